"""The sampling tail on the GPU (na_core_lm_tail_sample, DecodeModel.set_sampling) against the CPU oracle.

Bars: temp <= 0 gives the greedy tail's token; with temp > 0 the token is the oracle's Gumbel-max draw over the
kernel's own logits and the same uniforms (the on-device seeded draws reproduced exactly by oracle.uniform_draws, or
a caller array), or a near tie of the scores; over 6000 seeds the draws follow softmax(logits / temp) (chi-square at
1e-4); a captured decode step samples at every position with no host work, and replays equal eager steps.
"""
import numpy as np
import pytest
from scipy.stats import chi2

from oracle.bf16 import rb
from oracle.model_oracle import gumbel_scores, sample_token, uniform_draws

pytestmark = pytest.mark.gpu

H = 2880


class Tail:
    def __init__(self, vocab, rng, scale=1.0):
        import torch
        from neural_amd import _native as N
        self.N, self.torch = N, torch
        dev = self.dev = torch.device("cuda", 0)
        bf = torch.bfloat16
        t = lambda a: torch.from_numpy(np.asarray(a, np.float32)).to(bf).to(dev)  # noqa: E731
        self.vocab = vocab
        self.mid = t(rb(rng.standard_normal(H).astype(np.float32)))
        self.fw = t(np.ones(H, np.float32))
        self.Wl = t(rb((rng.standard_normal((vocab, H)) * scale / np.sqrt(H)).astype(np.float32)))
        self.hn = torch.empty(H, dtype=bf, device=dev)
        self.logits = torch.empty(vocab, dtype=bf, device=dev)
        self.part = torch.empty(N.lib().na_core_lm_partials(vocab), dtype=torch.int64, device=dev)
        self.tok = torch.zeros(1, dtype=torch.int64, device=dev)
        self.pos = torch.zeros(1, dtype=torch.int64, device=dev)
        self.temp = torch.zeros(1, dtype=torch.float32, device=dev)
        self.seed = torch.zeros(1, dtype=torch.int64, device=dev)

    def run(self, temp=None, seed=None, pos=None, u=None, sample=True):
        N = self.N
        if temp is not None:
            self.temp.fill_(temp)
        if seed is not None:
            self.seed.fill_(seed)
        if pos is not None:
            self.pos.fill_(pos)
        args = (self.mid.data_ptr(), None, None, self.fw.data_ptr(), 1e-5, self.Wl.data_ptr(), self.vocab,
                self.hn.data_ptr(), self.logits.data_ptr(), self.part.data_ptr(), self.tok.data_ptr(),
                self.pos.data_ptr(), 0, None, None, None, 0)
        if sample:
            N.call("na_core_lm_tail_sample", *args, self.temp.data_ptr(), N.ptr(u), self.seed.data_ptr(),
                   N.stream(self.dev))
        else:
            N.call("na_core_lm_tail", *args, N.stream(self.dev))


def _near_tie(scores, a, b):
    return abs(float(scores[a]) - float(scores[b])) <= 4 * np.finfo(np.float32).eps * max(1.0, abs(float(scores[a])))


def test_zero_temperature_is_greedy_and_draws_match_the_oracle():
    import torch
    print("case sampling tail vocab 4096", flush=True)
    tl = Tail(4096, np.random.default_rng(1), scale=4.0)
    tl.run(sample=False)
    torch.cuda.synchronize()
    greedy = int(tl.tok.item())
    tl.run(temp=0.0, seed=5, pos=9)
    torch.cuda.synchronize()
    assert int(tl.tok.item()) == greedy
    lg = tl.logits.float().cpu().numpy()
    for seed, pos, temp in ((0, 0, 1.0), (7, 123, 0.7), (2 ** 40 + 3, 4095, 1.3), (99, 7, 0.05)):
        tl.run(temp=temp, seed=seed, pos=pos)
        torch.cuda.synchronize()
        got = int(tl.tok.item())
        u = uniform_draws(seed, pos, 4096)
        want = sample_token(lg, temp, u)
        sc = gumbel_scores(lg, temp, u)
        assert got == want or _near_tie(sc, got, want), (seed, pos, temp, got, want)
    # caller-provided uniforms (the reference's u_dev)
    rng = np.random.default_rng(3)
    u = rng.random(4096).astype(np.float32)
    ud = torch.from_numpy(u).cuda()
    tl.run(temp=0.9, u=ud)
    torch.cuda.synchronize()
    got, want = int(tl.tok.item()), sample_token(lg, 0.9, u)
    assert got == want or _near_tie(gumbel_scores(lg, 0.9, u), got, want)


def test_draws_follow_the_softmax():
    import torch
    print("case sampling tail distribution", flush=True)
    V, n, temp = 12, 6000, 0.8
    tl = Tail(V, np.random.default_rng(2), scale=1.2)
    toks = torch.empty(n, dtype=torch.int64, device=tl.dev)
    tl.run(temp=temp, pos=11)
    for s in range(n):
        tl.run(seed=s)
        toks[s:s + 1].copy_(tl.tok)
    torch.cuda.synchronize()
    lg = tl.logits.float().cpu().numpy()
    p = np.exp((lg - lg.max()) / temp)
    p /= p.sum()
    assert p.max() < 0.9 and (p > 0.01).sum() >= 4, p           # a spread the test can see
    counts = np.bincount(toks.cpu().numpy(), minlength=V)
    keep = n * p >= 5
    stat = float(((counts[keep] - n * p[keep]) ** 2 / (n * p[keep])).sum())
    assert stat < chi2.ppf(1 - 1e-4, df=int(keep.sum()) - 1), (stat, counts, n * p)
    assert counts[~keep].sum() <= max(10, 5 * n * p[~keep].sum())


def test_model_sampling_graph_equals_eager():
    """A DecodeModel with the sampling tail: greedy decode by graph replays with temperature 0 equals the greedy
    model; with temperature 1 the captured steps sample (tokens vary with the seed) and replays equal eager steps."""
    import torch
    from neural_amd import synth, tiles
    from neural_amd.model import DecodeModel, random_weights
    from neural_amd.moe.experts import ResidentExperts
    from neural_amd.moe.layout import GPTOSS_LAYOUT_T950 as LT
    print("case sampling model 2 layers", flush=True)
    dev = torch.device("cuda", 0)
    w = random_weights(n_layers=2, vocab=2048, device="cpu", seed=4, window=16).to(dev)
    rng = np.random.default_rng(8)
    raw = torch.from_numpy(np.stack([synth.slot_raw(rng) for _ in range(4)])).to(dev)
    pool = torch.empty(4, LT.slot_bytes, dtype=torch.uint8, device=dev)
    tiles.repack_to_t950(raw, pool)
    tab = torch.from_numpy(np.arange(LT.n_layers * LT.n_experts) % 4).to(dev)
    rx = ResidentExperts(pool, LT, slot_tab=tab, max_batch=1)
    prompt = np.random.default_rng(9).integers(0, 2048, 10)

    def run(sample, temp, seed, graph):
        m = DecodeModel(w, rx, smax=40, n_split=4, sample=sample)
        if sample:
            m.set_sampling(temp, seed)
        m.prefill(prompt)
        m.run(12, graph=graph)
        torch.cuda.synchronize()
        return m.seq[:23].cpu().numpy()

    greedy = run(False, 0, 0, True)
    assert np.array_equal(run(True, 0.0, 3, True), greedy)
    a = run(True, 1.0, 3, True)
    assert np.array_equal(a, run(True, 1.0, 3, False))
    b = run(True, 1.0, 4, True)
    assert np.array_equal(a[:10], prompt) and not np.array_equal(a[10:], b[10:])
