"""The fused attention block of a decode layer (na_core_attn_block: QKV, attention, o_proj and router as four phases
of one launch, reference fused_core.py:581-629) against the four separate launches it replaces, on the GPU.

Bar: bit-identical outputs (q, the K / V rows, xbuf, att, mid, hn, router logits' selection and weights, here made
by the single-launch expert body from the block's logits) and caches
over consecutive decode steps of a 2-layer model with a sliding layer on a 16-row ring and a full layer, for the full
layer's attention in 1, 4 and 32 chunks (chunks past the position are empty), across the ring wrap; each launch
leaves its split counters at zero, advances its generation word (the tag of its handoff words) by one and leaves the
error flag clear; graph replays equal eager steps.  The same bar at configuration 4's geometry (window 128 on a
128-row ring, 4360 cache rows, 18 and 32 chunks) after a 4090-token prefill, across two ring wraps.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

H, NE, VOCAB, WIN, N_SLOTS, SMAX = 2880, 128, 4096, 16, 8, 64
LINE = 64                                   # uint32 words per line of the sync buffer: 0 error, 1 generation, 2-9 split
ENTERED = 203                               # the router workgroups' entry count (the expert body selects the top 4)


def _sync_state(sync):
    """(error word, generation word, split counters + router entry count): every completed launch leaves the
    counters at zero."""
    s = sync.cpu().numpy().view(np.uint32)
    return int(s[0]), int(s[LINE]), int(s[2 * LINE:10 * LINE].sum()) + int(s[ENTERED * LINE])


@pytest.fixture(scope="module")
def parts():
    import torch
    from neural_amd import synth
    from neural_amd.model import random_weights
    from neural_amd.moe.experts import ResidentExperts
    from neural_amd.moe.layout import GPTOSS_LAYOUT_T950 as LT

    dev = torch.device("cuda", 0)
    print("case attention block fixture: 2 layers, vocab 4096, window 16", flush=True)
    w = random_weights(n_layers=2, vocab=VOCAB, device="cpu", seed=17, window=WIN, norm_std=0.1).to(dev)
    pool = synth.t950_pool_device(2 * N_SLOTS, dev, seed=61)
    n = LT.n_layers * LT.n_experts
    tab = np.zeros(n, np.int64)
    for li in range(2):
        tab[li * NE:(li + 1) * NE] = li * N_SLOTS + np.arange(NE) % N_SLOTS
    rx = ResidentExperts(pool, LT, None, None, torch.from_numpy(tab).to(dev), max_batch=1)
    return dict(dev=dev, w=w, rx=rx)


def _pair(parts, ns):
    from neural_amd.model import DecodeModel
    a = DecodeModel(parts["w"], parts["rx"], smax=SMAX, n_split=ns, fused_attn=True)
    b = DecodeModel(parts["w"], parts["rx"], smax=SMAX, n_split=ns, fused_attn=False)
    return a, b


@pytest.mark.parametrize("ns", [1, 4, 32])
def test_fused_block_equals_four_launches(parts, ns):
    import torch
    print(f"case attention block fused vs 4 launches, n_split={ns}", flush=True)
    fa, fb = _pair(parts, ns)
    prompt = np.random.default_rng(300 + ns).integers(0, VOCAB, 12)
    fa.reset(prompt)
    fb.reset(prompt)
    for p in range(40):                                  # past the 16-row ring's wrap, prompt then greedy
        for m in (fa, fb):
            m.embed()
        for li in range(2):
            fa.layer(li)
            fb.layer(li)
            torch.cuda.synchronize()
            for nm in ("q", "att", "xbuf", "mid", "hn", "ids", "wts", "g"):
                assert torch.equal(getattr(fa, nm), getattr(fb, nm)), (p, li, nm)
            assert torch.equal(fa.kc[li], fb.kc[li]) and torch.equal(fa.vc[li], fb.vc[li]), (p, li)
        for m in (fa, fb):
            m.tail()
        torch.cuda.synchronize()
        assert int(fa.tok.item()) == int(fb.tok.item()), p
    assert torch.equal(fa.seq, fb.seq)
    assert not fa.sync_error()
    assert _sync_state(fa.sync) == (0, 40 * 2, 0)


def test_fused_block_graph_replay_equals_eager(parts):
    import torch
    print("case attention block graph replay vs eager", flush=True)
    fa, _ = _pair(parts, 8)
    prompt = np.random.default_rng(5).integers(0, VOCAB, 9)
    eager = fa.generate(prompt, 30, graph=False)
    first = fa.generate(prompt, 30, graph=True)
    again = fa.generate(prompt, 30, graph=True)
    assert torch.equal(eager, first) and torch.equal(first, again)
    err, gen, counters = _sync_state(fa.sync)
    assert not fa.sync_error() and err == 0 and counters == 0 and gen > 0


@pytest.mark.parametrize("ns", [18, 32])
def test_fused_block_equals_four_launches_at_model_size(parts, ns):
    """Configuration 4's attention geometry: a sliding layer with window 128 on a 128-row ring and a full layer of
    4360 cache rows whose attention runs in 18 chunks (the bench's automatic split: one 256-key pass per chunk) or 32.  A 4090-token context is prefilled into both models' caches
    (the same kernels, so the caches start equal), then 140 greedy steps at positions 4090 .. 4229 (the ring wraps
    at 4096 and 4224): every output of every layer and the caches bit for bit, the error word clear."""
    import torch
    from neural_amd.model import DecodeModel, random_weights
    print(f"case attention block fused vs 4 launches at window 128, smax 4360, n_split {ns}", flush=True)
    w = random_weights(n_layers=2, vocab=VOCAB, device="cpu", seed=23, window=128, norm_std=0.1).to(parts["dev"])
    assert [ly.sliding for ly in w.layers] == [128, 0]
    fa = DecodeModel(w, parts["rx"], smax=4360, n_split=ns, fused_attn=True)
    fb = DecodeModel(w, parts["rx"], smax=4360, n_split=ns, fused_attn=False)
    assert fa.ring == 128 and tuple(fa.kc[0].shape) == (1, 8, 128, 64) and tuple(fa.kc[1].shape) == (1, 8, 4360, 64)
    prompt = np.random.default_rng(4090).integers(0, VOCAB, 4090)
    for m in (fa, fb):
        m.prefill(prompt)
    torch.cuda.synchronize()
    for li in range(2):
        assert torch.equal(fa.kc[li], fb.kc[li]) and torch.equal(fa.vc[li], fb.vc[li]), li
    assert int(fa.pos.item()) == 4090 and torch.equal(fa.seq, fb.seq)
    for step in range(140):
        for m in (fa, fb):
            m.embed()
        for li in range(2):
            fa.layer(li)
            fb.layer(li)
            torch.cuda.synchronize()
            for nm in ("q", "att", "xbuf", "mid", "hn", "ids", "wts", "g"):
                assert torch.equal(getattr(fa, nm), getattr(fb, nm)), (4090 + step, li, nm)
            assert torch.equal(fa.kc[li], fb.kc[li]) and torch.equal(fa.vc[li], fb.vc[li]), (4090 + step, li)
        for m in (fa, fb):
            m.tail()
        torch.cuda.synchronize()
        assert int(fa.tok.item()) == int(fb.tok.item()), 4090 + step
    assert torch.equal(fa.seq, fb.seq) and int(fa.pos.item()) == 4230
    assert not fa.sync_error()
    err, _, counters = _sync_state(fa.sync)
    assert err == 0 and counters == 0
