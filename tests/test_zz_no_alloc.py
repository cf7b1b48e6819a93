"""na_moe_decode_t950_noalloc (the decode expert body with its scratch in the library's own device array) against
na_moe_decode_t950 with caller scratch, through the C ABI: bit-identical outputs on consecutive calls that share the
array, a larger batch first and then smaller ones (B = 8, then 2, then 1 on the two-launch path, then 4 with the
expert-major down), with invalid and duplicate ids; the size and argument errors.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

H, NE, N_SLOTS = 2880, 128, 12


@pytest.fixture(scope="module")
def setup():
    import torch
    from neural_amd import synth
    from neural_amd.moe.layout import GPTOSS_LAYOUT_T950 as LT

    dev = torch.device("cuda", 0)
    print("case no-alloc decode fixture: 12 distinct t950 slots", flush=True)
    pool = synth.t950_pool_device(N_SLOTS, dev, seed=515)
    n = LT.n_layers * LT.n_experts
    tab = torch.from_numpy((np.arange(n) * 7 % N_SLOTS).astype(np.int64)).to(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    bgu = (torch.randn(n, LT.gate_up_n, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    bdn = (torch.randn(n, LT.down_n, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    return dict(dev=dev, pool=pool, tab=tab, bgu=bgu, bdn=bdn, LT=LT)


def _inputs(s, B, seed):
    import torch
    from neural_amd import synth
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(NE, 4, replace=False) for _ in range(B)]).astype(np.int64)
    if B >= 2:
        ids[1, 3] = -1                     # an invalid id: +0, no weights read
        ids[B - 1, 2] = ids[B - 1, 0]      # a token listing one expert twice
    w = rng.dirichlet(np.ones(4), size=B).astype(np.float32)
    x = synth.bf16_normal(rng, (B, H)).to(s["dev"])
    return x, torch.from_numpy(ids).to(s["dev"]), torch.from_numpy(w).to(torch.bfloat16).to(s["dev"])


def _with_scratch(s, x, ids, w, layer, down_mode):
    import torch
    from neural_amd import _native as N
    B = x.shape[0]
    h = torch.empty(4 * B, H, dtype=torch.bfloat16, device=s["dev"])
    yw = torch.empty(4 * B, H, dtype=torch.bfloat16, device=s["dev"])
    out = torch.empty(B, H, dtype=torch.bfloat16, device=s["dev"])
    N.call("na_moe_decode_t950", x.data_ptr(), ids.data_ptr(), w.data_ptr(), B, s["pool"].data_ptr(),
           s["LT"].slot_bytes, s["tab"].data_ptr(), layer * NE, s["bgu"].data_ptr(), s["bdn"].data_ptr(),
           h.data_ptr(), yw.data_ptr(), out.data_ptr(), 1.702, 7.0, 0, down_mode, None, N.stream(s["dev"]))
    return out


def _no_alloc(s, x, ids, w, layer, down_mode, out=None):
    import torch
    from neural_amd import _native as N
    B = x.shape[0]
    out = torch.full((B, H), float("nan"), dtype=torch.bfloat16, device=s["dev"]) if out is None else out
    rc = N.lib().na_moe_decode_t950_noalloc(x.data_ptr(), ids.data_ptr(), w.data_ptr(), B, s["pool"].data_ptr(),
                                            s["LT"].slot_bytes, s["tab"].data_ptr(), layer * NE, s["bgu"].data_ptr(),
                                            s["bdn"].data_ptr(), N.ptr(out), 1.702, 7.0, 0, down_mode,
                                            N.stream(s["dev"]))
    return rc, out


def test_no_alloc_equals_caller_scratch_on_consecutive_calls(setup):
    import torch
    s = setup
    for i, (B, layer, mode) in enumerate(((8, 3, 1), (2, 17, 1), (1, 35, 0), (4, 0, 1), (1, 5, 1))):
        print(f"case no-alloc decode call {i}: B={B} layer={layer} down_mode={mode}", flush=True)
        x, ids, w = _inputs(s, B, 100 + i)
        want = _with_scratch(s, x, ids, w, layer, mode)
        rc, got = _no_alloc(s, x, ids, w, layer, mode)
        torch.cuda.synchronize()
        assert rc == 0
        assert torch.equal(got, want), (B, layer, mode)
        assert bool(torch.isfinite(got.float()).all())


def test_no_alloc_size_and_argument_errors(setup):
    import torch
    s = setup
    print("case no-alloc decode errors", flush=True)
    x, ids, w = _inputs(s, 8, 7)
    x9 = torch.cat([x, x[:1]])
    ids9 = torch.cat([ids, ids[:1]])
    w9 = torch.cat([w, w[:1]])
    assert _no_alloc(s, x9, ids9, w9, 0, 1)[0] == -3            # beyond the array's 8 tokens
    from neural_amd import _native as N
    rc = N.lib().na_moe_decode_t950_noalloc(x.data_ptr(), ids.data_ptr(), w.data_ptr(), 8, s["pool"].data_ptr(),
                                            s["LT"].slot_bytes, s["tab"].data_ptr(), 0, None, None, None, 1.702, 7.0,
                                            0, 1, N.stream(s["dev"]))
    assert rc == -1                                              # no output: the result would stay in the array
    torch.cuda.synchronize()
