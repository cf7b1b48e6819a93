"""CPU: what constructing neural_amd.fused_core.FusedCore does to the core-graphs object it is given (the drop-in
contract of the reference's fused_core.py:505-607), and run()'s host-side refusals, which happen before any launch.

- every layer's q/k/v weights and biases end up as row views of one fused [5120, 2880] / [5120] buffer holding the
  original values, and the modules compute with the same values as before;
- lg.ring is set on every layer; with ring > 0 each sliding layer gets new zeroed [1, 8, ring, 64] caches, the full
  layers keep their own cache tensors; a ring smaller than the window is refused;
- split_k > 1 builds one chunked-attention workspace for the full layers, which must share one smax;
- snapshot_rings / restore_rings copy the ring contents back into the same tensors;
- run() refuses a cache override of the wrong layout (AssertionError, checked on the host).
"""
import pytest
import torch

from neural_amd import fused_core as fc
from neural_amd.model import random_weights

H, NQ, NKV, HD = 2880, 64, 8, 64


@pytest.fixture()
def cg():
    w = random_weights(n_layers=3, vocab=256, device="cpu", seed=9, window=32)
    return fc.core_graphs(w, 96, "cpu")


def _attn(lg):
    return lg.layer.self_attn


def test_projections_become_views_of_one_fused_buffer(cg):
    before = [[(getattr(_attn(lg), p).weight.clone(), getattr(_attn(lg), p).bias.clone())
               for p in ("q_proj", "k_proj", "v_proj")] for lg in cg.layers]
    core = fc.FusedCore(cg, "cpu")
    for L, lg in enumerate(cg.layers):
        W, B = core.W[L], core.B[L]
        assert tuple(W.shape) == ((NQ + 2 * NKV) * HD, H) and tuple(B.shape) == ((NQ + 2 * NKV) * HD,)
        rows = [(0, 4096), (4096, 4608), (4608, 5120)]
        for (lo, hi), p, (w0, b0) in zip(rows, ("q_proj", "k_proj", "v_proj"), before[L]):
            proj = getattr(_attn(lg), p)
            assert torch.equal(W[lo:hi], w0) and torch.equal(B[lo:hi], b0)
            assert proj.weight.data_ptr() == W.data_ptr() + lo * H * 2
            assert proj.bias.data_ptr() == B.data_ptr() + lo * 2
            assert torch.equal(proj.weight, w0)
        W[0, 0] = 7.0                                  # one storage: a write through the fused buffer shows in q_proj
        assert _attn(lg).q_proj.weight[0, 0].item() == 7.0


def test_rings_and_cfg(cg):
    sliding = [bool(lg.sliding) for lg in cg.layers]
    assert sliding == [True, False, True]
    full_k = cg.layers[1].k
    core = fc.FusedCore(cg, "cpu", ring=48, qkv_bk=64, attn_bn=32)
    assert [lg.ring for lg in cg.layers] == [48, 0, 48] == [core.layer_ring(L) for L in range(3)]
    for lg in (cg.layers[0], cg.layers[2]):
        assert tuple(lg.k.shape) == tuple(lg.v.shape) == (1, NKV, 48, HD)
        assert lg.k.dtype == torch.bfloat16 and not lg.k.any() and lg.k.data_ptr() != lg.v.data_ptr()
    assert cg.layers[1].k is full_k and core.split is None
    assert core.cfg == dict(qkv_bk=64, qkv_warps=4, o_rows=16, o_bk=256, o_warps=4, r_rows=8, r_bk=256, attn_bn=32,
                            ring=48, split_k=1, split_bn=64, split_cache_s=True, near_miss=False)
    assert fc.FusedCore(cg, "cpu").layer_ring(0) == 0           # ring = 0 resets every layer to linear


def test_ring_must_cover_the_window(cg):
    with pytest.raises(AssertionError, match="smaller than the sliding window"):
        fc.FusedCore(cg, "cpu", ring=16)


def test_split_workspace(cg):
    core = fc.FusedCore(cg, "cpu", split_k=8)
    assert core.split is not None and core.split.ns == 8 and core.split.smax == 96
    cg2 = fc.core_graphs(random_weights(n_layers=4, vocab=256, device="cpu", seed=1, window=32), 96, "cpu")
    cg2.layers[3].smax = 128
    with pytest.raises(AssertionError, match="different smax"):
        fc.FusedCore(cg2, "cpu", split_k=4)
    fc.FusedCore(cg2, "cpu", split_k=1)                          # without split-K the full layers may differ
    for bad in (0, 65):
        with pytest.raises(AssertionError):
            fc.FusedCore(cg, "cpu", split_k=bad)


def test_snapshot_and_restore_keep_the_tensors(cg):
    core = fc.FusedCore(cg, "cpu", ring=32)
    for i, lg in enumerate(cg.layers):
        lg.k.fill_(i + 1)
        lg.v.fill_(-(i + 1))
    snap = core.snapshot_rings()
    assert snap[1] is None and all(s is not None for s in (snap[0], snap[2]))
    ptrs = [(lg.k.data_ptr(), lg.v.data_ptr()) for lg in cg.layers]
    for lg in cg.layers:
        lg.k.zero_()
        lg.v.zero_()
    core.restore_rings(snap)
    assert [(lg.k.data_ptr(), lg.v.data_ptr()) for lg in cg.layers] == ptrs
    assert cg.layers[0].k.eq(1).all() and cg.layers[2].v.eq(-3).all()
    assert not cg.layers[1].k.any()                              # a linear layer is neither saved nor restored


def test_run_refuses_a_cache_of_the_wrong_layout(cg):
    core = fc.FusedCore(cg, "cpu", ring=32)
    linear = torch.zeros(1, NKV, 96, HD, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="ring layout"):
        core.run(0, None, None, None, None, None, None, None, None, None, kc=linear)
    with pytest.raises(AssertionError, match="linear layout"):
        core.run(1, None, None, None, None, None, None, None, None, None, vc=linear[:, :, :64].contiguous())
    with pytest.raises(AssertionError, match="contiguous bf16"):
        core.run(1, None, None, None, None, None, None, None, None, None, kc=linear.float())
