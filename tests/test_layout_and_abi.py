"""CPU: store geometry and pool views (the reference's tests/test_scale_layout.py:44-116 restated for this
package), ragged tile plans (tests/test_grouped_gemm_plan.py), and the C-ABI library: it loads and exports every
symbol include/neural_amd.h declares (no compute call: there is no GPU here)."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from neural_amd import scale_pack as sp
from neural_amd import synth
from neural_amd.moe.layout import (GPTOSS_LAYOUT, GPTOSS_LAYOUT_PS4, ExpertLayout, gptoss_layout_for_repr,
                                   mxfp4_pool_views, prepacked_descriptor)
from neural_amd.q80.mxfp4_kernels import GroupedGemmPlan, _grouped_tile_rows, _scale_layout

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

RAW_STORE_DESCRIPTOR = {"slot_bytes": 13219200, "n_layers": 36, "n_experts": 128, "hidden": 2880, "gate_up_n": 5760,
                        "down_n": 2880, "down_k": 2880, "int4_group": 32, "inner_k_tiles": 2,
                        "kernel": "neural.q80.mxfp4_kernels (Triton, fp32-accum)", "weight_repr": "mxfp4_g32"}


def test_layout_arithmetic():
    assert GPTOSS_LAYOUT.slot_bytes == 13_219_200 == sp.SLOT_RAW
    assert GPTOSS_LAYOUT_PS4.slot_bytes == 12_839_040 == sp.SLOT_PACKED
    assert GPTOSS_LAYOUT_PS4.gate_saz_bytes == 5760 * 46 and GPTOSS_LAYOUT_PS4.down_saz_bytes == 2880 * 46
    assert GPTOSS_LAYOUT.gate_pack_bytes == GPTOSS_LAYOUT_PS4.gate_pack_bytes == 5760 * 1440
    assert (GPTOSS_LAYOUT.scale_layout_mode, GPTOSS_LAYOUT_PS4.scale_layout_mode) == (0, 1)
    assert GPTOSS_LAYOUT.is_mxfp4 and GPTOSS_LAYOUT_PS4.is_mxfp4
    assert gptoss_layout_for_repr("mxfp4_g32") is GPTOSS_LAYOUT
    assert gptoss_layout_for_repr("mxfp4_g32_ps4") is GPTOSS_LAYOUT_PS4
    assert round(100 * (1 - 12_839_040 / 13_219_200), 2) == 2.88
    with pytest.raises(KeyError):
        gptoss_layout_for_repr("int4_g32")
    with pytest.raises(ValueError):
        ExpertLayout("q", 1, 1, 1, 64, 64, 64, 32, weight_repr="int4_g32")


def test_descriptors():
    raw = prepacked_descriptor(GPTOSS_LAYOUT)
    assert {k: v for k, v in raw.items() if k != "row"} == RAW_STORE_DESCRIPTOR
    ps4 = prepacked_descriptor(GPTOSS_LAYOUT_PS4)
    assert ps4["weight_repr"] == "mxfp4_g32_ps4" and ps4["slot_bytes"] == 12_839_040
    diff = {k for k in set(raw) | set(ps4) if raw.get(k) != ps4.get(k)}
    assert {"slot_bytes", "weight_repr", "kernel"} <= diff


def _pools(cap=3, seed=1):
    rng = np.random.default_rng(seed)
    raws = [synth.slot_raw(rng) for _ in range(cap)]
    return torch.from_numpy(np.stack(raws)), torch.from_numpy(np.stack([sp.pack_slot(r) for r in raws]))


def test_pool_views_place_the_scales():
    raw_pool, pk_pool = _pools()
    gb, db, gs, ds = mxfp4_pool_views(raw_pool, GPTOSS_LAYOUT)
    gb2, db2, gs2, ds2 = mxfp4_pool_views(pk_pool, GPTOSS_LAYOUT_PS4)
    assert gs.shape == (3, 5760, 90) and ds.shape == (3, 2880, 90)
    assert gs2.shape == (3, 5760, 46) and ds2.shape == (3, 2880, 46)
    assert gb.shape == gb2.shape == (3, 5760, 90, 16) and db.shape == db2.shape == (3, 2880, 90, 16)
    assert gs.stride(0) == 13_219_200 and gs2.stride(0) == 12_839_040 and gs2.stride(1) == 46 and gs2.stride(2) == 1
    for i in range(3):
        assert torch.equal(gb[i], gb2[i]) and torch.equal(db[i], db2[i])
        assert np.array_equal(sp.unpack_scale_rows(gs2[i].numpy()), gs[i].numpy())
        assert np.array_equal(sp.unpack_scale_rows(ds2[i].numpy()), ds[i].numpy())
    with pytest.raises(AssertionError):
        mxfp4_pool_views(raw_pool, GPTOSS_LAYOUT_PS4)


def test_launchers_infer_the_layout_from_the_view():
    raw_pool, pk_pool = _pools(cap=2)
    _, _, gs, ds = mxfp4_pool_views(raw_pool, GPTOSS_LAYOUT)
    _, _, gs2, ds2 = mxfp4_pool_views(pk_pool, GPTOSS_LAYOUT_PS4)
    GK = 90
    assert _scale_layout(gs, GK, None) is False and _scale_layout(ds, GK, None) is False
    assert _scale_layout(gs2, GK, None) is True and _scale_layout(ds2, GK, None) is True
    assert _scale_layout(gs, GK, False) is False and _scale_layout(gs2, GK, True) is True
    with pytest.raises(ValueError):
        _scale_layout(gs, GK, True)
    with pytest.raises(ValueError):
        _scale_layout(gs2, GK, False)
    with pytest.raises(ValueError):
        _scale_layout(torch.zeros(2, 8, 47, dtype=torch.uint8), GK, None)
    with pytest.raises(ValueError):
        _scale_layout(torch.zeros(2, 8, 180, dtype=torch.uint8)[:, :, ::2], GK, None)


# ---------------------------------------------------------------- ragged tile plans (reference test_grouped_gemm_plan)
def test_pair_local_tiles_at_every_bm_boundary():
    descs = [(100, 200, i, m) for i, m in enumerate((0, 1, 15, 16, 17, 63, 64, 65, 128, 129))]
    for bm in (16, 32, 64, 128):
        rows = _grouped_tile_rows(descs, bm)
        for desc in descs:
            actual = [r for r in rows if r[2] == desc[2]]
            assert [r[4] for r in actual] == list(range((desc[3] + bm - 1) // bm))
            assert all(r[:4] == desc for r in actual)
            positions = [p for r in actual for p in range(r[4] * bm, min((r[4] + 1) * bm, r[3]))]
            assert positions == list(range(desc[3]))


def test_plan_keeps_pointer_offsets_and_original_pair_boundaries():
    xs = torch.empty(140 * 64 + 9, dtype=torch.bfloat16)
    ys = torch.empty(140 * 33 + 13, dtype=torch.bfloat16)
    pairs = [(xs[1:1 + 65 * 64].view(65, 64), 2, ys[3:3 + 65 * 33].view(65, 33)),
             (xs[1 + 65 * 64:1 + 130 * 64].view(65, 64), 2, ys[3 + 65 * 33:3 + 130 * 33].view(65, 33))]
    plan = GroupedGemmPlan(pairs, block_m=64)
    assert plan.metadata.device.type == "cpu"
    assert (plan.K, plan.N, plan.ntiles, plan.slots) == (64, 33, 4, (2, 2))
    assert plan.metadata.tolist() == [
        [pairs[0][0].data_ptr(), pairs[0][2].data_ptr(), 2, 65, 0],
        [pairs[0][0].data_ptr(), pairs[0][2].data_ptr(), 2, 65, 1],
        [pairs[1][0].data_ptr(), pairs[1][2].data_ptr(), 2, 65, 0],
        [pairs[1][0].data_ptr(), pairs[1][2].data_ptr(), 2, 65, 1]]
    assert plan.pairs[0][0] is pairs[0][0]


@pytest.mark.parametrize("bm", [0, 1, 15, 24, 63])
def test_invalid_tile_height(bm):
    with pytest.raises(ValueError, match="power of two"):
        _grouped_tile_rows((), bm)


@pytest.mark.parametrize("desc", [(1, 2, -1, 3), (1, 2, 0, -3), (1, 2, 0, 2 ** 31), (-1, 2, 0, 3), (1, 2, 0)])
def test_invalid_descriptor(desc):
    with pytest.raises(ValueError):
        _grouped_tile_rows([desc], 64)


def test_empty_pairs_are_safe():
    assert GroupedGemmPlan([]).metadata.shape == (0, 5)
    plan = GroupedGemmPlan([(torch.empty(0, 64, dtype=torch.bfloat16), 0, torch.empty(0, 16, dtype=torch.bfloat16))])
    assert plan.ntiles == 0


def test_alignment_hint_requires_both_pointers_and_row_pitches():
    x = torch.empty(4, 64, dtype=torch.bfloat16)
    y = torch.empty(4, 32, dtype=torch.bfloat16)
    assert GroupedGemmPlan([(x, 0, y)]).aligned
    xp = torch.empty(4 * 64 + 1, dtype=torch.bfloat16)
    yp = torch.empty(4 * 32 + 1, dtype=torch.bfloat16)
    assert not GroupedGemmPlan([(xp[1:].view(4, 64), 0, y)]).aligned
    assert not GroupedGemmPlan([(x, 0, yp[1:].view(4, 32))]).aligned
    odd_pitch = torch.empty(4, 33, dtype=torch.bfloat16)
    assert not GroupedGemmPlan([(x, 0, odd_pitch)]).aligned
    assert GroupedGemmPlan([(x, 0, y), (x[:0], 1, y[:0])]).aligned


def test_reject_overlapping_outputs_and_input_output_alias():
    x = torch.empty(32, 64, dtype=torch.bfloat16)
    y = torch.empty(32, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="output slices overlap"):
        GroupedGemmPlan([(x[:16], 0, y[:16]), (x[16:], 1, y[8:24])])
    with pytest.raises(ValueError, match="overlap an input"):
        GroupedGemmPlan([(x[:16], 0, x[16:]), (x[16:], 1, y[:16])])
    with pytest.raises(ValueError, match="overlap an input"):
        GroupedGemmPlan([(x, 0, x)])


def test_reject_bad_shapes_dtypes_and_strides():
    x = torch.empty(3, 64, dtype=torch.bfloat16)
    y = torch.empty(3, 16, dtype=torch.bfloat16)
    for pairs in ([(x, 0, y[:2])], [(x.float(), 0, y)], [(x[:, ::2], 0, y)],
                  [(x, 0, y), (torch.empty(3, 32, dtype=torch.bfloat16), 1, y.clone())]):
        with pytest.raises(ValueError):
            GroupedGemmPlan(pairs)


# -------------------------------------------------------------------------------------------------------- ABI
def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "neural_amd.h")).read()
    return sorted(set(re.findall(r"\b(?:int|long long)\s+(na_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from neural_amd import _native as N
    lib = N.lib()
    syms = _declared_symbols()
    assert len(syms) >= 4
    for s in syms:
        assert hasattr(lib, s), s
        assert s in N.SIGNATURES, f"{s} has no ctypes signature"
    assert set(N.SIGNATURES) == set(syms)
    assert lib.na_version() == 1
    assert lib.na_t950_slot_bytes() == 13_271_040


def test_library_rejects_bad_arguments_without_launching():
    """Argument validation happens before any HIP call, so it is checkable without a GPU."""
    from neural_amd import _native as N
    lib = N.lib()
    assert lib.na_mxfp4_gemv(None, 0, None, 0, None, 0, 0, None, 4, None, 0, None, 5760, 2880, 0, None) == -1
    assert lib.na_moe_decode(None, None, None, 1, None, 0, 0, None, 0, None, None, None, None, None,
                             ctypes.c_float(1.702), ctypes.c_float(7.0), 0, 0, None, None) == -1


def test_product_code_never_touches_the_oracle():
    """The oracle is the checker only: no module of the package imports, loads or runs anything under oracle/."""
    pkg = os.path.join(ROOT, "neural_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"\boracle\b", text), f"{f} mentions the oracle"


def test_ring_reuse_rule_truth_table():
    """reference tests/test_attention.py:309-311"""
    from neural_amd import attention as A
    rr = [A.ring_reuse_ok(1000, 999, 128), A.ring_reuse_ok(1000, 998, 128), A.ring_reuse_ok(100, 7, 128),
          A.ring_reuse_ok(1000, 1001, 128), A.ring_reuse_ok(2000, 1200, 1024)]
    assert rr == [True, False, True, False, True]


def test_attention_workspace_and_argument_checks():
    from neural_amd import _native as N
    lib = N.lib()
    assert lib.na_attn_workspace_floats(1, 32) == 1 * 8 * 32 * (8 + 8 + 512)
    assert lib.na_attn_workspace_floats(1, 65) == -1
    assert lib.na_decode_attention(None, None, None, 1, None, None, None, 1, ctypes.c_float(0.125), 0, 0, 1,
                                   None, None, None, None) == -1


def test_prefill_attention_argument_checks():
    """Host-side validation of na_prefill_attention / na_ring_write (no launch happens on any of these)."""
    from neural_amd import _native as N
    lib = N.lib()
    f = ctypes.c_float(0.125)
    a = 1 << 20                                   # an aligned non-null stand-in; never dereferenced here
    # missing pointers; ring without a window; ring != cache_rows; positions beyond the cache; negative T
    assert lib.na_prefill_attention(None, a, a, 64, None, None, 0, 0, 0, 0, a, a, 0, 4, f, 0, 0, None, None) == -1
    assert lib.na_prefill_attention(a, a, a, 128, a, a, 512, 64, 512, 64, a, a, 0, 4, f, 0, 128, None, None) == -1
    assert lib.na_prefill_attention(a, a, a, 64, a, a, 512, 64, 512, 64, a, a, 0, 4, f, 128, 128, None, None) == -1
    assert lib.na_prefill_attention(a, a, a, 64, None, None, 0, 0, 0, 0, a, a, 62, 4, f, 0, 0, None, None) == -1
    assert lib.na_prefill_attention(a, a, a, 64, None, None, 0, 0, 0, 0, a, a, 0, -1, f, 0, 0, None, None) == -1
    # strides not a multiple of 8 elements in ring mode; misaligned q
    assert lib.na_prefill_attention(a, a, a, 128, a, a, 510, 64, 512, 64, a, a, 0, 4, f, 128, 128, None, None) == -1
    assert lib.na_prefill_attention(a + 2, a, a, 64, None, None, 0, 0, 0, 0, a, a, 0, 4, f, 0, 0, None, None) == -1
    # T = 0 is a valid empty call and launches nothing
    assert lib.na_prefill_attention(a, a, a, 64, None, None, 0, 0, 0, 0, a, a, 0, 0, f, 0, 0, None, None) == 0
    assert lib.na_prefill_attention(None, a, a, 64, None, None, 0, 0, 0, 0, a, a, 0, 0, f, 0, 0, None, None) == 0
    assert lib.na_ring_write(a, a, 0, a, a, 512, 64, 512, 64, 0, 4, None) == -1
    assert lib.na_ring_write(a, a, 128, a, a, 512, 64, 512, 64, 0, 0, None) == 0
