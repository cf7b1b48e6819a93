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
    assert GPTOSS_LAYOUT.slot_bytes == 13_219_200 == sp.RAW_SLOT_BYTES
    assert GPTOSS_LAYOUT_PS4.slot_bytes == 12_839_040 == sp.PS4_SLOT_BYTES
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


# ------------------------------------------------------------------- ragged tile plans (contract: mxfp4_kernels.py:298-382)
# The tile table of a grouped launch lists, pair by pair in the order given, one row (x address, out address, slot,
# M, pm) per block of block_m rows of the pair; tiles never span two pairs and empty pairs get none.

def test_tile_rows_known_answer():
    descs = [(0x1000, 0x9000, 5, 40), (0x2000, 0xA000, 7, 0), (0x3000, 0xB000, 1, 33), (0x1000, 0xC000, 5, 32)]
    assert _grouped_tile_rows(descs, 32) == [
        (0x1000, 0x9000, 5, 40, 0), (0x1000, 0x9000, 5, 40, 1),
        (0x3000, 0xB000, 1, 33, 0), (0x3000, 0xB000, 1, 33, 1),
        (0x1000, 0xC000, 5, 32, 0)]
    assert [r[4] for r in _grouped_tile_rows(descs, 16)] == [0, 1, 2, 0, 1, 2, 0, 1]
    assert len(_grouped_tile_rows(descs, 256)) == 3
    assert _grouped_tile_rows([], 16) == []


@pytest.mark.parametrize("bm", [16, 64, 512])
def test_tile_rows_cover_each_pair_exactly_once(bm):
    rng = np.random.default_rng(bm)
    ms = [0, 2, 31, 96, 97, 255, 256, 257, 1000] + rng.integers(0, 700, 6).tolist()
    descs = [(0x4000 + 64 * i, 0x800000 + 64 * i, int(rng.integers(0, 4608)), m) for i, m in enumerate(ms)]
    rows = _grouped_tile_rows(descs, bm)
    covered = {}
    for x, y, slot, m, pm in rows:
        assert 0 <= pm * bm < m
        covered.setdefault((x, y, slot, m), []).extend(range(pm * bm, min(m, (pm + 1) * bm)))
    for d in descs:
        assert covered.get(d, []) == list(range(d[3]))
    assert len(rows) == sum(-(-m // bm) for m in ms)


def test_plan_tables_follow_the_tensors_addresses():
    K, N = 128, 48
    xbuf = torch.empty(90 * K + 24, dtype=torch.bfloat16)
    ybuf = torch.empty(90 * N + 40, dtype=torch.bfloat16)
    xa = xbuf[8:8 + 70 * K].view(70, K)
    xb = xbuf[8 + 70 * K:8 + 80 * K].view(10, K)
    ya = ybuf[40:40 + 70 * N].view(70, N)
    yb = ybuf[40 + 70 * N:40 + 80 * N].view(10, N)
    plan = GroupedGemmPlan([(xa, 9, ya), (xb, 4, yb), (xa[:0], 3, ybuf[40 + 80 * N:40 + 90 * N].view(10, N)[:0])],
                           block_m=32)
    assert (plan.K, plan.N, plan.block_m, plan.slots, plan.ntiles) == (K, N, 32, (9, 4, 3), 4)
    x0, y0 = xbuf.data_ptr() + 2 * 8, ybuf.data_ptr() + 2 * 40
    assert plan.metadata.tolist() == [[x0, y0, 9, 70, 0], [x0, y0, 9, 70, 1], [x0, y0, 9, 70, 2],
                                      [x0 + 2 * 70 * K, y0 + 2 * 70 * N, 4, 10, 0]]
    assert plan.metadata.device.type == "cpu" and plan.metadata_host.shape == (4, 5)
    assert plan.pairs[1][0] is xb


@pytest.mark.parametrize("bm", [-16, 0, 8, 48, 100, 2 ** 20 + 1])
def test_tile_height_must_be_a_power_of_two_of_16_or_more(bm):
    with pytest.raises(ValueError, match="power of two"):
        _grouped_tile_rows([(0, 0, 0, 5)], bm)


@pytest.mark.parametrize("desc", [(0x10, 0x20, -4, 8), (0x10, 0x20, 1, -1), (0x10, 0x20, 1, 2 ** 31),
                                  (0x10, -0x20, 1, 8), (0x10, 0x20, 1), (0x10, 0x20, 1, 8, 0)])
def test_malformed_descriptors_are_refused(desc):
    with pytest.raises(ValueError):
        _grouped_tile_rows([desc], 16)


def test_plans_without_rows():
    plan = GroupedGemmPlan([])
    assert plan.ntiles == 0 and tuple(plan.metadata.shape) == (0, 5) and plan.slots == ()
    z = torch.empty(0, 96, dtype=torch.bfloat16)
    plan = GroupedGemmPlan([(z, 3, torch.empty(0, 8, dtype=torch.bfloat16)), (z, 5, torch.empty(0, 8,
                                                                                             dtype=torch.bfloat16))])
    assert plan.ntiles == 0 and plan.slots == (3, 5) and plan.aligned


def test_alignment_flag():
    buf = torch.empty(4096, dtype=torch.bfloat16)
    x, y = buf[:6 * 96].view(6, 96), buf[1024:1024 + 6 * 16].view(6, 16)
    assert GroupedGemmPlan([(x, 0, y)]).aligned
    assert not GroupedGemmPlan([(buf[4:4 + 6 * 96].view(6, 96), 0, y)]).aligned            # 8-byte offset
    assert not GroupedGemmPlan([(x, 0, buf[1025:1025 + 6 * 16].view(6, 16))]).aligned     # 2-byte offset
    assert not GroupedGemmPlan([(x, 0, buf[1024:1024 + 6 * 12].view(6, 12))]).aligned     # 24-byte rows
    assert GroupedGemmPlan([(x, 0, y), (buf[4:4].view(0, 96), 1, buf[2049:2049].view(0, 16))]).aligned  # empty: ignored


def test_outputs_must_be_disjoint_from_each_other_and_the_inputs():
    buf = torch.empty(64 * 64, dtype=torch.bfloat16)
    a, b = buf[:8 * 64].view(8, 64), buf[8 * 64:16 * 64].view(8, 64)
    GroupedGemmPlan([(a, 0, b), (a, 1, buf[16 * 64:24 * 64].view(8, 64))])              # repeated input: fine
    with pytest.raises(ValueError, match="output slices overlap"):
        GroupedGemmPlan([(a, 0, buf[16 * 64:24 * 64].view(8, 64)), (a, 1, buf[20 * 64:28 * 64].view(8, 64))])
    with pytest.raises(ValueError, match="overlap an input"):
        GroupedGemmPlan([(a, 0, buf[4 * 64:12 * 64].view(8, 64))])
    with pytest.raises(ValueError, match="overlap an input"):
        GroupedGemmPlan([(a, 0, buf[30 * 64:38 * 64].view(8, 64)), (b, 1, a)])


def test_pair_shapes_dtypes_strides_and_widths_are_checked():
    x = torch.empty(5, 96, dtype=torch.bfloat16)
    y = torch.empty(5, 24, dtype=torch.bfloat16)
    bad = ([(x, 0, y[:4])],                                                 # row counts differ
           [(x.half(), 0, y)],                                              # not bf16
           [(x, 0, y.t().contiguous().t())],                                # not contiguous
           [(x[:, :80], 0, y)],                                             # strided view
           [(torch.empty(5, 48, dtype=torch.bfloat16), 0, y)],              # K not a multiple of 32
           [(x, 0, y), (x, 1, torch.empty(5, 16, dtype=torch.bfloat16))],   # N differs between pairs
           [(x.view(5, 96, 1), 0, y)])                                      # not 2-D
    for pairs in bad:
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
    assert lib.na_mxfp4_gemv(None, 0, None, 0, None, 0, 0, None, 4, None, 0, None, 5760, 2880, 0, None, None) == -1
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
