"""CPU: slot geometry and pool views against the byte format (neural_amd/moe/layout.py; the reference's
neural/moe/layout.py:17-212 and tools/scale_pack.py:6-12 define it), ragged tile plans (the contract of the
reference's mxfp4_kernels.py:298-382), and the C-ABI library: it loads and exports every
symbol include/neural_amd.h declares (no compute call: there is no GPU here)."""
import ctypes
import dataclasses
import os
import re

import numpy as np
import pytest
import torch

from neural_amd import scale_pack as sp
from neural_amd import synth
from neural_amd.moe.layout import (GPTOSS_LAYOUT, GPTOSS_LAYOUT_PS4, GPTOSS_LAYOUT_T950, MXFP4_REPRS, TILE_REPR,
                                   ExpertLayout, gptoss_layout_for_repr, mxfp4_pool_views, prepacked_descriptor)
from neural_amd.q80.mxfp4_kernels import GroupedGemmPlan, _grouped_tile_rows, _scale_layout

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

RAW_STORE_DESCRIPTOR = {"slot_bytes": 13219200, "n_layers": 36, "n_experts": 128, "hidden": 2880, "gate_up_n": 5760,
                        "down_n": 2880, "down_k": 2880, "int4_group": 32, "inner_k_tiles": 2,
                        "kernel": "neural.q80.mxfp4_kernels (Triton, fp32-accum)", "weight_repr": "mxfp4_g32"}


# Slot byte counts derived by hand from the format: a row of K = 2880 inputs has 90 groups of 32 E2M1 codes
# (16 bytes each, 1,440 bytes per row), and either 90 E8M0 bytes (raw) or 1 base byte + 45 delta bytes (PS4).
GATE_CODES = 5760 * 90 * 16            # 8,294,400
DOWN_CODES = 2880 * 90 * 16            # 4,147,200
RAW_SCALES = (5760 + 2880) * 90        # 777,600
PS4_SCALES = (5760 + 2880) * (1 + 45)  # 397,440
T950_SLOT = (5760 + 2880) // 16 * (22 * 1024 + 512 + 16 * 96)   # 540 blocks of 16 rows x 24,576 B


def test_slot_bytes_derived_from_the_format():
    assert GPTOSS_LAYOUT.slot_bytes == GATE_CODES + DOWN_CODES + RAW_SCALES == 13_219_200
    assert GPTOSS_LAYOUT_PS4.slot_bytes == GATE_CODES + DOWN_CODES + PS4_SCALES == 12_839_040
    assert GPTOSS_LAYOUT_T950.slot_bytes == T950_SLOT == 13_271_040
    assert (sp.RAW_SLOT_BYTES, sp.PS4_SLOT_BYTES) == (13_219_200, 12_839_040)
    for L, scale_row in ((GPTOSS_LAYOUT, 90), (GPTOSS_LAYOUT_PS4, 46)):
        assert (L.off_down_codes, L.off_gate_scales) == (GATE_CODES, GATE_CODES + DOWN_CODES)
        assert L.off_down_scales == GATE_CODES + DOWN_CODES + 5760 * scale_row
        assert L.off_down_scales + L.down_saz_bytes == L.slot_bytes
        assert (L.gate_groups, L.down_groups) == (90, 90)
    assert GPTOSS_LAYOUT_PS4.scale_layout_mode == 1 and GPTOSS_LAYOUT.scale_layout_mode == 0
    assert not GPTOSS_LAYOUT_T950.is_mxfp4            # not a store representation the views or the CPU kernels read


def test_layout_rules_on_small_geometries():
    # hidden 64 (2 groups), intermediate 96 (3 groups): raw is fine, PS4 needs an even group count per row
    small = ExpertLayout("s", 1, 4, 2, hidden=64, gate_up_n=192, down_n=64, down_k=96)
    assert small.slot_bytes == 192 * 2 * 16 + 64 * 3 * 16 + 192 * 2 + 64 * 3 == 9_792
    with pytest.raises(AssertionError):
        ExpertLayout("s", 1, 4, 2, hidden=64, gate_up_n=192, down_n=64, down_k=96, weight_repr="mxfp4_g32_ps4")
    even = ExpertLayout("e", 1, 4, 2, hidden=128, gate_up_n=128, down_n=128, down_k=64, weight_repr="mxfp4_g32_ps4")
    assert even.slot_bytes == 128 * 4 * 16 + 128 * 2 * 16 + 128 * 3 + 128 * 2 == 12_928
    with pytest.raises(AssertionError):               # gate_up must stack gate | up over the intermediate
        ExpertLayout("g", 1, 4, 2, hidden=64, gate_up_n=100, down_n=64, down_k=64)
    with pytest.raises(ValueError):                   # the int4 / int8 representations are outside this path
        ExpertLayout("q", 1, 4, 2, hidden=64, gate_up_n=128, down_n=64, down_k=64, weight_repr="int8_g32")
    for bad in ("int4_g32", TILE_REPR, ""):            # only the two store representations have a gpt-oss layout
        with pytest.raises(KeyError):
            gptoss_layout_for_repr(bad)
    assert [gptoss_layout_for_repr(r).weight_repr for r in MXFP4_REPRS] == list(MXFP4_REPRS)


def test_descriptors():
    raw = prepacked_descriptor(GPTOSS_LAYOUT)
    assert raw["row"] == "gate_codes|down_codes|gate_scales|down_scales"
    assert {k: v for k, v in raw.items() if k != "row"} == RAW_STORE_DESCRIPTOR
    ps4, t950 = prepacked_descriptor(GPTOSS_LAYOUT_PS4), prepacked_descriptor(GPTOSS_LAYOUT_T950)
    assert set(raw) == set(ps4) == set(t950)
    for d, L in ((ps4, GPTOSS_LAYOUT_PS4), (t950, GPTOSS_LAYOUT_T950)):
        assert d["slot_bytes"] == L.slot_bytes and d["weight_repr"] == L.weight_repr
        assert {k for k in raw if raw[k] != d[k]} == {"slot_bytes", "weight_repr", "kernel", "row"}
    fewer = dataclasses.replace(GPTOSS_LAYOUT, n_experts=64)
    assert {k for k, v in prepacked_descriptor(fewer).items() if raw[k] != v} == {"n_experts"}


def test_pool_views_cover_each_slot_byte_once():
    """Each view's offset, shape and strides, from the byte order gate codes | down codes | gate scales | down
    scales, and the four views together tile the slot without a gap or an overlap."""
    for L, w in ((GPTOSS_LAYOUT, 90), (GPTOSS_LAYOUT_PS4, 46)):
        pool = torch.empty(3, L.slot_bytes, dtype=torch.uint8)
        views = mxfp4_pool_views(pool, L)
        want = [(0, (3, 5760, 90, 16), (L.slot_bytes, 1440, 16, 1)),
                (GATE_CODES, (3, 2880, 90, 16), (L.slot_bytes, 1440, 16, 1)),
                (GATE_CODES + DOWN_CODES, (3, 5760, w), (L.slot_bytes, w, 1)),
                (GATE_CODES + DOWN_CODES + 5760 * w, (3, 2880, w), (L.slot_bytes, w, 1))]
        spans = []
        for v, (off, shape, stride) in zip(views, want):
            assert (v.storage_offset(), tuple(v.shape), v.stride()) == (off, shape, stride)
            assert v.untyped_storage().data_ptr() == pool.untyped_storage().data_ptr()
            spans.append((off, off + int(np.prod(shape[1:]))))
        assert [a for a, _ in spans[1:]] == [b for _, b in spans[:-1]] and spans[-1][1] == L.slot_bytes
    with pytest.raises(AssertionError):                # a pool whose rows are not the layout's slot size
        mxfp4_pool_views(torch.empty(2, GPTOSS_LAYOUT.slot_bytes, dtype=torch.uint8), GPTOSS_LAYOUT_PS4)
    with pytest.raises(AssertionError):                # the tile layout has no store views
        mxfp4_pool_views(torch.empty(1, T950_SLOT, dtype=torch.uint8), GPTOSS_LAYOUT_T950)


def test_pool_views_read_the_bytes_the_format_names():
    """Individual codes and scales read through the views are the bytes at their hand-computed slot offsets; a PS4
    row's base is its smallest exponent."""
    rng = np.random.default_rng(2027)
    raw = synth.slot_raw(rng)
    pool = torch.from_numpy(np.stack([np.zeros_like(raw), raw]))
    gb, db, gs, ds = mxfp4_pool_views(pool, GPTOSS_LAYOUT)
    for n, g, b in ((0, 0, 0), (5759, 89, 15), (2880, 44, 7), (17, 3, 9)):
        assert int(gb[1, n, g, b]) == raw[n * 1440 + g * 16 + b]
        assert int(gs[1, n, g]) == raw[GATE_CODES + DOWN_CODES + n * 90 + g]
    for n, g, b in ((0, 0, 0), (2879, 89, 15), (1234, 60, 1)):
        assert int(db[1, n, g, b]) == raw[GATE_CODES + n * 1440 + g * 16 + b]
        assert int(ds[1, n, g]) == raw[GATE_CODES + DOWN_CODES + 5760 * 90 + n * 90 + g]
    ps4 = torch.from_numpy(sp.pack_slot(raw)[None])
    _, _, gs2, ds2 = mxfp4_pool_views(ps4, GPTOSS_LAYOUT_PS4)
    for n in (0, 777, 5759):
        row = gs[1, n].numpy().astype(int)
        base = int(gs2[0, n, 0])
        assert base == row.min()
        deltas = [(int(gs2[0, n, 1 + j // 2]) >> (4 * (j % 2))) & 15 for j in range(90)]
        assert [base + d for d in deltas] == row.tolist()
    assert int(ds2[0, 2879, 0]) == int(ds[1, 2879].min())


def test_scale_layout_reads_the_row_width():
    GK = 4                                              # raw rows 4 bytes wide, PS4 rows 1 + 2
    raw2d, ps42d = torch.zeros(7, 4, dtype=torch.uint8), torch.zeros(7, 3, dtype=torch.uint8)
    assert _scale_layout(raw2d, GK, None) is False and _scale_layout(ps42d, GK, None) is True
    assert _scale_layout(raw2d, GK, 0) is False and _scale_layout(ps42d, GK, 1) is True
    with pytest.raises(ValueError, match="says raw"):
        _scale_layout(raw2d, GK, True)
    with pytest.raises(ValueError, match="says packed"):
        _scale_layout(ps42d, GK, False)
    with pytest.raises(ValueError, match="row width 5"):
        _scale_layout(torch.zeros(7, 5, dtype=torch.uint8), GK, None)
    with pytest.raises(ValueError, match="contiguous"):  # rows of 3 inside a pitch of 8
        _scale_layout(torch.zeros(7, 8, dtype=torch.uint8)[:, :3], GK, None)
    with pytest.raises(ValueError, match="contiguous"):  # a transposed view: unit stride across rows
        _scale_layout(torch.zeros(3, 7, dtype=torch.uint8).t(), GK, None)
    # the GPT-OSS pool views: 90 raw, 46 PS4, whatever the slot stride between experts
    for L, want in ((GPTOSS_LAYOUT, False), (GPTOSS_LAYOUT_PS4, True)):
        _, _, gs, ds = mxfp4_pool_views(torch.empty(2, L.slot_bytes, dtype=torch.uint8), L)
        assert _scale_layout(gs, 90, None) is want and _scale_layout(ds, 90, want) is want


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
    # the fused attention block: every argument valid except a sync buffer that is not 16-byte aligned (its handoff
    # words are 64-bit atomics), and a misaligned q; neither call reaches a launch
    a, f = 1 << 20, ctypes.c_float
    blk = lambda q, sync: lib.na_core_attn_block(a, None, None, a, a, a, a, a, a, a, a, 4352, 0, q, f(1e-5), f(1.0),  # noqa: E731
                                                 a, f(0.125), 0, 32, a, a, a, a, a, a, a, a, a, a, a, sync, None, None)
    assert blk(a, a + 8) == -1 and blk(a, a + 4) == -1 and blk(a + 2, a) == -1


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


def test_auto_split_is_the_fewest_chunks_of_one_pass():
    """attention.auto_split(smax): under the chunk rule (64-key blocks, ceil(blocks / ns) blocks per chunk) every
    chunk of a full cache stays within one 256-key pass, and one chunk fewer would give some chunk a second pass
    (up to the 64-chunk limit).  Brute force over the cache sizes."""
    from neural_amd import attention as A
    for smax in list(range(1, 3000, 7)) + [4096, 4354, 4360, 8192, 16384, 16385, 40000]:
        ns, blocks = A.auto_split(smax), -(-smax // 64)
        keys = [min(64 * -(-blocks // k), 64 * blocks) for k in range(1, 65)]   # largest chunk at k chunks
        assert 1 <= ns <= 64 and (keys[ns - 1] <= 256 or ns == 64), smax
        assert ns == 1 or keys[ns - 2] > 256, smax
    assert (A.auto_split(4354), A.auto_split(1024), A.auto_split(256), A.auto_split(257)) == (18, 4, 1, 2)


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
