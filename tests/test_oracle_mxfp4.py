"""CPU: pin the MXFP4 oracle (dequant, PS4 codec, expert forward, combine, router) against the reference's own
artefacts: its 16-entry E2M1 table (gptoss_adapter.py:55-56), the known-answer scale rows of
tools/scale_pack.py:114-133, and its C expert kernels compiled from source (oracle/_ref)."""
import os

import numpy as np
import pytest

from oracle import mxfp4_oracle as mo
from oracle.bf16 import rb
from neural_amd import scale_pack as sp
from neural_amd import synth

# transformers' FP4_VALUES as restated by the reference (gptoss_adapter.py:55-56), typed in as the known answer
FP4_VALUES = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def test_e2m1_bit_formula_matches_reference_table():
    got = mo.E2M1
    assert np.array_equal(got, np.array(FP4_VALUES))
    assert np.array_equal(np.signbit(got), np.signbit(np.array(FP4_VALUES)))      # code 8 is -0.0


def test_e8m0_scale_values():
    assert mo.e8m0_value(127) == 1.0 and mo.e8m0_value(128) == 2.0 and mo.e8m0_value(119) == 2.0 ** -8
    assert np.isinf(mo.e8m0_value(255))
    assert mo.e8m0_value(0) == np.float32(2.0 ** -127)


def test_dequant_layout_low_nibble_even():
    codes = np.zeros((1, 1, 16), np.uint8)
    codes[0, 0, 0] = 0x72          # element 0 <- low nibble 2 (1.0), element 1 <- high nibble 7 (6.0)
    codes[0, 0, 15] = 0x9F        # element 30 <- 0xF (-6.0), element 31 <- 0x9 (-0.5)
    w = mo.dequant_rows(codes, np.array([[128]], np.uint8))
    assert w.shape == (1, 32)
    assert (w[0, 0], w[0, 1], w[0, 30], w[0, 31]) == (2.0, 12.0, -12.0, -1.0)
    assert np.count_nonzero(w) == 4


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 100,
                        np.array([0.0, -0.0, 1.0, 65504.0, 3.3895314e38, 1e-40, -1e-40, np.inf, -np.inf], np.float32),
                        (np.arange(1 << 16, dtype=np.uint32) << 16 | 0x8000).view(np.float32)[:-1]])  # exact ties
    x = x[np.isfinite(x) | np.isinf(x)]
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = rb(x)
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all()


# ----------------------------------------------------------------------------------------------- PS4 codec
def _edge_slot(rng):
    """The known-answer edge rows of reference tools/scale_pack.py:122-125 on a synthetic slot."""
    raw = synth.slot_raw(rng, 105, 120)
    sc = raw[sp.SCALES_AT:].reshape(sp.SCALE_ROWS, sp.GROUPS)
    sc[0, :] = 0
    sc[1, :] = 255
    sc[2, :] = 240
    sc[2, 17] = 255
    sc[3, :] = 7
    sc[3, ::2] = 22
    sc[4, 89] = 200
    sc[4, :89] = 185
    return raw


def test_ps4_known_answer_rows_round_trip():
    rng = np.random.default_rng(1)
    raw = _edge_slot(rng)
    for packer in (sp.pack_slot, mo.ps4_pack_slot):
        p = packer(raw)
        assert p.shape == (sp.PS4_SLOT_BYTES,)
        assert np.array_equal(p[:sp.SCALES_AT], raw[:sp.SCALES_AT])
        assert np.array_equal(sp.unpack_slot(p), raw) and np.array_equal(mo.ps4_unpack_slot(p), raw)
    rows = sp.pack_slot(raw)[sp.SCALES_AT:].reshape(sp.SCALE_ROWS, sp.PS4_ROW_BYTES)
    assert rows[0, 0] == 0 and not rows[0, 1:].any()                     # constant row: base, zero deltas
    assert rows[1, 0] == 255 and not rows[1, 1:].any()
    assert rows[2, 0] == 240 and rows[2, 1 + 17 // 2] >> 4 == 15         # group 17 (odd) in the high nibble
    assert rows[3, 0] == 7 and (rows[3, 1:] == 15).all()                 # even groups 22 = 7 + 15, odd 7
    assert rows[4, 0] == 185 and rows[4, 1 + 44] == 15 << 4             # group 89 = base + 15 (high nibble)


def test_ps4_span16_refused_never_clipped():
    rng = np.random.default_rng(2)
    raw = _edge_slot(rng)
    sc = raw[sp.SCALES_AT:].reshape(sp.SCALE_ROWS, sp.GROUPS)
    sc[5, :] = 100
    sc[5, 44] = 116
    with pytest.raises(sp.SpanError) as ei:
        sp.pack_slot(raw)
    assert 5 in ei.value.rows.tolist()
    with pytest.raises(mo.SpanError):
        mo.ps4_pack_slot(raw)


def test_ps4_product_codec_equals_oracle_codec():
    rng = np.random.default_rng(7)
    sc = rng.integers(110, 126, size=(500, sp.GROUPS)).astype(np.uint8)
    assert np.array_equal(sp.pack_scale_rows(sc), mo.ps4_pack_rows(sc))
    assert np.array_equal(sp.unpack_scale_rows(sp.pack_scale_rows(sc)), sc)


# ------------------------------------------------------------------------------ reference C kernels (oracle/_ref)
def _ref(name="portable"):
    from oracle.refkernels import RefExperts
    try:
        return RefExperts(name)
    except (FileNotFoundError, RuntimeError) as e:
        pytest.skip(str(e))


@pytest.fixture(scope="module")
def experts4():
    rng = np.random.default_rng(20261201)
    slots = [synth.slot_raw(rng) for _ in range(4)]
    x = rb(rng.standard_normal(2880).astype(np.float32))
    bgu = [rb(rng.standard_normal(5760).astype(np.float32) * 0.02) for _ in range(4)]
    bdn = [rb(rng.standard_normal(2880).astype(np.float32) * 0.02) for _ in range(4)]
    w = rb(np.array([0.41, 0.29, 0.18, 0.12], np.float32))
    return slots, x, bgu, bdn, w


def test_reference_c_kernel_reads_our_ps4_slots_bit_identically(experts4):
    slots, x, bgu, bdn, w = experts4
    ref = _ref()
    raw = ref.experts(slots, x, bgu, bdn, w, threads=4)
    packed = ref.experts([sp.pack_slot(s) for s in slots], x, bgu, bdn, w, threads=4, packed=True)
    assert np.array_equal(raw, packed)
    # negative control: one flipped delta nibble must change the output
    bad = sp.pack_slot(slots[0])
    bad[sp.SCALES_AT + 46 * 3000 + 20] ^= 0x01
    moved = ref.experts([bad] + [sp.pack_slot(s) for s in slots[1:]], x, bgu, bdn, w, threads=4, packed=True)
    assert not np.array_equal(moved, raw)


def test_oracle_fp32_forward_matches_reference_c_kernel(experts4):
    slots, x, bgu, bdn, w = experts4
    ref = _ref().experts(slots, x, bgu, bdn, w, threads=4)
    ora = mo.experts_cpu_f64(x, slots, bgu, bdn, w)
    scale = np.abs(ref).max()
    assert np.abs(ref - ora).max() <= 2e-5 * scale + 1e-4
    # a dropped term (one expert missing) must fail the same check
    ora3 = mo.experts_cpu_f64(x, slots[:3], bgu[:3], bdn[:3], w[:3])
    assert np.abs(ref - ora3).max() > 100 * (2e-5 * scale + 1e-4)


def test_oracle_bf16_path_within_tolerance_of_reference_c_kernel(experts4):
    """The GPU reference's bf16 rounding points vs the CPU kernel's fp32 arithmetic: same mathematics, so they agree
    to a few bf16 ulps of the output scale; a transposed operand or a wrong gate/up split would not."""
    slots, x, bgu, bdn, w = experts4
    ref = _ref().experts(slots, x, bgu, bdn, w, threads=4)
    ys = np.stack([mo.expert_forward_bf16(x[None], s, bg, bd)[0] for s, bg, bd in zip(slots, bgu, bdn)])
    got = mo.combine_bf16(ys, w)
    scale = np.abs(ref).max()
    err = np.abs(got - ref)
    assert err.max() <= 2e-2 * scale, (err.max(), scale)
    assert np.median(err) <= 2e-3 * scale


def test_avx512_build_agrees_with_portable_build(experts4):
    slots, x, bgu, bdn, w = experts4
    a = _ref("portable").experts(slots, x, bgu, bdn, w, threads=4)
    b = _ref("multi").experts(slots, x, bgu, bdn, w, threads=4)
    assert np.abs(a - b).max() <= 2e-5 * np.abs(a).max()


def test_golden_vectors_from_reference_kernel():
    """tests/golden/experts_ref.npz: outputs of the reference C kernel on seeded slots (tests/golden/make_golden.py)."""
    path = os.path.join(os.path.dirname(__file__), "golden", "experts_ref.npz")
    g = np.load(path)
    rng = np.random.default_rng(int(g["seed"]))
    slots = [synth.slot_raw(rng) for _ in range(int(g["n_experts"]))]
    import hashlib
    h = hashlib.sha256(b"".join(s.tobytes() for s in slots)).hexdigest()
    assert h == str(g["slots_sha256"]), "the synthetic slot generator changed: regenerate the golden vectors"
    ora = mo.experts_cpu_f64(g["x"], slots, g["bgu"], g["bdn"], g["w"])
    ref = g["out"]
    assert np.abs(ora - ref).max() <= 2e-5 * np.abs(ref).max() + 1e-4


# ----------------------------------------------------------------------------------------------------- router
def test_router_top4_ties_and_softmax():
    v = np.zeros(128, np.float32)
    ids, w = mo.router_top4(v)
    assert ids.tolist() == [0, 1, 2, 3] and np.all(w == np.float32(0.25))
    v[[5, 77, 9, 100]] = [3.0, 3.0, 2.0, 2.0]
    ids, w = mo.router_top4(v)
    assert ids.tolist() == [5, 77, 9, 100]
    e = np.exp(np.array([0, 0, -1, -1], np.float64))
    assert np.allclose(w, e / e.sum(), rtol=4e-3)
    assert abs(float(w.astype(np.float64).sum()) - 1.0) < 1e-2


def test_combine_order_and_rounding():
    y = np.array([[1.0, 3.0], [2.0, 5.0], [0.5, 7.0], [0.25, 1.0]], np.float32)
    w = np.array([0.5, 0.25, 2.0, 4.0], np.float32)
    assert np.array_equal(mo.combine_bf16(y, w), np.array([0.5 + 0.5 + 1.0 + 1.0, 1.5 + 1.25 + 14.0 + 4.0],
                                                          np.float32))


def test_swiglu_clamp_special_values():
    gu = np.array([[100.0, -100.0, 0.0, 7.0, 100.0, -100.0, 3.0, -9.0]], np.float32)   # gate | up
    h = mo.swiglu_clamp_bf16(gu)
    gate = np.array([7.0, -100.0, 0.0, 7.0])
    up = np.array([7.0, -7.0, 3.0, -7.0])
    want = (up + 1) * gate / (1 + np.exp(-1.702 * gate))
    assert np.allclose(h[0], want, rtol=1e-2, atol=1e-6)
    assert h[0, 2] == 0.0
