"""MXFP4 expert path restated on the CPU in numpy (test infrastructure; see oracle/__init__.py).

Geometry (reference neural/moe/layout.py:143-157, tools/scale_pack.py:25-33): hidden H = 2880, gate_up rows GU = 5760
([gate | up], de-interleaved, reference neural/moe/gptoss_adapter.py:83-88), GK = 90 groups of 32 per row, 16 code
bytes per group, raw slot 13,219,200 B, PS4 slot 12,839,040 B.
"""
import numpy as np

from .bf16 import rb

H, GU, GK, RB = 2880, 5760, 90, 1440
OFF_DC = GU * RB
OFF_GS = OFF_DC + H * RB
OFF_DS = OFF_GS + GU * GK
SLOT_RAW = OFF_DS + H * GK
SR_P4 = 1 + GK // 2
SLOT_PACKED = OFF_GS + (GU + H) * SR_P4
assert SLOT_RAW == 13_219_200 and SLOT_PACKED == 12_839_040

ACT_ALPHA, ACT_LIMIT = 1.702, 7.0   # reference neural/moe/layout.py:143-146


# ----------------------------------------------------------------------------------------------------- dequant
def e2m1_value(code: int) -> float:
    """One E2M1 code -> value from the OCP MX bit fields (sign | 2-bit exponent, bias 1 | 1-bit mantissa).
    Restates reference neural/q80/mxfp4_kernels.py:62-69 (_e2m1) bit for bit; the 16-entry table of
    neural/moe/gptoss_adapter.py:55-56 is the independent second derivation the tests compare against."""
    s = -1.0 if code & 8 else 1.0
    e = (code >> 1) & 3
    m = code & 1
    mag = 0.5 * m if e == 0 else 2.0 ** (e - 1) * (1.0 + 0.5 * m)
    return s * mag


E2M1 = np.array([e2m1_value(c) for c in range(16)], dtype=np.float64)


def e8m0_value(s) -> np.ndarray:
    """E8M0 byte -> 2^(s-127), formed in fp32 as the reference GPU path does (mxfp4_kernels.py:118 tl.exp2(sc-127)):
    s = 255 -> +inf, s = 0 -> 2^-127 (an fp32 subnormal).  The reference's CPU kernels give +0.0 for s = 0
    (gptoss_cpu_portable.c:104 forms s << 23); the configs only use s in [119, 125] where both agree."""
    s = np.asarray(s, dtype=np.int32)
    with np.errstate(over="ignore"):
        return np.ldexp(np.float32(1.0), s - 127).astype(np.float32)


def dequant_rows(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """codes u8 [N, GK, 16] + raw scales u8 [N, GK] -> fp32 [N, GK*32] (reference gptoss_adapter.py:63-80:
    low nibble -> even element, high nibble -> odd element, value = E2M1[code] * 2^(s-127); exact in fp32)."""
    codes = np.asarray(codes, dtype=np.uint8)
    n, g, b = codes.shape
    out = np.empty((n, g, 2 * b), dtype=np.float32)
    out[..., 0::2] = E2M1[codes & 0x0F]
    out[..., 1::2] = E2M1[codes >> 4]
    out *= e8m0_value(scales)[..., None]
    return out.reshape(n, g * 2 * b)


# ------------------------------------------------------------------------------------------------- slot access
def slot_views(slot: np.ndarray, packed: bool):
    """(gate_codes [GU,GK,16], down_codes [H,GK,16], gate_scales raw [GU,GK], down_scales raw [H,GK]) of one slot.
    PS4 scale rows are decoded with ps4_unpack_rows (reference layout.py:168-186, scale_pack.py:6-12)."""
    slot = np.asarray(slot, dtype=np.uint8)
    gc = slot[:OFF_DC].reshape(GU, GK, 16)
    dc = slot[OFF_DC:OFF_GS].reshape(H, GK, 16)
    if packed:
        assert slot.size == SLOT_PACKED
        rows = ps4_unpack_rows(slot[OFF_GS:].reshape(GU + H, SR_P4))
    else:
        assert slot.size == SLOT_RAW
        rows = slot[OFF_GS:].reshape(GU + H, GK)
    return gc, dc, rows[:GU], rows[GU:]


def expert_weights(slot: np.ndarray, packed: bool = False):
    """Exact fp32 dequant of one expert: (W_gu [5760, 2880], W_dn [2880, 2880])."""
    gc, dc, gs, ds = slot_views(slot, packed)
    return dequant_rows(gc, gs), dequant_rows(dc, ds)


# ---------------------------------------------------------------------------------------------------- PS4 codec
class SpanError(ValueError):
    """A scale row whose max - min exceeds 15 cannot be stored as 4-bit deltas (reference scale_pack.py:36-40)."""

    def __init__(self, rows):
        self.rows = list(rows)
        super().__init__(f"{len(self.rows)} scale row(s) with span > 15: {self.rows[:8]}")


def ps4_pack_rows(sc: np.ndarray) -> np.ndarray:
    """raw scale rows u8 [n, 90] -> PS4 rows u8 [n, 46]: byte 0 = row minimum, byte 1+k = d[2k] | d[2k+1] << 4
    (reference tools/scale_pack.py:49-64).  Refuses rows with span > 15 (never clips).  Written row by row on
    purpose: an independent formulation of the product's vectorised codec."""
    sc = np.asarray(sc, dtype=np.uint8)
    n = sc.shape[0]
    out = np.zeros((n, SR_P4), dtype=np.uint8)
    bad = []
    for r in range(n):
        row = [int(v) for v in sc[r]]
        base = min(row)
        if max(row) - base > 15:
            bad.append(r)
            continue
        out[r, 0] = base
        for k in range(GK // 2):
            out[r, 1 + k] = (row[2 * k] - base) | ((row[2 * k + 1] - base) << 4)
    if bad:
        raise SpanError(bad)
    return out


def ps4_unpack_rows(rows: np.ndarray) -> np.ndarray:
    """PS4 rows u8 [n, 46] -> raw rows u8 [n, 90] (reference scale_pack.py:67-75): s[g] = base + nibble(g)."""
    rows = np.asarray(rows, dtype=np.uint8)
    base = rows[:, :1].astype(np.int32)
    d = rows[:, 1:].astype(np.int32)
    out = np.empty((rows.shape[0], GK), dtype=np.int32)
    out[:, 0::2] = base + (d & 15)
    out[:, 1::2] = base + (d >> 4)
    return (out & 0xFF).astype(np.uint8)


def ps4_pack_slot(raw: np.ndarray) -> np.ndarray:
    raw = np.asarray(raw, dtype=np.uint8)
    assert raw.shape == (SLOT_RAW,)
    out = np.empty(SLOT_PACKED, dtype=np.uint8)
    out[:OFF_GS] = raw[:OFF_GS]
    out[OFF_GS:] = ps4_pack_rows(raw[OFF_GS:].reshape(GU + H, GK)).ravel()
    return out


def ps4_unpack_slot(packed: np.ndarray) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.uint8)
    assert packed.shape == (SLOT_PACKED,)
    out = np.empty(SLOT_RAW, dtype=np.uint8)
    out[:OFF_GS] = packed[:OFF_GS]
    out[OFF_GS:] = ps4_unpack_rows(packed[OFF_GS:].reshape(GU + H, SR_P4)).ravel()
    return out


# ------------------------------------------------------------------------------------------------- products
def gemv_f64(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """out[t, n] = sum_k x[t, k] * w[n, k] in fp64 (the closed form of reference mxfp4_kernels.py:430-471)."""
    return np.asarray(x, np.float64) @ np.asarray(w, np.float64).T


def mxfp4_gemv(x, slots, which: str, packed=False, per_expert_x=False):
    """Reference mxfp4_gemv semantics (mxfp4_kernels.py:474-489): out [E, N] = bf16(fp32-accumulated x . w_e).
    ``slots`` is a list of slot byte arrays; ``which`` = "gate" or "down"; x [1, K] or [E, K] (per_expert_x)."""
    x = np.asarray(x, np.float32)
    outs = []
    for e, slot in enumerate(slots):
        wg, wd = expert_weights(slot, packed)
        w = wg if which == "gate" else wd
        xe = x[e:e + 1] if per_expert_x else x[:1]
        outs.append(rb(gemv_f64(xe, w).astype(np.float32))[0])
    return np.stack(outs)


def swiglu_clamp_bf16(gu: np.ndarray, alpha=ACT_ALPHA, limit=ACT_LIMIT) -> np.ndarray:
    """Clamped SwiGLU with torch's bf16 op-by-op rounding (reference neural/q80/expert_runtime.py:63-72; the in-place
    twin server.py:2014-2021): gate = min(g, limit); up = clamp(u, -limit, limit); t = bf16(gate * alpha);
    s = bf16(sigmoid(t)); glu = bf16(gate * s); h = bf16(bf16(up + 1) * glu).  gu: [..., 2I] bf16 values (fp32)."""
    gu = np.asarray(gu, np.float32)
    i = gu.shape[-1] // 2
    gate = np.minimum(gu[..., :i], np.float32(limit))
    up = np.clip(gu[..., i:], np.float32(-limit), np.float32(limit))
    t = rb(gate * np.float32(alpha))
    with np.errstate(over="ignore"):                  # exp(-t) = inf for t < -709 gives sigmoid 0, as it should
        s = rb((1.0 / (1.0 + np.exp(-t.astype(np.float64)))).astype(np.float32))
    glu = rb(gate * s)
    return rb(rb(up + np.float32(1.0)) * glu)


def expert_forward_bf16(x, slot, bias_gu, bias_dn, packed=False, weights=None):
    """One expert at the reference GPU path's rounding points (server.py:508-518 per expert, _pf_run_chunk
    server.py:2092-2181 per row): gu = bf16(x.Wgu) ; gu = bf16(gu + b_gu) ; h = act(gu) ; y = bf16(h.Wdn) ;
    y = bf16(y + b_dn).  x [T, 2880] bf16 values; biases bf16 values.  Returns y [T, 2880] (bf16 values, fp32)."""
    wg, wd = weights if weights is not None else expert_weights(slot, packed)
    x = np.atleast_2d(np.asarray(x, np.float32))
    gu = rb(gemv_f64(x, wg).astype(np.float32))
    gu = rb(gu + np.asarray(bias_gu, np.float32))
    h = swiglu_clamp_bf16(gu)
    y = rb(gemv_f64(h, wd).astype(np.float32))
    return rb(y + np.asarray(bias_dn, np.float32))


def combine_bf16(y_k: np.ndarray, w_k: np.ndarray) -> np.ndarray:
    """Weighted top-k combine of one token: bf16(sum_k fp32(bf16(y_k * w_k))) in top-k order (server.py:518 decode,
    server.py:2340-2341 prefill: bf16 products, fp32 sum, one rounding)."""
    y_k = np.asarray(y_k, np.float32)
    w_k = np.asarray(w_k, np.float32).reshape(-1, 1)
    prod = rb(y_k * w_k)
    acc = np.zeros(y_k.shape[1:], np.float32)
    for k in range(prod.shape[0]):
        acc = (acc + prod[k]).astype(np.float32)
    return rb(acc)


def moe_token_bf16(x, slots, ids, w, bias_gu, bias_dn, packed=False, cache=None):
    """MoE output of one token: combine over its top-k experts (ids index ``slots``; bias tables [E, .])."""
    ys = []
    for e in ids:
        wts = cache.get(e) if cache is not None else None
        if wts is None:
            wts = expert_weights(slots[e], packed)
            if cache is not None:
                cache[e] = wts
        ys.append(expert_forward_bf16(x, None, bias_gu[e], bias_dn[e], weights=wts)[0])
    return combine_bf16(np.stack(ys), w)


# ---------------------------------------------------------------- the reference C kernel's arithmetic (fp32)
def activation_f32(g, u, alpha=ACT_ALPHA, limit=ACT_LIMIT):
    """The CPU kernels' activation (reference gptoss_cpu_portable.c:197-201): fp32, expf, no intermediate rounding."""
    g = np.asarray(g, np.float32)
    u = np.asarray(u, np.float32)
    gt = np.minimum(g, np.float32(limit))
    up = np.minimum(np.maximum(u, np.float32(-limit)), np.float32(limit))
    with np.errstate(over="ignore"):          # expf(+large) = inf -> h = -0, as in C
        return ((up + np.float32(1.0)) * gt / (np.float32(1.0) + np.exp(np.float32(-alpha) * gt))).astype(np.float32)


def experts_cpu_f64(x, slots, bgu, bdn, w, packed=False):
    """gptoss_experts (reference gptoss_cpu_portable.c:214-294) in fp64 products with fp32 activation: out[n] =
    sum_e w[e] * (h_e . Wdn_e[n] + bdn_e[n]),  h_e = act(x . Wgu_e + bgu_e).  Agrees with the C kernel to ~1e-5."""
    x = np.asarray(x, np.float32).reshape(1, H)
    out = np.zeros(H, np.float64)
    for e, slot in enumerate(slots):
        wg, wd = expert_weights(slot, packed)
        gu = (gemv_f64(x, wg)[0] + np.asarray(bgu[e], np.float64)).astype(np.float32)
        h = activation_f32(gu[:H], gu[H:])
        y = gemv_f64(h.reshape(1, H), wd)[0] + np.asarray(bdn[e], np.float64)
        out += float(w[e]) * y
    return out


# ------------------------------------------------------------------------------------------------------ router
def router_top4(logits, k=4):
    """top-k by repeated argmax (first index wins ties), softmax over the k values relative to the max, weights
    rounded to bf16 (reference fused_core.py:460-486 k_topk/_emit: e_i = exp(v_i - v_0), sc = bf16(e_i / sum))."""
    v = np.asarray(logits, np.float32).copy()
    ids, vals = [], []
    for _ in range(k):
        i = int(np.argmax(v))          # numpy argmax returns the first maximal index
        ids.append(i)
        vals.append(v[i])
        v[i] = -np.inf
    vals = np.asarray(vals, np.float32)
    e = np.exp((vals - vals[0]).astype(np.float32)).astype(np.float32)
    ssum = np.float32(0.0)
    for t in e:
        ssum = np.float32(ssum + t)
    return np.asarray(ids, np.int64), rb(e / ssum)


def router_logits_bf16(xn, w_router, b_router):
    """Router GEMV with one bf16 rounding (reference fused_core.py:431-441): logits = bf16(xn . Wr^T + br)."""
    return rb((gemv_f64(np.atleast_2d(xn), w_router) + np.asarray(b_router, np.float64)).astype(np.float32))
