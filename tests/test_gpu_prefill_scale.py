"""The fused prefill layer's routing and products at the sizes of configurations 2 and 4 (reference moe_prefill_layer
server.py:2222-2345: stable argsort of the flattened top-k ids, bincount, gather; tile rows mxfp4_kernels.py:298-315).

na_moe_prefill is called through the C ABI with a caller-owned workspace, and its routing tables are read back from
the offsets na_moe_prefill_workspace_layout reports:
- counts == np.bincount of the valid ids; order == np.argsort(ids, kind="stable") over the valid pairs (bit-exact,
  index work); ntiles and the tile table == ceil(count / 64) tiles per expert in expert order, each (expert, first
  sorted position, rows), derived here from the counts;
- at T = 600, 2048 (Zipf(1.1), 8,192 pairs: every wave of the order kernel's first round), 2,100 and 4,096 (16,384
  pairs: the second round), with a few invalid ids (-1, 128) that must join no expert's list;
- sampled tokens against the oracle's expert forward and top-k combine (moe_rows), chosen so their pairs fall in
  every wave of both rounds (pair indices past 2,048 and past 8,192);
- raw, PS4 and t950 pools give bit-identical outputs at T = 2048.
The pool holds 8 distinct slots that a slot table maps onto the 128 experts (routing still spans 128 experts; the
oracle's dequantised weights stay in memory), biases N(0, 0.02) per expert.
"""
import ctypes

import numpy as np
import pytest

from oracle import mxfp4_oracle as mo
from oracle.model_oracle import DecodeOracle

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

H, NE, N_SLOTS = 2880, 128, 8


@pytest.fixture(scope="module")
def pools():
    import torch
    from neural_amd import synth, tiles
    from neural_amd.moe.layout import GPTOSS_LAYOUT, GPTOSS_LAYOUT_PS4, GPTOSS_LAYOUT_T950

    dev = torch.device("cuda", 0)
    print("case prefill scale fixture: 8 distinct slots in raw, PS4 and t950 pools", flush=True)
    rng = np.random.default_rng(2222)
    slots = [synth.slot_raw(rng) for _ in range(N_SLOTS)]
    raw = torch.from_numpy(np.stack(slots)).to(dev)
    ps4 = torch.from_numpy(np.stack([mo.ps4_pack_slot(s) for s in slots])).to(dev)
    t950 = torch.empty(N_SLOTS, GPTOSS_LAYOUT_T950.slot_bytes, dtype=torch.uint8, device=dev)
    tiles.repack_to_t950(raw, t950)
    n = 36 * NE
    tab = np.arange(n, dtype=np.int64) % N_SLOTS
    g = torch.Generator().manual_seed(23)
    bgu = (torch.randn(n, 5760, generator=g) * 0.02).to(torch.bfloat16)
    bdn = (torch.randn(n, 2880, generator=g) * 0.02).to(torch.bfloat16)
    f = lambda t: t.float().numpy()  # noqa: E731
    bgu_np, bdn_np = f(bgu), f(bdn)
    orc = DecodeOracle(np.zeros((1, H), np.float32), [], np.ones(H, np.float32), np.zeros((1, H), np.float32),
                       lambda li, e: (slots[tab[e]], bgu_np[e], bdn_np[e]), np.zeros(32, np.float32), 1.0, smax=1)
    return dict(dev=dev, slots=slots, layouts={
        "raw": (raw, GPTOSS_LAYOUT.slot_bytes, 0), "ps4": (ps4, GPTOSS_LAYOUT_PS4.slot_bytes, 1),
        "t950": (t950, GPTOSS_LAYOUT_T950.slot_bytes, 2)}, tab=torch.from_numpy(tab).to(dev), bgu=bgu.to(dev),
        bdn=bdn.to(dev), orc=orc)


def _routing(T, seed):
    from neural_amd import synth
    rng = np.random.default_rng(seed)
    ids, w = synth.zipf_routing(rng, T)
    bad = rng.choice(4 * T, size=max(4, T // 300), replace=False)
    flat = ids.reshape(-1)
    flat[bad[::2]] = -1
    flat[bad[1::2]] = NE
    return ids, w, rng


def _run(pools, layout, x, ids, w):
    """One na_moe_prefill call with a caller-owned workspace; returns (out, workspace, offsets)."""
    import torch
    from neural_amd import _native as N
    dev = pools["dev"]
    pool, slot_bytes, code = pools["layouts"][layout]
    T = x.shape[0]
    nbytes = N.lib().na_moe_prefill_workspace_bytes(T)
    offs = (ctypes.c_longlong * 9)()
    assert N.lib().na_moe_prefill_workspace_layout(T, offs) == 0
    assert offs[7] == nbytes
    ws = torch.full((nbytes,), 0xA5, dtype=torch.uint8, device=dev)       # stale bytes everywhere
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    N.call("na_moe_prefill", x.data_ptr(), ids.data_ptr(), w.data_ptr(), T, pool.data_ptr(), slot_bytes, code,
           pools["tab"].data_ptr(), 0, pools["bgu"].data_ptr(), pools["bdn"].data_ptr(), ws.data_ptr(), nbytes,
           out.data_ptr(), 1.702, 7.0, None, N.stream(dev))
    torch.cuda.synchronize()
    return out, ws, list(offs)


def _tables(ws, offs, P):
    w = ws.cpu().numpy()
    i32 = lambda o, n: w[o:o + 4 * n].view(np.int32)  # noqa: E731
    counts = i32(offs[0], NE).copy()
    ntiles = int(i32(offs[1], 1)[0])
    order = i32(offs[2], P).copy()
    tiles = i32(offs[3], 4 * ntiles).reshape(ntiles, 4).copy()
    return counts, ntiles, order, tiles


@pytest.mark.parametrize("T", [600, 2048, 2100, 4096])
def test_prefill_routing_tables_bit_exact(pools, T):
    import torch
    from neural_amd import synth
    dev = pools["dev"]
    print(f"case prefill routing tables T={T} ({4 * T} pairs)", flush=True)
    ids, w, rng = _routing(T, 7000 + T)
    x = synth.bf16_normal(rng, (T, H)).to(dev)
    ids_d = torch.from_numpy(ids).to(dev)
    w_d = torch.from_numpy(w).to(torch.bfloat16).to(dev)
    out, ws, offs = _run(pools, "t950", x, ids_d, w_d)
    P = 4 * T
    counts, ntiles, order, tiles = _tables(ws, offs, P)
    flat = ids.reshape(-1)
    valid = (flat >= 0) & (flat < NE)
    want_counts = np.bincount(flat[valid], minlength=NE)
    assert np.array_equal(counts, want_counts)
    nv = int(valid.sum())
    want_order = np.argsort(np.where(valid, flat, NE), kind="stable")[:nv]
    assert np.array_equal(order[:nv], want_order)
    rows = []                                           # expected tile table, written out from the counts
    start = 0
    for e in range(NE):
        c = int(want_counts[e])
        for m0 in range(0, c, 64):
            rows.append((e, start + m0, min(64, c - m0), 0))
        start += c
    assert ntiles == len(rows) == int(sum((c + 63) // 64 for c in want_counts))
    assert ntiles <= offs[8]
    assert np.array_equal(tiles, np.array(rows, np.int32).reshape(-1, 4))
    # sampled tokens in every wave of both order rounds (pair p = 4 t + k: waves of 2,048 pairs, rounds of 8,192)
    bands = [(0, 512), (512, 1024), (1024, 1536), (1536, 2048), (2048, 3072), (3072, 4096)]
    pick = []
    for lo, hi in bands:
        if lo < T:
            pick += list(rng.choice(np.arange(lo, min(hi, T)), size=min(12, min(hi, T) - lo), replace=False))
    pick = np.array(sorted(set(pick + [T - 1])))
    if T >= 2048:
        assert len(pick) >= 48 and (4 * pick > 2048).sum() >= 36
    if T > 2048:
        assert (4 * pick >= 8192).sum() >= 12
    hn = x.float().cpu().numpy()[pick]
    gw = w_d.float().cpu().numpy()[pick]
    want = pools["orc"].moe_rows(0, hn, ids[pick], gw)
    got = out.float().cpu().numpy()[pick]
    d = np.abs(got - want)
    scale = np.abs(want).max()
    assert d.max() <= 2e-2 + 1e-2 * scale and d.mean() <= 1e-3 * scale, (d.max(), d.mean(), scale)
    # a token whose four ids are all invalid gets +0
    allbad = np.all(~valid.reshape(T, 4), axis=1)
    if allbad.any():
        assert not bool(out[torch.from_numpy(np.nonzero(allbad)[0]).to(dev)].float().abs().sum())


def test_prefill_raw_ps4_t950_bitwise_at_2048(pools):
    import torch
    from neural_amd import synth
    dev = pools["dev"]
    print("case prefill raw == ps4 == t950 T=2048", flush=True)
    T = 2048
    ids, w, rng = _routing(T, 99)
    x = synth.bf16_normal(rng, (T, H)).to(dev)
    ids_d = torch.from_numpy(ids).to(dev)
    w_d = torch.from_numpy(w).to(torch.bfloat16).to(dev)
    outs = {nm: _run(pools, nm, x, ids_d, w_d)[0] for nm in ("raw", "ps4", "t950")}
    assert torch.equal(outs["raw"], outs["t950"]) and torch.equal(outs["ps4"], outs["t950"])
