"""The fp32 -> bf16 rounding every kernel uses (gfx950's v_cvt_pk_bf16_f32, single and paired forms) against the
oracle's integer round-to-nearest-even (oracle/bf16.py, the rounding of torch's .to(bfloat16)) over every bf16 boundary
case: each of the 65536 upper halves with the lower halves 0, 1, 0x4000, 0x7fff, 0x8000 (the tie), 0x8001, 0xc000,
0xffff (this covers zeros, subnormals, the largest finite values rounding to infinity, infinities and NaNs), and 4M
random bit patterns.  NaN inputs must give a NaN; every other input the exact bf16 bits."""
import numpy as np
import pytest

from oracle.bf16 import f32_to_bf16_bits

pytestmark = pytest.mark.gpu


def _bits():
    hi = np.arange(65536, dtype=np.uint32) << 16
    lows = np.array([0, 1, 0x4000, 0x7FFF, 0x8000, 0x8001, 0xC000, 0xFFFF], np.uint32)
    edge = (hi[:, None] | lows[None, :]).reshape(-1)
    rnd = np.random.default_rng(0).integers(0, 2 ** 32, 1 << 22, dtype=np.uint64).astype(np.uint32)
    return np.concatenate([edge, rnd])


def test_hardware_bf16_rounding_matches_integer_rne():
    import torch
    from neural_amd import _native as N
    dev = torch.device("cuda", 0)
    print("case bf16 conversion self-check", flush=True)
    bits = _bits()
    x = bits.view(np.float32)
    xin = torch.from_numpy(x.copy()).to(dev)
    n = x.size
    hw = torch.empty(n, dtype=torch.int16, device=dev)
    pk = torch.empty_like(hw)
    it = torch.empty_like(hw)
    N.call("na_selftest_bf16", xin.data_ptr(), hw.data_ptr(), pk.data_ptr(), it.data_ptr(), n, N.stream(dev))
    torch.cuda.synchronize()
    want = f32_to_bf16_bits(x)
    nan_in = np.isnan(x)
    for nm, t in (("single", hw), ("pair", pk), ("integer", it)):
        got = t.cpu().numpy().view(np.uint16)
        got_nan = ((got & 0x7F80) == 0x7F80) & ((got & 0x7F) != 0)
        assert np.array_equal(got_nan, nan_in), nm
        bad = (got != want) & ~nan_in
        assert not bad.any(), (nm, int(bad.sum()), hex(int(bits[bad][0])), hex(int(got[bad][0])),
                               hex(int(want[bad][0])))
