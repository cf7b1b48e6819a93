"""CPU: ResidentExperts.forward_decode's dispatch when the single-launch expert body cannot run (the library reports
that the device cannot hold its 720 workgroups at once, status -4): nothing is launched, and this call and every later
one take the two-launch form.  The library is replaced by a stub that records the calls (no GPU here)."""
import torch

from neural_amd import _native as N
from neural_amd.moe.experts import ResidentExperts
from neural_amd.moe.layout import GPTOSS_LAYOUT_T950 as LT


class _StubLib:
    def __init__(self, one_status):
        self.calls, self.one_status = [], one_status

    def na_moe_decode_t950_one(self, *args):
        self.calls.append("one")
        return self.one_status

    def na_moe_decode_t950(self, *args):
        self.calls.append("two")
        return 0


def _experts():
    rx = object.__new__(ResidentExperts)
    t = lambda n: torch.zeros(n, dtype=torch.uint8)  # noqa: E731
    rx.layout, rx.pool, rx.slot_tab, rx.bias_gu, rx.bias_dn = LT, t(16), None, None, None
    rx.h, rx.yw, rx.sync = t(16), t(16), torch.zeros(4, dtype=torch.int32)
    rx.max_batch, rx.tiled, rx.one, rx.k_split, rx.down_mode = 1, True, True, 0, 0
    return rx


def _run(monkeypatch, status):
    stub = _StubLib(status)
    monkeypatch.setattr(N, "lib", lambda: stub)
    monkeypatch.setattr(N, "stream", lambda dev=None: None)
    rx = _experts()
    x = torch.zeros(1, 2880, dtype=torch.bfloat16)
    ids = torch.zeros(1, 4, dtype=torch.int64)
    w = torch.zeros(1, 4, dtype=torch.bfloat16)
    rx.forward_decode(3, x, ids, w)
    rx.forward_decode(4, x, ids, w)
    return rx, stub.calls


def test_single_launch_when_resident(monkeypatch):
    rx, calls = _run(monkeypatch, 0)
    assert calls == ["one", "one"] and rx.one


def test_two_launch_form_when_the_device_cannot_hold_the_grid(monkeypatch):
    rx, calls = _run(monkeypatch, N.ERR_RESIDENT)
    assert calls == ["one", "two", "two"] and not rx.one


def test_other_failures_still_raise(monkeypatch):
    import pytest
    with pytest.raises(RuntimeError, match="invalid arguments"):
        _run(monkeypatch, -1)
