"""Host-side scratch policy of qmoe._lib (no GPU): the per-device counters
array grows to the largest request, keeps every array it replaced alive (a
HIP graph captured earlier may still hold its address) and refuses to grow
while a stream is being captured."""
import pytest
import torch

from qmoe import _lib

CPU = torch.device("cpu")


@pytest.fixture
def fresh_counters(monkeypatch):
    monkeypatch.setattr(_lib, "_COUNTERS", {})
    monkeypatch.setattr(_lib, "_RETIRED", [])
    monkeypatch.setattr(_lib, "_COUNTER_SLOTS", 64)
    return _lib


def test_counters_grow_and_retire(fresh_counters):
    L = fresh_counters
    a = L.counters(CPU, 10)
    assert a.dtype == torch.int32 and a.numel() == 64 and int(a.abs().sum()) == 0
    assert L.counters(CPU, 64) is a and L.counters(CPU) is a      # no growth for requests that fit
    a[3] = 7                                                      # state the kernels would leave
    b = L.counters(CPU, 200)
    assert b is not a and b.numel() == 200 and int(b.abs().sum()) == 0
    assert L._RETIRED == [a] and int(a[3]) == 7                   # the old array stays alive, untouched
    c = L.counters(CPU, 1000)
    assert L._RETIRED == [a, b] and c.numel() == 1000
    assert L.counters(CPU, 5) is c


def test_counters_refuse_to_grow_under_capture(fresh_counters, monkeypatch):
    L = fresh_counters
    a = L.counters(CPU, 32)
    monkeypatch.setattr(L, "_capturing", lambda device: True)
    assert L.counters(CPU, 64) is a                               # fits: returned during capture
    with pytest.raises(RuntimeError, match="outside graph capture"):
        L.counters(CPU, 65)
    assert L._COUNTERS[("cpu", None)] is a and L._RETIRED == []   # nothing replaced


def test_counters_first_use_under_capture_refused(fresh_counters, monkeypatch):
    L = fresh_counters
    monkeypatch.setattr(L, "_capturing", lambda device: True)
    with pytest.raises(RuntimeError, match="outside graph capture"):
        L.counters(CPU, 1)
    assert L._COUNTERS == {}


def test_new_counters_are_independent(fresh_counters):
    L = fresh_counters
    a = L.new_counters(CPU, 10)
    b = L.new_counters(CPU, 10)
    assert a.data_ptr() != b.data_ptr() and a.numel() == b.numel() == 64
    assert L._COUNTERS == {}                                      # caller-owned, not the device's array
