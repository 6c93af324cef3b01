"""Host-side bookkeeping of the opt-in decode tiles of ExpW4 (no GPU): tiles
built earlier are returned only while they match the weights they were built
from (same tensor, same storage, same version), rebinding drops them, a
failed build is not retried until the weights are rebound, and shapes the
tiled launch does not take get none."""
import pytest
import torch

from qmoe import engine
from qmoe.engine import ExpW4, _tiles_for


def _exp(E=4, K=256, N=256, gs=64, expert_major=True):
    shape = (E, K, N // 8) if expert_major else (K, E, N // 8)
    return ExpW4(torch.zeros(shape, dtype=torch.int32), None, None, gs, expert_major=expert_major)


def _plant(e, kind):
    """Tiles as decode_tiles records them after a build."""
    w = e.w4
    t = torch.ones_like(w)
    e._dtile = (kind, t, (w.data_ptr(), w.untyped_storage().data_ptr(), w._version))
    return t


def test_cached_tiles_returned_while_weights_unchanged():
    e = _exp()
    assert e.cached_decode_tiles("gate_up") is None
    t = _plant(e, "gate_up")
    assert e.cached_decode_tiles("gate_up") is t
    assert e.decode_tiles("gate_up") is t                          # built once: no second build
    with pytest.raises(ValueError, match="built as 'gate_up'"):
        e.cached_decode_tiles("down")


def test_rebinding_drops_tiles():
    e = _exp()
    _plant(e, "down")
    e.w4 = torch.zeros_like(e.w4)
    assert e._dtile is None and e.cached_decode_tiles("down") is None


def test_in_place_update_drops_tiles():
    e = _exp()
    _plant(e, "gate_up")
    e.w4[0, 0, 0] = 5                                              # bumps the tensor version
    assert e.cached_decode_tiles("gate_up") is None
    assert e._dtile is None


def test_view_of_other_storage_drops_tiles():
    e = _exp()
    _plant(e, "gate_up")
    bigger = torch.zeros((2,) + tuple(e.w4.shape), dtype=torch.int32)
    e._w4 = bigger[1]                                              # same shape, other storage and address
    assert e.cached_decode_tiles("gate_up") is None


def test_failed_build_not_retried_until_rebind(monkeypatch):
    e = _exp()
    calls = []

    def no_memory(*a, **k):
        calls.append(1)
        raise torch.OutOfMemoryError("no memory for the copy")

    monkeypatch.setattr(engine.torch, "empty_like", no_memory)
    monkeypatch.setattr(engine.torch.cuda, "is_current_stream_capturing", lambda: False)
    assert e.decode_tiles("gate_up") is None and e._dtile_failed
    assert e.decode_tiles("gate_up") is None and len(calls) == 1   # not tried again
    e.w4 = torch.zeros(tuple(e.w4.shape), dtype=torch.int32)
    assert not e._dtile_failed
    assert e.decode_tiles("gate_up") is None and len(calls) == 2


@pytest.mark.parametrize("kind,K,N,em", [
    ("gate_up", 256, 256, False),      # K-major weights: never tiled
    ("gate_up", 128, 256, True),       # H below 256
    ("gate_up", 384, 256, True),       # H not a multiple of 256
    ("gate_up", 256, 192, True),       # MI = 96 not a multiple of 128
    ("down", 64, 512, True),           # MI = 64 below 128
    ("down", 256, 384, True),          # H = 384 not a multiple of 256
])
def test_untiled_shapes_get_none(monkeypatch, kind, K, N, em):
    e = _exp(K=K, N=N, expert_major=em)
    monkeypatch.setattr(engine.torch, "empty_like", lambda *a, **k: pytest.fail("no copy for this shape"))
    assert e.decode_tiles(kind) is None and not e._dtile_failed


def test_bad_kind():
    with pytest.raises(ValueError, match="'gate_up' or 'down'"):
        _exp().decode_tiles("up")


def test_tiles_for_pairs():
    gu, dn = _exp(), _exp()
    assert _tiles_for(gu, dn, False) == (None, None)
    assert _tiles_for(gu, dn, None) == (None, None)                # nothing built: the decode reads w4
    tg = _plant(gu, "gate_up")
    assert _tiles_for(gu, dn, None) == (None, None)                # both or neither
    td = _plant(dn, "down")
    g, d = _tiles_for(gu, dn, None)
    assert g is tg and d is td
    assert _tiles_for(gu, dn, False) == (None, None)               # tiles=False ignores built tiles
    dn.w4 = torch.zeros_like(dn.w4)
    assert _tiles_for(gu, dn, None) == (None, None)
