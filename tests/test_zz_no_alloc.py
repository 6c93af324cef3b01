"""qmoe_moe_decode_noalloc: the decode block with no workspace and no counters
argument (its scratch is a fixed per-device array), called through the C ABI
and compared bit for bit with qmoe_moe_decode on the same inputs, over two
calls in a row (the second with smaller inputs, so stale mailbox words of the
first are in the array), plus the size limit and the error flag."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import bf16_normal, layer, layer_dev, log
from parity import to_dev


def _noalloc(L, x, lg, gu, dn, k, sh=None, sg=None):
    B, H = x.shape
    out = torch.empty((B, H), dtype=torch.bfloat16, device=x.device)
    idx = torch.empty((B, k), dtype=torch.int64, device=x.device)
    w = torch.empty((B, k), dtype=torch.bfloat16, device=x.device)
    from qmoe import _lib
    rc = L.qmoe_moe_decode_noalloc(x.data_ptr(), lg.data_ptr(), gu.w4.data_ptr(), gu._scales.data_ptr(),
                                   dn.w4.data_ptr(), dn._scales.data_ptr(), _lib.ptr(sh), _lib.ptr(sg),
                                   out.data_ptr(), idx.data_ptr(), w.data_ptr(), B, gu.E, k, H, dn.K, gu.gs, dn.gs,
                                   _lib.stream_of(x))
    _lib.check(rc, "moe_decode_noalloc")
    return out, idx, w


@pytest.mark.gpu
def test_noalloc_decode_matches_allocating_entry(device):
    from qmoe import _lib, moe_decode
    L = _lib.lib()
    cases = [  # (B, E, H, MI, gs, k, shared): the second call is smaller than the first
        (4, 512, 2048, 512, 128, 10, True),
        (1, 64, 512, 128, 64, 8, False),
    ]
    for i, (B, E, H, MI, gs, k, with_shared) in enumerate(cases):
        log(f"noalloc call {i}: B={B} E={E} H={H} MI={MI} k={k}")
        lay = layer(E, H, MI, gs, 900 + i)
        gu, dn = layer_dev(lay, device)
        x = to_dev(bf16_normal((B, H), 910 + i), device)
        lg = to_dev(bf16_normal((B, E), 920 + i), device)
        sh = to_dev(bf16_normal((B, H), 930 + i), device) if with_shared else None
        sg = to_dev(bf16_normal((B, 1), 940 + i), device) if with_shared else None
        out_n, idx_n, w_n = _noalloc(L, x, lg, gu, dn, k, sh, sg)
        out_a, idx_a, w_a = moe_decode(x, lg, gu, dn, k, sh, sg)
        torch.cuda.synchronize()
        assert torch.equal(idx_n, idx_a)
        assert torch.equal(w_n.view(torch.int16), w_a.view(torch.int16))
        assert torch.equal(out_n.view(torch.int16), out_a.view(torch.int16)), f"call {i}"
    flag = ctypes.c_int(-1)
    _lib.check(L.qmoe_moe_decode_status(None, 1, ctypes.byref(flag), _lib.stream_of(x)), "status")
    assert flag.value == 0


@pytest.mark.gpu
def test_noalloc_decode_rejects_oversize(device):
    from qmoe import _lib
    L = _lib.lib()
    limit = L.qmoe_moe_decode_noalloc_max_bytes()
    assert limit == 8 << 20
    assert 4 * L.qmoe_moe_decode_counters(4, 10, 3072, 768) <= limit
    B, E, H, MI, k = 4, 512, 8192, 2048, 16
    assert 4 * L.qmoe_moe_decode_counters(B, k, H, MI) > limit
    dummy = torch.zeros(16, dtype=torch.int32, device=device)
    p = dummy.data_ptr()
    rc = L.qmoe_moe_decode_noalloc(p, p, p, p, p, p, None, None, p, p, p, B, E, k, H, MI, 128, 128,
                                   _lib.stream_of(dummy))
    assert rc == -3      # QMOE_ESCRATCH, before any launch


@pytest.mark.gpu
def test_noalloc_decode_graph_replay(device):
    """The no-allocation entry captured in a graph (after one eager call) and
    replayed with fresh inputs gives the eager bits every time."""
    from qmoe import _lib
    from test_gpu_decode_paths import _replay_matches_eager
    L = _lib.lib()
    B, E, H, MI, gs, k = 1, 512, 2048, 512, 128, 10
    log("noalloc decode graph replay")
    lay = layer(E, H, MI, gs, 950)
    gu, dn = layer_dev(lay, device)
    x = torch.randn(B, H, device=device).to(torch.bfloat16)
    lg = torch.randn(B, E, device=device).to(torch.bfloat16)
    fresh = [(torch.randn(B, H, device=device).to(torch.bfloat16), torch.randn(B, E, device=device).to(torch.bfloat16))
             for _ in range(3)]
    _replay_matches_eager(lambda a, b: _noalloc(L, a, b, gu, dn, k), [x, lg], fresh, "moe_decode_noalloc")
    flag = ctypes.c_int(-1)
    _lib.check(L.qmoe_moe_decode_status(None, 1, ctypes.byref(flag), _lib.stream_of(x)), "status")
    assert flag.value == 0
