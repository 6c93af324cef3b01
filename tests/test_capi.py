"""The C-ABI library loads and exports every entry point include/qmoe.h declares (CPU only)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "qmoe.h"


def declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qmoe_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert "qmoe_w4a16_gemv" in names and "qmoe_grouped_gemm" in names and len(names) >= 20


def test_library_exports_every_declared_symbol():
    from qmoe import _lib
    path = _lib.library_path()
    if not path.exists():
        pytest.fail(f"{path} not built")
    so = ctypes.CDLL(str(path))
    missing = [n for n in declared() if not hasattr(so, n)]
    assert not missing, missing


def test_python_binding_covers_header():
    from qmoe import _lib
    assert sorted(_lib.SIGNATURES) == declared()
    so = _lib.lib()
    for name in _lib.SIGNATURES:
        assert getattr(so, name).restype is not None or name == ""


def test_host_side_shape_queries():
    from qmoe import _lib
    L = _lib.lib()
    assert L.qmoe_gemm_tile_rows() == 128
    assert L.qmoe_max_row_tiles(40960, 512, 128) == 320 + 512
    assert L.qmoe_w4a16_gemm_workspace(1, 2048, 4096) == 0          # partials live in the counters mailbox
    assert L.qmoe_w4a16_gemm_counters(1, 2048, 4096) == 65536 + 2 * 16 * 15 * 4 * 256
    assert L.qmoe_moe_decode_workspace(1, 10, 2048, 512) > 0
    assert L.qmoe_route_group_workspace(40960, 512) == (160 + 1) * 512 * 4  # chunk histograms + expert totals
    # argument validation happens on the host, before any launch
    assert L.qmoe_w4a16_gemv(None, None, None, None, 5, 2048, 4096, 128, None, 0, None, None) == -1
    assert L.qmoe_w4a16_gemv(None, None, None, None, 1, 2048, 4096, 128, None, 0, None, None) == -1  # no counters
    assert L.qmoe_router_topk(None, None, None, 1, 512, 17, None) == -1
    assert L.qmoe_moe_decode(*([None] * 11), 5, 512, 10, 2048, 512, 128, 128, None, 0, None, None) == -1
