"""ctypes binding of libqmoe.so and per-device scratch management.

Mirrors the reference's wrapper convention (``fnx/expert_gather.py:19-24``,
``fnx/weighted_reduce.py:32-41``): the library path can be overridden by an
environment variable (``QMOE_SO``), it is loaded lazily into a module global,
every launch goes to the caller's current stream, and a non-zero return code
raises ``RuntimeError``. There is no fallback: if the library is missing the
call fails loudly.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

_LIB = None
_LOCK = threading.Lock()
_SO = Path(__file__).with_name("libqmoe.so")

P = ctypes.c_void_p
I = ctypes.c_int
L = ctypes.c_long
Z = ctypes.c_size_t
EINVAL = -1  # QMOE_EINVAL: a shape or argument the entry point does not take

# name -> (restype, argtypes); every entry point declared in include/qmoe.h
SIGNATURES = {
    "qmoe_w4a16_gemm_workspace": (Z, [I, I, I]),
    "qmoe_w4a16_gemm_counters": (I, [I, I, I]),
    "qmoe_w4a16_gemv": (I, [P, P, P, P, I, I, I, I, P, Z, P, P]),
    "qmoe_w4a16_gemm_mfma_workspace": (Z, [I, I]),
    "qmoe_w4a16_gemm_mfma": (I, [P, P, P, P, I, I, I, I, P, Z, P]),
    "qmoe_moe_decode_workspace": (Z, [I, I, I, I]),
    "qmoe_moe_decode_counters": (I, [I, I, I, I]),
    "qmoe_moe_decode_layout": (I, [I, I, I, I, P, P, P]),
    "qmoe_moe_decode": (I, [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, P, Z, P, P]),
    "qmoe_moe_decode_tiled": (I, [P, P, P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, P, Z, P, P]),
    "qmoe_moe_block_decode": (I, [P, P, P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, P, P]),
    "qmoe_decode_tiles_gate_up": (I, [P, P, I, I, I, I, P]),
    "qmoe_decode_tiles_down": (I, [P, P, I, I, I, P]),
    "qmoe_moe_decode_status": (I, [P, I, P, P]),
    "qmoe_xcd_placement": (I, [I, P]),
    "qmoe_moe_decode_noalloc_max_bytes": (Z, []),
    "qmoe_moe_decode_noalloc": (I, [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, P]),
    "qmoe_moe_decode_gate_up": (I, [P, P, P, P, P, P, I, I, I, I, I, I, P, Z, P, P]),
    "qmoe_moe_decode_down": (I, [P, P, P, P, P, I, I, I, I, I, P, Z, P, P]),
    "qmoe_router_topk": (I, [P, P, P, I, I, I, P]),
    "qmoe_route_group_workspace": (Z, [I, I]),
    "qmoe_max_row_tiles": (I, [I, I, I]),
    "qmoe_route_group": (I, [P, I, I, P, P, P, P, I, P, P, P, P, P, Z, P]),
    "qmoe_tiles_from_ends": (I, [P, I, I, I, P, P, P, P, P]),
    "qmoe_tiles_from_ids": (I, [P, I, I, P, P, P, P, P]),
    "qmoe_gemm_tile_rows": (I, []),
    "qmoe_grouped_gemm_workspace": (Z, [I, I]),
    "qmoe_grouped_gemm": (I, [P, I, I, I, I, I, P, P, P, P, P, P, I, P, P, Z, P]),
    "qmoe_moe_prefill_workspace": (Z, [I, I, I, I]),
    "qmoe_moe_prefill_layout": (I, [I, I, I, I, P, P]),
    "qmoe_moe_experts_grouped": (I, [P, I, I, I, I, I, P, P, P, P, I, P, P, I, P, P, P, P, I, P, P, P, Z, P]),
    "qmoe_expert_gather": (I, [P, P, P, P, P, I, I, I, I, I, P]),
    "qmoe_expert_gather_kmajor": (I, [P, P, P, P, P, I, I, I, I, I, P]),
    "qmoe_weighted_reduce": (I, [P, P, P, P, I, I, I, L, L, P]),
    "qmoe_moe_epilogue": (I, [P, P, P, P, P, I, I, P]),
    "qmoe_moe_merge": (I, [P, P, P, P, I, I, P]),
    "qmoe_swiglu": (I, [P, P, I, I, P]),
    "qmoe_lqp_to_int4pack": (I, [P, P, I, I, I, I, P]),
    "qmoe_lqp_scales": (I, [P, P, P, P, P, I, I, I, P]),
    "qmoe_scale_cache": (I, [P, P, P, I, I, I, P]),
    "qmoe_bf16_gemv": (I, [P, L, P, P, L, I, I, I, P]),
    "qmoe_bf16_gemv_split": (I, [P, L, P, P, L, P, L, I, I, I, I, P]),
    "qmoe_bf16_gemm": (I, [P, L, P, P, L, I, I, I, P]),
    "qmoe_bf16_gemv_swiglu": (I, [P, L, P, P, L, I, I, I, P]),
    "qmoe_swiglu_bf16": (I, [P, L, P, L, I, P]),
    "qmoe_shared_gate": (I, [P, P, L, P, L, I, P]),
    "qmoe_w8a16_gemv_workspace": (Z, [I, I, I]),
    "qmoe_w8a16_gemv_counters": (I, [I]),
    "qmoe_w8a16_gemv": (I, [P, P, P, P, I, I, I, I, P, Z, P, P]),
    "qmoe_w8a16_gemm_mfma": (I, [P, P, P, P, I, I, I, I, P]),
}


def library_path() -> Path:
    return Path(os.environ.get("QMOE_SO", str(_SO)))


def lib():
    """Load libqmoe.so once (thread-safe) and declare every signature."""
    global _LIB
    if _LIB is None:
        with _LOCK:
            if _LIB is None:
                path = library_path()
                if not path.exists():
                    raise RuntimeError(f"{path} is not built; run __graft_entry__.build() "
                                       "(or python -m qmoe._build) first")
                so = ctypes.CDLL(str(path))
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(so, name)
                    fn.restype = res
                    fn.argtypes = args
                _LIB = so
    return _LIB


def check(rc: int, what: str) -> None:
    if rc:
        kind = {-1: "rejected arguments", -2: "workspace too small",
                -3: "shape beyond the fixed no-allocation scratch"}.get(rc, f"HIP error {rc}")
        raise RuntimeError(f"{what} launch failed: {kind} ({rc})")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------- scratch

_COUNTERS: dict = {}
_RETIRED: list = []
_COUNTER_SLOTS = 1 << 20
DECODE_MAILBOX_BASE = 1 << 16  # QMOE_DECODE_MAILBOX_BASE of qmoe.h
DECODE_EPOCH_SLOT = DECODE_MAILBOX_BASE - 2
DECODE_ERROR_SLOT = DECODE_MAILBOX_BASE - 1


def counters(device: torch.device, min_slots: int = 0) -> torch.Tensor:
    """Per-device counters array (int32, zero at first use).

    Kernels that use it leave its counters at zero when they finish; the
    decode kernels also keep their launch epoch, error flag and tagged mailbox
    in it. One array serves every call issued in stream order on that device;
    calls that overlap on different streams must pass arrays of their own
    (:func:`new_counters`).

    A call needing more slots than the current array has gets a larger,
    zeroed one. The smaller array is kept alive for the life of the process,
    because a HIP graph captured earlier may still hold its address. Growing
    allocates, so it is refused during graph capture: make one eager call of
    the largest shape before capturing.
    """
    key = (device.type, device.index)
    buf = _COUNTERS.get(key)
    if buf is None or buf.numel() < min_slots:
        if _capturing(device):
            raise RuntimeError("qmoe counters must grow outside graph capture: run the call once eagerly first")
        if buf is not None:
            _RETIRED.append(buf)
        buf = new_counters(device, min_slots)
        _COUNTERS[key] = buf
    return buf


def _capturing(device: torch.device) -> bool:
    return device.type == "cuda" and torch.cuda.is_current_stream_capturing()


def new_counters(device: torch.device, min_slots: int = 0) -> torch.Tensor:
    """A zeroed counters array owned by the caller (for a second stream).

    On a GPU, creating one (outside graph capture) also settles the device's
    workgroup placement check (:func:`xcd_placement`), so later calls, captured
    ones included, take the same launch forms as the first eager call."""
    buf = torch.zeros(max(_COUNTER_SLOTS, int(min_slots)), dtype=torch.int32, device=device)
    if device.type == "cuda" and not _capturing(device):
        xcd_placement(device)
    return buf


def xcd_placement(device: torch.device, mode: int = 0) -> int:
    """Workgroup placement check of a GPU (``qmoe_xcd_placement``): mode 0
    returns 1 when workgroup b of a launch runs on XCD (b + c) mod 8, which the
    one-token decode launch and the one-row GEMV rely on to keep hand-offs
    in one XCD's L2 (probed once, synchronising); otherwise those calls run
    their device-coherent forms. Mode 1 switches the device to those forms,
    mode 2 forgets the verdict."""
    with torch.cuda.device(device):
        rc = lib().qmoe_xcd_placement(int(mode), torch.cuda.current_stream(device).cuda_stream)
    if rc < 0 or rc > 1:
        check(rc, "xcd_placement")
    return rc


def decode_status(cnt: torch.Tensor, clear: bool = True) -> int:
    """The decode error flag of a counters array: 1 if a bounded wait of an
    earlier decode call timed out (that call's output is wrong), else 0.
    Synchronises the current stream; ``clear`` resets the flag."""
    flag = ctypes.c_int(0)
    check(lib().qmoe_moe_decode_status(cnt.data_ptr(), int(clear), ctypes.byref(flag), stream_of(cnt)),
          "moe_decode_status")
    return flag.value


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Per-call scratch from the caching allocator (stream-ordered reuse)."""
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)
