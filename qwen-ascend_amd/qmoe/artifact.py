"""Expert weight artifacts: the LQP layout, the W4A16 container and its loader.

Two on-disk formats of the reference hold the expert weights of a layer
(``mlp.experts.{gate_up_proj,down_proj}``):

* LQP, ``L{nn}.safetensors`` (``tools/repack_v2.py:8-11``): ``.v2o`` uint8
  [E, N, K/2] (offset-binary int4 packed along K, two 64-wide halves of each
  128-wide K segment per byte), ``.s8`` int8 [E, N, G], ``.base`` fp16 [E, N].
* W4A16, ``L{nn}.w4.safetensors`` (``tools/repack_w4a16.py:8-16``): ``.w4``
  int32 int4pack [K, E, N/8], ``.s8t`` int8 [G, E, N], ``.base`` bf16 [E, N];
  its ``-em`` twin (``tools/repack_w4_em.py``) holds ``.w4`` expert-major
  [E, K, N/8].

:func:`conv_proj` and :func:`repack_lqp_layer` do on the GPU what the
reference's offline tools do on the NPU (``npu_convert_weight_to_int4pack``
plus host-side unpacking and transposes); :func:`load_layer_w4` is the
W4A16 branch of ``fnx/load.py:56-77``. The kernels are
``qmoe_lqp_to_int4pack`` and ``qmoe_lqp_scales`` in libqmoe.so.
"""
from __future__ import annotations

import os
from pathlib import Path

import torch

from . import _lib
from .engine import ExpW4

PROJS = ("gate_up_proj", "down_proj")
PREFIX = "mlp.experts."


def _device_tensor(t, dtype, what):
    if t.device.type != "cuda":
        raise RuntimeError(f"{what} must be a device tensor")
    if t.dtype != dtype:
        raise RuntimeError(f"{what} must be {dtype}")
    return t.contiguous()


def lqp_to_int4pack(v2o, expert_major=True):
    """v2o uint8 [E, N, K/2] -> int4pack int32 [E, K, N/8] (``expert_major``)
    or [K, E, N/8]: the same int4 values, unpacked from offset binary along K
    and packed in two's complement along N (``tools/repack_w4a16.py:41-70``,
    ``tools/repack_w4_em.py:16``)."""
    v2o = _device_tensor(v2o, torch.uint8, "v2o")
    if v2o.dim() != 3:
        raise RuntimeError("v2o must be [E, N, K/2]")
    E, N, half = v2o.shape
    K = 2 * half
    shape = (E, K, N // 8) if expert_major else (K, E, N // 8)
    w4 = torch.empty(shape, dtype=torch.int32, device=v2o.device)
    if E == 0:
        return w4
    rc = _lib.lib().qmoe_lqp_to_int4pack(v2o.data_ptr(), w4.data_ptr(), E, N, K, int(bool(expert_major)),
                                        _lib.stream_of(v2o))
    _lib.check(rc, "lqp_to_int4pack")
    return w4


def lqp_scales(s8, base):
    """LQP scales int8 [E, N, G] + base fp16 [E, N] -> (s8t int8 [G, E, N],
    base bf16 [E, N], the bf16 scale cache [E, G, N] = bf16(s8 * base_bf16))
    (``tools/repack_w4a16.py:71-72``, ``fnx/engine.py:653-659``)."""
    s8 = _device_tensor(s8, torch.int8, "s8")
    base = _device_tensor(base, torch.float16, "base")
    if s8.dim() != 3 or base.shape != s8.shape[:2]:
        raise RuntimeError("s8 must be [E, N, G] and base [E, N]")
    E, N, G = s8.shape
    dev = s8.device
    s8t = torch.empty((G, E, N), dtype=torch.int8, device=dev)
    base_bf = torch.empty((E, N), dtype=torch.bfloat16, device=dev)
    scales = torch.empty((E, G, N), dtype=torch.bfloat16, device=dev)
    if s8.numel():
        rc = _lib.lib().qmoe_lqp_scales(s8.data_ptr(), base.data_ptr(), s8t.data_ptr(), base_bf.data_ptr(),
                                        scales.data_ptr(), E, N, G, _lib.stream_of(s8))
        _lib.check(rc, "lqp_scales")
    return s8t, base_bf, scales


def conv_proj(v2o, s8, base, expert_major=False):
    """One projection of an LQP layer -> the W4A16 artifact tensors
    (w4, s8t, base bf16); ``tools/repack_w4a16.py:58-76`` (K-major w4) or,
    with ``expert_major``, followed by ``tools/repack_w4_em.py:16``."""
    w4 = lqp_to_int4pack(v2o, expert_major)
    s8t, base_bf, _ = lqp_scales(s8, base)
    return w4, s8t, base_bf


def to_expert_major(w4):
    """K-major int4pack [K, E, N/8] -> expert-major [E, K, N/8]
    (``tools/repack_w4_em.py:16``: a permute; byte-for-byte the same words)."""
    return w4.permute(1, 0, 2).contiguous()


def exp_w4_from_lqp(v2o, s8, base):
    """An expert-major :class:`ExpW4` straight from LQP tensors (the container
    and its bf16 scale cache built on the GPU)."""
    w4 = lqp_to_int4pack(v2o, expert_major=True)
    _, _, scales = lqp_scales(s8, base)
    return ExpW4.from_scales(w4, scales)


def layer_path(directory, layer_idx, expert_major=True):
    """``{dir}/L{nn}.w4.safetensors`` or, expert-major, ``{dir}-em/...``
    (``fnx/load.py:63-69``)."""
    d = str(directory).rstrip("/")
    if expert_major:
        d += "-em"
    return Path(d) / f"L{layer_idx:02d}.w4.safetensors"


def load_layer_w4(path, device, expert_major=None, gs=None):
    """Expert projections of one W4A16 artifact file -> {name: ExpW4}.

    The W4A16 branch of ``fnx/load.py:56-77``: for every
    ``mlp.experts.<proj>`` the ``.w4``, ``.s8t`` and ``.base`` tensors go to
    ``device`` and become ``ExpW4(w4, s8t, base, gs, expert_major)``. When
    ``expert_major`` is None the layout follows the reference's directory
    convention: files under a directory whose name ends in ``-em`` are
    expert-major (``fnx/load.py:66-69``). The group size is K / G unless
    given (the reference fixes it at 64).
    """
    from safetensors.torch import load_file

    em = expert_major if expert_major is not None else Path(path).resolve().parent.name.endswith("-em")
    sd = load_file(str(path), device=str(device))
    res = {}
    try:
        for key in sorted(k[: -len(".w4")] for k in sd if k.endswith(".w4")):
            w4, s8t, base = sd[key + ".w4"], sd[key + ".s8t"], sd[key + ".base"]
            K = w4.shape[1] if em else w4.shape[0]
            g = gs if gs is not None else K // s8t.shape[0]
            res[key] = ExpW4(w4, s8t, base, g, expert_major=em)
    finally:
        del sd
    return res


def repack_lqp_layer(src, dst, device, expert_major=True):
    """LQP layer file -> W4A16 artifact file (``tools/repack_w4a16.py:79-106``
    for one layer; expert-major output as ``tools/repack_w4_em.py`` writes
    it). Converts on ``device``; writes through a temporary file that is
    renamed at the end, like the reference tools."""
    from safetensors.torch import load_file, save_file

    sd = load_file(str(src), device=str(device))
    out = {}
    for proj in PROJS:
        key = PREFIX + proj
        if key + ".v2o" not in sd:
            continue
        w4, s8t, base_bf = conv_proj(sd[key + ".v2o"], sd[key + ".s8"], sd[key + ".base"], expert_major)
        out[key + ".w4"], out[key + ".s8t"], out[key + ".base"] = w4.cpu(), s8t.cpu(), base_bf.cpu()
    del sd
    if not out:
        raise RuntimeError(f"{src}: no LQP expert tensors")
    tmp = str(dst) + ".tmp"
    save_file(out, tmp)
    os.replace(tmp, str(dst))
    return dst
