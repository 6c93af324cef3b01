"""Seeded inputs for the GPU parity tests (host numpy -> device tensors)."""
import numpy as np
import torch

from oracle import qmoe_oracle as O
from parity import to_dev


def rng(seed):
    return np.random.default_rng(seed)


def bf16_normal(shape, seed, scale=1.0):
    return O.f32_to_bf16_bits(rng(seed).standard_normal(shape).astype(np.float32) * np.float32(scale))


def int4_words(shape, seed):
    return rng(seed).integers(0, 2**32, size=shape, dtype=np.uint32).view(np.int32)


def scales(shape, seed):
    return O.f32_to_bf16_bits(np.abs(rng(seed).standard_normal(shape).astype(np.float32)) * np.float32(0.02))


def layer(E, H, MI, gs, seed):
    """Expert-major MoE layer (host arrays)."""
    return dict(gu_w=int4_words((E, H, 2 * MI // 8), seed + 1), gu_s=scales((E, H // gs, 2 * MI), seed + 2),
                dn_w=int4_words((E, MI, H // 8), seed + 3), dn_s=scales((E, MI // gs, H), seed + 4))


def layer_dev(lay, device):
    from qmoe import ExpW4
    gu = ExpW4.from_scales(to_dev(lay["gu_w"], device), to_dev(lay["gu_s"], device))
    dn = ExpW4.from_scales(to_dev(lay["dn_w"], device), to_dev(lay["dn_s"], device))
    return gu, dn


def log(msg):
    print(f"[case] {msg}", flush=True)


def prod_interval(y_exact, y_abs, w_bits):
    """Admissible bf16(bf16(y) * w) for w >= 0 (the product of two bf16 is
    exact in fp32, so only y's rounding is uncertain)."""
    lo, hi = O.bf16_interval(y_exact, y_abs)
    wv = O.bf16_bits_to_f32(np.asarray(w_bits).view(np.uint16)).reshape(-1, 1)
    return (O.f32_to_bf16_bits(O.bf16_bits_to_f32(lo) * wv), O.f32_to_bf16_bits(O.bf16_bits_to_f32(hi) * wv))


def check_expert_rows(x_rows, experts, wts, act_gpu, prod_gpu, lay, gs_gu, gs_dn, what):
    """Stage-wise rounding exactness of routed rows.

    x_rows [n, H] bf16 bits, experts [n] ids, wts [n] bf16 bits of the routing
    weight, act_gpu [n, MI] and prod_gpu [n, H] bf16 bits from the GPU.
    gate_up + SwiGLU must give an admissible rounding of the exact values
    (oracle fed x), down + weight an admissible rounding given the GPU's own
    act rows."""
    from parity import assert_in_interval
    n = len(experts)
    MI = act_gpu.shape[1]
    a_lo, a_hi, p_lo, p_hi = [], [], [], []
    for r in range(n):
        e = int(experts[r])
        ge, ga = O.w4a16_gemm_exact(x_rows[r:r + 1], lay["gu_w"][e], lay["gu_s"][e], gs_gu)
        lo, hi = O.swiglu_interval(ge[0, :MI], ga[0, :MI], ge[0, MI:], ga[0, MI:])
        a_lo.append(lo)
        a_hi.append(hi)
        ye, ya = O.w4a16_gemm_exact(act_gpu[r:r + 1], lay["dn_w"][e], lay["dn_s"][e], gs_dn)
        lo, hi = prod_interval(ye, ya, wts[r:r + 1])
        p_lo.append(lo[0])
        p_hi.append(hi[0])
    assert_in_interval(act_gpu, np.stack(a_lo), np.stack(a_hi), what + " act")
    assert_in_interval(prod_gpu, np.stack(p_lo), np.stack(p_hi), what + " prod")
