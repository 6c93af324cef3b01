"""Seeded synthetic inputs for the W4A16 MoE workloads (numpy, CPU).

Weights: signed int4 uniform in [-8, 7], int4pack along N (a uniformly random
int32 word holds 8 independent uniform nibbles, so packed words are drawn
directly). Scales: bf16(|N(0,1)| * 0.02). Activations and router logits:
bf16(N(0,1)). Skewed routing: expert popularity p_e ~ rank(e)^-s over a
seeded permutation and logits = bf16(ln p_e + Gumbel(0,1)), so top-k is
sampling without replacement proportional to p. Seeds follow
seed = 1000*workload + 10*layer + tensor_id.
"""
from __future__ import annotations

import numpy as np


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def f32_to_bf16_bits(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def int4_words(shape, seed):
    """int32 int4pack words of the given shape (last axis = N/8)."""
    return _rng(seed).integers(0, 1 << 32, size=shape, dtype=np.uint32).view(np.int32)


def scales(shape, seed):
    return f32_to_bf16_bits(np.abs(_rng(seed).standard_normal(shape, dtype=np.float32)) * np.float32(0.02))


def normal_bf16(shape, seed):
    return f32_to_bf16_bits(_rng(seed).standard_normal(shape, dtype=np.float32))


def zipf_logits(T, E, s, seed):
    rng = _rng(seed)
    perm = rng.permutation(E)
    rank = np.empty(E, dtype=np.float64)
    rank[perm] = np.arange(1, E + 1)
    logp = -s * np.log(rank)
    logp -= np.log(np.exp(logp).sum())
    g = rng.gumbel(size=(T, E))
    return f32_to_bf16_bits((logp[None, :] + g).astype(np.float32))


def moe_layer(H, MI, E, gs, seed_base):
    """Expert-major weights of one MoE layer: gate_up [E,H,2MI/8] + scales
    [E,H/gs,2MI], down [E,MI,H/8] + scales [E,MI/gs,H]."""
    return {
        "gu_w": int4_words((E, H, 2 * MI // 8), seed_base + 1),
        "gu_s": scales((E, H // gs, 2 * MI), seed_base + 2),
        "dn_w": int4_words((E, MI, H // 8), seed_base + 3),
        "dn_s": scales((E, MI // gs, H), seed_base + 4),
    }


# The five workloads of the W4A16 MoE expert path.
WORKLOADS = {
    "w4a16_proj_2048x4096_g128": dict(kind="proj", M=1, K=2048, N=4096, gs=128),
    "moe_decode_b1_h2048_e512_mi512_top10_g128": dict(kind="decode", B=1, H=2048, MI=512, E=512, k=10, gs=128),
    "moe_decode_b4_48layers_h2048_e512_mi512_top10_g128": dict(kind="decode_layers", B=4, layers=48, H=2048,
                                                                MI=512, E=512, k=10, gs=128),
    "moe_prefill_t512_zipf1.1_h2048_e512_mi512_top10_g128": dict(kind="prefill", T=512, H=2048, MI=512, E=512,
                                                                  k=10, gs=128, zipf=1.1),
    "moe_prefill_t4096_h3072_e512_mi768_top10_g64": dict(kind="prefill", T=4096, H=3072, MI=768, E=512, k=10,
                                                         gs=64, zipf=None),
}


def routed_bytes_per_expert(H, MI, gs):
    """Algorithmic HBM bytes of one expert: int4 weights + bf16 scales."""
    return (H * 2 * MI + MI * H) // 2 + (H // gs * 2 * MI + MI // gs * H) * 2


# ---------------------------------------------------------------- on-device generation (benchmarks)

def device_int4_words(shape, generator, device):
    """Uniform random int4pack words generated on the device (uniform bytes)."""
    import math
    import torch
    n = math.prod(shape)
    b = torch.empty(n * 4, dtype=torch.uint8, device=device).random_(0, 256, generator=generator)
    return b.view(torch.int32).view(shape)


def device_scales(shape, generator, device):
    import torch
    return (torch.randn(shape, generator=generator, device=device).abs_().mul_(0.02)).to(torch.bfloat16)


def device_layer(H, MI, E, gs, seed, device):
    """Expert-major MoE layer on the device: (gate_up ExpW4, down ExpW4)."""
    import torch
    from .engine import ExpW4
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    gu = ExpW4.from_scales(device_int4_words((E, H, 2 * MI // 8), g, device), device_scales((E, H // gs, 2 * MI), g, device))
    dn = ExpW4.from_scales(device_int4_words((E, MI, H // 8), g, device), device_scales((E, MI // gs, H), g, device))
    return gu, dn
