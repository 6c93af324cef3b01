"""Shared expert and router projection (fnx/engine.py:1786-1802) and the whole
MoE block: bf16 GEMV, the bf16 SwiGLU and sigmoid gate, and the block end to
end, each stage checked against the oracle fed the GPU's previous stage."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_normal, layer, layer_dev, log
from oracle import qmoe_oracle as O
from parity import assert_block_output, assert_in_interval, bits, to_dev


def check_linear(y_gpu_bits, x_bits, w_bits, what):
    ex, ab = O.linear_exact(x_bits, w_bits)
    lo, hi = O.bf16_interval(ex, ab)
    assert_in_interval(y_gpu_bits, lo, hi, what)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("K,N", [(2048, 1537), (512, 2048), (3072, 1537), (768, 3072), (40, 17), (4096, 64)])
def test_bf16_linear_gemv(device, M, K, N):
    from qmoe.shared import linear
    log(f"bf16 linear M={M} K={K} N={N}")
    x = bf16_normal((M, K), K + M)
    w = bf16_normal((N, K), N, 0.02)
    y = linear(to_dev(x, device), to_dev(w, device))
    torch.cuda.synchronize()
    check_linear(bits(y), x, w, "linear")


@pytest.mark.gpu
@pytest.mark.parametrize("rows,MI", [(1, 512), (3, 768), (300, 640), (2, 8)])
def test_swiglu_bf16_and_gate(device, rows, MI):
    from qmoe.shared import gate_shared, swiglu_bf16
    log(f"swiglu_bf16 rows={rows} MI={MI}")
    gu = bf16_normal((rows, 2 * MI + 5), rows + MI, 3.0)          # extra columns: row stride > 2 MI
    act = swiglu_bf16(to_dev(gu, device), MI)
    torch.cuda.synchronize()
    ref = O.swiglu_bf16(gu, MI)
    # silu goes through exp in fp32 on both sides: a result may differ in the
    # last place only where bf16(silu(g)) sits on a rounding boundary
    diff = bits(act) != ref
    if diff.any():
        g = O.bf16_bits_to_f32(gu[:, :MI]).astype(np.float64)
        s = g / (1 + np.exp(-g))
        lo, hi = O.bf16_interval(s)
        assert np.all(lo[diff] != hi[diff]), "swiglu differs away from a rounding boundary"
    gate = gu[:, 2 * MI:2 * MI + 1]
    for H in (96, 100, 3072):  # 16-byte rows (vector kernel) and not
        sh = bf16_normal((rows, H), rows + H)
        out = gate_shared(to_dev(sh, device), to_dev(np.ascontiguousarray(gu), device)[:, 2 * MI:2 * MI + 1])
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), O.shared_gate(sh, gate)), f"H={H}"


@pytest.mark.gpu
@pytest.mark.parametrize("b", [1, 3, 64])
def test_shared_router_stages(device, b):
    from qmoe.shared import shared_router, swiglu_bf16
    H, MI, E = 2048, 512, 512
    log(f"shared_router b={b} H={H} MI={MI} E={E}")
    x = bf16_normal((b, H), b)
    sh_gu = bf16_normal((2 * MI + 1 + E, H), 11, 0.03)
    sh_down = bf16_normal((H, MI), 12, 0.03)
    from qmoe.shared import linear
    sh, gate2, logits = shared_router(to_dev(x, device), to_dev(sh_gu, device), to_dev(sh_down, device), MI)
    # the fused projection (gate | up | gate2 | router), as shared_router computes it
    gu_gpu = bits(linear(to_dev(x, device), to_dev(sh_gu, device)))
    torch.cuda.synchronize()
    check_linear(gu_gpu, x, sh_gu, "gu")
    assert np.array_equal(bits(gate2), gu_gpu[:, 2 * MI:2 * MI + 1])
    assert np.array_equal(bits(logits), gu_gpu[:, 2 * MI + 1:])
    if b <= 4:
        # rows of their own, aligned for the one-token decode kernel's vector loads
        assert logits.is_contiguous() and logits.data_ptr() % 16 == 0
    # shared down over the GPU's own SwiGLU of gu (same device arithmetic)
    act_gpu = bits(swiglu_bf16(to_dev(gu_gpu, device), MI))
    torch.cuda.synchronize()
    check_linear(bits(sh), act_gpu, sh_down, "shared down")


@pytest.mark.gpu
@pytest.mark.parametrize("split", [0, 7, 1025, 1537])
def test_bf16_gemv_split(device, split):
    """Output columns from split on go to the second matrix, the same bits as
    the one-matrix GEMV; nothing outside the written columns changes."""
    from qmoe import _lib
    M, K, N, ldy, ldy2 = 2, 2048, 1537, 1032, 520
    x = bf16_normal((M, K), 5)
    w = bf16_normal((N, K), 6, 0.03)
    xd, wd = to_dev(x, device), to_dev(w, device)
    log(f"bf16 gemv split={split} M={M} K={K} N={N}")
    L, st = _lib.lib(), _lib.stream_of(xd)
    full = torch.empty((M, N), dtype=torch.bfloat16, device=device)
    _lib.check(L.qmoe_bf16_gemv(xd.data_ptr(), K, wd.data_ptr(), full.data_ptr(), N, M, K, N, st), "gemv")
    ld2 = max(ldy2, N - split)
    y2 = torch.full((M, ld2), 7.0, dtype=torch.bfloat16, device=device)
    yl = torch.full((M, max(ldy, split)), 7.0, dtype=torch.bfloat16, device=device)
    _lib.check(L.qmoe_bf16_gemv_split(xd.data_ptr(), K, wd.data_ptr(), yl.data_ptr(), yl.shape[1], y2.data_ptr(),
                                      ld2, split, M, K, N, st), "gemv split")
    torch.cuda.synchronize()
    fb = bits(full)
    assert np.array_equal(bits(yl[:, :split]), fb[:, :split])
    assert np.array_equal(bits(y2[:, :N - split]), fb[:, split:])
    assert torch.all(yl[:, split:] == 7.0) and torch.all(y2[:, N - split:] == 7.0)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [5, 64, 130, 700])
@pytest.mark.parametrize("K,N", [(2048, 1537), (512, 2048), (3072, 2049), (32, 17), (768, 3072)])
def test_bf16_linear_gemm(device, M, K, N):
    """More than four rows: the MFMA GEMM (partial row and column tiles,
    K of one chunk, the fused shared/router width of the prefill shapes)."""
    from qmoe.shared import linear
    log(f"bf16 GEMM M={M} K={K} N={N}")
    x = bf16_normal((M, K), K + M)
    w = bf16_normal((N, K), N, 0.02)
    y = linear(to_dev(x, device), to_dev(w, device))
    torch.cuda.synchronize()
    check_linear(bits(y), x, w, f"gemm M={M} K={K} N={N}")


@pytest.mark.gpu
def test_bf16_gemm_strided_rows(device):
    """Row strides of a and y wider than K and N (views of wider buffers)."""
    from qmoe import _lib
    M, K, N, lda, ldy = 200, 256, 300, 264, 304
    a = bf16_normal((M, lda), 3)
    w = bf16_normal((N, K), 4, 0.05)
    ad, wd = to_dev(a, device), to_dev(w, device)
    y = torch.full((M, ldy), 7.0, dtype=torch.bfloat16, device=device)
    _lib.check(_lib.lib().qmoe_bf16_gemm(ad.data_ptr(), lda, wd.data_ptr(), y.data_ptr(), ldy, M, K, N,
                                         _lib.stream_of(ad)), "gemm")
    torch.cuda.synchronize()
    check_linear(bits(y[:, :N]), np.ascontiguousarray(a[:, :K]), w, "strided gemm")
    assert torch.all(y[:, N:] == 7.0)                     # columns past N untouched


@pytest.mark.gpu
@pytest.mark.parametrize("b", [1, 2, 64, 300])
def test_moe_block_end_to_end(device, b):
    """Shared + router + experts: rel-L2 <= 2e-3 against the oracle's block
    fed the GPU's router logits and shared output (routing must agree)."""
    from qmoe.shared import moe_block, shared_router
    E, H, MI, gs, k = 64, 512, 256, 64, 8
    log(f"moe_block b={b} E={E} H={H} MI={MI}")
    lay = layer(E, H, MI, gs, 300 + b)
    gu_e, dn_e = layer_dev(lay, device)
    x = bf16_normal((b, H), 40 + b)
    sh_gu = bf16_normal((2 * MI + 1 + E, H), 41, 0.04)
    sh_down = bf16_normal((H, MI), 42, 0.04)
    xd, gd, dd = to_dev(x, device), to_dev(sh_gu, device), to_dev(sh_down, device)
    out = moe_block(xd, gd, dd, gu_e, dn_e, k)
    sh, gate2, logits = shared_router(xd, gd, dd, MI)
    torch.cuda.synchronize()
    sh_b, g2_b, lg_b = bits(sh), np.ascontiguousarray(bits(gate2)), np.ascontiguousarray(bits(logits))
    if b <= 4:
        ref = np.stack([O.moe_decode(x[t], lg_b[t], lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"], k,
                                     shared_bits=sh_b[t:t + 1], gate_bits=g2_b[t])["out"].reshape(-1)
                        for t in range(b)])
    else:
        ref = O.moe_prefill(x, lg_b, lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"], k,
                            shared_bits=O.shared_gate(sh_b, g2_b))["out"]
    if b <= 4:
        idx = O.router(lg_b, k)[0]
        lo, hi = zip(*(O.moe_output_interval(x[t:t + 1], idx[t:t + 1], lg_b[t:t + 1], lay["gu_w"], lay["gu_s"],
                                             lay["dn_w"], lay["dn_s"], shared_bits=sh_b[t:t + 1], gate_bits=g2_b[t])
                       for t in range(b)))
        bounds = (np.concatenate(lo), np.concatenate(hi))
    else:
        bounds = O.moe_output_interval(x, O.router(lg_b, k)[0], lg_b, lay["gu_w"], lay["gu_s"], lay["dn_w"],
                                       lay["dn_s"], shared_bits=O.shared_gate(sh_b, g2_b))
    assert_block_output(out, ref, bounds, f"moe_block b={b}")


@pytest.mark.gpu
@pytest.mark.parametrize("E,H,MI,gs,k", [(512, 2048, 512, 128, 10), (64, 512, 256, 64, 8)])
def test_moe_block_one_token_two_launches(device, E, H, MI, gs, k):
    """One token: the block in two launches (projection, then the experts
    with the shared expert's down projection in the same launch) gives the
    bits of the three-launch form (projection, shared-down GEMV, experts)."""
    from qmoe import _lib, moe_decode
    from qmoe.shared import moe_block, shared_router
    log(f"moe_block one token E={E} H={H} MI={MI}")
    lay = layer(E, H, MI, gs, 500 + E)
    gu_e, dn_e = layer_dev(lay, device)
    sh_gu = to_dev(bf16_normal((2 * MI + 1 + E, H), 51, 0.04), device)
    sh_down = to_dev(bf16_normal((H, MI), 52, 0.04), device)
    cnt = _lib.counters(device)
    for seed in (53, 54):
        x = to_dev(bf16_normal((1, H), seed), device)
        fused = moe_block(x, sh_gu, sh_down, gu_e, dn_e, k)
        sh, gate2, logits = shared_router(x, sh_gu, sh_down, MI)
        three = moe_decode(x, logits, gu_e, dn_e, k, shared=sh, shared_gate=gate2.contiguous())[0]
        torch.cuda.synchronize()
        assert torch.equal(fused.view(torch.int16), three.view(torch.int16)), f"seed {seed}"
    assert _lib.decode_status(cnt) == 0


@pytest.mark.gpu
def test_moe_block_one_token_misaligned_falls_back(device):
    """x not 16-byte aligned: the one-token block cannot take the XCD-group
    launch (QMOE_EINVAL) and runs the three launches (projection, shared-down
    GEMV, the per-pair decode launch), with their bits."""
    from qmoe import _lib, moe_decode
    from qmoe.shared import moe_block, shared_router
    E, H, MI, gs, k = 64, 512, 256, 64, 8
    lay = layer(E, H, MI, gs, 611)
    gu_e, dn_e = layer_dev(lay, device)
    sh_gu = to_dev(bf16_normal((2 * MI + 1 + E, H), 61, 0.04), device)
    sh_down = to_dev(bf16_normal((H, MI), 62, 0.04), device)
    wide = to_dev(bf16_normal((1, H + 8), 63), device)
    x_mis = wide[:, 1:H + 1]
    assert x_mis.is_contiguous() and x_mis.data_ptr() % 16 != 0
    log("moe_block one token, x misaligned")
    a = moe_block(x_mis, sh_gu, sh_down, gu_e, dn_e, k)
    sh, gate2, logits = shared_router(x_mis, sh_gu, sh_down, MI)
    b = moe_decode(x_mis, logits, gu_e, dn_e, k, shared=sh, shared_gate=gate2.contiguous())[0]
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert _lib.decode_status(_lib.counters(device)) == 0
