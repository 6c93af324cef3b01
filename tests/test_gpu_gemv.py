"""W4A16 GEMM (npu_weight_quant_batchmatmul replacement) vs the oracle."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_normal, int4_words, log, scales
from oracle import qmoe_oracle as O
from parity import assert_bf16_close, assert_rounds_exactly, to_dev

CASES = [
    (1, 2048, 4096, 128),   # the single-projection workload
    (1, 512, 2048, 128),
    (2, 256, 1024, 64),
    (3, 640, 2560, 64),     # reference down shape, g64
    (4, 2560, 1280, 64),    # reference gate_up shape, g64
    (1, 96, 32, 32),        # partial K slice and partial column tile
    (1, 3072, 1536, 64),    # one row, a tile count that is not a multiple of 8 (write-through partials)
    (1, 128, 512, 64),      # one row, a single K-slice (no partials to wait for)
    (8, 256, 256, 64),      # M > 4: MFMA path
    (130, 512, 384, 128),   # MFMA, two row tiles, partial
    (10, 2560, 2560, 64),
]


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N,gs", CASES)
def test_weight_quant_batchmatmul(device, M, K, N, gs):
    from qmoe import weight_quant_batchmatmul
    log(f"wqbm M={M} K={K} N={N} gs={gs}")
    seed = M * 7 + K + N
    x = bf16_normal((M, K), seed)
    w = int4_words((K, N // 8), seed + 1)
    s = scales((K // gs, N), seed + 2)
    y = weight_quant_batchmatmul(to_dev(x, device), to_dev(w, device), to_dev(s, device), antiquant_group_size=gs)
    torch.cuda.synchronize()
    assert_rounds_exactly(y, *O.w4a16_gemm_exact(x, w, s, gs), f"wqbm M={M} K={K} N={N} gs={gs}")
    assert_bf16_close(y, O.w4a16_gemm(x, w, s, gs), f"wqbm M={M} K={K} N={N} gs={gs}")


@pytest.mark.gpu
def test_weight_quant_batchmatmul_repeatable_and_counters_reset(device):
    """Split-K arrival counters return to zero: back-to-back calls give identical bits."""
    from qmoe import weight_quant_batchmatmul
    log("wqbm repeat")
    x = to_dev(bf16_normal((1, 2048), 3), device)
    w = to_dev(int4_words((2048, 512), 4), device)
    s = to_dev(scales((16, 4096), 5), device)
    ys = [weight_quant_batchmatmul(x, w, s, antiquant_group_size=128) for _ in range(5)]
    torch.cuda.synchronize()
    for y in ys[1:]:
        assert torch.equal(y.view(torch.int16), ys[0].view(torch.int16))


@pytest.mark.gpu
def test_weight_quant_batchmatmul_rejects_bad_shapes(device):
    from qmoe import weight_quant_batchmatmul
    x = torch.zeros((1, 256), dtype=torch.bfloat16, device=device)
    w = torch.zeros((256, 32), dtype=torch.int32, device=device)
    s = torch.zeros((2, 256), dtype=torch.bfloat16, device=device)
    with pytest.raises(RuntimeError):
        weight_quant_batchmatmul(x.view(1, 1, 256), w, s, antiquant_group_size=128)
    with pytest.raises(RuntimeError):
        weight_quant_batchmatmul(x, w, s.half(), antiquant_group_size=128)
    with pytest.raises(RuntimeError):
        weight_quant_batchmatmul(x, w, s, antiquant_group_size=64)
