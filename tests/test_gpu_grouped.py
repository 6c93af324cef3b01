"""Grouped W4A16 GEMM (npu_grouped_matmul replacement) vs the oracle."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_normal, int4_words, log, scales
from oracle import qmoe_oracle as O
from parity import assert_bf16_close, assert_rounds_exactly, bits, to_dev


@pytest.mark.gpu
@pytest.mark.parametrize("counts,K,N,gs", [
    ([3, 0, 1, 0, 300, 17], 256, 384, 64),     # empty experts, a 3-tile expert, partial tiles
    ([1] * 10, 512, 2048, 128),                 # one row per expert (the diagonal decode shape)
    ([0, 0, 5], 2048, 1024, 128),
    ([128, 129], 768, 3072, 64),
    ([40] * 16, 3072, 1536, 64),
])
def test_grouped_matmul(device, counts, K, N, gs):
    from qmoe import grouped_matmul
    E = len(counts)
    log(f"grouped counts={counts[:8]} K={K} N={N} gs={gs}")
    seed = K + N + E
    ends = np.cumsum(counts).astype(np.int64)
    R = int(ends[-1])
    x = bf16_normal((R, K), seed)
    w = int4_words((E, K, N // 8), seed + 1)
    s = scales((E, K // gs, N), seed + 2)
    y = grouped_matmul([to_dev(x, device)], [to_dev(w, device)], antiquant_scale=[to_dev(s, device)],
                       group_list=to_dev(ends, device), split_item=3, group_type=0, output_dtype=torch.bfloat16)[0]
    torch.cuda.synchronize()
    assert_rounds_exactly(y, *O.grouped_gemm_exact(x, w, s, ends), f"grouped E={E} K={K} N={N}")
    assert_bf16_close(y, O.grouped_gemm(x, w, s, ends), f"grouped E={E} K={K} N={N}")


@pytest.mark.gpu
def test_grouped_matmul_row_permutation_invariance(device):
    """Each output row depends only on its own input row: permuting rows within an
    expert permutes the output rows bit for bit."""
    from qmoe import grouped_matmul
    log("grouped permutation invariance")
    counts = [70, 0, 200]
    E, K, N, gs = 3, 512, 256, 128
    ends = torch.tensor(np.cumsum(counts), dtype=torch.int64, device=device)
    x = to_dev(bf16_normal((270, K), 11), device)
    w = to_dev(int4_words((E, K, N // 8), 12), device)
    s = to_dev(scales((E, K // gs, N), 13), device)
    p = torch.cat([torch.randperm(70, generator=torch.Generator().manual_seed(1)),
                   70 + torch.randperm(200, generator=torch.Generator().manual_seed(2))]).to(device)
    y = grouped_matmul([x], [w], antiquant_scale=[s], group_list=ends, split_item=3, group_type=0)[0]
    yp = grouped_matmul([x[p].contiguous()], [w], antiquant_scale=[s], group_list=ends, split_item=3,
                        group_type=0)[0]
    torch.cuda.synchronize()
    assert torch.equal(yp.view(torch.int16), y[p].view(torch.int16))
