"""Router top-k and the GPU grouping (histogram, stable permutation) vs the oracle: bit-exact."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_normal, log
from oracle import qmoe_oracle as O
from parity import bits, to_dev


@pytest.mark.gpu
@pytest.mark.parametrize("T,E,k", [(1, 512, 10), (4, 512, 10), (37, 512, 10), (512, 512, 10), (3, 1000, 16),
                                   (5, 64, 1), (8, 40, 8)])
def test_router_topk(device, T, E, k):
    from qmoe import router_topk
    log(f"router T={T} E={E} k={k}")
    lg = bf16_normal((T, E), T * 31 + E)
    if T > 1:
        lg[1, :] = 0x3F80                   # all equal: ids 0..k-1
        lg[0, 3] = lg[0, E - 1] = 0x4200    # tie at the max: lower id first
    idx, w = router_topk(to_dev(lg, device), k)
    torch.cuda.synchronize()
    ridx, rw = O.router(lg, k)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    from parity import assert_rounds_exactly
    assert_rounds_exactly(w, O.router_weights_exact(lg, ridx), None, f"router weights T={T}")


@pytest.mark.gpu
@pytest.mark.parametrize("T,k,E,skew", [(1, 10, 512, 0), (4, 10, 512, 0), (512, 10, 512, 1), (4096, 10, 512, 0),
                                        (300, 7, 64, 1), (1000, 4, 4096, 0), (25, 10, 512, 2)])
def test_route_group(device, T, k, E, skew):
    from qmoe import route_group
    log(f"route_group T={T} k={k} E={E} skew={skew}")
    r = np.random.default_rng(T + E)
    if skew == 1:
        p = 1.0 / np.arange(1, E + 1) ** 1.1
        ids = np.stack([r.choice(E, size=k, replace=False, p=p / p.sum()) for _ in range(T)])
    elif skew == 2:
        ids = np.tile(np.arange(k), (T, 1))          # every token picks experts 0..k-1
    else:
        ids = np.stack([r.choice(E, size=k, replace=False) for _ in range(T)])
    ids = ids.astype(np.int64)
    counts, ends, order, inverse, tiles, mt = route_group(to_dev(ids, device), E, with_tiles=True)
    torch.cuda.synchronize()
    rc, re, ro, ri = O.group_routing(ids, E)
    assert np.array_equal(counts.cpu().numpy(), rc)
    assert np.array_equal(ends.cpu().numpy(), re)
    assert np.array_equal(order.cpu().numpy(), ro)
    assert np.array_equal(inverse.cpu().numpy(), ri)
    # row-tile table: every row covered once, tiles of <= 128 rows inside one expert
    t = tiles.cpu().numpy()
    n = int(t[3 * mt])
    te, t0, tr = t[:n], t[mt:mt + n], t[2 * mt:2 * mt + n]
    assert n == int(np.sum((rc + 127) // 128))
    covered = np.zeros(ids.size, dtype=np.int64)
    for e_, a, c in zip(te, t0, tr):
        assert 0 < c <= 128 and re[e_] - rc[e_] <= a and a + c <= re[e_]
        covered[a:a + c] += 1
    assert np.all(covered == 1)
    # longest first: rows never increase along the table; equal rows in expert order
    assert np.all(np.diff(tr) <= 0)
    same = np.diff(tr) == 0
    assert np.all(np.diff(te)[same] >= 0)


@pytest.mark.gpu
def test_route_group_ignores_invalid_ids(device):
    from qmoe import route_group
    log("route_group invalid ids")
    ids = np.array([[3, 9, -1], [3, 70, 1]], dtype=np.int64)
    counts, ends, order, inverse = route_group(to_dev(ids, device), 64)
    torch.cuda.synchronize()
    assert counts.cpu().numpy()[[1, 3, 9]].tolist() == [1, 2, 1] and int(counts.sum()) == 4
    inv = inverse.cpu().numpy()
    assert inv[2] == -1 and inv[4] == -1
    assert order.cpu().numpy()[:4].tolist() == [5, 0, 3, 1]
