"""The benchmark workloads at their full sizes on one MI355X, checked through properties that hold at any size.

The oracle's dense star is out of reach at these sizes (a 32768 x 32768 star is 4.3 GB and about 3e11 semiring
operations), so each workload is checked against what the mathematics fixes:
- MinPlus mstar, directed 32 x 32 x 32 grid (Float32, integer weights): the whole n x n star, delivered to host
  memory, satisfies C = I (+) C (x) A entry by entry, bit for bit.  With every arc weight >= 1 that equation has
  exactly one solution, the star (a finite entry not given by a path would need an infinite strictly decreasing
  chain of finite entries); path lengths are integers below 2^24, so Float32 holds every candidate exactly.  Sampled
  rows and columns also equal Dijkstra's distances bit for bit.
- MaxMin lmul! of 1024 unit columns on the n = 65536 geometric graph: sampled columns equal widest-path (bottleneck
  Dijkstra) values exactly, -Inf between components; every column equals the batched source path bit for bit.
- PlusProd rmul! of 512 unit rows on the directed 256 x 256 grid (Float64): every row x satisfies its defining
  equation x = x A + e_s to 1e-12 componentwise (relative to |x| + |x| |A|), and equals the batched source path to
  1e-12.
- MinPlus GEMM 8192^3 (Float32): a full row and column of C and sampled entries equal min(C, min_k A + B) exactly.
- 16384 batched 64 x 64 fronts: sampled fronts equal the oracle's LU and stars exactly.
"""

import heapq

import numpy as np
import pytest

import oracle as O
import pathpack_hip as P
from pathpack_hip import workloads as W

pytestmark = pytest.mark.gpu


def widest_to(g: W.Graph, s: int) -> np.ndarray:
    """Widest-path values into s: best[v] = max over paths v -> ... -> s of the smallest capacity (+Inf at s, -Inf
    where s is unreachable): bottleneck Dijkstra from s over the reversed arcs."""
    n = g.n
    # reversed arcs: for the arc v -> u (row v of column u of A) walk u -> v
    best = np.full(n, -np.inf)
    best[s] = np.inf
    colptr, rowval, w = g.colptr, g.rowval, g.nzval.astype(np.float64)
    done = np.zeros(n, dtype=bool)
    heap = [(-np.inf, s)]
    while heap:
        negb, u = heapq.heappop(heap)
        if done[u]:
            continue
        done[u] = True
        bu = -negb
        for q in range(colptr[u], colptr[u + 1]):
            v = rowval[q]
            c = min(bu, w[q])
            if c > best[v]:
                best[v] = c
                heapq.heappush(heap, (-c, v))
    return best


def minplus_fixed_point_violations(C: np.ndarray, g: W.Graph, cols: np.ndarray) -> int:
    """Entries of the columns `cols` of C with C[:, j] != min(I[:, j], min over arcs k -> j of C[:, k] + w(k -> j)),
    compared bit for bit.  Column j of the CSC matrix lists the arcs into j; the columns of the column-major C are
    the rows of its transpose, so every gather reads whole contiguous rows."""
    CT = C.T
    lo, hi = g.colptr[cols], g.colptr[cols + 1]
    q = np.concatenate([np.arange(a, b) for a, b in zip(lo, hi)]).astype(np.int64)
    G = CT[g.rowval[q], :]
    G += g.nzval[q].astype(np.float32)[:, None]   # one gathered column per arc
    starts = np.concatenate([[0], np.cumsum(hi - lo)[:-1]])
    R = np.full((cols.size, C.shape[0]), np.inf, np.float32)
    has = hi > lo
    R[has, :] = np.minimum.reduceat(G, starts[has], axis=0)
    R[np.arange(cols.size), cols] = np.minimum(R[np.arange(cols.size), cols], 0)
    return int(np.count_nonzero(R.view(np.uint32) != CT[cols, :].view(np.uint32)))


def test_config3_mstar_full_size_vs_dijkstra():
    from concurrent.futures import ThreadPoolExecutor

    g = W.config_graph(3)
    n = g.n
    print(f"MinPlus mstar n={n}", flush=True)
    C = P.mstar(P.MinPlus(), g)               # the full star, through the chunked copy to host memory
    assert C.shape == (n, n) and C.dtype == np.float32
    assert np.all(np.diag(C) == 0)
    assert g.nzval.min() >= 1
    # the whole star against its defining equation, 256 columns at a time on the host's threads
    chunks = [np.arange(j, min(n, j + 256)) for j in range(0, n, 256)]
    bad = 0
    with ThreadPoolExecutor(max_workers=8) as ex:
        for k, v in enumerate(ex.map(lambda c: minplus_fixed_point_violations(C, g, c), chunks)):
            bad += v
            if k % 32 == 31:
                print(f"  fixed point: {k + 1} of {len(chunks)} column chunks, {bad} violations", flush=True)
    assert bad == 0
    rng = np.random.default_rng(3)
    src = np.concatenate([[0, n - 1, n // 2], rng.choice(n, 5, replace=False)])
    rows = O.dijkstra_rows(g, src)           # rows: distances from each source
    assert np.array_equal(C[src, :], rows.astype(np.float32))
    gt = W.Graph(n, *_transpose(g))
    cols = O.dijkstra_rows(gt, src)          # columns: distances into each source
    assert np.array_equal(C[:, src], cols.T.astype(np.float32))


def _transpose(g: W.Graph):
    A = g.scipy().T.tocsc()
    A.sort_indices()
    return A.indptr.astype(np.int64), A.indices.astype(np.int64), A.data


def test_config4_lmul_full_size_vs_widest_paths():
    g = W.config_graph(4)
    n, nrhs = g.n, 1024
    src = (W.splitmix64(W.SEED_BASE + 4 + 100, nrhs) % np.uint64(n)).astype(np.int64)
    B = np.full((n, nrhs), -np.inf, np.float32, order="F")
    B[src, np.arange(nrhs)] = np.inf
    print(f"MaxMin lmul! n={n} nrhs={nrhs}", flush=True)
    F = P.mlu(P.MaxMin(), g)
    P.lmul_(F, B)
    # the same columns through the batched source path, bit for bit
    assert np.array_equal(P.star_cols(F, src).view(np.uint32), B.view(np.uint32))
    for k in (0, 517):
        ref = widest_to(g, int(src[k])).astype(np.float32)
        assert np.array_equal(B[:, k], ref), f"column {k} (source {src[k]})"
    assert np.isneginf(B).any()                # the geometric graph has several components


def test_config5_rmul_full_size_defining_equation():
    g = W.config_graph(5)
    n, nrhs = g.n, 512
    src = (W.splitmix64(W.SEED_BASE + 5 + 100, nrhs) % np.uint64(n)).astype(np.int64)
    B = np.zeros((nrhs, n), np.float64, order="F")
    B[np.arange(nrhs), src] = 1.0
    print(f"PlusProd rmul! n={n} nrhs={nrhs}", flush=True)
    F = P.mlu(P.PlusProd(), g)
    X = B.copy(order="F")
    P.rmul_(X, F)
    A = g.scipy().tocsr()
    # x = x A + e_s, componentwise relative to |x| + |x||A| (A >= 0, x >= 0: the bound is x + x A).  Entries decay
    # like 0.2^distance and reach the subnormal range far from the source, where only an absolute slack of 1e-300
    # (far above the subnormal rounding, far below every normal entry's 1e-12 share) is meaningful.
    XA = np.asarray((A.T @ X.T).T)
    resid = np.abs(X - XA - B)
    scale = np.abs(X) + XA
    assert np.all(resid <= 1e-12 * scale + 1e-300), float(np.max(resid / np.maximum(scale, 1e-300)))
    assert np.all(X[np.arange(nrhs), src] >= 1.0)
    Y = P.star_rows(F, src)
    assert np.all(np.abs(Y - X) <= 1e-12 * np.abs(X) + 1e-300)


def test_config2a_gemm_full_size():
    N = 8192
    seed = W.SEED_BASE + 2
    A = W.dense_minplus(N, N, seed)
    B = W.dense_minplus(N, N, seed + 10)
    C = W.dense_minplus(N, N, seed + 20)
    ctx = P.context(0)
    dA, dB, dC = P.DeviceArray.from_numpy(A), P.DeviceArray.from_numpy(B), P.DeviceArray.from_numpy(C)
    print(f"MinPlus GEMM {N}^3", flush=True)
    ctx.check(P.lib().pp_sgemx(ctx.handle, 0, 0, N, N, N, dA.ptr, N, dB.ptr, N, dC.ptr, N))
    ctx.synchronize()
    R = dC.numpy()
    i, j = 4097, 8191
    assert np.array_equal(R[i, :], np.minimum(C[i, :], np.min(A[i, :, None] + B, axis=0)))
    assert np.array_equal(R[:, j], np.minimum(C[:, j], np.min(A + B[:, j][None, :], axis=1)))
    rng = np.random.default_rng(2)
    for i, j in rng.integers(0, N, (64, 2)):
        assert R[i, j] == min(C[i, j], np.min(A[i, :] + B[:, j]))


def test_config2b_batched_fronts_full_size():
    nb, batch = 64, 16384
    seed = W.SEED_BASE + 2
    A3 = np.asfortranarray(W.dense_minplus(nb, nb * batch, seed + 30)).reshape(nb, nb, batch, order="F")
    idx = np.arange(nb)
    A3[idx, idx, :] = 0.0
    A = A3.reshape(nb, nb * batch, order="F")
    ctx = P.context(0)
    dA = P.DeviceArray.from_numpy(A)
    dL = P.DeviceArray(A.shape, np.float32)
    dU = P.DeviceArray(A.shape, np.float32)
    print(f"batched fronts {batch} x {nb}^2", flush=True)
    ctx.check(P.lib().pp_getrf_star_batched(ctx.handle, 0, 0, nb, batch, dA.ptr, dL.ptr, dU.ptr))
    ctx.synchronize()
    got = [d.numpy().reshape(nb, nb, batch, order="F") for d in (dA, dL, dU)]
    pick = np.array([0, 1, 777, 8191, 12000, batch - 1])
    # the oracle takes fronts as (batch, nb, nb) blocks holding each column-major front as A[b].T
    LU, TL, TU = O.getrf_star_batched(O.MINPLUS, np.ascontiguousarray(A3[:, :, pick].transpose(2, 1, 0)))
    for r, ref in zip(got, (LU, TL, TU)):
        assert np.array_equal(r[:, :, pick].transpose(2, 1, 0), ref)
