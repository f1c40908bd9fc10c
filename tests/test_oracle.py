"""The oracle, pinned: the reference's own factors, its README answers, its test graphs against Floyd-Warshall, and
closed forms (Dijkstra, (I - A)^-1, the star of a dense LU).  CPU only."""

import numpy as np
import pytest

import oracle as O
import site_fixtures as SF
from helpers import assert_star_equal, bits, dtype_for, oracle_sym, weighted
import pathpack_hip as P
from pathpack_hip import workloads as W


def fixture_D(F: O.Factor) -> np.ndarray:
    """The fixture's D: upper triangle and diagonal of UDval, strict lower triangle of LDval (site_factors.jl:162-170)."""
    nn = np.diff(F.sym.Rptr)
    Dp = np.concatenate([[0], np.cumsum(nn * nn)])
    D = np.empty_like(F.LD)
    for f in range(F.sym.nf):
        k = nn[f]
        blk = slice(Dp[f], Dp[f + 1])
        ud = F.UD[blk].reshape(k, k, order="F")
        ld = F.LD[blk].reshape(k, k, order="F")
        D[blk] = np.where(np.triu(np.ones((k, k), bool)), ud, ld).ravel(order="F")
    return D


@pytest.mark.parametrize("name", ["paris", "bunny"])
def test_oracle_reproduces_reference_factors(name):
    """mlu(MinPlus(), A) in Float32 with the reference's ordering and fronts equals the reference's factor bit for bit
    (docs/site_factors.jl wrote it; non-integer weights, so this pins the LU's arithmetic, not just its algebra)."""
    n, cp, rv, nz = SF.graph_csc(name)
    fx = SF.factor_fixture(name)
    sym = O.Sym(n, fx["Rptr"], fx["Sptr"], fx["Stgt"], fx["perm"])
    F = O.factor(O.MINPLUS, sym, cp, rv, nz)
    assert np.array_equal(bits(fixture_D(F)), bits(fx["D"]))
    assert np.array_equal(bits(F.UL), bits(fx["UL"]))
    assert np.array_equal(bits(F.LL), bits(fx["LL"]))


def test_oracle_fixture_rows_match_dijkstra():
    """rmul! rows of the reference's Paris factor are shortest-path distances (site_factors_test.mjs:77-91 checks the
    same against Dijkstra to Float32 rounding)."""
    n, cp, rv, nz = SF.graph_csc("paris")
    fx = SF.factor_fixture("paris")
    F = O.factor(O.MINPLUS, O.Sym(n, fx["Rptr"], fx["Sptr"], fx["Stgt"], fx["perm"]), cp, rv, nz)
    srcs = np.array([0, n - 1, 1, n - 2, 4321])
    B = np.full((srcs.size, n), np.inf, np.float32)
    B[np.arange(srcs.size), srcs] = 0
    R = O.rmul(F, B)
    D = O.dijkstra_rows(W.Graph(n, cp, rv, nz), srcs)
    assert np.all(np.isfinite(R) == np.isfinite(D))
    fin = np.isfinite(D)
    assert np.max(np.abs(R[fin] - D[fin]) / np.maximum(D[fin], 1e-30)) < 4e-6


@pytest.mark.parametrize("n,p,seed", [(40, 0.08, 1), (150, 0.02, 2), (300, 0.01, 3)])
@pytest.mark.parametrize("s", [O.MINPLUS, O.MAXPLUS, O.MAXMIN, O.MINMAX, O.ORAND, O.PLUSPROD])
def test_oracle_star_vs_floyd_warshall(n, p, seed, s):
    """The reference's CPU test (test/core.jl:13-20): mstar of random directed graphs against Floyd-Warshall, here for
    all six semirings, with the product's symbolic structure (amalgamated and fundamental)."""
    dtype = dtype_for(s)
    g = weighted(W.random_digraph(n, p, seed), s, dtype)
    ref = O.plusprod_inverse(g.dense(0.0)) if s == O.PLUSPROD else O.floyd_warshall(s, g.dense(O.zero(s, dtype)))
    for amalg in (True, False):
        sym = P.symbolic(g, amalgamate=amalg)
        C = O.star(O.factor(s, oracle_sym(sym), g.colptr, g.rowval, g.nzval))
        assert_star_equal(s, C, ref)


DAG_LIKE = {
    "layered": lambda: W.layered_digraph(6, (8, 6), fwd=0.5, seed=3),   # a chain of six strongly connected layers
    "dag": lambda: W.random_dag(150, 0.04, 9),                          # 150 components of one vertex
}


@pytest.mark.parametrize("name", list(DAG_LIKE))
@pytest.mark.parametrize("s", [O.MINPLUS, O.MAXPLUS, O.MAXMIN, O.MINMAX, O.ORAND, O.PLUSPROD])
def test_oracle_star_of_dag_like_graphs(name, s):
    """Graphs whose strongly connected components form a chain or a deep DAG: the blocked star and solves over the
    components (blocked/sgetri.jl, blocked/sgetrs.jl; N applied between them) against Floyd-Warshall / (I - A)^-1,
    with the amalgamated and the fundamental structure."""
    dtype = dtype_for(s)
    g = weighted(DAG_LIKE[name](), s, dtype)
    ref = O.plusprod_inverse(g.dense(0.0)) if s == O.PLUSPROD else O.floyd_warshall(s, g.dense(O.zero(s, dtype)))
    for amalg in (True, False):
        sym = P.symbolic(g, amalgamate=amalg)
        assert sym.components()["nB"] > 5 and sym.components()["Nptr"][-1] > 0
        F = O.factor(s, oracle_sym(sym), g.colptr, g.rowval, g.nzval)
        assert_star_equal(s, O.star(F), ref)
        I = np.full((g.n, g.n), O.zero(s, dtype), dtype=dtype)
        np.fill_diagonal(I, O.one(s, dtype))
        assert_star_equal(s, O.rmul(F, I), ref)
        assert_star_equal(s, O.lmul(F, I), ref)


@pytest.mark.parametrize("s", [O.MINPLUS, O.MAXMIN, O.ORAND, O.PLUSPROD])
def test_oracle_star_of_disconnected_graph(s):
    """Eleven components (grids, a random digraph, a geometric graph, isolated vertices) with interleaved labels:
    entries between components are the semiring zero."""
    dtype = dtype_for(s)
    g = weighted(W.disjoint_union([W.grid((9, 7)), W.random_digraph(60, 0.05, 4), W.rgg(200, seed=5),
                                   W.grid((3, 4, 2))], isolated=5), s, dtype)
    ref = O.plusprod_inverse(g.dense(0.0)) if s == O.PLUSPROD else O.floyd_warshall(s, g.dense(O.zero(s, dtype)))
    sym = P.symbolic(g)
    C = O.star(O.factor(s, oracle_sym(sym), g.colptr, g.rowval, g.nzval))
    assert_star_equal(s, C, ref)


def readme_graph():
    """sparse([1, 1, 2, 3, 4, 4], [2, 3, 4, 2, 1, 5], [3.0, 8.0, 1.0, 4.0, 2.0, 7.0], 5, 5) (README.md:73)."""
    return W.from_arcs(5, np.array([1, 1, 2, 3, 4, 4]) - 1, np.array([2, 3, 4, 2, 1, 5]) - 1,
                       np.array([3.0, 8.0, 1.0, 4.0, 2.0, 7.0]))


def test_readme_known_answers():
    """README.md:83-128: mstar over MinPlus and MaxMin, lmul! of the unit vector at vertex 5, rmul! of the unit row at
    vertex 1."""
    g = readme_graph()
    assert g.dense(0.0)[0, 1] == 3.0 and g.dense(0.0)[3, 4] == 7.0
    inf = np.inf
    minplus = np.array([[0, 3, 8, 4, 11], [3, 0, 11, 1, 8], [7, 4, 0, 5, 12], [2, 5, 10, 0, 7],
                        [inf, inf, inf, inf, 0]], float)
    maxmin = np.array([[inf, 4, 8, 1, 1], [1, inf, 1, 1, 1], [1, 4, inf, 1, 1], [2, 2, 2, inf, 7],
                       [-inf, -inf, -inf, -inf, inf]], float)
    sym = P.symbolic(g)
    F = O.factor(O.MINPLUS, oracle_sym(sym), g.colptr, g.rowval, g.nzval)
    assert np.array_equal(O.star(F), minplus)
    b = np.full(5, inf)
    b[4] = 0
    assert np.array_equal(O.lmul(F, b)[:, 0], [11, 8, 12, 7, 0])
    B = np.full((1, 5), inf)
    B[0, 0] = 0
    assert np.array_equal(O.rmul(F, B)[0], [0, 3, 8, 4, 11])
    Fm = O.factor(O.MAXMIN, oracle_sym(sym), g.colptr, g.rowval, g.nzval)
    assert np.array_equal(O.star(Fm), maxmin)


def test_three_cycle_label_convention():
    """D[i, j] = A*[i, j] is the path i -> j (test/gpu/test_api.jl:105-115): arcs 1->2 (1), 2->3 (2), 3->1 (4)."""
    g = W.from_arcs(3, np.array([0, 1, 2]), np.array([1, 2, 0]), np.array([1.0, 2.0, 4.0], np.float32))
    sym = P.symbolic(g)
    C = O.star(O.factor(O.MINPLUS, oracle_sym(sym), g.colptr, g.rowval, g.nzval))
    assert np.array_equal(C, np.array([[0, 1, 3], [6, 0, 2], [4, 5, 0]], np.float32))


def test_grid_minplus_vs_dijkstra():
    """Configuration 1 (64 x 64 directed grid, Float64): the full star equals Dijkstra exactly (integer weights)."""
    g = W.config_graph(1)
    sym = P.symbolic(g)
    C = O.star(O.factor(O.MINPLUS, oracle_sym(sym), g.colptr, g.rowval, g.nzval))
    assert np.array_equal(C, O.dijkstra_rows(g))


ALL = [O.MINPLUS, O.MAXPLUS, O.MAXMIN, O.MINMAX, O.PLUSPROD, O.ORAND]


def semiring_matmul(s, A, B):
    """A (x) B over the semiring by brute force (numpy broadcasting; PlusProd by BLAS)."""
    if s == O.PLUSPROD:
        return A @ B
    C = np.full((A.shape[0], B.shape[1]), O.zero(s, A.dtype), dtype=A.dtype)
    for k in range(A.shape[1]):
        C = O.plus(s, C, O.times(s, A[:, k:k + 1], B[k:k + 1, :]))
    return C


def dense_rhs(s, dtype, shape, rng):
    if s == O.ORAND:
        return rng.integers(0, 128, shape).astype(np.int32)
    if s == O.PLUSPROD:
        return rng.random(shape).astype(dtype)
    B = rng.integers(0, 50, shape).astype(dtype)
    B[rng.random(shape) < 0.3] = O.zero(s, dtype)
    return B


@pytest.mark.parametrize("s", ALL)
def test_solves_are_rows_and_columns_of_the_star(s):
    """lmul!(F, I) and rmul!(I, F) are the star itself (abstract_slu.jl:123-145: B <- A* B, B <- B A*), and for dense
    right-hand sides lmul!(F, B) = A* (x) B and rmul!(B, F) = B (x) A*, with the star pinned against Floyd-Warshall
    or (I - A)^-1 and the products computed by brute force; all six semirings."""
    dtype = dtype_for(s)
    g = weighted(W.random_digraph(120, 0.03, 5), s, dtype)
    sym = P.symbolic(g)
    F = O.factor(s, oracle_sym(sym), g.colptr, g.rowval, g.nzval)
    C = O.star(F)
    ref = O.plusprod_inverse(g.dense(0.0)) if s == O.PLUSPROD else O.floyd_warshall(s, g.dense(O.zero(s, dtype)))
    assert_star_equal(s, C, ref)
    I = np.full((g.n, g.n), O.zero(s, dtype), dtype=dtype)
    np.fill_diagonal(I, O.one(s, dtype))
    assert_star_equal(s, O.rmul(F, I), C)
    assert_star_equal(s, O.lmul(F, I), C)
    rng = np.random.default_rng(s)
    B = dense_rhs(s, dtype, (g.n, 7), rng)
    assert_star_equal(s, O.lmul(F, B), semiring_matmul(s, ref, B))
    Bt = np.asfortranarray(dense_rhs(s, dtype, (5, g.n), rng))
    assert_star_equal(s, O.rmul(F, Bt), semiring_matmul(s, Bt, ref))
    # transposed solves (lmul!/rmul! with transpose(F)): (A^T)* B and B (A^T)*, against the star's transpose
    refT = np.ascontiguousarray(ref.T)
    assert_star_equal(s, O.lmul_t(F, B), semiring_matmul(s, refT, B))
    assert_star_equal(s, O.rmul_t(F, Bt), semiring_matmul(s, Bt, refT))


@pytest.mark.parametrize("s", ALL)
def test_dense_sgemx_vs_brute_force(s):
    """sgemx!: C <- C (+) A (x) B (dense/sgemx.jl:606-635) against a brute-force loop over k for every semiring, and
    PlusProd against BLAS (A B + C)."""
    rng = np.random.default_rng(0)
    dtype = dtype_for(s, np.float32 if s != O.PLUSPROD else np.float64)
    if s == O.ORAND:
        A, B, C = (rng.integers(0, 2 ** 20, sh).astype(np.int32) for sh in ((37, 19), (19, 23), (37, 23)))
    elif s == O.PLUSPROD:
        A, B, C = (rng.random(sh) for sh in ((37, 19), (19, 23), (37, 23)))
    else:
        A = rng.integers(0, 1000, (37, 19)).astype(dtype)
        B = rng.integers(0, 1000, (19, 23)).astype(dtype)
        C = rng.integers(0, 3000, (37, 23)).astype(dtype)
        A[rng.random(A.shape) < 0.1] = O.zero(s, dtype)
        B[rng.random(B.shape) < 0.1] = O.zero(s, dtype)
    got = O.sgemx(s, A, B, C)
    if s == O.PLUSPROD:
        ref = A @ B + C
        assert np.max(np.abs(got - ref) / np.abs(ref)) < 1e-14
        return
    ref = O.plus(s, C, semiring_matmul(s, A, B))
    assert np.array_equal(bits(got), bits(ref))
    # the same with every (x) spelled out for MinPlus / MaxMin
    if s == O.MINPLUS:
        assert np.array_equal(got, np.minimum(C, (A[:, :, None] + B[None, :, :]).min(axis=1)))
    if s == O.MAXMIN:
        assert np.array_equal(got, np.maximum(C, np.minimum(A[:, :, None], B[None, :, :]).max(axis=1)))


@pytest.mark.parametrize("s", ALL)
def test_getrf_star_gives_the_closure(s):
    """A* = U* L* for a dense front: the semiring product of the batched kernel's TU and TL is Floyd-Warshall's
    closure of A (dense/sgetrf.jl:151-175; batched/sgetrf.jl:11-120); for PlusProd it is (I - A)^-1, and MaxPlus
    takes nonpositive weights (no positive cycle)."""
    dtype = dtype_for(s, np.float32 if s != O.PLUSPROD else np.float64)
    rng = np.random.default_rng(1)
    nb, batch = 24, 3
    if s == O.ORAND:
        A = rng.integers(0, 64, (batch, nb, nb)).astype(np.int32)
    elif s == O.PLUSPROD:
        A = rng.random((batch, nb, nb)) * (0.9 / nb)
    else:
        A = rng.integers(0, 1000, (batch, nb, nb)).astype(dtype)
        if s == O.MAXPLUS:
            A = -A
        A[rng.random(A.shape) < 0.1] = O.zero(s, dtype)
        if s in (O.MINPLUS, O.MAXPLUS):
            A[:, np.arange(nb), np.arange(nb)] = 0
    LU, TL, TU = O.getrf_star_batched(s, A)
    for b in range(batch):
        a = A[b].T   # each front is column-major: element (i, j) at A[b][j, i]
        tu, tl = TU[b].T, TL[b].T
        prod = semiring_matmul(s, tu, tl)
        if s == O.PLUSPROD:
            assert_star_equal(s, prod, O.plusprod_inverse(a), rtol=1e-12)
        else:
            assert np.array_equal(bits(prod), bits(O.floyd_warshall(s, a)))


def test_plusprod_grid_vs_inverse():
    g = W.grid_float((12, 12), 0.2, np.float64, seed=99)
    sym = P.symbolic(g)
    C = O.star(O.factor(O.PLUSPROD, oracle_sym(sym), g.colptr, g.rowval, g.nzval))
    assert_star_equal(O.PLUSPROD, C, O.plusprod_inverse(g.dense(0.0)), rtol=1e-12)


def dense_matrix(s, dtype, n, rng, zeros=0.6):
    """A dense n x n matrix with weights suited to s and a share of semiring zeros (no arc)."""
    if s == O.ORAND:
        A = rng.integers(1, 128, (n, n)).astype(np.int32)
    elif s == O.PLUSPROD:
        A = (rng.random((n, n)) * (0.9 / max(1, n))).astype(dtype)
    elif s == O.MAXPLUS:
        A = (-rng.integers(1, 101, (n, n))).astype(dtype)
    else:
        A = rng.integers(1, 101, (n, n)).astype(dtype)
    A[rng.random((n, n)) < zeros] = O.zero(s, A.dtype)
    return np.asfortranarray(A)


def dense_pattern(A):
    """A dense matrix as the stored entries of a one-front structure in its own order (every entry stored)."""
    n = A.shape[0]
    cp = np.arange(0, n * n + 1, n, dtype=np.int64)
    rv = np.tile(np.arange(n, dtype=np.int64), n)
    sym = O.Sym(n, [0, n] if n else [0], [0, 0] if n else [0], np.zeros(0, np.int64), np.arange(n))
    return sym, cp, rv, np.asfortranarray(A).ravel(order="F")


@pytest.mark.parametrize("s", ALL)
def test_dense_lu_factors_the_closure(s):
    """The dense LU (DenseSLU, dense/sgetrf.jl:5-175): A <- L + U with A* = U* L*, L unit lower.  The stars of the two
    triangles are taken by Floyd-Warshall (by (I - T)^-1 for PlusProd), and the one-front multifrontal factor of the
    same matrix is the same LU."""
    rng = np.random.default_rng(100 + s)
    dtype = dtype_for(s)
    n = 37
    A = dense_matrix(s, dtype, n, rng)
    LU = O.getrf(s, A)
    z = O.zero(s, LU.dtype)
    U = np.where(np.triu(np.ones((n, n), bool)), LU, z).astype(LU.dtype)
    L = np.where(np.tril(np.ones((n, n), bool), -1), LU, z).astype(LU.dtype)
    if s == O.PLUSPROD:
        I = np.eye(n)
        got = np.linalg.inv(I - U) @ np.linalg.inv(I - L)
        assert np.allclose(got, O.plusprod_inverse(A), rtol=1e-12, atol=0)
    else:
        got = semiring_matmul(s, O.floyd_warshall(s, U), O.floyd_warshall(s, L))
        assert np.array_equal(got, O.floyd_warshall(s, A))
    sym, cp, rv, nz = dense_pattern(A)
    Fo = O.factor(s, sym, cp, rv, nz)
    assert_star_equal(s, Fo.LD.reshape(n, n, order="F"), LU)
