"""The oracle: ctypes binding of the CPU restatement (libpporacle.so) plus brute-force checkers.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, and there only
as the checker (or the timed CPU baseline); the product never imports it.

Brute-force checkers, independent of the factorization:
* ``floyd_warshall``: the closure A* = I + A + A^2 + ... by Floyd-Warshall in the semiring, as the reference's own
  test does (test/core.jl:5-11), vectorized over (i, j) for each k.
* ``dijkstra_rows``: scipy's Dijkstra for MinPlus with nonnegative weights.
* ``plusprod_inverse``: (I - A)^-1 by LAPACK for PlusProd (real.jl:9-16).
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libpporacle.so")

MINPLUS, MAXPLUS, MAXMIN, MINMAX, PLUSPROD, ORAND = range(6)
F32, F64, I32 = range(3)
NAMES = {"MinPlus": MINPLUS, "MaxPlus": MAXPLUS, "MaxMin": MAXMIN, "MinMax": MINMAX, "PlusProd": PLUSPROD,
         "OrAnd": ORAND}

_lib = None


def build():
    import subprocess

    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = ctypes.CDLL(LIB)
        _lib.ppo_offd.restype = ctypes.c_int64
    return _lib


def dtype_code(dtype) -> int:
    dtype = np.dtype(dtype)
    return {np.dtype(np.float32): F32, np.dtype(np.float64): F64, np.dtype(np.int32): I32}[dtype]


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


# ===== scalar semantics (App. A of the reference's semirings) =====

def zero(s: int, dtype):
    dtype = np.dtype(dtype)
    if s == ORAND:
        return dtype.type(0)
    return dtype.type({MINPLUS: np.inf, MAXPLUS: -np.inf, MAXMIN: -np.inf, MINMAX: np.inf, PLUSPROD: 0.0}[s])


def one(s: int, dtype):
    dtype = np.dtype(dtype)
    if s == ORAND:
        return dtype.type(np.iinfo(dtype).max)
    return dtype.type({MINPLUS: 0.0, MAXPLUS: 0.0, MAXMIN: np.inf, MINMAX: -np.inf, PLUSPROD: 1.0}[s])


def plus(s: int, a, b):
    if s in (MINPLUS, MINMAX):
        return np.where(a < b, a, b)
    if s in (MAXPLUS, MAXMIN):
        return np.where(a > b, a, b)
    if s == PLUSPROD:
        return a + b
    return a | b


def times(s: int, a, b):
    with np.errstate(invalid="ignore"):
        if s in (MINPLUS, MAXPLUS):
            c = a + b
            return np.where(np.isnan(c), zero(s, np.asarray(c).dtype), c)
        if s == MAXMIN:
            return np.where(a < b, a, b)
        if s == MINMAX:
            return np.where(a > b, a, b)
        if s == PLUSPROD:
            return a * b
        return a & b


class Sym:
    """A symbolic structure in the oracle's terms (0-based): res(f) = [Rptr[f], Rptr[f+1]), sep(f) =
    Stgt[Sptr[f]:Sptr[f+1]] (sorted), perm[new] = old.  Bptr (optional): the strongly connected components in a
    topological order, component c holding the permuted vertices [Bptr[c], Bptr[c+1]); the fronts are then those of
    the diagonal blocks, and the arcs between components (N) are applied by the blocked algorithms."""

    def __init__(self, n, Rptr, Sptr, Stgt, perm, Bptr=None):
        self.n = int(n)
        self.Bptr = None if Bptr is None or len(Bptr) <= 2 else np.ascontiguousarray(Bptr, dtype=np.int64)
        self.nB = 1 if self.Bptr is None else self.Bptr.size - 1
        self.Rptr = np.ascontiguousarray(Rptr, dtype=np.int64)
        self.Sptr = np.ascontiguousarray(Sptr, dtype=np.int64)
        self.Stgt = np.ascontiguousarray(Stgt, dtype=np.int64)
        self.perm = np.ascontiguousarray(perm, dtype=np.int64)
        self.nf = self.Rptr.size - 1
        nn = np.diff(self.Rptr)
        na = np.diff(self.Sptr)
        self.nD = int((nn * nn).sum())
        self.nL = int((nn * na).sum())

    def args(self):
        return (ctypes.c_int64(self.n), ctypes.c_int64(self.nf), _p(self.Rptr), _p(self.Sptr), _p(self.Stgt),
                _p(self.perm))


class Factor:
    def __init__(self, s, sym: Sym, dtype, LD, UD, LL, UL, N=None):
        self.s, self.sym, self.dtype = s, sym, np.dtype(dtype)
        self.LD, self.UD, self.LL, self.UL = LD, UD, LL, UL
        self.N = N   # (Nptr, Nidx, Nval) of a structure with components, else None

    def _fargs(self):
        return (_p(self.LD), _p(self.UD), _p(self.LL), _p(self.UL))

    def _nargs(self):
        Nptr, Nidx, Nval = self.N
        return (ctypes.c_int64(self.sym.nB), _p(self.sym.Bptr), _p(Nptr), _p(Nidx), _p(Nval))


def _check(rc, what):
    if rc != 0:
        raise RuntimeError(f"oracle {what} failed with code {rc}")


def factor(s: int, sym: Sym, colptr, rowval, nzval, scatter_only: bool = False) -> Factor:
    """scopyto! then the multifrontal sgetrf! (chordal/sgetrf.jl)."""
    nzval = np.ascontiguousarray(nzval)
    dt = nzval.dtype
    colptr = np.ascontiguousarray(colptr, dtype=np.int64)
    rowval = np.ascontiguousarray(rowval, dtype=np.int64)
    LD = np.empty(sym.nD, dt)
    UD = np.empty(sym.nD, dt)
    LL = np.empty(sym.nL, dt)
    UL = np.empty(sym.nL, dt)
    fn = lib().ppo_scatter if scatter_only else lib().ppo_factor
    rc = fn(ctypes.c_int(s), ctypes.c_int(dtype_code(dt)), *sym.args(), _p(colptr), _p(rowval), _p(nzval),
            _p(LD), _p(UD), _p(LL), _p(UL))
    _check(rc, "factor")
    N = None
    if sym.nB > 1:
        # soffd (chordal_ssymbolic.jl:212-269): the arcs between components, by permuted column
        Nptr = np.empty(sym.n + 1, np.int64)
        cap = max(1, int(colptr[-1]))
        Nidx = np.empty(cap, np.int64)
        Nval = np.empty(cap, dt)
        cnt = lib().ppo_offd(ctypes.c_int(s), ctypes.c_int(dtype_code(dt)), *sym.args(), ctypes.c_int64(sym.nB),
                             _p(sym.Bptr), _p(colptr), _p(rowval), _p(nzval), _p(Nptr), _p(Nidx), _p(Nval))
        if cnt < 0:
            raise RuntimeError(f"oracle offd failed with code {cnt}")
        N = (Nptr, Nidx[:max(1, cnt)].copy(), Nval[:max(1, cnt)].copy())
    return Factor(s, sym, dt, LD, UD, LL, UL, N)


def rmul(F: Factor, B: np.ndarray) -> np.ndarray:
    """B (nrhs x n) <- B A*."""
    B = np.asfortranarray(B, dtype=F.dtype).copy(order="F")
    if F.N is not None:
        rc = lib().ppo_rmul_scc(ctypes.c_int(F.s), ctypes.c_int(dtype_code(F.dtype)), *F.sym.args(), *F._fargs(),
                                *F._nargs(), _p(B), ctypes.c_int64(B.shape[0]))
        _check(rc, "rmul")
        return B
    rc = lib().ppo_rmul(ctypes.c_int(F.s), ctypes.c_int(dtype_code(F.dtype)), *F.sym.args(), *F._fargs(), _p(B),
                        ctypes.c_int64(B.shape[0]))
    _check(rc, "rmul")
    return B


def lmul(F: Factor, B: np.ndarray) -> np.ndarray:
    """B (n x nrhs) <- A* B."""
    B = np.asfortranarray(B, dtype=F.dtype).copy(order="F")
    if B.ndim == 1:
        B = B.reshape(-1, 1, order="F")
    if F.N is not None:
        rc = lib().ppo_lmul_scc(ctypes.c_int(F.s), ctypes.c_int(dtype_code(F.dtype)), *F.sym.args(), *F._fargs(),
                                *F._nargs(), _p(B), ctypes.c_int64(B.shape[1]))
        _check(rc, "lmul")
        return B
    rc = lib().ppo_lmul(ctypes.c_int(F.s), ctypes.c_int(dtype_code(F.dtype)), *F.sym.args(), *F._fargs(), _p(B),
                        ctypes.c_int64(B.shape[1]))
    _check(rc, "lmul")
    return B


def lmul_t(F: Factor, B: np.ndarray) -> np.ndarray:
    """lmul!(transpose(F), B): B (n x nrhs) <- (A^T)* B, the least solution of X = A^T X (+) B.  The reference
    runs sgetrs!(P, Val(:L), Val(:T), B) (src/CPU/abstract_slu.jl:131-134, chordal_slu.jl:337-377); since
    (A^T)* = (A*)^T this is rmul!(B^T, F)^T, which the oracle computes with the same triangular sweeps."""
    B = np.asarray(B)
    if B.ndim == 1:
        B = B.reshape(-1, 1)
    return np.asfortranarray(rmul(F, np.asfortranarray(B.T)).T)


def rmul_t(F: Factor, B: np.ndarray) -> np.ndarray:
    """rmul!(B, transpose(F)): B (nrhs x n) <- B (A^T)* = (A* B^T)^T (sgetrs!(P, Val(:R), Val(:T), B))."""
    return np.asfortranarray(lmul(F, np.asfortranarray(np.asarray(B).T)).T)


def star(F: Factor, rows: tuple[int, int] | None = None, relabel: bool = True, nthreads: int = 0) -> np.ndarray:
    """Matrix(F): the full star in the original labels (n x n, column-major); ``rows`` restricts the computed rows
    of the permuted star (a timing sample), in which case ``relabel=False`` keeps the permuted labels."""
    n = F.sym.n
    r0, r1 = rows if rows is not None else (0, n)
    C = np.empty((n, n), dtype=F.dtype, order="F")
    if F.N is not None:
        if rows is not None or not relabel:
            raise ValueError("the star of a structure with components is computed whole and relabelled")
        rc = lib().ppo_star_scc(ctypes.c_int(F.s), ctypes.c_int(dtype_code(F.dtype)), *F.sym.args(), *F._fargs(),
                                *F._nargs(), _p(C), ctypes.c_int(nthreads))
        _check(rc, "star")
        return C
    rc = lib().ppo_star(ctypes.c_int(F.s), ctypes.c_int(dtype_code(F.dtype)), *F.sym.args(), *F._fargs(), _p(C),
                        ctypes.c_int64(r0), ctypes.c_int64(r1), ctypes.c_int(1 if relabel else 0),
                        ctypes.c_int(nthreads))
    _check(rc, "star")
    return C


def sgemx(s: int, A: np.ndarray, B: np.ndarray, C: np.ndarray, nthreads: int = 0) -> np.ndarray:
    """C <- C + A B over the semiring (column-major operands)."""
    A = np.asfortranarray(A)
    B = np.asfortranarray(B)
    C = np.asfortranarray(C).copy(order="F")
    m, k = A.shape
    n = B.shape[1]
    rc = lib().ppo_sgemx(ctypes.c_int(s), ctypes.c_int(dtype_code(C.dtype)), ctypes.c_int64(m), ctypes.c_int64(n),
                         ctypes.c_int64(k), _p(A), ctypes.c_int64(m), _p(B), ctypes.c_int64(k), _p(C),
                         ctypes.c_int64(m), ctypes.c_int(nthreads))
    _check(rc, "sgemx")
    return C


def getrf(s: int, A: np.ndarray) -> np.ndarray:
    """Dense sgetrf2! (no pivoting): A <- L + U with A* = U* L*."""
    A = np.asfortranarray(A).copy(order="F")
    rc = lib().ppo_getrf(ctypes.c_int(s), ctypes.c_int(dtype_code(A.dtype)), ctypes.c_int64(A.shape[0]), _p(A),
                         ctypes.c_int64(A.shape[0]))
    _check(rc, "getrf")
    return A


def getrf_star_batched(s: int, A: np.ndarray, nthreads: int = 0):
    """A: (batch, nb, nb) with each front column-major in A[b].T layout; returns (LU, TL, TU) in the same layout."""
    A = np.ascontiguousarray(A).copy()
    batch, nb, _ = A.shape
    TL = np.empty_like(A)
    TU = np.empty_like(A)
    rc = lib().ppo_getrf_star_batched(ctypes.c_int(s), ctypes.c_int(dtype_code(A.dtype)), ctypes.c_int64(nb),
                                      ctypes.c_int64(batch), _p(A), _p(TL), _p(TU), ctypes.c_int(nthreads))
    _check(rc, "getrf_star_batched")
    return A, TL, TU


def num_threads() -> int:
    return int(lib().ppo_num_threads())


# ===== brute force =====

def floyd_warshall(s: int, A: np.ndarray) -> np.ndarray:
    """test/core.jl:5-11: D = I (+) A, then D[i,j] = D[i,j] (+) D[i,k] (x) D[k,j] for k = 1..n."""
    n = A.shape[0]
    D = A.copy()
    d = np.arange(n)
    D[d, d] = plus(s, D[d, d], np.full(n, one(s, A.dtype), dtype=A.dtype))
    for k in range(n):
        D = plus(s, D, times(s, D[:, k:k + 1], D[k:k + 1, :]))
    return D


def dijkstra_rows(graph, sources=None) -> np.ndarray:
    """MinPlus rows of A* by Dijkstra (nonnegative weights), in float64."""
    from scipy.sparse.csgraph import dijkstra

    return dijkstra(graph.scipy().astype(np.float64), directed=True, indices=sources)


def plusprod_inverse(A: np.ndarray) -> np.ndarray:
    """(I - A)^-1 (the PlusProd star of A when the series converges)."""
    n = A.shape[0]
    return np.linalg.inv(np.eye(n) - A)
