"""pathpack_hip: PATHPACK.jl's multifrontal semiring LU on one MI355X.

The host-side mirror of the reference's CPU API (src/CPU/abstract_slu.jl), over the C ABI of libpathpack_hip.so:

    F = mlu(MinPlus(), A)        # abstract_slu.jl:44-58   ordering + symbolic on the host, factorization on the GPU
    C = Matrix(F)                # abstract_slu.jl:10-14   the full star A* (n x n, original labels)
    D = mstar(MinPlus(), A)      # abstract_slu.jl:81-87   Matrix(mlu(s, A))
    lmul_(F, B)                  # lmul!(F, B), :131-134    B <- A* B  (columns of the star)
    rmul_(B, F)                  # rmul!(B, F), :142-145    B <- B A*  (rows of the star)

Python has no ``!`` in names, so ``lmul!``/``rmul!`` are ``lmul_``/``rmul_`` (the in-place convention of torch).
``A`` is a square sparse matrix (scipy.sparse, or ``(n, colptr, rowval, nzval)``, or a ``workloads.Graph``) with
``A[i, j]`` the weight of the arc i -> j, or a dense numpy array (one dense front, as the reference's DenseSLU).  The
element type follows the values, as ``ChordalSLU{Sem, T}`` does: float32 / float64, int32 for OrAnd.  Host arrays
come back as numpy arrays; ``device=True`` keeps results in HBM as ``DeviceArray`` buffers owned by the library
(torch is not used on the device path: it ships its own HIP runtime, and one process cannot drive the GPU through
two runtimes).
"""

from __future__ import annotations

import ctypes
import threading

import numpy as np

from . import _lib
from ._lib import (PathpackArgumentError, PathpackDeviceError, PathpackError, PathpackMemoryError,
                   PathpackUnsupportedError, check, lib)

__all__ = [
    "AbstractSemiring", "MinPlus", "MaxPlus", "MaxMin", "MinMax", "PlusProd", "OrAnd",
    "szero", "sone", "mlu", "lu_", "mstar", "lmul_", "rmul_", "transpose", "adjoint", "Matrix", "star_rows", "star_cols", "Factorization", "Symbolic", "symbolic",
    "DenseFactorization", "dense_mlu", "sgetrf_",
    "Context", "context", "DeviceArray", "PathpackError", "PathpackArgumentError", "PathpackMemoryError",
    "PathpackUnsupportedError", "PathpackDeviceError",
]

F32, F64, I32 = 0, 1, 2


# ===== semirings (src/CPU/semiring/*.jl) =====

class AbstractSemiring:
    id = -1
    name = ""
    integral = False

    def __repr__(self):
        return f"{self.name}()"

    def __eq__(self, other):
        return type(self) is type(other)

    def __hash__(self):
        return hash(self.id)


class MinPlus(AbstractSemiring):
    """([-Inf, Inf], min, +): shortest paths (tropical.jl:15)."""
    id, name = 0, "MinPlus"


class MaxPlus(AbstractSemiring):
    """([-Inf, Inf], max, +): longest paths (tropical.jl:31)."""
    id, name = 1, "MaxPlus"


class MaxMin(AbstractSemiring):
    """([-Inf, Inf], max, min): widest paths (bottleneck.jl:31)."""
    id, name, integral = 2, "MaxMin", True


class MinMax(AbstractSemiring):
    """([-Inf, Inf], min, max): minimax paths (bottleneck.jl:15)."""
    id, name, integral = 3, "MinMax", True


class PlusProd(AbstractSemiring):
    """([0, Inf], +, *): walk sums (I - A)^-1 (real.jl:16)."""
    id, name = 4, "PlusProd"


class OrAnd(AbstractSemiring):
    """(2^n, |, &) on int32 bit sets: label reachability (boolean.jl:31)."""
    id, name, integral = 5, "OrAnd", True


def szero(s: AbstractSemiring, dtype):
    """The semiring zero as a value of ``dtype`` (szero, semiring.jl:54-59)."""
    dtype = np.dtype(dtype)
    if isinstance(s, OrAnd):
        return dtype.type(0)
    return dtype.type({0: np.inf, 1: -np.inf, 2: -np.inf, 3: np.inf, 4: 0.0}[s.id])


def sone(s: AbstractSemiring, dtype):
    """The semiring one as a value of ``dtype`` (sone, semiring.jl:61-66)."""
    dtype = np.dtype(dtype)
    if isinstance(s, OrAnd):
        return dtype.type(np.iinfo(dtype).max)
    return dtype.type({0: 0.0, 1: 0.0, 2: np.inf, 3: -np.inf, 4: 1.0}[s.id])


def _dtype_code(dtype) -> int:
    dtype = np.dtype(dtype)
    if dtype == np.float32:
        return F32
    if dtype == np.float64:
        return F64
    if dtype == np.int32:
        return I32
    raise PathpackUnsupportedError(_lib.PP_EUNSUPPORTED, f"element type {dtype} is not supported")


def _p(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


# ===== device context =====

class Context:
    """One HIP stream on one device (pp_ctx)."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        check(lib().pp_init(ctypes.byref(h), int(device)))
        self.handle = h
        self.device = int(device)

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            lib().pp_destroy(h)
            self.handle = None

    def check(self, status: int):
        check(status, self.handle)

    def synchronize(self):
        self.check(lib().pp_synchronize(self.handle))

    def set_timing(self, on: bool):
        self.check(lib().pp_set_timing(self.handle, 1 if on else 0))

    def set_poison(self, on: bool):
        """Fill every sweep buffer with NaN (-1 for OrAnd) before the sweeps (pp_set_debug, PP_DEBUG_POISON)."""
        self.check(lib().pp_set_debug(self.handle, 1 if on else 0))

    def timing(self) -> np.ndarray:
        t = (ctypes.c_double * 8)()
        self.check(lib().pp_get_timing(self.handle, t))
        return np.array(t[:])


_contexts: dict[int, Context] = {}
_ctx_lock = threading.Lock()


def context(device: int = 0) -> Context:
    """The shared context of a device (created on first use)."""
    with _ctx_lock:
        if device not in _contexts:
            _contexts[device] = Context(device)
        return _contexts[device]


# ===== device buffers =====

class DeviceArray:
    """A column-major array in HBM allocated through the library (pp_buffer_alloc).  ``DeviceArray.from_numpy``
    uploads, ``numpy()`` downloads; ``ptr`` is the device address."""

    def __init__(self, shape, dtype, ctx: Context | None = None):
        self.ctx = ctx or context(0)
        self.shape = tuple(int(x) for x in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        h = ctypes.c_void_p()
        self.ctx.check(lib().pp_buffer_alloc(self.ctx.handle, max(1, self.nbytes), ctypes.byref(h)))
        self.ptr = h.value

    @classmethod
    def from_numpy(cls, a: np.ndarray, ctx: Context | None = None) -> "DeviceArray":
        d = cls(a.shape, a.dtype, ctx)
        d.upload(a)
        return d

    def upload(self, a: np.ndarray):
        a = np.asfortranarray(a, dtype=self.dtype)
        if a.shape != self.shape:
            raise PathpackArgumentError(_lib.PP_EINVAL, "shape mismatch")
        self.ctx.check(lib().pp_upload(self.ctx.handle, ctypes.c_void_p(self.ptr), _p(a), self.nbytes))

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype, order="F")
        self.ctx.check(lib().pp_download(self.ctx.handle, _p(out), ctypes.c_void_p(self.ptr), self.nbytes))
        return out

    def __del__(self):
        p = getattr(self, "ptr", None)
        if p:
            lib().pp_buffer_free(self.ctx.handle, ctypes.c_void_p(p))
            self.ptr = None


# ===== sparse input =====

def _as_csc(A):
    """(n, colptr int64, rowval int64, nzval) of a square sparse matrix, canonical (sorted, no duplicates)."""
    if hasattr(A, "colptr") and hasattr(A, "rowval"):
        return int(A.n), np.ascontiguousarray(A.colptr, np.int64), np.ascontiguousarray(A.rowval, np.int64), \
            np.ascontiguousarray(A.nzval)
    if isinstance(A, tuple) and len(A) == 4:
        n, cp, rv, nz = A
        return int(n), np.ascontiguousarray(cp, np.int64), np.ascontiguousarray(rv, np.int64), np.ascontiguousarray(nz)
    try:
        import scipy.sparse as sp
    except ImportError:  # pragma: no cover
        sp = None
    if sp is not None and sp.issparse(A):
        if A.shape[0] != A.shape[1]:
            raise PathpackArgumentError(_lib.PP_EINVAL, "the matrix must be square")
        M = sp.csc_matrix(A, copy=True)
        M.sort_indices()
        cp = M.indptr.astype(np.int64)
        rv = M.indices.astype(np.int64)
        dup = (np.diff(rv) == 0) & (np.repeat(np.arange(M.shape[1]), np.diff(cp))[1:] ==
                                    np.repeat(np.arange(M.shape[1]), np.diff(cp))[:-1])
        if dup.any():
            raise PathpackArgumentError(_lib.PP_EINVAL, "duplicate entries: combine parallel arcs with the semiring's "
                                                        "(+) before the call")
        return int(M.shape[0]), cp, rv, np.ascontiguousarray(M.data)
    raise PathpackArgumentError(_lib.PP_EINVAL, f"unsupported matrix type {type(A)}")


# ===== symbolic analysis =====

class Symbolic:
    """Ordering, supernodal elimination tree and separators of a pattern (pp_sym; ssymbolic,
    chordal_ssymbolic.jl:26-57).  Host only."""

    def __init__(self, handle: ctypes.c_void_p, n: int, nnz: int, colptr=None, rowval=None):
        self.handle = handle
        self.n = n
        self.nnz = nnz
        # the pattern, kept to check that later values (mlu(..., sym=), lu_) belong to it
        self._colptr = None if colptr is None else np.array(colptr, np.int64)
        self._rowval = None if rowval is None else np.array(rowval, np.int64)
        nn = ctypes.c_int64()
        nf = ctypes.c_int64()
        ns = ctypes.c_int64()
        mf = ctypes.c_int64()
        check(lib().pp_sym_size(handle, ctypes.byref(nn), ctypes.byref(nf), ctypes.byref(ns), ctypes.byref(mf)))
        self.nf = nf.value
        self.nstgt = ns.value
        self.maxfront = mf.value
        self._export = None

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            lib().pp_sym_destroy(h)
            self.handle = None

    def export(self) -> dict:
        """perm (new -> old), Rptr, Sptr, Stgt, parent, all 0-based."""
        if self._export is None:
            perm = np.empty(self.n, np.int64)
            R = np.empty(self.nf + 1, np.int64)
            S = np.empty(self.nf + 1, np.int64)
            T = np.empty(max(1, self.nstgt), np.int64)
            P = np.empty(max(1, self.nf), np.int64)
            check(lib().pp_sym_export(self.handle, _p(perm), _p(R), _p(S), _p(T), _p(P)))
            self._export = {"perm": perm, "Rptr": R, "Sptr": S, "Stgt": T[:self.nstgt], "parent": P[:self.nf]}
        return self._export

    def components(self) -> dict:
        """The strongly connected components in a topological order (sccs, soffd; chordal_ssymbolic.jl:26-57,
        212-269): nB, Bptr (component c holds the permuted vertices [Bptr[c], Bptr[c+1])), and N, the arcs between
        components by permuted column: Nptr (n + 1), Nidx (permuted rows), Nsrc (positions in the analysed nzval)."""
        nB, nN = ctypes.c_int64(), ctypes.c_int64()
        check(lib().pp_sym_components(self.handle, ctypes.byref(nB), None, ctypes.byref(nN), None, None, None))
        B = np.empty(nB.value + 1, np.int64)
        Np = np.empty(self.n + 1, np.int64)
        Ni = np.empty(max(1, nN.value), np.int64)
        Ns = np.empty(max(1, nN.value), np.int64)
        check(lib().pp_sym_components(self.handle, None, _p(B), None, _p(Np), _p(Ni), _p(Ns)))
        return {"nB": nB.value, "Bptr": B, "Nptr": Np, "Nidx": Ni[:nN.value], "Nsrc": Ns[:nN.value]}

    def check_pattern(self, n: int, colptr, rowval):
        """PathpackArgumentError unless (n, colptr, rowval) is the analysed pattern."""
        same = n == self.n and len(rowval) == self.nnz
        if same and self._colptr is not None:
            same = np.array_equal(colptr, self._colptr) and np.array_equal(rowval, self._rowval)
        if not same:
            raise PathpackArgumentError(_lib.PP_EINVAL, "the matrix does not have the pattern of the analysis; "
                                                        "analyse it again")

    def stats(self) -> dict:
        st = (ctypes.c_double * 10)()
        check(lib().pp_sym_stats(self.handle, st))
        keys = ["madds_factor_alg", "madds_star_alg", "madds_rhs_alg", "nnzL_alg", "madds_factor", "madds_star",
                "madds_rhs", "nnzL", "seconds_order", "seconds_total"]
        return dict(zip(keys, st[:]))


_ALGS = {None: 0, "nd": 0, "ND": 0, "natural": 1, "amd": 3, "AMD": 3, "auto": 4}


def symbolic(A, alg=None, amalgamate: bool = True) -> Symbolic:
    """Symbolic analysis of the pattern of A.  ``alg``: None / "nd" (nested dissection), "amd" (approximate minimum
    degree), "auto" (both, keeping the order with the smaller factor), "natural", or a permutation (0-based,
    perm[new] = old) -- the reference's ``alg`` keyword (abstract_slu.jl:44)."""
    n, cp, rv, _ = _as_csc(A)
    h = ctypes.c_void_p()
    if isinstance(alg, (str, type(None))):
        if alg not in _ALGS:
            raise PathpackArgumentError(_lib.PP_EINVAL, f"unknown ordering {alg!r}")
        check(lib().pp_symbolic(n, _p(cp), _p(rv), _ALGS[alg], 1 if amalgamate else 0, None, ctypes.byref(h)))
    else:
        perm = np.ascontiguousarray(alg, np.int64)
        if perm.shape != (n,):
            raise PathpackArgumentError(_lib.PP_EINVAL, "the permutation must have n entries")
        check(lib().pp_symbolic(n, _p(cp), _p(rv), 2, 1 if amalgamate else 0, _p(perm), ctypes.byref(h)))
    return Symbolic(h, n, int(cp[-1]), cp, rv)


def symbolic_given(A, perm, Rptr) -> Symbolic:
    """The structure for a given permutation and partition into fronts (e.g. the reference's own)."""
    n, cp, rv, _ = _as_csc(A)
    perm = np.ascontiguousarray(perm, np.int64)
    Rptr = np.ascontiguousarray(Rptr, np.int64)
    h = ctypes.c_void_p()
    check(lib().pp_symbolic_given(n, _p(cp), _p(rv), _p(perm), Rptr.size - 1, _p(Rptr), ctypes.byref(h)))
    return Symbolic(h, n, int(cp[-1]), cp, rv)


# ===== factorization =====

class Factorization:
    """A* = U* L* on the device (pp_fac; the reference's ChordalSLU, chordal_slu.jl:1-26)."""

    def __init__(self, s: AbstractSemiring, sym: Symbolic, dtype, handle, ctx: Context):
        self.s = s
        self.sym = sym
        self.dtype = np.dtype(dtype)
        self.handle = handle
        self.ctx = ctx
        self.n = sym.n

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            lib().pp_fac_destroy(h)
            self.handle = None

    @property
    def shape(self):
        return (self.n, self.n)

    @property
    def perm(self) -> np.ndarray:
        return self.sym.export()["perm"]

    def export(self) -> dict:
        """The factor in the reference's storage layout: LD/UD (diagonal blocks), LL (na x nn), UL (nn x na)."""
        e = self.sym.export()
        nn = np.diff(e["Rptr"])
        na = np.diff(e["Sptr"])
        nD = int((nn * nn).sum())
        nL = int((nn * na).sum())
        LD = np.empty(max(1, nD), self.dtype)
        UD = np.empty(max(1, nD), self.dtype)
        LL = np.empty(max(1, nL), self.dtype)
        UL = np.empty(max(1, nL), self.dtype)
        self.ctx.check(lib().pp_fac_export(self.ctx.handle, self.handle, _p(LD), _p(UD), _p(LL), _p(UL)))
        return {"LD": LD[:nD], "UD": UD[:nD], "LL": LL[:nL], "UL": UL[:nL]}


class DenseFactorization(Factorization):
    """A* = U* L* of a dense matrix in its own order (pp_dense_factor; the reference's DenseSLU, dense_slu.jl:1-44):
    one front, no structure to analyse.  ``A`` (``export()["A"]``) is the in-place L + U of DenseSLU.A."""

    def __init__(self, s: AbstractSemiring, n: int, dtype, handle, ctx: Context):
        self.s = s
        self.sym = None
        self.dtype = np.dtype(dtype)
        self.handle = handle
        self.ctx = ctx
        self.n = n

    @property
    def perm(self) -> np.ndarray:
        return np.arange(self.n, dtype=np.int64)

    def export(self) -> dict:
        n = self.n
        LD = np.empty(max(1, n * n), self.dtype)
        self.ctx.check(lib().pp_fac_export(self.ctx.handle, self.handle, _p(LD), None, None, None))
        A = LD[:n * n].reshape((n, n), order="F")
        return {"A": A, "LD": LD[:n * n], "UD": LD[:n * n], "LL": LD[:0], "UL": LD[:0]}


def _dense_operand(A):
    """(n, pointer, lda, on_device, keep-alive) of a square dense matrix: a numpy array (column-major copy) or an
    n x n DeviceArray (column-major in HBM)."""
    if isinstance(A, DeviceArray):
        if len(A.shape) != 2 or A.shape[0] != A.shape[1]:
            raise PathpackArgumentError(_lib.PP_EINVAL, "the matrix must be square")
        return A.shape[0], ctypes.c_void_p(A.ptr), max(1, A.shape[0]), 1, A, A.dtype
    if A.ndim != 2 or A.shape[0] != A.shape[1]:
        raise PathpackArgumentError(_lib.PP_EINVAL, "the matrix must be square")
    M = np.asfortranarray(A)
    return M.shape[0], _p(M), max(1, M.shape[0]), 0, M, M.dtype


def dense_mlu(s: AbstractSemiring, A, device: int = 0) -> DenseFactorization:
    """mlu(s, A::AbstractMatrix) -> DenseSLU (abstract_slu.jl:55-58): the dense matrix factorized in its own
    order on the device (pp_dense_factor).  ``A``: a square numpy array or DeviceArray."""
    ctx = context(device)
    n, ptr, lda, on_dev, keep, dtype = _dense_operand(A)
    dt = _dtype_code(dtype)
    if (dt == I32) != isinstance(s, OrAnd):
        raise PathpackUnsupportedError(_lib.PP_EUNSUPPORTED, f"{s.name} does not support {dtype}")
    h = ctypes.c_void_p()
    ctx.check(lib().pp_dense_factor(ctx.handle, s.id, dt, n, ptr, lda, on_dev, ctypes.byref(h)))
    del keep
    return DenseFactorization(s, n, dtype, h, ctx)


def sgetrf_(s: AbstractSemiring, A: "DeviceArray") -> "DeviceArray":
    """sgetrf!(s, A) on a device matrix (dense/sgetrf.jl:5-17): A <- L + U with A* = U* L*, in place."""
    n, ptr, lda, on_dev, keep, dtype = _dense_operand(A)
    if not on_dev:
        raise PathpackArgumentError(_lib.PP_EINVAL, "sgetrf_: A must be a DeviceArray")
    dt = _dtype_code(dtype)
    if (dt == I32) != isinstance(s, OrAnd):
        raise PathpackUnsupportedError(_lib.PP_EUNSUPPORTED, f"{s.name} does not support {dtype}")
    A.ctx.check(lib().pp_dense_sgetrf(A.ctx.handle, s.id, dt, n, ptr, lda))
    return A


def _factor(s: AbstractSemiring, sym: Symbolic, nzval, ctx: Context) -> Factorization:
    dt = _dtype_code(nzval.dtype)
    if (dt == I32) != isinstance(s, OrAnd):
        raise PathpackUnsupportedError(_lib.PP_EUNSUPPORTED, f"{s.name} does not support {nzval.dtype}")
    h = ctypes.c_void_p()
    nz = np.ascontiguousarray(nzval)
    ctx.check(lib().pp_factor(ctx.handle, sym.handle, s.id, dt, _p(nz), ctypes.byref(h)))
    return Factorization(s, sym, nz.dtype, h, ctx)


def mlu(s: AbstractSemiring, A, alg=None, amalgamate: bool = True, device: int = 0, sym: Symbolic | None = None):
    """Factorize the star of A over the semiring s: A* = U* L* (mlu, abstract_slu.jl:44-58).  A dense numpy A is one
    dense front in its natural order (the reference's DenseSLU path, abstract_slu.jl:65-68)."""
    ctx = context(device)
    if isinstance(A, np.ndarray) and sym is None:
        return dense_mlu(s, A, device)
    if isinstance(A, np.ndarray):
        # a dense matrix with a structure given from outside: one stored entry per matrix entry
        if A.ndim != 2 or A.shape[0] != A.shape[1]:
            raise PathpackArgumentError(_lib.PP_EINVAL, "the matrix must be square")
        n = A.shape[0]
        cp = np.arange(0, n * n + 1, n, dtype=np.int64)
        rv = np.tile(np.arange(n, dtype=np.int64), n)
        nz = np.asfortranarray(A).ravel(order="F")
        sym.check_pattern(n, cp, rv)
        return _factor(s, sym, nz, ctx)
    n, cp, rv, nz = _as_csc(A)
    if sym is None:
        sym = symbolic((n, cp, rv, nz), alg=alg, amalgamate=amalgamate)
    else:
        sym.check_pattern(n, cp, rv)
    return _factor(s, sym, nz, ctx)


def lu_(F: Factorization, A):
    """copyto!(F, A) then lu!(F) (chordal_slu.jl:116-118, abstract_slu.jl:119-121): the values of A, which must
    have the pattern F was analysed for, factorized in place on the device (no new analysis, plan upload or factor
    buffers; the reference GPU API's repeated-weights plan, ext/PATHPACKCUDAExt/api.jl:545-600).  ``A`` may also be
    a DeviceArray of the nnz values in the pattern's CSC order.  Returns F."""
    if isinstance(F, DenseFactorization):
        n, ptr, lda, on_dev, keep, dtype = _dense_operand(A)
        if n != F.n or np.dtype(dtype) != F.dtype:
            raise PathpackArgumentError(_lib.PP_EINVAL, "lu_: the matrix must be n x n of the factor's type")
        F.ctx.check(lib().pp_dense_refactor(F.ctx.handle, F.handle, ptr, lda, on_dev))
        del keep
        return F
    if isinstance(A, DeviceArray):
        if A.dtype != F.dtype or int(np.prod(A.shape)) != F.sym.nnz:
            raise PathpackArgumentError(_lib.PP_EINVAL, "lu_: the values must be nnz entries of the factor's type")
        F.ctx.check(lib().pp_refactor(F.ctx.handle, F.handle, ctypes.c_void_p(A.ptr), 1))
        return F
    if isinstance(A, np.ndarray):
        n = A.shape[0]
        if A.ndim != 2 or A.shape != (F.n, F.n):
            raise PathpackArgumentError(_lib.PP_EINVAL, "lu_: the matrix must be n x n")
        cp = np.arange(0, n * n + 1, n, dtype=np.int64)
        rv = np.tile(np.arange(n, dtype=np.int64), n)
        nz = np.asfortranarray(A).ravel(order="F")
    else:
        n, cp, rv, nz = _as_csc(A)
    F.sym.check_pattern(n, cp, rv)
    if nz.dtype != F.dtype:
        raise PathpackArgumentError(_lib.PP_EINVAL, f"lu_: the values must have the factor's type {F.dtype}")
    nz = np.ascontiguousarray(nz)
    F.ctx.check(lib().pp_refactor(F.ctx.handle, F.handle, _p(nz), 0))
    return F


def Matrix(F: Factorization, device: bool = False, out=None):
    """The full star A* of a factorization (Matrix(F), abstract_slu.jl:10-14), n x n in the original labels,
    column-major.  ``device=True`` (or a DeviceArray ``out``) leaves it in HBM as a DeviceArray."""
    n = F.n
    if device or isinstance(out, DeviceArray):
        if out is None:
            out = DeviceArray((n, n), F.dtype, F.ctx)
        if out.shape != (n, n) or out.dtype != F.dtype:
            raise PathpackArgumentError(_lib.PP_EINVAL, "out must be an n x n DeviceArray of the factor's type")
        F.ctx.check(lib().pp_star(F.ctx.handle, F.handle, ctypes.c_void_p(out.ptr), n, 1))
        return out
    C = out if out is not None else np.empty((n, n), dtype=F.dtype, order="F")
    if not C.flags.f_contiguous or C.shape != (n, n) or C.dtype != F.dtype:
        raise PathpackArgumentError(_lib.PP_EINVAL, "out must be a Fortran-ordered n x n array of the factor's type")
    F.ctx.check(lib().pp_star(F.ctx.handle, F.handle, _p(C), n, 0))
    return C


def mstar(s: AbstractSemiring, A, alg=None, amalgamate: bool = True, device: bool = False, sym: Symbolic | None = None,
          out=None, keep_factor: bool = False):
    """The star A* = I (+) A (+) A^2 (+) ... as a dense matrix (mstar, abstract_slu.jl:81-87): the symbolic analysis,
    then factorization and star in one device call (pp_mstar).  ``A`` may be a CSC triple / scipy matrix, or
    ``(n, colptr, rowval, values)`` with the values a DeviceArray already in HBM.  ``device=True`` (or a DeviceArray
    ``out``) leaves the star in HBM.  ``keep_factor=True`` returns ``(star, F)``."""
    if isinstance(A, np.ndarray):
        F = mlu(s, A, alg=alg, amalgamate=amalgamate, sym=sym)
        C = Matrix(F, device=device, out=out)
        return (C, F) if keep_factor else C
    ctx = context(0)
    if isinstance(A, tuple) and len(A) == 4 and isinstance(A[3], DeviceArray):
        n, cp, rv, dnz = A
        cp = np.ascontiguousarray(cp, np.int64)
        rv = np.ascontiguousarray(rv, np.int64)
        if int(np.prod(dnz.shape)) != int(cp[-1]):
            raise PathpackArgumentError(_lib.PP_EINVAL, "mstar: the device values must hold nnz entries")
        dtype, nzp, on_dev, keep = dnz.dtype, ctypes.c_void_p(dnz.ptr), 1, None
        if sym is None:
            sym = symbolic((n, cp, rv, np.zeros(cp[-1], dtype)), alg=alg, amalgamate=amalgamate)
    else:
        n, cp, rv, nz = _as_csc(A)
        keep = np.ascontiguousarray(nz)
        dtype, nzp, on_dev = keep.dtype, _p(keep), 0
        if sym is None:
            sym = symbolic((n, cp, rv, nz), alg=alg, amalgamate=amalgamate)
    sym.check_pattern(n, cp, rv)
    dt = _dtype_code(dtype)
    if (dt == I32) != isinstance(s, OrAnd):
        raise PathpackUnsupportedError(_lib.PP_EUNSUPPORTED, f"{s.name} does not support {dtype}")
    h = ctypes.c_void_p()
    hp = ctypes.byref(h) if keep_factor else None
    if device or isinstance(out, DeviceArray):
        C = out if out is not None else DeviceArray((n, n), dtype, ctx)
        if C.shape != (n, n) or C.dtype != dtype:
            raise PathpackArgumentError(_lib.PP_EINVAL, "out must be an n x n DeviceArray of the values' type")
        ctx.check(lib().pp_mstar(ctx.handle, sym.handle, s.id, dt, nzp, on_dev, ctypes.c_void_p(C.ptr), n, 1, hp))
    else:
        C = out if out is not None else np.empty((n, n), dtype=dtype, order="F")
        if not C.flags.f_contiguous or C.shape != (n, n) or C.dtype != dtype:
            raise PathpackArgumentError(_lib.PP_EINVAL, "out must be a Fortran-ordered n x n array of the values' type")
        ctx.check(lib().pp_mstar(ctx.handle, sym.handle, s.id, dt, nzp, on_dev, _p(C), n, 0, hp))
    del keep
    if keep_factor:
        return C, Factorization(s, sym, np.dtype(dtype), h, ctx)
    return C


def _star_sources(F: Factorization, src, which: int, device: bool):
    name = "star_rows" if which == 0 else "star_cols"
    idx = np.ascontiguousarray(np.asarray(src, dtype=np.int64).reshape(-1))
    if idx.size and (idx.min() < 0 or idx.max() >= F.n):
        raise PathpackArgumentError(_lib.PP_EINVAL, f"{name}: source index out of range")
    k, n = idx.size, F.n
    shape = (k, n) if which == 0 else (n, k)
    if device:
        out = DeviceArray(shape, F.dtype, F.ctx)
        if k and n:
            F.ctx.check(lib().pp_star_sources(F.ctx.handle, F.handle, which, k, _p(idx), ctypes.c_void_p(out.ptr),
                                              max(1, shape[0]), 1))
        return out
    out = np.empty(shape, dtype=F.dtype, order="F")
    if k and n:
        F.ctx.check(lib().pp_star_sources(F.ctx.handle, F.handle, which, k, _p(idx), _p(out), max(1, shape[0]), 0))
    return out


def star_rows(F: Factorization, src, device: bool = False):
    """Rows src of A* (len(src) x n; row k is the least solution x of x = x A (+) e_src[k]^T), for many sources in
    one pass: sgetre!(F, Val(:L), Val(:T), b, k) (chordal_slu.jl:445-493) over a batch of sources."""
    return _star_sources(F, src, 0, device)


def star_cols(F: Factorization, src, device: bool = False):
    """Columns src of A* (n x len(src); column k is the least solution x of x = A x (+) e_src[k]), for many
    sources in one pass: sgetre!(F, Val(:L), Val(:N), b, k) (chordal_slu.jl:445-493) over a batch of sources."""
    return _star_sources(F, src, 1, device)


class TransposedFactorization:
    """transpose(F) (equivalently adjoint(F) for these real semirings): the factorization of A^T that F implies,
    (A^T)* = (A*)^T, for lmul_ / rmul_ (the reference's MaybeTransSLU, abstract_slu.jl:131-145)."""

    def __init__(self, F: Factorization):
        self.parent = F

    @property
    def shape(self):
        return self.parent.shape


def transpose(F):
    """transpose(F): lmul_(transpose(F), B) solves X = A^T X (+) B, rmul_(B, transpose(F)) solves X = X A^T (+) B."""
    return F.parent if isinstance(F, TransposedFactorization) else TransposedFactorization(F)


adjoint = transpose


def _solve(F, B, left: bool):
    name = "lmul_" if left else "rmul_"
    trans = isinstance(F, TransposedFactorization)
    if trans:
        F = F.parent

    def fn(ctxh, fh, ptr, ld, nrhs, on_dev):
        return lib().pp_sgetrs(ctxh, fh, 0 if left else 1, 1 if trans else 0, ptr, ld, nrhs, on_dev)

    if isinstance(B, np.ndarray):
        if B.dtype != F.dtype:
            raise PathpackArgumentError(_lib.PP_EINVAL, f"{name}: B must have the factor's element type {F.dtype}")
        vec = B.ndim == 1
        if vec and not left:
            raise PathpackArgumentError(_lib.PP_EINVAL, "rmul_: B must be a matrix")
        M = B.reshape(-1, 1) if vec else B
        if left and M.shape[0] != F.n or (not left and M.shape[1] != F.n):
            raise PathpackArgumentError(_lib.PP_EINVAL, f"{name}: B has the wrong size")
        W = np.asfortranarray(M)
        nrhs = W.shape[1] if left else W.shape[0]
        ld = max(1, W.shape[0])
        F.ctx.check(fn(F.ctx.handle, F.handle, _p(W), ld, nrhs, 0))
        if W is not M:
            M[...] = W
        return B
    if not isinstance(B, DeviceArray) or len(B.shape) != 2:
        raise PathpackArgumentError(_lib.PP_EINVAL, f"{name}: B must be a numpy array or a 2-D DeviceArray")
    if B.dtype != F.dtype:
        raise PathpackArgumentError(_lib.PP_EINVAL, f"{name}: B must have the factor's element type {F.dtype}")
    rows, cols = B.shape
    if left and rows != F.n or (not left and cols != F.n):
        raise PathpackArgumentError(_lib.PP_EINVAL, f"{name}: B has the wrong size")
    nrhs = cols if left else rows
    F.ctx.check(fn(F.ctx.handle, F.handle, ctypes.c_void_p(B.ptr), max(1, rows), nrhs, 1))
    return B


def lmul_(F, B):
    """lmul!(F, B): B <- A* B, the least solution of X = A X (+) B (abstract_slu.jl:131-134); with
    F = transpose(F0), B <- (A^T)* B."""
    return _solve(F, B, True)


def rmul_(B, F):
    """rmul!(B, F): B <- B A*, the least solution of X = X A (+) B (abstract_slu.jl:142-145); with
    F = transpose(F0), B <- B (A^T)*."""
    return _solve(F, B, False)
