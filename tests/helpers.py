"""Shared helpers of the tests: the oracle's view of a product symbolic structure, brute-force closures, inputs."""

import numpy as np

import oracle as O
import pathpack_hip as P
from pathpack_hip import workloads as W

SEMIRINGS = {O.MINPLUS: P.MinPlus(), O.MAXPLUS: P.MaxPlus(), O.MAXMIN: P.MaxMin(), O.MINMAX: P.MinMax(),
             O.PLUSPROD: P.PlusProd(), O.ORAND: P.OrAnd()}


def oracle_sym(sym: P.Symbolic) -> O.Sym:
    e = sym.export()
    return O.Sym(sym.n, e["Rptr"], e["Sptr"], e["Stgt"], e["perm"], sym.components()["Bptr"])


def weighted(g: W.Graph, s: int, dtype, seed: int = 11) -> W.Graph:
    """The pattern of g with weights suited to semiring s: integers 1..100 (MinPlus, MaxMin, MinMax), their
    negatives (MaxPlus: longest paths need no positive cycle), bit sets 1..127 (OrAnd), and uniform(0, 0.2) scaled
    so the walk series converges (PlusProd)."""
    m = g.nnz
    if s == O.ORAND:
        v = W.uniform_int(seed, m, 1, 127).astype(np.int32)
    elif s == O.PLUSPROD:
        deg = np.maximum(1, np.bincount(g.rowval, minlength=g.n).max())
        v = (W.uniform_float(seed, m) * (0.9 / deg)).astype(dtype)
    elif s == O.MAXPLUS:
        v = (-W.uniform_int(seed, m, 1, 100)).astype(dtype)
    else:
        v = W.uniform_int(seed, m, 1, 100).astype(dtype)
    return W.Graph(g.n, g.colptr, g.rowval, v, g.name)


def dtype_for(s: int, float_dtype=np.float64):
    return np.int32 if s == O.ORAND else float_dtype


def assert_star_equal(s: int, C, D, rtol=1e-12):
    """Bit-exact for the idempotent semirings, relative tolerance for PlusProd."""
    if s == O.PLUSPROD:
        # relative error in the normal range of the compared type; below its smallest normal number (gradual
        # underflow, where the relative precision is gone) the error is measured against that number
        floor = np.finfo(np.result_type(np.asarray(C).dtype, np.asarray(D).dtype)).tiny
        C = np.asarray(C, np.float64)
        D = np.asarray(D, np.float64)
        assert C.shape == D.shape, f"shapes {C.shape} and {D.shape}"
        if C.size == 0:
            return
        scale = np.maximum(np.abs(D), floor)
        err = np.abs(C - D) / scale
        err[(C == 0) & (D == 0)] = 0
        assert err.max() <= rtol, f"max relative error {err.max()}"
    else:
        c, d = bits(C), bits(D)
        assert c.shape == d.shape and np.array_equal(c, d), f"{np.sum(c != d)} entries differ"


def bits(a) -> np.ndarray:
    """The bit patterns of an array (C order), for bit-exact comparisons."""
    a = np.ascontiguousarray(a)
    return a.view({1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[a.dtype.itemsize])
