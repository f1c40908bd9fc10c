"""pp_sgetrs_noalloc: the solves with no device allocation, their scratch in a fixed device array (64 MiB per device).

Checked against pp_sgetrs (the allocating entry point, same kernels) through the C ABI, to the parity bar: bit for bit
for the idempotent semirings, 1e-12 relative for PlusProd (its forward scatter adds atomically, so two runs may round
differently).  Two calls in a row on one context, the second with a smaller factor and fewer right-hand sides (the
array keeps the first call's contents), for both sides and both transposes; requests larger than the array are refused
before anything is queued.
"""

import ctypes

import numpy as np
import pytest

import oracle as O
from helpers import SEMIRINGS, assert_star_equal, bits, dtype_for, weighted
import pathpack_hip as P
from pathpack_hip import workloads as W

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20


def rhs(s, dtype, n, k, rng, left):
    """k unit right-hand sides and three dense ones, as columns (left) or rows (right)."""
    B = np.full((n, k), O.zero(s, dtype), dtype=dtype, order="F")
    B[rng.integers(0, n, k), np.arange(k)] = O.one(s, dtype)
    if s == O.ORAND:
        B[:, -3:] = rng.integers(0, 128, (n, 3)).astype(np.int32)
    elif s == O.PLUSPROD:
        B[:, -3:] = rng.random((n, 3))
    else:
        B[:, -3:] = rng.integers(0, 50, (n, 3)).astype(dtype)
    return B if left else np.asfortranarray(B.T)


def solve_both(F, B, side, trans):
    """(pp_sgetrs on a device copy, pp_sgetrs_noalloc on another device copy), both downloaded."""
    ld, nrhs = B.shape[0], (B.shape[1] if side == 0 else B.shape[0])
    d1, d2 = P.DeviceArray.from_numpy(B, F.ctx), P.DeviceArray.from_numpy(B, F.ctx)
    F.ctx.check(P.lib().pp_sgetrs(F.ctx.handle, F.handle, side, trans, ctypes.c_void_p(d1.ptr), ld, nrhs, 1))
    F.ctx.check(P.lib().pp_sgetrs_noalloc(F.ctx.handle, F.handle, side, trans, ctypes.c_void_p(d2.ptr), ld, nrhs))
    F.ctx.synchronize()
    return d1.numpy(), d2.numpy()


@pytest.mark.parametrize("side,trans", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("s,fdtype", [(O.MINPLUS, np.float32), (O.MAXMIN, np.float64), (O.PLUSPROD, np.float64),
                                      (O.ORAND, np.float32)])
def test_noalloc_solve_matches_allocating_solve(s, fdtype, side, trans):
    dtype = dtype_for(s, fdtype)
    print(f"case noalloc s={s} dtype={np.dtype(dtype)} side={side} trans={trans}", flush=True)
    rng = np.random.default_rng(17)
    big = weighted(W.random_digraph(260, 0.012, 8), s, dtype)
    small = weighted(W.random_digraph(90, 0.05, 12), s, dtype)
    F1 = P.mlu(SEMIRINGS[s], big)
    F2 = P.mlu(SEMIRINGS[s], small)
    for F, g, k in ((F1, big, 40), (F2, small, 7)):   # the second call is smaller
        B = rhs(s, dtype, g.n, k, rng, side == 0)
        ref, got = solve_both(F, B, side, trans)
        if s == O.PLUSPROD:
            assert_star_equal(s, got, ref, rtol=1e-12)
        else:
            assert np.array_equal(bits(got), bits(ref))


def test_noalloc_refuses_requests_beyond_the_scratch():
    g = weighted(W.random_digraph(260, 0.012, 8), O.MINPLUS, np.float64)
    F = P.mlu(P.MinPlus(), g)
    nrhs = SCRATCH_BYTES // (8 * g.n) + 1                  # one right-hand side too many
    B = P.DeviceArray((g.n, nrhs), np.float64, F.ctx)      # a real buffer of that size
    st = P.lib().pp_sgetrs_noalloc(F.ctx.handle, F.handle, 0, 0, ctypes.c_void_p(B.ptr), g.n, nrhs)
    assert st == 1   # PP_EINVAL
    assert b"fixed scratch" in P.lib().pp_last_error(F.ctx.handle)
    # the largest request that fits is accepted, and the context keeps working
    k = SCRATCH_BYTES // (8 * g.n)
    Bk = np.full((g.n, k), np.inf)
    Bk[np.arange(k) % g.n, np.arange(k)] = 0.0
    ref, got = solve_both(F, np.asfortranarray(Bk), 0, 0)
    assert np.array_equal(bits(got), bits(ref))
