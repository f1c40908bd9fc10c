"""The dense path (mlu(s, A::AbstractMatrix) -> DenseSLU, src/CPU/abstract_slu.jl:55-58, dense_slu.jl:1-44) on the
device through the C ABI (pp_dense_factor, pp_dense_refactor, pp_dense_sgetrf), against the oracle's dense LU
(dense/sgetrf.jl, pinned by test_oracle.test_dense_lu_factors_the_closure), its star and its solves.  Bit-exact for
the idempotent semirings (integer weights), relative 1e-12 for PlusProd in Float64."""

import numpy as np
import pytest

import oracle as O
import pathpack_hip as P
from helpers import SEMIRINGS, assert_star_equal, dtype_for
from test_oracle import ALL, dense_matrix, dense_pattern, dense_rhs

pytestmark = pytest.mark.gpu

# 1 and 7: one small front in LDS; 64 and 65 at the edge of it; 200 and 300: blocked steps and star blocks
SIZES = [1, 7, 64, 65, 200, 300]


def oracle_factor(s, A):
    sym, cp, rv, nz = dense_pattern(A)
    return O.factor(s, sym, cp, rv, nz)


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("s", ALL)
def test_dense_factor_star_and_solves_match_oracle(s, n):
    rng = np.random.default_rng(1000 * s + n)
    dtype = dtype_for(s)
    A = dense_matrix(s, dtype, n, rng)
    F = P.dense_mlu(SEMIRINGS[s], A)
    assert isinstance(F, P.DenseFactorization) and F.shape == (n, n)
    assert_star_equal(s, F.export()["A"], O.getrf(s, A))
    Fo = oracle_factor(s, A)
    assert_star_equal(s, P.Matrix(F), O.star(Fo))
    B = dense_rhs(s, dtype, (n, 5), rng)
    assert_star_equal(s, P.lmul_(F, np.asfortranarray(B.copy())), O.lmul(Fo, B))
    Bt = np.asfortranarray(dense_rhs(s, dtype, (3, n), rng))
    assert_star_equal(s, P.rmul_(np.asfortranarray(Bt.copy()), F), O.rmul(Fo, Bt))


@pytest.mark.parametrize("s", [O.MINPLUS, O.PLUSPROD])
def test_dense_float32(s):
    rng = np.random.default_rng(7 + s)
    A = dense_matrix(s, np.float32, 150, rng)
    F = P.dense_mlu(SEMIRINGS[s], A)
    Fo = oracle_factor(s, A)
    if s == O.PLUSPROD:
        np.testing.assert_allclose(F.export()["A"], O.getrf(s, A), rtol=2e-5, atol=1e-7)
        np.testing.assert_allclose(P.Matrix(F), O.star(Fo), rtol=2e-5, atol=1e-7)
    else:
        assert_star_equal(s, F.export()["A"], O.getrf(s, A))
        assert_star_equal(s, P.Matrix(F), O.star(Fo))


def test_dense_device_input_refactor_and_inplace_lu():
    """A matrix already in HBM factorizes like the host one; lu!(F, A2) with new values equals a fresh factor;
    sgetrf!(s, A) on a device matrix leaves L + U in A; a dense factor refuses the sparse refactorization."""
    s = O.MINPLUS
    rng = np.random.default_rng(31)
    n = 180
    A = dense_matrix(s, np.float64, n, rng)
    A2 = dense_matrix(s, np.float64, n, rng)
    dA = P.DeviceArray.from_numpy(A)
    F = P.dense_mlu(P.MinPlus(), dA)
    assert_star_equal(s, F.export()["A"], O.getrf(s, A))
    P.lu_(F, A2)
    assert_star_equal(s, F.export()["A"], O.getrf(s, A2))
    assert_star_equal(s, P.Matrix(F), O.floyd_warshall(s, A2))
    P.lu_(F, P.DeviceArray.from_numpy(A))
    assert_star_equal(s, P.Matrix(F), O.floyd_warshall(s, A))
    P.sgetrf_(P.MinPlus(), dA)
    assert_star_equal(s, dA.numpy(), O.getrf(s, A))
    with pytest.raises(P.PathpackArgumentError):
        F.ctx.check(P.lib().pp_refactor(F.ctx.handle, F.handle, None, 1))


def test_dense_mstar_through_mlu():
    """mstar(s, A::AbstractMatrix) = Matrix(mlu(s, A)) (abstract_slu.jl:81-83)."""
    rng = np.random.default_rng(5)
    A = dense_matrix(O.MAXMIN, np.float64, 90, rng)
    assert np.array_equal(P.mstar(P.MaxMin(), A), O.floyd_warshall(O.MAXMIN, A))
