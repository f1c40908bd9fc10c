// pp_oracle.cpp -- CPU restatement of PATHPACK.CPU's multifrontal semiring LU.
//
// TEST INFRASTRUCTURE ONLY.  This file is the oracle: only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg load it, and only as the checker (or as the timed CPU baseline).  The product path
// (libpathpack_hip.so) never links or calls it.
//
// It restates, loop for loop where that matters for the result, the reference's CPU algorithm:
//   scalar semirings          src/CPU/semiring/{semiring,tropical,bottleneck,real,boolean}.jl
//   scatter of A              src/CPU/chordal_slu.jl:221-321 (scopyto_loop!)
//   multifrontal LU           src/CPU/chordal/sgetrf.jl:35-290 (sgetrf_loop!, sgetrf_loop_1!, sgetrf_send!)
//   dense LU                  src/CPU/dense/sgetrf.jl:151-175 (sgetrf2!, generic method)
//   dense TRSM                src/CPU/dense/strsx.jl (strsx2!: B <- B A*, B <- A* B)
//   dense TRTRI               src/CPU/dense/strtri.jl:203-269 (strtri2!)
//   solves lmul!/rmul!        src/CPU/chordal_slu.jl:337-377, src/CPU/chordal/sgetrs.jl:29-51,
//                             src/CPU/chordal/strsx.jl (strsx_fwd*/strsx_bwd*)
//   full star                 src/CPU/chordal/sgetri.jl:13-31, src/CPU/chordal/strtri.jl:171-319,
//                             src/CPU/chordal/strsx.jl:729-867, src/CPU/utils.jl:261-505 (permuterowscols!)
//   components                src/CPU/chordal_ssymbolic.jl:212-269 (soffd: the arcs between components, N),
//                             src/CPU/blocked/sgetri.jl:3-162 (sgetri_offd!: the off-diagonal blocks of the star),
//                             src/CPU/blocked/sgetrs.jl:80-122 (sgetrs_mt!: the solves over the components),
//                             src/CPU/sparse/sgemx.jl (sgemx_sparse!: products with N)
//   dense semiring GEMM       src/CPU/dense/sgemx.jl:606-635 (generic loop)
//   batched getrf + star      ext/PATHPACKCUDAExt/batched/sgetrf.jl:11-120 (front_diag_kernel!)
//
// The symbolic structure (ordering, supernodes, separators) is an input: it is either the reference's own
// (read from its factor fixtures) or the one the product computes.  Everything below uses 0-based indices.
// Fronts are in postorder; res(f) = [Rptr[f], Rptr[f+1]); sep(f) = Stgt[Sptr[f] .. Sptr[f+1]) sorted ascending;
// perm[new] = old.  Factor layout (the reference's, App. B of the survey of CliqueTrees' storage):
//   LDval/UDval: nn x nn column-major at Dptr[f] = sum_{g<f} nn_g^2
//   LLval: na x nn column-major at Lptr[f] = sum_{g<f} nn_g na_g   (L21[i,j] = LLval[Lp + i + j*na])
//   ULval: nn x na column-major at Lptr[f]                         (U12[i,j] = ULval[Lp + i + j*nn])
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>
#include <algorithm>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef int64_t i64;

enum { S_MINPLUS = 0, S_MAXPLUS = 1, S_MAXMIN = 2, S_MINMAX = 3, S_PLUSPROD = 4, S_ORAND = 5 };
enum { D_F32 = 0, D_F64 = 1, D_I32 = 2 };

// ===== scalar semirings (src/CPU/semiring/*.jl) =====
//
// vmin(x, y) = ifelse(x < y, x, y) and vmax(x, y) = ifelse(x > y, x, y) on x86 (semiring.jl:124-138).

template <class T> static inline T vmin(T x, T y) { return x < y ? x : y; }
template <class T> static inline T vmax(T x, T y) { return x > y ? x : y; }

// MinPlus: tropical.jl:84-218.  zero +Inf, one 0; smuladd on x86 = vmin(a + b, c) (tropical.jl:188-191);
// sprod maps NaN to szero (tropical.jl:164-167); sstar(a) = 0 if a >= 0 else -Inf (tropical.jl:210-218).
template <class T> struct MinPlus {
    static constexpr bool integral = false;
    static T zero() { return std::numeric_limits<T>::infinity(); }
    static T one() { return T(0); }
    static T plus(T a, T b) { return vmin(a, b); }
    static T prod(T a, T b) { T c = a + b; return c != c ? zero() : c; }
    static T muladd(T a, T b, T c) { return vmin(T(a + b), c); }
    static T star(T a) { return a >= T(0) ? one() : -std::numeric_limits<T>::infinity(); }
};

// MaxPlus = DualQuantale{MinPlus}: zero -Inf, one 0, plus vmax, sprod NaN -> -Inf, sstar(a) = 0 if a <= 0 else +Inf
// (semiring.jl:259-265,305-307,343-349; tropical.jl:31,164-191,210-218).
template <class T> struct MaxPlus {
    static constexpr bool integral = false;
    static T zero() { return -std::numeric_limits<T>::infinity(); }
    static T one() { return T(0); }
    static T plus(T a, T b) { return vmax(a, b); }
    static T prod(T a, T b) { T c = a + b; return c != c ? zero() : c; }
    static T muladd(T a, T b, T c) { return vmax(T(a + b), c); }
    static T star(T a) { return a <= T(0) ? one() : std::numeric_limits<T>::infinity(); }
};

// MaxMin = DualQuantale{MinMax}: zero -Inf, one +Inf, plus vmax, prod vmin, star = one, integral
// (bottleneck.jl:31,63-65; semiring.jl:247-253,293-299,413-423).
template <class T> struct MaxMin {
    static constexpr bool integral = true;
    static T zero() { return -std::numeric_limits<T>::infinity(); }
    static T one() { return std::numeric_limits<T>::infinity(); }
    static T plus(T a, T b) { return vmax(a, b); }
    static T prod(T a, T b) { return vmin(a, b); }
    static T muladd(T a, T b, T c) { return vmax(vmin(a, b), c); }
    static T star(T) { return one(); }
};

// MinMax = Lattice{MinPlus}: zero +Inf, one -Inf, plus vmin, prod vmax, star = one, integral (bottleneck.jl:15).
template <class T> struct MinMax {
    static constexpr bool integral = true;
    static T zero() { return std::numeric_limits<T>::infinity(); }
    static T one() { return -std::numeric_limits<T>::infinity(); }
    static T plus(T a, T b) { return vmin(a, b); }
    static T prod(T a, T b) { return vmax(a, b); }
    static T muladd(T a, T b, T c) { return vmin(vmax(a, b), c); }
    static T star(T) { return one(); }
};

// PlusProd: zero 0, one 1, smuladd = muladd (fused), sstar(a) = 1/(1-a) if a < 1 else +Inf (real.jl:16-58).
template <class T> struct PlusProd {
    static constexpr bool integral = false;
    static T zero() { return T(0); }
    static T one() { return T(1); }
    static T plus(T a, T b) { return a + b; }
    static T prod(T a, T b) { return a * b; }
    static T muladd(T a, T b, T c) { return std::fma(a, b, c); }
    static T star(T a) { return a < T(1) ? T(1) / (T(1) - a) : std::numeric_limits<T>::infinity(); }
};

// OrAnd = DualQuantale{AndOr} on integers: zero 0, one typemax, plus |, prod &, star = one, integral
// (boolean.jl:31-71).
template <class T> struct OrAnd {
    static constexpr bool integral = true;
    static T zero() { return T(0); }
    static T one() { return std::numeric_limits<T>::max(); }
    static T plus(T a, T b) { return a | b; }
    static T prod(T a, T b) { return a & b; }
    static T muladd(T a, T b, T c) { return (a & b) | c; }
    static T star(T) { return one(); }
};

// ===== symbolic structure, derived maps =====

struct Sym {
    i64 n, nf;
    const i64 *Rptr, *Sptr, *Stgt, *perm;
    std::vector<i64> invp, idx, parent, fdsc, Dptr, Lptr;
    std::vector<std::vector<i64>> chd;   // children, increasing
    std::vector<std::vector<i64>> rel;   // rel[f][k]: position of Stgt[Sptr[f]+k] in bag(parent(f))
    i64 nFmax;
};

static int build_sym(Sym &S, i64 n, i64 nf, const i64 *Rptr, const i64 *Sptr, const i64 *Stgt, const i64 *perm) {
    S.n = n; S.nf = nf; S.Rptr = Rptr; S.Sptr = Sptr; S.Stgt = Stgt; S.perm = perm;
    S.invp.assign(n, -1);
    for (i64 i = 0; i < n; i++) {
        if (perm[i] < 0 || perm[i] >= n || S.invp[perm[i]] >= 0) return -1;
        S.invp[perm[i]] = i;
    }
    if (Rptr[0] != 0 || Rptr[nf] != n || Sptr[0] != 0) return -2;
    S.idx.assign(n, -1);
    for (i64 f = 0; f < nf; f++)
        for (i64 v = Rptr[f]; v < Rptr[f + 1]; v++) S.idx[v] = f;
    S.parent.assign(nf, -1);
    S.chd.assign(nf, {});
    S.Dptr.assign(nf + 1, 0);
    S.Lptr.assign(nf + 1, 0);
    S.nFmax = 0;
    for (i64 f = 0; f < nf; f++) {
        i64 nn = Rptr[f + 1] - Rptr[f], na = Sptr[f + 1] - Sptr[f];
        S.Dptr[f + 1] = S.Dptr[f] + nn * nn;
        S.Lptr[f + 1] = S.Lptr[f] + nn * na;
        S.nFmax = std::max(S.nFmax, nn + na);
        if (na > 0) {
            i64 p = S.idx[Stgt[Sptr[f]]];
            if (p <= f) return -3;
            S.parent[f] = p;
            S.chd[p].push_back(f);
        }
    }
    // fdsc: first descendant of each front (strtri.jl:63-77)
    S.fdsc.resize(nf);
    for (i64 f = 0; f < nf; f++) S.fdsc[f] = f;
    for (i64 f = 0; f < nf; f++)
        if (S.parent[f] >= 0) S.fdsc[S.parent[f]] = std::min(S.fdsc[S.parent[f]], S.fdsc[f]);
    // rel: sep(f) -> bag(parent(f)); bag = res ++ sep
    S.rel.assign(nf, {});
    std::vector<i64> pos(n, -1);
    for (i64 f = 0; f < nf; f++) {
        i64 p = S.parent[f];
        if (p < 0) continue;
        i64 pnn = Rptr[p + 1] - Rptr[p];
        for (i64 v = Rptr[p]; v < Rptr[p + 1]; v++) pos[v] = v - Rptr[p];
        for (i64 q = Sptr[p]; q < Sptr[p + 1]; q++) pos[Stgt[q]] = pnn + (q - Sptr[p]);
        for (i64 q = Sptr[f]; q < Sptr[f + 1]; q++) {
            i64 r = pos[Stgt[q]];
            if (r < 0) return -4;
            S.rel[f].push_back(r);
        }
        for (i64 v = Rptr[p]; v < Rptr[p + 1]; v++) pos[v] = -1;
        for (i64 q = Sptr[p]; q < Sptr[p + 1]; q++) pos[Stgt[q]] = -1;
    }
    return 0;
}

// ===== dense kernels on column-major views =====

// sgetrf2! generic (dense/sgetrf.jl:151-175): A <- L + U, A* = U* L*, no pivoting.
template <class S, class T> static void sgetrf2(T *A, i64 lda, i64 n) {
    for (i64 i = 0; i < n; i++) {
        if (!S::integral) {
            T s = S::star(A[i + i * lda]);
            for (i64 k = i + 1; k < n; k++) A[k + i * lda] = S::prod(A[k + i * lda], s);
        }
        for (i64 j = i + 1; j < n; j++) {
            T Aij = A[i + j * lda];
            for (i64 q = i + 1; q < n; q++) A[q + j * lda] = S::muladd(A[q + i * lda], Aij, A[q + j * lda]);
        }
    }
}

// B <- B A*, A upper, non-unit (strsx2!, Val(:R), Val(:U), Val(:N)): B is m x n.
template <class S, class T> static void trsm_right_upper_nonunit(const T *A, i64 lda, T *B, i64 ldb, i64 m, i64 n) {
    for (i64 j = 0; j < n; j++) {
        for (i64 k = 0; k < j; k++) {
            T Akj = A[k + j * lda];
            for (i64 r = 0; r < m; r++) B[r + j * ldb] = S::muladd(B[r + k * ldb], Akj, B[r + j * ldb]);
        }
        if (!S::integral) {
            T s = S::star(A[j + j * lda]);
            for (i64 r = 0; r < m; r++) B[r + j * ldb] = S::prod(B[r + j * ldb], s);
        }
    }
}

// B <- B A*, A lower, unit (strsx2!, Val(:R), Val(:L), Val(:U)): backward over columns.
template <class S, class T> static void trsm_right_lower_unit(const T *A, i64 lda, T *B, i64 ldb, i64 m, i64 n) {
    for (i64 j = n - 1; j >= 0; j--)
        for (i64 k = j + 1; k < n; k++) {
            T Akj = A[k + j * lda];
            for (i64 r = 0; r < m; r++) B[r + j * ldb] = S::muladd(B[r + k * ldb], Akj, B[r + j * ldb]);
        }
}

// B <- A* B, A lower, unit (strsx2!, Val(:L), Val(:L), Val(:U)): forward over rows.
template <class S, class T> static void trsm_left_lower_unit(const T *A, i64 lda, T *B, i64 ldb, i64 n, i64 m) {
    for (i64 c = 0; c < m; c++)
        for (i64 i = 0; i < n; i++) {
            T acc = B[i + c * ldb];
            for (i64 k = 0; k < i; k++) acc = S::muladd(A[i + k * lda], B[k + c * ldb], acc);
            B[i + c * ldb] = acc;
        }
}

// B <- A* B, A upper, non-unit (strsx2!, Val(:L), Val(:U), Val(:N)): backward over rows.
template <class S, class T> static void trsm_left_upper_nonunit(const T *A, i64 lda, T *B, i64 ldb, i64 n, i64 m) {
    for (i64 c = 0; c < m; c++)
        for (i64 i = n - 1; i >= 0; i--) {
            T acc = B[i + c * ldb];
            for (i64 k = i + 1; k < n; k++) acc = S::muladd(A[i + k * lda], B[k + c * ldb], acc);
            if (!S::integral) acc = S::prod(S::star(A[i + i * lda]), acc);
            B[i + c * ldb] = acc;
        }
}

// C <- C + A B (sgemx2! generic, dense/sgemx.jl:606-635): C[i,k] = smuladd(A[i,j], B[j,k], C[i,k]), j ascending.
template <class S, class T>
static void sgemx(T *C, i64 ldc, const T *A, i64 lda, const T *B, i64 ldb, i64 m, i64 n, i64 k) {
    for (i64 c = 0; c < n; c++)
        for (i64 j = 0; j < k; j++) {
            T Bjc = B[j + c * ldb];
            for (i64 r = 0; r < m; r++) C[r + c * ldc] = S::muladd(A[r + j * lda], Bjc, C[r + c * ldc]);
        }
}

// strtri2! upper (dense/strtri.jl:242-269): A <- A* in place for an upper triangle (diag :N or :U).
template <class S, class T> static void strtri2_upper(T *A, i64 lda, i64 n, bool nonunit) {
    if (nonunit)
        for (i64 k = 0; k < n; k++) A[k + k * lda] = S::star(A[k + k * lda]);
    for (i64 j = n - 1; j >= 0; j--) {
        if (nonunit && !S::integral)
            for (i64 i = 0; i < j; i++) A[i + j * lda] = S::prod(A[i + j * lda], A[j + j * lda]);
        for (i64 k = j - 1; k >= 0; k--) {
            if (nonunit && !S::integral) A[k + j * lda] = S::prod(A[k + k * lda], A[k + j * lda]);
            T Akj = A[k + j * lda];
            for (i64 q = 0; q < k; q++) A[q + j * lda] = S::muladd(A[q + k * lda], Akj, A[q + j * lda]);
        }
    }
}

// ===== scatter of A into the factor storage (scopyto_loop!, chordal_slu.jl:221-321) =====

template <class S, class T>
static void scopyto(const Sym &Y, const i64 *colptr, const i64 *rowval, const T *nzval, T *LD, T *UD, T *LL, T *UL) {
    const i64 n = Y.n, nf = Y.nf;
    std::fill(LD, LD + Y.Dptr[nf], S::zero());
    std::fill(UD, UD + Y.Dptr[nf], S::zero());
    std::fill(LL, LL + Y.Lptr[nf], S::zero());
    std::fill(UL, UL + Y.Lptr[nf], S::zero());
    std::vector<i64> ind(n, -1);
    for (i64 f = 0; f < nf; f++) {
        const i64 rlo = Y.Rptr[f], rhi = Y.Rptr[f + 1], nn = rhi - rlo;
        const i64 s0 = Y.Sptr[f], s1 = Y.Sptr[f + 1], na = s1 - s0;
        for (i64 q = s0; q < s1; q++) ind[Y.Stgt[q]] = q - s0;
        for (i64 j = rlo; j < rhi; j++) {
            i64 c = Y.perm[j];
            for (i64 p = colptr[c]; p < colptr[c + 1]; p++) {
                i64 i = Y.invp[rowval[p]];
                T v = nzval[p];
                if (i >= rlo && i < rhi) {
                    i64 o = Y.Dptr[f] + (i - rlo) + (j - rlo) * nn;
                    LD[o] = v; UD[o] = v;
                } else if (i > j) {
                    i64 k = ind[i];
                    if (k >= 0) LL[Y.Lptr[f] + k + (j - rlo) * na] = v;
                } else {
                    i64 g = Y.idx[i];
                    i64 q0 = Y.Sptr[g], q1 = Y.Sptr[g + 1];
                    const i64 *b = std::lower_bound(Y.Stgt + q0, Y.Stgt + q1, j);
                    if (b != Y.Stgt + q1 && *b == j) {
                        i64 mm = Y.Rptr[g + 1] - Y.Rptr[g];
                        UL[Y.Lptr[g] + (i - Y.Rptr[g]) + (i64)(b - (Y.Stgt + q0)) * mm] = v;
                    }
                }
            }
        }
        for (i64 q = s0; q < s1; q++) ind[Y.Stgt[q]] = -1;
    }
}

// ===== multifrontal LU (chordal/sgetrf.jl:9-290) =====

template <class S, class T> static void sgetrf_chordal(const Sym &Y, T *LD, T *UD, T *LL, T *UL) {
    const i64 nf = Y.nf;
    std::vector<std::vector<T>> M(nf);   // update matrices (the reference keeps them on a stack, Mptr/Mval)
    std::vector<T> F;
    for (i64 f = 0; f < nf; f++) {
        const i64 nn = Y.Rptr[f + 1] - Y.Rptr[f], na = Y.Sptr[f + 1] - Y.Sptr[f], nj = nn + na;
        F.assign(nj * nj, S::zero());
        // F <- F + inj M inj^T for each child, children in reverse (sgetrf_send!, :257-290)
        for (auto it = Y.chd[f].rbegin(); it != Y.chd[f].rend(); ++it) {
            i64 c = *it, nc = Y.Sptr[c + 1] - Y.Sptr[c];
            const std::vector<i64> &inj = Y.rel[c];
            const T *Mc = M[c].data();
            for (i64 w = 0; w < nc; w++)
                for (i64 v = 0; v < nc; v++)
                    F[inj[v] + inj[w] * nj] = S::plus(F[inj[v] + inj[w] * nj], Mc[v + w * nc]);
            std::vector<T>().swap(M[c]);
        }
        T *L11 = LD + Y.Dptr[f], *U11 = UD + Y.Dptr[f];
        T *L21 = LL + Y.Lptr[f], *U12 = UL + Y.Lptr[f];
        if (nn == 1) {
            // sgetrf_loop_1! (:153-255)
            T d11 = S::plus(U11[0], F[0]);
            L11[0] = d11; U11[0] = d11;
            if (na > 0) {
                for (i64 i = 0; i < na; i++) {
                    L21[i] = S::plus(L21[i], F[1 + i]);
                    U12[i] = S::plus(U12[i], F[(1 + i) * nj]);
                }
                if (!S::integral) {
                    T ds = S::star(d11);
                    for (i64 i = 0; i < na; i++) L21[i] = S::prod(L21[i], ds);
                }
                M[f].resize(na * na);
                T *Mf = M[f].data();
                for (i64 w = 0; w < na; w++)
                    for (i64 v = 0; v < na; v++) Mf[v + w * na] = F[(1 + v) + (1 + w) * nj];
                // sger_mt!(s, N, N, R, l21, u12, M22): M[v,w] = smuladd(l21[v], u12[w], M[v,w])
                for (i64 w = 0; w < na; w++)
                    for (i64 v = 0; v < na; v++) Mf[v + w * na] = S::muladd(L21[v], U12[w], Mf[v + w * na]);
            }
            continue;
        }
        // sgetrf_loop! (:35-151)
        for (i64 j = 0; j < nn; j++)
            for (i64 i = 0; i < nn; i++) {
                if (i > j) L11[i + j * nn] = S::plus(F[i + j * nj], L11[i + j * nn]);
                else L11[i + j * nn] = S::plus(F[i + j * nj], U11[i + j * nn]);
            }
        sgetrf2<S>(L11, nn, nn);
        for (i64 j = 0; j < nn; j++)   // copytri!(U11, L11, Val(:U))
            for (i64 i = 0; i <= j; i++) U11[i + j * nn] = L11[i + j * nn];
        if (na > 0) {
            for (i64 c = 0; c < nn; c++)
                for (i64 r = 0; r < na; r++) L21[r + c * na] = S::plus(L21[r + c * na], F[(nn + r) + c * nj]);
            for (i64 c = 0; c < na; c++)
                for (i64 r = 0; r < nn; r++) U12[r + c * nn] = S::plus(U12[r + c * nn], F[r + (nn + c) * nj]);
            trsm_right_upper_nonunit<S>(L11, nn, L21, na, na, nn);   // L21 <- L21 U11*
            trsm_left_lower_unit<S>(L11, nn, U12, nn, nn, na);       // U12 <- L11* U12
            M[f].resize(na * na);
            T *Mf = M[f].data();
            for (i64 w = 0; w < na; w++)
                for (i64 v = 0; v < na; v++) Mf[v + w * na] = F[(nn + v) + (nn + w) * nj];
            sgemx<S>(Mf, na, L21, na, U12, nn, na, na, nn);          // M22 <- L21 U12 + M22
        }
    }
}

// ===== solves (chordal_slu.jl:337-377, chordal/sgetrs.jl:29-51, chordal/strsx.jl) =====
//
// rmul!: B (nrhs x n, column-major, ldb = nrhs) <- B A*.   In the permuted order: U forward, then L backward.
template <class S, class T> static void rmul(const Sym &Y, const T *LD, const T *UD, const T *LL, const T *UL, T *B, i64 nrhs) {
    const i64 n = Y.n, nf = Y.nf;
    std::vector<T> C(n * nrhs);
    // permutecols!(B, work, invp): C[:, invp[j]] = B[:, j]
    for (i64 j = 0; j < n; j++) std::memcpy(&C[Y.invp[j] * nrhs], &B[j * nrhs], nrhs * sizeof(T));
    std::vector<T> Mv;
    // U, forward: C[:, res] <- C[:, res] U11*;  C[:, sep] <- C[:, sep] + C[:, res] U12
    for (i64 f = 0; f < nf; f++) {
        const i64 Rp = Y.Rptr[f], nn = Y.Rptr[f + 1] - Rp, s0 = Y.Sptr[f], na = Y.Sptr[f + 1] - s0;
        const T *D11 = UD + Y.Dptr[f], *U12 = UL + Y.Lptr[f];
        trsm_right_upper_nonunit<S>(D11, nn, &C[Rp * nrhs], nrhs, nrhs, nn);
        for (i64 k = 0; k < na; k++) {
            T *ck = &C[Y.Stgt[s0 + k] * nrhs];
            for (i64 i = 0; i < nn; i++) {
                T u = U12[i + k * nn];
                const T *ci = &C[(Rp + i) * nrhs];
                for (i64 r = 0; r < nrhs; r++) ck[r] = S::muladd(ci[r], u, ck[r]);
            }
        }
    }
    // L, backward: C[:, res] <- C[:, res] + C[:, sep] L21;  C[:, res] <- C[:, res] L11*
    for (i64 f = nf - 1; f >= 0; f--) {
        const i64 Rp = Y.Rptr[f], nn = Y.Rptr[f + 1] - Rp, s0 = Y.Sptr[f], na = Y.Sptr[f + 1] - s0;
        const T *D11 = LD + Y.Dptr[f], *L21 = LL + Y.Lptr[f];
        for (i64 j = 0; j < nn; j++) {
            T *cj = &C[(Rp + j) * nrhs];
            for (i64 k = 0; k < na; k++) {
                T l = L21[k + j * na];
                const T *ck = &C[Y.Stgt[s0 + k] * nrhs];
                for (i64 r = 0; r < nrhs; r++) cj[r] = S::muladd(ck[r], l, cj[r]);
            }
        }
        trsm_right_lower_unit<S>(D11, nn, &C[Rp * nrhs], nrhs, nrhs, nn);
    }
    // permutecols!(B, work, perm): B[:, perm[j]] = C[:, j]
    for (i64 j = 0; j < n; j++) std::memcpy(&B[Y.perm[j] * nrhs], &C[j * nrhs], nrhs * sizeof(T));
}

// lmul!: B (n x nrhs, column-major, ldb = n) <- A* B.  In the permuted order: L forward, then U backward.
template <class S, class T> static void lmul(const Sym &Y, const T *LD, const T *UD, const T *LL, const T *UL, T *B, i64 nrhs) {
    const i64 n = Y.n, nf = Y.nf;
    std::vector<T> C(n * nrhs);
    for (i64 c = 0; c < nrhs; c++)
        for (i64 i = 0; i < n; i++) C[Y.invp[i] + c * n] = B[i + c * n];
    for (i64 c = 0; c < nrhs; c++) {
        T *x = &C[c * n];
        // L, forward: x[res] <- L11* x[res];  x[sep] <- x[sep] + L21 x[res]
        for (i64 f = 0; f < nf; f++) {
            const i64 Rp = Y.Rptr[f], nn = Y.Rptr[f + 1] - Rp, s0 = Y.Sptr[f], na = Y.Sptr[f + 1] - s0;
            const T *D11 = LD + Y.Dptr[f], *L21 = LL + Y.Lptr[f];
            trsm_left_lower_unit<S>(D11, nn, x + Rp, n, nn, 1);
            for (i64 k = 0; k < na; k++) {
                T acc = x[Y.Stgt[s0 + k]];
                for (i64 j = 0; j < nn; j++) acc = S::muladd(L21[k + j * na], x[Rp + j], acc);
                x[Y.Stgt[s0 + k]] = acc;
            }
        }
        // U, backward: x[res] <- x[res] + U12 x[sep];  x[res] <- U11* x[res]
        for (i64 f = nf - 1; f >= 0; f--) {
            const i64 Rp = Y.Rptr[f], nn = Y.Rptr[f + 1] - Rp, s0 = Y.Sptr[f], na = Y.Sptr[f + 1] - s0;
            const T *D11 = UD + Y.Dptr[f], *U12 = UL + Y.Lptr[f];
            for (i64 i = 0; i < nn; i++) {
                T acc = x[Rp + i];
                for (i64 k = 0; k < na; k++) acc = S::muladd(U12[i + k * nn], x[Y.Stgt[s0 + k]], acc);
                x[Rp + i] = acc;
            }
            trsm_left_upper_nonunit<S>(D11, nn, x + Rp, n, nn, 1);
        }
    }
    for (i64 c = 0; c < nrhs; c++)
        for (i64 i = 0; i < n; i++) B[Y.perm[i] + c * n] = C[i + c * n];
}

// ===== full star (chordal/sgetri.jl:13-31) =====
//
// X <- U* (strtri_fwd! per front over the rows of its descendants, chordal/strtri.jl:171-319), then X <- X L*
// (strsx_bwd! over all rows, fronts root to leaves, chordal/strsx.jl:729-867), then the relabel
// C[perm[i], perm[j]] = X[i, j] (permuterowscols!, utils.jl:261-505).  Every row of the star depends only on the
// factor, so the rows are split into blocks of RB and the blocks run in parallel, as the reference's threads do.
// Rows outside [row0, row1) are not computed (a bounded sample for timing); X is the caller's n x n buffer in the
// PERMUTED labels when relabel == 0.

template <class S, class T>
static void star(const Sym &Y, const T *LD, const T *UD, const T *LL, const T *UL, T *C, i64 row0, i64 row1, int relabel, int nthreads) {
    const i64 n = Y.n, nf = Y.nf;
    // X11 = strtri(D11) of every front, once (dense/strtri.jl: strtri2! upper, diag :N)
    std::vector<T> T11(Y.Dptr[nf]);
    for (i64 f = 0; f < nf; f++) {
        const i64 nn = Y.Rptr[f + 1] - Y.Rptr[f];
        T *t = &T11[Y.Dptr[f]];
        const T *d = UD + Y.Dptr[f];
        for (i64 j = 0; j < nn; j++)
            for (i64 i = 0; i < nn; i++) t[i + j * nn] = i <= j ? d[i + j * nn] : S::zero();
        strtri2_upper<S>(t, nn, nn, true);
    }
    T *X = C;
    std::vector<T> Xbuf;
    if (relabel) { Xbuf.resize((size_t)n * n); X = Xbuf.data(); }
    const i64 RB = 32;
    const i64 nblk = (row1 - row0 + RB - 1) / RB;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        std::vector<T> M2, Xrow;
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (i64 b = 0; b < nblk; b++) {
            const i64 r0 = row0 + b * RB, r1 = std::min(row1, r0 + RB);
            for (i64 c = 0; c < n; c++)
                for (i64 r = r0; r < r1; r++) X[r + c * n] = S::zero();
            // X <- U*, rows [r0, r1) only
            for (i64 f = 0; f < nf; f++) {
                const i64 Rp = Y.Rptr[f], nn = Y.Rptr[f + 1] - Rp, s0 = Y.Sptr[f], na = Y.Sptr[f + 1] - s0;
                const i64 rs = std::max(r0, Y.Rptr[Y.fdsc[f]]), re = std::min(r1, Rp + nn);
                if (rs >= re) continue;
                const T *D11 = UD + Y.Dptr[f], *U12 = UL + Y.Lptr[f];
                // X11 <- strtri(D11) for the rows in res(f)
                for (i64 r = std::max(rs, Rp); r < re; r++)
                    for (i64 j = 0; j < nn; j++) X[r + (Rp + j) * n] = T11[Y.Dptr[f] + (r - Rp) + j * nn];
                // X01 <- X01 D11* for the rows of strict descendants
                const i64 qe = std::min(re, Rp);
                if (rs < qe) trsm_right_upper_nonunit<S>(D11, nn, &X[rs + Rp * n], n, qe - rs, nn);
                // M2 <- X1 U12;  X2 <- X2 + M2
                const i64 nr = re - rs;
                M2.assign(nr * na, S::zero());
                sgemx<S>(M2.data(), nr, &X[rs + Rp * n], n, U12, nn, nr, na, nn);
                for (i64 k = 0; k < na; k++) {
                    T *x = &X[rs + Y.Stgt[s0 + k] * n];
                    for (i64 r = 0; r < nr; r++) x[r] = S::plus(x[r], M2[r + k * nr]);
                }
            }
            // X <- X L*, fronts root to leaves
            const i64 nr = r1 - r0;
            for (i64 f = nf - 1; f >= 0; f--) {
                const i64 Rp = Y.Rptr[f], nn = Y.Rptr[f + 1] - Rp, s0 = Y.Sptr[f], na = Y.Sptr[f + 1] - s0;
                const T *D11 = LD + Y.Dptr[f], *L21 = LL + Y.Lptr[f];
                if (na > 0) {
                    // M2 <- X[:, sep] (copygatherrec!);  X1 <- X1 + M2 L21
                    M2.resize(nr * na);
                    for (i64 k = 0; k < na; k++) std::memcpy(&M2[k * nr], &X[r0 + Y.Stgt[s0 + k] * n], nr * sizeof(T));
                    sgemx<S>(&X[r0 + Rp * n], n, M2.data(), nr, L21, na, nr, nn, na);
                }
                trsm_right_lower_unit<S>(D11, nn, &X[r0 + Rp * n], n, nr, nn);
            }
            if (relabel)
                for (i64 c = 0; c < n; c++) {
                    T *dst = C + Y.perm[c] * n;
                    const T *src = X + c * n;
                    for (i64 r = r0; r < r1; r++) dst[Y.perm[r]] = src[r];
                }
        }
    }
}

// ===== strongly connected components (src/CPU/blocked/*.jl) =====
//
// The structure's vertices are grouped by component in a topological order: component c holds the permuted vertices
// [Bptr[c], Bptr[c+1]) and the fronts [Fptr[c], Fptr[c+1]); the factor is that of the diagonal blocks.  N holds the
// arcs between components in the permuted labels, by column j (Nptr, Nidx = rows i < Bptr[comp(j)], ascending;
// Nval = A[i, j]).

// soffd (chordal_ssymbolic.jl:212-269): the entries of column j of the permuted A whose row lies in an earlier
// component.  Returns their number; with Nidx / Nval null only Nptr is filled.
template <class T>
static i64 offd(const Sym &Y, const i64 *Bptr, i64 nB, const i64 *colptr, const i64 *rowval, const T *nzval, i64 *Nptr,
                i64 *Nidx, T *Nval) {
    const i64 n = Y.n;
    std::vector<i64> start(n);
    for (i64 c = 0; c < nB; c++)
        for (i64 j = Bptr[c]; j < Bptr[c + 1]; j++) start[j] = Bptr[c];
    Nptr[0] = 0;
    std::vector<std::pair<i64, T>> col;
    for (i64 j = 0; j < n; j++) {
        const i64 oc = Y.perm[j];
        col.clear();
        for (i64 p = colptr[oc]; p < colptr[oc + 1]; p++) {
            const i64 i = Y.invp[rowval[p]];
            if (i < start[j]) col.push_back({i, nzval ? nzval[p] : T(0)});
        }
        std::sort(col.begin(), col.end(), [](const std::pair<i64, T> &a, const std::pair<i64, T> &b) { return a.first < b.first; });
        if (Nidx)
            for (size_t k = 0; k < col.size(); k++) {
                Nidx[Nptr[j] + k] = col[k].first;
                Nval[Nptr[j] + k] = col[k].second;
            }
        Nptr[j + 1] = Nptr[j] + (i64)col.size();
    }
    return Nptr[n];
}

// The fronts of component c, from the vertex ranges.
static void comp_fronts(const Sym &Y, const i64 *Bptr, i64 nB, std::vector<i64> &Fptr) {
    Fptr.assign(nB + 1, Y.nf);
    for (i64 c = nB - 1; c >= 0; c--) Fptr[c] = Bptr[c] < Bptr[c + 1] ? Y.idx[Bptr[c]] : Fptr[c + 1];
}

// C[:, cols] with the rows of fronts [f0, f1) <- A_cc* C (lmul! over one component's fronts: L forward, then U
// backward; chordal/sgetrs.jl:29-51 restricted to fronts fstrt:fstop, as blocked/sgetri.jl:109 calls it); C is
// n x m column-major (ldc).
template <class S, class T>
static void lmul_fronts(const Sym &Y, const T *LD, const T *UD, const T *LL, const T *UL, T *C, i64 ldc, i64 m, i64 f0,
                        i64 f1) {
    for (i64 col = 0; col < m; col++) {
        T *x = C + col * ldc;
        for (i64 f = f0; f < f1; f++) {
            const i64 Rp = Y.Rptr[f], nn = Y.Rptr[f + 1] - Rp, s0 = Y.Sptr[f], na = Y.Sptr[f + 1] - s0;
            const T *D11 = LD + Y.Dptr[f], *L21 = LL + Y.Lptr[f];
            trsm_left_lower_unit<S>(D11, nn, x + Rp, ldc, nn, 1);
            for (i64 k = 0; k < na; k++) {
                T acc = x[Y.Stgt[s0 + k]];
                for (i64 j = 0; j < nn; j++) acc = S::muladd(L21[k + j * na], x[Rp + j], acc);
                x[Y.Stgt[s0 + k]] = acc;
            }
        }
        for (i64 f = f1 - 1; f >= f0; f--) {
            const i64 Rp = Y.Rptr[f], nn = Y.Rptr[f + 1] - Rp, s0 = Y.Sptr[f], na = Y.Sptr[f + 1] - s0;
            const T *D11 = UD + Y.Dptr[f], *U12 = UL + Y.Lptr[f];
            for (i64 i = 0; i < nn; i++) {
                T acc = x[Rp + i];
                for (i64 k = 0; k < na; k++) acc = S::muladd(U12[i + k * nn], x[Y.Stgt[s0 + k]], acc);
                x[Rp + i] = acc;
            }
            trsm_left_upper_nonunit<S>(D11, nn, x + Rp, ldc, nn, 1);
        }
    }
}

// C (nrhs x n, ldc = nrhs, permuted columns) <- C A_cc* over the fronts [f0, f1) (rmul!: U forward, then L backward)
template <class S, class T>
static void rmul_fronts(const Sym &Y, const T *LD, const T *UD, const T *LL, const T *UL, T *C, i64 nrhs, i64 f0, i64 f1) {
    for (i64 f = f0; f < f1; f++) {
        const i64 Rp = Y.Rptr[f], nn = Y.Rptr[f + 1] - Rp, s0 = Y.Sptr[f], na = Y.Sptr[f + 1] - s0;
        const T *D11 = UD + Y.Dptr[f], *U12 = UL + Y.Lptr[f];
        trsm_right_upper_nonunit<S>(D11, nn, &C[Rp * nrhs], nrhs, nrhs, nn);
        for (i64 k = 0; k < na; k++) {
            T *ck = &C[Y.Stgt[s0 + k] * nrhs];
            for (i64 i = 0; i < nn; i++) {
                T u = U12[i + k * nn];
                const T *ci = &C[(Rp + i) * nrhs];
                for (i64 r = 0; r < nrhs; r++) ck[r] = S::muladd(ci[r], u, ck[r]);
            }
        }
    }
    for (i64 f = f1 - 1; f >= f0; f--) {
        const i64 Rp = Y.Rptr[f], nn = Y.Rptr[f + 1] - Rp, s0 = Y.Sptr[f], na = Y.Sptr[f + 1] - s0;
        const T *D11 = LD + Y.Dptr[f], *L21 = LL + Y.Lptr[f];
        for (i64 j = 0; j < nn; j++) {
            T *cj = &C[(Rp + j) * nrhs];
            for (i64 k = 0; k < na; k++) {
                T l = L21[k + j * na];
                const T *ck = &C[Y.Stgt[s0 + k] * nrhs];
                for (i64 r = 0; r < nrhs; r++) cj[r] = S::muladd(ck[r], l, cj[r]);
            }
        }
        trsm_right_lower_unit<S>(D11, nn, &C[Rp * nrhs], nrhs, nrhs, nn);
    }
}

// rmul! over the components (blocked/sgetrs.jl:80-122 with side :R, trans :N: components in increasing order, each
// first gathering its arcs from earlier components, X[:, j] <- X[:, j] (+) sum_i X[:, i] (x) N[i, j]
// (sgemx_sparse!), then solving with its own fronts).  B: nrhs x n.
template <class S, class T>
static void rmul_scc(const Sym &Y, const T *LD, const T *UD, const T *LL, const T *UL, const i64 *Bptr, i64 nB,
                     const i64 *Nptr, const i64 *Nidx, const T *Nval, T *B, i64 nrhs) {
    const i64 n = Y.n;
    std::vector<i64> Fptr;
    comp_fronts(Y, Bptr, nB, Fptr);
    std::vector<T> C(n * nrhs);
    for (i64 j = 0; j < n; j++) std::memcpy(&C[Y.invp[j] * nrhs], &B[j * nrhs], nrhs * sizeof(T));
    for (i64 c = 0; c < nB; c++) {
        for (i64 j = Bptr[c]; j < Bptr[c + 1]; j++) {
            T *cj = &C[j * nrhs];
            for (i64 q = Nptr[j]; q < Nptr[j + 1]; q++) {
                const T *ci = &C[Nidx[q] * nrhs];
                for (i64 r = 0; r < nrhs; r++) cj[r] = S::muladd(ci[r], Nval[q], cj[r]);
            }
        }
        rmul_fronts<S>(Y, LD, UD, LL, UL, C.data(), nrhs, Fptr[c], Fptr[c + 1]);
    }
    for (i64 j = 0; j < n; j++) std::memcpy(&B[Y.perm[j] * nrhs], &C[j * nrhs], nrhs * sizeof(T));
}

// lmul! over the components (side :L, trans :N: components in decreasing order, each solving with its own fronts,
// then pushing its rows to the earlier components, X[i, :] <- X[i, :] (+) N[i, j] (x) X[j, :]).  B: n x nrhs.
template <class S, class T>
static void lmul_scc(const Sym &Y, const T *LD, const T *UD, const T *LL, const T *UL, const i64 *Bptr, i64 nB,
                     const i64 *Nptr, const i64 *Nidx, const T *Nval, T *B, i64 nrhs) {
    const i64 n = Y.n;
    std::vector<i64> Fptr;
    comp_fronts(Y, Bptr, nB, Fptr);
    std::vector<T> C(n * nrhs);
    for (i64 col = 0; col < nrhs; col++)
        for (i64 i = 0; i < n; i++) C[Y.invp[i] + col * n] = B[i + col * n];
    for (i64 c = nB - 1; c >= 0; c--) {
        lmul_fronts<S>(Y, LD, UD, LL, UL, C.data(), n, nrhs, Fptr[c], Fptr[c + 1]);
        for (i64 col = 0; col < nrhs; col++) {
            T *x = &C[col * n];
            for (i64 j = Bptr[c]; j < Bptr[c + 1]; j++)
                for (i64 q = Nptr[j]; q < Nptr[j + 1]; q++) x[Nidx[q]] = S::muladd(Nval[q], x[j], x[Nidx[q]]);
        }
    }
    for (i64 col = 0; col < nrhs; col++)
        for (i64 i = 0; i < n; i++) B[Y.perm[i] + col * n] = C[i + col * n];
}

// The star over the components (blocked/sgetri.jl:3-162): the diagonal blocks A_cc* by the chordal star (star(),
// rows of other components stay zero), then for each component d whose columns N reaches, the components with a
// path into d (sgetri_reach!) in an order that visits every component after all those it has arcs into (decreasing
// number: every arc goes to a higher one): C[rows of c, cols of d] <- A_cc* C[rows of c, cols of d] (c != d), then
// C[rows of b, cols of d] <- (+) N[b, c] (x) C[rows of c, cols of d] for the arcs b -> c (sgemx_sparse!).
template <class S, class T>
static void star_scc(const Sym &Y, const T *LD, const T *UD, const T *LL, const T *UL, const i64 *Bptr, i64 nB,
                     const i64 *Nptr, const i64 *Nidx, const T *Nval, T *C, int nthreads) {
    const i64 n = Y.n;
    std::vector<T> X((size_t)n * n);
    star<S>(Y, LD, UD, LL, UL, X.data(), 0, n, 0, nthreads);
    std::vector<i64> Fptr, comp(n);
    comp_fronts(Y, Bptr, nB, Fptr);
    for (i64 c = 0; c < nB; c++)
        for (i64 j = Bptr[c]; j < Bptr[c + 1]; j++) comp[j] = c;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        std::vector<char> anc(nB);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (i64 d = 0; d < nB; d++) {
            const i64 j0 = Bptr[d], j1 = Bptr[d + 1];
            if (Nptr[j0] == Nptr[j1]) continue;
            // the components with a path into d (sgetri_reach!)
            std::fill(anc.begin(), anc.end(), 0);
            anc[d] = 1;
            for (i64 c = d; c >= 0; c--) {
                if (!anc[c]) continue;
                for (i64 j = Bptr[c]; j < Bptr[c + 1]; j++)
                    for (i64 q = Nptr[j]; q < Nptr[j + 1]; q++) anc[comp[Nidx[q]]] = 1;
            }
            T *Cd = X.data() + j0 * n;
            const i64 m = j1 - j0;
            for (i64 c = d; c >= 0; c--) {
                if (!anc[c]) continue;
                if (c != d) lmul_fronts<S>(Y, LD, UD, LL, UL, Cd, n, m, Fptr[c], Fptr[c + 1]);
                for (i64 j = Bptr[c]; j < Bptr[c + 1]; j++)
                    for (i64 q = Nptr[j]; q < Nptr[j + 1]; q++)
                        for (i64 col = 0; col < m; col++) {
                            T *x = Cd + col * n;
                            x[Nidx[q]] = S::muladd(Nval[q], x[j], x[Nidx[q]]);
                        }
            }
        }
    }
    for (i64 c = 0; c < n; c++) {
        T *dst = C + Y.perm[c] * n;
        const T *src = X.data() + c * n;
        for (i64 r = 0; r < n; r++) dst[Y.perm[r]] = src[r];
    }
}

// ===== batched getrf + star of dense fronts (ext/PATHPACKCUDAExt/batched/sgetrf.jl:11-120) =====
//
// A (nb x nb, column-major, batch of them back to back) <- L + U;  TU <- U*;  TL <- L* (unit lower).
// TU[r, j] = (TU[r, j] + sum_{k<j} TU[r, k] U[k, j]) U[j, j]*, starting from I;
// TL[i, c] = TL[i, c] + sum_{k<i} L[i, k] TL[k, c], starting from I.
template <class S, class T> static void getrf_star_batched(i64 nb, i64 batch, T *A, T *TL, T *TU, int nthreads) {
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
    for (i64 b = 0; b < batch; b++) {
        T *a = A + b * nb * nb, *tl = TL + b * nb * nb, *tu = TU + b * nb * nb;
        sgetrf2<S>(a, nb, nb);
        for (i64 j = 0; j < nb; j++)
            for (i64 i = 0; i < nb; i++) {
                tu[i + j * nb] = i == j ? S::one() : S::zero();
                tl[i + j * nb] = i == j ? S::one() : S::zero();
            }
        for (i64 j = 0; j < nb; j++)
            for (i64 r = 0; r < nb; r++) {
                T part = S::zero();
                for (i64 k = 0; k < j; k++) part = S::muladd(tu[r + k * nb], a[k + j * nb], part);
                T acc = S::plus(tu[r + j * nb], part);
                if (!S::integral) acc = S::prod(acc, S::star(a[j + j * nb]));
                tu[r + j * nb] = acc;
            }
        for (i64 i = 0; i < nb; i++)
            for (i64 c = 0; c < nb; c++) {
                T part = S::zero();
                for (i64 k = 0; k < i; k++) part = S::muladd(a[i + k * nb], tl[k + c * nb], part);
                tl[i + c * nb] = S::plus(tl[i + c * nb], part);
            }
    }
}

// C <- C + A B over output columns in parallel (the GEMM microbenchmark's CPU side)
template <class S, class T>
static void sgemx_omp(T *C, i64 ldc, const T *A, i64 lda, const T *B, i64 ldb, i64 m, i64 n, i64 k, int nthreads) {
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
    for (i64 c = 0; c < n; c++) sgemx<S>(C + c * ldc, ldc, A, lda, B + c * ldb, ldb, m, 1, k);
}

// ===== dispatch =====

#define PPO_DISPATCH(sr, dt, CALL)                                                                   \
    do {                                                                                             \
        if (dt == D_F32) {                                                                           \
            typedef float T;                                                                         \
            switch (sr) {                                                                            \
            case S_MINPLUS: { typedef MinPlus<T> S; CALL; return 0; }                               \
            case S_MAXPLUS: { typedef MaxPlus<T> S; CALL; return 0; }                               \
            case S_MAXMIN: { typedef MaxMin<T> S; CALL; return 0; }                                 \
            case S_MINMAX: { typedef MinMax<T> S; CALL; return 0; }                                 \
            case S_PLUSPROD: { typedef PlusProd<T> S; CALL; return 0; }                             \
            }                                                                                        \
        } else if (dt == D_F64) {                                                                    \
            typedef double T;                                                                        \
            switch (sr) {                                                                            \
            case S_MINPLUS: { typedef MinPlus<T> S; CALL; return 0; }                               \
            case S_MAXPLUS: { typedef MaxPlus<T> S; CALL; return 0; }                               \
            case S_MAXMIN: { typedef MaxMin<T> S; CALL; return 0; }                                 \
            case S_MINMAX: { typedef MinMax<T> S; CALL; return 0; }                                 \
            case S_PLUSPROD: { typedef PlusProd<T> S; CALL; return 0; }                             \
            }                                                                                        \
        } else if (dt == D_I32 && sr == S_ORAND) {                                                   \
            typedef int32_t T;                                                                       \
            typedef OrAnd<T> S;                                                                      \
            CALL;                                                                                    \
            return 0;                                                                                \
        }                                                                                            \
        return -100;                                                                                 \
    } while (0)

extern "C" {

int ppo_factor(int sr, int dt, i64 n, i64 nf, const i64 *Rptr, const i64 *Sptr, const i64 *Stgt, const i64 *perm,
               const i64 *colptr, const i64 *rowval, const void *nzval, void *LD, void *UD, void *LL, void *UL) {
    Sym Y;
    int e = build_sym(Y, n, nf, Rptr, Sptr, Stgt, perm);
    if (e) return e;
    PPO_DISPATCH(sr, dt, (scopyto<S, T>(Y, colptr, rowval, (const T *)nzval, (T *)LD, (T *)UD, (T *)LL, (T *)UL),
                          sgetrf_chordal<S, T>(Y, (T *)LD, (T *)UD, (T *)LL, (T *)UL)));
}

// scatter only (no LU): the initial factor storage, for tests of the scatter itself
int ppo_scatter(int sr, int dt, i64 n, i64 nf, const i64 *Rptr, const i64 *Sptr, const i64 *Stgt, const i64 *perm,
                const i64 *colptr, const i64 *rowval, const void *nzval, void *LD, void *UD, void *LL, void *UL) {
    Sym Y;
    int e = build_sym(Y, n, nf, Rptr, Sptr, Stgt, perm);
    if (e) return e;
    PPO_DISPATCH(sr, dt, (scopyto<S, T>(Y, colptr, rowval, (const T *)nzval, (T *)LD, (T *)UD, (T *)LL, (T *)UL)));
}

int ppo_rmul(int sr, int dt, i64 n, i64 nf, const i64 *Rptr, const i64 *Sptr, const i64 *Stgt, const i64 *perm,
             const void *LD, const void *UD, const void *LL, const void *UL, void *B, i64 nrhs) {
    Sym Y;
    int e = build_sym(Y, n, nf, Rptr, Sptr, Stgt, perm);
    if (e) return e;
    PPO_DISPATCH(sr, dt, (rmul<S, T>(Y, (const T *)LD, (const T *)UD, (const T *)LL, (const T *)UL, (T *)B, nrhs)));
}

int ppo_lmul(int sr, int dt, i64 n, i64 nf, const i64 *Rptr, const i64 *Sptr, const i64 *Stgt, const i64 *perm,
             const void *LD, const void *UD, const void *LL, const void *UL, void *B, i64 nrhs) {
    Sym Y;
    int e = build_sym(Y, n, nf, Rptr, Sptr, Stgt, perm);
    if (e) return e;
    PPO_DISPATCH(sr, dt, (lmul<S, T>(Y, (const T *)LD, (const T *)UD, (const T *)LL, (const T *)UL, (T *)B, nrhs)));
}

int ppo_star(int sr, int dt, i64 n, i64 nf, const i64 *Rptr, const i64 *Sptr, const i64 *Stgt, const i64 *perm,
             const void *LD, const void *UD, const void *LL, const void *UL, void *C, i64 row0, i64 row1, int relabel,
             int nthreads) {
    Sym Y;
    int e = build_sym(Y, n, nf, Rptr, Sptr, Stgt, perm);
    if (e) return e;
    if (row0 < 0 || row1 > n || row0 > row1) return -5;
    PPO_DISPATCH(sr, dt, (star<S, T>(Y, (const T *)LD, (const T *)UD, (const T *)LL, (const T *)UL, (T *)C, row0, row1, relabel, nthreads)));
}

// N of a structure with components (soffd): Nptr (n + 1) always; Nidx / Nval (capacity nnz) when not null.
// Returns the number of arcs, or a negative error.
i64 ppo_offd(int sr, int dt, i64 n, i64 nf, const i64 *Rptr, const i64 *Sptr, const i64 *Stgt, const i64 *perm, i64 nB,
             const i64 *Bptr, const i64 *colptr, const i64 *rowval, const void *nzval, i64 *Nptr, i64 *Nidx, void *Nval) {
    Sym Y;
    int e = build_sym(Y, n, nf, Rptr, Sptr, Stgt, perm);
    if (e) return e;
    i64 cnt = -100;
    if (dt == D_F32) cnt = offd<float>(Y, Bptr, nB, colptr, rowval, (const float *)nzval, Nptr, Nidx, (float *)Nval);
    else if (dt == D_F64) cnt = offd<double>(Y, Bptr, nB, colptr, rowval, (const double *)nzval, Nptr, Nidx, (double *)Nval);
    else if (dt == D_I32) cnt = offd<int32_t>(Y, Bptr, nB, colptr, rowval, (const int32_t *)nzval, Nptr, Nidx, (int32_t *)Nval);
    (void)sr;
    return cnt;
}

int ppo_rmul_scc(int sr, int dt, i64 n, i64 nf, const i64 *Rptr, const i64 *Sptr, const i64 *Stgt, const i64 *perm,
                 const void *LD, const void *UD, const void *LL, const void *UL, i64 nB, const i64 *Bptr, const i64 *Nptr,
                 const i64 *Nidx, const void *Nval, void *B, i64 nrhs) {
    Sym Y;
    int e = build_sym(Y, n, nf, Rptr, Sptr, Stgt, perm);
    if (e) return e;
    PPO_DISPATCH(sr, dt, (rmul_scc<S, T>(Y, (const T *)LD, (const T *)UD, (const T *)LL, (const T *)UL, Bptr, nB, Nptr,
                                         Nidx, (const T *)Nval, (T *)B, nrhs)));
}

int ppo_lmul_scc(int sr, int dt, i64 n, i64 nf, const i64 *Rptr, const i64 *Sptr, const i64 *Stgt, const i64 *perm,
                 const void *LD, const void *UD, const void *LL, const void *UL, i64 nB, const i64 *Bptr, const i64 *Nptr,
                 const i64 *Nidx, const void *Nval, void *B, i64 nrhs) {
    Sym Y;
    int e = build_sym(Y, n, nf, Rptr, Sptr, Stgt, perm);
    if (e) return e;
    PPO_DISPATCH(sr, dt, (lmul_scc<S, T>(Y, (const T *)LD, (const T *)UD, (const T *)LL, (const T *)UL, Bptr, nB, Nptr,
                                         Nidx, (const T *)Nval, (T *)B, nrhs)));
}

int ppo_star_scc(int sr, int dt, i64 n, i64 nf, const i64 *Rptr, const i64 *Sptr, const i64 *Stgt, const i64 *perm,
                 const void *LD, const void *UD, const void *LL, const void *UL, i64 nB, const i64 *Bptr, const i64 *Nptr,
                 const i64 *Nidx, const void *Nval, void *C, int nthreads) {
    Sym Y;
    int e = build_sym(Y, n, nf, Rptr, Sptr, Stgt, perm);
    if (e) return e;
    PPO_DISPATCH(sr, dt, (star_scc<S, T>(Y, (const T *)LD, (const T *)UD, (const T *)LL, (const T *)UL, Bptr, nB, Nptr,
                                         Nidx, (const T *)Nval, (T *)C, nthreads)));
}

int ppo_sgemx(int sr, int dt, i64 m, i64 n, i64 k, const void *A, i64 lda, const void *B, i64 ldb, void *C, i64 ldc, int nthreads) {
    PPO_DISPATCH(sr, dt, (sgemx_omp<S>((T *)C, ldc, (const T *)A, lda, (const T *)B, ldb, m, n, k, nthreads)));
}

int ppo_getrf(int sr, int dt, i64 n, void *A, i64 lda) {
    PPO_DISPATCH(sr, dt, (sgetrf2<S>((T *)A, lda, n)));
}

int ppo_getrf_star_batched(int sr, int dt, i64 nb, i64 batch, void *A, void *TL, void *TU, int nthreads) {
    PPO_DISPATCH(sr, dt, (getrf_star_batched<S>(nb, batch, (T *)A, (T *)TL, (T *)TU, nthreads)));
}

int ppo_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

}  // extern "C"
