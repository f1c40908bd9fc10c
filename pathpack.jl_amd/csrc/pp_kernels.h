// pp_kernels.h -- gfx950 kernels and the numeric drivers of the multifrontal semiring LU (templates).
//
// Included once per semiring/element type by the pp_inst_*.hip translation units, which instantiate the drivers.
//
// Reference behaviour (file:line in AlgebraicJulia/PATHPACK.jl):
//   factorization     src/CPU/chordal/sgetrf.jl:35-290, src/CPU/dense/sgetrf.jl:151-175
//   star              src/CPU/chordal/sgetri.jl:13-31 (X <- U*, X <- X L*), src/CPU/utils.jl:261-505 (relabel)
//   solves            src/CPU/chordal_slu.jl:337-377, src/CPU/chordal/sgetrs.jl:29-51, src/CPU/chordal/strsx.jl
//   dense GEMM        src/CPU/dense/sgemx.jl:606-635
//   front LU + stars  ext/PATHPACKCUDAExt/batched/sgetrf.jl:11-120
// The plans these kernels run are described in pp_internal.h.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cstdio>
#include <cstring>
#include <functional>
#include <type_traits>

#include "pathpack_hip.h"
#include "pp_internal.h"
#include "pp_semiring.h"

namespace pp {

#define HIPCHK(x)                                                                  \
    do {                                                                           \
        hipError_t e_ = (x);                                                       \
        if (e_ != hipSuccess) return std::string(#x ": ") + hipGetErrorString(e_); \
    } while (0)

#define LAUNCHCHK()                                                                            \
    do {                                                                                       \
        hipError_t e_ = hipGetLastError();                                                     \
        if (e_ != hipSuccess) return std::string("kernel launch: ") + hipGetErrorString(e_);   \
    } while (0)

constexpr int NT = 256;


static inline unsigned grid1(i64 work, int per = NT) {
    i64 g = (work + per - 1) / per;
    return (unsigned)std::max<i64>(1, std::min<i64>(g, 1 << 20));
}

// ===== elementwise =====

template <class T> __global__ void k_fill(T *__restrict__ p, i64 n, T v) {
    for (i64 i = blockIdx.x * (i64)NT + threadIdx.x; i < n; i += (i64)gridDim.x * NT) p[i] = v;
}

// F[pos[i]] = val[i] for the entries with a position (pos < 0: an arc between components, which N holds)
template <class T>
__global__ void k_scatter_entries(T *__restrict__ F, const i64 *__restrict__ pos, const T *__restrict__ val, i64 nnz) {
    for (i64 i = blockIdx.x * (i64)NT + threadIdx.x; i < nnz; i += (i64)gridDim.x * NT) {
        const i64 q = pos[i];
        if (q >= 0) F[q] = val[i];
    }
}

// dst[q] = src[idx[q]]: the values of N (by column and by row) from A's values
// dst[i + j ldd] = src[i + j lds] for i < rows, j < cols: blockIdx.y strides over the columns, the threads of x over
// the rows
template <class T>
__global__ __launch_bounds__(NT) void k_copy2d(T *__restrict__ dst, i64 ldd, const T *__restrict__ src, i64 lds,
                                                i64 rows, i64 cols) {
    for (i64 j = blockIdx.y; j < cols; j += gridDim.y)
        for (i64 i = blockIdx.x * (i64)NT + threadIdx.x; i < rows; i += (i64)gridDim.x * NT) dst[i + j * ldd] = src[i + j * lds];
}

template <class T>
__global__ void k_gather(T *__restrict__ dst, const T *__restrict__ src, const i64 *__restrict__ idx, i64 m) {
    for (i64 q = blockIdx.x * (i64)NT + threadIdx.x; q < m; q += (i64)gridDim.x * NT) dst[q] = src[idx[q]];
}

// X <- I in the semiring (the start of X <- U*; row i is the unit vector of source rsrc[i], or of i), on the entries
// the sweeps read before writing them, for the units p (units[], or all panels): column c of p over the rows
// [alo[p], ahi[p]) of its subtree (every forward write into column c comes from a panel of
// that subtree; the backward sweep takes the other rows of its component as zero), and over the rows outside the
// component [blo[p], bhi[p]), which no sweep visits.
template <class S>
__global__ __launch_bounds__(NT) void k_identity_panels(typename S::value_type *__restrict__ X, i64 n,
                                                        const int32_t *__restrict__ units, const int32_t *__restrict__ rsrc,
                                                        i64 ncols,
                                                        const int32_t *__restrict__ c0, const int32_t *__restrict__ w,
                                                        const int32_t *__restrict__ alo, const int32_t *__restrict__ ahi,
                                                        const int32_t *__restrict__ blo,
                                                        const int32_t *__restrict__ bhi) {
    typedef typename S::value_type T;
    const int p = units ? units[blockIdx.x] : (int)blockIdx.x;
    for (int j = blockIdx.y; j < w[p]; j += gridDim.y) {
        const i64 col = c0[p] + j;
        T *x = X + col * n;
        for (i64 i = alo[p] + threadIdx.x; i < ahi[p]; i += NT)
            x[i] = (rsrc ? (i64)rsrc[i] : i) == col ? S::one() : S::zero();
        for (i64 i = threadIdx.x; i < blo[p]; i += NT) x[i] = S::zero();
        for (i64 i = bhi[p] + threadIdx.x; i < n; i += NT) x[i] = S::zero();
    }
    (void)ncols;
}

// ===== extend-add: F_f <- F_f (+) inj M_c inj^T for every child c (sgetrf_send!, chordal/sgetrf.jl:257-290) =====
//
// One workgroup per (parent front, block of `blk` parent columns; blk = ASM_BLOCK, or down to 4 on a level with few
// parent columns).  A child's map into its parent's bag (relpos)
// is increasing, so the child columns landing in the block are a contiguous range found by binary search; blocks of
// one parent never write the same entry, and the children of a parent are added one after another.
template <class S>
__global__ __launch_bounds__(NT) void k_assemble(typename S::value_type *__restrict__ F, const i64 *__restrict__ Foff,
                                                 const int32_t *__restrict__ nn, const int32_t *__restrict__ na,
                                                 const int32_t *__restrict__ nj, const i64 *__restrict__ Sptr,
                                                 const int32_t *__restrict__ relpos, const int32_t *__restrict__ chptr,
                                                 const int32_t *__restrict__ chidx, const int32_t *__restrict__ tasks,
                                                 int blk) {
    typedef typename S::value_type T;
    const int f = tasks[2 * blockIdx.x], a = tasks[2 * blockIdx.x + 1];
    const int ldf = nj[f];
    const int b = min(ldf, a + blk);
    T *Ff = F + Foff[f];
    for (int q = chptr[f]; q < chptr[f + 1]; q++) {
        const int c = chidx[q];
        const int nc = na[c], ldc = nj[c], off = nn[c];
        const T *M = F + Foff[c] + off + (i64)off * ldc;
        const int32_t *rp = relpos + Sptr[c];
        // child columns w with a <= rp[w] < b
        int lo = 0, hi = nc;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (rp[mid] < a) lo = mid + 1;
            else hi = mid;
        }
        int w1 = lo;
        while (w1 < nc && rp[w1] < b) w1++;
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        for (int w = lo + wave; w < w1; w += NT / 64) {
            T *dcol = Ff + (i64)rp[w] * ldf;
            const T *scol = M + (i64)w * ldc;
            // four rows per lane in flight: every load of a batch is issued before its stores (the rows of one child
            // column land on distinct parent rows, and the child's update block does not overlap the parent front)
            int v = lane;
            for (; v + 192 < nc; v += 256) {
                int q[4];
                T x[4], y[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    q[u] = rp[v + 64 * u];
                    x[u] = scol[v + 64 * u];
                }
#pragma unroll
                for (int u = 0; u < 4; u++) y[u] = dcol[q[u]];
#pragma unroll
                for (int u = 0; u < 4; u++) dcol[q[u]] = S::plus(y[u], x[u]);
            }
            for (; v < nc; v += 64) dcol[rp[v]] = S::plus(dcol[rp[v]], scol[v]);
        }
        __syncthreads();
    }
}

// ===== dense LU of an n x n block in LDS (ld = lda), first p pivots (dense/sgetrf.jl:151-175) =====

template <class S>
__device__ inline void lds_lu(typename S::value_type *A, int n, int lda, int p) {
    // waves take columns, lanes take rows: no integer division in the update
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int i = 0; i < p; i++) {
        if (!S::integral) {
            const typename S::value_type s = S::star(A[i + i * lda]);
            for (int k = i + 1 + (int)threadIdx.x; k < n; k += (int)blockDim.x) A[k + i * lda] = S::prod(A[k + i * lda], s);
            __syncthreads();
        }
        for (int j = i + 1 + wave; j < n; j += nw) {
            const typename S::value_type aij = A[i + j * lda];
            for (int k = i + 1 + lane; k < n; k += 64) A[k + j * lda] = S::muladd(A[k + i * lda], aij, A[k + j * lda]);
        }
        __syncthreads();
    }
}

// fronts with nj <= MAXN: the whole partial LU (nn pivots of the nj x nj front) in one workgroup
template <class S, int MAXN>
__global__ __launch_bounds__(NT) void k_front_small(typename S::value_type *__restrict__ F, const i64 *__restrict__ Foff,
                                                    const int32_t *__restrict__ nn, const int32_t *__restrict__ nj,
                                                    const int32_t *__restrict__ list) {
    typedef typename S::value_type T;
    __shared__ T A[MAXN * MAXN];
    const int f = list[blockIdx.x];
    const int n = nj[f], p = nn[f];
    T *G = F + Foff[f];
    for (int e = threadIdx.x; e < n * n; e += NT) A[e] = G[e];
    __syncthreads();
    lds_lu<S>(A, n, n, p);
    for (int e = threadIdx.x; e < n * n; e += NT) G[e] = A[e];
}

// value of v in lane `src` of the wave (src uniform)
template <class T> __device__ inline T bcast_lane(T v, int src) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int32_t, v), src));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int32_t)(uint32_t)u, src);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int32_t)(uint32_t)(u >> 32), src);
        return __builtin_bit_cast(T, (uint64_t)lo | ((uint64_t)hi << 32));
    }
}

// Fronts with nj > SMALL_NJ, step at pivot `off` (b = min(NB, nn - off) pivots, trailing block from m0 = off + b):
// one workgroup per 64 x 64 tile (ti, tj) of the trailing block, which
//   - factors the b x b diagonal block D in registers (wave 0; every tile does it),
//   - solves its 64 rows of the column panel, L <- A U_D* (wave 1), and its 64 columns of the row panel,
//     U <- L_D* A (wave 2), into LDS,
//   - applies the Schur update of its tile, A <- A (+) L (x) U (all waves; sgemx_mt!, chordal/sgetrf.jl:146).
// The solved panels and D are final factor entries: the tiles of the first tile column / row store them straight
// into the reference layout (LD, LL, UL), not into the arena, whose panel entries other tiles of the step still
// read.  The arena keeps only the trailing blocks, down to the update matrix for the parent.
//
// D is padded to NB x NB by repeating its last row and column.  A real entry (i, j < b) only ever meets real
// entries: the LU updates it with pivots k < min(i, j), and a real unknown j of the solves reads unknowns i < j
// and block entries D[i, j] with i, j < b.  The padded entries and unknowns hold whatever the same arithmetic gives
// and are never stored or used by the update (which runs over k < b).
template <class S>
__global__ __launch_bounds__(NT) void k_front_step(typename S::value_type *__restrict__ F, const i64 *__restrict__ Foff,
                                                   const int32_t *__restrict__ nn, const int32_t *__restrict__ nj,
                                                   const i64 *__restrict__ Dptr, const i64 *__restrict__ Lptr,
                                                   typename S::value_type *__restrict__ LD,
                                                   typename S::value_type *__restrict__ LL,
                                                   typename S::value_type *__restrict__ UL,
                                                   const int32_t *__restrict__ tasks) {
    typedef typename S::value_type T;
    constexpr int LDd = NB + 1, TG = 64;
    __shared__ T Dl[NB * LDd];
    __shared__ T Ls[NB][TG];   // the tile's rows of L, by pivot column
    __shared__ T Us[NB][TG];   // the tile's columns of U, by pivot row
    const int32_t *t = tasks + 4 * (i64)blockIdx.x;
    const int f = t[0], off = t[1], ti = t[2], tj = t[3];
    const int n = nj[f], a = nn[f];
    const int b = min(NB, a - off), m0 = off + b;
    T *A = F + Foff[f];
    const int r0 = m0 + ti * TG, c0 = m0 + tj * TG;
    const int mr = max(0, min(TG, n - r0)), mc = max(0, min(TG, n - c0));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    // the tile of the trailing block, 4 x 4 per thread (rows 4 tx + i, columns 4 ty + j)
    T acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = 4 * tx + i, c = 4 * ty + j;
            acc[i][j] = (r < mr && c < mc) ? A[(r0 + r) + (i64)(c0 + c) * n] : S::zero();
        }
    // the panel rows (wave 1) and columns (wave 2) of this tile; lanes past the end repeat the last one
    T v[NB];
    if (wave == 1 && mr > 0) {
        const int r = r0 + min(lane, mr - 1);
#pragma unroll
        for (int j = 0; j < NB; j++) v[j] = A[r + (i64)(off + min(j, b - 1)) * n];
    }
    // the row panel's block (NB rows x the tile's TG columns) into Us, by waves 2 and 3: 32 consecutive threads read a
    // column's NB consecutive rows (coalesced); wave 2 takes its column from Us after the barrier below
    if (wave >= 2 && mc > 0) {
        const int t = threadIdx.x - 128;
#pragma unroll
        for (int q = 0; q < NB * TG / 128; q++) {
            const int idx = t + 128 * q, row = idx % NB, col = idx / NB;
            Us[row][col] = A[(off + min(row, b - 1)) + (i64)(c0 + min(col, mc - 1)) * n];
        }
    }
    if (wave == 0) {
        // LU of D in registers (dense/sgetrf.jl:151-175, the operations of lds_lu in the same order): lane i holds
        // row i (lanes NB.. repeat lanes 0..NB-1), and pivot row k is read from lane k
        const int i = lane & (NB - 1);
        const int ic = min(i, b - 1);
        T d[NB];
#pragma unroll
        for (int j = 0; j < NB; j++) d[j] = A[(off + ic) + (i64)(off + min(j, b - 1)) * n];
        // Rows at or above the pivot keep their entries.  Except for PlusProd, their multiplier is the semiring zero
        // instead of a select per entry: zero (x) u (+) d = d for every u these semirings can hold (min/max drop the
        // NaN of inf - inf), and the entries stay canonical, so the update is readlane, (x), (+).  PlusProd selects:
        // 0 * inf is NaN.
        constexpr bool zero_mul = S::id != S_PLUSPROD;
#pragma unroll
        for (int k = 0; k < NB; k++) {
            const bool below = i > k;
            if (!S::integral) {
                const T l = S::prod(d[k], S::star(bcast_lane(d[k], k)));
                d[k] = below ? l : d[k];
            }
            const T lm = below ? d[k] : S::zero();
#pragma unroll
            for (int j = k + 1; j < NB; j++) {
                if constexpr (zero_mul) {
                    d[j] = S::muladd(lm, bcast_lane(d[j], k), d[j]);
                } else {
                    const T w = S::muladd(d[k], bcast_lane(d[j], k), d[j]);
                    d[j] = below ? w : d[j];
                }
            }
        }
        if (lane < NB) {
#pragma unroll
            for (int j = 0; j < NB; j++) Dl[i + j * LDd] = d[j];
            if (ti == 0 && tj == 0 && i < b) {
                T *dst = LD + Dptr[f] + (off + i) + (i64)off * a;
#pragma unroll
                for (int j = 0; j < NB; j++)
                    if (j < b) dst[(i64)j * a] = d[j];
            }
        }
    }
    __syncthreads();
    if (wave == 1 && mr > 0) {
        // rows of the column panel: x <- x U_D*, right-looking (x_i is final after step i and then updates every later
        // x_j): each x_j receives the terms i = 0, 1, ... in the order of the one-by-one substitution, and a step's
        // updates are independent of each other
#pragma unroll
        for (int i = 0; i < NB; i++) {
            if (!S::integral) v[i] = S::prod(v[i], S::star(Dl[i + i * LDd]));
#pragma unroll
            for (int j = i + 1; j < NB; j++) v[j] = S::muladd(v[i], Dl[i + j * LDd], v[j]);
        }
#pragma unroll
        for (int j = 0; j < NB; j++) Ls[j][lane] = v[j];
        if (tj == 0 && lane < mr) {
            const int r = r0 + lane;
            T *dst = r < a ? LD + Dptr[f] + r + (i64)off * a : LL + Lptr[f] + (r - a) + (i64)off * (n - a);
            const i64 ldd = r < a ? a : n - a;
#pragma unroll
            for (int j = 0; j < NB; j++)
                if (j < b) dst[j * ldd] = v[j];
        }
    }
    if (wave == 2 && mc > 0) {
        // columns of the row panel: y <- L_D* y, right-looking as above (L unit lower)
#pragma unroll
        for (int i = 0; i < NB; i++) v[i] = Us[i][lane];
#pragma unroll
        for (int k = 0; k < NB; k++)
#pragma unroll
            for (int i = k + 1; i < NB; i++) v[i] = S::muladd(Dl[i + k * LDd], v[k], v[i]);
#pragma unroll
        for (int i = 0; i < NB; i++) Us[i][lane] = v[i];
        if (ti == 0 && lane < mc) {
            const int c = c0 + lane;
            T *dst = c < a ? LD + Dptr[f] + off + (i64)c * a : UL + Lptr[f] + off + (i64)(c - a) * a;
#pragma unroll
            for (int i = 0; i < NB; i++)
                if (i < b) dst[i] = v[i];
        }
    }
    __syncthreads();
    if (mr == 0 || mc == 0) return;
    // the Schur update of the tile over the step's b pivots
    int k = 0;
    for (; k + 2 <= b; k += 2) {
        T a0[4], a1[4], b0[4], b1[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            a0[i] = Ls[k][4 * tx + i];
            a1[i] = Ls[k + 1][4 * tx + i];
            b0[i] = Us[k][4 * ty + i];
            b1[i] = Us[k + 1][4 * ty + i];
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = S::muladd2(a0[i], b0[j], a1[i], b1[j], acc[i][j]);
    }
    if (k < b) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = S::muladd(Ls[k][4 * tx + i], Us[k][4 * ty + j], acc[i][j]);
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = 4 * tx + i, c = 4 * ty + j;
            if (r < mr && c < mc) A[(r0 + r) + (i64)(c0 + c) * n] = acc[i][j];
        }
}

// ===== semiring GEMM tile: C[64 x 64] <- C (+) A[64 x k] (x) B[k x 64], column-major operands =====

constexpr int GT = 64, GK = 32;

template <class S>
__device__ inline void gemm_tile(typename S::value_type *__restrict__ C, i64 ldc, const typename S::value_type *__restrict__ A,
                                 i64 lda, const typename S::value_type *__restrict__ B, i64 ldb, int m, int n, int k) {
    typedef typename S::value_type T;
    __shared__ T As[GK][GT + 4];
    __shared__ T Bs[GK][GT + 4];
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    T acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = tx * 4 + i, c = ty * 4 + j;
            acc[i][j] = (r < m && c < n) ? C[r + c * ldc] : S::zero();
        }
    for (int k0 = 0; k0 < k; k0 += GK) {
        const int kc = min(GK, k - k0);
        __syncthreads();
        for (int e = threadIdx.x; e < GK * GT; e += NT) {
            const int r = e % GT, kk = e / GT;
            As[kk][r] = (kk < kc && r < m) ? A[r + (i64)(k0 + kk) * lda] : S::zero();
        }
        for (int e = threadIdx.x; e < GK * GT; e += NT) {
            const int kk = e % GK, c = e / GK;
            Bs[kk][c] = (kk < kc && c < n) ? B[(k0 + kk) + (i64)c * ldb] : S::zero();
        }
        __syncthreads();
        for (int kk = 0; kk < kc; kk++) {
            T a[4], bb[4];
#pragma unroll
            for (int i = 0; i < 4; i++) a[i] = As[kk][tx * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; j++) bb[j] = Bs[kk][ty * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = S::muladd(a[i], bb[j], acc[i][j]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = tx * 4 + i, c = ty * 4 + j;
            if (r < m && c < n) C[r + c * ldc] = acc[i][j];
        }
}

template <class S>
__global__ __launch_bounds__(NT) void k_gemm(typename S::value_type *__restrict__ C, i64 ldc,
                                             const typename S::value_type *__restrict__ A, i64 lda,
                                             const typename S::value_type *__restrict__ B, i64 ldb, i64 m, i64 n, i64 k) {
    const i64 r0 = (i64)blockIdx.x * GT, c0 = (i64)blockIdx.y * GT;
    gemm_tile<S>(C + r0 + c0 * ldc, ldc, A + r0, lda, B + c0 * ldb, ldb, (int)min<i64>(GT, m - r0),
                 (int)min<i64>(GT, n - c0), (int)k);
}

// 16-byte vectors of each element type, and of their int32 indices
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
template <class T> struct Vec16;
template <> struct Vec16<float> { typedef f32x4 type; typedef i32x4 idx; };
template <> struct Vec16<double> { typedef f64x2 type; typedef i32x2 idx; };
template <> struct Vec16<int32_t> { typedef i32x4 type; typedef i32x4 idx; };

// ===== dense semiring GEMM: C <- C (+) A (x) B (sgemx!, dense/sgemx.jl:26-60; generic loop :606-635) =====
//
// Workgroups of 256 threads (16 x 16) own a BM x BN tile of C (BM = 16 TM, BN = 16 TN; 128 x 128 for 4-byte
// elements, 64 x 64 for 8-byte ones), each thread a TM x TN register block whose rows are groups of four, 64 rows
// apart, and likewise its columns (16-byte LDS reads without bank conflicts).  K runs in steps of BK = 16 through
// two LDS buffers: the next step's A and B tiles are loaded into registers while the current step is computed, then
// stored into the other buffer (one barrier per step).  Two k at a time go into each accumulator (muladd2: v_min3 /
// v_max3 for the tropical semirings, 1.5 VALU instructions per multiply-add).  Out-of-range rows, columns and k
// read the semiring zero.
constexpr int GBK = 16;

template <class S, int TM, int TN>
__global__ __launch_bounds__(256) void k_gemm_tiled(typename S::value_type *__restrict__ C, i64 ldc,
                                                    const typename S::value_type *__restrict__ A, i64 lda,
                                                    const typename S::value_type *__restrict__ B, i64 ldb, i64 m,
                                                    i64 n, i64 k) {
    typedef typename S::value_type T;
    constexpr int BM = 16 * TM, BN = 16 * TN, BK = GBK, PAD = 4;
    constexpr int AL = BM * BK / 256, BL = BN * BK / 256;   // tile elements per thread
    __shared__ __attribute__((aligned(16))) T As[2][BK][BM];
    __shared__ __attribute__((aligned(16))) T Bs[2][BK][BN + PAD];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const i64 r0 = (i64)blockIdx.x * BM, c0 = (i64)blockIdx.y * BN;
    T ra[AL], rb[BL];
    // 16-byte loads when the tile is inside the matrices and the columns are 16-byte aligned (uniform)
    typedef typename Vec16<T>::type V;
    constexpr int VW = 16 / (int)sizeof(T);
    const bool vec = r0 + BM <= m && c0 + BN <= n && lda % VW == 0 && ldb % VW == 0 &&
                     ((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0;
    auto gload = [&](i64 k0) {
        if (vec && k0 + BK <= k) {
#pragma unroll
            for (int q = 0; q < AL / VW; q++) {
                const int e = (tid + 256 * q) * VW, r = e % BM, kk = e / BM;
                const V v = *reinterpret_cast<const V *>(A + (r0 + r) + (k0 + kk) * lda);
#pragma unroll
                for (int u = 0; u < VW; u++) ra[q * VW + u] = v[u];
            }
#pragma unroll
            for (int q = 0; q < BL / VW; q++) {
                const int e = (tid + 256 * q) * VW, kk = e % BK, c = e / BK;
                const V v = *reinterpret_cast<const V *>(B + (k0 + kk) + (c0 + c) * ldb);
#pragma unroll
                for (int u = 0; u < VW; u++) rb[q * VW + u] = v[u];
            }
        } else {
#pragma unroll
            for (int q = 0; q < AL / VW; q++)
#pragma unroll
                for (int u = 0; u < VW; u++) {
                    const int e = (tid + 256 * q) * VW + u, r = e % BM, kk = e / BM;
                    ra[q * VW + u] = (r0 + r < m && k0 + kk < k) ? A[(r0 + r) + (k0 + kk) * lda] : S::zero();
                }
#pragma unroll
            for (int q = 0; q < BL / VW; q++)
#pragma unroll
                for (int u = 0; u < VW; u++) {
                    const int e = (tid + 256 * q) * VW + u, kk = e % BK, c = e / BK;
                    rb[q * VW + u] = (c0 + c < n && k0 + kk < k) ? B[(k0 + kk) + (c0 + c) * ldb] : S::zero();
                }
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int q = 0; q < AL / VW; q++) {
            const int e = (tid + 256 * q) * VW;
            V v;
#pragma unroll
            for (int u = 0; u < VW; u++) v[u] = ra[q * VW + u];
            *reinterpret_cast<V *>(&As[buf][e / BM][e % BM]) = v;
        }
#pragma unroll
        for (int q = 0; q < BL / VW; q++)
#pragma unroll
            for (int u = 0; u < VW; u++) {
                const int e = (tid + 256 * q) * VW + u;
                Bs[buf][e % BK][e / BK] = rb[q * VW + u];
            }
    };
    // row i of the register block: 64 (i / 4) + 4 tx + i % 4; column j likewise with ty
    auto rowof = [&](int i) { return 64 * (i >> 2) + 4 * tx + (i & 3); };
    auto colof = [&](int j) { return 64 * (j >> 2) + 4 * ty + (j & 3); };
    T acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const i64 r = r0 + rowof(i), c = c0 + colof(j);
            acc[i][j] = (r < m && c < n) ? C[r + c * ldc] : S::zero();
        }
    gload(0);
    sstore(0);
    __syncthreads();
    int buf = 0;
    for (i64 k0 = 0; k0 < k; k0 += BK) {
        const bool more = k0 + BK < k;
        if (more) gload(k0 + BK);
#pragma unroll 1
        for (int kk = 0; kk < BK; kk += 2) {
            T a0[TM], a1[TM], b0[TN], b1[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                a0[i] = As[buf][kk][rowof(i)];
                a1[i] = As[buf][kk + 1][rowof(i)];
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                b0[j] = Bs[buf][kk][colof(j)];
                b1[j] = Bs[buf][kk + 1][colof(j)];
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) acc[i][j] = S::muladd2(a0[i], b0[j], a1[i], b1[j], acc[i][j]);
        }
        if (more) sstore(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const i64 r = r0 + rowof(i), c = c0 + colof(j);
            if (r < m && c < n) C[r + c * ldc] = acc[i][j];
        }
}

// ===== PlusProd over doubles on the fp64 matrix cores =====
//
// PlusProd is the ordinary (+, x) algebra, so its GEMMs are dense contractions for v_mfma_f64_16x16x4f64.  Lane
// layout of one 16 x 16 x 4 product, as measured on gfx950: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16]
// and holds D[4 r + l / 16][l % 16] in element r of its four accumulators.
typedef double v4d __attribute__((ext_vector_type(4)));

__device__ inline v4d mfma_f64_16x16x4(double a, double b, v4d c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// C <- C + A B (column-major, f64): a 64 x 64 tile per workgroup of four waves, each wave a 32 x 32 quarter
// (2 x 2 products per k step of 4); K in steps of 16 through two LDS buffers with the next step's loads in registers,
// as k_gemm_tiled.  Operands outside the matrices load as 0.
template <class T>
__global__ __launch_bounds__(256) void k_gemm_mfma64(T *__restrict__ C, i64 ldc, const T *__restrict__ A, i64 lda,
                                                    const T *__restrict__ B, i64 ldb, i64 m, i64 n, i64 k) {
    static_assert(std::is_same<T, double>::value, "the fp64 matrix cores");
    constexpr int BM = 64, BN = 64, BK = 16, PAD = 4;
    __shared__ __attribute__((aligned(16))) double As[2][BK][BM + PAD];
    __shared__ __attribute__((aligned(16))) double Bs[2][BK][BN + PAD];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int li = lane & 15, lq = lane >> 4;
    const int wr = (wv & 1) * 32, wc = (wv >> 1) * 32;   // the wave's quarter of the tile
    const i64 r0 = (i64)blockIdx.x * BM, c0 = (i64)blockIdx.y * BN;
    const bool vec = r0 + BM <= m && c0 + BN <= n && lda % 2 == 0 && ldb % 2 == 0 && ((uintptr_t)A & 15) == 0 &&
                     ((uintptr_t)B & 15) == 0;
    double ra[4], rb[4];   // two pairs of consecutive elements each: A down a column, B down a column (along k)
    auto gload = [&](i64 k0) {
        const bool full = vec && k0 + BK <= k;
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int e = (tid + 256 * q) * 2;
            const int ar = e % BM, ak = e / BM, bk = e % BK, bc = e / BK;
            if (full) {
                const double2 va = *reinterpret_cast<const double2 *>(A + (r0 + ar) + (k0 + ak) * lda);
                const double2 vb = *reinterpret_cast<const double2 *>(B + (k0 + bk) + (c0 + bc) * ldb);
                ra[2 * q] = va.x;
                ra[2 * q + 1] = va.y;
                rb[2 * q] = vb.x;
                rb[2 * q + 1] = vb.y;
            } else {
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    ra[2 * q + u] = (r0 + ar + u < m && k0 + ak < k) ? A[(r0 + ar + u) + (k0 + ak) * lda] : 0.0;
                    rb[2 * q + u] = (k0 + bk + u < k && c0 + bc < n) ? B[(k0 + bk + u) + (c0 + bc) * ldb] : 0.0;
                }
            }
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int e = (tid + 256 * q) * 2;
            As[buf][e / BM][e % BM] = ra[2 * q];
            As[buf][e / BM][e % BM + 1] = ra[2 * q + 1];
            Bs[buf][e % BK][e / BK] = rb[2 * q];
            Bs[buf][e % BK + 1][e / BK] = rb[2 * q + 1];
        }
    };
    v4d acc[2][2];
#pragma unroll
    for (int bi = 0; bi < 2; bi++)
#pragma unroll
        for (int bj = 0; bj < 2; bj++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const i64 row = r0 + wr + 16 * bi + 4 * r + lq, col = c0 + wc + 16 * bj + li;
                acc[bi][bj][r] = (row < m && col < n) ? C[row + col * ldc] : 0.0;
            }
    gload(0);
    sstore(0);
    __syncthreads();
    int buf = 0;
    for (i64 k0 = 0; k0 < k; k0 += BK) {
        const bool more = k0 + BK < k;
        if (more) gload(k0 + BK);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 4) {
            double a[2], b[2];
#pragma unroll
            for (int bi = 0; bi < 2; bi++) a[bi] = As[buf][kk + lq][wr + 16 * bi + li];
#pragma unroll
            for (int bj = 0; bj < 2; bj++) b[bj] = Bs[buf][kk + lq][wc + 16 * bj + li];
#pragma unroll
            for (int bi = 0; bi < 2; bi++)
#pragma unroll
                for (int bj = 0; bj < 2; bj++) acc[bi][bj] = mfma_f64_16x16x4(a[bi], b[bj], acc[bi][bj]);
        }
        if (more) sstore(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }
#pragma unroll
    for (int bi = 0; bi < 2; bi++)
#pragma unroll
        for (int bj = 0; bj < 2; bj++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const i64 row = r0 + wr + 16 * bi + 4 * r + lq, col = c0 + wc + 16 * bj + li;
                if (row < m && col < n) C[row + col * ldc] = acc[bi][bj][r];
            }
}

// ===== factor extraction: the reference layout and the sweep packs =====

// LD (nn x nn at Dptr), LL (na x nn at Lptr), UL (nn x na at Lptr); one workgroup per (front, EXTRACT_COLS columns)
template <class T>
__global__ __launch_bounds__(NT) void k_extract_ref(const T *__restrict__ F, const i64 *__restrict__ Foff,
                                                   const int32_t *__restrict__ nn, const int32_t *__restrict__ nj,
                                                   const i64 *__restrict__ Dptr, const i64 *__restrict__ Lptr,
                                                   const int32_t *__restrict__ tasks, T *__restrict__ LD,
                                                   T *__restrict__ LL, T *__restrict__ UL) {
    const int f = tasks[2 * blockIdx.x], c0 = tasks[2 * blockIdx.x + 1];
    const int a = nn[f], n = nj[f], c = n - a;
    const T *G = F + Foff[f];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c1 = min(n, c0 + EXTRACT_COLS);
    for (int col = c0 + wave; col < c1; col += NT / 64) {
        if (col < a) {
            for (int r = lane; r < a; r += 64) LD[Dptr[f] + r + (i64)col * a] = G[r + (i64)col * n];
            for (int r = lane; r < c; r += 64) LL[Lptr[f] + r + (i64)col * c] = G[(a + r) + (i64)col * n];   // F[a+r, col]
        } else {
            for (int r = lane; r < a; r += 64) UL[Lptr[f] + r + (i64)(col - a) * a] = G[r + (i64)col * n];   // F[r, col]
        }
    }
}

// Dpack (Wc x Wc) / Upack / Lpack (e x Wc) of every panel, Wc = the panel's width class; padding holds the semiring
// zero.  Dpack's diagonal holds the stars of the panel's diagonal entries (the triangle solves read the diagonal only
// through its star), so the division of the real semirings' star is made once per entry, not once per row tile.
// One workgroup per panel.
template <class S>
__global__ __launch_bounds__(NT) void k_build_packs(const typename S::value_type *__restrict__ LD,
                                                   const typename S::value_type *__restrict__ LL,
                                                   const typename S::value_type *__restrict__ UL,
                                                   const i64 *__restrict__ Dptr, const i64 *__restrict__ Lptr,
                                                   const int32_t *__restrict__ nn, const int32_t *__restrict__ nj,
                                                   const i64 *__restrict__ Rptr,
                                                   const int32_t *__restrict__ p_front, const int32_t *__restrict__ p_c0,
                                                   const int32_t *__restrict__ p_w, const int32_t *__restrict__ p_e,
                                                   const int32_t *__restrict__ p_lo, const i64 *__restrict__ p_poff,
                                                   const i64 *__restrict__ p_doff, typename S::value_type *__restrict__ Dpack,
                                                   typename S::value_type *__restrict__ Upack,
                                                   typename S::value_type *__restrict__ Lpack) {
    typedef typename S::value_type T;
    const int p = blockIdx.x;
    const int f = p_front[p], w = p_w[p], e = p_e[p], lo = p_lo[p];
    const int Wc = class_width(width_class(w));
    const int a = nn[f], c = nj[f] - a;
    const int lj0 = p_c0[p] - (int)Rptr[f];
    const T *D = LD + Dptr[f];
    const T *Lf = LL + Lptr[f];   // c x a
    const T *Uf = UL + Lptr[f];   // a x c
    for (int q = threadIdx.x; q < Wc * Wc; q += NT) {
        const int j = q / Wc, i = q - j * Wc;
        T d = S::zero();
        if (i < w && j < w) {
            d = D[(lj0 + i) + (i64)(lj0 + j) * a];
            if (i == j) d = S::star(d);
        }
        Dpack[p_doff[p] + q] = d;
    }
    for (int q = threadIdx.x; q < Wc * e; q += NT) {
        const int t = q / Wc, j = q - t * Wc;      // element (j, t) at t*Wc + j
        const int col = lo + t;                    // local index of the extension column
        T u = S::zero(), l = S::zero();
        if (j < w) {
            if (col < a) {
                u = D[(lj0 + j) + (i64)col * a];
                l = D[col + (i64)(lj0 + j) * a];
            } else {
                u = Uf[(lj0 + j) + (i64)(col - a) * a];
                l = Lf[(col - a) + (i64)(lj0 + j) * c];
            }
        }
        Upack[p_poff[p] + q] = u;
        Lpack[p_poff[p] + q] = l;
    }
}

// ===== sweeps over the rows of X (X column-major, ld rows) =====
//
// Forward (leaves to root), one panel with columns c_0..c_{w-1}:
//   x_j <- (x_j (+) sum_{i<j} x_i (x) D(i,j)) (x) star(D(j,j))?          (k_fwd; stored by k_sweep_bwd)
//   X[:, E_t] <- X[:, E_t] (+) sum_j x_j (x) P(j,t)                        (k_fwd)
// Backward (root to leaves):
//   x_j <- x_j (+) sum_t X[:, E_t] (x) Q(t,j),   then   x_j <- (x_j (+) sum_{i>j} x_i (x) D(i,j)) (x) star(D(j,j))?
// DMODE 0 reads the panel block as stored (U upper with star for forward, L strict lower unit for backward);
// DMODE 1 reads it transposed (L^T unit for forward, U^T with star for backward): lmul! runs on B^T.
// A panel of width w runs in the kernel of its width class W (power of two >= w); its packs are padded to W columns
// with the semiring zero, so every inner loop runs over W without branches (a zero term changes nothing).  The padded
// unknowns j >= w are reset to the semiring zero after each triangular solve: under PlusProd an Inf times a zero pad
// entry is NaN, which must not reach a real column.
// The column indices and pack values are wave-uniform (scalar loads); X is read and written one row per lane, so
// each gathered column is a coalesced 256-byte wave access.

struct SweepArgs {
    const int32_t *plist;            // the list's panel ids
    const int32_t *pre;              // per-panel prefix of work units over each panel's own rows (null: rows [0, nrows))
    const int32_t *cpre;             // per-panel prefix of target chunks (k_fwd, rows [0, nrows))
    int32_t np, nrows, row_base;     // without a prefix: rows [row_base, row_base + nrows)
    const int32_t *p_c0, *p_w, *p_e, *p_chunks, *row_lo, *row_hi;
    const i64 *p_eoff, *p_poff, *p_doff;
    const int32_t *Eidx;
    // backward star sweep: the rows [init_lo[p], init_hi[p]) where the forward sweep left panel p's columns; the
    // other rows of those columns are zero (null: X holds every row, as in the solves)
    const int32_t *init_lo, *init_hi;
};

// largest i in [0, np) with pre[i] <= u
__device__ inline int search(const int32_t *pre, int np, int u) {
    int lo = 0, hi = np;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (pre[mid] <= u) lo = mid;
        else hi = mid;
    }
    return lo;
}

// Element offset of column col of a column-major array with leading dimension ld: a 32 x 32 -> 64-bit product
// (two scalar instructions for uniform operands, where the 64 x 64 product of a sign-extended index takes seven).
// Exact: column indices are int32 and non-negative, and every leading dimension here is below 2^32.
__device__ __forceinline__ i64 cofs(int col, i64 ld) {
    return (i64)((uint64_t)(uint32_t)col * (uint64_t)(uint32_t)ld);
}

// p[i] of a plan array (read-only for the whole launch) through the constant address space: a wave-uniform index
// then gives a scalar load even after the kernel's own stores to X, which the compiler cannot otherwise tell apart
// from the plan's memory (it would load the index into a vector register and wait for it before the gather).
template <class T> __device__ __forceinline__ T cld(const T *p, i64 i) {
    return ((const __attribute__((address_space(4))) T *)p)[i];
}

// X[addr] <- X[addr] (+) v by compare-and-swap on the bit pattern; returns at once when (+) leaves the value
// unchanged (the common case for min / max / or).  Exact and order-independent for the idempotent semirings.
// PlusProd uses the hardware's atomic add (order-dependent rounding, as any parallel sum).
template <class S> __device__ inline void atomic_plus(typename S::value_type *addr, typename S::value_type v) {
    typedef typename S::value_type T;
    if constexpr (std::is_same<S, PlusProd<T>>::value) {
        // (+) is the hardware's floating-point atomic add; a zero term changes nothing (unit right-hand sides make
        // many of them)
        if (v != T(0)) unsafeAtomicAdd(addr, v);
        return;
    }
    typedef typename std::conditional<sizeof(T) == 8, unsigned long long, unsigned int>::type U;
    U *a = reinterpret_cast<U *>(addr);
    U old = __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    while (true) {
        const T nv = S::plus(__builtin_bit_cast(T, old), v);
        const U nb = __builtin_bit_cast(U, nv);
        if (nb == old) return;
        const U prev = atomicCAS(a, old, nb);
        if (prev == old) return;
        old = prev;
    }
}

// Forward step of one panel for a 64-row tile and a chunk of at most SCATTER_T targets: wave 0 solves the rows'
// panel columns (x <- x D*, DMODE as above), the solution goes through LDS, and the four waves scatter it into the
// chunk's targets, X[:, E_t] <- X[:, E_t] (+) sum_j x_j (x) P(j, t).  The solution is not stored: the workgroups of
// the other chunks read the same unsolved columns, and no later forward step reads them; the backward sweep solves
// them again as it loads them (the same operations in the same order).
// (panel, row tile, target chunk) of a forward workgroup
__device__ inline void locate_fwd(const SweepArgs &a, int &pi, int &tile, int &chunk) {
    if (a.pre) {
        pi = search(a.pre, a.np, blockIdx.x);
        const int u = blockIdx.x - a.pre[pi];
        const int nc = a.p_chunks[a.plist[pi]];
        tile = u / nc;
        chunk = u - tile * nc;
    } else {
        const int total = a.cpre[a.np];
        tile = blockIdx.x / total;
        const int u = blockIdx.x - tile * total;
        pi = search(a.cpre, a.np, u);
        chunk = u - a.cpre[pi];
    }
}

// The forward step of list entry pi (width class W) for a row tile and target chunk; xsh: W x TILE_ROWS of LDS.
template <class S, int W, bool ATOMIC, int DMODE>
__device__ __forceinline__ void fwd_step(typename S::value_type *__restrict__ X, i64 ld, const SweepArgs &a,
                                         const typename S::value_type *__restrict__ Dpack,
                                         const typename S::value_type *__restrict__ P, int pi, int tile, int chunk,
                                         typename S::value_type (*xsh)[TILE_ROWS]) {
    typedef typename S::value_type T;
    const int p = a.plist[pi];
    const int lo = a.pre ? a.row_lo[p] : 0, hi = a.pre ? a.row_hi[p] : a.nrows;
    const int lane = threadIdx.x & 63;
    const int q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // the wave: uniform, so pack loads are scalar
    if (lo + tile * TILE_ROWS >= hi) return;                          // (whole workgroup)
    const int r = lo + tile * TILE_ROWS + lane;
    const bool valid = r < hi;
    const int w = a.p_w[p], e = a.p_e[p], c0 = a.p_c0[p];
    const T *Pp = P + a.p_poff[p];
    const int32_t *E = a.Eidx + a.p_eoff[p];
    const int t1 = min(e, (chunk + 1) * SCATTER_T);
    // the wave's targets t = tb + 4 i, in groups of four; the first two groups' loads are issued before the solve
    // (they do not depend on it), and later the next two groups' loads stay in flight (three register sets in
    // rotation).  The targets of a panel are distinct columns, so a load never meets a pending store.  Loads past
    // the last target repeat it and are dropped.
    const int tb = chunk * SCATTER_T + q;
    const int ng = tb < t1 ? ((t1 - tb + 3) / 4 + 3) / 4 : 0;
    T *xr = X + (valid ? r : hi - 1);
    auto ldg = [&](int g, T(&v)[4]) {
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = xr[cofs(cld(E, min(tb + 4 * (4 * g + u), t1 - 1)), ld)];
        __builtin_amdgcn_sched_barrier(0);   // issue the loads here, ahead of the arithmetic that follows
    };
    T A[4], B[4], C[4];
    if (!ATOMIC && ng > 0) {
        ldg(0, A);
        ldg(1, B);
    }
    T x[W];
    if (q == 0) {
        const T *D = Dpack + a.p_doff[p];
#pragma unroll
        for (int j = 0; j < W; j++) {
            const T v = xr[cofs(c0 + min(j, w - 1), ld)];
            x[j] = j < w ? v : S::zero();
        }
#pragma unroll
        for (int j = 0; j < W; j++) {
            T acc = x[j];
#pragma unroll
            for (int i = 0; i < j; i++) acc = S::muladd(x[i], DMODE == 0 ? D[i + j * W] : D[j + i * W], acc);
            if (DMODE == 0 && !S::integral) acc = S::prod(acc, D[j + j * W]);
            x[j] = j < w ? acc : S::zero();
        }
#pragma unroll
        for (int j = 0; j < W; j++) xsh[j][lane] = x[j];
    }
    __syncthreads();
    if (!valid) return;
    if (q != 0) {
#pragma unroll
        for (int j = 0; j < W; j++) x[j] = xsh[j][lane];
    }
    if (ATOMIC) {
        auto contribution = [&](int t) {
            const T *pc = Pp + (i64)t * W;
            T v = S::zero();
            if (W == 1) {
                v = S::muladd(x[0], pc[0], v);
            } else {
#pragma unroll
                for (int j = 0; j < W; j += 2) v = S::muladd2(x[j], pc[j], x[j + 1], pc[j + 1], v);
            }
            return v;
        };
        if constexpr (std::is_same<S, PlusProd<T>>::value) {
            for (int t = tb; t < t1; t += 4) atomic_plus<S>(X + cofs(cld(E, t), ld) + r, contribution(t));
        } else {
            // (+) is min, max or or: the current values of four targets are loaded together, then each
            // contribution goes in by compare-and-swap from its loaded value.  A value changed since the load has
            // moved further in the direction of (+), so a contribution that the loaded value absorbs is absorbed
            // by the current one too; a failed swap retries from the value it returns.
            // The four swaps of a group are issued together and checked after; the next group's loads are issued
            // before them (two register sets in rotation).
            typedef typename std::conditional<sizeof(T) == 8, unsigned long long, unsigned int>::type U;
            auto load4 = [&](int t0, U *(&ad)[4], U(&old)[4]) {
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    ad[u] = reinterpret_cast<U *>(X + cofs(cld(E, min(t0 + 4 * u, t1 - 1)), ld) + r);
                    old[u] = __hip_atomic_load(ad[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            };
            auto swap4 = [&](int t0, U *const(&ad)[4], const U(&old)[4]) {
                T c[4];
                U nb[4], prev[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    c[u] = t0 + 4 * u < t1 ? contribution(t0 + 4 * u) : S::zero();
                    nb[u] = __builtin_bit_cast(U, S::plus(__builtin_bit_cast(T, old[u]), c[u]));
                    prev[u] = old[u];
                    if (t0 + 4 * u < t1 && nb[u] != old[u]) prev[u] = atomicCAS(ad[u], old[u], nb[u]);
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    if (prev[u] == old[u]) continue;   // swapped, absorbed, or past the chunk
                    U o = prev[u];                     // the swap failed: retry from the value it returned
                    while (true) {
                        const U n2 = __builtin_bit_cast(U, S::plus(__builtin_bit_cast(T, o), c[u]));
                        if (n2 == o) break;
                        const U p2 = atomicCAS(ad[u], o, n2);
                        if (p2 == o) break;
                        o = p2;
                    }
                }
            };
            U *adA[4], *adB[4];
            U oldA[4], oldB[4];
            if (tb < t1) load4(tb, adA, oldA);
            for (int t0 = tb; t0 < t1; t0 += 32) {
                if (t0 + 16 < t1) load4(t0 + 16, adB, oldB);
                swap4(t0, adA, oldA);
                if (t0 + 16 >= t1) break;
                if (t0 + 32 < t1) load4(t0 + 32, adA, oldA);
                swap4(t0 + 16, adB, oldB);
            }
        }
        return;
    }
    if (ng == 0) return;
    auto upd = [&](int g, const T(&v)[4]) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int t = tb + 4 * (4 * g + u);
            if (t < t1) {
                const T *pc = Pp + (i64)t * W;
                T acc = v[u];
                if (W == 1) {
                    acc = S::muladd(x[0], pc[0], acc);
                } else {
#pragma unroll
                    for (int j = 0; j < W; j += 2) acc = S::muladd2(x[j], pc[j], x[j + 1], pc[j + 1], acc);
                }
                xr[cofs(cld(E, t), ld)] = acc;
            }
        }
    };
    int g = 0;
    for (; g + 3 <= ng; g += 3) {
        ldg(g + 2, C);
        upd(g, A);
        ldg(g + 3, A);
        upd(g + 1, B);
        ldg(g + 4, B);
        upd(g + 2, C);
    }
    if (g < ng) {
        upd(g, A);
        if (g + 1 < ng) upd(g + 1, B);
    }
}

template <class S, int W, bool ATOMIC, int DMODE>
__global__ __launch_bounds__(NT) void k_fwd(typename S::value_type *__restrict__ X, i64 ld, SweepArgs a,
                                            const typename S::value_type *__restrict__ Dpack,
                                            const typename S::value_type *__restrict__ P) {
    __shared__ typename S::value_type xsh[W][TILE_ROWS];
    int pi, tile, chunk;
    locate_fwd(a, pi, tile, chunk);
    fwd_step<S, W, ATOMIC, DMODE>(X, ld, a, Dpack, P, pi, tile, chunk, xsh);
}

// A list whose panels have different width classes (one level of the solves): each workgroup takes its panel's
// class.  One launch per level instead of one per level and class.
template <class S, bool ATOMIC, int DMODE>
__global__ __launch_bounds__(NT) void k_fwd_mixed(typename S::value_type *__restrict__ X, i64 ld, SweepArgs a,
                                                  const typename S::value_type *__restrict__ Dpack,
                                                  const typename S::value_type *__restrict__ P) {
    __shared__ typename S::value_type xsh[PANEL_W][TILE_ROWS];
    int pi, tile, chunk;
    locate_fwd(a, pi, tile, chunk);
    const int w = a.p_w[a.plist[pi]];
    const int cls = width_class(w);
    switch (cls) {
    case 0: fwd_step<S, 1, ATOMIC, DMODE>(X, ld, a, Dpack, P, pi, tile, chunk, xsh); break;
    case 1: fwd_step<S, 2, ATOMIC, DMODE>(X, ld, a, Dpack, P, pi, tile, chunk, xsh); break;
    case 2: fwd_step<S, 4, ATOMIC, DMODE>(X, ld, a, Dpack, P, pi, tile, chunk, xsh); break;
    case 3: fwd_step<S, 8, ATOMIC, DMODE>(X, ld, a, Dpack, P, pi, tile, chunk, xsh); break;
    case 4: fwd_step<S, 12, ATOMIC, DMODE>(X, ld, a, Dpack, P, pi, tile, chunk, xsh); break;
    case 5: fwd_step<S, 16, ATOMIC, DMODE>(X, ld, a, Dpack, P, pi, tile, chunk, xsh); break;
    case 6: fwd_step<S, 24, ATOMIC, DMODE>(X, ld, a, Dpack, P, pi, tile, chunk, xsh); break;
    default: fwd_step<S, 32, ATOMIC, DMODE>(X, ld, a, Dpack, P, pi, tile, chunk, xsh); break;
    }
}

// Locate (panel, row tile) of a backward / solve workgroup.  With a prefix (star rows): panel-major over each
// panel's own rows.  Without (one row range [row_base, row_base + nrows) for the whole list): workgroups are dealt to
// the 8 XCDs round-robin, so XCD x gets the tiles t = x mod 8; within an XCD the workgroups run panel by panel, so a
// CU's consecutive workgroups share the panel's pack in its scalar cache, and neighbouring panels of the list (the
// children of one front share their parent's columns) meet in the XCD's L2.
__device__ inline void locate_tile(const SweepArgs &a, int np, int &pi, int &tile) {
    const int bid = blockIdx.x;
    if (a.pre) {
        pi = search(a.pre, np, bid);
        tile = bid - a.pre[pi];
    } else {
        const int xcd = bid & 7, local = bid >> 3, tpx = (int)(gridDim.x >> 3) / np;
        pi = local / tpx;
        tile = (local - pi * tpx) * 8 + xcd;
    }
}

constexpr int BWD_NSET = 5;

// The backward step of list entry pi (width class W) for a row tile; red: (KSPLIT - 1) W TILE_ROWS of LDS for the
// split gather list's partial sums.
template <class S, int W, int DMODE, int KSPLIT>
__device__ __forceinline__ void bwd_step(typename S::value_type *__restrict__ X, i64 ld, const SweepArgs &a,
                                         const typename S::value_type *__restrict__ Dpack,
                                         const typename S::value_type *__restrict__ Q, int pi, int tile,
                                         typename S::value_type *__restrict__ red) {
    typedef typename S::value_type T;
    const int p = a.plist[pi];
    const int lo = a.pre ? a.row_lo[p] : a.row_base, hi = a.pre ? a.row_hi[p] : a.row_base + a.nrows;
    const int lane = threadIdx.x & 63;
    const int q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // the wave: uniform, so pack loads are scalar
    if (lo + tile * TILE_ROWS >= hi) return;   // a padding tile of the XCD-aware mapping (whole workgroup)
    const int r = lo + tile * TILE_ROWS + lane;
    const bool valid = r < hi;
    const T *xr = X + (valid ? r : hi - 1);   // lanes past the last row compute on a valid row and store nothing
    const int w = a.p_w[p], e = a.p_e[p], c0 = a.p_c0[p];
    const T *Qp = Q + a.p_poff[p];
    const int32_t *E = a.Eidx + a.p_eoff[p];
    const T *D = Dpack + a.p_doff[p];
    T acc[W];
    // this wave's share of the gather list, in groups of four columns, with the next BWD_NSET - 1 groups' loads in
    // flight (register sets used in rotation, so no copy waits on a load); the lookahead reads up to
    // 4 (BWD_NSET - 1) entries past the share, into the following lists or the zero padding after the last one
    const int ng = e >> 2;
    const int g0 = (int)(((i64)ng * q) / KSPLIT), g1 = (int)(((i64)ng * (q + 1)) / KSPLIT);
    const int kt = 4 * g1, kend = q == KSPLIT - 1 ? e : kt;
    const int32_t *ep = E + 4 * g0;
    const T *qp = Qp + (i64)(4 * g0) * W;
    auto ld4 = [&](const int32_t *ei, T(&v)[4]) {
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = xr[cofs(ei[u], ld)];
        __builtin_amdgcn_sched_barrier(0);   // issue the loads here, ahead of the arithmetic that follows
    };
    auto mad4 = [&](const T(&v)[4], const T *qq) {
#pragma unroll
        for (int j = 0; j < W; j++) {
            acc[j] = S::muladd2(v[0], qq[j], v[1], qq[W + j], acc[j]);
            acc[j] = S::muladd2(v[2], qq[2 * W + j], v[3], qq[3 * W + j], acc[j]);
        }
    };
    const int ngw = g1 - g0;
    // the first groups are issued before wave 0 loads the panel's own columns (not among the gathered ones), so
    // that the two loads' latencies overlap
    T xs[BWD_NSET][4];
    if (ngw > 0) {
#pragma unroll
        for (int u = 0; u + 1 < BWD_NSET; u++) ld4(ep + 4 * u, xs[u]);
    }
#pragma unroll
    for (int j = 0; j < W; j++) acc[j] = S::zero();
    if (q == 0 && (!a.init_lo || (r >= a.init_lo[p] && r < a.init_hi[p]))) {
        // the panel's columns as the forward sweep left them, unsolved: finish its step x <- x D* here
#pragma unroll
        for (int j = 0; j < W; j++) {
            const T v = xr[cofs(c0 + min(j, w - 1), ld)];
            acc[j] = j < w ? v : S::zero();
        }
#pragma unroll
        for (int j = 0; j < W; j++) {
            T s = acc[j];
#pragma unroll
            for (int i = 0; i < j; i++) s = S::muladd(acc[i], DMODE == 0 ? D[i + j * W] : D[j + i * W], s);
            if (DMODE == 0 && !S::integral) s = S::prod(s, D[j + j * W]);
            acc[j] = j < w ? s : S::zero();
        }
    }
    if (ngw > 0) {
        int g = 0;
        for (; g + BWD_NSET <= ngw; g += BWD_NSET) {
#pragma unroll
            for (int u = 0; u < BWD_NSET; u++) {
                ld4(ep + 4 * (u + BWD_NSET - 1), xs[(u + BWD_NSET - 1) % BWD_NSET]);
                mad4(xs[u], qp + 4 * u * W);
            }
            ep += 4 * BWD_NSET;
            qp += 4 * BWD_NSET * W;
        }
#pragma unroll
        for (int u = 0; u + 1 < BWD_NSET; u++)
            if (g + u < ngw) mad4(xs[u], qp + 4 * u * W);
    }
    for (int k = kt; k < kend; k++) {
        const T v0 = xr[cofs(E[k], ld)];
        const T *q0 = Qp + (i64)k * W;
#pragma unroll
        for (int j = 0; j < W; j++) acc[j] = S::muladd(v0, q0[j], acc[j]);
    }
    if (KSPLIT > 1) {
        if (q > 0) {
#pragma unroll
            for (int j = 0; j < W; j++) red[((q - 1) * W + j) * TILE_ROWS + lane] = acc[j];
        }
        __syncthreads();
        if (q != 0) return;
#pragma unroll
        for (int qq = 0; qq < KSPLIT - 1; qq++)
#pragma unroll
            for (int j = 0; j < W; j++) acc[j] = S::plus(acc[j], red[(qq * W + j) * TILE_ROWS + lane]);
    }
#pragma unroll
    for (int j = W - 1; j >= 0; j--) {
        T s = acc[j];
#pragma unroll
        for (int i = j + 1; i < W; i++) s = S::muladd(acc[i], DMODE == 0 ? D[i + j * W] : D[j + i * W], s);
        if (DMODE == 1 && !S::integral) s = S::prod(s, D[j + j * W]);
        acc[j] = j < w ? s : S::zero();
    }
    if (valid) {
#pragma unroll
        for (int j = 0; j < W; j++)
            if (j < w) X[cofs(c0 + j, ld) + r] = acc[j];
    }
}

template <class S, int W, int DMODE, int KSPLIT>
__global__ __launch_bounds__(64 * KSPLIT) __attribute__((amdgpu_waves_per_eu(sizeof(typename S::value_type) == 4 ? 4 : 2))) void k_sweep_bwd(typename S::value_type *__restrict__ X, i64 ld, SweepArgs a,
                                                           const typename S::value_type *__restrict__ Dpack,
                                                           const typename S::value_type *__restrict__ Q) {
    __shared__ typename S::value_type red[(KSPLIT > 1 ? KSPLIT - 1 : 1) * W * TILE_ROWS];
    int pi, tile;
    locate_tile(a, a.np, pi, tile);
    bwd_step<S, W, DMODE, KSPLIT>(X, ld, a, Dpack, Q, pi, tile, red);
}

// A list whose panels have different width classes (one level of the solves): each workgroup takes its panel's
// class.
template <class S, int DMODE, int KSPLIT>
__global__ __launch_bounds__(64 * KSPLIT) __attribute__((amdgpu_waves_per_eu(sizeof(typename S::value_type) == 4 ? 4 : 2))) void k_sweep_bwd_mixed(typename S::value_type *__restrict__ X, i64 ld, SweepArgs a,
                                                                 const typename S::value_type *__restrict__ Dpack,
                                                                 const typename S::value_type *__restrict__ Q) {
    __shared__ typename S::value_type red[(KSPLIT > 1 ? KSPLIT - 1 : 1) * PANEL_W * TILE_ROWS];
    int pi, tile;
    locate_tile(a, a.np, pi, tile);
    const int w = a.p_w[a.plist[pi]];
    const int cls = width_class(w);
    switch (cls) {
    case 0: bwd_step<S, 1, DMODE, KSPLIT>(X, ld, a, Dpack, Q, pi, tile, red); break;
    case 1: bwd_step<S, 2, DMODE, KSPLIT>(X, ld, a, Dpack, Q, pi, tile, red); break;
    case 2: bwd_step<S, 4, DMODE, KSPLIT>(X, ld, a, Dpack, Q, pi, tile, red); break;
    case 3: bwd_step<S, 8, DMODE, KSPLIT>(X, ld, a, Dpack, Q, pi, tile, red); break;
    case 4: bwd_step<S, 12, DMODE, KSPLIT>(X, ld, a, Dpack, Q, pi, tile, red); break;
    case 5: bwd_step<S, 16, DMODE, KSPLIT>(X, ld, a, Dpack, Q, pi, tile, red); break;
    case 6: bwd_step<S, 24, DMODE, KSPLIT>(X, ld, a, Dpack, Q, pi, tile, red); break;
    default: bwd_step<S, 32, DMODE, KSPLIT>(X, ld, a, Dpack, Q, pi, tile, red); break;
    }
}

// ===== star subtrees: a wave steps through a small subtree's panels for its 64 rows =====

struct SubArgs {
    const int32_t *ptr, *pan, *rows, *pre;   // subtree panel lists, rows, prefix of 64-row tiles
    int32_t nsub;
    const int32_t *p_c0, *p_w, *p_e, *rowA_lo, *rowA_hi;
    const i64 *p_eoff, *p_poff, *p_doff;
    const int32_t *Eidx;
};

// Forward step of panel p (width class W) on row r (the lane stores only when `store`): x <- x D* over the panel's
// columns, then X[r, E_t] <- X[r, E_t] (+) sum_j x_j (x) P(j, t) for every t, four targets at a time with the next
// four loads in flight (the targets are distinct columns, so no load meets a pending store).
template <class S, int W>
__device__ inline void sub_fwd_panel(typename S::value_type *__restrict__ X, i64 ld, const SubArgs &a, int p, i64 r,
                                     bool store, const typename S::value_type *__restrict__ Dpack,
                                     const typename S::value_type *__restrict__ Pk) {
    typedef typename S::value_type T;
    const int w = cld(a.p_w, p), e = cld(a.p_e, p), c0 = cld(a.p_c0, p);
    const T *D = Dpack + cld(a.p_doff, p);
    const T *Pp = Pk + cld(a.p_poff, p);
    const int32_t *E = a.Eidx + cld(a.p_eoff, p);
    T *xr = X + r;
    // (a group's four indices are read unclamped, so they merge into one scalar load: up to three entries past the
    // list are the next panel's or the zero padding after the last list, in range, and their loads go unused)
    T x[W];
#pragma unroll
    for (int j = 0; j < W; j++) {
        const T v = xr[cofs(c0 + min(j, w - 1), ld)];
        x[j] = j < w ? v : S::zero();
    }
#pragma unroll
    for (int j = 0; j < W; j++) {
        T acc = x[j];
#pragma unroll
        for (int i = 0; i < j; i++) acc = S::muladd(x[i], D[i + j * W], acc);
        if (!S::integral) acc = S::prod(acc, D[j + j * W]);
        x[j] = j < w ? acc : S::zero();
    }
    if (e == 0) return;
    T A[4], B[4];
    auto ld4 = [&](int t0, T(&v)[4]) {
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = xr[cofs(cld(E, t0 + u), ld)];
    };
    auto upd4 = [&](int t0, const T(&v)[4]) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int t = t0 + u;
            if (t < e) {
                const T *pc = Pp + (i64)t * W;
                T acc = v[u];
                if (W == 1) {
                    acc = S::muladd(x[0], pc[0], acc);
                } else {
#pragma unroll
                    for (int j = 0; j < W; j += 2) acc = S::muladd2(x[j], pc[j], x[j + 1], pc[j + 1], acc);
                }
                if (store) xr[cofs(cld(E, t), ld)] = acc;
            }
        }
    };
    ld4(0, A);
    for (int t0 = 0; t0 < e; t0 += 8) {   // A holds targets t0.., B then t0 + 4..
        if (t0 + 4 < e) ld4(t0 + 4, B);
        upd4(t0, A);
        if (t0 + 4 >= e) break;
        if (t0 + 8 < e) ld4(t0 + 8, A);
        upd4(t0 + 4, B);
    }
}

// Backward step of panel p on row r: x <- (the panel's unsolved forward values, solved, on its own rows [alo, ahi);
// zero elsewhere) (+) sum_t X[r, E_t] (x) Q(t, :), then the unit lower triangle of D; stored when `store`.
template <class S, int W>
__device__ inline void sub_bwd_panel(typename S::value_type *__restrict__ X, i64 ld, const SubArgs &a, int p, i64 r,
                                     bool store, const typename S::value_type *__restrict__ Dpack,
                                     const typename S::value_type *__restrict__ Qk) {
    typedef typename S::value_type T;
    const int w = cld(a.p_w, p), e = cld(a.p_e, p), c0 = cld(a.p_c0, p);
    const T *D = Dpack + cld(a.p_doff, p);
    const T *Qp = Qk + cld(a.p_poff, p);
    const int32_t *E = a.Eidx + cld(a.p_eoff, p);
    const T *xr = X + r;
    T acc[W];
    // gathers in groups of four, three register sets in rotation (eight loads in flight)
    auto ld4 = [&](int t0, T(&v)[4]) {
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = xr[cofs(cld(E, t0 + u), ld)];
    };
    auto mad4 = [&](int t0, const T(&v)[4]) {
        const T *qq = Qp + (i64)t0 * W;
        if (t0 + 4 <= e) {
            // in chunks of 8 columns; a chunk's pack pointer passes through an empty asm that takes the 8 results of
            // the chunk before (of the previous group, for the first), so its scalar loads cannot be hoisted above
            // that chunk: 32 pack scalars live at a time rather than the whole loop body's (which spill into vector
            // lanes, a readlane per operand)
            constexpr int JC = W % 8 == 0 ? 8 : W;
#pragma unroll
            for (int jc = 0; jc < W; jc += JC) {
                const T *qc = qq + jc;
                if constexpr (W >= 16) {
                    const int b = jc == 0 ? W - JC : jc - JC;
                    asm volatile("" : "+s"(qc) : "v"(acc[b]), "v"(acc[b + 1]), "v"(acc[b + 2]), "v"(acc[b + 3]),
                                 "v"(acc[b + 4]), "v"(acc[b + 5]), "v"(acc[b + 6]), "v"(acc[b + 7]));
                }
#pragma unroll
                for (int j = 0; j < JC; j++) {
                    acc[jc + j] = S::muladd2(v[0], cld(qc, j), v[1], cld(qc, W + j), acc[jc + j]);
                    acc[jc + j] = S::muladd2(v[2], cld(qc, 2 * W + j), v[3], cld(qc, 3 * W + j), acc[jc + j]);
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (t0 + u < e) {
#pragma unroll
                    for (int j = 0; j < W; j++) acc[j] = S::muladd(v[u], qq[u * W + j], acc[j]);
                }
        }
    };
    // NS register sets of four in rotation: group g + NS - 1 is loaded while group g is multiplied (deeper rotations
    // spill at the kernel's 80-register budget and run slower).  The first groups are issued before the panel's own
    // columns are loaded, so that the two loads' latencies overlap (the gathered columns are not the panel's own).
    constexpr int NS = 3;
    T xs[NS][4];
#pragma unroll
    for (int u = 0; u + 1 < NS; u++)
        if (4 * u < e) ld4(4 * u, xs[u]);
#pragma unroll
    for (int j = 0; j < W; j++) acc[j] = S::zero();
    if (r >= cld(a.rowA_lo, p) && r < cld(a.rowA_hi, p)) {
#pragma unroll
        for (int j = 0; j < W; j++) {
            const T v = xr[cofs(c0 + min(j, w - 1), ld)];
            acc[j] = j < w ? v : S::zero();
        }
#pragma unroll
        for (int j = 0; j < W; j++) {
            T s = acc[j];
#pragma unroll
            for (int i = 0; i < j; i++) s = S::muladd(acc[i], D[i + j * W], s);
            if (!S::integral) s = S::prod(s, D[j + j * W]);
            acc[j] = j < w ? s : S::zero();
        }
    }
    if (e > 0) {
        int t0 = 0;
        for (; t0 + 4 * NS <= e; t0 += 4 * NS) {
#pragma unroll
            for (int u = 0; u < NS; u++) {
                if (t0 + 4 * (u + NS - 1) < e) ld4(t0 + 4 * (u + NS - 1), xs[(u + NS - 1) % NS]);
                mad4(t0 + 4 * u, xs[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < NS; u++)
            if (t0 + 4 * u < e) {
                if (u == NS - 1) ld4(t0 + 4 * u, xs[u]);
                mad4(t0 + 4 * u, xs[u]);
            }
    }
#pragma unroll
    for (int j = W - 1; j >= 0; j--) {
        T s = acc[j];
#pragma unroll
        for (int i = j + 1; i < W; i++) s = S::muladd(acc[i], D[i + j * W], s);
        acc[j] = j < w ? s : S::zero();
    }
    if (store) {
#pragma unroll
        for (int j = 0; j < W; j++)
            if (j < w) X[cofs(c0 + j, ld) + r] = acc[j];
    }
}

// One wave per (subtree, 64-row tile): forward over the subtree's rows in postorder, or backward over the
// component's rows in reverse postorder.  Every value a panel reads on row r was last written by this lane.
template <class S, bool FWD>
// (backward: at least 6 waves per SIMD, at the cost of a few spilled registers; the gathers need the occupancy)
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(FWD ? 1 : 6))) void k_sub(typename S::value_type *__restrict__ X, i64 ld, SubArgs a,
                                            const typename S::value_type *__restrict__ Dpack,
                                            const typename S::value_type *__restrict__ Pk) {
    const int task = blockIdx.x;
    const int s = search(a.pre, a.nsub, task);
    const int tile = task - a.pre[s];
    const int lo = a.rows[4 * s + (FWD ? 0 : 2)], hi = a.rows[4 * s + (FWD ? 1 : 3)];
    const i64 r = (i64)lo + (i64)tile * TILE_ROWS + threadIdx.x;
    const int k0 = a.ptr[s], k1 = a.ptr[s + 1];
    for (int kk = 0; kk < k1 - k0; kk++) {
        const int p = __builtin_amdgcn_readfirstlane(cld(a.pan, FWD ? k0 + kk : k1 - 1 - kk));
        const int w = cld(a.p_w, p);
        // rows of this step: the panel's own rows [alo, ahi) forward, all the tile's rows backward; lanes outside
        // compute on a row inside and store nothing
        const int plo = FWD ? cld(a.rowA_lo, p) : lo, phi = FWD ? cld(a.rowA_hi, p) : hi;
        const i64 t0 = (i64)lo + (i64)tile * TILE_ROWS;
        if (plo >= phi || t0 >= phi || t0 + TILE_ROWS <= plo) continue;   // (a source subset can leave none)
        const bool store = r >= plo && r < phi;
        const i64 rr = r < plo ? plo : (r >= phi ? phi - 1 : r);
        const int cls = width_class(w);
        if (FWD) {
            switch (cls) {
            case 0: sub_fwd_panel<S, 1>(X, ld, a, p, rr, store, Dpack, Pk); break;
            case 1: sub_fwd_panel<S, 2>(X, ld, a, p, rr, store, Dpack, Pk); break;
            case 2: sub_fwd_panel<S, 4>(X, ld, a, p, rr, store, Dpack, Pk); break;
            case 3: sub_fwd_panel<S, 8>(X, ld, a, p, rr, store, Dpack, Pk); break;
            case 4: sub_fwd_panel<S, 12>(X, ld, a, p, rr, store, Dpack, Pk); break;
            case 5: sub_fwd_panel<S, 16>(X, ld, a, p, rr, store, Dpack, Pk); break;
            case 6: sub_fwd_panel<S, 24>(X, ld, a, p, rr, store, Dpack, Pk); break;
            default: sub_fwd_panel<S, 32>(X, ld, a, p, rr, store, Dpack, Pk); break;
            }
        } else {
            switch (cls) {
            case 0: sub_bwd_panel<S, 1>(X, ld, a, p, rr, store, Dpack, Pk); break;
            case 1: sub_bwd_panel<S, 2>(X, ld, a, p, rr, store, Dpack, Pk); break;
            case 2: sub_bwd_panel<S, 4>(X, ld, a, p, rr, store, Dpack, Pk); break;
            case 3: sub_bwd_panel<S, 8>(X, ld, a, p, rr, store, Dpack, Pk); break;
            case 4: sub_bwd_panel<S, 12>(X, ld, a, p, rr, store, Dpack, Pk); break;
            case 5: sub_bwd_panel<S, 16>(X, ld, a, p, rr, store, Dpack, Pk); break;
            case 6: sub_bwd_panel<S, 24>(X, ld, a, p, rr, store, Dpack, Pk); break;
            default: sub_bwd_panel<S, 32>(X, ld, a, p, rr, store, Dpack, Pk); break;
            }
        }
    }
}

// ===== star blocks: fronts with more than PANEL_W columns, in blocks of at most BLK_W columns =====
//
// Per block b (columns c_0 .. c_{w-1} of front f, local start cb; extension E_b as for a panel):
//   Lstar = L_bb* (unit lower), Ustar = U_bb* (upper, with the diagonal stars for non-integral semirings), the two
//   recurrences the panel kernels run in registers (the forward solve x <- x U_bb*, the backward x <- x L_bb*);
//   Bpack = [Ustar (x) Lstar; L[E, blk] (x) Lstar] and Hpack = Ustar (x) U[blk, E].

// L[E_t, c_i] and U[c_i, E_t] of block-local column i and extension entry t (frontal local index lo + t), read from
// the reference layout: LD (nn x nn, L strict lower and U upper), LL (na x nn), UL (nn x na)
template <class T> struct FrontView {
    const T *D, *Lf, *Uf;
    int nn, na, cb, lo;
    __device__ T L_ext(int t, int i) const {
        const int col = lo + t;
        return col < nn ? D[col + (i64)(cb + i) * nn] : Lf[(col - nn) + (i64)(cb + i) * na];
    }
    __device__ T U_ext(int i, int t) const {
        const int col = lo + t;
        return col < nn ? D[(cb + i) + (i64)col * nn] : Uf[(cb + i) + (i64)(col - nn) * nn];
    }
    __device__ T diag(int i, int j) const { return D[(cb + i) + (i64)(cb + j) * nn]; }
};

template <class T>
__device__ inline FrontView<T> front_view(const T *LD, const T *LL, const T *UL, const i64 *Dptr, const i64 *Lptr,
                                          const int32_t *nn, const int32_t *nj, const i64 *Rptr, int f, int c0, int lo) {
    FrontView<T> v;
    v.nn = nn[f];
    v.na = nj[f] - v.nn;
    v.D = LD + Dptr[f];
    v.Lf = LL + Lptr[f];
    v.Uf = UL + Lptr[f];
    v.cb = c0 - (int)Rptr[f];
    v.lo = lo;
    return v;
}

// One workgroup per block: Lstar (column c per thread) and then Ustar (row r per thread) in LDS, written to
// `stars` at 2 BLK_W^2 per block (Lstar, then Ustar; column-major, zero outside w x w).  A column of Lstar is zero
// above its diagonal and a row of Ustar left of it, so each thread starts at its own index.  For 4-byte elements the
// diagonal block is staged in LDS as well.
template <class S>
__global__ __launch_bounds__(NT) void k_blk_stars(const typename S::value_type *__restrict__ LD,
                                                 const i64 *__restrict__ Dptr, const int32_t *__restrict__ nn,
                                                 const i64 *__restrict__ Rptr, const int32_t *__restrict__ p_front,
                                                 const int32_t *__restrict__ p_c0, const int32_t *__restrict__ p_w,
                                                 int np, typename S::value_type *__restrict__ stars) {
    typedef typename S::value_type T;
    constexpr int LDX = BLK_W + 1;
    constexpr bool DLDS = sizeof(T) == 4;
    __shared__ T x[BLK_W * LDX];                  // x[k * LDX + thread]
    __shared__ T dl[DLDS ? BLK_W * LDX : 1];      // dl[i + j * LDX] = diagonal-block entry (i, j)
    const int id = np + blockIdx.x;
    const int f = p_front[id], w = p_w[id];
    const int a = nn[f], cb = p_c0[id] - (int)Rptr[f];
    const T *Dg = LD + Dptr[f] + cb + (i64)cb * a;   // Dg[i + j a] = diagonal-block entry (i, j)
    if (DLDS)
        for (int q = threadIdx.x; q < w * w; q += NT) dl[(q % w) + (q / w) * LDX] = Dg[(q % w) + (i64)(q / w) * a];
    __syncthreads();
    auto Dv = [&](int i, int j) -> T { return DLDS ? dl[i + j * LDX] : Dg[i + (i64)j * a]; };
    T *Ls = stars + (i64)blockIdx.x * 2 * BLK_W * BLK_W, *Us = Ls + BLK_W * BLK_W;
    const int c = threadIdx.x;
    // Lstar, column c: y_i = [i == c] (+) sum_{c <= k < i} L(i, k) y_k  (y_k = zero for k < c)
    if (c < w) {
        x[c * LDX + c] = S::one();
        for (int i = c + 1; i < w; i++) {
            T a0 = S::zero(), a1 = S::zero();
            int k = c;
            for (; k + 1 < i; k += 2) {
                a0 = S::muladd(Dv(i, k), x[k * LDX + c], a0);
                a1 = S::muladd(Dv(i, k + 1), x[(k + 1) * LDX + c], a1);
            }
            if (k < i) a0 = S::muladd(Dv(i, k), x[k * LDX + c], a0);
            x[i * LDX + c] = S::plus(a0, a1);
        }
    }
    __syncthreads();
    for (int q = threadIdx.x; q < BLK_W * BLK_W; q += NT) {
        const int i = q % BLK_W, j = q / BLK_W;
        Ls[q] = (i < w && j < w && i >= j) ? x[i * LDX + j] : S::zero();
    }
    __syncthreads();
    // Ustar, row r: y_j = ([j == r] (+) sum_{r <= k < j} y_k U(k, j)) (x) U(j, j)*  (y_j = zero for j < r)
    if (c < w) {
        for (int j = c; j < w; j++) {
            T a0 = S::zero(), a1 = S::zero();
            int k = c;
            for (; k + 1 < j; k += 2) {
                a0 = S::muladd(x[k * LDX + c], Dv(k, j), a0);
                a1 = S::muladd(x[(k + 1) * LDX + c], Dv(k + 1, j), a1);
            }
            if (k < j) a0 = S::muladd(x[k * LDX + c], Dv(k, j), a0);
            T acc = S::plus(j == c ? S::one() : S::zero(), S::plus(a0, a1));
            if (!S::integral) acc = S::prod(acc, S::star(Dv(j, j)));
            x[j * LDX + c] = acc;
        }
    }
    __syncthreads();
    for (int q = threadIdx.x; q < BLK_W * BLK_W; q += NT) {
        const int i = q % BLK_W, j = q / BLK_W;   // Ustar(i, j) = y_j of row i
        Us[q] = (i < w && j < w && j >= i) ? x[j * LDX + i] : S::zero();
    }
}

// The packs, one PREP_T x PREP_T output tile per workgroup, K = w <= BLK_W with both operands in LDS:
//   part 0: Bpack rows 0..w-1      = Ustar (x) Lstar      (row stride bn)
//   part 1: Bpack rows w..w+e-1    = L[E, blk] (x) Lstar
//   part 2: Hpack (w x e, stride ep) = Ustar (x) U[blk, E]
template <class S>
__global__ __launch_bounds__(NT) void k_blk_prep(const typename S::value_type *__restrict__ LD,
                                                const typename S::value_type *__restrict__ LL,
                                                const typename S::value_type *__restrict__ UL,
                                                const i64 *__restrict__ Dptr, const i64 *__restrict__ Lptr,
                                                const int32_t *__restrict__ nn, const int32_t *__restrict__ nj,
                                                const i64 *__restrict__ Rptr, const int32_t *__restrict__ p_front,
                                                const int32_t *__restrict__ p_c0, const int32_t *__restrict__ p_w,
                                                const int32_t *__restrict__ p_e, const int32_t *__restrict__ p_lo,
                                                int np, const int32_t *__restrict__ tasks,
                                                const typename S::value_type *__restrict__ stars,
                                                const i64 *__restrict__ b_boff, const i64 *__restrict__ b_hoff,
                                                const int32_t *__restrict__ b_ep, const int32_t *__restrict__ b_bn,
                                                typename S::value_type *__restrict__ Bpack,
                                                typename S::value_type *__restrict__ Hpack) {
    typedef typename S::value_type T;
    constexpr int PT = PREP_T;
    __shared__ T As[BLK_W][PT];   // As[i][r]
    __shared__ T Bs[BLK_W][PT];   // Bs[i][c]
    const int b = tasks[4 * blockIdx.x], part = tasks[4 * blockIdx.x + 1];
    const int r0 = tasks[4 * blockIdx.x + 2] * PT, q0 = tasks[4 * blockIdx.x + 3] * PT;
    const int id = np + b, f = p_front[id], w = p_w[id], e = p_e[id];
    const FrontView<T> fv = front_view(LD, LL, UL, Dptr, Lptr, nn, nj, Rptr, f, p_c0[id], p_lo[id]);
    const T *Ls = stars + (i64)b * 2 * BLK_W * BLK_W, *Us = Ls + BLK_W * BLK_W;
    const int rows = part == 1 ? e : w, cols = part == 2 ? e : w;
    for (int q = threadIdx.x; q < BLK_W * PT; q += NT) {
        const int r = q % PT, i = q / PT;   // A(r0 + r, i)
        T v = S::zero();
        if (i < w && r0 + r < rows) v = part == 1 ? fv.L_ext(r0 + r, i) : Us[(r0 + r) + i * BLK_W];
        As[i][r] = v;
    }
    for (int q = threadIdx.x; q < BLK_W * PT; q += NT) {
        const int i = q % BLK_W, cc = q / BLK_W;   // B(i, q0 + cc)
        T v = S::zero();
        if (i < w && q0 + cc < cols) v = part == 2 ? fv.U_ext(i, q0 + cc) : Ls[i + (q0 + cc) * BLK_W];
        Bs[i][cc] = v;
    }
    __syncthreads();
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    T acc[4][4];
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
        for (int v = 0; v < 4; v++) acc[u][v] = S::zero();
    for (int i = 0; i < w; i++) {
        T av[4], bv[4];
#pragma unroll
        for (int u = 0; u < 4; u++) av[u] = As[i][4 * tx + u];
#pragma unroll
        for (int v = 0; v < 4; v++) bv[v] = Bs[i][4 * ty + v];
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int v = 0; v < 4; v++) acc[u][v] = S::muladd(av[u], bv[v], acc[u][v]);
    }
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int r = r0 + 4 * tx + u, cc = q0 + 4 * ty + v;
            if (r >= rows || cc >= cols) continue;
            if (part == 0) Bpack[b_boff[b] + (i64)r * b_bn[b] + cc] = acc[u][v];
            else if (part == 1) Bpack[b_boff[b] + (i64)(w + r) * b_bn[b] + cc] = acc[u][v];
            else Hpack[b_hoff[b] + (i64)r * b_ep[b] + cc] = acc[u][v];
        }
}

struct BlkArgs {
    const int32_t *ulist;        // the list's unit ids (blocks: id >= np)
    const int32_t *pre;          // per-unit prefix of GEMM tiles (for this kernel's rows per tile)
    int32_t nu, np, ntask;
    i64 nrows;                   // rows of X
    const int32_t *p_c0, *p_w, *p_e;
    const int32_t *rlo, *rhi;    // the rows this sweep writes
    const int32_t *olo, *ohi;    // backward: the rows where the forward sweep left the block's columns
    const i64 *p_eoff;
    const int32_t *Eidx;
    const i64 *b_boff, *b_hoff;
    const int32_t *b_ep;
};

// Block step as a semiring GEMM over a BM x BN tile (BM = 16 TM, BN = 16 TN; 256 threads, 16 x 16, each a TM x TN
// register block whose rows are groups of four, 64 apart, and likewise its columns; K in steps of BK through two
// LDS buffers with the next step's loads in registers, as k_gemm_tiled).  The backward's BN is the block's tile
// width bn; the forward's tiles cover BLK_W extension entries.  Row tiles start at multiples of BM; rows outside the
// sweep's range are computed from in-range memory and not stored.
//   FWD:  C = X[r, E_t] (t in the tile's 128 extension entries) <- C (+) sum_{k < w} X[r, c_k] (x) Hpack[k, t]
//   !FWD: X[r, c_j] <- sum_{k < w} X'[r, c_k] (x) Bpack[k, j] (+) sum_{t < e} X[r, E_t] (x) Bpack[w + t, j], with
//         X' = X on the rows [olo, ohi) and zero elsewhere; a workgroup owns all w columns of its rows, reads them
//         before it writes them, and no other workgroup touches them.
// Workgroups are dealt to the 8 XCDs round-robin; XCD x takes the consecutive tiles [x per, (x + 1) per), so
// neighbouring tiles (the same rows of a forward block, the same pack of a backward block) share its L2.
template <class S, int TM, int TN, int BK, bool FWD>
__global__ __launch_bounds__(256) void k_blk(typename S::value_type *__restrict__ X, i64 ld, BlkArgs a,
                                             const typename S::value_type *__restrict__ Pk) {
    typedef typename S::value_type T;
    static_assert(BLK_K % BK == 0, "pack rows are padded to BLK_K");
    constexpr int BM = 16 * TM, BN = 16 * TN, PAD = 4;
    typedef typename Vec16<T>::type V;
    constexpr int VW = 16 / (int)sizeof(T);
    constexpr int AQ = BM * BK / (256 * VW), BQ = BN * BK / (256 * VW);   // vectors per thread per k step
    __shared__ __attribute__((aligned(16))) T As[2][BK][BM];
    __shared__ __attribute__((aligned(16))) T Bs[2][BK][BN + PAD];
    const int per = (int)(gridDim.x >> 3);
    const int task = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    if (task >= a.ntask) return;
    const int ui = search(a.pre, a.nu, task);
    const int u = task - a.pre[ui];
    const int id = a.ulist[ui], b = id - a.np;
    const int c0 = a.p_c0[id], w = a.p_w[id], e = a.p_e[id];
    const int32_t *E = a.Eidx + a.p_eoff[id];
    const int lo = a.rlo[id], hi = a.rhi[id];
    int rt = u, ct = 0;
    if (FWD) {
        const int nct = (e + BN - 1) / BN;
        rt = u / nct;
        ct = u - rt * nct;
    }
    const i64 r0 = (i64)(lo / BM) * BM + (i64)rt * BM;
    const int K = FWD ? w : w + e;
    const int olo = FWD ? 0 : a.olo[id], ohi = FWD ? 0 : a.ohi[id];
    const T *B = FWD ? Pk + a.b_hoff[b] + (i64)ct * BN : Pk + a.b_boff[b];
    const i64 ldb = FWD ? a.b_ep[b] : BN;
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    // the backward's own columns contribute only on the rows [olo, ohi): a tile without such rows starts at w
    const bool own = FWD || (r0 < ohi && r0 + BM > olo);
    const int kbeg = own ? 0 : (w / BK) * BK, kend = (K + BK - 1) / BK * BK;
    const bool vec = r0 + BM <= a.nrows && ld % VW == 0 && ((uintptr_t)X & 15) == 0;
    auto colA = [&](int k) -> i64 {
        if (FWD) return c0 + min(k, w - 1);
        return k < w ? c0 + k : (k < K ? E[k - w] : c0);
    };
    T ra[AQ * VW], rb[BQ * VW];
    // backward: the extension indices of the A columns of the next step to load.  A wave's lanes of load q cover
    // ND consecutive k (wave-uniform), so the indices are scalar loads (from clamped, always valid positions),
    // issued a step ahead; each lane picks its own at the load.  No gathered load waits on a vector index load.
    constexpr int ND = 64 * VW / BM;
    static_assert(ND >= 1 && (64 * VW) % BM == 0, "a wave's loads cover whole k");
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int dl = (tid & 63) * VW / BM;
    int32_t craw[AQ][ND];
    auto cols = [&](int k0) {
        if constexpr (!FWD) {
#pragma unroll
            for (int q = 0; q < AQ; q++) {
                const int kl = k0 + (64 * wv + 256 * q) * VW / BM - w;
#pragma unroll
                for (int d = 0; d < ND; d++) craw[q][d] = E[min(max(kl + d, 0), max(e - 1, 0))];
            }
        }
    };
    auto pick = [&](int q) {
        int32_t v = craw[q][0];
#pragma unroll
        for (int d = 1; d < ND; d++) v = dl == d ? craw[q][d] : v;
        return v;
    };
    auto gload = [&](int k0) {
        const T *srcs[AQ];   // every address first: a load issued before an index is used would be waited for
#pragma unroll
        for (int q = 0; q < AQ; q++) {
            const int ev = (tid + 256 * q) * VW, r = ev % BM, k = k0 + ev / BM;
            int col;
            if constexpr (FWD) col = c0 + min(k, w - 1);
            else col = k < w ? c0 + k : (k < K ? pick(q) : c0);
            srcs[q] = X + (r0 + r) + cofs(col, ld);
        }
#pragma unroll
        for (int q = 0; q < AQ; q++) {
            const int r = (tid + 256 * q) * VW % BM;
            const T *src = srcs[q];
            if (vec) {
                const V v = *reinterpret_cast<const V *>(src);
#pragma unroll
                for (int t = 0; t < VW; t++) ra[q * VW + t] = v[t];
            } else {
#pragma unroll
                for (int t = 0; t < VW; t++) ra[q * VW + t] = r0 + r + t < a.nrows ? src[t] : S::zero();
            }
        }
#pragma unroll
        for (int q = 0; q < BQ; q++) {
            const int ev = (tid + 256 * q) * VW, c = ev % BN, kk = ev / BN;
            const V v = *reinterpret_cast<const V *>(B + (i64)(k0 + kk) * ldb + c);
#pragma unroll
            for (int t = 0; t < VW; t++) rb[q * VW + t] = v[t];
        }
    };
    // the loaded step k0 into LDS buffer buf; the backward's own columns (k < w) are zero outside the rows
    // [olo, ohi), applied here rather than at the load so that nothing waits on the load before the step's math.
    // The padded steps k >= K load an in-range column (c0, or the block's last column forward) whose rows outside
    // the block's subtree no kernel has written yet: they are replaced by the semiring zero too (a zero pack row
    // times such a value is not zero for PlusProd when it holds Inf or NaN).
    auto sstore = [&](int buf, int k0) {
#pragma unroll
        for (int q = 0; q < AQ; q++) {
            const int ev = (tid + 256 * q) * VW;
            const int kq = k0 + ev / BM;
            V v;
#pragma unroll
            for (int t = 0; t < VW; t++) v[t] = ra[q * VW + t];
            if (kq >= K) {
#pragma unroll
                for (int t = 0; t < VW; t++) v[t] = S::zero();
            } else if (!FWD && kq < w) {
#pragma unroll
                for (int t = 0; t < VW; t++) {
                    const i64 rr = r0 + ev % BM + t;
                    if (rr < olo || rr >= ohi) v[t] = S::zero();
                }
            }
            *reinterpret_cast<V *>(&As[buf][ev / BM][ev % BM]) = v;
        }
#pragma unroll
        for (int q = 0; q < BQ; q++) {
            const int ev = (tid + 256 * q) * VW;
            V v;
#pragma unroll
            for (int t = 0; t < VW; t++) v[t] = rb[q * VW + t];
            *reinterpret_cast<V *>(&Bs[buf][ev / BN][ev % BN]) = v;
        }
    };
    auto rowof = [&](int i) { return 64 * (i >> 2) + 4 * tx + (i & 3); };
    auto colof = [&](int j) { return 64 * (j >> 2) + 4 * ty + (j & 3); };
    // a register block's rows come in groups of four consecutive rows: 16-byte accesses when all four are in range
    auto rows_in = [&](int g) -> int {   // 2: all four rows of group g in [lo, hi), 1: some, 0: none
        const i64 r = r0 + 64 * g + 4 * tx;
        if (r >= lo && r + 4 <= hi) return 2;
        return (r + 4 <= lo || r >= hi) ? 0 : 1;
    };
    // PlusProd over doubles runs on the fp64 matrix cores: each wave takes 32 rows x BN / 2 columns as 2 x NBJ
    // products of 16 x 16, computed transposed (C^T = Bpack^T X^T), so that lane l holds rows r0 + wr + 16 bi + l % 16
    // of the columns wc + 16 bj + 4 r + l / 16: sixteen consecutive rows of a column per access
    constexpr bool MF = std::is_same<S, PlusProd<double>>::value;
    static_assert(!MF || BM == 64, "matrix-core tiles are 64 rows");
    constexpr int NBJ = MF ? BN / 32 : 1;
    const int lane = tid & 63, li = lane & 15, lq = lane >> 4;
    const int wr = ((tid >> 6) & 1) * 32, wc = (tid >> 7) * (BN / 2);
    v4d macc[2][NBJ];
    if constexpr (MF) {
#pragma unroll
        for (int bi = 0; bi < 2; bi++) {
            const i64 row = r0 + wr + 16 * bi + li;
#pragma unroll
            for (int bj = 0; bj < NBJ; bj++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int t = ct * BN + wc + 16 * bj + 4 * r + lq;
                    macc[bi][bj][r] = (FWD && row >= lo && row < hi && t < e) ? X[row + cofs(E[t], ld)] : 0.0;
                }
        }
    }
    T acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = S::zero();
    if (FWD && !MF) {
#pragma unroll
        for (int g = 0; g < TM / 4; g++) {
            const int st = rows_in(g);
            if (st == 0) continue;
            const i64 r = r0 + 64 * g + 4 * tx;
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int t = ct * BN + colof(j);
                if (t >= e) continue;
                const T *src = X + r + cofs(E[t], ld);
                if (st == 2 && vec) {
#pragma unroll
                    for (int h = 0; h < 4; h += VW) {
                        const V v = *reinterpret_cast<const V *>(src + h);
#pragma unroll
                        for (int u = 0; u < VW; u++) acc[4 * g + h + u][j] = v[u];
                    }
                } else {
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        if (r + u >= lo && r + u < hi) acc[4 * g + u][j] = src[u];
                }
            }
        }
    }
    if (kbeg < kend) {
        cols(kbeg);
        gload(kbeg);
        if (kbeg + BK < kend) cols(kbeg + BK);
        sstore(0, kbeg);
    }
    __syncthreads();
    int buf = 0;
    for (int k0 = kbeg; k0 < kend; k0 += BK) {
        const bool more = k0 + BK < kend;
        if (more) gload(k0 + BK);
        if constexpr (MF) {
#pragma unroll
            for (int kk = 0; kk < BK; kk += 4) {
                double af[2], bf[NBJ];
#pragma unroll
                for (int bi = 0; bi < 2; bi++) af[bi] = As[buf][kk + lq][wr + 16 * bi + li];
#pragma unroll
                for (int bj = 0; bj < NBJ; bj++) bf[bj] = Bs[buf][kk + lq][wc + 16 * bj + li];
#pragma unroll
                for (int bi = 0; bi < 2; bi++)
#pragma unroll
                    for (int bj = 0; bj < NBJ; bj++) macc[bi][bj] = mfma_f64_16x16x4(bf[bj], af[bi], macc[bi][bj]);
            }
        } else
#pragma unroll 2
        for (int kk = 0; kk < BK; kk += 2) {
            T a0[TM], a1[TM], b0[TN], b1[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                a0[i] = As[buf][kk][rowof(i)];
                a1[i] = As[buf][kk + 1][rowof(i)];
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                b0[j] = Bs[buf][kk][colof(j)];
                b1[j] = Bs[buf][kk + 1][colof(j)];
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) acc[i][j] = S::muladd2(a0[i], b0[j], a1[i], b1[j], acc[i][j]);
        }
        if (k0 + 2 * BK < kend) cols(k0 + 2 * BK);
        if (more) sstore(buf ^ 1, k0 + BK);
        __syncthreads();
        buf ^= 1;
    }
    if constexpr (MF) {
#pragma unroll
        for (int bi = 0; bi < 2; bi++) {
            const i64 row = r0 + wr + 16 * bi + li;
            if (row < lo || row >= hi) continue;
#pragma unroll
            for (int bj = 0; bj < NBJ; bj++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int cc = wc + 16 * bj + 4 * r + lq;
                    i64 col;
                    if (FWD) {
                        const int t = ct * BN + cc;
                        if (t >= e) continue;
                        col = E[t];
                    } else {
                        if (cc >= w) continue;
                        col = c0 + cc;
                    }
                    X[row + col * ld] = macc[bi][bj][r];
                }
        }
        return;
    }
#pragma unroll
    for (int g = 0; g < TM / 4; g++) {
        const int st = rows_in(g);
        if (st == 0) continue;
        const i64 r = r0 + 64 * g + 4 * tx;
#pragma unroll
        for (int j = 0; j < TN; j++) {
            i64 col;
            if (FWD) {
                const int t = ct * BN + colof(j);
                if (t >= e) continue;
                col = E[t];
            } else {
                const int jj = colof(j);
                if (jj >= w) continue;
                col = c0 + jj;
            }
            T *dst = X + r + col * ld;
            if (st == 2 && vec) {
#pragma unroll
                for (int h = 0; h < 4; h += VW) {
                    V v;
#pragma unroll
                    for (int u = 0; u < VW; u++) v[u] = acc[4 * g + h + u][j];
                    *reinterpret_cast<V *>(dst + h) = v;
                }
            } else {
#pragma unroll
                for (int u = 0; u < 4; u++)
                    if (r + u >= lo && r + u < hi) dst[u] = acc[4 * g + u][j];
            }
        }
    }
}

// ===== relabel and permutations =====

// C[i, j - j0] = X[invp[i], invp[j]] for the columns j0 <= j < j0 + gridDim (C <- P^-1 X Q^-1, permuterowscols!,
// utils.jl:261-505): one workgroup per column
template <class T>
__global__ __launch_bounds__(NT) void k_relabel(const T *__restrict__ X, i64 n, T *__restrict__ C, i64 ldc,
                                               const i64 *__restrict__ invp, i64 j0, const int32_t *__restrict__ cols) {
    const i64 j = j0 + blockIdx.x;
    const T *src = X + (cols ? (i64)cols[j] : invp[j]) * n;
    T *dst = C + (j - j0) * ldc;
    for (i64 i = threadIdx.x; i < n; i += NT) dst[i] = src[invp[i]];
}

// With `cols`, output column j - j0 is instead X's column cols[j] with its rows relabelled (C[i, j - j0] =
// X[invp[i], cols[j]]): the columns of X in a given order (the streamed star).
// The same for the columns [j0, j1), with the source column staged in LDS (coalesced read, gather from LDS, coalesced
// write), for columns of
// at most RELABEL_LDS bytes; persistent workgroups, one per CU.  Rows move in 16-byte vectors (n and ldc multiples
// of the vector width, 16-byte aligned output), and the next column's loads are in flight while the current one is
// gathered and written.
constexpr int RELABEL_LDS = 131072;
constexpr int RELABEL_NT = 1024;


template <class T>
__global__ __launch_bounds__(RELABEL_NT) void k_relabel_lds(const T *__restrict__ X, i64 n, T *__restrict__ C, i64 ldc,
                                                           const int32_t *__restrict__ invp, i64 j0, i64 j1,
                                                           const int32_t *__restrict__ cols) {
    typedef typename Vec16<T>::type V;
    typedef typename Vec16<T>::idx I;
    constexpr int VW = 16 / sizeof(T);
    constexpr int RV = RELABEL_LDS / 16 / RELABEL_NT;   // vectors per thread and column
    __shared__ V col[RELABEL_LDS / 16];
    const T *cs = reinterpret_cast<const T *>(col);
    const int nv = (int)(n / VW);
    V buf[RV];
    auto load = [&](i64 j) {
        const V *src = reinterpret_cast<const V *>(X + (i64)(cols ? cols[j] : invp[j]) * n);
#pragma unroll
        for (int u = 0; u < RV; u++) {
            const int v = threadIdx.x + u * RELABEL_NT;
            if (v < nv) buf[u] = __builtin_nontemporal_load(src + v);
        }
    };
    i64 j = j0 + blockIdx.x;
    if (j < j1) load(j);
    for (; j < j1; j += gridDim.x) {
#pragma unroll
        for (int u = 0; u < RV; u++) {
            const int v = threadIdx.x + u * RELABEL_NT;
            if (v < nv) col[v] = buf[u];
        }
        __syncthreads();
        if (j + gridDim.x < j1) load(j + gridDim.x);
        V *dst = reinterpret_cast<V *>(C + (j - j0) * ldc);
        const I *ip = reinterpret_cast<const I *>(invp);
        for (int v = threadIdx.x; v < nv; v += RELABEL_NT) {
            const I p = ip[v];
            V o;
            if constexpr (VW == 4) o = V{cs[p.x], cs[p.y], cs[p.z], cs[p.w]};
            else o = V{cs[p.x], cs[p.y]};
            __builtin_nontemporal_store(o, dst + v);
        }
        __syncthreads();
    }
}

// rmul!: Y[:, invp[c]] = B[:, c] (dir 0) or B[:, c] = Y[:, invp[c]] (dir 1); B nrhs x n (ldb), Y nrhs x n (nrhs)
template <class T>
__global__ __launch_bounds__(NT) void k_permute_cols(T *__restrict__ B, i64 ldb, T *__restrict__ Y, i64 n, i64 nrhs,
                                                    const i64 *__restrict__ invp, int dir) {
    for (i64 c = blockIdx.x; c < n; c += gridDim.x) {
        T *b = B + c * ldb;
        T *y = Y + invp[c] * nrhs;
        for (i64 r = threadIdx.x; r < nrhs; r += NT) {
            if (dir == 0) y[r] = b[r];
            else b[r] = y[r];
        }
    }
}

// lmul!: Y[r, invp[c]] = B[c, r] (dir 0) or back (dir 1); B n x nrhs (ldb), Y nrhs x n (ld nrhs).  64 x 64 tiles
// through LDS: both sides move 64 consecutive elements per row of the tile, 16 elements per thread.
template <class T>
__global__ __launch_bounds__(NT) void k_transpose_perm(T *__restrict__ B, i64 ldb, T *__restrict__ Y, i64 n, i64 nrhs,
                                                      const i64 *__restrict__ invp, int dir) {
    constexpr int TT = 64, TR = NT / TT;
    __shared__ T tile[TT][TT + 1];
    const i64 c0 = (i64)blockIdx.x * TT, r0 = (i64)blockIdx.y * TT;
    const int tx = threadIdx.x % TT, ty = threadIdx.x / TT;
    if (dir == 0) {
        for (int k = ty; k < TT; k += TR) {
            const i64 c = c0 + tx, r = r0 + k;
            if (c < n && r < nrhs) tile[k][tx] = B[c + r * ldb];
        }
        __syncthreads();
        for (int k = ty; k < TT; k += TR) {
            const i64 c = c0 + k, r = r0 + tx;
            if (c < n && r < nrhs) Y[r + invp[c] * nrhs] = tile[tx][k];
        }
    } else {
        for (int k = ty; k < TT; k += TR) {
            const i64 c = c0 + k, r = r0 + tx;
            if (c < n && r < nrhs) tile[tx][k] = Y[r + invp[c] * nrhs];
        }
        __syncthreads();
        for (int k = ty; k < TT; k += TR) {
            const i64 c = c0 + tx, r = r0 + k;
            if (c < n && r < nrhs) B[c + r * ldb] = tile[k][tx];
        }
    }
}

// ===== arcs between strongly connected components (blocked/sgetrs.jl, sparse/sgemx.jl) =====
//
// Y[r, t] <- Y[r, t] (+) sum_q Y[r, idx[q]] (x) val[q], q in [ptr[t], ptr[t + 1]), for the gather columns t =
// cols[blockIdx.x] of one level of the component DAG: with N by column (idx = rows i of the arcs i -> t, from earlier
// components) or by row (idx = columns j of the arcs t -> j, to later components).  Rows [rlo[b], rhi[b]) (the star's
// second pass), or [0, nrows).  The sources lie in components of earlier levels, so no block writes what another
// reads; every row is one lane, the arc lists are wave-uniform (scalar loads), the columns coalesced.
template <class S>
__global__ __launch_bounds__(NT) void k_spmm_pull(typename S::value_type *__restrict__ Y, i64 ld,
                                                  const int32_t *__restrict__ cols, const int32_t *__restrict__ rlo,
                                                  const int32_t *__restrict__ rhi, i64 nrows, const i64 *__restrict__ ptr,
                                                  const int32_t *__restrict__ idx,
                                                  const typename S::value_type *__restrict__ val) {
    typedef typename S::value_type T;
    const int b = blockIdx.x;
    const i64 t = cols[b];
    const i64 lo = rlo ? rlo[b] : 0, hi = rhi ? rhi[b] : nrows;
    const i64 q0 = ptr[t], q1 = ptr[t + 1];
    for (i64 r = lo + (i64)blockIdx.y * NT + threadIdx.x; r < hi; r += (i64)gridDim.y * NT) {
        T acc = Y[r + t * ld];
        for (i64 q = q0; q < q1; q++) acc = S::muladd(Y[r + (i64)idx[q] * ld], val[q], acc);
        Y[r + t * ld] = acc;
    }
}

// Y[k, js[k]] = one for the m rows of the source-row buffer (its other entries are zero)
template <class S>
__global__ void k_set_units(typename S::value_type *__restrict__ Y, i64 m, const int32_t *__restrict__ js) {
    for (i64 k = blockIdx.x * (i64)NT + threadIdx.x; k < m; k += (i64)gridDim.x * NT) Y[k + (i64)js[k] * m] = S::one();
}

// ===== batched getrf + star of dense fronts (nb <= 64), one workgroup per front =====

template <class S>
__global__ __launch_bounds__(NT) void k_getrf_star(typename S::value_type *__restrict__ Aall,
                                                   typename S::value_type *__restrict__ TLall,
                                                   typename S::value_type *__restrict__ TUall, int nb) {
    typedef typename S::value_type T;
    constexpr int LD = 65;
    __shared__ T A[64 * LD];
    __shared__ T X[64 * LD];
    const i64 base = (i64)blockIdx.x * nb * nb;
    T *G = Aall + base;
    for (int e = threadIdx.x; e < nb * nb; e += NT) A[(e % nb) + (e / nb) * LD] = G[e];
    __syncthreads();
    lds_lu<S>(A, nb, LD, nb);
    for (int e = threadIdx.x; e < nb * nb; e += NT) G[e] = A[(e % nb) + (e / nb) * LD];
    // TU = U*: row r: X[r, j] = (X[r, j] (+) sum_{k<j} X[r, k] U[k, j]) (x) U[j, j]*, from X = I
    if (TUall) {
        const int r = threadIdx.x;
        if (r < nb) {
            T *x = X + r;   // row r at stride LD
            for (int j = 0; j < nb; j++) x[j * LD] = j == r ? S::one() : S::zero();
            for (int j = 0; j < nb; j++) {
                T part = S::zero();
                for (int k = 0; k < j; k++) part = S::muladd(x[k * LD], A[k + j * LD], part);
                T acc = S::plus(x[j * LD], part);
                if (!S::integral) acc = S::prod(acc, S::star(A[j + j * LD]));
                x[j * LD] = acc;
            }
        }
        __syncthreads();
        T *TU = TUall + base;
        for (int e = threadIdx.x; e < nb * nb; e += NT) TU[e] = X[(e % nb) + (e / nb) * LD];
        __syncthreads();
    }
    // TL = L*: column c: X[i, c] = X[i, c] (+) sum_{k<i} L[i, k] X[k, c], from X = I
    if (TLall) {
        const int c = threadIdx.x;
        if (c < nb) {
            T *x = X + c * LD;   // column c
            for (int i = 0; i < nb; i++) x[i] = i == c ? S::one() : S::zero();
            for (int i = 0; i < nb; i++) {
                T part = S::zero();
                for (int k = 0; k < i; k++) part = S::muladd(A[i + k * LD], x[k], part);
                x[i] = S::plus(x[i], part);
            }
        }
        __syncthreads();
        T *TL = TLall + base;
        for (int e = threadIdx.x; e < nb * nb; e += NT) TL[e] = X[(e % nb) + (e / nb) * LD];
    }
}

// One wave per front (4-byte elements, nb <= 64): lane r holds row r of the front in registers (a[j] = A[r, j]),
// the factor and both stars are computed there and the pivot rows and columns are broadcast with readlane.  Every
// entry gets the same terms in the same order as the CPU loops (k_getrf_star, the oracle): the LU pivot by pivot
// (l = A[k, p] (x) A[p, p]*, then A[k, j] <- A[k, j] (+) l (x) A[p, j]); TU = U* by rows, lane r computing
// X[r, j] = (X[r, j] (+) sum_{k<j} X[r, k] (x) U[k, j]) (x) U[j, j]*; TL = L* by columns, lane c computing
// X[i, c] = X[i, c] (+) sum_{k<i} L[i, k] (x) X[k, c].  For the idempotent semirings the k-sums take two terms per
// v_min3 / v_max3 (min and max are exact, so their grouping changes nothing); PlusProd sums them one by one.
// TL leaves through an LDS transpose (32 rows at a time) so that every store is a coalesced column segment.
template <class S>
__global__ __launch_bounds__(256) void k_getrf_star_wave(typename S::value_type *__restrict__ Aall,
                                                        typename S::value_type *__restrict__ TLall,
                                                        typename S::value_type *__restrict__ TUall, int nb, i64 batch) {
    typedef typename S::value_type T;
    static_assert(sizeof(T) == 4, "128 registers of 4 bytes per lane");
    constexpr int N = 64;
    __shared__ T tbuf[4][32 * (N + 1)];
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const i64 f = (i64)blockIdx.x * 4 + wv;
    if (f >= batch) return;   // whole waves; no barrier in this kernel
    const i64 base = f * nb * nb;
    T *G = Aall + base;
    const bool act = lane < nb;
    T a[N];
#pragma unroll
    for (int j = 0; j < N; j++) a[j] = (act && j < nb) ? G[lane + (i64)j * nb] : S::zero();
    // the LU (sgetrf2): pivot p scales column p below it by A[p, p]*, then updates the trailing rows.  The loops
    // run over all 64 rows and columns: a real entry (both indices < nb) only meets pivots and terms with smaller
    // indices, so the padding (the semiring zero, then whatever the arithmetic makes of it) never reaches one.
#pragma unroll
    for (int p = 0; p < N; p++) {
        const bool below = lane > p;
        if (!S::integral) {
            const T sp = S::star(bcast_lane(a[p], p));
            const T l = S::prod(a[p], sp);
            a[p] = below ? l : a[p];
        }
#pragma unroll
        for (int j = p + 1; j < N; j++) {
            const T nv = S::muladd(a[p], bcast_lane(a[j], p), a[j]);
            a[j] = below ? nv : a[j];
        }
    }
    if (act) {
#pragma unroll
        for (int j = 0; j < N; j++)
            if (j < nb) G[lane + (i64)j * nb] = a[j];
    }
    constexpr bool PAIR = S::id != S_PLUSPROD;
    if (TUall) {
        T x[N];
#pragma unroll
        for (int j = 0; j < N; j++) x[j] = j == lane ? S::one() : S::zero();
#pragma unroll
        for (int j = 0; j < N; j++) {
            T part = S::zero();
            int k = 0;
            if (PAIR) {
#pragma unroll
                for (; k + 2 <= j; k += 2)
                    part = S::muladd2(x[k], bcast_lane(a[j], k), x[k + 1], bcast_lane(a[j], k + 1), part);
            }
#pragma unroll
            for (; k < j; k++) part = S::muladd(x[k], bcast_lane(a[j], k), part);
            T acc = S::plus(x[j], part);
            if (!S::integral) acc = S::prod(acc, S::star(bcast_lane(a[j], j)));
            x[j] = acc;
        }
        if (act) {
            T *TU = TUall + base;
#pragma unroll
            for (int j = 0; j < N; j++)
                if (j < nb) TU[lane + (i64)j * nb] = x[j];
        }
    }
    if (TLall) {
        T x[N];   // lane c: column c of L*
#pragma unroll
        for (int i = 0; i < N; i++) x[i] = i == lane ? S::one() : S::zero();
#pragma unroll
        for (int i = 0; i < N; i++) {
            T part = S::zero();
            int k = 0;
            if (PAIR) {
#pragma unroll
                for (; k + 2 <= i; k += 2)
                    part = S::muladd2(bcast_lane(a[k], i), x[k], bcast_lane(a[k + 1], i), x[k + 1], part);
            }
#pragma unroll
            for (; k < i; k++) part = S::muladd(bcast_lane(a[k], i), x[k], part);
            x[i] = S::plus(x[i], part);
        }
        // TL[i, c] = x[i] of lane c: through LDS, 32 rows at a time; then each store instruction writes 32
        // consecutive rows of two columns
        T *TL = TLall + base;
        T *tb = tbuf[wv];
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int i = 0; i < 32; i++) tb[i * (N + 1) + lane] = x[32 * h + i];
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            const int r = lane & 31, c0 = lane >> 5;
#pragma unroll
            for (int c = 0; c < N; c += 2) {
                const int cc = c + c0, ii = 32 * h + r;
                if (cc < nb && ii < nb) TL[ii + (i64)cc * nb] = tb[r * (N + 1) + cc];
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
}

// ===== drivers =====

// Timing slots: events on the context's stream, read by pp_get_timing (no synchronization here).
inline void timer_start(pp_ctx *ctx, int slot) {
    if (ctx->timing) hipEventRecord(ctx->ev[2 * slot], ctx->stream);
}
inline void timer_stop(pp_ctx *ctx, int slot) {
    if (!ctx->timing) return;
    hipEventRecord(ctx->ev[2 * slot + 1], ctx->stream);
    ctx->pending[slot] = true;
}

// Debug (PP_DEBUG_POISON): fill a fresh sweep buffer with the all-ones bit pattern (NaN in both float types, -1 for
// OrAnd) before the sweeps, so that any read of an element no kernel has written shows in the result.  A fill kernel,
// not a memset, on the context's stream.
inline std::string poison_fill(pp_ctx *ctx, void *p, size_t bytes) {
    if (!(ctx->debug & PP_DEBUG_POISON) || bytes < 4) return "";
    const i64 words = (i64)(bytes / 4);
    k_fill<uint32_t><<<grid1(words), NT, 0, ctx->stream>>>((uint32_t *)p, words, 0xffffffffu);
    LAUNCHCHK();
    return "";
}

template <class S> struct FactorRun {
    pp_ctx *ctx;
    pp_fac *fac;
    const void *nz;
    std::string err;
    void operator()() { err = run(); }
    std::string run() {
        typedef typename S::value_type T;
        const FactorPlan &P = *fac->sym->fplan;
        const DevPlan &d = fac->plan;
        hipStream_t st = ctx->stream;
        // the previous star blocks' packs read the factor buffers this run overwrites
        if (ctx->aux_pending) HIPCHK(hipStreamWaitEvent(st, ctx->aux_done, 0));
        timer_start(ctx, 0);
        T *F = nullptr;
        HIPCHK(ctx_alloc(ctx, (void **)&F, std::max<i64>(1, P.arena) * sizeof(T), st));
        const i64 nd = fac->sym->S.n;
        if (fac->dense_src && nd > 0) {
            // a dense matrix: its one front is the whole matrix (column-major, leading dimension nj = n)
            if (P.arena != nd * nd || P.Foff.empty() || P.Foff[0] != 0) return "dense factor: unexpected front arena";
            const unsigned gx = (unsigned)std::min<i64>(16, (nd + NT - 1) / NT), gy = (unsigned)std::min<i64>(nd, 8192);
            k_copy2d<T><<<dim3(gx, gy), NT, 0, st>>>(F, nd, (const T *)fac->dense_src, fac->dense_lda, nd, nd);
        } else {
            k_fill<T><<<grid1(P.arena), NT, 0, st>>>(F, P.arena, S::zero());
        }
        LAUNCHCHK();
        if (fac->sym->S.nnz > 0)
            k_scatter_entries<T><<<grid1(fac->sym->S.nnz), NT, 0, st>>>(F, d.entry_pos, (const T *)nz, fac->sym->S.nnz);
        LAUNCHCHK();
        if (fac->Nval) {
            // the arcs between strongly connected components: N's values by column and by row
            const i64 nN = fac->sym->S.nN;
            k_gather<T><<<grid1(nN), NT, 0, st>>>((T *)fac->Nval, (const T *)nz, d.Nsrc, nN);
            k_gather<T><<<grid1(nN), NT, 0, st>>>((T *)fac->NTval, (const T *)nz, d.NTsrc, nN);
            LAUNCHCHK();
        }
        for (const auto &L : P.levels) {
            if (L.asm_cnt)
                k_assemble<S><<<(unsigned)L.asm_cnt, NT, 0, st>>>(F, d.Foff, d.nn, d.na, d.nj, d.Sptr, d.relpos, d.chptr,
                                                                 d.chidx, d.atask + 2 * L.asm_off, L.asm_blk);
            if (L.small_cnt)
                k_front_small<S, SMALL_NJ><<<(unsigned)L.small_cnt, NT, 0, st>>>(F, d.Foff, d.nn, d.nj,
                                                                                  d.flist + L.small_off);
            for (const auto &s : L.steps)
                if (s.cnt)
                    k_front_step<S><<<(unsigned)s.cnt, NT, 0, st>>>(F, d.Foff, d.nn, d.nj, d.Dptr, d.Lptr, (T *)fac->LD,
                                                                    (T *)fac->LL, (T *)fac->UL, d.stask + 4 * s.off);
            LAUNCHCHK();
        }
        if (P.etask.size())
            k_extract_ref<T><<<(unsigned)(P.etask.size() / 2), NT, 0, st>>>(F, d.Foff, d.nn, d.nj, d.Dptr, d.Lptr, d.etask,
                                                                            (T *)fac->LD, (T *)fac->LL, (T *)fac->UL);
        LAUNCHCHK();
        HIPCHK(hipFreeAsync(F, st));
        return "";
    }
};

// The sweep packs from the factor in the reference layout (the end of the factorization's timing).
template <class S> struct PacksRun {
    pp_ctx *ctx;
    pp_fac *fac;
    std::string err;
    void operator()() { err = run(); }
    std::string run() {
        typedef typename S::value_type T;
        const SweepPlan &W = *fac->sym->splan;
        const DevPlan &d = fac->plan;
        hipStream_t st = ctx->stream;
        if (W.np > 0)
            k_build_packs<S><<<(unsigned)W.np, NT, 0, st>>>((const T *)fac->LD, (const T *)fac->LL, (const T *)fac->UL,
                                                            d.Dptr, d.Lptr, d.nn, d.nj, d.Rptr, d.p_front, d.p_c0, d.p_w,
                                                            d.p_e, d.p_lo, d.p_poff, d.p_doff, (T *)fac->Dpack,
                                                            (T *)fac->Upack, (T *)fac->Lpack);
        LAUNCHCHK();
        if (W.nb > 0) {
            // star blocks: L_bb*, U_bb* into a scratch, then the GEMM packs (zero padding first).  They run on the
            // second stream, after everything queued so far (the factorization, and any earlier star still reading
            // the packs), while the star's first launches (identity, small subtrees, panels) need only the panel
            // packs; block GEMMs and the next factorization wait for aux_done.
            hipStream_t as = ctx->aux_stream;
            HIPCHK(hipEventRecord(ctx->aux_from, st));
            HIPCHK(hipStreamWaitEvent(as, ctx->aux_from, 0));
            T *stars = nullptr;
            HIPCHK(ctx_alloc(ctx, (void **)&stars, (size_t)W.nb * 2 * BLK_W * BLK_W * sizeof(T), as));
            k_fill<T><<<grid1(W.nbpack), NT, 0, as>>>((T *)fac->Bpack, W.nbpack, S::zero());
            if (W.nhpack) k_fill<T><<<grid1(W.nhpack), NT, 0, as>>>((T *)fac->Hpack, W.nhpack, S::zero());
            k_blk_stars<S><<<(unsigned)W.nb, NT, 0, as>>>((const T *)fac->LD, d.Dptr, d.nn, d.Rptr, d.p_front, d.p_c0,
                                                          d.p_w, (int)W.np, stars);
            if (W.prep.size())
                k_blk_prep<S><<<(unsigned)(W.prep.size() / 4), NT, 0, as>>>(
                    (const T *)fac->LD, (const T *)fac->LL, (const T *)fac->UL, d.Dptr, d.Lptr, d.nn, d.nj, d.Rptr,
                    d.p_front, d.p_c0, d.p_w, d.p_e, d.p_lo, (int)W.np, d.prep, stars, d.b_boff, d.b_hoff, d.b_ep,
                    d.b_bn, (T *)fac->Bpack, (T *)fac->Hpack);
            LAUNCHCHK();
            HIPCHK(hipFreeAsync(stars, as));
            HIPCHK(hipEventRecord(ctx->aux_done, as));
            ctx->aux_pending = true;
        }
        timer_stop(ctx, 0);
        return "";
    }
};

// LDS of the backward kernel's split-K combine
template <class T, int W> constexpr i64 bwd_lds(int ks) { return (i64)(ks > 1 ? ks - 1 : 1) * W * TILE_ROWS * sizeof(T); }

template <class S, int W, int KS>
static void launch_bwd(unsigned grid, int dmode, typename S::value_type *X, i64 ld, const SweepArgs &a,
                       const typename S::value_type *D, const typename S::value_type *Pk, hipStream_t st) {
    typedef typename S::value_type T;
    if constexpr (bwd_lds<T, W>(KS) <= 98304) {
        if (dmode == 0) k_sweep_bwd<S, W, 0, KS><<<grid, 64 * KS, 0, st>>>(X, ld, a, D, Pk);
        else k_sweep_bwd<S, W, 1, KS><<<grid, 64 * KS, 0, st>>>(X, ld, a, D, Pk);
    }
}

// Rows of the sweeps: ROWS_ALL, every list on rows [0, nrows) (the solves); ROWS_STAR, each unit its star rows
// (rowA forward, rowB backward); ROWS_OFFD, each unit the rows [rowC_lo, rowC_hi) of the star's second pass.
enum { ROWS_ALL = 0, ROWS_STAR = 1, ROWS_OFFD = 2 };

template <class S, int W>
static void launch_list(bool fwd, int dmode, bool atomic, typename S::value_type *X, i64 ld, const SweepArgs &base,
                        const SweepPlan &Wp, const SweepPlan::List &li, int rows_mode, i64 nrows, const void *Dpack,
                        const void *pack, hipStream_t st, const RowSub *rs) {
    typedef typename S::value_type T;
    const T *D = (const T *)Dpack, *Pk = (const T *)pack;
    const int32_t *tiles = base.pre;   // device copy of the prefix arrays
    const std::vector<int32_t> &HT = rs ? rs->tiles : Wp.tiles;
    const bool star_rows = rows_mode == ROWS_STAR;
    SweepArgs a = base;
    if (fwd) {
        // one launch per list: the panels' own columns solved and scattered, per (64-row tile, target chunk)
        unsigned grid;
        a.cpre = tiles + li.pC;
        if (rows_mode != ROWS_ALL) {
            const i64 pu = rows_mode == ROWS_OFFD ? li.pCu : li.pAu;
            a.pre = tiles + pu;
            grid = (unsigned)HT[pu + li.cnt];
        } else {
            a.pre = nullptr;
            grid = (unsigned)(((nrows + TILE_ROWS - 1) / TILE_ROWS) * HT[li.pC + li.cnt]);
        }
        if (grid) {
            if (atomic) {
                if (dmode == 0) k_fwd<S, W, true, 0><<<grid, NT, 0, st>>>(X, ld, a, D, Pk);
                else k_fwd<S, W, true, 1><<<grid, NT, 0, st>>>(X, ld, a, D, Pk);
            } else {
                if (dmode == 0) k_fwd<S, W, false, 0><<<grid, NT, 0, st>>>(X, ld, a, D, Pk);
                else k_fwd<S, W, false, 1><<<grid, NT, 0, st>>>(X, ld, a, D, Pk);
            }
        }
    } else {
        unsigned grid;
        i64 ntile = 0;
        if (rows_mode == ROWS_OFFD || (star_rows && !li.uniB)) {
            const i64 pb = rows_mode == ROWS_OFFD ? li.pC64 : li.pB64;
            a.pre = tiles + pb;
            grid = (unsigned)HT[pb + li.cnt];
            ntile = grid / std::max<i64>(1, li.cnt);
        } else {
            a.pre = nullptr;
            if (star_rows) {
                a.row_base = rs ? rs->map(li.rowB_lo) : li.rowB_lo;
                a.nrows = (rs ? rs->map(li.rowB_hi) : li.rowB_hi) - a.row_base;
            }
            ntile = (a.nrows + TILE_ROWS - 1) / TILE_ROWS;
            grid = (unsigned)(li.cnt * ((ntile + 7) / 8) * 8);
        }
        // split each row tile's gather list over ks waves when the list has too few tiles to fill the chip (8192
        // waves: the gathers' latency wants several waves per SIMD), keeping at least 32 gather columns per wave of its longest list (which sets the launch's
        // duration) and the split's LDS within 96 KiB
        const i64 tiles_total = li.cnt * ntile;
        int ks = 1;
        while (ks < 8 && tiles_total * ks < 8192 && li.emax >= 64 * ks && bwd_lds<T, W>(2 * ks) <= 98304) ks *= 2;
        if (grid) {
            switch (ks) {
            case 1: launch_bwd<S, W, 1>(grid, dmode, X, ld, a, D, Pk, st); break;
            case 2: launch_bwd<S, W, 2>(grid, dmode, X, ld, a, D, Pk, st); break;
            case 4: launch_bwd<S, W, 4>(grid, dmode, X, ld, a, D, Pk, st); break;
            default: launch_bwd<S, W, 8>(grid, dmode, X, ld, a, D, Pk, st); break;
            }
        }
    }
}

// Run the forward or backward lists of the sweep plan over X.  star_rows: each panel's own row range of the star;
// otherwise rows [0, nrows) for every panel (solves), where forward scatters of one level may meet: atomic.
// A list of star blocks: one launch of the block GEMM over all the list's tiles.  Rows per tile: 128 for 4-byte
// elements when the list has at least two such tiles per compute unit, otherwise 64.
template <class S, int TM, int TN>
static void launch_blk(pp_ctx *ctx, bool fwd, typename S::value_type *X, i64 ld, const BlkArgs &a, const void *Hp,
                       const void *Bp) {
    typedef typename S::value_type T;
    const unsigned grid = (unsigned)((a.ntask + 7) / 8 * 8);
    if (fwd) k_blk<S, TM, 8, 16, true><<<grid, 256, 0, ctx->stream>>>(X, ld, a, (const T *)Hp);
    else k_blk<S, TM, TN, 16, false><<<grid, 256, 0, ctx->stream>>>(X, ld, a, (const T *)Bp);
}

template <class S>
static void launch_blocks(pp_ctx *ctx, const pp_fac *fac, bool fwd, typename S::value_type *X, i64 ld, i64 nrows,
                          const SweepPlan::List &li, const RowSub *rs) {
    typedef typename S::value_type T;
    const SweepPlan &Wp = *fac->sym->splan;
    const DevPlan &d = fac->plan;
    const std::vector<int32_t> &HT = rs ? rs->tiles : Wp.tiles;
    int q = sizeof(T) == 4 && HT[li.pT[1] + li.cnt] >= 2 * ctx->num_cu ? 1 : 0;
    BlkArgs a;
    a.ulist = d.plist + li.off;
    a.pre = (rs ? rs->d_tiles : d.tiles) + li.pT[q];
    a.nu = (int32_t)li.cnt;
    a.np = (int32_t)Wp.np;
    a.ntask = HT[li.pT[q] + li.cnt];
    a.nrows = nrows;
    a.p_c0 = d.p_c0;
    a.p_w = d.p_w;
    a.p_e = d.p_e;
    const int32_t *rAlo = rs ? rs->d_rowA_lo : d.p_rowA_lo, *rAhi = rs ? rs->d_rowA_hi : d.p_rowA_hi;
    const int32_t *rBlo = rs ? rs->d_rowB_lo : d.p_rowB_lo, *rBhi = rs ? rs->d_rowB_hi : d.p_rowB_hi;
    a.rlo = fwd ? rAlo : rBlo;
    a.rhi = fwd ? rAhi : rBhi;
    a.olo = rAlo;
    a.ohi = rAhi;
    a.p_eoff = d.p_eoff;
    a.Eidx = d.Eidx;
    a.b_boff = d.b_boff;
    a.b_hoff = d.b_hoff;
    a.b_ep = d.b_ep;
    if (a.ntask == 0) return;
    const bool wide = li.cls == BLK_CLS;
    if constexpr (sizeof(T) == 4) {
        if (q == 1) {
            if (wide) launch_blk<S, 8, 8>(ctx, fwd, X, ld, a, fac->Hpack, fac->Bpack);
            else launch_blk<S, 8, 4>(ctx, fwd, X, ld, a, fac->Hpack, fac->Bpack);
            return;
        }
    }
    if (wide) launch_blk<S, 4, 8>(ctx, fwd, X, ld, a, fac->Hpack, fac->Bpack);
    else launch_blk<S, 4, 4>(ctx, fwd, X, ld, a, fac->Hpack, fac->Bpack);
}

// A list of every width class (cls < 0) over the rows [0, nrows): the class is taken per workgroup.
template <class S, int KS>
static void launch_bwd_mixed(unsigned grid, int dmode, typename S::value_type *X, i64 ld, const SweepArgs &a,
                             const typename S::value_type *D, const typename S::value_type *Pk, hipStream_t st) {
    typedef typename S::value_type T;
    if constexpr (bwd_lds<T, PANEL_W>(KS) <= 98304) {
        if (dmode == 0) k_sweep_bwd_mixed<S, 0, KS><<<grid, 64 * KS, 0, st>>>(X, ld, a, D, Pk);
        else k_sweep_bwd_mixed<S, 1, KS><<<grid, 64 * KS, 0, st>>>(X, ld, a, D, Pk);
    }
}

template <class S>
static void launch_list_mixed(bool fwd, int dmode, bool atomic, typename S::value_type *X, i64 ld,
                              const SweepArgs &base, const SweepPlan &Wp, const SweepPlan::List &li, int rows_mode,
                              i64 nrows, const void *Dpack, const void *pack, hipStream_t st, const RowSub *rs) {
    typedef typename S::value_type T;
    const T *D = (const T *)Dpack, *Pk = (const T *)pack;
    SweepArgs a = base;
    const i64 ntile = (nrows + TILE_ROWS - 1) / TILE_ROWS;
    if (fwd) {
        // as launch_list: per (64-row tile, target chunk) of each panel's rows, or of rows [0, nrows)
        const std::vector<int32_t> &HT = rs ? rs->tiles : Wp.tiles;
        a.cpre = base.pre + li.pC;
        unsigned grid;
        if (rows_mode != ROWS_ALL) {
            const i64 pu = rows_mode == ROWS_OFFD ? li.pCu : li.pAu;
            a.pre = base.pre + pu;
            grid = (unsigned)HT[pu + li.cnt];
        } else {
            a.pre = nullptr;
            grid = (unsigned)(ntile * HT[li.pC + li.cnt]);
        }
        if (!grid) return;
        if (atomic) {
            if (dmode == 0) k_fwd_mixed<S, true, 0><<<grid, NT, 0, st>>>(X, ld, a, D, Pk);
            else k_fwd_mixed<S, true, 1><<<grid, NT, 0, st>>>(X, ld, a, D, Pk);
        } else {
            if (dmode == 0) k_fwd_mixed<S, false, 0><<<grid, NT, 0, st>>>(X, ld, a, D, Pk);
            else k_fwd_mixed<S, false, 1><<<grid, NT, 0, st>>>(X, ld, a, D, Pk);
        }
        return;
    }
    // backward, as launch_list: per-panel row tiles (the star's rows when they differ across the list, or the rows
    // of the second pass), the list's common star rows, or rows [0, nrows) (the solves)
    const std::vector<int32_t> &HT = rs ? rs->tiles : Wp.tiles;
    unsigned grid;
    i64 nt = ntile;
    if (rows_mode == ROWS_OFFD || (rows_mode == ROWS_STAR && !li.uniB)) {
        const i64 pb = rows_mode == ROWS_OFFD ? li.pC64 : li.pB64;
        a.pre = base.pre + pb;
        grid = (unsigned)HT[pb + li.cnt];
        nt = grid / std::max<i64>(1, li.cnt);
    } else {
        a.pre = nullptr;
        if (rows_mode == ROWS_STAR) {
            a.row_base = rs ? rs->map(li.rowB_lo) : li.rowB_lo;
            a.nrows = (rs ? rs->map(li.rowB_hi) : li.rowB_hi) - a.row_base;
            nt = (a.nrows + TILE_ROWS - 1) / TILE_ROWS;
        }
        grid = (unsigned)(li.cnt * ((nt + 7) / 8) * 8);
    }
    if (!grid) return;
    // as launch_list: split each tile's gather list over ks waves when the list has too few tiles to fill the chip
    const i64 tiles_total = li.cnt * nt;
    int ks = 1;
    while (ks < 8 && tiles_total * ks < 8192 && li.emax >= 64 * ks && bwd_lds<T, PANEL_W>(2 * ks) <= 98304) ks *= 2;
    switch (ks) {
    case 1: launch_bwd_mixed<S, 1>(grid, dmode, X, ld, a, D, Pk, st); break;
    case 2: launch_bwd_mixed<S, 2>(grid, dmode, X, ld, a, D, Pk, st); break;
    case 4: launch_bwd_mixed<S, 4>(grid, dmode, X, ld, a, D, Pk, st); break;
    default: launch_bwd_mixed<S, 8>(grid, dmode, X, ld, a, D, Pk, st); break;
    }
}

// One panel list, dispatched on its width class.
template <class S>
static void launch_panels(bool fwd, int dmode, bool atomic, typename S::value_type *X, i64 ld, const SweepArgs &a,
                          const SweepPlan &Wp, const SweepPlan::List &li, int rows_mode, i64 nrows, const void *Dpack,
                          const void *pack, hipStream_t st, const RowSub *rs) {
    if (li.cls < 0) {
        launch_list_mixed<S>(fwd, dmode, atomic, X, ld, a, Wp, li, rows_mode, nrows, Dpack, pack, st, rs);
        return;
    }
    switch (li.cls) {
    case 0: launch_list<S, 1>(fwd, dmode, atomic, X, ld, a, Wp, li, rows_mode, nrows, Dpack, pack, st, rs); break;
    case 1: launch_list<S, 2>(fwd, dmode, atomic, X, ld, a, Wp, li, rows_mode, nrows, Dpack, pack, st, rs); break;
    case 2: launch_list<S, 4>(fwd, dmode, atomic, X, ld, a, Wp, li, rows_mode, nrows, Dpack, pack, st, rs); break;
    case 3: launch_list<S, 8>(fwd, dmode, atomic, X, ld, a, Wp, li, rows_mode, nrows, Dpack, pack, st, rs); break;
    case 4: launch_list<S, 12>(fwd, dmode, atomic, X, ld, a, Wp, li, rows_mode, nrows, Dpack, pack, st, rs); break;
    case 5: launch_list<S, 16>(fwd, dmode, atomic, X, ld, a, Wp, li, rows_mode, nrows, Dpack, pack, st, rs); break;
    case 6: launch_list<S, 24>(fwd, dmode, atomic, X, ld, a, Wp, li, rows_mode, nrows, Dpack, pack, st, rs); break;
    default: launch_list<S, 32>(fwd, dmode, atomic, X, ld, a, Wp, li, rows_mode, nrows, Dpack, pack, st, rs); break;
    }
}

// star_rows: each unit's own rows (those of the plan, or of the source subset rs); otherwise rows [0, nrows) for
// every panel (the solves; atomic forward scatter).  star_lists: the star's units (blocks for the large fronts, the
// small subtrees first forward and last backward; dmode 0 only) rather than panels only.
template <class S>
static std::string run_sweeps(pp_ctx *ctx, const pp_fac *fac, bool fwd, int dmode, typename S::value_type *X, i64 ld,
                              bool star_rows, i64 nrows, const void *pack, const RowSub *rs = nullptr,
                              int star_lists = -1, const std::function<std::string(i64)> *after = nullptr) {
    const SweepPlan &Wp = *fac->sym->splan;
    const DevPlan &d = fac->plan;
    hipStream_t st = ctx->stream;
    const bool sl = star_lists < 0 ? star_rows : star_lists != 0;
    // the star's lists (blocks, panels, subtrees), or panels only (the solves, and the transposed sweeps of source
    // columns): both take one launch per level for the panels, their width classes together
    const auto &lists = sl ? (fwd ? Wp.sfwd : Wp.sbwd) : (fwd ? Wp.fwdm : Wp.bwdm);
    if (nrows == 0) return "";
    auto subtrees = [&]() {
        typedef typename S::value_type T;
        const i64 nsub = (i64)Wp.sub_ptr.size() - 1;
        const int32_t ntask = rs ? (fwd ? rs->sub_preF.back() : rs->sub_preB.back())
                                 : (fwd ? Wp.sub_preF.back() : Wp.sub_preB.back());
        if (nsub <= 0 || ntask == 0) return;
        SubArgs b;
        b.ptr = d.sub_ptr;
        b.pan = d.sub_pan;
        b.rows = rs ? rs->d_sub_rows : d.sub_rows;
        b.pre = rs ? (fwd ? rs->d_sub_preF : rs->d_sub_preB) : (fwd ? d.sub_preF : d.sub_preB);
        b.nsub = (int32_t)nsub;
        b.p_c0 = d.p_c0;
        b.p_w = d.p_w;
        b.p_e = d.p_e;
        b.rowA_lo = rs ? rs->d_rowA_lo : d.p_rowA_lo;
        b.rowA_hi = rs ? rs->d_rowA_hi : d.p_rowA_hi;
        b.p_eoff = d.p_eoff;
        b.p_poff = d.p_poff;
        b.p_doff = d.p_doff;
        b.Eidx = d.Eidx;
        if (fwd) k_sub<S, true><<<(unsigned)ntask, 64, 0, st>>>(X, ld, b, (const T *)fac->Dpack, (const T *)pack);
        else k_sub<S, false><<<(unsigned)ntask, 64, 0, st>>>(X, ld, b, (const T *)fac->Dpack, (const T *)pack);
    };
    if (sl && fwd) {
        subtrees();
        LAUNCHCHK();
    }
    bool packs_ready = !ctx->aux_pending;
    for (const auto &li : lists) {
        if (li.cls >= BLK_CLS) {
            if (!packs_ready) {
                // the block packs come from the second stream
                if (hipStreamWaitEvent(st, ctx->aux_done, 0) != hipSuccess) return "hipStreamWaitEvent failed";
                packs_ready = true;
            }
            launch_blocks<S>(ctx, fac, fwd, X, ld, nrows, li, rs);
            LAUNCHCHK();
            if (after) {
                const std::string ae = (*after)(&li - lists.data());
                if (!ae.empty()) return ae;
            }
            continue;
        }
        SweepArgs a;
        a.plist = d.plist + li.off;
        a.pre = rs ? rs->d_tiles : d.tiles;   // base of the prefix arrays; launch_list offsets it
        a.cpre = nullptr;
        a.np = (int32_t)li.cnt;
        a.nrows = (int32_t)nrows;
        a.row_base = 0;
        a.p_c0 = d.p_c0;
        a.p_w = d.p_w;
        a.p_e = d.p_e;
        a.p_chunks = d.p_chunks;
        const int32_t *rAlo = rs ? rs->d_rowA_lo : d.p_rowA_lo, *rAhi = rs ? rs->d_rowA_hi : d.p_rowA_hi;
        const int32_t *rBlo = rs ? rs->d_rowB_lo : d.p_rowB_lo, *rBhi = rs ? rs->d_rowB_hi : d.p_rowB_hi;
        a.row_lo = fwd ? rAlo : rBlo;
        a.row_hi = fwd ? rAhi : rBhi;
        a.p_eoff = d.p_eoff;
        a.p_poff = d.p_poff;
        a.p_doff = d.p_doff;
        a.Eidx = d.Eidx;
        a.init_lo = star_rows ? rAlo : nullptr;
        a.init_hi = star_rows ? rAhi : nullptr;
        const bool atomic = !star_rows;
        launch_panels<S>(fwd, dmode, atomic, X, ld, a, Wp, li, star_rows ? ROWS_STAR : ROWS_ALL, nrows, fac->Dpack, pack,
                         st, rs);
        LAUNCHCHK();
        if (after) {
            const std::string ae = (*after)(&li - lists.data());
            if (!ae.empty()) return ae;
        }
    }
    if (sl && !fwd) {
        subtrees();
        LAUNCHCHK();
        if (after) {
            const std::string ae = (*after)((i64)lists.size());
            if (!ae.empty()) return ae;
        }
    }
    return "";
}

// The sweeps over the component DAG when components are coupled by N (blocked/sgetrs.jl:80-122,
// blocked/sgetri.jl:44-121).  up: Y <- Y A*, the levels of lev_up, each gathering N by column into its columns and
// then running its panels (U forward, L backward); !up: Y <- Y (A*)^T, the levels of lev_dn, gathering N by row, then
// the transposed sweeps (L^T forward, U^T backward).  offd: the star's second pass, each gather column and panel on
// the rows of the earlier components of its own component ([anc_lo, first row)); else every row [0, nrows).  The
// forward scatter is atomic: the rows of the panels of one level overlap.
template <class S>
static std::string run_coupled(pp_ctx *ctx, const pp_fac *fac, bool up, bool offd, typename S::value_type *Y, i64 ld,
                               i64 nrows) {
    typedef typename S::value_type T;
    const SweepPlan &Wp = *fac->sym->splan;
    const DevPlan &d = fac->plan;
    hipStream_t st = ctx->stream;
    if (nrows == 0) return "";
    const int dmode = up ? 0 : 1;
    const void *fpack = up ? fac->Upack : fac->Lpack, *bpack = up ? fac->Lpack : fac->Upack;
    SweepArgs a;
    a.pre = d.tiles;
    a.cpre = nullptr;
    a.nrows = (int32_t)nrows;
    a.row_base = 0;
    a.p_c0 = d.p_c0;
    a.p_w = d.p_w;
    a.p_e = d.p_e;
    a.p_chunks = d.p_chunks;
    a.row_lo = offd ? d.p_rowC_lo : nullptr;
    a.row_hi = offd ? d.p_rowC_hi : nullptr;
    a.p_eoff = d.p_eoff;
    a.p_poff = d.p_poff;
    a.p_doff = d.p_doff;
    a.Eidx = d.Eidx;
    a.init_lo = a.init_hi = nullptr;   // every row of a panel holds its forward values
    const int rows_mode = offd ? ROWS_OFFD : ROWS_ALL;
    i64 maxrows = nrows;
    if (offd) {
        maxrows = 0;
        for (size_t k = 0; k < Wp.ccols.size(); k++) maxrows = std::max<i64>(maxrows, Wp.ccol_hi[k] - Wp.ccol_lo[k]);
    }
    const unsigned gy = (unsigned)std::max<i64>(1, std::min<i64>(64, (maxrows + NT - 1) / NT));
    for (const auto &cl : up ? Wp.cup : Wp.cdn) {
        if (cl.cols_cnt)
            k_spmm_pull<S><<<dim3((unsigned)cl.cols_cnt, gy), NT, 0, st>>>(
                Y, ld, d.ccols + cl.cols_off, offd ? d.ccol_lo + cl.cols_off : nullptr,
                offd ? d.ccol_hi + cl.cols_off : nullptr, nrows, up ? d.Nptr : d.NTptr, up ? d.Nidx : d.NTidx,
                (const T *)(up ? fac->Nval : fac->NTval));
        LAUNCHCHK();
        for (i64 k = 0; k < cl.fwd_cnt; k++) {
            const auto &li = Wp.cfwd[cl.fwd_off + k];
            SweepArgs b = a;
            b.plist = d.plist + li.off;
            b.np = (int32_t)li.cnt;
            launch_panels<S>(true, dmode, true, Y, ld, b, Wp, li, rows_mode, nrows, fac->Dpack, fpack, st, nullptr);
            LAUNCHCHK();
        }
        for (i64 k = 0; k < cl.bwd_cnt; k++) {
            const auto &li = Wp.cbwd[cl.bwd_off + k];
            SweepArgs b = a;
            b.plist = d.plist + li.off;
            b.np = (int32_t)li.cnt;
            launch_panels<S>(false, dmode, true, Y, ld, b, Wp, li, rows_mode, nrows, fac->Dpack, bpack, st, nullptr);
            LAUNCHCHK();
        }
    }
    return "";
}

template <class S> struct StarRun {
    pp_ctx *ctx;
    const pp_fac *fac;
    void *out;
    i64 ldc;
    int host;
    std::string err;
    void operator()() { err = run(); }
    // C[:, j0:j1] <- X relabelled, into device memory at C (leading dimension ldc); with `cols`, C[:, j - j0] <- X's
    // column cols[j] with its rows relabelled, on stream `st` with at most `wgs` workgroups
    void relabel(const typename S::value_type *X, i64 n, typename S::value_type *C, i64 ld, i64 j0, i64 j1,
                 const int32_t *cols = nullptr, hipStream_t st = nullptr, int wgs = 0) {
        typedef typename S::value_type T;
        if (!st) st = ctx->stream;
        if (j1 <= j0) return;
        constexpr i64 VW = 16 / sizeof(T);
        const i64 g = std::min<i64>(j1 - j0, wgs > 0 ? wgs : ctx->num_cu);
        if (n * (i64)sizeof(T) <= RELABEL_LDS && n % VW == 0 && ld % VW == 0 && ((uintptr_t)C & 15) == 0)
            k_relabel_lds<T><<<(unsigned)g, RELABEL_NT, 0, st>>>(X, n, C, ld, fac->plan.invp32, j0, j1, cols);
        else
            k_relabel<T><<<(unsigned)(j1 - j0), NT, 0, st>>>(X, n, C, ld, fac->plan.invp, j0, cols);
    }
    // The order in which the backward sweep leaves X's columns final (a unit's columns are final once its launch has
    // run: later launches only read them), cut into groups at list boundaries: group g is X's columns
    // order[gend[g - 1] .. gend[g]), final after list glist[g] (the subtree launch: lists.size()).  False when the
    // columns are not each covered once.
    bool stream_order(std::vector<int32_t> &order, std::vector<i64> &gend, std::vector<i64> &glist, i64 group) {
        const SweepPlan &Wp = *fac->sym->splan;
        const i64 n = fac->sym->S.n;
        std::vector<char> seen(n, 0);
        order.clear();
        gend.clear();
        glist.clear();
        auto take = [&](int32_t id) {
            for (i64 c = Wp.c0[id]; c < Wp.c0[id] + Wp.w[id]; c++) {
                if (c < 0 || c >= n || seen[c]) return false;
                seen[c] = 1;
                order.push_back((int32_t)c);
            }
            return true;
        };
        i64 last = 0;
        for (size_t l = 0; l < Wp.sbwd.size(); l++) {
            const auto &li = Wp.sbwd[l];
            for (i64 k = li.off; k < li.off + li.cnt; k++)
                if (!take(Wp.plist[k])) return false;
            if ((i64)order.size() - last >= group) {
                gend.push_back((i64)order.size());
                glist.push_back((i64)l);
                last = (i64)order.size();
            }
        }
        // (lists after the last cut join the subtrees' group)
        for (size_t q = 0; q + 1 < Wp.sub_ptr.size(); q++)
            for (i64 k = Wp.sub_ptr[q]; k < Wp.sub_ptr[q + 1]; k++)
                if (!take(Wp.sub_pan[k])) return false;
        if ((i64)order.size() != n) return false;
        if ((i64)order.size() > last) {
            gend.push_back(n);
            glist.push_back((i64)Wp.sbwd.size());
        }
        return true;
    }
    std::string run() {
        typedef typename S::value_type T;
        const i64 n = fac->sym->S.n;
        hipStream_t st = ctx->stream;
        T *X = nullptr;
        HIPCHK(ctx_alloc(ctx, (void **)&X, std::max<i64>(1, n * n) * sizeof(T), st));
        std::string pe = poison_fill(ctx, X, (size_t)(n * n) * sizeof(T));
        if (!pe.empty()) return pe;
        timer_start(ctx, 1);
        const DevPlan &d = fac->plan;
        const i64 nsu = (i64)fac->sym->splan->sunits.size();
        if (nsu > 0)
            k_identity_panels<S><<<dim3((unsigned)nsu, PANEL_W), NT, 0, st>>>(X, n, d.sunits, nullptr, n, d.p_c0, d.p_w,
                                                                            d.p_rowA_lo, d.p_rowA_hi, d.p_rowB_lo,
                                                                            d.p_rowB_hi);
        LAUNCHCHK();
        std::string e = run_sweeps<S>(ctx, fac, true, 0, X, n, true, n, fac->Upack);
        if (!e.empty()) return e;
        timer_stop(ctx, 1);
        // star into host memory, components not coupled: each group of columns is relabelled and delivered while the
        // rest of the backward sweep runs
        if (host && n > 0 && !fac->sym->splan->coupled) {
            std::vector<int32_t> order;
            std::vector<i64> gend, glist;
            const i64 CB = chunk_cols(n);
            if (stream_order(order, gend, glist, 1)) {
                timer_start(ctx, 2);
                e = stream_to_host(X, n, order, gend, glist, CB);
                if (!e.empty()) {
                    hipStreamSynchronize(ctx->aux_stream);
                    hipStreamSynchronize(st);
                    hipFreeAsync(X, st);
                    return e;
                }
                timer_stop(ctx, 2);
                timer_start(ctx, 3);
                timer_stop(ctx, 3);
                HIPCHK(hipFreeAsync(X, st));
                return "";
            }
        }
        timer_start(ctx, 2);
        e = run_sweeps<S>(ctx, fac, false, 0, X, n, true, n, fac->Lpack);
        if (!e.empty()) return e;
        timer_stop(ctx, 2);
        if (fac->sym->splan->coupled) {
            // the off-diagonal blocks between strongly connected components (the first pass left A_cc* on the
            // diagonal blocks and zero elsewhere)
            e = run_coupled<S>(ctx, fac, true, true, X, n, n);
            if (!e.empty()) return e;
        }
        timer_start(ctx, 3);
        if (!host) {
            relabel(X, n, (T *)out, ldc, 0, n);
            LAUNCHCHK();
        } else if (n > 0) {
            e = to_host(X, n);
            if (!e.empty()) {
                hipStreamSynchronize(st);
                hipFreeAsync(X, st);
                return e;
            }
        }
        timer_stop(ctx, 3);
        HIPCHK(hipFreeAsync(X, st));
        return "";
    }
    // Relabel into host memory in K >= 4 column chunks: the relabel kernel writes chunk k straight into pinned buffer
    // k % 2 over PCIe (its device-side address; the writes are coalesced 16-byte vectors), then the host's worker
    // threads copy it into `out`; the relabel of chunk k + 2 is queued once the host has read chunk k's buffer.  The
    // device writes one chunk while the host copies the other.  (A copy-engine transfer from a device-side chunk
    // buffer ran at half the PCIe rate in some states of the device memory pool; the kernel's writes do not depend
    // on them.)
    // columns per chunk of the star into host memory: K >= 4 chunks of about STAR_CHUNK_BYTES
    i64 chunk_cols(i64 n) const {
        const i64 total = n * n * (i64)sizeof(typename S::value_type);
        const i64 K = std::min<i64>(n, std::max<i64>(4, (total + STAR_CHUNK_BYTES - 1) / STAR_CHUNK_BYTES));
        return (n + K - 1) / K;
    }
    // the two pinned chunk buffers (and their device-side addresses) for chunks of CB columns
    std::string pinned_chunks(i64 n, i64 CB) {
        const size_t cbytes = (size_t)(CB * n) * sizeof(typename S::value_type);
        for (auto &ev : ctx->pev)
            if (!ev) HIPCHK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
        if (ctx->outpin_bytes >= cbytes) return "";
        HIPCHK(hipStreamSynchronize(ctx->stream));
        HIPCHK(hipStreamSynchronize(ctx->aux_stream));
        for (auto &p : ctx->outpin)
            if (p) hipHostFree(p);
        ctx->outpin[0] = ctx->outpin[1] = nullptr;
        ctx->outpin_dev[0] = ctx->outpin_dev[1] = nullptr;
        ctx->outpin_bytes = 0;
        for (int b = 0; b < 2; b++) {
            HIPCHK(hipHostMalloc(&ctx->outpin[b], cbytes, hipHostMallocDefault));
            HIPCHK(hipHostGetDevicePointer(&ctx->outpin_dev[b], ctx->outpin[b], 0));
        }
        ctx->outpin_bytes = cbytes;
        return "";
    }
    // The backward sweep queued on the context's stream with an event after each group's last list; the columns, in
    // the order the sweep finishes them, relabelled on the second stream into the pinned buffers by chunks of CB
    // columns (each chunk after the event of the group holding its last column), and copied by the host's worker
    // threads into their columns of `out` (X's column j is column perm[j] of the star).  The relabel uses 32
    // workgroups: it waits on PCIe writes, and the sweep keeps the rest of the device.
    std::string stream_to_host(typename S::value_type *X, i64 n, const std::vector<int32_t> &order,
                               const std::vector<i64> &gend, const std::vector<i64> &glist, i64 CB) {
        typedef typename S::value_type T;
        hipStream_t st = ctx->stream, as = ctx->aux_stream;
        std::string e = pinned_chunks(n, CB);
        if (!e.empty()) return e;
        const i64 ng = (i64)gend.size();
        std::vector<hipEvent_t> gev(ng, nullptr);
        auto cleanup = [&]() {
            for (auto &ev : gev)
                if (ev) hipEventDestroy(ev);
        };
        for (auto &ev : gev)
            if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
                cleanup();
                return "hipEventCreate failed";
            }
        // the column order on the device (second stream: the sweep does not wait for it)
        int32_t *d_order = nullptr;
        if (ctx_alloc(ctx, (void **)&d_order, (size_t)n * sizeof(int32_t), as) != hipSuccess) {
            cleanup();
            return "stream-ordered allocation of the column order failed";
        }
        if (hipMemcpyAsync(d_order, order.data(), (size_t)n * sizeof(int32_t), hipMemcpyHostToDevice, as) != hipSuccess) {
            cleanup();
            return "upload of the column order failed";
        }
        // the sweep, recording each group's event after its last list
        i64 gnext = 0;
        const std::function<std::string(i64)> after = [&](i64 l) -> std::string {
            while (gnext < ng && glist[gnext] == l) {
                if (hipEventRecord(gev[gnext], st) != hipSuccess) return "hipEventRecord failed";
                gnext++;
            }
            return "";
        };
        e = run_sweeps<S>(ctx, fac, false, 0, X, n, true, n, fac->Lpack, nullptr, -1, &after);
        while (e.empty() && gnext < ng) e = after(glist[gnext]);   // (groups after the last list run: none expected)
        if (!e.empty()) {
            hipStreamSynchronize(as);
            hipFreeAsync(d_order, as);
            cleanup();
            return e;
        }
        // chunks of CB consecutive positions of the order (the last one shorter), each after the group of its last
        // position: (first position, end, group)
        std::vector<std::array<i64, 3>> ch;
        for (i64 k = 0; k < n; k += CB) {
            const i64 k1 = std::min(n, k + CB);
            const i64 g = std::upper_bound(gend.begin(), gend.end(), k1 - 1) - gend.begin();
            ch.push_back({k, k1, std::min(g, ng - 1)});
        }
        const i64 nchunk = (i64)ch.size();
        i64 waited = -1;   // last group the second stream waits for
        auto produce = [&](i64 c) -> std::string {
            const int b = (int)(c & 1);
            const i64 g = ch[c][2];
            if (g > waited) {
                HIPCHK(hipStreamWaitEvent(as, gev[g], 0));
                waited = g;
            }
            relabel(X, n, (T *)ctx->outpin_dev[b], n, ch[c][0], ch[c][1], d_order, as, 32);
            LAUNCHCHK();
            HIPCHK(hipEventRecord(ctx->pev[b], as));
            return "";
        };
        for (i64 c = 0; c < std::min<i64>(2, nchunk) && e.empty(); c++) e = produce(c);
        for (i64 c = 0; c < nchunk && e.empty(); c++) {
            const int b = (int)(c & 1);
            hipError_t he = hipEventSynchronize(ctx->pev[b]);
            if (he != hipSuccess) {
                e = std::string("hipEventSynchronize: ") + hipGetErrorString(he);
                break;
            }
            const T *src = (const T *)ctx->outpin[b];
            const i64 k0 = ch[c][0], m = ch[c][1] - k0;
            const int nt = (int)std::max<i64>(1, std::min<i64>(16, (m * n * (i64)sizeof(T)) >> 22));   // 4 MiB a thread
            const i64 *perm = fac->sym->S.perm.data();
            pool_run(nt, [&](int t) {
                for (i64 k = m * t / nt; k < m * (t + 1) / nt; k++)
                    std::memcpy((T *)out + perm[order[k0 + k]] * ldc, src + k * n, (size_t)n * sizeof(T));
            });
            if (c + 2 < nchunk) e = produce(c + 2);
        }
        hipError_t se = hipStreamSynchronize(as);
        hipFreeAsync(d_order, st);
        cleanup();
        if (e.empty() && se != hipSuccess) e = std::string("hipStreamSynchronize: ") + hipGetErrorString(se);
        return e;
    }
    std::string to_host(const typename S::value_type *X, i64 n) {
        typedef typename S::value_type T;
        hipStream_t st = ctx->stream;
        const i64 CB = chunk_cols(n);   // columns per chunk
        const i64 nchunk = (n + CB - 1) / CB;
        std::string pe = pinned_chunks(n, CB);
        if (!pe.empty()) return pe;
        auto cols = [&](i64 k, i64 &j0, i64 &j1) {
            j0 = k * CB;
            j1 = std::min(n, j0 + CB);
        };
        auto produce = [&](i64 k) -> std::string {   // relabel chunk k into its pinned buffer
            i64 j0, j1;
            cols(k, j0, j1);
            const int b = (int)(k & 1);
            relabel(X, n, (T *)ctx->outpin_dev[b], n, j0, j1);
            LAUNCHCHK();
            HIPCHK(hipEventRecord(ctx->pev[b], st));
            return "";
        };
        std::string e;
        for (i64 k = 0; k < std::min<i64>(2, nchunk) && e.empty(); k++) e = produce(k);
        for (i64 k = 0; k < nchunk && e.empty(); k++) {
            const int b = (int)(k & 1);
            hipError_t he = hipEventSynchronize(ctx->pev[b]);
            if (he != hipSuccess) {
                e = std::string("hipEventSynchronize: ") + hipGetErrorString(he);
                break;
            }
            i64 j0, j1;
            cols(k, j0, j1);
            const T *src = (const T *)ctx->outpin[b];
            T *dst = (T *)out + j0 * ldc;
            const i64 m = j1 - j0;
            const int nt = (int)std::max<i64>(1, std::min<i64>(16, (m * n * (i64)sizeof(T)) >> 22));   // 4 MiB a thread
            pool_run(nt, [&](int t) {
                if (ldc == n) {
                    const i64 a = m * n * t / nt, z = m * n * (t + 1) / nt;
                    std::memcpy(dst + a, src + a, (size_t)(z - a) * sizeof(T));
                } else {
                    for (i64 j = m * t / nt; j < m * (t + 1) / nt; j++)
                        std::memcpy(dst + j * ldc, src + j * n, (size_t)n * sizeof(T));
                }
            });
            if (k + 2 < nchunk) e = produce(k + 2);
        }
        HIPCHK(hipStreamSynchronize(st));
        return e;
    }
};

// Rows of the star for sources: out[k + j ldo] = Y[pos[k], invp[j]] (Y m x n, leading dimension m); one workgroup per
// output column j
template <class T>
__global__ __launch_bounds__(NT) void k_src_rows_out(const T *__restrict__ Y, i64 m, const int32_t *__restrict__ pos,
                                                    i64 nsrc, const i64 *__restrict__ invp, T *__restrict__ out,
                                                    i64 ldo) {
    const i64 j = blockIdx.x;
    const T *src = Y + invp[j] * m;
    T *dst = out + j * ldo;
    for (i64 k = threadIdx.x; k < nsrc; k += NT) dst[k] = src[pos[k]];
}

// Columns of the star for sources: out[i + k ldo] = Y[pos[k], invp[i]]; 32 x 32 tiles through LDS (reads down the
// columns of Y, writes down the columns of out)
template <class T>
__global__ __launch_bounds__(NT) void k_src_cols_out(const T *__restrict__ Y, i64 m, const int32_t *__restrict__ pos,
                                                    i64 nsrc, const i64 *__restrict__ invp, i64 n, T *__restrict__ out,
                                                    i64 ldo) {
    __shared__ T tile[32][33];
    const i64 i0 = (i64)blockIdx.x * 32, k0 = (i64)blockIdx.y * 32;
    const int tx = threadIdx.x % 32, ty = threadIdx.x / 32;   // 8 rows of 32
    for (int r = ty; r < 32; r += 8) {
        const i64 i = i0 + r, k = k0 + tx;
        if (i < n && k < nsrc) tile[r][tx] = Y[pos[k] + invp[i] * m];
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const i64 k = k0 + r, i = i0 + tx;
        if (i < n && k < nsrc) out[i + k * ldo] = tile[tx][r];
    }
}

// Rows (cols = 0) or columns (cols = 1) of the star for a set of sources (the reference's sgetre!, chordal_slu.jl:
// 445-493, for many sources at once): the sweep buffer Y has one row per source (sorted by elimination label); the
// forward sweep visits, for each unit, only the sources in its subtree.  Rows run the star's units (blocks, subtrees,
// panels) with X <- U* then X <- X L*; columns run the transposed panel sweeps (L^T forward, U^T backward), as lmul!.
template <class S> struct StarSrcRun {
    pp_ctx *ctx;
    const pp_fac *fac;
    const RowSub *R;
    i64 nsrc;
    int cols;
    void *out;
    i64 ldo;
    std::string err;
    void operator()() { err = run(); }
    std::string run() {
        typedef typename S::value_type T;
        const i64 n = fac->sym->S.n, m = (i64)R->js.size();
        hipStream_t st = ctx->stream;
        if (n == 0 || m == 0) return "";
        const SweepPlan &Wp = *fac->sym->splan;
        const DevPlan &d = fac->plan;
        T *Y = nullptr;
        HIPCHK(ctx_alloc(ctx, (void **)&Y, m * n * sizeof(T), st));
        std::string pe = poison_fill(ctx, Y, (size_t)(m * n) * sizeof(T));
        if (!pe.empty()) return pe;
        timer_start(ctx, 4);
        std::string e;
        if (Wp.coupled) {
            // components coupled by N: the rows (columns) of A* as the solve of unit rows, Y <- Y A* (Y (A*)^T)
            k_fill<T><<<grid1(m * n), NT, 0, st>>>(Y, m * n, S::zero());
            k_set_units<S><<<grid1(m), NT, 0, st>>>(Y, m, R->d_js);
            LAUNCHCHK();
            e = run_coupled<S>(ctx, fac, !cols, false, Y, m, m);
        } else if (!cols) {
            const i64 nsu = (i64)Wp.sunits.size();
            if (nsu > 0)
                k_identity_panels<S><<<dim3((unsigned)nsu, PANEL_W), NT, 0, st>>>(Y, m, d.sunits, R->d_js, n, d.p_c0, d.p_w,
                                                                                R->d_rowA_lo, R->d_rowA_hi, R->d_rowB_lo,
                                                                                R->d_rowB_hi);
            LAUNCHCHK();
            e = run_sweeps<S>(ctx, fac, true, 0, Y, m, true, m, fac->Upack, R, 1);
            if (e.empty()) e = run_sweeps<S>(ctx, fac, false, 0, Y, m, true, m, fac->Lpack, R, 1);
        } else {
            if (Wp.np > 0)
                k_identity_panels<S><<<dim3((unsigned)Wp.np, PANEL_W), NT, 0, st>>>(Y, m, nullptr, R->d_js, n, d.p_c0,
                                                                                  d.p_w, R->d_rowA_lo, R->d_rowA_hi,
                                                                                  R->d_rowB_lo, R->d_rowB_hi);
            LAUNCHCHK();
            e = run_sweeps<S>(ctx, fac, true, 1, Y, m, true, m, fac->Lpack, R, 0);
            if (e.empty()) e = run_sweeps<S>(ctx, fac, false, 1, Y, m, true, m, fac->Upack, R, 0);
        }
        if (!e.empty()) return e;
        if (!cols)
            k_src_rows_out<T><<<(unsigned)n, NT, 0, st>>>(Y, m, R->d_pos, nsrc, d.invp, (T *)out, ldo);
        else
            k_src_cols_out<T><<<dim3((unsigned)((n + 31) / 32), (unsigned)((nsrc + 31) / 32)), NT, 0, st>>>(
                Y, m, R->d_pos, nsrc, d.invp, n, (T *)out, ldo);
        LAUNCHCHK();
        timer_stop(ctx, 4);
        HIPCHK(hipFreeAsync(Y, st));
        return "";
    }
};

// The solves (chordal_slu.jl:337-377 -> chordal/sgetrs.jl:29-51).  The right-hand sides go into Y (nrhs x n, one
// row per right-hand side, vertex-major in the elimination order): rmul!'s B (nrhs x n) by a column permutation,
// lmul!'s B (n x nrhs) transposed.  On Y the sweeps compute either Y <- Y A* (U forward, then L backward; the panel
// blocks as stored) or Y <- Y (A*)^T (L^T forward, then U^T backward; the blocks transposed):
//   rmul!(B, F)            Y = B     Y <- Y A*        lmul!(F, B)            Y = B^T   Y <- Y (A*)^T
//   rmul!(B, transpose(F)) Y = B     Y <- Y (A*)^T    lmul!(transpose(F), B) Y = B^T   Y <- Y A*
// since (A^T)* = (A*)^T.  For the real semirings here transpose(F) and adjoint(F) are the same.
template <class S> struct SolveRun {
    pp_ctx *ctx;
    const pp_fac *fac;
    void *B;
    i64 ldb, nrhs;
    bool left, trans;
    void *scratch;                   // Y's memory when not null (at least n * nrhs elements), else a pool allocation
    std::string err;
    void operator()() { err = run(); }
    std::string run() {
        typedef typename S::value_type T;
        const i64 n = fac->sym->S.n;
        hipStream_t st = ctx->stream;
        if (n == 0 || nrhs == 0) return "";
        T *Y = (T *)scratch;
        if (!Y) HIPCHK(ctx_alloc(ctx, (void **)&Y, n * nrhs * sizeof(T), st));
        std::string pe = poison_fill(ctx, Y, (size_t)(n * nrhs) * sizeof(T));
        if (!pe.empty()) return pe;
        timer_start(ctx, 4);
        const dim3 g((unsigned)((n + 63) / 64), (unsigned)((nrhs + 63) / 64));
        auto layout = [&](int dir) {
            if (left) k_transpose_perm<T><<<g, NT, 0, st>>>((T *)B, ldb, Y, n, nrhs, fac->plan.invp, dir);
            else k_permute_cols<T><<<(unsigned)std::min<i64>(n, 65536), NT, 0, st>>>((T *)B, ldb, Y, n, nrhs,
                                                                                      fac->plan.invp, dir);
        };
        layout(0);
        LAUNCHCHK();
        std::string e;
        if (fac->sym->splan->coupled) {
            // components coupled by N: level by level over the component DAG
            e = run_coupled<S>(ctx, fac, left == trans, false, Y, nrhs, nrhs);
        } else if (left == trans) {
            // Y <- Y A*: U forward, then L backward
            e = run_sweeps<S>(ctx, fac, true, 0, Y, nrhs, false, nrhs, fac->Upack);
            if (e.empty()) e = run_sweeps<S>(ctx, fac, false, 0, Y, nrhs, false, nrhs, fac->Lpack);
        } else {
            // Y <- Y (A*)^T: L^T forward, then U^T backward
            e = run_sweeps<S>(ctx, fac, true, 1, Y, nrhs, false, nrhs, fac->Lpack);
            if (e.empty()) e = run_sweeps<S>(ctx, fac, false, 1, Y, nrhs, false, nrhs, fac->Upack);
        }
        if (!e.empty()) return e;
        layout(1);
        LAUNCHCHK();
        timer_stop(ctx, 4);
        if (!scratch) HIPCHK(hipFreeAsync(Y, st));
        return "";
    }
};

template <class S> struct GemmRun {
    pp_ctx *ctx;
    i64 m, n, k;
    const void *A;
    i64 lda;
    const void *B;
    i64 ldb;
    void *C;
    i64 ldc;
    std::string err;
    void operator()() { err = run(); }
    std::string run() {
        typedef typename S::value_type T;
        if (m == 0 || n == 0) return "";
        // (+, x) over doubles: the matrix cores (PP_GEMM_VALU=1 selects the VALU tile kernel instead, for comparison)
        static const bool valu = std::getenv("PP_GEMM_VALU") != nullptr;
        if constexpr (std::is_same<S, PlusProd<double>>::value) if (!valu) {
            dim3 g((unsigned)((m + 63) / 64), (unsigned)((n + 63) / 64));
            k_gemm_mfma64<double><<<g, 256, 0, ctx->stream>>>((double *)C, ldc, (const double *)A, lda,
                                                              (const double *)B, ldb, m, n, k);
            LAUNCHCHK();
            return "";
        }
        constexpr int TM = sizeof(T) == 4 ? 8 : 4, BM = 16 * TM;
        dim3 g((unsigned)((m + BM - 1) / BM), (unsigned)((n + BM - 1) / BM));
        k_gemm_tiled<S, TM, TM><<<g, 256, 0, ctx->stream>>>((T *)C, ldc, (const T *)A, lda, (const T *)B, ldb, m, n, k);
        LAUNCHCHK();
        return "";
    }
};

template <class S> struct GetrfStarRun {
    pp_ctx *ctx;
    i64 nb, batch;
    void *A, *TL, *TU;
    std::string err;
    void operator()() { err = run(); }
    std::string run() {
        typedef typename S::value_type T;
        if (batch == 0) return "";
        if constexpr (sizeof(T) == 4) {
            k_getrf_star_wave<S><<<(unsigned)((batch + 3) / 4), 256, 0, ctx->stream>>>((T *)A, (T *)TL, (T *)TU,
                                                                                     (int)nb, batch);
        } else {
            k_getrf_star<S><<<(unsigned)batch, NT, 0, ctx->stream>>>((T *)A, (T *)TL, (T *)TU, (int)nb);
        }
        LAUNCHCHK();
        return "";
    }
};

template <class S> std::string factor_impl(pp_ctx *ctx, pp_fac *fac, const void *nz) {
    FactorRun<S> r{ctx, fac, nz};
    r();
    return r.err;
}
template <class S> std::string packs_impl(pp_ctx *ctx, pp_fac *fac) {
    PacksRun<S> r{ctx, fac};
    r();
    return r.err;
}
template <class S> std::string star_impl(pp_ctx *ctx, const pp_fac *fac, void *out, i64 ldc, int host) {
    StarRun<S> r{ctx, fac, out, ldc, host};
    r();
    return r.err;
}
template <class S>
std::string star_src_impl(pp_ctx *ctx, const pp_fac *fac, const RowSub &R, i64 nsrc, int cols, void *out, i64 ldo) {
    StarSrcRun<S> r{ctx, fac, &R, nsrc, cols, out, ldo};
    r();
    return r.err;
}
template <class S>
std::string solve_impl(pp_ctx *ctx, const pp_fac *fac, void *B, i64 ldb, i64 nrhs, bool left, bool trans,
                       void *scratch) {
    SolveRun<S> r{ctx, fac, B, ldb, nrhs, left, trans, scratch};
    r();
    return r.err;
}
template <class S>
std::string gemm_impl(pp_ctx *ctx, i64 m, i64 n, i64 k, const void *A, i64 lda, const void *B, i64 ldb, void *C, i64 ldc) {
    GemmRun<S> r{ctx, m, n, k, A, lda, B, ldb, C, ldc};
    r();
    return r.err;
}
template <class S> std::string getrf_impl(pp_ctx *ctx, i64 nb, i64 batch, void *A, void *TL, void *TU) {
    GetrfStarRun<S> r{ctx, nb, batch, A, TL, TU};
    r();
    return r.err;
}

}  // namespace pp
