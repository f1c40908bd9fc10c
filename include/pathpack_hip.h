/*
 * pathpack_hip.h -- C ABI of libpathpack_hip.so, the MI355X (gfx950) backend of PATHPACK.jl's multifrontal semiring
 * LU path.
 *
 * The entry points replace what the reference computes on the CPU behind its public API (reference citations are
 * file:line in AlgebraicJulia/PATHPACK.jl):
 *
 *   mlu(s, A; alg)        src/CPU/abstract_slu.jl:44-48      -> pp_symbolic + pp_factor
 *   mstar(s, A; alg)      src/CPU/abstract_slu.jl:85-87      -> pp_symbolic + pp_mstar (= pp_factor + pp_star)
 *   Matrix(F)             src/CPU/abstract_slu.jl:10-14      -> pp_star
 *   copyto!(F, A); lu!(F) src/CPU/chordal_slu.jl:116, abstract_slu.jl:119 -> pp_refactor
 *   sgetre! (many k)      src/CPU/chordal_slu.jl:445-493     -> pp_star_sources   (rows / columns of A*)
 *   lmul!(F, B)           src/CPU/abstract_slu.jl:131-134    -> pp_lmul
 *   rmul!(B, F)           src/CPU/abstract_slu.jl:142-145    -> pp_rmul
 *   lmul!/rmul! with transpose(F) or F'  (sgetrs!, chordal_slu.jl:337)  -> pp_sgetrs
 *   sgemx!(s, C, A, B)    src/CPU/dense/sgemx.jl:26-60       -> pp_sgemx           (dense kernel, device operands)
 *   front LU + stars      ext/PATHPACKCUDAExt/batched/sgetrf.jl:11-120 -> pp_getrf_star_batched
 *
 * Conventions
 *   - Matrices are column-major (Julia's layout).  A sparse matrix is CSC: colptr (n+1), rowval (nnz, 0-based,
 *     sorted and unique within each column), nzval (nnz).  A[i, j] is the weight of the arc i -> j
 *     (README.md:40-41).
 *   - Indices and sizes are int64_t.  Element types: PP_F32 (float), PP_F64 (double), PP_I32 (int32_t, OrAnd only).
 *   - Every function returns a pp_status; on failure pp_last_error(ctx) (or pp_last_error(NULL) for the functions
 *     without a context) returns a message.  Nothing aborts and nothing throws across the ABI.  Sizes are
 *     checked against free device memory before any work is launched (PP_ENOMEM).
 *   - A pp_ctx owns one HIP stream on one device and every device buffer it allocates.  Every result a call
 *     leaves in device memory is ordered on that stream.  (The packs of the star's large fronts are built on a
 *     second, internal stream overlapped with the start of the star; the library orders its own readers and
 *     writers of them.)  A context must not be used by two threads at once; distinct contexts are independent.
 *   - Host buffers passed in are borrowed for the duration of the call.
 */
#ifndef PATHPACK_HIP_H
#define PATHPACK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    PP_OK = 0,
    PP_EINVAL = 1,        /* invalid argument (the reference's ArgumentError) */
    PP_ENOMEM = 2,        /* not enough device memory; nothing was launched */
    PP_EUNSUPPORTED = 3,  /* unsupported semiring / element type combination */
    PP_EHIP = 4,          /* a HIP runtime call failed */
    PP_ENODEV = 5         /* no usable GPU */
} pp_status;

/* Semirings (src/CPU/semiring/*.jl).  MinPlus/MaxPlus/MaxMin/MinMax/PlusProd take PP_F32 or PP_F64; OrAnd takes
 * PP_I32. */
typedef enum {
    PP_MINPLUS = 0,   /* ([-Inf, Inf], min, +)   tropical.jl:15  */
    PP_MAXPLUS = 1,   /* ([-Inf, Inf], max, +)   tropical.jl:31  */
    PP_MAXMIN = 2,    /* ([-Inf, Inf], max, min) bottleneck.jl:31 */
    PP_MINMAX = 3,    /* ([-Inf, Inf], min, max) bottleneck.jl:15 */
    PP_PLUSPROD = 4,  /* ([0, Inf], +, *)        real.jl:16      */
    PP_ORAND = 5      /* (2^n, |, &)             boolean.jl:31   */
} pp_semiring;

typedef enum { PP_F32 = 0, PP_F64 = 1, PP_I32 = 2 } pp_dtype;

/* Orderings for pp_symbolic (the reference's `alg` keyword, abstract_slu.jl:44). */
typedef enum {
    PP_ORDER_ND = 0,       /* nested dissection (default) */
    PP_ORDER_NATURAL = 1,  /* identity */
    PP_ORDER_GIVEN = 2,    /* the permutation passed in `perm` (perm[new] = old, 0-based) */
    PP_ORDER_AMD = 3,      /* approximate minimum degree (for irregular graphs: road networks, meshes) */
    PP_ORDER_AUTO = 4      /* both ND and AMD (concurrently), keeping the order whose factor has fewer entries */
} pp_ordering;

typedef struct pp_ctx pp_ctx;
typedef struct pp_sym pp_sym;
typedef struct pp_fac pp_fac;

/* ===== context ===== */

/* Open a context on HIP device `device` (creates its stream).  Replaces nothing in the reference: Julia's threads
 * need no handle. */
pp_status pp_init(pp_ctx **ctx, int device);
pp_status pp_destroy(pp_ctx *ctx);
/* Message of the last failure on ctx; with ctx == NULL, of the calling thread's last context-free call. */
const char *pp_last_error(const pp_ctx *ctx);
/* Wait for all work queued on the context's streams. */
pp_status pp_synchronize(pp_ctx *ctx);
/* The context's HIP stream (hipStream_t) as an opaque pointer, for callers that order their own work after it. */
pp_status pp_stream(pp_ctx *ctx, void **stream);

/* ===== symbolic analysis (host only; no GPU needed) ===== */

/* Order the symmetrized pattern of A, build the postordered supernodal elimination tree and the separators.
 * Replaces ssymbolic(A; alg) (src/CPU/chordal_ssymbolic.jl:26-57) and the CliqueTrees calls behind it.
 * ordering: pp_ordering; amalgamate: merge small fronts into their parents (1) or keep fundamental supernodes (0);
 * perm: used when ordering == PP_ORDER_GIVEN, else may be NULL. */
pp_status pp_symbolic(int64_t n, const int64_t *colptr, const int64_t *rowval, int ordering, int amalgamate,
                      const int64_t *perm, pp_sym **sym);
/* The symbolic structure for a given permutation (perm[new] = old) and partition of the permuted vertices into
 * fronts (Rptr, nf + 1 entries, fronts in postorder), e.g. a structure the reference computed
 * (docs/site_factors.jl:136-160 writes one).  Separators are derived. */
pp_status pp_symbolic_given(int64_t n, const int64_t *colptr, const int64_t *rowval, const int64_t *perm, int64_t nf,
                            const int64_t *Rptr, pp_sym **sym);
/* Sizes: vertices, fronts, total separator length, largest front (nn + na). */
pp_status pp_sym_size(const pp_sym *sym, int64_t *n, int64_t *nf, int64_t *nstgt, int64_t *maxfront);
/* Copy out the structure (0-based): perm (n), Rptr (nf+1), Sptr (nf+1), Stgt (nstgt), parent (nf, -1 = root).
 * Any pointer may be NULL. */
pp_status pp_sym_export(const pp_sym *sym, int64_t *perm, int64_t *Rptr, int64_t *Sptr, int64_t *Stgt,
                        int64_t *parent);
/* Work counts in semiring multiply-adds, stats[0..9]: factor, star, one right-hand side, nnz(L) of the exact
 * (fundamental-supernode) structure; the same four of the executed (amalgamated) structure; seconds spent in the
 * ordering and in the whole analysis. */
pp_status pp_sym_stats(const pp_sym *sym, double *stats);
/* The strongly connected components (sccs and soffd, src/CPU/chordal_ssymbolic.jl:26-57,212-269): nB components in a
 * topological order, component c holding the permuted vertices [Bptr[c], Bptr[c+1]) (nB + 1 entries); and N, the nN
 * arcs between components, by column of the permuted labels (CSC: Nptr, n + 1 entries; Nidx, the permuted row of
 * each arc, ascending per column; Nsrc, its position in the nzval of the matrix given to pp_symbolic).  Every arc of
 * N goes from a lower to a higher component.  Any output pointer may be NULL (call with the arrays NULL for the
 * sizes). */
pp_status pp_sym_components(const pp_sym *sym, int64_t *nB, int64_t *Bptr, int64_t *nN, int64_t *Nptr, int64_t *Nidx,
                            int64_t *Nsrc);
pp_status pp_sym_destroy(pp_sym *sym);

/* ===== numeric factorization (device) ===== */

/* mlu: upload the values of A (nzval, host, in the CSC order given to pp_symbolic) and factorize on the device,
 * A* = U* L*.  Replaces copyto!(F, A) + lu!(F) (src/CPU/chordal_slu.jl:116-328, src/CPU/chordal/sgetrf.jl:3-290).
 * The factor stays on the device; the symbolic object must outlive it. */
pp_status pp_factor(pp_ctx *ctx, const pp_sym *sym, int semiring, int dtype, const void *nzval, pp_fac **fac);
/* Same, with nzval already in device memory. */
pp_status pp_factor_device(pp_ctx *ctx, const pp_sym *sym, int semiring, int dtype, const void *d_nzval,
                           pp_fac **fac);
/* New values of the same pattern into an existing factor, factorized in place: copyto!(F, A) + lu!(F)
 * (src/CPU/chordal_slu.jl:116-118, src/CPU/abstract_slu.jl:119-121), the repeated-weights plan of the reference's GPU
 * API (apsp_plan / apsp_gpu(plan, A2), ext/PATHPACKCUDAExt/api.jl:545-600).  No analysis, no plan upload and no new
 * factor buffers: nzval holds the values in the CSC order of the pattern given to pp_symbolic (the caller keeps the
 * pattern; a device pointer when on_device != 0).  Later pp_star / pp_lmul / pp_rmul use the new factor. */
pp_status pp_refactor(pp_ctx *ctx, pp_fac *fac, const void *nzval, int on_device);
/* Copy the factor to the host in the reference's layout (CliqueTrees' FChordalTriangular storage):
 * LD/UD: diagonal blocks (sum nn^2; LD holds L (strict lower) + U, UD's upper triangle holds U),
 * LL: na x nn blocks of L (sum nn*na), UL: nn x na blocks of U.  Pointers may be NULL. */
pp_status pp_fac_export(pp_ctx *ctx, const pp_fac *fac, void *LD, void *UD, void *LL, void *UL);
pp_status pp_fac_destroy(pp_fac *fac);

/* mlu(s, A::AbstractMatrix): the dense n x n matrix A (column-major, leading dimension lda >= n; device memory when
 * on_device != 0, else host) factorized in its own vertex order, A* = U* L* -- the reference's DenseSLU
 * (src/CPU/abstract_slu.jl:55-58, src/CPU/dense_slu.jl:1-44, dense sgetrf! src/CPU/dense/sgetrf.jl:5-70).  The
 * factor owns its structure (one front, no separator) and takes every call that takes a pp_fac: pp_star (sgetri!,
 * src/CPU/dense/sgetri.jl:3-35), pp_lmul / pp_rmul / pp_sgetrs (sgetrs!, src/CPU/dense/sgetrs.jl:3-57),
 * pp_fac_export (LD: the n x n in-place L + U of DenseSLU.A). */
pp_status pp_dense_factor(pp_ctx *ctx, int semiring, int dtype, int64_t n, const void *A, int64_t lda, int on_device,
                          pp_fac **fac);
/* copyto!(F, A) + lu!(F) of a dense factorization (src/CPU/dense_slu.jl:23-33): new values, factorized in place. */
pp_status pp_dense_refactor(pp_ctx *ctx, pp_fac *fac, const void *A, int64_t lda, int on_device);
/* sgetrf!(s, A) on a device matrix: A <- L + U with A* = U* L*, in place (src/CPU/dense/sgetrf.jl:5-17; the
 * reference's GPU method CPU.sgetrf!(s, A::CuMatrix), ext/PATHPACKCUDAExt/dense/dense.jl:31-33). */
pp_status pp_dense_sgetrf(pp_ctx *ctx, int semiring, int dtype, int64_t n, void *A, int64_t lda);

/* ===== star and solves (device) ===== */

/* Matrix(F): the full star A* (n x n, column-major, ldc >= n, original labels) into `out`: a device pointer when
 * out_on_device != 0, else a host pointer (the star is assembled in HBM, then copied back).  Replaces sgetri!(F, C)
 * (src/CPU/chordal_slu.jl:501-513 -> chordal/sgetri.jl:13-31, utils.jl:261-505). */
pp_status pp_star(pp_ctx *ctx, const pp_fac *fac, void *out, int64_t ldc, int out_on_device);
/* mstar: pp_factor then pp_star in one call, the star queued behind the factorization with no wait in between.
 * Replaces mstar(s, A) = Matrix(mlu(s, A)) (src/CPU/abstract_slu.jl:85-87) after the symbolic analysis.  nzval is in
 * host memory (nz_on_device == 0) or device memory; out and ldc as for pp_star.  fac_out may be NULL (the factor is
 * freed before returning), else it receives the factor for later solves. */
pp_status pp_mstar(pp_ctx *ctx, const pp_sym *sym, int semiring, int dtype, const void *nzval, int nz_on_device,
                   void *out, int64_t ldc, int out_on_device, pp_fac **fac_out);
/* Rows (which = 0) or columns (which = 1) of A* for the sources src[0..nsrc) (0-based original labels, in any
 * order, repeats allowed): rows: out (nsrc x n, ldo >= nsrc) row k <- row src[k] of A*; columns: out (n x nsrc,
 * ldo >= n) column k <- column src[k] of A*.  The sweeps visit, for each front, only the sources of its subtree
 * (forward) and of its component (backward).  Replaces sgetre!(F, Val(:L), Val(:T), b, k) (rows) and
 * sgetre!(F, Val(:L), Val(:N), b, k) (columns), one source at a time in the reference
 * (src/CPU/chordal_slu.jl:445-493, chordal/sgetre.jl).  `out` is a device pointer when out_on_device != 0. */
pp_status pp_star_sources(pp_ctx *ctx, const pp_fac *fac, int which, int64_t nsrc, const int64_t *src, void *out,
                          int64_t ldo, int out_on_device);
/* lmul!(F, B): B (n x nrhs, column-major, ldb >= n) <- A* B, the least solution of X = A X (+) B.
 * B is a device pointer when on_device != 0, else a host pointer.  (abstract_slu.jl:131-134) */
pp_status pp_lmul(pp_ctx *ctx, const pp_fac *fac, void *B, int64_t ldb, int64_t nrhs, int on_device);
/* rmul!(B, F): B (nrhs x n, column-major, ldb >= nrhs) <- B A*, the least solution of X = X A (+) B.
 * (abstract_slu.jl:142-145) */
pp_status pp_rmul(pp_ctx *ctx, const pp_fac *fac, void *B, int64_t ldb, int64_t nrhs, int on_device);
/* The solves with the factor or its transpose: sgetrs!(F, side, trans, B) (src/CPU/chordal_slu.jl:337-377), which
 * lmul!(F, B) / rmul!(B, F) call for F, transpose(F) and F' (abstract_slu.jl:131-145, MaybeTransSLU).
 *   side = PP_SIDE_LEFT:  B (n x nrhs, ldb >= n)    <- op(A)* B, the least solution of X = op(A) X (+) B
 *   side = PP_SIDE_RIGHT: B (nrhs x n, ldb >= nrhs) <- B op(A)*, the least solution of X = X op(A) (+) B
 * with op(A) = A (PP_NOTRANS) or A^T (PP_TRANS; for these real semirings F' is transpose(F)).  (A^T)* = (A*)^T, so the
 * transposed solves run the same sweeps as the plain ones of the other side.  B is a device pointer when
 * on_device != 0. */
enum { PP_SIDE_LEFT = 0, PP_SIDE_RIGHT = 1 };
enum { PP_NOTRANS = 0, PP_TRANS = 1 };
pp_status pp_sgetrs(pp_ctx *ctx, const pp_fac *fac, int side, int trans, void *B, int64_t ldb, int64_t nrhs,
                    int on_device);
/* pp_sgetrs with B in device memory and no device allocation at all.  No counterpart in the reference: for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * solve's scratch (the vertex-major copy of B) is a fixed device array of 64 MiB per device, held until the process
 * ends; requests with n * nrhs * element size above 64 MiB are refused with PP_EINVAL.  The work is queued on the
 * context's stream and not waited for (pp_synchronize).  Every call on one device shares that device's array:
 * calls that overlap on one device (two contexts, two threads) race; calls on one context are ordered. */
pp_status pp_sgetrs_noalloc(pp_ctx *ctx, const pp_fac *fac, int side, int trans, void *B, int64_t ldb, int64_t nrhs);

/* ===== dense kernels (device operands) ===== */

/* C <- C (+) A (x) B over the semiring; A m x k, B k x n, C m x n, column-major device pointers.
 * (src/CPU/dense/sgemx.jl:26-60, the reference GPU's sgemx_gpu! ext/PATHPACKCUDAExt/dense/sgemx.jl) */
pp_status pp_sgemx(pp_ctx *ctx, int semiring, int dtype, int64_t m, int64_t n, int64_t k, const void *A, int64_t lda,
                   const void *B, int64_t ldb, void *C, int64_t ldc);
/* For each of `batch` dense nb x nb fronts (column-major, back to back, nb <= 64): A <- L + U (in place, no
 * pivoting, dense/sgetrf.jl:151-175), TU <- U* and TL <- L* (unit lower), as the reference's fused front diagonal
 * kernel (ext/PATHPACKCUDAExt/batched/sgetrf.jl:11-120).  Device pointers; TL or TU may be NULL. */
pp_status pp_getrf_star_batched(pp_ctx *ctx, int semiring, int dtype, int64_t nb, int64_t batch, void *A, void *TL,
                                void *TU);

/* ===== device buffers ===== */

pp_status pp_buffer_alloc(pp_ctx *ctx, size_t bytes, void **dptr);
pp_status pp_buffer_free(pp_ctx *ctx, void *dptr);
pp_status pp_upload(pp_ctx *ctx, void *dst_device, const void *src_host, size_t bytes);
pp_status pp_download(pp_ctx *ctx, void *dst_host, const void *src_device, size_t bytes);
/* Device-to-device copy by a plain copy kernel on the context's stream (also the calibration kernel for memory
 * counters).  Replaces nothing in the reference. */
pp_status pp_copy(pp_ctx *ctx, void *dst_device, const void *src_device, size_t bytes);

/* ===== measurement ===== */

/* VALU throughput probe (replaces nothing in the reference; the calibration of the VALU roofline): every lane of
 * 8 workgroups per CU runs `iters` iterations of eight independent chains of (kind 0) v_add_f32 or (kind 1) the
 * Float32 MinPlus double multiply-add of the kernels (two v_add_f32 and one v_min3_f32; plus two v_mov_b32 per
 * eight of them in the probe's loop).  Returns the kernel's seconds (HIP events) and the lane instructions it
 * executed. */
pp_status pp_calibrate_valu(pp_ctx *ctx, int kind, int64_t iters, double *seconds, double *lane_instr);

/* Per-phase device time of the last pp_factor / pp_star / pp_lmul / pp_rmul on ctx, in seconds (HIP events on the
 * context's stream): t[0] factor total, t[1] star U* sweep, t[2] star L* sweep, t[3] star relabel, t[4] solve,
 * t[5] host-side setup of the last call, t[6] the dominant sweep kernel's summed duration, t[7] its launch count.
 * Timing adds synchronization: enable with pp_set_timing(ctx, 1). */
pp_status pp_set_timing(pp_ctx *ctx, int on);
pp_status pp_get_timing(const pp_ctx *ctx, double *t);

/* Debug flags of a context (replaces nothing in the reference).  PP_DEBUG_POISON: every sweep buffer (the n x n star,
 * the rows of pp_star_sources, the right-hand sides of the solves) is filled with the all-ones bit pattern -- NaN in
 * Float32 and Float64, -1 in Int32 -- before the sweeps start, so that a kernel reading an element that nothing wrote
 * shows it in the result.  Costs one extra pass over each buffer. */
enum { PP_DEBUG_POISON = 1 };
pp_status pp_set_debug(pp_ctx *ctx, int flags);

#ifdef __cplusplus
}
#endif

#endif /* PATHPACK_HIP_H */
