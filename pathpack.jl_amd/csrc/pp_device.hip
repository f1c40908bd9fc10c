// pp_device.hip -- dispatch of the numeric drivers over the semiring / element type pairs.
//
// The kernels and drivers are templates (pp_kernels.h); each pair is instantiated in its own translation unit
// (pp_inst_*.hip) so that they compile in parallel.
#include <cstdint>
#include <mutex>
#include <string>

#include "pp_internal.h"
#include "pp_semiring.h"

namespace pp {

template <class S> std::string factor_impl(pp_ctx *ctx, pp_fac *fac, const void *nz);
template <class S> std::string packs_impl(pp_ctx *ctx, pp_fac *fac);
template <class S> std::string star_impl(pp_ctx *ctx, const pp_fac *fac, void *out, i64 ldc, int host);
template <class S>
std::string star_src_impl(pp_ctx *ctx, const pp_fac *fac, const RowSub &R, i64 nsrc, int cols, void *out, i64 ldo);
template <class S>
std::string solve_impl(pp_ctx *ctx, const pp_fac *fac, void *B, i64 ldb, i64 nrhs, bool left, bool trans,
                       void *scratch);
template <class S>
std::string gemm_impl(pp_ctx *ctx, i64 m, i64 n, i64 k, const void *A, i64 lda, const void *B, i64 ldb, void *C, i64 ldc);
template <class S> std::string getrf_impl(pp_ctx *ctx, i64 nb, i64 batch, void *A, void *TL, void *TU);

// ===== the scratch of the allocation-free solves (pp_sgetrs_noalloc) =====
//
// Y, the vertex-major copy of the right-hand sides, lives in this fixed array instead of a pool allocation.  Every
// device the library runs on holds its own copy until the process ends.  The array's name is a host-side stand-in, not
// a device address: host code uses only the address hipGetSymbolAddress returns for each device, taken once per
// device with that device current (pp_init calls noalloc_scratch_setup).  Every call on one device shares that
// device's array: calls that overlap on one device (two contexts, two threads) race.  Y is written in full by the
// layout kernel before any sweep reads it, so nothing in the array needs clearing between calls.
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
void *scratch_ptr[MAX_DEVICES] = {};
}  // namespace

std::string noalloc_scratch_setup(int device) {
    if (device < 0 || device >= MAX_DEVICES) return "device index beyond the scratch table";
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (scratch_ptr[device]) return "";
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return std::string("hipGetSymbolAddress of the solve scratch: ") + hipGetErrorString(e);
    scratch_ptr[device] = p;
    return "";
}

void *noalloc_scratch(int device) {
    if (device < 0 || device >= MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lock(scratch_mu);
    return scratch_ptr[device];
}

// plain copy, 16 bytes per thread per step (the memory-counter calibration kernel)
__global__ __launch_bounds__(256) void k_copy16(uint4 *__restrict__ dst, const uint4 *__restrict__ src, i64 n16) {
    for (i64 i = blockIdx.x * (i64)256 + threadIdx.x; i < n16; i += (i64)gridDim.x * 256) dst[i] = src[i];
}

__global__ __launch_bounds__(256) void k_copy1(unsigned char *__restrict__ dst, const unsigned char *__restrict__ src,
                                               i64 n) {
    for (i64 i = blockIdx.x * (i64)256 + threadIdx.x; i < n; i += (i64)gridDim.x * 256) dst[i] = src[i];
}

std::string device_copy(pp_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return "";
    const bool aligned = ((uintptr_t)dst % 16 == 0) && ((uintptr_t)src % 16 == 0) && bytes % 16 == 0;
    if (aligned) k_copy16<<<2048, 256, 0, ctx->stream>>>((uint4 *)dst, (const uint4 *)src, (i64)(bytes / 16));
    else k_copy1<<<2048, 256, 0, ctx->stream>>>((unsigned char *)dst, (const unsigned char *)src, (i64)bytes);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? "" : std::string("kernel launch: ") + hipGetErrorString(e);
}

// VALU throughput probe: eight independent chains per lane of (kind 0) v_add_f32, or (kind 1) the MinPlus Float32
// double multiply-add of the sweeps and GEMMs, min3(p + q_i, r + q_7-i, acc_i) = v_add_f32, v_add_f32, v_min3_f32
// (the chains' inputs change every iteration, so nothing is hoisted).  Lane instructions per lane and iteration, as
// compiled for gfx950: 8 v_add_f32 (kind 0); 16 v_add_f32, 8 v_min3_f32 and the 2 v_mov_b32 that carry p and r
// (kind 1).
template <int KIND> __global__ __launch_bounds__(256) void k_valu_peak(float *__restrict__ out, int iters, float s0) {
    float acc[8], q[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        acc[i] = s0 * (float)(threadIdx.x + i);
        q[i] = s0 + (float)i;
    }
    float p = acc[0], r = acc[1];
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (KIND == 0) acc[i] = acc[i] + q[i];
            else acc[i] = MinPlus<float>::muladd2(p, q[i], r, q[7 - i], acc[i]);
        }
        if (KIND != 0) {
            p = acc[0];
            r = acc[1];
        }
    }
    float t = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) t += acc[i];
    out[blockIdx.x * 256 + threadIdx.x] = t;
}

std::string device_valu_peak(pp_ctx *ctx, int kind, int iters, double *seconds, double *lane_instr) {
    const int blocks = ctx->num_cu * 8;
    float *out = nullptr;
    hipStream_t st = ctx->stream;
    if (ctx_alloc(ctx, (void **)&out, (size_t)blocks * 256 * sizeof(float), st) != hipSuccess) return "hipMallocAsync failed";
    hipEvent_t e0, e1;
    hipEventCreate(&e0);
    hipEventCreate(&e1);
    auto launch = [&](int it) {
        if (kind == 0) k_valu_peak<0><<<blocks, 256, 0, st>>>(out, it, 1e-3f);
        else k_valu_peak<1><<<blocks, 256, 0, st>>>(out, it, 1e-3f);
    };
    launch(iters / 10 + 1);   // warm-up
    hipEventRecord(e0, st);
    launch(iters);
    hipEventRecord(e1, st);
    hipError_t e = hipEventSynchronize(e1);
    float ms = 0;
    hipEventElapsedTime(&ms, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipFreeAsync(out, st);
    if (e != hipSuccess) return std::string("valu probe: ") + hipGetErrorString(e);
    *seconds = ms * 1e-3;
    *lane_instr = (double)blocks * 256 * (double)iters * (kind == 0 ? 8 : 26);
    return "";
}

#define PP_DISPATCH(sr, dt, EXPR)                                        \
    do {                                                                 \
        std::string err_;                                                \
        bool ok_ = dispatch(sr, dt, [&]<class S>() { err_ = EXPR; });    \
        if (!ok_) return "unsupported semiring / element type";          \
        return err_;                                                     \
    } while (0)

std::string device_factor(pp_ctx *ctx, pp_fac *fac, const void *d_nzval) {
    PP_DISPATCH(fac->semiring, fac->dtype, factor_impl<S>(ctx, fac, d_nzval));
}

std::string device_factor_packs(pp_ctx *ctx, pp_fac *fac) { PP_DISPATCH(fac->semiring, fac->dtype, packs_impl<S>(ctx, fac)); }

std::string device_star(pp_ctx *ctx, const pp_fac *fac, void *out, i64 ldc, int host) {
    PP_DISPATCH(fac->semiring, fac->dtype, star_impl<S>(ctx, fac, out, ldc, host));
}

std::string device_star_sources(pp_ctx *ctx, const pp_fac *fac, const RowSub &R, i64 nsrc, int cols, void *out, i64 ldo) {
    PP_DISPATCH(fac->semiring, fac->dtype, star_src_impl<S>(ctx, fac, R, nsrc, cols, out, ldo));
}

std::string device_solve(pp_ctx *ctx, const pp_fac *fac, void *d_B, i64 ldb, i64 nrhs, bool left, bool trans,
                         void *scratch) {
    PP_DISPATCH(fac->semiring, fac->dtype, solve_impl<S>(ctx, fac, d_B, ldb, nrhs, left, trans, scratch));
}

std::string device_sgemx(pp_ctx *ctx, int sr, int dt, i64 m, i64 n, i64 k, const void *A, i64 lda, const void *B,
                         i64 ldb, void *C, i64 ldc) {
    PP_DISPATCH(sr, dt, gemm_impl<S>(ctx, m, n, k, A, lda, B, ldb, C, ldc));
}

std::string device_getrf_star_batched(pp_ctx *ctx, int sr, int dt, i64 nb, i64 batch, void *A, void *TL, void *TU) {
    PP_DISPATCH(sr, dt, getrf_impl<S>(ctx, nb, batch, A, TL, TU));
}

}  // namespace pp
