// pp_device.hip -- dispatch of the numeric drivers over the semiring / element type pairs.
//
// The kernels and drivers are templates (pp_kernels.h); each pair is instantiated in its own translation unit
// (pp_inst_*.hip) so that they compile in parallel.
#include <cstdint>
#include <string>

#include "pp_internal.h"
#include "pp_semiring.h"

namespace pp {

template <class S> std::string factor_impl(pp_ctx *ctx, pp_fac *fac, const void *nz);
template <class S> std::string star_impl(pp_ctx *ctx, const pp_fac *fac, void *out, i64 ldc);
template <class S> std::string solve_impl(pp_ctx *ctx, const pp_fac *fac, void *B, i64 ldb, i64 nrhs, bool left);
template <class S>
std::string gemm_impl(pp_ctx *ctx, i64 m, i64 n, i64 k, const void *A, i64 lda, const void *B, i64 ldb, void *C, i64 ldc);
template <class S> std::string getrf_impl(pp_ctx *ctx, i64 nb, i64 batch, void *A, void *TL, void *TU);

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

std::string device_star(pp_ctx *ctx, const pp_fac *fac, void *d_out, i64 ldc) {
    PP_DISPATCH(fac->semiring, fac->dtype, star_impl<S>(ctx, fac, d_out, ldc));
}

std::string device_rmul(pp_ctx *ctx, const pp_fac *fac, void *d_B, i64 ldb, i64 nrhs) {
    PP_DISPATCH(fac->semiring, fac->dtype, solve_impl<S>(ctx, fac, d_B, ldb, nrhs, false));
}

std::string device_lmul(pp_ctx *ctx, const pp_fac *fac, void *d_B, i64 ldb, i64 nrhs) {
    PP_DISPATCH(fac->semiring, fac->dtype, solve_impl<S>(ctx, fac, d_B, ldb, nrhs, true));
}

std::string device_sgemx(pp_ctx *ctx, int sr, int dt, i64 m, i64 n, i64 k, const void *A, i64 lda, const void *B,
                         i64 ldb, void *C, i64 ldc) {
    PP_DISPATCH(sr, dt, gemm_impl<S>(ctx, m, n, k, A, lda, B, ldb, C, ldc));
}

std::string device_getrf_star_batched(pp_ctx *ctx, int sr, int dt, i64 nb, i64 batch, void *A, void *TL, void *TU) {
    PP_DISPATCH(sr, dt, getrf_impl<S>(ctx, nb, batch, A, TL, TU));
}

}  // namespace pp
