// pp_api.cpp -- the C ABI of libpathpack_hip.so (declared in include/pathpack_hip.h).
//
// Handles, argument checks, device-memory checks before any launch, plan upload; the numeric work is in
// pp_device.hip, the symbolic analysis in pp_symbolic.cpp, the plans in pp_plan.cpp.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <thread>

#include "../../include/pathpack_hip.h"
#include "pp_internal.h"
#include "pp_semiring.h"

using pp::i64;

static thread_local std::string g_err;

static pp_status fail(pp_ctx *ctx, pp_status code, const std::string &msg) {
    if (ctx) ctx->err = msg;
    else g_err = msg;
    return code;
}

#define CHECK_HIP(ctx, x)                                                                     \
    do {                                                                                      \
        hipError_t e_ = (x);                                                                  \
        if (e_ != hipSuccess) return fail(ctx, PP_EHIP, std::string(#x ": ") + hipGetErrorString(e_)); \
    } while (0)

pp_sym::~pp_sym() {
    delete fplan;
    delete splan;
}

pp_fac::~pp_fac() {
    // one block (stream-ordered pool of the context's stream): the plans and the factor arrays
    for (void *p : plan.owned) hipFreeAsync(p, ctx->stream);
}

static bool supported(int semiring, int dtype) {
    if (dtype == PP_I32) return semiring == PP_ORAND;
    if (dtype == PP_F32 || dtype == PP_F64) return semiring >= PP_MINPLUS && semiring <= PP_PLUSPROD;
    return false;
}

extern "C" {

pp_status pp_init(pp_ctx **out, int device) {
    if (!out) return fail(nullptr, PP_EINVAL, "pp_init: null output");
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) return fail(nullptr, PP_ENODEV, "pp_init: no HIP device");
    if (device < 0 || device >= count) return fail(nullptr, PP_ENODEV, "pp_init: device index out of range");
    if (hipSetDevice(device) != hipSuccess) return fail(nullptr, PP_EHIP, "pp_init: hipSetDevice failed");
    pp_ctx *ctx = new (std::nothrow) pp_ctx;
    if (!ctx) return fail(nullptr, PP_ENOMEM, "pp_init: out of host memory");
    ctx->device = device;
    {
        int cu = 0;
        if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cu > 0)
            ctx->num_cu = cu;
    }
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return fail(nullptr, PP_EHIP, "pp_init: hipStreamCreate failed");
    }
    for (auto &e : ctx->ev)
        if (hipEventCreate(&e) != hipSuccess) {
            delete ctx;
            return fail(nullptr, PP_EHIP, "pp_init: hipEventCreate failed");
        }
    *out = ctx;
    return PP_OK;
}

pp_status pp_destroy(pp_ctx *ctx) {
    if (!ctx) return PP_OK;
    hipSetDevice(ctx->device);
    if (ctx->stream) {
        hipStreamSynchronize(ctx->stream);
        hipStreamDestroy(ctx->stream);
    }
    for (auto &e : ctx->ev)
        if (e) hipEventDestroy(e);
    if (ctx->staging) hipHostFree(ctx->staging);
    delete ctx;
    return PP_OK;
}

const char *pp_last_error(const pp_ctx *ctx) { return ctx ? ctx->err.c_str() : g_err.c_str(); }

pp_status pp_synchronize(pp_ctx *ctx) {
    if (!ctx) return fail(nullptr, PP_EINVAL, "pp_synchronize: null context");
    CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return PP_OK;
}

pp_status pp_stream(pp_ctx *ctx, void **stream) {
    if (!ctx || !stream) return fail(ctx, PP_EINVAL, "pp_stream: null argument");
    *stream = (void *)ctx->stream;
    return PP_OK;
}

// ===== symbolic =====

pp_status pp_symbolic(int64_t n, const int64_t *colptr, const int64_t *rowval, int ordering, int amalgamate,
                      const int64_t *perm, pp_sym **out) {
    if (!out) return fail(nullptr, PP_EINVAL, "pp_symbolic: null output");
    *out = nullptr;
    if (n < 0 || !colptr || (n > 0 && colptr[n] > 0 && !rowval)) return fail(nullptr, PP_EINVAL, "pp_symbolic: bad matrix");
    if (ordering < 0 || ordering > 2) return fail(nullptr, PP_EINVAL, "pp_symbolic: unknown ordering");
    if (ordering == PP_ORDER_GIVEN && !perm) return fail(nullptr, PP_EINVAL, "pp_symbolic: ordering GIVEN needs perm");
    pp_sym *s = new (std::nothrow) pp_sym;
    if (!s) return fail(nullptr, PP_ENOMEM, "pp_symbolic: out of host memory");
    pp::SymOptions o;
    o.ordering = ordering;
    o.amalgamate = amalgamate;
    std::string err;
    try {
        err = pp::analyze(n, colptr, rowval, o, perm, s->S);
    } catch (const std::bad_alloc &) {
        err = "out of host memory";
    }
    if (!err.empty()) {
        delete s;
        return fail(nullptr, PP_EINVAL, "pp_symbolic: " + err);
    }
    *out = s;
    return PP_OK;
}

pp_status pp_symbolic_given(int64_t n, const int64_t *colptr, const int64_t *rowval, const int64_t *perm, int64_t nf,
                            const int64_t *Rptr, pp_sym **out) {
    if (!out) return fail(nullptr, PP_EINVAL, "pp_symbolic_given: null output");
    *out = nullptr;
    if (n < 0 || !colptr || !perm || !Rptr || nf < 0) return fail(nullptr, PP_EINVAL, "pp_symbolic_given: bad arguments");
    pp_sym *s = new (std::nothrow) pp_sym;
    if (!s) return fail(nullptr, PP_ENOMEM, "pp_symbolic_given: out of host memory");
    std::string err;
    try {
        err = pp::analyze_given(n, colptr, rowval, perm, nf, Rptr, s->S);
    } catch (const std::bad_alloc &) {
        err = "out of host memory";
    }
    if (!err.empty()) {
        delete s;
        return fail(nullptr, PP_EINVAL, "pp_symbolic_given: " + err);
    }
    *out = s;
    return PP_OK;
}

pp_status pp_sym_size(const pp_sym *sym, int64_t *n, int64_t *nf, int64_t *nstgt, int64_t *maxfront) {
    if (!sym) return fail(nullptr, PP_EINVAL, "pp_sym_size: null symbolic");
    if (n) *n = sym->S.n;
    if (nf) *nf = sym->S.nf;
    if (nstgt) *nstgt = (int64_t)sym->S.Stgt.size();
    if (maxfront) {
        int64_t m = 0;
        for (i64 f = 0; f < sym->S.nf; f++)
            m = std::max<int64_t>(m, (sym->S.Rptr[f + 1] - sym->S.Rptr[f]) + (sym->S.Sptr[f + 1] - sym->S.Sptr[f]));
        *maxfront = m;
    }
    return PP_OK;
}

pp_status pp_sym_export(const pp_sym *sym, int64_t *perm, int64_t *Rptr, int64_t *Sptr, int64_t *Stgt, int64_t *parent) {
    if (!sym) return fail(nullptr, PP_EINVAL, "pp_sym_export: null symbolic");
    const pp::Symbolic &S = sym->S;
    if (perm) std::copy(S.perm.begin(), S.perm.end(), perm);
    if (Rptr) std::copy(S.Rptr.begin(), S.Rptr.end(), Rptr);
    if (Sptr) std::copy(S.Sptr.begin(), S.Sptr.end(), Sptr);
    if (Stgt) std::copy(S.Stgt.begin(), S.Stgt.end(), Stgt);
    if (parent) std::copy(S.parent.begin(), S.parent.end(), parent);
    return PP_OK;
}

pp_status pp_sym_stats(const pp_sym *sym, double *st) {
    if (!sym || !st) return fail(nullptr, PP_EINVAL, "pp_sym_stats: null argument");
    const pp::Symbolic &S = sym->S;
    const double v[10] = {S.madds_factor_alg, S.madds_star_alg, S.madds_rhs_alg, S.nnzL_alg, S.madds_factor,
                          S.madds_star,       S.madds_rhs,      S.nnzL,          S.seconds_order, S.seconds_total};
    std::copy(v, v + 10, st);
    return PP_OK;
}

pp_status pp_sym_destroy(pp_sym *sym) {
    delete sym;
    return PP_OK;
}

}  // extern "C"

// ===== factor =====

// The factor and sweep plans of a structure (a cache of the immutable structure), built on two threads.
static std::string ensure_plans(const pp_sym *csym) {
    pp_sym *sym = const_cast<pp_sym *>(csym);
    if (sym->fplan && sym->splan) return "";
    auto *f = sym->fplan ? nullptr : new pp::FactorPlan;
    auto *s = sym->splan ? nullptr : new pp::SweepPlan;
    std::string ef, es;
    std::thread t;
    if (s) t = std::thread([&] { es = pp::build_sweep_plan(sym->S, *s); });
    if (f) ef = pp::build_factor_plan(sym->S, *f);
    if (t.joinable()) t.join();
    if (!ef.empty() || !es.empty()) {
        delete f;
        delete s;
        return ef.empty() ? es : ef;
    }
    if (f) sym->fplan = f;
    if (s) sym->splan = s;
    return "";
}

static pp_status factor_common(pp_ctx *ctx, const pp_sym *sym, int semiring, int dtype, const void *nzval,
                               bool on_device, pp_fac **out) {
    if (!ctx) return fail(nullptr, PP_EINVAL, "pp_factor: null context");
    if (!sym || !out) return fail(ctx, PP_EINVAL, "pp_factor: null argument");
    *out = nullptr;
    if (!supported(semiring, dtype)) return fail(ctx, PP_EUNSUPPORTED, "pp_factor: unsupported semiring / element type");
    if (sym->S.nnz > 0 && !nzval) return fail(ctx, PP_EINVAL, "pp_factor: null nzval");
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    const bool htime = std::getenv("PP_SYMTIME") != nullptr;   // host phases of pp_factor to stderr
    auto hnow = [] { return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count(); };
    double th = hnow();
    auto hstage = [&](const char *what) {
        if (!htime) return;
        const double t = hnow();
        std::fprintf(stderr, "pp_factor: %-28s %8.2f ms\n", what, (t - th) * 1e3);
        th = t;
    };
    std::string e = ensure_plans(sym);
    if (!e.empty()) return fail(ctx, PP_EINVAL, "pp_factor: " + e);
    hstage("plans");
    const pp::FactorPlan &P = *sym->fplan;
    const pp::SweepPlan &W = *sym->splan;
    const pp::Symbolic &S = sym->S;
    const size_t es = (size_t)pp::dtype_size(dtype);
    // device memory needed at the peak: the frontal arena, the factor in both layouts, the plans, the values
    const size_t nD = (size_t)S.Dptr[S.nf], nL = (size_t)S.Lptr[S.nf];
    const size_t need = es * ((size_t)P.arena + nD + 2 * nL + (size_t)W.ndpack + 2 * (size_t)W.npack + (size_t)S.nnz) +
                        sizeof(i64) * (3 * (size_t)S.nnz + 6 * (size_t)S.nf + 2 * (size_t)S.n) +
                        sizeof(int32_t) * (W.Eidx.size() + W.plist.size() + W.tiles.size() + 16 * (size_t)W.np +
                                           P.ftask.size() + P.stask.size() + P.flist.size() + P.atask.size() +
                                           P.relpos.size());
    size_t freeb = 0, totalb = 0;
    CHECK_HIP(ctx, hipMemGetInfo(&freeb, &totalb));
    if (need > freeb)
        return fail(ctx, PP_ENOMEM, "pp_factor: needs " + std::to_string(need) + " bytes of device memory, " +
                                        std::to_string(freeb) + " free");
    pp_fac *fac = new (std::nothrow) pp_fac;
    if (!fac) return fail(ctx, PP_ENOMEM, "pp_factor: out of host memory");
    fac->ctx = ctx;
    fac->sym = sym;
    fac->semiring = semiring;
    fac->dtype = dtype;
    hipStream_t st = ctx->stream;
    pp::DevPlan &d = fac->plan;
    // One device block holds the plans (uploaded by one copy from pinned staging) and the factor arrays.
    std::vector<int32_t> invp32(S.invp.begin(), S.invp.end());
    struct Part { const void *src; size_t bytes; size_t off; void **dst; };
    std::vector<Part> parts;
    size_t total = 0;
    auto place = [&](size_t bytes) {
        const size_t off = total;
        total += (std::max<size_t>(bytes, 1) + 255) & ~size_t(255);
        return off;
    };
    auto plan_part = [&](const auto &vec, auto **ptr) {
        const size_t bytes = vec.size() * sizeof(vec[0]);
        parts.push_back({vec.data(), bytes, place(bytes), (void **)ptr});
    };
    plan_part(P.nn, &d.nn);
    plan_part(P.na, &d.na);
    plan_part(P.nj, &d.nj);
    plan_part(P.relpos, &d.relpos);
    plan_part(P.chptr, &d.chptr);
    plan_part(P.chidx, &d.chidx);
    plan_part(P.Foff, &d.Foff);
    plan_part(P.Sptr32, &d.Sptr);
    plan_part(P.entry_pos, &d.entry_pos);
    plan_part(P.flist, &d.flist);
    plan_part(P.atask, &d.atask);
    plan_part(P.etask, &d.etask);
    plan_part(P.ftask, &d.ftask);
    plan_part(P.stask, &d.stask);
    plan_part(S.Dptr, &d.Dptr);
    plan_part(S.Lptr, &d.Lptr);
    plan_part(S.Rptr, &d.Rptr);
    plan_part(W.front, &d.p_front);
    plan_part(W.c0, &d.p_c0);
    plan_part(W.w, &d.p_w);
    plan_part(W.e, &d.p_e);
    plan_part(W.lo_ext, &d.p_lo);
    plan_part(W.chunks, &d.p_chunks);
    plan_part(W.eoff, &d.p_eoff);
    plan_part(W.poff, &d.p_poff);
    plan_part(W.doff, &d.p_doff);
    plan_part(W.rowA_lo, &d.p_rowA_lo);
    plan_part(W.rowA_hi, &d.p_rowA_hi);
    plan_part(W.rowB_lo, &d.p_rowB_lo);
    plan_part(W.rowB_hi, &d.p_rowB_hi);
    plan_part(W.Eidx, &d.Eidx);
    plan_part(W.plist, &d.plist);
    plan_part(W.tiles, &d.tiles);
    plan_part(S.perm, &d.perm);
    plan_part(S.invp, &d.invp);
    plan_part(invp32, &d.invp32);
    const size_t plan_bytes = total;
    const size_t oLD = place(nD * es), oLL = place(nL * es), oUL = place(nL * es), oD = place(W.ndpack * es),
                 oU = place(W.npack * es), oL = place(W.npack * es);
    if (ctx->staging_bytes < plan_bytes) {
        if (ctx->staging) hipHostFree(ctx->staging);
        ctx->staging = nullptr;
        ctx->staging_bytes = 0;
        if (hipHostMalloc(&ctx->staging, plan_bytes, hipHostMallocDefault) != hipSuccess) {
            delete fac;
            return fail(ctx, PP_ENOMEM, "pp_factor: pinned staging allocation failed");
        }
        ctx->staging_bytes = plan_bytes;
    }
    hstage("layout + staging alloc");
    for (const Part &q : parts)
        if (q.bytes) std::memcpy((char *)ctx->staging + q.off, q.src, q.bytes);
    hstage("staging copy");
    void *block = nullptr;
    if (hipMallocAsync(&block, total, st) != hipSuccess) {
        delete fac;
        return fail(ctx, PP_ENOMEM, "pp_factor: hipMalloc of the factor failed");
    }
    d.owned.push_back(block);
    for (const Part &q : parts) *q.dst = q.bytes ? (void *)((char *)block + q.off) : nullptr;
    fac->LD = (char *)block + oLD;
    fac->LL = (char *)block + oLL;
    fac->UL = (char *)block + oUL;
    fac->Dpack = (char *)block + oD;
    fac->Upack = (char *)block + oU;
    fac->Lpack = (char *)block + oL;
    if (hipMemcpyAsync(block, ctx->staging, plan_bytes, hipMemcpyHostToDevice, st) != hipSuccess) {
        delete fac;
        return fail(ctx, PP_EHIP, "pp_factor: upload of the plans failed");
    }
    const void *dnz = nzval;
    void *tmpnz = nullptr;
    if (!on_device && S.nnz > 0) {
        if (hipMalloc(&tmpnz, S.nnz * es) != hipSuccess) {
            delete fac;
            return fail(ctx, PP_ENOMEM, "pp_factor: hipMalloc of the values failed");
        }
        if (hipMemcpyAsync(tmpnz, nzval, S.nnz * es, hipMemcpyHostToDevice, st) != hipSuccess) {
            hipFree(tmpnz);
            delete fac;
            return fail(ctx, PP_EHIP, "pp_factor: upload of the values failed");
        }
        dnz = tmpnz;
    }
    hstage("alloc + upload issue");
    e = pp::device_factor(ctx, fac, dnz);
    hstage("launches");
    hipError_t se = hipStreamSynchronize(st);
    hstage("device wait");
    if (tmpnz) hipFree(tmpnz);
    if (!e.empty() || se != hipSuccess) {
        delete fac;
        return fail(ctx, PP_EHIP, "pp_factor: " + (e.empty() ? std::string(hipGetErrorString(se)) : e));
    }
    *out = fac;
    return PP_OK;
}

extern "C" {

pp_status pp_factor(pp_ctx *ctx, const pp_sym *sym, int semiring, int dtype, const void *nzval, pp_fac **fac) {
    return factor_common(ctx, sym, semiring, dtype, nzval, false, fac);
}

pp_status pp_factor_device(pp_ctx *ctx, const pp_sym *sym, int semiring, int dtype, const void *d_nzval, pp_fac **fac) {
    return factor_common(ctx, sym, semiring, dtype, d_nzval, true, fac);
}

pp_status pp_fac_export(pp_ctx *ctx, const pp_fac *fac, void *LD, void *UD, void *LL, void *UL) {
    if (!ctx || !fac) return fail(ctx, PP_EINVAL, "pp_fac_export: null argument");
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    const pp::Symbolic &S = fac->sym->S;
    const size_t es = (size_t)pp::dtype_size(fac->dtype);
    const size_t nD = (size_t)S.Dptr[S.nf] * es, nL = (size_t)S.Lptr[S.nf] * es;
    if (LD && nD) CHECK_HIP(ctx, hipMemcpy(LD, fac->LD, nD, hipMemcpyDeviceToHost));
    if (UD && nD) CHECK_HIP(ctx, hipMemcpy(UD, fac->LD, nD, hipMemcpyDeviceToHost));
    if (LL && nL) CHECK_HIP(ctx, hipMemcpy(LL, fac->LL, nL, hipMemcpyDeviceToHost));
    if (UL && nL) CHECK_HIP(ctx, hipMemcpy(UL, fac->UL, nL, hipMemcpyDeviceToHost));
    return PP_OK;
}

pp_status pp_fac_destroy(pp_fac *fac) {
    if (!fac) return PP_OK;
    hipSetDevice(fac->ctx->device);
    hipStreamSynchronize(fac->ctx->stream);
    delete fac;
    return PP_OK;
}

// ===== star and solves =====

pp_status pp_star(pp_ctx *ctx, const pp_fac *fac, void *out, int64_t ldc, int out_on_device) {
    if (!ctx || !fac || !out) return fail(ctx, PP_EINVAL, "pp_star: null argument");
    const i64 n = fac->sym->S.n;
    if (ldc < n) return fail(ctx, PP_EINVAL, "pp_star: ldc < n");
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    const size_t es = (size_t)pp::dtype_size(fac->dtype);
    size_t freeb = 0, totalb = 0;
    CHECK_HIP(ctx, hipMemGetInfo(&freeb, &totalb));
    const size_t need = (size_t)n * n * es * (out_on_device ? 1 : 2);
    if (need > freeb)
        return fail(ctx, PP_ENOMEM, "pp_star: needs " + std::to_string(need) + " bytes of device memory, " +
                                        std::to_string(freeb) + " free");
    void *dout = out;
    if (!out_on_device) CHECK_HIP(ctx, hipMalloc(&dout, std::max<size_t>(1, (size_t)n * n * es)));
    std::string e = pp::device_star(ctx, fac, dout, out_on_device ? ldc : n);
    hipError_t se = hipStreamSynchronize(ctx->stream);
    if (e.empty() && se == hipSuccess && !out_on_device) {
        if (ldc == n) se = hipMemcpy(out, dout, (size_t)n * n * es, hipMemcpyDeviceToHost);
        else se = hipMemcpy2D(out, ldc * es, dout, n * es, n * es, n, hipMemcpyDeviceToHost);
    }
    if (!out_on_device) hipFree(dout);
    if (!e.empty() || se != hipSuccess)
        return fail(ctx, PP_EHIP, "pp_star: " + (e.empty() ? std::string(hipGetErrorString(se)) : e));
    return PP_OK;
}

static pp_status solve(pp_ctx *ctx, const pp_fac *fac, void *B, int64_t ldb, int64_t nrhs, int on_device, bool left) {
    const char *name = left ? "pp_lmul" : "pp_rmul";
    if (!ctx || !fac || (!B && nrhs > 0)) return fail(ctx, PP_EINVAL, std::string(name) + ": null argument");
    const i64 n = fac->sym->S.n;
    if (nrhs < 0) return fail(ctx, PP_EINVAL, std::string(name) + ": nrhs < 0");
    if (left ? ldb < n : ldb < nrhs) return fail(ctx, PP_EINVAL, std::string(name) + ": leading dimension too small");
    if (nrhs == 0 || n == 0) return PP_OK;
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    const size_t es = (size_t)pp::dtype_size(fac->dtype);
    const size_t bytesB = (size_t)ldb * (size_t)(left ? nrhs : n) * es;
    size_t freeb = 0, totalb = 0;
    CHECK_HIP(ctx, hipMemGetInfo(&freeb, &totalb));
    const size_t need = (size_t)n * nrhs * es + (on_device ? 0 : bytesB);
    if (need > freeb) return fail(ctx, PP_ENOMEM, std::string(name) + ": not enough device memory");
    void *dB = B;
    if (!on_device) {
        CHECK_HIP(ctx, hipMalloc(&dB, bytesB));
        hipError_t ue = hipMemcpy(dB, B, bytesB, hipMemcpyHostToDevice);
        if (ue != hipSuccess) {
            hipFree(dB);
            return fail(ctx, PP_EHIP, std::string(name) + ": upload failed");
        }
    }
    std::string e = left ? pp::device_lmul(ctx, fac, dB, ldb, nrhs) : pp::device_rmul(ctx, fac, dB, ldb, nrhs);
    hipError_t se = hipStreamSynchronize(ctx->stream);
    if (e.empty() && se == hipSuccess && !on_device) se = hipMemcpy(B, dB, bytesB, hipMemcpyDeviceToHost);
    if (!on_device) hipFree(dB);
    if (!e.empty() || se != hipSuccess)
        return fail(ctx, PP_EHIP, std::string(name) + ": " + (e.empty() ? std::string(hipGetErrorString(se)) : e));
    return PP_OK;
}

pp_status pp_lmul(pp_ctx *ctx, const pp_fac *fac, void *B, int64_t ldb, int64_t nrhs, int on_device) {
    return solve(ctx, fac, B, ldb, nrhs, on_device, true);
}

pp_status pp_rmul(pp_ctx *ctx, const pp_fac *fac, void *B, int64_t ldb, int64_t nrhs, int on_device) {
    return solve(ctx, fac, B, ldb, nrhs, on_device, false);
}

// ===== dense kernels =====

pp_status pp_sgemx(pp_ctx *ctx, int semiring, int dtype, int64_t m, int64_t n, int64_t k, const void *A, int64_t lda,
                   const void *B, int64_t ldb, void *C, int64_t ldc) {
    if (!ctx) return fail(nullptr, PP_EINVAL, "pp_sgemx: null context");
    if (!supported(semiring, dtype)) return fail(ctx, PP_EUNSUPPORTED, "pp_sgemx: unsupported semiring / element type");
    if (m < 0 || n < 0 || k < 0 || lda < std::max<int64_t>(1, m) || ldb < std::max<int64_t>(1, k) ||
        ldc < std::max<int64_t>(1, m))
        return fail(ctx, PP_EINVAL, "pp_sgemx: bad sizes");
    if ((m > 0 && n > 0) && (!C || (k > 0 && (!A || !B)))) return fail(ctx, PP_EINVAL, "pp_sgemx: null operand");
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    std::string e = pp::device_sgemx(ctx, semiring, dtype, m, n, k, A, lda, B, ldb, C, ldc);
    if (!e.empty()) return fail(ctx, PP_EHIP, "pp_sgemx: " + e);
    return PP_OK;
}

pp_status pp_getrf_star_batched(pp_ctx *ctx, int semiring, int dtype, int64_t nb, int64_t batch, void *A, void *TL,
                                void *TU) {
    if (!ctx) return fail(nullptr, PP_EINVAL, "pp_getrf_star_batched: null context");
    if (!supported(semiring, dtype)) return fail(ctx, PP_EUNSUPPORTED, "pp_getrf_star_batched: unsupported semiring / element type");
    if (nb < 1 || nb > 64 || batch < 0) return fail(ctx, PP_EINVAL, "pp_getrf_star_batched: need 1 <= nb <= 64");
    if (batch > 0 && !A) return fail(ctx, PP_EINVAL, "pp_getrf_star_batched: null A");
    if (batch > 0x7fffffff) return fail(ctx, PP_EINVAL, "pp_getrf_star_batched: batch too large");
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    std::string e = pp::device_getrf_star_batched(ctx, semiring, dtype, nb, batch, A, TL, TU);
    if (!e.empty()) return fail(ctx, PP_EHIP, "pp_getrf_star_batched: " + e);
    return PP_OK;
}

// ===== buffers =====

pp_status pp_buffer_alloc(pp_ctx *ctx, size_t bytes, void **dptr) {
    if (!ctx || !dptr) return fail(ctx, PP_EINVAL, "pp_buffer_alloc: null argument");
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    size_t freeb = 0, totalb = 0;
    CHECK_HIP(ctx, hipMemGetInfo(&freeb, &totalb));
    if (bytes > freeb) return fail(ctx, PP_ENOMEM, "pp_buffer_alloc: not enough device memory");
    if (hipMalloc(dptr, std::max<size_t>(1, bytes)) != hipSuccess) return fail(ctx, PP_ENOMEM, "pp_buffer_alloc: hipMalloc failed");
    return PP_OK;
}

pp_status pp_buffer_free(pp_ctx *ctx, void *dptr) {
    if (!ctx) return fail(nullptr, PP_EINVAL, "pp_buffer_free: null context");
    if (dptr) CHECK_HIP(ctx, hipFree(dptr));
    return PP_OK;
}

pp_status pp_upload(pp_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(ctx, PP_EINVAL, "pp_upload: null argument");
    if (bytes) CHECK_HIP(ctx, hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return PP_OK;
}

pp_status pp_download(pp_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(ctx, PP_EINVAL, "pp_download: null argument");
    if (bytes) {
        CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
        CHECK_HIP(ctx, hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    }
    return PP_OK;
}

pp_status pp_copy(pp_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(ctx, PP_EINVAL, "pp_copy: null argument");
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    std::string e = pp::device_copy(ctx, dst, src, bytes);
    if (!e.empty()) return fail(ctx, PP_EHIP, "pp_copy: " + e);
    CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return PP_OK;
}

pp_status pp_calibrate_valu(pp_ctx *ctx, int kind, int64_t iters, double *seconds, double *lane_instr) {
    if (!ctx || !seconds || !lane_instr) return fail(ctx, PP_EINVAL, "pp_calibrate_valu: null argument");
    if (kind < 0 || kind > 1 || iters < 1 || iters > (1 << 24)) return fail(ctx, PP_EINVAL, "pp_calibrate_valu: bad kind / iters");
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    std::string e = pp::device_valu_peak(ctx, kind, (int)iters, seconds, lane_instr);
    if (!e.empty()) return fail(ctx, PP_EHIP, "pp_calibrate_valu: " + e);
    return PP_OK;
}

pp_status pp_set_timing(pp_ctx *ctx, int on) {
    if (!ctx) return fail(nullptr, PP_EINVAL, "pp_set_timing: null context");
    ctx->timing = on;
    return PP_OK;
}

pp_status pp_get_timing(const pp_ctx *ctx, double *t) {
    if (!ctx || !t) return fail(nullptr, PP_EINVAL, "pp_get_timing: null argument");
    std::copy(ctx->t, ctx->t + 8, t);
    return PP_OK;
}

}  // extern "C"
