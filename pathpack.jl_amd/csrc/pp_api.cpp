// pp_api.cpp -- the C ABI of libpathpack_hip.so (declared in include/pathpack_hip.h).
//
// Handles, argument checks, device-memory checks before any launch, plan upload; the numeric work is in
// pp_device.hip, the symbolic analysis in pp_symbolic.cpp, the plans in pp_plan.cpp.
#include <hip/hip_runtime.h>

#include <malloc.h>

#include <algorithm>
#include <mutex>
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
    // the blocks (stream-ordered pool of the context's stream): the plans and the factor arrays
    for (void *p : plan.owned) hipFreeAsync(p, ctx->stream);
    delete own_sym;   // a dense factorization's own structure (host only)
}

static bool supported(int semiring, int dtype) {
    if (dtype == PP_I32) return semiring == PP_ORAND;
    if (dtype == PP_F32 || dtype == PP_F64) return semiring >= PP_MINPLUS && semiring <= PP_PLUSPROD;
    return false;
}

// Free device memory for the size checks: the driver's free memory plus what the context's pool holds cached (freed
// stream-ordered allocations, which the pool keeps for the next call).
static hipError_t mem_free(pp_ctx *ctx, size_t *freeb, size_t *totalb) {
    hipError_t e = hipMemGetInfo(freeb, totalb);
    if (e != hipSuccess) return e;
    uint64_t res = 0, used = 0;
    if (ctx->pool && hipMemPoolGetAttribute(ctx->pool, hipMemPoolAttrReservedMemCurrent, &res) == hipSuccess &&
        hipMemPoolGetAttribute(ctx->pool, hipMemPoolAttrUsedMemCurrent, &used) == hipSuccess && res > used)
        *freeb += (size_t)(res - used);
    return hipSuccess;
}

// hipMalloc outside the pool: when the driver is short, the pool's cached memory is returned to it first
static hipError_t dev_malloc(pp_ctx *ctx, void **p, size_t bytes) {
    hipError_t e = hipMalloc(p, bytes);
    if (e == hipSuccess) return e;
    (void)hipGetLastError();
    hipStreamSynchronize(ctx->stream);
    hipStreamSynchronize(ctx->aux_stream);
    if (ctx->pool) hipMemPoolTrimTo(ctx->pool, 0);
    return hipMalloc(p, bytes);
}

extern "C" {

// The host analysis allocates a few dozen arrays of n or nnz elements per call.  glibc serves blocks above its mmap
// threshold (128 KiB at first) with fresh mappings, which every call then faults in again, page by page (about 2 ms of
// an 11 ms analysis of a 32768-vertex graph on a 16-thread host).  Once per process, before the first analysis, the
// library raises the mmap threshold to glibc's maximum (32 MiB) and the trim threshold to 512 MiB, so that freed
// blocks stay in the heap and later calls reuse warm pages.  PP_KEEP_MALLOC=1 leaves the process's allocator alone.
static void host_heap_setup() {
    static std::once_flag once;
    std::call_once(once, [] {
        const char *keep = std::getenv("PP_KEEP_MALLOC");
        if (keep && keep[0] == '1') return;
        mallopt(M_MMAP_THRESHOLD, 32 << 20);
        mallopt(M_TRIM_THRESHOLD, 512 << 20);
    });
}

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
            pp_destroy(ctx);
            return fail(nullptr, PP_EHIP, "pp_init: hipEventCreate failed");
        }
    {
        // the context's own pool (stream-ordered allocations), which keeps freed memory until the context ends
        hipMemPoolProps props = {};
        props.allocType = hipMemAllocationTypePinned;
        props.handleTypes = hipMemHandleTypeNone;
        props.location.type = hipMemLocationTypeDevice;
        props.location.id = device;
        uint64_t keep = UINT64_MAX;
        if (hipMemPoolCreate(&ctx->pool, &props) != hipSuccess ||
            hipMemPoolSetAttribute(ctx->pool, hipMemPoolAttrReleaseThreshold, &keep) != hipSuccess) {
            pp_destroy(ctx);
            return fail(nullptr, PP_EHIP, "pp_init: creating the memory pool failed");
        }
    }
    {
        // the device address of the allocation-free solves' scratch array, taken once per device (device current)
        const std::string se = pp::noalloc_scratch_setup(device);
        if (!se.empty()) {
            pp_destroy(ctx);
            return fail(nullptr, PP_EHIP, "pp_init: " + se);
        }
    }
    if (hipStreamCreateWithFlags(&ctx->aux_stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&ctx->aux_from, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&ctx->aux_done, hipEventDisableTiming) != hipSuccess) {
        pp_destroy(ctx);
        return fail(nullptr, PP_EHIP, "pp_init: creating the second stream failed");
    }
    *out = ctx;
    return PP_OK;
}

pp_status pp_destroy(pp_ctx *ctx) {
    if (!ctx) return PP_OK;
    hipSetDevice(ctx->device);
    if (ctx->aux_stream) {
        hipStreamSynchronize(ctx->aux_stream);
        hipStreamDestroy(ctx->aux_stream);
    }
    if (ctx->aux_from) hipEventDestroy(ctx->aux_from);
    if (ctx->aux_done) hipEventDestroy(ctx->aux_done);
    if (ctx->stream) {
        hipStreamSynchronize(ctx->stream);
        hipStreamDestroy(ctx->stream);
    }
    for (auto &e : ctx->ev)
        if (e) hipEventDestroy(e);
    if (ctx->staging) hipHostFree(ctx->staging);
    if (ctx->staging2) hipHostFree(ctx->staging2);
    for (auto &e : ctx->pev)
        if (e) hipEventDestroy(e);
    for (auto &p : ctx->outpin)
        if (p) hipHostFree(p);
    for (auto &p : ctx->xfer)
        if (p) hipHostFree(p);
    for (auto &e : ctx->xev)
        if (e) hipEventDestroy(e);
    if (ctx->pool) {
        // every stream is synchronized: the pool's memory goes back to the driver (the factors of a context are
        // destroyed before it)
        hipMemPoolTrimTo(ctx->pool, 0);
        hipMemPoolDestroy(ctx->pool);
    }
    delete ctx;
    return PP_OK;
}

const char *pp_last_error(const pp_ctx *ctx) { return ctx ? ctx->err.c_str() : g_err.c_str(); }

pp_status pp_synchronize(pp_ctx *ctx) {
    if (!ctx) return fail(nullptr, PP_EINVAL, "pp_synchronize: null context");
    CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    CHECK_HIP(ctx, hipStreamSynchronize(ctx->aux_stream));
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
    host_heap_setup();
    if (!out) return fail(nullptr, PP_EINVAL, "pp_symbolic: null output");
    *out = nullptr;
    if (n < 0 || !colptr || (n > 0 && colptr[n] > 0 && !rowval)) return fail(nullptr, PP_EINVAL, "pp_symbolic: bad matrix");
    if (ordering < 0 || ordering > 4) return fail(nullptr, PP_EINVAL, "pp_symbolic: unknown ordering");
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
    host_heap_setup();
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

pp_status pp_sym_components(const pp_sym *sym, int64_t *nB, int64_t *Bptr, int64_t *nN, int64_t *Nptr, int64_t *Nidx,
                            int64_t *Nsrc) {
    if (!sym) return fail(nullptr, PP_EINVAL, "pp_sym_components: null symbolic");
    const pp::Symbolic &S = sym->S;
    if (nB) *nB = S.nB;
    if (nN) *nN = S.nN;
    if (Bptr) std::copy(S.Bptr.begin(), S.Bptr.end(), Bptr);
    if (Nptr) std::copy(S.Nptr.begin(), S.Nptr.end(), Nptr);
    if (Nidx) std::copy(S.Nidx.begin(), S.Nidx.end(), Nidx);
    if (Nsrc) std::copy(S.Nsrc.begin(), S.Nsrc.end(), Nsrc);
    return PP_OK;
}

pp_status pp_sym_destroy(pp_sym *sym) {
    delete sym;
    return PP_OK;
}

}  // extern "C"

// ===== factor =====

// Device-plan upload: the host arrays of one block are laid out at 256-byte offsets, copied into a pinned staging
// buffer and uploaded by one asynchronous copy; the bytes placed after them (the factor arrays) are not uploaded.
struct Upload {
    struct Part { const void *src; size_t bytes; size_t off; void **dst; };
    std::vector<Part> parts;
    size_t total = 0;
    size_t place(size_t bytes) {
        const size_t off = total;
        total += (std::max<size_t>(bytes, 1) + 255) & ~size_t(255);
        return off;
    }
    template <class V, class P> void add(const V &vec, P **ptr) {
        const size_t bytes = vec.size() * sizeof(vec[0]);
        parts.push_back({vec.data(), bytes, place(bytes), (void **)ptr});
    }
    // allocate the block (stream-ordered pool), stage and upload the parts; the block's address into *block
    std::string run(pp_ctx *ctx, hipStream_t st, void *&staging, size_t &staging_bytes, size_t plan_bytes, void **block) {
        if (staging_bytes < plan_bytes) {
            if (staging) hipHostFree(staging);
            staging = nullptr;
            staging_bytes = 0;
            if (hipHostMalloc(&staging, plan_bytes, hipHostMallocDefault) != hipSuccess)
                return "pinned staging allocation failed";
            staging_bytes = plan_bytes;
        }
        for (const Part &q : parts)
            if (q.bytes) std::memcpy((char *)staging + q.off, q.src, q.bytes);
        if (pp::ctx_alloc(ctx, block, total, st) != hipSuccess) return "stream-ordered allocation of the factor failed";
        for (const Part &q : parts) *q.dst = q.bytes ? (void *)((char *)*block + q.off) : nullptr;
        if (hipMemcpyAsync(*block, staging, plan_bytes, hipMemcpyHostToDevice, st) != hipSuccess)
            return "upload of the plans failed";
        return "";
    }
};

// Device memory of a factorization, from the structure alone (nothing is queued before the check): the plans and
// the factor, then the larger of the factorization's scratch (the frontal arena, the uploaded values) and what the
// sweeps keep (their plan, the panel and block packs, the block stars' scratch) plus `extra` (the star of pp_mstar).
// The plan arrays are bounded per unit (panels and blocks); everything else is exact.
static size_t factor_bytes(const pp::Symbolic &S, const pp::FactorPlan &P, size_t es, bool values_on_device,
                           size_t extra) {
    const size_t nD = (size_t)S.Dptr[S.nf], nL = (size_t)S.Lptr[S.nf];
    const pp::SweepSizes z = pp::sweep_sizes(S);
    const size_t plan1 = sizeof(i64) * (3 * (size_t)S.nnz + 6 * (size_t)S.nf + 2 * (size_t)S.n) +
                         sizeof(int32_t) * (P.stask.size() + P.flist.size() + P.atask.size() + P.etask.size() +
                                            P.relpos.size() + 3 * (size_t)S.nf) +
                         32 * 256;
    const size_t factor = es * (nD + 2 * nL);
    const size_t scratch = es * ((size_t)P.arena + (values_on_device ? 0 : (size_t)S.nnz));
    const size_t plan2 = sizeof(int32_t) * ((size_t)z.eidx + 80 * (size_t)z.units + 4 * (size_t)z.prep + (size_t)S.n) +
                         sizeof(i64) * (5 * (size_t)z.units + 2 * (size_t)S.n) + 40 * 256;
    const size_t packs = es * (2 * (size_t)z.npack + (size_t)z.ndpack + (size_t)z.nbpack + (size_t)z.nhpack +
                               (size_t)z.nb * 2 * pp::BLK_W * pp::BLK_W);
    // N (components coupled by arcs): values and sources by column and by row, pointers, indices, gather lists
    const size_t ncoup = z.nN ? (2 * es + 2 * sizeof(i64) + 2 * sizeof(int32_t) + 3 * sizeof(int32_t)) * (size_t)z.nN +
                                    2 * sizeof(i64) * ((size_t)S.n + 1) + 2 * sizeof(int32_t) * (size_t)z.units + 8 * 256
                              : 0;
    return plan1 + factor + ncoup + std::max(scratch, plan2 + packs + extra);
}

// finish: wait for the factorization before returning (pp_factor); pp_mstar queues the star behind it instead, and
// passes the star's bytes as `extra` so that the one check covers both before anything is queued
// dense: nzval is a dense n x n matrix with leading dimension dense_lda (pp_dense_factor; csym its one-front
// structure), in device memory when on_device, else in host memory
static pp_status factor_common(pp_ctx *ctx, const pp_sym *csym, int semiring, int dtype, const void *nzval,
                               bool on_device, pp_fac **out, bool finish = true, size_t extra = 0,
                               const char *who = "pp_factor", i64 dense_lda = 0) {
    if (!ctx) return fail(nullptr, PP_EINVAL, "pp_factor: null context");
    if (!csym || !out) return fail(ctx, PP_EINVAL, "pp_factor: null argument");
    *out = nullptr;
    if (!supported(semiring, dtype)) return fail(ctx, PP_EUNSUPPORTED, "pp_factor: unsupported semiring / element type");
    if ((csym->S.nnz > 0 || (dense_lda && csym->S.n > 0)) && !nzval) return fail(ctx, PP_EINVAL, "pp_factor: null nzval");
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    pp_sym *sym = const_cast<pp_sym *>(csym);   // the plans are a cache of the immutable structure
    const pp::Symbolic &S = sym->S;
    const size_t es = (size_t)pp::dtype_size(dtype);
    // The sweep plan is built on a second thread while this one builds the factor plan and the device factorizes;
    // it is needed only for the packs at the end.
    pp::SweepPlan *splan = sym->splan ? nullptr : new pp::SweepPlan;
    std::string es_err;
    std::thread sweep_thread;
    if (splan) sweep_thread = std::thread([&] { es_err = pp::build_sweep_plan(S, *splan); });
    auto join_sweep = [&]() -> std::string {
        if (!sweep_thread.joinable()) return "";
        sweep_thread.join();
        if (!es_err.empty()) {
            delete splan;
            splan = nullptr;
            return es_err;
        }
        sym->splan = splan;
        splan = nullptr;
        return "";
    };
    auto failj = [&](pp_status code, const std::string &msg) {
        join_sweep();
        return fail(ctx, code, msg);
    };
    if (!sym->fplan) {
        auto *f = new pp::FactorPlan;
        std::string e = pp::build_factor_plan(S, *f);
        if (!e.empty()) {
            delete f;
            return failj(PP_EINVAL, "pp_factor: " + e);
        }
        sym->fplan = f;
    }
    const pp::FactorPlan &P = *sym->fplan;
    const size_t nD = (size_t)S.Dptr[S.nf], nL = (size_t)S.Lptr[S.nf];
    const size_t dense_tmp = dense_lda && !on_device ? (size_t)S.n * (size_t)S.n * es : 0;   // the uploaded matrix
    const size_t need = factor_bytes(S, P, es, on_device, extra) + dense_tmp;
    size_t freeb = 0, totalb = 0;
    if (mem_free(ctx, &freeb, &totalb) != hipSuccess) return failj(PP_EHIP, std::string(who) + ": hipMemGetInfo failed");
    if (need > freeb) {
        // work still queued on the context may hold pool memory that it is about to free: wait and look again
        hipStreamSynchronize(ctx->stream);
        hipStreamSynchronize(ctx->aux_stream);
        if (mem_free(ctx, &freeb, &totalb) != hipSuccess) return failj(PP_EHIP, std::string(who) + ": hipMemGetInfo failed");
    }
    if (need > freeb)
        return failj(PP_ENOMEM, std::string(who) + ": needs " + std::to_string(need) + " bytes of device memory, " +
                                    std::to_string(freeb) + " free; nothing was launched");
    pp_fac *fac = new (std::nothrow) pp_fac;
    if (!fac) return failj(PP_ENOMEM, "pp_factor: out of host memory");
    fac->ctx = ctx;
    fac->sym = sym;
    fac->semiring = semiring;
    fac->dtype = dtype;
    hipStream_t st = ctx->stream;
    pp::DevPlan &d = fac->plan;
    auto failf = [&](pp_status code, const std::string &msg) {
        hipStreamSynchronize(st);
        hipStreamSynchronize(ctx->aux_stream);   // the block packs may still read and write this factor
        delete fac;
        return failj(code, msg);
    };
    // block 1: the factor plan and the factor in the reference layout
    Upload u1;
    u1.add(P.nn, &d.nn);
    u1.add(P.na, &d.na);
    u1.add(P.nj, &d.nj);
    u1.add(P.relpos, &d.relpos);
    u1.add(P.chptr, &d.chptr);
    u1.add(P.chidx, &d.chidx);
    u1.add(P.Foff, &d.Foff);
    u1.add(P.Sptr32, &d.Sptr);
    u1.add(P.entry_pos, &d.entry_pos);
    u1.add(P.flist, &d.flist);
    u1.add(P.atask, &d.atask);
    u1.add(P.etask, &d.etask);
    u1.add(P.stask, &d.stask);
    u1.add(S.Dptr, &d.Dptr);
    u1.add(S.Lptr, &d.Lptr);
    u1.add(S.Rptr, &d.Rptr);
    const bool coupled = S.nB > 1 && S.nN > 0;
    if (coupled) {
        u1.add(S.Nsrc, &d.Nsrc);
        u1.add(S.NTsrc, &d.NTsrc);
    }
    const size_t plan1 = u1.total;
    const size_t oLD = u1.place(nD * es), oLL = u1.place(nL * es), oUL = u1.place(nL * es);
    const size_t oNv = coupled ? u1.place((size_t)S.nN * es) : 0, oNTv = coupled ? u1.place((size_t)S.nN * es) : 0;
    void *block1 = nullptr;
    std::string e = u1.run(ctx, st, ctx->staging, ctx->staging_bytes, plan1, &block1);
    if (!e.empty()) return failf(PP_ENOMEM, "pp_factor: " + e);
    d.owned.push_back(block1);
    fac->LD = (char *)block1 + oLD;
    fac->LL = (char *)block1 + oLL;
    fac->UL = (char *)block1 + oUL;
    if (coupled) {
        fac->Nval = (char *)block1 + oNv;
        fac->NTval = (char *)block1 + oNTv;
    }
    const void *dnz = nzval;
    void *tmpnz = nullptr;
    if (dense_lda) {
        const size_t n = (size_t)S.n;
        fac->dense_src = nzval;
        fac->dense_lda = dense_lda;
        if (!on_device && n > 0) {
            if (pp::ctx_alloc(ctx, &tmpnz, n * n * es, st) != hipSuccess)
                return failf(PP_ENOMEM, std::string(who) + ": allocation of the matrix failed");
            if (hipMemcpy2DAsync(tmpnz, n * es, nzval, (size_t)dense_lda * es, n * es, n, hipMemcpyHostToDevice, st) !=
                hipSuccess) {
                hipFreeAsync(tmpnz, st);
                return failf(PP_EHIP, std::string(who) + ": upload of the matrix failed");
            }
            fac->dense_src = tmpnz;
            fac->dense_lda = (i64)n;
        }
        dnz = nullptr;
    } else if (!on_device && S.nnz > 0) {
        if (pp::ctx_alloc(ctx, &tmpnz, S.nnz * es, st) != hipSuccess) return failf(PP_ENOMEM, "pp_factor: hipMalloc of the values failed");
        if (hipMemcpyAsync(tmpnz, nzval, S.nnz * es, hipMemcpyHostToDevice, st) != hipSuccess) {
            hipFreeAsync(tmpnz, st);
            return failf(PP_EHIP, "pp_factor: upload of the values failed");
        }
        dnz = tmpnz;
    }
    e = pp::device_factor(ctx, fac, dnz);
    fac->dense_src = nullptr;
    fac->dense_lda = 0;
    if (tmpnz) hipFreeAsync(tmpnz, st);
    if (!e.empty()) return failf(PP_EHIP, "pp_factor: " + e);
    // block 2: the sweep plan, the permutation and the sweep packs (built from the factor)
    e = join_sweep();
    if (!e.empty()) return failf(PP_EINVAL, "pp_factor: " + e);
    const pp::SweepPlan &W = *sym->splan;
    std::vector<int32_t> invp32(S.invp.begin(), S.invp.end());
    Upload u2;
    u2.add(W.front, &d.p_front);
    u2.add(W.c0, &d.p_c0);
    u2.add(W.w, &d.p_w);
    u2.add(W.e, &d.p_e);
    u2.add(W.lo_ext, &d.p_lo);
    u2.add(W.chunks, &d.p_chunks);
    u2.add(W.eoff, &d.p_eoff);
    u2.add(W.poff, &d.p_poff);
    u2.add(W.doff, &d.p_doff);
    u2.add(W.rowA_lo, &d.p_rowA_lo);
    u2.add(W.rowA_hi, &d.p_rowA_hi);
    u2.add(W.rowB_lo, &d.p_rowB_lo);
    u2.add(W.rowB_hi, &d.p_rowB_hi);
    u2.add(W.Eidx, &d.Eidx);
    u2.add(W.plist, &d.plist);
    u2.add(W.tiles, &d.tiles);
    u2.add(W.b_boff, &d.b_boff);
    u2.add(W.b_hoff, &d.b_hoff);
    u2.add(W.b_kp, &d.b_kp);
    u2.add(W.b_ep, &d.b_ep);
    u2.add(W.b_bn, &d.b_bn);
    u2.add(W.prep, &d.prep);
    u2.add(W.sunits, &d.sunits);
    u2.add(W.sub_ptr, &d.sub_ptr);
    u2.add(W.sub_pan, &d.sub_pan);
    u2.add(W.sub_rows, &d.sub_rows);
    u2.add(W.sub_preF, &d.sub_preF);
    u2.add(W.sub_preB, &d.sub_preB);
    u2.add(S.perm, &d.perm);
    u2.add(S.invp, &d.invp);
    u2.add(invp32, &d.invp32);
    if (W.coupled) {
        u2.add(S.Nptr, &d.Nptr);
        u2.add(S.Nidx, &d.Nidx);
        u2.add(S.NTptr, &d.NTptr);
        u2.add(S.NTidx, &d.NTidx);
        u2.add(W.ccols, &d.ccols);
        u2.add(W.ccol_lo, &d.ccol_lo);
        u2.add(W.ccol_hi, &d.ccol_hi);
        u2.add(W.rowC_lo, &d.p_rowC_lo);
        u2.add(W.rowC_hi, &d.p_rowC_hi);
    }
    const size_t plan2 = u2.total;
    const size_t oD = u2.place(W.ndpack * es), oU = u2.place(W.npack * es), oL = u2.place(W.npack * es);
    const size_t oB = u2.place(W.nbpack * es), oH = u2.place(W.nhpack * es);
    // (no free-memory query here: the factorization is already queued and the query would wait for it; the packs'
    // stream-ordered allocation reports a shortage itself)
    void *block2 = nullptr;
    e = u2.run(ctx, st, ctx->staging2, ctx->staging2_bytes, plan2, &block2);
    if (!e.empty()) return failf(PP_ENOMEM, "pp_factor: " + e);
    d.owned.push_back(block2);
    fac->Dpack = (char *)block2 + oD;
    fac->Upack = (char *)block2 + oU;
    fac->Lpack = (char *)block2 + oL;
    fac->Bpack = (char *)block2 + oB;
    fac->Hpack = (char *)block2 + oH;
    e = pp::device_factor_packs(ctx, fac);
    hipError_t se = finish ? hipStreamSynchronize(st) : hipGetLastError();
    if (!e.empty() || se != hipSuccess)
        return failf(PP_EHIP, "pp_factor: " + (e.empty() ? std::string(hipGetErrorString(se)) : e));
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

pp_status pp_refactor(pp_ctx *ctx, pp_fac *fac, const void *nzval, int on_device) {
    if (!ctx || !fac) return fail(ctx, PP_EINVAL, "pp_refactor: null argument");
    if (fac->ctx != ctx) return fail(ctx, PP_EINVAL, "pp_refactor: the factor belongs to another context");
    if (fac->own_sym) return fail(ctx, PP_EINVAL, "pp_refactor: a dense factorization takes pp_dense_refactor");
    const pp::Symbolic &S = fac->sym->S;
    if (S.nnz > 0 && !nzval) return fail(ctx, PP_EINVAL, "pp_refactor: null nzval");
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    const size_t es = (size_t)pp::dtype_size(fac->dtype);
    const pp::SweepPlan &W = *fac->sym->splan;
    // the factorization's fronts, the star blocks' scratch and the uploaded values: the factor's own buffers are reused
    const size_t need = es * ((size_t)fac->sym->fplan->arena + (on_device ? 0 : (size_t)S.nnz) +
                              (size_t)W.nb * 2 * pp::BLK_W * pp::BLK_W);
    size_t freeb = 0, totalb = 0;
    CHECK_HIP(ctx, mem_free(ctx, &freeb, &totalb));
    if (need > freeb)
        return fail(ctx, PP_ENOMEM, "pp_refactor: needs " + std::to_string(need) + " bytes of device memory, " +
                                        std::to_string(freeb) + " free");
    hipStream_t st = ctx->stream;
    const void *dnz = nzval;
    void *tmpnz = nullptr;
    if (!on_device && S.nnz > 0) {
        if (pp::ctx_alloc(ctx, &tmpnz, S.nnz * es, st) != hipSuccess) return fail(ctx, PP_ENOMEM, "pp_refactor: hipMalloc of the values failed");
        if (hipMemcpyAsync(tmpnz, nzval, S.nnz * es, hipMemcpyHostToDevice, st) != hipSuccess) {
            hipFreeAsync(tmpnz, st);
            hipStreamSynchronize(st);
            return fail(ctx, PP_EHIP, "pp_refactor: upload of the values failed");
        }
        dnz = tmpnz;
    }
    std::string e = pp::device_factor(ctx, fac, dnz);
    if (tmpnz) hipFreeAsync(tmpnz, st);
    if (e.empty()) e = pp::device_factor_packs(ctx, fac);
    hipError_t se = hipStreamSynchronize(st);
    if (!e.empty() || se != hipSuccess)
        return fail(ctx, PP_EHIP, "pp_refactor: " + (e.empty() ? std::string(hipGetErrorString(se)) : e));
    return PP_OK;
}

pp_status pp_dense_factor(pp_ctx *ctx, int semiring, int dtype, int64_t n, const void *A, int64_t lda, int on_device,
                          pp_fac **fac) {
    if (!ctx) return fail(nullptr, PP_EINVAL, "pp_dense_factor: null context");
    if (!fac) return fail(ctx, PP_EINVAL, "pp_dense_factor: null output");
    *fac = nullptr;
    if (n < 0 || n > (int64_t)1 << 30) return fail(ctx, PP_EINVAL, "pp_dense_factor: n out of range");
    if (n > 0 && (!A || lda < n)) return fail(ctx, PP_EINVAL, "pp_dense_factor: null matrix or lda < n");
    pp_sym *sym = new (std::nothrow) pp_sym;
    if (!sym) return fail(ctx, PP_ENOMEM, "pp_dense_factor: out of host memory");
    try {
        pp::dense_structure(n, sym->S);
    } catch (const std::bad_alloc &) {
        delete sym;
        return fail(ctx, PP_ENOMEM, "pp_dense_factor: out of host memory");
    }
    pp_status st = factor_common(ctx, sym, semiring, dtype, A, on_device != 0, fac, true, 0, "pp_dense_factor",
                                 std::max<int64_t>(1, lda));
    if (st != PP_OK) {
        delete sym;
        return st;
    }
    (*fac)->own_sym = sym;
    return PP_OK;
}

pp_status pp_dense_refactor(pp_ctx *ctx, pp_fac *fac, const void *A, int64_t lda, int on_device) {
    if (!ctx || !fac) return fail(ctx, PP_EINVAL, "pp_dense_refactor: null argument");
    if (fac->ctx != ctx) return fail(ctx, PP_EINVAL, "pp_dense_refactor: the factor belongs to another context");
    if (!fac->own_sym) return fail(ctx, PP_EINVAL, "pp_dense_refactor: not a dense factorization (pp_refactor)");
    const i64 n = fac->sym->S.n;
    if (n > 0 && (!A || lda < n)) return fail(ctx, PP_EINVAL, "pp_dense_refactor: null matrix or lda < n");
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    const size_t es = (size_t)pp::dtype_size(fac->dtype);
    const pp::SweepPlan &W = *fac->sym->splan;
    const size_t need = es * ((size_t)fac->sym->fplan->arena + (on_device ? 0 : (size_t)n * (size_t)n) +
                              (size_t)W.nb * 2 * pp::BLK_W * pp::BLK_W);
    size_t freeb = 0, totalb = 0;
    CHECK_HIP(ctx, mem_free(ctx, &freeb, &totalb));
    if (need > freeb)
        return fail(ctx, PP_ENOMEM, "pp_dense_refactor: needs " + std::to_string(need) + " bytes of device memory, " +
                                        std::to_string(freeb) + " free");
    hipStream_t st = ctx->stream;
    void *tmp = nullptr;
    fac->dense_src = A;
    fac->dense_lda = std::max<int64_t>(1, lda);
    if (!on_device && n > 0) {
        if (pp::ctx_alloc(ctx, &tmp, (size_t)n * n * es, st) != hipSuccess) {
            fac->dense_src = nullptr;
            fac->dense_lda = 0;
            return fail(ctx, PP_ENOMEM, "pp_dense_refactor: allocation of the matrix failed");
        }
        if (hipMemcpy2DAsync(tmp, n * es, A, (size_t)lda * es, n * es, n, hipMemcpyHostToDevice, st) != hipSuccess) {
            hipFreeAsync(tmp, st);
            hipStreamSynchronize(st);
            fac->dense_src = nullptr;
            fac->dense_lda = 0;
            return fail(ctx, PP_EHIP, "pp_dense_refactor: upload of the matrix failed");
        }
        fac->dense_src = tmp;
        fac->dense_lda = n;
    }
    std::string e = pp::device_factor(ctx, fac, nullptr);
    fac->dense_src = nullptr;
    fac->dense_lda = 0;
    if (tmp) hipFreeAsync(tmp, st);
    if (e.empty()) e = pp::device_factor_packs(ctx, fac);
    hipError_t se = hipStreamSynchronize(st);
    if (!e.empty() || se != hipSuccess)
        return fail(ctx, PP_EHIP, "pp_dense_refactor: " + (e.empty() ? std::string(hipGetErrorString(se)) : e));
    return PP_OK;
}

pp_status pp_dense_sgetrf(pp_ctx *ctx, int semiring, int dtype, int64_t n, void *A, int64_t lda) {
    pp_fac *fac = nullptr;
    pp_status st = pp_dense_factor(ctx, semiring, dtype, n, A, lda, 1, &fac);
    if (st != PP_OK) return st;
    const size_t es = (size_t)pp::dtype_size(dtype);
    hipError_t e = hipSuccess;
    if (n > 0)
        e = hipMemcpy2DAsync(A, (size_t)lda * es, fac->LD, (size_t)n * es, (size_t)n * es, (size_t)n,
                             hipMemcpyDeviceToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    pp_fac_destroy(fac);
    if (e != hipSuccess) return fail(ctx, PP_EHIP, std::string("pp_dense_sgetrf: ") + hipGetErrorString(e));
    return PP_OK;
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
    hipStreamSynchronize(fac->ctx->aux_stream);
    delete fac;
    return PP_OK;
}

// ===== star and solves =====

// Device memory the star needs: the star buffer X, plus two column chunks of at most STAR_CHUNK_BYTES each when the
// output is in host memory
static size_t star_bytes(i64 n, size_t es, int out_on_device) {
    return (size_t)n * n * es + (out_on_device ? 0 : 2 * (size_t)pp::STAR_CHUNK_BYTES + 2 * (size_t)n * es);
}

static pp_status star_common(pp_ctx *ctx, const pp_fac *fac, void *out, int64_t ldc, int out_on_device, bool check);

pp_status pp_star(pp_ctx *ctx, const pp_fac *fac, void *out, int64_t ldc, int out_on_device) {
    if (!ctx || !fac || !out) return fail(ctx, PP_EINVAL, "pp_star: null argument");
    return star_common(ctx, fac, out, ldc, out_on_device, true);
}

// check: compare the star's memory with the free memory first (pp_mstar checks before it queues the factorization:
// the query would wait for the queued work)
static pp_status star_common(pp_ctx *ctx, const pp_fac *fac, void *out, int64_t ldc, int out_on_device, bool check) {
    const i64 n = fac->sym->S.n;
    if (ldc < n) return fail(ctx, PP_EINVAL, "pp_star: ldc < n");
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    const size_t es = (size_t)pp::dtype_size(fac->dtype);
    size_t freeb = 0, totalb = 0;
    const size_t need = star_bytes(n, es, out_on_device);
    if (check) CHECK_HIP(ctx, mem_free(ctx, &freeb, &totalb));
    if (check && need > freeb) {
        // work still queued (a factorization's fronts) may hold memory: wait for it and look again
        CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
        CHECK_HIP(ctx, hipStreamSynchronize(ctx->aux_stream));
        CHECK_HIP(ctx, mem_free(ctx, &freeb, &totalb));
    }
    if (check && need > freeb)
        return fail(ctx, PP_ENOMEM, "pp_star: needs " + std::to_string(need) + " bytes of device memory, " +
                                        std::to_string(freeb) + " free");
    std::string e = pp::device_star(ctx, fac, out, ldc, out_on_device ? 0 : 1);
    hipError_t se = hipStreamSynchronize(ctx->stream);
    if (!e.empty() || se != hipSuccess)
        return fail(ctx, PP_EHIP, "pp_star: " + (e.empty() ? std::string(hipGetErrorString(se)) : e));
    return PP_OK;
}

pp_status pp_mstar(pp_ctx *ctx, const pp_sym *sym, int semiring, int dtype, const void *nzval, int nz_on_device,
                   void *out, int64_t ldc, int out_on_device, pp_fac **fac_out) {
    if (fac_out) *fac_out = nullptr;
    if (!ctx) return fail(nullptr, PP_EINVAL, "pp_mstar: null context");
    if (!sym || !out) return fail(ctx, PP_EINVAL, "pp_mstar: null argument");
    if (ldc < sym->S.n) return fail(ctx, PP_EINVAL, "pp_mstar: ldc < n");
    if (!supported(semiring, dtype)) return fail(ctx, PP_EUNSUPPORTED, "pp_mstar: unsupported semiring / element type");
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    pp_fac *fac = nullptr;
    // the factorization is queued without waiting for it; the star's launches follow it on the same stream.  Its
    // memory check includes the star's, so a request that does not fit is refused before anything is queued.
    pp_status st = factor_common(ctx, sym, semiring, dtype, nzval, nz_on_device != 0, &fac, false,
                                 star_bytes(sym->S.n, (size_t)pp::dtype_size(dtype), out_on_device), "pp_mstar");
    if (st != PP_OK) return st;
    st = star_common(ctx, fac, out, ldc, out_on_device, false);
    if (st != PP_OK || !fac_out) {
        const std::string msg = ctx->err;
        pp_fac_destroy(fac);
        ctx->err = msg;
        return st;
    }
    *fac_out = fac;
    return PP_OK;
}

pp_status pp_star_sources(pp_ctx *ctx, const pp_fac *fac, int which, int64_t nsrc, const int64_t *src, void *out,
                          int64_t ldo, int out_on_device) {
    if (!ctx || !fac || (nsrc > 0 && (!src || !out))) return fail(ctx, PP_EINVAL, "pp_star_sources: null argument");
    if (which != 0 && which != 1) return fail(ctx, PP_EINVAL, "pp_star_sources: which must be 0 (rows) or 1 (columns)");
    const pp::Symbolic &S = fac->sym->S;
    const i64 n = S.n;
    if (nsrc < 0) return fail(ctx, PP_EINVAL, "pp_star_sources: nsrc < 0");
    if (which == 0 ? ldo < std::max<i64>(1, nsrc) : ldo < std::max<i64>(1, n))
        return fail(ctx, PP_EINVAL, "pp_star_sources: leading dimension too small");
    if (nsrc > (i64)1 << 30) return fail(ctx, PP_EINVAL, "pp_star_sources: too many sources");
    for (i64 k = 0; k < nsrc; k++)
        if (src[k] < 0 || src[k] >= n) return fail(ctx, PP_EINVAL, "pp_star_sources: source index out of range");
    if (nsrc == 0 || n == 0) return PP_OK;
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    const pp::SweepPlan &P = *fac->sym->splan;
    // the sweep rows: the distinct sources in elimination order
    pp::RowSub R;
    R.js.resize(nsrc);
    for (i64 k = 0; k < nsrc; k++) R.js[k] = (int32_t)S.invp[src[k]];
    std::sort(R.js.begin(), R.js.end());
    R.js.erase(std::unique(R.js.begin(), R.js.end()), R.js.end());
    std::vector<int32_t> pos(nsrc);
    for (i64 k = 0; k < nsrc; k++) pos[k] = R.map((int32_t)S.invp[src[k]]);
    pp::build_row_subset(P, S, R);
    const i64 m = (i64)R.js.size();
    const size_t es = (size_t)pp::dtype_size(fac->dtype);
    const size_t bytesO = (size_t)ldo * (size_t)(which == 0 ? n : nsrc) * es;
    // one device block for the row-subset arrays
    std::vector<int32_t> blk;
    std::vector<std::pair<int32_t **, size_t>> where;
    auto add = [&](const std::vector<int32_t> &v, int32_t **dst) {
        where.push_back({dst, blk.size()});
        blk.insert(blk.end(), v.begin(), v.end());
        blk.resize((blk.size() + 63) / 64 * 64);   // 256-byte aligned pieces
    };
    add(R.js, &R.d_js);
    add(R.rowA_lo, &R.d_rowA_lo);
    add(R.rowA_hi, &R.d_rowA_hi);
    add(R.rowB_lo, &R.d_rowB_lo);
    add(R.rowB_hi, &R.d_rowB_hi);
    add(R.tiles, &R.d_tiles);
    add(R.sub_rows, &R.d_sub_rows);
    add(R.sub_preF, &R.d_sub_preF);
    add(R.sub_preB, &R.d_sub_preB);
    add(pos, &R.d_pos);
    size_t freeb = 0, totalb = 0;
    CHECK_HIP(ctx, mem_free(ctx, &freeb, &totalb));
    const size_t need = (size_t)m * n * es + blk.size() * sizeof(int32_t) + (out_on_device ? 0 : bytesO);
    if (need > freeb)
        return fail(ctx, PP_ENOMEM, "pp_star_sources: needs " + std::to_string(need) + " bytes of device memory, " +
                                        std::to_string(freeb) + " free");
    void *dblk = nullptr;
    CHECK_HIP(ctx, dev_malloc(ctx, &dblk, blk.size() * sizeof(int32_t)));
    for (auto &w : where) *w.first = (int32_t *)dblk + w.second;
    void *dO = out;
    hipError_t ue = hipMemcpy(dblk, blk.data(), blk.size() * sizeof(int32_t), hipMemcpyHostToDevice);
    if (ue == hipSuccess && !out_on_device) ue = dev_malloc(ctx, &dO, bytesO);
    if (ue != hipSuccess) {
        hipFree(dblk);
        return fail(ctx, PP_EHIP, std::string("pp_star_sources: ") + hipGetErrorString(ue));
    }
    std::string e = pp::device_star_sources(ctx, fac, R, nsrc, which, dO, ldo);
    hipError_t se = hipStreamSynchronize(ctx->stream);
    if (e.empty() && se == hipSuccess && !out_on_device) se = hipMemcpy(out, dO, bytesO, hipMemcpyDeviceToHost);
    if (!out_on_device) hipFree(dO);
    hipFree(dblk);
    if (!e.empty() || se != hipSuccess)
        return fail(ctx, PP_EHIP, "pp_star_sources: " + (e.empty() ? std::string(hipGetErrorString(se)) : e));
    return PP_OK;
}

static pp_status solve(pp_ctx *ctx, const pp_fac *fac, void *B, int64_t ldb, int64_t nrhs, int on_device, bool left,
                       bool trans, const char *name) {
    if (!ctx || !fac || (!B && nrhs > 0)) return fail(ctx, PP_EINVAL, std::string(name) + ": null argument");
    const i64 n = fac->sym->S.n;
    if (nrhs < 0) return fail(ctx, PP_EINVAL, std::string(name) + ": nrhs < 0");
    if (left ? ldb < n : ldb < nrhs) return fail(ctx, PP_EINVAL, std::string(name) + ": leading dimension too small");
    if (nrhs == 0 || n == 0) return PP_OK;
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    const size_t es = (size_t)pp::dtype_size(fac->dtype);
    const size_t bytesB = (size_t)ldb * (size_t)(left ? nrhs : n) * es;
    size_t freeb = 0, totalb = 0;
    CHECK_HIP(ctx, mem_free(ctx, &freeb, &totalb));
    const size_t need = (size_t)n * nrhs * es + (on_device ? 0 : bytesB);
    if (need > freeb) return fail(ctx, PP_ENOMEM, std::string(name) + ": not enough device memory; nothing was launched");
    void *dB = B;
    if (!on_device) {
        CHECK_HIP(ctx, dev_malloc(ctx, &dB, bytesB));
        hipError_t ue = hipMemcpy(dB, B, bytesB, hipMemcpyHostToDevice);
        if (ue != hipSuccess) {
            hipFree(dB);
            return fail(ctx, PP_EHIP, std::string(name) + ": upload failed");
        }
    }
    std::string e = pp::device_solve(ctx, fac, dB, ldb, nrhs, left, trans, nullptr);
    hipError_t se = hipStreamSynchronize(ctx->stream);
    if (e.empty() && se == hipSuccess && !on_device) se = hipMemcpy(B, dB, bytesB, hipMemcpyDeviceToHost);
    if (!on_device) hipFree(dB);
    if (!e.empty() || se != hipSuccess)
        return fail(ctx, PP_EHIP, std::string(name) + ": " + (e.empty() ? std::string(hipGetErrorString(se)) : e));
    return PP_OK;
}

pp_status pp_lmul(pp_ctx *ctx, const pp_fac *fac, void *B, int64_t ldb, int64_t nrhs, int on_device) {
    return solve(ctx, fac, B, ldb, nrhs, on_device, true, false, "pp_lmul");
}

pp_status pp_rmul(pp_ctx *ctx, const pp_fac *fac, void *B, int64_t ldb, int64_t nrhs, int on_device) {
    return solve(ctx, fac, B, ldb, nrhs, on_device, false, false, "pp_rmul");
}

pp_status pp_sgetrs(pp_ctx *ctx, const pp_fac *fac, int side, int trans, void *B, int64_t ldb, int64_t nrhs,
                    int on_device) {
    if (side != PP_SIDE_LEFT && side != PP_SIDE_RIGHT) return fail(ctx, PP_EINVAL, "pp_sgetrs: side must be PP_SIDE_LEFT or PP_SIDE_RIGHT");
    if (trans != PP_NOTRANS && trans != PP_TRANS) return fail(ctx, PP_EINVAL, "pp_sgetrs: trans must be PP_NOTRANS or PP_TRANS");
    return solve(ctx, fac, B, ldb, nrhs, on_device, side == PP_SIDE_LEFT, trans == PP_TRANS, "pp_sgetrs");
}

pp_status pp_sgetrs_noalloc(pp_ctx *ctx, const pp_fac *fac, int side, int trans, void *B, int64_t ldb, int64_t nrhs) {
    if (!ctx || !fac || (!B && nrhs > 0)) return fail(ctx, PP_EINVAL, "pp_sgetrs_noalloc: null argument");
    if (fac->ctx != ctx) return fail(ctx, PP_EINVAL, "pp_sgetrs_noalloc: the factor belongs to another context");
    if (side != PP_SIDE_LEFT && side != PP_SIDE_RIGHT)
        return fail(ctx, PP_EINVAL, "pp_sgetrs_noalloc: side must be PP_SIDE_LEFT or PP_SIDE_RIGHT");
    if (trans != PP_NOTRANS && trans != PP_TRANS)
        return fail(ctx, PP_EINVAL, "pp_sgetrs_noalloc: trans must be PP_NOTRANS or PP_TRANS");
    const bool left = side == PP_SIDE_LEFT;
    const i64 n = fac->sym->S.n;
    if (nrhs < 0) return fail(ctx, PP_EINVAL, "pp_sgetrs_noalloc: nrhs < 0");
    if (left ? ldb < n : ldb < nrhs) return fail(ctx, PP_EINVAL, "pp_sgetrs_noalloc: leading dimension too small");
    if (nrhs == 0 || n == 0) return PP_OK;
    const size_t bytes = (size_t)n * (size_t)nrhs * (size_t)pp::dtype_size(fac->dtype);
    if (bytes > pp::NOALLOC_SCRATCH_BYTES)
        return fail(ctx, PP_EINVAL, "pp_sgetrs_noalloc: n * nrhs * element size = " + std::to_string(bytes) +
                                        " bytes is more than the fixed scratch of " +
                                        std::to_string(pp::NOALLOC_SCRATCH_BYTES) + " bytes (use pp_sgetrs)");
    void *scr = pp::noalloc_scratch(ctx->device);
    if (!scr) return fail(ctx, PP_EHIP, "pp_sgetrs_noalloc: the scratch of this device is not set up");
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    std::string e = pp::device_solve(ctx, fac, B, ldb, nrhs, left, trans == PP_TRANS, scr);
    if (!e.empty()) return fail(ctx, PP_EHIP, "pp_sgetrs_noalloc: " + e);
    return PP_OK;
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
    CHECK_HIP(ctx, mem_free(ctx, &freeb, &totalb));
    if (bytes > freeb) return fail(ctx, PP_ENOMEM, "pp_buffer_alloc: not enough device memory");
    if (dev_malloc(ctx, dptr, std::max<size_t>(1, bytes)) != hipSuccess) return fail(ctx, PP_ENOMEM, "pp_buffer_alloc: hipMalloc failed");
    return PP_OK;
}

pp_status pp_buffer_free(pp_ctx *ctx, void *dptr) {
    if (!ctx) return fail(nullptr, PP_EINVAL, "pp_buffer_free: null context");
    if (dptr) CHECK_HIP(ctx, hipFree(dptr));
    return PP_OK;
}

}  // extern "C"

// Large transfers between pageable host memory and the device go through two pinned chunks: a copy straight
// between pageable memory and the device runs at a few GB/s, the pinned path at the PCIe rate.  Download: a copy
// kernel writes chunk k into pinned buffer k % 2 (its device-side address) while the host's worker threads copy chunk
// k - 1 out; upload: the host threads fill one buffer while the copy engine moves the other.
static constexpr size_t XFER_CHUNK = 64u << 20, XFER_MIN = 1u << 20;

static std::string xfer_setup(pp_ctx *ctx) {
    for (int b = 0; b < 2; b++) {
        if (!ctx->xev[b] && hipEventCreateWithFlags(&ctx->xev[b], hipEventDisableTiming) != hipSuccess)
            return "hipEventCreate failed";
        if (ctx->xfer[b]) continue;
        if (hipHostMalloc(&ctx->xfer[b], XFER_CHUNK, hipHostMallocDefault) != hipSuccess) return "hipHostMalloc failed";
        if (hipHostGetDevicePointer(&ctx->xfer_dev[b], ctx->xfer[b], 0) != hipSuccess) return "hipHostGetDevicePointer failed";
    }
    return "";
}

static void host_copy(void *dst, const void *src, size_t bytes) {
    const int nt = (int)std::max<size_t>(1, std::min<size_t>(16, bytes >> 22));   // 4 MiB a thread
    pp::pool_run(nt, [&](int t) {
        const size_t a = bytes * t / nt, z = bytes * (t + 1) / nt;
        std::memcpy((char *)dst + a, (const char *)src + a, z - a);
    });
}

static std::string staged_download(pp_ctx *ctx, void *dst, const void *src, size_t bytes) {
    std::string e = xfer_setup(ctx);
    if (!e.empty()) return e;
    const size_t nchunk = (bytes + XFER_CHUNK - 1) / XFER_CHUNK;
    auto produce = [&](size_t k) -> std::string {
        const size_t off = k * XFER_CHUNK, len = std::min(XFER_CHUNK, bytes - off);
        std::string ce = pp::device_copy(ctx, ctx->xfer_dev[k & 1], (const char *)src + off, len);
        if (!ce.empty()) return ce;
        return hipEventRecord(ctx->xev[k & 1], ctx->stream) == hipSuccess ? "" : "hipEventRecord failed";
    };
    for (size_t k = 0; k < std::min<size_t>(2, nchunk) && e.empty(); k++) e = produce(k);
    for (size_t k = 0; k < nchunk && e.empty(); k++) {
        if (hipEventSynchronize(ctx->xev[k & 1]) != hipSuccess) return "hipEventSynchronize failed";
        const size_t off = k * XFER_CHUNK, len = std::min(XFER_CHUNK, bytes - off);
        host_copy((char *)dst + off, ctx->xfer[k & 1], len);
        if (k + 2 < nchunk) e = produce(k + 2);
    }
    return e;
}

static std::string staged_upload(pp_ctx *ctx, void *dst, const void *src, size_t bytes) {
    std::string e = xfer_setup(ctx);
    if (!e.empty()) return e;
    const size_t nchunk = (bytes + XFER_CHUNK - 1) / XFER_CHUNK;
    for (size_t k = 0; k < nchunk; k++) {
        const int b = (int)(k & 1);
        if (k >= 2 && hipEventSynchronize(ctx->xev[b]) != hipSuccess) return "hipEventSynchronize failed";
        const size_t off = k * XFER_CHUNK, len = std::min(XFER_CHUNK, bytes - off);
        host_copy(ctx->xfer[b], (const char *)src + off, len);
        if (hipMemcpyAsync((char *)dst + off, ctx->xfer[b], len, hipMemcpyHostToDevice, ctx->stream) != hipSuccess)
            return "hipMemcpyAsync failed";
        if (hipEventRecord(ctx->xev[b], ctx->stream) != hipSuccess) return "hipEventRecord failed";
    }
    return hipStreamSynchronize(ctx->stream) == hipSuccess ? "" : "hipStreamSynchronize failed";
}

extern "C" {

pp_status pp_upload(pp_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(ctx, PP_EINVAL, "pp_upload: null argument");
    if (!bytes) return PP_OK;
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    if (bytes < XFER_MIN) {
        CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
        CHECK_HIP(ctx, hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
        return PP_OK;
    }
    CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    std::string e = staged_upload(ctx, dst, src, bytes);
    if (!e.empty()) {
        hipStreamSynchronize(ctx->stream);
        return fail(ctx, PP_EHIP, "pp_upload: " + e);
    }
    return PP_OK;
}

pp_status pp_download(pp_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(ctx, PP_EINVAL, "pp_download: null argument");
    if (!bytes) return PP_OK;
    CHECK_HIP(ctx, hipSetDevice(ctx->device));
    CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (bytes < XFER_MIN) {
        CHECK_HIP(ctx, hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
        return PP_OK;
    }
    std::string e = staged_download(ctx, dst, src, bytes);
    hipError_t se = hipStreamSynchronize(ctx->stream);
    if (!e.empty() || se != hipSuccess) return fail(ctx, PP_EHIP, "pp_download: " + (e.empty() ? std::string(hipGetErrorString(se)) : e));
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

pp_status pp_set_debug(pp_ctx *ctx, int flags) {
    if (!ctx) return fail(nullptr, PP_EINVAL, "pp_set_debug: null context");
    if (flags & ~PP_DEBUG_POISON) return fail(ctx, PP_EINVAL, "pp_set_debug: unknown flag");
    ctx->debug = flags;
    return PP_OK;
}

pp_status pp_get_timing(const pp_ctx *ctx, double *t) {
    if (!ctx || !t) return fail(nullptr, PP_EINVAL, "pp_get_timing: null argument");
    pp_ctx *c = const_cast<pp_ctx *>(ctx);   // the times of recorded slots are read lazily
    for (int s = 0; s < 8; s++)
        if (c->pending[s]) {
            float ms = 0;
            if (hipEventSynchronize(c->ev[2 * s + 1]) == hipSuccess &&
                hipEventElapsedTime(&ms, c->ev[2 * s], c->ev[2 * s + 1]) == hipSuccess)
                c->t[s] = ms * 1e-3;
            c->pending[s] = false;
        }
    std::copy(c->t, c->t + 8, t);
    return PP_OK;
}

}  // extern "C"
