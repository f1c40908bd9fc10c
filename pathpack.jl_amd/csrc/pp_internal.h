// pp_internal.h -- device plans for the factorization and the sweeps (internal).
//
// Factorization plan.  Every frontal matrix F_f (nj x nj, nj = nn + na, column-major, local order res(f) then
// sep(f)) has a fixed place in one arena.  Fronts are grouped by height in the front tree (leaves 0); a height level
// runs: extend-add of the children's update blocks F_c[nn_c:, nn_c:] into the parents (one workgroup per parent
// column block, children one after another), then the partial LU of the fronts' first nn pivots.  Fronts with
// nj <= SMALL_NJ are factorized by one workgroup in LDS and their factor values copied into the reference's storage
// layout afterwards; larger fronts take blocked steps of NB pivots, one launch per step over the 64 x 64 tiles of all
// the level's trailing blocks (each tile factors the NB x NB diagonal block, solves its share of the row and column
// panels and updates itself), and the steps write the factor values into the reference layout directly.  The
// per-panel packs of the sweeps are built from the reference layout.
//
// Sweep plan.  Each front's residual is cut into panels of at most PANEL_W columns.  A panel p of front f covers
// the permuted columns [c0, c0 + w); its "extension" E_p is the rest of the residual after the panel followed by
// sep(f), i.e. the frontal-matrix local indices lo_ext .. nj-1 with lo_ext = c0 - Rptr[f] + w.  Packs:
//   Dpack[p]: the panel's w x w diagonal block of F (L strict lower, U upper with diagonal), at i + j*Wc
//   Upack[p]: U[c_j, E_t] at t*Wc + j         Lpack[p]: L[E_t, c_j] at t*Wc + j
// with Wc the panel's width class (the power of two >= w); the padding holds the semiring zero.
// A forward sweep visits panels leaves to root (each panel after its front's previous panel and after all
// panels of its children), a backward sweep root to leaves.
//
// Star blocks.  For the star, a front with more than PANEL_W columns is cut into blocks of at most BLK_W columns
// (and panels for a rest of at most PANEL_W columns), which run as register-tiled semiring GEMMs over whole row
// tiles.  A block b of width w, tile width bn (BLK_W, or BLK_W / 2 when w fits), with diagonal blocks L_bb (unit
// lower) and U_bb (upper) and extension E_b (as for a panel) carries two packs built at factor time:
//   Bpack[b]  (kp x bn, k-major, kp = w + e rounded up to BLK_K): rows 0..w-1 hold M_b = U_bb* (x) L_bb*, rows
//             w + t hold G_b[t, :] = L[E_t, blk] (x) L_bb*;
//   Hpack[b]  (wp x ep, k-major, wp = w rounded up to BLK_K, ep = e rounded up to BLK_W): H_b = U_bb* (x) U[blk, E].
//
// Star subtrees.  A maximal subtree of fronts with at most PANEL_W columns (one panel each) whose columns plus its
// root's separator number at most SUB_L runs in one launch per sweep: a wave takes a 64-row tile and steps through
// the subtree's panels in postorder (forward) or reverse postorder (backward), so what a panel reads was written just
// before by the same lane (no synchronization) and is still in the cache.
// Forward step:  X[R, E] <- X[R, E] (+) X[R, blk] (x) H_b over the rows R of the block's subtree (X[R, blk] as
// accumulated, unsolved).  Backward step: X[:, blk] <- X[:, blk] (x) M_b (+) X[:, E] (x) G_b over the component's
// rows, X[:, blk] taken as zero outside R.  In exact arithmetic this is the panel recurrence (U_bb* solves the
// forward step, L_bb* the backward one).  Block units have ids np .. np + nb - 1 in the per-panel arrays; the solves
// use the panels only.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "pp_symbolic.h"

namespace pp {

constexpr int SMALL_NJ = 64;   // fronts up to this size are factorized in one workgroup's LDS
constexpr int ASM_BLOCK = 16;  // parent columns per extend-add workgroup (at most; 4 at least)
constexpr int EXTRACT_COLS = 32;  // frontal columns per factor-extraction workgroup
constexpr int EIDX_PAD = 32;      // zero entries after the last gather list: sweeps read up to 16 entries ahead
constexpr int NB = 32;         // pivot block of the blocked front factorization
constexpr int PANEL_W = 32;    // widest sweep panel
constexpr int NCLASS = 8;      // sweep width classes 1, 2, 4, 8, 12, 16, 24, 32
constexpr int TILE_ROWS = 64;    // rows per scatter / backward workgroup (one per lane, 4 waves)
constexpr int SCATTER_T = 32;    // extension columns per scatter workgroup
constexpr int BLK_W = 128;       // widest star block (the GEMM tile's column count)
constexpr int BLK_K = 32;        // pack rows are padded to a multiple (of every k step of the block GEMMs)
constexpr int BLK_CLS = NCLASS;  // list class of star blocks with bn = BLK_W (BLK_CLS + 1: bn = BLK_W / 2)
constexpr int PREP_T = 64;       // output tile of the block-pack GEMMs
constexpr int SUB_L = 512;       // largest star subtree: columns plus the root's separator
constexpr long STAR_CHUNK_BYTES = 128L << 20;   // column chunk of a star written to host memory

// The width class of a panel of w columns: the narrowest of 1, 2, 4, 8, 12, 16, 24, 32 that holds it.  Its packs
// are padded to that width, and its sweep steps run in the kernels instantiated for it.  (Classes 12 and 24 cut the
// padded work of the common 9-12 and 17-24 column panels by a quarter against powers of two.)
__host__ __device__ constexpr int width_class(int w) {
    return w <= 1 ? 0 : w <= 2 ? 1 : w <= 4 ? 2 : w <= 8 ? 3 : w <= 12 ? 4 : w <= 16 ? 5 : w <= 24 ? 6 : 7;
}
__host__ __device__ constexpr int class_width(int c) {
    return c < 4 ? 1 << c : (c & 1) ? 16 << ((c - 5) >> 1) : 12 << ((c - 4) >> 1);
}
static_assert(class_width(4) == 12 && class_width(5) == 16 && class_width(6) == 24 && class_width(7) == 32 &&
                  class_width(NCLASS - 1) == PANEL_W,
              "width classes");

inline i64 round_up(i64 x, i64 m) { return (x + m - 1) / m * m; }
// The star's cut of a front wider than PANEL_W: blocks of BLK_W columns while more than 3/4 BLK_W remain, then one
// block of the rest if it is wider than PANEL_W (a BLK_W / 2 tile class when it fits), then panels.
inline i64 star_block_w(i64 rest) {
    return rest > BLK_W * 3 / 4 ? (rest < BLK_W ? rest : BLK_W) : rest > BLK_W / 2 ? BLK_W / 2 : rest;
}
inline i64 star_block_bn(i64 w) { return w > BLK_W / 2 ? BLK_W : BLK_W / 2; }

struct FactorPlan {
    i64 nf = 0;
    std::vector<int32_t> nn, na, nj;
    std::vector<i64> Foff;           // arena offset of each front
    i64 arena = 0;                   // elements
    std::vector<int32_t> relpos;     // Sptr-aligned: local index of sep(f)[k] in bag(parent(f))
    std::vector<i64> Sptr32;         // copy of Sptr (offsets into relpos)
    std::vector<int32_t> chptr, chidx;   // children (CSR)
    std::vector<i64> entry_pos;      // arena position of each stored entry of A
    // schedule
    struct Step {
        i64 off, cnt;                // (front, pivot offset, ti, tj) tile tasks in stask
    };
    struct Level {
        i64 asm_off, asm_cnt;        // extend-add tasks (front, first parent column) in atask
        int32_t asm_blk;             // parent columns per extend-add task (ASM_BLOCK, or fewer on a narrow level)
        i64 small_off, small_cnt;    // fronts with nj <= SMALL_NJ, in flist
        std::vector<Step> steps;     // blocked steps for the larger fronts
    };
    std::vector<Level> levels;
    std::vector<int32_t> flist;      // front lists of all levels
    std::vector<int32_t> atask;      // (front, first column) per extend-add task: 2 ints
    std::vector<int32_t> etask;      // (front, first column) per extraction task of a small front: 2 ints
    std::vector<int32_t> stask;      // (front, step offset, ti, tj) per step tile: 4 ints
    i64 max_nj = 0;
};

struct SweepPlan {
    i64 np = 0;                      // panels (ids 0 .. np-1)
    i64 nb = 0;                      // star blocks (ids np .. np+nb-1)
    // per panel, then per block
    std::vector<int32_t> front, c0, w, e, lo_ext, chunks;   // chunks: ceil(e / SCATTER_T), at least 1
    std::vector<i64> eoff, poff, doff;
    std::vector<int32_t> rowA_lo, rowA_hi, rowB_lo, rowB_hi;   // rows of the star sweeps
    std::vector<int32_t> Eidx;       // extension column indices (permuted labels)
    i64 npack = 0, ndpack = 0;
    // per block (index id - np)
    std::vector<i64> b_boff, b_hoff;     // Bpack / Hpack offsets
    std::vector<int32_t> b_kp, b_ep;     // Bpack rows, Hpack row stride
    std::vector<int32_t> b_bn;           // tile width (Bpack row stride)
    i64 nbpack = 0, nhpack = 0;
    std::vector<int32_t> prep;           // block-pack GEMM tiles: (block, part, tile row, tile column)
    std::vector<int32_t> sunits;         // the star's units: panels of fronts with at most PANEL_W columns, blocks
    // star subtrees: panels of subtree s at sub_pan[sub_ptr[s] .. sub_ptr[s + 1]) in postorder; rows (forward lo, hi,
    // backward lo, hi) and per-subtree prefixes of 64-row tiles (forward, backward); their panels are in no list
    std::vector<int32_t> sub_ptr, sub_pan, sub_rows, sub_preF, sub_preB;
    struct List {
        int cls;                     // width class (BLK_CLS, BLK_CLS + 1: star blocks)
        i64 off, cnt;                // panel ids in plist
        // offsets into `tiles` of per-panel prefix sums (cnt + 1 entries each): forward units (tiles x chunks)
        // over the star's forward rows, backward tiles over its backward rows, chunks
        i64 pAu, pB64, pC;
        i64 esum, emax;              // sum and maximum of the panels' gather-list lengths
        bool uniB;                   // every panel of the list has the same backward rows [rowB_lo, rowB_hi)
        int32_t rowB_lo, rowB_hi;
        i64 pT[2];                   // block lists: per-block prefix of GEMM tiles for 64 and 128 rows per tile
        i64 pCu, pC64;               // forward units (tiles x chunks) and backward tiles over the rows [rowC_lo, rowC_hi)
    };
    // the panels of every front (the solves, the transposed sweeps of source columns): one list per level holding
    // every width class (cls = -1), one launch each, in execution order
    std::vector<List> fwdm, bwdm;
    std::vector<List> sfwd, sbwd;    // the star's (panels of small fronts and blocks)
    // Strongly connected components coupled by N (several components and arcs between them): schedules over the
    // component DAG, one entry per level.  "up" (Y <- Y A*: rmul!, the rows and the off-diagonal blocks of the star):
    // the components by increasing lev_up; a level first gathers, into each of its columns j, the arcs i -> j from
    // earlier components (Y[:, j] (+)= Y[:, i] (x) N[i, j], N by column), then runs its panels (U forward, L backward).
    // "dn" (Y <- Y (A*)^T: lmul!, the columns of the star): by increasing lev_dn, gathering into row i the arcs i -> j
    // to later components (N by row), then the transposed sweeps.  The solves run every list on all their rows; the
    // star's second pass runs the "up" lists on each panel's rows [rowC_lo, rowC_hi) = [anc_lo, first row) of its
    // component, i.e. the rows of the earlier components (the diagonal blocks come from the first pass).
    bool coupled = false;
    struct CLevel {
        i64 cols_off, cols_cnt;      // the level's columns with arcs to gather (in ccols)
        i64 fwd_off, fwd_cnt;        // its forward panel lists (in cfwd)
        i64 bwd_off, bwd_cnt;        // its backward panel lists (in cbwd)
    };
    std::vector<CLevel> cup, cdn;
    std::vector<List> cfwd, cbwd;
    std::vector<int32_t> ccols;      // gather columns of all levels
    std::vector<int32_t> ccol_lo, ccol_hi;   // per gather column of an "up" level: the rows of the star's second pass
    std::vector<int32_t> rowC_lo, rowC_hi;   // per unit
    std::vector<int32_t> plist;
    std::vector<int32_t> tiles;      // the prefix sums of all lists
    i64 max_e = 0;
};

std::string build_factor_plan(const Symbolic &S, FactorPlan &P);
std::string build_sweep_plan(const Symbolic &S, SweepPlan &P);

// Element counts of the sweep plan's packs and index lists, from the front sizes alone (the cut of build_sweep_plan,
// without building the plan): for the device-memory checks made before anything is queued.
struct SweepSizes {
    i64 units = 0, nb = 0;           // panels plus star blocks; star blocks
    i64 eidx = 0;                    // gather-list entries (with the padding)
    i64 npack = 0, ndpack = 0, nbpack = 0, nhpack = 0;
    i64 prep = 0;                    // block-pack GEMM tiles
    i64 nN = 0;                      // arcs between strongly connected components
};
SweepSizes sweep_sizes(const Symbolic &S);

// The sweeps over the rows of a set of sources instead of all n (rows or columns of the star for chosen vertices).
// Row k of the sweep buffer starts as the unit vector of source js[k] (elimination labels, ascending).  A unit's
// forward rows are then the sources in its subtree, a contiguous range of js, and its backward rows the sources of
// its component: the plan's row ranges mapped through js, with the tile prefixes of every list recomputed in the
// plan's layout.
struct RowSub {
    std::vector<int32_t> js;                        // sorted sources (elimination labels)
    std::vector<int32_t> rowA_lo, rowA_hi, rowB_lo, rowB_hi;   // per unit
    std::vector<int32_t> tiles;                     // the plan's prefix arrays for these rows
    std::vector<int32_t> sub_rows, sub_preF, sub_preB;
    // device copies
    int32_t *d_js = nullptr, *d_rowA_lo = nullptr, *d_rowA_hi = nullptr, *d_rowB_lo = nullptr, *d_rowB_hi = nullptr;
    int32_t *d_tiles = nullptr, *d_sub_rows = nullptr, *d_sub_preF = nullptr, *d_sub_preB = nullptr;
    int32_t *d_pos = nullptr;                       // row of the sweep buffer of each requested source (input order)
    int32_t map(int32_t r) const;                   // plan row r (a source label) -> first sweep row with js >= r
};
void build_row_subset(const SweepPlan &P, const Symbolic &S, RowSub &R);

// Device copies of the plans.
struct DevPlan {
    // factor
    int32_t *nn = nullptr, *na = nullptr, *nj = nullptr, *relpos = nullptr, *chptr = nullptr, *chidx = nullptr;
    i64 *Foff = nullptr, *Sptr = nullptr, *entry_pos = nullptr;
    int32_t *flist = nullptr, *stask = nullptr, *atask = nullptr, *etask = nullptr;
    i64 *Dptr = nullptr, *Lptr = nullptr, *Rptr = nullptr;
    // sweeps
    int32_t *p_front = nullptr, *p_c0 = nullptr, *p_w = nullptr, *p_e = nullptr, *p_lo = nullptr, *p_chunks = nullptr;
    i64 *p_eoff = nullptr, *p_poff = nullptr, *p_doff = nullptr;
    int32_t *p_rowA_lo = nullptr, *p_rowA_hi = nullptr, *p_rowB_lo = nullptr, *p_rowB_hi = nullptr;
    int32_t *Eidx = nullptr, *plist = nullptr, *tiles = nullptr;
    i64 *b_boff = nullptr, *b_hoff = nullptr;
    int32_t *b_kp = nullptr, *b_ep = nullptr, *b_bn = nullptr, *prep = nullptr, *sunits = nullptr;
    int32_t *sub_ptr = nullptr, *sub_pan = nullptr, *sub_rows = nullptr, *sub_preF = nullptr, *sub_preB = nullptr;
    // components coupled by N: N by column and by row, the value sources, the gather columns, per-unit rows
    i64 *Nptr = nullptr, *NTptr = nullptr, *Nsrc = nullptr, *NTsrc = nullptr;
    int32_t *Nidx = nullptr, *NTidx = nullptr, *ccols = nullptr, *ccol_lo = nullptr, *ccol_hi = nullptr;
    int32_t *p_rowC_lo = nullptr, *p_rowC_hi = nullptr;
    // permutation
    i64 *perm = nullptr, *invp = nullptr;
    int32_t *invp32 = nullptr;
    std::vector<void *> owned;
};

}  // namespace pp

// Opaque handles of the C ABI.
struct pp_sym {
    pp::Symbolic S;
    pp::FactorPlan *fplan = nullptr;
    pp::SweepPlan *splan = nullptr;
    ~pp_sym();
};

struct pp_ctx {
    int device = 0;
    int num_cu = 256;                // compute units of the device
    hipStream_t stream = nullptr;
    // the context's own stream-ordered memory pool: fronts, the n x n star buffer, scratch.  It keeps freed memory
    // for the next call (re-mapping the 4 GB star buffer of a 32768-vertex graph costs about a millisecond) and is
    // trimmed and destroyed with the context; the device's default pool and other contexts are not touched.
    hipMemPool_t pool = nullptr;
    std::string err;
    int timing = 0;
    int debug = 0;                   // PP_DEBUG_* flags (pp_set_debug)
    double t[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    hipEvent_t ev[16] = {};          // start and stop event of each timing slot
    bool pending[8] = {};            // a slot's events are recorded and its time not yet read
    void *staging = nullptr;        // pinned host staging of the factor plan
    size_t staging_bytes = 0;
    void *staging2 = nullptr;       // pinned host staging of the sweep plan
    size_t staging2_bytes = 0;
    // star to host memory: the pipeline's events and two pinned chunk buffers (kept between calls)
    hipEvent_t pev[2] = {};
    // the star blocks' packs are built on a second stream, overlapped with the start of the star: aux_from orders
    // them after the factorization, aux_done orders every later reader (block GEMMs) and writer (the next
    // factorization of the same buffers) after them
    hipStream_t aux_stream = nullptr;
    hipEvent_t aux_from = nullptr, aux_done = nullptr;
    bool aux_pending = false;        // aux_done is recorded
    void *outpin[2] = {nullptr, nullptr};
    size_t outpin_bytes = 0;
    void *outpin_dev[2] = {nullptr, nullptr};   // their device-side addresses (the relabel kernel writes them)
    // pp_upload / pp_download of large buffers: two pinned staging chunks and their device-side addresses
    void *xfer[2] = {nullptr, nullptr}, *xfer_dev[2] = {nullptr, nullptr};
    hipEvent_t xev[2] = {};
};

struct pp_fac {
    pp_ctx *ctx = nullptr;
    const pp_sym *sym = nullptr;
    int semiring = 0, dtype = 0;
    pp::DevPlan plan;
    void *LD = nullptr, *LL = nullptr, *UL = nullptr;     // reference layout
    void *Dpack = nullptr, *Upack = nullptr, *Lpack = nullptr;
    void *Bpack = nullptr, *Hpack = nullptr;             // star blocks
    void *Nval = nullptr, *NTval = nullptr;              // N's values by column and by row (components coupled)
    // a dense factorization (pp_dense_factor) owns its one-front structure; while it factorizes, the values are the
    // n x n matrix dense_src (device memory, leading dimension dense_lda) instead of stored entries
    pp_sym *own_sym = nullptr;
    const void *dense_src = nullptr;
    int64_t dense_lda = 0;
    ~pp_fac();
};

namespace pp {
// A stream-ordered allocation from the context's pool (freed with hipFreeAsync).
inline hipError_t ctx_alloc(pp_ctx *ctx, void **p, size_t bytes, hipStream_t st) {
    return hipMallocFromPoolAsync(p, bytes, ctx->pool, st);
}

// Numeric drivers (pp_device.hip).  Return "" or an error message.
std::string device_factor(pp_ctx *ctx, pp_fac *fac, const void *d_nzval);   // up to the reference layout
std::string device_factor_packs(pp_ctx *ctx, pp_fac *fac);                 // the sweep packs; frees the fronts
// The star into out (ldc): device memory, or host memory (host != 0) through pinned chunks overlapped with the
// device-to-host copies.
std::string device_star(pp_ctx *ctx, const pp_fac *fac, void *out, i64 ldc, int host);
// Rows (cols = 0: out[k, j] = A*[src_k, j], nsrc x n, leading dimension ldo) or columns (cols = 1: out[i, k] =
// A*[i, src_k], n x nsrc) of the star for the sources of R (device copies uploaded), into device memory.
std::string device_star_sources(pp_ctx *ctx, const pp_fac *fac, const RowSub &R, i64 nsrc, int cols, void *out, i64 ldo);
// The solves on B in device memory: left (lmul!, B n x nrhs) or right (rmul!, B nrhs x n), with A or A^T; Y in
// `scratch` (device memory of at least n * nrhs elements) when it is not null, else in a pool allocation.
std::string device_solve(pp_ctx *ctx, const pp_fac *fac, void *d_B, i64 ldb, i64 nrhs, bool left, bool trans,
                         void *scratch);
// The fixed device array of the allocation-free solves: its size, the per-device set-up (hipGetSymbolAddress with
// the device current; once per device) and the device address it gave (null before the set-up).
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(64) << 20;
std::string noalloc_scratch_setup(int device);
void *noalloc_scratch(int device);
std::string device_sgemx(pp_ctx *ctx, int sr, int dt, i64 m, i64 n, i64 k, const void *A, i64 lda, const void *B,
                         i64 ldb, void *C, i64 ldc);
std::string device_getrf_star_batched(pp_ctx *ctx, int sr, int dt, i64 nb, i64 batch, void *A, void *TL, void *TU);
std::string device_valu_peak(pp_ctx *ctx, int kind, int iters, double *seconds, double *lane_instr);
std::string device_copy(pp_ctx *ctx, void *dst, const void *src, size_t bytes);
}  // namespace pp
