// star_plan_emu.cpp -- CPU replay of the star's device schedule (test infrastructure).
//
// Builds the real symbolic structure and sweep plan (pp_symbolic.cpp, pp_plan.cpp), factorizes with the oracle, then
// replays the star launch by launch with the device kernels' index arithmetic: the block-pack stars and GEMM tiles
// (k_blk_stars, k_blk_prep), the identity initialisation, the subtree launches (k_sub), the panel lists (k_fwd,
// k_sweep_bwd) and the block GEMM tiles (k_blk, with the tile heights the launcher picks for a given compute-unit
// count).  Every access is bounds-checked; within a launch, a task that reads an element another task of the same
// launch writes, two writers of one element, and a read of an element nothing has initialised are reported.  The
// relabelled result is compared with the oracle's star: bit for bit, or within 1e-4 relative error for PlusProd.
//
// With a source modulus M > 0 the replay runs the rows of the star for a subset of sources instead (the source-row
// path: the sweep buffer holds one row per source, and every unit's row ranges are those of the subset, as
// build_row_subset maps them): the sources are the labels s with (s * 2654435761) mod 2^32 mod M == 0 (M = 1: all).
//
// usage: star_plan_emu graph.bin semiring dtype ncu [M]   (graph.bin: n, nnz, colptr, rowval as int64, nzval)
// exit status 0 when no error is reported and the star (or its rows) matches.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "pp_internal.h"
#include "pp_semiring.h"

using namespace pp;

extern "C" {
int ppo_factor(int sr, int dt, i64 n, i64 nf, const i64 *Rptr, const i64 *Sptr, const i64 *Stgt, const i64 *perm,
               const i64 *colptr, const i64 *rowval, const void *nzval, void *LD, void *UD, void *LL, void *UL);
int ppo_star(int sr, int dt, i64 n, i64 nf, const i64 *Rptr, const i64 *Sptr, const i64 *Stgt, const i64 *perm,
             const void *LD, const void *UD, const void *LL, const void *UL, void *C, i64 row0, i64 row1, int relabel,
             int nthreads);
int ppo_star_scc(int sr, int dt, i64 n, i64 nf, const i64 *Rptr, const i64 *Sptr, const i64 *Stgt, const i64 *perm,
                 const void *LD, const void *UD, const void *LL, const void *UL, i64 nB, const i64 *Bptr, const i64 *Nptr,
                 const i64 *Nidx, const void *Nval, void *C, int nthreads);
}

static long nerr = 0;
#define FAIL(...)                          \
    do {                                   \
        if (nerr++ < 20) {                 \
            fprintf(stderr, __VA_ARGS__);  \
            fprintf(stderr, "\n");         \
        }                                  \
    } while (0)

template <class T> T poison() {
    if constexpr (std::is_floating_point<T>::value) return std::numeric_limits<T>::quiet_NaN();
    else return T(-1);
}

template <class T> struct Chk {
    const std::vector<T> *v;
    const char *name;
    T at(i64 i, i64 lo = 0, i64 hi = -1) const {
        if (hi < 0) hi = (i64)v->size();
        if (i < lo || i >= hi || i >= (i64)v->size()) {
            FAIL("OOB read %s[%lld] not in [%lld, %lld)", name, (long long)i, (long long)lo, (long long)hi);
            return T(0);
        }
        return (*v)[i];
    }
};

template <class S> struct Emu {
    typedef typename S::value_type T;
    i64 n;
    i64 m;                                     // rows of X (n, or the number of sources)
    Symbolic Sy;
    SweepPlan P;
    // the rows of each unit and the launches' prefix arrays: the plan's, or the source subset's
    std::vector<int32_t> rsrc;                 // row -> source label (empty: row i is label i)
    const int32_t *rAlo = nullptr, *rAhi = nullptr, *rBlo = nullptr, *rBhi = nullptr;
    const std::vector<int32_t> *TL = nullptr, *SR = nullptr, *SPF = nullptr, *SPB = nullptr;
    void use_plan_rows() {
        m = n;
        rAlo = P.rowA_lo.data(); rAhi = P.rowA_hi.data(); rBlo = P.rowB_lo.data(); rBhi = P.rowB_hi.data();
        TL = &P.tiles; SR = &P.sub_rows; SPF = &P.sub_preF; SPB = &P.sub_preB;
    }
    void use_subset(const RowSub &R) {
        m = (i64)R.js.size();
        rsrc = R.js;
        rAlo = R.rowA_lo.data(); rAhi = R.rowA_hi.data(); rBlo = R.rowB_lo.data(); rBhi = R.rowB_hi.data();
        TL = &R.tiles; SR = &R.sub_rows; SPF = &R.sub_preF; SPB = &R.sub_preB;
    }
    std::vector<T> LD, LL, UL;                 // device layout
    std::vector<T> Bpack, Hpack, stars;
    std::vector<T> X, X0;                      // X0: snapshot before a launch
    std::vector<int32_t> wtask;                // writer task of the current launch, -1 (ATOMIC_W: atomic updates)
    std::vector<char> init;                    // element initialised
    int phase = 0;                             // 1: collect writes, 2: compute + check reads
    bool live = false;                         // reads see this launch's own writes (subtree launches)
    int cur = 0;
    int ncu;

    T D(int f, int i, int j) {   // diagonal-block entry of front f, local (i, j)
        i64 a = Sy.Rptr[f + 1] - Sy.Rptr[f];
        return Chk<T>{&LD, "LD"}.at(Sy.Dptr[f] + i + (i64)j * a, Sy.Dptr[f], Sy.Dptr[f + 1]);
    }
    T Lext(int f, int cb, int lo, int t, int i) {
        i64 a = Sy.Rptr[f + 1] - Sy.Rptr[f], c = Sy.Sptr[f + 1] - Sy.Sptr[f];
        int col = lo + t;
        if (col < a) return D(f, col, cb + i);
        return Chk<T>{&LL, "LL"}.at(Sy.Lptr[f] + (col - a) + (i64)(cb + i) * c, Sy.Lptr[f], Sy.Lptr[f + 1]);
    }
    T Uext(int f, int cb, int lo, int i, int t) {
        i64 a = Sy.Rptr[f + 1] - Sy.Rptr[f];
        int col = lo + t;
        if (col < a) return D(f, cb + i, col);
        return Chk<T>{&UL, "UL"}.at(Sy.Lptr[f] + (cb + i) + (i64)(col - a) * a, Sy.Lptr[f], Sy.Lptr[f + 1]);
    }

    // X access with launch semantics
    static constexpr int32_t ATOMIC_W = -2;
    T rd(i64 r, i64 c, bool used) {
        if (r < 0 || r >= m || c < 0 || c >= n) {
            FAIL("OOB X read (%lld, %lld)", (long long)r, (long long)c);
            return S::zero();
        }
        i64 idx = r + c * m;
        if (phase == 2 && used) {
            if (wtask[idx] == ATOMIC_W) FAIL("race: task %d reads (%lld,%lld), which the launch updates atomically", cur, (long long)r, (long long)c);
            if (wtask[idx] >= 0 && wtask[idx] != cur) FAIL("race: task %d reads (%lld,%lld) written by task %d", cur, (long long)r, (long long)c, wtask[idx]);
            if (!init[idx]) FAIL("read of uninitialised X(%lld, %lld) by task %d", (long long)r, (long long)c, cur);
        }
        return live ? X[idx] : X0[idx];
    }
    // an atomic X[r, c] (+)= v of the forward scatter: any number of tasks may do it; no task of the launch may read
    // the element or write it plainly
    void wr_atomic(i64 r, i64 c, T v) {
        if (r < 0 || r >= m || c < 0 || c >= n) {
            FAIL("OOB X atomic (%lld, %lld)", (long long)r, (long long)c);
            return;
        }
        const i64 idx = r + c * m;
        if (phase == 1) {
            if (wtask[idx] >= 0) FAIL("race: atomic and plain writers of (%lld,%lld)", (long long)r, (long long)c);
            wtask[idx] = ATOMIC_W;
        } else {
            if (!init[idx]) FAIL("atomic update of uninitialised X(%lld, %lld)", (long long)r, (long long)c);
            X[idx] = S::plus(X[idx], v);
        }
    }
    void wr(i64 r, i64 c, T v) {
        if (r < 0 || r >= m || c < 0 || c >= n) {
            FAIL("OOB X write (%lld, %lld)", (long long)r, (long long)c);
            return;
        }
        i64 idx = r + c * m;
        if (phase == 1) {
            if (wtask[idx] == ATOMIC_W) FAIL("race: plain and atomic writers of (%lld,%lld)", (long long)r, (long long)c);
            if (wtask[idx] >= 0 && wtask[idx] != cur) FAIL("race: two writers of (%lld,%lld): %d, %d", (long long)r, (long long)c, wtask[idx], cur);
            wtask[idx] = cur;
        } else {
            X[idx] = v;
            init[idx] = 1;
        }
    }

    // ---- block packs (k_blk_stars, k_blk_prep) ----
    void packs() {
        const int BW = BLK_W;
        stars.assign((size_t)P.nb * 2 * BW * BW, S::zero());
        Bpack.assign(P.nbpack, S::zero());
        Hpack.assign(P.nhpack, S::zero());
        for (i64 b = 0; b < P.nb; b++) {
            i64 id = P.np + b;
            int f = P.front[id], w = P.w[id], cb = P.c0[id] - (int)Sy.Rptr[f];
            T *Ls = &stars[b * 2 * BW * BW], *Us = Ls + BW * BW;
            std::vector<T> x((size_t)BW * BW);
            for (int c = 0; c < BW; c++)
                for (int i = 0; i < w; i++) {
                    T acc = i == c ? S::one() : S::zero();
                    for (int k = 0; k < i; k++) acc = S::muladd(D(f, cb + i, cb + k), x[k * BW + c], acc);
                    x[i * BW + c] = acc;
                }
            for (int i = 0; i < w; i++)
                for (int j = 0; j < w; j++) Ls[i + j * BW] = x[i * BW + j];
            for (int c = 0; c < BW; c++)
                for (int j = 0; j < w; j++) {
                    T part = S::zero();
                    for (int k = 0; k < j; k++) part = S::muladd(x[k * BW + c], D(f, cb + k, cb + j), part);
                    T acc = S::plus(j == c ? S::one() : S::zero(), part);
                    if (!S::integral) acc = S::prod(acc, S::star(D(f, cb + j, cb + j)));
                    x[j * BW + c] = acc;
                }
            for (int i = 0; i < w; i++)
                for (int j = 0; j < w; j++) Us[i + j * BW] = x[j * BW + i];
        }
        for (size_t q = 0; q < P.prep.size() / 4; q++) {
            int b = P.prep[4 * q], part = P.prep[4 * q + 1], r0 = P.prep[4 * q + 2] * PREP_T, q0 = P.prep[4 * q + 3] * PREP_T;
            i64 id = P.np + b;
            int f = P.front[id], w = P.w[id], e = P.e[id], cb = P.c0[id] - (int)Sy.Rptr[f], lo = P.lo_ext[id];
            T *Ls = &stars[b * 2 * BW * BW], *Us = Ls + BW * BW;
            int rows = part == 1 ? e : w, cols = part == 2 ? e : w;
            for (int r = r0; r < std::min(rows, r0 + PREP_T); r++)
                for (int cc = q0; cc < std::min(cols, q0 + PREP_T); cc++) {
                    T acc = S::zero();
                    for (int i = 0; i < w; i++) {
                        T av = part == 1 ? Lext(f, cb, lo, r, i) : Us[r + i * BW];
                        T bv = part == 2 ? Uext(f, cb, lo, i, cc) : Ls[i + cc * BW];
                        acc = S::muladd(av, bv, acc);
                    }
                    i64 pos;
                    std::vector<T> *dst;
                    i64 lo_, hi_;
                    const int bn = P.b_bn[b];
                    if (part == 0) { pos = P.b_boff[b] + (i64)r * bn + cc; dst = &Bpack; lo_ = P.b_boff[b]; hi_ = lo_ + (i64)P.b_kp[b] * bn; }
                    else if (part == 1) { pos = P.b_boff[b] + (i64)(w + r) * bn + cc; dst = &Bpack; lo_ = P.b_boff[b]; hi_ = lo_ + (i64)P.b_kp[b] * bn; }
                    else { pos = P.b_hoff[b] + (i64)r * P.b_ep[b] + cc; dst = &Hpack; lo_ = P.b_hoff[b]; hi_ = lo_ + (i64)((w + BLK_K - 1) / BLK_K * BLK_K) * P.b_ep[b]; }
                    if (pos < lo_ || pos >= hi_) FAIL("prep write out of the block's pack: part %d b %d", part, b);
                    else (*dst)[pos] = acc;
                }
        }
    }

    // ---- sweeps ----
    void identity() {
        for (int32_t p : P.sunits) {
            for (int j = 0; j < P.w[p]; j++) {
                i64 col = P.c0[p] + j;
                for (i64 i = rAlo[p]; i < rAhi[p]; i++) {
                    const i64 src = rsrc.empty() ? i : rsrc[i];
                    X[i + col * m] = src == col ? S::one() : S::zero();
                    init[i + col * m] = 1;
                }
                for (i64 i = 0; i < rBlo[p]; i++) { X[i + col * m] = S::zero(); init[i + col * m] = 1; }
                for (i64 i = rBhi[p]; i < m; i++) { X[i + col * m] = S::zero(); init[i + col * m] = 1; }
            }
        }
    }

    int search(const int32_t *pre, int np, int u) {
        int lo = 0, hi = np;
        while (hi - lo > 1) {
            int mid = (lo + hi) >> 1;
            if (pre[mid] <= u) lo = mid;
            else hi = mid;
        }
        return lo;
    }

    // panel forward, star rows (k_fwd semantics)
    void panel_fwd(int p, int task0) {
        int f = P.front[p], w = P.w[p], e = P.e[p], c0 = P.c0[p], lj0 = c0 - (int)Sy.Rptr[f], lo = P.lo_ext[p];
        i64 eo = P.eoff[p];
        for (i64 r = rAlo[p]; r < rAhi[p]; r++) {
            cur = task0 + (int)((r - rAlo[p]) / 64);
            std::vector<T> x(w);
            for (int j = 0; j < w; j++) x[j] = rd(r, c0 + j, true);
            for (int j = 0; j < w; j++) {
                T acc = x[j];
                for (int i = 0; i < j; i++) acc = S::muladd(x[i], D(f, lj0 + i, lj0 + j), acc);
                if (!S::integral) acc = S::prod(acc, S::star(D(f, lj0 + j, lj0 + j)));
                x[j] = acc;
            }
            for (int t = 0; t < e; t++) {
                int col = P.Eidx[eo + t];
                T acc = rd(r, col, true);
                for (int j = 0; j < w; j++) acc = S::muladd(x[j], Uext(f, lj0, lo, j, t), acc);
                wr(r, col, acc);
            }
        }
    }
    void panel_bwd(int p, int task0) {
        int f = P.front[p], w = P.w[p], e = P.e[p], c0 = P.c0[p], lj0 = c0 - (int)Sy.Rptr[f], lo = P.lo_ext[p];
        i64 eo = P.eoff[p];
        for (i64 r = rBlo[p]; r < rBhi[p]; r++) {
            cur = task0 + (int)((r - rBlo[p]) / 64);
            std::vector<T> acc(w, S::zero());
            if (r >= rAlo[p] && r < rAhi[p]) {
                for (int j = 0; j < w; j++) acc[j] = rd(r, c0 + j, true);
                for (int j = 0; j < w; j++) {
                    T s = acc[j];
                    for (int i = 0; i < j; i++) s = S::muladd(acc[i], D(f, lj0 + i, lj0 + j), s);
                    if (!S::integral) s = S::prod(s, S::star(D(f, lj0 + j, lj0 + j)));
                    acc[j] = s;
                }
            }
            for (int t = 0; t < e; t++) {
                T v = rd(r, P.Eidx[eo + t], true);
                for (int j = 0; j < w; j++) acc[j] = S::muladd(v, Lext(f, lj0, lo, t, j), acc[j]);
            }
            for (int j = w - 1; j >= 0; j--) {
                T s = acc[j];
                for (int i = j + 1; i < w; i++) s = S::muladd(acc[i], D(f, lj0 + i, lj0 + j), s);
                acc[j] = s;
            }
            for (int j = 0; j < w; j++) wr(r, c0 + j, acc[j]);
        }
    }

    // block launch (k_blk semantics)
    void blocks(const SweepPlan::List &li, bool fwd) {
        const int q = sizeof(T) == 4 && (*TL)[li.pT[1] + li.cnt] >= 2 * ncu ? 1 : 0;
        const int TM = q ? 8 : 4, TN = fwd || li.cls == BLK_CLS ? 8 : 4;
        const int BM = 16 * TM, BN = 16 * TN, BK = 16;
        const int32_t *pre = &(*TL)[li.pT[q]];
        const int32_t *ulist = &P.plist[li.off];
        int nu = (int)li.cnt, ntask = pre[nu];
        int grid = (ntask + 7) / 8 * 8, per = grid / 8;
        std::vector<char> seen(ntask, 0);
        for (int bid = 0; bid < grid; bid++) {
            int task = (bid & 7) * per + (bid >> 3);
            if (task >= ntask) continue;
            if (seen[task]++) FAIL("task %d twice", task);
            cur = task;
            int ui = search(pre, nu, task), u = task - pre[ui];
            int id = ulist[ui], b = id - (int)P.np;
            if (b < 0 || b >= P.nb) { FAIL("block list holds a panel"); continue; }
            if (!fwd && P.b_bn[b] != BN) FAIL("block of tile width %d in a list of %d", P.b_bn[b], BN);
            int c0 = P.c0[id], w = P.w[id], e = P.e[id];
            i64 eo = P.eoff[id];
            int lo = fwd ? rAlo[id] : rBlo[id], hi = fwd ? rAhi[id] : rBhi[id];
            int rt = u, ct = 0;
            if (fwd) { int nct = (e + BN - 1) / BN; if (nct == 0) { FAIL("fwd task with e = 0"); continue; } rt = u / nct; ct = u - rt * nct; }
            i64 r0 = (i64)(lo / BM) * BM + (i64)rt * BM;
            if (r0 >= hi) FAIL("tile beyond its rows");
            int K = fwd ? w : w + e;
            int olo = fwd ? 0 : rAlo[id], ohi = fwd ? 0 : rAhi[id];
            i64 boff = fwd ? P.b_hoff[b] + (i64)ct * BN : P.b_boff[b];
            i64 ldb = fwd ? P.b_ep[b] : BN;
            i64 plo = fwd ? P.b_hoff[b] : P.b_boff[b];
            i64 phi = fwd ? plo + (i64)((w + BLK_K - 1) / BLK_K * BLK_K) * P.b_ep[b] : plo + (i64)P.b_kp[b] * P.b_bn[b];
            const std::vector<T> &Pk = fwd ? Hpack : Bpack;
            bool own = fwd || (r0 < ohi && r0 + BM > olo);
            int kbeg = own ? 0 : (w / BK) * BK, kend = (K + BK - 1) / BK * BK;
            bool vec = r0 + BM <= m && m % (16 / (int)sizeof(T)) == 0;
            auto colA = [&](int k) -> i64 {
                if (fwd) return c0 + std::min(k, w - 1);
                if (k < w) return c0 + k;
                if (k < K) {
                    if (k - w >= e) FAIL("E index beyond the list");
                    return P.Eidx[eo + (k - w)];
                }
                return c0;
            };
            if (kbeg >= kend) {
                // no loads
            }
            for (int rr = 0; rr < BM; rr++) {
                i64 r = r0 + rr;
                bool stored = r >= lo && r < hi;
                if (!vec && r >= m) continue;   // not loaded (zero)
                for (int c = 0; c < BN; c++) {
                    T acc = S::zero();
                    if (fwd) {
                        int t = ct * BN + c;
                        if (stored && t < e) acc = rd(r, P.Eidx[eo + t], true);
                    }
                    if (kbeg < kend) {
                        for (int k = kbeg; k < kend; k += 2) {
                            T av[2], bv[2];
                            for (int h = 0; h < 2; h++) {
                                int kk = k + h;
                                i64 col = colA(kk);
                                // the kernel's LDS store selects the semiring zero for the backward's own columns
                                // outside [olo, ohi) and for the padded steps k >= K; every other value read enters
                                // the accumulator (also on rows that are not stored, which only this lane computes)
                                bool masked = !fwd && ((kk < w && (r < olo || r >= ohi)) || kk >= K);
                                T v = rd(r, col, stored && !masked);
                                if (masked) v = S::zero();
                                av[h] = v;
                                i64 pos = boff + (i64)kk * ldb + c;
                                if (pos < plo || pos >= phi) { FAIL("B read outside the block's pack (fwd %d b %d k %d c %d)", fwd, b, kk, c); bv[h] = S::zero(); }
                                else bv[h] = Pk[pos];
                            }
                            acc = S::muladd2(av[0], bv[0], av[1], bv[1], acc);
                        }
                    }
                    if (!stored) continue;
                    if (fwd) {
                        int t = ct * BN + c;
                        if (t < e) wr(r, P.Eidx[eo + t], acc);
                    } else if (c < w) wr(r, c0 + c, acc);
                }
            }
        }
    }

    // k_sub: one task per (subtree, 64-row tile)
    void subtrees(bool fwd) {
        const i64 nsub = (i64)P.sub_ptr.size() - 1;
        if (nsub <= 0) return;
        const std::vector<int32_t> &pre = fwd ? *SPF : *SPB;
        X0 = X;
        std::fill(wtask.begin(), wtask.end(), -1);
        live = true;
        for (phase = 1; phase <= 2; phase++) {
            for (int task = 0; task < pre[nsub]; task++) {
                cur = task;
                const int s = search(pre.data(), (int)nsub, task);
                const int tile = task - pre[s];
                const int lo = (*SR)[4 * s + (fwd ? 0 : 2)], hi = (*SR)[4 * s + (fwd ? 1 : 3)];
                const int k0 = P.sub_ptr[s], k1 = P.sub_ptr[s + 1];
                for (int lane = 0; lane < 64; lane++) {
                    const i64 r = (i64)lo + (i64)tile * 64 + lane;
                    for (int kk = 0; kk < k1 - k0; kk++) {
                        const int p = P.sub_pan[fwd ? k0 + kk : k1 - 1 - kk];
                        const int plo = fwd ? rAlo[p] : lo, phi = fwd ? rAhi[p] : hi;
                        const i64 t0 = (i64)lo + (i64)tile * 64;
                        if (plo >= phi || t0 >= phi || t0 + 64 <= plo) continue;
                        const bool store = r >= plo && r < phi;
                        const i64 rr = r < plo ? plo : (r >= phi ? phi - 1 : r);
                        int f = P.front[p], w = P.w[p], e = P.e[p], c0 = P.c0[p], lj0 = c0 - (int)Sy.Rptr[f], lo_ = P.lo_ext[p];
                        i64 eo = P.eoff[p];
                        if (fwd) {
                            std::vector<T> x(w);
                            for (int j = 0; j < w; j++) x[j] = rd(rr, c0 + j, store);
                            for (int j = 0; j < w; j++) {
                                T acc = x[j];
                                for (int i = 0; i < j; i++) acc = S::muladd(x[i], D(f, lj0 + i, lj0 + j), acc);
                                if (!S::integral) acc = S::prod(acc, S::star(D(f, lj0 + j, lj0 + j)));
                                x[j] = acc;
                            }
                            for (int t = 0; t < e; t++) {
                                int col = P.Eidx[eo + t];
                                T acc = rd(rr, col, store);
                                for (int j = 0; j < w; j++) acc = S::muladd(x[j], Uext(f, lj0, lo_, j, t), acc);
                                if (store) wr(rr, col, acc);
                            }
                        } else {
                            std::vector<T> acc(w, S::zero());
                            if (rr >= rAlo[p] && rr < rAhi[p]) {
                                for (int j = 0; j < w; j++) acc[j] = rd(rr, c0 + j, store);
                                for (int j = 0; j < w; j++) {
                                    T sv = acc[j];
                                    for (int i = 0; i < j; i++) sv = S::muladd(acc[i], D(f, lj0 + i, lj0 + j), sv);
                                    if (!S::integral) sv = S::prod(sv, S::star(D(f, lj0 + j, lj0 + j)));
                                    acc[j] = sv;
                                }
                            }
                            for (int t = 0; t < e; t++) {
                                T v = rd(rr, P.Eidx[eo + t], store);
                                for (int j = 0; j < w; j++) acc[j] = S::muladd(v, Lext(f, lj0, lo_, t, j), acc[j]);
                            }
                            for (int j = w - 1; j >= 0; j--) {
                                T sv = acc[j];
                                for (int i = j + 1; i < w; i++) sv = S::muladd(acc[i], D(f, lj0 + i, lj0 + j), sv);
                                acc[j] = sv;
                            }
                            if (store)
                                for (int j = 0; j < w; j++) wr(rr, c0 + j, acc[j]);
                        }
                    }
                }
            }
        }
        phase = 0;
        live = false;
    }

    // ---- the second pass over coupled components (run_coupled with up, offd) ----
    std::vector<i64> Nptr, Nidx;             // N by column (permuted labels)
    std::vector<T> Nval;
    // k_spmm_pull: gather columns t of a level, rows [ccol_lo, ccol_hi), one task per (column, 256-row tile)
    void spmm(const SweepPlan::CLevel &cl) {
        X0 = X;
        std::fill(wtask.begin(), wtask.end(), -1);
        for (phase = 1; phase <= 2; phase++) {
            for (i64 b = 0; b < cl.cols_cnt; b++) {
                const i64 t = P.ccols[cl.cols_off + b];
                const i64 lo = P.ccol_lo[cl.cols_off + b], hi = P.ccol_hi[cl.cols_off + b];
                if (hi != Sy.Bptr[Sy.comp[t]] || lo != Sy.anc_lo[Sy.comp[t]]) FAIL("gather column %lld: wrong rows", (long long)t);
                for (i64 r = lo; r < hi; r++) {
                    cur = (int)(b * 100000 + (r - lo) / 256);
                    T acc = rd(r, t, true);
                    for (i64 q = Nptr[t]; q < Nptr[t + 1]; q++) acc = S::muladd(rd(r, Nidx[q], true), Nval[q], acc);
                    wr(r, t, acc);
                }
            }
        }
        phase = 0;
    }
    // k_fwd with ATOMIC and per-panel rows [rowC_lo, rowC_hi): solve the panel's columns (not stored), then
    // X[r, E_t] (+)= sum_j x_j (x) U(j, t) atomically
    void panel_fwd_offd(int p, int task0) {
        int f = P.front[p], w = P.w[p], e = P.e[p], c0 = P.c0[p], lj0 = c0 - (int)Sy.Rptr[f], lo = P.lo_ext[p];
        i64 eo = P.eoff[p];
        for (i64 r = P.rowC_lo[p]; r < P.rowC_hi[p]; r++) {
            cur = task0 + (int)((r - P.rowC_lo[p]) / 64);
            std::vector<T> x(w);
            for (int j = 0; j < w; j++) x[j] = rd(r, c0 + j, true);
            for (int j = 0; j < w; j++) {
                T acc = x[j];
                for (int i = 0; i < j; i++) acc = S::muladd(x[i], D(f, lj0 + i, lj0 + j), acc);
                if (!S::integral) acc = S::prod(acc, S::star(D(f, lj0 + j, lj0 + j)));
                x[j] = acc;
            }
            for (int t = 0; t < e; t++) {
                T v = S::zero();
                for (int j = 0; j < w; j++) v = S::muladd(x[j], Uext(f, lj0, lo, j, t), v);
                wr_atomic(r, P.Eidx[eo + t], v);
            }
        }
    }
    // k_sweep_bwd on the rows [rowC_lo, rowC_hi), every row holding the panel's forward values
    void panel_bwd_offd(int p, int task0) {
        int f = P.front[p], w = P.w[p], e = P.e[p], c0 = P.c0[p], lj0 = c0 - (int)Sy.Rptr[f], lo = P.lo_ext[p];
        i64 eo = P.eoff[p];
        for (i64 r = P.rowC_lo[p]; r < P.rowC_hi[p]; r++) {
            cur = task0 + (int)((r - P.rowC_lo[p]) / 64);
            std::vector<T> acc(w);
            for (int j = 0; j < w; j++) acc[j] = rd(r, c0 + j, true);
            for (int j = 0; j < w; j++) {
                T sv = acc[j];
                for (int i = 0; i < j; i++) sv = S::muladd(acc[i], D(f, lj0 + i, lj0 + j), sv);
                if (!S::integral) sv = S::prod(sv, S::star(D(f, lj0 + j, lj0 + j)));
                acc[j] = sv;
            }
            for (int t = 0; t < e; t++) {
                T v = rd(r, P.Eidx[eo + t], true);
                for (int j = 0; j < w; j++) acc[j] = S::muladd(v, Lext(f, lj0, lo, t, j), acc[j]);
            }
            for (int j = w - 1; j >= 0; j--) {
                T sv = acc[j];
                for (int i = j + 1; i < w; i++) sv = S::muladd(acc[i], D(f, lj0 + i, lj0 + j), sv);
                acc[j] = sv;
            }
            for (int j = 0; j < w; j++) wr(r, c0 + j, acc[j]);
        }
    }
    void run_list_offd(const SweepPlan::List &li, bool fwd) {
        X0 = X;
        std::fill(wtask.begin(), wtask.end(), -1);
        if (li.cls >= BLK_CLS) FAIL("a block in a list of the second pass");
        for (phase = 1; phase <= 2; phase++) {
            int task0 = 0;
            for (i64 k = 0; k < li.cnt; k++) {
                int p = P.plist[li.off + k];
                if (fwd) panel_fwd_offd(p, task0);
                else panel_bwd_offd(p, task0);
                task0 += 100000;
            }
        }
        phase = 0;
    }
    void second_pass() {
        for (const auto &cl : P.cup) {
            if (cl.cols_cnt) spmm(cl);
            for (i64 k = 0; k < cl.fwd_cnt; k++) run_list_offd(P.cfwd[cl.fwd_off + k], true);
            for (i64 k = 0; k < cl.bwd_cnt; k++) run_list_offd(P.cbwd[cl.bwd_off + k], false);
        }
    }

    void run_list(const SweepPlan::List &li, bool fwd) {
        // phase 1 writes, phase 2 values
        X0 = X;
        std::fill(wtask.begin(), wtask.end(), -1);
        for (phase = 1; phase <= 2; phase++) {
            if (li.cls >= BLK_CLS) blocks(li, fwd);
            else {
                int task0 = 0;
                for (i64 k = 0; k < li.cnt; k++) {
                    int p = P.plist[li.off + k];
                    if (p >= P.np) FAIL("panel list holds a block");
                    if (fwd) panel_fwd(p, task0);
                    else panel_bwd(p, task0);
                    task0 += 100000;
                }
            }
        }
        phase = 0;
    }
};

template <class S> int run(const char *path, int sr, int dt, int ncu, long mod) {
    typedef typename S::value_type T;
    FILE *fp = fopen(path, "rb");
    if (!fp) return 2;
    i64 n, nnz;
    if (fread(&n, 8, 1, fp) != 1 || fread(&nnz, 8, 1, fp) != 1) return 2;
    std::vector<i64> colptr(n + 1), rowval(nnz);
    std::vector<T> nzval(nnz);
    if (fread(colptr.data(), 8, n + 1, fp) != (size_t)(n + 1)) return 2;
    if (fread(rowval.data(), 8, nnz, fp) != (size_t)nnz) return 2;
    if (fread(nzval.data(), sizeof(T), nnz, fp) != (size_t)nnz) return 2;
    fclose(fp);
    Emu<S> E;
    E.n = n;
    E.ncu = ncu;
    SymOptions opts;
    std::string err = analyze(n, colptr.data(), rowval.data(), opts, nullptr, E.Sy);
    if (!err.empty()) { fprintf(stderr, "analyze: %s\n", err.c_str()); return 3; }
    err = build_sweep_plan(E.Sy, E.P);
    if (!err.empty()) { fprintf(stderr, "plan: %s\n", err.c_str()); return 3; }
    Symbolic &Sy = E.Sy;
    i64 nD = Sy.Dptr[Sy.nf], nL = Sy.Lptr[Sy.nf];
    std::vector<T> LDo(nD), UDo(nD), LLo(nL), ULo(nL);
    int rc = ppo_factor(sr, dt, n, Sy.nf, Sy.Rptr.data(), Sy.Sptr.data(), Sy.Stgt.data(), Sy.perm.data(), colptr.data(),
                        rowval.data(), nzval.data(), LDo.data(), UDo.data(), LLo.data(), ULo.data());
    if (rc) { fprintf(stderr, "oracle factor %d\n", rc); return 4; }
    E.LD.assign(nD, S::zero());
    for (i64 f = 0; f < Sy.nf; f++) {
        i64 a = Sy.Rptr[f + 1] - Sy.Rptr[f];
        for (i64 j = 0; j < a; j++)
            for (i64 i = 0; i < a; i++) {
                i64 q = Sy.Dptr[f] + i + j * a;
                E.LD[q] = i > j ? LDo[q] : UDo[q];
            }
    }
    E.LL = LLo;
    E.UL = ULo;
    printf("n=%lld nf=%lld np=%lld nb=%lld sfwd=%zu sbwd=%zu bpack=%lld hpack=%lld subtrees=%zu (%zu panels)\n", (long long)n, (long long)Sy.nf,
           (long long)E.P.np, (long long)E.P.nb, E.P.sfwd.size(), E.P.sbwd.size(), (long long)E.P.nbpack,
           (long long)E.P.nhpack, E.P.sub_ptr.size() - 1, E.P.sub_pan.size());
    E.packs();
    E.use_plan_rows();
    RowSub R;
    std::vector<i64> srcs;   // requested sources, original labels
    if (mod > 0) {
        for (i64 s = 0; s < n; s++)
            if ((uint32_t)((uint64_t)s * 2654435761ull) % (uint64_t)mod == 0) srcs.push_back(s);
        for (i64 s : srcs) R.js.push_back((int32_t)Sy.invp[s]);
        std::sort(R.js.begin(), R.js.end());
        build_row_subset(E.P, Sy, R);
        E.use_subset(R);
        printf("sources %zu\n", srcs.size());
    }
    const i64 m = E.m;
    // X starts poisoned, as device memory that no kernel wrote: NaN (a bit pattern with every bit set for OrAnd), so
    // that a value read before it is written shows in the result as well as in the initialisation check
    E.X.assign(m * n, poison<T>());
    E.init.assign(m * n, 0);
    E.wtask.assign(m * n, -1);
    E.identity();
    E.subtrees(true);
    for (auto &li : E.P.sfwd) E.run_list(li, true);
    for (auto &li : E.P.sbwd) E.run_list(li, false);
    E.subtrees(false);
    // the off-diagonal blocks between components coupled by N (the rows of a source subset take the solve path
    // instead, which this replay does not cover)
    const bool coupled = E.P.coupled && mod <= 0;
    std::vector<i64> Bptr(Sy.Bptr.begin(), Sy.Bptr.end());
    if (coupled) {
        E.Nptr.assign(Sy.Nptr.begin(), Sy.Nptr.end());
        E.Nidx.assign(Sy.Nidx.begin(), Sy.Nidx.end());
        E.Nval.resize(Sy.nN);
        for (i64 q = 0; q < Sy.nN; q++) E.Nval[q] = nzval[Sy.Nsrc[q]];
        printf("components %lld, arcs between them %lld, levels %zu\n", (long long)Sy.nB, (long long)Sy.nN, E.P.cup.size());
        E.second_pass();
    }
    std::vector<T> C(n * n), Co(n * n);
    if (mod <= 0)
        for (i64 j = 0; j < n; j++)
            for (i64 i = 0; i < n; i++) C[i + j * n] = E.X[Sy.invp[i] + Sy.invp[j] * n];
    if (coupled)
        rc = ppo_star_scc(sr, dt, n, Sy.nf, Sy.Rptr.data(), Sy.Sptr.data(), Sy.Stgt.data(), Sy.perm.data(), LDo.data(),
                          UDo.data(), LLo.data(), ULo.data(), Sy.nB, Bptr.data(), E.Nptr.data(), E.Nidx.data(),
                          E.Nval.data(), Co.data(), 8);
    else
        rc = ppo_star(sr, dt, n, Sy.nf, Sy.Rptr.data(), Sy.Sptr.data(), Sy.Stgt.data(), Sy.perm.data(), LDo.data(),
                      UDo.data(), LLo.data(), ULo.data(), Co.data(), 0, n, 1, 8);
    if (rc) { fprintf(stderr, "oracle star %d\n", rc); return 4; }
    // the entries compared: all of the star, or the rows of the sources (row k of X is source js[k])
    std::vector<i64> qs;
    if (mod > 0) {
        C.assign(n * n, S::zero());
        for (i64 s : srcs) {
            const i64 k = R.map((int32_t)Sy.invp[s]);
            for (i64 j = 0; j < n; j++) {
                C[s + j * n] = E.X[k + Sy.invp[j] * m];
                qs.push_back(s + j * n);
            }
        }
    } else
        for (i64 q = 0; q < n * n; q++) qs.push_back(q);
    long ndiff = 0;
    double maxrel = 0;
    for (i64 q : qs) {
        T a = C[q], b = Co[q];
        if (sr == S_PLUSPROD) {
            double d = std::fabs((double)a - (double)b) / std::max(1e-300, std::fabs((double)b));
            if (d > maxrel) maxrel = d;
            // below the smallest normal number of T the relative precision is gone: measure against it there
            const double floor_ = (double)std::numeric_limits<T>::min();
            const double dd = std::fabs((double)a - (double)b) / std::max(floor_, std::fabs((double)b));
            if (!(dd <= 1e-4) && !(a == b)) {
                if (ndiff < 5) fprintf(stderr, "diff (%lld,%lld): %.9g vs %.9g\n", (long long)(q % n), (long long)(q / n), (double)a, (double)b);
                ndiff++;
            }
        } else if (std::memcmp(&a, &b, sizeof(T)) != 0) {
            if (ndiff < 5) fprintf(stderr, "diff at (%lld, %lld): %g vs %g\n", (long long)(q % n), (long long)(q / n), (double)a, (double)b);
            ndiff++;
        }
    }
    printf("errors %ld, differing entries %ld, max rel %.3g\n", nerr, ndiff, maxrel);
    return (nerr || ndiff) ? 1 : 0;
}

int main(int argc, char **argv) {
    if (argc < 5) { fprintf(stderr, "usage: star_plan_emu graph.bin semiring dtype ncu [M]\n"); return 2; }
    int sr = atoi(argv[2]), dt = atoi(argv[3]), ncu = atoi(argv[4]);
    long mod = argc > 5 ? atol(argv[5]) : 0;
    if (dt == D_F32) {
        switch (sr) {
        case S_MINPLUS: return run<MinPlus<float>>(argv[1], sr, dt, ncu, mod);
        case S_MAXPLUS: return run<MaxPlus<float>>(argv[1], sr, dt, ncu, mod);
        case S_MAXMIN: return run<MaxMin<float>>(argv[1], sr, dt, ncu, mod);
        case S_MINMAX: return run<MinMax<float>>(argv[1], sr, dt, ncu, mod);
        case S_PLUSPROD: return run<PlusProd<float>>(argv[1], sr, dt, ncu, mod);
        }
    } else if (dt == D_F64) {
        switch (sr) {
        case S_MINPLUS: return run<MinPlus<double>>(argv[1], sr, dt, ncu, mod);
        case S_MAXPLUS: return run<MaxPlus<double>>(argv[1], sr, dt, ncu, mod);
        case S_MAXMIN: return run<MaxMin<double>>(argv[1], sr, dt, ncu, mod);
        case S_MINMAX: return run<MinMax<double>>(argv[1], sr, dt, ncu, mod);
        case S_PLUSPROD: return run<PlusProd<double>>(argv[1], sr, dt, ncu, mod);
        }
    } else if (dt == D_I32) {
        return run<OrAnd>(argv[1], sr, dt, ncu, mod);
    }
    return 2;
}
