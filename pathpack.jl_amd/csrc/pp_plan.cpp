// pp_plan.cpp -- host construction of the device plans (see pp_internal.h).
#include <algorithm>
#include <atomic>

#include "pp_internal.h"

namespace pp {

namespace {
// Workers to ask the analysis's thread pool for, for a loop of `count` items: one per 8192 items, at most 16 (the
// loops take their items in chunks, so any number of workers that the pool runs covers them).
int plan_workers(i64 count) { return (int)std::min<i64>(16, std::max<i64>(1, count / 8192)); }
}  // namespace

std::string build_factor_plan(const Symbolic &S, FactorPlan &P) {
    const i64 nf = S.nf;
    P.nf = nf;
    P.nn.resize(nf);
    P.na.resize(nf);
    P.nj.resize(nf);
    P.Foff.resize(nf + 1);
    P.Foff[0] = 0;
    P.max_nj = 0;
    for (i64 f = 0; f < nf; f++) {
        i64 nn = S.Rptr[f + 1] - S.Rptr[f], na = S.Sptr[f + 1] - S.Sptr[f];
        if (nn + na > (i64)0x7fffffff / 2) return "front too large";
        P.nn[f] = (int32_t)nn;
        P.na[f] = (int32_t)na;
        P.nj[f] = (int32_t)(nn + na);
        P.Foff[f + 1] = P.Foff[f] + (nn + na) * (nn + na);
        P.max_nj = std::max(P.max_nj, nn + na);
    }
    P.arena = P.Foff[nf];
    P.Sptr32 = S.Sptr;
    // positions of each separator in its parent's bag: the parent's bag positions are scattered into a map over the
    // vertices, which its children then read (linear in the bags and separators)
    P.relpos.assign(S.Stgt.size(), 0);
    {
        std::vector<int32_t> kids(nf + 1, 0), kid(nf);
        for (i64 f = 0; f < nf; f++)
            if (S.parent[f] >= 0) kids[S.parent[f] + 1]++;
        for (i64 f = 0; f < nf; f++) kids[f + 1] += kids[f];
        {
            std::vector<int32_t> pos(kids.begin(), kids.end() - 1);
            for (i64 f = 0; f < nf; f++)
                if (S.parent[f] >= 0) kid[pos[S.parent[f]]++] = (int32_t)f;
        }
        // parents in chunks of 64 taken in turn by the pool's workers, each with its own map (every child's
        // positions are written by its parent's worker alone)
        const int nw = plan_workers((i64)S.Stgt.size());
        std::atomic<i64> next(0);
        std::atomic<bool> bad(false);
        auto work = [&](int) {
            std::vector<int32_t> where(S.n, -1);
            for (i64 p0; (p0 = next.fetch_add(64)) < nf && !bad.load(std::memory_order_relaxed);)
                for (i64 p = p0; p < std::min<i64>(nf, p0 + 64); p++) {
                    if (kids[p + 1] == kids[p]) continue;
                    const i64 a = S.Rptr[p + 1] - S.Rptr[p];
                    for (i64 v = S.Rptr[p]; v < S.Rptr[p + 1]; v++) where[v] = (int32_t)(v - S.Rptr[p]);
                    for (i64 q = S.Sptr[p]; q < S.Sptr[p + 1]; q++) where[S.Stgt[q]] = (int32_t)(a + (q - S.Sptr[p]));
                    for (int32_t k = kids[p]; k < kids[p + 1]; k++) {
                        const int32_t f = kid[k];
                        for (i64 q = S.Sptr[f]; q < S.Sptr[f + 1]; q++) {
                            const int32_t r = where[S.Stgt[q]];
                            if (r < 0) bad.store(true);
                            P.relpos[q] = r;
                        }
                    }
                    for (i64 v = S.Rptr[p]; v < S.Rptr[p + 1]; v++) where[v] = -1;
                    for (i64 q = S.Sptr[p]; q < S.Sptr[p + 1]; q++) where[S.Stgt[q]] = -1;
                }
        };
        if (nw > 1) pool_run(nw, work);
        else work(0);
        if (bad.load()) return "separator not contained in the parent's bag";
    }
    // children
    P.chptr.assign(nf + 1, 0);
    for (i64 f = 0; f < nf; f++)
        if (S.parent[f] >= 0) P.chptr[S.parent[f] + 1]++;
    for (i64 f = 0; f < nf; f++) P.chptr[f + 1] += P.chptr[f];
    P.chidx.assign(P.chptr[nf], 0);
    {
        std::vector<int32_t> pos(P.chptr.begin(), P.chptr.end() - 1);
        for (i64 f = 0; f < nf; f++)
            if (S.parent[f] >= 0) P.chidx[pos[S.parent[f]]++] = (int32_t)f;
    }
    // entries of A
    // (an arc between two strongly connected components belongs to N, not to a front: position -1, skipped)
    P.entry_pos.resize(S.nnz);
    {
        // chunks taken in turn (the pool may run fewer workers than asked)
        constexpr i64 CH = 8192;
        std::atomic<i64> next(0);
        auto work = [&](int) {
            for (i64 p0; (p0 = next.fetch_add(CH)) < S.nnz;)
                for (i64 p = p0; p < std::min<i64>(S.nnz, p0 + CH); p++) {
                    const i64 f = S.entry_front[p];
                    P.entry_pos[p] = f < 0 ? -1 : P.Foff[f] + S.entry_row[p] + (i64)S.entry_col[p] * P.nj[f];
                }
        };
        const int nw = plan_workers(S.nnz);
        if (nw > 1) pool_run(nw, work);
        else work(0);
    }
    // heights
    std::vector<i64> h(nf, 0);
    i64 H = 0;
    for (i64 f = 0; f < nf; f++) {
        if (S.parent[f] >= 0) h[S.parent[f]] = std::max(h[S.parent[f]], h[f] + 1);
        H = std::max(H, h[f] + 1);
    }
    std::vector<std::vector<int32_t>> byh(H);
    for (i64 f = 0; f < nf; f++) byh[h[f]].push_back((int32_t)f);
    P.etask.clear();   // the small fronts' factors are copied out of the arena; the steps write theirs directly
    for (i64 f = 0; f < nf; f++)
        if (P.nj[f] <= SMALL_NJ)
            for (int32_t c = 0; c < P.nj[f]; c += EXTRACT_COLS) {
                P.etask.push_back((int32_t)f);
                P.etask.push_back(c);
            }
    P.levels.clear();
    P.flist.clear();
    P.atask.clear();
    P.stask.clear();
    for (i64 l = 0; l < H; l++) {
        FactorPlan::Level L;
        L.asm_off = (i64)P.atask.size() / 2;
        // narrower column blocks while the level has fewer than four tasks per compute unit (the upper levels: few
        // parents with large update matrices), down to one column per wave
        i64 ncols = 0;
        for (int32_t f : byh[l])
            if (P.chptr[f + 1] > P.chptr[f]) ncols += P.nj[f];
        int32_t blk = ASM_BLOCK;
        while (blk > 4 && ncols / blk < 1024) blk /= 2;
        L.asm_blk = blk;
        for (int32_t f : byh[l])
            if (P.chptr[f + 1] > P.chptr[f])
                for (int32_t a = 0; a < P.nj[f]; a += blk) {
                    P.atask.push_back(f);
                    P.atask.push_back(a);
                }
        L.asm_cnt = (i64)P.atask.size() / 2 - L.asm_off;
        L.small_off = (i64)P.flist.size();
        for (int32_t f : byh[l])
            if (P.nj[f] <= SMALL_NJ) P.flist.push_back(f);
        L.small_cnt = (i64)P.flist.size() - L.small_off;
        i64 maxsteps = 0;
        for (int32_t f : byh[l])
            if (P.nj[f] > SMALL_NJ) maxsteps = std::max<i64>(maxsteps, (P.nn[f] + NB - 1) / NB);
        for (i64 s = 0; s < maxsteps; s++) {
            FactorPlan::Step st;
            st.off = (i64)P.stask.size() / 4;
            for (int32_t f : byh[l]) {
                if (P.nj[f] <= SMALL_NJ || s * NB >= P.nn[f]) continue;
                // one task per 64 x 64 tile of the trailing block; a step with no trailing block still has one
                // task, for its diagonal block
                const i64 off = s * NB, b = std::min<i64>(NB, P.nn[f] - off), m = P.nj[f] - off - b;
                const i64 T = std::max<i64>(1, (m + 63) / 64);
                for (i64 ti = 0; ti < T; ti++)
                    for (i64 tj = 0; tj < T; tj++) {
                        P.stask.push_back(f);
                        P.stask.push_back((int32_t)off);
                        P.stask.push_back((int32_t)ti);
                        P.stask.push_back((int32_t)tj);
                    }
            }
            st.cnt = (i64)P.stask.size() / 4 - st.off;
            L.steps.push_back(st);
        }
        P.levels.push_back(std::move(L));
    }
    return "";
}

std::string build_sweep_plan(const Symbolic &S, SweepPlan &P) {
    const i64 nf = S.nf;
    // panels
    std::vector<i64> first(nf), last(nf);
    P.np = 0;
    P.front.clear();
    P.c0.clear();
    P.w.clear();
    P.e.clear();
    P.lo_ext.clear();
    P.chunks.clear();
    P.rowA_lo.clear();
    P.rowA_hi.clear();
    P.rowB_lo.clear();
    P.rowB_hi.clear();
    P.eoff.clear();
    P.poff.clear();
    P.doff.clear();
    P.Eidx.clear();
    P.npack = 0;
    P.ndpack = 0;
    P.max_e = 0;
    std::vector<i64> root(nf);
    for (i64 f = nf - 1; f >= 0; f--) root[f] = S.parent[f] >= 0 ? root[S.parent[f]] : f;
    for (i64 f = 0; f < nf; f++) {
        const i64 Rp = S.Rptr[f], nn = S.Rptr[f + 1] - Rp, nj = nn + (S.Sptr[f + 1] - S.Sptr[f]);
        first[f] = P.np;
        for (i64 k = 0; k * PANEL_W < nn; k++) {
            const i64 c0 = Rp + k * PANEL_W, w = std::min<i64>(PANEL_W, nn - k * PANEL_W);
            const i64 lo = k * PANEL_W + w, e = nj - lo;
            P.front.push_back((int32_t)f);
            P.c0.push_back((int32_t)c0);
            P.w.push_back((int32_t)w);
            P.e.push_back((int32_t)e);
            P.lo_ext.push_back((int32_t)lo);
            P.chunks.push_back((int32_t)std::max<i64>(1, (e + SCATTER_T - 1) / SCATTER_T));
            const i64 Wc = class_width(width_class((int)w));
            P.eoff.push_back((i64)P.Eidx.size());
            for (i64 v = c0 + w; v < Rp + nn; v++) P.Eidx.push_back((int32_t)v);
            for (i64 q = S.Sptr[f]; q < S.Sptr[f + 1]; q++) P.Eidx.push_back((int32_t)S.Stgt[q]);
            P.poff.push_back(P.npack);
            P.npack += Wc * e;
            P.doff.push_back(P.ndpack);
            P.ndpack += Wc * Wc;
            P.rowA_lo.push_back((int32_t)S.Rptr[S.fdsc[f]]);
            P.rowA_hi.push_back((int32_t)(c0 + w));
            P.rowB_lo.push_back((int32_t)S.Rptr[S.fdsc[root[f]]]);
            P.rowB_hi.push_back((int32_t)S.Rptr[root[f] + 1]);
            P.max_e = std::max(P.max_e, e);
            P.np++;
        }
        last[f] = P.np - 1;
    }
    P.np = (i64)P.front.size();
    // star units: a front with at most PANEL_W columns keeps its panels; a wider front is cut into blocks of
    // BLK_W columns while more than 3/4 BLK_W remain, then one block of the rest if it is wider than PANEL_W (a
    // 64-column tile class when it fits), and the panels that cover a rest of at most PANEL_W columns
    std::vector<std::vector<int32_t>> su(nf);
    P.b_boff.clear();
    P.b_hoff.clear();
    P.b_kp.clear();
    P.b_ep.clear();
    P.b_bn.clear();
    P.prep.clear();
    P.nbpack = 0;
    P.nhpack = 0;
    for (i64 f = 0; f < nf; f++) {
        const i64 Rp = S.Rptr[f], nn = S.Rptr[f + 1] - Rp, nj = nn + (S.Sptr[f + 1] - S.Sptr[f]);
        i64 done = 0;
        while (nn > PANEL_W && nn - done > PANEL_W) {
            const i64 w = star_block_w(nn - done), bn = star_block_bn(w);
            const i64 c0 = Rp + done, lo = done + w, e = nj - lo;
            const i64 b = (i64)P.b_boff.size();
            su[f].push_back((int32_t)P.front.size());
            P.front.push_back((int32_t)f);
            P.c0.push_back((int32_t)c0);
            P.w.push_back((int32_t)w);
            P.e.push_back((int32_t)e);
            P.lo_ext.push_back((int32_t)lo);
            P.chunks.push_back(1);
            P.eoff.push_back((i64)P.Eidx.size());
            for (i64 v = c0 + w; v < Rp + nn; v++) P.Eidx.push_back((int32_t)v);
            for (i64 q = S.Sptr[f]; q < S.Sptr[f + 1]; q++) P.Eidx.push_back((int32_t)S.Stgt[q]);
            P.poff.push_back(0);
            P.doff.push_back(0);
            P.rowA_lo.push_back((int32_t)S.Rptr[S.fdsc[f]]);
            P.rowA_hi.push_back((int32_t)(c0 + w));
            P.rowB_lo.push_back((int32_t)S.Rptr[S.fdsc[root[f]]]);
            P.rowB_hi.push_back((int32_t)S.Rptr[root[f] + 1]);
            P.max_e = std::max(P.max_e, e);
            const i64 kp = round_up(w + e, BLK_K), wp = round_up(w, BLK_K), ep = round_up(e, BLK_W);
            P.b_boff.push_back(P.nbpack);
            P.b_kp.push_back((int32_t)kp);
            P.b_bn.push_back((int32_t)bn);
            P.nbpack += kp * bn;
            P.b_hoff.push_back(P.nhpack);
            P.b_ep.push_back((int32_t)ep);
            P.nhpack += wp * ep;
            // pack GEMM tiles: M (w x w), G (e x w), H (w x e)
            const i64 tw = (w + PREP_T - 1) / PREP_T, te = (e + PREP_T - 1) / PREP_T;
            auto task = [&](int part, i64 tr, i64 tc) {
                P.prep.push_back((int32_t)b);
                P.prep.push_back(part);
                P.prep.push_back((int32_t)tr);
                P.prep.push_back((int32_t)tc);
            };
            for (i64 tr = 0; tr < tw; tr++)
                for (i64 tc = 0; tc < tw; tc++) task(0, tr, tc);
            for (i64 tr = 0; tr < te; tr++)
                for (i64 tc = 0; tc < tw; tc++) task(1, tr, tc);
            for (i64 tr = 0; tr < tw; tr++)
                for (i64 tc = 0; tc < te; tc++) task(2, tr, tc);
            done += w;
        }
        // the rest, if any: panels (every block before a rest is 64 or 128 wide, so done is a multiple of PANEL_W)
        if (done < nn)
            for (i64 p = first[f] + done / PANEL_W; p <= last[f]; p++) su[f].push_back((int32_t)p);
    }
    P.nb = (i64)P.front.size() - P.np;
    P.Eidx.insert(P.Eidx.end(), EIDX_PAD, 0);
    // forward levels (leaves to root) and backward levels (root to leaves) of a sequence of units per front
    const i64 nu = (i64)P.front.size();
    auto levels = [&](const std::vector<std::vector<int32_t>> &units, std::vector<i64> &lvA, std::vector<i64> &lvB) {
        lvA.assign(nu, -1);
        lvB.assign(nu, -1);
        std::vector<i64> baseA(nf, 0);   // fronts are in postorder: a front's children come before it
        for (i64 f = 0; f < nf; f++) {
            const auto &U = units[f];
            for (size_t k = 0; k < U.size(); k++) lvA[U[k]] = baseA[f] + (i64)k;
            if (S.parent[f] >= 0 && !U.empty()) baseA[S.parent[f]] = std::max(baseA[S.parent[f]], lvA[U.back()] + 1);
        }
        std::vector<i64> endB(nf, -1);   // level of the front's first unit (the last one visited)
        for (i64 f = nf - 1; f >= 0; f--) {
            const auto &U = units[f];
            const i64 base = S.parent[f] >= 0 ? endB[S.parent[f]] + 1 : 0;
            for (size_t k = 0; k < U.size(); k++) lvB[U[k]] = base + (i64)(U.size() - 1 - k);
            endB[f] = U.empty() ? base - 1 : lvB[U[0]];
        }
    };
    // star subtrees (fronts with at most PANEL_W columns have exactly one panel); their panels leave the star lists
    P.sub_ptr.assign(1, 0);
    P.sub_pan.clear();
    P.sub_rows.clear();
    P.sub_preF.assign(1, 0);
    P.sub_preB.assign(1, 0);
    {
        std::vector<char> small(nf), ok(nf);
        for (i64 f = 0; f < nf; f++) small[f] = S.Rptr[f + 1] - S.Rptr[f] <= PANEL_W;
        for (i64 f = 0; f < nf; f++)   // postorder: a front's children come before it
            if (!small[f] && S.parent[f] >= 0) small[S.parent[f]] = 0;
        for (i64 f = 0; f < nf; f++)
            ok[f] = small[f] && (S.Rptr[f + 1] - S.Rptr[S.fdsc[f]]) + (S.Sptr[f + 1] - S.Sptr[f]) <= SUB_L;
        for (i64 r = 0; r < nf; r++) {
            if (!ok[r] || (S.parent[r] >= 0 && ok[S.parent[r]])) continue;
            for (i64 f = S.fdsc[r]; f <= r; f++) {
                P.sub_pan.push_back((int32_t)first[f]);
                su[f].clear();
            }
            P.sub_ptr.push_back((int32_t)P.sub_pan.size());
            const int32_t p = (int32_t)first[r];
            const int32_t flo = (int32_t)S.Rptr[S.fdsc[r]], fhi = (int32_t)S.Rptr[r + 1];
            P.sub_rows.insert(P.sub_rows.end(), {flo, fhi, P.rowB_lo[p], P.rowB_hi[p]});
            P.sub_preF.push_back(P.sub_preF.back() + (fhi - flo + TILE_ROWS - 1) / TILE_ROWS);
            P.sub_preB.push_back(P.sub_preB.back() + (P.rowB_hi[p] - P.rowB_lo[p] + TILE_ROWS - 1) / TILE_ROWS);
        }
    }
    std::vector<i64> lvA, lvB, slvA, slvB;
    {
        std::vector<std::vector<int32_t>> pu(nf);
        for (i64 f = 0; f < nf; f++)
            for (i64 p = first[f]; p <= last[f]; p++) pu[f].push_back((int32_t)p);
        levels(pu, lvA, lvB);
    }
    levels(su, slvA, slvB);
    P.sunits.clear();
    for (i64 f = 0; f < nf; f++) P.sunits.insert(P.sunits.end(), su[f].begin(), su[f].end());
    P.sunits.insert(P.sunits.end(), P.sub_pan.begin(), P.sub_pan.end());
    auto rowtiles = [](i64 lo, i64 hi, i64 bm) { return hi > lo ? (hi - lo / bm * bm + bm - 1) / bm : 0; };
    auto unit_class = [&](i64 p) {
        return p < P.np ? width_class(P.w[p]) : P.b_bn[p - P.np] == BLK_W ? BLK_CLS : BLK_CLS + 1;
    };
    // the rows of the star's second pass (components coupled by N): those of the earlier components with a path in
    P.coupled = S.nB > 1 && S.nN > 0;
    P.rowC_lo.assign(nu, 0);
    P.rowC_hi.assign(nu, 0);
    if (P.coupled)
        for (i64 p = 0; p < nu; p++) {
            const i64 c = S.comp[P.c0[p]];
            P.rowC_lo[p] = (int32_t)S.anc_lo[c];
            P.rowC_hi[p] = (int32_t)S.Bptr[c];
        }
    // one list of units of one level and width class, with the prefix arrays of its launches
    auto emit = [&](int cls, const std::vector<int32_t> &bucket, bool fwd, std::vector<SweepPlan::List> &out) {
        {
            SweepPlan::List li;
            li.cls = cls;
            li.off = (i64)P.plist.size();
            li.cnt = (i64)bucket.size();
            P.plist.insert(P.plist.end(), bucket.begin(), bucket.end());
            auto prefix = [&](auto units) {
                const i64 off = (i64)P.tiles.size();
                int64_t acc = 0;
                P.tiles.push_back(0);
                for (int32_t p : bucket) {
                    acc += units(p);
                    P.tiles.push_back((int32_t)acc);
                }
                return off;
            };
            auto tiles_of = [&](i64 lo, i64 hi, i64 rows) { return hi > lo ? (hi - lo + rows - 1) / rows : 0; };
            li.pAu = prefix([&](int32_t p) { return tiles_of(P.rowA_lo[p], P.rowA_hi[p], TILE_ROWS) * P.chunks[p]; });
            li.pB64 = prefix([&](int32_t p) { return tiles_of(P.rowB_lo[p], P.rowB_hi[p], TILE_ROWS); });
            li.pC = prefix([&](int32_t p) { return (i64)P.chunks[p]; });
            li.pCu = prefix([&](int32_t p) { return tiles_of(P.rowC_lo[p], P.rowC_hi[p], TILE_ROWS) * P.chunks[p]; });
            li.pC64 = prefix([&](int32_t p) { return tiles_of(P.rowC_lo[p], P.rowC_hi[p], TILE_ROWS); });
            li.pT[0] = li.pT[1] = 0;
            if (li.cls >= BLK_CLS)
                for (int q = 0; q < 2; q++) {
                    const i64 bm = 64 << q;
                    li.pT[q] = prefix([&](int32_t p) {
                        if (fwd) return P.e[p] > 0 ? rowtiles(P.rowA_lo[p], P.rowA_hi[p], bm) * ((P.e[p] + BLK_W - 1) / BLK_W) : 0;
                        return rowtiles(P.rowB_lo[p], P.rowB_hi[p], bm);
                    });
                }
            li.esum = li.emax = 0;
            for (int32_t p : bucket) {
                li.esum += P.e[p];
                li.emax = std::max<i64>(li.emax, P.e[p]);
            }
            li.uniB = true;
            li.rowB_lo = P.rowB_lo[bucket[0]];
            li.rowB_hi = P.rowB_hi[bucket[0]];
            for (int32_t p : bucket)
                if (P.rowB_lo[p] != li.rowB_lo || P.rowB_hi[p] != li.rowB_hi) li.uniB = false;
            out.push_back(li);
        }
    };
    // the lists of the units with lv >= 0: by level (increasing), then width class
    // the lists of a subset of the units with lv >= 0: by level (increasing), then width class
    auto make_lists_of = [&](const std::vector<int32_t> &units, const std::vector<i64> &lv, bool fwd,
                             std::vector<SweepPlan::List> &out) {
        std::vector<std::pair<i64, int32_t>> key;   // (level * classes + class, unit)
        constexpr int NC = BLK_CLS + 2;
        for (int32_t p : units) key.push_back({lv[p] * NC + unit_class(p), p});
        std::sort(key.begin(), key.end());
        std::vector<int32_t> bucket;
        for (size_t k = 0; k < key.size(); k++) {
            bucket.push_back(key[k].second);
            if (k + 1 == key.size() || key[k + 1].first != key[k].first) {
                emit((int)(key[k].first % NC), bucket, fwd, out);
                bucket.clear();
            }
        }
    };
    P.plist.clear();
    P.tiles.clear();
    P.sfwd.clear();
    P.sbwd.clear();
    // the panels (every front's) by level, the width classes of a level in one list (wider panels first)
    auto make_mixed = [&](const std::vector<i64> &lv, bool fwd, std::vector<SweepPlan::List> &out) {
        i64 L = 0;
        for (i64 p = 0; p < nu; p++) L = std::max(L, lv[p] + 1);
        std::vector<std::vector<int32_t>> buckets(L);
        for (i64 p = 0; p < P.np; p++)
            if (lv[p] >= 0) buckets[lv[p]].push_back((int32_t)p);
        for (auto &b : buckets) {
            if (b.empty()) continue;
            std::stable_sort(b.begin(), b.end(), [&](int32_t x, int32_t y) { return P.w[x] > P.w[y]; });
            emit(-1, b, fwd, out);
        }
    };
    P.fwdm.clear();
    P.bwdm.clear();
    make_mixed(lvA, true, P.fwdm);
    make_mixed(lvB, false, P.bwdm);
    // the star's lists: per level, its panels of every width class in one list (one launch, wider panels first)
    // and its blocks by tile width
    auto make_star_lists = [&](const std::vector<i64> &lv, bool fwd, std::vector<SweepPlan::List> &out) {
        i64 L = 0;
        for (i64 p = 0; p < nu; p++) L = std::max(L, lv[p] + 1);
        constexpr int NC = BLK_CLS + 2;
        std::vector<std::vector<int32_t>> buckets(L * NC);
        for (i64 p = 0; p < nu; p++)
            if (lv[p] >= 0) buckets[lv[p] * NC + (p < P.np ? 0 : unit_class(p))].push_back((int32_t)p);
        for (i64 b = 0; b < (i64)buckets.size(); b++) {
            auto &bk = buckets[b];
            if (bk.empty()) continue;
            if (b % NC == 0) {
                std::stable_sort(bk.begin(), bk.end(), [&](int32_t x, int32_t y) { return P.w[x] > P.w[y]; });
                emit(-1, bk, fwd, out);
            } else {
                emit((int)(b % NC), bk, fwd, out);
            }
        }
    };
    make_star_lists(slvA, true, P.sfwd);
    make_star_lists(slvB, false, P.sbwd);
    // the schedules over the component DAG (panels only, as the solves)
    P.cup.clear();
    P.cdn.clear();
    P.cfwd.clear();
    P.cbwd.clear();
    P.ccols.clear();
    P.ccol_lo.clear();
    P.ccol_hi.clear();
    if (P.coupled) {
        std::vector<std::vector<int32_t>> cpan(S.nB);   // panels of each component
        for (i64 p = 0; p < P.np; p++) cpan[S.comp[P.c0[p]]].push_back((int32_t)p);
        auto schedule = [&](const std::vector<i32> &lev, bool up, std::vector<SweepPlan::CLevel> &out) {
            i64 L = 0;
            for (i64 c = 0; c < S.nB; c++) L = std::max<i64>(L, lev[c] + 1);
            std::vector<std::vector<int32_t>> bylev(L);
            for (i64 c = 0; c < S.nB; c++) bylev[lev[c]].push_back((int32_t)c);
            std::vector<int32_t> units;
            for (i64 l = 0; l < L; l++) {
                SweepPlan::CLevel cl;
                cl.cols_off = (i64)P.ccols.size();
                units.clear();
                for (int32_t c : bylev[l]) {
                    for (i64 j = S.Bptr[c]; j < S.Bptr[c + 1]; j++) {
                        const bool any = up ? S.Nptr[j + 1] > S.Nptr[j] : S.NTptr[j + 1] > S.NTptr[j];
                        if (!any) continue;
                        P.ccols.push_back((int32_t)j);
                        P.ccol_lo.push_back((int32_t)S.anc_lo[c]);
                        P.ccol_hi.push_back((int32_t)S.Bptr[c]);
                    }
                    units.insert(units.end(), cpan[c].begin(), cpan[c].end());
                }
                cl.cols_cnt = (i64)P.ccols.size() - cl.cols_off;
                cl.fwd_off = (i64)P.cfwd.size();
                make_lists_of(units, lvA, true, P.cfwd);
                cl.fwd_cnt = (i64)P.cfwd.size() - cl.fwd_off;
                cl.bwd_off = (i64)P.cbwd.size();
                make_lists_of(units, lvB, false, P.cbwd);
                cl.bwd_cnt = (i64)P.cbwd.size() - cl.bwd_off;
                out.push_back(cl);
            }
        };
        schedule(S.lev_up, true, P.cup);
        schedule(S.lev_dn, false, P.cdn);
    }
    return "";
}

SweepSizes sweep_sizes(const Symbolic &S) {
    SweepSizes z;
    for (i64 f = 0; f < S.nf; f++) {
        const i64 nn = S.Rptr[f + 1] - S.Rptr[f], nj = nn + (S.Sptr[f + 1] - S.Sptr[f]);
        for (i64 k = 0; k * PANEL_W < nn; k++) {   // panels (every front)
            const i64 w = std::min<i64>(PANEL_W, nn - k * PANEL_W), e = nj - (k * PANEL_W + w);
            const i64 Wc = class_width(width_class((int)w));
            z.units++;
            z.eidx += e;
            z.npack += Wc * e;
            z.ndpack += Wc * Wc;
        }
        for (i64 done = 0; nn > PANEL_W && nn - done > PANEL_W;) {   // star blocks (fronts wider than a panel)
            const i64 w = star_block_w(nn - done), e = nj - (done + w);
            z.units++;
            z.eidx += e;
            z.nbpack += round_up(w + e, BLK_K) * star_block_bn(w);
            z.nhpack += round_up(w, BLK_K) * round_up(e, BLK_W);
            const i64 tw = (w + PREP_T - 1) / PREP_T, te = (e + PREP_T - 1) / PREP_T;
            z.prep += tw * tw + 2 * te * tw;
            z.nb++;
            done += w;
        }
    }
    z.eidx += EIDX_PAD;
    z.nN = S.nB > 1 ? S.nN : 0;
    return z;
}

int32_t RowSub::map(int32_t r) const { return (int32_t)(std::lower_bound(js.begin(), js.end(), r) - js.begin()); }

void build_row_subset(const SweepPlan &P, const Symbolic &S, RowSub &R) {
    const i64 nu = (i64)P.front.size();
    R.rowA_lo.resize(nu);
    R.rowA_hi.resize(nu);
    R.rowB_lo.resize(nu);
    R.rowB_hi.resize(nu);
    for (i64 p = 0; p < nu; p++) {
        R.rowA_lo[p] = R.map(P.rowA_lo[p]);
        R.rowA_hi[p] = R.map(P.rowA_hi[p]);
        R.rowB_lo[p] = R.map(P.rowB_lo[p]);
        R.rowB_hi[p] = R.map(P.rowB_hi[p]);
    }
    // the prefix arrays of every list, in the plan's layout (make_lists)
    R.tiles = P.tiles;
    auto tiles_of = [](i64 lo, i64 hi, i64 rows) { return hi > lo ? (hi - lo + rows - 1) / rows : 0; };
    auto rowtiles = [](i64 lo, i64 hi, i64 bm) { return hi > lo ? (hi - lo / bm * bm + bm - 1) / bm : 0; };
    auto redo = [&](const SweepPlan::List &li, bool fwd) {
        auto prefix = [&](i64 off, auto units) {
            int32_t acc = 0;
            R.tiles[off] = 0;
            for (i64 k = 0; k < li.cnt; k++) {
                acc += (int32_t)units(P.plist[li.off + k]);
                R.tiles[off + 1 + k] = acc;
            }
        };
        prefix(li.pAu, [&](int32_t p) { return tiles_of(R.rowA_lo[p], R.rowA_hi[p], TILE_ROWS) * P.chunks[p]; });
        prefix(li.pB64, [&](int32_t p) { return tiles_of(R.rowB_lo[p], R.rowB_hi[p], TILE_ROWS); });
        if (li.cls >= BLK_CLS)
            for (int q = 0; q < 2; q++) {
                const i64 bm = 64 << q;
                prefix(li.pT[q], [&](int32_t p) -> i64 {
                    if (fwd) return P.e[p] > 0 ? rowtiles(R.rowA_lo[p], R.rowA_hi[p], bm) * ((P.e[p] + BLK_W - 1) / BLK_W) : 0;
                    return rowtiles(R.rowB_lo[p], R.rowB_hi[p], bm);
                });
            }
    };
    for (const auto &li : P.fwdm) redo(li, true);
    for (const auto &li : P.bwdm) redo(li, false);
    for (const auto &li : P.sfwd) redo(li, true);
    for (const auto &li : P.sbwd) redo(li, false);
    // subtrees
    const i64 nsub = (i64)P.sub_ptr.size() - 1;
    R.sub_rows.resize(4 * std::max<i64>(nsub, 0));
    R.sub_preF.assign(1, 0);
    R.sub_preB.assign(1, 0);
    for (i64 s = 0; s < nsub; s++) {
        for (int k = 0; k < 4; k++) R.sub_rows[4 * s + k] = R.map(P.sub_rows[4 * s + k]);
        R.sub_preF.push_back(R.sub_preF.back() + (int32_t)tiles_of(R.sub_rows[4 * s], R.sub_rows[4 * s + 1], TILE_ROWS));
        R.sub_preB.push_back(R.sub_preB.back() + (int32_t)tiles_of(R.sub_rows[4 * s + 2], R.sub_rows[4 * s + 3], TILE_ROWS));
    }
    (void)S;
}

}  // namespace pp
