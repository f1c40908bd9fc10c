// pp_symbolic.cpp -- host symbolic analysis: ordering, elimination tree, supernodes, separators.
//
// Replaces the CliqueTrees.jl calls of the reference (src/CPU/chordal_ssymbolic.jl:26-184: cliquetree,
// symmetric, ChordalSymbolic).  See pp_symbolic.h for what is computed and how it differs.
#include "pp_symbolic.h"

#include <algorithm>
#include <climits>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <mutex>
#include <thread>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <numeric>
#include <unistd.h>

namespace pp {

namespace {
int max_threads();
}

// A pool of worker threads kept for the life of the process (created at the first parallel call, again in a
// forked child): starting and joining 15 threads costs about a millisecond, several times per analysis.  A job is
// published as one atomic word, (generation << 8) | workers, so a worker never pairs one job's worker count with
// another's generation.  Idle workers spin on that word for about 50 microseconds before they sleep on a condition
// variable: the analysis runs a dozen short parallel steps with short serial steps between them, and waking a
// sleeping thread costs tens of microseconds; a longer spin would take the cores from the serial steps and from the
// thread that launches the GPU work after the analysis.
namespace {
inline void cpu_relax() {
#if defined(__x86_64__)
    __builtin_ia32_pause();
#endif
}

class ThreadPool {
  public:
    explicit ThreadPool(int n) {
        for (int i = 1; i < n; i++) th_.emplace_back([this, i] { loop(i); });
    }
    ~ThreadPool() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_.store(true);
        }
        cv_.notify_all();
        for (auto &t : th_) t.join();
    }
    int size() const { return (int)th_.size() + 1; }
    void run(int n, const std::function<void(int)> &fn) {
        std::lock_guard<std::mutex> one(run_mu_);   // one job at a time
        job_ = &fn;
        pending_.store(n - 1, std::memory_order_relaxed);
        bool wake;
        {
            std::lock_guard<std::mutex> lk(mu_);
            const uint64_t g = (word_.load(std::memory_order_relaxed) >> 8) + 1;
            word_.store(g << 8 | (uint64_t)n, std::memory_order_release);
            wake = sleepers_ > 0;
        }
        if (wake) cv_.notify_all();
        fn(0);
        for (unsigned spins = 0; pending_.load(std::memory_order_acquire) != 0; spins++) {
            if (spins < 4096) cpu_relax();
            else std::this_thread::yield();
        }
    }

  private:
    void loop(int i) {
        uint64_t seen = 0;   // the word before the first job: a job published before this thread starts still runs
        while (true) {
            uint64_t w = word_.load(std::memory_order_acquire);
            if (w == seen) {
                const double t0 = now_s();
                for (unsigned spins = 1; (w = word_.load(std::memory_order_acquire)) == seen; spins++) {
                    if (stop_.load(std::memory_order_relaxed)) return;
                    cpu_relax();
                    if ((spins & 255) == 0 && now_s() - t0 > 5e-5) {
                        std::unique_lock<std::mutex> lk(mu_);
                        sleepers_++;
                        cv_.wait(lk, [&] { return stop_.load() || word_.load() != seen; });
                        sleepers_--;
                        if (stop_.load()) return;
                    }
                }
            }
            seen = w;
            if (i >= (int)(w & 0xff)) continue;
            (*job_)(i);
            pending_.fetch_sub(1, std::memory_order_acq_rel);
        }
    }
    static double now_s() {
        return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
    }
    std::vector<std::thread> th_;
    std::mutex mu_, run_mu_;
    std::condition_variable cv_;
    const std::function<void(int)> *job_ = nullptr;
    std::atomic<uint64_t> word_{0};
    std::atomic<int> pending_{0};
    std::atomic<bool> stop_{false};
    int sleepers_ = 0;
};
}  // namespace

void pool_run(int n, const std::function<void(int)> &fn) {
    static std::mutex mu;
    static ThreadPool *pool = nullptr;
    static pid_t owner = 0;
    if (n <= 1) {
        fn(0);
        return;
    }
    ThreadPool *p;
    {
        std::lock_guard<std::mutex> lk(mu);
        if (!pool || owner != getpid()) {   // a forked child does not have its parent's threads
            pool = new ThreadPool(std::max(2, max_threads()));   // kept to the end of the process
            owner = getpid();
        }
        p = pool;
    }
    if (n > p->size()) n = p->size();
    p->run(n, fn);
}

namespace {

double now() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// PP_SYMTIME=1 prints the time of each stage of the analysis to stderr
void stage(const char *name, double &t) {
    static const bool on = std::getenv("PP_SYMTIME") != nullptr;
    const double t1 = now();
    if (on) std::fprintf(stderr, "pp_symbolic: %-28s %8.2f ms\n", name, (t1 - t) * 1e3);
    t = t1;
}

struct Adj {
    i64 n = 0;
    std::vector<i64> xadj;
    std::vector<i32> adj;
};

// Threads for the host analysis: up to 16 (PP_SYMBOLIC_THREADS overrides), one for small graphs.
int max_threads() {
    int threads = (int)std::min<unsigned>(16, std::max(1u, std::thread::hardware_concurrency()));
    if (const char *e = std::getenv("PP_SYMBOLIC_THREADS")) threads = std::max(1, std::min(64, std::atoi(e)));
    return threads;
}
int analysis_threads(i64 n) { return n < 4096 ? 1 : max_threads(); }

// fn(lo, hi) over [0, count) in contiguous blocks on `threads` threads of the pool (the caller's thread takes the
// first block)
template <class Fn> void parallel_for(i64 count, int threads, Fn fn) {
    threads = (int)std::max<i64>(1, std::min<i64>(threads, count / 1024));
    if (threads <= 1) {
        fn((i64)0, count);
        return;
    }
    pool_run(threads, [&](int t) { fn(count * t / threads, count * (t + 1) / threads); });
}

// The CSC arrays of an n x n pattern: "" when they are well formed (the message names the first bad column's fault).
std::string check_csc(i64 n, const i64 *colptr, const i64 *rowval, int threads = 1) {
    if (n < 0 || n > (i64)0x7fffffff) return "n out of range";
    if (colptr[0] != 0) return "colptr[0] must be 0";
    for (i64 j = 0; j < n; j++)
        if (colptr[j + 1] < colptr[j]) return "colptr must be nondecreasing";
    std::atomic<i64> bad(n);   // first column with a bad row list
    parallel_for(n, threads, [&](i64 a, i64 b) {
        for (i64 j = a; j < b && j < bad.load(std::memory_order_relaxed); j++)
            for (i64 p = colptr[j]; p < colptr[j + 1]; p++)
                if (rowval[p] < 0 || rowval[p] >= n || (p > colptr[j] && rowval[p] <= rowval[p - 1])) {
                    i64 cur = bad.load();
                    while (j < cur && !bad.compare_exchange_weak(cur, j)) {}
                    break;
                }
    });
    if (bad.load() < n) {
        const i64 j = bad.load();
        for (i64 p = colptr[j]; p < colptr[j + 1]; p++) {
            if (rowval[p] < 0 || rowval[p] >= n) return "row index out of range";
            if (p > colptr[j] && rowval[p] <= rowval[p - 1]) return "row indices must be sorted and unique in each column";
        }
    }
    return "";
}

// Whether the pattern is symmetric (A[i, j] stored iff A[j, i] stored): each off-diagonal entry's mirror is looked up
// in its column (binary search; the rows are sorted).  Then the symmetrized pattern is A without its diagonal.
bool pattern_symmetric(i64 n, const i64 *colptr, const i64 *rowval, int threads) {
    std::atomic<bool> ok(true);
    parallel_for(n, threads, [&](i64 a, i64 b) {
        for (i64 j = a; j < b && ok.load(std::memory_order_relaxed); j++)
            for (i64 p = colptr[j]; p < colptr[j + 1]; p++) {
                const i64 i = rowval[p];
                if (i != j && !std::binary_search(rowval + colptr[i], rowval + colptr[i + 1], j)) {
                    ok = false;
                    break;
                }
            }
    });
    return ok.load();
}

// The symmetrized pattern of a symmetric A: its columns without the diagonal, in parallel.
void offdiagonal(i64 n, const i64 *colptr, const i64 *rowval, Adj &G, int threads) {
    G.n = n;
    G.xadj.assign(n + 1, 0);
    parallel_for(n, threads, [&](i64 a, i64 b) {
        for (i64 j = a; j < b; j++) {
            i64 c = colptr[j + 1] - colptr[j];
            if (c > 0 && std::binary_search(rowval + colptr[j], rowval + colptr[j + 1], j)) c--;
            G.xadj[j + 1] = c;
        }
    });
    for (i64 j = 0; j < n; j++) G.xadj[j + 1] += G.xadj[j];
    G.adj.resize(G.xadj[n]);
    parallel_for(n, threads, [&](i64 a, i64 b) {
        for (i64 j = a; j < b; j++) {
            i64 w = G.xadj[j];
            for (i64 p = colptr[j]; p < colptr[j + 1]; p++)
                if (rowval[p] != j) G.adj[w++] = (i32)rowval[p];
        }
    });
}

// Connected components of G (a symmetric pattern: they are its strongly connected components), numbered in the order
// of their smallest vertex -- the numbering strong_components gives a symmetric pattern.  A lock-free disjoint-set
// forest over the edges in parallel, a root always linked under a smaller one, so each set's root ends at its smallest
// vertex whatever the threads' interleaving.
i64 connected_components(const Adj &G, std::vector<i32> &comp, int threads) {
    const i64 n = G.n;
    std::vector<i32> up(n);
    parallel_for(n, threads, [&](i64 a, i64 b) {
        for (i64 v = a; v < b; v++) up[v] = (i32)v;
    });
    auto find = [&](i32 x) {
        while (true) {
            const i32 p = std::atomic_ref<i32>(up[x]).load(std::memory_order_relaxed);
            if (p == x) return x;
            const i32 g = std::atomic_ref<i32>(up[p]).load(std::memory_order_relaxed);
            if (g != p) {   // path halving
                i32 e = p;
                std::atomic_ref<i32>(up[x]).compare_exchange_weak(e, g, std::memory_order_relaxed);
            }
            x = p;
        }
    };
    parallel_for(n, threads, [&](i64 a, i64 b) {
        for (i64 v = a; v < b; v++)
            for (i64 q = G.xadj[v]; q < G.xadj[v + 1]; q++) {
                const i32 u = G.adj[q];
                if (u >= v) continue;   // each edge once
                while (true) {
                    i32 ru = find(u), rv = find((i32)v);
                    if (ru == rv) break;
                    if (ru < rv) std::swap(ru, rv);   // link the larger root under the smaller
                    i32 expect = ru;
                    if (std::atomic_ref<i32>(up[ru]).compare_exchange_strong(expect, rv)) break;
                }
            }
    });
    comp.assign(n, -1);
    i32 nc = 0;
    for (i64 v = 0; v < n; v++) {
        const i32 r = find((i32)v);
        comp[v] = r == v ? nc++ : comp[r];
    }
    return nc;
}

// Symmetric pattern of A without the diagonal, neighbours sorted; with `comp`, only the pairs inside one component
// (the pattern of the diagonal blocks).  The CSC arrays must have passed check_csc.
std::string symmetrize(i64 n, const i64 *colptr, const i64 *rowval, Adj &G, const std::vector<i32> *comp = nullptr) {
    // A^T by a counting sort over the columns of A: the entries of each of its columns come out in increasing order
    const i64 nnz = colptr[n];
    std::vector<i64> tptr(n + 1, 0);
    std::vector<i32> tidx(nnz);
    for (i64 p = 0; p < nnz; p++) tptr[rowval[p] + 1]++;
    for (i64 v = 0; v < n; v++) tptr[v + 1] += tptr[v];
    {
        std::vector<i64> pos(tptr.begin(), tptr.end() - 1);
        for (i64 j = 0; j < n; j++)
            for (i64 p = colptr[j]; p < colptr[j + 1]; p++) tidx[pos[rowval[p]]++] = (i32)j;
    }
    // adj(v): the sorted union of column v of A and of A^T, without v
    G.n = n;
    std::vector<i64> nx(n + 1, 0);
    G.adj.resize(2 * nnz);
    i64 w = 0;
    for (i64 v = 0; v < n; v++) {
        nx[v] = w;
        i64 a = colptr[v], ae = colptr[v + 1], b = tptr[v], be = tptr[v + 1];
        while (a < ae || b < be) {
            i64 x;
            if (b >= be || (a < ae && rowval[a] <= (i64)tidx[b])) {
                x = rowval[a];
                if (b < be && (i64)tidx[b] == x) b++;
                a++;
            } else {
                x = tidx[b++];
            }
            if (x != v && (!comp || (*comp)[x] == (*comp)[v])) G.adj[w++] = (i32)x;
        }
    }
    nx[n] = w;
    G.xadj = nx;
    G.adj.resize(w);
    return "";
}

// ===== strongly connected components (Tarjan 1972, iterative) =====
//
// The digraph has the arc i -> j for every stored A[i, j], i != j.  The search walks the arcs backwards, from
// column j to its rows i, so a component is completed only after every component with an arc into it; numbering the
// components in the order of completion therefore puts every arc between two components from a lower to a higher
// number.  The reference's sccs! (utils.jl:18-70) walks the same column lists from the same roots.
i64 strong_components(i64 n, const i64 *colptr, const i64 *rowval, std::vector<i32> &comp) {
    comp.assign(n, -1);
    std::vector<i32> index(n, -1), low(n, 0), stack, call;
    std::vector<i64> edge(n, 0);
    std::vector<char> on(n, 0);
    stack.reserve(n);
    i32 counter = 0, nc = 0;
    for (i64 s0 = 0; s0 < n; s0++) {
        if (index[s0] >= 0) continue;
        auto enter = [&](i64 v) {
            index[v] = low[v] = counter++;
            edge[v] = colptr[v];
            stack.push_back((i32)v);
            on[v] = 1;
            call.push_back((i32)v);
        };
        enter(s0);
        while (!call.empty()) {
            const i64 v = call.back();
            if (edge[v] < colptr[v + 1]) {
                const i64 w = rowval[edge[v]++];
                if (index[w] < 0) enter(w);
                else if (on[w]) low[v] = std::min(low[v], index[w]);
                continue;
            }
            call.pop_back();
            if (!call.empty()) low[call.back()] = std::min(low[call.back()], low[v]);
            if (low[v] == index[v]) {
                while (true) {
                    const i64 w = stack.back();
                    stack.pop_back();
                    on[w] = 0;
                    comp[w] = nc;
                    if (w == v) break;
                }
                nc++;
            }
        }
    }
    return nc;
}

// Columns [a, b) of an order whose lower neighbours all lie in [lo, b), filled at depth `level` of a nested
// dissection (INT_MAX: a whole subtree of it).  Ranges of a deeper level never depend on shallower ones, and ranges of
// one level are independent of each other.
struct NDRange {
    int level;
    i64 lo, a, b;
};

// perm (perm[new] = old) with the vertices of each component moved together, the components in increasing number,
// and the vertices of one component in their order in perm (a stable counting sort).  The fill of each component's
// own order is unchanged: no pattern entry joins two components.
// With `sub`, each range of positions in it is moved along; a range that the regrouping does not keep in one piece is
// dropped.
void group_by_component(std::vector<i64> &perm, const std::vector<i32> &comp, i64 nc,
                        std::vector<NDRange> *sub = nullptr) {
    const i64 n = (i64)perm.size();
    std::vector<i64> ptr(nc + 1, 0), out(n), newpos(sub ? n : 0);
    for (i64 k = 0; k < n; k++) ptr[comp[perm[k]] + 1]++;
    for (i64 c = 0; c < nc; c++) ptr[c + 1] += ptr[c];
    for (i64 k = 0; k < n; k++) {
        const i64 q = ptr[comp[perm[k]]]++;
        out[q] = perm[k];
        if (sub) newpos[k] = q;
    }
    perm.swap(out);
    if (sub) {
        std::vector<NDRange> moved;
        for (auto &r : *sub)
            if (r.b > r.lo && newpos[r.b - 1] - newpos[r.lo] == r.b - 1 - r.lo) {
                const i64 lo = newpos[r.lo];
                moved.push_back(NDRange{r.level, lo, lo + (r.a - r.lo), lo + (r.b - r.lo)});
            }
        sub->swap(moved);
    }
}

// ===== nested dissection on level structures =====
//
// A work item is a vertex subset, held as the subgraph it induces, that owns the output positions [hi - size, hi).
// Each item carries its own compact adjacency, so a search reads only the item's edges and the workers share no
// per-vertex arrays.  A connected item is split by one level of a breadth-first level structure rooted at a
// pseudo-peripheral vertex (George & Liu, "Computer Solution of Large Sparse Positive Definite Systems", 1981):
// the level with the fewest vertices among those leaving at least 35% of the item on each side.  The separator
// takes the last positions; the two sides recurse.  Small items are ordered by minimum degree.

struct ND {
    // A work item: the subgraph induced by its vertices in a local numbering (local vertex v is G's glob[v]; its
    // neighbours inside the item are adj[xadj[v] .. xadj[v + 1]), in the order of G's lists).  The whole graph is
    // the first item and is read from G itself.
    struct Item {
        std::vector<i64> xadj_s;
        std::vector<i32> adj_s, glob_s;
        bool whole = false;
        i64 m = 0, hi = 0;
    };
    // per worker, indexed by local vertex: BFS queue and levels (-1 outside a search), side / component of each
    // vertex and its index in the item it goes to
    struct Scratch {
        std::vector<i32> queue, level, side, cid;
        std::vector<i64> lptr, lptr2;
        explicit Scratch(i64 n) : queue(n + 1), level(n, -1), side(n), cid(n) {}   // queue: one slot past the end
    };
    const Adj &G;
    int leaf;
    std::vector<i64> order;   // order[k] = vertex eliminated k-th
    // Where each position was ordered: columns [a, b) of `order`, whose lower neighbours all lie in [lo, b), were
    // filled at depth `level` of the dissection (one entry per item split at the top, its separator), or hold a whole
    // subtree of it (level INT_MAX).  Entries of a deeper level never depend on shallower ones.
    using Range = NDRange;
    std::vector<Range> ranges;

    ND(const Adj &g, int leaf_) : G(g), leaf(std::max(2, std::min(leaf_, 64))), order(g.n, -1) {}

    const i64 *X(const Item &it) const { return it.whole ? G.xadj.data() : it.xadj_s.data(); }
    const i32 *A(const Item &it) const { return it.whole ? G.adj.data() : it.adj_s.data(); }
    i64 glob(const Item &it, i32 v) const { return it.whole ? (i64)v : (i64)it.glob_s[v]; }

    // BFS inside the item from root; returns the number of levels; fills queue[0..cnt), level[] and the level
    // pointers (a BFS visits the levels in order)
    int bfs(const Item &it, Scratch &s, i32 root, i64 &cnt, std::vector<i64> &lptr) const {
        const i64 *xa = X(it);
        const i32 *ad = A(it);
        i32 *queue = s.queue.data(), *level = s.level.data();
        lptr.clear();
        lptr.push_back(0);
        cnt = 0;
        queue[cnt++] = root;
        level[root] = 0;
        i64 head = 0;
        i32 cur = 0;
        while (head < cnt) {
            const i32 v = queue[head];
            if (level[v] != cur) {
                lptr.push_back(head);
                cur = level[v];
            }
            head++;
            const i32 lv = cur + 1;
            // branch-free: every neighbour is written at the queue's end, and the end moves past it only when it was
            // not visited yet (a neighbour list has no repeats)
            for (i64 p = xa[v]; p < xa[v + 1]; p++) {
                const i32 u = ad[p];
                const i32 lu = level[u];
                const bool fresh = lu < 0;
                queue[cnt] = u;
                level[u] = fresh ? lv : lu;
                cnt += fresh;
            }
        }
        lptr.push_back(cnt);
        return (int)lptr.size() - 1;
    }

    static void clear_levels(Scratch &s, i64 cnt) {
        for (i64 k = 0; k < cnt; k++) s.level[s.queue[k]] = -1;
    }

    // minimum degree on a small item (at most 64 vertices): explicit elimination graph in bit masks; ties go to the
    // vertex listed first
    void md_leaf(const Item &it, i64 lo) {
        const int m = (int)it.m;
        const i64 *xa = X(it);
        const i32 *ad = A(it);
        uint64_t mask[64];
        for (int a = 0; a < m; a++) {
            mask[a] = 0;
            for (i64 p = xa[a]; p < xa[a + 1]; p++) mask[a] |= uint64_t(1) << ad[p];
        }
        uint64_t alive = m == 64 ? ~uint64_t(0) : ((uint64_t(1) << m) - 1);
        for (int k = 0; k < m; k++) {
            int best = -1, bd = 1 << 30;
            for (uint64_t rest = alive; rest; rest &= rest - 1) {   // alive vertices in increasing index
                const int a = __builtin_ctzll(rest);
                const int d = __builtin_popcountll(mask[a] & alive);
                if (d < bd) { bd = d; best = a; }
            }
            const uint64_t nb = mask[best] & alive & ~(uint64_t(1) << best);
            for (uint64_t rest = nb; rest; rest &= rest - 1) {
                const int a = __builtin_ctzll(rest);
                mask[a] |= nb & ~(uint64_t(1) << a);
            }
            alive &= ~(uint64_t(1) << best);
            order[lo + k] = glob(it, best);
        }
    }

    // the item of the vertices `list` (in that order) of `it`: those with side[v] == code, local index cid[v]
    Item extract(const Item &it, const Scratch &s, const std::vector<i32> &list, i32 code, i64 hi) const {
        const i64 *xa = X(it);
        const i32 *ad = A(it);
        Item c;
        c.m = (i64)list.size();
        c.hi = hi;
        c.glob_s.resize(c.m);
        c.xadj_s.resize(c.m + 1);
        i64 deg = 0;
        for (i32 v : list) deg += xa[v + 1] - xa[v];
        c.adj_s.resize(deg);
        i64 w = 0;
        c.xadj_s[0] = 0;
        for (i64 k = 0; k < c.m; k++) {
            const i32 v = list[k];
            c.glob_s[k] = (i32)glob(it, v);
            for (i64 p = xa[v]; p < xa[v + 1]; p++) {
                const i32 u = ad[p];
                if (s.side[u] == code) c.adj_s[w++] = s.cid[u];
            }
            c.xadj_s[k + 1] = w;
        }
        c.adj_s.resize(w);
        return c;
    }

    // One item: split it (components, or sides + separator) or order it (leaf); new items go to `out`.  Returns
    // the positions of `order` filled by this item itself (its separator, or all of it).
    std::pair<i64, i64> process(const Item &it, Scratch &s, std::vector<Item> &out) {
        const i64 sz = it.m;
        if (sz == 0) return {it.hi, it.hi};
        const i64 lo = it.hi - sz;
        if (sz <= leaf) {
            md_leaf(it, lo);
            return {lo, it.hi};
        }
        const i64 *xa = X(it);
        const i32 *ad = A(it);
        std::vector<i64> &lptr = s.lptr;
        // connected components of the item; the first breadth-first search starts at the item's first vertex and
        // the pseudo-peripheral search below moves the root to the far end
        i64 cnt;
        i32 root = 0;
        int nlev = bfs(it, s, root, cnt, lptr);
        if (cnt < sz) {
            // disconnected: every component becomes an item of its own, the first one found taking the last
            // positions; a component lists its vertices in the order its search visits them
            std::vector<std::vector<i32>> comps;
            comps.emplace_back(s.queue.begin(), s.queue.begin() + cnt);
            for (i32 v = 0; v < (i32)sz; v++) {
                if (s.level[v] >= 0) continue;
                i64 c2;
                bfs(it, s, v, c2, s.lptr2);
                comps.emplace_back(s.queue.begin(), s.queue.begin() + c2);
            }
            for (i32 v = 0; v < (i32)sz; v++) s.level[v] = -1;
            for (i32 c = 0; c < (i32)comps.size(); c++)
                for (i64 k = 0; k < (i64)comps[c].size(); k++) {
                    s.side[comps[c][k]] = c;
                    s.cid[comps[c][k]] = (i32)k;
                }
            i64 hi = it.hi;
            for (i32 c = 0; c < (i32)comps.size(); c++) {
                out.push_back(extract(it, s, comps[c], c, hi));
                hi -= (i64)comps[c].size();
            }
            return {it.hi, it.hi};
        }
        // pseudo-peripheral root: restart from a vertex of minimum degree in the last level while the level
        // structure gets deeper; a structure as deep as the current one is kept as it is
        for (int iter = 0; iter < 4; iter++) {
            i32 best = -1;
            i64 bd = 1LL << 60;
            for (i64 k = lptr[nlev - 1]; k < lptr[nlev]; k++) {
                const i32 v = s.queue[k];
                const i64 d = xa[v + 1] - xa[v];
                if (d < bd) { bd = d; best = v; }
            }
            clear_levels(s, cnt);
            i64 cnt2;
            const int nlev2 = bfs(it, s, best, cnt2, s.lptr2);
            if (nlev2 >= nlev) {
                const bool deeper = nlev2 > nlev;
                nlev = nlev2;
                lptr.swap(s.lptr2);
                cnt = cnt2;
                root = best;
                if (!deeper) break;
            } else {
                clear_levels(s, cnt2);
                nlev = bfs(it, s, root, cnt, lptr);
                break;
            }
        }
        if (nlev < 3) {
            // too shallow to dissect: minimum degree would be too slow on a large item; natural order
            for (i64 k = 0; k < cnt; k++) order[lo + k] = glob(it, s.queue[k]);
            clear_levels(s, cnt);
            return {lo, it.hi};
        }
        // the separator level
        int sl = -1;
        i64 ssz = 1LL << 60, sbal = 1LL << 60;
        const i64 minside = (i64)(0.35 * (double)sz);
        for (int k = 1; k + 1 < nlev; k++) {
            i64 a = lptr[k], sn = lptr[k + 1] - lptr[k], b = sz - a - sn;
            if (a < minside || b < minside) continue;
            i64 bal = a > b ? a - b : b - a;
            if (sn < ssz || (sn == ssz && bal < sbal)) { ssz = sn; sbal = bal; sl = k; }
        }
        if (sl < 0) {
            for (int k = 1; k + 1 < nlev; k++)
                if (lptr[k + 1] * 2 >= sz) { sl = k; break; }
            if (sl < 0) sl = nlev / 2;
        }
        // sides: A (0) = levels < sl, B (1) = levels > sl, S (2) = level sl; then separator vertices that touch
        // only one side move to it, one after another (a minimal separator)
        for (i64 k = 0; k < cnt; k++) {
            const i32 v = s.queue[k];
            s.side[v] = s.level[v] < sl ? 0 : (s.level[v] > sl ? 1 : 2);
        }
        clear_levels(s, cnt);
        std::vector<i32> keep;
        for (i64 k = lptr[sl]; k < lptr[sl + 1]; k++) {
            const i32 v = s.queue[k];
            bool ta = false, tb = false;
            for (i64 p = xa[v]; p < xa[v + 1]; p++) {
                const i32 sd = s.side[ad[p]];
                ta |= sd == 0;
                tb |= sd == 1;
            }
            if (!tb) s.side[v] = 0;
            else if (!ta) s.side[v] = 1;
            else keep.push_back(v);
        }
        std::vector<i32> Av, Bv;
        for (i32 v = 0; v < (i32)sz; v++) {
            if (s.side[v] == 0) {
                s.cid[v] = (i32)Av.size();
                Av.push_back(v);
            } else if (s.side[v] == 1) {
                s.cid[v] = (i32)Bv.size();
                Bv.push_back(v);
            }
        }
        const i64 ns = (i64)keep.size();
        for (i64 k = 0; k < ns; k++) order[it.hi - ns + k] = glob(it, keep[k]);
        const i64 na = (i64)Av.size();
        out.push_back(extract(it, s, Bv, 1, it.hi - ns));
        out.push_back(extract(it, s, Av, 0, lo + na));
        return {it.hi - ns, it.hi};
    }

    // The top of the dissection runs level by level, the large items of one level in parallel (an item is large when
    // it holds more than a quarter of a thread's share of the vertices), until none is large; then the threads take
    // the remaining items largest first and order each one's whole subtree themselves (depth first).  Every item writes its own positions of `order`, so the result does not
    // depend on the threads.
    void run(int nthreads) {
        std::vector<Item> level;
        {
            Item all;
            all.whole = true;
            all.m = G.n;
            all.hi = G.n;
            level.push_back(std::move(all));
        }
        const i64 big = std::max<i64>(2048, G.n / (4 * (i64)std::max(1, nthreads)));
        std::vector<Scratch *> scratch(std::max(1, nthreads), nullptr);
        auto scr = [&](int t) -> Scratch & {
            if (!scratch[t]) scratch[t] = new Scratch(G.n);
            return *scratch[t];
        };
        double tl = now();
        for (int depth = 0; nthreads > 1; depth++) {
            bool any = false;
            for (auto &it : level) any |= it.m >= big;
            if (!any) break;
            std::vector<std::vector<Item>> outs(level.size());
            std::vector<Range> own(level.size(), Range{depth, 0, 0, 0});
            std::atomic<size_t> next(0);
            pool_run((int)std::min<size_t>(nthreads, level.size()), [&](int t) {
                for (size_t k; (k = next.fetch_add(1)) < level.size();) {
                    if (level[k].m >= big) {
                        const auto ab = process(level[k], scr(t), outs[k]);
                        own[k] = Range{depth, level[k].hi - level[k].m, ab.first, ab.second};
                    } else {
                        outs[k].push_back(std::move(level[k]));
                    }
                }
            });
            for (auto &r : own)
                if (r.b > r.a) ranges.push_back(r);
            stage("      dissection depth", tl);
            std::vector<Item> nl;
            for (auto &o : outs)
                for (auto &it : o) nl.push_back(std::move(it));
            level.swap(nl);
        }
        std::sort(level.begin(), level.end(), [](const Item &a, const Item &b) { return a.m > b.m; });
        for (auto &it : level)
            if (it.m > 0) ranges.push_back(Range{INT_MAX, it.hi - it.m, it.hi - it.m, it.hi});
        std::atomic<size_t> next(0);
        pool_run(std::max(1, (int)std::min<size_t>(nthreads, level.size())), [&](int t) {
            Scratch &s = scr(t);
            std::vector<Item> out, local;
            for (size_t k; (k = next.fetch_add(1)) < level.size();) {
                local.clear();
                local.push_back(std::move(level[k]));
                while (!local.empty()) {
                    Item cur = std::move(local.back());
                    local.pop_back();
                    out.clear();
                    process(cur, s, out);
                    for (auto &o : out) local.push_back(std::move(o));
                }
            }
        });
        stage("      dissection subtrees", tl);
        for (Scratch *p : scratch) delete p;
    }
};

// ===== approximate minimum degree (Amestoy, Davis & Duff, SIAM J. Matrix Anal. Appl. 17(4):886-905, 1996) =====
//
// The quotient graph: eliminating a pivot turns it into an element, the clique of its remaining neighbours (Lme),
// which absorbs the elements adjacent to the pivot.  A variable's list holds its adjacent elements first, then its
// adjacent variables.  Variables whose lists become equal merge into supervariables (nv = size); a variable left
// adjacent to the new element only is eliminated with the pivot (mass elimination).  The degree of a variable is
// the AMD upper bound min(n - k, d_old + |Lme \ i|, |A_i \ i| + |Lme \ i| + sum_e |Le \ Lme|), where |Le \ Lme| comes
// from one pass over the elements adjacent to Lme.  The pivot is a variable of least degree.  Returns the
// elimination order (order[k] = vertex eliminated k-th).
std::vector<i64> amd_order(const Adj &G) {
    const i64 n = G.n;
    std::vector<i64> order;
    order.reserve(n);
    if (n == 0) return order;
    std::vector<i32> iw(G.adj.begin(), G.adj.end());   // lists; element lists are appended at the end
    std::vector<i64> pe(G.xadj.begin(), G.xadj.end() - 1);
    std::vector<i32> len(n), elen(n, 0), nv(n, 1), degree(n);
    std::vector<char> isel(n, 0), dead(n, 0);            // node is an element; node absorbed (element or variable)
    std::vector<i64> w(n, 0);                           // element marks: |Le \ Lme| + wflg
    std::vector<i32> head(n + 1, -1), next(n, -1), last(n, -1);
    std::vector<i32> gnext(n, -1), gtail(n);            // members of each supervariable / pivot group
    std::vector<i32> mark(n, -1);
    std::vector<i64> hkey(n, 0);
    for (i64 i = 0; i < n; i++) {
        len[i] = (i32)(G.xadj[i + 1] - G.xadj[i]);
        degree[i] = len[i];
        gtail[i] = (i32)i;
    }
    auto dl_insert = [&](i32 i, i32 d) {
        next[i] = head[d];
        last[i] = -1;
        if (head[d] >= 0) last[head[d]] = i;
        head[d] = i;
    };
    auto dl_remove = [&](i32 i) {
        if (last[i] >= 0) next[last[i]] = next[i];
        else head[degree[i]] = next[i];
        if (next[i] >= 0) last[next[i]] = last[i];
    };
    auto gappend = [&](i32 a, i32 b) {   // members of b after those of a
        gnext[gtail[a]] = b;
        gtail[a] = gtail[b];
    };
    for (i64 i = 0; i < n; i++) dl_insert((i32)i, degree[i]);
    i64 nel = 0, mindeg = 0, wflg = 1;
    std::vector<i32> lme, bucket_members;
    while (nel < n) {
        while (mindeg <= n && head[mindeg] < 0) mindeg++;
        const i32 me = head[mindeg];
        dl_remove(me);
        i32 nvpiv = nv[me];
        nv[me] = -nvpiv;
        // 1. Lme: the principal variables of me's list and of its elements, which me absorbs
        lme.clear();
        i64 degme = 0;
        auto take = [&](i32 i) {
            if (isel[i] || dead[i] || nv[i] <= 0) return;   // an element, absorbed, already in Lme, or me
            degme += nv[i];
            nv[i] = -nv[i];
            dl_remove(i);
            lme.push_back(i);
        };
        for (i32 q = 0; q < len[me]; q++) {
            const i32 x = iw[pe[me] + q];
            if (q < elen[me]) {
                if (dead[x]) continue;
                for (i32 r = 0; r < len[x]; r++) take(iw[pe[x] + r]);
                dead[x] = 1;   // absorbed into me
                w[x] = 0;
            } else {
                take(x);
            }
        }
        isel[me] = 1;
        // 2. |Le \ Lme| for the elements adjacent to Lme
        for (i32 i : lme) {
            const i32 nvi = -nv[i];
            for (i32 q = 0; q < elen[i]; q++) {
                const i32 e = iw[pe[i] + q];
                if (dead[e] || e == me) continue;
                if (w[e] >= wflg) w[e] -= nvi;
                else w[e] = degree[e] + wflg - nvi;
            }
        }
        // 3. new lists and degree bounds of the variables of Lme; mass elimination
        std::vector<i32> &keep = bucket_members;
        i64 kept_lme = 0;
        for (i32 i : lme) {
            const i32 nvi = -nv[i];
            const i64 p0 = pe[i];
            i64 deg = 0, h = me;
            keep.clear();
            for (i32 q = 0; q < elen[i]; q++) {
                const i32 e = iw[p0 + q];
                if (dead[e] || e == me) continue;
                const i64 we = w[e] - wflg;
                if (we > 0) {
                    deg += we;
                    keep.push_back(e);
                    h += e;
                } else {
                    dead[e] = 1;   // Le within Lme: absorbed into me (aggressive absorption)
                    w[e] = 0;
                }
            }
            const i32 ne = (i32)keep.size();
            for (i32 q = elen[i]; q < len[i]; q++) {
                const i32 j = iw[p0 + q];
                if (isel[j] || dead[j] || nv[j] <= 0) continue;   // elements, absorbed, Lme (covered by me)
                deg += nv[j];
                keep.push_back(j);
                h += j;
            }
            if (keep.empty()) {
                // adjacent to me only: eliminated together with the pivot
                dead[i] = 1;
                nvpiv += nvi;
                nv[i] = 0;
                gappend(me, i);
                continue;
            }
            iw[p0] = me;
            for (i32 q = 0; q < (i32)keep.size(); q++) iw[p0 + 1 + q] = keep[q];
            len[i] = (i32)keep.size() + 1;
            elen[i] = ne + 1;
            degree[i] = (i32)std::min<i64>(degree[i], deg);   // the two bounds without |Lme \ i|
            hkey[i] = h % n;
            lme[kept_lme++] = i;
        }
        lme.resize(kept_lme);
        // 4. supervariables: variables of Lme with equal lists merge (candidates share a hash of their lists)
        if (lme.size() > 1) {
            std::sort(lme.begin(), lme.end(), [&](i32 a, i32 b) { return hkey[a] != hkey[b] ? hkey[a] < hkey[b] : a < b; });
            for (size_t a = 0; a < lme.size(); a++) {
                const i32 i = lme[a];
                if (dead[i]) continue;
                bool marked = false;
                for (size_t b = a + 1; b < lme.size() && hkey[lme[b]] == hkey[i]; b++) {
                    const i32 j = lme[b];
                    if (dead[j] || len[j] != len[i] || elen[j] != elen[i]) continue;
                    if (!marked) {
                        for (i32 q = 0; q < len[i]; q++) mark[iw[pe[i] + q]] = i;
                        marked = true;
                    }
                    bool same = true;
                    for (i32 q = 0; q < len[j] && same; q++) same = mark[iw[pe[j] + q]] == i;
                    if (!same) continue;
                    nv[i] += nv[j];   // both negative while in Lme
                    nv[j] = 0;
                    dead[j] = 1;
                    degree[i] = std::min(degree[i], degree[j]);
                    gappend(i, j);
                }
                if (marked)
                    for (i32 q = 0; q < len[i]; q++) mark[iw[pe[i] + q]] = -1;
            }
        }
        // 5. the element me and the final degrees of its variables
        nel += nvpiv;
        i64 degme2 = 0;
        const i64 start = (i64)iw.size();
        for (i32 i : lme)
            if (!dead[i]) {
                degme2 += -nv[i];
                iw.push_back(i);
            }
        for (i64 q = start; q < (i64)iw.size(); q++) {
            const i32 i = iw[q];
            const i32 nvi = -nv[i];
            nv[i] = nvi;
            const i64 d = std::min<i64>({(i64)degree[i] + degme2 - nvi, n - nel - nvi});
            degree[i] = (i32)std::max<i64>(d, 0);
            dl_insert(i, degree[i]);
            mindeg = std::min<i64>(mindeg, degree[i]);
        }
        pe[me] = start;
        len[me] = (i32)((i64)iw.size() - start);
        elen[me] = 0;
        degree[me] = (i32)degme2;
        nv[me] = nvpiv;
        if (len[me] == 0) dead[me] = 1;
        for (i32 m = me; m >= 0; m = gnext[m]) order.push_back(m);
        wflg += n + 1;
    }
    return order;
}

// ===== elimination tree and postorder (Liu 1986, path compression) =====
//
// The columns of a nested-dissection item (a range of positions holding a whole subtree of the dissection) have
// their lower neighbours inside the item: the vertices ordered before it lie in other items, which only the later
// separators touch.  So Liu's algorithm runs on the whole subtrees at the bottom in parallel, then on the separators
// of the items above them, one depth of the dissection at a time (deepest first, the items of one depth in
// parallel); each item writes only its own nodes, and every column still sees the columns before it in its item, so
// the tree is the one a single pass over all columns gives.

// post_perm: a postorder of the elimination tree of perm (the children of a node in increasing order);
// post_parent: the elimination tree in the postorder's labels.  sub: the nested dissection's ranges of perm, or null.
void etree_postorder(const Adj &G, const std::vector<i64> &perm, std::vector<i64> &post_perm,
                     std::vector<i64> &post_parent, const std::vector<NDRange> *sub = nullptr, int threads = 1) {
    const i64 n = G.n;
    double ts = now();
    std::vector<i64> invp(n);
    parallel_for(n, threads, [&](i64 a, i64 b) {
        for (i64 k = a; k < b; k++) invp[perm[k]] = k;
    });
    std::vector<i64> parent(n, -1), anc(n, -1);
    // Liu's algorithm on the columns [j0, j1); false when a lower neighbour lies below lo
    auto cols = [&](i64 j0, i64 j1, i64 lo) {
        for (i64 j = j0; j < j1; j++) {
            const i64 v = perm[j];
            for (i64 p = G.xadj[v]; p < G.xadj[v + 1]; p++) {
                const i64 i = invp[G.adj[p]];
                if (i >= j) continue;
                if (i < lo) return false;
                i64 r = i;
                while (anc[r] != -1 && anc[r] != j) {
                    const i64 t = anc[r];
                    anc[r] = j;
                    r = t;
                }
                if (anc[r] == -1) {
                    anc[r] = j;
                    parent[r] = j;
                }
            }
        }
        return true;
    };
    bool done = false;
    if (sub && threads > 1 && sub->size() > 1) {
        // the ranges must cover every column once
        std::vector<NDRange> rs(*sub);
        std::sort(rs.begin(), rs.end(), [](const NDRange &x, const NDRange &y) { return x.a < y.a; });
        bool ok = true;
        i64 at = 0;
        for (auto &r : rs) {
            ok &= r.a == at && r.b > r.a && r.lo >= 0 && r.lo <= r.a;
            at = r.b;
        }
        ok &= at == n;
        if (ok) {
            // deepest level first; the ranges of one level in parallel
            std::stable_sort(rs.begin(), rs.end(), [](const NDRange &x, const NDRange &y) { return x.level > y.level; });
            std::atomic<bool> bad(false);
            stage("      etree setup", ts);
            for (size_t g0 = 0; g0 < rs.size() && !bad;) {
                size_t g1 = g0;
                while (g1 < rs.size() && rs[g1].level == rs[g0].level) g1++;
                std::atomic<size_t> next(g0);
                pool_run((int)std::min<size_t>(threads, g1 - g0), [&](int) {
                    for (size_t k; (k = next.fetch_add(1)) < g1;)
                        if (!cols(rs[k].a, rs[k].b, rs[k].lo)) bad = true;
                });
                stage(rs[g0].level == INT_MAX ? "      etree subtrees" : "      etree depth", ts);
                g0 = g1;
            }
            if (!bad) {
                done = true;
            } else {
                std::fill(parent.begin(), parent.end(), -1);
                std::fill(anc.begin(), anc.end(), -1);
            }
        }
    }
    if (!done) cols(0, n, 0);
    stage(done ? "    etree (dissection ranges)" : "    etree", ts);
    // postorder with the children of a node in increasing order, roots in increasing order: the subtree of j takes
    // size[j] consecutive labels starting after its earlier siblings' subtrees, j last
    std::vector<i64> &size = anc, &post = invp;   // reused
    std::fill(size.begin(), size.end(), 1);
    for (i64 j = 0; j < n; j++)
        if (parent[j] >= 0) size[parent[j]] += size[j];
    stage("    postorder sizes", ts);
    std::vector<i64> start(n), acc(n, 0);
    i64 roots = 0;
    for (i64 j = 0; j < n; j++) {   // offset of j among its siblings
        if (parent[j] >= 0) {
            start[j] = acc[parent[j]];
            acc[parent[j]] += size[j];
        } else {
            start[j] = roots;
            roots += size[j];
        }
    }
    for (i64 j = n - 1; j >= 0; j--) {
        if (parent[j] >= 0) start[j] += start[parent[j]];
        post[j] = start[j] + size[j] - 1;
    }
    stage("    postorder starts", ts);
    post_perm.resize(n);
    post_parent.resize(n);
    parallel_for(n, threads, [&](i64 a, i64 b) {
        for (i64 j = a; j < b; j++) {
            post_perm[post[j]] = perm[j];
            post_parent[post[j]] = parent[j] >= 0 ? post[parent[j]] : -1;
        }
    });
    stage("    postorder", ts);
}

// ===== column counts of L (Gilbert, Ng & Peyton, "An efficient algorithm to compute row and column counts for
// sparse Cholesky factorization", SIMAX 1994) =====
//
// The labels are a postorder of the elimination tree.  L[i, j] != 0 iff j lies in the row subtree T_i, whose leaves
// are among the j < i with A[i, j] != 0.  Every node counts +1; for each row subtree, each leaf j (a neighbour of i
// that is not a descendant of the previous leaf, visiting the neighbours in increasing order) adds +1 at j and -1 at
// the least common ancestor of j and the previous leaf; each leaf of the tree counts 1 and each non-root node
// subtracts 1 from its parent.  The column count of j (with the diagonal) is then the sum of these weights over the
// subtree of j.
//
// The rows are independent, so they run in parallel.  In a postorder the least common ancestor of a < b is the first
// ancestor of a labelled b or more; it is found by climbing with jump pointers (Myers, "An applicative random-access
// stack", IPL 17, 1983: each node keeps its parent and one longer jump, so a monotone search along the path to the
// root takes O(log depth) steps).
void column_counts(const Adj &G, const std::vector<i64> &perm, const std::vector<i64> &parent, std::vector<i64> &cc,
                   int threads = 1) {
    const i64 n = G.n;
    double ts = now();
    std::vector<i64> invp(n);
    parallel_for(n, threads, [&](i64 a, i64 b) {
        for (i64 k = a; k < b; k++) invp[perm[k]] = k;
    });
    stage("      cc invp", ts);
    // first descendant of every node (a subtree is the range [first[j], j]), depth and jump pointer
    std::vector<i64> first(n), depth(n), jump(n);
    for (i64 j = 0; j < n; j++) first[j] = j;
    for (i64 j = 0; j < n; j++)
        if (parent[j] >= 0) first[parent[j]] = std::min(first[parent[j]], first[j]);
    for (i64 j = n - 1; j >= 0; j--) {
        const i64 p = parent[j];
        if (p < 0) {
            depth[j] = 0;
            jump[j] = j;
            continue;
        }
        depth[j] = depth[p] + 1;
        const i64 jp = jump[p];
        jump[j] = (jp != p && depth[p] - depth[jp] == depth[jp] - depth[jump[jp]]) ? jump[jp] : p;
    }
    stage("      cc jump", ts);
    // the first ancestor of a (a < b) labelled b or more
    auto lca = [&](i64 a, i64 b) {
        while (true) {
            const i64 s = jump[a];
            if (s != a && s < b) {
                a = s;
                continue;
            }
            const i64 p = parent[a];
            if (p < 0 || p >= b) return p;
            a = p;
        }
    };
    std::vector<i64> delta(n, 0);
    for (i64 j = 0; j < n; j++) {
        if (first[j] == j) delta[j]++;   // leaves of the elimination tree
        if (parent[j] >= 0) delta[parent[j]]--;
    }
    stage("      cc delta", ts);
    // rows in blocks on the threads, each adding into its own copy of the weights (or, for a very large tree, into the
    // shared ones with atomic adds)
    const int T = (int)std::max<i64>(1, std::min<i64>(threads, n / 1024));
    const bool own = (double)n * T <= (double)(1 << 26);
    std::vector<std::vector<i32>> part(own && T > 1 ? T : 0);
    pool_run(T, [&](int t) {
        i32 *mine = nullptr;
        if (!part.empty()) {
            part[t].assign(n, 0);
            mine = part[t].data();
        }
        auto add = [&](i64 k, i64 v) {
            if (T == 1) delta[k] += v;
            else if (mine) mine[k] += (i32)v;
            else std::atomic_ref<i64>(delta[k]).fetch_add(v, std::memory_order_relaxed);
        };
        std::vector<i64> nb;
        for (i64 i = n * t / T; i < n * (t + 1) / T; i++) {
            nb.clear();
            const i64 v = perm[i];
            for (i64 p = G.xadj[v]; p < G.xadj[v + 1]; p++) {
                const i64 j = invp[G.adj[p]];
                if (j < i) nb.push_back(j);
            }
            std::sort(nb.begin(), nb.end());
            i64 maxfirst = -1, jprev = -1;
            for (i64 j : nb) {
                if (first[j] <= maxfirst) continue;   // j is no new leaf of the row subtree of i
                maxfirst = first[j];
                add(j, 1);
                if (jprev >= 0) {
                    const i64 q = lca(jprev, j);   // exists: jprev and j both descend from i
                    if (q >= 0) add(q, -1);
                }
                jprev = j;
            }
        }
    });
    if (!part.empty())
        parallel_for(n, threads, [&](i64 a, i64 b) {
            for (int t = 0; t < T; t++) {
                const i32 *mine = part[t].data();
                for (i64 k = a; k < b; k++) delta[k] += mine[k];
            }
        });
    stage("      cc rows", ts);
    cc = delta;
    for (i64 j = 0; j < n; j++)
        if (parent[j] != -1) cc[parent[j]] += cc[j];
    stage("    column counts", ts);
}

// ===== supernodal symbolic factorization for (perm, Rptr) =====
//
// sep(f) = (adj(res(f)) and the separators of f's children) restricted to vertices after res(f); parent(f) is the
// front holding min sep(f).  Fronts must be in a postorder of the resulting tree.
std::string supernodal(const Adj &G, const std::vector<i64> &perm, const std::vector<i64> &Rptr,
                       std::vector<i64> &Sptr, std::vector<i32> &Stgt, std::vector<i64> &parent) {
    const i64 n = G.n, nf = (i64)Rptr.size() - 1;
    std::vector<i64> invp(n), idx(n);
    for (i64 k = 0; k < n; k++) invp[perm[k]] = k;
    for (i64 f = 0; f < nf; f++)
        for (i64 v = Rptr[f]; v < Rptr[f + 1]; v++) idx[v] = f;
    std::vector<i64> mark(n, -1), chead(nf, -1), cnext(nf, -1), ctail(nf, -1);
    Sptr.assign(nf + 1, 0);
    Stgt.clear();
    parent.assign(nf, -1);
    std::vector<i32> buf;
    for (i64 f = 0; f < nf; f++) {
        const i64 r0 = Rptr[f], r1 = Rptr[f + 1];
        buf.clear();
        for (i64 v = r0; v < r1; v++) {
            i64 ov = perm[v];
            for (i64 p = G.xadj[ov]; p < G.xadj[ov + 1]; p++) {
                i64 u = invp[G.adj[p]];
                if (u >= r1 && mark[u] != f) {
                    mark[u] = f;
                    buf.push_back((i32)u);
                }
            }
        }
        for (i64 c = chead[f]; c >= 0; c = cnext[c])
            for (i64 q = Sptr[c]; q < Sptr[c + 1]; q++) {
                i64 u = Stgt[q];
                if (u < r0) return "front structure is not a postorder of its tree";
                if (u >= r1 && mark[u] != f) {
                    mark[u] = f;
                    buf.push_back((i32)u);
                }
            }
        std::sort(buf.begin(), buf.end());
        Stgt.insert(Stgt.end(), buf.begin(), buf.end());
        Sptr[f + 1] = (i64)Stgt.size();
        if (!buf.empty()) {
            i64 p = idx[buf[0]];
            parent[f] = p;
            if (ctail[p] < 0) chead[p] = f;
            else cnext[ctail[p]] = f;
            ctail[p] = f;
        }
    }
    return "";
}

// The same with the front tree known in advance (parent[f] > f, fronts in postorder): disjoint subtrees are
// independent, so the fronts below a cut of the tree run on `threads` threads (one subtree after another, each in
// postorder, into per-thread buffers), then the fronts above the cut in postorder.  The result equals supernodal()'s.
std::string supernodal_tree(const Adj &G, const std::vector<i64> &perm, const std::vector<i64> &Rptr,
                            const std::vector<i64> &parent_in, int threads, std::vector<i64> &Sptr,
                            std::vector<i32> &Stgt, std::vector<i64> &parent) {
    const i64 n = G.n, nf = (i64)Rptr.size() - 1;
    if (threads <= 1 || nf < 64) return supernodal(G, perm, Rptr, Sptr, Stgt, parent);
    std::vector<i64> invp(n);
    for (i64 k = 0; k < n; k++) invp[perm[k]] = k;
    std::vector<i64> chead(nf, -1), cnext(nf, -1), ctail(nf, -1), first(nf), size(nf);
    for (i64 f = 0; f < nf; f++) {
        const i64 p = parent_in[f];
        if (p >= 0) {
            if (p <= f) return supernodal(G, perm, Rptr, Sptr, Stgt, parent);
            if (ctail[p] < 0) chead[p] = f;
            else cnext[ctail[p]] = f;
            ctail[p] = f;
        }
    }
    for (i64 f = 0; f < nf; f++) first[f] = f;
    for (i64 f = 0; f < nf; f++)
        if (parent_in[f] >= 0) first[parent_in[f]] = std::min(first[parent_in[f]], first[f]);
    for (i64 f = 0; f < nf; f++) size[f] = Rptr[f + 1] - Rptr[first[f]];   // vertices in the subtree
    // cut: split every subtree larger than n / (4 threads) into its children; the split fronts form the top
    const i64 limit = std::max<i64>(1, n / (4 * (i64)threads));
    std::vector<i64> tasks, stack;
    std::vector<char> top(nf, 0);
    for (i64 f = 0; f < nf; f++)
        if (parent_in[f] < 0) stack.push_back(f);
    while (!stack.empty()) {
        const i64 f = stack.back();
        stack.pop_back();
        if (size[f] <= limit || chead[f] < 0) {
            tasks.push_back(f);
        } else {
            top[f] = 1;
            for (i64 c = chead[f]; c >= 0; c = cnext[c]) stack.push_back(c);
        }
    }
    std::sort(tasks.begin(), tasks.end(), [&](i64 a, i64 b) { return size[a] > size[b]; });
    // per front: (buffer, offset, length) of its separator
    std::vector<int32_t> fbuf(nf, -1);
    std::vector<i64> foff(nf, 0), flen(nf, 0);
    std::vector<std::vector<i32>> bufs(threads), topsep(nf), marks(threads);
    constexpr int32_t TOP = -2;   // fbuf of a front above the cut: its separator is topsep[f]
    std::atomic<bool> bad(false);
    auto front = [&](i64 f, std::vector<i32> &out, int bid, std::vector<i32> &mark, std::vector<i32> &buf) {
        const i64 r0 = Rptr[f], r1 = Rptr[f + 1];
        buf.clear();
        for (i64 v = r0; v < r1; v++) {
            const i64 ov = perm[v];
            for (i64 q = G.xadj[ov]; q < G.xadj[ov + 1]; q++) {
                const i64 u = invp[G.adj[q]];
                if (u >= r1 && mark[u] != (i32)f) {
                    mark[u] = (i32)f;
                    buf.push_back((i32)u);
                }
            }
        }
        for (i64 c = chead[f]; c >= 0; c = cnext[c]) {
            const i32 *sc = fbuf[c] == TOP ? topsep[c].data() : bufs[fbuf[c]].data() + foff[c];
            for (i64 k = 0; k < flen[c]; k++) {
                const i64 u = sc[k];
                if (u < r0) bad = true;
                if (u >= r1 && mark[u] != (i32)f) {
                    mark[u] = (i32)f;
                    buf.push_back((i32)u);
                }
            }
        }
        std::sort(buf.begin(), buf.end());
        fbuf[f] = bid;
        foff[f] = bid == TOP ? 0 : (i64)out.size();
        flen[f] = (i64)buf.size();
        out.insert(out.end(), buf.begin(), buf.end());
    };
    double tst = now();
    std::atomic<i64> next(0);
    auto worker = [&](int t) {
        std::vector<i32> &mark = marks[t], buf;
        mark.assign(n, -1);
        while (true) {
            const i64 k = next.fetch_add(1);
            if (k >= (i64)tasks.size()) break;
            const i64 root = tasks[k];
            for (i64 f = first[root]; f <= root; f++) front(f, bufs[t], t, mark, buf);
        }
    };
    {
        pool_run(threads, worker);
    }
    stage("    separators below the cut", tst);
    {
        // above the cut: the fronts of one height (longest path down to the cut) are independent; heights in order
        std::vector<i64> height(nf, 0), hptr, hidx;
        i64 hmax = -1;
        for (i64 f = 0; f < nf; f++) {
            if (!top[f]) continue;
            for (i64 c = chead[f]; c >= 0; c = cnext[c])
                if (top[c]) height[f] = std::max(height[f], height[c] + 1);
            hmax = std::max(hmax, height[f]);
        }
        hptr.assign(hmax + 2, 0);
        for (i64 f = 0; f < nf; f++)
            if (top[f]) hptr[height[f] + 1]++;
        for (i64 h = 0; h <= hmax; h++) hptr[h + 1] += hptr[h];
        hidx.resize(hptr[hmax + 1]);
        {
            std::vector<i64> pos(hptr.begin(), hptr.end() - 1);
            for (i64 f = 0; f < nf; f++)
                if (top[f]) hidx[pos[height[f]]++] = f;
        }
        for (i64 h = 0; h <= hmax; h++) {
            std::atomic<i64> nx(hptr[h]);
            pool_run((int)std::min<i64>(threads, hptr[h + 1] - hptr[h]), [&](int t) {
                std::vector<i32> buf;
                for (i64 k; (k = nx.fetch_add(1)) < hptr[h + 1];) {
                    const i64 f = hidx[k];
                    front(f, topsep[f], TOP, marks[t], buf);
                }
            });
        }
    }
    stage("    separators above the cut", tst);
    if (bad) return "front structure is not a postorder of its tree";
    Sptr.assign(nf + 1, 0);
    for (i64 f = 0; f < nf; f++) Sptr[f + 1] = Sptr[f] + flen[f];
    Stgt.resize(Sptr[nf]);
    parallel_for(nf, threads, [&](i64 a, i64 b) {
        for (i64 f = a; f < b; f++) {
            const i32 *src = fbuf[f] == TOP ? topsep[f].data() : bufs[fbuf[f]].data() + foff[f];
            std::copy(src, src + flen[f], Stgt.begin() + Sptr[f]);
        }
    });
    // the tree the separators define must be the one given
    parent.assign(nf, -1);
    std::vector<i64> fof(n);
    for (i64 f = 0; f < nf; f++)
        for (i64 v = Rptr[f]; v < Rptr[f + 1]; v++) fof[v] = f;
    for (i64 f = 0; f < nf; f++) {
        parent[f] = flen[f] ? fof[Stgt[Sptr[f]]] : -1;
        if (parent[f] != parent_in[f]) return supernodal(G, perm, Rptr, Sptr, Stgt, parent);
    }
    return "";
}



// Work counts of a structure (the formulas of the reference's per-front costs): factor sum nn^3/3 + nn^2 na +
// nn na^2; star n * sum nn (na + (nn-1)/2) for X <- X L* plus sum |subtree(f)| nn (na + (nn-1)/2) for X <- U*;
// one right-hand side 2 sum nn (na + (nn-1)/2).
void work_counts(i64 n, const std::vector<i64> &Rptr, const std::vector<i64> &Sptr, const std::vector<i64> &parent,
                 double &factor, double &star, double &rhs, double &nnzL) {
    const i64 nf = (i64)Rptr.size() - 1;
    std::vector<i64> fdsc(nf);
    for (i64 f = 0; f < nf; f++) fdsc[f] = f;
    for (i64 f = 0; f < nf; f++)
        if (parent[f] >= 0) fdsc[parent[f]] = std::min(fdsc[parent[f]], fdsc[f]);
    factor = star = rhs = nnzL = 0;
    for (i64 f = 0; f < nf; f++) {
        double nn = (double)(Rptr[f + 1] - Rptr[f]), na = (double)(Sptr[f + 1] - Sptr[f]);
        double per = nn * (na + (nn - 1) / 2);
        double sub = (double)(Rptr[f + 1] - Rptr[fdsc[f]]);
        factor += nn * nn * nn / 3 + nn * nn * na + nn * na * na;
        star += (double)n * per + sub * per;
        rhs += 2 * per;
        nnzL += per;
    }
}

// The component structure of out (perm, Rptr, invp set) from the components of the old labels: Bptr, Fptr, comp,
// N by column and by row, the two level orders and the earliest ancestor rows.  "" or an error when the order does
// not keep each component's vertices together in increasing component number.
std::string components(i64 n, const i64 *colptr, const i64 *rowval, const std::vector<i32> &comp_old, i64 nB,
                       Symbolic &out) {
    const i64 nf = out.nf;
    out.nB = nB;
    out.comp.resize(n);
    for (i64 k = 0; k < n; k++) out.comp[k] = comp_old[out.perm[k]];
    for (i64 k = 1; k < n; k++)
        if (out.comp[k] < out.comp[k - 1]) return "the order does not group the strongly connected components";
    out.Bptr.assign(nB + 1, 0);
    for (i64 k = 0; k < n; k++) out.Bptr[out.comp[k] + 1]++;
    for (i64 c = 0; c < nB; c++) out.Bptr[c + 1] += out.Bptr[c];
    out.Fptr.assign(nB + 1, nf);
    for (i64 f = nf - 1; f >= 0; f--) out.Fptr[out.comp[out.Rptr[f]]] = f;
    for (i64 f = 0; f < nf; f++)
        if (out.comp[out.Rptr[f]] != out.comp[out.Rptr[f + 1] - 1]) return "a front spans two components";
    for (i64 c = nB - 1; c >= 0; c--)
        if (out.Fptr[c] > out.Fptr[c + 1]) out.Fptr[c] = out.Fptr[c + 1];
    // N by column (new labels), rows ascending, then by row
    out.Nptr.assign(n + 1, 0);
    for (i64 c = 0; c < n; c++) {
        const i64 j = out.invp[c];
        for (i64 p = colptr[c]; p < colptr[c + 1]; p++) {
            const i64 i = out.invp[rowval[p]];
            if (out.comp[i] == out.comp[j]) continue;
            if (out.comp[i] > out.comp[j]) return "internal error: an arc against the component order";
            out.Nptr[j + 1]++;
        }
    }
    for (i64 j = 0; j < n; j++) out.Nptr[j + 1] += out.Nptr[j];
    out.nN = out.Nptr[n];
    out.Nidx.resize(out.nN);
    out.Nsrc.resize(out.nN);
    {
        std::vector<i64> pos(out.Nptr.begin(), out.Nptr.end() - 1);
        for (i64 c = 0; c < n; c++) {
            const i64 j = out.invp[c];
            for (i64 p = colptr[c]; p < colptr[c + 1]; p++) {
                const i64 i = out.invp[rowval[p]];
                if (out.comp[i] == out.comp[j]) continue;
                out.Nidx[pos[j]] = (i32)i;
                out.Nsrc[pos[j]++] = p;
            }
        }
        std::vector<std::pair<i32, i64>> tmp;
        for (i64 j = 0; j < n; j++) {
            tmp.clear();
            for (i64 q = out.Nptr[j]; q < out.Nptr[j + 1]; q++) tmp.push_back({out.Nidx[q], out.Nsrc[q]});
            std::sort(tmp.begin(), tmp.end());
            for (i64 q = out.Nptr[j]; q < out.Nptr[j + 1]; q++) {
                out.Nidx[q] = tmp[q - out.Nptr[j]].first;
                out.Nsrc[q] = tmp[q - out.Nptr[j]].second;
            }
        }
    }
    // by row: a counting sort over the columns keeps each row's columns ascending
    out.NTptr.assign(n + 1, 0);
    for (i64 q = 0; q < out.nN; q++) out.NTptr[out.Nidx[q] + 1]++;
    for (i64 i = 0; i < n; i++) out.NTptr[i + 1] += out.NTptr[i];
    out.NTidx.resize(out.nN);
    out.NTsrc.resize(out.nN);
    {
        std::vector<i64> pos(out.NTptr.begin(), out.NTptr.end() - 1);
        for (i64 j = 0; j < n; j++)
            for (i64 q = out.Nptr[j]; q < out.Nptr[j + 1]; q++) {
                const i64 i = out.Nidx[q];
                out.NTidx[pos[i]] = (i32)j;
                out.NTsrc[pos[i]++] = out.Nsrc[q];
            }
    }
    out.lev_up.assign(nB, 0);
    out.lev_dn.assign(nB, 0);
    out.anc_lo.resize(nB);
    for (i64 c = 0; c < nB; c++) {
        out.anc_lo[c] = out.Bptr[c];
        for (i64 j = out.Bptr[c]; j < out.Bptr[c + 1]; j++)
            for (i64 q = out.Nptr[j]; q < out.Nptr[j + 1]; q++) {
                const i64 b = out.comp[out.Nidx[q]];
                out.lev_up[c] = std::max(out.lev_up[c], out.lev_up[b] + 1);
                out.anc_lo[c] = std::min(out.anc_lo[c], out.anc_lo[b]);
            }
    }
    for (i64 c = nB - 1; c >= 0; c--)
        for (i64 i = out.Bptr[c]; i < out.Bptr[c + 1]; i++)
            for (i64 q = out.NTptr[i]; q < out.NTptr[i + 1]; q++)
                out.lev_dn[c] = std::max(out.lev_dn[c], out.lev_dn[out.comp[out.NTidx[q]]] + 1);
    return "";
}

std::string finish(const Adj &G, i64 n, const i64 *colptr, const i64 *rowval, std::vector<i64> perm,
                   std::vector<i64> Rptr, Symbolic &out, const std::vector<i64> *tree = nullptr,
                   const std::vector<i32> *comp_old = nullptr, i64 nB = 1) {
    std::vector<i64> Sptr, parent;
    std::vector<i32> Stgt;
    double ts = now();
    std::string err = tree ? supernodal_tree(G, perm, Rptr, *tree, analysis_threads(n), Sptr, Stgt, parent)
                           : supernodal(G, perm, Rptr, Sptr, Stgt, parent);
    if (!err.empty()) return err;
    stage("  separators", ts);
    const i64 nf = (i64)Rptr.size() - 1;
    out.n = n;
    out.perm = std::move(perm);
    out.invp.assign(n, 0);
    for (i64 k = 0; k < n; k++) out.invp[out.perm[k]] = k;
    out.nf = nf;
    out.Rptr = std::move(Rptr);
    out.Sptr = std::move(Sptr);
    out.Stgt.assign(Stgt.begin(), Stgt.end());
    out.parent = std::move(parent);
    out.fdsc.resize(nf);
    for (i64 f = 0; f < nf; f++) out.fdsc[f] = f;
    for (i64 f = 0; f < nf; f++)
        if (out.parent[f] >= 0) out.fdsc[out.parent[f]] = std::min(out.fdsc[out.parent[f]], out.fdsc[f]);
    out.Dptr.assign(nf + 1, 0);
    out.Lptr.assign(nf + 1, 0);
    for (i64 f = 0; f < nf; f++) {
        i64 nn = out.Rptr[f + 1] - out.Rptr[f], na = out.Sptr[f + 1] - out.Sptr[f];
        out.Dptr[f + 1] = out.Dptr[f] + nn * nn;
        out.Lptr[f + 1] = out.Lptr[f] + nn * na;
    }
    out.nB = 1;
    out.nN = 0;
    out.Bptr = {0, n};
    out.Fptr = {0, nf};
    out.comp.clear();
    out.Nptr.assign(n + 1, 0);
    out.NTptr.assign(n + 1, 0);
    out.Nidx.clear(); out.Nsrc.clear(); out.NTidx.clear(); out.NTsrc.clear();
    out.lev_up.assign(1, 0);
    out.lev_dn.assign(1, 0);
    out.anc_lo.assign(1, 0);
    if (comp_old && nB > 1) {
        err = components(n, colptr, rowval, *comp_old, nB, out);
        if (!err.empty()) return err;
    }
    // where each stored entry (i, j) lands (new labels): the front f of min(i, j), at the local positions of i and j
    // in bag(f) = res(f) then sep(f); an arc between two components is in N instead (entry_front = -1).  Entries are
    // grouped by front (counting sort), and each front's bag positions are scattered into a per-thread map over the
    // vertices that its entries then read; in parallel over fronts.
    stage("  structure copies", ts);
    out.nnz = colptr[n];
    const i64 nnz = out.nnz;
    out.entry_front.resize(nnz);
    out.entry_row.resize(nnz);
    out.entry_col.resize(nnz);
    stage("    entry arrays", ts);
    const int nth = analysis_threads(n);
    std::vector<i32> fof(n);
    parallel_for(nf, nth, [&](i64 a, i64 b) {
        for (i64 f = a; f < b; f++)
            for (i64 v = out.Rptr[f]; v < out.Rptr[f + 1]; v++) fof[v] = (i32)f;
    });
    // blocks of columns on the threads: per-block counts per front, then each block places its entries after those
    // of the blocks before it (the order a serial pass over the columns gives)
    const bool split = out.nB > 1;
    const int T = (int)std::max<i64>(1, std::min<i64>(nth, n / 1024));
    std::vector<std::vector<i64>> cnt(T);
    std::vector<i64> eptr(nf + 1, 0), colof(nnz);   // colof: column of A of each entry
    std::vector<i32> eidx(nnz);
    pool_run(T, [&](int t) {
        std::vector<i64> &h = cnt[t];
        h.assign(nf, 0);
        for (i64 c = n * t / T; c < n * (t + 1) / T; c++) {
            const i64 j = out.invp[c];
            for (i64 p = colptr[c]; p < colptr[c + 1]; p++) {
                colof[p] = c;
                const i64 i = out.invp[rowval[p]];
                if (split && out.comp[i] != out.comp[j]) {
                    out.entry_front[p] = -1;
                    continue;
                }
                const i64 f = fof[std::min<i64>(i, j)];
                out.entry_front[p] = f;
                h[f]++;
            }
        }
    });
    stage("    entry fronts", ts);
    for (i64 f = 0; f < nf; f++) {
        i64 run = eptr[f];
        for (int t = 0; t < T; t++) {
            const i64 c = cnt[t][f];
            cnt[t][f] = run;
            run += c;
        }
        eptr[f + 1] = run;
    }
    pool_run(T, [&](int t) {
        std::vector<i64> &pos = cnt[t];
        for (i64 p = colptr[n * t / T]; p < colptr[n * (t + 1) / T]; p++)
            if (out.entry_front[p] >= 0) eidx[pos[out.entry_front[p]]++] = (i32)p;
    });
    stage("  entry lists", ts);
    std::atomic<bool> outside(false);
    std::atomic<i64> nextf(0);
    pool_run(nth, [&](int) {
        std::vector<i32> where(n, -1);
        while (true) {
            const i64 f0 = nextf.fetch_add(64);
            if (f0 >= nf) break;
            for (i64 f = f0; f < std::min<i64>(nf, f0 + 64); f++) {
                const i64 r0 = out.Rptr[f], r1 = out.Rptr[f + 1];
                for (i64 q = out.Sptr[f]; q < out.Sptr[f + 1]; q++) where[out.Stgt[q]] = (i32)((r1 - r0) + (q - out.Sptr[f]));
                for (i64 k = eptr[f]; k < eptr[f + 1]; k++) {
                    const i64 p = eidx[k];
                    const i64 i = out.invp[rowval[p]], j = out.invp[colof[p]];
                    const i64 hi = std::max(i, j);
                    const i64 lhi = hi < r1 ? hi - r0 : where[hi];
                    if (lhi < 0) {
                        outside = true;
                        continue;
                    }
                    out.entry_row[p] = (i32)(i < j ? i - r0 : lhi);
                    out.entry_col[p] = (i32)(j <= i ? j - r0 : lhi);
                }
                for (i64 q = out.Sptr[f]; q < out.Sptr[f + 1]; q++) where[out.Stgt[q]] = -1;
            }
        }
    });
    if (outside) return "an entry of A falls outside the structure";
    stage("  entries", ts);
    work_counts(n, out.Rptr, out.Sptr, out.parent, out.madds_factor, out.madds_star, out.madds_rhs, out.nnzL);
    out.madds_star_offd = 0;
    if (out.nB > 1 && out.nN > 0) {
        for (i64 c = 0; c < out.nB; c++) {
            const double rows = (double)(out.Bptr[c] - out.anc_lo[c]);
            if (rows <= 0) continue;
            double per = (double)(out.Nptr[out.Bptr[c + 1]] - out.Nptr[out.Bptr[c]]);
            for (i64 f = out.Fptr[c]; f < out.Fptr[c + 1]; f++) {
                const double nn = (double)(out.Rptr[f + 1] - out.Rptr[f]), na = (double)(out.Sptr[f + 1] - out.Sptr[f]);
                per += 2 * nn * (na + (nn - 1) / 2);
            }
            out.madds_star_offd += rows * per;
        }
        out.madds_star += out.madds_star_offd;
    }
    return "";
}

}  // namespace

std::string analyze_given(i64 n, const i64 *colptr, const i64 *rowval, const i64 *perm, i64 nf, const i64 *Rptr,
                          Symbolic &out) {
    double t0 = now();
    std::string err = check_csc(n, colptr, rowval);
    if (!err.empty()) return err;
    std::vector<i64> p(perm, perm + n), R(Rptr, Rptr + nf + 1);
    std::vector<char> seen(n, 0);
    for (i64 k = 0; k < n; k++) {
        if (p[k] < 0 || p[k] >= n || seen[p[k]]) return "perm is not a permutation";
        seen[p[k]] = 1;
    }
    if (R[0] != 0 || R[nf] != n) return "Rptr must run from 0 to n";
    for (i64 f = 0; f < nf; f++)
        if (R[f + 1] <= R[f]) return "fronts must be nonempty";
    // the strongly connected components, renumbered in the order the given permutation visits them (any topological
    // order of the components is the reference's; components() checks that they come out grouped)
    std::vector<i32> comp;
    i64 nB = strong_components(n, colptr, rowval, comp);
    if (nB > 1) {
        std::vector<i32> ren(nB, -1);
        i32 next = 0;
        for (i64 k = 0; k < n; k++)
            if (ren[comp[p[k]]] < 0) ren[comp[p[k]]] = next++;
        for (i64 v = 0; v < n; v++) comp[v] = ren[comp[v]];
        for (i64 j = 0; j < n; j++)
            for (i64 q = colptr[j]; q < colptr[j + 1]; q++)
                if (comp[rowval[q]] > comp[j]) return "the given order puts a strongly connected component before one with an arc into it";
    }
    Adj G;
    err = symmetrize(n, colptr, rowval, G, nB > 1 ? &comp : nullptr);
    if (!err.empty()) return err;
    err = finish(G, n, colptr, rowval, p, R, out, nullptr, nB > 1 ? &comp : nullptr, nB);
    if (!err.empty()) return err;
    out.madds_factor_alg = out.madds_factor;
    out.madds_star_alg = out.madds_star;
    out.madds_rhs_alg = out.madds_rhs;
    out.nnzL_alg = out.nnzL;
    out.seconds_total = now() - t0;
    return "";
}

void dense_structure(i64 n, Symbolic &out) {
    out = Symbolic();
    out.n = n;
    out.perm.resize(n);
    std::iota(out.perm.begin(), out.perm.end(), 0);
    out.invp = out.perm;
    out.nf = n > 0 ? 1 : 0;
    out.Rptr = n > 0 ? std::vector<i64>{0, n} : std::vector<i64>{0};
    out.Sptr.assign(out.nf + 1, 0);
    out.parent.assign(out.nf, -1);
    out.fdsc.assign(out.nf, 0);
    out.Dptr = n > 0 ? std::vector<i64>{0, n * n} : std::vector<i64>{0};
    out.Lptr.assign(out.nf + 1, 0);
    out.nB = 1;
    out.Bptr = {0, n};
    out.Fptr = {0, out.nf};
    out.nN = 0;
    out.Nptr.assign(n + 1, 0);
    out.NTptr.assign(n + 1, 0);
    out.lev_up.assign(1, 0);
    out.lev_dn.assign(1, 0);
    out.anc_lo.assign(1, 0);
    out.nnz = 0;
    work_counts(n, out.Rptr, out.Sptr, out.parent, out.madds_factor, out.madds_star, out.madds_rhs, out.nnzL);
    out.madds_factor_alg = out.madds_factor;
    out.madds_star_alg = out.madds_star;
    out.madds_rhs_alg = out.madds_rhs;
    out.nnzL_alg = out.nnzL;
}

std::string analyze(i64 n, const i64 *colptr, const i64 *rowval, const SymOptions &opts, const i64 *given_perm,
                    Symbolic &out) {
    double t0 = now();
    const int nth = analysis_threads(n);
    std::string err = check_csc(n, colptr, rowval, nth);
    if (!err.empty()) return err;
    // 0. strongly connected components in a topological order (sccs, chordal_ssymbolic.jl:26-57): the pattern that is
    //    ordered and factorized is that of the diagonal blocks; every order below is regrouped by component.  A
    //    symmetric pattern has no arcs between its components, which are its connected components.
    std::vector<i32> comp;
    double tsc = t0;
    stage("  check", tsc);
    Adj G;
    i64 nB;
    if (pattern_symmetric(n, colptr, rowval, nth)) {
        offdiagonal(n, colptr, rowval, G, nth);
        stage("  symmetric pattern", tsc);
        nB = connected_components(G, comp, nth);
        stage("  connected components", tsc);
    } else {
        nB = strong_components(n, colptr, rowval, comp);
        stage("  strong components", tsc);
        err = symmetrize(n, colptr, rowval, G, nB > 1 ? &comp : nullptr);
        if (!err.empty()) return err;
        stage("  symmetrize", tsc);
    }
    const std::vector<i32> *cp = nB > 1 ? &comp : nullptr;
    // 1. fill-reducing order
    std::vector<i64> perm0(n);
    std::vector<i64> perm1, pcol, ccol;   // set here by the automatic choice (2. and 3. below otherwise)
    std::vector<NDRange> sub;   // nested dissection's ranges
    if (opts.ordering == 4) {
        // both orders (minimum degree on its own thread while nested dissection uses the pool); keep the one whose
        // factor has fewer entries
        std::vector<i64> pa;
        std::thread tamd([&] { pa = amd_order(G); });
        ND nd(G, opts.nd_leaf);
        nd.run(analysis_threads(n));
        tamd.join();
        std::vector<i64> p1[2], pc[2], cc[2];
        if (cp) {
            group_by_component(nd.order, comp, nB, &nd.ranges);
            group_by_component(pa, comp, nB);
        }
        const std::vector<i64> *cand[2] = {&nd.order, &pa};
        std::thread t1([&] {
            etree_postorder(G, *cand[1], p1[1], pc[1]);
            column_counts(G, p1[1], pc[1], cc[1]);
        });
        etree_postorder(G, *cand[0], p1[0], pc[0], &nd.ranges, nth);
        column_counts(G, p1[0], pc[0], cc[0], nth);
        t1.join();
        i64 fill[2] = {0, 0};
        for (int c = 0; c < 2; c++)
            for (i64 v : cc[c]) fill[c] += v;
        const int pick = fill[1] < fill[0] ? 1 : 0;
        perm0 = *cand[pick];
        perm1 = std::move(p1[pick]);
        pcol = std::move(pc[pick]);
        ccol = std::move(cc[pick]);
    } else if (opts.ordering == 0) {
        ND nd(G, opts.nd_leaf);
        nd.run(analysis_threads(n));
        perm0.swap(nd.order);
        sub.swap(nd.ranges);
    } else if (opts.ordering == 3) {
        perm0 = amd_order(G);
    } else if (opts.ordering == 1) {
        std::iota(perm0.begin(), perm0.end(), 0);
    } else {
        if (!given_perm) return "no permutation given";
        std::vector<char> seen(n, 0);
        for (i64 k = 0; k < n; k++) {
            if (given_perm[k] < 0 || given_perm[k] >= n || seen[given_perm[k]]) return "perm is not a permutation";
            seen[given_perm[k]] = 1;
            perm0[k] = given_perm[k];
        }
    }
    if (cp && opts.ordering != 4) group_by_component(perm0, comp, nB, &sub);
    out.seconds_order = now() - t0;
    double ts = t0;
    stage("symmetrize + order", ts);
    // 2. postordered elimination tree
    if (opts.ordering != 4) etree_postorder(G, perm0, perm1, pcol, sub.empty() ? nullptr : &sub, nth);
    stage("etree + postorder", ts);
    // 3. column counts, then fundamental supernodes: j + 1 continues j's supernode when it is j's parent, has no
    //    other child, and its column holds exactly one entry fewer
    if (opts.ordering != 4) column_counts(G, perm1, pcol, ccol, nth);
    std::vector<i64> nchild(n, 0);
    for (i64 j = 0; j < n; j++)
        if (pcol[j] >= 0) nchild[pcol[j]]++;
    std::vector<i64> R1;
    R1.push_back(0);
    for (i64 j = 1; j < n; j++) {
        const bool cont = pcol[j - 1] == j && nchild[j] == 1 && ccol[j] == ccol[j - 1] - 1;
        if (!cont) R1.push_back(j);
    }
    R1.push_back(n);
    stage("column counts + supernodes", ts);
    // the fundamental supernodes' separator sizes and tree, from the counts: na = count(first column) - nn, and
    // the parent holds the elimination-tree parent of the last column
    const i64 ns = (i64)R1.size() - 1;
    std::vector<i64> S1(ns + 1, 0), par1(ns, -1), sidx(n);
    for (i64 s = 0; s < ns; s++) {
        for (i64 v = R1[s]; v < R1[s + 1]; v++) sidx[v] = s;
        S1[s + 1] = S1[s] + (ccol[R1[s]] - (R1[s + 1] - R1[s]));
    }
    for (i64 s = 0; s < ns; s++) {
        const i64 pj = pcol[R1[s + 1] - 1];
        par1[s] = pj >= 0 ? sidx[pj] : -1;
    }
    {
        double f, s, r, l;
        work_counts(n, R1, S1, par1, f, s, r, l);
        out.madds_factor_alg = f;
        out.madds_star_alg = s;
        out.madds_rhs_alg = r;
        out.nnzL_alg = l;
    }
    if (!opts.amalgamate) {
        err = finish(G, n, colptr, rowval, perm1, R1, out, &par1, cp, nB);
        out.madds_star_alg += out.madds_star_offd;
        out.seconds_total = now() - t0;
        return err;
    }
    // 4. relaxed amalgamation: merge a child front into its parent when the merged front's share of explicit
    //    zeros stays below a size-dependent bound (the rule of CHOLMOD's relaxed supernodes, Ashcraft & Grimes
    //    1989); the merged front has the parent's separator.
    std::vector<i64> mnn(ns), mna(ns), rep(ns);
    std::vector<double> mtrue(ns);
    for (i64 s = 0; s < ns; s++) {
        i64 nn = R1[s + 1] - R1[s], na = S1[s + 1] - S1[s];
        mnn[s] = nn;
        mna[s] = na;
        mtrue[s] = (double)nn * (nn - 1) / 2 + (double)nn * na;
        rep[s] = s;
    }
    auto find = [&](i64 s) {
        while (rep[s] != s) {
            rep[s] = rep[rep[s]];
            s = rep[s];
        }
        return s;
    };
    // children of every supernode and, after the merges, members and children of every merged front: lists in
    // increasing order, stored as (pointer, index) arrays
    auto csr = [&](i64 m, auto key, std::vector<i64> &ptr, std::vector<i64> &idx) {   // idx lists s with key(s) = k
        ptr.assign(ns + 1, 0);
        for (i64 s = 0; s < m; s++) {
            const i64 k = key(s);
            if (k >= 0) ptr[k + 1]++;
        }
        for (i64 k = 0; k < ns; k++) ptr[k + 1] += ptr[k];
        idx.assign(ptr[ns], 0);
        std::vector<i64> pos(ptr.begin(), ptr.end() - 1);
        for (i64 s = 0; s < m; s++) {
            const i64 k = key(s);
            if (k >= 0) idx[pos[k]++] = s;
        }
    };
    stage("    amalgamation setup", ts);
    std::vector<i64> kptr, kidx;
    csr(ns, [&](i64 s) { return par1[s]; }, kptr, kidx);
    std::vector<i64> cs, ckey;
    for (i64 p = 0; p < ns; p++) {
        // children with few columns first: they gain the most (a stable insertion sort: a front has few children)
        cs.assign(kidx.begin() + kptr[p], kidx.begin() + kptr[p + 1]);
        ckey.resize(cs.size());
        for (size_t a = 0; a < cs.size(); a++) ckey[a] = mnn[find(cs[a])];
        for (size_t a = 1; a < cs.size(); a++) {
            const i64 c = cs[a], k = ckey[a];
            size_t b = a;
            for (; b > 0 && ckey[b - 1] > k; b--) {
                cs[b] = cs[b - 1];
                ckey[b] = ckey[b - 1];
            }
            cs[b] = c;
            ckey[b] = k;
        }
        for (i64 c : cs) {
            i64 rc = find(c), rp = find(p);
            i64 nn = mnn[rp] + mnn[rc], na = mna[rp];
            if (nn > opts.max_front_cols) continue;
            double dense = (double)nn * (nn - 1) / 2 + (double)nn * na;
            double z = dense > 0 ? 1.0 - (mtrue[rp] + mtrue[rc]) / dense : 0.0;
            bool merge;
            if (nn <= opts.relax_small) merge = true;
            else if (nn <= opts.relax_cols[0]) merge = z < opts.relax_z[0];
            else if (nn <= opts.relax_cols[1]) merge = z < opts.relax_z[1];
            else merge = z < opts.relax_z[2];
            if (!merge) continue;
            rep[rc] = rp;
            mnn[rp] = nn;
            mtrue[rp] += mtrue[rc];
        }
    }
    stage("    merges", ts);
    // 5. renumber: postorder of the merged tree; a merged front lists its members' columns in the members'
    //    (post)order, so the new order is still a topological order of the elimination tree
    std::vector<i64> root(ns);
    for (i64 s = 0; s < ns; s++) root[s] = find(s);
    std::vector<i64> mptr, midx, cptr, cidx;
    csr(ns, [&](i64 s) { return root[s]; }, mptr, midx);
    auto top_of = [&](i64 s) { return midx[mptr[s + 1] - 1]; };   // the last member of merged front s
    // parent of a merged front: the merged front of its top member's parent
    csr(ns, [&](i64 s) { return root[s] == s && par1[top_of(s)] >= 0 ? root[par1[top_of(s)]] : (i64)-1; }, cptr, cidx);
    std::vector<i64> perm2, R2, fid(ns, -1);
    perm2.reserve(n);
    R2.push_back(0);
    std::vector<std::pair<i64, i64>> stack;
    for (i64 s = 0; s < ns; s++) {
        if (root[s] != s || par1[top_of(s)] >= 0) continue;
        stack.push_back({s, cptr[s]});
        while (!stack.empty()) {
            auto &tp = stack.back();
            const i64 m = tp.first;
            if (tp.second < cptr[m + 1]) {
                const i64 c = cidx[tp.second++];
                stack.push_back({c, cptr[c]});
            } else {
                for (i64 q = mptr[m]; q < mptr[m + 1]; q++)
                    for (i64 v = R1[midx[q]]; v < R1[midx[q] + 1]; v++) perm2.push_back(perm1[v]);
                fid[m] = (i64)R2.size() - 1;
                R2.push_back((i64)perm2.size());
                stack.pop_back();
            }
        }
    }
    if ((i64)perm2.size() != n) return "internal error: amalgamation lost vertices";
    // the merged tree in the final numbering: a merged front's parent holds its top member's parent
    std::vector<i64> tree2((i64)R2.size() - 1, -1);
    for (i64 s = 0; s < ns; s++)
        if (root[s] == s) {
            const i64 top = top_of(s);
            if (par1[top] >= 0) tree2[fid[s]] = fid[root[par1[top]]];
        }
    stage("amalgamation", ts);
    err = finish(G, n, colptr, rowval, perm2, R2, out, &tree2, cp, nB);
    out.madds_star_alg += out.madds_star_offd;
    stage("final structure + entries", ts);
    out.seconds_total = now() - t0;
    return err;
}

}  // namespace pp
