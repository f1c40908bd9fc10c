// pp_symbolic.h -- host symbolic analysis of the multifrontal semiring LU (internal header).
//
// The reference delegates this step to CliqueTrees.jl (cliquetree(symmetric(graph); alg), ChordalSymbolic,
// src/CPU/chordal_ssymbolic.jl:26-184): a fill-reducing order, the elimination tree and the supernodes ("fronts")
// with their separators.  This is an independent implementation of the same objects:
//   * the pattern is symmetrized (the reference orders symmetric(graph), chordal_ssymbolic.jl:67);
//   * the order is nested dissection on level structures, with minimum degree on the leaves;
//   * the elimination tree is postordered, fundamental supernodes are found from the column counts, and small
//     fronts are merged into their parents (relaxed amalgamation: explicit semiring zeros in exchange for wider
//     fronts);
//   * separators are computed by the supernodal symbolic factorization, so a structure given from outside (a
//     permutation plus a partition into fronts, e.g. the reference's own) yields the same separators.
// Strongly connected components are split as the reference does (sccs, chordal_ssymbolic.jl:26-57; utils.jl:3-70):
// the components are numbered in a topological order of the graph (every arc between two components goes from a
// lower to a higher number), each component's vertices get consecutive labels in that order, and only arcs inside a
// component enter the symmetrized pattern.  So the pattern is block upper triangular, the fronts are per component
// (one elimination tree each), and the arcs between components are kept apart as the sparse matrix N (soffd,
// chordal_ssymbolic.jl:212-269), applied by the coupled sweeps.
#pragma once
#include <cstdint>
#include <functional>
#include <string>
#include <vector>

namespace pp {

typedef int64_t i64;
typedef int32_t i32;

struct SymOptions {
    int ordering = 0;          // 0 = nested dissection, 1 = natural (identity), 2 = given permutation,
                               // 3 = approximate minimum degree, 4 = the one of 0 and 3 with the smaller factor
    int amalgamate = 1;        // relaxed amalgamation on/off
    int nd_leaf = 32;          // subgraphs of at most this many vertices are ordered by minimum degree
    int relax_small = 4;       // fronts of at most this many columns always merge
    double relax_z[3] = {0.8, 0.1, 0.05};   // zero fraction allowed at <= 16, <= 48, > 48 columns
    int relax_cols[2] = {16, 48};
    int max_front_cols = 1 << 30;
};

struct Symbolic {
    i64 n = 0;
    std::vector<i64> perm, invp;        // perm[new] = old, invp[old] = new
    i64 nf = 0;
    std::vector<i64> Rptr, Sptr, Stgt;  // res(f) = [Rptr[f], Rptr[f+1]), sep(f) = Stgt[Sptr[f]..Sptr[f+1]) ascending
    std::vector<i64> parent;            // parent front, -1 for roots
    std::vector<i64> fdsc;              // first descendant front of each front
    std::vector<i64> Dptr, Lptr;        // running sums of nn^2 and nn*na
    // strongly connected components (in a topological order; nB == 1: one block, nothing below is used)
    i64 nB = 1;
    std::vector<i64> Bptr;              // vertices of component c: [Bptr[c], Bptr[c+1]) (new labels)
    std::vector<i64> Fptr;              // fronts of component c: [Fptr[c], Fptr[c+1])
    std::vector<i32> comp;              // component of each vertex (new labels)
    // N: the arcs between components, A[i, j] with comp(i) < comp(j), in the new labels.  By column (CSC: rows i of
    // column j ascending) and by row (CSR: columns j of row i ascending); *src is the position in A's nzval.
    i64 nN = 0;
    std::vector<i64> Nptr, Nsrc, NTptr, NTsrc;
    std::vector<i32> Nidx, NTidx;
    // per component: level in the arcs' direction (1 + the largest level of a component with an arc into it), level
    // against it (1 + the largest level of a component it has an arc into), and the first vertex of the earliest
    // component with a path into it (its own first vertex if none)
    std::vector<i32> lev_up, lev_dn;
    std::vector<i64> anc_lo;
    // the input pattern: where each stored entry of A lands in the frontal matrices
    i64 nnz = 0;
    std::vector<i64> entry_front;       // front owning entry p (the front of min(new row, new col)); -1: an arc of N
    std::vector<i32> entry_row, entry_col;   // local row / column of entry p in that front's bag (res then sep)
    // work counts (semiring multiply-adds) of the exact structure, before amalgamation, and of the executed one
    double madds_factor_alg = 0, madds_star_alg = 0, madds_rhs_alg = 0, nnzL_alg = 0;
    double madds_factor = 0, madds_star = 0, madds_rhs = 0, nnzL = 0;
    // the star's pass over coupled components (included in both star counts): for each component, the rows of the
    // earlier components with a path into it times its per-row solve and its arcs in N
    double madds_star_offd = 0;
    double seconds_order = 0, seconds_total = 0;
};

// Build the symbolic structure of the CSC pattern (colptr, rowval) of an n x n matrix.  Returns "" on success,
// otherwise an error message.  `given_perm` is used when opts.ordering == 2.
std::string analyze(i64 n, const i64 *colptr, const i64 *rowval, const SymOptions &opts, const i64 *given_perm,
                    Symbolic &out);

// fn(0), ..., fn(n - 1) concurrently on the library's worker threads (fn(0) on the caller's); one job at a time.
void pool_run(int n, const std::function<void(int)> &fn);

// The symbolic structure for a given permutation and partition into fronts (Rptr, fronts in postorder).
std::string analyze_given(i64 n, const i64 *colptr, const i64 *rowval, const i64 *perm, i64 nf, const i64 *Rptr,
                          Symbolic &out);

// The structure of a dense n x n matrix factorized in its own order (the reference's DenseSLU, dense_slu.jl:1-44):
// one front holding every vertex, no separator, no stored entries (the values are copied into the front whole).
void dense_structure(i64 n, Symbolic &out);

}  // namespace pp
