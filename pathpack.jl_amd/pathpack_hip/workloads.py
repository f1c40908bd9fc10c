"""Seeded synthetic inputs for the multifrontal semiring solver.

One generator serves the tests, the benchmark and the CPU baseline, so every side reads the same matrices.

* The stream is SplitMix64 (Steele, Lea & Flood, "Fast splittable pseudorandom number generators", OOPSLA 2014):
  the k-th draw of a stream with seed ``s`` is ``mix(s + (k + 1) * 0x9E3779B97F4A7C15)``.  It is counter based, so a
  vector of draws is one numpy expression.
* A uniform integer in ``[a, b]`` is ``a + draw % (b - a + 1)``; a uniform float in ``[0, 1)`` is the top 53 bits
  times ``2**-53``.
* Graphs are square matrices in CSC form with ``A[i, j]`` the weight of the arc ``i -> j`` (the reference's
  convention, README.md:40-41).  "Both ways" means two arcs per undirected edge with independently drawn weights.
  Arcs are numbered source-major (vertex ``v`` ascending, then its neighbours in a fixed direction order) and the
  k-th arc takes the k-th draw.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
SEED_BASE = 0x5EED


def splitmix64(seed: int, count: int, start: int = 0) -> np.ndarray:
    """Draws ``start .. start + count - 1`` of the SplitMix64 stream ``seed`` as uint64."""
    with np.errstate(over="ignore"):
        k = np.arange(start + 1, start + count + 1, dtype=np.uint64)
        z = np.uint64(seed) + k * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def uniform_int(seed: int, count: int, lo: int, hi: int, start: int = 0) -> np.ndarray:
    """Uniform integers in ``[lo, hi]`` (int64)."""
    z = splitmix64(seed, count, start)
    return (np.int64(lo) + (z % np.uint64(hi - lo + 1)).astype(np.int64)).astype(np.int64)


def uniform_float(seed: int, count: int, start: int = 0) -> np.ndarray:
    """Uniform floats in ``[0, 1)`` from the top 53 bits (float64)."""
    z = splitmix64(seed, count, start)
    return (z >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


@dataclass
class Graph:
    """A square sparse matrix in CSC form: column ``j`` holds the arcs ``i -> j`` (``rowval``) and their weights."""

    n: int
    colptr: np.ndarray  # int64, n + 1
    rowval: np.ndarray  # int64, nnz, sorted within each column, no duplicates
    nzval: np.ndarray   # weights
    name: str = ""
    coords: np.ndarray | None = None

    @property
    def nnz(self) -> int:
        return int(self.colptr[-1])

    def dense(self, zero) -> np.ndarray:
        """The matrix as a dense array with ``zero`` off the pattern."""
        A = np.full((self.n, self.n), zero, dtype=self.nzval.dtype)
        cols = np.repeat(np.arange(self.n), np.diff(self.colptr))
        A[self.rowval, cols] = self.nzval
        return A

    def scipy(self):
        import scipy.sparse as sp

        return sp.csc_matrix((self.nzval, self.rowval, self.colptr), shape=(self.n, self.n))

    def astype(self, dtype) -> "Graph":
        return Graph(self.n, self.colptr, self.rowval, self.nzval.astype(dtype), self.name, self.coords)


def from_arcs(n: int, src: np.ndarray, dst: np.ndarray, w: np.ndarray, combine: str = "min", name: str = "") -> Graph:
    """CSC of the arcs ``src -> dst`` with weights ``w``; parallel arcs are combined with ``min``, ``max`` or ``or``."""
    src = np.asarray(src, dtype=np.int64)
    dst = np.asarray(dst, dtype=np.int64)
    w = np.asarray(w)
    key = dst * n + src
    order = np.lexsort((w, key)) if combine == "min" else np.lexsort((-w if combine == "max" else w, key))
    key = key[order]
    w = w[order]
    if combine == "or" and key.size:
        first = np.ones(key.size, dtype=bool)
        first[1:] = key[1:] != key[:-1]
        starts = np.flatnonzero(first)
        w = np.bitwise_or.reduceat(w, starts)
        key = key[first]
    else:
        first = np.ones(key.size, dtype=bool)
        first[1:] = key[1:] != key[:-1]
        key = key[first]
        w = w[first]
    cols = key // n
    rows = key % n
    colptr = np.zeros(n + 1, dtype=np.int64)
    np.add.at(colptr, cols + 1, 1)
    colptr = np.cumsum(colptr)
    return Graph(n, colptr, rows.astype(np.int64), w, name)


def _grid_arcs(dims: tuple[int, ...]) -> tuple[np.ndarray, np.ndarray]:
    """Arcs between lattice neighbours, both ways, source-major; vertex id = x + nx*y + nx*ny*z."""
    n = int(np.prod(dims))
    v = np.arange(n, dtype=np.int64)
    coord = []
    rem = v.copy()
    for d in dims:
        coord.append(rem % d)
        rem //= d
    stride = np.cumprod((1,) + dims[:-1])
    srcs, dsts, order = [], [], []
    k = 0
    for axis in range(len(dims)):
        for sgn in (+1, -1):
            ok = (coord[axis] + sgn >= 0) & (coord[axis] + sgn < dims[axis])
            s = v[ok]
            srcs.append(s)
            dsts.append(s + sgn * stride[axis])
            order.append(np.full(s.size, k))
            k += 1
    src = np.concatenate(srcs)
    dst = np.concatenate(dsts)
    direction = np.concatenate(order)
    o = np.lexsort((direction, src))
    return src[o], dst[o]


def grid(dims: tuple[int, ...], lo: int = 1, hi: int = 100, dtype=np.float32, seed: int = SEED_BASE, name: str = "") -> Graph:
    """Directed grid graph, arcs both ways between lattice neighbours, weights uniform integers in [lo, hi]."""
    src, dst = _grid_arcs(tuple(dims))
    w = uniform_int(seed, src.size, lo, hi).astype(dtype)
    n = int(np.prod(dims))
    return from_arcs(n, src, dst, w, "min", name or "grid" + "x".join(map(str, dims)))


def grid_float(dims: tuple[int, ...], scale: float, dtype=np.float64, seed: int = SEED_BASE, name: str = "") -> Graph:
    """Directed grid graph with weights uniform in [0, scale) (the PlusProd workload)."""
    src, dst = _grid_arcs(tuple(dims))
    w = (uniform_float(seed, src.size) * scale).astype(dtype)
    n = int(np.prod(dims))
    return from_arcs(n, src, dst, w, "min", name or "grid" + "x".join(map(str, dims)))


def rgg(n: int, degree: float = 8.0, lo: int = 1, hi: int = 1000, dtype=np.float32, seed: int = SEED_BASE) -> Graph:
    """Random geometric graph: n points uniform in the unit square, radius sqrt(degree / (pi n)), arcs both ways,
    weights uniform integers in [lo, hi].  Points use draws 2i, 2i+1 of the stream ``seed``; weights use the stream
    ``seed + 1``."""
    u = uniform_float(seed, 2 * n)
    xy = u.reshape(n, 2)
    r = math.sqrt(degree / (math.pi * n))
    cells = max(1, int(1.0 / r))
    cx = np.minimum((xy[:, 0] * cells).astype(np.int64), cells - 1)
    cy = np.minimum((xy[:, 1] * cells).astype(np.int64), cells - 1)
    cell = cx + cells * cy
    order = np.argsort(cell, kind="stable")
    start = np.searchsorted(cell[order], np.arange(cells * cells + 1))
    src_l, dst_l = [], []
    for dx in (-1, 0, 1):
        for dy in (-1, 0, 1):
            nx = cx + dx
            ny = cy + dy
            ok = (nx >= 0) & (nx < cells) & (ny >= 0) & (ny < cells)
            i_idx = np.flatnonzero(ok)
            c2 = (nx + cells * ny)[ok]
            cnt = start[c2 + 1] - start[c2]
            rep_i = np.repeat(i_idx, cnt)
            offs = np.repeat(start[c2], cnt) + (np.arange(cnt.sum()) - np.repeat(np.cumsum(cnt) - cnt, cnt))
            j = order[offs]
            keep = (j != rep_i)
            rep_i, j = rep_i[keep], j[keep]
            d2 = ((xy[rep_i] - xy[j]) ** 2).sum(axis=1)
            near = d2 < r * r
            src_l.append(rep_i[near])
            dst_l.append(j[near])
    src = np.concatenate(src_l)
    dst = np.concatenate(dst_l)
    o = np.lexsort((dst, src))
    src, dst = src[o], dst[o]
    w = uniform_int(seed + 1, src.size, lo, hi).astype(dtype)
    g = from_arcs(n, src, dst, w, "min", f"rgg{n}")
    g.coords = xy
    return g


def random_digraph(n: int, p: float, seed: int, lo: int = 1, hi: int = 100, dtype=np.float64) -> Graph:
    """Random directed graph (each ordered pair i != j an arc with probability p) with weights in [lo, hi]: the
    shape of the reference's Floyd-Warshall test graphs (test/core.jl:13-20), from this module's own stream."""
    u = uniform_float(seed, n * n).reshape(n, n)
    src, dst = np.nonzero((u < p) & ~np.eye(n, dtype=bool))
    w = uniform_int(seed + 7, src.size, lo, hi).astype(dtype)
    return from_arcs(n, src, dst, w, "min", f"digraph{n}")


def layered_digraph(layers: int, dims: tuple[int, ...], fwd: float = 0.3, seed: int = SEED_BASE, lo: int = 1,
                    hi: int = 100, dtype=np.float64) -> Graph:
    """A DAG of strongly connected layers: ``layers`` copies of the lattice ``dims`` with arcs both ways between
    neighbours (each layer one strongly connected component), plus arcs from layer k to layer k + 1 only: vertex v of
    layer k to the same vertex of layer k + 1, and each further pair (v in k, u in k + 1) with probability ``fwd``
    divided by the layer size.  The condensation is a chain of ``layers`` components; vertex labels are shuffled."""
    m = int(np.prod(dims))
    n = layers * m
    s0, d0 = _grid_arcs(dims)
    src = [s0 + k * m for k in range(layers)]
    dst = [d0 + k * m for k in range(layers)]
    for k in range(layers - 1):
        src.append(np.arange(m) + k * m)
        dst.append(np.arange(m) + (k + 1) * m)
        u = uniform_float(seed + 31 + k, m * m).reshape(m, m)
        a, b = np.nonzero(u < fwd / m)
        src.append(a + k * m)
        dst.append(b + (k + 1) * m)
    src, dst = np.concatenate(src), np.concatenate(dst)
    lab = np.argsort(uniform_float(seed + 17, n), kind="stable")
    w = uniform_int(seed + 7, src.size, lo, hi).astype(dtype)
    return from_arcs(n, lab[src], lab[dst], w, "min", f"layered{layers}x{m}")


def random_dag(n: int, p: float, seed: int, lo: int = 1, hi: int = 100, dtype=np.float64) -> Graph:
    """A random DAG: arc i -> j with probability p for i < j in a seeded random order of the vertices (every vertex is
    its own strongly connected component)."""
    u = uniform_float(seed, n * n).reshape(n, n)
    src, dst = np.nonzero((u < p) & np.triu(np.ones((n, n), dtype=bool), 1))
    lab = np.argsort(uniform_float(seed + 3, n), kind="stable")
    w = uniform_int(seed + 7, src.size, lo, hi).astype(dtype)
    return from_arcs(n, lab[src], lab[dst], w, "min", f"dag{n}")


def disjoint_union(parts: list[Graph], isolated: int = 0, seed: int = SEED_BASE, name: str = "") -> Graph:
    """The disjoint union of ``parts`` plus ``isolated`` vertices without arcs, with the vertices relabelled by a
    seeded permutation so that the components interleave."""
    n = sum(g.n for g in parts) + isolated
    lab = np.argsort(uniform_float(seed, n), kind="stable")
    src, dst, w, base = [], [], [], 0
    for g in parts:
        cols = np.repeat(np.arange(g.n), np.diff(g.colptr))
        src.append(lab[base + g.rowval])
        dst.append(lab[base + cols])
        w.append(g.nzval)
        base += g.n
    dtype = parts[0].nzval.dtype if parts else np.float64
    return from_arcs(n, np.concatenate(src), np.concatenate(dst), np.concatenate(w).astype(dtype), "min", name)


def dense_minplus(rows: int, cols: int, seed: int, inf_frac: float = 0.1, lo: int = 0, hi: int = 1000,
                  dtype=np.float32) -> np.ndarray:
    """Column-major (Fortran order) matrix of uniform integers in [lo, hi] with a fraction ``inf_frac`` set to
    +Inf (Bernoulli per entry from the independent stream ``seed + 1``)."""
    cnt = rows * cols
    v = uniform_int(seed, cnt, lo, hi).astype(dtype)
    mask = uniform_float(seed + 1, cnt) < inf_frac
    v[mask] = np.inf
    return v.reshape(cols, rows).T  # element (i, j) at j * rows + i: a Fortran-ordered view


# ===== the benchmark configurations =====

def config_graph(cfg: int) -> Graph:
    """The graph of benchmark configuration ``cfg`` (1-based: 1, 3, 4, 5), seed 0x5EED + cfg."""
    seed = SEED_BASE + cfg
    if cfg == 1:
        return grid((64, 64), 1, 100, np.float64, seed, "grid64x64")
    if cfg == 3:
        return grid((32, 32, 32), 1, 100, np.float32, seed, "grid32x32x32")
    if cfg == 4:
        return rgg(65536, 8.0, 1, 1000, np.float32, seed)
    if cfg == 5:
        return grid_float((256, 256), 0.2, np.float64, seed, "grid256x256")
    raise ValueError(f"configuration {cfg} has no graph")
