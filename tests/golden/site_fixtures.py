"""Reader for the reference's own factor fixtures and the graphs they were made from.

The four data files next to this module are data the reference ships (docs/src/public/data/):
* ``paris.bin.gz``, ``bunny.bin.gz``: the two demo graphs;
* ``paris-lu.bin.gz``, ``bunny-lu.bin.gz``: ``mlu(MinPlus(), A)`` of those graphs in Float32, written by the
  reference's docs/site_factors.jl:136-207 (permutation, fronts, separators and the factor values D, UL, LL).

File format (docs/site_factors.jl:111-133): uint32 header length, a JSON header
``{meta, arrays: {name: [dtype, offset, count]}}``, then the arrays, each aligned to 4 bytes; all gzip-compressed.

The graphs are rebuilt exactly as docs/site_factors.jl:44-104 builds them (the browser's construction):
* paris: arc weights ``Float32(wm[e] / 1000)``, every street an arc both ways, parallel arcs combined with min;
* bunny: vertex coordinates ``Float32(lo[i % 3] + pos[i] / scale)``, each triangle edge once in the order the
  triangles list them, weight ``Float32(hypot)`` with V8's Math.hypot (scale by the largest magnitude, Kahan-summed
  squares, scale back; site_factors.jl:78-95), arcs both ways, combined with min.
"""

from __future__ import annotations

import gzip
import json
import math
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def readbin(path: str):
    raw = gzip.open(path).read()
    hl = struct.unpack("<I", raw[:4])[0]
    head = json.loads(raw[4:4 + hl])
    base = 4 + hl
    arrays = {}
    for k, (dt, off, cnt) in head["arrays"].items():
        arrays[k] = np.frombuffer(raw, dtype=np.dtype(dt).newbyteorder("<"), count=cnt, offset=base + off)
    return head["meta"], arrays


def _jshypot(dx: float, dy: float, dz: float) -> float:
    xs = (dx, dy, dz)
    mx = 0.0
    for x in xs:
        mx = max(mx, abs(x))
    if mx == 0:
        return 0.0
    s = 0.0
    comp = 0.0
    for x in xs:
        r = abs(x) / mx
        t = r * r - comp
        prel = s + t
        comp = (prel - s) - t
        s = prel
    return math.sqrt(s) * mx


def graph_arcs(name: str):
    """(n, I, J, W) of the demo graph: undirected edges (0-based), Float32 weights."""
    meta, a = readbin(os.path.join(HERE, f"{name}.bin.gz"))
    if name == "paris":
        n = int(meta["n"])
        I = a["ei"].astype(np.int64)
        J = a["ej"].astype(np.int64)
        W = (a["wm"].astype(np.float64) / 1000.0).astype(np.float32)
        return n, I, J, W
    if name == "bunny":
        n = int(meta["n"])
        nf = int(meta["f"])
        lo = [float(x) for x in meta["lo"]]
        scale = float(meta["scale"])
        pos = a["pos"].astype(np.float64)
        P = np.array([lo[i % 3] + pos[i] / scale for i in range(3 * n)], dtype=np.float64).astype(np.float32)
        tri = a["tri"].astype(np.int64)
        seen = set()
        I, J, W = [], [], []
        for f in range(nf):
            i, j, k = int(tri[3 * f]), int(tri[3 * f + 1]), int(tri[3 * f + 2])
            for p, q in ((i, j), (j, k), (k, i)):
                key = min(p, q) * 65536 + max(p, q)
                if key in seen:
                    continue
                seen.add(key)
                dx = float(P[3 * p]) - float(P[3 * q])
                dy = float(P[3 * p + 1]) - float(P[3 * q + 1])
                dz = float(P[3 * p + 2]) - float(P[3 * q + 2])
                I.append(p)
                J.append(q)
                W.append(_jshypot(dx, dy, dz))
        return n, np.array(I, np.int64), np.array(J, np.int64), np.array(W, np.float64).astype(np.float32)
    raise ValueError(name)


def graph_csc(name: str):
    """(n, colptr, rowval, nzval): the matrix sparse(vcat(I, J), vcat(J, I), vcat(W, W), n, n, min)."""
    n, I, J, W = graph_arcs(name)
    src = np.concatenate([I, J])
    dst = np.concatenate([J, I])
    w = np.concatenate([W, W])
    key = dst * n + src
    order = np.lexsort((w, key))
    key, w = key[order], w[order]
    first = np.ones(key.size, bool)
    first[1:] = key[1:] != key[:-1]
    key, w = key[first], w[first]
    cols, rows = key // n, key % n
    colptr = np.zeros(n + 1, np.int64)
    np.add.at(colptr, cols + 1, 1)
    return n, np.cumsum(colptr), rows.astype(np.int64), w.astype(np.float32)


def factor_fixture(name: str):
    """The reference's factor of the demo graph, 0-based: dict with n, perm (new -> old), Rptr, Sptr, Stgt and the
    values D (diag blocks: upper+diag of U, strict lower of L), UL (nn x na), LL (na x nn)."""
    meta, a = readbin(os.path.join(HERE, f"{name}-lu.bin.gz"))
    n = int(meta["n"])
    rperm = a["rperm"].astype(np.int64) - 1
    cinvp = a["cinvp"].astype(np.int64) - 1
    assert np.array_equal(cinvp[rperm], np.arange(n))
    return {
        "n": n,
        "nB": int(meta["nB"]),
        "perm": rperm,
        "Rptr": a["Rptr"].astype(np.int64) - 1,
        "Sptr": a["Sptr"].astype(np.int64) - 1,
        "Stgt": a["Stgt"].astype(np.int64) - 1,
        "D": np.array(a["D"], dtype=np.float32),
        "UL": np.array(a["UL"], dtype=np.float32),
        "LL": np.array(a["LL"], dtype=np.float32),
        "Nval": np.array(a["Nval"], dtype=np.float32),
    }
