"""CPU replay of the star's device schedule (tests/emu/star_plan_emu.cpp): the real plan and block packs, the device
kernels' index arithmetic launch by launch, bounds / race / initialisation checks, and the result against the oracle
(its blocked star when strongly connected components are coupled by arcs between them).

The replay is built with hipcc as host code (it includes the plan headers) and linked with the oracle library; it is
skipped where hipcc is absent.  Graphs are chosen so that large fronts cut into 128- and 64-column blocks, blocks are
followed by panels, small subtrees form, n is odd (guarded row loads) and the graph has several components.  The source-row path (rows of the star for a
subset of sources, each unit's rows mapped into the subset) is replayed the same way.
"""

import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle as O
from helpers import dtype_for, weighted
from pathpack_hip import workloads as W

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(REPO, "pathpack.jl_amd", "csrc")


def _hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    return None


@pytest.fixture(scope="module")
def emu(tmp_path_factory):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    O.build()
    exe = str(tmp_path_factory.mktemp("emu") / "star_plan_emu")
    cmd = [hipcc, "-O2", "-std=c++20", "-I", CSRC, "-I", os.path.join(REPO, "include"),
           os.path.join(HERE, "emu", "star_plan_emu.cpp"), os.path.join(CSRC, "pp_symbolic.cpp"),
           os.path.join(CSRC, "pp_plan.cpp"), "-L", os.path.join(REPO, "oracle"), "-lpporacle",
           "-Wl,-rpath," + os.path.join(REPO, "oracle"), "-lpthread", "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


GRAPHS = {
    "grid12x12x12": lambda: W.grid((12, 12, 12)),          # 144-column top front: a 128 block and a 16 panel
    "grid15x13x11": lambda: W.grid((15, 13, 11)),          # odd n; a 161-column front: 128 + 33 (a 64-wide tile)
    "grid9x9x9": lambda: W.grid((9, 9, 9)),                # an 82-column front: a 64 block and an 18 panel
    "components": lambda: W.disjoint_union([W.grid((10, 10, 9)), W.grid((30, 29)), W.rgg(300, seed=5)],
                                           isolated=3, name="components"),
    # one 64-wide block whose component rows reach far outside its subtree: the padded K steps of the backward
    # block GEMM read rows that nothing has written yet (NaN under PlusProd before the fix); also 30 strongly
    # connected components with 88 arcs between them (the coupled second pass)
    "digraph300": lambda: W.random_digraph(300, 0.01, 3),
    # strongly connected layers in a chain, and a DAG of 150 one-vertex components: the second pass over the
    # component DAG (the gathers of N, then the panel lists on the rows of the earlier components, atomic forward)
    "layered": lambda: W.layered_digraph(6, (8, 6), fwd=0.5, seed=3),
    "dag": lambda: W.random_dag(150, 0.04, 9),
}

# X starts as NaN (-1 for OrAnd) in the replay, so every semiring checks that no value read before it is written
# reaches a stored result
ALL = [(O.MINPLUS, np.float32), (O.MINPLUS, np.float64), (O.MAXPLUS, np.float32), (O.MAXPLUS, np.float64),
       (O.MAXMIN, np.float32), (O.MINMAX, np.float64), (O.PLUSPROD, np.float32), (O.PLUSPROD, np.float64),
       (O.ORAND, np.float32)]
FEW = [(O.MINPLUS, np.float32), (O.MINPLUS, np.float64), (O.PLUSPROD, np.float32), (O.PLUSPROD, np.float64)]
CASES = [(name, s, d) for name in GRAPHS
         for (s, d) in (ALL if name in ("grid9x9x9", "components", "digraph300", "layered", "dag") else FEW)]


@pytest.mark.parametrize("name,s,fdtype", CASES)
def test_star_schedule_replay(emu, tmp_path, name, s, fdtype):
    dtype = dtype_for(s, fdtype)
    g = weighted(GRAPHS[name](), s, dtype)
    path = tmp_path / "graph.bin"
    with open(path, "wb") as f:
        np.array([g.n, len(g.rowval)], np.int64).tofile(f)
        np.asarray(g.colptr, np.int64).tofile(f)
        np.asarray(g.rowval, np.int64).tofile(f)
        np.asarray(g.nzval, dtype).tofile(f)
    dcode = {np.dtype(np.float32): 0, np.dtype(np.float64): 1, np.dtype(np.int32): 2}[np.dtype(dtype)]
    # a compute-unit count of 1 makes every launch with a 128-row tile take it; a huge one forces 64-row tiles
    for ncu in ([1, 1 << 20] if s == O.MINPLUS and np.dtype(dtype).itemsize == 4 else [1]):
        r = subprocess.run([emu, str(path), str(s), str(dcode), str(ncu)], capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, f"ncu={ncu}: {r.stdout[-500:]} {r.stderr[-2000:]}"


def _write(g, dtype, path):
    with open(path, "wb") as f:
        np.array([g.n, len(g.rowval)], np.int64).tofile(f)
        np.asarray(g.colptr, np.int64).tofile(f)
        np.asarray(g.rowval, np.int64).tofile(f)
        np.asarray(g.nzval, dtype).tofile(f)


SOURCE_CASES = [("grid15x13x11", O.MINPLUS, np.float32), ("components", O.MINPLUS, np.float64),
                ("components", O.PLUSPROD, np.float64), ("grid9x9x9", O.MAXMIN, np.float32)]


@pytest.mark.parametrize("name,s,fdtype", SOURCE_CASES)
def test_source_rows_schedule_replay(emu, tmp_path, name, s, fdtype):
    """Rows of the star for sources s with hash(s) mod M == 0: M = 1 (every source, the subset map is the
    identity), 3, 17 and a modulus that leaves a handful of sources."""
    dtype = dtype_for(s, fdtype)
    g = weighted(GRAPHS[name](), s, dtype)
    path = tmp_path / "graph.bin"
    _write(g, dtype, path)
    dcode = {np.dtype(np.float32): 0, np.dtype(np.float64): 1, np.dtype(np.int32): 2}[np.dtype(dtype)]
    for mod in (1, 3, 17, max(2, g.n // 4)):
        r = subprocess.run([emu, str(path), str(s), str(dcode), "1", str(mod)], capture_output=True, text=True,
                           timeout=300)
        assert r.returncode == 0, f"M={mod}: {r.stdout[-500:]} {r.stderr[-2000:]}"
