"""Benchmark: MinPlus mstar of the directed 32 x 32 x 32 grid (n = 32768, Float32) on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--config 3] [--no-cpu]

One step is one mstar(MinPlus(), A) (abstract_slu.jl:85-87): the host symbolic analysis (ordering, elimination tree,
supernodes), the device factorization and the device star, with A's values already in HBM and the n x n star left in
HBM.  `value` is semiring Gop/s = 1e-9 * madds_alg / step seconds, where madds_alg is the multiply-add count of the
exact (unamalgamated) factor of the same ordering (the reference's per-front formulas).  One JSON line on stdout.

Other configurations (--config 1, 4, 5, gemm, getrf) are the other workloads of the benchmark suite; the default is the
headline one.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for sub in ("pathpack.jl_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)

import pathpack_hip as P  # noqa: E402
from pathpack_hip import workloads as W  # noqa: E402

VALU_PEAK_MADD = 26.2e12   # MinPlus f32: 2 v_add_f32 + 1 v_min3_f32 per 2 multiply-adds; 256 CU x 4 SIMD x 16 x 2.4 GHz
HBM_PEAK = 8.0e12


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def step_mstar(g, dnz, out, ctx, timing):
    """One mstar: returns (seconds, symbolic, phases)."""
    ctx.synchronize()
    t0 = time.perf_counter()
    sym = P.symbolic(g)
    t1 = time.perf_counter()
    import ctypes

    h = ctypes.c_void_p()
    ctx.check(P.lib().pp_factor_device(ctx.handle, sym.handle, 0, 0, ctypes.c_void_p(dnz.ptr), ctypes.byref(h)))
    F = P.Factorization(P.MinPlus(), sym, np.float32, h, ctx)
    t2 = time.perf_counter()
    ph_f = ctx.timing() if timing else None
    P.Matrix(F, out=out)
    ctx.synchronize()
    t3 = time.perf_counter()
    ph_s = ctx.timing() if timing else None
    phases = {"symbolic_s": t1 - t0, "factor_s": t2 - t1, "star_s": t3 - t2}
    if timing:
        phases.update({"factor_device_s": ph_f[0], "star_Ustar_s": ph_s[1], "star_Lstar_s": ph_s[2],
                       "relabel_s": ph_s[3]})
    return t3 - t0, sym, phases, F


def cpu_baseline(g, sym, budget_s=15.0):
    """The oracle (CPU restatement of PATHPACK.CPU, OpenMP on all host cores) on a bounded sample: the factorization
    once, then the star's rows in evenly spread blocks until about budget_s of work; scaled to all n rows."""
    import oracle as O

    e = sym.export()
    osym = O.Sym(g.n, e["Rptr"], e["Sptr"], e["Stgt"], e["perm"])
    threads = O.num_threads()
    t0 = time.perf_counter()
    F = O.factor(O.MINPLUS, osym, g.colptr, g.rowval, g.nzval)
    t_factor = time.perf_counter() - t0
    n = g.n
    C = np.empty((n, n), np.float32, order="F")   # the oracle writes the sampled rows of the permuted star here
    import ctypes

    rows_done = 0
    t_star = 0.0
    blk = max(32, 32 * threads)
    k = 0
    order = np.random.default_rng(0).permutation(n // blk)
    while t_star < budget_s and k < order.size:
        r0 = int(order[k]) * blk
        t = time.perf_counter()
        rc = O.lib().ppo_star(ctypes.c_int(O.MINPLUS), ctypes.c_int(O.F32), *osym.args(), *F._fargs(),
                              C.ctypes.data_as(ctypes.c_void_p), ctypes.c_int64(r0), ctypes.c_int64(r0 + blk),
                              ctypes.c_int(0), ctypes.c_int(threads))
        t_star += time.perf_counter() - t
        if rc != 0:
            raise RuntimeError(f"oracle star failed {rc}")
        rows_done += blk
        k += 1
    est_star = t_star * n / rows_done
    return {"factor_s": t_factor, "star_sample_s": t_star, "rows": rows_done, "threads": threads,
            "est_mstar_s": t_factor + est_star}


def bench_mstar(args):
    cfg = args.config
    g = W.config_graph(cfg)
    if cfg == 1:
        g = g.astype(np.float64)
    ctx = P.context(0)
    ctx.set_timing(args.timing)
    dnz = P.DeviceArray.from_numpy(np.ascontiguousarray(g.nzval).reshape(-1, 1))
    out = P.DeviceArray((g.n, g.n), g.nzval.dtype)
    assert g.nzval.dtype == np.float32 or cfg == 1
    if cfg == 1:
        raise SystemExit("--config 1 is Float64; use the parity tests")
    log(f"bench: {g.name} n={g.n} nnz={g.nnz} warmup={args.warmup} steps={args.steps}")
    for i in range(args.warmup):
        t, sym, ph, F = step_mstar(g, dnz, out, ctx, args.timing)
        log(f"warmup {i}: {t * 1e3:.1f} ms {json.dumps({k: round(v * 1e3, 2) for k, v in ph.items()})}")
        del F
    times, phases = [], []
    for i in range(args.steps):
        t, sym, ph, F = step_mstar(g, dnz, out, ctx, args.timing)
        times.append(t)
        phases.append(ph)
        log(f"step {i}: {t * 1e3:.1f} ms {json.dumps({k: round(v * 1e3, 2) for k, v in ph.items()})}")
        del F
    T = float(np.mean(times))
    st = sym.stats()
    madds = st["madds_factor_alg"] + st["madds_star_alg"]
    value = madds / T / 1e9
    ph = {k: float(np.mean([p[k] for p in phases])) for k in phases[0]}
    result = {
        "metric": "mstar sec + semiring Gop/s, MinPlus 3D grid n=32768; % VALU/HBM roofline",
        "value": round(value, 2),
        "unit": "semiring Gop/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(T * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"MinPlus mstar, directed 32x32x32 grid, n=32768, 6-neighbour arcs both ways, "
                               f"weights U{{1..100}} Float32 (SplitMix64 seed 0x5EED+3); star left in HBM",
                   "n": g.n, "nnz": g.nnz, "fronts": sym.nf, "madds_alg": madds,
                   "madds_executed": st["madds_factor"] + st["madds_star"], "nnzL_alg": st["nnzL_alg"],
                   "mstar_s": round(T, 5)},
        "phases_ms": {k: round(v * 1e3, 3) for k, v in ph.items()},
    }
    if args.timing:
        # dominant kernel family: the X <- X L* sweep (k_sweep_bwd); algorithmic work n * nnz(L) madds
        n = g.n
        lstar_madds = n * st["nnzL_alg"]
        t_l = ph["star_Lstar_s"]
        ach = lstar_madds / t_l
        result["roofline"] = {"bound": "valu", "kernel": "k_sweep_bwd (X <- X L*, all launches of one star)",
                              "achieved": round(ach / 1e12, 4), "peak": VALU_PEAK_MADD / 1e12, "unit": "Tmadd/s",
                              "frac": round(ach / VALU_PEAK_MADD, 4), "traffic": None,
                              "algorithmic_madds": lstar_madds, "seconds": round(t_l, 6),
                              "output_floor_GBps": round(4.0 * n * n / T / 1e9, 1)}
    if not args.no_cpu:
        cb = cpu_baseline(g, sym, budget_s=args.cpu_budget)
        result["cpu_baseline"] = {"value": round(madds / cb["est_mstar_s"] / 1e9, 3), "unit": "semiring Gop/s",
                                  "cores": cb["threads"], "kind": "port",
                                  "sample": f"oracle factorization (single thread, full) + star rows "
                                            f"{cb['rows']} of {g.n} in blocks spread over the rows "
                                            f"({cb['star_sample_s']:.1f} s on {cb['threads']} threads), scaled to "
                                            f"n rows; symbolic excluded",
                                  "est_mstar_s": round(cb["est_mstar_s"], 3), "factor_s": round(cb["factor_s"], 3)}
        result["speedup_vs_cpu"] = round(cb["est_mstar_s"] / T, 1)
    print(json.dumps(result), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--no-timing", dest="timing", action="store_false")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MiB",
                    help="only run the plain copy kernel (pp_copy) over this many MiB: the calibration of the memory "
                         "counters FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.calibrate_copy:
        import ctypes

        ctx = P.context(0)
        nb = args.calibrate_copy << 20
        src = P.DeviceArray((nb // 4,), np.float32)
        dst = P.DeviceArray((nb // 4,), np.float32)
        for _ in range(2):
            ctx.check(P.lib().pp_copy(ctx.handle, ctypes.c_void_p(dst.ptr), ctypes.c_void_p(src.ptr), nb))
        print(json.dumps({"calibrate_copy_bytes": nb, "launches": 2}))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU: the star's row blocks would shard across GPUs "
                                   "with a replicated factor, which this build does not implement"}))
        sys.exit(2)
    bench_mstar(args)


if __name__ == "__main__":
    main()
