"""Benchmark: MinPlus mstar of the directed 32 x 32 x 32 grid (n = 32768, Float32) on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--config 3] [--no-cpu]

One step is one mstar(MinPlus(), A) (abstract_slu.jl:85-87): the host symbolic analysis (ordering, elimination tree,
supernodes), the device factorization and the device star, with A's values already in HBM and the n x n star left in
HBM.  `value` is semiring Gop/s = 1e-9 * madds_alg / step seconds, where madds_alg is the multiply-add count of the
exact (unamalgamated) factor of the same ordering (the reference's per-front formulas).  One JSON line on stdout.

Other configurations of the benchmark suite (one JSON line each, same keys):
    --config 1    MinPlus mstar, directed 64 x 64 grid, Float64 (wall time of a small case)
    --config 2a   dense MinPlus GEMM C <- min(C, A + B), 8192^3, Float32 (pp_sgemx; % of VALU peak)
    --config 2b   batched front LU + stars, 16384 fronts of 64 x 64, Float32 (pp_getrf_star_batched)
    --config 4    MaxMin lmul! of 1024 unit columns on a random geometric graph, n = 65536, Float32
    --config 5    PlusProd rmul! of 512 unit rows on the directed 256 x 256 grid, Float64
    --config dag  MinPlus mstar of a chain of 16 strongly connected layers (components coupled by arcs), n = 16384
The default is the headline configuration 3.
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

# MI355X's published FP32 vector rate is 157.3 TFLOP/s: 78.65e12 lane FMAs/s (256 CU x 4 SIMD x 32 lanes x 2.4 GHz),
# one full-rate VALU instruction per lane and clock.  The roofline counts one semiring multiply-add as one FMA (two
# flops), so its peak is the published 157.3 TFLOP/s.  Beside it the instruction-mix bound: a MinPlus / MaxPlus Float32
# multiply-add costs 1.5 VALU instructions (v_add_f32, v_add_f32, v_min3_f32 per two; packed FP32 is not used), which
# caps the min-plus kernels at 52.4e12 madds/s.  The VALU probe (--calibrate-valu) measures the compiled sequence.
FP32_PEAK_TFLOPS = 157.3
VALU_PEAK_MADD = FP32_PEAK_TFLOPS * 1e12 / 2          # madds/s at one FMA slot per madd
INSTR_PER_MADD = 1.5
INSTR_MIX_PEAK_MADD = VALU_PEAK_MADD / INSTR_PER_MADD
HBM_PEAK = 8.0e12


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def valu_roofline(kernel: str, madds: float, seconds: float, extra=None) -> dict:
    """The roofline object of a VALU-bound min/max kernel: achieved and peak in TFLOP/s (one madd = one FMA = two
    flops, against the published FP32 rate), and the same rate against the 1.5-instruction mix."""
    rate = madds / seconds
    r = {"bound": "valu", "kernel": kernel, "achieved": round(2 * rate / 1e12, 3), "peak": FP32_PEAK_TFLOPS,
         "unit": "TFLOP/s", "frac": round(rate / VALU_PEAK_MADD, 4), "traffic": None,
         "madds_per_s": round(rate / 1e12, 3),
         "instr_mix": {"instr_per_madd": INSTR_PER_MADD, "peak_Tmadd_s": round(INSTR_MIX_PEAK_MADD / 1e12, 2),
                       "frac": round(rate / INSTR_MIX_PEAK_MADD, 4)}}
    if extra:
        r.update(extra)
    return r
PROFILES = os.path.join(ROOT, "profiles")


def measured_traffic(kernel: str):
    """HBM bytes per mstar of a kernel family, from the committed rocprofv3 --pmc summary (a line
    `traffic_bytes_per_star <kernel> <bytes>`), or None."""
    try:
        with open(os.path.join(PROFILES, "memory_traffic_mstar_minplus_grid32x32x32.md")) as f:
            for line in f:
                parts = line.replace("`", " ").split()
                if len(parts) == 3 and parts[0] == "traffic_bytes_per_star" and parts[1] == kernel:
                    return float(parts[2])
    except OSError:
        pass
    return None


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def factor_device(s, sym, dnz, ctx):
    """mlu with the values already in HBM (pp_factor_device)."""
    import ctypes

    h = ctypes.c_void_p()
    dt = {np.dtype(np.float32): 0, np.dtype(np.float64): 1, np.dtype(np.int32): 2}[dnz.dtype]
    ctx.check(P.lib().pp_factor_device(ctx.handle, sym.handle, s.id, dt, ctypes.c_void_p(dnz.ptr), ctypes.byref(h)))
    return P.Factorization(s, sym, dnz.dtype, h, ctx)


ORDERING = ["nd"]   # the analysis's fill-reducing order (--ordering)


def mstar_device(s, sym, dnz, out, ctx):
    """mstar with the values already in HBM and the star left in HBM (pp_mstar: the factorization and the star in
    one call, the star queued behind the factorization); returns the factor."""
    import ctypes

    h = ctypes.c_void_p()
    dt = {np.dtype(np.float32): 0, np.dtype(np.float64): 1, np.dtype(np.int32): 2}[dnz.dtype]
    ctx.check(P.lib().pp_mstar(ctx.handle, sym.handle, s.id, dt, ctypes.c_void_p(dnz.ptr), 1,
                               ctypes.c_void_p(out.ptr), sym.n, 1, ctypes.byref(h)))
    return P.Factorization(s, sym, dnz.dtype, h, ctx)


def step_mstar(g, dnz, out, ctx, timing):
    """One mstar: returns (seconds, symbolic, phases)."""
    ctx.synchronize()
    t0 = time.perf_counter()
    sym = P.symbolic(g, alg=ORDERING[0])
    t1 = time.perf_counter()
    F = mstar_device(P.MinPlus(), sym, dnz, out, ctx)
    ctx.synchronize()
    t3 = time.perf_counter()
    ph = ctx.timing() if timing else None
    phases = {"symbolic_s": t1 - t0, "factor_star_s": t3 - t1}
    if timing:
        phases.update({"factor_device_s": ph[0], "star_Ustar_s": ph[1], "star_Lstar_s": ph[2], "relabel_s": ph[3]})
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
    cfg = int(args.config)
    g = W.config_graph(cfg)
    ctx = P.context(0)
    ctx.set_timing(args.timing)
    dnz = P.DeviceArray.from_numpy(np.ascontiguousarray(g.nzval).reshape(-1, 1))
    out = P.DeviceArray((g.n, g.n), g.nzval.dtype)
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
    # repeated weights on one pattern (copyto! + lu! + Matrix, the plan idiom): the analysis, the plans and the
    # factor's buffers are reused; each step refactorizes from values in HBM and assembles the star (not `value`)
    import ctypes
    Tp = None
    if args.plan:
        Fp = factor_device(P.MinPlus(), sym, dnz, ctx)

        def plan_step():
            ctx.check(P.lib().pp_refactor(ctx.handle, Fp.handle, ctypes.c_void_p(dnz.ptr), 1))
            P.Matrix(Fp, out=out)

        Tp = timed(plan_step, ctx, args.steps, 1)
        del Fp
    if cfg == 3:
        metric = "mstar sec + semiring Gop/s, MinPlus 3D grid n=32768; % VALU/HBM roofline"
        workload = (f"MinPlus mstar, directed 32x32x32 grid, n=32768, 6-neighbour arcs both ways, "
                    f"weights U{{1..100}} Float32 (SplitMix64 seed 0x5EED+3); star left in HBM")
    else:
        metric = "mstar sec + semiring Gop/s, MinPlus 2D grid n=4096 (Float64)"
        workload = (f"MinPlus mstar, directed 64x64 grid, n=4096, 4-neighbour arcs both ways, weights U{{1..100}} "
                    f"Float64 (SplitMix64 seed 0x5EED+1); star left in HBM")
    result = {
        "metric": metric,
        "value": round(value, 2),
        "unit": "semiring Gop/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(T * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if g.nzval.dtype == np.float32 else "f64",
        "data": "synthetic",
        "config": {"workload": workload,
                   "n": g.n, "nnz": g.nnz, "fronts": sym.nf, "ordering": ORDERING[0], "madds_alg": madds,
                   "madds_executed": st["madds_factor"] + st["madds_star"], "nnzL_alg": st["nnzL_alg"],
                   "mstar_s": round(T, 5)},
        "phases_ms": {k: round(v * 1e3, 3) for k, v in ph.items()},
    }
    if Tp is not None:
        result["plan"] = {"ms_per_step": round(Tp * 1e3, 3), "semiring_Gops": round(madds / Tp / 1e9, 2),
                          "step": "pp_refactor (new values of the same pattern, in HBM) + pp_star; analysis reused"}
    if args.timing and cfg == 3:
        # dominant kernel family: the X <- X L* sweep (k_blk backward, k_sweep_bwd, k_sub backward), timed with HIP
        # events around all its launches on the context's stream; algorithmic work n * nnz(L) madds
        n = g.n
        lstar_madds = n * st["nnzL_alg"]
        t_l = ph["star_Lstar_s"]
        result["roofline"] = valu_roofline(
            "X <- X L* sweep: k_blk<..., false> + k_sweep_bwd + k_sub<..., false>, all launches of one star",
            lstar_madds, t_l,
            {"traffic": measured_traffic("lstar_sweep"), "algorithmic_madds": lstar_madds, "seconds": round(t_l, 6),
             "output_floor_GBps": round(4.0 * n * n / T / 1e9, 1)})
    Th = None
    if args.host_steps > 0:
        # mstar as the reference returns it: the n x n star in host memory (the analysis, the device factorization
        # and star, then the relabelled star copied back through pinned chunks), timed in the same run
        Th = mstar_to_host(g, args.host_steps)
        result["mstar_to_host"] = {"ms_per_step": round(Th * 1e3, 2), "semiring_Gops": round(madds / Th / 1e9, 2),
                                   "step": "symbolic + pp_mstar with the star delivered into a host array (n x n, "
                                           "original labels)"}
    if not args.no_cpu and cfg == 3:
        cb = cpu_baseline(g, sym, budget_s=args.cpu_budget)
        result["cpu_baseline"] = {"value": round(madds / cb["est_mstar_s"] / 1e9, 3), "unit": "semiring Gop/s",
                                  "cores": cb["threads"], "kind": "port", "cpu_model": cpu_model(),
                                  "sample": f"oracle factorization (single thread, full) + star rows "
                                            f"{cb['rows']} of {g.n} in blocks spread over the rows "
                                            f"({cb['star_sample_s']:.1f} s on {cb['threads']} threads), scaled to "
                                            f"n rows; symbolic excluded; star left in host memory",
                                  "est_mstar_s": round(cb["est_mstar_s"], 3), "factor_s": round(cb["factor_s"], 3)}
        # like for like: both stars end in host memory
        if Th is not None:
            result["speedup_vs_cpu"] = round(cb["est_mstar_s"] / Th, 1)
        result["speedup_vs_cpu_star_in_hbm"] = round(cb["est_mstar_s"] / T, 1)
    print(json.dumps(result), flush=True)


def mstar_to_host(g, steps):
    """Mean seconds of mstar(MinPlus(), A) with the star delivered into host memory (symbolic included), after one
    warm-up call; the host array is allocated and touched once beforehand."""
    C = np.empty((g.n, g.n), g.nzval.dtype, order="F")
    C.fill(0)
    ts = []
    for i in range(steps + 1):
        t0 = time.perf_counter()
        P.mstar(P.MinPlus(), g, out=C)
        t = time.perf_counter() - t0
        if i:
            ts.append(t)
        log(f"mstar to host {i}: {t * 1e3:.1f} ms")
    del C
    return float(np.mean(ts))


def timed(fn, ctx, steps, warmup):
    """Mean seconds of fn() over `steps` calls after `warmup` calls, each bracketed by stream synchronisation."""
    for _ in range(warmup):
        fn()
    ctx.synchronize()
    ts = []
    for _ in range(steps):
        ctx.synchronize()
        t0 = time.perf_counter()
        fn()
        ctx.synchronize()
        ts.append(time.perf_counter() - t0)
    return float(np.mean(ts))


def base_result(args, metric, value, unit, T, dtype, workload, extra):
    r = {"metric": metric, "value": round(value, 3), "unit": unit, "n_gpus": 1, "steps": args.steps,
         "warmup": args.warmup, "ms_per_step": round(T * 1e3, 4), "higher_is_better": True, "scaling": "weak",
         "vs_baseline": None, "dtype": dtype, "data": "synthetic", "config": {"workload": workload}}
    r["config"].update(extra)
    return r


def bench_gemm_plusprod(args):
    """2a with --semiring plusprod: C <- C + A B over Float64, M = N = K = 8192, entries U[0, 1/N) (fp64 MFMA)."""
    import ctypes

    N = 8192
    seed = W.SEED_BASE + 2
    A, B, C = [np.asfortranarray((W.uniform_float(seed + 10 * q, N * N) / N).reshape(N, N).T) for q in range(3)]
    ctx = P.context(0)
    dA, dB, dC = P.DeviceArray.from_numpy(A), P.DeviceArray.from_numpy(B), P.DeviceArray.from_numpy(C)

    def run():
        ctx.check(P.lib().pp_sgemx(ctx.handle, 4, 1, N, N, N, ctypes.c_void_p(dA.ptr), N, ctypes.c_void_p(dB.ptr), N,
                                   ctypes.c_void_p(dC.ptr), N))

    T = timed(run, ctx, args.steps, args.warmup)
    flops = 2.0 * float(N) ** 3
    valu = bool(os.environ.get("PP_GEMM_VALU"))
    r = base_result(args, "semiring GEMM TFLOP/s, PlusProd 8192^3 Float64; % fp64 MFMA roofline", flops / T / 1e12,
                    "TFLOP/s", T, "f64",
                    "dense PlusProd GEMM C <- C + A B, M=N=K=8192, entries U[0, 1/N) (SplitMix64 seeds 0x5EED+2, "
                    "+12, +22), operands in HBM", {"m": N, "n": N, "k": N})
    r["roofline"] = {"bound": "valu" if valu else "mfma",
                     "kernel": "k_gemm_tiled<PlusProd<double>, 4, 4>" if valu else "k_gemm_mfma64<double>",
                     "achieved": round(flops / T / 1e12, 3), "peak": 78.6, "unit": "TFLOP/s",
                     "frac": round(flops / T / 78.6e12, 4), "traffic": None}
    print(json.dumps(r), flush=True)


def bench_gemm(args):
    """2a: C <- min(C, A + B), M = N = K = 8192, Float32, A/B/C ~ U{0..1000} with 10 % +Inf."""
    import ctypes
    import oracle as O

    if args.semiring == "plusprod":
        return bench_gemm_plusprod(args)
    N = 8192
    seed = W.SEED_BASE + 2
    A = W.dense_minplus(N, N, seed)
    B = W.dense_minplus(N, N, seed + 10)
    C = W.dense_minplus(N, N, seed + 20)
    ctx = P.context(0)
    dA, dB, dC = P.DeviceArray.from_numpy(A), P.DeviceArray.from_numpy(B), P.DeviceArray.from_numpy(C)

    def run():
        ctx.check(P.lib().pp_sgemx(ctx.handle, 0, 0, N, N, N, ctypes.c_void_p(dA.ptr), N, ctypes.c_void_p(dB.ptr), N,
                                   ctypes.c_void_p(dC.ptr), N))

    T = timed(run, ctx, args.steps, args.warmup)
    madds = float(N) ** 3
    r = base_result(args, "semiring GEMM Gop/s, MinPlus 8192^3 Float32; % VALU roofline", madds / T / 1e9,
                    "semiring Gop/s", T, "f32",
                    "dense MinPlus GEMM C <- min(C, A + B), M=N=K=8192, entries U{0..1000} with 10% +Inf "
                    "(SplitMix64 seeds 0x5EED+2, +12, +22), operands in HBM", {"m": N, "n": N, "k": N})
    r["roofline"] = valu_roofline("k_gemm_tiled<MinPlus<float>, 8, 8>", madds, T)
    if not args.no_cpu:
        # the oracle's OpenMP GEMM on a 1024 x 1024 block of C with the full K
        mb = 1024
        t0 = time.perf_counter()
        O.sgemx(O.MINPLUS, np.asfortranarray(A[:mb, :]), np.asfortranarray(B[:, :mb]), np.asfortranarray(C[:mb, :mb]))
        tc = time.perf_counter() - t0
        r["cpu_baseline"] = {"value": round(float(mb) * mb * N / tc / 1e9, 3), "unit": "semiring Gop/s",
                             "cores": O.num_threads(), "kind": "port", "cpu_model": cpu_model(),
                             "sample": f"oracle sgemx on a {mb}x{mb} block of C with K={N} ({tc:.1f} s)"}
    print(json.dumps(r), flush=True)


def bench_getrf(args):
    """2b: 16384 independent 64 x 64 Float32 fronts: LU + L* + U* (pp_getrf_star_batched)."""
    import ctypes
    import oracle as O

    nb, batch = 64, 16384
    seed = W.SEED_BASE + 2
    A3 = np.asfortranarray(W.dense_minplus(nb, nb * batch, seed + 30)).reshape(nb, nb, batch, order="F")
    idx = np.arange(nb)
    A3[idx, idx, :] = 0.0   # front b is A3[:, :, b]; its diagonal is 0
    A = A3.reshape(nb, nb * batch, order="F")
    ctx = P.context(0)
    d0 = P.DeviceArray.from_numpy(A)
    dA = P.DeviceArray(A.shape, np.float32)
    dL = P.DeviceArray(A.shape, np.float32)
    dU = P.DeviceArray(A.shape, np.float32)

    def run():
        ctx.check(P.lib().pp_copy(ctx.handle, ctypes.c_void_p(dA.ptr), ctypes.c_void_p(d0.ptr), dA.nbytes))
        ctx.check(P.lib().pp_getrf_star_batched(ctx.handle, 0, 0, nb, batch, ctypes.c_void_p(dA.ptr),
                                                ctypes.c_void_p(dL.ptr), ctypes.c_void_p(dU.ptr)))

    T = timed(run, ctx, args.steps, args.warmup)
    per = nb ** 3 / 3 + 2 * nb ** 3 / 6
    madds = per * batch
    r = base_result(args, "batched front LU + stars Gop/s, 16384 x 64x64 Float32", madds / T / 1e9, "semiring Gop/s",
                    T, "f32", "16384 independent 64x64 MinPlus fronts, entries U{0..1000} with 10% +Inf, diagonal 0 "
                    "(SplitMix64 seed 0x5EED+32); A <- L+U, TL <- L*, TU <- U*; step includes a 268 MB device copy "
                    "restoring A", {"nb": nb, "batch": batch, "madds_per_front": per})
    r["roofline"] = valu_roofline("k_getrf_star_wave<MinPlus<float>>", madds, T,
                                  {"hbm_floor_ms": round(4.0 * A.size * 4 / HBM_PEAK * 1e3, 3)})
    if not args.no_cpu:
        sb = 512
        t0 = time.perf_counter()
        flat = A.ravel(order="F")[:sb * nb * nb]
        O.getrf_star_batched(O.MINPLUS, flat.reshape(sb, nb, nb))   # front b at [b] (column-major: [b, j, i])
        tc = time.perf_counter() - t0
        r["cpu_baseline"] = {"value": round(per * sb / tc / 1e9, 3), "unit": "semiring Gop/s",
                             "cores": O.num_threads(), "kind": "port", "cpu_model": cpu_model(), "sample": f"oracle on {sb} of the fronts"}
    print(json.dumps(r), flush=True)


def bench_solve(args, cfg):
    """4: MaxMin lmul! with 1024 unit columns on the RGG n=65536 (Float32); 5: PlusProd rmul! with 512 unit rows on
    the 256 x 256 grid (Float64).  mlu once; a step restores B (device copy) and applies the solve."""
    import ctypes
    import oracle as O

    g = W.config_graph(cfg)
    n = g.n
    ctx = P.context(0)
    ctx.set_timing(True)
    left = cfg == 4
    s = P.MaxMin() if left else P.PlusProd()
    nrhs = 1024 if left else 512
    src = (W.splitmix64(W.SEED_BASE + cfg + 100, nrhs) % np.uint64(n)).astype(np.int64)
    if left:
        B = np.full((n, nrhs), -np.inf, np.float32, order="F")
        B[src, np.arange(nrhs)] = np.inf
    else:
        B = np.zeros((nrhs, n), np.float64, order="F")
        B[np.arange(nrhs), src] = 1.0
    t0 = time.perf_counter()
    sym = P.symbolic(g, alg=ORDERING[0])
    t_sym = time.perf_counter() - t0
    dnz = P.DeviceArray.from_numpy(np.ascontiguousarray(g.nzval).reshape(-1, 1))
    ctx.synchronize()
    t0 = time.perf_counter()
    F = factor_device(s, sym, dnz, ctx)
    ctx.synchronize()
    t_fac = time.perf_counter() - t0
    d0 = P.DeviceArray.from_numpy(B)
    dB = P.DeviceArray(B.shape, B.dtype)
    fn = P.lib().pp_lmul if left else P.lib().pp_rmul
    ld = B.shape[0]

    def run():
        ctx.check(P.lib().pp_copy(ctx.handle, ctypes.c_void_p(dB.ptr), ctypes.c_void_p(d0.ptr), dB.nbytes))
        ctx.check(fn(ctx.handle, F.handle, ctypes.c_void_p(dB.ptr), ld, nrhs, 1))

    T = timed(run, ctx, args.steps, args.warmup)
    t_dev = ctx.timing()[4]
    st = sym.stats()
    madds = st["madds_rhs_alg"] * nrhs
    name = "lmul!" if left else "rmul!"
    # the same unit-vector right-hand sides as one batch of sources (columns / rows of A*, pp_star_sources): the
    # sweeps visit only the sources under each front; the result must equal the solve's
    which = 1 if left else 0
    dO = P.DeviceArray(B.shape, B.dtype)
    csrc = np.ascontiguousarray(src, dtype=np.int64)

    def run_src():
        ctx.check(P.lib().pp_star_sources(ctx.handle, F.handle, which, nrhs, csrc.ctypes.data_as(ctypes.c_void_p),
                                          ctypes.c_void_p(dO.ptr), ld, 1))

    T2 = timed(run_src, ctx, args.steps, args.warmup)
    got, ref = dO.numpy(), dB.numpy()
    if left:
        same = bool(np.array_equal(got.view(np.uint32), ref.view(np.uint32)))
        maxrel = 0.0
    else:
        maxrel = float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), np.finfo(np.float64).tiny)))
        same = maxrel <= 1e-12
    r = base_result(args, f"{name} sec + semiring Gop/s, {s.name} {nrhs} RHS, n={n}", madds / T / 1e9,
                    "semiring Gop/s", T, "f32" if left else "f64",
                    (f"MaxMin lmul! of 1024 unit columns (+Inf at a seeded source, -Inf elsewhere) on a random "
                     f"geometric graph n=65536, mean degree 8, capacities U{{1..1000}} Float32 (seed 0x5EED+4)"
                     if left else
                     f"PlusProd rmul! of 512 unit rows (1 at a seeded source) on the directed 256x256 grid, weights "
                     f"U(0,0.2) Float64 (seed 0x5EED+5)") + "; B in HBM, restored by a device copy in each step",
                    {"n": n, "nrhs": nrhs, "madds_alg": madds, "fronts": sym.nf, "ordering": ORDERING[0],
                     "nnzL_alg": st["nnzL_alg"]})
    r["phases_ms"] = {"symbolic_s": round(t_sym * 1e3, 3), "factor_s": round(t_fac * 1e3, 3),
                      "solve_device_s": round(t_dev * 1e3, 3)}
    r["unit_sources"] = {"entry": "pp_star_sources", "ms_per_step": round(T2 * 1e3, 3),
                         "speedup_vs_solve": round(T / T2, 2), "matches_solve": same, "max_rel": maxrel}
    if not args.no_cpu:
        k = 32
        e = sym.export()
        osym = O.Sym(n, e["Rptr"], e["Sptr"], e["Stgt"], e["perm"])
        Fo = O.factor(O.MAXMIN if left else O.PLUSPROD, osym, g.colptr, g.rowval, g.nzval)
        Bs = np.asfortranarray(B[:, :k] if left else B[:k, :])
        t0 = time.perf_counter()
        (O.lmul if left else O.rmul)(Fo, Bs)
        tc = time.perf_counter() - t0
        r["cpu_baseline"] = {"value": round(st["madds_rhs_alg"] * k / tc / 1e9, 3), "unit": "semiring Gop/s",
                             "cores": O.num_threads(), "kind": "port", "cpu_model": cpu_model(),
                             "sample": f"oracle {name} on {k} of the {nrhs} right-hand sides"}
    print(json.dumps(r), flush=True)


def bench_dag(args):
    """Strongly connected components coupled by arcs: MinPlus mstar of a chain of 16 strongly connected layers (each
    a 16 x 16 x 4 grid with arcs both ways; arcs from layer k to k + 1 only), n = 16384, Float32, star left in HBM.
    Beside it, the same graph with every arc made two-way (one strongly connected block: the fill a symmetrized
    pattern pays)."""
    import ctypes

    g = W.layered_digraph(16, (16, 16, 4), seed=W.SEED_BASE + 6, dtype=np.float32)
    cols = np.repeat(np.arange(g.n), np.diff(g.colptr))
    gs = W.from_arcs(g.n, np.concatenate([g.rowval, cols]), np.concatenate([cols, g.rowval]),
                     np.concatenate([g.nzval, g.nzval]))
    ctx = P.context(0)
    out = P.DeviceArray((g.n, g.n), np.float32)
    res = {}
    for label, gg in (("components", g), ("one_block", gs)):
        dnz = P.DeviceArray.from_numpy(np.ascontiguousarray(gg.nzval).reshape(-1, 1))

        def step():
            sym = P.symbolic(gg)
            h = ctypes.c_void_p()
            ctx.check(P.lib().pp_mstar(ctx.handle, sym.handle, 0, 0, ctypes.c_void_p(dnz.ptr), 1, ctypes.c_void_p(out.ptr),
                                       gg.n, 1, None))
            return sym

        T = timed(step, ctx, args.steps, args.warmup)
        sym = P.symbolic(gg)
        st, cm = sym.stats(), sym.components()
        res[label] = {"ms_per_step": round(T * 1e3, 3), "components": cm["nB"], "arcs_between": int(cm["Nptr"][-1]),
                      "nnzL_alg": st["nnzL_alg"], "madds_alg": st["madds_factor_alg"] + st["madds_star_alg"]}
        log(f"{label}: {res[label]}")
    T = res["components"]["ms_per_step"] * 1e-3
    r = base_result(args, "mstar sec + semiring Gop/s, MinPlus chain of 16 strongly connected 16x16x4 layers, n=16384",
                    res["components"]["madds_alg"] / T / 1e9, "semiring Gop/s", T, "f32",
                    "MinPlus mstar of layered_digraph(16, (16, 16, 4)) (arcs both ways inside a layer, forward between "
                    "layers), weights U{1..100} Float32 (seed 0x5EED+6); star left in HBM", {"n": g.n})
    r["components"] = res["components"]
    r["one_block_two_way_arcs"] = res["one_block"]
    print(json.dumps(r), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="3", choices=["1", "2a", "2b", "3", "4", "5", "dag"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-plan", dest="plan", action="store_false",
                    help="configurations 1 and 3: skip the repeated-weights (pp_refactor + pp_star) timing")
    ap.add_argument("--semiring", default="minplus", choices=["minplus", "plusprod"],
                    help="configuration 2a only: MinPlus Float32 (default) or PlusProd Float64 (fp64 matrix cores)")
    ap.add_argument("--ordering", default="nd", choices=["nd", "amd"],
                    help="fill-reducing order of the analysis: nested dissection (default) or approximate minimum degree")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--host-steps", type=int, default=2,
                    help="configurations 1 and 3: timed mstar calls with the star delivered to host memory (0: skip)")
    ap.add_argument("--no-timing", dest="timing", action="store_false")
    ap.add_argument("--calibrate-valu", action="store_true",
                    help="only run the VALU probe (pp_calibrate_valu): v_add_f32 and MinPlus multiply-add rates")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MiB",
                    help="only run the plain copy kernel (pp_copy) over this many MiB: the calibration of the memory "
                         "counters FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    ORDERING[0] = args.ordering
    if args.calibrate_valu:
        import ctypes

        ctx = P.context(0)
        out = {}
        for kind, name in ((0, "v_add_f32"), (1, "minplus_madd2")):
            sec, ins = ctypes.c_double(), ctypes.c_double()
            ctx.check(P.lib().pp_calibrate_valu(ctx.handle, kind, 200000, ctypes.byref(sec), ctypes.byref(ins)))
            out[name] = {"seconds": sec.value, "lane_instr_per_s": ins.value / sec.value}
        out["minplus_madd_per_s"] = out["minplus_madd2"]["lane_instr_per_s"] * 16 / 26
        print(json.dumps(out))
        return
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
    if args.config in ("1", "3"):
        bench_mstar(args)
    elif args.config == "2a":
        bench_gemm(args)
    elif args.config == "2b":
        bench_getrf(args)
    elif args.config == "dag":
        bench_dag(args)
    else:
        bench_solve(args, int(args.config))


if __name__ == "__main__":
    main()
