"""Benchmark: coded-weight GB/s of the fused Huffman decode + Q4_K dequant + GEMV on Mistral-7B-shaped layers.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers L] [--m 1]

Workload: per layer the matrices q 4096x4096, k, v 1024x4096, o 4096x4096, gate, up
14336x4096, down 4096x14336, Q4_K coded (huf4p, one Huffman table per matrix, entropy 2.3 bits per code), fp16
activations x ~ N(0, 1) resident in HBM, batch 1. L distinct layers (default 8, > 600 MB of coded weights, beyond
the 256 MB Infinity Cache) are generated with their own seeds. A step = one pass over all L layers, each layer's
seven GEMVs launched back to back (grouped per layer). value = algorithmic coded bytes per step / step time, where
the algorithmic bytes of a GEMV are blob + side tensor + 2 K (x) + 4 m N (y) (the reference's own size
accounting; device-layout padding is not credited).

roofline: the dominant kernel (k_fused_tiles: a tile per wave copied to LDS, 8 chains per lane; one grouped launch
per layer that also sums the tile-column partials)
timed with HIP events around each pass of the layers' launches on their stream (the launches run back to back),
divided by the launches per pass; achieved = the layer's algorithmic bytes / that mean duration, peak = 8 TB/s. serial_per_matrix: the same step with every GEMV launched on its own (latency view);
decode_step_forward_order: the same GEMVs as a forward pass orders them (per layer q, k, v grouped, then o, then gate
and up grouped, then down: 4 dependent launches, kernels/llmrt.cu:2366-2411). traffic = HBM
bytes per layer launch from two rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE) over `bench.py --profile`,
each scaled by what the counter reads for the 256 MiB device copy that --profile also runs (null when rocprofv3 is
unavailable or a pass fails). cpu_baseline: the oracle's restatement of the reference CPU path (cpu_decode,
kernels/llmrt.cu:2513-2541, then dequant + fp32 GEMV) on layer 0, timed on this host.
One JSON line on stdout.
"""
import argparse
import json
import math
import os
import shutil
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "coded-weight GB/s and % HBM roofline, fused decode+GEMV, Mistral-7B-shaped Q4_K"
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def counter_pass(counter, layers, tmp, timeout=240):
    """One rocprofv3 --pmc pass over `bench.py --profile`: {kernel: [(grid, KiB), ...]} or None."""
    import csv
    import signal
    import subprocess
    exe = shutil.which("rocprofv3")
    if not exe:
        return None
    out = os.path.join(tmp, counter)
    cmd = [exe, "--pmc", counter, "--output-format", "csv", "-d", out, "-o", "t", "--", sys.executable,
           os.path.abspath(__file__), "--profile", "--steps", "2", "--layers", str(layers)]
    log("bench: counter pass %s" % counter)
    p = subprocess.Popen(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL, start_new_session=True)
    timed_out = False
    try:
        p.wait(timeout=timeout)
    except subprocess.TimeoutExpired:
        timed_out = True
    # the pass's own process group (its session, started above) is reaped whether or not rocprofv3 ended by itself:
    # a child of the profiler that outlives it would otherwise outlive bench.py
    try:
        os.killpg(p.pid, signal.SIGKILL)
    except (ProcessLookupError, PermissionError):
        pass
    p.wait()
    if timed_out:
        log("bench: counter pass %s timed out" % counter)
        return None
    rows = {}
    for root, _, files in os.walk(out):
        for f in files:
            if f.endswith("counter_collection.csv"):
                with open(os.path.join(root, f)) as fh:
                    for r in csv.DictReader(fh):
                        if r["Counter_Name"] == counter:
                            rows.setdefault(r["Kernel_Name"], []).append((int(r["Grid_Size"]),
                                                                          float(r["Counter_Value"])))
    return rows or None


def measure_traffic(layers):
    """HBM bytes per full-layer fused launch: calibrated FETCH_SIZE + WRITE_SIZE (see the module docstring)."""
    tmp = tempfile.mkdtemp(prefix="lw_pmc_")
    try:
        res = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            rows = counter_pass(counter, layers, tmp)
            if not rows:
                return None
            ring = [v for k, vs in rows.items() if any(n in k for n in ("k_fused_tiles", "k_fused_flat", "k_fused_ring"))
                    for v in vs]
            copy = [v for k, vs in rows.items() if "copyBuffer" in k for v in vs]
            if not ring or not copy:
                return None
            grid = max(g for g, _ in ring)
            vals = [v for g, v in ring if g == grid]
            cal = max(copy)[1]                      # the 256 MiB copy: 262144 KiB read and written
            factor = (256 << 10) / cal if cal > 0 else 0.0
            res[counter] = (sum(vals) / len(vals), factor, grid)
        f, w = res["FETCH_SIZE"], res["WRITE_SIZE"]
        log("bench: traffic per layer launch (grid %d): FETCH %.0f KiB x %.3f, WRITE %.0f KiB x %.3f"
            % (f[2], f[0], f[1], w[0], w[1]))
        return (f[0] * f[1] + w[0] * w[1]) * 1024.0, f[1], w[1]
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def time_prefill(lib, rt, torch, names, infos, ms=(128, 512), reps=5):
    """Prefill shapes (fp32 x resident) over the named matrices through path 2 (decode to scratch + GEMM), per m
    with the default GEMM (hand-written on the matrix cores over tiled codes) and with rocBLAS over fp16 hi + lo
    weights (lw_set_prefill_gemm 4): ms per pass over the matrices and useful TFLOP/s (2 m N K per matrix)."""
    import ctypes
    stream = torch.cuda.current_stream().cuda_stream
    g = torch.Generator().manual_seed(5)
    runs = []
    for pm in ms:
        XP = [torch.randn(pm, inf["K"], generator=g).float().cuda() for inf in infos]
        YP = [torch.zeros(pm, inf["N"], device="cuda") for inf in infos]

        def one_pass():
            for nm, inf, x, y in zip(names, infos, XP, YP):
                if lib.lw_matmul_dev(rt.h, nm, ctypes.c_void_p(x.data_ptr()), 0, pm, ctypes.c_void_p(y.data_ptr()),
                                     inf["N"], stream) != 0:
                    raise RuntimeError(lib.lw_last_error().decode())
        flops = sum(2.0 * pm * inf["N"] * inf["K"] for inf in infos)
        run = {"m": pm}
        try:
            for which, key in ((0, "own_mfma"), (4, "rocblas")):
                lib.lw_set_prefill_gemm(which)
                one_pass()
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for _ in range(reps):
                    one_pass()
                torch.cuda.synchronize()
                fms = (time.perf_counter() - t0) * 1e3 / reps
                run[key] = {"ms_per_pass": round(fms, 3), "TFLOPs": round(flops / (fms * 1e-3) / 1e12, 1)}
        finally:
            lib.lw_set_prefill_gemm(0)
        run["own_over_rocblas"] = round(run["rocblas"]["ms_per_pass"] / run["own_mfma"]["ms_per_pass"], 2)
        runs.append(run)
        del XP, YP
    return runs


def time_config(lib, rt_cls, bundle, torch, work, key, mats, layers, ms, steps, prefill=False):
    """A further configuration of the benchmark contract: `layers` copies of its matrices (own seeds, together beyond
    the 256 MB Infinity Cache), one grouped call per layer and step, fp16 x resident. Per m: ms per step, GB/s of
    algorithmic coded bytes (as the headline), and the kernels alone timed with HIP events (lw_bench_groups) against
    the HBM peak; for m > 1 also the same tokens as m consecutive m = 1 steps. prefill: also the prefill shapes over
    layer 0's matrices, one figure per format (time_prefill)."""
    import ctypes
    d = os.path.join(work, key)
    lm = [("l%d.%s" % (l, nm), kqt, N, K, H, seed + 97 * l) for l in range(layers)
          for nm, kqt, N, K, H, seed in mats]
    bundle.write_synthetic_bundle(d, lm, threads=16)
    rt = rt_cls(d)
    try:
        infos = [rt.info(mt[0]) for mt in lm]
        n, per = len(lm), len(mats)
        stream = torch.cuda.current_stream().cuda_stream
        g = torch.Generator().manual_seed(11)
        mmax = max(ms)
        X = [torch.randn(mmax, inf["K"], generator=g).half().cuda() for inf in infos]
        Y = [torch.zeros(mmax, inf["N"], device="cuda") for inf in infos]
        names = (ctypes.c_char_p * n)(*[mt[0].encode() for mt in lm])
        xp = (ctypes.c_void_p * n)(*[x.data_ptr() for x in X])
        yp = (ctypes.c_void_p * n)(*[y.data_ptr() for y in Y])
        groups = [slice(per * l, per * l + per) for l in range(layers)]
        calls = [((ctypes.c_char_p * per)(*names[sl]), (ctypes.c_void_p * per)(*xp[sl]),
                  (ctypes.c_void_p * per)(*yp[sl])) for sl in groups]

        def timed(fn):
            # untimed runs for about 20 ms first: the clocks settle again after a change of workload
            t0 = time.perf_counter()
            while time.perf_counter() - t0 < 0.02:
                for _ in range(10):
                    fn()
                torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                fn()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e3 / steps

        res = {"layers": layers, "matrices": ["%s kqt %d %dx%d H=%.1f" % (nm, kqt, N, K, H)
                                              for nm, kqt, N, K, H, _ in mats],
               "coded_MB": round(sum(inf["blob_bytes"] + inf["side_bytes"] for inf in infos) / 1e6, 1)}
        for m in ms:
            def step():
                for nm, xx, yy in calls:
                    if lib.lw_group_matmul_dev(rt.h, per, nm, xx, m, yy, stream) != 0:
                        raise RuntimeError(lib.lw_last_error().decode())
            sms = timed(step)
            sbytes = float(sum(inf["blob_bytes"] + inf["side_bytes"] + 2 * inf["K"] * m + 4 * m * inf["N"]
                               for inf in infos))
            kbytes = float(sum(inf["blob_bytes"] + inf["side_bytes"] + 2 * inf["K"] * m for inf in infos))
            sizes = (ctypes.c_int * layers)(*([per] * layers))
            out = (ctypes.c_double * 3)()
            if lib.lw_bench_groups(rt.h, layers, sizes, names, xp, m, yp, 10, max(3, steps // 2), out) != 0:
                raise RuntimeError(lib.lw_last_error().decode())
            rec = {"ms_per_step": round(sms, 4), "GBps_coded": round(sbytes / (sms * 1e-3) / 1e9, 1),
                   "kernel_ms_per_pass": round(out[1], 4), "launches_per_pass": int(out[2]),
                   "roofline_frac": round(kbytes / (out[1] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            if m > 1:  # the same m tokens as m steps at m = 1 (config 4's comparison)
                singles = []
                for t in range(m):
                    for sl in groups:
                        singles.append(((ctypes.c_char_p * per)(*names[sl]),
                                        (ctypes.c_void_p * per)(*[X[i].data_ptr() + 2 * t * infos[i]["K"]
                                                                  for i in range(sl.start, sl.stop)]),
                                        (ctypes.c_void_p * per)(*[Y[i].data_ptr() + 4 * t * infos[i]["N"]
                                                                  for i in range(sl.start, sl.stop)])))

                def rep():
                    for nm, xx, yy in singles:
                        if lib.lw_group_matmul_dev(rt.h, per, nm, xx, 1, yy, stream) != 0:
                            raise RuntimeError(lib.lw_last_error().decode())
                rms = timed(rep)
                rec["repeated_m1"] = {"ms_per_step": round(rms, 4), "gemm_over_repeated": round(sms / rms, 3),
                                      "gemm_over_one_m1_step": None}
            res["m%d" % m] = rec
            log("bench: %s m=%d: %.3f ms per step (%d layers), %.1f GB/s coded, kernels %.1f%% of HBM peak%s"
                % (key, m, sms, layers, rec["GBps_coded"], 100 * rec["roofline_frac"],
                   "" if m == 1 else "; %d x m=1: %.3f ms" % (m, rec["repeated_m1"]["ms_per_step"])))
        if 1 in ms:
            for m in ms:
                if m > 1:
                    res["m%d" % m]["repeated_m1"]["gemm_over_one_m1_step"] = round(
                        res["m%d" % m]["ms_per_step"] / res["m1"]["ms_per_step"], 3)
        if prefill:
            res["prefill_path2"] = {}
            for kqt in sorted({mt[1] for mt in mats}):
                sel = [i for i in range(per) if lm[i][1] == kqt]
                fmt = {1: "Q4_K", 2: "Q5_K", 3: "Q6_K", 4: "IQ4_XS"}[kqt]
                runs = time_prefill(lib, rt, torch, [lm[i][0].encode() for i in sel], [infos[i] for i in sel])
                res["prefill_path2"][fmt] = {"matrices": [lm[i][0] for i in sel], "runs": runs}
                for r in runs:
                    log("bench: %s prefill %s m=%d: own %.3f ms (%.1f TFLOP/s), rocblas %.3f ms (%.1f TFLOP/s)"
                        % (key, fmt, r["m"], r["own_mfma"]["ms_per_pass"], r["own_mfma"]["TFLOPs"],
                           r["rocblas"]["ms_per_pass"], r["rocblas"]["TFLOPs"]))
        return res
    finally:
        rt.close()
        shutil.rmtree(d, ignore_errors=True)


def cpu_share():
    """Threads for the CPU baseline: every core this process may run on (its affinity mask), capped by the cgroup's
    CPU quota when one is set (a share of a larger host); plus what the host reports, for the record."""
    aff = len(os.sched_getaffinity(0))
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()
        if q != "max":
            quota = int(q) / int(period)
    except (OSError, ValueError):
        pass
    n = aff if quota is None else max(1, min(aff, int(math.ceil(quota))))
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return n, {"nproc": os.cpu_count(), "affinity_cores": aff, "cgroup_cpu_quota": quota, "cpu_model": model}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--m", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--workdir", default=None)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the two rocprofv3 counter passes")
    ap.add_argument("--no-packed", action="store_true", help="skip the packed-twin control")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill-shape figures (m = 128 and 512)")
    ap.add_argument("--no-configs", action="store_true", help="skip configs 1, 3 and 4 (Q5_K)")
    ap.add_argument("--only-configs", action="store_true",
                    help="time configs 1, 3 and 4 (Q5_K) only (for a kernel trace of their kernels)")
    ap.add_argument("--kernel-mode", type=int, default=0, help="lw_set_kernel_mode for the whole run (0 = auto)")
    ap.add_argument("--act8", action="store_true",
                    help="with --profile: int8 activations (lw_set_act8) for the passes, e.g. with --m 5")
    ap.add_argument("--profile", action="store_true",
                    help="counter-collection run: a few grouped passes over the layers plus a 256 MiB device copy "
                         "(the calibration for FETCH_SIZE / WRITE_SIZE), no timing, no JSON")
    ap.add_argument("--profile-config3", action="store_true",
                    help="with --profile: the passes over 4 config-3 layers (Q6_K down + IQ4_XS gate / up, one "
                         "grouped call per layer) instead, at --m tokens")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the path has no multi-GPU leg); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from lazyweights_amd import Runtime, bundle, load_library
    from lazyweights_amd.configs import CONFIG1, CONFIG3, CONFIG4, Q5_K, config2_layer

    def further_configs(work):
        steps = max(3, a.steps // 2)
        return {"config1": time_config(lib, Runtime, bundle, torch, work, "config1", CONFIG1, 8, (1,), steps),
                "config3": time_config(lib, Runtime, bundle, torch, work, "config3", CONFIG3, 4, (1, 5), steps,
                                       prefill=not a.no_prefill),
                "config4_q5k": time_config(lib, Runtime, bundle, torch, work, "config4_q5k",
                                           [mt for mt in CONFIG4 if mt[1] == Q5_K], 3, (1, 5), steps)}

    lib = load_library()
    if lib.lw_set_kernel_mode(a.kernel_mode) != 0:
        raise SystemExit("bench.py: unknown kernel mode %d" % a.kernel_mode)
    work = a.workdir or tempfile.mkdtemp(prefix="lw_bench_")
    os.makedirs(work, exist_ok=True)
    if a.only_configs:
        try:
            print(json.dumps(further_configs(work)), flush=True)
        finally:
            if not a.workdir:
                shutil.rmtree(work, ignore_errors=True)
        return
    if a.profile and a.profile_config3:
        import ctypes
        try:
            lm = [("l%d.%s" % (l, nm), kqt, N, K, H, seed + 97 * l) for l in range(4)
                  for nm, kqt, N, K, H, seed in CONFIG3]
            bundle.write_synthetic_bundle(work, lm, threads=16)
            rt = Runtime(work)
            infos = [rt.info(mt[0]) for mt in lm]
            g = torch.Generator().manual_seed(11)
            X = [torch.randn(a.m, inf["K"], generator=g).half().cuda() for inf in infos]
            Y = [torch.zeros(a.m, inf["N"], device="cuda") for inf in infos]
            stream = torch.cuda.current_stream().cuda_stream
            per = len(CONFIG3)
            calls = [((ctypes.c_char_p * per)(*[mt[0].encode() for mt in lm[per * l:per * l + per]]),
                      (ctypes.c_void_p * per)(*[x.data_ptr() for x in X[per * l:per * l + per]]),
                      (ctypes.c_void_p * per)(*[y.data_ptr() for y in Y[per * l:per * l + per]])) for l in range(4)]
            for _ in range(max(1, a.steps)):
                for nm, xx, yy in calls:
                    if lib.lw_group_matmul_dev(rt.h, per, nm, xx, a.m, yy, stream) != 0:
                        raise RuntimeError(lib.lw_last_error().decode())
            torch.cuda.synchronize()
            log("bench --profile --profile-config3: %d passes over 4 config-3 layers at m = %d done"
                % (max(1, a.steps), a.m))
            rt.close()
        finally:
            if not a.workdir:
                shutil.rmtree(work, ignore_errors=True)
        return
    try:
        t0 = time.time()
        mats = [m for l in range(a.layers) for m in config2_layer(l)]
        bundle.write_synthetic_bundle(work, mats, threads=16)
        log("bench: generated %d layers in %.1f s" % (a.layers, time.time() - t0))
        t0 = time.time()
        rt = Runtime(work)
        log("bench: opened (device layout built) in %.1f s; coded %.1f MB, device layout %.1f MB"
            % (time.time() - t0, rt.stat("coded_bytes") / 1e6, rt.stat("device_bytes") / 1e6))
        m = a.m
        infos = [rt.info(mt[0]) for mt in mats]
        algo = [inf["blob_bytes"] + inf["side_bytes"] + 2 * inf["K"] * m + 4 * m * inf["N"] for inf in infos]
        bytes_per_step = float(sum(algo))
        g = torch.Generator().manual_seed(0)
        X = [torch.randn(m, inf["K"], generator=g).half().cuda() for inf in infos]
        Y = [torch.zeros(m, inf["N"], device="cuda") for inf in infos]
        import ctypes
        n = len(mats)
        names = (ctypes.c_char_p * n)(*[mt[0].encode() for mt in mats])
        xp = (ctypes.c_void_p * n)(*[x.data_ptr() for x in X])
        yp = (ctypes.c_void_p * n)(*[y.data_ptr() for y in Y])
        stream = torch.cuda.current_stream().cuda_stream

        per_layer = []
        for l in range(a.layers):
            sl = slice(7 * l, 7 * l + 7)
            per_layer.append(((ctypes.c_char_p * 7)(*names[sl]), (ctypes.c_void_p * 7)(*xp[sl]),
                              (ctypes.c_void_p * 7)(*yp[sl])))

        def step():
            for nm, xx, yy in per_layer:
                if lib.lw_group_matmul_dev(rt.h, 7, nm, xx, m, yy, stream) != 0:
                    raise RuntimeError(lib.lw_last_error().decode())

        singles = [((ctypes.c_char_p * 1)(names[i]), (ctypes.c_void_p * 1)(xp[i]), (ctypes.c_void_p * 1)(yp[i]))
                   for i in range(n)]

        def serial_step():
            for nm, xx, yy in singles:
                if lib.lw_group_matmul_dev(rt.h, 1, nm, xx, m, yy, stream) != 0:
                    raise RuntimeError(lib.lw_last_error().decode())

        # a decode step in the order the reference's forward pass issues a layer's matmuls (rt_forward,
        # kernels/llmrt.cu:2366-2411): q, k, v together, then o, then gate and up together, then down, each launch
        # on the same stream after the one before (4 dependent launches per layer)
        dep = []
        for l in range(a.layers):
            for part in ((0, 1, 2), (3,), (4, 5), (6,)):
                ii = [7 * l + i for i in part]
                k_ = len(ii)
                dep.append((k_, (ctypes.c_char_p * k_)(*[names[i] for i in ii]),
                            (ctypes.c_void_p * k_)(*[xp[i] for i in ii]), (ctypes.c_void_p * k_)(*[yp[i] for i in ii])))

        def dependent_step():
            for k_, nm, xx, yy in dep:
                if lib.lw_group_matmul_dev(rt.h, k_, nm, xx, m, yy, stream) != 0:
                    raise RuntimeError(lib.lw_last_error().decode())

        if a.profile:
            if a.act8 and lib.lw_set_act8(1) != 0:
                raise SystemExit("bench.py: int8 activations refused: " + lib.lw_last_error().decode())
            for _ in range(max(1, a.steps)):
                step()
            lib.lw_set_act8(0)
            src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
            dst = torch.empty_like(src)
            dst.copy_(src)  # calibration: 256 MiB read + 256 MiB written
            torch.cuda.synchronize()
            lib.lw_stream_read_gbps(256 << 20, 1)  # calibration: k_stream_read, 256 MiB read per launch
            log("bench --profile: %d passes over %d layers + 256 MiB copy done" % (max(1, a.steps), a.layers))
            rt.close()
            return
        # dominant kernel: HIP events around each pass of the fused launches, on the library's stream (an event
        # between two launches costs the stream about 2 us). It runs first, after 60
        # untimed passes (about 20 ms): under sustained load the GPU's clocks ramp up over the first 10-15 ms (the
        # kernel trace shows the layer launch going from 43-44 us to 39.7-40 us over its first ~300 launches), which
        # would otherwise land in whichever measurement came first; the headline's W warmup and K timed steps follow
        sizes = (ctypes.c_int * a.layers)(*([7] * a.layers))
        out = (ctypes.c_double * 3)()
        rc = lib.lw_bench_groups(rt.h, a.layers, sizes, names, xp, m, yp, 60, max(3, a.steps // 2), out)
        if rc != 0:
            raise RuntimeError(lib.lw_last_error().decode())
        kernel_ms_per_pass = out[1]
        launches = int(out[2])
        kbytes = float(sum(inf["blob_bytes"] + inf["side_bytes"] + 2 * inf["K"] * m for inf in infos))
        achieved = kbytes / (kernel_ms_per_pass * 1e-3) / 1e9
        layer_us = kernel_ms_per_pass * 1e3 / a.layers
        log("bench: fused kernels %.3f ms per pass (%d launches for %d layers, %.1f us per layer), %.1f GB/s"
            % (kernel_ms_per_pass, launches, a.layers, layer_us, achieved))
        for _ in range(a.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            step()
        torch.cuda.synchronize()
        ms_per_step = (time.perf_counter() - t0) * 1e3 / a.steps
        value = bytes_per_step / (ms_per_step * 1e-3) / 1e9
        log("bench: %.3f ms per step (%d GEMVs), %.1f GB/s coded" % (ms_per_step, n, value))
        # speculative verify (config 4: m = 5 tokens on the same layers, one grouped call per layer), timed right
        # after the m = 1 step it is compared with, before the other measurements' allocations: fp16 x and
        # int8 x (one pass over the weights for all tokens); bytes as m = 1 plus 5x the x and y traffic
        verify = None
        if m == 1:
            vm = 5
            XV = [torch.randn(vm, inf["K"], generator=g).half().cuda() for inf in infos]
            YV = [torch.zeros(vm, inf["N"], device="cuda") for inf in infos]
            vcalls = []
            for l in range(a.layers):
                sl = slice(7 * l, 7 * l + 7)
                vcalls.append(((ctypes.c_char_p * 7)(*names[sl]),
                               (ctypes.c_void_p * 7)(*[x.data_ptr() for x in XV[sl]]),
                               (ctypes.c_void_p * 7)(*[y.data_ptr() for y in YV[sl]])))
            vbytes = float(sum(inf["blob_bytes"] + inf["side_bytes"] + 2 * inf["K"] * vm + 4 * vm * inf["N"]
                               for inf in infos))
            verify = {"m": vm}
            for a8, key in ((0, "fp16_x"), (1, "int8_x")):
                lib.lw_set_act8(a8)
                try:
                    def vstep():
                        for nm, xx, yy in vcalls:
                            if lib.lw_group_matmul_dev(rt.h, 7, nm, xx, vm, yy, stream) != 0:
                                raise RuntimeError(lib.lw_last_error().decode())
                    for _ in range(max(40, a.warmup)):  # about 17 ms: the clocks settle again after the switch
                        vstep()
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                    for _ in range(a.steps):
                        vstep()
                    torch.cuda.synchronize()
                    vms = (time.perf_counter() - t0) * 1e3 / a.steps
                finally:
                    lib.lw_set_act8(0)
                verify[key] = {"ms_per_step": round(vms, 4), "GBps_coded": round(vbytes / (vms * 1e-3) / 1e9, 1),
                               "over_one_m1_step": round(vms / ms_per_step, 3)}
                log("bench: verify m=%d (%s): %.3f ms per step, %.1f GB/s coded" % (vm, key, vms, verify[key]["GBps_coded"]))
            # config 4's comparison: the 5 tokens as 5 m = 1 steps over the same layers (the headline step, timed above)
            verify["five_m1_steps_ms"] = round(vm * ms_per_step, 4)
            verify["fp16_x"]["over_five_m1_steps"] = round(verify["fp16_x"]["ms_per_step"] / (vm * ms_per_step), 3)
            del XV, YV

        serial_step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            serial_step()
        torch.cuda.synchronize()
        serial_ms = (time.perf_counter() - t0) * 1e3 / a.steps
        log("bench: serial per-matrix launches %.3f ms per step, %.1f GB/s coded"
            % (serial_ms, bytes_per_step / (serial_ms * 1e-3) / 1e9))
        for _ in range(max(20, a.warmup)):
            dependent_step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            dependent_step()
        torch.cuda.synchronize()
        dep_ms = (time.perf_counter() - t0) * 1e3 / a.steps
        log("bench: decode step in forward order (4 launches per layer) %.3f ms per step, %.1f GB/s coded"
            % (dep_ms, bytes_per_step / (dep_ms * 1e-3) / 1e9))

        ctrl = lib.lw_stream_read_gbps(1 << 31, 10)
        log("bench: streaming-read control %.1f GB/s" % ctrl)
        # decode only (the reference's decode bench, rt_gpu_decode_all): every matrix of the workload to code bytes,
        # median of 5 passes
        dsec = lib.rt_gpu_decode_all(rt.h, 5)
        ncodes = float(sum(inf["N"] * inf["K"] for inf in infos))
        decode_only = {"ms_per_pass": round(dsec * 1e3, 4), "Gcodes_per_s": round(ncodes / dsec / 1e9, 1),
                       "kernel": "k_decode_split"} if dsec > 0 else None
        if decode_only:
            log("bench: decode only %.3f ms per pass over %d layers, %.1f G codes/s"
                % (dsec * 1e3, a.layers, decode_only["Gcodes_per_s"]))

        # int8 activations (the reference's default act8 mode; m = 1 only): the same step with x quantized per block
        # of 32 on the device (one quantization launch per distinct x) and integer sub-block dot products
        act8 = None
        if m == 1:
            lib.lw_set_act8(1)
            try:
                for _ in range(max(40, a.warmup)):  # about 14 ms: the clocks settle again after the decode pass
                    step()
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for _ in range(a.steps):
                    step()
                torch.cuda.synchronize()
                ams = (time.perf_counter() - t0) * 1e3 / a.steps
                out8 = (ctypes.c_double * 3)()
                if lib.lw_bench_groups(rt.h, a.layers, sizes, names, xp, m, yp, 1, max(3, a.steps // 2), out8) != 0:
                    raise RuntimeError(lib.lw_last_error().decode())
            finally:
                lib.lw_set_act8(0)
            act8 = {"ms_per_step": round(ams, 4), "GBps_coded": round(bytes_per_step / (ams * 1e-3) / 1e9, 1),
                    "kernel_ms_per_pass": round(out8[1], 4), "launches_per_pass": int(out8[2]),
                    "speed_vs_fp16_x": round(ms_per_step / ams, 3)}
            log("bench: int8 activations %.3f ms per step (%.1f GB/s coded; kernels %.3f ms per pass, %d launches)"
                % (ams, act8["GBps_coded"], out8[1], int(out8[2])))

        # prefill shapes (m = 128 and 512, fp32 x resident): the decode-to-scratch path (path 2) over layer 0's seven
        # matrices, with the default GEMM (the hand-written matrix-core GEMM over the codes, k_gemm_prefill) and with
        # rocBLAS over fp16 hi + lo weights (a reported figure, not the metric); config 3 adds Q6_K and IQ4_XS
        prefill = None
        if not a.no_prefill:
            prefill = {"path": "own_mfma (default): codes decoded to scratch in a tiled layout, v_mfma_f32_32x32x16_f16 "
                               "with fp16 hi + lo x and fp32 accumulation (Q4_K / Q5_K: weights scaled by their 6-bit "
                               "sub-scales, exact in fp16; Q6_K / IQ4_XS: grid values, folded per sub-block in fp32); "
                               "rocblas: codes dequantized to fp16 hi + lo weights, rocBLAS fp16 GEMM (one GEMM over "
                               "2m columns up to m = 512)",
                       "matrices": "config 2 layer 0 (Q4_K)",
                       "runs": time_prefill(lib, rt, torch, [names[i] for i in range(7)], infos[:7])}
            for r in prefill["runs"]:
                log("bench: prefill m=%d: own %.3f ms per layer (%.1f TFLOP/s), rocblas %.3f ms (%.1f TFLOP/s)"
                    % (r["m"], r["own_mfma"]["ms_per_pass"], r["own_mfma"]["TFLOPs"], r["rocblas"]["ms_per_pass"],
                       r["rocblas"]["TFLOPs"]))

        configs = None if a.no_configs else further_configs(work)

        # packed-twin control: the same codes stored fixed-rate (pk4 / pk8), no decode chain; the achievable rate of
        # this access pattern and arithmetic without entropy decoding (the reference's pk4 baseline)
        packed = None
        if not a.no_packed:
            pdir = os.path.join(work, "packed")
            bundle.write_packed_bundle(pdir, mats, threads=16)
            rtp = Runtime(pdir)
            pbytes = float(sum(rtp.info(mt[0])["blob_bytes"] + rtp.info(mt[0])["side_bytes"] + 2 * mt[3] * m
                               + 4 * m * mt[2] for mt in mats))

            def pstep():
                for nm, xx, yy in per_layer:
                    if lib.lw_group_matmul_dev(rtp.h, 7, nm, xx, m, yy, stream) != 0:
                        raise RuntimeError(lib.lw_last_error().decode())
            pstep()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(a.steps):
                pstep()
            torch.cuda.synchronize()
            pms = (time.perf_counter() - t0) * 1e3 / a.steps
            rtp.close()
            packed = {"ms_per_step": round(pms, 4), "GBps_packed_bytes": round(pbytes / (pms * 1e-3) / 1e9, 1),
                      "speed_vs_coded": round(ms_per_step / pms, 3), "kernel": "k_fused_packed"}
            log("bench: packed-twin control %.3f ms per step, %.1f GB/s of packed bytes (%.2fx the coded step)"
                % (pms, packed["GBps_packed_bytes"], ms_per_step / pms))

        traffic = None
        if not a.no_traffic:
            t = measure_traffic(a.layers)
            if t:
                traffic = {"bytes_per_layer_launch": int(t[0]), "algorithmic_bytes_per_layer": int(kbytes / a.layers),
                           "fetch_factor": round(t[1], 3), "write_factor": round(t[2], 3)}
                log("bench: HBM traffic %.1f MB per layer launch vs %.1f MB algorithmic"
                    % (t[0] / 1e6, kbytes / a.layers / 1e6))

        cpu = None
        if not a.no_cpu:
            from oracle import oracle as orc
            threads, host = cpu_share()
            coded_total = float(sum(inf["blob_bytes"] for inf in infos))
            cfg, ts = bundle.read_manifest(work)
            by = {t["name"]: t for t in ts}
            layer0 = config2_layer(0)
            blobs = [(bundle.read_tensor(work, by[nm]), bundle.read_tensor(work, by[nm + ".kqs"]), N, K)
                     for nm, _, N, K, _, _ in layer0]
            xs = [X[i][0].float().cpu().numpy() for i in range(7)]
            sample_bytes = sum(len(b) + len(s) + 2 * K + 4 * N for b, s, N, K in blobs)
            reps, t_cpu = 0, 0.0
            while t_cpu < a.cpu_seconds and reps < 1000:
                t0 = time.perf_counter()
                for (b, s, N, K), x in zip(blobs, xs):
                    orc.decode_gemv(1, b, s, N, K, x, threads)
                t_cpu += time.perf_counter() - t0
                reps += 1
            cpu_gbs = sample_bytes * reps / t_cpu / 1e9
            # the reference's own CPU setting (6 threads, results/a2_orin/decode7), a shorter sample
            reps6, t6 = 0, 0.0
            while t6 < a.cpu_seconds / 2 and reps6 < 1000:
                t0 = time.perf_counter()
                for (b, s, N, K), x in zip(blobs, xs):
                    orc.decode_gemv(1, b, s, N, K, x, min(6, threads))
                t6 += time.perf_counter() - t0
                reps6 += 1
            # decode only, the reference's CPU decode bench (rt_cpu_decode_all: every coded matrix of the workload,
            # blobs read before the clock starts, kernels/llmrt.cu:2558-2573), on all cores and on 6
            dec = {}
            for nth in sorted({threads, min(6, threads)}, reverse=True):
                s_dec, nsym = rt.cpu_decode_all(nth)
                dec[nth] = {"threads": nth, "seconds": round(s_dec, 3), "symbols": int(nsym),
                            "Gsym_per_s": round(nsym / s_dec / 1e9, 3),
                            "GBps_coded": round(coded_total / s_dec / 1e9, 3)}
            cpu = {"value": round(cpu_gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
                   "sample": "layer 0 of the workload (7 matrices, %.1f MB coded), %d passes, %.1f s; "
                             "oracle cpu_decode + dequant + fp32 GEMV" % (sample_bytes / 1e6, reps, t_cpu),
                   "value_6_threads": round(sample_bytes * reps6 / t6 / 1e9, 3),
                   "host": host,
                   "decode_only": {"what": "rt_cpu_decode_all over the %d layers (%.1f MB coded), symbols to memory"
                                           % (a.layers, coded_total / 1e6),
                                   "all_cores": dec[threads], "six_threads": dec[min(6, threads)]}}
            log("bench: cpu baseline %.2f GB/s on %d threads, %.2f GB/s on %d; decode only %.2f G symbols/s on %d"
                % (cpu_gbs, threads, cpu["value_6_threads"], min(6, threads), dec[threads]["Gsym_per_s"], threads))

        res = {
            "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
            "warmup": a.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp16*fp16->fp32", "data": "synthetic",
            "config": {"workload": "config2: Mistral-7B-shaped Q4_K layers (q,k,v,o,gate,up,down), H=2.3 bits/code, "
                                   "fp16 x, batch %d, %d distinct layers per step, grouped per layer" % (m, a.layers),
                       "layers": a.layers, "m": m, "coded_bytes_per_step": int(bytes_per_step),
                       "hbm_fraction": round(value / HBM_PEAK_GBS, 4)},
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "traffic": traffic["bytes_per_layer_launch"] if traffic else None,
                         "traffic_detail": traffic,
                         "kernel": {0: "k_fused_tiles", 6: "k_fused_tiles", 8: "k_fused_halves",
                                    9: "k_fused_tiles (comparator lookup)"}.get(a.kernel_mode, "k_fused_flat"),
                         "launch": "one grouped launch per layer",
                         "mean_launch_us": round(layer_us, 2), "launches_per_pass": launches},
            "serial_per_matrix": {"ms_per_step": round(serial_ms, 4),
                                  "GBps": round(bytes_per_step / (serial_ms * 1e-3) / 1e9, 1)},
            "decode_step_forward_order": {"launches_per_layer": 4, "ms_per_step": round(dep_ms, 4),
                                          "us_per_layer": round(dep_ms * 1e3 / a.layers, 2),
                                          "GBps": round(bytes_per_step / (dep_ms * 1e-3) / 1e9, 1)},
            "cpu_baseline": cpu,
            "control_stream_read_GBps": round(ctrl, 1),
            "control_packed_twin": packed,
            "act8": act8,
            "decode_only": decode_only,
            "verify_m5": verify,
            "prefill_path2": prefill,
            "configs": configs,
        }
        print(json.dumps(res), flush=True)
        rt.close()
    finally:
        if not a.workdir:
            shutil.rmtree(work, ignore_errors=True)


if __name__ == "__main__":
    main()
