"""Per-wave timeline of the whole-tile kernel (k_fused_tiles) on config-2 layers: where a layer launch's time goes.

    python -m lazyweights_amd.build --timeline      # once: liblazyweights_amd_timeline.so (device code -DLW_TIMELINE)
    python -m lazyweights_amd.timeline [--layers 8] [--steps 20]

The diagnostic library is the product's source with timestamps added (s_memrealtime, 100 MHz, stored by lane 0 of
each wave: its start, the tables' barrier, each tile in LDS / decoded / next copy issued, its end; nothing else
changes, the results are the same bits). After warm-up steps (clocks at their working level) the timestamps of the
last layer launch of one step are read back and summarised as Markdown: when the first tiles land, how many waves
decode per CU over the launch, each wave index's start, tiles and end (medians over the blocks), and the end phase
(the last decode to each block's last wave end: the in-launch reductions).
"""
import argparse
import ctypes
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TL_BLOCKS, TL_WAVES, TL_SLOTS = 1024, 16, 32


def summarise(ts, W, clk_hz=1e8):
    """ts [blocks, TL_WAVES, TL_SLOTS] int64 timestamps of one launch (0 = unset) -> Markdown lines."""
    live = ts[:, :, 0] > 0
    blocks = int(live.any(1).sum())
    t0 = ts[:, :, 0][live].min()
    us = lambda v: (v - t0) / clk_hz * 1e6
    units = []  # (block, wave, tile index, landed us, decoded us)
    for b in range(blocks):
        for w in range(W):
            if not live[b, w]:
                continue
            a0, a1 = ts[b, w, 0], ts[b, w, 3]
            for i in range(8):
                r, e = ts[b, w, 4 + 3 * i], ts[b, w, 5 + 3 * i]
                if a0 <= r <= e <= a1:
                    units.append((b, w, i, us(r), us(e)))
    u = np.array(units)
    end = us(ts[:, :, 3][live].max())
    first = np.array([u[u[:, 0] == b][:, 3].min() for b in range(blocks)])
    last_dec = np.array([u[u[:, 0] == b][:, 4].max() for b in range(blocks)])
    blk_end = np.array([us(ts[b, :, 3][live[b]].max()) for b in range(blocks)])
    out = ["| launch | blocks | waves per block | tiles | last wave end |", "|---|---|---|---|---|",
           "| one config-2 layer | %d | %d | %d (%.1f per block) | %.2f us |" % (blocks, W, len(u), len(u) / blocks, end),
           "",
           "| phase | median over blocks | p10 | p90 |", "|---|---|---|---|",
           "| first tile in LDS | %.2f us | %.2f | %.2f |" % (np.median(first), np.percentile(first, 10),
                                                          np.percentile(first, 90)),
           "| last decode done | %.2f us | %.2f | %.2f |" % (np.median(last_dec), np.percentile(last_dec, 10),
                                                           np.percentile(last_dec, 90)),
           "| block end (last wave) | %.2f us | %.2f | %.2f |" % (np.median(blk_end), np.percentile(blk_end, 10),
                                                               np.percentile(blk_end, 90)),
           "| block end - last decode (in-launch reductions) | %.2f us | %.2f | %.2f |" % (
               np.median(blk_end - last_dec), np.percentile(blk_end - last_dec, 10),
               np.percentile(blk_end - last_dec, 90)),
           "", "Decoding waves per CU (mean over the window) and tiles finished per CU:", "",
           "| window | decoding waves | tiles finished |", "|---|---|---|"]
    grid = np.arange(0, end, 0.25)
    occ = np.array([((u[:, 3] <= g) & (u[:, 4] > g)).sum() / blocks for g in grid])
    for lo in range(0, int(np.ceil(end / 5.0)) * 5, 5):
        m = (grid >= lo) & (grid < lo + 5)
        done = ((u[:, 4] >= lo) & (u[:, 4] < lo + 5)).sum() / blocks
        out.append("| %d-%d us | %.2f | %.2f |" % (lo, lo + 5, occ[m].mean() if m.any() else 0.0, done))
    out += ["", "Per wave index (medians over the blocks): its first tile in LDS, its last decode done, tiles decoded, "
            "the first and second tile's decode time:", "",
            "| wave | first tile in LDS | last decode done | tiles | decode 1 | decode 2 |", "|---|---|---|---|---|---|"]
    for w in range(W):
        uw = u[u[:, 1] == w]
        if not len(uw):
            continue
        firsts, lasts, counts, d1, d2 = [], [], [], [], []
        for b in range(blocks):
            ub = uw[uw[:, 0] == b]
            if not len(ub):
                continue
            ub = ub[np.argsort(ub[:, 2])]
            firsts.append(ub[0, 3])
            lasts.append(ub[-1, 4])
            counts.append(len(ub))
            d1.append(ub[0, 4] - ub[0, 3])
            if len(ub) > 1:
                d2.append(ub[1, 4] - ub[1, 3])
        out.append("| %d | %.2f us | %.2f us | %.2f | %.2f us | %s |" % (
            w, np.median(firsts), np.median(lasts), np.mean(counts), np.median(d1),
            ("%.2f us" % np.median(d2)) if d2 else "-"))
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--lib", default=None, help="the diagnostic library (default: the in-tree timeline build)")
    a = ap.parse_args()
    sys.path.insert(0, ROOT)
    from lazyweights_amd import build as lwbuild
    path = a.lib or lwbuild.TIMELINE_LIB
    if not os.path.exists(path):
        raise SystemExit("timeline: %s is not built (python -m lazyweights_amd.build --timeline)" % path)
    os.environ["LAZYWEIGHTS_AMD_LIB"] = path  # the runtime's library for this process
    import torch
    from lazyweights_amd import bundle, configs
    from lazyweights_amd import runtime as lwrt
    from lazyweights_amd._lib import load_library
    lib = load_library()
    lib.lw_timeline_read.restype = ctypes.c_int
    lib.lw_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    lib.lw_timeline_clear.restype = ctypes.c_int
    work = tempfile.mkdtemp(prefix="lw_timeline_")
    mats = [m for l in range(a.layers) for m in configs.config2_layer(l)]
    bundle.write_synthetic_bundle(work, mats, threads=16)
    rt = lwrt.Runtime(work)
    names = [m[0] for m in mats]
    infos = [rt.info(n) for n in names]
    g = torch.Generator().manual_seed(3)
    X = [torch.randn(1, i["K"], generator=g).half().cuda() for i in infos]
    Y = [torch.zeros(1, i["N"], device="cuda") for i in infos]
    stream = torch.cuda.current_stream().cuda_stream
    calls = []
    for l in range(a.layers):
        sl = slice(7 * l, 7 * l + 7)
        calls.append(((ctypes.c_char_p * 7)(*[n.encode() for n in names[sl]]),
                      (ctypes.c_void_p * 7)(*[x.data_ptr() for x in X[sl]]),
                      (ctypes.c_void_p * 7)(*[y.data_ptr() for y in Y[sl]])))

    def step():
        for nm, xp, yp in calls:
            if lib.lw_group_matmul_dev(rt.h, 7, nm, xp, 1, yp, ctypes.c_void_p(stream)) != 0:
                raise RuntimeError(lib.lw_last_error().decode())
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.05:  # clocks up to their working level
        for _ in range(5):
            step()
        torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / a.steps
    if lib.lw_timeline_clear() != 0:
        raise RuntimeError("lw_timeline_clear failed")
    step()
    torch.cuda.synchronize()
    buf = np.zeros(TL_BLOCKS * TL_WAVES * TL_SLOTS, np.uint64)
    if lib.lw_timeline_read(buf.ctypes.data, buf.nbytes) != 0:
        raise RuntimeError("lw_timeline_read failed")
    ts = buf.reshape(TL_BLOCKS, TL_WAVES, TL_SLOTS).astype(np.int64)
    W = int((ts[0, :, 0] > 0).sum())
    rt.close()
    print("Diagnostic build, %d config-2 layers: %.4f ms per step (%.2f us per layer launch); the timestamps of the "
          "last layer launch of one step." % (a.layers, ms, ms * 1e3 / a.layers))
    print()
    print("\n".join(summarise(ts, W)))


if __name__ == "__main__":
    main()
