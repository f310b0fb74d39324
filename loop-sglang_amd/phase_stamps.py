"""Per-row phase table of the sampler, from the phase-stamp profiling build.

Build the profiling library first (here, not on the GPU):
    python loop-sglang_amd/build.py --stamps
then, on the GPU:
    python loop-sglang_amd/phase_stamps.py [--workload sample_huginn] [--nbuf 5]
(`--workload coda_ouro` samples the bf16 logits of the package's LM head on the
fused-coda inputs.)

The profiling build (libloopsgl_tok_stamps.so, -DLSG_PHASE_STAMPS) has thread 0
of every workgroup of the streamed-row sampler (or, for batches of no more rows
than compute units, of the one-row-per-workgroup sampler) write the 100 MHz
real-time counter at fixed points of its row (start, wave 0's pass done, barrier 1 passed,
floor known, candidates staged, end), its hardware/XCC ids and the path the row
took.  The script rotates `nbuf` logits buffers (so the timed launch reads from
HBM, not from the Infinity Cache), times eager launches, then reads the stamps
of one launch and prints the per-phase percentiles, the start/end spread of the
workgroups and the path counts.
"""
from __future__ import annotations

import argparse
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SLOTS, ROWS = 8, 8192
PATHS = {1: "window", 2: "two-pass top-p", 3: "exact refinement", 4: "unfiltered walk", 5: "argmax",
         6: "small window"}
# the one-row-per-workgroup sampler (batches of no more rows than compute units)
ROW_PATHS = {1: "unfiltered walk", 2: "window <= 128", 3: "ranked window", 4: "dense top-p", 5: "exact refinement",
             6: "argmax"}


ROW_SLOTS = 16


def row_sampler_table(st, B):
    """Phases of the one-row-per-workgroup sampler (slots: 0 entry, 1 passes
    done, 2 window staged, 3-5 dense path: histogram, bracket, gather,
    7 threshold known, 8 id written, 9 dense path: kept masses, 10 inverse-CDF
    barrier passed, 6 ids and path)."""
    info = st[:, 6]
    path_of = (info >> 40) & 0xFF
    base = st[:, 0].min()
    rel = (st - base) * 0.01
    # slots a row's path does not write keep values of earlier launches: count a stamp only when it
    # is not earlier than the row's own entry stamp
    have = lambda c: (st[:, c] > 0) & (st[:, c] >= st[:, 0])
    pct = lambda v: "p50 %6.2f  p90 %6.2f  max %6.2f" % (np.median(v), np.percentile(v, 90), v.max())
    print("kernel entry (rel. first):", pct(rel[:, 0]))
    print("threshold known (rel. first):", pct(rel[have(7), 7]))
    print("id written (rel. first):", pct(rel[have(8), 8]))
    for name, c0, c1 in [("entry -> passes done", 0, 1), ("passes done -> window staged", 1, 2),
                         ("window staged -> threshold", 2, 7), ("dense: staged -> histogram", 2, 3),
                         ("dense: histogram -> bracket", 3, 4), ("dense: bracket -> gathered", 4, 5),
                         ("dense: gathered -> threshold", 5, 7), ("threshold -> id written", 7, 8),
                         ("dense: threshold -> kept masses", 7, 9), ("kept masses -> walk barrier", 9, 10),
                         ("walk barrier -> id written", 10, 8)]:
        ok = have(c0) & have(c1) & (st[:, c1] >= st[:, c0])
        if ok.any():
            print(f"{name:34s} ({ok.sum():4d} rows): {pct(rel[ok, c1] - rel[ok, c0])}")
    for code in sorted(set(path_of.tolist())):
        sel = (path_of == code) & have(7)
        if sel.any():
            print(f"path {ROW_PATHS.get(code, code)!s:18s}: {sel.sum():4d} rows, entry -> threshold "
                  f"{pct(rel[sel, 7] - rel[sel, 0])}")
            end = sel & have(8)
            if end.any():
                print(f"{'':23s}{end.sum():4d} rows, entry -> id written  {pct(rel[end, 8] - rel[end, 0])}")
            steps = [("passes", 0, 1), ("window attempt", 1, 2), ("to threshold", 2, 7), ("walk", 7, 8)]
            print(f"{'':23s}p50 " + ", ".join(
                f"{nm} {np.median(rel[sel & have(c1), c1] - rel[sel & have(c1), c0]):.2f}"
                for nm, c0, c1 in steps if (sel & have(c1)).any()))


def coda_logits(torch, pkg, dev, nbuf):
    """bf16 logits [256, 49152] of the package's LM head (lsg_lm_head) on the fused-coda bench inputs:
    h ~ N(0, 1) [256, 2048], W ~ N(0, 0.02^2) [49152, 2048] (one W per buffer, drawn in the bench's
    order from the same seeded generator), with the bench's temperatures, top-k, top-p and uniforms."""
    B, H, V = 256, 2048, 49152
    g = torch.Generator(device=dev).manual_seed(1)
    h = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
    bufs = []
    for _ in range(3):  # the bench draws three weight copies before the sampling arguments
        W = (torch.randn(V, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        bufs.append(pkg.coda.lm_head(h, W))
        del W
    T = 0.3 + 0.9 * torch.rand(B, generator=g, device=dev)
    Kt = torch.tensor([1, 20, 50, V], dtype=torch.int32, device=dev)[
        torch.randint(0, 4, (B,), generator=g, device=dev)].contiguous()
    P = 0.8 + 0.2 * torch.rand(B, generator=g, device=dev)
    U = torch.rand(B, generator=g, device=dev)
    g2 = torch.Generator(device=dev).manual_seed(2)
    while len(bufs) < nbuf:  # further buffers: more weight draws of the same distribution
        W = (torch.randn(V, H, generator=g2, device=dev) * 0.02).to(torch.bfloat16)
        bufs.append(pkg.coda.lm_head(h, W))
        del W
    return bufs[:nbuf], (T, Kt, P, U)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="sample_huginn",
                    choices=["sample_huginn", "sample_ouro", "cdb_mixed_depth", "coda_ouro"])
    ap.add_argument("--nbuf", type=int, default=5)
    ap.add_argument("--launches", type=int, default=20)
    ap.add_argument("--lib", default=os.path.join(HERE, "libloopsgl_tok_stamps.so"),
                    help="profiling library (a -DLSG_PHASE_STAMPS build)")
    a = ap.parse_args()
    sys.path.insert(0, ROOT)
    import torch

    import __graft_entry__

    pkg = __graft_entry__.package()
    path = a.lib
    if not os.path.exists(path):
        raise SystemExit(f"{path} missing: run python loop-sglang_amd/build.py --stamps first")
    pkg._lib.use_library(path)
    L = pkg._lib.load()
    L.lsg_phase_stamps_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    L.lsg_phase_stamps_read.restype = ctypes.c_int
    dev = torch.device("cuda:0")
    if a.workload == "coda_ouro":
        bufs, args = coda_logits(torch, pkg, dev, a.nbuf)
    else:
        make = getattr(pkg.workloads, a.workload)
        wl = make(dev, seed=3 if a.workload == "sample_huginn" else 1)
        bufs = [wl["logits"]] + [make(dev, seed=100 + i)["logits"] for i in range(a.nbuf - 1)]
        args = (wl["temperatures"], wl.get("top_k"), wl["top_p"], wl["uniforms"])
    B = bufs[0].shape[0]
    for i in range(2 * a.nbuf):
        pkg.sample_rows(bufs[i % a.nbuf], *args)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(a.launches):
        pkg.sample_rows(bufs[i % a.nbuf], *args)
    t1.record()
    torch.cuda.synchronize()
    print(f"{a.workload}: {a.nbuf} buffers rotated, eager launch {t0.elapsed_time(t1) / a.launches * 1e3:.1f} us")
    # the stamped launch reads a buffer the previous launch did not touch
    pkg.sample_rows(bufs[(a.launches + 1) % a.nbuf], *args)
    torch.cuda.synchronize()
    raw = np.zeros(ROWS * SLOTS, dtype=np.uint64)
    if B <= torch.cuda.get_device_properties(dev).multi_processor_count:
        L.lsg_row_stamps_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
        L.lsg_row_stamps_read.restype = ctypes.c_int
        raw = np.zeros(ROWS * ROW_SLOTS, dtype=np.uint64)
        if L.lsg_row_stamps_read(raw.ctypes.data, raw.nbytes) != 0:
            raise SystemExit("lsg_row_stamps_read failed")
        row_sampler_table(raw.reshape(ROWS, ROW_SLOTS)[:B].astype(np.int64), B)
        return
    if L.lsg_phase_stamps_read(raw.ctypes.data, raw.nbytes) != 0:
        raise SystemExit("lsg_phase_stamps_read failed")
    st = raw.reshape(ROWS, SLOTS)[:min(B, ROWS)].astype(np.int64)
    info = st[:, 6]
    path_of = (info >> 40) & 0xFF
    xcc = (info >> 32) & 0xFF
    cu = (xcc << 8) | ((info >> 8) & 0xFF)  # XCC id, then HW_ID's CU, SH and SE fields
    ts = st[:, [0, 7, 1, 2, 3, 4, 5]]  # entry, loads issued, pass done, barrier 1, floor, staged, end
    base = ts[:, 0].min()
    rel = (ts - base) * 0.01  # us (100 MHz counter)
    have = lambda c: ts[:, c] > 0
    pct = lambda v: "p50 %6.2f  p90 %6.2f  max %6.2f" % (np.median(v), np.percentile(v, 90), v.max())
    print("kernel entry (rel. first):", pct(rel[:, 0]))
    print("row end      (rel. first):", pct(rel[:, 6]))
    order = np.argsort(rel[:, 0])
    q = [0, B // 4, B // 2, 3 * B // 4, B - 1]
    print("sorted entries at ranks", q, ":", np.round(rel[order[q], 0], 2))
    phases = [("entry -> loads issued", 0, 1), ("loads issued -> wave 0 pass done", 1, 2),
              ("pass done -> barrier 1", 2, 3), ("barrier 1 -> floor", 3, 4),
              ("floor -> staged (barrier 2)", 4, 5), ("staged -> end", 5, 6), ("row total", 0, 6)]
    for name, c0, c1 in phases:
        ok = have(c0) & have(c1) & (ts[:, c1] >= ts[:, c0])
        if ok.any():
            print(f"{name:34s} ({ok.sum():5d} rows): {pct(rel[ok, c1] - rel[ok, c0])}")
    for code in sorted(set(path_of.tolist())):
        sel = path_of == code
        dur = rel[sel, 6] - rel[sel, 0]
        print(f"path {PATHS.get(code, code)!s:18s}: {sel.sum():5d} rows, row time {pct(dur)}")
    per_cu = np.bincount(np.unique(cu, return_inverse=True)[1])
    print(f"distinct compute units: {len(per_cu)}, rows per unit: min {per_cu.min()} max {per_cu.max()}")
    for x in sorted(set(xcc.tolist())):
        sel = xcc == x
        print(f"  XCC {x}: {sel.sum():4d} rows, entry {pct(rel[sel, 0])} | end {pct(rel[sel, 6])}")
    # per compute unit: the order its rows finished and the gaps between their ends
    units = np.unique(cu)
    last_end = np.array([rel[cu == c, 6].max() for c in units])
    print("compute-unit last row end:", pct(last_end))
    # timelines of the compute units finishing first, at the median and last
    for c in units[np.argsort(last_end)[[0, len(units) // 2, -1]]]:
        rows = np.nonzero(cu == c)[0]
        rows = rows[np.argsort(rel[rows, 1])]
        print(f"unit {c:#x}: rows (loads issued / pass done / barrier 1 / floor / staged / end)")
        for r in rows:
            print("   row %5d:" % r, " ".join("%6.2f" % v for v in rel[r, 1:7]))

if __name__ == "__main__":
    main()
