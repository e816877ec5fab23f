"""Per-tile phase timing of the onesweep pass and the scan kernel (diagnostic build).

Loads ``liblcpp_hip_trace.so`` (``python build.py --phase-trace``), whose kernels stamp ``s_memtime`` at
every phase boundary and write one 16-word record per tile (layout in ``csrc/common.hpp``,
``PhaseClock``), runs one SortKeys of 2^28 uniform u32 keys and one ExclusiveSum of 2^28 u32 values in
[0, 16) after warm-up calls, and prints one JSON line per onesweep pass and one for the scan:

* onesweep phases: load (issue to last key in registers), rank (to the barrier after every wave
  ranked), publish (PARTIAL counts, in-tile digit scan), reorder (keys into LDS by digit), look-back
  (walk over predecessors until every digit's prefix is known, including spinning), offsets (INCLUSIVE
  publish, global offsets), scatter (stores out of LDS to their final positions);
* scan phases: load + in-register scan, look-back, store;
* per phase the mean and median in microseconds (cycles converted with the clock measured from the
  100 MHz real-time counter over the same records), look-back steps, spin polls and fallback counts.

The trace build perturbs what it measures a little (a wait for outstanding memory operations before two
stamps); the product library has no trace code.

``--pairs`` traces SortPairs of 2^27 uniform u64 keys with u32 values (8 passes) instead.  ``--rank-mode M``
traces SortKeys only, with the in-wave ranking set by the library's test hook (0 ballots, 1 LDS tables,
2 both), after printing the untraced time per sort of the same library.

Usage: python luisacompute-parallelprimitive_amd/phase_trace.py [--log2n 28] [--pairs] [--rank-mode M]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))

WORDS = 16
SORT_PHASES = ("load", "rank", "publish", "reorder", "lookback", "offsets", "scatter")
SCAN_PHASES = ("load_scan", "lookback", "store")


def _stats(cycles: np.ndarray, mhz: float) -> dict:
    us = cycles / mhz
    return {"mean_us": round(float(us.mean()), 3), "median_us": round(float(np.median(us)), 3)}


def _clock_mhz(rec: np.ndarray, last_stamp: int) -> float:
    cyc = (rec[:, 1 + last_stamp] - rec[:, 1]).astype(np.float64)
    real_us = (rec[:, 15] - rec[:, 0]).astype(np.float64) / 100.0
    ok = real_us > 0.5
    return float(np.median(cyc[ok] / real_us[ok]))


def summarize_sort(rec: np.ndarray, p: int) -> dict:
    # Stamps: t0 start, t1 loaded, t2 ranked, t3 published, t4 reordered, t5 looked back (tiles > 0),
    # t6 offsets known, t7 stored.
    t = rec[:, 1:9].astype(np.int64)
    # A pass with offsets precomputed by the histogram (the first pass, by default) does not look back:
    # its look-back stamp stays 0, and the phase counts as empty.
    t[:, 5] = np.where(t[:, 5] == 0, t[:, 4], t[:, 5])
    mhz = _clock_mhz(rec, 7)
    body = rec[1:]  # tile 0 has no look-back
    tb = t[1:]
    phases = {}
    bounds = [(0, 1), (1, 2), (2, 3), (3, 4), (4, 5), (5, 6), (6, 7)]
    for name, (a, b) in zip(SORT_PHASES, bounds):
        phases[name] = _stats((tb[:, b] - tb[:, a]).astype(np.float64), mhz)
    counters = body[:, 13]
    steps = counters & 0xFFFF
    spins = (counters >> 16) & 0xFFFF
    fallbacks = (counters >> 32) & 0xFFFF
    resident = (tb[:, 7] - tb[:, 0]).astype(np.float64)
    span_us = (rec[:, 15].max() - rec[:, 0].min()) / 100.0
    lb = (tb[:, 5] - tb[:, 4]).astype(np.float64)
    return {"kernel": "onesweep", "pass": p, "tiles": int(rec.shape[0]), "clock_mhz": round(mhz, 1),
            "span_us": round(float(span_us), 1), "resident": _stats(resident, mhz), "phases": phases,
            "lookback_share_of_resident": round(float(lb.sum() / resident.sum()), 4),
            "lookback_cycles_mean": round(float(lb.mean()), 1),
            "lookback_steps_mean": round(float(steps.mean()), 3),
            "spin_polls_mean": round(float(spins.mean()), 3),
            "tiles_that_spun": int((spins > 0).sum()),
            "fallback_tiles": int(fallbacks.sum())}


def summarize_scan(rec: np.ndarray) -> dict:
    t = rec[:, 1:5].astype(np.int64)
    mhz = _clock_mhz(rec, 3)
    tb = t[1:]
    phases = {name: _stats((tb[:, b] - tb[:, a]).astype(np.float64), mhz)
              for name, (a, b) in zip(SCAN_PHASES, [(0, 1), (1, 2), (2, 3)])}
    counters = rec[1:, 13]
    resident = (tb[:, 3] - tb[:, 0]).astype(np.float64)
    lb = (tb[:, 2] - tb[:, 1]).astype(np.float64)
    return {"kernel": "scan_sum", "tiles": int(rec.shape[0]), "clock_mhz": round(mhz, 1),
            "span_us": round(float((rec[:, 15].max() - rec[:, 0].min()) / 100.0), 1),
            "resident": _stats(resident, mhz), "phases": phases,
            "lookback_share_of_resident": round(float(lb.sum() / resident.sum()), 4),
            "lookback_cycles_mean": round(float(lb.mean()), 1),
            "lookback_steps_mean": round(float((counters & 0xFFFF).mean()), 3),
            "spin_polls_mean": round(float(((counters >> 16) & 0xFFFF).mean()), 3),
            "fallback_tiles": int(((counters >> 32) & 0xFFFF).sum())}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--log2n", type=int, default=28)
    ap.add_argument("--pairs", action="store_true", help="SortPairs 2^27 u64 + u32 (8 passes) only")
    ap.add_argument("--rank-mode", type=int, default=None, choices=(0, 1, 2),
                    help="SortKeys in-wave ranking: 0 ballots in every wave, 1 LDS tables in every wave, 2 both "
                         "(the default); also prints the untraced time per sort")
    args = ap.parse_args()
    import torch
    import lcpp_hip as hip

    trace_lib = HERE / "liblcpp_hip_trace.so"
    if not trace_lib.exists():
        raise SystemExit(f"{trace_lib} is missing: run `python build.py --phase-trace` first")
    hip.LIB_PATH = trace_lib
    lib = hip.lib()
    lib.lcpp_hip_trace_set_buffer.restype = C.c_int
    lib.lcpp_hip_trace_set_buffer.argtypes = [C.c_void_p, C.c_uint64]

    dev = torch.device("cuda:0")
    if args.pairs:
        m = 1 << 27
        k = torch.empty(m, dtype=torch.int64, device=dev)
        hip.generate(hip.GEN_U64, k, m, 114521)
        v = torch.empty(m, dtype=torch.int32, device=dev)
        hip.generate(hip.GEN_U32_IOTA, v, m, 0)
        ko, vo = torch.empty_like(k), torch.empty_like(v)
        pt = torch.empty(hip.bytes_to_uint_count(hip.sort_pairs_temp_bytes(m, 8, 4)), dtype=torch.int32, device=dev)
        tile = hip.lib().lcpp_hip_radix_tile_items(8, 4)
        tiles = (m + tile - 1) // tile
        pbuf = torch.zeros(8 * tiles * WORDS, dtype=torch.int64, device=dev)
        assert lib.lcpp_hip_trace_set_buffer(None, 0) == 0
        for _ in range(2):
            hip.sort_pairs("u64", 4, k, ko, v, vo, m, temp=pt)
        torch.cuda.synchronize()
        assert lib.lcpp_hip_trace_set_buffer(C.c_void_p(pbuf.data_ptr()), 8 * tiles) == 0
        hip.sort_pairs("u64", 4, k, ko, v, vo, m, temp=pt)
        torch.cuda.synchronize()
        assert lib.lcpp_hip_trace_set_buffer(None, 0) == 0
        rec = pbuf.cpu().numpy().view(np.uint64).reshape(-1, WORDS)
        for p in range(8):
            print(json.dumps({"workload": "SortPairs 2^27 u64+u32", **summarize_sort(rec[p * tiles:(p + 1) * tiles], p)}),
                  flush=True)
        return 0
    n = 1 << args.log2n
    keys = torch.empty(n, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_HI, keys, n, 114521)
    out = torch.empty_like(keys)
    temp = torch.empty(hip.bytes_to_uint_count(hip.sort_keys_temp_bytes(n, 4)), dtype=torch.int32, device=dev)
    tiles = (n + hip.lib().lcpp_hip_radix_tile_items(4, 0) - 1) // hip.lib().lcpp_hip_radix_tile_items(4, 0)
    buf = torch.zeros(4 * tiles * WORDS, dtype=torch.int64, device=dev)

    def traced(fn, records):
        assert lib.lcpp_hip_trace_set_buffer(None, 0) == 0
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        buf.zero_()
        assert lib.lcpp_hip_trace_set_buffer(C.c_void_p(buf.data_ptr()), records) == 0
        fn()
        torch.cuda.synchronize()
        assert lib.lcpp_hip_trace_set_buffer(None, 0) == 0
        return buf.cpu().numpy().view(np.uint64).reshape(-1, WORDS)[:records].copy()

    sort = lambda: hip.sort_keys("u32", keys, out, n, temp=temp)
    if args.rank_mode is not None:
        # The trace library's own test hook; the untraced time is of the same library with tracing off.
        assert lib.lcpp_hip_internal_radix_rank_mode(args.rank_mode) == 0
        assert lib.lcpp_hip_trace_set_buffer(None, 0) == 0
        for _ in range(15):
            sort()
        events = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        events[0].record()
        for _ in range(10):
            sort()
        events[1].record()
        torch.cuda.synchronize()
        print(json.dumps({"rank_mode": args.rank_mode, "untraced_ms_per_sort": round(events[0].elapsed_time(events[1]) / 10, 4)}),
              flush=True)
    rec = traced(sort, 4 * tiles)
    for p in range(4):
        print(json.dumps(summarize_sort(rec[p * tiles:(p + 1) * tiles], p)), flush=True)
    if args.rank_mode is not None:
        lib.lcpp_hip_internal_radix_rank_mode(2)
        return 0
    del temp

    vals = torch.empty(n, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_LT16, vals, n, 114521)
    st = torch.empty(hip.bytes_to_uint_count(hip.scan_temp_bytes(n, 4)), dtype=torch.int32, device=dev)
    scan_tiles = (n + 24576 - 1) // 24576
    rec = traced(lambda: hip.scan_sum("u32", vals, out, n, temp=st), scan_tiles)
    print(json.dumps(summarize_scan(rec)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
