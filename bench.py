"""Benchmark of the LCPP device hot path on one MI355X.

Headline (`value`): onesweep SortKeys of 2^28 uniform uint32 keys (4 x 8-bit passes), Gkeys/s, inputs
resident in HBM, one step = one SortKeys call.  Every timed configuration records one HIP event per
step on the launch stream and reports the mean (`ms`) with the median, minimum and maximum step.  The
JSON line also carries the roofline of the dominant kernel (the onesweep pass) with the achievable copy
rate measured in the same run (a 1 GiB device-to-device copy by the library's copy kernel), the CPU
baseline of every benchmark configuration (the oracle's host restatement, one thread and all host
threads, median of five runs on a stated sample), and the other benchmark configurations (reduce,
scan, SortPairs, CsrMV) plus ExclusiveSumByKey / ReduceByKey and the stream-compaction family (select,
partition, unique, run-length encode), the segmented reduce / scan and the segmented sorts as achieved
GB/s against the 8 TB/s HBM peak.

`roofline.traffic` is the HBM bytes per onesweep launch read from the committed rocprofv3
FETCH_SIZE/WRITE_SIZE summary (profiles/radix_onesweep_sortkeys_2p28_u32.md); `--copy-calibration`
runs the plain copy whose counter readings scale those counters to bytes.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu] [--copy-calibration MIB]
                       [--only bykey|compact|reduce|scan|segmented|segsort|segsort-sweep|sortpairs|spmv|spmv-footprint]
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import platform
import sys
import time

REPO = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "luisacompute-parallelprimitive_amd"))

HBM_PEAK_GBS = 8000.0
SEED = 114521


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


class Timing:
    """Per-step times of one timed loop, in ms."""

    def __init__(self, per_step: list[float]):
        self.per_step = per_step
        self.mean = sum(per_step) / len(per_step)

    def fields(self, key: str = "ms") -> dict:
        import statistics
        return {key: round(self.mean, 5), f"{key}_median": round(statistics.median(self.per_step), 5),
                f"{key}_min": round(min(self.per_step), 5), f"{key}_max": round(max(self.per_step), 5)}


def time_steps(fn, steps: int, warmup: int) -> Timing:
    """Runs `warmup` untimed steps, then times exactly `steps` steps on the current stream with one event
    per step boundary."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    events = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    events[0].record()
    for i in range(steps):
        fn()
        events[i + 1].record()
    torch.cuda.synchronize()
    return Timing([events[i].elapsed_time(events[i + 1]) for i in range(steps)])


def achievable_copy_gbps(hip, dev, reps: int = 10) -> dict:
    """1 GiB device-to-device copy by the library's copy kernel (grid-stride, 32 workgroups per CU, four
    16-byte non-temporal loads and stores per thread and step, the fastest copy form measured on this GPU):
    the copy rate this GPU reaches in this run, median of `reps`."""
    import torch
    src = torch.ones(1 << 28, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    t = time_steps(lambda: hip.device_copy(dst, src, 1 << 30), reps, 5)
    import statistics
    ms = statistics.median(t.per_step)
    del src, dst
    torch.cuda.empty_cache()
    return {"bytes": 2 << 30, "ms_median": round(ms, 5), "GBps": round((2 << 30) / ms / 1e6, 1)}


def kernel_avg_ms(hip, fn, kernel: str, reps: int):
    """Average device duration of `kernel` over `reps` calls (events recorded around each launch on the
    launch stream by the library)."""
    import torch
    torch.cuda.synchronize()
    hip.profile_reset()
    hip.profile_enable(True)
    try:
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        ms, launches = hip.profile_query(kernel)
    finally:
        hip.profile_enable(False)
    return ms / max(launches, 1), launches


def flush_mall(buf):
    buf.add_(1)  # writes 1 GiB, evicting the 256 MB MALL


def graph_call_ms(fn, calls: int, reps: int) -> Timing:
    """Per-call device time of `fn` with the host out of the loop: `calls` calls recorded into one HIP graph
    (torch.cuda.CUDAGraph), replayed `reps` times with an event pair around each replay; per call = replay
    time / calls.  (The calls' kernels then run back to back, as they would in a loop the host outpaces.)"""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for e0, e1 in events:
        e0.record()
        graph.replay()
        e1.record()
    torch.cuda.synchronize()
    per = [e0.elapsed_time(e1) / calls for e0, e1 in events]
    del graph
    return Timing(per)


def cold_call_ms(fn, flush_buf, reps: int) -> Timing:
    """Device time of the whole call (every kernel it launches) after the MALL is flushed: an event pair
    around each call; the flush before it gives the host time to enqueue the call's launches."""
    import torch
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for e0, e1 in events:
        flush_mall(flush_buf)
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    return Timing([e0.elapsed_time(e1) for e0, e1 in events])


TRAFFIC_PROFILE = REPO / "profiles" / "radix_onesweep_sortkeys_2p28_u32.md"


def measured_traffic():
    """HBM bytes per onesweep launch from the committed FETCH_SIZE/WRITE_SIZE summary (the line
    `traffic_bytes_per_launch: N`), already scaled by the plain-copy calibration; None if absent."""
    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            if line.strip().startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip().strip("`"))
    except (OSError, ValueError):
        pass
    return None


def copy_calibration(mib: int) -> int:
    """Runs a plain device-to-device copy of `mib` MiB three times: the reference kernel whose
    FETCH_SIZE/WRITE_SIZE readings scale the onesweep counters to bytes."""
    import torch
    src = torch.ones(mib << 18, dtype=torch.int32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": mib << 20, "launches": 3}))
    return 0


_CSR = {}


def zipf_matrix():
    """The config-5 CSR matrix (built once per run; the host generation takes tens of seconds)."""
    if "m" not in _CSR:
        import workloads
        _CSR["m"] = workloads.zipf_csr(1 << 20, 1 << 20, SEED)
    return _CSR["m"]


def rate(nbytes: float, ms: float) -> float:
    return round(nbytes / ms / 1e6, 1)


def extra_reduce(hip, dev, steps, warmup, extra):
    import torch
    flush = torch.empty(1 << 28, dtype=torch.int32, device=dev)
    # Reduce 2^24 int32 in [-1000, 1000]: hot (MALL-resident) and cold (MALL flushed before each call).
    m = 1 << 24
    a = torch.empty(m, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_I32_PM1000, a, m, SEED)
    s = torch.empty(1, dtype=torch.int32, device=dev)
    rt = torch.empty(hip.bytes_to_uint_count(hip.reduce_temp_bytes(m, 4)), dtype=torch.int32, device=dev)
    call = lambda: hip.reduce_sum("i32", a, s, m, temp=rt)
    # Per call from the host (one event per step: Python and launch gaps included), per call inside a
    # HIP graph of 20 calls (device time only), the whole call after a MALL flush, and the floor of the
    # call's shape: the same two launches (partials + final fold) over 8,192 items, in a graph.
    hot = time_steps(call, steps, warmup)
    hot_graph = graph_call_ms(call, 20, 10)
    cold = cold_call_ms(call, flush, 10)
    tiny = torch.empty(8192, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_I32_PM1000, tiny, 8192, SEED)
    floor = graph_call_ms(lambda: hip.reduce_sum("i32", tiny, s, 8192, temp=rt), 20, 10)
    extra["reduce_sum_i32_2p24"] = {**hot.fields("ms_hot"), "GBps_hot": rate(4 * m, hot.mean),
                                    **hot_graph.fields("ms_hot_graph"), "GBps_hot_graph": rate(4 * m, hot_graph.mean),
                                    **cold.fields("ms_cold"), "GBps_cold": rate(4 * m, cold.mean),
                                    "ms_two_launch_floor_graph": round(floor.mean, 5)}
    del flush
    # Reduce 2^28 int32 (1 GiB read).
    m = 1 << 28
    a = torch.empty(m, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_I32_PM1000, a, m, SEED)
    rt = torch.empty(hip.bytes_to_uint_count(hip.reduce_temp_bytes(m, 4)), dtype=torch.int32, device=dev)
    t = time_steps(lambda: hip.reduce_sum("i32", a, s, m, temp=rt), steps, warmup)
    extra["reduce_sum_i32_2p28"] = {**t.fields(), "GBps": rate(4 * m, t.mean),
                                    "frac": round(4 * m / t.mean / 1e6 / HBM_PEAK_GBS, 4)}
    # DeviceReduce::Min and ArgMin over the same 2^28 int32 items (the same bytes read).
    t = time_steps(lambda: hip.reduce_minmax("min", "i32", a, s, m, temp=rt), steps, warmup)
    extra["reduce_min_i32_2p28"] = {**t.fields(), "GBps": rate(4 * m, t.mean),
                                    "frac": round(4 * m / t.mean / 1e6 / HBM_PEAK_GBS, 4)}
    at = torch.empty(hip.bytes_to_uint_count(hip.reduce_arg_temp_bytes(m, 4)), dtype=torch.int32, device=dev)
    ix = torch.empty(1, dtype=torch.int32, device=dev)
    t = time_steps(lambda: hip.reduce_arg("min", "i32", a, s, ix, m, temp=at), steps, warmup)
    extra["reduce_argmin_i32_2p28"] = {**t.fields(), "GBps": rate(4 * m, t.mean),
                                       "frac": round(4 * m / t.mean / 1e6 / HBM_PEAK_GBS, 4)}


def extra_scan(hip, dev, steps, warmup, extra, copy=None):
    import torch
    # ExclusiveSum 2^28 uint32 in [0, 16).
    m = 1 << 28
    b = torch.empty(m, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_LT16, b, m, SEED)
    c = torch.empty_like(b)
    st = torch.empty(hip.bytes_to_uint_count(hip.scan_temp_bytes(m, 4)), dtype=torch.int32, device=dev)
    t = time_steps(lambda: hip.scan_sum("u32", b, c, m, temp=st), steps, warmup)
    sk, _ = kernel_avg_ms(hip, lambda: hip.scan_sum("u32", b, c, m, temp=st), "scan_sum", 5)
    e = {**t.fields(), "GBps": rate(8 * m, t.mean), "frac": round(8 * m / t.mean / 1e6 / HBM_PEAK_GBS, 4),
         "kernel_ms": round(sk, 5)}
    if copy:
        e["frac_of_achievable_copy"] = round(copy["ms_median"] / t.mean, 4)
    extra["exclusive_sum_u32_2p28"] = e
    # ExclusiveSum 2^27 uint64 (the same 1 GiB in, 1 GiB out, 8-byte items).
    del b, c
    m = 1 << 27
    b = torch.empty(m, dtype=torch.int64, device=dev)
    hip.generate(hip.GEN_U64, b, m, SEED)
    c = torch.empty_like(b)
    st = torch.empty(hip.bytes_to_uint_count(hip.scan_temp_bytes(m, 8)), dtype=torch.int32, device=dev)
    t = time_steps(lambda: hip.scan_sum("u64", b, c, m, temp=st), steps, warmup)
    extra["exclusive_sum_u64_2p27"] = {**t.fields(), "GBps": rate(16 * m, t.mean),
                                       "frac": round(16 * m / t.mean / 1e6 / HBM_PEAK_GBS, 4)}


def extra_sort_pairs(hip, dev, steps, warmup, extra):
    import torch
    # SortPairs 2^27 u64 keys + u32 index values, uniform and AND-of-3 keys.
    m = 1 << 27
    for kind, gen in (("uniform", hip.GEN_U64), ("and3", hip.GEN_U64_AND3)):
        k = torch.empty(m, dtype=torch.int64, device=dev)
        hip.generate(gen, k, m, SEED)
        v = torch.empty(m, dtype=torch.int32, device=dev)
        hip.generate(hip.GEN_U32_IOTA, v, m, 0)
        ko, vo = torch.empty_like(k), torch.empty_like(v)
        pt = torch.empty(hip.bytes_to_uint_count(hip.sort_pairs_temp_bytes(m, 8, 4)), dtype=torch.int32, device=dev)
        t = time_steps(lambda: hip.sort_pairs("u64", 4, k, ko, v, vo, m, temp=pt), max(3, steps // 2), warmup)
        extra[f"sort_pairs_u64_u32_2p27_{kind}"] = {
            **t.fields(), "Gpairs_per_s": round(m / t.mean / 1e6, 3),
            "GBps_8pass_model": rate(2 * 8 * m * 12, t.mean),
            "frac": round(2 * 8 * m * 12 / t.mean / 1e6 / HBM_PEAK_GBS, 4)}
        del k, v, ko, vo, pt


def extra_spmv(hip, dev, steps, warmup, extra):
    import torch
    # CsrMV fp32: 2^20 x 2^20, Zipf(1.5) row lengths in [1, 4096], built on the host.
    rows = cols = 1 << 20
    va, ro, ci, xv, nnz = zipf_matrix()
    d = [torch.from_numpy(t).to(dev) for t in (va, ro, ci, xv)]
    y = torch.empty(rows, dtype=torch.float32, device=dev)
    spmv = lambda: hip.spmv_csr("f32", "i32", d[0], d[1], d[2], d[3], y, rows, cols, nnz)
    t = time_steps(spmv, steps, warmup)
    sk, _ = kernel_avg_ms(hip, spmv, "spmv_csr", 5)
    spmv_bytes = 8 * nnz + 4 * (rows + 1) + 4 * rows + 4 * cols
    extra["spmv_csr_f32_zipf1.5_2p20"] = {"nnz": nnz, **t.fields(), "kernel_ms": round(sk, 5),
                                          "GBps": rate(spmv_bytes, sk),
                                          "frac": round(spmv_bytes / sk / 1e6 / HBM_PEAK_GBS, 4)}


def extra_by_key(hip, dev, steps, warmup, extra):
    import torch
    # ExclusiveSumByKey and ReduceByKey over 2^28 uint32 values in [0, 16) with int32 keys in runs of
    # geometric length (mean 64: an item starts a run when 6 random bits are zero).
    m = 1 << 28
    r = torch.empty(m, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_HI, r, m, SEED + 7)
    keys = torch.cumsum(((r & 63) == 0).to(torch.int32), 0, dtype=torch.int32)
    del r
    vals = torch.empty(m, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_LT16, vals, m, SEED)
    out = torch.empty_like(vals)
    st = torch.empty(hip.bytes_to_uint_count(hip.scan_by_key_temp_bytes(m, 4, 4)), dtype=torch.int32, device=dev)
    t = time_steps(lambda: hip.scan_by_key("i32", "u32", keys, vals, out, m, inclusive=False, temp=st), steps, warmup)
    sk, _ = kernel_avg_ms(hip, lambda: hip.scan_by_key("i32", "u32", keys, vals, out, m, temp=st), "scan_by_key", 5)
    extra["exclusive_sum_by_key_i32_u32_2p28"] = {**t.fields(), "GBps": rate(12 * m, t.mean),
                                                  "frac": round(12 * m / t.mean / 1e6 / HBM_PEAK_GBS, 4),
                                                  "kernel_ms": round(sk, 5)}
    runs_out = torch.zeros(1, dtype=torch.int32, device=dev)
    rt = torch.empty(hip.bytes_to_uint_count(hip.reduce_by_key_temp_bytes(m, 4, 4)), dtype=torch.int32, device=dev)
    uniq, agg = out, torch.empty_like(vals)
    t = time_steps(lambda: hip.reduce_by_key("i32", "u32", keys, vals, uniq, agg, runs_out, m, temp=rt), steps, warmup)
    runs = int(runs_out.item())
    moved = 8 * m + 8 * runs
    extra["reduce_by_key_i32_u32_2p28"] = {**t.fields(), "runs": runs, "GBps": rate(moved, t.mean),
                                           "frac": round(moved / t.mean / 1e6 / HBM_PEAK_GBS, 4)}


def extra_compact(hip, dev, steps, warmup, extra):
    import torch
    # DeviceSelect::If and DevicePartition::If over 2^28 uniform uint32 items with x < 2^31 (half
    # selected); DeviceSelect::Unique and DeviceRunLengthEncode::Encode over 2^28 uint32 items in runs of
    # geometric length (mean 64).
    m = 1 << 28
    x = torch.empty(m, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_HI, x, m, SEED + 11)
    out = torch.empty_like(x)
    num = torch.zeros(2, dtype=torch.int32, device=dev)
    temp = torch.empty(hip.bytes_to_uint_count(hip.run_length_encode_temp_bytes(m)), dtype=torch.int32, device=dev)
    half = hip.predicate("u32", (hip.PRED_LT, 1 << 31))
    for name, fn, written in (("select_if_u32_half_2p28", hip.select_if, None),
                              ("partition_if_u32_half_2p28", hip.partition_if, m)):
        call = lambda fn=fn: fn("u32", x, out, num, m, half, temp=temp)
        t = time_steps(call, steps, warmup)
        kept = int(num[0].item())
        moved = 4 * m + 4 * (kept if written is None else written)
        kms, _ = kernel_avg_ms(hip, call, "compact", 5)
        extra[name] = {**t.fields(), "kernel_ms": round(kms, 5), "selected": kept,
                       "GBps": rate(moved, t.mean), "frac": round(moved / t.mean / 1e6 / HBM_PEAK_GBS, 4)}
    r = x
    hip.generate(hip.GEN_U32_HI, r, m, SEED + 7)
    runs_in = torch.cumsum(((r & 63) == 0).to(torch.int32), 0, dtype=torch.int32)
    del x, r
    counts = torch.empty_like(out)
    for name, call, per_run in (
            ("unique_u32_runs64_2p28", lambda: hip.select_unique("u32", runs_in, out, num, m, temp=temp), 4),
            ("run_length_encode_u32_runs64_2p28",
             lambda: hip.run_length_encode("u32", runs_in, out, counts, num, m, temp=temp), 8)):
        t = time_steps(call, steps, warmup)
        runs = int(num[0].item())
        moved = 4 * m + per_run * runs
        kms, _ = kernel_avg_ms(hip, call, "runs_by_key", 5)
        extra[name] = {**t.fields(), "kernel_ms": round(kms, 5), "runs": runs,
                       "GBps": rate(moved, t.mean), "frac": round(moved / t.mean / 1e6 / HBM_PEAK_GBS, 4)}


def extra_segmented(hip, dev, steps, warmup, extra):
    import torch
    # DeviceSegmentReduce::Sum and DeviceSegmentedScan::InclusiveSegmentedSum over 2^28 int32 items in
    # 2^16 segments of 4096 (begin/end offsets).
    m, segs = 1 << 28, 1 << 16
    x = torch.empty(m, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_I32_PM1000, x, m, SEED)
    begins = torch.arange(segs, dtype=torch.int64, device=dev).mul_(m // segs).to(torch.int32)
    ends = begins + (m // segs)
    out = torch.empty(segs, dtype=torch.int32, device=dev)
    call = lambda: hip.segment_reduce("sum", "i32", x, out, segs, begins=begins, ends=ends)
    t = time_steps(call, steps, warmup)
    kms, _ = kernel_avg_ms(hip, call, "segment_reduce", 5)
    moved = 4 * m + 12 * segs
    extra["segment_reduce_sum_i32_2p28_4096"] = {**t.fields(), "kernel_ms": round(kms, 5),
                                                 "GBps": rate(moved, t.mean),
                                                 "frac": round(moved / t.mean / 1e6 / HBM_PEAK_GBS, 4)}
    y = torch.empty_like(x)
    call = lambda: hip.segmented_scan("i32", x, y, begins, ends, segs, inclusive=True)
    t = time_steps(call, steps, warmup)
    kms, _ = kernel_avg_ms(hip, call, "segmented_scan", 5)
    moved = 8 * m + 8 * segs
    extra["segmented_inclusive_sum_i32_2p28_4096"] = {**t.fields(), "kernel_ms": round(kms, 5),
                                                      "GBps": rate(moved, t.mean),
                                                      "frac": round(moved / t.mean / 1e6 / HBM_PEAK_GBS, 4)}


def extra_segsort(hip, dev, steps, warmup, extra):
    import torch
    # DeviceSegmentedRadixSort::SortPairs over 2^26 uint32 keys + uint32 values in 2^14 segments of 4096
    # (the chunk kernel sorts their 2048-item chunks, then one global merge pass), and SortKeys over 2^26
    # uint32 keys in 2^16 segments of 1024 (the block kernel, one workgroup per segment).  Algorithmic
    # bytes: every key (and value) read once and written once.
    m = 1 << 26
    keys = torch.empty(m, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_HI, keys, m, SEED + 13)
    vals = torch.empty(m, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_IOTA, vals, m, 0)
    ko, vo = torch.empty_like(keys), torch.empty_like(vals)
    temp = torch.empty(hip.bytes_to_uint_count(hip.segmented_sort_pairs_temp_bytes(m, 4, 4)), dtype=torch.int32,
                       device=dev)
    for name, seg_len, pairs in (("segmented_radix_sort_pairs_u32_2p26_4096", 4096, True),
                                 ("segmented_radix_sort_keys_u32_2p26_1024", 1024, False)):
        segs = m // seg_len
        begins = torch.arange(segs, dtype=torch.int64, device=dev).mul_(seg_len).to(torch.int32)
        ends = begins + seg_len
        if pairs:
            call = lambda: hip.segmented_sort("u32", keys, ko, m, segs, begins, ends, values_in=vals, values_out=vo,
                                              temp=temp)
        else:
            call = lambda: hip.segmented_sort("u32", keys, ko, m, segs, begins, ends, temp=temp)
        t = time_steps(call, steps, warmup)
        block_ms, _ = kernel_avg_ms(hip, call, "segsort_block", 3)
        chunk_ms, _ = kernel_avg_ms(hip, call, "segsort_chunk", 3)
        merge_ms, merges = kernel_avg_ms(hip, call, "segsort_merge", 3)
        moved = (16 if pairs else 8) * m
        extra[name] = {**t.fields(), "Gkeys_per_s": round(m / t.mean / 1e6, 2),
                       "block_kernel_ms": round(block_ms, 5), "chunk_kernel_ms": round(chunk_ms, 5),
                       "merge_kernel_ms": round(merge_ms, 5),
                       "merge_launches_per_call": merges // 3,
                       "GBps": rate(moved, t.mean), "frac": round(moved / t.mean / 1e6 / HBM_PEAK_GBS, 4)}


def study_spmv_footprint(hip, dev, steps, warmup, extra):
    import torch
    import workloads
    # CsrMV time against the footprint of x: the same Zipf(1.5) row lengths over 2^20 rows with 2^20,
    # 2^19, 2^17 and 2^15 columns (x of 4 MB down to 128 KB), so that the x gathers go from missing
    # the L2 to hitting it (and, at 128 KB, partly the L1) while the streamed matrix bytes stay fixed.
    # Not part of the default run.
    rows = 1 << 20
    for lc in (20, 19, 17, 15):
        cols = 1 << lc
        va, ro, ci, xv, nnz = zipf_matrix() if lc == 20 else workloads.zipf_csr(rows, cols, SEED)
        d = [torch.from_numpy(a).to(dev) for a in (va, ro, ci, xv)]
        y = torch.empty(rows, dtype=torch.float32, device=dev)
        call = lambda: hip.spmv_csr("f32", "i32", d[0], d[1], d[2], d[3], y, rows, cols, nnz)
        t = time_steps(call, steps, warmup)
        extra[f"spmv_csr_f32_zipf1.5_2p20_x{4 * cols // 1024}KiB"] = {"cols": cols, "nnz": nnz, **t.fields()}
        del d, y
        torch.cuda.empty_cache()


EXTRAS = {"reduce": extra_reduce, "scan": extra_scan, "sortpairs": extra_sort_pairs, "spmv": extra_spmv,
          "bykey": extra_by_key, "compact": extra_compact,
          "segmented": extra_segmented, "segsort": extra_segsort}
# Studies run only when named with --only.
def study_segsort_sweep(hip, dev, steps, warmup, extra):
    import torch
    # DeviceSegmentedRadixSort::SortKeys over 2^24 uint32 keys in equal segments of 4 .. 65,536 items (the
    # tile kernel's joint sorts, the block kernel's one sort per segment, the chunk kernel plus global
    # merge passes), and SortPairs with uint32 values at three of the lengths.  Not part of the default run.
    m = 1 << 24
    keys = torch.empty(m, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_HI, keys, m, SEED + 13)
    vals = torch.empty(m, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_IOTA, vals, m, 0)
    ko, vo = torch.empty_like(keys), torch.empty_like(vals)
    temp = torch.empty(hip.bytes_to_uint_count(hip.segmented_sort_pairs_temp_bytes(m, 4, 4)), dtype=torch.int32,
                       device=dev)
    for seg_len, pairs in ((4, False), (16, False), (64, False), (256, False), (1024, False), (2048, False),
                           (4096, False), (65536, False), (64, True), (1024, True), (4096, True)):
        segs = m // seg_len
        begins = torch.arange(segs, dtype=torch.int64, device=dev).mul_(seg_len).to(torch.int32)
        ends = begins + seg_len
        if pairs:
            call = lambda: hip.segmented_sort("u32", keys, ko, m, segs, begins, ends, values_in=vals, values_out=vo,
                                              temp=temp)
        else:
            call = lambda: hip.segmented_sort("u32", keys, ko, m, segs, begins, ends, temp=temp)
        t = time_steps(call, steps, warmup)
        moved = (16 if pairs else 8) * m
        extra[f"segmented_radix_sort_{'pairs' if pairs else 'keys'}_u32_2p24_{seg_len}"] = {
            **t.fields(), "Gkeys_per_s": round(m / t.mean / 1e6, 2), "GBps": rate(moved, t.mean),
            "frac": round(moved / t.mean / 1e6 / HBM_PEAK_GBS, 4)}
        del begins, ends


STUDIES = {"spmv-footprint": study_spmv_footprint, "segsort-sweep": study_segsort_sweep}


def run_extras(hip, dev, steps, warmup, names, copy=None):
    import torch
    extra = {}
    for name in names:
        if name == "scan":
            extra_scan(hip, dev, steps, warmup, extra, copy)
        else:
            {**EXTRAS, **STUDIES}[name](hip, dev, steps, warmup, extra)
        torch.cuda.empty_cache()
    return extra


# ---- CPU baseline ----------------------------------------------------------------------------------
def cpu_baseline(keys_dev, reps: int = 5) -> dict:
    """The oracle's host restatement of every benchmark configuration (oracle/cpu_baseline.cpp), on one
    thread and on every host thread, median of `reps` runs after one untimed run, on the samples named
    in each entry.  Inputs are the same seeded streams as the GPU runs (the SortKeys sample is the first
    2^24 of the GPU's keys)."""
    import statistics
    import numpy as np
    sys.path.insert(0, str(REPO))
    import oracle
    threads_all = os.cpu_count() or 1

    def timed(fn, prep=None):
        out = {}
        for label, th in (("1_thread", 1), (f"{threads_all}_threads", threads_all)):
            ts = []
            for r in range(reps + 1):
                args = prep() if prep else ()
                t0 = time.perf_counter()
                fn(th, *args)
                dt = time.perf_counter() - t0
                if r:
                    ts.append(dt)
            out[label] = statistics.median(ts)
        return out

    res = {}
    # Reduce: all 2^24 int32 items in [-1000, 1000].
    n = 1 << 24
    a = oracle.generate(2, n, SEED)
    t = timed(lambda th: oracle.par_reduce_sum_i32(a, th))
    res["reduce_sum_i32_2p24"] = {"sample": "all 2^24 items", "unit": "GB/s",
                                  **{k: round(4 * n / v / 1e9, 2) for k, v in t.items()}}
    # Scan: 2^26 of the 2^28 u32 in [0, 16).
    n = 1 << 26
    b = oracle.generate(3, n, SEED)
    out = np.empty_like(b)
    t = timed(lambda th: oracle.par_scan_sum_u32(b, th, out))
    res["exclusive_sum_u32_2p28"] = {"sample": "first 2^26 of the 2^28 items", "unit": "GB/s",
                                     **{k: round(8 * n / v / 1e9, 2) for k, v in t.items()}}
    del b, out
    # SortKeys: 2^24 of the 2^28 uniform u32 keys (stable 8-bit LSD, as on the GPU), plus std::sort on one thread.
    n = 1 << 24
    sample = keys_dev[:n].cpu().numpy().view(np.uint32).copy()
    work, tmp = np.empty_like(sample), np.empty_like(sample)

    def fresh():
        np.copyto(work, sample)
        return ()
    t = timed(lambda th: oracle.par_radix_sort_u32(work, th, tmp), fresh)
    std_ts = []
    for r in range(reps + 1):
        fresh()
        t0 = time.perf_counter()
        oracle.std_sort_u32(work)
        if r:
            std_ts.append(time.perf_counter() - t0)
    res["sort_keys_u32_2p28"] = {"sample": "first 2^24 of the 2^28 keys", "unit": "Gkeys/s",
                                 **{k: round(n / v / 1e9, 4) for k, v in t.items()},
                                 "std_sort_1_thread": round(n / statistics.median(std_ts) / 1e9, 4)}
    del sample, work, tmp
    # SortPairs: 2^22 uniform u64 keys with u32 index values (the uniform SortPairs key stream).
    n = 1 << 22
    k0 = oracle.generate(0, n, SEED)
    v0 = np.arange(n, dtype=np.uint32)
    kw, vw, tk, tv = np.empty_like(k0), np.empty_like(v0), np.empty_like(k0), np.empty_like(v0)

    def fresh_pairs():
        np.copyto(kw, k0)
        np.copyto(vw, v0)
        return ()
    t = timed(lambda th: oracle.par_radix_sort_u64_u32(kw, vw, th, (tk, tv)), fresh_pairs)
    res["sort_pairs_u64_u32_2p27_uniform"] = {"sample": "2^22 pairs of the same key stream", "unit": "Gpairs/s",
                                              **{k: round(n / v / 1e9, 4) for k, v in t.items()}}
    del k0, v0, kw, vw, tk, tv
    # CsrMV: the whole config-5 matrix.
    rows = cols = 1 << 20
    va, ro, ci, xv, nnz = zipf_matrix()
    y = np.empty(rows, np.float32)
    t = timed(lambda th: oracle.par_spmv_csr_f32(va, ro, ci, xv, rows, th, y))
    spmv_bytes = 8 * nnz + 4 * (rows + 1) + 4 * rows + 4 * cols
    res["spmv_csr_f32_zipf1.5_2p20"] = {"sample": f"the whole matrix ({nnz} nonzeros)", "unit": "GB/s",
                                        **{k: round(spmv_bytes / v / 1e9, 2) for k, v in t.items()}}
    res["threads_all"] = threads_all
    return res


def device_info(torch, dev) -> dict:
    props = torch.cuda.get_device_properties(dev)
    return {"device": props.name, "gcnArchName": getattr(props, "gcnArchName", ""),
            "compute_units": props.multi_processor_count,
            "hbm_GiB": round(props.total_memory / 2**30, 1)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # The first dozen sorts after the GPU idles run slower (2.8 -> 2.05 ms for SortKeys 2^28) while the
    # clock settles; the default warm-up covers that ramp so the timed steps measure the steady state.
    ap.add_argument("--warmup", type=int, default=15)
    ap.add_argument("--no-extra", action="store_true", help="headline SortKeys only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", choices=sorted(EXTRAS) + sorted(STUDIES), default=None,
                    help="run only this secondary configuration (for profiling); prints its extra entry")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain MIB-MiB device copy (counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this library runs on one GPU; sharding across GPUs is design-only",
                          "n_gpus": args.gpus}))
        return 2
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)

    import torch
    import lcpp_hip as hip

    dev = torch.device("cuda:0")
    steps, warmup = args.steps, args.warmup
    if args.only:
        print(json.dumps({"only": args.only, "extra": run_extras(hip, dev, steps, warmup, [args.only])}))
        return 0

    # ---- headline: SortKeys 2^28 u32 ---------------------------------------------------------------
    n = 1 << 28
    keys = torch.empty(n, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_HI, keys, n, SEED)
    out = torch.empty_like(keys)
    temp = torch.empty(hip.bytes_to_uint_count(hip.sort_keys_temp_bytes(n, 4)), dtype=torch.int32, device=dev)

    def sort_step():
        hip.sort_keys("u32", keys, out, n, temp=temp)

    t = time_steps(sort_step, steps, warmup)
    ms = t.mean
    gkeys = n / (ms * 1e-3) / 1e9
    onesweep_ms, launches = kernel_avg_ms(hip, sort_step, "radix_onesweep", max(3, steps // 4))
    hist_ms, _ = kernel_avg_ms(hip, sort_step, "radix_histogram", 3)
    pass_bytes = 2 * n * 4  # read + write of the keys in one 8-bit pass
    achieved = pass_bytes / (onesweep_ms * 1e-3) / 1e9
    del temp, out
    torch.cuda.empty_cache()
    copy = achievable_copy_gbps(hip, dev)  # after the sort, with the GPU at its working clocks
    line = {
        "metric": "onesweep SortKeys 2^28 u32 Gkeys/s; reduce/scan achieved HBM GB/s vs peak",
        "value": round(gkeys, 3),
        "unit": "Gkeys/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic (splitmix64, seed 114521), generated on the device",
        "config": {"workload": "DeviceRadixSort::SortKeys, 2^28 uniform uint32 keys, 4 x 8-bit onesweep passes",
                   "items": n, **device_info(torch, dev)},
        "timing": t.fields("ms_per_step"),
        "roofline": {
            "kernel": "radix_onesweep",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "avg_launch_ms": round(onesweep_ms, 5),
            "algorithmic_bytes_per_launch": pass_bytes,
            "whole_sort_frac_4pass_model": round((32 * n) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "histogram_avg_ms": round(hist_ms, 5),
            "achievable_copy_GBps": copy["GBps"],
            "frac_of_achievable_copy": round(achieved / copy["GBps"], 4),
        },
    }

    # ---- CPU baseline: every configuration on the host, one thread and all threads -----------------
    if not args.no_cpu:
        per_config = cpu_baseline(keys)
        sk = per_config["sort_keys_u32_2p28"]
        threads_all = per_config.pop("threads_all")
        line["cpu_baseline"] = {
            "value": sk[f"{threads_all}_threads"],
            "unit": "Gkeys/s",
            "cores": threads_all,
            "kind": "port",
            "sample": "first 2^24 of the same keys, stable 8-bit LSD sort (oracle/cpu_baseline.cpp) on every "
                      "host thread, median of 5",
            "cpu": cpu_model(),
            "per_config": per_config,
        }

    # ---- other configurations -----------------------------------------------------------------------
    if not args.no_extra:
        del keys
        torch.cuda.empty_cache()
        line["extra"] = run_extras(hip, dev, steps, warmup, list(EXTRAS), copy)
        line["extra"]["achievable_copy_1GiB"] = copy

    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
