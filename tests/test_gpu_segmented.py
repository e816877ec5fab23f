"""DeviceSegmentReduce (Sum, Min, Max, ArgMin, ArgMax; offsets and fixed-size) and DeviceSegmentedScan
(exclusive / inclusive / with initial value; same and separate output offsets) on the GPU through the
C-ABI.

Known answers of the reference's tests (device_segment_reduce.cpp:438-548,
device_segmented_scan_test.cpp:104-257) exactly.  Integer results bit-exact against the oracle;
float Min / Max / Arg bit-exact (selection, no rounding); float sums within
|got - exact| <= rel * (sum of |terms|), rel 1e-5 (f32) / 1e-12 (f64), the oracle summing in long
double.  Also: empty and reversed segments, overlapping segments, segments of 1 to 2^20 items, and
a 2^26-item input."""
import numpy as np
import pytest
import torch

from gpu_util import fill_dev, log, to_dev, to_host

pytestmark = pytest.mark.gpu

NP = {"i32": np.int32, "u32": np.uint32, "f32": np.float32, "i64": np.int64, "u64": np.uint64, "f64": np.float64}
REL = {"f32": 1e-5, "f64": 1e-12}


def values_for(rng, n, ts):
    if ts in ("f32", "f64"):
        return rng.uniform(-1.0, 1.0, n).astype(NP[ts])
    info = np.iinfo(NP[ts])
    return rng.integers(info.min, info.max, n, dtype=NP[ts], endpoint=True)


def random_segments(rng, n, m, max_len):
    b = rng.integers(0, n, m).astype(np.uint32)
    e = np.minimum(b.astype(np.int64) + rng.integers(0, max_len + 1, m), n).astype(np.uint32)
    e[::13] = b[::13]                       # empty
    e[7::29] = b[7::29] // 2                # begin > end: empty
    return b, e


def g_reduce(hip, op, x, b=None, e=None, size=None, m=None):
    ts = {v: k for k, v in NP.items()}[x.dtype.type]
    m = m if m is not None else len(b)
    d = to_dev(x) if x.size else torch.empty(1, dtype=torch.int32, device="cuda:0")
    out = fill_dev(m, x.itemsize, 0x5A)
    idx = fill_dev(m, 4, 0x5A) if op.startswith("arg") else None
    if size is not None:
        hip.segment_reduce(op, ts, d, out, m, segment_size=size, index_out=idx)
    else:
        hip.segment_reduce(op, ts, d, out, m, begins=to_dev(np.asarray(b, np.uint32)), ends=to_dev(np.asarray(e, np.uint32)),
                           index_out=idx)
    return to_host(out, x.dtype, m), (to_host(idx, np.uint32, m) if idx is not None else None)


def check_reduce(orc, op, x, b, e, got, idx, ts):
    want, widx, ab = orc.segment_reduce(op, x, b, e)
    if op == "sum" and ts in REL:
        exact = want.astype(np.float64)
        assert np.all(np.abs(got.astype(np.float64) - exact) <= REL[ts] * np.maximum(ab, 1e-30) + 1e-30)
    else:
        np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))
    if widx is not None:
        np.testing.assert_array_equal(idx, widx)


def g_scan(hip, x, b, e, ob=None, inclusive=False, init=None, in_place=False, out_size=None):
    ts = {v: k for k, v in NP.items()}[x.dtype.type]
    d = to_dev(x)
    out = d if in_place else fill_dev(out_size or x.size, x.itemsize, 0)
    hip.segmented_scan(ts, d, out, to_dev(np.asarray(b, np.uint32)), to_dev(np.asarray(e, np.uint32)), len(b),
                       inclusive=inclusive, init=init,
                       out_begins=to_dev(np.asarray(ob, np.uint32)) if ob is not None else None)
    return to_host(out, x.dtype, out_size or x.size)


def written_mask(n_out, b, e, ob):
    m = np.zeros(n_out, bool)
    for s in range(len(b)):
        if e[s] > b[s]:
            m[ob[s]:ob[s] + (e[s] - b[s])] = True
    return m


# ---- known answers ---------------------------------------------------------------------------------
def test_segment_reduce_known_answers(hip, dev):
    """device_segment_reduce.cpp:438-548."""
    got, _ = g_reduce(hip, "sum", np.array([4, 6, 8, 10], np.int32), [0, 2, 2], [2, 2, 4])
    assert got.tolist() == [10, 0, 18]
    v, i = g_reduce(hip, "argmax", np.array([-9, -2, -2, -8, -5], np.float32), [0, 1, 4], [0, 4, 4])
    lo = float(np.finfo(np.float32).min)
    assert v.tolist() == [lo, -2.0, lo] and i.tolist() == [1, 0, 1]
    v, i = g_reduce(hip, "argmin", np.array([7, 1, 1, 9, 4, 2], np.int32), [0, 3], [3, 6])
    assert v.tolist() == [1, 2] and i.tolist() == [1, 2]


@pytest.mark.parametrize("op", ["argmin", "argmax"])
def test_arg_nan_among_unaligned_head_items(hip, orc, dev, op):
    """Float ArgMin / ArgMax over segments of 512 to 70,000 items that start 1-3 items before a 16-byte
    boundary (the items the lanes read one by one before the 16-byte vectors), with NaNs among those head
    items: NaN items never win, so the true extremum and its index come out, as the oracle's fold that skips
    NaN items gives."""
    rng = np.random.default_rng(61)
    n = 1 << 19
    x = rng.standard_normal(n).astype(np.float32)
    begins, ends = [], []
    pos = 5
    for length in (512, 513, 700, 1024, 1500, 4096, 5000, 70000):
        for r in (1, 2, 3):  # b % 4 == r: 4 - r items before the boundary (the input is 16-byte aligned)
            b = pos - pos % 4 + r + 4
            x[b] = np.nan
            if r == 1:
                x[b + 1] = np.nan  # two of the three head items
            begins.append(b)
            ends.append(b + length)
            pos = b + length + 7
    assert pos < n
    log(f"segment {op}: NaN head items in {len(begins)} unaligned segments")
    got, idx = g_reduce(hip, op, x, begins, ends)
    check_reduce(orc, op, x, begins, ends, got, idx, "f32")
    assert not np.isnan(got).any()


def test_segmented_scan_known_answers(hip, orc, dev):
    """device_segmented_scan_test.cpp:104-257: same and packed output offsets, exclusive, inclusive,
    inclusive with initial value 10, and the exact in-place inclusive sum (items outside every segment
    keep their values)."""
    x = np.array([100, 1, 2, 3, 5, 6, 7, 200, 9, 10, 11, 12, 300, 400], np.int32)
    b, e, packed = [1, 4, 4, 8], [4, 4, 7, 12], [0, 4, 6, 10]
    for ob in (b, packed):
        for kw in ({}, {"inclusive": True}, {"inclusive": True, "init": 10}):
            got = g_scan(hip, x, b, e, ob=ob, **kw)
            want, _ = orc.segmented_scan(x, b, e, out_begins=ob, **kw)
            mask = written_mask(14, b, e, ob)
            assert got[mask].tolist() == want[mask].tolist()
    got = g_scan(hip, x, b, e, inclusive=True, in_place=True)
    want, _ = orc.segmented_scan(x, b, e, inclusive=True)
    mask = written_mask(14, b, e, b)
    assert got.tolist() == np.where(mask, want, x).tolist()
    hip.segmented_scan("i32", to_dev(x), to_dev(x), None, None, 0, inclusive=True)  # zero segments: no-op


# ---- types, shapes, sizes ------------------------------------------------------------------------------
@pytest.mark.parametrize("ts", ["i32", "u32", "f32", "i64", "u64", "f64"])
def test_segment_reduce_types(hip, orc, dev, ts):
    rng = np.random.default_rng(sum(map(ord, ts)))
    n = 200_000
    x = values_for(rng, n, ts)
    b, e = random_segments(rng, n, 3000, 3000)
    ops = ["sum", "min", "max"] + (["argmin", "argmax"] if ts in ("i32", "u32", "f32") else [])
    for op in ops:
        got, idx = g_reduce(hip, op, x, b, e)
        check_reduce(orc, op, x, b, e, got, idx, ts)


@pytest.mark.parametrize("size", [1, 7, 255, 256, 257, 2048, 2049, 100_000])
def test_segment_reduce_fixed_size(hip, orc, dev, size):
    """Fixed segment_size (device_segment_reduce.cpp:165-202,269-318): full tiles and tails."""
    rng = np.random.default_rng(size)
    m = max(1, 300_000 // size)
    x = rng.integers(-1000, 1000, m * size).astype(np.int32)
    b = (np.arange(m) * size).astype(np.uint32)
    e = (b + size).astype(np.uint32)
    for op in ("sum", "max", "argmin"):
        got, idx = g_reduce(hip, op, x, size=size, m=m)
        check_reduce(orc, op, x, b, e, got, idx, "i32")


def test_segment_reduce_ties_and_long_segments(hip, orc, dev):
    """Many equal values (ties go to the lower index) and segments up to 2^20 items."""
    rng = np.random.default_rng(3)
    n = 1 << 22
    x = rng.integers(0, 4, n).astype(np.float32)
    b = np.array([0, 5, 1 << 20, 3 << 20, 100, 77], np.uint32)
    e = np.array([1 << 20, 6, 2 << 20, (3 << 20) + 1, 100, 1 << 22], np.uint32)
    for op in ("argmin", "argmax", "min", "max", "sum"):
        got, idx = g_reduce(hip, op, x, b, e)
        check_reduce(orc, op, x, b, e, got, idx, "f32")


@pytest.mark.parametrize("ts", ["i32", "u32", "f32", "i64", "u64", "f64"])
def test_segmented_scan_types(hip, orc, dev, ts):
    rng = np.random.default_rng(sum(map(ord, ts)) + 1)
    n = 150_000
    x = values_for(rng, n, ts)
    # Disjoint segments (packed output offsets) so that every output position has one writer.
    cuts = np.sort(rng.choice(n, 800, replace=False)).astype(np.uint32)
    b, e = cuts[:-1:2], cuts[1::2]
    e[::9] = b[::9]
    lengths = np.where(e > b, e - b, 0)
    ob = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.uint32)
    out_size = int(lengths.sum())
    for kw in ({}, {"inclusive": True}, {"inclusive": True, "init": 3}, {"init": 5}):
        got = g_scan(hip, x, b, e, ob=ob, out_size=out_size, **kw)
        want, ab = orc.segmented_scan(x, b, e, out_begins=ob, out_size=out_size, **kw)
        if ts in REL:
            assert np.all(np.abs(got.astype(np.float64) - want.astype(np.float64)) <= REL[ts] * ab + 1e-30), kw
        else:
            np.testing.assert_array_equal(got, want)


def test_large_segmented(hip, orc, dev):
    """2^26 int32 items in 2^14 segments of 4096: sums, maxima, argmin and an inclusive scan."""
    rng = np.random.default_rng(26)
    n, m = 1 << 26, 1 << 14
    x = rng.integers(-(1 << 31), 1 << 31, n, dtype=np.int64).astype(np.int32)
    b = (np.arange(m, dtype=np.uint64) * (n // m)).astype(np.uint32)
    e = (b.astype(np.uint64) + n // m).astype(np.uint32)
    for op in ("sum", "max", "argmin"):
        log(f"segmented large {op}")
        got, idx = g_reduce(hip, op, x, b, e)
        check_reduce(orc, op, x, b, e, got, idx, "i32")
    log("segmented large scan")
    got = g_scan(hip, x, b, e, inclusive=True)
    want, _ = orc.segmented_scan(x, b, e, inclusive=True)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("ts", ["i32", "f32", "u64"])
def test_segment_reduce_many_segments_grouped(hip, orc, dev, ts):
    """More than 65,536 segments, so workgroups take several segments each: tiny segments reduced by one
    wave, some longer than 1,024 items by the whole workgroup, empty and reversed ones, all ops."""
    rng = np.random.default_rng(90 + len(ts))
    m = 150_000
    lengths = np.where(rng.random(m) < 0.002, rng.integers(1025, 6000, m), rng.integers(0, 12, m))
    b = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.uint32)
    e = (b.astype(np.int64) + lengths).astype(np.uint32)
    n = int(e[-1])
    x = values_for(rng, n, ts)
    e[5::1000] = b[5::1000] // 2  # begin > end: empty
    ops = ["sum", "min", "max"] + (["argmin", "argmax"] if ts in ("i32", "f32") else [])
    for op in ops:
        got, idx = g_reduce(hip, op, x, b, e)
        check_reduce(orc, op, x, b, e, got, idx, ts)


@pytest.mark.parametrize("ts", ["i32", "f32", "u64"])
def test_segment_reduce_millions_of_segments(hip, orc, dev, ts):
    """About 4.2 M segments, so every wave takes batches of 64 consecutive segments: batches of segments of
    at most 16 items reduced one segment per lane, batches holding a longer one (up to 1,024 items: by the
    wave; over 1,024: by the workgroup) one segment at a time; empty and reversed segments; all ops."""
    rng = np.random.default_rng(700 + len(ts))
    m = (1 << 22) + 77
    r = rng.random(m)
    lengths = np.where(r < 0.0005, rng.integers(1025, 3000, m),
                       np.where(r < 0.003, rng.integers(17, 1025, m), rng.integers(0, 17, m)))
    b = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.uint32)
    e = (b.astype(np.int64) + lengths).astype(np.uint32)
    n = int(e[-1])
    x = values_for(rng, n, ts)
    e[7::5000] = b[7::5000] // 2  # begin > end: empty
    ops = ["sum", "min", "argmax"] if ts in ("i32", "f32") else ["sum", "max"]
    log(f"segment reduce {m} segments {ts}")
    for op in ops:
        got, idx = g_reduce(hip, op, x, b, e)
        check_reduce(orc, op, x, b, e, got, idx, ts)


@pytest.mark.parametrize("ts", ["i32", "f64"])
def test_segmented_scan_millions_of_segments(hip, orc, dev, ts):
    """About 2.1 M segments in batches of 32 per wave: batches of segments of at most 16 items scanned one
    segment per lane, other batches one segment at a time (by the wave, or the workgroup beyond 1,024
    items); empty and reversed segments; exclusive with an initial value, and inclusive."""
    rng = np.random.default_rng(800 + len(ts))
    m = (1 << 21) + 33
    r = rng.random(m)
    lengths = np.where(r < 0.0005, rng.integers(1025, 2500, m),
                       np.where(r < 0.003, rng.integers(17, 1025, m), rng.integers(0, 17, m)))
    b = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.uint32)
    e = (b.astype(np.int64) + lengths).astype(np.uint32)
    n = int(e[-1])
    x = values_for(rng, n, ts)
    e[9::4000] = b[9::4000] // 2  # begin > end: empty
    log(f"segmented scan {m} segments {ts}")
    for kw in ({"init": 5}, {"inclusive": True}):
        got = g_scan(hip, x, b, e, ob=b.copy(), out_size=n, **kw)
        want, ab = orc.segmented_scan(x, b, e, out_begins=b.copy(), out_size=n, **kw)
        if ts in REL:
            assert np.all(np.abs(got.astype(np.float64) - want.astype(np.float64)) <= REL[ts] * ab + 1e-30), kw
        else:
            np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("ts", ["i32", "u64", "f64"])
def test_segmented_scan_many_segments_grouped(hip, orc, dev, ts):
    """More than 65,536 segments: short segments scanned by one wave, some longer than 1,024 items by the
    whole workgroup; exclusive, inclusive and with an initial value, packed output offsets."""
    rng = np.random.default_rng(120 + len(ts))
    m = 140_000
    lengths = np.where(rng.random(m) < 0.002, rng.integers(1025, 5000, m), rng.integers(0, 150, m))
    b = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.uint32)
    e = (b.astype(np.int64) + lengths).astype(np.uint32)
    n = int(e[-1])
    x = values_for(rng, n, ts)
    ob = b.copy()
    for kw in ({}, {"inclusive": True}, {"inclusive": True, "init": 3}):
        got = g_scan(hip, x, b, e, ob=ob, out_size=n, **kw)
        want, ab = orc.segmented_scan(x, b, e, out_begins=ob, out_size=n, **kw)
        if ts in REL:
            assert np.all(np.abs(got.astype(np.float64) - want.astype(np.float64)) <= REL[ts] * ab + 1e-30), kw
        else:
            np.testing.assert_array_equal(got, want)
