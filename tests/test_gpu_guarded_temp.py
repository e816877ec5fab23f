"""Temp storage and outputs are written only where a call owns them, through the C-ABI.

Every entry-point family gets temp storage of exactly the size its temp query returns (the reference's
Get*TempStorageBytes, rounded up to whole uint words as bytes_to_uint_count does) inside a buffer with 256
canary words on each side, as the reference's GuardedTemp does (tests/scan_optimization_regression_test.cpp:
75-103, tests/pr6_review_regression_test.cpp:427-457); after the call every canary must be intact.  Outputs
are followed by 8 sentinel items that must be intact too.

The scans also run the reference's exact binary-fraction cases (value(i) = i % 7 + 1, times 0.25 for
floats, :49-61,116-208): int, uint, float and double ExclusiveSum / InclusiveSum at its 19 boundary sizes up to
262,147 items, equal exactly to the host's sequential sums (every partial sum is a multiple of 0.25 below
2^24, so any summation order gives it exactly), and at 16,003 items ExclusiveScan / InclusiveScanInit with
init 3 in place and out of place, and InclusiveScan with the left projection."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import fill_dev, log, to_dev, to_host

pytestmark = pytest.mark.gpu

GUARD = 256
CANARY = 0x5EED5EED  # fits int32
SENTINEL_ITEMS = 8
DT = {"i32": np.int32, "u32": np.uint32, "f32": np.float32, "i64": np.int64, "u64": np.uint64, "f64": np.float64}


class GuardedTemp:
    def __init__(self, nbytes: int, dev):
        self.words = max(1, (nbytes + 3) // 4)
        self.backing = torch.full((self.words + 2 * GUARD,), CANARY, dtype=torch.int32, device=dev)
        self.view = self.backing[GUARD:GUARD + self.words]

    @property
    def ptr(self):
        return ctypes.c_void_p(self.view.data_ptr())

    @property
    def nbytes(self):
        return self.words * 4

    def verify(self, label: str):
        h = self.backing.cpu().numpy()
        assert (h[:GUARD] == CANARY).all(), f"{label}: wrote below temp storage"
        assert (h[GUARD + self.words:] == CANARY).all(), f"{label}: wrote past temp storage"


def sentinel(dt):
    return np.array(-777).astype(dt)


def padded(a: np.ndarray) -> np.ndarray:
    return np.concatenate([a, np.full(SENTINEL_ITEMS, sentinel(a.dtype), a.dtype)])


def same_bits(x, y):
    return np.array_equal(x.view(f"u{x.itemsize}"), y.view(f"u{y.itemsize}"))


def value(i: np.ndarray, dt):
    q = i % 7 + 1
    return (q * 0.25).astype(dt) if np.dtype(dt).kind == "f" else q.astype(dt)


def host_scan(x, inclusive, init=0):
    """Sequential sums in int64 (integers, wrapped into the type) or float64 (exact here)."""
    acc = np.cumsum(x.astype(np.float64 if x.dtype.kind == "f" else np.int64)) + init
    excl = np.concatenate([[init], acc[:-1]]) if x.size else acc
    r = acc if inclusive else excl
    return r.astype(x.dtype) if x.dtype.kind == "f" else (r.astype(np.int64) & ((1 << (8 * x.itemsize)) - 1)).astype(
        np.uint64).astype(x.dtype)


SIZES = [0, 1, 31, 32, 33, 255, 256, 257, 3839, 3840, 3841, 4095, 4096, 4097, 7999, 8000, 8001, 16003, 262147]


@pytest.mark.parametrize("suffix", ["i32", "u32", "f32", "f64"])
def test_exact_scans_at_reference_sizes_with_guarded_temp(hip, dev, suffix):
    dt = DT[suffix]
    for n in SIZES:
        host = padded(value(np.arange(n), dt))
        d_in = to_dev(host)
        g = GuardedTemp(hip.scan_temp_bytes(n, np.dtype(dt).itemsize), dev)
        for inclusive in (False, True):
            d_out = to_dev(np.full(n + SENTINEL_ITEMS, sentinel(dt), dt))
            hip.scan_sum(suffix, d_in, d_out, n, inclusive=inclusive, temp=g.view)
            want = padded(host_scan(host[:n], inclusive))
            assert same_bits(to_host(d_out, dt), want), (n, inclusive)
            g.verify(f"{suffix} n={n} inclusive={inclusive}")
        if n != 16003:
            continue
        log(f"exact scans {suffix}: init 3, in place and out of place, left projection")
        for mode in range(4):
            inclusive, in_place = mode % 2 == 1, mode < 2
            src = to_dev(host)
            dst = src if in_place else to_dev(np.full(n + SENTINEL_ITEMS, sentinel(dt), dt))
            hip.scan_sum(suffix, src, dst, n, inclusive=inclusive, init=3, temp=g.view)
            want = padded(host_scan(host[:n], inclusive, init=3))
            assert same_bits(to_host(dst, dt), want), (mode, in_place)
            g.verify(f"{suffix} init mode={mode}")
        d_out = to_dev(np.full(n + SENTINEL_ITEMS, sentinel(dt), dt))
        hip.scan_minmax("left", suffix, d_in, d_out, n, inclusive=True, temp=g.view)
        assert same_bits(to_host(d_out, dt), padded(np.full(n, host[0], dt)))
        g.verify(f"{suffix} left projection")


def _sorted_check(got, keys):
    assert np.array_equal(got[:keys.size], np.sort(keys, kind="stable"))
    assert same_bits(got[keys.size:], np.full(SENTINEL_ITEMS, sentinel(keys.dtype), keys.dtype))


@pytest.mark.parametrize("n", [5000, (1 << 22) + 5])
def test_reduce_scan_sort_spmv_stay_inside_their_temp(hip, orc, dev, n):
    rng = np.random.default_rng(n)
    log(f"guarded temp: reduce / scan / sort / spmv n={n}")
    a = rng.integers(-1000, 1000, n).astype(np.int32)
    d = to_dev(a)
    out = fill_dev(1 + SENTINEL_ITEMS, 8, -777)
    for name, call in (
            ("Sum i32", lambda t: hip.reduce_sum("i32", d, out, n, temp=t)),
            ("Min i32", lambda t: hip.reduce_minmax("min", "i32", d, out, n, temp=t)),
            ("Reduce max i32", lambda t: hip.reduce_op("max", "i32", d, out, n, init=5, temp=t)),
            ("TransformReduce sum i32", lambda t: hip.transform_reduce("sum", "square", "i32", d, out, n, temp=t))):
        g = GuardedTemp(hip.reduce_temp_bytes(n, 4), dev)
        call(g.view)
        g.verify(name)
        assert (to_host(out, np.int64)[1:] == -777).all(), name
    g = GuardedTemp(hip.reduce_arg_temp_bytes(n, 4), dev)
    idx = fill_dev(1 + SENTINEL_ITEMS, 4, -777)
    hip.reduce_arg("min", "i32", d, out, idx, n, temp=g.view)
    g.verify("ArgMin i32")
    assert (to_host(idx, np.int32)[1:] == -777).all()
    f64 = rng.standard_normal(n)
    g = GuardedTemp(hip.reduce_temp_bytes(n, 8), dev)
    hip.reduce_sum("f64", to_dev(f64), out, n, temp=g.view)
    g.verify("Sum f64")

    for suffix, op in (("i64", "min"), ("u32", "left"), ("f32", "max")):
        x = rng.integers(0, 1 << 20, n).astype(DT[suffix])
        dst = to_dev(padded(np.zeros(n, x.dtype)))
        g = GuardedTemp(hip.scan_temp_bytes(n, x.itemsize), dev)
        hip.scan_minmax(op, suffix, to_dev(x), dst, n, inclusive=True, temp=g.view)
        g.verify(f"scan {op} {suffix}")
        assert same_bits(to_host(dst, x.dtype)[n:], np.full(SENTINEL_ITEMS, sentinel(x.dtype), x.dtype))

    for suffix in ("u32", "f32", "i64"):
        keys = rng.integers(0, 1 << 40, n).astype(DT[suffix])
        kb = keys.itemsize
        ko = to_dev(padded(np.zeros(n, keys.dtype)))
        g = GuardedTemp(hip.sort_keys_temp_bytes(n, kb), dev)
        hip.sort_keys(suffix, to_dev(keys), ko, n, temp=g.view)
        g.verify(f"SortKeys {suffix}")
        _sorted_check(to_host(ko, keys.dtype), keys)
        vals = np.arange(n, dtype=np.uint32)
        vo = to_dev(padded(np.zeros(n, np.uint32)))
        ko = to_dev(padded(np.zeros(n, keys.dtype)))
        g = GuardedTemp(hip.sort_pairs_temp_bytes(n, kb, 4), dev)
        hip.sort_pairs(suffix, 4, to_dev(keys), ko, to_dev(vals), vo, n, temp=g.view)
        g.verify(f"SortPairs {suffix}")
        _sorted_check(to_host(ko, keys.dtype), keys)
        g = GuardedTemp(hip.sort_keys_temp_bytes(n, kb), dev)
        b0, b1 = to_dev(padded(keys)), to_dev(padded(np.zeros(n, keys.dtype)))
        sel = hip.sort_keys_db(suffix, b0, b1, 0, n, temp=g.view)
        g.verify(f"SortKeys DoubleBuffer {suffix}")
        _sorted_check(to_host((b0, b1)[sel], keys.dtype), keys)

    rows = cols = 2000
    lengths = rng.integers(0, 30, rows)
    ro = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    nnz = int(ro[-1])
    ci = rng.integers(0, cols, nnz).astype(np.int32)
    va, xv = rng.standard_normal(nnz).astype(np.float32), rng.standard_normal(cols).astype(np.float32)
    y = to_dev(padded(np.zeros(rows, np.float32)))
    g = GuardedTemp(0, dev)
    rc = hip.lib().lcpp_hip_spmv_csr_f32_i32(g.ptr, g.nbytes, to_dev(va).data_ptr(), to_dev(ro).data_ptr(),
                                              to_dev(ci).data_ptr(), to_dev(xv).data_ptr(), y.data_ptr(), rows, cols,
                                              nnz, None)
    assert rc == hip.OK
    g.verify("CsrMV")
    assert same_bits(to_host(y, np.float32)[rows:], np.full(SENTINEL_ITEMS, sentinel(np.float32), np.float32))


@pytest.mark.parametrize("n", [5000, (1 << 22) + 5])
def test_by_key_compaction_segmented_stay_inside_their_temp(hip, orc, dev, n):
    rng = np.random.default_rng(n + 1)
    log(f"guarded temp: by-key / compaction / segmented n={n}")
    keys = np.repeat(np.arange(n), rng.integers(1, 6, n))[:n].astype(np.int32)
    vals = rng.integers(-100, 100, n).astype(np.int32)
    dk, dv = to_dev(keys), to_dev(vals)

    g = GuardedTemp(hip.scan_by_key_temp_bytes(n, 4, 4), dev)
    out = to_dev(padded(np.zeros(n, np.int32)))
    hip.scan_by_key("i32", "i32", dk, dv, out, n, inclusive=True, temp=g.view)
    g.verify("InclusiveSumByKey")
    assert (to_host(out, np.int32)[n:] == -777).all()

    g = GuardedTemp(hip.reduce_by_key_temp_bytes(n, 4, 4), dev)
    uniq, agg = to_dev(padded(np.zeros(n, np.int32))), to_dev(padded(np.zeros(n, np.int32)))
    runs = fill_dev(1, 4, 0)
    hip.reduce_by_key("i32", "i32", dk, dv, uniq, agg, runs, n, temp=g.view)
    g.verify("ReduceByKey")
    r = int(to_host(runs, np.int32)[0])
    ou, oa = orc.reduce_by_key_int(keys, vals)
    assert r == ou.size and np.array_equal(to_host(uniq, np.int32)[:r], ou)

    pred = hip.predicate("i32", (hip.PRED_LT, 0))
    num = fill_dev(2, 4, 0)
    for name, tb, call in (
            ("select_if", hip.select_temp_bytes(n), lambda t, o: hip.select_if("i32", dv, o, num, n, pred, temp=t)),
            ("partition_if", hip.select_temp_bytes(n),
             lambda t, o: hip.partition_if("i32", dv, o, num, n, pred, temp=t)),
            ("select_unique", hip.select_temp_bytes(n), lambda t, o: hip.select_unique("i32", dk, o, num, n, temp=t)),
            ("run_length_encode", hip.run_length_encode_temp_bytes(n),
             lambda t, o: hip.run_length_encode("i32", dk, o, agg, num, n, temp=t))):
        g = GuardedTemp(tb, dev)
        o = to_dev(padded(np.zeros(n, np.int32)))
        call(g.view, o)
        g.verify(name)
        assert (to_host(o, np.int32)[n:] == -777).all(), name
    g = GuardedTemp(hip.partition_three_way_temp_bytes(n), dev)
    outs = [to_dev(padded(np.zeros(n, np.int32))) for _ in range(3)]
    hip.partition_three_way("i32", dv, *outs, num, n, pred, hip.predicate("i32", (hip.PRED_GT, 50)), temp=g.view)
    g.verify("partition three-way")

    m = max(1, n // 100)
    begins = np.sort(rng.integers(0, n, m)).astype(np.int64)
    ends = np.minimum(np.minimum(begins + rng.integers(0, 300, m), n), np.r_[begins[1:], n])  # disjoint segments
    begins, ends = begins.astype(np.uint32), ends.astype(np.uint32)
    db, de = to_dev(begins), to_dev(ends)
    lib = hip.lib()
    seg_out = to_dev(padded(np.zeros(m, np.int32)))
    g = GuardedTemp(lib.lcpp_hip_segment_reduce_temp_bytes(n), dev)
    assert lib.lcpp_hip_segment_reduce_sum_i32(g.ptr, g.nbytes, dv.data_ptr(), seg_out.data_ptr(), m, db.data_ptr(),
                                               de.data_ptr(), None) == hip.OK
    g.verify("segment reduce")
    assert (to_host(seg_out, np.int32)[m:] == -777).all()
    g = GuardedTemp(lib.lcpp_hip_segmented_scan_temp_bytes(n, m), dev)
    scan_out = to_dev(padded(np.zeros(n, np.int32)))
    assert lib.lcpp_hip_segmented_scan_sum_i32(g.ptr, g.nbytes, dv.data_ptr(), scan_out.data_ptr(), db.data_ptr(),
                                               de.data_ptr(), None, m, 1, 0, 0, None) == hip.OK
    g.verify("segmented scan")
    assert (to_host(scan_out, np.int32)[n:] == -777).all()
    for with_values in (False, True):
        nb = hip.segmented_sort_pairs_temp_bytes(n, 4, 4) if with_values else hip.segmented_sort_keys_temp_bytes(n, 4)
        g = GuardedTemp(nb, dev)
        ko = to_dev(padded(keys[::-1].copy()))
        vo = to_dev(padded(np.zeros(n, np.int32))) if with_values else None
        hip.segmented_sort("i32", to_dev(keys[::-1].copy()), ko, n, m, db, de,
                           values_in=dv if with_values else None, values_out=vo, temp=g.view)
        g.verify(f"segmented sort values={with_values}")
        assert (to_host(ko, np.int32)[n:] == -777).all()
