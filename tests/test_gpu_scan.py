"""DeviceScan::ExclusiveSum / InclusiveSum on the GPU vs the oracle (bit-exact for 32-bit integers).

Cases follow the reference tests: sums of 2^i ones (tests/device_scan_test.cpp:80-127), (i%7)-3 data
(:189-265), InclusiveScanInit {1,2,3,4}+10 (:288-321), the regression sizes around tile edges
(tests/scan_optimization_regression_test.cpp:49-61,116-208), the decoupled look-back over many tiles
(tests/decoupled_look_back.cpp:56-186), and the benchmark input (2^28 uint32 in [0, 16)).  8-byte items
(int64 / uint64 / double; device_scan.h accepts any NumericT) follow the reference's InclusiveSum<double>
case (tests/device_scan_test.cpp:267-286) and are bit-exact for integers (64-bit wrap-around), within a
stated bound for doubles.
"""
import numpy as np
import pytest
import torch

from gpu_util import empty_dev, fill_dev, log, to_dev, to_host

pytestmark = pytest.mark.gpu

REGRESSION_SIZES = [1, 31, 32, 33, 255, 256, 257, 3839, 3840, 3841, 4095, 4096, 4097, 7999, 8000, 8001, 16003,
                    262147]


def gpu_scan(hip, suffix, a, inclusive=False, init=None, offset_in=0, offset_out=0):
    n = a.size - offset_in
    d_in = to_dev(a)[offset_in:]
    out_full = fill_dev(n + offset_out, a.dtype.itemsize, 0x7E7E7E7E)
    d_out = out_full[offset_out:]
    hip.scan_sum(suffix, d_in, d_out, n, inclusive=inclusive, init=init)
    return to_host(out_full, a.dtype)[offset_out:offset_out + n]


@pytest.mark.parametrize("i", list(range(0, 24)))
def test_ones(hip, orc, dev, i):
    n = 1 << i
    log(f"scan ones n={n}")
    ones = np.ones(n, np.uint32)
    assert np.array_equal(gpu_scan(hip, "u32", ones), np.arange(n, dtype=np.uint32))
    assert np.array_equal(gpu_scan(hip, "u32", ones, inclusive=True), np.arange(1, n + 1, dtype=np.uint32))


@pytest.mark.parametrize("n", REGRESSION_SIZES)
def test_regression_sizes_signed(hip, orc, dev, n):
    a = ((np.arange(n) % 7) - 3).astype(np.int32)
    for inclusive in (False, True):
        assert np.array_equal(gpu_scan(hip, "i32", a, inclusive), orc.scan_sum_u32(a, inclusive))


def test_inclusive_scan_init_known_answer(hip, dev):
    a = np.array([1, 2, 3, 4], np.int32)
    assert gpu_scan(hip, "i32", a, inclusive=True, init=10).tolist() == [11, 13, 16, 20]
    assert gpu_scan(hip, "i32", a, inclusive=False, init=10).tolist() == [10, 11, 13, 16]


def test_many_tiles_lookback(hip, orc, dev):
    # 102,400 tiles of ones in the reference's look-back test; here 2^26 items = 16,384 tiles of 4096.
    n = 1 << 26
    ones = torch.ones(n, dtype=torch.int32, device=dev)
    out = torch.empty_like(ones)
    hip.scan_sum("u32", ones, out, n)
    assert torch.equal(out, torch.arange(n, dtype=torch.int32, device=dev))


@pytest.mark.parametrize("offset_in,offset_out", [(1, 0), (0, 3), (2, 1)])
def test_unaligned_views(hip, orc, dev, offset_in, offset_out):
    a = orc.generate(3, 100003, 3)
    got = gpu_scan(hip, "u32", a, offset_in=offset_in, offset_out=offset_out)
    assert np.array_equal(got, orc.scan_sum_u32(a[offset_in:]))


def test_wraparound(hip, orc, dev):
    a = orc.generate(1, 1000003, 8)  # full 32-bit values: the running sum wraps many times
    for inclusive in (False, True):
        assert np.array_equal(gpu_scan(hip, "u32", a, inclusive), orc.scan_sum_u32(a, inclusive))


def test_float_within_tolerance(hip, orc, dev):
    # |gpu - exact| <= (i+1) * eps * running sum|x| per element (any summation order satisfies it).
    n = 262147
    a = orc.generate(6, n, 21)
    got = gpu_scan(hip, "f32", a).astype(np.float64)
    exact, absum = orc.scan_sum_f32(a)
    bound = (np.arange(n) + 2) * np.finfo(np.float32).eps * absum
    assert np.all(np.abs(got - exact) <= bound)


def test_empty_is_noop(hip, dev):
    out = fill_dev(4, 4, 77)
    hip.scan_sum("u32", out, out, 0)
    assert to_host(out, np.int32).tolist() == [77] * 4


def test_temp_too_small_is_an_error(hip, dev):
    a = torch.zeros(100000, dtype=torch.int32, device=dev)
    temp = torch.empty(2, dtype=torch.int32, device=dev)
    with pytest.raises(hip.LcppHipError) as e:
        hip.scan_sum("u32", a, a, 100000, temp=temp)
    assert e.value.status == hip.ERR_TEMP_TOO_SMALL


def test_benchmark_input_2p28(hip, orc, dev):
    """2^28 uint32 in [0, 16) from seed 114521, full output compared bit-exact."""
    n = 1 << 28
    log("scan 2^28")
    d = torch.empty(n, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_LT16, d, n, 114521)
    out = torch.empty_like(d)
    hip.scan_sum("u32", d, out, n)
    host_in = to_host(d, np.uint32)
    assert np.array_equal(to_host(out, np.uint32), orc.scan_sum_u32(host_in))


@pytest.fixture
def forced_fallback(hip):
    """Every look-back predecessor that is not yet published is computed by the waiting workgroup."""
    lib = hip.lib()
    old = lib.lcpp_hip_get_lookback_spin_limit()
    lib.lcpp_hip_set_lookback_spin_limit(0)
    try:
        yield
    finally:
        lib.lcpp_hip_set_lookback_spin_limit(old)


@pytest.mark.parametrize("n", [4097, 65536 * 3 + 5, (1 << 22) + 77])
def test_forced_fallback_integer(hip, orc, dev, forced_fallback, n):
    log(f"scan forced fallback n={n}")
    a = orc.generate(1, n, n)
    for inclusive in (False, True):
        assert np.array_equal(gpu_scan(hip, "u32", a, inclusive), orc.scan_sum_u32(a, inclusive))
    assert np.array_equal(gpu_scan(hip, "u32", a, False, offset_in=1), orc.scan_sum_u32(a[1:]))


def test_forced_fallback_float_within_tolerance(hip, orc, dev, forced_fallback):
    # Float prefixes combine PARTIAL and INCLUSIVE aggregates in a timing-dependent grouping (as in any
    # decoupled look-back), so the check is the order-independent bound of test_float_within_tolerance.
    n = (1 << 22) + 123
    a = orc.generate(6, n, 5)
    got = gpu_scan(hip, "f32", a).astype(np.float64)
    exact, absum = orc.scan_sum_f32(a)
    bound = (np.arange(n) + 2) * np.finfo(np.float32).eps * absum
    assert np.all(np.abs(got - exact) <= bound)


def gpu_scan_in_place(hip, suffix, a, inclusive=False, init=None):
    """Scans `a` with d_in == d_out, as the reference's InclusiveScanInit test does
    (tests/device_scan_test.cpp:288-321)."""
    d = to_dev(a)
    hip.scan_sum(suffix, d, d, a.size, inclusive=inclusive, init=init)
    return to_host(d, a.dtype)


def test_in_place_known_answer(hip, dev):
    a = np.array([1, 2, 3, 4], np.int32)
    assert gpu_scan_in_place(hip, "i32", a, inclusive=True, init=10).tolist() == [11, 13, 16, 20]


@pytest.mark.parametrize("n", [24576 * 3 + 11, (1 << 22) + 77])
def test_in_place_matches_oracle(hip, orc, dev, n):
    a = orc.generate(1, n, n + 1)
    for inclusive in (False, True):
        assert np.array_equal(gpu_scan_in_place(hip, "u32", a, inclusive), orc.scan_sum_u32(a, inclusive))


@pytest.mark.parametrize("n", [24576 * 5 + 3, (1 << 22) + 77])
def test_in_place_forced_fallback(hip, orc, dev, forced_fallback, n):
    """Every look-back claims and recomputes its unpublished predecessors while their owners may be
    overwriting the same buffer: the claim protocol keeps the in-place result exact."""
    log(f"scan in-place forced fallback n={n}")
    a = orc.generate(1, n, n + 2)
    for inclusive in (False, True):
        assert np.array_equal(gpu_scan_in_place(hip, "u32", a, inclusive), orc.scan_sum_u32(a, inclusive))


# ---- 8-byte items --------------------------------------------------------------------------------
TILE64 = 12288  # 8-byte items per scan tile
SIZES64 = [1, 17, 255, 256, 257, TILE64 - 1, TILE64, TILE64 + 1, 3 * TILE64 + 5, 1000003]


def test_inclusive_sum_double_known_answer(hip, dev):
    """tests/device_scan_test.cpp:267-286: InclusiveSum<double> of 17 ones is 1..17 exactly."""
    got = gpu_scan(hip, "f64", np.ones(17))
    assert got.tolist() == list(range(17))
    got = gpu_scan(hip, "f64", np.ones(17), inclusive=True)
    assert got.tolist() == [float(i + 1) for i in range(17)]


@pytest.mark.parametrize("n", SIZES64)
def test_u64_ones(hip, orc, dev, n):
    ones = np.ones(n, np.uint64)
    assert np.array_equal(gpu_scan(hip, "u64", ones), np.arange(n, dtype=np.uint64))
    assert np.array_equal(gpu_scan(hip, "u64", ones, inclusive=True), np.arange(1, n + 1, dtype=np.uint64))


@pytest.mark.parametrize("n", SIZES64)
def test_i64_wraparound(hip, orc, dev, n):
    a = orc.generate(0, n, n + 5).view(np.int64)  # full 64-bit words: the running sum wraps
    for inclusive in (False, True):
        assert np.array_equal(gpu_scan(hip, "i64", a, inclusive), orc.scan_sum_u64(a, inclusive))
    assert np.array_equal(gpu_scan(hip, "i64", a, True, init=-3), orc.scan_sum_u64(a, True, -3))
    u = a.view(np.uint64)
    assert np.array_equal(gpu_scan(hip, "u64", u, False, init=12345), orc.scan_sum_u64(u, False, 12345))


def test_64bit_unaligned_views(hip, orc, dev):
    a = orc.generate(0, 100003, 11)
    for offset_in, offset_out in ((1, 0), (0, 1), (1, 1)):
        got = gpu_scan(hip, "u64", a, offset_in=offset_in, offset_out=offset_out)
        assert np.array_equal(got, orc.scan_sum_u64(a[offset_in:]))


def test_f64_within_tolerance(hip, orc, dev):
    # |gpu - exact| <= (i+2) * eps64 * running sum|x| per element (any summation order satisfies it).
    n = 1000003
    rng = np.random.default_rng(17)
    a = rng.uniform(-1.0, 1.0, n)
    for inclusive in (False, True):
        got = gpu_scan(hip, "f64", a, inclusive).astype(np.longdouble)
        exact, absum = orc.scan_sum_f64(a, inclusive)
        bound = (np.arange(n) + 2) * np.finfo(np.float64).eps * absum
        assert np.all(np.abs(got - exact) <= bound)


def test_u64_2p27_full(hip, orc, dev):
    """2^27 uint64 words (10,923 tiles of look-back), full output compared bit-exact."""
    n = 1 << 27
    log("scan u64 2^27")
    d = torch.empty(n, dtype=torch.int64, device=dev)
    hip.generate(hip.GEN_U64, d, n, 114521)
    out = torch.empty_like(d)
    hip.scan_sum("u64", d, out, n)
    assert np.array_equal(to_host(out, np.uint64), orc.scan_sum_u64(to_host(d, np.uint64)))


@pytest.mark.parametrize("n", [TILE64 * 3 + 7, (1 << 22) + 77])
def test_64bit_forced_fallback(hip, orc, dev, forced_fallback, n):
    """Claimed predecessors publish both words of their state; readers accept only matching pairs."""
    log(f"scan u64 forced fallback n={n}")
    a = orc.generate(0, n, n + 9)
    for inclusive in (False, True):
        assert np.array_equal(gpu_scan(hip, "u64", a, inclusive), orc.scan_sum_u64(a, inclusive))
    b = np.ones(n, np.float64)
    assert gpu_scan(hip, "f64", b, inclusive=True).tolist() == [float(i + 1) for i in range(n)]


@pytest.mark.parametrize("n", [TILE64 * 5 + 3, (1 << 22) + 77])
def test_64bit_in_place_forced_fallback(hip, orc, dev, forced_fallback, n):
    log(f"scan u64 in-place forced fallback n={n}")
    a = orc.generate(0, n, n + 13)
    for inclusive in (False, True):
        assert np.array_equal(gpu_scan_in_place(hip, "u64", a, inclusive), orc.scan_sum_u64(a, inclusive))


# ---- min / max operators -------------------------------------------------------------------------
# DeviceScan<>::ExclusiveScan / InclusiveScan / InclusiveScanInit with MinOp / MaxOp (device_scan.h:321-368,
# common/thread_operators.h:58-74), bit-exact against the oracle's left-to-right fold for every type.
MINMAX_SUFFIX = {"i32": np.int32, "u32": np.uint32, "f32": np.float32, "i64": np.int64, "u64": np.uint64,
                 "f64": np.float64}
TILE32 = 24576  # 4-byte items per scan tile


def gpu_scan_minmax(hip, op, suffix, a, inclusive=False, init=None):
    n = a.size
    d_in = to_dev(a)
    d_out = fill_dev(n, a.dtype.itemsize, 0x7E7E7E7E)
    hip.scan_minmax(op, suffix, d_in, d_out, n, inclusive=inclusive, init=init)
    return to_host(d_out, a.dtype)


def minmax_input(suffix, n, seed, nan_fraction=0.02):
    """Full-range integers, or floats with canonical NaNs and no zeros (the sign of a zero tie is tested
    apart)."""
    dtype = np.dtype(MINMAX_SUFFIX[suffix])
    rng = np.random.default_rng(seed)
    if dtype.kind == "f":
        a = (rng.standard_normal(n) * 1000).astype(dtype)
        a[a == 0] = 1
        a[rng.random(n) < nan_fraction] = np.nan
        return a
    info = np.iinfo(dtype)
    return rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)


def same_bits(x, y):
    return x.dtype == y.dtype and np.array_equal(x.view(f"u{x.dtype.itemsize}"), y.view(f"u{y.dtype.itemsize}"))


def test_scan_max_exclusive_known_answer(hip, dev):
    """tests/pr6_review_regression_test.cpp:146-151,247-265: exclusive max with init 0 over i % 7 + 1."""
    n = 4097
    a = (np.arange(n) % 7 + 1).astype(np.int32)
    assert np.array_equal(gpu_scan_minmax(hip, "max", "i32", a, init=0), np.minimum(np.arange(n), 7))


@pytest.mark.parametrize("suffix", list(MINMAX_SUFFIX))
@pytest.mark.parametrize("op", ["min", "max"])
@pytest.mark.parametrize("n", [1, 31, 257, TILE64 - 1, TILE64 + 1, TILE32 + 1, 3 * TILE32 + 7, (1 << 22) + 77])
def test_scan_minmax_vs_oracle(hip, orc, dev, suffix, op, n):
    log(f"scan {op} {suffix} n={n}")
    a = minmax_input(suffix, n, n * 7 + len(suffix))
    inits = [None, np.nan, 0.5] if a.dtype.kind == "f" else [None, 0, 12345]
    for inclusive in (False, True):
        for init in inits:
            got = gpu_scan_minmax(hip, op, suffix, a, inclusive, init)
            assert same_bits(got, orc.scan_minmax(op, a, inclusive, init)), (inclusive, init)


@pytest.mark.parametrize("suffix", ["i32", "u64", "f32", "f64"])
def test_scan_minmax_monotone(hip, orc, dev, suffix):
    """Descending input: every item is a new minimum, so every tile's prefix comes from the look-back."""
    n = (1 << 22) + 77
    a = np.arange(n, 0, -1).astype(MINMAX_SUFFIX[suffix])
    for op in ("min", "max"):
        for inclusive in (False, True):
            got = gpu_scan_minmax(hip, op, suffix, a, inclusive)
            assert same_bits(got, orc.scan_minmax(op, a, inclusive))


@pytest.mark.parametrize("suffix", ["f32", "f64"])
def test_scan_minmax_signed_zero_order(hip, orc, dev, suffix):
    """Zeros of both signs compare equal and the earlier is kept: +0.0 first and -0.0 everywhere after
    must give +0.0 at every position across lanes, waves, rows, tiles and look-back windows (an operand
    swapped anywhere lets a -0.0 through), and the mirror case -0.0 first."""
    n = (1 << 22) + 77
    dtype = MINMAX_SUFFIX[suffix]
    a = np.full(n, -0.0, dtype)
    a[0] = 0.0
    rng = np.random.default_rng(5)
    b = np.where(rng.random(n) < 0.5, dtype(0.0), dtype(-0.0)).astype(dtype)
    b[0] = -0.0
    for op in ("min", "max"):
        for x in (a, b):
            got = gpu_scan_minmax(hip, op, suffix, x, inclusive=True)
            assert same_bits(got, orc.scan_minmax(op, x, inclusive=True))
            assert np.all(np.signbit(got) == np.signbit(x[0]))


@pytest.mark.parametrize("suffix", ["u32", "f32", "i64", "f64"])
def test_scan_minmax_forced_fallback(hip, orc, dev, forced_fallback, suffix):
    """Predecessors computed by the waiting workgroup fold in the owner's order, signed zeros included."""
    n = (1 << 22) + 77
    log(f"scan minmax forced fallback {suffix}")
    a = minmax_input(suffix, n, 23)
    for op in ("min", "max"):
        for inclusive in (False, True):
            got = gpu_scan_minmax(hip, op, suffix, a, inclusive)
            assert same_bits(got, orc.scan_minmax(op, a, inclusive))
    if suffix.startswith("f"):
        z = np.full(n, -0.0, MINMAX_SUFFIX[suffix])
        z[0] = 0.0
        assert not np.any(np.signbit(gpu_scan_minmax(hip, "min", suffix, z, inclusive=True)))


def test_scan_minmax_all_nan_prefix(hip, orc, dev):
    """Floats like fmin / fmax: NaN items are skipped, an all-NaN prefix stays NaN."""
    for suffix in ("f32", "f64"):
        a = np.full(TILE32 * 2 + 5, np.nan, MINMAX_SUFFIX[suffix])
        a[TILE32 + 3] = 2.0
        a[TILE32 + 9] = -1.0
        for op in ("min", "max"):
            got = gpu_scan_minmax(hip, op, suffix, a, inclusive=True)
            assert same_bits(got, orc.scan_minmax(op, a, inclusive=True))
            assert np.all(np.isnan(got[:TILE32 + 3])) and got[TILE32 + 3] == 2.0


def test_scan_minmax_empty_and_errors(hip, dev):
    d = torch.empty(0, dtype=torch.int32, device=dev)
    hip.scan_minmax("min", "i32", d, d, 0)
    with pytest.raises(ValueError):
        hip.scan_minmax("sum", "i32", d, d, 0)
    a = torch.zeros(1 << 20, dtype=torch.int32, device=dev)
    with pytest.raises(hip.LcppHipError) as e:
        hip.scan_minmax("max", "i32", a, a, 1 << 20, temp=torch.empty(2, dtype=torch.int32, device=dev))
    assert e.value.status == hip.ERR_TEMP_TOO_SMALL


def test_scan_minmax_in_place_forced_fallback(hip, orc, dev, forced_fallback):
    """In place: a claimed tile's owner stores only after its claimer has read the tile."""
    n = (1 << 22) + 77
    for suffix in ("i32", "f64"):
        a = minmax_input(suffix, n, 31)
        d = to_dev(a)
        hip.scan_minmax("min", suffix, d, d, n, inclusive=True)
        assert same_bits(to_host(d, a.dtype), orc.scan_minmax("min", a, inclusive=True))


# ---- the left projection op(lhs, rhs) = lhs ------------------------------------------------------------
# An associative operator that does not commute: every output is the scan's first operand, so any level
# (lane, wave, row, tile, look-back window, fallback) that combined operands in the wrong order would show.
# Bit-exact against the oracle's literal left-to-right fold.
LEFT_DTYPES = {"i32": np.int32, "u32": np.uint32, "f32": np.float32, "i64": np.int64, "u64": np.uint64,
               "f64": np.float64}


def test_scan_left_reference_cases(hip, dev):
    """tests/device_scan_test.cpp:129-155: ExclusiveScan with lhs and init 42 over 3,841 sevens is 42
    everywhere.  tests/scan_optimization_regression_test.cpp:195-205: InclusiveScan with lhs over
    value(i) (i % 7 + 1, times 0.25 for floats) at 16,003 items is in[0] everywhere, for int, uint, float
    and double."""
    assert (gpu_scan_minmax(hip, "left", "i32", np.full(3841, 7, np.int32), inclusive=False, init=42) == 42).all()
    q = np.arange(16003) % 7 + 1
    for suffix in ("i32", "u32", "f32", "f64"):
        dt = LEFT_DTYPES[suffix]
        h = (q * 0.25).astype(dt) if np.dtype(dt).kind == "f" else q.astype(dt)
        got = gpu_scan_minmax(hip, "left", suffix, h, inclusive=True)
        assert same_bits(got, np.full(h.size, h[0], dt)), suffix


@pytest.mark.parametrize("suffix", ["u32", "f32", "i64", "f64"])
@pytest.mark.parametrize("n", [1, 31, TILE32 + 1, 3 * TILE32 + 7, (1 << 22) + 77])
def test_scan_left_vs_oracle(hip, orc, dev, suffix, n):
    """Random bit patterns with all-ones words among them, a first item that is all ones, and initial values
    of every kind (an all-ones one too)."""
    dt = np.dtype(LEFT_DTYPES[suffix])
    u = np.dtype(f"u{dt.itemsize}")
    rng = np.random.default_rng(n + dt.itemsize)
    bits = rng.integers(0, np.iinfo(u).max, n, dtype=u, endpoint=True)
    bits[rng.random(n) < 0.01] = np.iinfo(u).max
    a = bits.view(dt)
    log(f"scan left {suffix} n={n}")
    ones = np.array([np.iinfo(u).max], u).view(dt)[0]  # a quiet NaN for floats: it survives ctypes
    first_ones = bits.copy()
    first_ones[0] = np.iinfo(u).max
    for x in (a, first_ones.view(dt)):
        got = gpu_scan_minmax(hip, "left", suffix, x, inclusive=True)
        assert same_bits(got, orc.scan_left(x, inclusive=True))
        for init in (dt.type(3), ones, np.array(-7).astype(dt)):
            for inclusive in (False, True):
                got = gpu_scan_minmax(hip, "left", suffix, x, inclusive=inclusive, init=init)
                assert same_bits(got, orc.scan_left(x, inclusive=inclusive, init=init)), (inclusive, init)


@pytest.mark.parametrize("suffix", ["u32", "f64"])
def test_scan_left_forced_fallback_and_in_place(hip, orc, dev, forced_fallback, suffix):
    """Predecessors computed by the waiting workgroup fold in the owner's order; an in-place scan reads in[0]
    that the scan writes back unchanged."""
    n = (1 << 22) + 77
    dt = LEFT_DTYPES[suffix]
    a = np.random.default_rng(12).integers(1, 1 << 30, n).astype(dt)
    for init in (None, dt(9)):
        got = gpu_scan_minmax(hip, "left", suffix, a, inclusive=True, init=init)
        assert same_bits(got, orc.scan_left(a, inclusive=True, init=init))
    d = to_dev(a)
    hip.scan_minmax("left", suffix, d, d, n, inclusive=True)
    assert same_bits(to_host(d, a.dtype), np.full(n, a[0], dt))


def test_scan_left_exclusive_without_init_is_rejected(hip, dev):
    a = torch.ones(1000, dtype=torch.int32, device=dev)
    with pytest.raises(hip.LcppHipError) as e:
        hip.scan_minmax("left", "i32", a, torch.empty_like(a), 1000, inclusive=False)
    assert e.value.status == hip.ERR_INVALID_ARGUMENT
