"""DeviceScan::ExclusiveSum / InclusiveSum on the GPU vs the oracle (bit-exact for 32-bit integers).

Cases follow the reference tests: sums of 2^i ones (tests/device_scan_test.cpp:80-127), (i%7)-3 data
(:189-265), InclusiveScanInit {1,2,3,4}+10 (:288-321), the regression sizes around tile edges
(tests/scan_optimization_regression_test.cpp:49-61,116-208), the decoupled look-back over many tiles
(tests/decoupled_look_back.cpp:56-186), and the benchmark input (2^28 uint32 in [0, 16)).
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
    yield
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
