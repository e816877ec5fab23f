"""DeviceReduce::Sum on the GPU vs the oracle (bit-exact for integers; a stated tolerance for floats).

Cases follow the reference tests: sums of 2^k+1 ones (tests/device_reduce_test.cpp:95-119), shuffled
iota (:85-91), transform sizes {1,31,256,1023,1024,1025,1048577,4194304} (:148-173), 2^24+1 zeros
plus a tail value (tests/pr6_review_regression_test.cpp:427-457), the benchmark input (2^24 int32 in
[-1000, 1000] from seed 114521) and the 2^28 north-star size.
"""
import numpy as np
import pytest
import torch

from gpu_util import empty_dev, fill_dev, log, to_dev, to_host

pytestmark = pytest.mark.gpu


def run_sum(hip, suffix, a: np.ndarray, offset: int = 0):
    d = to_dev(a)
    d_in = d[offset:]
    out = fill_dev(1, a.dtype.itemsize, 0x5A5A5A5A)
    hip.reduce_sum(suffix, d_in, out, a.size - offset)
    return to_host(out, a.dtype, 1)[0]


@pytest.mark.parametrize("k", list(range(0, 24)))
def test_sum_of_ones(hip, orc, dev, k):
    n = (1 << k) + 1
    log(f"reduce ones n={n}")
    assert run_sum(hip, "i32", np.ones(n, np.int32)) == n


def test_shuffled_iota(hip, orc, dev):
    a = np.random.default_rng(114521).permutation(4096).astype(np.int32)
    assert run_sum(hip, "i32", a) == 4095 * 4096 // 2


@pytest.mark.parametrize("n", [1, 2, 3, 5, 31, 256, 1023, 1024, 1025, 4095, 4097, 65537, 1000003, 1048577, 4194304])
def test_ragged_sizes_i32(hip, orc, dev, n):
    a = orc.generate(2, n, 1234 + n)
    log(f"reduce ragged n={n}")
    assert run_sum(hip, "i32", a) == orc.reduce_sum_i32(a)[0]


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_unaligned_input_subview(hip, orc, dev, offset):
    a = orc.generate(2, 100003, 99)
    assert run_sum(hip, "i32", a, offset) == orc.reduce_sum_i32(a[offset:])[0]


def test_zeros_plus_tail(hip, orc, dev):
    n = (1 << 24) + 1
    a = np.zeros(n, np.int32)
    a[-1] = 7
    assert run_sum(hip, "i32", a) == 7


def test_empty_writes_init(hip, dev):
    out = fill_dev(1, 4, 0x12345)
    hip.reduce_sum("i32", out, out, 0)
    assert to_host(out, np.int32, 1)[0] == 0


def test_wraparound_u32_and_signed(hip, orc, dev):
    a = np.full(1 << 20, 0xFFFFFFFF, np.uint32)
    assert run_sum(hip, "u32", a) == orc.reduce_sum_u32(a)
    b = np.full(1 << 20, 2**31 - 1, np.int32)
    assert run_sum(hip, "i32", b) == orc.reduce_sum_i32(b)[0]


def test_64bit_integers(hip, orc, dev):
    a = orc.generate(0, 1000003, 5)
    assert int(run_sum(hip, "u64", a)) == orc.reduce_sum_u64(a)
    b = a.view(np.int64)
    expected = int(np.array([orc.reduce_sum_u64(a)], dtype=np.uint64).view(np.int64)[0])
    assert int(run_sum(hip, "i64", b)) == expected


@pytest.mark.parametrize("suffix,dtype", [("f32", np.float32), ("f64", np.float64)])
def test_floating_point_within_tolerance(hip, orc, dev, suffix, dtype):
    # Tolerance: |gpu - exact| <= n * eps(dtype) * sum|x| (the summation order differs from the
    # reference's tree; any order satisfies this bound).
    n = 1000003
    a = orc.generate(6, n, 17).astype(dtype)
    exact, absum = orc.reduce_sum_fp(a)
    got = float(run_sum(hip, suffix, a))
    eps = np.finfo(dtype).eps
    assert abs(got - exact) <= n * eps * absum


def test_benchmark_input_2p24(hip, orc, dev):
    """2^24 int32 in [-1000, 1000] from seed 114521: bit-exact and int64-safe."""
    n = 1 << 24
    d = torch.empty(n, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_I32_PM1000, d, n, 114521)
    host = orc.generate(2, n, 114521)
    assert np.array_equal(to_host(d, np.int32), host)
    out = fill_dev(1, 4, 0)
    hip.reduce_sum("i32", d, out, n)
    wrapped, exact = orc.reduce_sum_i32(host)
    assert -2**31 <= exact < 2**31
    assert to_host(out, np.int32, 1)[0] == wrapped


def test_north_star_size_2p28(hip, orc, dev):
    n = 1 << 28
    log("reduce 2^28")
    d = torch.empty(n, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_I32_PM1000, d, n, 4242)
    out = fill_dev(1, 4, 0)
    hip.reduce_sum("i32", d, out, n)
    assert to_host(out, np.int32, 1)[0] == orc.reduce_sum_i32(to_host(d, np.int32))[0]
