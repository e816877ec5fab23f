"""Pins the CPU oracle (oracle/oracle.c) before the GPU tests compare their results with it.

Each oracle function is checked against (a) the known-answer cases of the reference's own tests
(paths relative to the LCPP root), (b) closed forms, and (c) an independent algorithm (numpy / Python
comparison sorts), chosen so that a dropped term, a wrong sign or index, or a wrong twiddle fails.
"""
import math
import os
import shutil
import struct
import subprocess
import sys

import numpy as np
import pytest


# ---- splitmix64 ----------------------------------------------------------------------------------
def test_splitmix64_known_answers(orc):
    # Published SplittableRandom / splitmix64 outputs for seed 0.
    assert orc.splitmix64_at(0, 0) == 0xE220A8397B1DCDAF
    assert orc.splitmix64_at(0, 1) == 0x6E789E6AA1B965F4
    assert orc.splitmix64_at(0, 2) == 0x06C45D188009454F


def test_generator_mappings(orc):
    seed = 114521
    r = orc.generate(0, 1000, seed)
    assert np.array_equal(orc.generate(1, 1000, seed), (r >> np.uint64(32)).astype(np.uint32))
    pm = orc.generate(2, 1000, seed)
    assert np.array_equal(pm, (r % np.uint64(2001)).astype(np.int64) - 1000)
    assert pm.min() >= -1000 and pm.max() <= 1000
    assert np.array_equal(orc.generate(3, 1000, seed), (r & np.uint64(15)).astype(np.uint32))
    r3 = orc.generate(0, 3000, seed)
    assert np.array_equal(orc.generate(4, 1000, seed), r3[0::3] & r3[1::3] & r3[2::3])
    assert np.array_equal(orc.generate(5, 10, seed, start=7), np.arange(7, 17, dtype=np.uint32))
    # counter-based: a window equals the slice of a longer stream
    assert np.array_equal(orc.generate(0, 10, seed, start=500), r[500:510])


# ---- reduce --------------------------------------------------------------------------------------
@pytest.mark.parametrize("k", range(0, 24, 3))
def test_reduce_ones_known_answer(orc, k):
    # tests/device_reduce_test.cpp:95-119: Sum of 2^k+1 ones is 2^k+1.
    n = (1 << k) + 1
    assert orc.reduce_sum_i32(np.ones(n, np.int32)) == (n, n)


def test_reduce_shuffled_iota_and_empty(orc):
    # tests/device_reduce_test.cpp:85-91: shuffled iota 0..4095.
    a = np.random.default_rng(114521).permutation(4096).astype(np.int32)
    assert orc.reduce_sum_i32(a)[0] == 4095 * 4096 // 2
    assert orc.reduce_sum_i32(np.zeros(0, np.int32)) == (0, 0)


def test_reduce_wraps_modulo_2_32(orc):
    a = np.full(3, 2**31 - 1, np.int32)
    wrapped, exact = orc.reduce_sum_i32(a)
    assert exact == 3 * (2**31 - 1)
    assert wrapped == ((exact + 2**31) % 2**32) - 2**31
    assert orc.reduce_sum_u32(np.array([2**32 - 1, 2], np.uint32)) == 1
    assert orc.reduce_sum_u64(np.array([2**64 - 1, 5], np.uint64)) == 4


def test_reduce_closed_form_random(orc):
    a = orc.generate(2, 1 << 20, 114521)
    assert orc.reduce_sum_i32(a)[1] == int(a.astype(np.int64).sum())
    f = orc.generate(6, 10000, 7)
    s, absum = orc.reduce_sum_fp(f)
    assert math.isclose(s, math.fsum(f.astype(np.float64)), rel_tol=0, abs_tol=1e-9)
    assert math.isclose(absum, math.fsum(np.abs(f.astype(np.float64))), rel_tol=1e-12)


def test_reduce_sum_f64_closed_forms(orc):
    """The double branch (oracle_reduce_sum_f64).  Integers below 2^63 add exactly in long double, so the
    result is the int64 sum rounded once to double (a double accumulator would round along the way);
    the reference's exact binary fractions (i % 7 + 1) * 0.25 (tests/scan_optimization_regression_test.cpp:49-61)
    give 0.25 * the integer sum; random doubles agree with math.fsum (correctly rounded) to the long
    double's error bound."""
    rng = np.random.default_rng(21)
    a = rng.integers(-2**40, 2**40, 100000)
    s, absum = orc.reduce_sum_fp(a.astype(np.float64))
    assert s == float(int(a.sum()))
    assert absum == float(int(np.abs(a).sum()))
    big = np.array([2.0**53, 1.0, 1.0, -2.0**53], np.float64)  # a double accumulator loses both ones
    assert orc.reduce_sum_fp(big)[0] == 2.0
    q = np.arange(262147) % 7 + 1
    assert orc.reduce_sum_fp(q * 0.25)[0] == 0.25 * int(q.sum())
    r = rng.standard_normal(20000) * 1e3
    s, absum = orc.reduce_sum_fp(r)
    assert abs(s - math.fsum(r)) <= 1e-15 * absum
    assert math.isclose(absum, math.fsum(np.abs(r)), rel_tol=1e-15)
    assert orc.reduce_sum_fp(np.zeros(0, np.float64)) == (0.0, 0.0)


# ---- Reduce(op, init) / TransformReduce -------------------------------------------------------------
def test_transform_reduce_known_answers(orc):
    """tests/device_reduce_test.cpp:120-173: max of squares over a permutation of 0..4095 with init 0 is
    4095^2; the sum of 2x + 1 over x = i % 13 - 6 with init 17 at eight sizes.
    tests/pr6_review_regression_test.cpp:144-240 over i % 7 + 1 (4,097 items): sum and max with init 0,
    the transforms x + 1, x + 7, 2x, x * x and the identity under the sum."""
    a = np.random.default_rng(114521).permutation(4096).astype(np.int32)
    assert orc.transform_reduce(a, "max", "square", init=0)[0] == 4095 ** 2
    for size in (1, 31, 256, 1023, 1024, 1025, 1048577, 4194304):
        x = (np.arange(size) % 13 - 6).astype(np.int32)
        assert orc.transform_reduce(x, "sum", "affine", 2, 1, 17)[0] == 17 + int((2 * x.astype(np.int64) + 1).sum())
    h = (np.arange(4097) % 7 + 1).astype(np.int32)
    s, n = int(h.sum()), h.size
    assert orc.transform_reduce(h, "sum")[0] == s and orc.transform_reduce(h, "max")[0] == 7
    assert orc.transform_reduce(h, "sum", "affine", 1, 1)[0] == s + n
    assert orc.transform_reduce(h, "sum", "affine", 1, 7)[0] == s + 7 * n
    assert orc.transform_reduce(h, "sum", "affine", 2, 0)[0] == 2 * s
    assert orc.transform_reduce(h, "sum", "square")[0] == int((h.astype(np.int64) ** 2).sum())
    assert orc.transform_reduce(h, "sum", "identity", 5, 5)[0] == s  # scale / shift unused
    for op in ("sum", "min", "max"):
        assert orc.transform_reduce(np.zeros(0, np.int32), op, "square", init=-9)[0] == -9  # empty: init


def _numpy_transform(x, transform, scale, shift):
    """The transform in the item type, wrapping integers through the unsigned type of the same width."""
    if transform == "identity":
        return x
    if x.dtype.kind == "f":
        with np.errstate(over="ignore", invalid="ignore"):
            return {"affine": lambda: (x * x.dtype.type(scale)) + x.dtype.type(shift), "square": lambda: x * x,
                    "abs": lambda: np.abs(x)}[transform]()
    u = x.view(f"u{x.itemsize}")
    with np.errstate(over="ignore"):
        if transform == "affine":
            r = u * u.dtype.type(np.array(scale).astype(x.dtype).view(u.dtype)) + \
                u.dtype.type(np.array(shift).astype(x.dtype).view(u.dtype))
        elif transform == "square":
            r = u * u
        else:
            r = np.where(x < 0, u.dtype.type(0) - u, u) if x.dtype.kind == "i" else u
    return r.astype(u.dtype).view(x.dtype)


@pytest.mark.parametrize("dtype", [np.int32, np.uint32, np.float32, np.int64, np.uint64, np.float64])
def test_transform_reduce_vs_numpy(orc, dtype):
    """Every operator and transform against an independent numpy formulation: integer sums wrap (uint64
    numpy sums), min / max are numpy's fmin / fmax (NaN skipped) or minimum / maximum reductions with the
    initial value as the left operand, float sums within the long double's bound of math.fsum."""
    rng = np.random.default_rng(np.dtype(dtype).itemsize * 7 + np.dtype(dtype).kind.encode()[0])
    n = 5003
    if np.dtype(dtype).kind == "f":
        x = (rng.standard_normal(n) * 100).astype(dtype)
        x[rng.random(n) < 0.01] = np.nan
        params = [(dtype(1.5), dtype(-0.25), dtype(3.0))]
    else:
        info = np.iinfo(dtype)
        x = rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)
        params = [(3, 11, 7), (-5 if info.min < 0 else 2**31 + 3, 0, info.max)]
    for transform in ("identity", "affine", "square", "abs"):
        for scale, shift, init in params:
            y = _numpy_transform(x, transform, scale, shift)
            for op in ("sum", "min", "max"):
                got, exact, absum = orc.transform_reduce(x, op, transform, scale, shift, init)
                if op == "sum" and y.dtype.kind == "f":
                    if np.isnan(y).any():
                        assert np.isnan(exact)
                        continue
                    assert abs(exact - math.fsum([float(init)] + y.astype(np.float64).tolist())) <= 1e-15 * absum
                    assert math.isclose(absum, math.fsum([abs(float(init))] + np.abs(y.astype(np.float64)).tolist()),
                                        rel_tol=1e-15)
                elif op == "sum":
                    w = (int(init) + int(y.astype(object).sum())) % (1 << (8 * y.itemsize))
                    assert int(np.array(got).astype(y.dtype).view(f"u{y.itemsize}")) == w
                else:
                    red = (np.fmin if op == "min" else np.fmax) if y.dtype.kind == "f" else \
                          (np.minimum if op == "min" else np.maximum)
                    agg = red.reduce(y)
                    want = red(dtype(init), agg) if not np.isnan(agg) else dtype(init)
                    assert got == want or (np.isnan(got) and np.isnan(want)), (op, transform)


def test_transform_reduce_float_edges(orc):
    """Min / max: NaN items are skipped, an all-NaN input gives init, the initial value is the left
    operand (of +0.0 and -0.0, which compare equal, init is kept), and an initial NaN yields the aggregate."""
    z = np.array([-0.0, -0.0, -0.0], np.float32)
    assert not np.signbit(orc.transform_reduce(z, "min", init=0.0)[0])
    assert np.signbit(orc.transform_reduce(-z, "max", init=-0.0)[0])
    nan = np.full(4, np.nan, np.float32)
    assert orc.transform_reduce(nan, "min", init=2.5)[0] == np.float32(2.5)
    v = np.array([3.0, np.nan, -7.0, 1.0], np.float64)
    assert orc.transform_reduce(v, "min", init=np.nan)[0] == -7.0
    assert orc.transform_reduce(v, "max", "square", init=0.0)[0] == 49.0
    assert orc.transform_reduce(v, "max", "abs", init=-1.0)[0] == 7.0


# ---- scan ----------------------------------------------------------------------------------------
@pytest.mark.parametrize("i", [0, 1, 5, 12, 17])
def test_scan_ones_known_answer(orc, i):
    # tests/device_scan_test.cpp:80-127: exclusive sum of 2^i ones is iota, inclusive is iota+1.
    n = 1 << i
    ones = np.ones(n, np.uint32)
    assert np.array_equal(orc.scan_sum_u32(ones), np.arange(n, dtype=np.uint32))
    assert np.array_equal(orc.scan_sum_u32(ones, inclusive=True), np.arange(1, n + 1, dtype=np.uint32))


def test_scan_sum_f32_exact_fractions(orc):
    """oracle_scan_sum_f32 (double accumulation of float items).  Ones give iota; the reference's exact
    binary fractions (i % 7 + 1) * 0.25 over 262,147 items (tests/scan_optimization_regression_test.cpp:49-61,
    116-193) sum exactly, so each output is 0.25 * the int64 prefix sum plus init; inclusive outputs are the
    exclusive ones shifted by one item; the running magnitudes start at |init| and add |x|."""
    n = 262147
    ones = np.ones(n, np.float32)
    assert np.array_equal(orc.scan_sum_f32(ones)[0], np.arange(n, dtype=np.float64))
    assert np.array_equal(orc.scan_sum_f32(ones, inclusive=True)[0], np.arange(1, n + 1, dtype=np.float64))
    q = np.arange(n) % 7 + 1
    sign = np.where(np.arange(n) % 3 == 1, -1, 1)
    a = (sign * q * 0.25).astype(np.float32)
    c = np.cumsum(sign * q)
    cabs = np.cumsum(q)
    for init in (0.0, 3.0, -2.0):
        ex, exa = orc.scan_sum_f32(a, init=init)
        assert np.array_equal(ex, np.r_[0, c[:-1]] * 0.25 + init)
        assert np.array_equal(exa, np.r_[0, cabs[:-1]] * 0.25 + abs(init))
        inc, inca = orc.scan_sum_f32(a, inclusive=True, init=init)
        assert np.array_equal(inc, c * 0.25 + init)
        assert np.array_equal(inca, cabs * 0.25 + abs(init))
    assert orc.scan_sum_f32(np.zeros(0, np.float32))[0].size == 0


def test_scan_left_projection(orc):
    """oracle_scan_left against the reference's cases (ExclusiveScan with lhs and init 42 over 3,841 sevens
    gives 42 everywhere, tests/device_scan_test.cpp:129-155; InclusiveScan with lhs gives in[0] everywhere,
    tests/scan_optimization_regression_test.cpp:195-205) and itertools.accumulate with the same lambda over
    the items' bits (NaN payloads, -0.0 and all-ones words included)."""
    import itertools
    assert orc.scan_left(np.full(3841, 7, np.int32), inclusive=False, init=42).tolist() == [42] * 3841
    h = ((np.arange(16003) % 7 + 1) * 0.25).astype(np.float32)
    assert np.array_equal(orc.scan_left(h), np.full(16003, h[0], np.float32))
    rng = np.random.default_rng(4)
    for dt in (np.uint32, np.uint64):
        bits = rng.integers(0, np.iinfo(dt).max, 500, dtype=dt, endpoint=True)
        bits[[0, 7, 9]] = np.iinfo(dt).max  # all-ones words are ordinary items
        left = lambda a, b: a
        for start in (bits, bits[1:]):
            assert orc.scan_left(start).tolist() == list(itertools.accumulate(start.tolist(), left))
            for init in (0, 5, int(np.iinfo(dt).max)):
                acc = list(itertools.accumulate([init] + start.tolist(), left))
                assert orc.scan_left(start, inclusive=True, init=dt(init)).tolist() == acc[1:]
                assert orc.scan_left(start, inclusive=False, init=dt(init)).tolist() == acc[:-1]
    f = np.array([np.nan, -0.0, 1.0], np.float64)
    assert np.array_equal(orc.scan_left(f).view(np.uint64), np.full(3, f.view(np.uint64)[0]))
    with pytest.raises(ValueError):
        orc.scan_left(np.ones(3, np.int32), inclusive=False)


def test_scan_inclusive_init_known_answer(orc):
    # tests/device_scan_test.cpp:288-321: InclusiveScanInit {1,2,3,4} + 10 -> {11,13,16,20}.
    a = np.array([1, 2, 3, 4], np.int32)
    assert orc.scan_sum_u32(a, inclusive=True, init=10).tolist() == [11, 13, 16, 20]


def test_scan_matches_cumsum_with_wrap(orc):
    # (i % 7) - 3 data of tests/device_scan_test.cpp:189-265 and tests/lcpp_cub_bench.cpp:666-672.
    n = 100003
    a = ((np.arange(n) % 7) - 3).astype(np.int32)
    ref = np.concatenate([[0], np.cumsum(a.astype(np.int64))[:-1]])
    assert np.array_equal(orc.scan_sum_u32(a).astype(np.int64), ref)
    big = np.full(10, 2**31, np.uint32)
    got = orc.scan_sum_u32(big, inclusive=True)
    assert got.tolist() == [(2**31 * (i + 1)) % 2**32 for i in range(10)]


# ---- radix sort ----------------------------------------------------------------------------------
def _stable_order(keys, keyfunc):
    return sorted(range(len(keys)), key=lambda i: keyfunc(keys[i]))


def test_radix_partial_bits_known_answer(orc):
    # tests/device_radix_sort_interface_test.cpp:68-159: 257 items, bits [1, 6), asc/desc, pairs.
    n, b, e = 257, 1, 6
    keys = np.array([((i * 53) % 64) | (((i * 17) % 11) << 8) for i in range(n)], np.uint32)
    vals = np.arange(n, dtype=np.uint32)
    sel = lambda k: (int(k) >> b) & ((1 << (e - b)) - 1)
    asc = _stable_order(keys, sel)
    desc = _stable_order(keys, lambda k: -sel(k))
    assert np.array_equal(orc.radix_sort(keys, begin_bit=b, end_bit=e), keys[asc])
    assert np.array_equal(orc.radix_sort(keys, begin_bit=b, end_bit=e, descending=True), keys[desc])
    ko, vo = orc.radix_sort(keys, vals, begin_bit=b, end_bit=e)
    assert np.array_equal(ko, keys[asc]) and np.array_equal(vo, vals[asc])
    ko, vo = orc.radix_sort(keys, vals, begin_bit=b, end_bit=e, descending=True)
    assert np.array_equal(ko, keys[desc]) and np.array_equal(vo, vals[desc])


def test_radix_double_buffer_case_known_answer(orc):
    # tests/device_radix_sort_interface_test.cpp:205-283: 65 items, bits [0, 5).
    n = 65
    keys = np.array([((i * 19) % 32) | ((i % 7) << 8) for i in range(n)], np.uint32)
    asc = _stable_order(keys, lambda k: int(k) & 31)
    assert np.array_equal(orc.radix_sort(keys, begin_bit=0, end_bit=5), keys[asc])


def test_radix_u64_reversed_known_answer(orc):
    # tests/device_radix_sort_one_sweep.cpp:175-205: 65,536 u64 keys (n-i-1)*2654435761.
    n = 65536
    keys = ((n - np.arange(n, dtype=np.uint64) - 1) * np.uint64(2654435761)).astype(np.uint64)
    assert np.array_equal(orc.radix_sort(keys), np.sort(keys))


@pytest.mark.parametrize("dtype", [np.uint32, np.int32, np.uint64, np.int64])
@pytest.mark.parametrize("descending", [False, True])
def test_radix_integer_keys_vs_numpy_stable(orc, dtype, descending):
    rng = np.random.default_rng(5)
    n = 20000
    info = np.iinfo(dtype)
    keys = rng.integers(info.min, info.max, size=n, dtype=dtype, endpoint=True)
    keys[::7] = keys[3]  # many duplicates for the stability check
    vals = np.arange(n, dtype=np.uint32)
    if descending:
        order = sorted(range(n), key=lambda i: -int(keys[i]))
    else:
        order = np.argsort(keys, kind="stable")
    ko, vo = orc.radix_sort(keys, vals, descending=descending)
    assert np.array_equal(ko, keys[order])
    assert np.array_equal(vo, vals[order])


def test_radix_float_keys_total_order(orc):
    # Float twiddle (common/util_type.h:141-175): -NaN < -inf < ... < -0.0 == +0.0 < ... < +inf < +NaN,
    # with -0.0 and +0.0 ranked as equal keys (agent/radix_rank_sort_operations.h:31-42), so they
    # keep their input order.
    neg_nan = struct.unpack("<f", struct.pack("<I", 0xFFC00000))[0]
    pos_nan = struct.unpack("<f", struct.pack("<I", 0x7FC00000))[0]
    keys = np.array([1.5, -0.0, 0.0, -2.0, float("inf"), pos_nan, -0.0, float("-inf"), neg_nan, 0.0, -1e-30],
                    np.float32)
    bits = keys.view(np.uint32)
    vals = np.arange(keys.size, dtype=np.uint32)
    ko, vo = orc.radix_sort(keys, vals)
    assert vo.tolist() == [8, 7, 3, 10, 1, 2, 6, 9, 0, 4, 5]
    assert np.array_equal(ko.view(np.uint32), bits[vo])
    ko, vo = orc.radix_sort(keys, vals, descending=True)
    assert vo.tolist() == [5, 4, 0, 1, 2, 6, 9, 10, 3, 7, 8]


def test_radix_float_keys_vs_python_sort(orc):
    rng = np.random.default_rng(9)
    keys = rng.standard_normal(5000).astype(np.float32)
    keys[::5] = 0.0
    keys[1::11] = -0.0
    vals = np.arange(keys.size, dtype=np.uint32)
    for desc in (False, True):
        order = sorted(range(keys.size), key=lambda i: (-1 if desc else 1) * float(keys[i]))
        ko, vo = orc.radix_sort(keys, vals, descending=desc)
        assert vo.tolist() == order
        kd = rng.standard_normal(3000)
        od = sorted(range(kd.size), key=lambda i: (-1 if desc else 1) * float(kd[i]))
        assert np.array_equal(orc.radix_sort(kd, descending=desc), kd[od])


def test_radix_brute_force_tiny(orc):
    rng = np.random.default_rng(11)
    for n in range(0, 40):
        keys = rng.integers(0, 4, size=n).astype(np.uint32)
        vals = np.arange(n, dtype=np.uint32)
        ko, vo = orc.radix_sort(keys, vals)
        # brute force: rank of i = #{j: k_j < k_i} + #{j < i: k_j == k_i}
        exp = np.empty(n, np.uint32)
        for i in range(n):
            r = int(np.sum(keys < keys[i]) + np.sum(keys[:i] == keys[i]))
            exp[r] = i
        assert np.array_equal(vo, exp)


def test_radix_digit_known_values(orc):
    # signed: 0x80000000 (INT_MIN) is the smallest ordered key; descending inverts.
    assert orc.radix_digit(0x80000000, np.int32, False, 24, 8) == 0x00
    assert orc.radix_digit(0x7FFFFFFF, np.int32, False, 24, 8) == 0xFF
    assert orc.radix_digit(0x80000000, np.int32, True, 24, 8) == 0xFF
    # float -0.0 digits equal +0.0 digits in both directions
    for d in (False, True):
        for s in (0, 8, 16, 24):
            assert orc.radix_digit(0x80000000, np.float32, d, s, 8) == orc.radix_digit(0, np.float32, d, s, 8)


# ---- spmv ----------------------------------------------------------------------------------------
def reference_int_csr():
    """tests/device_spmv_test.cpp:41-108 (8x13 int CSR with row lengths {0,1,5,33,2,64,0,7})."""
    rows, cols = 8, 13
    lengths = [0, 1, 5, 33, 2, 64, 0, 7]
    ro = np.zeros(rows + 1, np.int32)
    for r in range(rows):
        ro[r + 1] = ro[r] + lengths[r]
    nnz = int(ro[-1])
    ci = np.zeros(nnz, np.int32)
    va = np.zeros(nnz, np.int32)
    for r in range(rows):
        for it in range(lengths[r]):
            idx = ro[r] + it
            ci[idx] = (r * 5 + it * 7) % cols
            va[idx] = ((r + it * 3) % 9) - 4
    x = np.arange(cols, dtype=np.int32) - 6
    return va, ro, ci, x, rows, cols, nnz


def test_spmv_int_known_answer(orc):
    va, ro, ci, x, rows, cols, nnz = reference_int_csr()
    expected = [sum(int(va[i]) * int(x[ci[i]]) for i in range(ro[r], ro[r + 1])) for r in range(rows)]
    got = orc.spmv_csr_u32(va, ro, ci, x, rows, cols, nnz).view(np.int32)
    assert got.tolist() == expected
    # dense cross-check
    dense = np.zeros((rows, cols), np.int64)
    for r in range(rows):
        for i in range(ro[r], ro[r + 1]):
            dense[r, ci[i]] += va[i]
    assert (dense @ x.astype(np.int64)).tolist() == expected


def test_spmv_float_known_answer(orc):
    # tests/device_spmv_test.cpp:110-155.
    ro = np.array([0, 3, 3, 6, 8], np.uint32)
    ci = np.array([0, 2, 4, 1, 2, 3, 0, 4], np.uint32)
    va = np.array([1.5, -2.0, 0.25, 3.0, 1.25, -0.5, 2.0, 4.0], np.float32)
    x = np.array([2.0, -1.0, 0.5, 3.0, -2.0], np.float32)
    y, ay = orc.spmv_csr_fp(va, ro, ci, x, 4, 5, 8)
    assert y.tolist() == [1.5 * 2 - 2.0 * 0.5 + 0.25 * -2, 0.0, -3.0 + 0.625 - 1.5, 4.0 - 8.0]
    assert ay[0] == 3.0 + 1.0 + 0.5


def test_spmv_invalid_rows_and_columns(orc):
    # device_spmv.h:97-108: decreasing offsets or offsets past nnz -> 0; columns >= cols skipped.
    ro = np.array([0, 2, 1, 4, 9], np.uint32)
    ci = np.array([0, 5, 1, 2], np.uint32)
    va = np.array([1, 2, 3, 4], np.uint32)
    x = np.array([10, 20, 30], np.uint32)
    y = orc.spmv_csr_u32(va, ro, ci, x, 4, 3, 4)
    assert y.tolist() == [10, 0, 3 * 20 + 4 * 30, 0]
    zero = orc.spmv_csr_u32(va, np.zeros(5, np.uint32), ci, x, 4, 3, 0)
    assert zero.tolist() == [0, 0, 0, 0]


def test_spmv_f64_vs_fsum_row_loop(orc):
    """The double branch of oracle_spmv_csr_fp.  The reference's 4x5 case (tests/device_spmv_test.cpp:110-155)
    with values float32 cannot hold (a float read would be off by ~1e-8), then a random matrix with empty
    rows and out-of-range columns against a math.fsum row loop over the double products."""
    ro = np.array([0, 3, 3, 6, 8], np.uint32)
    ci = np.array([0, 2, 4, 1, 2, 3, 0, 4], np.uint32)
    va = np.array([1.1, -2.0, 0.3, 3.0, 1.7, -0.5, 2.0, 4.0], np.float64)
    x = np.array([2.0, -1.0, 0.1, 3.0, -2.0], np.float64)
    y, ay = orc.spmv_csr_fp(va, ro, ci, x, 4, 5, 8)
    want = [math.fsum([1.1 * 2.0, -2.0 * 0.1, 0.3 * -2.0]), 0.0, math.fsum([-3.0, 1.7 * 0.1, -1.5]), 4.0 - 8.0]
    assert np.all(np.abs(y - want) <= 1e-15 * ay)
    assert ay[1] == 0.0 and ay[3] == 12.0
    rng = np.random.default_rng(13)
    rows, cols = 3000, 2500
    lengths = rng.integers(0, 60, rows)
    lengths[::41] = 0
    ro = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint32)
    nnz = int(ro[-1])
    ci = rng.integers(0, cols + 20, nnz).astype(np.uint32)  # some columns out of range: skipped
    va = rng.standard_normal(nnz)
    x = rng.standard_normal(cols)
    y, ay = orc.spmv_csr_fp(va, ro, ci, x, rows, cols, nnz)
    for r in range(rows):
        terms = [va[j] * x[ci[j]] for j in range(ro[r], ro[r + 1]) if ci[j] < cols]
        assert abs(y[r] - math.fsum(terms)) <= 1e-15 * ay[r] + 1e-300, r
        assert math.isclose(ay[r], math.fsum(np.abs(terms)), rel_tol=1e-15, abs_tol=1e-300), r


def test_twiddle_in_known_values_and_order(orc):
    """oracle_twiddle_in (common/util_type.h:97-175): unsigned keys keep their bits, signed keys flip the
    high bit, floats flip the high bit when positive and every bit when negative, descending inverts the
    image.  The unsigned order of the images is the keys' numeric order."""
    assert orc.twiddle_in(0x12345678, np.uint32) == 0x12345678
    assert orc.twiddle_in(0x12345678, np.uint32, True) == 0xEDCBA987
    assert orc.twiddle_in(0x80000000, np.int32) == 0 and orc.twiddle_in(0xFFFFFFFF, np.int32) == 0x7FFFFFFF
    assert orc.twiddle_in(0x3F800000, np.float32) == 0xBF800000  # +1.0
    assert orc.twiddle_in(0xBF800000, np.float32) == 0x407FFFFF  # -1.0
    assert orc.twiddle_in(1 << 63, np.int64) == 0
    assert orc.twiddle_in(1 << 63, np.float64) == (1 << 63) - 1  # -0.0 sits just below +0.0's 1 << 63
    assert orc.twiddle_in(0, np.float64, True) == (1 << 63) - 1
    rng = np.random.default_rng(17)
    f = (rng.standard_normal(3000) * 10.0 ** rng.integers(-30, 30, 3000)).astype(np.float32)
    f[:4] = [np.inf, -np.inf, 0.0, 3.0e38]
    img = np.array([orc.twiddle_in(int(b), np.float32) for b in f.view(np.uint32)], np.uint64)
    assert np.all(np.diff(f[np.argsort(img, kind="stable")]) >= 0)
    s = rng.integers(-2**63, 2**63 - 1, 3000, dtype=np.int64)
    img = np.array([orc.twiddle_in(int(b), np.int64) for b in s.view(np.uint64)], np.uint64)
    assert np.array_equal(np.argsort(img, kind="stable"), np.argsort(s, kind="stable"))
    imgd = np.array([orc.twiddle_in(int(b), np.int64, True) for b in s.view(np.uint64)], np.uint64)
    assert np.array_equal(imgd, ~img)


def test_scan_u64_ones_and_wrap(orc):
    # Exclusive sums of ones are iota; full-range 64-bit words wrap like numpy's uint64 cumsum.
    ones = np.ones(1000, np.uint64)
    assert np.array_equal(orc.scan_sum_u64(ones), np.arange(1000, dtype=np.uint64))
    rng = np.random.default_rng(9)
    a = rng.integers(0, 2**64 - 1, 5000, dtype=np.uint64, endpoint=True)
    with np.errstate(over="ignore"):
        ref = np.cumsum(a, dtype=np.uint64)
    assert np.array_equal(orc.scan_sum_u64(a, inclusive=True), ref)
    assert np.array_equal(orc.scan_sum_u64(a)[1:], ref[:-1])
    assert orc.scan_sum_u64(a)[0] == 0
    # init: every output shifts by init (mod 2^64); int64 through the same bits.
    assert np.array_equal(orc.scan_sum_u64(a, inclusive=True, init=7), ref + np.uint64(7))
    s = a.view(np.int64)
    assert np.array_equal(orc.scan_sum_u64(s, inclusive=True).view(np.uint64), ref)


def test_scan_f64_known_answer_and_exactness(orc):
    # tests/device_scan_test.cpp:267-286: InclusiveSum<double> of 17 ones is 1..17.
    out, _ = orc.scan_sum_f64(np.ones(17), inclusive=True)
    assert [float(x) for x in out] == [float(i + 1) for i in range(17)]
    # Integer-valued doubles below 2^53 sum exactly in any order: the long-double scan equals int64 cumsum.
    rng = np.random.default_rng(3)
    a = rng.integers(-1000, 1000, 100000)
    out, absum = orc.scan_sum_f64(a.astype(np.float64))
    assert np.array_equal(out.astype(np.int64)[1:], np.cumsum(a)[:-1])
    assert np.array_equal(absum.astype(np.int64)[1:], np.cumsum(np.abs(a))[:-1])


# ---- min / max scans ----------------------------------------------------------------------------
def test_scan_max_exclusive_known_answer(orc):
    """tests/pr6_review_regression_test.cpp:146-151,247-265: ExclusiveScan with max and init 0 over
    host[i] = i % 7 + 1 (4,097 items) gives the running maximum before i: min(i, 7)."""
    n = 4097
    a = (np.arange(n) % 7 + 1).astype(np.int32)
    assert np.array_equal(orc.scan_minmax("max", a, init=0), np.minimum(np.arange(n), 7).astype(np.int32))


def _accumulate(ufunc, a, inclusive, init):
    """Running min / max by numpy's ufunc.accumulate, with `init` put in front of the items."""
    if init is None:
        if inclusive:
            return ufunc.accumulate(a)
        init = np.nan if a.dtype.kind == "f" else (np.iinfo(a.dtype).max if ufunc in (np.minimum, np.fmin)
                                                     else np.iinfo(a.dtype).min)
    run = ufunc.accumulate(np.concatenate([np.array([init], a.dtype), a]))
    return run[1:] if inclusive else run[:-1]


@pytest.mark.parametrize("dtype", [np.int32, np.uint32, np.int64, np.uint64, np.float32, np.float64])
@pytest.mark.parametrize("op", ["min", "max"])
def test_scan_minmax_vs_numpy_accumulate(orc, dtype, op):
    """Integers against np.minimum / np.maximum.accumulate; floats (with NaNs, no signed zeros) against
    np.fmin / np.fmax.accumulate, which ignore a NaN operand as the operators do."""
    rng = np.random.default_rng(17)
    n = 20000
    if np.dtype(dtype).kind == "f":
        a = rng.standard_normal(n).astype(dtype) * 1000
        a[a == 0] = 1
        a[rng.random(n) < 0.05] = np.nan
        a[:3] = np.nan  # an all-NaN prefix stays NaN
        ufunc = np.fmin if op == "min" else np.fmax
        inits = [None, 1.5, np.nan]
    else:
        info = np.iinfo(dtype)
        a = rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)
        ufunc = np.minimum if op == "min" else np.maximum
        inits = [None, 0, info.max, info.min]
    for inclusive in (False, True):
        for init in inits:
            got = orc.scan_minmax(op, a, inclusive=inclusive, init=init)
            ref = _accumulate(ufunc, a, inclusive, init)
            assert np.array_equal(got, ref, equal_nan=np.dtype(dtype).kind == "f"), (inclusive, init)


def test_scan_minmax_signed_zero_keeps_earlier(orc):
    """-0.0 and +0.0 compare equal, so the running value keeps the earlier of the two (sign bit checked)."""
    a = np.array([0.0, -0.0, -0.0, 0.0], np.float32)
    for op in ("min", "max"):
        assert np.signbit(orc.scan_minmax(op, a, inclusive=True)).tolist() == [False] * 4
        assert np.signbit(orc.scan_minmax(op, -a, inclusive=True)).tolist() == [True] * 4
    assert np.signbit(orc.scan_minmax("min", a, init=-0.0)).tolist() == [True] * 4


@pytest.mark.parametrize("kdt", [np.int32, np.uint64])
@pytest.mark.parametrize("vdt", [np.int32, np.uint32, np.int64, np.uint64, np.float32, np.float64])
def test_minmax_by_key_vs_numpy(orc, kdt, vdt):
    """Per run (split at the heads): np.minimum / maximum.accumulate (integers), np.fmin / fmax.accumulate
    (floats with NaNs) for the scans, with the initial value put in front; reduceat for the reduce.  Every
    value type is covered, since each has its own identity (the type's max / lowest, NaN for floats) that
    opens a run without init.  The 8-byte keys differ only above bit 32, so reading them as 4-byte words
    would merge every run."""
    rng = np.random.default_rng(8)
    n = 3000
    ids = np.repeat(np.arange(400), rng.integers(1, 14, 400))[:n]
    keys = ids.astype(np.int32) if kdt is np.int32 else (ids.astype(np.uint64) << np.uint64(33)) | np.uint64(5)
    n = keys.size
    if np.dtype(vdt).kind == "f":
        vals = rng.integers(-50, 50, n).astype(vdt)
        vals[rng.random(n) < 0.05] = np.nan
        fmin, fmax, ident = np.fmin, np.fmax, (np.nan, np.nan)
    else:
        info = np.iinfo(vdt)
        vals = rng.integers(info.min, info.max, n, dtype=vdt, endpoint=True)
        fmin, fmax, ident = np.minimum, np.maximum, (info.max, info.min)
    heads = np.flatnonzero(np.r_[True, keys[1:] != keys[:-1]])
    for op, uf, idv in (("min", fmin, ident[0]), ("max", fmax, ident[1])):
        for inclusive in (False, True):
            for init in (None, vdt(5)):
                want = np.empty_like(vals)
                start = idv if init is None else init
                for a, b in zip(heads, np.r_[heads[1:], n]):
                    run = uf.accumulate(np.r_[np.array([start], vals.dtype), vals[a:b]])
                    want[a:b] = run[1:] if inclusive else run[:-1]
                got = orc.scan_by_key_minmax(op, keys, vals, inclusive, init)
                assert np.array_equal(got, want, equal_nan=np.dtype(vdt).kind == "f"), (op, inclusive, init)
        u, agg = orc.reduce_by_key_minmax(op, keys, vals)
        assert np.array_equal(u, keys[heads])
        assert np.array_equal(agg, uf.reduceat(vals, heads), equal_nan=np.dtype(vdt).kind == "f")


# ---- min / max / arg reductions ------------------------------------------------------------------
def test_reduce_min_max_arg_known_answers(orc):
    """tests/device_reduce_test.cpp:218-345: float Max from the lowest identity, ArgMax's first equal
    extremum, ArgMax of negative floats, empty-input sentinels (value max / lowest, index 1)."""
    assert orc.reduce_minmax("max", np.array([-8.0, -2.5, -9.0, -4.0], np.float32)) == np.float32(-2.5)
    assert orc.reduce_arg("max", np.array([1, 9, 4, 9, 3], np.int32)) == (9, 1)
    assert orc.reduce_arg("max", np.array([-7.0, -3.0, -5.0], np.float32)) == (np.float32(-3.0), 1)
    e = np.array([], np.int32)
    assert orc.reduce_arg("min", e) == (np.iinfo(np.int32).max, 1)
    assert orc.reduce_arg("max", e) == (np.iinfo(np.int32).min, 1)
    assert orc.reduce_minmax("min", e) == np.iinfo(np.int32).max


@pytest.mark.parametrize("dtype", [np.int32, np.uint32, np.int64, np.uint64, np.float32, np.float64])
def test_reduce_min_max_arg_vs_numpy(orc, dtype):
    """Integers against np.min / max / argmin / argmax (first occurrence); floats with NaNs against np.nanmin /
    nanmax / nanargmin / nanargmax, which skip NaNs as the operators do."""
    rng = np.random.default_rng(5)
    for n in (1, 2, 100, 20001):
        if np.dtype(dtype).kind == "f":
            a = rng.integers(-40, 40, n).astype(dtype)   # many ties
            a[rng.random(n) < 0.1] = np.nan
            a[0] = 7 if np.isnan(a).all() else a[0]
            fmin, fmax, amin, amax = np.nanmin, np.nanmax, np.nanargmin, np.nanargmax
        else:
            info = np.iinfo(dtype)
            a = rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)
            a[rng.integers(0, n, 3)] = a.max()
            fmin, fmax, amin, amax = np.min, np.max, np.argmin, np.argmax
        assert orc.reduce_minmax("min", a) == fmin(a) and orc.reduce_minmax("max", a) == fmax(a)
        assert orc.reduce_arg("min", a) == (fmin(a), int(amin(a)))
        assert orc.reduce_arg("max", a) == (fmax(a), int(amax(a)))


def test_reduce_arg_float_edges(orc):
    """The fold starts at the type's max / lowest: +inf items leave Min at FLT_MAX; all-NaN gives the initial
    pair with index 0xFFFFFFFF; -0.0 and +0.0 tie, the first wins."""
    f = np.float32
    assert orc.reduce_minmax("min", np.array([np.inf], f)) == np.finfo(f).max
    assert orc.reduce_arg("min", np.full(5, np.nan, f)) == (np.finfo(f).max, 0xFFFFFFFF)
    v, i = orc.reduce_arg("min", np.array([1.0, -0.0, 0.0], f))
    assert i == 1 and np.signbit(v)


# ---- scan-by-key / reduce-by-key ---------------------------------------------------------------

def numpy_by_key(keys, values, key_mask=-1):
    """Independent formulation: head flags, then running totals per run from one cumulative sum
    (modulo 2^64 in uint64).  Returns (heads, inclusive-within-run, per-run sums, run starts)."""
    k = keys.astype(np.uint64) if keys.dtype.kind == "u" else keys.view(f"u{keys.itemsize}").astype(np.uint64)
    m = np.uint64(key_mask & 0xFFFFFFFFFFFFFFFF)
    heads = np.ones(k.size, bool)
    heads[1:] = ((k[1:] ^ k[:-1]) & m) != 0
    v = values.view(f"u{values.itemsize}").astype(np.uint64)
    with np.errstate(over="ignore"):
        cs = np.cumsum(v, dtype=np.uint64)
        starts = np.flatnonzero(heads)
        seg = np.cumsum(heads) - 1
        base = cs[starts] - v[starts]
        incl = cs - base[seg]
        sums = np.add.reduceat(v, starts, dtype=np.uint64) if v.size else np.zeros(0, np.uint64)
    return heads, incl, sums, starts


@pytest.mark.parametrize("log_n", [5, 8, 12, 16])
def test_exclusive_sum_by_key_ones_known_answer(orc, log_n):
    """device_scan_test.cpp:325-385: ones with keys i / 100 give i % 100 (per-segment exclusive sum)."""
    n = 1 << log_n
    keys = (np.arange(n) // 100).astype(np.int32)
    out = orc.scan_by_key_int(keys, np.ones(n, np.int32))
    assert np.array_equal(out, (np.arange(n) % 100).astype(np.int32))


def test_inclusive_sum_by_key_three_tiles_known_answer(orc):
    """device_scan_test.cpp:387-417: int keys 1 | 2 | 3 split at tile + 1 and 2 tile + 1 (tile = 256 x 15),
    int64 ones; the inclusive sums restart at every key change."""
    tile = 256 * 15
    n = 2 * tile + 2
    idx = np.arange(n)
    keys = np.where(idx < tile + 1, 1, np.where(idx < 2 * tile + 1, 2, 3)).astype(np.int32)
    out = orc.scan_by_key_int(keys, np.ones(n, np.int64), inclusive=True)
    expected = np.concatenate([np.arange(1, tile + 2), np.arange(1, tile + 1), np.arange(1, 2)]).astype(np.int64)
    assert np.array_equal(out, expected)


def test_inclusive_sum_by_key_parity_equality_known_answer(orc):
    """device_scan_test.cpp:419-447: equality (lhs & 1) == (rhs & 1) over keys {1,3,5,2,4} gives {1,2,3,1,2}."""
    out = orc.scan_by_key_int(np.array([1, 3, 5, 2, 4], np.int32), np.ones(5, np.int32), inclusive=True, key_mask=1)
    assert out.tolist() == [1, 2, 3, 1, 2]


def test_reduce_by_key_blocks_of_100_known_answer(orc):
    """device_reduce_test.cpp:420-478: 4096 items, keys i / 100, values a permutation of 0..4095: 41 runs,
    unique keys 0..40 and block sums (the reference shuffles with std::shuffle, whose permutation is
    implementation-defined; any permutation exercises the same closed form)."""
    n = 4096
    keys = (np.arange(n) // 100).astype(np.int32)
    vals = np.random.default_rng(114521).permutation(n).astype(np.int32)
    uniq, agg = orc.reduce_by_key_int(keys, vals)
    assert uniq.tolist() == list(range(41))
    expected = [int(vals[i * 100:(i + 1) * 100].sum()) for i in range(41)]
    assert agg.astype(np.int64).tolist() == expected


def test_reduce_by_key_empty_input(orc):
    """device_reduce_test.cpp:480-512: n == 0 gives 0 runs."""
    uniq, agg = orc.reduce_by_key_int(np.zeros(0, np.int32), np.zeros(0, np.int32))
    assert uniq.size == 0 and agg.size == 0


@pytest.mark.parametrize("kdt,vdt,mask", [(np.uint32, np.uint32, -1), (np.int32, np.int64, -1),
                                          (np.uint64, np.uint32, 0xFF00), (np.int64, np.uint64, -1)])
@pytest.mark.parametrize("mode", ["exclusive", "inclusive", "inclusive_init"])
def test_scan_by_key_vs_numpy(orc, kdt, vdt, mask, mode):
    rng = np.random.default_rng(5)
    n = 20000
    runs = np.repeat(rng.integers(0, 1 << 20, 6000), rng.integers(1, 12, 6000))[:n]
    assert runs.size == n
    keys = runs.astype(kdt)
    vals = rng.integers(0, np.iinfo(vdt).max, n, dtype=vdt, endpoint=True)
    init = 0x9E3779B9 if mode != "inclusive" else 0
    heads, incl, _, _ = numpy_by_key(keys, vals, mask)
    vmask = np.uint64((1 << (8 * vals.itemsize)) - 1)
    v = vals.view(f"u{vals.itemsize}").astype(np.uint64)
    with np.errstate(over="ignore"):
        if mode == "exclusive":
            want = np.where(heads, np.uint64(init), np.uint64(init) + incl - v)
        elif mode == "inclusive":
            want = incl
        else:
            want = np.uint64(init) + incl
    want = (want & vmask).astype(f"u{vals.itemsize}").view(vdt)
    got = orc.scan_by_key_int(keys, vals, inclusive=mode != "exclusive", use_init=mode == "inclusive_init",
                              init=init, key_mask=mask)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("kdt,vdt,mask", [(np.int32, np.int32, -1), (np.uint64, np.uint64, -1), (np.uint32, np.int64, 3)])
def test_reduce_by_key_vs_numpy(orc, kdt, vdt, mask):
    rng = np.random.default_rng(9)
    n = 30000
    keys = np.repeat(rng.integers(0, 50, 12000), rng.integers(1, 9, 12000))[:n].astype(kdt)
    assert keys.size == n
    vals = rng.integers(np.iinfo(vdt).min, np.iinfo(vdt).max, n, dtype=vdt, endpoint=True)
    heads, _, sums, starts = numpy_by_key(keys, vals, mask)
    vmask = np.uint64((1 << (8 * vals.itemsize)) - 1)
    uniq, agg = orc.reduce_by_key_int(keys, vals, key_mask=mask)
    assert np.array_equal(uniq, keys[starts])
    assert np.array_equal(agg, (sums & vmask).astype(f"u{vals.itemsize}").view(vdt))


def test_by_key_float_paths_match_exact_sums(orc):
    """Float values: every output equals the exactly rounded (math.fsum) sum of its run prefix."""
    rng = np.random.default_rng(13)
    keys = np.repeat(np.arange(40), rng.integers(1, 30, 40)).astype(np.int32)
    vals = rng.uniform(-1e3, 1e3, keys.size).astype(np.float32)
    heads, _, _, starts = numpy_by_key(keys, vals)
    incl, _ = orc.scan_by_key_fp(keys, vals, inclusive=True)
    excl, _ = orc.scan_by_key_fp(keys, vals, inclusive=False, init=2.5)
    uniq, agg, _ = orc.reduce_by_key_fp(keys, vals)
    seg_start = np.maximum.accumulate(np.where(heads, np.arange(keys.size), 0))
    for i in range(keys.size):
        part = [float(x) for x in vals[seg_start[i]:i + 1]]
        assert incl[i] == pytest.approx(math.fsum(part), rel=1e-15, abs=1e-12)
        assert excl[i] == pytest.approx(2.5 + math.fsum(part[:-1]), rel=1e-15, abs=1e-12)
    ends = np.r_[starts[1:], keys.size]
    assert np.array_equal(uniq, keys[starts])
    for r, (b, e) in enumerate(zip(starts, ends)):
        assert agg[r] == pytest.approx(math.fsum(float(x) for x in vals[b:e]), rel=1e-15, abs=1e-12)


# ---- stream compaction --------------------------------------------------------------------------
# Known answers from the reference's tests, then an independent pure-Python formulation on small
# random inputs (list comprehensions and explicit C remainders, sharing nothing with oracle.c).

def test_run_length_encode_cub_example_known_answer(orc):
    """tests/device_run_length_encode_test.cpp:172-245 (CUB's documented example)."""
    x = np.array([0, 2, 2, 9, 5, 5, 5, 8], np.int32)
    u, c = orc.run_length_encode(x)
    assert u.tolist() == [0, 2, 9, 5, 8] and c.tolist() == [1, 2, 1, 3, 1]
    o, ln = orc.non_trivial_runs(x)
    assert o.tolist() == [1, 4] and ln.tolist() == [2, 3]


def test_run_length_encode_wide_values_known_answer(orc):
    """tests/device_run_length_encode_test.cpp:41-72: 64-bit values 2^40, 2^40, 2^41, 2^42 x3, 2^43."""
    x = np.array([1 << 40, 1 << 40, 1 << 41, 1 << 42, 1 << 42, 1 << 42, 1 << 43], np.uint64)
    u, c = orc.run_length_encode(x)
    assert u.tolist() == [1 << 40, 1 << 41, 1 << 42, 1 << 43] and c.tolist() == [2, 1, 3, 1]


def test_run_length_encode_host_reference_runs(orc):
    """tests/device_run_length_encode_test.cpp:282-340: 180 runs of length run % 7 + 1."""
    x = np.concatenate([np.full(r % 7 + 1, r, np.int32) for r in range(180)])
    u, c = orc.run_length_encode(x)
    assert u.tolist() == list(range(180)) and c.tolist() == [r % 7 + 1 for r in range(180)]
    o, ln = orc.non_trivial_runs(x)
    starts = np.cumsum([0] + [r % 7 + 1 for r in range(179)])
    want = [(int(starts[r]), r % 7 + 1) for r in range(180) if r % 7 + 1 > 1]
    assert list(zip(o.tolist(), ln.tolist())) == want


def test_partition_three_way_known_answer(orc):
    """tests/device_partition_test.cpp:292-349: 0..11, first = x % 3 == 0, second = x < 8."""
    x = np.arange(12, dtype=np.int32)
    f = orc.predicate(x, [(10, 3, 0)])
    s = orc.predicate(x, [(1, 8, 0)])
    o1, o2, o3, (c1, c2) = orc.partition_three_way(x, f, s)
    assert (c1, c2) == (4, 5)
    assert o1[:4].tolist() == [0, 3, 6, 9] and o2[:5].tolist() == [1, 2, 4, 5, 7] and o3[:3].tolist() == [11, 10, 8]


def test_partition_flagged_and_if_ordering_known_answer(orc):
    """tests/device_partition_test.cpp:103-177: flags i % 3 == 0 and x < 7 over 0..11."""
    x = np.arange(12, dtype=np.int32)
    out, k = orc.select(x, (np.arange(12) % 3 == 0).astype(np.uint8), partition=True)
    assert k == 4 and out.tolist() == [0, 3, 6, 9, 11, 10, 8, 7, 5, 4, 2, 1]
    out, k = orc.select(x, orc.predicate(x, [(1, 7, 0)]), partition=True)
    assert k == 7 and out.tolist() == [0, 1, 2, 3, 4, 5, 6, 11, 10, 9, 8, 7]


def test_select_unique_and_unique_by_key_known_answer(orc):
    """tests/device_select_test.cpp:301-357: keys {1,1,2,2,2,4,7,7,9}."""
    keys = np.array([1, 1, 2, 2, 2, 4, 7, 7, 9], np.int32)
    vals = np.array([10, 11, 20, 21, 22, 40, 70, 71, 90], np.int32)
    heads = orc.run_heads(keys)
    uk, k = orc.select(keys, heads)
    uv, kv = orc.select(vals, heads)
    assert k == kv == 5 and uk[:5].tolist() == [1, 2, 4, 7, 9] and uv[:5].tolist() == [10, 20, 40, 70, 90]


def test_select_flagged_if_positive_odd_known_answer(orc):
    """tests/device_select_test.cpp:359-425: flags -3..5, flag > 0 and flag % 2 != 0 -> 104, 106, 108."""
    data = np.arange(100, 109, dtype=np.int32)
    flags = np.arange(-3, 6, dtype=np.int32)
    sel = orc.predicate(flags, [(3, 0, 0), (11, 2, 0)])
    out, k = orc.select(data, sel)
    assert k == 3 and out[:3].tolist() == [104, 106, 108]


def test_select_in_place_cases_known_answer(orc):
    """tests/device_select_test.cpp:427-500: aliased flags, x > 0, same-parity Unique, default Unique."""
    aliased = np.array([0, 2, 0, 3, 4, 0, 5, 0], np.int32)
    out, k = orc.select(aliased, (aliased != 0).astype(np.uint8))
    assert out[:k].tolist() == [2, 3, 4, 5]
    pred = np.array([-3, 4, -1, 6, 0, 2, 7, -8], np.int32)
    out, k = orc.select(pred, orc.predicate(pred, [(3, 0, 0)]))
    assert out[:k].tolist() == [4, 6, 2, 7]
    uni = np.array([1, 3, 2, 4, 5, 7, 8, 10], np.int32)
    out, k = orc.select(uni, orc.run_heads(uni, key_mask=1))
    assert out[:k].tolist() == [1, 2, 5, 8]
    dflt = np.array([1, 1, 2, 2, 2, 4, 4, 9], np.int32)
    out, k = orc.select(dflt, orc.run_heads(dflt))
    assert out[:k].tolist() == [1, 2, 4, 9]


def _c_rem(x: int, a: int) -> int:
    q = abs(x) // abs(a)
    return x - (q if (x < 0) == (a < 0) else -q) * a


def _py_clause(x, op, a, b, bits):
    if op == 0:
        return True
    if op in (8, 9):
        m = (1 << bits) - 1
        xv = int(np.array([x]).view({8: np.uint8, 32: np.uint32, 64: np.uint64}[bits])[0]) if bits else x
        eq = (xv & a & m) == (b & m)
        return eq if op == 8 else not eq
    return {1: x < a, 2: x <= a, 3: x > a, 4: x >= a, 5: x == a, 6: x != a, 7: a <= x < b,
            10: a != 0 and _c_rem(x, a) == b, 11: a != 0 and _c_rem(x, a) != b}[op]


@pytest.mark.parametrize("dtype", [np.int32, np.uint32, np.int64, np.uint64])
def test_predicate_vs_python(orc, dtype):
    rng = np.random.default_rng(71)
    info = np.iinfo(dtype)
    x = rng.integers(max(info.min, -50), min(info.max, 50), size=300, endpoint=True).astype(dtype)
    bits = 8 * np.dtype(dtype).itemsize
    for op, a, b in [(1, 7, 0), (2, -3, 0), (3, 0, 0), (4, 9, 0), (5, 4, 0), (6, 0, 0), (7, -5, 12), (10, 3, 0),
                     (10, 4, 1), (11, 2, 0), (8, 1, 0), (9, 6, 2)]:
        if info.min == 0 and (a < 0 or b < 0):
            continue
        got = orc.predicate(x, [(op, a, b)])
        want = [_py_clause(int(v), op, a, b, bits) if op not in (8, 9) else
                ((int(v) & ((1 << bits) - 1)) & a) == b if op == 8 else ((int(v) & ((1 << bits) - 1)) & a) != b
                for v in x]
        assert got.astype(bool).tolist() == want, (op, a, b)


def test_predicate_float_and_two_clauses(orc):
    x = np.array([-2.5, -0.0, 0.0, 1.0, 6.99, 7.0, np.nan, np.inf], np.float32)
    assert orc.predicate(x, [(1, 7.0, 0)]).tolist() == [1, 1, 1, 1, 1, 0, 0, 0]
    assert orc.predicate(x, [(5, 0.0, 0)]).tolist() == [0, 1, 1, 0, 0, 0, 0, 0]
    assert orc.predicate(x, [(7, 0.0, 7.0)]).tolist() == [0, 1, 1, 1, 1, 0, 0, 0]
    assert orc.predicate(x, [(3, -1.0, 0), (2, 1.0, 0)]).tolist() == [0, 1, 1, 1, 0, 0, 0, 0]


@pytest.mark.parametrize("dtype", [np.int32, np.uint64, np.float32, np.float64])
def test_compaction_vs_python(orc, dtype):
    rng = np.random.default_rng(5)
    for n in (0, 1, 2, 7, 64, 257):
        raw = rng.integers(0, 4, size=n)
        x = np.repeat(raw, rng.integers(1, 4, size=n))[:n].astype(dtype)
        if dtype == np.float32 and n > 3:
            x[1] = -0.0  # equal to +0.0 by value
            x[2] = 0.0
        sel = (rng.integers(0, 3, size=n) == 0).astype(np.uint8)
        xs = x.tolist()
        out, k = orc.select(x, sel)
        assert out[:k].tolist() == [v for v, s in zip(xs, sel) if s]
        out, k = orc.select(x, sel, partition=True)
        assert out.tolist() == [v for v, s in zip(xs, sel) if s] + [v for v, s in zip(xs, sel) if not s][::-1]
        sel2 = (rng.integers(0, 2, size=n) == 0).astype(np.uint8)
        o1, o2, o3, (c1, c2) = orc.partition_three_way(x, sel, sel2)
        first = [v for v, s in zip(xs, sel) if s]
        second = [v for v, s, t in zip(xs, sel, sel2) if not s and t]
        rest = [v for v, s, t in zip(xs, sel, sel2) if not s and not t]
        assert (c1, c2) == (len(first), len(second))
        assert o1[:c1].tolist() == first and o2[:c2].tolist() == second and o3[:len(rest)].tolist() == rest[::-1]
        runs = []
        for v in xs:
            if runs and runs[-1][0] == v:
                runs[-1][1] += 1
            else:
                runs.append([v, 1])
        u, c = orc.run_length_encode(x)
        assert u.tolist() == [r[0] for r in runs] and c.tolist() == [r[1] for r in runs]
        starts = np.cumsum([0] + [r[1] for r in runs])[:-1] if runs else []
        o, ln = orc.non_trivial_runs(x)
        assert list(zip(o.tolist(), ln.tolist())) == [(int(s), r[1]) for s, r in zip(starts, runs) if r[1] > 1]
        heads = orc.run_heads(x)
        assert heads.tolist() == [int(i == 0 or xs[i] != xs[i - 1]) for i in range(n)]


def test_select_stability_with_index_payload(orc):
    """Kept items keep their order: selecting indices returns an increasing sequence."""
    rng = np.random.default_rng(9)
    idx = np.arange(5000, dtype=np.uint32)
    sel = (rng.random(5000) < 0.3).astype(np.uint8)
    out, k = orc.select(idx, sel)
    assert np.all(np.diff(out[:k].astype(np.int64)) > 0) and k == int(sel.sum())


# ---- segmented reductions and scans -----------------------------------------------------------------
def test_segment_reduce_known_answers(orc):
    """tests/device_segment_reduce.cpp:438-548: empty segments take the initial value; ArgMax of
    negative ties and empty segments; ArgMin's first relative index."""
    assert orc.segment_reduce("sum", np.array([4, 6, 8, 10], np.int32), [0, 2, 2], [2, 2, 4])[0].tolist() == [10, 0, 18]
    v, i, _ = orc.segment_reduce("argmax", np.array([-9, -2, -2, -8, -5], np.float32), [0, 1, 4], [0, 4, 4])
    lo = float(np.finfo(np.float32).min)
    assert v.tolist() == [lo, -2.0, lo] and i.tolist() == [1, 0, 1]
    v, i, _ = orc.segment_reduce("argmin", np.array([7, 1, 1, 9, 4, 2], np.int32), [0, 3], [3, 6])
    assert v.tolist() == [1, 2] and i.tolist() == [1, 2]


def test_segmented_scan_known_answers(orc):
    """tests/device_segmented_scan_test.cpp:11-103 (expected_values), same and packed output offsets."""
    x = np.array([100, 1, 2, 3, 5, 6, 7, 200, 9, 10, 11, 12, 300, 400], np.int32)
    b, e, packed = [1, 4, 4, 8], [4, 4, 7, 12], [0, 4, 6, 10]

    def expected(out_begins, mode):
        want = [None] * 14
        for s in range(4):
            if b[s] == e[s]:
                continue
            agg = 0 if mode == "ex" else (10 if mode == "init" else None)
            for k, idx in enumerate(range(b[s], e[s])):
                if mode == "ex":
                    want[out_begins[s] + k] = agg
                    agg += int(x[idx])
                else:
                    agg = int(x[idx]) if agg is None else agg + int(x[idx])
                    want[out_begins[s] + k] = agg
        return want

    for ob in (b, packed):
        for mode, kw in (("ex", {}), ("in", {"inclusive": True}), ("init", {"inclusive": True, "init": 10})):
            got, _ = orc.segmented_scan(x, b, e, out_begins=ob, **kw)
            want = expected(ob, mode)
            assert [int(g) for g, w in zip(got, want) if w is not None] == [w for w in want if w is not None]


@pytest.mark.parametrize("dtype", [np.int32, np.uint32, np.int64, np.float32])
def test_segment_ops_vs_numpy(orc, dtype):
    """Independent numpy formulation on random ragged, empty and reversed segments."""
    rng = np.random.default_rng(17)
    n = 3000
    x = (rng.integers(-1000, 1000, n) if dtype != np.uint32 else rng.integers(0, 2000, n)).astype(dtype)
    b = rng.integers(0, n, 200).astype(np.uint32)
    e = np.minimum(b + rng.integers(0, 60, 200), n).astype(np.uint32)
    e[::17] = b[::17]          # empty
    e[5::23] = b[5::23] // 2   # reversed: empty
    for op in ("sum", "min", "max") + (("argmin", "argmax") if np.dtype(dtype).itemsize == 4 else ()):
        out, idx, _ = orc.segment_reduce(op, x, b, e)
        for s in range(200):
            seg = x[b[s]:e[s]] if e[s] > b[s] else x[:0]
            if op == "sum":
                want = seg.astype(np.float64).sum() if dtype == np.float32 else int(seg.astype(np.int64).sum())
                if dtype != np.float32:
                    want = np.array([want]).astype(np.int64).astype(dtype)[0] if seg.size else 0
                assert np.isclose(float(out[s]), float(want)), (op, s)
            elif seg.size == 0:
                info = np.finfo(dtype) if dtype == np.float32 else np.iinfo(dtype)
                assert out[s] == (info.max if op in ("min", "argmin") else info.min)
                if idx is not None:
                    assert idx[s] == 1
            else:
                f = np.argmin if op in ("min", "argmin") else np.argmax
                k = int(f(seg))
                assert out[s] == seg[k]
                if idx is not None:
                    assert idx[s] == k
    got, _ = orc.segmented_scan(x, b, e, inclusive=True)
    for s in range(0, 200, 7):
        if e[s] > b[s] and all(not (b[t] < e[s] and b[s] < e[t]) or t == s for t in range(200)):
            want = np.cumsum(x[b[s]:e[s]].astype(np.float64 if dtype == np.float32 else np.int64))
            assert np.allclose(got[b[s]:e[s]].astype(np.float64), want.astype(dtype).astype(np.float64))


# ---- segmented sorts ----------------------------------------------------------------------------------
SEG_KEYS = [91, 3, -2, 3, 92, 8, 1, 8, 4, 93, 5, -1, 5, 2, -1, 7, 2, 5, 0]
SEG_B, SEG_E = [1, 5, 5, 10], [4, 5, 9, 19]


def _py_segmented(keys, begins, ends, key_fn, reverse=False):
    out = list(range(len(keys)))
    for b, e in zip(begins, ends):
        if b < e:
            # Python's sort is stable; descending keeps ties in order with reverse=True on a stable sort.
            out[b:e] = sorted(range(b, e), key=lambda i: key_fn(keys[i]), reverse=reverse)
    return out


def test_segmented_sort_known_answer(orc):
    """tests/device_segmented_sort_test.cpp:19-264: int keys {91, 3, -2, ...}, segments [1,4) [5,5) [5,9)
    [10,19), values = index; items outside every segment untouched."""
    keys = np.array(SEG_KEYS, np.int32)
    vals = np.arange(19, dtype=np.uint32)
    for desc in (False, True):
        for value_order in (False, True):
            ko, vo = orc.segmented_sort(keys, SEG_B, SEG_E, values=vals, descending=desc, value_order=value_order,
                                        keys_out=np.full(19, -777, np.int32), values_out=np.full(19, 2**32 - 1, np.uint32))
            order = _py_segmented(SEG_KEYS, SEG_B, SEG_E, lambda k: k, reverse=desc)
            inside = [any(b <= i < e for b, e in zip(SEG_B, SEG_E)) for i in range(19)]
            assert [int(k) for k, f in zip(ko, inside) if f] == [SEG_KEYS[order[i]] for i in range(19) if inside[i]]
            assert [int(v) for v, f in zip(vo, inside) if f] == [order[i] for i in range(19) if inside[i]]
            assert all(int(k) == -777 for k, f in zip(ko, inside) if not f)


@pytest.mark.parametrize("dtype", [np.uint32, np.int32, np.int64, np.float32])
def test_segmented_radix_bits_vs_python(orc, dtype):
    """Radix order over bit ranges: stable by ((twiddled bits >> begin) & mask)."""
    rng = np.random.default_rng(4)
    n = 3000
    keys = (rng.integers(-500, 500, n) if dtype != np.uint32 else rng.integers(0, 1000, n)).astype(dtype)
    if dtype == np.float32:
        keys = (keys / 7.0).astype(np.float32)
    b = np.sort(rng.choice(n, 40, replace=False)).astype(np.uint32)
    e = np.append(b[1:], n).astype(np.uint32)
    e[::5] = b[::5]
    bits = np.dtype(dtype).itemsize * 8
    ubits = keys.view({4: np.uint32, 8: np.uint64}[keys.itemsize]).astype(object)
    sign = 1 << (bits - 1)

    def tw(u):
        if dtype in (np.int32, np.int64):
            return u ^ sign
        if dtype == np.float32:
            return (~u & ((1 << bits) - 1)) if u & sign else u | sign
        return u
    for lo, hi in ((0, bits), (2, 6), (3, bits - 1)):
        mask = (1 << (hi - lo)) - 1
        for desc in (False, True):
            ko, _ = orc.segmented_sort(keys, b, e, begin_bit=lo, end_bit=hi, descending=desc)
            order = _py_segmented(list(ubits), b, e, lambda u: (tw(int(u)) >> lo) & mask, reverse=desc)
            np.testing.assert_array_equal(ko.view(np.uint8), keys[order].view(np.uint8))


def test_segmented_sort_value_order_floats(orc):
    """DeviceSegmentedSort's default comparator (lhs < rhs, device_segmented_sort.h:77-105) on floats:
    -0.0 and +0.0 are equal, so they keep their input order; against Python's stable sorted()."""
    rng = np.random.default_rng(12)
    n = 2000
    keys = (rng.integers(-40, 40, n) / 4.0).astype(np.float64)
    keys[rng.random(n) < 0.05] = -0.0
    b = np.array([0, 700, 701, 1500], np.uint32)
    e = np.array([700, 701, 1500, n], np.uint32)
    for dtype in (np.float32, np.float64):
        k = keys.astype(dtype)
        for desc in (False, True):
            ko, _ = orc.segmented_sort(k, b, e, value_order=True, descending=desc)
            order = _py_segmented([float(x) for x in k], b, e, lambda x: x, reverse=desc)
            np.testing.assert_array_equal(ko.view(np.uint8), k[order].view(np.uint8))
    # Radix order of the same keys puts -0.0 before +0.0 (ascending).
    k = np.array([0.0, -0.0, 0.0, -0.0], np.float32)
    ko, _ = orc.segmented_sort(k, [0], [4])
    assert np.signbit(ko).tolist() == [True, True, False, False]


# ---- host baselines (oracle/cpu_baseline.cpp) ------------------------------------------------------
# Each multi-threaded baseline must give the serial oracle's result for every thread count, including
# thread counts that do not divide n and more threads than items.
@pytest.mark.parametrize("threads", [1, 2, 3, 8, 17])
def test_par_reduce_and_scan_match_serial(orc, threads):
    rng = np.random.default_rng(threads)
    for n in (0, 1, 5, 1000003):
        a = rng.integers(-1000, 1001, n).astype(np.int32)
        assert orc.par_reduce_sum_i32(a, threads) == int(a.astype(np.int64).sum())
        u = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
        assert np.array_equal(orc.par_scan_sum_u32(u, threads), orc.scan_sum_u32(u))


@pytest.mark.parametrize("threads", [1, 2, 5, 16])
def test_par_sorts_match_serial(orc, threads):
    rng = np.random.default_rng(100 + threads)
    for n in (1, 7, 300001):
        k = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
        got = orc.par_radix_sort_u32(k.copy(), threads)
        assert np.array_equal(got, orc.radix_sort(k))
        assert np.array_equal(orc.std_sort_u32(k.copy()), got)
        # Pairs with index values and low-entropy keys: stability is visible in the values.
        k64 = (rng.integers(0, 2**63, n, dtype=np.int64).astype(np.uint64) & np.uint64(0x0101010101010101))
        v = np.arange(n, dtype=np.uint32)
        gk, gv = orc.par_radix_sort_u64_u32(k64.copy(), v.copy(), threads)
        ek, ev = orc.radix_sort(k64, v)
        assert np.array_equal(gk, ek) and np.array_equal(gv, ev)


@pytest.mark.parametrize("threads", [1, 4, 9])
def test_par_spmv_matches_row_loop(orc, threads):
    rng = np.random.default_rng(7)
    rows = cols = 4000
    lengths = rng.integers(0, 40, rows)
    lengths[::97] = 0  # empty rows
    ro = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    nnz = int(ro[-1])
    ci = rng.integers(0, cols, nnz).astype(np.int32)
    av = rng.uniform(-1, 1, nnz).astype(np.float32)
    xv = rng.uniform(-1, 1, cols).astype(np.float32)
    y = orc.par_spmv_csr_f32(av, ro, ci, xv, rows, threads)
    ref = np.zeros(rows, np.float32)
    for r in range(rows):  # the same float row loop, in order
        s = np.float32(0)
        for j in range(ro[r], ro[r + 1]):
            s = np.float32(s + np.float32(av[j] * xv[ci[j]]))
        ref[r] = s
    assert np.array_equal(y, ref)
    exact, absum = orc.spmv_csr_fp(av, ro, ci, xv, rows, cols, nnz)
    assert np.all(np.abs(y.astype(np.float64) - exact) <= 1e-5 * np.maximum(np.abs(exact), absum))


# ---- every exported oracle function is exercised by the tests above --------------------------------
_CALLED: set[str] = set()


class _CallRecorder:
    """Stands in for the oracle's ctypes handle and records the name of every function looked up."""

    def __init__(self, handle):
        self._handle = handle

    def __getattr__(self, name):
        _CALLED.add(name)
        return getattr(self._handle, name)


@pytest.fixture(scope="module", autouse=True)
def _record_oracle_calls(orc):
    real = orc.lib()
    orc._lib = _CallRecorder(real)
    yield
    orc._lib = real


def test_zz_every_exported_oracle_function_is_exercised(orc, request):
    """Each `oracle_*` symbol the library exports must have been called by a test of this module, each of
    which compares it with an independent result.  Runs only when the whole module ran in this process."""
    this = sys.modules[__name__]
    names = {n for n in dir(this) if n.startswith("test_") and n != request.function.__name__}
    ran = {item.originalname for item in request.session.items if getattr(item, "module", None) is this}
    if not names <= ran or os.environ.get("PYTEST_XDIST_WORKER"):
        pytest.skip("needs every test of this module in one process")
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm (binutils) not found")
    out = subprocess.run([nm, "-D", "--defined-only", str(orc.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {f[-1] for f in (line.split() for line in out.splitlines()) if f and f[-1].startswith("oracle_")}
    assert len(exported) > 50
    assert exported - _CALLED == set()
