"""DeviceReduce::Sum on the GPU vs the oracle (bit-exact for integers; a stated tolerance for floats).

Cases follow the reference tests: sums of 2^k+1 ones (tests/device_reduce_test.cpp:95-119), shuffled
iota (:85-91), transform sizes {1,31,256,1023,1024,1025,1048577,4194304} (:148-173), 2^24+1 zeros
plus a tail value (tests/pr6_review_regression_test.cpp:427-457), the benchmark input (2^24 int32 in
[-1000, 1000] from seed 114521) and 2^28 items (1 GiB of int32).
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


def test_sum_2p28_i32(hip, orc, dev):
    """Sum of 2^28 int32 values in [-1000, 1000], bit-exact against the oracle."""
    n = 1 << 28
    log("reduce 2^28")
    d = torch.empty(n, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_I32_PM1000, d, n, 4242)
    out = fill_dev(1, 4, 0)
    hip.reduce_sum("i32", d, out, n)
    assert to_host(out, np.int32, 1)[0] == orc.reduce_sum_i32(to_host(d, np.int32))[0]


# ---- Min / Max / ArgMin / ArgMax -------------------------------------------------------------------
# device_reduce.h:291-436 (MinOp / MaxOp / ArgMinOp / ArgMaxOp): bit-exact against the oracle's left-to-right
# fold for every type; the reference's cases of tests/device_reduce_test.cpp:175-345.
EXT_TYPES = {"i32": np.int32, "u32": np.uint32, "f32": np.float32, "i64": np.int64, "u64": np.uint64,
             "f64": np.float64}


def ext_input(suffix, n, seed, nan_fraction=0.0):
    dtype = np.dtype(EXT_TYPES[suffix])
    rng = np.random.default_rng(seed)
    if dtype.kind == "f":
        a = (rng.standard_normal(n) * 1e3).astype(dtype)
        if nan_fraction:
            a[rng.random(n) < nan_fraction] = np.nan
        return a
    info = np.iinfo(dtype)
    return rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)


def gpu_ext(hip, op, suffix, a, offset=0):
    d = to_dev(a)[offset:]
    out = fill_dev(1, a.dtype.itemsize, 0x5A5A5A5A)
    hip.reduce_minmax(op, suffix, d, out, a.size - offset)
    return to_host(out, a.dtype, 1)[0]


def gpu_arg(hip, op, suffix, a, offset=0):
    d = to_dev(a)[offset:]
    out = fill_dev(1, a.dtype.itemsize, 0x5A5A5A5A)
    idx = fill_dev(1, 4, 0x5A5A5A5A)
    hip.reduce_arg(op, suffix, d, out, idx, a.size - offset)
    return to_host(out, a.dtype, 1)[0], int(to_host(idx, np.uint32, 1)[0])


def same(x, y):
    return np.asarray(x).tobytes() == np.asarray(y).tobytes()


def test_reference_cases_min_max_arg(hip, dev):
    """device_reduce_test.cpp:218-345: float Max from the lowest identity, ArgMax's first equal extremum,
    ArgMax of negative floats, empty-input sentinels."""
    assert gpu_ext(hip, "max", "f32", np.array([-8.0, -2.5, -9.0, -4.0], np.float32)) == np.float32(-2.5)
    assert gpu_arg(hip, "max", "i32", np.array([1, 9, 4, 9, 3], np.int32)) == (9, 1)
    assert gpu_arg(hip, "max", "f32", np.array([-7.0, -3.0, -5.0], np.float32)) == (np.float32(-3.0), 1)
    for op, want in (("min", np.iinfo(np.int32).max), ("max", np.iinfo(np.int32).min)):
        d = torch.empty(0, dtype=torch.int32, device=dev)
        out, idx = fill_dev(1, 4, 7), fill_dev(1, 4, 7)
        hip.reduce_arg(op, "i32", d, out, idx, 0)
        assert int(to_host(out, np.int32, 1)[0]) == want and int(to_host(idx, np.uint32, 1)[0]) == 1
        hip.reduce_minmax(op, "i32", d, out, 0)
        assert int(to_host(out, np.int32, 1)[0]) == want


@pytest.mark.parametrize("suffix", list(EXT_TYPES))
@pytest.mark.parametrize("n", [1, 3, 31, 1025, 4097, 65537, 1000003, (1 << 22) + 5])
def test_min_max_arg_vs_oracle(hip, orc, dev, suffix, n):
    log(f"reduce min/max/arg {suffix} n={n}")
    a = ext_input(suffix, n, n + len(suffix))
    for op in ("min", "max"):
        assert same(gpu_ext(hip, op, suffix, a), orc.reduce_minmax(op, a)), op
        v, i = gpu_arg(hip, op, suffix, a)
        ov, oi = orc.reduce_arg(op, a)
        assert same(v, ov) and i == oi, (op, v, i, ov, oi)
        want_i = int(np.argmin(a) if op == "min" else np.argmax(a))
        assert i == want_i


@pytest.mark.parametrize("suffix", ["i32", "f64"])
def test_min_max_arg_unaligned_and_ties(hip, orc, dev, suffix):
    """Subviews off the 16-byte grid; many equal extrema: the lowest index wins wherever the copies sit."""
    n = (1 << 20) + 77
    dtype = EXT_TYPES[suffix]
    rng = np.random.default_rng(4)
    a = rng.integers(-50, 50, n).astype(dtype)
    a[rng.integers(0, n, 40)] = dtype(-1000)
    a[rng.integers(0, n, 40)] = dtype(1000)
    for offset in (1, 2, 3):
        b = a[offset:]
        for op in ("min", "max"):
            assert same(gpu_ext(hip, op, suffix, a, offset), orc.reduce_minmax(op, b))
            v, i = gpu_arg(hip, op, suffix, a, offset)
            assert (v, i) == orc.reduce_arg(op, b)


def test_float_nan_and_signed_zero(hip, orc, dev):
    """NaN items never win; -0.0 == +0.0, so ArgMin / ArgMax take the first zero (its sign bit included);
    an all-NaN input gives the initial pair (the type's max / lowest, index 0xFFFFFFFF); Min / Max of
    +-infinity stop at the initial value (the type's max / lowest), as the reference's fold does."""
    for dtype, sfx in ((np.float32, "f32"), (np.float64, "f64")):
        n = (1 << 21) + 9
        a = ext_input(sfx, n, 3, nan_fraction=0.1)
        for op in ("min", "max"):
            assert same(gpu_ext(hip, op, sfx, a), orc.reduce_minmax(op, a))
            assert gpu_arg(hip, op, sfx, a) == orc.reduce_arg(op, a)
        z = np.full(70000, np.nan, dtype)
        z[5000], z[9000], z[65000] = 0.0, -0.0, 0.0
        for op in ("min", "max"):
            v, i = gpu_arg(hip, op, sfx, z)
            assert i == 5000 and not np.signbit(v)
        z[5000] = -0.0
        v, i = gpu_arg(hip, "min", sfx, z)
        assert i == 5000 and np.signbit(v)
        allnan = np.full(3000, np.nan, dtype)
        assert gpu_arg(hip, "min", sfx, allnan) == (np.finfo(dtype).max, 0xFFFFFFFF)
        assert gpu_arg(hip, "max", sfx, allnan) == (np.finfo(dtype).min, 0xFFFFFFFF)
        inf = np.array([np.inf, 1.0, np.inf], dtype)
        assert gpu_ext(hip, "max", sfx, inf) == np.inf and gpu_ext(hip, "min", sfx, -inf) == -np.inf
        assert gpu_ext(hip, "min", sfx, np.array([np.inf], dtype)) == np.finfo(dtype).max


def test_min_max_arg_2p28(hip, orc, dev):
    """The 2^28 benchmark size: int32 from the on-device generator, the extremes planted late."""
    n = 1 << 28
    log("reduce min/max/arg 2^28")
    d = torch.empty(n, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_I32_PM1000, d, n, 114521)
    d[n - 3] = -5000
    d[n - 7] = 5000
    d[n - 2] = -5000
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    idx = torch.zeros(1, dtype=torch.int32, device=dev)
    hip.reduce_arg("min", "i32", d, out, idx, n)
    assert int(out.item()) == -5000 and int(idx.item()) == n - 3
    hip.reduce_arg("max", "i32", d, out, idx, n)
    assert int(out.item()) == 5000 and int(idx.item()) == n - 7
    hip.reduce_minmax("min", "i32", d, out, n)
    assert int(out.item()) == -5000


# ---- Reduce(op, init) and TransformReduce(op, transform, init) ----------------------------------------
# device_reduce.h:229-252,491-515: op(init, fold of transform(items)), n == 0 writes init.  Integer
# results and float min / max (selections) bit-exact against the oracle; float sums within
# |got - exact| <= rel * (|init| + sum of |terms|), rel 1e-5 (f32) / 1e-12 (f64), the oracle summing in
# long double.
NP_OF = {"i32": np.int32, "u32": np.uint32, "f32": np.float32, "i64": np.int64, "u64": np.uint64, "f64": np.float64}


def run_transform_reduce(hip, suffix, a, op, transform="identity", scale=0, shift=0, init=0, offset=0):
    d = to_dev(a) if a.size else torch.empty(1, dtype=torch.int32, device="cuda:0")
    out = fill_dev(1, a.dtype.itemsize, 0x5A5A5A5A)
    if transform == "identity" and scale == 0 and shift == 0:
        hip.reduce_op(op, suffix, d[offset:], out, a.size - offset, init=init)
    else:
        hip.transform_reduce(op, transform, suffix, d[offset:], out, a.size - offset, scale=scale, shift=shift,
                             init=init)
    return to_host(out, a.dtype, 1)[0]


def test_transform_reduce_reference_cases(hip, dev):
    """tests/device_reduce_test.cpp:120-173 and tests/pr6_review_regression_test.cpp:144-240."""
    a = np.random.default_rng(114521).permutation(4096).astype(np.int32)
    assert run_transform_reduce(hip, "i32", a, "max", "square") == 4095 ** 2
    for size in (1, 31, 256, 1023, 1024, 1025, 1048577, 4194304):
        x = (np.arange(size) % 13 - 6).astype(np.int32)
        log(f"transform reduce 2x+1 n={size}")
        assert run_transform_reduce(hip, "i32", x, "sum", "affine", 2, 1, 17) == \
            17 + int((2 * x.astype(np.int64) + 1).sum())
    h = (np.arange(4097) % 7 + 1).astype(np.int32)
    s, n = int(h.sum()), h.size
    assert run_transform_reduce(hip, "i32", h, "sum") == s
    assert run_transform_reduce(hip, "i32", h, "max") == 7
    assert run_transform_reduce(hip, "i32", h, "sum", "affine", 1, 1) == s + n
    assert run_transform_reduce(hip, "i32", h, "sum", "affine", 1, 7) == s + 7 * n
    assert run_transform_reduce(hip, "i32", h, "sum", "affine", 2, 0) == 2 * s
    assert run_transform_reduce(hip, "i32", h, "sum", "square") == int((h.astype(np.int64) ** 2).sum())
    assert run_transform_reduce(hip, "i32", h, "sum", "identity", 5, 5) == s
    for op in ("sum", "min", "max"):
        assert run_transform_reduce(hip, "i32", np.zeros(0, np.int32), op, "square", init=-9) == -9


def _check_transform_reduce(orc, suffix, got, a, op, transform, scale, shift, init):
    want, exact, absum = orc.transform_reduce(a, op, transform, scale, shift, init)
    if op == "sum" and suffix in ("f32", "f64"):
        rel = 1e-5 if suffix == "f32" else 1e-12
        assert abs(float(got) - exact) <= rel * max(absum, 1e-30), (got, exact)
    else:
        assert np.array([got]).view(f"u{a.itemsize}")[0] == np.array([want]).view(f"u{a.itemsize}")[0], (got, want)


@pytest.mark.parametrize("suffix", ["i32", "u32", "f32", "i64", "u64", "f64"])
@pytest.mark.parametrize("n", [1, 17, 4097, 1000003, (1 << 24) + 1])
def test_transform_reduce_vs_oracle(hip, orc, dev, suffix, n):
    dtype = NP_OF[suffix]
    rng = np.random.default_rng(n + len(suffix))
    if np.dtype(dtype).kind == "f":
        a = (rng.standard_normal(n) * 100).astype(dtype)
        a[rng.random(n) < 0.01] = np.nan if n < 5000 else a[0]
        params = (1.5, -0.25, 3.0)
    else:
        info = np.iinfo(dtype)
        a = rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)
        params = (3, 11, 7)
    log(f"transform reduce {suffix} n={n}")
    for transform in ("identity", "affine", "square", "abs"):
        for op in ("sum", "min", "max"):
            if op == "sum" and np.dtype(dtype).kind == "f" and np.isnan(a).any():
                continue  # a NaN sum has no tolerance to check against
            got = run_transform_reduce(hip, suffix, a, op, transform, *params)
            _check_transform_reduce(orc, suffix, got, a, op, transform, *params)


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_transform_reduce_unaligned_and_float_edges(hip, orc, dev, offset):
    """Views that start off a 16-byte boundary, float min / max with NaNs (skipped), all-NaN input (init),
    the initial value as the left operand (of +0.0 and -0.0 init is kept) and a NaN initial value."""
    rng = np.random.default_rng(offset)
    a = rng.integers(-1000, 1000, 300_001).astype(np.int32)
    for op, transform in (("sum", "affine"), ("max", "square"), ("min", "abs")):
        got = run_transform_reduce(hip, "i32", a, op, transform, 3, -2, 5, offset=offset)
        _check_transform_reduce(orc, "i32", got, a[offset:], op, transform, 3, -2, 5)
    z = np.full(100_000, -0.0, np.float32)
    assert not np.signbit(run_transform_reduce(hip, "f32", z, "min", init=0.0))
    assert np.signbit(run_transform_reduce(hip, "f32", -z, "max", init=-0.0))
    assert run_transform_reduce(hip, "f32", np.full(70_000, np.nan, np.float32), "min", init=2.5) == np.float32(2.5)
    v = rng.standard_normal(90_001)
    v[::7] = np.nan
    for op in ("min", "max"):
        got = run_transform_reduce(hip, "f64", v, op, "square", init=np.nan)
        _check_transform_reduce(orc, "f64", got, v, op, "square", 0, 0, np.nan)


def test_transform_reduce_rejects_unknown_op_and_transform(hip, dev):
    lib = hip.lib()
    a = torch.ones(1000, dtype=torch.int32, device=dev)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    temp = torch.empty(hip.bytes_to_uint_count(hip.reduce_temp_bytes(1000, 4)), dtype=torch.int32, device=dev)
    tb = temp.numel() * 4
    assert lib.lcpp_hip_reduce_op_i32(temp.data_ptr(), tb, a.data_ptr(), out.data_ptr(), 1000, 3, 0, None) == \
        hip.ERR_INVALID_ARGUMENT
    assert lib.lcpp_hip_transform_reduce_i32(temp.data_ptr(), tb, a.data_ptr(), out.data_ptr(), 1000, 0, 4, 1, 0, 0,
                                             None) == hip.ERR_INVALID_ARGUMENT
    torch.cuda.synchronize()
    assert int(out.item()) == 0
