"""Scan-by-key and reduce-by-key (sum operator) on the GPU, through the C-ABI.

Known answers of the reference's tests (device_scan_test.cpp:325-447, device_reduce_test.cpp:420-512)
exactly; integer values bit-exact against the oracle for every key/value type and scan mode; float
values within |got - exact| <= rel * (sum of |terms|) with rel 1e-5 (f32) / 1e-12 (f64), where the
oracle sums in long double.  Also: tile-boundary sizes (the scan's 16,384-item and the reduce's 15,360-item
tiles of 4-byte keys and values), runs spanning many tiles, reduce tiles with fewer and with more runs than
the kernel stages in LDS (4,096 for 4-byte keys and values, 2,048 for 8-byte ones), in-place scans, the forced
look-back fallback (spin limit 0) and misaligned (element-offset) views."""
import numpy as np
import pytest
import torch

from gpu_util import fill_dev, log, to_dev, to_host

pytestmark = pytest.mark.gpu

NP = {"i32": np.int32, "u32": np.uint32, "f32": np.float32, "i64": np.int64, "u64": np.uint64, "f64": np.float64}
TILE = 12288         # scan tile, 4-byte keys and values
REDUCE_TILE = 15360  # reduce tile, 4-byte keys and values


def run_keys(rng, n, mean_len, key_dtype, distinct=1 << 30):
    """Keys in runs of geometric length (mean `mean_len`); consecutive runs get different keys."""
    lengths = rng.geometric(1.0 / mean_len, size=n // max(1, int(mean_len)) + 16)
    while lengths.sum() < n:
        lengths = np.concatenate([lengths, rng.geometric(1.0 / mean_len, size=len(lengths))])
    ids = np.repeat(np.arange(lengths.size), lengths)[:n]
    base = rng.integers(0, distinct, lengths.size)
    base[1:] = np.where(base[1:] == base[:-1], base[1:] + 1, base[1:])  # neighbours differ
    return base[ids].astype(key_dtype)


def values_for(rng, n, vs):
    dt = NP[vs]
    if vs in ("f32", "f64"):
        return rng.uniform(-1.0, 1.0, n).astype(dt)
    info = np.iinfo(dt)
    return rng.integers(info.min, info.max, n, dtype=dt, endpoint=True)


def gpu_scan_by_key(hip, ks, vs, keys, vals, inclusive, init=None, key_mask=-1, in_place=False, op="sum"):
    n = keys.size
    d_k, d_v = to_dev(keys), to_dev(vals)
    d_o = d_v if in_place else torch.empty_like(d_v)
    hip.scan_by_key(ks, vs, d_k, d_v, d_o, n, inclusive=inclusive, init=init, key_mask=key_mask, op=op)
    return to_host(d_o, NP[vs], n)


def gpu_reduce_by_key(hip, ks, vs, keys, vals, key_mask=-1, op="sum"):
    n = keys.size
    d_k, d_v = to_dev(keys), to_dev(vals)
    uniq = fill_dev(max(n, 1), keys.itemsize, 0x5A5A5A5A)
    agg = fill_dev(max(n, 1), vals.itemsize, 0x5A5A5A5A)
    runs = fill_dev(1, 4, 17)
    hip.reduce_by_key(ks, vs, d_k, d_v, uniq, agg, runs, n, key_mask=key_mask, op=op)
    r = int(to_host(runs, np.uint32, 1)[0])
    return to_host(uniq, keys.dtype, r), to_host(agg, NP[vs], r), r


def check_scan(orc, keys, vals, got, vs, inclusive, init, key_mask):
    if vs in ("f32", "f64"):
        exact, ab = orc.scan_by_key_fp(keys, vals, inclusive=inclusive, use_init=init is not None,
                                       init=0.0 if init is None else init, key_mask=key_mask)
        rel = 1e-5 if vs == "f32" else 1e-12
        err = np.abs(got.astype(np.float64) - exact)
        assert np.all(err <= rel * np.maximum(ab, 1e-30)), f"worst {np.max(err / np.maximum(ab, 1e-30))}"
    else:
        want = orc.scan_by_key_int(keys, vals, inclusive=inclusive, use_init=init is not None,
                                   init=0 if init is None else init, key_mask=key_mask)
        assert np.array_equal(got, want)


def check_reduce(orc, keys, vals, uniq, agg, runs, vs, key_mask):
    if vs in ("f32", "f64"):
        ou, oa, ab = orc.reduce_by_key_fp(keys, vals, key_mask=key_mask)
        assert runs == ou.size and np.array_equal(uniq, ou)
        rel = 1e-5 if vs == "f32" else 1e-12
        assert np.all(np.abs(agg.astype(np.float64) - oa) <= rel * np.maximum(ab, 1e-30))
    else:
        ou, oa = orc.reduce_by_key_int(keys, vals, key_mask=key_mask)
        assert runs == ou.size and np.array_equal(uniq, ou) and np.array_equal(agg, oa)


# ---- the reference's known answers ---------------------------------------------------------------

@pytest.mark.parametrize("log_n", [5, 9, 12, 13, 16, 20])
def test_exclusive_sum_by_key_ones_known_answer(hip, dev, log_n):
    """device_scan_test.cpp:325-385: ones with keys i / 100 give i % 100."""
    n = 1 << log_n
    keys = (np.arange(n) // 100).astype(np.int32)
    got = gpu_scan_by_key(hip, "i32", "i32", keys, np.ones(n, np.int32), inclusive=False)
    assert np.array_equal(got, (np.arange(n) % 100).astype(np.int32))


def test_inclusive_sum_by_key_three_tiles_known_answer(hip, dev):
    """device_scan_test.cpp:387-417 (reference tile 256 x 15): int keys, int64 ones."""
    tile = 256 * 15
    n = 2 * tile + 2
    idx = np.arange(n)
    keys = np.where(idx < tile + 1, 1, np.where(idx < 2 * tile + 1, 2, 3)).astype(np.int32)
    got = gpu_scan_by_key(hip, "i32", "i64", keys, np.ones(n, np.int64), inclusive=True)
    expected = np.concatenate([np.arange(1, tile + 2), np.arange(1, tile + 1), np.arange(1, 2)]).astype(np.int64)
    assert np.array_equal(got, expected)


def test_inclusive_sum_by_key_parity_equality_known_answer(hip, dev):
    """device_scan_test.cpp:419-447: (lhs & 1) == (rhs & 1) over {1,3,5,2,4} gives {1,2,3,1,2}."""
    got = gpu_scan_by_key(hip, "i32", "i32", np.array([1, 3, 5, 2, 4], np.int32), np.ones(5, np.int32),
                          inclusive=True, key_mask=1)
    assert got.tolist() == [1, 2, 3, 1, 2]


def test_reduce_by_key_blocks_of_100_known_answer(hip, orc, dev):
    """device_reduce_test.cpp:420-478: 4096 items, keys i / 100, values a permutation of 0..4095."""
    n = 4096
    keys = (np.arange(n) // 100).astype(np.int32)
    vals = np.random.default_rng(114521).permutation(n).astype(np.int32)
    uniq, agg, runs = gpu_reduce_by_key(hip, "i32", "i32", keys, vals)
    assert runs == 41 and uniq.tolist() == list(range(41))
    assert agg.astype(np.int64).tolist() == [int(vals[i * 100:(i + 1) * 100].sum()) for i in range(41)]


def test_reduce_by_key_empty_input_writes_zero_runs(hip, dev):
    """device_reduce_test.cpp:480-512: the run count is preset to 17 and must read 0 afterwards."""
    runs = fill_dev(1, 4, 17)
    one = torch.zeros(1, dtype=torch.int32, device=dev)
    hip.reduce_by_key("i32", "i32", one, one, one, one, runs, 0)
    assert int(to_host(runs, np.uint32, 1)[0]) == 0


def test_scan_by_key_empty_input_is_a_no_op(hip, dev):
    out = fill_dev(4, 4, 0x77)
    one = torch.zeros(1, dtype=torch.int32, device=dev)
    hip.scan_by_key("i32", "i32", one, one, out, 0, inclusive=True)
    assert to_host(out, np.uint32).tolist() == [0x77] * 4


# ---- oracle parity -------------------------------------------------------------------------------

@pytest.mark.parametrize("ks", ["i32", "u32", "i64", "u64"])
@pytest.mark.parametrize("vs", ["i32", "u32", "f32", "i64", "u64", "f64"])
def test_scan_by_key_types_and_modes(hip, orc, dev, ks, vs):
    rng = np.random.default_rng(sum(map(ord, ks + vs)))
    n = 3 * TILE + 1234
    keys = run_keys(rng, n, 7.0, NP[ks])
    vals = values_for(rng, n, vs)
    log(f"scan_by_key {ks}/{vs} n={n}")
    init = 2.5 if vs in ("f32", "f64") else 0x1234567
    for inclusive, use_init in ((False, True), (True, False), (True, True)):
        iv = init if use_init else None
        got = gpu_scan_by_key(hip, ks, vs, keys, vals, inclusive, iv)
        check_scan(orc, keys, vals, got, vs, inclusive, iv, -1)


@pytest.mark.parametrize("ks", ["i32", "u64"])
@pytest.mark.parametrize("vs", ["i32", "f32", "u64", "f64"])
def test_reduce_by_key_types(hip, orc, dev, ks, vs):
    rng = np.random.default_rng(7 + len(ks + vs))
    n = 5 * TILE + 77
    keys = run_keys(rng, n, 5.0, NP[ks])
    vals = values_for(rng, n, vs)
    log(f"reduce_by_key {ks}/{vs} n={n}")
    uniq, agg, runs = gpu_reduce_by_key(hip, ks, vs, keys, vals)
    check_reduce(orc, keys, vals, uniq, agg, runs, vs, -1)


@pytest.mark.parametrize("n", [1, 2, 15, 16, 17, 255, 256, 257, 1023, 1024, 1025, REDUCE_TILE - 1, REDUCE_TILE,
                               REDUCE_TILE + 1, 2 * REDUCE_TILE + 1, TILE - 1, TILE, TILE + 1, 2 * TILE + 1,
                               64 * TILE + 3])
def test_tile_boundary_sizes(hip, orc, dev, n):
    rng = np.random.default_rng(n)
    keys = run_keys(rng, n, 3.0, np.int32)
    vals = values_for(rng, n, "u32")
    log(f"by_key boundary n={n}")
    check_scan(orc, keys, vals, gpu_scan_by_key(hip, "i32", "u32", keys, vals, True), "u32", True, None, -1)
    check_scan(orc, keys, vals, gpu_scan_by_key(hip, "i32", "u32", keys, vals, False, 5), "u32", False, 5, -1)
    uniq, agg, runs = gpu_reduce_by_key(hip, "i32", "u32", keys, vals)
    check_reduce(orc, keys, vals, uniq, agg, runs, "u32", -1)


@pytest.mark.parametrize("kind", ["all_distinct", "one_run", "long_runs", "runs_on_tile_edges"])
def test_run_structures(hip, orc, dev, kind):
    rng = np.random.default_rng(3)
    n = 200 * TILE + 11
    if kind == "all_distinct":
        keys = np.arange(n, dtype=np.uint32)
    elif kind == "one_run":
        keys = np.full(n, 42, np.uint32)
    elif kind == "long_runs":
        keys = run_keys(rng, n, 60000.0, np.uint32)   # runs spanning ~15 tiles on average
    else:
        keys = (np.arange(n) // TILE).astype(np.uint32)  # every run starts exactly on a tile
    vals = values_for(rng, n, "i32")
    log(f"by_key runs {kind} n={n}")
    check_scan(orc, keys, vals, gpu_scan_by_key(hip, "u32", "i32", keys, vals, True), "i32", True, None, -1)
    check_scan(orc, keys, vals, gpu_scan_by_key(hip, "u32", "i32", keys, vals, False, -3), "i32", False, -3, -1)
    uniq, agg, runs = gpu_reduce_by_key(hip, "u32", "i32", keys, vals)
    check_reduce(orc, keys, vals, uniq, agg, runs, "i32", -1)


def test_key_mask_classes(hip, orc, dev):
    """Keys equal when they agree on the masked bits (bit classes across tiles)."""
    rng = np.random.default_rng(21)
    n = 7 * TILE + 5
    keys = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    keys = (keys & ~np.uint32(0xF0)) | ((np.arange(n, dtype=np.uint32) // 37 % 3) << np.uint32(4))
    vals = values_for(rng, n, "u32")
    check_scan(orc, keys, vals, gpu_scan_by_key(hip, "u32", "u32", keys, vals, True, key_mask=0xF0), "u32", True,
               None, 0xF0)
    uniq, agg, runs = gpu_reduce_by_key(hip, "u32", "u32", keys, vals, key_mask=0xF0)
    check_reduce(orc, keys, vals, uniq, agg, runs, "u32", 0xF0)


@pytest.mark.parametrize("vs", ["i32", "f64"])
def test_in_place_scan_with_forced_fallback(hip, orc, dev, vs):
    """values_out == values_in while every look-back takes the fallback (spin limit 0): helpers read a
    predecessor's input while its owner may be about to overwrite it."""
    rng = np.random.default_rng(99)
    n = 300 * TILE + 9
    keys = run_keys(rng, n, 3000.0, np.int32)
    vals = values_for(rng, n, vs)
    lib = hip.lib()
    old = lib.lcpp_hip_get_lookback_spin_limit()
    try:
        lib.lcpp_hip_set_lookback_spin_limit(0)
        for inclusive in (True, False):
            log(f"in-place fallback {vs} inclusive={inclusive}")
            got = gpu_scan_by_key(hip, "i32", vs, keys, vals, inclusive, None if inclusive else 0, in_place=True)
            check_scan(orc, keys, vals, got, vs, inclusive, None if inclusive else 0, -1)
        uniq, agg, runs = gpu_reduce_by_key(hip, "i32", vs, keys, vals)
        check_reduce(orc, keys, vals, uniq, agg, runs, vs, -1)
    finally:
        lib.lcpp_hip_set_lookback_spin_limit(old)


@pytest.mark.parametrize("which", ["keys", "values", "out"])
def test_misaligned_views(hip, orc, dev, which):
    """Views offset by one element are not 16-byte aligned and take the element-wise load/store path."""
    rng = np.random.default_rng(55)
    n = 9 * TILE + 3
    keys = run_keys(rng, n, 11.0, np.int32)
    vals = values_for(rng, n, "u32")
    d_k = to_dev(np.concatenate([[7], keys]).astype(np.int32))[1:] if which == "keys" else to_dev(keys)
    d_v = to_dev(np.concatenate([[7], vals]).astype(np.uint32))[1:] if which == "values" else to_dev(vals)
    d_o = (torch.empty(n + 1, dtype=torch.int32, device=dev)[1:] if which == "out"
           else torch.empty(n, dtype=torch.int32, device=dev))
    hip.scan_by_key("i32", "u32", d_k, d_v, d_o, n, inclusive=True)
    check_scan(orc, keys, vals, to_host(d_o, np.uint32, n), "u32", True, None, -1)


@pytest.mark.parametrize("ks,vs", [("u32", "u32"), ("i32", "f32"), ("u64", "i64"), ("i64", "f64"), ("u32", "u64")])
def test_reduce_staged_and_direct_tiles(hip, orc, dev, ks, vs):
    """Run lengths 1..6 in 4,096-item stretches: some reduce tiles hold more runs than the LDS stage (they
    write their outputs row by row after the look-back), others fewer (staged outputs), side by side."""
    rng = np.random.default_rng(77)
    n = 40 * TILE + 321
    length = 1 + (np.arange(n) // 4096) % 6
    starts = np.zeros(n, bool)
    pos = 0
    while pos < n:
        starts[pos] = True
        pos += int(length[pos])
    keys = np.cumsum(starts).astype(NP[ks]) * NP[ks](3)
    vals = values_for(rng, n, vs)
    log(f"reduce staged/direct {ks} {vs}")
    uniq, agg, runs = gpu_reduce_by_key(hip, ks, vs, keys, vals)
    check_reduce(orc, keys, vals, uniq, agg, runs, vs, -1)


def test_reduce_misaligned_keys_and_values(hip, orc, dev):
    rng = np.random.default_rng(56)
    n = 9 * TILE + 3
    keys = run_keys(rng, n, 11.0, np.int32)
    vals = values_for(rng, n, "u32")
    d_k = to_dev(np.concatenate([[7], keys]).astype(np.int32))[1:]
    d_v = to_dev(np.concatenate([[7], vals]).astype(np.uint32))[1:]
    uniq = fill_dev(n, 4, 0x5A5A5A5A)
    agg = fill_dev(n, 4, 0x5A5A5A5A)
    runs = fill_dev(1, 4, 17)
    hip.reduce_by_key("i32", "u32", d_k, d_v, uniq, agg, runs, n)
    r = int(to_host(runs, np.uint32, 1)[0])
    check_reduce(orc, keys, vals, to_host(uniq, np.int32, r), to_host(agg, np.uint32, r), r, "u32", -1)


def test_large_random_runs(hip, orc, dev):
    """2^26 items with geometric runs (mean 50): scan and reduce bit-exact against the oracle."""
    rng = np.random.default_rng(2024)
    n = 1 << 26
    keys = run_keys(rng, n, 50.0, np.int32)
    vals = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    log("by_key large 2^26")
    check_scan(orc, keys, vals, gpu_scan_by_key(hip, "i32", "u32", keys, vals, False, 0), "u32", False, 0, -1)
    uniq, agg, runs = gpu_reduce_by_key(hip, "i32", "u32", keys, vals)
    check_reduce(orc, keys, vals, uniq, agg, runs, "u32", -1)


def test_temp_too_small_is_an_error(hip, dev):
    n = 10 * TILE
    one = torch.zeros(n, dtype=torch.int32, device=dev)
    temp = torch.empty(4, dtype=torch.int32, device=dev)
    with pytest.raises(hip.LcppHipError) as e:
        hip.scan_by_key("i32", "i32", one, one, one.clone(), n, temp=temp)
    assert e.value.status == hip.ERR_TEMP_TOO_SMALL


@pytest.mark.parametrize("op", ["sum", "max"])
def test_reduce_by_key_runs_sized_outputs_below_inputs(hip, orc, dev, op):
    """Outputs sized to the run count sit directly below the inputs in one allocation, as a caching
    allocator may place them: accepted and exact, on tiles with more runs than the LDS stage (runs of 1-3
    items, so every tile reads its input again after its look-back).  An output whose first item lies
    inside an input overlaps it whatever the run count; such calls are rejected and write nothing."""
    rng = np.random.default_rng(41)
    n = 12 * REDUCE_TILE + 5
    starts = np.zeros(n, bool)
    pos = np.cumsum(rng.integers(1, 4, n))
    starts[pos[pos < n]] = True
    starts[0] = True
    keys = np.cumsum(starts).astype(np.uint32)
    vals = rng.integers(-(1 << 31), 1 << 31, n).astype(np.int32)
    ou, oa = orc.reduce_by_key_int(keys, vals) if op == "sum" else orc.reduce_by_key_minmax(op, keys, vals)
    runs = ou.size
    kbuf = torch.empty(runs + n, dtype=torch.int32, device=dev)
    vbuf = torch.empty(runs + n, dtype=torch.int32, device=dev)
    kbuf[runs:] = to_dev(keys)
    vbuf[runs:] = to_dev(vals)
    d_runs = fill_dev(1, 4, 17)
    log(f"reduce_by_key {op}: runs-sized outputs below the inputs, {runs} runs")
    hip.reduce_by_key("u32", "i32", kbuf[runs:], vbuf[runs:], kbuf[:runs], vbuf[:runs], d_runs, n, op=op)
    assert int(to_host(d_runs, np.uint32, 1)[0]) == runs
    assert np.array_equal(to_host(kbuf[:runs], np.uint32), ou)
    assert np.array_equal(to_host(vbuf[:runs], np.int32), oa)
    assert np.array_equal(to_host(kbuf[runs:], np.uint32), keys)
    assert np.array_equal(to_host(vbuf[runs:], np.int32), vals)
    spare_k, spare_v = fill_dev(n, 4, 7), fill_dev(n, 4, 7)
    d_keys, d_vals = kbuf[runs:], vbuf[runs:]
    for uniq, agg in ((d_keys, spare_v), (spare_k, d_vals), (d_keys[n - 1:], spare_v), (spare_k, d_keys[5:]),
                      (d_vals[1000:], spare_v)):
        with pytest.raises(hip.LcppHipError) as e:
            hip.reduce_by_key("u32", "i32", d_keys, d_vals, uniq, agg, d_runs, n, op=op)
        assert e.value.status == hip.ERR_INVALID_ARGUMENT
    assert np.array_equal(to_host(kbuf[runs:], np.uint32), keys)
    assert np.array_equal(to_host(vbuf[runs:], np.int32), vals)
    assert np.array_equal(to_host(spare_k, np.int32), np.full(n, 7, np.int32))


# ---- min / max operators -----------------------------------------------------------------------------
# ScanByKey / ReduceByKey with MinOp / MaxOp (device_scan.h:424-597, device_reduce.h:437-487): bit-exact
# against the oracle's left-to-right fold for every value type (floats included: the result is one of the
# items or the initial value, and ties of -0.0 / +0.0 keep the older, as the oracle does).
def minmax_values(rng, n, vs):
    dt = np.dtype(NP[vs])
    if dt.kind == "f":
        v = np.round(rng.standard_normal(n) * 100).astype(dt)   # many ties, zeros of both signs
        v[rng.random(n) < 0.3] *= -0.0
        v[rng.random(n) < 0.02] = np.nan
        return v
    info = np.iinfo(dt)
    return rng.integers(info.min, info.max, n, dtype=dt, endpoint=True)


def same_bits(x, y):
    return x.dtype == y.dtype and x.tobytes() == y.tobytes()


@pytest.mark.parametrize("ks", ["i32", "u64"])
@pytest.mark.parametrize("vs", ["i32", "u32", "f32", "i64", "u64", "f64"])
@pytest.mark.parametrize("op", ["min", "max"])
def test_minmax_by_key_vs_oracle(hip, orc, dev, ks, vs, op):
    rng = np.random.default_rng(hash((ks, vs, op)) % 1000)
    n = 5 * TILE + 1234
    keys = run_keys(rng, n, 40.0, NP[ks])
    vals = minmax_values(rng, n, vs)
    log(f"by_key {op} {ks} {vs}")
    for inclusive in (False, True):
        for init in (None, NP[vs](3)):
            got = gpu_scan_by_key(hip, ks, vs, keys, vals, inclusive, init, op=op)
            want = orc.scan_by_key_minmax(op, keys, vals, inclusive, init)
            assert same_bits(got, want), (inclusive, init)
    uniq, agg, runs = gpu_reduce_by_key(hip, ks, vs, keys, vals, op=op)
    ou, oa = orc.reduce_by_key_minmax(op, keys, vals)
    assert runs == ou.size and np.array_equal(uniq, ou) and same_bits(agg, oa)


@pytest.mark.parametrize("op", ["min", "max"])
def test_minmax_by_key_long_runs_and_fallback(hip, orc, dev, op):
    """Runs spanning many tiles (the look-back folds whole windows of predecessors), with every look-back
    taking the fallback (spin limit 0) on the second pass."""
    rng = np.random.default_rng(31)
    n = 120 * TILE + 7
    keys = run_keys(rng, n, 50000.0, np.int32)
    vals = minmax_values(rng, n, "f32")
    lib = hip.lib()
    old = lib.lcpp_hip_get_lookback_spin_limit()
    try:
        for spin in (old, 0):
            lib.lcpp_hip_set_lookback_spin_limit(spin)
            log(f"by_key {op} long runs spin={spin}")
            got = gpu_scan_by_key(hip, "i32", "f32", keys, vals, True, op=op)
            assert same_bits(got, orc.scan_by_key_minmax(op, keys, vals, True))
            uniq, agg, runs = gpu_reduce_by_key(hip, "i32", "f32", keys, vals, op=op)
            ou, oa = orc.reduce_by_key_minmax(op, keys, vals)
            assert runs == ou.size and same_bits(agg, oa)
    finally:
        lib.lcpp_hip_set_lookback_spin_limit(old)


def test_minmax_by_key_staged_and_direct_tiles(hip, orc, dev):
    """Reduce tiles with more runs than the LDS stage (runs of length 1-2) beside staged ones."""
    n = 20 * REDUCE_TILE + 9
    length = 1 + (np.arange(n) // 4096) % 6
    starts = np.zeros(n, bool)
    pos = 0
    while pos < n:
        starts[pos] = True
        pos += int(length[pos])
    keys = np.cumsum(starts).astype(np.uint32)
    vals = minmax_values(np.random.default_rng(2), n, "i64")
    for op in ("min", "max"):
        uniq, agg, runs = gpu_reduce_by_key(hip, "u32", "i64", keys, vals, op=op)
        ou, oa = orc.reduce_by_key_minmax(op, keys, vals)
        assert runs == ou.size and np.array_equal(agg, oa)
