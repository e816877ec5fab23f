"""DeviceSpmv::CsrMV on the GPU: reference known answers (tests/device_spmv_test.cpp:41-203) exactly,
32-bit integer matrices bit-exact against the oracle, and fp32/fp64 within the condition-aware bound
|y - y_exact| <= 1e-5 * max(|y_exact|, sum_j |a_ij x_j|) (fp32) / 1e-12 * (...) (fp64)."""
import numpy as np
import pytest
import torch

from gpu_util import fill_dev, log, to_dev, to_host
from test_oracle import reference_int_csr

pytestmark = pytest.mark.gpu


def gpu_spmv(hip, vs, isfx, va, ro, ci, x, rows, cols, nnz, y_init=0x12345678):
    y = fill_dev(rows, va.dtype.itemsize if va.size else 4, y_init)
    hip.spmv_csr(vs, isfx, to_dev(va) if va.size else None, to_dev(ro), to_dev(ci) if ci.size else None,
                 to_dev(x) if x.size else None, y, rows, cols, nnz)
    return y


def test_int_csr_known_answer(hip, orc, dev):
    va, ro, ci, x, rows, cols, nnz = reference_int_csr()
    y = gpu_spmv(hip, "i32", "i32", va, ro, ci, x, rows, cols, nnz)
    expected = [sum(int(va[i]) * int(x[ci[i]]) for i in range(ro[r], ro[r + 1])) for r in range(rows)]
    assert to_host(y, np.int32, rows).tolist() == expected


def test_float_unsigned_index_known_answer(hip, dev):
    ro = np.array([0, 3, 3, 6, 8], np.uint32)
    ci = np.array([0, 2, 4, 1, 2, 3, 0, 4], np.uint32)
    va = np.array([1.5, -2.0, 0.25, 3.0, 1.25, -0.5, 2.0, 4.0], np.float32)
    x = np.array([2.0, -1.0, 0.5, 3.0, -2.0], np.float32)
    y = to_host(gpu_spmv(hip, "f32", "u32", va, ro, ci, x, 4, 5, 8), np.float32, 4)
    expected = [1.5 * 2 - 2.0 * 0.5 + 0.25 * -2, 0.0, -3.0 + 0.625 - 1.5, 4.0 - 8.0]
    assert np.all(np.abs(y - np.array(expected)) < 1e-5)


def test_empty_and_zero_matrix(hip, dev):
    hip.spmv_csr("f32", "i32", None, None, None, None, None, 0, 0, 0)
    ro = np.zeros(6, np.int32)
    y = torch.full((5,), 42.0, dtype=torch.float32, device=dev)
    hip.spmv_csr("f32", "i32", None, to_dev(ro), None, None, y, 5, 7, 0)
    assert to_host(y, np.float32).tolist() == [0.0] * 5


def random_csr(orc, rows, cols, seed, max_len):
    rng = np.random.default_rng(seed)
    lengths = np.minimum(rng.zipf(1.5, size=rows), max_len).astype(np.int64)
    ro = np.zeros(rows + 1, np.int64)
    ro[1:] = np.cumsum(lengths)
    nnz = int(ro[-1])
    ci = np.concatenate([np.sort(rng.choice(cols, size=int(L), replace=False)) for L in lengths]).astype(np.int32)
    return ro.astype(np.int32), ci, nnz


@pytest.mark.parametrize("vs,dtype,rel", [("f32", np.float32, 1e-5), ("f64", np.float64, 1e-12)])
def test_power_law_rows_within_tolerance(hip, orc, dev, vs, dtype, rel):
    rows, cols = 20000, 5000
    ro, ci, nnz = random_csr(orc, rows, cols, 3, 2000)
    log(f"spmv {vs} nnz={nnz}")
    va = orc.generate(6, nnz, 4).astype(dtype)
    x = orc.generate(6, cols, 5).astype(dtype)
    y = to_host(gpu_spmv(hip, vs, "i32", va, ro, ci, x, rows, cols, nnz), dtype, rows).astype(np.float64)
    ye, ay = orc.spmv_csr_fp(va, ro, ci, x, rows, cols, nnz)
    assert np.all(np.abs(y - ye) <= rel * np.maximum(np.abs(ye), ay))


@pytest.mark.parametrize("isfx", ["i32", "u32"])
def test_integer_values_bit_exact_with_invalid_entries(hip, orc, dev, isfx):
    rows, cols = 5000, 3000
    ro, ci, nnz = random_csr(orc, rows, cols, 8, 700)
    ci = ci.copy()
    ci[::97] = cols + 5          # out-of-range columns are skipped
    ro = ro.copy()
    ro[100] = ro[101] + 1        # row 99 and row 100 get invalid (decreasing) bounds
    va = orc.generate(1, nnz, 9)
    x = orc.generate(1, cols, 10)
    y = gpu_spmv(hip, "u32", isfx, va, ro.view(np.uint32) if isfx == "u32" else ro,
                 ci.view(np.uint32) if isfx == "u32" else ci, x, rows, cols, nnz)
    assert np.array_equal(to_host(y, np.uint32, rows), orc.spmv_csr_u32(va, ro, ci, x, rows, cols, nnz))


def test_benchmark_matrix_zipf_2p20(hip, orc, dev):
    """The SpMV benchmark matrix: 2^20 x 2^20, Zipf(1.5) row lengths in [1, 4096] (about 51.7 M nonzeros),
    distinct sorted columns per row, fp32 values and x in [-1, 1).  y within the condition-aware
    1e-5 bound of the oracle's long-double sums, and bit-identical between two runs."""
    import workloads
    log("spmv zipf 2^20 generate")
    rows = cols = 1 << 20
    va, ro, ci, x, nnz = workloads.zipf_csr(rows, cols, 114521)
    d_va, d_ro, d_ci, d_x = to_dev(va), to_dev(ro), to_dev(ci), to_dev(x)
    y1 = torch.empty(rows, dtype=torch.float32, device=dev)
    y2 = torch.empty(rows, dtype=torch.float32, device=dev)
    log(f"spmv zipf 2^20 nnz={nnz}")
    hip.spmv_csr("f32", "i32", d_va, d_ro, d_ci, d_x, y1, rows, cols, nnz)
    hip.spmv_csr("f32", "i32", d_va, d_ro, d_ci, d_x, y2, rows, cols, nnz)
    got = to_host(y1, np.float32).astype(np.float64)
    assert torch.equal(y1.view(torch.int32), y2.view(torch.int32))
    exact, absum = orc.spmv_csr_fp(va, ro, ci, x, rows, cols, nnz)
    err = np.abs(got - exact)
    bound = 1e-5 * np.maximum(np.abs(exact), absum)
    assert np.all(err <= bound), f"worst ratio {np.max(err / bound)}"


def test_integer_stream_segments_bit_exact(hip, orc, dev):
    """Integer sums are exact in any order, so this pins the nonzero-stream walk: runs of empty rows
    (also at the start and end of a wave's 64 rows), rows of length 1, and rows long enough to span
    several 512-nonzero chunks and lane boundaries."""
    rng = np.random.default_rng(77)
    rows, cols = 6000, 9000
    kind = rng.integers(0, 10, rows)
    lengths = np.where(kind < 3, 0, np.where(kind < 6, 1, rng.integers(2, 40, rows)))
    lengths[rng.integers(0, rows, 25)] = rng.integers(500, 4000, 25)  # multi-chunk rows
    lengths[0:70] = 0              # a fully empty wave and the start of the next one
    lengths[127] = 0
    lengths[128:140] = 1
    lengths[191] = 2000            # a long row as the last row of a wave
    lengths[-5:] = 0               # trailing empty rows
    ro = np.zeros(rows + 1, np.int64)
    ro[1:] = np.cumsum(lengths)
    nnz = int(ro[-1])
    ci = np.concatenate([np.sort(rng.choice(cols, size=int(L), replace=False)) if L else np.zeros(0, np.int64)
                         for L in lengths]).astype(np.uint32)
    ro = ro.astype(np.uint32)
    va = orc.generate(1, nnz, 31)
    x = orc.generate(1, cols, 32)
    log(f"spmv integer stream nnz={nnz}")
    y = gpu_spmv(hip, "u32", "u32", va, ro, ci, x, rows, cols, nnz)
    assert np.array_equal(to_host(y, np.uint32, rows), orc.spmv_csr_u32(va, ro, ci, x, rows, cols, nnz))


@pytest.mark.parametrize("offset_values,offset_columns", [(False, False), (True, True), (True, False), (False, True)])
def test_grouped_long_rows_bit_exact(hip, orc, dev, offset_values, offset_columns):
    """Rows longer than 64 nonzeros stream their columns and values in 16-byte groups when both arrays
    are 16-byte aligned.  Integer sums are exact in any order, so this pins that path: rows whose
    groups start before and end after the row, a last row whose final group crosses nnz (nnz not a
    multiple of the group), and streams passed as views offset by one element (4 bytes), which must
    take the element-wise path."""
    rng = np.random.default_rng(91)
    rows, cols = 3000, 7000
    lengths = np.where(rng.integers(0, 4, rows) == 0, rng.integers(65, 700, rows), rng.integers(0, 70, rows))
    lengths[-1] = 517              # the last row is long and nnz % 8 != 0 below
    ro = np.zeros(rows + 1, np.int64)
    ro[1:] = np.cumsum(lengths)
    nnz = int(ro[-1])
    if nnz % 8 == 0:
        lengths[-1] += 3
        ro[-1] += 3
        nnz += 3
    assert nnz % 8 != 0
    ci = np.concatenate([np.sort(rng.choice(cols, size=int(L), replace=False)) if L else np.zeros(0, np.int64)
                         for L in lengths]).astype(np.uint32)
    ci[::131] = cols + 9           # out-of-range columns are skipped
    ro = ro.astype(np.uint32)
    va = orc.generate(1, nnz, 41)
    x = orc.generate(1, cols, 42)
    log(f"spmv grouped rows nnz={nnz} offsets={offset_values},{offset_columns}")
    d_va = to_dev(np.concatenate([np.array([7], np.uint32), va]))[1:] if offset_values else to_dev(va)
    d_ci = to_dev(np.concatenate([np.array([3], np.uint32), ci]))[1:] if offset_columns else to_dev(ci)
    y = fill_dev(rows, 4, 0x12345678)
    hip.spmv_csr("u32", "u32", d_va, to_dev(ro), d_ci, to_dev(x), y, rows, cols, nnz)
    assert np.array_equal(to_host(y, np.uint32, rows), orc.spmv_csr_u32(va, ro, ci, x, rows, cols, nnz))
