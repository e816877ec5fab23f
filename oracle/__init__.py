"""CPU oracle for the LCPP device hot path — TEST INFRASTRUCTURE ONLY.

Loaded only by tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg, always as the
checker or the timed CPU baseline, never by the product library.  The C sources (``oracle.c``) cite
the reference lines each function restates.  Build: ``make -C oracle``.
"""
from __future__ import annotations

import ctypes as C
import pathlib

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = _HERE / "liblcpp_oracle.so"
_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run `make -C oracle`")
        h = C.CDLL(str(LIB_PATH))
        vp, u64, u32, i32 = C.c_void_p, C.c_uint64, C.c_uint32, C.c_int
        h.oracle_splitmix64_at.restype = u64
        h.oracle_splitmix64_at.argtypes = [u64, u64]
        h.oracle_generate.restype = i32
        h.oracle_generate.argtypes = [i32, vp, u64, u64, u64]
        h.oracle_reduce_sum_i32.restype = C.c_int32
        h.oracle_reduce_sum_i32.argtypes = [vp, u64, C.POINTER(C.c_int64)]
        h.oracle_reduce_sum_u32.restype = u32
        h.oracle_reduce_sum_u32.argtypes = [vp, u64]
        h.oracle_reduce_sum_u64.restype = u64
        h.oracle_reduce_sum_u64.argtypes = [vp, u64]
        h.oracle_reduce_sum_f32.restype = C.c_double
        h.oracle_reduce_sum_f32.argtypes = [vp, u64, C.POINTER(C.c_double)]
        h.oracle_reduce_sum_f64.restype = C.c_double
        h.oracle_reduce_sum_f64.argtypes = [vp, u64, C.POINTER(C.c_double)]
        h.oracle_scan_sum_u32.restype = None
        h.oracle_scan_sum_u32.argtypes = [vp, vp, u64, i32, u32]
        h.oracle_scan_sum_f32.restype = None
        h.oracle_scan_sum_f32.argtypes = [vp, vp, vp, u64, i32, C.c_float]
        h.oracle_twiddle_in.restype = u64
        h.oracle_twiddle_in.argtypes = [u64, i32, i32, i32]
        h.oracle_radix_digit.restype = u32
        h.oracle_radix_digit.argtypes = [u64, i32, i32, i32, u32, u32]
        h.oracle_radix_sort.restype = i32
        h.oracle_radix_sort.argtypes = [vp, vp, vp, vp, u64, i32, i32, i32, u32, u32, i32]
        h.oracle_spmv_csr_fp.restype = None
        h.oracle_spmv_csr_fp.argtypes = [vp, i32, vp, vp, vp, vp, vp, u64, u64, u64]
        h.oracle_spmv_csr_u32.restype = None
        h.oracle_spmv_csr_u32.argtypes = [vp, vp, vp, vp, vp, u64, u64, u64]
        h.oracle_scan_by_key_int.restype = None
        h.oracle_scan_by_key_int.argtypes = [vp, i32, vp, i32, vp, u64, i32, i32, u64, u64]
        h.oracle_scan_by_key_fp.restype = None
        h.oracle_scan_by_key_fp.argtypes = [vp, i32, vp, i32, vp, vp, u64, i32, i32, C.c_double, u64]
        h.oracle_reduce_by_key_int.restype = u64
        h.oracle_reduce_by_key_int.argtypes = [vp, i32, vp, i32, vp, vp, u64, u64]
        h.oracle_reduce_by_key_fp.restype = u64
        h.oracle_reduce_by_key_fp.argtypes = [vp, i32, vp, i32, vp, vp, vp, u64, u64]
        _lib = h
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


GEN_DTYPES = {0: np.uint64, 1: np.uint32, 2: np.int32, 3: np.uint32, 4: np.uint64, 5: np.uint32, 6: np.float32}


def generate(kind: int, n: int, seed: int, start: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=GEN_DTYPES[kind])
    if lib().oracle_generate(kind, _p(out), n, seed, start) != 0:
        raise ValueError(f"bad generator kind {kind}")
    return out


def splitmix64_at(seed: int, index: int) -> int:
    return lib().oracle_splitmix64_at(seed, index)


def reduce_sum_i32(a: np.ndarray) -> tuple[int, int]:
    a = np.ascontiguousarray(a, dtype=np.int32)
    exact = C.c_int64()
    r = lib().oracle_reduce_sum_i32(_p(a), a.size, C.byref(exact))
    return int(r), int(exact.value)


def reduce_sum_u32(a: np.ndarray) -> int:
    a = np.ascontiguousarray(a, dtype=np.uint32)
    return int(lib().oracle_reduce_sum_u32(_p(a), a.size))


def reduce_sum_u64(a: np.ndarray) -> int:
    a = np.ascontiguousarray(a, dtype=np.uint64)
    return int(lib().oracle_reduce_sum_u64(_p(a), a.size))


def reduce_sum_fp(a: np.ndarray) -> tuple[float, float]:
    absum = C.c_double()
    if a.dtype == np.float32:
        a = np.ascontiguousarray(a)
        r = lib().oracle_reduce_sum_f32(_p(a), a.size, C.byref(absum))
    else:
        a = np.ascontiguousarray(a, dtype=np.float64)
        r = lib().oracle_reduce_sum_f64(_p(a), a.size, C.byref(absum))
    return float(r), float(absum.value)


def scan_sum_u32(a: np.ndarray, inclusive: bool = False, init: int = 0) -> np.ndarray:
    """32-bit wrap-around sum scan (int32 inputs are scanned through their bits)."""
    src = np.ascontiguousarray(a).view(np.uint32)
    out = np.empty_like(src)
    lib().oracle_scan_sum_u32(_p(src), _p(out), src.size, int(inclusive), init & 0xFFFFFFFF)
    return out.view(a.dtype)


def scan_sum_f32(a: np.ndarray, inclusive: bool = False, init: float = 0.0) -> tuple[np.ndarray, np.ndarray]:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.size, dtype=np.float64)
    aout = np.empty(a.size, dtype=np.float64)
    lib().oracle_scan_sum_f32(_p(a), _p(out), _p(aout), a.size, int(inclusive), init)
    return out, aout


KEY_KINDS = {np.dtype(np.uint32): (4, 0), np.dtype(np.int32): (4, 1), np.dtype(np.float32): (4, 2),
             np.dtype(np.uint64): (8, 0), np.dtype(np.int64): (8, 1), np.dtype(np.float64): (8, 2)}


def radix_sort(keys: np.ndarray, values: np.ndarray | None = None, begin_bit: int = 0, end_bit: int | None = None,
               descending: bool = False):
    keys = np.ascontiguousarray(keys)
    kb, kind = KEY_KINDS[keys.dtype]
    end_bit = kb * 8 if end_bit is None else end_bit
    ko = np.empty_like(keys)
    vb = 0
    vo = None
    if values is not None:
        values = np.ascontiguousarray(values)
        vb = values.dtype.itemsize
        vo = np.empty_like(values)
    st = lib().oracle_radix_sort(_p(keys), _p(ko), _p(values), _p(vo), keys.size, kb, kind, vb, begin_bit, end_bit,
                                 int(descending))
    if st != 0:
        raise ValueError(f"oracle_radix_sort failed ({st})")
    return (ko, vo) if values is not None else ko


def radix_digit(key: int, dtype, descending: bool, shift: int, bits: int) -> int:
    kb, kind = KEY_KINDS[np.dtype(dtype)]
    return int(lib().oracle_radix_digit(key, kb, kind, int(descending), shift, bits))


def spmv_csr_fp(values, row_offsets, cols_idx, x, rows: int, cols: int, nnz: int):
    values = np.ascontiguousarray(values)
    ro = np.ascontiguousarray(row_offsets).view(np.uint32)
    ci = np.ascontiguousarray(cols_idx).view(np.uint32)
    x = np.ascontiguousarray(x, dtype=values.dtype)
    y = np.empty(rows, dtype=np.float64)
    ay = np.empty(rows, dtype=np.float64)
    lib().oracle_spmv_csr_fp(_p(values), values.dtype.itemsize, _p(ro), _p(ci), _p(x), _p(y), _p(ay), rows, cols, nnz)
    return y, ay


def spmv_csr_u32(values, row_offsets, cols_idx, x, rows: int, cols: int, nnz: int) -> np.ndarray:
    v = np.ascontiguousarray(values).view(np.uint32)
    ro = np.ascontiguousarray(row_offsets).view(np.uint32)
    ci = np.ascontiguousarray(cols_idx).view(np.uint32)
    xx = np.ascontiguousarray(x).view(np.uint32)
    y = np.empty(rows, dtype=np.uint32)
    lib().oracle_spmv_csr_u32(_p(v), _p(ro), _p(ci), _p(xx), _p(y), rows, cols, nnz)
    return y


def _mask(key_mask: int) -> int:
    return key_mask & 0xFFFFFFFFFFFFFFFF


def scan_by_key_int(keys: np.ndarray, values: np.ndarray, inclusive: bool = False, use_init: bool = False,
                    init: int = 0, key_mask: int = -1) -> np.ndarray:
    """Sum scan by key over 4/8-byte integer values, exact modulo 2^bits (oracle.c)."""
    keys, values = np.ascontiguousarray(keys), np.ascontiguousarray(values)
    out = np.empty_like(values)
    lib().oracle_scan_by_key_int(_p(keys), keys.itemsize, _p(values), values.itemsize, _p(out), values.size,
                                 int(inclusive), int(use_init), int(init) & ((1 << (8 * values.itemsize)) - 1),
                                 _mask(key_mask))
    return out


def scan_by_key_fp(keys: np.ndarray, values: np.ndarray, inclusive: bool = False, use_init: bool = False,
                   init: float = 0.0, key_mask: int = -1) -> tuple[np.ndarray, np.ndarray]:
    """Sum scan by key over float/double values in long double: (result, sum of |terms|)."""
    keys, values = np.ascontiguousarray(keys), np.ascontiguousarray(values)
    out = np.empty(values.size, np.float64)
    ab = np.empty(values.size, np.float64)
    lib().oracle_scan_by_key_fp(_p(keys), keys.itemsize, _p(values), values.itemsize, _p(out), _p(ab), values.size,
                                int(inclusive), int(use_init), float(init), _mask(key_mask))
    return out, ab


def reduce_by_key_int(keys: np.ndarray, values: np.ndarray, key_mask: int = -1) -> tuple[np.ndarray, np.ndarray]:
    """(first key of each run, sum of each run) for integer values, exact modulo 2^bits."""
    keys, values = np.ascontiguousarray(keys), np.ascontiguousarray(values)
    uniq = np.empty(max(keys.size, 1), keys.dtype)
    agg = np.empty(max(values.size, 1), values.dtype)
    runs = lib().oracle_reduce_by_key_int(_p(keys), keys.itemsize, _p(values), values.itemsize, _p(uniq), _p(agg),
                                          values.size, _mask(key_mask))
    return uniq[:runs], agg[:runs]


def reduce_by_key_fp(keys: np.ndarray, values: np.ndarray, key_mask: int = -1):
    """(first key of each run, long-double sum of each run, sum of |items| of each run)."""
    keys, values = np.ascontiguousarray(keys), np.ascontiguousarray(values)
    uniq = np.empty(max(keys.size, 1), keys.dtype)
    agg = np.empty(max(values.size, 1), np.float64)
    ab = np.empty(max(values.size, 1), np.float64)
    runs = lib().oracle_reduce_by_key_fp(_p(keys), keys.itemsize, _p(values), values.itemsize, _p(uniq), _p(agg),
                                         _p(ab), values.size, _mask(key_mask))
    return uniq[:runs], agg[:runs], ab[:runs]
