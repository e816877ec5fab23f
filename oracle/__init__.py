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
        i64, i32p = C.c_int64, C.c_int
        h.oracle_par_reduce_sum_i32.restype = i64
        h.oracle_par_reduce_sum_i32.argtypes = [vp, u64, i32p]
        h.oracle_par_scan_sum_u32.restype = None
        h.oracle_par_scan_sum_u32.argtypes = [vp, vp, u64, i32p]
        h.oracle_par_radix_sort_u32.restype = None
        h.oracle_par_radix_sort_u32.argtypes = [vp, vp, u64, i32p]
        h.oracle_std_sort_u32.restype = None
        h.oracle_std_sort_u32.argtypes = [vp, u64]
        h.oracle_par_radix_sort_u64_u32.restype = None
        h.oracle_par_radix_sort_u64_u32.argtypes = [vp, vp, vp, vp, u64, i32p]
        h.oracle_par_spmv_csr_f32.restype = None
        h.oracle_par_spmv_csr_f32.argtypes = [vp, vp, vp, vp, vp, u64, i32p]
        h.oracle_scan_sum_u64.restype = None
        h.oracle_scan_sum_u64.argtypes = [vp, vp, u64, i32, u64]
        h.oracle_scan_sum_f64.restype = None
        h.oracle_scan_sum_f64.argtypes = [vp, vp, vp, u64, i32, C.c_double]
        for name, ct in (("i32", C.c_int32), ("u32", C.c_uint32), ("f32", C.c_float), ("i64", C.c_int64),
                         ("u64", C.c_uint64), ("f64", C.c_double)):
            for op in ("min", "max"):
                f = getattr(h, f"oracle_scan_{op}_{name}")
                f.restype = None
                f.argtypes = [vp, vp, u64, i32, ct]
                f = getattr(h, f"oracle_reduce_{op}_{name}")
                f.restype = ct
                f.argtypes = [vp, u64]
            f = getattr(h, f"oracle_reduce_arg_{name}")
            f.restype = None
            f.argtypes = [vp, u64, i32, C.POINTER(ct), C.POINTER(u32)]
            f = getattr(h, f"oracle_scan_by_key_minmax_{name}")
            f.restype = None
            f.argtypes = [vp, i32, vp, vp, u64, i32, i32, ct, u64, i32]
            f = getattr(h, f"oracle_reduce_by_key_minmax_{name}")
            f.restype = u64
            f.argtypes = [vp, i32, vp, vp, vp, u64, u64, i32]
        for name, ct in (("i32", C.c_int32), ("u32", C.c_uint32), ("f32", C.c_float), ("i64", C.c_int64),
                         ("u64", C.c_uint64), ("f64", C.c_double)):
            f = getattr(h, f"oracle_transform_reduce_{name}")
            f.restype = ct
            f.argtypes = [vp, u64, i32, i32, ct, ct, ct, C.POINTER(C.c_double), C.POINTER(C.c_double)]
        h.oracle_scan_left.restype = i32
        h.oracle_scan_left.argtypes = [vp, vp, u64, i32, i32, i32, u64]
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
        h.oracle_run_heads.restype = None
        h.oracle_run_heads.argtypes = [i32, vp, u64, u64, vp]
        h.oracle_predicate.restype = None
        h.oracle_predicate.argtypes = [i32, vp, u64, vp, vp, vp, vp]
        h.oracle_select.restype = u64
        h.oracle_select.argtypes = [i32, vp, vp, u64, vp, i32]
        h.oracle_partition_three_way.restype = None
        h.oracle_partition_three_way.argtypes = [i32, vp, vp, vp, u64, vp, vp, vp, vp]
        h.oracle_run_length_encode.restype = u64
        h.oracle_run_length_encode.argtypes = [i32, vp, u64, vp, vp]
        h.oracle_non_trivial_runs.restype = u64
        h.oracle_non_trivial_runs.argtypes = [i32, vp, u64, vp, vp]
        h.oracle_segment_reduce.restype = None
        h.oracle_segment_reduce.argtypes = [i32, i32, vp, vp, vp, u64, vp, vp, vp]
        h.oracle_segmented_scan.restype = None
        h.oracle_segmented_scan.argtypes = [i32, vp, vp, vp, vp, u64, i32, i32, u64, C.c_double, vp, vp]
        h.oracle_segmented_sort.restype = i32
        h.oracle_segmented_sort.argtypes = [i32, vp, vp, i32, vp, vp, u64, u64, vp, vp, u32, u32, i32, i32]
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


def scan_sum_u64(a: np.ndarray, inclusive: bool = False, init: int = 0) -> np.ndarray:
    """64-bit wrap-around sum scan (int64 inputs are scanned through their bits)."""
    src = np.ascontiguousarray(a).view(np.uint64)
    out = np.empty_like(src)
    lib().oracle_scan_sum_u64(_p(src), _p(out), src.size, int(inclusive), init & 0xFFFFFFFFFFFFFFFF)
    return out.view(a.dtype)


def scan_sum_f64(a: np.ndarray, inclusive: bool = False, init: float = 0.0) -> tuple[np.ndarray, np.ndarray]:
    """Double scan accumulated in long double: (values, running sums of |x|), both as float64 arrays
    of the long-double results."""
    a = np.ascontiguousarray(a, dtype=np.float64)
    out = np.empty(a.size, dtype=np.longdouble)
    aout = np.empty(a.size, dtype=np.longdouble)
    lib().oracle_scan_sum_f64(_p(a), _p(out), _p(aout), a.size, int(inclusive), init)
    return out, aout


_MINMAX_CTYPE = {np.dtype(np.int32): C.c_int32, np.dtype(np.uint32): C.c_uint32, np.dtype(np.float32): C.c_float,
                 np.dtype(np.int64): C.c_int64, np.dtype(np.uint64): C.c_uint64, np.dtype(np.float64): C.c_double}
_MINMAX_SUFFIX = {np.dtype(np.int32): "i32", np.dtype(np.uint32): "u32", np.dtype(np.float32): "f32",
                  np.dtype(np.int64): "i64", np.dtype(np.uint64): "u64", np.dtype(np.float64): "f64"}


def reduce_minmax(op: str, a: np.ndarray):
    """DeviceReduce::Min / Max: the fold from the type's max / lowest, NaN items skipped."""
    a = np.ascontiguousarray(a)
    return a.dtype.type(getattr(lib(), f"oracle_reduce_{op}_{_MINMAX_SUFFIX[a.dtype]}")(_p(a), a.size))


def reduce_arg(op: str, a: np.ndarray):
    """DeviceReduce::ArgMin / ArgMax: (value, index); first index among equal values, NaN never wins,
    (initial value, 1) for an empty input."""
    a = np.ascontiguousarray(a)
    ct = _MINMAX_CTYPE[a.dtype]
    v, i = ct(), C.c_uint32()
    getattr(lib(), f"oracle_reduce_arg_{_MINMAX_SUFFIX[a.dtype]}")(_p(a), a.size, int(op == "max"), C.byref(v),
                                                                  C.byref(i))
    return a.dtype.type(v.value), int(i.value)


def scan_minmax(op: str, a: np.ndarray, inclusive: bool = False, init=None) -> np.ndarray:
    """Min (op "min") or max ("max") scan in the array's own type; without `init` the operator's identity
    (the type's max / lowest; a quiet NaN for floats, which the NaN-ignoring min / max absorbs) stands in
    for it."""
    a = np.ascontiguousarray(a)
    sfx = _MINMAX_SUFFIX[a.dtype]
    if init is None:
        if a.dtype.kind == "f":
            init = np.nan
        else:
            info = np.iinfo(a.dtype)
            init = info.max if op == "min" else info.min
    out = np.empty_like(a)
    getattr(lib(), f"oracle_scan_{op}_{sfx}")(_p(a), _p(out), a.size, int(inclusive), a.dtype.type(init).item())
    return out


def scan_left(a: np.ndarray, inclusive: bool = True, init=None) -> np.ndarray:
    """Scan with the left projection op(lhs, rhs) = lhs over the items' bits (init, when given, is taken
    in the array's type)."""
    a = np.ascontiguousarray(a)
    u = a.view(f"u{a.itemsize}")
    out = np.empty_like(u)
    bits = 0 if init is None else int(np.array(init, dtype=a.dtype).view(u.dtype))
    if lib().oracle_scan_left(_p(u), _p(out), a.size, a.itemsize, int(inclusive), int(init is not None), bits) != 0:
        raise ValueError("an exclusive left-projection scan needs an initial value")
    return out.view(a.dtype)


REDUCE_OPS = {"sum": 0, "min": 1, "max": 2}
TRANSFORMS = {"identity": 0, "affine": 1, "square": 2, "abs": 3}


def transform_reduce(a: np.ndarray, op: str, transform: str = "identity", scale=0, shift=0, init=0):
    """DeviceReduce::Reduce(op, init) / TransformReduce(op, transform, init): (result in the item type,
    the result as a double (the long-double sum for float sums), the sum of |init| and |transformed items|
    (float sums only, else 0))."""
    a = np.ascontiguousarray(a)
    ct = _MINMAX_CTYPE[a.dtype]
    exact, absum = C.c_double(), C.c_double()
    t = a.dtype.type
    r = getattr(lib(), f"oracle_transform_reduce_{_MINMAX_SUFFIX[a.dtype]}")(
        _p(a), a.size, REDUCE_OPS[op], TRANSFORMS[transform], t(scale).item(), t(shift).item(), t(init).item(),
        C.byref(exact), C.byref(absum))
    return t(r), float(exact.value), float(absum.value)


# ---- host baselines (oracle/cpu_baseline.cpp): `threads` std::threads over contiguous chunks ----------
def par_reduce_sum_i32(a: np.ndarray, threads: int) -> int:
    a = np.ascontiguousarray(a, dtype=np.int32)
    return int(lib().oracle_par_reduce_sum_i32(_p(a), a.size, threads))


def par_scan_sum_u32(a: np.ndarray, threads: int, out: np.ndarray | None = None) -> np.ndarray:
    src = np.ascontiguousarray(a).view(np.uint32)
    out = np.empty_like(src) if out is None else out
    lib().oracle_par_scan_sum_u32(_p(src), _p(out), src.size, threads)
    return out


def par_radix_sort_u32(keys: np.ndarray, threads: int, tmp: np.ndarray | None = None) -> np.ndarray:
    """Sorts `keys` (uint32) in place, stable LSD with 8-bit digits."""
    tmp = np.empty_like(keys) if tmp is None else tmp
    lib().oracle_par_radix_sort_u32(_p(keys), _p(tmp), keys.size, threads)
    return keys


def std_sort_u32(keys: np.ndarray) -> np.ndarray:
    lib().oracle_std_sort_u32(_p(keys), keys.size)
    return keys


def par_radix_sort_u64_u32(keys: np.ndarray, vals: np.ndarray, threads: int, tmp=None):
    """Sorts (keys uint64, vals uint32) in place by key, stable."""
    tk, tv = (np.empty_like(keys), np.empty_like(vals)) if tmp is None else tmp
    lib().oracle_par_radix_sort_u64_u32(_p(keys), _p(vals), _p(tk), _p(tv), keys.size, threads)
    return keys, vals


def par_spmv_csr_f32(values, row_offsets, cols, x, rows: int, threads: int, y: np.ndarray | None = None) -> np.ndarray:
    y = np.empty(rows, np.float32) if y is None else y
    lib().oracle_par_spmv_csr_f32(_p(values), _p(row_offsets), _p(cols), _p(x), _p(y), rows, threads)
    return y


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


def twiddle_in(key: int, dtype, descending: bool = False) -> int:
    """The ordered unsigned image of a key's bits (oracle.c: signed XOR high bit, floats by sign,
    descending inverts)."""
    kb, kind = KEY_KINDS[np.dtype(dtype)]
    return int(lib().oracle_twiddle_in(key, kb, kind, int(descending)))


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


def scan_by_key_minmax(op: str, keys: np.ndarray, values: np.ndarray, inclusive: bool = False, init=None,
                       key_mask: int = -1) -> np.ndarray:
    """Min (op "min") / max ("max") scan by key in the values' own type; without `init` the operator's
    identity (the type's max / lowest, NaN for floats) starts every run."""
    keys, values = np.ascontiguousarray(keys), np.ascontiguousarray(values)
    out = np.empty_like(values)
    sfx = _MINMAX_SUFFIX[values.dtype]
    getattr(lib(), f"oracle_scan_by_key_minmax_{sfx}")(_p(keys), keys.itemsize, _p(values), _p(out), values.size,
                                                       int(inclusive), int(init is not None),
                                                       values.dtype.type(0 if init is None else init).item(),
                                                       _mask(key_mask), int(op == "max"))
    return out


def reduce_by_key_minmax(op: str, keys: np.ndarray, values: np.ndarray, key_mask: int = -1):
    """(first key of each run, min / max of each run)."""
    keys, values = np.ascontiguousarray(keys), np.ascontiguousarray(values)
    uniq = np.empty(max(keys.size, 1), keys.dtype)
    agg = np.empty(max(values.size, 1), values.dtype)
    runs = getattr(lib(), f"oracle_reduce_by_key_minmax_{_MINMAX_SUFFIX[values.dtype]}")(
        _p(keys), keys.itemsize, _p(values), _p(uniq), _p(agg), values.size, _mask(key_mask), int(op == "max"))
    return uniq[:runs], agg[:runs]


# ---- stream compaction (oracle.c: select, partition, run-length encode) -------------------------
_TYPE_CODES = {np.dtype(np.int32): 0, np.dtype(np.uint32): 1, np.dtype(np.float32): 2, np.dtype(np.int64): 3,
               np.dtype(np.uint64): 4, np.dtype(np.float64): 5, np.dtype(np.uint8): 6, np.dtype(np.bool_): 6}


def _code(a: np.ndarray) -> int:
    return _TYPE_CODES[a.dtype]


def _bits_of(value, dtype) -> int:
    """The operand's bits in the item type, as the C-ABI takes them (low bytes of a uint64)."""
    arr = np.array([value], dtype=dtype)
    return int(arr.view({1: np.uint8, 4: np.uint32, 8: np.uint64}[arr.itemsize])[0])


def predicate(x: np.ndarray, clauses) -> np.ndarray:
    """uint8 mask: both clauses hold.  `clauses` = [(op, a, b), (op, a, b)] with values of x's type."""
    x = np.ascontiguousarray(x)
    cl = [tuple(c) + (0,) * (3 - len(c)) for c in clauses] + [(0, 0, 0)] * (2 - len(clauses))
    ops = np.array([c[0] for c in cl], np.int32)
    a = np.array([_bits_of(c[1], x.dtype) for c in cl], np.uint64)
    b = np.array([_bits_of(c[2], x.dtype) for c in cl], np.uint64)
    sel = np.empty(x.size, np.uint8)
    lib().oracle_predicate(_code(x), _p(x), x.size, _p(ops), _p(a), _p(b), _p(sel))
    return sel


def run_heads(x: np.ndarray, key_mask: int = -1) -> np.ndarray:
    x = np.ascontiguousarray(x)
    heads = np.empty(x.size, np.uint8)
    lib().oracle_run_heads(_code(x), _p(x), x.size, _mask(key_mask), _p(heads))
    return heads


def select(x: np.ndarray, sel: np.ndarray, partition: bool = False) -> tuple[np.ndarray, int]:
    """(output of n items, kept count): kept items in order; partition puts rejects reversed at the end."""
    x = np.ascontiguousarray(x)
    sel = np.ascontiguousarray(sel, dtype=np.uint8)
    out = np.zeros_like(x)
    kept = lib().oracle_select(x.itemsize, _p(x), _p(sel), x.size, _p(out), int(partition))
    return out, int(kept)


def partition_three_way(x: np.ndarray, first: np.ndarray, second: np.ndarray):
    """(first_out, second_out, unselected_out, (c1, c2)); outputs are n-sized, written prefixes."""
    x = np.ascontiguousarray(x)
    f = np.ascontiguousarray(first, dtype=np.uint8)
    s = np.ascontiguousarray(second, dtype=np.uint8)
    o1, o2, o3 = np.zeros_like(x), np.zeros_like(x), np.zeros_like(x)
    counts = np.zeros(2, np.uint64)
    lib().oracle_partition_three_way(x.itemsize, _p(x), _p(f), _p(s), x.size, _p(o1), _p(o2), _p(o3), _p(counts))
    return o1, o2, o3, (int(counts[0]), int(counts[1]))


def run_length_encode(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x)
    uniq = np.zeros(max(x.size, 1), x.dtype)
    counts = np.zeros(max(x.size, 1), np.uint32)
    runs = lib().oracle_run_length_encode(_code(x), _p(x), x.size, _p(uniq), _p(counts))
    return uniq[:runs], counts[:runs]


def non_trivial_runs(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x)
    offs = np.zeros(max(x.size, 1), np.uint32)
    lens = np.zeros(max(x.size, 1), np.uint32)
    runs = lib().oracle_non_trivial_runs(_code(x), _p(x), x.size, _p(offs), _p(lens))
    return offs[:runs], lens[:runs]


# ---- segmented reductions and scans (oracle.c) --------------------------------------------------
SEG_OPS = {"sum": 0, "min": 1, "max": 2, "argmin": 3, "argmax": 4}


def segment_reduce(op: str, x: np.ndarray, begins, ends):
    """(out, index or None, sum of |items| or None) per segment."""
    x = np.ascontiguousarray(x)
    b = np.ascontiguousarray(begins, dtype=np.uint32)
    e = np.ascontiguousarray(ends, dtype=np.uint32)
    m = b.size
    out = np.zeros(max(m, 1), x.dtype)
    idx = np.zeros(max(m, 1), np.uint32) if op in ("argmin", "argmax") else None
    ab = np.zeros(max(m, 1), np.float64) if op == "sum" and x.dtype.kind == "f" else None
    lib().oracle_segment_reduce(_code(x), SEG_OPS[op], _p(x), _p(b), _p(e), m, _p(out), _p(idx), _p(ab))
    return out[:m], (idx[:m] if idx is not None else None), (ab[:m] if ab is not None else None)


def segmented_scan(x: np.ndarray, begins, ends, out_begins=None, inclusive=False, init=None, out_size=None):
    """(out, sum of |terms| or None); positions no segment writes hold 0."""
    x = np.ascontiguousarray(x)
    b = np.ascontiguousarray(begins, dtype=np.uint32)
    e = np.ascontiguousarray(ends, dtype=np.uint32)
    ob = b if out_begins is None else np.ascontiguousarray(out_begins, dtype=np.uint32)
    use_init = init is not None
    n_out = out_size if out_size is not None else x.size
    out = np.zeros(max(n_out, 1), x.dtype)
    ab = np.zeros(max(n_out, 1), np.float64) if x.dtype.kind == "f" else None
    init_v = init if use_init else 0
    init_bits = _bits_of(init_v, x.dtype) if x.dtype.kind != "f" else 0
    lib().oracle_segmented_scan(_code(x), _p(x), _p(b), _p(e), _p(ob), b.size, int(inclusive), int(use_init),
                                init_bits, float(init_v), _p(out), _p(ab))
    return out[:n_out], (ab[:n_out] if ab is not None else None)


def segmented_sort(keys: np.ndarray, begins, ends, values: np.ndarray | None = None, begin_bit: int = 0,
                   end_bit: int | None = None, descending: bool = False, value_order: bool = False,
                   keys_out: np.ndarray | None = None, values_out: np.ndarray | None = None):
    """Stable per-segment sort (oracle.c).  Items outside every segment keep keys_out / values_out
    (copies of the inputs unless given)."""
    keys = np.ascontiguousarray(keys)
    b = np.ascontiguousarray(begins, dtype=np.uint32)
    e = np.ascontiguousarray(ends, dtype=np.uint32)
    ko = keys.copy() if keys_out is None else np.ascontiguousarray(keys_out).copy()
    vin = None if values is None else np.ascontiguousarray(values)
    vo = None if vin is None else (vin.copy() if values_out is None else np.ascontiguousarray(values_out).copy())
    end_bit = keys.itemsize * 8 if end_bit is None else end_bit
    rc = lib().oracle_segmented_sort(_code(keys), _p(keys), _p(ko), 0 if vin is None else vin.itemsize, _p(vin),
                                     _p(vo), keys.size, b.size, _p(b), _p(e), begin_bit, end_bit, int(descending),
                                     int(value_order))
    if rc != 0:
        raise MemoryError("oracle_segmented_sort")
    return ko, vo
