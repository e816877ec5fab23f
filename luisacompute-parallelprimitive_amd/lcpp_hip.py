"""ctypes binding of ``liblcpp_hip.so`` (the C-ABI declared in ``include/lcpp_hip.h``).

Device memory and streams come from PyTorch (``tensor.data_ptr()``, ``torch.cuda.current_stream()``);
every call goes straight to the HIP library.  There is no CPU fallback: if the library cannot be
loaded, :func:`lib` raises.

The operation names follow the reference API (``DeviceReduce::Sum``, ``DeviceScan::ExclusiveSum``,
``DeviceRadixSort::SortKeys/SortPairs``, ``DeviceSpmv::CsrMV``, ``DeviceScan::*SumByKey``,
``DeviceReduce::ReduceByKey``, ``DeviceSelect``, ``DevicePartition``, ``DeviceRunLengthEncode``;
src/lcpp/device/*.h) and the
temp-storage queries return the reference's ``Get*TempStorageBytes`` values.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib

_HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = _HERE / "liblcpp_hip.so"

OK = 0
ERR_INVALID_ARGUMENT = -1
ERR_TEMP_TOO_SMALL = -2
ERR_HIP = -3
ERR_UNSUPPORTED = -4

GEN_U64, GEN_U32_HI, GEN_I32_PM1000, GEN_U32_LT16, GEN_U64_AND3, GEN_U32_IOTA, GEN_F32_PM1 = range(7)

SCALAR_SUFFIXES = ("i32", "u32", "f32", "i64", "u64", "f64")
SCAN_SUFFIXES = SCALAR_SUFFIXES
ARG_SUFFIXES = ("i32", "u32", "f32")  # segment ArgMin / ArgMax item types
SORT_KEY_SUFFIXES = ("u32", "i32", "f32", "u64", "i64", "f64")
SPMV_SUFFIXES = [(v, i) for v in ("f32", "f64", "i32", "u32") for i in ("i32", "u32")]
BY_KEY_KEY_SUFFIXES = ("i32", "u32", "i64", "u64")
BY_KEY_VALUE_SUFFIXES = SCALAR_SUFFIXES
FLAG_SUFFIXES = ("b8", "i32", "u32", "i64", "u64")

# Predicate clause ops (include/lcpp_hip.h LCPP_HIP_PRED_*).
(PRED_TRUE, PRED_LT, PRED_LE, PRED_GT, PRED_GE, PRED_EQ, PRED_NE, PRED_RANGE, PRED_MASK_EQ, PRED_MASK_NE,
 PRED_MOD_EQ, PRED_MOD_NE) = range(12)


class Predicate(C.Structure):
    """lcpp_hip_predicate: two clauses that must both hold; operands are bits of the item type."""
    _fields_ = [("op", C.c_int32 * 2), ("a", C.c_uint64 * 2), ("b", C.c_uint64 * 2)]

_CTYPE = {
    "i32": C.c_int32, "u32": C.c_uint32, "f32": C.c_float,
    "i64": C.c_int64, "u64": C.c_uint64, "f64": C.c_double,
}
ELEM_BYTES = {"i32": 4, "u32": 4, "f32": 4, "i64": 8, "u64": 8, "f64": 8}
_NP_DTYPE = {"i32": "int32", "u32": "uint32", "f32": "float32", "i64": "int64", "u64": "uint64", "f64": "float64",
             "b8": "uint8"}


class LcppHipError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"lcpp_hip status {status}: {message}")
        self.status = status


_lib = None


def _declare(lib: C.CDLL) -> None:
    vp, sz, u64, u32, i32 = C.c_void_p, C.c_size_t, C.c_uint64, C.c_uint32, C.c_int

    def sig(name, res, *args):
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = list(args)

    sig("lcpp_hip_version", C.c_char_p)
    sig("lcpp_hip_last_error", C.c_char_p)
    sig("lcpp_hip_profile_enable", i32, i32)
    sig("lcpp_hip_profile_reset", i32)
    sig("lcpp_hip_profile_query", i32, C.c_char_p, C.POINTER(C.c_double), C.POINTER(C.c_uint64))
    sig("lcpp_hip_profile_names", i32, C.c_char_p, sz)
    sig("lcpp_hip_device_copy", i32, vp, vp, u64, vp)
    sig("lcpp_hip_scan_exclusive_sum_u32_noalloc", i32, vp, vp, u64, vp)
    sig("lcpp_hip_internal_segsort_slot_kind", i32, vp)
    sig("lcpp_hip_reduce_temp_bytes_policy", sz, u64, sz, u32, u32)
    sig("lcpp_hip_reduce_temp_bytes", sz, u64, sz)
    sig("lcpp_hip_scan_temp_bytes_policy", sz, u64, sz, u32, u32, i32, i32)
    sig("lcpp_hip_scan_temp_bytes", sz, u64, sz)
    sig("lcpp_hip_radix_sort_temp_bytes_policy", sz, u32, sz, sz, i32, u32, u32, i32)
    sig("lcpp_hip_radix_sort_keys_temp_bytes", sz, u32, sz)
    sig("lcpp_hip_radix_sort_pairs_temp_bytes", sz, u32, sz, sz)
    sig("lcpp_hip_spmv_temp_bytes", sz, u64, u64, u64)
    sig("lcpp_hip_radix_set_portion_limit", i32, u32)
    sig("lcpp_hip_set_lookback_spin_limit", i32, u32)
    sig("lcpp_hip_get_lookback_spin_limit", u32)
    sig("lcpp_hip_radix_tile_items", u32, sz, sz)
    sig("lcpp_hip_internal_scan_needed_bytes", sz, u64, sz)
    sig("lcpp_hip_internal_radix_needed_bytes", sz, u32, sz, sz, u32, u32, i32)
    sig("lcpp_hip_internal_radix_portions", u32, u32, sz, sz, u32, u32, i32, sz)
    sig("lcpp_hip_internal_radix_rank_mode", i32, i32)
    sig("lcpp_hip_internal_radix_precount", i32, i32)
    sig("lcpp_hip_generate", i32, i32, vp, u64, u64, u64, vp)
    for s in SCALAR_SUFFIXES:
        sig(f"lcpp_hip_reduce_sum_{s}", i32, vp, sz, vp, vp, u64, vp)
        for op in ("min", "max"):
            sig(f"lcpp_hip_reduce_{op}_{s}", i32, vp, sz, vp, vp, u64, vp)
            sig(f"lcpp_hip_reduce_arg{op}_{s}", i32, vp, sz, vp, vp, vp, u64, vp)
        sig(f"lcpp_hip_reduce_op_{s}", i32, vp, sz, vp, vp, u64, i32, _CTYPE[s], vp)
        sig(f"lcpp_hip_transform_reduce_{s}", i32, vp, sz, vp, vp, u64, i32, i32, _CTYPE[s], _CTYPE[s], _CTYPE[s], vp)
    sig("lcpp_hip_reduce_arg_temp_bytes", sz, u64, sz)
    for s in SCAN_SUFFIXES:
        sig(f"lcpp_hip_scan_exclusive_sum_{s}", i32, vp, sz, vp, vp, u64, vp)
        sig(f"lcpp_hip_scan_inclusive_sum_{s}", i32, vp, sz, vp, vp, u64, vp)
        sig(f"lcpp_hip_scan_sum_init_{s}", i32, vp, sz, vp, vp, u64, i32, _CTYPE[s], vp)
        for op in ("min", "max", "left"):
            sig(f"lcpp_hip_scan_{op}_{s}", i32, vp, sz, vp, vp, u64, i32, i32, _CTYPE[s], vp)
    for k in SORT_KEY_SUFFIXES:
        sig(f"lcpp_hip_radix_sort_keys_{k}", i32, vp, sz, vp, vp, u32, u32, u32, i32, vp)
        sig(f"lcpp_hip_radix_sort_keys_db_{k}", i32, vp, sz, vp, vp, C.POINTER(C.c_int), u32, u32, u32, i32, vp)
        for v in ("v32", "v64"):
            sig(f"lcpp_hip_radix_sort_pairs_{k}_{v}", i32, vp, sz, vp, vp, vp, vp, u32, u32, u32, i32, vp)
            sig(f"lcpp_hip_radix_sort_pairs_db_{k}_{v}", i32, vp, sz, vp, vp, vp, vp, C.POINTER(C.c_int), u32, u32,
                u32, i32, vp)
    for v, i in SPMV_SUFFIXES:
        sig(f"lcpp_hip_spmv_csr_{v}_{i}", i32, vp, sz, vp, vp, vp, vp, vp, u64, u64, u64, vp)
    sig("lcpp_hip_scan_by_key_temp_bytes", sz, u64, sz, sz)
    sig("lcpp_hip_reduce_by_key_temp_bytes", sz, u64, sz, sz)
    sig("lcpp_hip_scan_by_key_temp_bytes_policy", sz, u64, sz, sz, u32, u32)
    sig("lcpp_hip_reduce_by_key_temp_bytes_policy", sz, u64, sz, sz, u32)
    sig("lcpp_hip_internal_by_key_needed_bytes", sz, u64, sz)
    for k in BY_KEY_KEY_SUFFIXES:
        for v in BY_KEY_VALUE_SUFFIXES:
            for op in ("sum", "min", "max"):
                sig(f"lcpp_hip_scan_by_key_{op}_{k}_{v}", i32, vp, sz, vp, vp, vp, u64, i32, i32, _CTYPE[v], u64, vp)
                sig(f"lcpp_hip_reduce_by_key_{op}_{k}_{v}", i32, vp, sz, vp, vp, vp, vp, vp, u64, u64, vp)
    sig("lcpp_hip_segment_reduce_temp_bytes", sz, u64)
    sig("lcpp_hip_segment_reduce_arg_temp_bytes", sz, u64, u64)
    sig("lcpp_hip_segmented_scan_temp_bytes", sz, u64, u64)
    for t in SCALAR_SUFFIXES:
        for op in ("sum", "min", "max"):
            sig(f"lcpp_hip_segment_reduce_{op}_{t}", i32, vp, sz, vp, vp, u64, vp, vp, vp)
            sig(f"lcpp_hip_segment_reduce_fixed_{op}_{t}", i32, vp, sz, vp, vp, u64, u32, vp)
        sig(f"lcpp_hip_segmented_scan_sum_{t}", i32, vp, sz, vp, vp, vp, vp, vp, u64, i32, i32, _CTYPE[t], vp)
    for t in ARG_SUFFIXES:
        for op in ("argmin", "argmax"):
            sig(f"lcpp_hip_segment_{op}_{t}", i32, vp, sz, vp, vp, vp, u64, vp, vp, vp)
            sig(f"lcpp_hip_segment_fixed_{op}_{t}", i32, vp, sz, vp, vp, vp, u64, u32, vp)
    sig("lcpp_hip_segmented_sort_keys_temp_bytes", sz, u64, sz)
    sig("lcpp_hip_segmented_sort_pairs_temp_bytes", sz, u64, sz, sz)
    ip = C.POINTER(C.c_int)
    for k in SORT_KEY_SUFFIXES:
        sig(f"lcpp_hip_segmented_sort_keys_{k}", i32, vp, sz, vp, vp, u64, u64, vp, vp, u32, u32, i32, i32, vp)
        sig(f"lcpp_hip_segmented_sort_keys_db_{k}", i32, vp, vp, ip, u64, u64, vp, vp, u32, u32, i32, i32, vp)
        for v in ("v32", "v64"):
            sig(f"lcpp_hip_segmented_sort_pairs_{k}_{v}", i32, vp, sz, vp, vp, vp, vp, u64, u64, vp, vp, u32, u32,
                i32, i32, vp)
            sig(f"lcpp_hip_segmented_sort_pairs_db_{k}_{v}", i32, vp, vp, ip, vp, vp, ip, u64, u64, vp, vp, u32, u32,
                i32, i32, vp)
    pp = C.POINTER(Predicate)
    for name in ("select", "partition_three_way", "run_length_encode"):
        sig(f"lcpp_hip_{name}_temp_bytes", sz, u64)
        sig(f"lcpp_hip_{name}_temp_bytes_policy", sz, u64, u32, u32)
    sig("lcpp_hip_internal_compact_needed_bytes", sz, u64, sz, i32, i32)
    sig("lcpp_hip_internal_compact_rows", i32, i32)
    for t in SCALAR_SUFFIXES:
        sig(f"lcpp_hip_select_if_{t}", i32, vp, sz, vp, vp, vp, u64, pp, vp)
        sig(f"lcpp_hip_partition_if_{t}", i32, vp, sz, vp, vp, vp, u64, pp, vp)
        sig(f"lcpp_hip_partition_three_way_{t}", i32, vp, sz, vp, vp, vp, vp, vp, u64, pp, pp, vp)
        sig(f"lcpp_hip_select_unique_{t}", i32, vp, sz, vp, vp, vp, u64, u64, vp)
        sig(f"lcpp_hip_run_length_encode_{t}", i32, vp, sz, vp, vp, vp, vp, u64, vp)
        sig(f"lcpp_hip_run_length_non_trivial_{t}", i32, vp, sz, vp, vp, vp, vp, u64, vp)
        for f in FLAG_SUFFIXES:
            sig(f"lcpp_hip_select_flagged_{t}_{f}", i32, vp, sz, vp, vp, vp, vp, u64, vp)
            sig(f"lcpp_hip_select_flagged_if_{t}_{f}", i32, vp, sz, vp, vp, vp, vp, u64, pp, vp)
            sig(f"lcpp_hip_partition_flagged_{t}_{f}", i32, vp, sz, vp, vp, vp, vp, u64, vp)
        for v in SCALAR_SUFFIXES:
            sig(f"lcpp_hip_select_unique_by_key_{t}_{v}", i32, vp, sz, vp, vp, vp, vp, vp, u64, u64, vp)


def lib() -> C.CDLL:
    """Loads liblcpp_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run `python luisacompute-parallelprimitive_amd/build.py`")
        handle = C.CDLL(str(LIB_PATH), mode=os.RTLD_GLOBAL if hasattr(os, "RTLD_GLOBAL") else 0)
        _declare(handle)
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != OK:
        raise LcppHipError(status, lib().lcpp_hip_last_error().decode(errors="replace"))


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


def ptr(t) -> int | None:
    """Device address of a torch tensor (None for an absent buffer)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_handle(stream=None) -> int | None:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


# ---- temp-storage queries (reference Get*TempStorageBytes) --------------------------------------
def reduce_temp_bytes(n: int, elem_bytes: int, block: int = 256, items: int = 8) -> int:
    return lib().lcpp_hip_reduce_temp_bytes_policy(n, elem_bytes, block, items)


def scan_temp_bytes(n: int, elem_bytes: int) -> int:
    return lib().lcpp_hip_scan_temp_bytes(n, elem_bytes)


def sort_keys_temp_bytes(n: int, key_bytes: int) -> int:
    return lib().lcpp_hip_radix_sort_keys_temp_bytes(n, key_bytes)


def sort_pairs_temp_bytes(n: int, key_bytes: int, value_bytes: int) -> int:
    return lib().lcpp_hip_radix_sort_pairs_temp_bytes(n, key_bytes, value_bytes)


def scan_by_key_temp_bytes(n: int, key_bytes: int, value_bytes: int) -> int:
    return lib().lcpp_hip_scan_by_key_temp_bytes(n, key_bytes, value_bytes)


def reduce_by_key_temp_bytes(n: int, key_bytes: int, value_bytes: int) -> int:
    return lib().lcpp_hip_reduce_by_key_temp_bytes(n, key_bytes, value_bytes)


def bytes_to_uint_count(nbytes: int) -> int:
    return (nbytes + 3) // 4


# ---- operations on torch tensors ----------------------------------------------------------------
def _temp(nbytes: int, device):
    import torch
    return torch.empty(max(1, bytes_to_uint_count(nbytes)), dtype=torch.int32, device=device)


def reduce_sum(suffix: str, d_in, d_out, n: int, temp=None, stream=None) -> None:
    """DeviceReduce::Sum over d_in[0:n) into d_out[0]."""
    if temp is None:
        temp = _temp(reduce_temp_bytes(n, ELEM_BYTES[suffix]), d_in.device)
    call(f"lcpp_hip_reduce_sum_{suffix}", ptr(temp), temp.numel() * temp.element_size(), ptr(d_in), ptr(d_out), n,
         stream_handle(stream))


REDUCE_OPS = {"sum": 0, "min": 1, "max": 2}  # LCPP_HIP_REDUCE_*
TRANSFORMS = {"identity": 0, "affine": 1, "square": 2, "abs": 3}  # LCPP_HIP_TRANSFORM_*


def reduce_op(op: str, suffix: str, d_in, d_out, n: int, init=0, temp=None, stream=None) -> None:
    """DeviceReduce::Reduce(op, init) with op "sum", "min" or "max": op(init, fold of the items) into d_out[0]."""
    if temp is None:
        temp = _temp(reduce_temp_bytes(n, ELEM_BYTES[suffix]), d_in.device)
    call(f"lcpp_hip_reduce_op_{suffix}", ptr(temp), temp.numel() * temp.element_size(), ptr(d_in), ptr(d_out), n,
         REDUCE_OPS[op], _CTYPE[suffix](init), stream_handle(stream))


def transform_reduce(op: str, transform: str, suffix: str, d_in, d_out, n: int, scale=0, shift=0, init=0, temp=None,
                     stream=None) -> None:
    """DeviceReduce::TransformReduce(op, transform, init): transform "identity", "affine" (scale * x + shift),
    "square" or "abs" applied to every item, then op(init, fold) into d_out[0]."""
    if temp is None:
        temp = _temp(reduce_temp_bytes(n, ELEM_BYTES[suffix]), d_in.device)
    ct = _CTYPE[suffix]
    call(f"lcpp_hip_transform_reduce_{suffix}", ptr(temp), temp.numel() * temp.element_size(), ptr(d_in), ptr(d_out),
         n, REDUCE_OPS[op], TRANSFORMS[transform], ct(scale), ct(shift), ct(init), stream_handle(stream))


def reduce_arg_temp_bytes(n: int, elem_bytes: int) -> int:
    return lib().lcpp_hip_reduce_arg_temp_bytes(n, elem_bytes)


def reduce_minmax(op: str, suffix: str, d_in, d_out, n: int, temp=None, stream=None) -> None:
    """DeviceReduce::Min (op "min") or Max ("max") over d_in[0:n) into d_out[0]."""
    if op not in ("min", "max"):
        raise ValueError(f"reduce operator {op!r}: min or max")
    if temp is None:
        temp = _temp(reduce_temp_bytes(n, ELEM_BYTES[suffix]), d_in.device)
    call(f"lcpp_hip_reduce_{op}_{suffix}", ptr(temp), temp.numel() * temp.element_size(), ptr(d_in), ptr(d_out), n,
         stream_handle(stream))


def reduce_arg(op: str, suffix: str, d_in, d_value, d_index, n: int, temp=None, stream=None) -> None:
    """DeviceReduce::ArgMin (op "min") or ArgMax ("max"): the extreme item into d_value[0], its index
    (uint32) into d_index[0]."""
    if op not in ("min", "max"):
        raise ValueError(f"reduce operator {op!r}: min or max")
    if temp is None:
        temp = _temp(reduce_arg_temp_bytes(n, ELEM_BYTES[suffix]), d_in.device)
    call(f"lcpp_hip_reduce_arg{op}_{suffix}", ptr(temp), temp.numel() * temp.element_size(), ptr(d_in),
         ptr(d_value), ptr(d_index), n, stream_handle(stream))


def scan_sum(suffix: str, d_in, d_out, n: int, inclusive: bool = False, init=None, temp=None, stream=None) -> None:
    """DeviceScan::ExclusiveSum / InclusiveSum (optionally with an initial value)."""
    if temp is None:
        temp = _temp(scan_temp_bytes(n, ELEM_BYTES[suffix]), d_in.device)
    tb = temp.numel() * temp.element_size()
    if init is None:
        kind = "inclusive" if inclusive else "exclusive"
        call(f"lcpp_hip_scan_{kind}_sum_{suffix}", ptr(temp), tb, ptr(d_in), ptr(d_out), n, stream_handle(stream))
    else:
        call(f"lcpp_hip_scan_sum_init_{suffix}", ptr(temp), tb, ptr(d_in), ptr(d_out), n, int(inclusive),
             _CTYPE[suffix](init), stream_handle(stream))


def scan_minmax(op: str, suffix: str, d_in, d_out, n: int, inclusive: bool = False, init=None, temp=None,
                stream=None) -> None:
    """DeviceScan::ExclusiveScan / InclusiveScan with MinOp (op "min"), MaxOp ("max") or the left projection
    ("left", lhs of every pair); without `init` the operator's identity stands in for it (the left projection
    has none and takes in[0])."""
    if op not in ("min", "max", "left"):
        raise ValueError(f"scan operator {op!r}: min, max or left")
    if temp is None:
        temp = _temp(scan_temp_bytes(n, ELEM_BYTES[suffix]), d_in.device)
    tb = temp.numel() * temp.element_size()
    call(f"lcpp_hip_scan_{op}_{suffix}", ptr(temp), tb, ptr(d_in), ptr(d_out), n, int(inclusive),
         int(init is not None), _CTYPE[suffix](0 if init is None else init), stream_handle(stream))


def device_copy(dst, src, nbytes: int, stream=None) -> None:
    """Device-to-device copy by the library's copy kernel."""
    call("lcpp_hip_device_copy", ptr(dst), ptr(src), nbytes, stream_handle(stream))


def sort_keys(key_suffix: str, keys_in, keys_out, n: int, begin_bit: int = 0, end_bit: int | None = None,
              descending: bool = False, temp=None, stream=None) -> None:
    """DeviceRadixSort::SortKeys / SortKeysDescending (copy form)."""
    kb = ELEM_BYTES[key_suffix]
    end_bit = kb * 8 if end_bit is None else end_bit
    if temp is None:
        temp = _temp(sort_keys_temp_bytes(n, kb), keys_in.device)
    call(f"lcpp_hip_radix_sort_keys_{key_suffix}", ptr(temp), temp.numel() * temp.element_size(), ptr(keys_in),
         ptr(keys_out), n, begin_bit, end_bit, int(descending), stream_handle(stream))


def sort_pairs(key_suffix: str, value_bytes: int, keys_in, keys_out, values_in, values_out, n: int,
               begin_bit: int = 0, end_bit: int | None = None, descending: bool = False, temp=None,
               stream=None) -> None:
    """DeviceRadixSort::SortPairs / SortPairsDescending (copy form)."""
    kb = ELEM_BYTES[key_suffix]
    end_bit = kb * 8 if end_bit is None else end_bit
    if temp is None:
        temp = _temp(sort_pairs_temp_bytes(n, kb, value_bytes), keys_in.device)
    v = "v32" if value_bytes == 4 else "v64"
    call(f"lcpp_hip_radix_sort_pairs_{key_suffix}_{v}", ptr(temp), temp.numel() * temp.element_size(), ptr(keys_in),
         ptr(keys_out), ptr(values_in), ptr(values_out), n, begin_bit, end_bit, int(descending),
         stream_handle(stream))


def sort_keys_db(key_suffix: str, buf0, buf1, selector: int, n: int, begin_bit: int = 0, end_bit: int | None = None,
                 descending: bool = False, temp=None, stream=None) -> int:
    """DeviceRadixSort::SortKeys(DoubleBuffer); returns the updated selector."""
    kb = ELEM_BYTES[key_suffix]
    end_bit = kb * 8 if end_bit is None else end_bit
    if temp is None:
        temp = _temp(sort_keys_temp_bytes(n, kb), buf0.device)
    sel = C.c_int(selector)
    call(f"lcpp_hip_radix_sort_keys_db_{key_suffix}", ptr(temp), temp.numel() * temp.element_size(), ptr(buf0),
         ptr(buf1), C.byref(sel), n, begin_bit, end_bit, int(descending), stream_handle(stream))
    return sel.value


def sort_pairs_db(key_suffix: str, value_bytes: int, k0, k1, v0, v1, selector: int, n: int, begin_bit: int = 0,
                  end_bit: int | None = None, descending: bool = False, temp=None, stream=None) -> int:
    """DeviceRadixSort::SortPairs(DoubleBuffer, DoubleBuffer); returns the updated selector."""
    kb = ELEM_BYTES[key_suffix]
    end_bit = kb * 8 if end_bit is None else end_bit
    if temp is None:
        temp = _temp(sort_pairs_temp_bytes(n, kb, value_bytes), k0.device)
    sel = C.c_int(selector)
    v = "v32" if value_bytes == 4 else "v64"
    call(f"lcpp_hip_radix_sort_pairs_db_{key_suffix}_{v}", ptr(temp), temp.numel() * temp.element_size(), ptr(k0),
         ptr(k1), ptr(v0), ptr(v1), C.byref(sel), n, begin_bit, end_bit, int(descending), stream_handle(stream))
    return sel.value


def spmv_csr(value_suffix: str, index_suffix: str, values, row_offsets, column_indices, x, y, rows: int, cols: int,
             nnz: int, stream=None) -> None:
    """DeviceSpmv::CsrMV: y = A x (temp storage: 0 bytes)."""
    call(f"lcpp_hip_spmv_csr_{value_suffix}_{index_suffix}", None, 0, ptr(values), ptr(row_offsets),
         ptr(column_indices), ptr(x), ptr(y), rows, cols, nnz, stream_handle(stream))


def generate(kind: int, out, n: int, seed: int, start: int = 0, stream=None) -> None:
    call("lcpp_hip_generate", kind, ptr(out), n, seed, start, stream_handle(stream))


# ---- per-kernel device time ---------------------------------------------------------------------
def profile_enable(on: bool = True) -> None:
    check(lib().lcpp_hip_profile_enable(int(on)))


def profile_reset() -> None:
    check(lib().lcpp_hip_profile_reset())


def profile_query(kernel: str) -> tuple[float, int]:
    ms, cnt = C.c_double(), C.c_uint64()
    check(lib().lcpp_hip_profile_query(kernel.encode(), C.byref(ms), C.byref(cnt)))
    return ms.value, cnt.value


def scan_by_key(key_suffix: str, value_suffix: str, keys, values_in, values_out, n: int, inclusive: bool = False,
                init=None, key_mask: int = -1, temp=None, stream=None, op: str = "sum") -> None:
    """DeviceScan::ExclusiveSumByKey / InclusiveSumByKey (op "sum"), or ExclusiveScanByKey / InclusiveScanByKey
    with MinOp ("min") or MaxOp ("max"); `init` as in the overloads with an initial value; keys equal when
    ((a ^ b) & key_mask) == 0."""
    if op not in ("sum", "min", "max"):
        raise ValueError(f"by-key operator {op!r}: sum, min or max")
    if temp is None:
        temp = _temp(scan_by_key_temp_bytes(n, ELEM_BYTES[key_suffix], ELEM_BYTES[value_suffix]), values_in.device)
    use_init = init is not None
    call(f"lcpp_hip_scan_by_key_{op}_{key_suffix}_{value_suffix}", ptr(temp), temp.numel() * temp.element_size(),
         ptr(keys), ptr(values_in), ptr(values_out), n, int(inclusive), int(use_init),
         _CTYPE[value_suffix](init if use_init else 0), key_mask & 0xFFFFFFFFFFFFFFFF, stream_handle(stream))


def reduce_by_key(key_suffix: str, value_suffix: str, keys, values, unique_out, aggregates_out, num_runs_out,
                  n: int, key_mask: int = -1, temp=None, stream=None, op: str = "sum") -> None:
    """DeviceReduce::ReduceByKey with SumOp (op "sum"), MinOp ("min") or MaxOp ("max"): first key and
    aggregate of each run, and the run count."""
    if op not in ("sum", "min", "max"):
        raise ValueError(f"by-key operator {op!r}: sum, min or max")
    if temp is None:
        temp = _temp(reduce_by_key_temp_bytes(n, ELEM_BYTES[key_suffix], ELEM_BYTES[value_suffix]),
                     num_runs_out.device)
    call(f"lcpp_hip_reduce_by_key_{op}_{key_suffix}_{value_suffix}", ptr(temp), temp.numel() * temp.element_size(),
         ptr(keys), ptr(values), ptr(unique_out), ptr(aggregates_out), ptr(num_runs_out), n,
         key_mask & 0xFFFFFFFFFFFFFFFF, stream_handle(stream))


# ---- stream compaction (DeviceSelect, DevicePartition, DeviceRunLengthEncode) -------------------
def operand_bits(value, suffix: str) -> int:
    """Bits of `value` as an item of type `suffix`, in the low bytes (how the C-ABI takes operands)."""
    import numpy as np
    arr = np.array([value], dtype=_NP_DTYPE[suffix])
    return int(arr.view({1: np.uint8, 4: np.uint32, 8: np.uint64}[arr.itemsize])[0])


def predicate(suffix: str, *clauses) -> Predicate:
    """Predicate from up to two (op, a[, b]) clauses with operands given as values of type `suffix`."""
    p = Predicate()
    for c in range(2):
        op, a, b = (tuple(clauses[c]) + (0, 0))[:3] if c < len(clauses) else (PRED_TRUE, 0, 0)
        p.op[c] = op
        p.a[c] = operand_bits(a, suffix)
        p.b[c] = operand_bits(b, suffix)
    return p


def select_temp_bytes(n: int, block: int = 256, items: int = 4) -> int:
    return lib().lcpp_hip_select_temp_bytes_policy(n, block, items)


def partition_three_way_temp_bytes(n: int, block: int = 256, items: int = 4) -> int:
    return lib().lcpp_hip_partition_three_way_temp_bytes_policy(n, block, items)


def run_length_encode_temp_bytes(n: int, block: int = 256, items: int = 4) -> int:
    return lib().lcpp_hip_run_length_encode_temp_bytes_policy(n, block, items)


def _temp_for(nbytes: int, like, temp):
    if temp is not None:
        return temp
    return _temp(nbytes, like.device)


def _tb(temp) -> int:
    return temp.numel() * temp.element_size()


def select_flagged(suffix: str, flag_suffix: str, d_in, flags, d_out, num_out, n: int, temp=None, stream=None):
    """DeviceSelect::Flagged: items whose flag != 0, in order (in place when d_out overlaps d_in)."""
    temp = _temp_for(select_temp_bytes(n), num_out, temp)
    call(f"lcpp_hip_select_flagged_{suffix}_{flag_suffix}", ptr(temp), _tb(temp), ptr(d_in), ptr(flags), ptr(d_out),
         ptr(num_out), n, stream_handle(stream))


def select_flagged_if(suffix: str, flag_suffix: str, d_in, flags, d_out, num_out, n: int, pred: Predicate,
                      temp=None, stream=None):
    """DeviceSelect::FlaggedIf: items whose flag satisfies `pred` (a predicate over the flag type)."""
    temp = _temp_for(select_temp_bytes(n), num_out, temp)
    call(f"lcpp_hip_select_flagged_if_{suffix}_{flag_suffix}", ptr(temp), _tb(temp), ptr(d_in), ptr(flags),
         ptr(d_out), ptr(num_out), n, C.byref(pred), stream_handle(stream))


def select_if(suffix: str, d_in, d_out, num_out, n: int, pred: Predicate, temp=None, stream=None):
    """DeviceSelect::If."""
    temp = _temp_for(select_temp_bytes(n), num_out, temp)
    call(f"lcpp_hip_select_if_{suffix}", ptr(temp), _tb(temp), ptr(d_in), ptr(d_out), ptr(num_out), n,
         C.byref(pred), stream_handle(stream))


def select_unique(suffix: str, d_in, d_out, num_out, n: int, key_mask: int = -1, temp=None, stream=None):
    """DeviceSelect::Unique: the first item of every run of equal items."""
    temp = _temp_for(select_temp_bytes(n), num_out, temp)
    call(f"lcpp_hip_select_unique_{suffix}", ptr(temp), _tb(temp), ptr(d_in), ptr(d_out), ptr(num_out), n,
         key_mask & 0xFFFFFFFFFFFFFFFF, stream_handle(stream))


def select_unique_by_key(key_suffix: str, value_suffix: str, keys_in, values_in, keys_out, values_out, num_out,
                         n: int, key_mask: int = -1, temp=None, stream=None):
    """DeviceSelect::UniqueByKey: the first (key, value) of every run of equal keys."""
    temp = _temp_for(select_temp_bytes(n), num_out, temp)
    call(f"lcpp_hip_select_unique_by_key_{key_suffix}_{value_suffix}", ptr(temp), _tb(temp), ptr(keys_in),
         ptr(values_in), ptr(keys_out), ptr(values_out), ptr(num_out), n, key_mask & 0xFFFFFFFFFFFFFFFF,
         stream_handle(stream))


def partition_flagged(suffix: str, flag_suffix: str, d_in, flags, d_out, num_out, n: int, temp=None, stream=None):
    """DevicePartition::Flagged: flagged items in order, then the others in reverse order."""
    temp = _temp_for(select_temp_bytes(n), num_out, temp)
    call(f"lcpp_hip_partition_flagged_{suffix}_{flag_suffix}", ptr(temp), _tb(temp), ptr(d_in), ptr(flags),
         ptr(d_out), ptr(num_out), n, stream_handle(stream))


def partition_if(suffix: str, d_in, d_out, num_out, n: int, pred: Predicate, temp=None, stream=None):
    """DevicePartition::If."""
    temp = _temp_for(select_temp_bytes(n), num_out, temp)
    call(f"lcpp_hip_partition_if_{suffix}", ptr(temp), _tb(temp), ptr(d_in), ptr(d_out), ptr(num_out), n,
         C.byref(pred), stream_handle(stream))


def partition_three_way(suffix: str, d_in, first_out, second_out, unselected_out, num_out, n: int,
                        select_first: Predicate, select_second: Predicate, temp=None, stream=None):
    """DevicePartition::If with two predicates (num_out[0..1] = the two category sizes)."""
    temp = _temp_for(partition_three_way_temp_bytes(n), num_out, temp)
    call(f"lcpp_hip_partition_three_way_{suffix}", ptr(temp), _tb(temp), ptr(d_in), ptr(first_out),
         ptr(second_out), ptr(unselected_out), ptr(num_out), n, C.byref(select_first), C.byref(select_second),
         stream_handle(stream))


def run_length_encode(suffix: str, d_in, unique_out, counts_out, num_runs_out, n: int, temp=None, stream=None):
    """DeviceRunLengthEncode::Encode."""
    temp = _temp_for(run_length_encode_temp_bytes(n), num_runs_out, temp)
    call(f"lcpp_hip_run_length_encode_{suffix}", ptr(temp), _tb(temp), ptr(d_in), ptr(unique_out), ptr(counts_out),
         ptr(num_runs_out), n, stream_handle(stream))


def run_length_non_trivial(suffix: str, d_in, offsets_out, lengths_out, num_runs_out, n: int, temp=None,
                           stream=None):
    """DeviceRunLengthEncode::NonTrivialRuns."""
    temp = _temp_for(run_length_encode_temp_bytes(n), num_runs_out, temp)
    call(f"lcpp_hip_run_length_non_trivial_{suffix}", ptr(temp), _tb(temp), ptr(d_in), ptr(offsets_out),
         ptr(lengths_out), ptr(num_runs_out), n, stream_handle(stream))


# ---- segmented reductions and scans (DeviceSegmentReduce, DeviceSegmentedScan) ------------------
def segment_reduce(op: str, suffix: str, d_in, d_out, num_segments: int, begins=None, ends=None,
                   segment_size: int | None = None, index_out=None, stream=None) -> None:
    """DeviceSegmentReduce::{Sum,Min,Max,ArgMin,ArgMax}: offsets (begins, ends) or a fixed segment_size."""
    arg = op in ("argmin", "argmax")
    if segment_size is not None:
        name = f"lcpp_hip_segment_fixed_{op}_{suffix}" if arg else f"lcpp_hip_segment_reduce_fixed_{op}_{suffix}"
        extra = (ptr(index_out),) if arg else ()
        call(name, None, 0, ptr(d_in), ptr(d_out), *extra, num_segments, segment_size, stream_handle(stream))
    else:
        name = f"lcpp_hip_segment_{op}_{suffix}" if arg else f"lcpp_hip_segment_reduce_{op}_{suffix}"
        extra = (ptr(index_out),) if arg else ()
        call(name, None, 0, ptr(d_in), ptr(d_out), *extra, num_segments, ptr(begins), ptr(ends),
             stream_handle(stream))


def segmented_scan(suffix: str, d_in, d_out, begins, ends, num_segments: int, inclusive: bool = False, init=None,
                   out_begins=None, stream=None) -> None:
    """DeviceSegmentedScan::{Exclusive,Inclusive}SegmentedSum, InclusiveSegmentedScanInit (sum)."""
    use_init = init is not None
    if not inclusive and not use_init:
        init, use_init = 0, True
    call(f"lcpp_hip_segmented_scan_sum_{suffix}", None, 0, ptr(d_in), ptr(d_out), ptr(begins), ptr(ends),
         ptr(out_begins), num_segments, int(inclusive), int(use_init), _CTYPE[suffix](init if use_init else 0),
         stream_handle(stream))


# ---- segmented sorts (DeviceSegmentedRadixSort, DeviceSegmentedSort) -----------------------------
def segmented_sort_keys_temp_bytes(n: int, key_bytes: int) -> int:
    return lib().lcpp_hip_segmented_sort_keys_temp_bytes(n, key_bytes)


def segmented_sort_pairs_temp_bytes(n: int, key_bytes: int, value_bytes: int) -> int:
    return lib().lcpp_hip_segmented_sort_pairs_temp_bytes(n, key_bytes, value_bytes)


def segmented_sort(key_suffix: str, keys_in, keys_out, n: int, num_segments: int, begins, ends, values_in=None,
                   values_out=None, begin_bit: int = 0, end_bit: int | None = None, descending: bool = False,
                   value_order: bool = False, temp=None, stream=None) -> None:
    """Stable per-segment sort (radix order of bits [begin_bit, end_bit), or value order)."""
    kb = ELEM_BYTES[key_suffix]
    end_bit = kb * 8 if end_bit is None else end_bit
    if values_in is None:
        nbytes = lib().lcpp_hip_segmented_sort_keys_temp_bytes(n, kb)
        temp = _temp_for(nbytes, keys_out, temp)
        call(f"lcpp_hip_segmented_sort_keys_{key_suffix}", ptr(temp), _tb(temp), ptr(keys_in), ptr(keys_out), n,
             num_segments, ptr(begins), ptr(ends), begin_bit, end_bit, int(descending), int(value_order),
             stream_handle(stream))
    else:
        vb = values_in.element_size()
        nbytes = lib().lcpp_hip_segmented_sort_pairs_temp_bytes(n, kb, vb)
        temp = _temp_for(nbytes, keys_out, temp)
        call(f"lcpp_hip_segmented_sort_pairs_{key_suffix}_v{8 * vb}", ptr(temp), _tb(temp), ptr(keys_in),
             ptr(keys_out), ptr(values_in), ptr(values_out), n, num_segments, ptr(begins), ptr(ends), begin_bit,
             end_bit, int(descending), int(value_order), stream_handle(stream))


def segmented_sort_db(key_suffix: str, keys0, keys1, selector: int, n: int, num_segments: int, begins, ends,
                      values0=None, values1=None, value_selector: int = 0, begin_bit: int = 0,
                      end_bit: int | None = None, descending: bool = False, value_order: bool = False,
                      stream=None):
    """DoubleBuffer form; returns the new (key selector, value selector)."""
    kb = ELEM_BYTES[key_suffix]
    end_bit = kb * 8 if end_bit is None else end_bit
    ks = C.c_int(selector)
    vs = C.c_int(value_selector)
    if values0 is None:
        call(f"lcpp_hip_segmented_sort_keys_db_{key_suffix}", ptr(keys0), ptr(keys1), C.byref(ks), n, num_segments,
             ptr(begins), ptr(ends), begin_bit, end_bit, int(descending), int(value_order), stream_handle(stream))
    else:
        call(f"lcpp_hip_segmented_sort_pairs_db_{key_suffix}_v{8 * values0.element_size()}", ptr(keys0), ptr(keys1),
             C.byref(ks), ptr(values0), ptr(values1), C.byref(vs), n, num_segments, ptr(begins), ptr(ends),
             begin_bit, end_bit, int(descending), int(value_order), stream_handle(stream))
    return ks.value, vs.value
