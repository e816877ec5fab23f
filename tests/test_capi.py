"""The C-ABI library loads without a GPU and exports every entry point include/lcpp_hip.h declares.
No compute call is made here (that needs the GPU)."""
import ctypes
import pathlib
import re
import subprocess

REPO = pathlib.Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "lcpp_hip.h"


def declared_symbols(*defines):
    """Function names declared in the header, with the declaration macros expanded by the C preprocessor."""
    out = subprocess.run(["gcc", "-E", "-P", *defines, "-x", "c", str(HEADER)], capture_output=True, text=True,
                         check=True)
    return sorted(set(re.findall(r"\b(lcpp_hip_\w+)\s*\(", out.stdout)))


def test_header_declares_the_hot_path():
    syms = declared_symbols()
    for s in ("lcpp_hip_reduce_sum_i32", "lcpp_hip_scan_exclusive_sum_u32", "lcpp_hip_radix_sort_keys_u32",
              "lcpp_hip_radix_sort_pairs_u64_v32", "lcpp_hip_spmv_csr_f32_i32", "lcpp_hip_reduce_temp_bytes",
              "lcpp_hip_scan_temp_bytes", "lcpp_hip_radix_sort_keys_temp_bytes", "lcpp_hip_radix_sort_pairs_temp_bytes"):
        assert s in syms
    assert len(syms) > 70


def test_library_exports_every_declared_symbol(hip):
    lib = ctypes.CDLL(str(hip.LIB_PATH))
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_phase_trace_library_exports_its_hook(hip):
    """The diagnostic build (build.py --phase-trace) exports everything, plus the trace hook; the product
    library has no trace hook."""
    import pytest
    trace = pathlib.Path(hip.LIB_PATH).with_name("liblcpp_hip_trace.so")
    if not trace.exists():
        pytest.skip("liblcpp_hip_trace.so is built by __graft_entry__.build() (build.py --phase-trace)")
    lib = ctypes.CDLL(str(trace))
    missing = [s for s in declared_symbols("-DLCPP_HIP_PHASE_TRACE") if not hasattr(lib, s)]
    assert not missing, missing
    assert hasattr(lib, "lcpp_hip_trace_set_buffer")
    assert not hasattr(ctypes.CDLL(str(hip.LIB_PATH)), "lcpp_hip_trace_set_buffer")


def test_error_reporting_without_gpu(hip):
    # Argument validation happens before any HIP call, so it works on a machine without a GPU.
    lib = hip.lib()
    st = lib.lcpp_hip_radix_sort_keys_u32(None, 0, None, None, 10, 9, 8, 0, None)
    assert st == hip.ERR_INVALID_ARGUMENT
    assert b"begin_bit" in lib.lcpp_hip_last_error()
    st = lib.lcpp_hip_radix_sort_keys_u32(None, 0, None, None, 10, 0, 33, 0, None)
    assert st == hip.ERR_INVALID_ARGUMENT
    assert lib.lcpp_hip_radix_sort_keys_u32(None, 0, None, None, 0, 0, 32, 0, None) == hip.OK
    assert lib.lcpp_hip_scan_exclusive_sum_u32(None, 0, None, None, 0, None) == hip.OK
    assert lib.lcpp_hip_reduce_sum_i32(None, 0, None, None, 1 << 33, None) == hip.ERR_INVALID_ARGUMENT
    assert lib.lcpp_hip_spmv_csr_f32_i32(None, 0, None, None, None, None, None, 0, 0, 0, None) == hip.OK
    assert lib.lcpp_hip_spmv_csr_f32_i32(None, 0, None, None, None, None, None, 1 << 30, 1, 1, None) == \
        hip.ERR_INVALID_ARGUMENT
    assert lib.lcpp_hip_version().startswith(b"lcpp-hip")


def test_facade_tests_build_and_list_cases():
    """The C++20 facade headers compile against the C-ABI and link (the binary lists its cases without
    touching a GPU)."""
    import pathlib
    import subprocess
    repo = pathlib.Path(__file__).resolve().parents[1]
    subprocess.run(["make", "-s", "-C", str(repo / "tests" / "cpp")], check=True)
    out = subprocess.run([str(repo / "tests" / "cpp" / "bin" / "facade_test"), "--list"], check=True,
                         capture_output=True, text=True).stdout.split()
    assert len(out) == 40 and "reduce_with_operator_and_transform" in out and "scan_double_inclusive_sum" in out and "radix_double_buffer_selectors" in out and "scan_inclusive_init_in_place" in out
    assert "scan_by_key_custom_equality" in out and "reduce_by_key_empty_input" in out
    assert "partition_ordering_and_three_way" in out and "run_length_encode_examples" in out
