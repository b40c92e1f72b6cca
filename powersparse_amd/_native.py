"""ctypes bindings of the two in-tree shared libraries.

lib/libpowersparse_hip.so     HIP kernels + C ABI        (include/powersparse_hip.h)
lib/libpowersparse.so         C++17 host API, C facade   (include/powersparse.h)
lib/libpowersparse_bench.so   the CSV benchmark harness (include/powersparse_bench.h),
                              loaded on demand (bench())
lib/libpowersparse_perf.so    the measurement tooling's calibration copy (not
                              product code), loaded only by powersparse_amd.perf
                              (perf_lib())

Loading fails loudly when the libraries are missing: there is no CPU fallback.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_HERE, "lib")
HIP_LIB_PATH = os.path.join(LIB_DIR, "libpowersparse_hip.so")
HOST_LIB_PATH = os.path.join(LIB_DIR, "libpowersparse.so")
PERF_LIB_PATH = os.path.join(LIB_DIR, "libpowersparse_perf.so")
BENCH_LIB_PATH = os.path.join(LIB_DIR, "libpowersparse_bench.so")

PS_OK = 0
PS_ERR_INVALID = 1
PS_ERR_RUNTIME = 2
PS_MAX_WORKSETS = 32
PS_TASK_CHUNK_AUTO = -1
PS_OP_SPMM = 0
PS_OP_SDDMM = 1

c_int_p = ctypes.POINTER(ctypes.c_int)
c_float_p = ctypes.POINTER(ctypes.c_float)
c_double_p = ctypes.POINTER(ctypes.c_double)
c_u8_p = ctypes.POINTER(ctypes.c_uint8)
c_u32_p = ctypes.POINTER(ctypes.c_uint32)
c_u64_p = ctypes.POINTER(ctypes.c_uint64)
c_void_p = ctypes.c_void_p


class BuildOptions(ctypes.Structure):
    """psx_build_options (include/powersparse.h)."""
    _fields_ = [("cu_count", ctypes.c_int), ("signature_order", ctypes.c_int),
                ("csr_positions", ctypes.c_int), ("task_order", ctypes.c_int),
                ("stored_order", ctypes.c_int), ("max_group_types", ctypes.c_int),
                ("parity_spmm", ctypes.c_int), ("no_hub_block", ctypes.c_int),
                ("hub_min_degree", ctypes.c_int * 3), ("hub_min_count", ctypes.c_int * 3)]


class DeviceProps(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
        ("cu_count", ctypes.c_int),
        ("major", ctypes.c_int),
        ("minor", ctypes.c_int),
        ("lds_per_block", ctypes.c_int),
        ("l2_bytes", ctypes.c_int),
        ("clock_khz", ctypes.c_int),
        ("mem_clock_khz", ctypes.c_int),
        ("mem_bus_width", ctypes.c_int),
        ("global_mem", ctypes.c_size_t),
    ]


class Workset(ctypes.Structure):
    """ps_workset: one workset as the kernels read it."""

    _fields_ = [
        ("col_ind", c_void_p),
        ("sp_data", c_void_p),
        ("group_des", c_void_p),
        ("group_num", ctypes.c_int),
        ("group_size", ctypes.c_int),
        ("order", c_void_p),
    ]


class HubBlock(ctypes.Structure):
    """ps_hub_block: the dense hub block of a matrix (device pointers)."""

    _fields_ = [
        ("matrix_rows", ctypes.c_int),
        ("matrix_cols", ctypes.c_int),
        ("rows", ctypes.c_int),
        ("cols", ctypes.c_int),
        ("hub_rows", c_void_p),
        ("hub_index", c_void_p),
        ("hot_cols", c_void_p),
        ("hot_rank", c_void_p),
        ("dense", c_void_p),
        ("stored", c_void_p),
    ]


# (name, restype, argtypes) of every exported entry point. Tests check that
# each symbol declared in include/*.h is exported.
HIP_API = [
    ("ps_guard_violations", ctypes.c_longlong, []),
    ("ps_last_error", ctypes.c_char_p, []),
    ("ps_set_device", ctypes.c_int, [ctypes.c_int]),
    ("ps_get_device", ctypes.c_int, [c_int_p]),
    ("ps_device_count", ctypes.c_int, [c_int_p]),
    ("ps_get_device_props", ctypes.c_int, [ctypes.c_int, ctypes.POINTER(DeviceProps)]),
    ("ps_runtime_version", ctypes.c_int, [c_int_p]),
    ("ps_driver_version", ctypes.c_int, [c_int_p]),
    ("ps_device_synchronize", ctypes.c_int, []),
    ("ps_malloc", ctypes.c_int, [ctypes.POINTER(c_void_p), ctypes.c_size_t]),
    ("ps_mem_get_info", ctypes.c_int,
     [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]),
    ("ps_free", ctypes.c_int, [c_void_p]),
    ("ps_memcpy_htod", ctypes.c_int, [c_void_p, c_void_p, ctypes.c_size_t]),
    ("ps_memcpy_dtoh", ctypes.c_int, [c_void_p, c_void_p, ctypes.c_size_t]),
    ("ps_host_malloc", ctypes.c_int, [ctypes.POINTER(c_void_p), ctypes.c_size_t]),
    ("ps_host_free", ctypes.c_int, [c_void_p]),
    ("ps_memcpy_htod_async", ctypes.c_int, [c_void_p, c_void_p, ctypes.c_size_t, c_void_p]),
    ("ps_memcpy_dtod_async", ctypes.c_int, [c_void_p, c_void_p, ctypes.c_size_t, c_void_p]),
    ("ps_memset_async", ctypes.c_int, [c_void_p, ctypes.c_int, ctypes.c_size_t, c_void_p]),
    ("ps_fill_random_async", ctypes.c_int,
     [c_void_p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_float, ctypes.c_float, ctypes.c_int,
      c_void_p]),
    ("ps_stream_create", ctypes.c_int, [ctypes.POINTER(c_void_p)]),
    ("ps_stream_destroy", ctypes.c_int, [c_void_p]),
    ("ps_stream_synchronize", ctypes.c_int, [c_void_p]),
    ("ps_event_create", ctypes.c_int, [ctypes.POINTER(c_void_p)]),
    ("ps_event_destroy", ctypes.c_int, [c_void_p]),
    ("ps_event_record", ctypes.c_int, [c_void_p, c_void_p]),
    ("ps_event_synchronize", ctypes.c_int, [c_void_p]),
    ("ps_event_elapsed_ms", ctypes.c_int, [c_float_p, c_void_p, c_void_p]),
    ("ps_stream_wait_event", ctypes.c_int, [c_void_p, c_void_p]),
    ("ps_spmm_launch", ctypes.c_int,
     [ctypes.c_int, ctypes.POINTER(Workset), c_void_p, c_void_p, ctypes.c_int, ctypes.c_int,
      ctypes.c_int, c_void_p, c_void_p, ctypes.c_int, c_void_p]),
    ("ps_spmm_workset_launch", ctypes.c_int,
     [ctypes.c_int, ctypes.POINTER(Workset), c_void_p, c_void_p, ctypes.c_int, ctypes.c_int,
      ctypes.c_int, c_void_p, c_void_p, c_void_p]),
    ("ps_sddmm_launch", ctypes.c_int,
     [ctypes.c_int, ctypes.POINTER(Workset), c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
      c_void_p, c_void_p, ctypes.POINTER(c_void_p), ctypes.c_int, c_void_p]),
    ("ps_sddmm_workset_launch", ctypes.c_int,
     [ctypes.c_int, ctypes.POINTER(Workset), c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
      c_void_p, c_void_p, c_void_p, c_void_p]),
    ("ps_sddmm_csr_launch", ctypes.c_int,
     [ctypes.c_int, ctypes.POINTER(Workset), c_void_p, ctypes.POINTER(c_void_p), ctypes.c_int,
      ctypes.c_int, ctypes.c_int, c_void_p, c_void_p, c_void_p, ctypes.c_int, c_void_p]),
    ("ps_sddmm_scatter_launch", ctypes.c_int,
     [ctypes.c_int, ctypes.POINTER(Workset), c_void_p, ctypes.POINTER(c_void_p), ctypes.c_int,
      ctypes.c_int, ctypes.c_int, c_void_p, c_void_p, ctypes.POINTER(c_void_p), ctypes.c_int,
      c_void_p]),
    ("ps_task_count", ctypes.c_int,
     [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(Workset), c_u32_p]),
    ("ps_task_order_build", ctypes.c_int,
     [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(Workset), c_void_p,
      ctypes.c_uint32, c_void_p]),
    ("ps_task_order_build_subset", ctypes.c_int,
     [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(Workset),
      ctypes.POINTER(c_void_p), c_void_p, ctypes.c_uint32, c_u32_p, c_void_p]),
    ("ps_hub_histogram", ctypes.c_int,
     [c_void_p, ctypes.c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("ps_hub_stored_words", ctypes.c_size_t, [ctypes.POINTER(HubBlock)]),
    ("ps_hub_dense_build", ctypes.c_int,
     [ctypes.POINTER(HubBlock), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("ps_hub_kept_counts", ctypes.c_int,
     [ctypes.POINTER(HubBlock), c_void_p, c_void_p, c_void_p, c_void_p]),
    ("ps_hub_compact", ctypes.c_int,
     [ctypes.POINTER(HubBlock), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
      c_void_p]),
    ("ps_hub_mark_atomic", ctypes.c_int,
     [ctypes.POINTER(HubBlock), c_void_p, ctypes.c_int, c_void_p, c_void_p]),
    ("ps_hub_tile_flags", ctypes.c_int,
     [ctypes.POINTER(HubBlock), ctypes.POINTER(Workset), c_void_p, c_void_p]),
    ("ps_hub_workspace_bytes", ctypes.c_size_t,
     [ctypes.POINTER(HubBlock), ctypes.c_int, ctypes.c_int]),
    ("ps_hub_spmm_launch", ctypes.c_int,
     [ctypes.POINTER(HubBlock), ctypes.c_int, c_void_p, c_void_p, c_void_p, ctypes.c_size_t,
      c_void_p]),
    ("ps_hub_dense_ld", ctypes.c_size_t, [ctypes.c_int]),
    ("ps_hub_dense_floats", ctypes.c_size_t, [ctypes.c_int, ctypes.c_int]),
    ("ps_hub_sddmm_plan_bytes", ctypes.c_size_t, [ctypes.POINTER(HubBlock), ctypes.c_uint32]),
    ("ps_hub_sddmm_plan", ctypes.c_int,
     [ctypes.POINTER(HubBlock), ctypes.c_int, ctypes.POINTER(Workset), c_void_p,
      ctypes.c_uint32, c_void_p, ctypes.c_size_t, c_void_p]),
    ("ps_hub_sddmm_launch", ctypes.c_int,
     [ctypes.POINTER(HubBlock), ctypes.c_int, ctypes.POINTER(Workset), c_void_p,
      ctypes.c_uint32, ctypes.c_int, c_void_p, c_void_p, ctypes.POINTER(c_void_p),
      ctypes.POINTER(c_void_p), c_void_p, c_void_p, ctypes.c_size_t, c_void_p]),
    ("ps_spmm_launch_ordered", ctypes.c_int,
     [ctypes.c_int, ctypes.POINTER(Workset), c_void_p, c_void_p, ctypes.c_int, ctypes.c_int,
      ctypes.c_int, c_void_p, c_void_p, ctypes.c_int, c_void_p, ctypes.c_uint32, c_void_p]),
    ("ps_sddmm_launch_ordered", ctypes.c_int,
     [ctypes.c_int, ctypes.POINTER(Workset), c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
      c_void_p, c_void_p, ctypes.POINTER(c_void_p), ctypes.c_int, c_void_p, ctypes.c_uint32,
      c_void_p]),
    ("ps_sddmm_csr_launch_ordered", ctypes.c_int,
     [ctypes.c_int, ctypes.POINTER(Workset), c_void_p, ctypes.POINTER(c_void_p), ctypes.c_int,
      ctypes.c_int, ctypes.c_int, c_void_p, c_void_p, c_void_p, ctypes.c_int, c_void_p,
      ctypes.c_uint32, c_void_p]),
    ("ps_pre_exec_positions", ctypes.c_int,
     [ctypes.c_int, c_void_p, ctypes.c_int, c_void_p, c_void_p, c_void_p]),
    ("ps_pre_locality_score", ctypes.c_int,
     [ctypes.c_int, ctypes.POINTER(c_void_p), ctypes.POINTER(ctypes.c_longlong), ctypes.c_int,
      ctypes.c_int, c_double_p, c_void_p]),
    ("ps_workset_to_csr", ctypes.c_int,
     [ctypes.c_int, ctypes.POINTER(ctypes.c_longlong), ctypes.POINTER(c_void_p),
      ctypes.POINTER(c_void_p), c_void_p, c_void_p]),
    ("ps_scan_workspace_bytes", ctypes.c_size_t, [ctypes.c_size_t]),
    ("ps_exclusive_scan_u32", ctypes.c_int,
     [c_void_p, c_void_p, ctypes.c_size_t, c_void_p, c_void_p]),
    ("ps_exclusive_scan_u32_noalloc", ctypes.c_int,
     [c_void_p, c_void_p, ctypes.c_size_t, c_void_p]),
    ("ps_radix_workspace_bytes", ctypes.c_size_t, [ctypes.c_size_t]),
    ("ps_radix_sort_pairs_u64", ctypes.c_int,
     [c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
      c_void_p, c_int_p, c_void_p]),
    ("ps_radix_sort_pairs_u32", ctypes.c_int,
     [c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
      c_void_p, c_int_p, c_void_p]),
    ("ps_iota_u32", ctypes.c_int, [c_void_p, ctypes.c_int, c_void_p]),
    ("ps_pre_degree_sums", ctypes.c_int, [c_void_p, ctypes.c_int, c_u64_p, c_void_p]),
    ("ps_pre_col_histogram", ctypes.c_int, [c_void_p, ctypes.c_int, c_void_p, c_void_p]),
    ("ps_pre_rank_keys", ctypes.c_int,
     [c_void_p, ctypes.c_int, c_void_p, ctypes.c_int, c_void_p, ctypes.c_int, ctypes.c_int,
      c_void_p, c_void_p, c_void_p]),
    ("ps_pre_rank_sort", ctypes.c_int,
     [c_void_p, ctypes.c_int, c_void_p, ctypes.c_int, c_void_p, ctypes.c_int, ctypes.c_int,
      c_void_p, c_void_p, c_void_p]),
    ("ps_pre_group_counts", ctypes.c_int,
     [c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, c_void_p]),
    ("ps_pre_group_meta", ctypes.c_int,
     [c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.POINTER(c_void_p),
      ctypes.POINTER(c_void_p), c_void_p, c_void_p, c_void_p]),
    ("ps_pre_signatures", ctypes.c_int,
     [c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int, c_void_p,
      ctypes.c_int, c_void_p, c_void_p, c_void_p, c_int_p, ctypes.POINTER(c_void_p), c_void_p]),
    ("ps_pre_signature_keys", ctypes.c_int,
     [c_void_p, c_void_p, ctypes.c_int, c_void_p, c_void_p]),
    ("ps_pre_signature_span", ctypes.c_int,
     [c_void_p, ctypes.c_int, ctypes.c_int, c_u32_p, c_u32_p, c_void_p]),
    ("ps_pre_signature_lists", ctypes.c_int,
     [c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int, c_void_p,
      ctypes.c_int, c_void_p, c_void_p, ctypes.c_int, c_void_p, c_int_p, c_void_p, c_void_p,
      c_void_p]),
    ("ps_pre_signature_order", ctypes.c_int,
     [c_void_p, c_void_p, ctypes.c_int, c_int_p, ctypes.c_int, ctypes.POINTER(c_void_p),
      c_void_p]),
    ("ps_pre_permute_meta", ctypes.c_int,
     [c_void_p, ctypes.c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
      c_void_p]),
    ("ps_pre_gather_workset", ctypes.c_int,
     [ctypes.c_int, c_void_p, ctypes.c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
      c_void_p, c_void_p, c_void_p, c_void_p]),
]

BENCH_API = [
    ("psx_bench_main", ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p)]),
]

PERF_API = [
    ("ps_perf_copy_f32_async", ctypes.c_int, [c_void_p, c_void_p, ctypes.c_size_t, c_void_p]),
]

HOST_API = [
    ("psx_last_error", ctypes.c_char_p, []),
    ("psx_matrix_create", ctypes.c_int,
     [ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, c_void_p, c_void_p, ctypes.c_int,
      c_double_p, ctypes.POINTER(c_void_p)]),
    ("psx_matrix_create_ex", ctypes.c_int,
     [ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, c_void_p, c_void_p,
      ctypes.POINTER(BuildOptions), c_double_p, ctypes.POINTER(c_void_p)]),
    ("psx_matrix_signature_order", ctypes.c_int, [c_void_p, c_int_p]),
    ("psx_matrix_task_order", ctypes.c_int, [c_void_p, c_int_p, c_double_p, c_double_p]),
    ("psx_matrix_run_order", ctypes.c_int, [c_void_p, c_int_p]),
    ("psx_matrix_spmm_worksets", ctypes.c_int, [c_void_p, c_int_p]),
    ("psx_matrix_hub_block", ctypes.c_int, [c_void_p, c_int_p, ctypes.c_int, c_int_p, c_int_p]),
    ("psx_matrix_destroy", ctypes.c_int, [c_void_p]),
    ("psx_matrix_info", ctypes.c_int,
     [c_void_p, c_int_p, c_int_p, c_int_p, c_int_p, c_int_p, c_int_p, c_int_p]),
    ("psx_matrix_group_num", ctypes.c_int, [c_void_p, c_int_p]),
    ("psx_matrix_workset", ctypes.c_int,
     [c_void_p, ctypes.c_int, ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p),
      ctypes.POINTER(c_void_p)]),
    ("psx_matrix_residue", ctypes.c_int,
     [c_void_p, ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p)]),
    ("psx_spmm", ctypes.c_int,
     [c_void_p, ctypes.c_int, c_void_p, c_void_p, ctypes.c_int, ctypes.POINTER(c_void_p)]),
    ("psx_spmm_async", ctypes.c_int, [c_void_p, ctypes.c_int, c_void_p, c_void_p, c_void_p]),
    ("psx_sddmm", ctypes.c_int,
     [c_void_p, ctypes.c_int, c_void_p, c_void_p, ctypes.POINTER(c_void_p), ctypes.c_int,
      ctypes.POINTER(c_void_p)]),
    ("psx_sddmm_async", ctypes.c_int,
     [c_void_p, ctypes.c_int, c_void_p, c_void_p, ctypes.POINTER(c_void_p), c_void_p]),
    ("psx_sddmm_csr", ctypes.c_int,
     [c_void_p, ctypes.c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("psx_workset_to_csr", ctypes.c_int,
     [c_void_p, ctypes.POINTER(c_void_p), c_void_p, c_void_p]),
    ("psx_matrix_csr_position", ctypes.c_int, [c_void_p, ctypes.c_int, ctypes.POINTER(c_void_p)]),
    ("psx_csr_read_mtx", ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(c_void_p)]),
    ("psx_csr_read_binary", ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(c_void_p)]),
    ("psx_csr_write_binary", ctypes.c_int, [c_void_p, ctypes.c_char_p]),
    ("psx_csr_synth", ctypes.c_int,
     [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_int, ctypes.POINTER(c_void_p)]),
    ("psx_csr_chung_lu", ctypes.c_int,
     [ctypes.c_int, ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_float,
      ctypes.c_float, ctypes.c_uint64, ctypes.POINTER(c_void_p)]),
    ("psx_csr_uniform_degree", ctypes.c_int,
     [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float,
      ctypes.c_uint64, ctypes.POINTER(c_void_p)]),
    ("psx_csr_community", ctypes.c_int,
     [ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_double, ctypes.c_double,
      ctypes.c_double, ctypes.c_float, ctypes.c_float, ctypes.c_uint64,
      ctypes.POINTER(c_void_p)]),
    ("psx_csr_info", ctypes.c_int, [c_void_p, c_int_p, c_int_p, c_int_p]),
    ("psx_csr_arrays", ctypes.c_int,
     [c_void_p, ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p)]),
    ("psx_csr_free", ctypes.c_int, [c_void_p]),
    ("psx_generate_sigbit", ctypes.c_int,
     [ctypes.c_int, c_void_p, ctypes.c_int, c_void_p, c_int_p]),
    ("psx_workset_count", ctypes.c_int, [c_u64_p, ctypes.c_int, c_int_p]),
    ("psx_dense_input", ctypes.c_int,
     [ctypes.c_uint, ctypes.c_size_t, c_void_p, ctypes.c_size_t, c_void_p]),
]

_hip = None
_host = None
_perf = None
_bench = None


def _bind(lib, api):
    for name, restype, argtypes in api:
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes


def libs():
    """Loads (once) and returns (hip_lib, host_lib)."""
    global _hip, _host
    if _host is None:
        for path in (HIP_LIB_PATH, HOST_LIB_PATH):
            if not os.path.exists(path):
                raise ImportError(
                    f"powersparse_amd: native library {path} is missing; build it with "
                    "`python -c 'import __graft_entry__ as g; g.build()'` or "
                    "`make -C powersparse_amd`")
        hip = ctypes.CDLL(HIP_LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        _bind(hip, HIP_API)
        host = ctypes.CDLL(HOST_LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        _bind(host, HOST_API)
        _hip, _host = hip, host
    return _hip, _host


def hip():
    return libs()[0]


def host():
    return libs()[1]


def bench():
    """Loads (once) and returns the CSV benchmark harness library."""
    global _bench
    if _bench is None:
        libs()
        if not os.path.exists(BENCH_LIB_PATH):
            raise ImportError(f"powersparse_amd: {BENCH_LIB_PATH} is missing; "
                              "build it with `make -C powersparse_amd`")
        lib = ctypes.CDLL(BENCH_LIB_PATH)
        _bind(lib, BENCH_API)
        _bench = lib
    return _bench


def perf_lib():
    """Loads (once) and returns the measurement tooling's calibration-copy library."""
    global _perf
    if _perf is None:
        libs()
        if not os.path.exists(PERF_LIB_PATH):
            raise ImportError(f"powersparse_amd: {PERF_LIB_PATH} is missing; "
                              "build it with `make -C powersparse_amd perf`")
        lib = ctypes.CDLL(PERF_LIB_PATH)
        _bind(lib, PERF_API)
        _perf = lib
    return _perf
