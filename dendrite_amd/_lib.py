"""ctypes binding of libdendrite_hip.so (the C ABI in include/dendrite_hip.h).

The library is loaded from the package directory (or from the path in
DENDRITE_HIP_LIB, e.g. the host-sanitized build); a missing library is a hard
error (there is no fallback implementation).
"""
from __future__ import annotations

import ctypes as C
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("DENDRITE_HIP_LIB") or os.path.join(_PKG, "libdendrite_hip.so")

# dh_status
DH_OK = 0
DH_EINVAL = 1
DH_ENOMEM = 2
DH_EHIP = 3
DH_EUNSUPPORTED = 4
DH_EINVALID_BLOCK = 5
DH_EINVALID_NODE = 6
DH_ECACHE = 7

# dh_dtype
DTYPE_F16, DTYPE_BF16, DTYPE_F32 = 0, 1, 2
# dh_kv_format
KV_F16, KV_BF16, KV_F32, KV_FP8_E4M3, KV_MXFP8 = 0, 1, 2, 3, 4
# dh_gqa_mapping
GQA_TILED, GQA_INTERLEAVED = 0, 1
# plan flags
PLAN_FLAT, PLAN_CASCADE = 0, 1
PLAN_APPEND, PLAN_REPLACE_LAST = 0, 1
# dh_plan_options.direct
DIRECT_AUTO, DIRECT_OFF = 0, 1

PAGE_SIZE = 16
STATIC_WORKSPACE_BYTES = 32 << 20   # DH_STATIC_WORKSPACE_BYTES
HOST_LENS_MAX_BATCH = 512           # DH_HOST_LENS_MAX_BATCH
MAX_SEQ_LEN = 131072
INVALID_PAGE = 0xFFFFFFFF
INVALID_NODE = 0xFFFFFFFFFFFFFFFF
ROOT_NODE = 0


class DhError(RuntimeError):
    """A dh_status other than DH_OK, with dh_last_error()'s text."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[dh_status {status}] {message}")
        self.status = status


class dh_attn_config(C.Structure):
    _fields_ = [("num_heads", C.c_uint32), ("num_kv_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("scale", C.c_float),
                ("sliding_window", C.c_uint32), ("gqa_mapping", C.c_uint32),
                ("q_dtype", C.c_uint32), ("kv_format", C.c_uint32)]


class dh_plan_options(C.Structure):
    _fields_ = [("shared_chunk_pages", C.c_uint32), ("private_chunk_pages", C.c_uint32),
                ("target_items", C.c_uint32), ("direct", C.c_uint32),
                ("reserved", C.c_uint32 * 4)]


class dh_plan_stats(C.Structure):
    _fields_ = [("batch_size", C.c_uint32), ("num_segments", C.c_uint32),
                ("num_shared_segments", C.c_uint32), ("num_items", C.c_uint32),
                ("num_tasks", C.c_uint32), ("num_group_items", C.c_uint32),
                ("num_partials", C.c_uint32), ("direct", C.c_uint32), ("unique_pages", C.c_uint64),
                ("page_reads", C.c_uint64), ("total_pages", C.c_uint64)]


class dh_plan_item(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("page_off", "npages", "seq_off", "row_begin", "nrows",
                                          "kv_head", "flags", "tail_seq")]


class dh_node_info(C.Structure):
    _fields_ = [("id", C.c_uint64), ("parent", C.c_uint64), ("num_tokens", C.c_uint64),
                ("num_children", C.c_uint32), ("is_active", C.c_uint32)]


_P = C.c_void_p
_U32 = C.c_uint32
_U64 = C.c_uint64
_I = C.c_int
_PU32 = C.POINTER(C.c_uint32)
_PU64 = C.POINTER(C.c_uint64)

# name -> (restype, argtypes); restype _I means dh_status.
SIGNATURES = {
    "dh_last_error": (C.c_char_p, []),
    "dh_version": (C.c_char_p, []),
    "dh_attn_config_init": (_I, [C.POINTER(dh_attn_config), _U32, _U32, _U32]),
    "dh_attn_config_num_queries_per_kv": (_U32, [C.POINTER(dh_attn_config)]),
    "dh_create": (_I, [_I, C.POINTER(_P)]),
    "dh_destroy": (_I, [_P]),
    "dh_is_available": (_I, []),
    "dh_device_count": (_I, [C.POINTER(_I)]),
    "dh_memory_info": (_I, [_P, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "dh_synchronize": (_I, [_P]),
    "dh_pool_create": (_I, [_P, _U32, _U32, _U32, _U32, _U32, C.POINTER(_P)]),
    "dh_pool_destroy": (_I, [_P]),
    "dh_pool_page_bytes": (C.c_size_t, [_P]),
    "dh_pool_scale_bytes": (C.c_size_t, [_P]),
    "dh_pool_num_pages": (_U32, [_P]),
    "dh_pool_data": (_P, [_P]),
    "dh_pool_scales": (_P, [_P]),
    "dh_pool_write_tokens": (_I, [_P, _U32, _U32, _U32, _P, _P, _P, _P, _P]),
    "dh_pool_write_pages": (_I, [_P, _PU32, _U32, _P, _P, _P]),
    "dh_pool_write_pages_device": (_I, [_P, _P, _U32, _P, _U32, _P]),
    "dh_pool_copy_page": (_I, [_P, _U32, _U32, _P]),
    "dh_pool_read_page": (_I, [_P, _U32, _P, _P]),
    "dh_plan_create": (_I, [_P, C.POINTER(dh_attn_config), _P, _PU32, _PU32, _U32, _U32,
                            C.POINTER(dh_plan_options), C.POINTER(_P)]),
    "dh_plan_create_prefill": (_I, [_P, C.POINTER(dh_attn_config), _P, _PU32, _PU32, _PU32, _PU32, _U32, _U32,
                                    _U32, C.POINTER(_P)]),
    "dh_plan_destroy": (_I, [_P]),
    "dh_plan_update": (_I, [_P, _U32, _PU32, _PU32, _PU32, _P, _PU32]),
    "dh_plan_workspace_size": (C.c_size_t, [_P]),
    "dh_plan_get_stats": (_I, [_P, C.POINTER(dh_plan_stats)]),
    "dh_plan_inspect": (_I, [_P, _U32, _PU32, _PU32, _U32, _U32, _P, C.POINTER(dh_plan_stats), _P, _PU32,
                             _PU32, _PU32, _PU32, _PU32]),
    "dh_decode_batch": (_I, [_P, _P, _P, _P, _P, _P, _P, C.c_size_t, _P]),
    "dh_decode_stages": (_I, [_P, _P, _P, _P, _P, _P, _P, C.c_size_t, _U32, _P]),
    "dh_decode_batch_static": (_I, [_P, _P, _P, _P, _P, _P, _P]),
    "dh_decode_batch_host_lens": (_I, [_P, _P, _P, _P, _P, _P, _P, C.c_size_t, _P]),
    "dh_csr_workspace_size": (C.c_size_t, [C.POINTER(dh_attn_config), _U32, _U32]),
    "dh_decode_csr": (_I, [_P, _P, C.POINTER(dh_attn_config), _U32, _P, _P, _P, _P, _P, _P, C.c_size_t, _P,
                           _P]),
    "dh_merge_states": (_I, [_P, _P, _P, _P, _P, _P, _U32, _U32, _P]),
    "dh_gather_debug": (_I, [_P, _PU32, _U32, _U32, _P, _PU32, _P]),
    "dh_debug_e4m3_to_bf16": (_I, [_I, _P, _P, _U32, _P]),
    "dh_block_pool_create": (_I, [_U32, _U32, C.POINTER(_P)]),
    "dh_block_pool_destroy": (_I, [_P]),
    "dh_block_pool_allocate": (_I, [_P, _PU32]),
    "dh_block_pool_free": (_I, [_P, _U32]),
    "dh_block_pool_share": (_I, [_P, _U32]),
    "dh_block_pool_copy_on_write": (_I, [_P, _U32, _PU32]),
    "dh_block_pool_free_count": (_U32, [_P]),
    "dh_block_pool_total": (_U32, [_P]),
    "dh_block_pool_refcount": (_U32, [_P, _U32]),
    "dh_block_table_create": (_I, [_U32, C.POINTER(_P)]),
    "dh_block_table_destroy": (_I, [_P]),
    "dh_block_table_num_blocks": (_U32, [_P]),
    "dh_block_table_num_tokens": (_U64, [_P]),
    "dh_block_table_get": (_I, [_P, _U64, _PU32]),
    "dh_block_table_block_for_token": (_I, [_P, _U64, _PU32]),
    "dh_block_table_push": (_I, [_P, _U32]),
    "dh_block_table_set": (_I, [_P, _U64, _U32]),
    "dh_block_table_set_num_tokens": (_I, [_P, _U64]),
    "dh_block_table_add_tokens": (_I, [_P, _U64]),
    "dh_block_table_needs_new_block": (_I, [_P]),
    "dh_block_table_fork": (_I, [_P, C.POINTER(_P)]),
    "dh_block_table_clear": (_I, [_P]),
    "dh_block_table_blocks": (_U32, [_P, _PU32, _U32]),
    "dh_tree_create": (_I, [_P, _U32, C.POINTER(_P)]),
    "dh_tree_destroy": (_I, [_P]),
    "dh_tree_fork": (_I, [_P, _U64, _PU64, _PU64, _PU64]),
    "dh_tree_append_token": (_I, [_P, _U64, _U32, _PU32, _PU32]),
    "dh_tree_release": (_I, [_P, _U64]),
    "dh_tree_get_node": (_I, [_P, _U64, C.POINTER(dh_node_info)]),
    "dh_tree_get_block_table": (_I, [_P, _U64, _PU32, _U32, _PU32]),
    "dh_tree_get_tokens": (_I, [_P, _U64, _PU32, _U32, _PU32]),
    "dh_tree_num_nodes": (_U32, [_P]),
    "dh_tree_tokens_per_block": (_U32, [_P]),
    "dh_plan_create_tree": (_I, [_P, C.POINTER(dh_attn_config), _P, _P, _PU64, _U32, _U32,
                                 C.POINTER(dh_plan_options), C.POINTER(_P)]),
    "dh_tree_last_page_len": (_I, [_P, _PU64, _U32, C.POINTER(C.c_int32)]),
}

# libdendrite_testdata.so (include/dendrite_testdata.h): the tests' and
# benchmark's seeded input generators, kept out of the backend library.
TESTDATA_PATH = os.path.join(_PKG, "libdendrite_testdata.so")
TESTDATA_SIGNATURES = {
    "dh_testdata_last_error": (C.c_char_p, []),
    "dh_synth_normal": (C.c_double, [_U64, _U64]),
    "dh_synth_fill": (_I, [_P, _U32, _U64, _U64, _U64]),
    "dh_synth_pages": (_I, [_U32, _U32, _U32, _U64, _PU32, _U32, C.c_double, _U32, _P, _P]),
}

_lib = None
_testdata = None


def lib() -> C.CDLL:
    """Loads the in-tree library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m dendrite_amd.build` "
                "(there is no non-HIP fallback)")
        # One HIP runtime per process: torch (which holds the device buffers
        # on the Python side) bundles its own libamdhip64.so.7.  Loading torch
        # first lets the dynamic loader satisfy this library's libamdhip64.so.7
        # dependency with that same, already loaded runtime (matched by
        # SONAME) instead of mapping a second runtime that would contend for
        # the device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def testdata_lib() -> C.CDLL:
    """Loads the in-tree test-data library (raises if it has not been built)."""
    global _testdata
    if _testdata is None:
        if not os.path.exists(TESTDATA_PATH):
            raise RuntimeError(f"{TESTDATA_PATH} is missing: build it with `python -m dendrite_amd.build`")
        L = C.CDLL(TESTDATA_PATH)
        for name, (res, args) in TESTDATA_SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _testdata = L
    return _testdata


def check_testdata(status: int) -> None:
    if status != DH_OK:
        raise DhError(status, testdata_lib().dh_testdata_last_error().decode())


def last_error() -> str:
    return lib().dh_last_error().decode()


def check(status: int) -> None:
    if status != DH_OK:
        raise DhError(status, last_error())


def u32_array(values) -> "C.Array":
    vals = list(values)
    return (C.c_uint32 * max(1, len(vals)))(*vals)
