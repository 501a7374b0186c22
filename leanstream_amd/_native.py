"""ctypes binding of libleanstream_hip.so (C ABI declared in include/leanstream_hip.h).

The library is built in-tree (``python -c 'import __graft_entry__; __graft_entry__.build()'``).
Nothing here falls back to Python or CPU code: a missing library is an error.
"""
import ctypes as C
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIBRARY_PATH = _HERE / "libleanstream_hip.so"

p = C.c_void_p
u32 = C.c_uint32
u64 = C.c_uint64
i32 = C.c_int32


class ExecDesc(C.Structure):
    """Five 32-bit words (include/leanstream/types.h ExecDesc)."""

    _fields_ = [("logical_group", u32), ("physical_group", u32), ("source_slot", u32), ("dest_slot", u32),
                ("source_kind", u32)]


class DeviceQueue(C.Structure):
    """DeviceExecQueue: descriptors, ready_indices, control, capacity."""

    _fields_ = [("descriptors", p), ("ready_indices", p), ("control", p), ("capacity", u32)]


class LayerBuffers(C.Structure):
    """HipLayerBuffers (include/leanstream/hip_backend.h)."""

    _fields_ = [("width", u32), ("group_size", u32), ("batch", u32), ("slot_capacity", u32),
                ("cache_groups", u32), ("staging_groups", u32), ("physical_groups", u32), ("queue_capacity", u32),
                ("cache", p), ("staging", p), ("scales", p), ("hidden", p), ("partial", p), ("y32", p),
                ("executions", p), ("first_compute", p), ("claim_log", p), ("stamps", p)]


class Epilogue(C.Structure):
    """ls_hip_epilogue / HipEpilogue (include/leanstream/hip_backend.h)."""

    _fields_ = [("residual", p), ("hidden", p), ("hidden_flag", p), ("norm_weight", p), ("norm_output", p),
                ("norm_flag", p), ("bell", p), ("norm_eps", C.c_float)]


class ChainLayer(C.Structure):
    """ls_hip_chain_layer / HipChainLayer (include/leanstream/hip_backend.h)."""

    _fields_ = [("core", p), ("cache", p), ("staging", p), ("scales", p), ("input", p), ("residual", p),
                ("norm_weight", p), ("output", p), ("output32", p), ("hidden", p), ("hidden_flag", p), ("bell", p),
                ("core_count", u32), ("cache_groups", u32), ("staging_groups", u32), ("physical_groups", u32),
                ("epoch", u32), ("norm_eps", C.c_float)]


class GroupLayout(C.Structure):
    """GroupLayout (include/leanstream/group_layout.h); file_offset = offset in the host store."""

    _fields_ = [("logical_group", u32), ("physical_group", u32), ("file_offset", u64), ("bytes", u32),
                ("reserved", u32)]


class StreamSetup(C.Structure):
    """ls_stream_setup (include/leanstream_hip.h)."""

    _fields_ = [("backend", p), ("host_store", p), ("host_bytes", u64), ("staging", p), ("staging_bytes", u64),
                ("group_bytes", u64), ("staging_stride", u64), ("group_count", u32), ("layers", u32), ("qd", u32),
                ("copy_engine", u32), ("copy_queues", u32), ("copy_chunk", u32), ("mode", u32), ("device", i32)]


class StreamLayer(C.Structure):
    """ls_stream_layer (include/leanstream_hip.h)."""

    _fields_ = [("layout", p), ("rank", p), ("rank_count", u32), ("final_ids", p), ("final_count", u32),
                ("arrival_ns", p), ("input", p), ("output", p)]


_SIGNATURES = [
    ("ls_hip_create", [], p),
    ("ls_hip_create_table", [p, u32, u32], p),
    ("ls_hip_destroy", [p], None),
    ("ls_hip_bind", [p, p], C.c_int),
    ("ls_hip_enqueue", [p, u32, u32, u32, p, p, p, p, u32, p, u32], C.c_int),
    ("ls_hip_complete", [p, u32], C.c_int),
    ("ls_hip_compute_backend", [p, p, u64], C.c_int),
    ("ls_hip_status", [p], u32),
    ("ls_hip_clear_status", [p], None),
    ("ls_hip_set_spin_limit", [p, u64], None),
    ("ls_hip_set_epilogue", [p, p], C.c_int),
    ("ls_hip_set_stage_hook", [p, p, p, p], C.c_int),
    ("ls_hip_enqueue_chain", [p, p, u32, p], C.c_int),
    ("ls_hip_set_chain_stamps", [p, p, u32], C.c_int),
    ("ls_hip_chain_workers", [p], u32),
    ("ls_hip_last_seq", [p], u32),
    ("ls_hip_done_seq", [p], u32),
    ("ls_hip_slices", [p], u32),
    ("ls_hip_set_workers", [p, u32], None),
    ("ls_hip_select", [p, u32, u32], u32),
    ("ls_hip_last_candidate", [p], C.c_int),
    ("ls_hip_max_workers", [p], u32),
    ("ls_quantize_io_load", [u32, u32, u32], u32),
    ("ls_hip_core_layer_noalloc", [u32, u32, u32, p, u32, p, u32, p, u32, p, p, p, p, p], C.c_int),
    ("ls_hip_host_alloc", [u64], p),
    ("ls_hip_host_free", [p], None),
    ("ls_hip_release_u32", [p, C.c_int64, u32], None),
    ("ls_hip_acquire_all", [p, i32, u32, i32], C.c_int),
    ("ls_queue_create", [p], p),
    ("ls_queue_destroy", [p], None),
    ("ls_queue_reset", [p, u32], None),
    ("ls_queue_prepare", [p, u32], None),
    ("ls_queue_append_unpublished", [p, u32], None),
    ("ls_queue_activate", [p], None),
    ("ls_queue_seal", [p, u32], None),
    ("ls_queue_publish_all", [p], None),
    ("ls_queue_publish", [p, u32], None),
    ("ls_queue_fail", [p, u32], None),
    ("ls_publisher_start", [p, p, p, u32, u32, u32], p),
    ("ls_publisher_join", [p], C.c_int),
    ("ls_rank_groups", [p, u32, u32, p], C.c_int),
    ("ls_stream_create", [p], p),
    ("ls_stream_destroy", [p], None),
    ("ls_stream_queue", [p, p], C.c_int),
    ("ls_stream_run", [p, p, u32, u32, p, p, p, i32], C.c_int),
    ("ls_stream_inject_copy_error", [p, u32, i32], C.c_int),
    ("ls_synth_bytes", [p, u64, u64, p], C.c_int),
    ("ls_synth_uniform_f16", [p, u64, u64, C.c_double, C.c_double, p], C.c_int),
    ("ls_synth_normal_f16", [p, u64, u64, p], C.c_int),
    ("ls_synth_normal_bf16", [p, u64, u64, p], C.c_int),
    ("ls_hold_stream", [p, p, u64], C.c_int),
]

EXPORTED = tuple(name for name, _, _ in _SIGNATURES)

_lib = None


def library():
    """Load the native library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIBRARY_PATH.is_file():
            raise RuntimeError(f"{LIBRARY_PATH} is missing: build the native HIP library first")
        lib = C.CDLL(str(LIBRARY_PATH))
        for name, args, res in _SIGNATURES:
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib
