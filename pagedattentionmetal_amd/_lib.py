"""ctypes binding of libpam.so (declarations mirror include/pam.h).

The library is built in-tree by ``pagedattentionmetal_amd.build``.  Loading fails
loudly when it is missing: there is no Python or CPU fallback for any
operation of the package.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libpam.so")

P = C.c_void_p
I32 = C.c_int32
I64 = C.c_int64
SZ = C.c_size_t


class LayerSpec(C.Structure):
    _fields_ = [("head_dim", I32), ("num_heads", I32), ("num_kv_heads", I32), ("block_size", I32),
                ("data_type", I32), ("window_size", I32)]


class Stats(C.Structure):
    _fields_ = [("operation", I32), ("batch_size", I32), ("sequence_length", I32), ("num_blocks", I32),
                ("temporary_bytes", I64), ("used_split_pass", I32), ("elapsed_ms", C.c_double),
                ("kernel_ms", C.c_double), ("reduce_ms", C.c_double), ("chunks", I32)]


class DecodeRequest(C.Structure):
    _fields_ = [("q", P), ("k_pool", P), ("v_pool", P), ("block_tables", P), ("seq_lengths", P), ("output", P),
                ("batch_size", I32), ("max_num_blocks", I32), ("layer", LayerSpec), ("k_scale", P), ("v_scale", P),
                ("q_bytes", SZ), ("k_pool_bytes", SZ), ("v_pool_bytes", SZ), ("block_tables_bytes", SZ),
                ("seq_lengths_bytes", SZ), ("output_bytes", SZ)]


class PrefillRequest(C.Structure):
    _fields_ = [("q", P), ("k_pool", P), ("v_pool", P), ("block_table", P), ("output", P), ("seq_len", I32),
                ("q_offset", I32), ("layer", LayerSpec), ("causal", C.c_bool), ("k_scale", P), ("v_scale", P),
                ("q_bytes", SZ), ("k_pool_bytes", SZ), ("v_pool_bytes", SZ), ("block_table_bytes", SZ),
                ("output_bytes", SZ)]


class FusedPrefillRequest(C.Structure):
    _fields_ = [("q", P), ("raw_k", P), ("raw_v", P), ("block_table", P), ("k_pool", P), ("v_pool", P),
                ("output", P), ("seq_len", I32), ("layer", LayerSpec), ("causal", C.c_bool), ("k_scale", P),
                ("v_scale", P), ("q_bytes", SZ), ("raw_k_bytes", SZ), ("raw_v_bytes", SZ), ("k_pool_bytes", SZ),
                ("v_pool_bytes", SZ), ("block_table_bytes", SZ), ("output_bytes", SZ)]


class BackwardRequest(C.Structure):
    _fields_ = [("q", P), ("k_pool", P), ("v_pool", P), ("block_table", P), ("d_out", P), ("m", P), ("l", P),
                ("d_q", P), ("d_k_pool", P), ("d_v_pool", P), ("seq_len", I32), ("layer", LayerSpec)]


class AppendRequest(C.Structure):
    _fields_ = [("keys", P), ("values", P), ("k_pool", P), ("v_pool", P), ("block_table", P), ("token_offset", I32),
                ("num_new_tokens", I32), ("layer", LayerSpec), ("k_scale", P), ("v_scale", P), ("slot_mapping", P),
                ("keys_bytes", SZ), ("values_bytes", SZ), ("k_pool_bytes", SZ), ("v_pool_bytes", SZ),
                ("block_table_bytes", SZ)]


class MixedRequest(C.Structure):
    _fields_ = [("q", P), ("output", P), ("new_keys", P), ("new_values", P), ("k_pool", P), ("v_pool", P),
                ("k_scale", P), ("v_scale", P), ("block_tables", P), ("bt_stride", I32), ("num_seqs", I32),
                ("context_lens", P), ("query_lens", P), ("layer", LayerSpec), ("q_bytes", SZ), ("output_bytes", SZ),
                ("new_keys_bytes", SZ), ("new_values_bytes", SZ), ("k_pool_bytes", SZ), ("v_pool_bytes", SZ),
                ("block_tables_bytes", SZ)]


class EngineConfig(C.Structure):
    _fields_ = [("split_threshold", I32), ("default_window_size", I32), ("default_chunk_size", I32)]


PP = C.POINTER(C.c_void_p)
PSZ = C.POINTER(C.c_size_t)


class DecodeLayersRequest(C.Structure):
    _fields_ = [("q", PP), ("output", PP), ("layers", C.POINTER(LayerSpec)), ("num_layers", I32), ("k_pool", P),
                ("v_pool", P), ("block_tables", P), ("seq_lengths", P), ("batch_size", I32), ("max_num_blocks", I32),
                ("window_size", I32), ("k_scale", P), ("v_scale", P), ("q_bytes", PSZ), ("output_bytes", PSZ),
                ("k_pool_bytes", SZ), ("v_pool_bytes", SZ), ("block_tables_bytes", SZ), ("seq_lengths_bytes", SZ)]


class PrefillLayersRequest(C.Structure):
    _fields_ = [("q", PP), ("output", PP), ("layers", C.POINTER(LayerSpec)), ("num_layers", I32), ("k_pool", P),
                ("v_pool", P), ("block_table", P), ("seq_len", I32), ("causal", C.c_bool), ("window_size", I32),
                ("k_scale", P), ("v_scale", P), ("q_bytes", PSZ), ("output_bytes", PSZ), ("k_pool_bytes", SZ),
                ("v_pool_bytes", SZ), ("block_table_bytes", SZ)]


class AppendLayersRequest(C.Structure):
    _fields_ = [("keys", PP), ("values", PP), ("layers", C.POINTER(LayerSpec)), ("num_layers", I32), ("k_pool", P),
                ("v_pool", P), ("block_table", P), ("token_offset", I32), ("num_new_tokens", I32), ("k_scale", PP),
                ("v_scale", PP), ("keys_bytes", PSZ), ("values_bytes", PSZ), ("k_pool_bytes", SZ),
                ("v_pool_bytes", SZ), ("block_table_bytes", SZ)]


class MemoryStats(C.Structure):
    _fields_ = [("total_blocks", I64), ("used_blocks", I64), ("free_blocks", I64), ("active_sequences", I64),
                ("total_memory_bytes", I64), ("used_memory_bytes", I64), ("partially_filled_blocks", I64),
                ("fragmentation_ratio", C.c_float), ("prefix_cache_hits", I64), ("prefix_cache_entries", I64),
                ("shared_blocks", I64), ("eviction_policy", I32)]


# name -> (restype, argtypes); every symbol declared in include/pam.h
SIGNATURES = {
    # Part 1
    "pam_create_context": (P, []),
    "pam_destroy_context": (None, [P]),
    "pam_last_error": (C.c_char_p, [P]),
    "pam_create_cache": (P, [P, I32, I32, I32, I32, I32]),
    "pam_destroy_cache": (None, [P]),
    "pam_reserve_sequence": (I32, [P, P, I64]),
    "pam_append_tokens": (I32, [P, P, I64, I32]),
    "pam_free_sequence": (None, [P, I64]),
    "pam_available_blocks": (I32, [P]),
    "pam_sequence_length": (I32, [P, P, I64]),
    "pam_append_kv": (I32, [P, P, I64, P, P, I32, I32, I32]),
    "pam_prefill": (I32, [P, P, I64, P, P, I32, I32, C.c_bool]),
    "pam_decode": (I32, [P, P, P, I32, P, P, I32]),
    # Part 2
    "pam_engine_decode": (I32, [P, C.POINTER(DecodeRequest)]),
    "pam_engine_prefill": (I32, [P, C.POINTER(PrefillRequest)]),
    "pam_engine_append": (I32, [P, C.POINTER(AppendRequest)]),
    "pam_engine_fused_prefill": (I32, [P, C.POINTER(FusedPrefillRequest)]),
    "pam_engine_backward": (I32, [P, C.POINTER(BackwardRequest)]),
    "pam_engine_last_stats": (I32, [P, C.POINTER(Stats)]),
    "pam_engine_set_graceful_degradation": (I32, [P, C.c_bool]),
    "pam_engine_set_max_retries": (I32, [P, I32]),
    "pam_append_tokens_hashed": (I32, [P, P, I64, I32, P, I32]),
    "pam_ensure_exclusive": (I32, [P, P, I64, I32]),
    "pam_register_block_hash": (I32, [P, C.c_uint64, I32]),
    "pam_set_eviction_policy": (I32, [P, I32]),
    "pam_block_table": (I32, [P, P, I64, P, I32]),
    "pam_cache_memory_stats": (I32, [P, C.POINTER(MemoryStats)]),
    "pam_cache_k_pool": (P, [P]),
    "pam_cache_v_pool": (P, [P]),
    "pam_cache_k_scale": (P, [P]),
    "pam_cache_v_scale": (P, [P]),
    "pam_cache_batch_view": (I32, [P, P, P, I32, I32, P, P]),
    "pam_scheduler_create": (P, [I32, I32]),
    "pam_scheduler_destroy": (None, [P]),
    "pam_scheduler_add_request": (I32, [P, I32, I32]),
    "pam_scheduler_complete": (None, [P, I32]),
    "pam_scheduler_step": (I32, [P, P, I32]),
    "pam_scheduler_mark_prefilled": (None, [P, I32]),
    "pam_scheduler_mark_decoded": (None, [P, I32]),
    "pam_scheduler_preempt": (None, [P, I32]),
    "pam_scheduler_handle_memory_pressure": (I32, [P, I32, P, P, I32]),
    "pam_scheduler_count": (I32, [P, I32]),
    "pam_scheduler_sequence": (I32, [P, I32, P, P, P]),
    # Part 3
    "pam_create_cache_host": (P, [P, I32, I32, I32, I32, I32]),
    "pam_buffer_alloc": (P, [P, SZ]),
    "pam_buffer_free": (None, [P, P]),
    "pam_buffer_upload": (I32, [P, P, P, SZ]),
    "pam_buffer_download": (I32, [P, P, P, SZ]),
    "pam_buffer_zero": (I32, [P, P, SZ]),
    "pam_set_stream": (I32, [P, P]),
    "pam_use_own_stream": (I32, [P]),
    "pam_set_synchronous": (I32, [P, C.c_bool]),
    "pam_synchronize": (I32, [P]),
    "pam_reserve_workspace": (I32, [P, SZ]),
    "pam_set_partition_tokens": (I32, [P, I32]),
    "pam_set_decode_kernel": (I32, [P, I32]),
    "pam_set_mixed_launch": (I32, [P, I32, I32, I32]),
    "pam_set_fused_prefill_kernel": (I32, [P, C.c_bool]),
    "pam_set_gpu_timing": (I32, [P, C.c_bool]),
    "pam_engine_mixed_step": (I32, [P, C.POINTER(MixedRequest)]),
    "pam_engine_set_config": (I32, [P, C.POINTER(EngineConfig)]),
    "pam_engine_get_config": (I32, [P, C.POINTER(EngineConfig)]),
    "pam_engine_prefill_flat": (I32, [P, C.POINTER(PrefillRequest), I32, I32]),
    "pam_engine_decode_flat": (I32, [P, C.POINTER(DecodeRequest), I32]),
    "pam_engine_append_flat": (I32, [P, C.POINTER(AppendRequest), I32]),
    "pam_engine_decode_layers": (I32, [P, C.POINTER(DecodeLayersRequest)]),
    "pam_engine_prefill_layers": (I32, [P, C.POINTER(PrefillLayersRequest)]),
    "pam_engine_append_layers": (I32, [P, C.POINTER(AppendLayersRequest)]),
    "pam_module_load": (I32, [P, C.c_char_p]),
    "pam_module_unload": (I32, [P]),
    "pam_module_set_strict": (I32, [P, I32]),
    "pam_decode_step": (I32, [P, P, I64, P, P, P, P, I32]),
    "pam_module_function": (I32, [P, C.c_char_p, C.POINTER(C.c_void_p)]),
    "pam_module_launch": (I32, [P, P, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                C.c_uint32, P, SZ]),
    "pam_module_default_path": (C.c_char_p, []),
    "pam_engine_setup_noalloc": (I32, [P]),
    "pam_engine_decode_noalloc": (I32, [P, C.POINTER(DecodeRequest)]),
    "pam_fp8_quantize": (I32, [P, P, P, P, I64]),
    "pam_fp8_dequant": (I32, [P, P, P, P, I64]),
    "pam_calib_stream_read": (I32, [P, P, SZ, I32, P]),
    "pam_calib_stream_copy": (I32, [P, P, P, SZ, I32, P]),
    "pam_calib_mfma": (I32, [P, I32, P]),
    "pam_synth_normal": (I32, [P, P, I32, C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, C.c_int64, C.c_float]),
    "pam_debug_fail_next_launches": (I32, [P, I32]),
    "pam_debug_dirty_counters": (I32, [P, I32]),
    "pam_version": (C.c_char_p, []),
}

_lib = None


def load() -> C.CDLL:
    """Load libpam.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"libpam.so not found at {LIB_PATH}; build it with "
                          "`python -m pagedattentionmetal_amd.build` (no fallback exists)")
    # One HIP runtime per process: torch ships its own libamdhip64 / libhsa-runtime64
    # with the same SONAMEs as ROCm's.  Loading torch first makes libpam bind to the
    # runtime torch's tensors and streams live in; loading libpam first would map a
    # second runtime that cannot share the device with torch's.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
