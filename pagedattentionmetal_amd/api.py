"""Python mirror of the reference's Swift API over libpam's C ABI.

Names, argument meaning and error behaviour follow
Sources/PagedAttentionMetal/{PagedAttentionTypes,PagedAttentionEngine,KVCacheManager,Scheduler}.swift:
``PagedLayerSpec``, ``PagedAttentionEngine.prefill/decode/append_to_cache``,
``KVCacheManager``, ``ContinuousBatchingScheduler``.  Buffers are torch device
tensors (torch provides HBM allocation and streams); every computation runs in
libpam's HIP kernels.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from enum import IntEnum

from . import _lib

L = None


def lib():
    global L
    if L is None:
        L = _lib.load()
    return L


class PagedAttentionDataType(IntEnum):
    """PagedAttentionTypes.swift:67-91"""
    float32 = 0
    float16 = 1
    float8 = 2

    @property
    def byte_width(self) -> int:
        return {0: 4, 1: 2, 2: 1}[int(self)]

    @property
    def is_quantized(self) -> bool:
        return self == PagedAttentionDataType.float8


class PagedAttentionError(RuntimeError):
    """PagedAttentionError / KVCacheError text from pam_last_error."""


class BlockEvictionPolicy(IntEnum):
    """KVCacheManager.swift:13-17"""
    fifo = 0
    lifo = 1
    best_fit = 2


@dataclass
class PagedLayerSpec:
    """PagedAttentionTypes.swift:94-152"""
    head_dim: int
    num_heads: int
    num_kv_heads: int
    block_size: int = 16
    data_type: PagedAttentionDataType = PagedAttentionDataType.float16
    window_size: int = 0

    def validate(self):
        if self.head_dim <= 0:
            raise PagedAttentionError("Invalid paged attention configuration: headDim must be positive.")
        if self.num_heads <= 0:
            raise PagedAttentionError("Invalid paged attention configuration: numHeads must be positive.")
        if self.num_kv_heads <= 0:
            raise PagedAttentionError("Invalid paged attention configuration: numKVHeads must be positive.")
        if self.num_heads % self.num_kv_heads:
            raise PagedAttentionError("Invalid paged attention configuration: numHeads must be divisible by "
                                      "numKVHeads for GQA/MQA mapping.")
        if self.block_size <= 0:
            raise PagedAttentionError("Invalid paged attention configuration: blockSize must be positive.")

    @property
    def q_elements_per_token(self):
        return self.num_heads * self.head_dim

    @property
    def kv_elements_per_token(self):
        return self.num_kv_heads * self.head_dim

    def c(self) -> _lib.LayerSpec:
        return _lib.LayerSpec(self.head_dim, self.num_heads, self.num_kv_heads, self.block_size, int(self.data_type),
                              self.window_size)


def _ptr(t):
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        if not t.is_contiguous():
            raise PagedAttentionError("buffers must be contiguous")
        return t.data_ptr()
    return int(t)


def _nbytes(t):
    if t is None or not hasattr(t, "element_size"):
        return 0
    return t.numel() * t.element_size()


class _DeviceArray:
    """__cuda_array_interface__ view of library-owned HBM (torch.as_tensor imports it)."""

    def __init__(self, ptr: int, shape, typestr: str):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": typestr, "data": (ptr, False),
                                         "version": 2, "strides": None}


class PagedAttentionEngine:
    """PagedAttentionEngine (PagedAttentionEngine.swift).  One libpam context: one
    HIP stream, synchronous calls unless ``synchronous = False``."""

    def __init__(self):
        self._ctx = lib().pam_create_context()
        if not self._ctx:
            raise PagedAttentionError("GPU device or stream could not be initialized.")

    def close(self):
        if getattr(self, "_ctx", None):
            lib().pam_destroy_context(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._ctx

    def _check(self, rc: int):
        if rc != 0:
            msg = lib().pam_last_error(self._ctx)
            raise PagedAttentionError(msg.decode() if msg else "libpam call failed")

    # --- configuration
    def set_stream(self, stream):
        """Launch on a torch stream (or a raw hipStream_t int; 0 = default stream);
        None -> the engine's own stream."""
        if stream is None:
            self._check(lib().pam_use_own_stream(self._ctx))
            return
        raw = stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)
        self._check(lib().pam_set_stream(self._ctx, raw or None))

    @property
    def synchronous(self):
        return self._sync if hasattr(self, "_sync") else True

    @synchronous.setter
    def synchronous(self, v: bool):
        self._check(lib().pam_set_synchronous(self._ctx, bool(v)))
        self._sync = bool(v)

    def synchronize(self):
        self._check(lib().pam_synchronize(self._ctx))

    def set_graceful_degradation(self, enabled: bool):
        self._check(lib().pam_engine_set_graceful_degradation(self._ctx, bool(enabled)))

    def set_max_retries(self, n: int):
        self._check(lib().pam_engine_set_max_retries(self._ctx, int(n)))

    def set_partition_tokens(self, n: int):
        self._check(lib().pam_set_partition_tokens(self._ctx, int(n)))

    def set_decode_kernel(self, choice: int):
        self._check(lib().pam_set_decode_kernel(self._ctx, int(choice)))

    def set_mixed_launch(self, mode: int, prefill_groups: int = 0, decode_groups: int = 0):
        """mixed_step's attention: 0 automatic, 1 separate prefill and decode
        launches, 2 one launch holding both; the one launch's workgroups per part
        (0 = automatic)."""
        self._check(lib().pam_set_mixed_launch(self._ctx, int(mode), int(prefill_groups), int(decode_groups)))

    def set_fused_prefill_one_kernel(self, one_kernel: bool):
        """fused_prefill for f16 with d = 128: append then prefill (False, the
        default) or the one kernel that appends as it reads (True)."""
        self._check(lib().pam_set_fused_prefill_kernel(self._ctx, bool(one_kernel)))

    def set_gpu_timing(self, enabled: bool):
        """HIP-event timing of every call (last_stats times); off: no events, times -1."""
        self._check(lib().pam_set_gpu_timing(self._ctx, bool(enabled)))

    def reserve_workspace(self, nbytes: int):
        self._check(lib().pam_reserve_workspace(self._ctx, int(nbytes)))

    # --- code-object loading (the reference's pipeline manager, PagedAttentionEngine.swift:151-198)
    def load_module(self, path: str = None):
        """Launch the code object's entries (hipModuleLoad / hipModuleLaunchKernel);
        default: libpam_kernels.hsaco beside libpam.so."""
        path = path or lib().pam_module_default_path().decode()
        self._check(lib().pam_module_load(self._ctx, path.encode()))

    def unload_module(self):
        self._check(lib().pam_module_unload(self._ctx))

    def set_module_strict(self, strict: bool):
        """Strict: launches the loaded code object has no entry for fail instead of
        running the library's kernel."""
        self._check(lib().pam_module_set_strict(self._ctx, int(bool(strict))))

    def module_function(self, name: str) -> int:
        f = C.c_void_p()
        self._check(lib().pam_module_function(self._ctx, name.encode(), C.byref(f)))
        return f.value

    def module_launch(self, function: int, grid, block, args: bytes, shared_bytes: int = 0):
        """Launch a code-object entry with its packed kernel arguments on the engine's stream."""
        g = tuple(grid) + (1,) * (3 - len(grid))
        b = tuple(block) + (1,) * (3 - len(block))
        buf = C.create_string_buffer(bytes(args), len(args))
        self._check(lib().pam_module_launch(self._ctx, function, *g, *b, int(shared_bytes), buf, len(args)))

    def debug_fail_next_launches(self, n: int):
        self._check(lib().pam_debug_fail_next_launches(self._ctx, int(n)))

    def debug_dirty_counters(self, arrivals: int):
        """Test hook: leave every split-merge counter as an abandoned launch would."""
        self._check(lib().pam_debug_dirty_counters(self._ctx, int(arrivals)))

    # --- splitThreshold / defaultWindowSize / defaultChunkSize (PagedAttentionEngine.swift:116-121)
    def _config(self) -> _lib.EngineConfig:
        c = _lib.EngineConfig()
        self._check(lib().pam_engine_get_config(self._ctx, C.byref(c)))
        return c

    def _set_config(self, **kw):
        c = self._config()
        for k, v in kw.items():
            setattr(c, k, int(v))
        self._check(lib().pam_engine_set_config(self._ctx, C.byref(c)))

    @property
    def split_threshold(self) -> int:
        """Tokens above which a prefill may run the multi-pass (split) form."""
        return self._config().split_threshold

    @split_threshold.setter
    def split_threshold(self, v: int):
        self._set_config(split_threshold=v)

    @property
    def default_window_size(self) -> int:
        return self._config().default_window_size

    @default_window_size.setter
    def default_window_size(self, v: int):
        self._set_config(default_window_size=v)

    @property
    def default_chunk_size(self) -> int:
        return self._config().default_chunk_size

    @default_chunk_size.setter
    def default_chunk_size(self, v: int):
        self._set_config(default_chunk_size=v)

    @property
    def last_stats(self) -> dict:
        s = _lib.Stats()
        self._check(lib().pam_engine_last_stats(self._ctx, C.byref(s)))
        return {f: getattr(s, f) for f, _ in _lib.Stats._fields_}

    # --- PagedAttentionEngine.decode (PagedAttentionEngine.swift:533-546)
    def decode(self, q, k_pool, v_pool, block_tables, seq_lengths, output, batch_size, max_num_blocks,
               layer: PagedLayerSpec, k_scale=None, v_scale=None):
        r = _lib.DecodeRequest(
            _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(block_tables), _ptr(seq_lengths), _ptr(output), int(batch_size),
            int(max_num_blocks), layer.c(), _ptr(k_scale), _ptr(v_scale), _nbytes(q), _nbytes(k_pool),
            _nbytes(v_pool), _nbytes(block_tables), _nbytes(seq_lengths), _nbytes(output))
        self._check(lib().pam_engine_decode(self._ctx, C.byref(r)))

    # --- PagedAttentionEngine.prefill (PagedAttentionEngine.swift:405-418) + query offset
    def prefill(self, q, k_pool, v_pool, block_table, output, seq_len, layer: PagedLayerSpec, causal=True,
                q_offset=0, k_scale=None, v_scale=None):
        r = _lib.PrefillRequest(
            _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(block_table), _ptr(output), int(seq_len), int(q_offset),
            layer.c(), bool(causal), _ptr(k_scale), _ptr(v_scale), _nbytes(q), _nbytes(k_pool), _nbytes(v_pool),
            _nbytes(block_table), _nbytes(output))
        self._check(lib().pam_engine_prefill(self._ctx, C.byref(r)))

    # --- PagedAttentionEngine.appendToCache (PagedAttentionEngine.swift:585-597)
    def append_to_cache(self, keys, values, k_pool, v_pool, block_table, token_offset, num_new_tokens,
                        layer: PagedLayerSpec, k_scale=None, v_scale=None, slot_mapping=None):
        r = _lib.AppendRequest(
            _ptr(keys), _ptr(values), _ptr(k_pool), _ptr(v_pool), _ptr(block_table), int(token_offset),
            int(num_new_tokens), layer.c(), _ptr(k_scale), _ptr(v_scale), _ptr(slot_mapping), _nbytes(keys),
            _nbytes(values), _nbytes(k_pool), _nbytes(v_pool), _nbytes(block_table))
        self._check(lib().pam_engine_append(self._ctx, C.byref(r)))

    # --- PagedAttentionEngine.fusedPrefill (PagedAttentionEngine.swift:633-710)
    def fused_prefill(self, q, raw_k, raw_v, block_table, k_pool, v_pool, output, seq_len, layer: PagedLayerSpec,
                      causal=True, k_scale=None, v_scale=None):
        """Append raw K/V rows 0 .. seq_len-1 into the pool and prefill over them, in one call."""
        r = _lib.FusedPrefillRequest(
            _ptr(q), _ptr(raw_k), _ptr(raw_v), _ptr(block_table), _ptr(k_pool), _ptr(v_pool), _ptr(output),
            int(seq_len), layer.c(), bool(causal), _ptr(k_scale), _ptr(v_scale), _nbytes(q), _nbytes(raw_k),
            _nbytes(raw_v), _nbytes(k_pool), _nbytes(v_pool), _nbytes(block_table), _nbytes(output))
        self._check(lib().pam_engine_fused_prefill(self._ctx, C.byref(r)))

    # --- PagedAttentionEngine.backward (PagedAttentionEngine.swift:1340-1396)
    def backward(self, q, k_pool, v_pool, block_table, d_out, m, l, d_q, d_k_pool, d_v_pool, seq_len,
                 layer: PagedLayerSpec):
        """Gradients of non-causal paged attention: d_q written, d_k_pool / d_v_pool accumulated."""
        r = _lib.BackwardRequest(_ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(block_table), _ptr(d_out), _ptr(m),
                                 _ptr(l), _ptr(d_q), _ptr(d_k_pool), _ptr(d_v_pool), int(seq_len), layer.c())
        self._check(lib().pam_engine_backward(self._ctx, C.byref(r)))

    # --- the flat overloads (PagedAttentionEngine.swift:713-760, 1012-1046, 1167-1201):
    # the layer is built from the arguments, its window is window_size or
    # defaultWindowSize; prefill's chunk_size (or defaultChunkSize) runs the chunk loop
    def prefill_flat(self, q, k_pool, v_pool, block_table, seq_len, head_dim, num_heads, num_kv_heads, block_size,
                     output, causal=True, data_type=PagedAttentionDataType.float16, window_size=0, chunk_size=0,
                     k_scale=None, v_scale=None):
        layer = PagedLayerSpec(head_dim, num_heads, num_kv_heads, block_size, data_type)
        r = _lib.PrefillRequest(
            _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(block_table), _ptr(output), int(seq_len), 0, layer.c(),
            bool(causal), _ptr(k_scale), _ptr(v_scale), _nbytes(q), _nbytes(k_pool), _nbytes(v_pool),
            _nbytes(block_table), _nbytes(output))
        self._check(lib().pam_engine_prefill_flat(self._ctx, C.byref(r), int(window_size), int(chunk_size)))

    def decode_flat(self, q, k_pool, v_pool, block_tables, seq_lengths, batch_size, max_num_blocks, head_dim,
                    num_heads, num_kv_heads, block_size, output, data_type=PagedAttentionDataType.float16,
                    window_size=0, k_scale=None, v_scale=None):
        layer = PagedLayerSpec(head_dim, num_heads, num_kv_heads, block_size, data_type)
        r = _lib.DecodeRequest(
            _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(block_tables), _ptr(seq_lengths), _ptr(output), int(batch_size),
            int(max_num_blocks), layer.c(), _ptr(k_scale), _ptr(v_scale), _nbytes(q), _nbytes(k_pool),
            _nbytes(v_pool), _nbytes(block_tables), _nbytes(seq_lengths), _nbytes(output))
        self._check(lib().pam_engine_decode_flat(self._ctx, C.byref(r), int(window_size)))

    def append_to_cache_flat(self, keys, values, k_pool, v_pool, block_table, token_offset, num_new_tokens,
                             num_heads, num_kv_heads, head_dim, block_size, data_type=PagedAttentionDataType.float16,
                             window_size=0, k_scale=None, v_scale=None):
        layer = PagedLayerSpec(head_dim, num_heads, num_kv_heads, block_size, data_type)
        r = _lib.AppendRequest(
            _ptr(keys), _ptr(values), _ptr(k_pool), _ptr(v_pool), _ptr(block_table), int(token_offset),
            int(num_new_tokens), layer.c(), _ptr(k_scale), _ptr(v_scale), None, _nbytes(keys), _nbytes(values),
            _nbytes(k_pool), _nbytes(v_pool), _nbytes(block_table))
        self._check(lib().pam_engine_append_flat(self._ctx, C.byref(r), int(window_size)))

    # --- multi-layer calls over one shared pool (PagedAttentionEngine.swift:1433-1895)
    @staticmethod
    def _arrays(bufs, layers):
        n = len(layers)
        ptrs = (C.c_void_p * max(n, 1))(*[_ptr(b) for b in bufs])
        sizes = (C.c_size_t * max(n, 1))(*[_nbytes(b) for b in bufs])
        return ptrs, sizes

    def decode_layers(self, q_buffers, k_pool, v_pool, block_tables, seq_lengths, output_buffers, batch_size,
                      max_num_blocks, layers, window_size=0, k_scale=None, v_scale=None):
        """decodeLayers: each layer's Q into its output over the one pool; layers of one
        spec share K/V reads (one launch for up to 16 query heads per kv head)."""
        if len(q_buffers) != len(layers) or len(output_buffers) != len(layers):
            raise PagedAttentionError("Invalid paged attention configuration: buffer/layer count mismatch")
        n = len(layers)
        qp, qs = self._arrays(q_buffers, layers)
        op, os_ = self._arrays(output_buffers, layers)
        specs = (_lib.LayerSpec * max(n, 1))(*[l.c() for l in layers])
        r = _lib.DecodeLayersRequest(
            C.cast(qp, _lib.PP), C.cast(op, _lib.PP), specs, n, _ptr(k_pool), _ptr(v_pool), _ptr(block_tables),
            _ptr(seq_lengths), int(batch_size), int(max_num_blocks), int(window_size), _ptr(k_scale), _ptr(v_scale),
            qs, os_, _nbytes(k_pool), _nbytes(v_pool), _nbytes(block_tables), _nbytes(seq_lengths))
        self._check(lib().pam_engine_decode_layers(self._ctx, C.byref(r)))

    def prefill_layers(self, q_buffers, k_pool, v_pool, block_table, output_buffers, seq_len, layers, causal=True,
                       window_size=0, k_scale=None, v_scale=None):
        """prefillLayers: rows 0 .. seq_len-1 of every layer over the one pool."""
        if len(q_buffers) != len(layers) or len(output_buffers) != len(layers):
            raise PagedAttentionError("Invalid paged attention configuration: buffer/layer count mismatch")
        n = len(layers)
        qp, qs = self._arrays(q_buffers, layers)
        op, os_ = self._arrays(output_buffers, layers)
        specs = (_lib.LayerSpec * max(n, 1))(*[l.c() for l in layers])
        r = _lib.PrefillLayersRequest(
            C.cast(qp, _lib.PP), C.cast(op, _lib.PP), specs, n, _ptr(k_pool), _ptr(v_pool), _ptr(block_table),
            int(seq_len), bool(causal), int(window_size), _ptr(k_scale), _ptr(v_scale), qs, os_, _nbytes(k_pool),
            _nbytes(v_pool), _nbytes(block_table))
        self._check(lib().pam_engine_prefill_layers(self._ctx, C.byref(r)))

    def append_layers(self, keys, values, k_pool, v_pool, block_table, token_offset, num_new_tokens, layers,
                      k_scale_buffers=None, v_scale_buffers=None):
        """appendLayers: every layer's keys/values at the same positions of the one pool, in order."""
        if len(keys) != len(layers) or len(values) != len(layers):
            raise PagedAttentionError("Invalid paged attention configuration: buffer/layer count mismatch")
        if k_scale_buffers is not None and len(k_scale_buffers) != len(layers):
            raise PagedAttentionError("Invalid paged attention configuration: kScaleBuffers count must match "
                                      "layers count")
        if v_scale_buffers is not None and len(v_scale_buffers) != len(layers):
            raise PagedAttentionError("Invalid paged attention configuration: vScaleBuffers count must match "
                                      "layers count")
        n = len(layers)
        kp, ks = self._arrays(keys, layers)
        vp, vs = self._arrays(values, layers)
        specs = (_lib.LayerSpec * max(n, 1))(*[l.c() for l in layers])
        ksp = C.cast(self._arrays(k_scale_buffers, layers)[0], _lib.PP) if k_scale_buffers is not None else None
        vsp = C.cast(self._arrays(v_scale_buffers, layers)[0], _lib.PP) if v_scale_buffers is not None else None
        r = _lib.AppendLayersRequest(
            C.cast(kp, _lib.PP), C.cast(vp, _lib.PP), specs, n, _ptr(k_pool), _ptr(v_pool), _ptr(block_table),
            int(token_offset), int(num_new_tokens), ksp, vsp, ks, vs, _nbytes(k_pool), _nbytes(v_pool),
            _nbytes(block_table))
        self._check(lib().pam_engine_append_layers(self._ctx, C.byref(r)))

    # --- mixed continuous-batching step (no reference counterpart)
    def mixed_step(self, q, output, k_pool, v_pool, block_tables, context_lens, query_lens, layer: PagedLayerSpec,
                   new_keys=None, new_values=None, k_scale=None, v_scale=None):
        import numpy as np
        cl = np.ascontiguousarray(context_lens, dtype=np.int32).reshape(-1)
        ql = np.ascontiguousarray(query_lens, dtype=np.int32).reshape(-1)
        if len(cl) != len(ql):
            raise PagedAttentionError("Invalid paged attention configuration: context_lens and query_lens must "
                                      f"have one entry per sequence ({len(cl)} != {len(ql)}).")
        if block_tables.dim() != 2 or block_tables.shape[0] < len(cl):
            raise PagedAttentionError("Invalid paged attention configuration: block_tables needs one row per "
                                      f"sequence ({len(cl)}).")
        # the library checks every buffer's byte length against the step's rows
        r = _lib.MixedRequest(
            _ptr(q), _ptr(output), _ptr(new_keys), _ptr(new_values), _ptr(k_pool), _ptr(v_pool), _ptr(k_scale),
            _ptr(v_scale), _ptr(block_tables), int(block_tables.shape[1]), len(cl),
            cl.ctypes.data_as(C.c_void_p), ql.ctypes.data_as(C.c_void_p), layer.c(), _nbytes(q), _nbytes(output),
            _nbytes(new_keys), _nbytes(new_values), _nbytes(k_pool), _nbytes(v_pool), _nbytes(block_tables))
        self._check(lib().pam_engine_mixed_step(self._ctx, C.byref(r)))

    # --- calibration streams (achievable HBM rates, counter scaling)
    def calib_stream_read(self, src, blocks=0) -> float:
        ms = C.c_float()
        self._check(lib().pam_calib_stream_read(self._ctx, _ptr(src), _nbytes(src), int(blocks), C.byref(ms)))
        return ms.value

    def calib_mfma(self, iters: int = 60000) -> float:
        """Dense f16 MFMA TFLOP/s the device sustains (pam_calib_mfma)."""
        t = C.c_double()
        self._check(lib().pam_calib_mfma(self._ctx, int(iters), C.byref(t)))
        return t.value

    def synth_normal(self, dst, seed: int, stream: int, stddev: float = 1.0, outlier_stream: int = -1,
                     outlier_frac: float = 0.0):
        """Fill a float32 / float16 device tensor with the counter-based normals of
        (seed, stream) (pam_synth_normal)."""
        import torch
        dt = {torch.float32: 0, torch.float16: 1}.get(dst.dtype)
        if dt is None:
            raise PagedAttentionError("synthetic data is float32 or float16")
        self._check(lib().pam_synth_normal(self._ctx, _ptr(dst), dt, dst.numel(), int(seed) & ((1 << 64) - 1),
                                           int(stream), float(stddev), int(outlier_stream), float(outlier_frac)))

    def calib_stream_copy(self, src, dst, blocks=0) -> float:
        ms = C.c_float()
        self._check(lib().pam_calib_stream_copy(self._ctx, _ptr(src), _ptr(dst), _nbytes(src), int(blocks),
                                                C.byref(ms)))
        return ms.value

    # --- FP8 codec (kernels.metal:553-601), elementwise
    def fp8_quantize(self, values_f16, scales_f16, out_u8):
        self._check(lib().pam_fp8_quantize(self._ctx, _ptr(values_f16), _ptr(scales_f16), _ptr(out_u8),
                                           values_f16.numel()))

    def fp8_dequant(self, codes_u8, scales_f16, out_f16):
        self._check(lib().pam_fp8_dequant(self._ctx, _ptr(codes_u8), _ptr(scales_f16), _ptr(out_f16),
                                          codes_u8.numel()))


class KVCacheManager:
    """KVCacheManager (KVCacheManager.swift:47-379) with pools in HBM.

    ``device=False`` keeps block bookkeeping only (no pools), usable without a GPU.
    """

    def __init__(self, engine: PagedAttentionEngine, max_blocks: int, block_size: int = 16, head_dim: int = 128,
                 num_kv_heads: int = 8, data_type=PagedAttentionDataType.float16, device: bool = True):
        self.engine = engine
        self.max_blocks = max_blocks
        self.block_size = block_size
        self.head_dim = head_dim
        self.num_kv_heads = num_kv_heads
        self.data_type = PagedAttentionDataType(data_type)
        fn = lib().pam_create_cache if device else lib().pam_create_cache_host
        self._cache = fn(engine.handle, max_blocks, block_size, head_dim, num_kv_heads, int(data_type))
        if not self._cache:
            msg = lib().pam_last_error(engine.handle)
            raise PagedAttentionError(msg.decode() if msg else "cache creation failed")

    def close(self):
        if getattr(self, "_cache", None):
            lib().pam_destroy_cache(self._cache)
            self._cache = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._cache

    def _check(self, rc):
        self.engine._check(rc)

    def allocate_sequence(self, sid: int):
        self._check(lib().pam_reserve_sequence(self.engine.handle, self._cache, int(sid)))

    def append_tokens(self, sid: int, count: int, block_hashes=None):
        if block_hashes is None:
            self._check(lib().pam_append_tokens(self.engine.handle, self._cache, int(sid), int(count)))
        else:
            arr = (C.c_uint64 * len(block_hashes))(*[int(h) & (2**64 - 1) for h in block_hashes])
            self._check(lib().pam_append_tokens_hashed(self.engine.handle, self._cache, int(sid), int(count), arr,
                                                       len(block_hashes)))

    def ensure_exclusive_access(self, sid: int, logical_block_index: int):
        self._check(lib().pam_ensure_exclusive(self.engine.handle, self._cache, int(sid), int(logical_block_index)))

    def register_block_hash(self, h: int, physical_block: int):
        if lib().pam_register_block_hash(self._cache, int(h) & (2**64 - 1), int(physical_block)) != 0:
            raise PagedAttentionError("invalid block")

    @property
    def eviction_policy(self):
        return BlockEvictionPolicy(self.memory_stats()["eviction_policy"])

    @eviction_policy.setter
    def eviction_policy(self, p):
        if lib().pam_set_eviction_policy(self._cache, int(p)) != 0:
            raise PagedAttentionError("invalid eviction policy")

    def free_sequence(self, sid: int):
        lib().pam_free_sequence(self._cache, int(sid))

    def get_block_table(self, sid: int):
        n = lib().pam_block_table(self.engine.handle, self._cache, int(sid), None, 0)
        self._check(0 if n >= 0 else -1)
        buf = (C.c_int32 * max(n, 1))()
        lib().pam_block_table(self.engine.handle, self._cache, int(sid), buf, n)
        return list(buf[:n])

    def get_sequence_length(self, sid: int) -> int:
        n = lib().pam_sequence_length(self.engine.handle, self._cache, int(sid))
        self._check(0 if n >= 0 else -1)
        return n

    @property
    def available_blocks(self) -> int:
        return lib().pam_available_blocks(self._cache)

    def memory_stats(self) -> dict:
        s = _lib.MemoryStats()
        if lib().pam_cache_memory_stats(self._cache, C.byref(s)) != 0:
            raise PagedAttentionError("memory stats failed")
        return {f: getattr(s, f) for f, _ in _lib.MemoryStats._fields_}

    def batch_view(self, ids, device_block_tables, device_seq_lengths, max_num_blocks=0) -> int:
        """getBatchBlockTableBuffer + getSeqLengthsBuffer into device tensors."""
        arr = (C.c_int64 * max(len(ids), 1))(*[int(i) for i in ids])
        n = lib().pam_cache_batch_view(self.engine.handle, self._cache, arr, len(ids), int(max_num_blocks),
                                       _ptr(device_block_tables), _ptr(device_seq_lengths))
        self._check(0 if n >= 0 else -1)
        return n

    # pools as torch tensors viewing library-owned HBM
    def _pool_shape(self):
        return (self.max_blocks, self.block_size, self.num_kv_heads, self.head_dim)

    def k_pool(self):
        import torch
        ts = {0: "<f4", 1: "<f2", 2: "|u1"}[int(self.data_type)]
        return torch.as_tensor(_DeviceArray(lib().pam_cache_k_pool(self._cache), self._pool_shape(), ts),
                               device="cuda")

    def v_pool(self):
        import torch
        ts = {0: "<f4", 1: "<f2", 2: "|u1"}[int(self.data_type)]
        return torch.as_tensor(_DeviceArray(lib().pam_cache_v_pool(self._cache), self._pool_shape(), ts),
                               device="cuda")

    def k_scale(self):
        import torch
        p = lib().pam_cache_k_scale(self._cache)
        return None if not p else torch.as_tensor(_DeviceArray(p, (self.max_blocks,), "<f2"), device="cuda")

    def v_scale(self):
        import torch
        p = lib().pam_cache_v_scale(self._cache)
        return None if not p else torch.as_tensor(_DeviceArray(p, (self.max_blocks,), "<f2"), device="cuda")


class SequenceStatus(IntEnum):
    """Scheduler.swift:5-10"""
    waiting = 0
    running = 1
    paused = 2
    completed = 3


class ContinuousBatchingScheduler:
    """ContinuousBatchingScheduler (Scheduler.swift:42-177), native in libpam."""

    def __init__(self, max_batch_size: int, max_sequences: int = 128):
        self.max_batch_size = max_batch_size
        self.max_sequences = max_sequences
        self._s = lib().pam_scheduler_create(max_batch_size, max_sequences)

    def __del__(self):
        try:
            if self._s:
                lib().pam_scheduler_destroy(self._s)
                self._s = None
        except Exception:
            pass

    def add_request(self, prompt_token_count: int, max_new_tokens: int) -> int:
        return lib().pam_scheduler_add_request(self._s, int(prompt_token_count), int(max_new_tokens))

    def complete_sequence(self, sid: int):
        lib().pam_scheduler_complete(self._s, int(sid))

    def step(self):
        buf = (C.c_int32 * max(self.max_batch_size, 1))()
        n = lib().pam_scheduler_step(self._s, buf, self.max_batch_size)
        return list(buf[:n])

    def mark_prefilled(self, sid):
        lib().pam_scheduler_mark_prefilled(self._s, int(sid))

    def mark_decoded(self, sid):
        lib().pam_scheduler_mark_decoded(self._s, int(sid))

    def preempt_sequence(self, sid):
        lib().pam_scheduler_preempt(self._s, int(sid))

    def handle_memory_pressure(self, required_blocks: int, cache: KVCacheManager):
        # every victim was running, and at most max_sequences sequences exist, so
        # the buffer holds all of them (a second call could not return them:
        # they are already paused)
        cap = max(1, self.max_sequences)
        buf = (C.c_int32 * cap)()
        n = lib().pam_scheduler_handle_memory_pressure(self._s, int(required_blocks), cache.handle, buf, cap)
        if n > cap:
            raise PagedAttentionError(f"memory pressure preempted {n} sequences, more than max_sequences ({cap})")
        return list(buf[:n])

    def count(self, status: SequenceStatus) -> int:
        return lib().pam_scheduler_count(self._s, int(status))

    @property
    def waiting_count(self):
        return self.count(SequenceStatus.waiting)

    @property
    def running_count(self):
        return self.count(SequenceStatus.running)

    @property
    def completed_count(self):
        return self.count(SequenceStatus.completed)

    def sequence(self, sid: int):
        st, gen, pr = C.c_int32(), C.c_int32(), C.c_int32()
        if lib().pam_scheduler_sequence(self._s, int(sid), C.byref(st), C.byref(gen), C.byref(pr)) != 0:
            return None
        return {"status": SequenceStatus(st.value), "generated": gen.value, "prompt": pr.value}
