"""Framework-facing KV cache: the semantics of the reference's MLX adapter
``PagedMetalKVCache`` (Sources/PagedAttentionMLXSupport/PagedMetalKVCache.swift:27-202)
for torch tensors in HBM.

One cache object holds one sequence.  ``paged_attention`` takes the attention
call of a model layer in the framework's layout (queries ``[B, H, S, d]``, keys
and values ``[B, Hkv, S, d]``), appends the new keys and values to the paged
pool at the current offset and runs decode (S = 1) or prefill (S > 1) through
libpam, returning ``[B, H, S, d]``.  Masks: ``"none"`` or ``"causal"``; a
materialised mask is refused, as in the reference (PagedMetalKVCache.swift:279-286).

``paged_attention_with_cache_update`` mirrors ``pagedAttentionWithCacheUpdate``
(PagedMetalKVCache.swift:244-264): it uses the paged path when the cache is a
``PagedTorchKVCache`` and the scale is 1/sqrt(d); otherwise it calls the
``fallback`` the caller passes (the framework's own attention, MLX's
``attentionWithCacheUpdate`` in the reference).  There is no built-in fallback.

Differences from the reference, both deliberate:
* a prompt that arrives in several chunks attends with its query offset (rows
  [offset, offset + S) of a causal prefill); the reference's adapter passes no
  offset, so its second chunk would attend over the sequence's first S tokens;
* FP8 caches work (queries and outputs in f16); the reference's adapter raises
  for FP8 when it converts the output.
"""
from __future__ import annotations

import ctypes as C

from . import api
from .api import PagedAttentionDataType, PagedAttentionError, PagedLayerSpec


class UnsupportedShape(PagedAttentionError):
    """PagedAttentionMLXError.unsupportedShape (PagedMetalKVCache.swift:10)"""


class UnsupportedMask(PagedAttentionError):
    """PagedAttentionMLXError.unsupportedMask (PagedMetalKVCache.swift:12)"""


def make_mask(n: int, offset: int, window_size=None, return_array: bool = False):
    """Mask mode for n new tokens after `offset` cached ones (PagedMetalKVCache.swift:178-190):
    "none" for one token; a boolean [n, offset + n] array (True = attend) when one is
    asked for or the window is shorter than n; "causal" otherwise.  The array is the
    causal window mask j <= offset + i < j + window_size."""
    if n == 1:
        return "none"
    if return_array or (window_size is not None and n > window_size):
        import torch
        rows = torch.arange(offset, offset + n)[:, None]
        cols = torch.arange(0, offset + n)[None, :]
        mask = rows >= cols
        if window_size is not None:
            mask &= rows < cols + window_size
        return mask
    return "causal"


def _is_tensor_mask(mask) -> bool:
    return not isinstance(mask, str)


class PagedTorchKVCache:
    """One sequence's paged KV cache behind a framework attention call
    (PagedMetalKVCache, PagedMetalKVCache.swift:27-62)."""

    def __init__(self, sequence_id: int, layer: PagedLayerSpec, max_blocks: int,
                 engine: api.PagedAttentionEngine | None = None):
        layer.validate()
        owns = engine is None
        if engine is None:
            # its own engine enqueues on the caller's current torch stream and
            # returns at once: the outputs are ordered after the inputs by the stream
            import torch
            engine = api.PagedAttentionEngine()
            engine.set_stream(torch.cuda.current_stream())
            engine.synchronous = False
            engine.set_gpu_timing(False)  # a serving loop: no per-call timing events
            self._stream = torch.cuda.current_stream().cuda_stream
        self._own_engine = owns
        self.engine = engine
        self.sequence_id = int(sequence_id)
        self.layer = layer
        self.cache_manager = api.KVCacheManager(self.engine, max_blocks, layer.block_size, layer.head_dim,
                                                layer.num_kv_heads, layer.data_type)
        self.cache_manager.allocate_sequence(self.sequence_id)
        self.offset = 0
        self._step = api.lib().pam_decode_step
        # the decode step's shapes and type ([1, H, 1, d] queries, [1, Hkv, 1, d]
        # keys and values): calls with exactly these take the short path of
        # paged_attention
        import torch
        self._io = torch.float32 if layer.data_type == PagedAttentionDataType.float32 else torch.float16
        self._q1 = torch.Size([1, layer.num_heads, 1, layer.head_dim])
        self._kv1 = torch.Size([1, layer.num_kv_heads, 1, layer.head_dim])
        self._short = layer.data_type != PagedAttentionDataType.float8

    # metaState (PagedMetalKVCache.swift:158-167)
    @property
    def meta_state(self):
        return ["paged-hip", str(self.sequence_id), str(self.offset), str(self.layer.block_size)]

    @meta_state.setter
    def meta_state(self, value):
        if len(value) >= 3:
            self.offset = int(value[2])

    is_trimmable = False

    def trim(self, n: int) -> int:
        return 0

    def make_mask(self, n: int, window_size=None, return_array: bool = False):
        return make_mask(n, self.offset, window_size, return_array)

    def paged_attention(self, queries, keys, values, mask="none"):
        """pagedAttention(queries:keys:values:mask:) (PagedMetalKVCache.swift:74-154)."""
        import torch
        if self._own_engine:
            # the cache's own engine follows the caller's current stream, so its
            # kernels stay ordered after the producers of the inputs and before
            # the consumers of the output (and the allocator's reuse of both)
            cur_stream = torch.cuda.current_stream().cuda_stream
            if cur_stream != self._stream:
                self.engine.set_stream(cur_stream)
                self._stream = cur_stream
        io = self._io
        if (self._short and isinstance(mask, str) and (mask == "none" or mask == "causal") and
                queries.shape == self._q1 and keys.shape == self._kv1 and values.shape == self._kv1 and
                queries.dtype == io and keys.dtype == io and values.dtype == io and queries.is_contiguous() and
                keys.is_contiguous() and values.is_contiguous()):
            # a decode step in one library call (pam_decode_step): bookkeeping,
            # the token's K/V append and the decode; the block table and length
            # stay on the device between steps.  [1, heads, 1, d] holds the same
            # bytes as [heads, d].
            out = torch.empty(self._q1, dtype=io, device=queries.device)
            rc = self._step(self.engine.handle, self.cache_manager.handle, self.sequence_id, keys.data_ptr(),
                            values.data_ptr(), queries.data_ptr(), out.data_ptr(), self.layer.num_heads)
            if rc != 0:
                self.engine._check(rc)
            self.offset += 1
            return out
        if _is_tensor_mask(mask):
            raise UnsupportedMask("materialized masks fall back to native attention")
        if mask not in ("none", "causal"):
            raise UnsupportedMask(f"unknown mask mode {mask!r}")
        L = self.layer
        if queries.dim() != 4:
            raise UnsupportedShape(f"queries must be [B, heads, seqLen, headDim]; got {list(queries.shape)}")
        B, H, S, d = queries.shape
        if B != 1:
            raise UnsupportedShape(f"PagedTorchKVCache supports batch size 1; got {B}.")
        if H != L.num_heads or d != L.head_dim:
            raise UnsupportedShape(f"queries are [{B}, {H}, {S}, {d}], expected heads={L.num_heads}, "
                                   f"headDim={L.head_dim}.")
        for name, t in (("keys", keys), ("values", values)):
            if t.dim() != 4:
                raise UnsupportedShape(f"{name} must be [B, kvHeads, seqLen, headDim]; got {list(t.shape)}")
            if t.shape[1] != L.num_kv_heads or t.shape[2] != S or t.shape[3] != L.head_dim:
                raise UnsupportedShape(f"keys/values must match seqLen={S}, kvHeads={L.num_kv_heads}, "
                                       f"headDim={L.head_dim}.")
        cm = self.cache_manager
        cur = self.offset
        if S == 1 and L.data_type != PagedAttentionDataType.float8:
            # a decode step in one library call (pam_decode_step): bookkeeping,
            # the token's K/V append and the decode; the block table and length
            # stay on the device between steps
            def flat(t, rows):
                if t.dtype == io and t.is_contiguous():
                    return t.view(rows, d)
                return t[0, :, 0].to(io).contiguous()
            k, v, q = flat(keys, L.num_kv_heads), flat(values, L.num_kv_heads), flat(queries, H)
            out = torch.empty((H, d), dtype=io, device=queries.device)
            rc = self._step(self.engine.handle, cm.handle, self.sequence_id, k.data_ptr(), v.data_ptr(),
                            q.data_ptr(), out.data_ptr(), H)
            if rc != 0:
                self.engine._check(rc)
            self.offset += 1
            out = out.view(1, H, 1, d)
            return out if out.dtype == queries.dtype else out.to(queries.dtype)
        cm.append_tokens(self.sequence_id, S)
        if S == 1:
            # FP8 caches: the cache's own calls (pam_append_kv, pam_decode)
            k = keys[0, :, 0].to(io).contiguous()    # [Hkv, d]
            v = values[0, :, 0].to(io).contiguous()
            q = queries[0, :, 0].to(io).contiguous()  # [H, d]
            out = torch.empty_like(q)
            self.engine._check(api.lib().pam_append_kv(self.engine.handle, cm.handle, self.sequence_id,
                                                       k.data_ptr(), v.data_ptr(), cur, 1, L.num_kv_heads))
            ids = (C.c_int64 * 1)(self.sequence_id)
            self.engine._check(api.lib().pam_decode(self.engine.handle, cm.handle, ids, 1, q.data_ptr(),
                                                    out.data_ptr(), L.num_heads))
            self.offset += 1
            return out.view(1, H, 1, d).to(queries.dtype)
        table = cm.get_block_table(self.sequence_id)
        bt = torch.tensor(table if table else [0], dtype=torch.int32, device=queries.device)
        k = keys[0].transpose(0, 1).to(io).contiguous()    # [S, Hkv, d]
        v = values[0].transpose(0, 1).to(io).contiguous()
        kp, vp, ks, vs = cm.k_pool(), cm.v_pool(), cm.k_scale(), cm.v_scale()
        self.engine.append_to_cache(k, v, kp, vp, bt, cur, S, L, k_scale=ks, v_scale=vs)
        self.offset += S
        q = queries[0].transpose(0, 1).to(io).contiguous()  # [S, H, d]
        out = torch.empty_like(q)
        if S == 1:
            lens = torch.tensor([self.offset], dtype=torch.int32, device=queries.device)
            self.engine.decode(q, kp, vp, bt.view(1, -1), lens, out, 1, bt.numel(), L, k_scale=ks, v_scale=vs)
        else:
            self.engine.prefill(q, kp, vp, bt, out, S, L, causal=(mask == "causal"), q_offset=cur,
                                k_scale=ks, v_scale=vs)
        return out.transpose(0, 1).unsqueeze(0).to(queries.dtype)


def paged_attention_with_cache_update(queries, keys, values, cache, scale: float, mask="none", fallback=None):
    """pagedAttentionWithCacheUpdate (PagedMetalKVCache.swift:244-264).  `fallback`
    (queries, keys, values, cache, scale, mask) -> output is the caller's own
    attention, used when the paged path does not apply or refuses the call."""
    if isinstance(cache, PagedTorchKVCache) and abs(scale - cache.layer.head_dim ** -0.5) < 1e-4:
        try:
            return cache.paged_attention(queries, keys, values, mask)
        except PagedAttentionError:
            if fallback is None:
                raise
    if fallback is None:
        raise PagedAttentionError("the paged path does not apply to this call and no fallback was given")
    return fallback(queries, keys, values, cache, scale, mask)
