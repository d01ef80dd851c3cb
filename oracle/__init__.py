"""CPU oracle for the paged-attention path (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker.  The product
(``pagedattentionmetal_amd`` + ``libpam.so``) never imports it.

The numerics live in ``pam_oracle.c`` (built by ``oracle/Makefile`` into
``oracle/_build/libpam_oracle.so``); this module wraps it for numpy arrays.
Host-logic restatements (block allocator, scheduler) are in ``allocator.py`` and
``scheduler.py``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libpam_oracle.so")
_lib = None


def build() -> str:
    """Compile the C oracle (gcc) into oracle/_build/."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        P = C.c_void_p
        i32, u16, f32 = C.c_int32, C.c_uint16, C.c_float
        L.pamo_f32_to_f16.argtypes, L.pamo_f32_to_f16.restype = [f32], u16
        L.pamo_f16_to_f32.argtypes, L.pamo_f16_to_f32.restype = [u16], f32
        L.pamo_quantize_fp8.argtypes, L.pamo_quantize_fp8.restype = [u16, u16], C.c_uint8
        L.pamo_dequant_fp8.argtypes, L.pamo_dequant_fp8.restype = [C.c_uint8, u16], u16
        L.pamo_fp8_scale.argtypes, L.pamo_fp8_scale.restype = [f32, u16], u16
        L.pamo_quantize_fp8_n.argtypes, L.pamo_quantize_fp8_n.restype = [P, P, P, C.c_int64], None
        L.pamo_dequant_fp8_n.argtypes, L.pamo_dequant_fp8_n.restype = [P, P, P, C.c_int64], None
        L.pamo_slot.argtypes, L.pamo_slot.restype = [P, C.c_int64, i32], C.c_int64
        L.pamo_append.argtypes = [C.c_int, P, P, P, P, P, P, P, i32, i32, i32, i32, i32, i32]
        L.pamo_append.restype = C.c_int
        L.pamo_sim_forward.argtypes = [P, P, P, P, i32, i32, i32, i32, P, P, P]
        L.pamo_sim_forward.restype = None
        L.pamo_decode.argtypes = [C.c_int, P, P, P, P, P, P, P, i32, i32, i32, i32, i32, i32, i32, P, C.c_int]
        L.pamo_decode.restype = C.c_int
        L.pamo_prefill.argtypes = [C.c_int, P, P, P, P, P, P, i32, i32, i32, i32, i32, i32, i32, i32, i32, P,
                                   C.c_int]
        L.pamo_prefill.restype = C.c_int
        L.pamo_merge.argtypes = [i32, P, P, P, i32, P]
        L.pamo_merge.restype = None
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ----------------------------------------------------------------- codec helpers

def quantize_fp8(values_f16: np.ndarray, scales_f16) -> np.ndarray:
    """kernels.metal:564-601, elementwise over half inputs and (broadcast) half scales."""
    v = _c(values_f16, np.float16)
    s = np.ascontiguousarray(np.broadcast_to(np.asarray(scales_f16, dtype=np.float16), v.shape))
    out = np.empty(v.shape, np.uint8)
    lib().pamo_quantize_fp8_n(_p(v), _p(s), _p(out), v.size)
    return out


def dequant_fp8(codes: np.ndarray, scales_f16) -> np.ndarray:
    """kernels.metal:553-562 (half arithmetic), elementwise, returns float16."""
    c = _c(codes, np.uint8)
    s = np.ascontiguousarray(np.broadcast_to(np.asarray(scales_f16, dtype=np.float16), c.shape))
    out = np.empty(c.shape, np.float16)
    lib().pamo_dequant_fp8_n(_p(c), _p(s), _p(out), c.size)
    return out


def dequant_pool(pool_u8: np.ndarray, scales_f16: np.ndarray) -> np.ndarray:
    """Dequantise a [nb][bs][Hkv][d] byte pool with per-block scales -> float16."""
    sc = _c(scales_f16, np.float16).reshape((-1,) + (1,) * (pool_u8.ndim - 1))
    return dequant_fp8(pool_u8, sc)


def fp8_scale(new_max_abs: float, old_scale_f16) -> np.float16:
    s = int(np.asarray(old_scale_f16, dtype=np.float16).view(np.uint16))
    return np.array([lib().pamo_fp8_scale(float(new_max_abs), s)], dtype=np.uint16).view(np.float16)[0]


# ----------------------------------------------------------------- append

def append(dtype: int, keys, values, k_pool, v_pool, block_table, token_offset: int,
           k_scale=None, v_scale=None):
    """In-place KV append (kernels.metal:1804-1961). keys/values [n][Hkv][d]."""
    n, hkv, d = keys.shape
    bs = k_pool.shape[1]
    bt = _c(block_table, np.int32)
    rc = lib().pamo_append(dtype, _p(keys), _p(values), _p(k_pool), _p(v_pool),
                           _p(k_scale), _p(v_scale), _p(bt), len(bt), int(token_offset), n, hkv, d, bs)
    if rc != 0:
        raise IndexError("block table too short for append")


def slot(block_table, pos: int, block_size: int) -> int:
    bt = _c(block_table, np.int32)
    return int(lib().pamo_slot(_p(bt), int(pos), int(block_size)))


# ----------------------------------------------------------------- attention

def sim_forward(q, k_pool, v_pool, block_table, block_size):
    """Reference/paged_attention_sim.py:12-138 restated in C (fp64).  Returns
    (output [S][d], m_history [nlb][S], l_history [nlb][S])."""
    q = _c(q, np.float32)
    k_pool = _c(k_pool, np.float32)
    v_pool = _c(v_pool, np.float32)
    bt = _c(block_table, np.int32)
    S, d = q.shape
    out = np.empty((S, d), np.float64)
    mh = np.empty((len(bt), S), np.float64)
    lh = np.empty((len(bt), S), np.float64)
    lib().pamo_sim_forward(_p(q), _p(k_pool), _p(v_pool), _p(bt), len(bt), S, block_size, d,
                           _p(out), _p(mh), _p(lh))
    return out, mh, lh


def decode(dtype, q, k_pool, v_pool, block_tables, seq_lengths, num_heads, window=0,
           k_scale=None, v_scale=None, n_threads=1):
    """Batched paged decode -> fp64 [B][H][d]."""
    nb, bs, hkv, d = k_pool.shape
    bt = _c(block_tables, np.int32)
    B, max_nb = bt.shape
    sl = _c(seq_lengths, np.uint32)
    out = np.empty((B, num_heads, d), np.float64)
    rc = lib().pamo_decode(dtype, _p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(k_pool)),
                           _p(np.ascontiguousarray(v_pool)), _p(k_scale), _p(v_scale), _p(bt), _p(sl),
                           B, max_nb, num_heads, hkv, d, bs, int(window), _p(out), int(n_threads))
    assert rc == 0
    return out


def prefill(dtype, q, k_pool, v_pool, block_table, q_offset, causal=True, window=0,
            k_scale=None, v_scale=None, n_threads=1):
    """Prefill rows [q_offset, q_offset+T) of one sequence -> fp64 [T][H][d]."""
    nb, bs, hkv, d = k_pool.shape
    T, H, _ = q.shape
    bt = _c(block_table, np.int32)
    out = np.empty((T, H, d), np.float64)
    rc = lib().pamo_prefill(dtype, _p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(k_pool)),
                            _p(np.ascontiguousarray(v_pool)), _p(k_scale), _p(v_scale), _p(bt), len(bt),
                            int(q_offset), T, H, hkv, d, bs, int(window), int(bool(causal)), _p(out),
                            int(n_threads))
    if rc != 0:
        raise IndexError("block table too short for prefill")
    return out


def merge(m, l, o):
    """LSE merge of P partial states: m [P] (natural log), l [P], o [P][d]."""
    m = _c(m, np.float64)
    l = _c(l, np.float64)
    o = _c(o, np.float64)
    out = np.empty(o.shape[1], np.float64)
    lib().pamo_merge(len(m), _p(m), _p(l), _p(o), o.shape[1], _p(out))
    return out


def _gather_rows(pool, block_table, seq_len):
    """Pool rows of tokens 0 .. seq_len-1 of one sequence: [seq_len][Hkv][d] fp64."""
    nb, bs, hkv, d = pool.shape
    j = np.arange(seq_len)
    return pool[np.asarray(block_table)[j // bs], j % bs].astype(np.float64)


def forward_stats(q, k_pool, v_pool, block_table, window=0):
    """Row max m and sum l (natural-log units, scores scaled by 1/sqrt(d)) of the
    non-causal attention the backward differentiates (rows 0 .. T-1 over keys
    [max(0, T - W), T)), as the forward's online softmax leaves them
    (kernels.metal:1217-1260 reads them as inputs).  Returns (m, l, O) in fp64."""
    T, H, d = q.shape
    hkv = k_pool.shape[2]
    G = H // hkv
    ws = max(0, T - window) if window > 0 else 0
    K = _gather_rows(k_pool, block_table, T)[ws:]
    V = _gather_rows(v_pool, block_table, T)[ws:]
    qf = q.astype(np.float64)
    m = np.empty((T, H))
    l = np.empty((T, H))
    o = np.empty((T, H, d))
    for h in range(H):
        s = qf[:, h] @ K[:, h // G].T / np.sqrt(d)
        m[:, h] = s.max(1)
        e = np.exp(s - m[:, h:h + 1])
        l[:, h] = e.sum(1)
        o[:, h] = e @ V[:, h // G] / l[:, h:h + 1]
    return m, l, o


def backward(q, k_pool, v_pool, block_table, d_out, m, l, window=0):
    """Gradients of paged attention (kernels.metal:1217-1314, paged_attention_backward):
    with P = exp(s - m) / l over keys [max(0, T - W), T), dP = dO V^T,
    D = rowsum(P * dP), dS = P (dP - D):
      dQ = scale dS K;  dK_j = scale sum_i dS_ij q_i;  dV_j = sum_i P_ij dO_i,
    the key gradients summed over the query heads of each kv head.  Returns
    (dQ [T][H][d], dK [T][Hkv][d], dV [T][Hkv][d]) in fp64; keys before the window
    get zero.  Pinned by central finite differences of the dense forward."""
    T, H, d = q.shape
    hkv = k_pool.shape[2]
    G = H // hkv
    ws = max(0, T - window) if window > 0 else 0
    K = _gather_rows(k_pool, block_table, T)
    V = _gather_rows(v_pool, block_table, T)
    qf, go = q.astype(np.float64), d_out.astype(np.float64)
    sc = 1.0 / np.sqrt(d)
    dq = np.zeros((T, H, d))
    dk = np.zeros((T, hkv, d))
    dv = np.zeros((T, hkv, d))
    for h in range(H):
        g = h // G
        s = qf[:, h] @ K[ws:, g].T * sc
        P = np.exp(s - np.asarray(m, np.float64)[:, h:h + 1]) / np.asarray(l, np.float64)[:, h:h + 1]
        dP = go[:, h] @ V[ws:, g].T
        D = (P * dP).sum(1, keepdims=True)
        dS = P * (dP - D)
        dq[:, h] = sc * dS @ K[ws:, g]
        dk[ws:, g] += sc * dS.T @ qf[:, h]
        dv[ws:, g] += P.T @ go[:, h]
    return dq, dk, dv
