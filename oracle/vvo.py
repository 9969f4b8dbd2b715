"""ctypes binding of the CPU oracle (oracle/vvo.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker, and by bench.py's cpu_baseline leg.  The product library never
imports this module.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

F32, F16, Q8_0, BF16 = 0, 1, 8, 30
EXACT, GGML, GGML_F32ACC = 0, 1, 2
MASK_NONE, MASK_EXPLICIT, MASK_CAUSAL = 0, 1, 2
THETA_RECURRENCE, THETA_POW = 0, 1
MAX_B = 16

_HERE = os.path.dirname(os.path.abspath(__file__))
# VVO_LIB names another build of the oracle (the sanitized lib/san/libvvo.so)
LIB_PATH = os.environ.get("VVO_LIB") or os.path.join(_HERE, "lib", "libvvo.so")


class AttnArgs(ctypes.Structure):
    _fields_ = [
        ("d", ctypes.c_int32), ("n_q_heads", ctypes.c_int32), ("n_kv_heads", ctypes.c_int32),
        ("T", ctypes.c_int32), ("B", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("k_type", ctypes.c_int32), ("v_type", ctypes.c_int32),
        ("k", ctypes.c_void_p * MAX_B), ("v", ctypes.c_void_p * MAX_B),
        ("L", ctypes.c_int32 * MAX_B), ("past", ctypes.c_int32 * MAX_B),
        ("mask", ctypes.c_void_p),
        ("mask_row_stride", ctypes.c_int64), ("mask_b_stride", ctypes.c_int64),
        ("mask_mode", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("out", ctypes.c_void_p),
        ("mode", ctypes.c_int32), ("q_round", ctypes.c_int32), ("n_threads", ctypes.c_int32),
        ("rows", ctypes.c_void_p), ("n_rows", ctypes.c_int32),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        L.vvo_f32_to_f16.restype = ctypes.c_uint16
        L.vvo_f32_to_f16.argtypes = [ctypes.c_float]
        L.vvo_f16_to_f32.restype = ctypes.c_float
        L.vvo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.vvo_f32_to_bf16.restype = ctypes.c_uint16
        L.vvo_f32_to_bf16.argtypes = [ctypes.c_float]
        L.vvo_bf16_to_f32.restype = ctypes.c_float
        L.vvo_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.vvo_row_bytes.restype = ctypes.c_int64
        L.vvo_row_bytes.argtypes = [ctypes.c_int, ctypes.c_int64]
        L.vvo_from_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int64]
        L.vvo_to_f32.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64]
        L.vvo_quantize_q8_0.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.vvo_dequantize_q8_0.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.vvo_rope_neox.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                    ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                    ctypes.c_float, ctypes.c_int]
        L.vvo_attn.restype = ctypes.c_int
        L.vvo_attn.argtypes = [ctypes.POINTER(AttnArgs)]
        L.vvo_n_cores.restype = ctypes.c_int
        L.vvo_set_simd.restype = None
        L.vvo_set_simd.argtypes = [ctypes.c_int]
        L.vvo_linear.restype = ctypes.c_int
        L.vvo_linear.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                 ctypes.c_int]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def row_bytes(type_: int, n: int) -> int:
    return int(lib().vvo_row_bytes(type_, n))


def from_f32(x: np.ndarray, type_: int) -> np.ndarray:
    """F32 array -> raw bytes of `type_` (last dim converted; Q8_0 needs a multiple of 32)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.size
    out = np.empty(row_bytes(type_, n), dtype=np.uint8)
    lib().vvo_from_f32(_ptr(x), _ptr(out), type_, n)
    return out


def to_f32(buf: np.ndarray, type_: int, n: int) -> np.ndarray:
    buf = np.ascontiguousarray(buf)
    out = np.empty(n, dtype=np.float32)
    lib().vvo_to_f32(_ptr(buf), type_, _ptr(out), n)
    return out


def f16_bits(x: np.ndarray) -> np.ndarray:
    return from_f32(x, F16).view(np.uint16).reshape(np.shape(x))


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return from_f32(x, BF16).view(np.uint16).reshape(np.shape(x))


def rope(x: np.ndarray, pos: np.ndarray, base: float = 1.0e6, mode: int = THETA_RECURRENCE) -> np.ndarray:
    """x: [B, T, H, d] f32; pos: [T] or [B, T] int32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    B, T, H, d = x.shape
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    stride_b = 0 if pos.ndim == 1 else T
    y = np.empty_like(x)
    lib().vvo_rope_neox(_ptr(x), _ptr(y), _ptr(pos), stride_b, d, H, T, B, base, mode)
    return y


def attn(q: np.ndarray, k_caches, v_caches, k_type: int, v_type: int, L, *, n_kv_heads: int,
         scale: float, mask_mode: int = MASK_CAUSAL, past=None, mask: np.ndarray | None = None,
         mode: int = EXACT, q_round: int = 1, n_threads: int = 0, rows=None) -> np.ndarray:
    """q: [B, T, Hq, d] f32.  k_caches/v_caches: per-batch raw byte arrays holding rows
    [L_b][Hkv][d] of k_type/v_type.  mask (explicit): f16 bits [B or 1, T, Lm]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, T, Hq, d = q.shape
    a = AttnArgs()
    a.d, a.n_q_heads, a.n_kv_heads, a.T, a.B = d, Hq, n_kv_heads, T, B
    a.q = _ptr(q)
    a.k_type, a.v_type = k_type, v_type
    keep = [q]
    for b in range(B):
        kc = np.ascontiguousarray(k_caches[b])
        vc = np.ascontiguousarray(v_caches[b])
        keep += [kc, vc]
        a.k[b] = _ptr(kc)
        a.v[b] = _ptr(vc)
        a.L[b] = int(L[b])
        a.past[b] = int(past[b]) if past is not None else int(L[b]) - T
    if mask is not None:
        m = np.ascontiguousarray(mask, dtype=np.uint16)
        keep.append(m)
        a.mask = _ptr(m)
        a.mask_row_stride = m.shape[-1]
        a.mask_b_stride = 0 if m.shape[0] == 1 else m.shape[-1] * m.shape[-2]
    a.mask_mode = mask_mode
    a.scale = scale
    out = np.zeros((B, T, Hq, d), dtype=np.float32)
    a.out = _ptr(out)
    a.mode, a.q_round, a.n_threads = mode, q_round, n_threads
    if rows is not None:
        r = np.ascontiguousarray(rows, dtype=np.int32)
        keep.append(r)
        a.rows = _ptr(r)
        a.n_rows = r.size
    rc = lib().vvo_attn(ctypes.byref(a))
    if rc != 0:
        raise RuntimeError(f"vvo_attn failed: {rc}")
    return out


def n_cores() -> int:
    return int(lib().vvo_n_cores())


def set_simd(on: bool) -> None:
    """F16C conversions in the ggml-order attention (default) or the scalar loops."""
    lib().vvo_set_simd(1 if on else 0)


def linear(x: np.ndarray, w_raw: np.ndarray, w_type: int, M: int, bias: np.ndarray | None = None,
           mode: int = GGML, n_threads: int = 0) -> np.ndarray:
    """y = x W^T + bias.  x: f32 [..., K]; w_raw: raw bytes of M rows of K
    elements of w_type (F16 or Q8_0); bias f32 [M] or None -> f32 [..., M]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = x.shape[-1]
    N = x.size // K
    w_raw = np.ascontiguousarray(w_raw).reshape(-1)
    rb = row_bytes(w_type, K)
    assert w_raw.size == M * rb
    y = np.empty(x.shape[:-1] + (M,), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = lib().vvo_linear(_ptr(w_raw), w_type, rb, None if b is None else _ptr(b), _ptr(x), _ptr(y),
                          N, K, M, mode, n_threads)
    if rc != 0:
        raise RuntimeError(f"vvo_linear failed: {rc}")
    return y
