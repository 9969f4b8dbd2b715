"""Python binding of libvva.so (include/vva.h) over ctypes.

A thin host-side mirror of the C ABI for tests, the benchmark and Python
callers.  Device memory and streams come from PyTorch (torch tensors on a HIP
device); every compute call goes through the native library.  There is no
fallback: if the library is missing or the device is not gfx950, the calls
raise.
"""
from __future__ import annotations

import atexit
import contextlib
import ctypes
import os
import weakref

F32, F16, Q8_0, I32, BF16 = 0, 1, 8, 26, 30
ROPE_NEOX = 2
MAX_BATCH = 16
Q8_BLOCK_BYTES = 34

OK, ERR_GENERIC, ERR_INVALID_ARG, ERR_OOM, ERR_NOT_IMPLEMENTED, ERR_DEVICE = 0, -1, -2, -5, -6, -9

_HERE = os.path.dirname(os.path.abspath(__file__))
# VVA_LIB names another build of the library (same ABI), e.g. to compare kernel variants.
LIB_PATH = os.environ.get("VVA_LIB") or os.path.join(_HERE, "lib", "libvva.so")

# Symbols declared in include/vva.h (checked by the CPU test suite).
EXPORTS = [
    "vva_create", "vva_destroy", "vva_set_stream", "vva_synchronize", "vva_last_error",
    "vva_version", "vva_kv_create", "vva_kv_free", "vva_kv_get_len", "vva_kv_set_len",
    "vva_kv_view", "vva_kv_upload", "vva_rope_ext", "vva_rope_append", "vva_attn",
    "vva_flash_attn_ext", "vva_supports", "vva_set_attn_path", "vva_last_decode_splits",
    "vva_set_schedule", "vva_attn_noalloc", "vva_qkv_rope_append", "vva_out_proj_residual",
    "vva_set_flash_attn", "vva_decode_step", "vva_qkv_proj", "vva_set_log_callback",
]

LOG_ERROR, LOG_WARN, LOG_INFO, LOG_DEBUG = 0, 1, 2, 3
# void (*)(vva_log_level lvl, const char* msg, void* user_data)
LOG_CB = ctypes.CFUNCTYPE(None, ctypes.c_int, ctypes.c_char_p, ctypes.c_void_p)


class VvaError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"vva status {status}: {msg}")
        self.status = status


class Tensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("type", ctypes.c_int32),
                ("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_size_t * 4)]


class KVDesc(ctypes.Structure):
    _fields_ = [("n_layers", ctypes.c_int32), ("n_kv_heads", ctypes.c_int32),
                ("head_dim", ctypes.c_int32), ("max_seq", ctypes.c_int32),
                ("n_seq", ctypes.c_int32), ("type", ctypes.c_int32)]


_lib = None
# Contexts still open when the interpreter exits are destroyed by an atexit
# hook, which runs before the C-level exit handlers of the HIP runtime and
# of any profiler attached to the process: no vva_destroy (stream
# synchronize, hipFree) then runs during or after their teardown.
_live_contexts = weakref.WeakSet()


@atexit.register
def _close_live_contexts():
    for c in list(_live_contexts):
        try:
            c.close()
        except Exception:  # noqa: BLE001 — best effort at exit
            pass


def load_library(path: str = LIB_PATH):
    """Load libvva.so (after torch, so both share one HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"libvva.so not built: {path} (run __graft_entry__.build())")
    L = ctypes.CDLL(path)
    P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    TP = ctypes.POINTER(Tensor)
    sig = {
        "vva_create": (I, [I, P, ctypes.POINTER(P)]),
        "vva_destroy": (None, [P]),
        "vva_set_stream": (I, [P, P]),
        "vva_synchronize": (I, [P]),
        "vva_last_error": (ctypes.c_char_p, [P]),
        "vva_version": (ctypes.c_char_p, []),
        "vva_kv_create": (I, [P, ctypes.POINTER(KVDesc), ctypes.POINTER(P)]),
        "vva_kv_free": (None, [P]),
        "vva_kv_get_len": (I, [P, I, ctypes.POINTER(ctypes.c_int32)]),
        "vva_kv_set_len": (I, [P, I, ctypes.c_int32]),
        "vva_kv_view": (I, [P, I, I, TP, TP]),
        "vva_kv_upload": (I, [P, P, I, I, ctypes.c_int32, ctypes.c_int32, P, P]),
        "vva_rope_ext": (I, [P, TP, TP, I, I, F, TP]),
        "vva_rope_append": (I, [P, P, I, TP, TP, TP, TP, P, F, TP]),
        "vva_attn": (I, [P, P, I, TP, P, TP, F, TP]),
        "vva_attn_noalloc": (I, [P, P, I, TP, P, TP, F, TP]),
        "vva_qkv_rope_append": (I, [P, P, I, TP, TP, TP, TP, TP, TP, TP, TP, P, F, TP]),
        "vva_out_proj_residual": (I, [P, TP, TP, TP, TP]),
        "vva_qkv_proj": (I, [P, TP, TP, TP, TP, TP, TP, TP, TP]),
        "vva_flash_attn_ext": (I, [P, TP, TP, TP, TP, F, F, F, TP]),
        "vva_supports": (I, [P, I, I, I, I, I]),
        "vva_set_attn_path": (I, [P, I]),
        "vva_last_decode_splits": (I, [P]),
        "vva_set_schedule": (I, [P, I, I, I]),
        "vva_set_flash_attn": (I, [P, I]),
        "vva_decode_step": (I, [P, P, I, TP, TP, TP, TP, P, F, F, TP, TP]),
        "vva_set_log_callback": (None, [LOG_CB, P, I]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


_log_cb_ref = None      # the installed ctypes callback (kept alive while set)


def set_log_callback(fn, max_level: int = LOG_INFO):
    """Deliver the library's messages to fn(level, message) up to max_level
    (fn None: none).  Mirrors vv_set_log_callback."""
    global _log_cb_ref
    lib = load_library()
    if fn is None:
        lib.vva_set_log_callback(LOG_CB(), None, LOG_ERROR)
        _log_cb_ref = None
        return
    cb = LOG_CB(lambda lvl, msg, _user: fn(int(lvl), msg.decode(errors="replace")))
    lib.vva_set_log_callback(cb, None, max_level)
    _log_cb_ref = cb


def _torch():
    import torch  # noqa: PLC0415 — imported lazily so the CPU tests need no GPU
    return torch


def vva_type_of(t) -> int:
    torch = _torch()
    m = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.int32: I32}
    if t.dtype not in m:
        raise TypeError(f"unsupported dtype {t.dtype}")
    return m[t.dtype]


def view(t, ggml_ne=None, ggml_nb=None, type_=None) -> Tensor:
    """ggml-shaped view of a torch tensor: ne/nb are the reversed shape/strides
    (ne[0] fastest) unless given explicitly (e.g. for Q8_0 byte buffers)."""
    tv = Tensor()
    tv.data = t.data_ptr()
    tv.type = vva_type_of(t) if type_ is None else type_
    if ggml_ne is None:
        es = t.element_size()
        ggml_ne = list(t.shape)[::-1]
        ggml_nb = [s * es for s in t.stride()][::-1]
        while len(ggml_ne) < 4:
            ggml_nb.append(ggml_nb[-1] * ggml_ne[-1] if ggml_nb else es)
            ggml_ne.append(1)
    for i in range(4):
        tv.ne[i] = int(ggml_ne[i])
        tv.nb[i] = int(ggml_nb[i])
    return tv


class Context:
    """vva_context bound to the current torch stream of `device`."""

    def __init__(self, device: int = 0, stream=None):
        torch = _torch()
        self.lib = load_library()
        self.device = device
        if stream is None:
            stream = torch.cuda.current_stream(device)
        self.stream = stream
        h = ctypes.c_void_p()
        st = self.lib.vva_create(device, ctypes.c_void_p(stream.cuda_stream), ctypes.byref(h))
        if st != OK:
            raise VvaError(st, self.lib.vva_last_error(None).decode())
        self.h = h
        self.caches = weakref.WeakSet()
        _live_contexts.add(self)

    def check(self, st: int):
        if st != OK:
            raise VvaError(st, self.lib.vva_last_error(self.h).decode())

    def close(self):
        if getattr(self, "h", None):
            for kv in list(self.caches):      # vva_destroy releases them natively
                kv.h = None
            self.lib.vva_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 — interpreter shutdown
            pass

    def synchronize(self):
        self.check(self.lib.vva_synchronize(self.h))

    def set_stream(self, stream):
        """Enqueue later calls on `stream` (a torch.cuda.Stream), e.g. the
        stream a torch.cuda.graph capture records."""
        self.check(self.lib.vva_set_stream(self.h, ctypes.c_void_p(stream.cuda_stream)))
        self.stream = stream

    def set_attn_path(self, path: int):
        self.check(self.lib.vva_set_attn_path(self.h, path))

    def set_flash_attn(self, use_flash_attn: bool):
        """F32 caches: True = F16 cast + MFMA prefill (the flash branch), False = fp32 eager branch."""
        self.check(self.lib.vva_set_flash_attn(self.h, int(bool(use_flash_attn))))

    def last_decode_splits(self) -> int:
        return int(self.lib.vva_last_decode_splits(self.h))

    def set_schedule(self, decode_wgs: int = 0, decode_splits: int = 0, prefill_splits: int = 0):
        """Scheduling overrides for tests and benchmarks (0 = automatic)."""
        self.check(self.lib.vva_set_schedule(self.h, decode_wgs, decode_splits, prefill_splits))

    @contextlib.contextmanager
    def schedule(self, decode_wgs: int = 0, decode_splits: int = 0, prefill_splits: int = 0):
        """`with ctx.schedule(...)`: overrides for the block, automatic after."""
        self.set_schedule(decode_wgs, decode_splits, prefill_splits)
        try:
            yield self
        finally:
            self.set_schedule(0, 0, 0)

    def supports(self, head_dim, n_q_heads, n_kv_heads, q_type, kv_type) -> bool:
        return bool(self.lib.vva_supports(self.h, head_dim, n_q_heads, n_kv_heads, q_type, kv_type))

    # ---- ops -----------------------------------------------------------
    def rope_ext(self, x, pos, freq_base: float = 1.0e6, dst=None):
        """x: torch [B, T, H, d]; pos: int32 [T] or [B, T]."""
        dst = x if dst is None else dst
        self.check(self.lib.vva_rope_ext(self.h, ctypes.byref(view(x)), ctypes.byref(view(pos)),
                                         x.shape[-1], ROPE_NEOX, freq_base, ctypes.byref(view(dst))))
        return dst

    def rope_append(self, kv: "KVCache", layer: int, q, k, v, pos, q_out, seq_ids=None,
                    freq_base: float = 1.0e6):
        """q/q_out: [B, T, Hq, d]; k, v: [B, T, Hkv, d]; pos int32 [T] or [B, T]."""
        ids = _ids(seq_ids)
        self.check(self.lib.vva_rope_append(self.h, kv.h, layer, ctypes.byref(view(q)), ctypes.byref(view(k)),
                                            ctypes.byref(view(v)), ctypes.byref(view(pos)), ids,
                                            freq_base, ctypes.byref(view(q_out))))

    def attn(self, kv: "KVCache", layer: int, q, out, scale: float, seq_ids=None, mask=None):
        """q: [B, T, Hq, d]; out: f32 [B, T, Hq, d]; mask: f16 [B or 1, T, >= L] or None (causal)."""
        ids = _ids(seq_ids)
        mp = ctypes.byref(_mask_view(mask)) if mask is not None else None
        self.check(self.lib.vva_attn(self.h, kv.h, layer, ctypes.byref(view(q)), ids, mp, scale,
                                     ctypes.byref(view(out))))

    def decode_step(self, kv: "KVCache", layer: int, q, k, v, pos, q_out, out, scale: float, seq_ids=None,
                    freq_base: float = 1.0e6):
        """One new token per sequence: RoPE + append + attention (q/k/v [B, 1, H, d], pos int32 [1] or [B, 1])."""
        ids = _ids(seq_ids)
        self.check(self.lib.vva_decode_step(self.h, kv.h, layer, ctypes.byref(view(q)), ctypes.byref(view(k)),
                                            ctypes.byref(view(v)), ctypes.byref(view(pos)), ids, freq_base, scale,
                                            ctypes.byref(view(q_out)), ctypes.byref(view(out))))

    def attn_noalloc(self, kv: "KVCache", layer: int, q, out, scale: float, seq_ids=None, mask=None):
        """vva_attn_noalloc: as attn, with the split partials in the device's
        static scratch (no device allocation)."""
        ids = _ids(seq_ids)
        mp = ctypes.byref(_mask_view(mask)) if mask is not None else None
        self.check(self.lib.vva_attn_noalloc(self.h, kv.h, layer, ctypes.byref(view(q)), ids, mp, scale,
                                             ctypes.byref(view(out))))

    def qkv_rope_append(self, kv: "KVCache", layer: int, x, wq: "Weight", wk: "Weight", wv: "Weight", pos,
                        q_out, bq=None, bk=None, bv=None, seq_ids=None, freq_base: float = 1.0e6):
        """x: [B, T, hidden]; weights: Weight; biases f32 [rows] or None; q_out [B, T, Hq, d]."""
        ids = _ids(seq_ids)
        bref = [ctypes.byref(view(t)) if t is not None else None for t in (bq, bk, bv)]
        self.check(self.lib.vva_qkv_rope_append(self.h, kv.h, layer, ctypes.byref(view(x)), ctypes.byref(wq.t),
                                                ctypes.byref(wk.t), ctypes.byref(wv.t), bref[0], bref[1], bref[2],
                                                ctypes.byref(view(pos)), ids, freq_base, ctypes.byref(view(q_out))))

    def qkv_proj(self, x, wq: "Weight", wk: "Weight", wv: "Weight", y, bq=None, bk=None, bv=None):
        """x: [B, T, hidden]; weights: Weight; biases f32 [rows] or None; y f32 [B, T, Mq + Mk + Mv]."""
        bref = [ctypes.byref(view(t)) if t is not None else None for t in (bq, bk, bv)]
        self.check(self.lib.vva_qkv_proj(self.h, ctypes.byref(view(x)), ctypes.byref(wq.t), ctypes.byref(wk.t),
                                         ctypes.byref(wv.t), bref[0], bref[1], bref[2], ctypes.byref(view(y))))

    def out_proj_residual(self, o, w_o: "Weight", x, h):
        """o: [B, T, Hq*d] (or [B, T, Hq, d], viewed as rows); x, h: f32 [B, T, hidden]."""
        if o.dim() == 4:
            o = o.reshape(o.shape[0], o.shape[1], -1)
        self.check(self.lib.vva_out_proj_residual(self.h, ctypes.byref(view(o)), ctypes.byref(w_o.t),
                                                  ctypes.byref(view(x)), ctypes.byref(view(h))))

    def flash_attn_ext(self, q, k, v, out, scale: float, mask=None, k_view=None, v_view=None):
        """ggml layout: q torch [B, Hq, T, d] (ne=[d,T,Hq,B]); k, v torch [B, Hkv, L, d] or
        explicit Tensor views; out f32 [B, T, Hq, d] (ne=[d,Hq,T,B])."""
        kt = k_view if k_view is not None else view(k)
        vt = v_view if v_view is not None else view(v)
        mp = ctypes.byref(_mask_view(mask)) if mask is not None else None
        self.check(self.lib.vva_flash_attn_ext(self.h, ctypes.byref(view(q)), ctypes.byref(kt), ctypes.byref(vt),
                                               mp, scale, 0.0, 0.0, ctypes.byref(view(out))))


def _ids(seq_ids):
    if seq_ids is None:
        return None
    arr = (ctypes.c_int32 * len(seq_ids))(*[int(s) for s in seq_ids])
    return ctypes.cast(arr, ctypes.c_void_p)


def _mask_view(mask) -> Tensor:
    """mask: f16 or f32 torch [Bm, T, Lm] -> ggml ne=[Lm, T, 1, Bm]."""
    Bm, T, Lm = mask.shape
    es = mask.element_size()
    return view(mask, ggml_ne=[Lm, T, 1, Bm],
                ggml_nb=[es, mask.stride(1) * es, mask.stride(0) * es * T, mask.stride(0) * es],
                type_=F32 if es == 4 else F16)


class KVCache:
    def __init__(self, ctx: Context, n_layers: int, n_kv_heads: int, head_dim: int, max_seq: int,
                 n_seq: int, type_: int):
        self.ctx = ctx
        d = KVDesc(n_layers, n_kv_heads, head_dim, max_seq, n_seq, type_)
        h = ctypes.c_void_p()
        ctx.check(ctx.lib.vva_kv_create(ctx.h, ctypes.byref(d), ctypes.byref(h)))
        self.h = h
        ctx.caches.add(self)
        self.n_layers, self.n_kv_heads, self.head_dim = n_layers, n_kv_heads, head_dim
        self.max_seq, self.n_seq, self.type = max_seq, n_seq, type_

    def free(self):
        if getattr(self, "h", None) and getattr(self.ctx, "h", None):
            self.ctx.lib.vva_kv_free(self.h)
        self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:  # noqa: BLE001
            pass

    def get_len(self, seq: int) -> int:
        n = ctypes.c_int32()
        self.ctx.check(self.ctx.lib.vva_kv_get_len(self.h, seq, ctypes.byref(n)))
        return n.value

    def set_len(self, seq: int, n: int):
        self.ctx.check(self.ctx.lib.vva_kv_set_len(self.h, seq, n))

    def views(self, layer: int, seq: int):
        k, v = Tensor(), Tensor()
        self.ctx.check(self.ctx.lib.vva_kv_view(self.h, layer, seq, ctypes.byref(k), ctypes.byref(v)))
        return k, v

    def row_bytes(self) -> int:
        k, _ = self.views(0, 0)
        return int(k.nb[2])

    def download(self, layer: int, seq: int, rows: int):
        """Raw bytes (uint8 numpy, [rows, row_bytes]) of K and V rows [0, rows)."""
        torch = _torch()
        import numpy as np  # noqa: PLC0415
        k, v = self.views(layer, seq)
        rb = int(k.nb[2])
        out = []
        for t in (k, v):
            buf = np.empty((rows, rb), dtype=np.uint8)
            self.ctx.synchronize()
            torch.cuda.synchronize(self.ctx.device)
            hip = _hip()
            rc = hip.hipMemcpy(ctypes.c_void_p(buf.ctypes.data), ctypes.c_void_p(t.data), ctypes.c_size_t(rows * rb), 2)
            if rc != 0:
                raise RuntimeError(f"hipMemcpy D2H failed: {rc}")
            out.append(buf)
        return out[0], out[1]

    def upload(self, layer: int, seq: int, start: int, k_rows, v_rows):
        """k_rows/v_rows: numpy f32 [len, Hkv, d]."""
        import numpy as np  # noqa: PLC0415
        k_rows = np.ascontiguousarray(k_rows, dtype=np.float32)
        v_rows = np.ascontiguousarray(v_rows, dtype=np.float32)
        self.ctx.check(self.ctx.lib.vva_kv_upload(self.ctx.h, self.h, layer, seq, start, k_rows.shape[0],
                                                  ctypes.c_void_p(k_rows.ctypes.data),
                                                  ctypes.c_void_p(v_rows.ctypes.data)))


class Weight:
    """A linear layer's weight on the device: M rows of K elements, F16 or
    Q8_0 (GGUF blocks along K), as ggml stores it (ne = [K, M]).  `raw` is a
    uint8 torch tensor holding the rows back to back."""

    def __init__(self, raw, w_type: int, K: int, M: int):
        self.raw, self.w_type, self.K, self.M = raw, w_type, K, M
        rb = K * 2 if w_type == F16 else K // 32 * Q8_BLOCK_BYTES
        assert raw.numel() == rb * M
        es = 2 if w_type == F16 else Q8_BLOCK_BYTES
        self.t = view(raw, ggml_ne=[K, M, 1, 1], ggml_nb=[es, rb, rb * M, rb * M], type_=w_type)


_hip_lib = None


def _hip():
    """The HIP runtime already loaded by torch (same SONAME as libvva's dependency)."""
    global _hip_lib
    if _hip_lib is None:
        _hip_lib = ctypes.CDLL("libamdhip64.so.7")
        _hip_lib.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _hip_lib.hipMemcpy.restype = ctypes.c_int
    return _hip_lib
