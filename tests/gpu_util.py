"""Helpers shared by the GPU parity tests (not a test module)."""
from __future__ import annotations

import numpy as np

import vva
import vvo

TORCH_DT = {}


def torch_dtype(torch, t):
    return {vva.F32: torch.float32, vva.F16: torch.float16, vva.BF16: torch.bfloat16}[t]


def to_gpu(torch, x: np.ndarray, t: int):
    """f32 numpy -> torch GPU tensor of vva type t (values rounded by torch)."""
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to("cuda").to(torch_dtype(torch, t))


def as_f32(torch, x) -> np.ndarray:
    return x.float().cpu().numpy()


def fill_cache(kv: vva.KVCache, lens, seed: int, layers=None, scale: float = 1.0):
    """Upload N(0,1)*scale rows [0, lens[s]) into every (layer, seq) and set len."""
    rng = np.random.default_rng(seed)
    layers = range(kv.n_layers) if layers is None else layers
    for layer in layers:
        for s, n in enumerate(lens):
            k = (rng.standard_normal((n, kv.n_kv_heads, kv.head_dim)) * scale).astype(np.float32)
            v = (rng.standard_normal((n, kv.n_kv_heads, kv.head_dim)) * scale).astype(np.float32)
            if n > 0:                                     # an empty upload is an argument error
                kv.upload(layer, s, 0, k, v)
    for s, n in enumerate(lens):
        kv.set_len(s, n)


def cache_raw(kv: vva.KVCache, layer: int, seq: int, rows: int):
    k, v = kv.download(layer, seq, rows)
    return k.reshape(-1), v.reshape(-1)


def oracle_attn(q32: np.ndarray, kv: vva.KVCache, layer: int, seqs, L, T: int, scale: float,
                mode=vvo.EXACT, mask=None, rows=None):
    ks, vs = [], []
    for b, s in enumerate(seqs):
        k, v = cache_raw(kv, layer, s, L[b])
        ks.append(k)
        vs.append(v)
    return vvo.attn(q32, ks, vs, kv.type, kv.type, L, n_kv_heads=kv.n_kv_heads, scale=scale,
                    mask_mode=vvo.MASK_EXPLICIT if mask is not None else vvo.MASK_CAUSAL,
                    past=[L[b] - T for b in range(len(L))], mask=mask, mode=mode, rows=rows)


def err_stats(got: np.ndarray, ref: np.ndarray):
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    return float(d.max()), float(d.mean())


def assert_close(got, ref, max_tol: float, mean_tol: float, what: str = ""):
    mx, mn = err_stats(got, ref)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert mx <= max_tol and mn <= mean_tol, f"{what}: max {mx:.3e} (tol {max_tol}) mean {mn:.3e} (tol {mean_tol})"
    return mx, mn


def check_ggml_order(got: np.ndarray, q32: np.ndarray, kv: vva.KVCache, layer: int, seqs, L, T: int, scale: float,
                     max_tol: float, mean_tol: float, mask=None, rows=None, what: str = ""):
    """Parity with the oracle's ggml CPU order (Q rounded to K's dot type,
    per-key online softmax with expf).

    Asserted at (max_tol, mean_tol) against that order with an F32 running V
    sum.  For F16 V the oracle's ggml order keeps the running V sum in F16
    (an f16 rounding per key); no fp32-accumulating implementation can track
    that sum's own rounding, which grows with the keys a row sees, so against
    it the mean is asserted at mean_tol and the max is returned for the
    record.  Returns (max, mean) against the F32-sum order and (max, mean)
    against the F16-sum order (equal to the former unless V is F16)."""
    sel = (lambda x: x[:, rows]) if rows is not None else (lambda x: x)
    g32 = oracle_attn(q32, kv, layer, seqs, L, T, scale, mode=vvo.GGML_F32ACC, mask=mask, rows=rows)
    a = assert_close(sel(got), sel(g32), max_tol, mean_tol, what=f"{what} vs ggml order (F32 V sum)")
    if kv.type != vva.F16:
        return a, a
    g16 = oracle_attn(q32, kv, layer, seqs, L, T, scale, mode=vvo.GGML, mask=mask, rows=rows)
    b = err_stats(sel(got), sel(g16))
    assert b[1] <= mean_tol, f"{what} vs ggml order (F16 V sum): mean {b[1]:.3e} (tol {mean_tol})"
    return a, b
