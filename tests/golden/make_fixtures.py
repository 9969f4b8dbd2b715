#!/usr/bin/env python3
"""Writes the golden fixtures under tests/golden/.

The reference's own hot-path tests compare ggml against fixtures produced by
Python dumpers (tests/dump_rope_reference.py, tests/dump_qwen2_reference.py)
that need the `gguf` package, which is not installed here, so their GGUF
files cannot be produced.  This script re-creates the same test cases with
the same generators, seeds and shapes and takes the expected values from
Hugging Face transformers' Qwen2 implementation (the library the reference's
dumper uses as ground truth), evaluated in float64:

  rope_seed2025.npz   tests/dump_rope_reference.py defaults: dim 64, 4 heads,
                      seq 128, theta 1e6, x = default_rng(2025).standard_normal
                      ((seq, heads, dim)); expected = Qwen2RotaryEmbedding +
                      apply_rotary_pos_emb (fp64).  A subset of token rows is
                      stored to keep the file small.
  attn_seed1234.npz   tests/dump_qwen2_reference.py attention shape: 4 q heads,
                      2 kv heads, head_dim 32, seq 64, theta 1e6, seed 1234;
                      q/k/v drawn N(0,1) (the projections are outside this
                      path), expected = HF RoPE + repeat_kv + causal
                      eager_attention_forward (fp64), output [seq, heads, dim].

Run:  python tests/golden/make_fixtures.py
"""
from __future__ import annotations

import os

import numpy as np
import torch
from transformers.models.qwen2.configuration_qwen2 import Qwen2Config
from transformers.models.qwen2.modeling_qwen2 import (
    Qwen2RotaryEmbedding,
    apply_rotary_pos_emb,
    eager_attention_forward,
)

HERE = os.path.dirname(os.path.abspath(__file__))
ROPE_ROWS = np.array(sorted(set(list(range(16)) + list(range(16, 112, 8)) + list(range(112, 128)))), dtype=np.int32)


def hf_rope(x: np.ndarray, pos: np.ndarray, theta: float, n_heads: int) -> np.ndarray:
    """x: [T, H, d] -> HF Qwen2 RoPE in float64."""
    T, H, d = x.shape
    cfg = Qwen2Config(hidden_size=H * d, num_attention_heads=H, num_key_value_heads=H,
                      rope_theta=theta, max_position_embeddings=max(T * 2, int(pos.max()) + 1))
    rot = Qwen2RotaryEmbedding(cfg).to(torch.float64)
    xt = torch.from_numpy(x.astype(np.float64)).permute(1, 0, 2).unsqueeze(0)      # [1, H, T, d]
    cos, sin = rot(xt, torch.from_numpy(pos.astype(np.int64)).unsqueeze(0))
    y, _ = apply_rotary_pos_emb(xt, xt, cos, sin)
    return y.squeeze(0).permute(1, 0, 2).numpy()


class _Mod(torch.nn.Module):
    def __init__(self, groups: int):
        super().__init__()
        self.num_key_value_groups = groups


def main() -> None:
    torch.set_grad_enabled(False)
    # ---- RoPE case of tests/dump_rope_reference.py
    dim, heads, seq, theta, seed = 64, 4, 128, 1.0e6, 2025
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((seq, heads, dim)).astype(np.float32)
    pos = np.arange(seq, dtype=np.int32)
    y = hf_rope(x, pos, theta, heads)
    np.savez_compressed(os.path.join(HERE, "rope_seed2025.npz"), rows=ROPE_ROWS,
                        expected=y[ROPE_ROWS].astype(np.float32), dim=dim, heads=heads, seq=seq,
                        theta=theta, seed=seed)

    # ---- attention case with the shape of tests/dump_qwen2_reference.py
    nh, nkv, hd, seq, seed = 4, 2, 32, 64, 1234
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((seq, nh, hd)).astype(np.float32)
    k = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    pos = np.arange(seq, dtype=np.int32)
    cfg = Qwen2Config(hidden_size=nh * hd, num_attention_heads=nh, num_key_value_heads=nkv,
                      rope_theta=theta, max_position_embeddings=seq * 2)
    rot = Qwen2RotaryEmbedding(cfg).to(torch.float64)
    qt = torch.from_numpy(q.astype(np.float64)).permute(1, 0, 2).unsqueeze(0)
    kt = torch.from_numpy(k.astype(np.float64)).permute(1, 0, 2).unsqueeze(0)
    vt = torch.from_numpy(v.astype(np.float64)).permute(1, 0, 2).unsqueeze(0)
    cos, sin = rot(qt, torch.from_numpy(pos.astype(np.int64)).unsqueeze(0))
    qr, kr = apply_rotary_pos_emb(qt, kt, cos, sin)
    causal = torch.full((seq, seq), float("-inf"), dtype=torch.float64).triu(1)[None, None]
    out, _ = eager_attention_forward(_Mod(nh // nkv), qr, kr, vt, causal, scaling=hd ** -0.5)
    np.savez_compressed(os.path.join(HERE, "attn_seed1234.npz"),
                        expected=out[0].numpy().astype(np.float32), theta=theta, seed=seed)
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
