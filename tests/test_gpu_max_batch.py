"""Calls at the largest batch one call may touch (VVA_MAX_BATCH = 16
sequences), ragged lengths, against the oracle on the cache bytes the GPU
holds; and the first batch past it refused before anything is enqueued.
Tolerance: 2e-3 max-abs / 1e-3 mean-abs (F16 / Q8_0 caches)."""
import numpy as np
import pytest

import vva
from gpu_util import as_f32, assert_close, fill_cache, oracle_attn, to_gpu

pytestmark = pytest.mark.gpu

TOL = (2e-3, 1e-3)
B = vva.MAX_BATCH


@pytest.mark.parametrize("d,Hq,Hkv,t", [
    (128, 28, 4, vva.Q8_0),     # the streamed Q8_0 decode kernel: grid (splits, 16 sequences x 2 head pairs)
    (64, 14, 2, vva.F16),       # the register-streamed kernel
])
def test_decode_sixteen_sequences(ctx, torch_gpu, d, Hq, Hkv, t):
    torch = torch_gpu
    lens = [1 + 97 * s + (s % 3) * 500 for s in range(B)]       # 1 .. ~2500 keys
    print(f"decode B={B} d={d} Hq={Hq} Hkv={Hkv} type={t} lens {min(lens)}..{max(lens)}", flush=True)
    kv = vva.KVCache(ctx, 1, Hkv, d, max(lens) + 4, B, t)
    fill_cache(kv, lens, seed=1600 + d)
    for s, n in enumerate(lens):
        kv.set_len(s, n - 1)
    rng = np.random.default_rng(16)
    q = to_gpu(torch, rng.standard_normal((B, 1, Hq, d)), vva.F32)
    out = torch.full((B, 1, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    ctx.attn(kv, 0, q, out, d ** -0.5)
    torch.cuda.synchronize()
    q32, o = as_f32(torch, q), as_f32(torch, out)
    ref = oracle_attn(q32, kv, 0, range(B), lens, 1, d ** -0.5)
    mx, mn = assert_close(o, ref, *TOL, what="16-sequence decode")
    print(f"  max {mx:.2e} mean {mn:.2e}; splits {ctx.last_decode_splits()}")
    kv.free()


def test_decode_step_sixteen_sequences(ctx, torch_gpu):
    """vva_decode_step (RoPE + append + attention) for 16 streams of a Q8_0
    cache: the output equals vva_rope_append followed by vva_attn."""
    torch = torch_gpu
    d, Hq, Hkv = 128, 28, 4
    lens = [40 + 61 * s for s in range(B)]
    kv_a = vva.KVCache(ctx, 1, Hkv, d, max(lens) + 4, B, vva.Q8_0)
    kv_b = vva.KVCache(ctx, 1, Hkv, d, max(lens) + 4, B, vva.Q8_0)
    fill_cache(kv_a, lens, seed=77)
    fill_cache(kv_b, lens, seed=77)
    rng = np.random.default_rng(5)
    q = to_gpu(torch, rng.standard_normal((B, 1, Hq, d)), vva.F32)
    k = to_gpu(torch, rng.standard_normal((B, 1, Hkv, d)), vva.F32)
    v = to_gpu(torch, rng.standard_normal((B, 1, Hkv, d)), vva.F32)
    pos = torch.tensor([[n] for n in lens], dtype=torch.int32, device="cuda")
    qa = torch.empty((B, 1, Hq, d), dtype=torch.float32, device="cuda")
    qb = torch.empty_like(qa)
    oa = torch.full((B, 1, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    ob = torch.full_like(oa, float("nan"))
    ctx.decode_step(kv_a, 0, q, k, v, pos, qa, oa, d ** -0.5)
    ctx.rope_append(kv_b, 0, q, k, v, pos, qb)
    ctx.attn(kv_b, 0, qb, ob, d ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(qa, qb)
    assert torch.equal(oa, ob), "the fused step and append + attention differ"
    for s, n in enumerate(lens):
        assert kv_a.get_len(s) == n and kv_b.get_len(s) == n       # the caller advances past_len
        ka, va = kv_a.download(0, s, n + 1)
        kb, vb = kv_b.download(0, s, n + 1)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb), f"cache rows of stream {s}"
    ref = oracle_attn(as_f32(torch, qa), kv_a, 0, range(B), [n + 1 for n in lens], 1, d ** -0.5)
    mx, mn = assert_close(as_f32(torch, oa), ref, *TOL, what="16-stream step vs exact")
    print(f"  16-stream step: max {mx:.2e} mean {mn:.2e}")
    kv_a.free()
    kv_b.free()


def test_prefill_sixteen_sequences(ctx, torch_gpu):
    torch = torch_gpu
    d, Hq, Hkv, T = 128, 12, 2, 24
    pasts = [33 * s for s in range(B)]
    L = [p + T for p in pasts]
    print(f"prefill B={B} T={T} pasts 0..{max(pasts)}", flush=True)
    kv = vva.KVCache(ctx, 1, Hkv, d, max(L), B, vva.F16)
    fill_cache(kv, L, seed=1616)
    for s in range(B):
        kv.set_len(s, pasts[s])
    rng = np.random.default_rng(17)
    q = to_gpu(torch, rng.standard_normal((B, T, Hq, d)), vva.BF16)
    out = torch.full((B, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    ctx.attn(kv, 0, q, out, d ** -0.5)
    torch.cuda.synchronize()
    q32, o = as_f32(torch, q), as_f32(torch, out)
    ref = oracle_attn(q32, kv, 0, range(B), L, T, d ** -0.5)
    mx, mn = assert_close(o, ref, *TOL, what="16-sequence prefill")
    print(f"  max {mx:.2e} mean {mn:.2e}")
    kv.free()


def test_seventeen_sequences_are_refused(ctx, torch_gpu):
    torch = torch_gpu
    d, Hq, Hkv = 64, 14, 2
    kv = vva.KVCache(ctx, 1, Hkv, d, 64, B + 1, vva.F16)
    fill_cache(kv, [10] * (B + 1), seed=3)
    q = torch.zeros((B + 1, 1, Hq, d), dtype=torch.float32, device="cuda")
    out = torch.full((B + 1, 1, Hq, d), 7.0, dtype=torch.float32, device="cuda")
    with pytest.raises(vva.VvaError) as e:
        ctx.attn(kv, 0, q, out, d ** -0.5)
    assert e.value.status == vva.ERR_INVALID_ARG
    torch.cuda.synchronize()
    assert bool((out == 7.0).all()), "a refused call wrote its output"
    kv.free()
