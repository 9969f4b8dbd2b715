"""GPU parity of the fused RoPE + KV append (src/qwen2.cpp:282-306) and of the
cache ingest (vva_kv_upload, src/vibevoice_tts.cpp:735-749), through the C ABI.

Byte-level results (the V rows of every cache type, Q8_0 blocks included) must
be bit-identical to the oracle's conversion of the same values; rotated
values (Q, K) must agree with the oracle's fp32-recurrence RoPE to fp32
rounding (the oracle and the kernel use the same operation order; sinf/cosf
come from different math libraries).
"""
import numpy as np
import pytest

import vva
import vvo
from gpu_util import as_f32, to_gpu

pytestmark = pytest.mark.gpu

CASES = [
    # d, Hq, Hkv, T, B, in_type, cache_type, past
    (64, 14, 2, 37, 1, vva.F32, vva.F16, [0]),
    (64, 14, 2, 1, 2, vva.F32, vva.F16, [1024, 700]),
    (128, 28, 4, 129, 1, vva.BF16, vva.F16, [5]),
    (128, 28, 4, 64, 2, vva.F32, vva.Q8_0, [0, 33]),
    (128, 12, 2, 16, 1, vva.F16, vva.BF16, [300]),
    (64, 14, 2, 8, 1, vva.F32, vva.F32, [3]),
    (128, 28, 4, 1, 2, vva.F32, vva.Q8_0, [32768, 32700]),
]


@pytest.mark.parametrize("d,Hq,Hkv,T,B,in_t,cache_t,past", CASES)
def test_rope_append_matches_oracle(ctx, torch_gpu, d, Hq, Hkv, T, B, in_t, cache_t, past):
    torch = torch_gpu
    print(f"case d={d} Hq={Hq} Hkv={Hkv} T={T} B={B} in={in_t} cache={cache_t} past={past}", flush=True)
    rng = np.random.default_rng(d * 1000 + T * 10 + B)
    max_seq = max(past) + T + 8
    kv = vva.KVCache(ctx, 2, Hkv, d, max_seq, B, cache_t)
    for s in range(B):
        kv.set_len(s, past[s])
    q = to_gpu(torch, rng.standard_normal((B, T, Hq, d)), in_t)
    k = to_gpu(torch, rng.standard_normal((B, T, Hkv, d)), in_t)
    v = to_gpu(torch, rng.standard_normal((B, T, Hkv, d)), in_t)
    pos = torch.tensor(np.array([[past[b] + t for t in range(T)] for b in range(B)], np.int32)).to("cuda")
    q_out = torch.empty((B, T, Hq, d), dtype=torch.float32, device="cuda")
    ctx.rope_append(kv, 1, q, k, v, pos, q_out)
    torch.cuda.synchronize()

    pos_np = pos.cpu().numpy()
    q_ref = vvo.rope(as_f32(torch, q), pos_np)
    k_ref = vvo.rope(as_f32(torch, k), pos_np)
    np.testing.assert_allclose(as_f32(torch, q_out), q_ref, atol=2e-6, rtol=0)

    rb = kv.row_bytes()
    for b in range(B):
        kraw, vraw = kv.download(1, b, past[b] + T)
        # rows before past untouched (still zero), new rows at [past, past+T)
        assert not kraw[: past[b]].any() and not vraw[: past[b]].any()
        v_expect = vvo.from_f32(as_f32(torch, v)[b], cache_t).reshape(T, rb)
        np.testing.assert_array_equal(vraw[past[b]:], v_expect)
        k_got = vvo.to_f32(kraw[past[b]:], cache_t, T * Hkv * d).reshape(T, Hkv, d)
        k_exp = vvo.to_f32(vvo.from_f32(k_ref[b], cache_t), cache_t, T * Hkv * d).reshape(T, Hkv, d)
        tol = {vva.F32: 2e-6, vva.F16: 2e-3, vva.BF16: 2e-2, vva.Q8_0: 4e-2}[cache_t]
        np.testing.assert_allclose(k_got, k_exp, atol=tol, rtol=0)
        same = np.mean(kraw[past[b]:] == vvo.from_f32(k_ref[b], cache_t).reshape(T, rb))
        # F32 rows expose 1-ulp sinf/cosf differences in their low bytes
        assert same > (0.9 if cache_t == vva.F32 else 0.99), same
        # the other layer is untouched
        k0, v0 = kv.download(0, b, past[b] + T)
        assert not k0.any() and not v0.any()
    kv.free()


def test_rope_ext_in_place_half_precision(ctx, torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(5)
    x32 = rng.standard_normal((2, 9, 7, 128)).astype(np.float32)
    pos = np.array([[p + t for t in range(9)] for p in (0, 4000)], np.int32)
    x = to_gpu(torch, x32, vva.F16)
    src = as_f32(torch, x)
    ctx.rope_ext(x, torch.tensor(pos).to("cuda"))
    torch.cuda.synchronize()
    ref = vvo.to_f32(vvo.from_f32(vvo.rope(src, pos), vvo.F16), vvo.F16, src.size).reshape(src.shape)
    np.testing.assert_allclose(as_f32(torch, x), ref, atol=2e-3, rtol=0)


@pytest.mark.parametrize("cache_t", [vva.F32, vva.F16, vva.BF16, vva.Q8_0])
def test_kv_upload_is_bit_exact(ctx, torch_gpu, cache_t):
    rng = np.random.default_rng(cache_t)
    Hkv, d, n = 4, 128, 37
    kv = vva.KVCache(ctx, 1, Hkv, d, 64, 1, cache_t)
    k = rng.standard_normal((n, Hkv, d)).astype(np.float32) * 3
    v = rng.standard_normal((n, Hkv, d)).astype(np.float32) * 3
    kv.upload(0, 0, 5, k, v)
    kraw, vraw = kv.download(0, 0, 5 + n)
    assert not kraw[:5].any()
    np.testing.assert_array_equal(kraw[5:].reshape(-1), vvo.from_f32(k, cache_t))
    np.testing.assert_array_equal(vraw[5:].reshape(-1), vvo.from_f32(v, cache_t))
    kv.free()


def test_errors_are_reported_not_raised_in_native_code(ctx, torch_gpu):
    torch = torch_gpu
    kv = vva.KVCache(ctx, 1, 2, 64, 16, 1, vva.F16)
    kv.set_len(0, 10)
    q = torch.zeros((1, 8, 14, 64), device="cuda")
    k = torch.zeros((1, 8, 2, 64), device="cuda")
    pos = torch.zeros(8, dtype=torch.int32, device="cuda")
    with pytest.raises(vva.VvaError) as e:          # 10 + 8 > max_seq 16
        ctx.rope_append(kv, 0, q, k, k, pos, q)
    assert e.value.status == vva.ERR_INVALID_ARG and "max_seq" in str(e.value)
    with pytest.raises(vva.VvaError):
        ctx.rope_append(kv, 3, q, k, k, pos, q)     # bad layer
    kv.free()


def test_a_sequence_written_twice_in_one_call_is_refused(ctx, torch_gpu):
    """Two rows of one call naming the same sequence would write the same
    cache rows from two places: every writer (vva_rope_append,
    vva_decode_step) refuses the call before anything is enqueued."""
    torch = torch_gpu
    d, Hq, Hkv = 64, 14, 2
    kv = vva.KVCache(ctx, 1, Hkv, d, 32, 2, vva.F16)
    kv.set_len(0, 4)
    kv.set_len(1, 4)
    before = kv.download(0, 0, 8)
    q = torch.ones((2, 1, Hq, d), device="cuda")
    k = torch.ones((2, 1, Hkv, d), device="cuda")
    q_out = torch.full((2, 1, Hq, d), 7.0, device="cuda")
    out = torch.full((2, 1, Hq, d), 7.0, device="cuda")
    pos = torch.tensor([[4], [4]], dtype=torch.int32, device="cuda")
    with pytest.raises(vva.VvaError) as e:
        ctx.rope_append(kv, 0, q, k, k, pos, q_out, seq_ids=[0, 0])
    assert e.value.status == vva.ERR_INVALID_ARG and "twice" in str(e.value)
    with pytest.raises(vva.VvaError) as e:
        ctx.decode_step(kv, 0, q, k, k, pos, q_out, out, d ** -0.5, seq_ids=[1, 1])
    assert e.value.status == vva.ERR_INVALID_ARG and "twice" in str(e.value)
    torch.cuda.synchronize()
    after = kv.download(0, 0, 8)
    assert all(np.array_equal(x, y) for x, y in zip(before, after)), "a refused call wrote the cache"
    assert bool((q_out == 7.0).all()) and bool((out == 7.0).all())
    assert kv.get_len(0) == 4 and kv.get_len(1) == 4
    kv.free()


@pytest.mark.parametrize("in_t,cache_t", [(vva.BF16, vva.F16), (vva.F32, vva.BF16), (vva.F16, vva.F32)])
def test_vector_and_scalar_paths_agree_bit_for_bit(ctx, torch_gpu, in_t, cache_t):
    """Rows on 16-byte boundaries take the vector path (8 pairs per lane), a
    view 8 bytes off a boundary the scalar one; both compute the same fp32
    operations, so Q and the cache bytes must be identical."""
    torch = torch_gpu
    d, Hq, Hkv, T, B = 128, 28, 4, 40, 2           # T * B >= 64: the vector path when aligned
    rng = np.random.default_rng(17)
    vals = [rng.standard_normal((B, T, H, d)) for H in (Hq, Hkv, Hkv)]
    aligned = [to_gpu(torch, x, in_t) for x in vals]
    eb = 4 if in_t == vva.F32 else 2
    off = 8 // eb                                          # 8 bytes: off every 16-byte boundary
    shifted = []
    for x in aligned:
        big = torch.zeros(x.shape[:-1] + (d + 8,), dtype=x.dtype, device="cuda")
        big[..., off:off + d] = x
        shifted.append(big[..., off:off + d])
    assert shifted[0].data_ptr() % 16 == 8
    pos = torch.tensor(np.array([[100 * b + t for t in range(T)] for b in range(B)], np.int32)).to("cuda")
    kv = vva.KVCache(ctx, 2, Hkv, d, T + 8, B, cache_t)
    outs = []
    for layer, (q, k, v) in enumerate((aligned, shifted)):
        for s in range(B):
            kv.set_len(s, 0)
        q_out = torch.empty((B, T, Hq, d), dtype=torch.float16, device="cuda")
        ctx.rope_append(kv, layer, q, k, v, pos, q_out)
        outs.append(q_out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    for b in range(B):
        a0, a1 = kv.download(0, b, T), kv.download(1, b, T)
        np.testing.assert_array_equal(a0[0], a1[0])
        np.testing.assert_array_equal(a0[1], a1[1])
    kv.free()
