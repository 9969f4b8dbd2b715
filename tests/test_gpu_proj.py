"""GPU parity of the fused projections (proj.hip) through the C ABI.

vva_qkv_rope_append: the q/k/v linear layers with bias (ggml_mul_mat +
ggml_add, src/qwen2.cpp:19-25, :273-275), NeoX RoPE (theta 1e6) and the
cache append (src/qwen2.cpp:282-306).  vva_out_proj_residual: the output
projection plus the residual (src/qwen2.cpp:348-349).

The oracle is vvo.linear in ggml's CPU order (x rounded to f16 for F16
weights, quantized to Q8_0 blocks with integer block sums for Q8_0 weights)
followed by vvo.rope (fp32 theta recurrence).  Tolerance 2e-3 max-abs /
1e-3 mean-abs on F32 outputs, plus, where the output is stored in a
narrower type, that type's own rounding of the oracle's value (half an ulp
for f16 / bf16, half a quantization step for Q8_0 blocks).  Weights are
N(0, 1/hidden), x N(0, 1), biases N(0, 0.25), so outputs are O(1).
"""
import numpy as np
import pytest

import vva
import vvo
from gpu_util import as_f32, to_gpu

pytestmark = pytest.mark.gpu

MAX_TOL, MEAN_TOL = 2e-3, 1e-3


def _weight(torch, rng, M, K, w_type):
    w = (rng.standard_normal((M, K)) * K ** -0.5).astype(np.float32)
    raw = vvo.from_f32(w, w_type)
    return raw, vva.Weight(torch.from_numpy(raw).cuda(), w_type, K, M)


def _round_bound(ref, t):
    """Per-element bound of storing ref in type t (before the compute tolerance)."""
    a = np.abs(ref)
    if t == vva.F32:
        return np.zeros_like(a)
    if t == vva.F16:
        return a * 2.0 ** -11 + 2.0 ** -25
    if t == vva.BF16:
        return a * 2.0 ** -8
    # Q8_0: half a step of the block's scale (amax / 127), per 32-value block
    blk = a.reshape(*a.shape[:-1], -1, 32)
    step = (blk.max(axis=-1, keepdims=True) + MAX_TOL) / 127.0
    return np.broadcast_to(0.5 * step * 1.001, blk.shape).reshape(a.shape)


def _check(got, ref, t, what):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = MAX_TOL + _round_bound(ref, t)
    assert np.isfinite(got).all(), f"{what}: non-finite"
    worst = float((err - bound).max())
    assert worst <= 0, f"{what}: error exceeds bound by {worst:.3e} (max err {err.max():.3e})"
    excess = np.maximum(err - _round_bound(ref, t), 0.0)
    assert excess.mean() <= MEAN_TOL, f"{what}: mean {excess.mean():.3e}"
    return float(err.max()), float(excess.mean())


QKV_CASES = [
    # hidden, Hq, Hkv, d, weights, cache, T, B, q_out type
    (896, 14, 2, 64, vva.F16, vva.F16, 512, 1, vva.F32),       # 0.5B prefill chunk
    (896, 14, 2, 64, vva.Q8_0, vva.Q8_0, 1, 2, vva.F32),       # 0.5B CFG decode step, Q8_0 cache
    (1536, 12, 2, 128, vva.F16, vva.BF16, 300, 1, vva.F32),    # 1.5B, ragged last token tile
    (3584, 28, 4, 128, vva.Q8_0, vva.Q8_0, 1, 2, vva.F32),     # 7B CFG decode step
    (3584, 28, 4, 128, vva.F16, vva.F16, 512, 1, vva.F16),     # 7B ASR chunk, f16 Q
    (3584, 28, 4, 128, vva.Q8_0, vva.F32, 129, 2, vva.BF16),   # Q8_0 weights, two sequences
    (3584, 28, 4, 128, vva.F16, vva.Q8_0, 200, 2, vva.F32),    # F16 weights into a Q8_0 cache, two sequences
    (3584, 28, 4, 128, vva.F16, vva.F16, 1, 2, vva.F32),       # 7B CFG decode step, F16 weights (GEMV)
    (896, 14, 2, 64, vva.F16, vva.Q8_0, 3, 2, vva.F32),        # 6 token rows, F16 weights (GEMV)
    # >= 1024 token rows, F16 weights: the 256 x 256 tile GEMM
    (3584, 28, 4, 128, vva.F16, vva.Q8_0, 1030, 1, vva.F32),   # ragged last token tile, Q8_0 cache (pair epilogue)
    (896, 14, 2, 64, vva.F16, vva.F16, 640, 2, vva.BF16),      # two sequences, a half-filled last feature tile
    (1536, 12, 2, 128, vva.F16, vva.BF16, 1500, 1, vva.F16),   # 1.5B long chunk
    (1536, 12, 2, 128, vva.Q8_0, vva.F16, 1100, 1, vva.F32),   # Q8_0 weights dequantized for the long-call GEMM
]


@pytest.mark.parametrize("hidden,Hq,Hkv,d,wt,ct,T,B,qt", QKV_CASES)
def test_qkv_rope_append_matches_oracle(ctx, torch_gpu, hidden, Hq, Hkv, d, wt, ct, T, B, qt):
    torch = torch_gpu
    print(f"qkv hidden={hidden} Hq={Hq} Hkv={Hkv} d={d} w={wt} cache={ct} T={T} B={B} q={qt}", flush=True)
    rng = np.random.default_rng(hidden + T + wt + ct)
    pasts = [5 + 17 * b for b in range(B)]
    kv = vva.KVCache(ctx, 1, Hkv, d, max(pasts) + T + 8, B, ct)
    for b, p in enumerate(pasts):
        kv.set_len(b, p)
    x = rng.standard_normal((B, T, hidden)).astype(np.float32)
    wq_raw, wq = _weight(torch, rng, Hq * d, hidden, wt)
    wk_raw, wk = _weight(torch, rng, Hkv * d, hidden, wt)
    wv_raw, wv = _weight(torch, rng, Hkv * d, hidden, wt)
    bq, bk, bv = [(rng.standard_normal(n) * 0.5).astype(np.float32) for n in (Hq * d, Hkv * d, Hkv * d)]
    pos = np.array([[p + t for t in range(T)] for p in pasts], np.int32)
    q_out = torch.full((B, T, Hq, d), float("nan"), dtype={vva.F32: torch.float32, vva.F16: torch.float16,
                                                           vva.BF16: torch.bfloat16}[qt], device="cuda")
    ctx.qkv_rope_append(kv, 0, torch.from_numpy(x).cuda(), wq, wk, wv, torch.from_numpy(pos).cuda(), q_out,
                        bq=torch.from_numpy(bq).cuda(), bk=torch.from_numpy(bk).cuda(),
                        bv=torch.from_numpy(bv).cuda())
    torch.cuda.synchronize()
    got_q = as_f32(torch, q_out)
    for b in range(B):
        yq = vvo.linear(x[b], wq_raw, wt, Hq * d, bq).reshape(1, T, Hq, d)
        yk = vvo.linear(x[b], wk_raw, wt, Hkv * d, bk).reshape(1, T, Hkv, d)
        yv = vvo.linear(x[b], wv_raw, wt, Hkv * d, bv).reshape(T, Hkv, d)
        rq = vvo.rope(yq, pos[b])[0]
        rk = vvo.rope(yk, pos[b])[0]
        mq = _check(got_q[b], rq, qt, f"q (b={b})")
        kraw, vraw = kv.download(0, b, pasts[b] + T + 1)
        rb = kraw.shape[1]
        kdec = vvo.to_f32(kraw[pasts[b]:pasts[b] + T].reshape(-1), ct, T * Hkv * d).reshape(T, Hkv, d)
        vdec = vvo.to_f32(vraw[pasts[b]:pasts[b] + T].reshape(-1), ct, T * Hkv * d).reshape(T, Hkv, d)
        mk = _check(kdec, rk, ct, f"k cache (b={b})")
        mv = _check(vdec, yv, ct, f"v cache (b={b})")
        # rows outside [past, past + T) are untouched (the cache starts zeroed)
        assert not kraw[:pasts[b]].any() and not kraw[pasts[b] + T:].any()
        assert not vraw[:pasts[b]].any() and not vraw[pasts[b] + T:].any()
        assert rb == vvo.row_bytes(ct, d) * Hkv
        print(f"  b={b}: q max {mq[0]:.2e} mean {mq[1]:.2e}; k max {mk[0]:.2e}; v max {mv[0]:.2e}")
    kv.free()


def test_qkv_rope_append_without_bias_equals_rope_append(ctx, torch_gpu):
    """No bias: the fused call's cache bytes and rotated Q equal projecting
    with the same GEMM (out_proj with a zero residual) and then running
    vva_rope_append on the projections: one RoPE and append implementation."""
    torch = torch_gpu
    hidden, Hq, Hkv, d, T = 896, 14, 2, 64, 40
    rng = np.random.default_rng(31)
    x = torch.from_numpy(rng.standard_normal((1, T, hidden)).astype(np.float32)).cuda()
    ws = [_weight(torch, rng, n, hidden, vva.F16) for n in (Hq * d, Hkv * d, Hkv * d)]
    pos = torch.arange(3, 3 + T, dtype=torch.int32, device="cuda")
    a = vva.KVCache(ctx, 1, Hkv, d, T + 8, 1, vva.F16)
    b = vva.KVCache(ctx, 1, Hkv, d, T + 8, 1, vva.F16)
    for kv in (a, b):
        kv.set_len(0, 3)
    qa = torch.empty((1, T, Hq, d), dtype=torch.float32, device="cuda")
    ctx.qkv_rope_append(a, 0, x, ws[0][1], ws[1][1], ws[2][1], pos, qa)
    proj = []
    for (_, w), n in zip(ws, (Hq, Hkv, Hkv)):
        y = torch.zeros((1, T, n * d), dtype=torch.float32, device="cuda")
        ctx.out_proj_residual(x, w, y, y)            # y = x w^T + 0
        proj.append(y.reshape(1, T, n, d))
    qb = torch.empty_like(qa)
    ctx.rope_append(b, 0, proj[0], proj[1], proj[2], pos, qb)
    torch.cuda.synchronize()
    assert torch.equal(qa, qb)
    ka, va = a.download(0, 0, T + 3)
    kb, vb = b.download(0, 0, T + 3)
    np.testing.assert_array_equal(ka, kb)
    np.testing.assert_array_equal(va, vb)
    a.free()
    b.free()


@pytest.mark.parametrize("d,Hq,Hkv,hidden,wt,ct,T,B", [
    (128, 28, 4, 3584, vva.F16, vva.F16, 1, 2),      # 7B CFG decode step
    (128, 28, 4, 3584, vva.Q8_0, vva.BF16, 1, 2),
    (64, 14, 2, 896, vva.F16, vva.F32, 2, 1),        # two tokens of one sequence
    (64, 14, 2, 896, vva.Q8_0, vva.F16, 1, 1),
])
def test_decode_step_fused_rope_equals_rope_append(ctx, torch_gpu, d, Hq, Hkv, hidden, wt, ct, T, B):
    """The decode step's one- and two-row call (RoPE and the append in the
    projection's epilogue, the angles tabulated once per workgroup) stores
    the same bits as projecting with out_proj (zero residual, the same
    kernel's dot products) and then running vva_rope_append, at positions
    whose angles need the large-argument reduction of cos / sin."""
    torch = torch_gpu
    rng = np.random.default_rng(d + T + wt)
    x = torch.from_numpy(rng.standard_normal((B, T, hidden)).astype(np.float32)).cuda()
    ws = [_weight(torch, rng, n * d, hidden, wt) for n in (Hq, Hkv, Hkv)]
    pos = torch.tensor([[30011 + 977 * b + t for t in range(T)] for b in range(B)], dtype=torch.int32, device="cuda")
    past = 5
    a = vva.KVCache(ctx, 1, Hkv, d, past + T + 4, B, ct)
    c = vva.KVCache(ctx, 1, Hkv, d, past + T + 4, B, ct)
    for kv in (a, c):
        for b in range(B):
            kv.set_len(b, past)
    qa = torch.empty((B, T, Hq, d), dtype=torch.float32, device="cuda")
    ctx.qkv_rope_append(a, 0, x, ws[0][1], ws[1][1], ws[2][1], pos, qa)
    proj = []
    for (_, w), n in zip(ws, (Hq, Hkv, Hkv)):
        y = torch.zeros((B, T, n * d), dtype=torch.float32, device="cuda")
        ctx.out_proj_residual(x, w, y, y)            # y = x w^T + 0
        proj.append(y.reshape(B, T, n, d))
    qc = torch.empty_like(qa)
    ctx.rope_append(c, 0, proj[0], proj[1], proj[2], pos, qc)
    torch.cuda.synchronize()
    assert torch.equal(qa, qc), f"q differs: max {float((qa - qc).abs().max()):.3e}"
    for b in range(B):
        ka, va = a.download(0, b, past + T)
        kc, vc = c.download(0, b, past + T)
        np.testing.assert_array_equal(ka, kc)
        np.testing.assert_array_equal(va, vc)
    a.free()
    c.free()


@pytest.mark.parametrize("hidden,Hq,Hkv,d,wt,T,B", [
    (3584, 28, 4, 128, vva.Q8_0, 1, 2),    # 7B CFG decode step, Q8_0 weights
    (3584, 28, 4, 128, vva.F16, 1, 2),
    (896, 14, 2, 64, vva.F16, 3, 2),       # 6 token rows
    (1536, 12, 2, 128, vva.Q8_0, 1, 1),
])
def test_qkv_proj_matches_oracle(ctx, torch_gpu, hidden, Hq, Hkv, d, wt, T, B):
    """vva_qkv_proj: the bare q/k/v projections with bias of a decode step,
    one [q | k | v] row per token, against the oracle's linear()."""
    torch = torch_gpu
    print(f"qkv_proj hidden={hidden} Hq={Hq} Hkv={Hkv} d={d} w={wt} T={T} B={B}", flush=True)
    rng = np.random.default_rng(5 * hidden + T + wt)
    x = rng.standard_normal((B, T, hidden)).astype(np.float32)
    wq_raw, wq = _weight(torch, rng, Hq * d, hidden, wt)
    wk_raw, wk = _weight(torch, rng, Hkv * d, hidden, wt)
    wv_raw, wv = _weight(torch, rng, Hkv * d, hidden, wt)
    bq, bk, bv = [(rng.standard_normal(n) * 0.5).astype(np.float32) for n in (Hq * d, Hkv * d, Hkv * d)]
    M = (Hq + 2 * Hkv) * d
    y = torch.full((B, T, M), float("nan"), dtype=torch.float32, device="cuda")
    ctx.qkv_proj(torch.from_numpy(x).cuda(), wq, wk, wv, y, bq=torch.from_numpy(bq).cuda(),
                 bk=torch.from_numpy(bk).cuda(), bv=torch.from_numpy(bv).cuda())
    torch.cuda.synchronize()
    got = as_f32(torch, y)
    for b in range(B):
        ref = np.concatenate([vvo.linear(x[b], wq_raw, wt, Hq * d, bq), vvo.linear(x[b], wk_raw, wt, Hkv * d, bk),
                              vvo.linear(x[b], wv_raw, wt, Hkv * d, bv)], axis=-1)
        m = _check(got[b], ref, vva.F32, f"y (b={b})")
        print(f"  b={b}: max {m[0]:.2e} mean {m[1]:.2e}")
    # a prefill chunk is vva_qkv_rope_append's
    x16 = torch.zeros((1, 16, hidden), dtype=torch.float32, device="cuda")
    y16 = torch.zeros((1, 16, M), dtype=torch.float32, device="cuda")
    with pytest.raises(vva.VvaError) as e:
        ctx.qkv_proj(x16, wq, wk, wv, y16)
    assert e.value.status == vva.ERR_NOT_IMPLEMENTED


O_CASES = [
    # in (Hq * d), hidden, weights, T, B, o type
    (896, 896, vva.F16, 256, 1, vva.F32),       # 0.5B layer of the TTS prefill
    (896, 896, vva.Q8_0, 1, 2, vva.F32),        # 0.5B CFG decode step
    (1536, 1536, vva.F16, 333, 1, vva.BF16),
    (3584, 3584, vva.Q8_0, 512, 1, vva.F32),    # 7B ASR chunk
    (3584, 3584, vva.F16, 2, 2, vva.F16),
    (1536, 1536, vva.F16, 4, 2, vva.BF16),      # 8 token rows: more row chunks than the staged batch
    (3584, 3584, vva.F16, 1, 2, vva.F32),       # 7B CFG decode step
    (3584, 3584, vva.F16, 1024, 2, vva.F32),    # 2048 token rows: the 256 x 256 tile GEMM
    (1536, 1536, vva.F16, 1100, 1, vva.BF16),   # ragged last token tile
    (3584, 3584, vva.Q8_0, 640, 2, vva.F32),    # Q8_0 weights dequantized for the long-call GEMM
]


@pytest.mark.parametrize("K,hidden,wt,T,B,ot", O_CASES)
def test_out_proj_residual_matches_oracle(ctx, torch_gpu, K, hidden, wt, T, B, ot):
    torch = torch_gpu
    print(f"out_proj K={K} hidden={hidden} w={wt} T={T} B={B} o={ot}", flush=True)
    rng = np.random.default_rng(K + T + wt)
    o = rng.standard_normal((B, T, K)).astype(np.float32)
    x = rng.standard_normal((B, T, hidden)).astype(np.float32)
    w_raw, w = _weight(torch, rng, hidden, K, wt)
    og = to_gpu(torch, o, ot)
    o_used = as_f32(torch, og)                        # o as the device holds it
    xg = torch.from_numpy(x).cuda()
    h = torch.full((B, T, hidden), float("nan"), dtype=torch.float32, device="cuda")
    ctx.out_proj_residual(og, w, xg, h)
    # in place: h aliasing x
    ctx.out_proj_residual(og, w, xg, xg)
    torch.cuda.synchronize()
    ref = vvo.linear(o_used, w_raw, wt, hidden) + x
    m = _check(as_f32(torch, h), ref, vva.F32, "h")
    assert torch.equal(h, xg)
    print(f"  max {m[0]:.2e} mean {m[1]:.2e}")


@pytest.mark.parametrize("wt", [vva.F16, vva.Q8_0])
def test_short_chunk_projections_repeat_bit_for_bit(ctx, torch_gpu, wt):
    """A 512-token ASR chunk fills few GEMM tiles, so the GEMM is split along
    K: every piece stores its partial and the tile's last piece sums them in
    split order.  The sum must not depend on which piece finishes last, and the
    tiles' tickets must be back at zero after each call: three calls in a row
    give the same bytes, and the result matches the oracle."""
    torch = torch_gpu
    hidden, Hq, Hkv, d, T = 3584, 28, 4, 128, 512
    print(f"split-K projections w={wt} T={T}", flush=True)
    rng = np.random.default_rng(77 + wt)
    x = rng.standard_normal((1, T, hidden)).astype(np.float32)
    wo_raw, wo = _weight(torch, rng, hidden, Hq * d, wt)
    o = rng.standard_normal((1, T, Hq * d)).astype(np.float32)
    xg, og = torch.from_numpy(x).cuda(), torch.from_numpy(o).cuda()
    hs = []
    for _ in range(3):
        h = torch.full((1, T, hidden), float("nan"), dtype=torch.float32, device="cuda")
        ctx.out_proj_residual(og, wo, xg, h)
        torch.cuda.synchronize()
        hs.append(as_f32(torch, h))
    assert np.array_equal(hs[0], hs[1]) and np.array_equal(hs[0], hs[2])
    ref = vvo.linear(o[0], wo_raw, wt, hidden) + x[0]
    m = _check(hs[0][0], ref, vva.F32, "h (split K)")
    wq_raw, wq = _weight(torch, rng, Hq * d, hidden, wt)
    wk_raw, wk = _weight(torch, rng, Hkv * d, hidden, wt)
    wv_raw, wv = _weight(torch, rng, Hkv * d, hidden, wt)
    pos = torch.arange(T, dtype=torch.int32, device="cuda").reshape(1, T)
    qs = []
    for _ in range(3):
        kv = vva.KVCache(ctx, 1, Hkv, d, T + 8, 1, vva.F16)
        q_out = torch.full((1, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
        ctx.qkv_rope_append(kv, 0, xg, wq, wk, wv, pos, q_out)
        torch.cuda.synchronize()
        qs.append(as_f32(torch, q_out))
        kv.free()
    assert np.array_equal(qs[0], qs[1]) and np.array_equal(qs[0], qs[2])
    yq = vvo.linear(x[0], wq_raw, wt, Hq * d).reshape(1, T, Hq, d)
    rq = vvo.rope(yq, np.arange(T, dtype=np.int32))[0]
    mq = _check(qs[0][0], rq, vva.F32, "q (split K)")
    print(f"  h max {m[0]:.2e}; q max {mq[0]:.2e}")


@pytest.mark.parametrize("wt", [vva.F16, vva.Q8_0])
def test_4096_token_projection_with_split_tail(ctx, torch_gpu, wt):
    """At 4096 tokens the 7B q/k/v GEMM has 576 (F16) or 1152 (Q8_0) tiles:
    two or more full rounds and a last round of a quarter of the CUs, whose
    tiles are split along K and merged by their last piece.  The first and
    last 256 token rows (the last ones are in the split tail) match the
    oracle, and two calls give the same bytes."""
    torch = torch_gpu
    hidden, Hq, Hkv, d, T = 3584, 28, 4, 128, 4096
    print(f"tail-split projections w={wt} T={T}", flush=True)
    rng = np.random.default_rng(91 + wt)
    x = rng.standard_normal((1, T, hidden)).astype(np.float32)
    wq_raw, wq = _weight(torch, rng, Hq * d, hidden, wt)
    wk_raw, wk = _weight(torch, rng, Hkv * d, hidden, wt)
    wv_raw, wv = _weight(torch, rng, Hkv * d, hidden, wt)
    xg = torch.from_numpy(x).cuda()
    pos = torch.arange(T, dtype=torch.int32, device="cuda").reshape(1, T)
    qs, ks = [], []
    for _ in range(2):
        kv = vva.KVCache(ctx, 1, Hkv, d, T + 8, 1, vva.F16)
        q_out = torch.full((1, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
        ctx.qkv_rope_append(kv, 0, xg, wq, wk, wv, pos, q_out)
        torch.cuda.synchronize()
        qs.append(as_f32(torch, q_out))
        kraw, _ = kv.download(0, 0, T)
        ks.append(kraw.copy())
        kv.free()
    assert np.array_equal(qs[0], qs[1]) and np.array_equal(ks[0], ks[1])
    rows = np.r_[0:256, T - 256:T]
    yq = vvo.linear(x[0][rows], wq_raw, wt, Hq * d).reshape(1, len(rows), Hq, d)
    rq = vvo.rope(yq, rows.astype(np.int32))[0]
    mq = _check(qs[0][0][rows], rq, vva.F32, "q rows (split tail)")
    yk = vvo.linear(x[0][rows], wk_raw, wt, Hkv * d).reshape(1, len(rows), Hkv, d)
    rk = vvo.rope(yk, rows.astype(np.int32))[0]
    kdec = vvo.to_f32(ks[0][rows].reshape(-1), vva.F16, len(rows) * Hkv * d).reshape(len(rows), Hkv, d)
    mk = _check(kdec, rk, vva.F16, "k cache rows (split tail)")
    print(f"  q max {mq[0]:.2e}; k max {mk[0]:.2e}")


def test_projection_argument_errors(ctx, torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(0)
    _, w = _weight(torch, rng, 896, 896, vva.F16)
    o = torch.zeros((1, 4, 896), dtype=torch.float32, device="cuda")
    x = torch.zeros((1, 4, 896), dtype=torch.float32, device="cuda")
    bad = torch.zeros((1, 4, 800), dtype=torch.float32, device="cuda")
    with pytest.raises(vva.VvaError) as e:
        ctx.out_proj_residual(o, w, bad, bad)          # residual of the wrong width
    assert e.value.status == vva.ERR_INVALID_ARG
    # h may alias x (in-place residual), never o: the few-row kernel reads
    # every row of o while other workgroups already write h
    with pytest.raises(vva.VvaError) as e:
        ctx.out_proj_residual(o, w, x, o)
    assert e.value.status == vva.ERR_INVALID_ARG and "overlaps" in str(e.value)
    ctx.out_proj_residual(o, w, x, x)                  # h == x is allowed
    torch.cuda.synchronize()
    kv = vva.KVCache(ctx, 1, 2, 64, 8, 1, vva.F16)
    kv.set_len(0, 6)
    q = torch.zeros((1, 4, 14, 64), dtype=torch.float32, device="cuda")
    pos = torch.arange(4, dtype=torch.int32, device="cuda")
    _, wkv = _weight(torch, rng, 128, 896, vva.F16)
    with pytest.raises(vva.VvaError) as e:             # 6 + 4 rows > max_seq 8
        ctx.qkv_rope_append(kv, 0, x, w, wkv, wkv, pos, q)
    assert e.value.status == vva.ERR_INVALID_ARG
    kv.free()
