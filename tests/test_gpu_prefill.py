"""GPU parity of the MFMA flash prefill through the C ABI.

Cases cover the three prefill shapes of the reference (0.5B / 1.5B / 7B
Qwen2.5 heads), single-shot and chunked (past > 0, the ASR 512-token chunk
loop, src/vibevoice_asr.cpp:542-652), ragged CFG batches, explicit masks and
the ggml-shaped vva_flash_attn_ext entry.  Tolerance 2e-3 max-abs / 1e-3
mean-abs against the oracle on the device's own cache bytes.  The chunked
replay mirrors tests/test_qwen2_resident.cpp paths B-D (single shot, two
chunks, four uneven chunks).  At the full 32768-token 7B shape the oracle
checks a deterministic row subset plus the first and last 128 rows.
"""
import numpy as np
import pytest

import vva
import vvo
from gpu_util import as_f32, assert_close, check_ggml_order, err_stats, fill_cache, oracle_attn, to_gpu

pytestmark = pytest.mark.gpu
TOL = (2e-3, 1e-3)

CASES = [
    # d, Hq, Hkv, type, T, past, q_type, B
    (128, 12, 2, vva.F16, 512, 0, vva.BF16, 1),     # 1.5B voice-cloning prefill shape
    (128, 12, 2, vva.BF16, 512, 0, vva.BF16, 1),
    (128, 28, 4, vva.F16, 300, 0, vva.F16, 1),      # 7B, tail tile
    (128, 28, 4, vva.F16, 512, 1536, vva.F16, 1),   # ASR chunk 4 of a 512-chunk prefill
    (128, 28, 4, vva.BF16, 77, 3000, vva.F32, 1),
    (64, 14, 2, vva.F16, 256, 0, vva.F32, 1),       # 0.5B
    (64, 14, 2, vva.F16, 5, 1030, vva.F32, 2),      # TTS text window on both CFG streams
    (128, 28, 4, vva.F16, 2, 0, vva.F32, 1),
    # Q8_0 caches: the window converted to f16 (contiguous rows: the flat
    # conversion), ragged sequences of one call included
    (128, 28, 4, vva.Q8_0, 512, 1536, vva.F32, 1),
    (128, 28, 4, vva.Q8_0, 33, 700, vva.BF16, 2),
    (64, 14, 2, vva.Q8_0, 40, 1030, vva.F32, 2),
]


@pytest.mark.parametrize("d,Hq,Hkv,t,T,past,q_type,B", CASES)
def test_prefill_matches_oracle(ctx, torch_gpu, d, Hq, Hkv, t, T, past, q_type, B):
    torch = torch_gpu
    print(f"prefill d={d} Hq={Hq} Hkv={Hkv} type={t} T={T} past={past} B={B}", flush=True)
    pasts = [past + 17 * b for b in range(B)]
    L = [p + T for p in pasts]
    kv = vva.KVCache(ctx, 1, Hkv, d, max(L), B, t)
    fill_cache(kv, L, seed=T + past + d)
    for b in range(B):
        kv.set_len(b, pasts[b])
    rng = np.random.default_rng(T)
    q = to_gpu(torch, rng.standard_normal((B, T, Hq, d)), q_type)
    out = torch.full((B, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    ctx.attn(kv, 0, q, out, d ** -0.5)
    torch.cuda.synchronize()
    q32, o = as_f32(torch, q), as_f32(torch, out)
    ref = oracle_attn(q32, kv, 0, range(B), L, T, d ** -0.5)
    mx, mn = assert_close(o, ref, *TOL, what="prefill vs exact")
    (gmx, gmn), (hmx, hmn) = check_ggml_order(o, q32, kv, 0, range(B), L, T, d ** -0.5, *TOL, what="prefill")
    print(f"  vs exact max {mx:.2e} mean {mn:.2e}; vs ggml order max {gmx:.2e} mean {gmn:.2e} "
          f"(F16 V sum: max {hmx:.2e} mean {hmn:.2e})")
    kv.free()


def test_prefill_explicit_mask_and_no_mask(ctx, torch_gpu):
    torch = torch_gpu
    d, Hq, Hkv, T, past = 128, 28, 4, 96, 40
    L = past + T
    kv = vva.KVCache(ctx, 1, Hkv, d, L, 1, vva.F16)
    fill_cache(kv, [L], seed=5)
    kv.set_len(0, past)
    rng = np.random.default_rng(6)
    m = np.where(np.arange(L)[None, :] > past + np.arange(T)[:, None], -np.inf, 0.0).astype(np.float32)
    m[:, 10:30] = -np.inf                              # a block of keys nobody sees
    m[7, :] = -np.inf                                  # a row with no visible key -> 0
    mbits = vvo.f16_bits(m)[None]
    q = to_gpu(torch, rng.standard_normal((1, T, Hq, d)), vva.F16)
    out = torch.empty((1, T, Hq, d), dtype=torch.float32, device="cuda")
    ctx.attn(kv, 0, q, out, d ** -0.5, mask=torch.from_numpy(mbits.view(np.float16)).cuda())
    torch.cuda.synchronize()
    o = as_f32(torch, out)
    ref = oracle_attn(as_f32(torch, q), kv, 0, [0], [L], T, d ** -0.5, mask=mbits)
    assert_close(o, ref, *TOL, what="explicit mask")
    assert not o[0, 7].any()
    # ggml_flash_attn_ext without a mask: every key visible
    kview, vview = kv.views(0, 0)
    for t_ in (kview, vview):
        t_.ne[1], t_.ne[2] = t_.ne[2], t_.ne[1]        # ne = [d, L, Hkv, 1] (permuted view)
        t_.nb[1], t_.nb[2] = t_.nb[2], t_.nb[1]
        t_.ne[1] = L
    qp = q.permute(0, 2, 1, 3)                          # ne = [d, T, Hq, 1]
    ctx.flash_attn_ext(qp, None, None, out, d ** -0.5, k_view=kview, v_view=vview)
    torch.cuda.synchronize()
    kraw, vraw = kv.download(0, 0, L)
    ref = vvo.attn(as_f32(torch, q), [kraw.reshape(-1)], [vraw.reshape(-1)], 1, 1, [L], n_kv_heads=Hkv,
                   scale=d ** -0.5, mask_mode=vvo.MASK_NONE)
    assert_close(as_f32(torch, out), ref, *TOL, what="no mask")
    kv.free()


def _resident_replay(ctx, torch, bounds, t, seed=1):
    """RoPE + append + attention of N tokens in the given chunks, one layer."""
    d, Hq, Hkv = 128, 28, 4
    N = bounds[-1]
    rng = np.random.default_rng(seed)
    q = to_gpu(torch, rng.standard_normal((1, N, Hq, d)), vva.BF16)
    k = to_gpu(torch, rng.standard_normal((1, N, Hkv, d)), vva.BF16)
    v = to_gpu(torch, rng.standard_normal((1, N, Hkv, d)), vva.BF16)
    kv = vva.KVCache(ctx, 1, Hkv, d, N, 1, t)
    out = torch.empty((1, N, Hq, d), dtype=torch.float32, device="cuda")
    qr = torch.empty((1, N, Hq, d), dtype=torch.float16, device="cuda")
    for a, b in zip(bounds[:-1], bounds[1:]):
        pos = torch.arange(a, b, dtype=torch.int32, device="cuda")
        ctx.rope_append(kv, 0, q[:, a:b], k[:, a:b], v[:, a:b], pos, qr[:, a:b])
        ctx.attn(kv, 0, qr[:, a:b], out[:, a:b], d ** -0.5)
        kv.set_len(0, b)
    torch.cuda.synchronize()
    res = as_f32(torch, out), kv.download(0, 0, N)
    kv.free()
    return res


def test_chunked_prefill_equals_single_shot(ctx, torch_gpu):
    """tests/test_qwen2_resident.cpp paths B (one shot), C (two chunks), D (four
    uneven).  Cache bytes are identical.  Outputs: the reference's tolerance
    for chunked flash attention, 1e-3 (tests/test_qwen2_resident.cpp:478-479),
    on the default path (later chunks split their keys over workgroups, with
    P rounded to f16 against another exponent base); with one key split per
    row tile the chunks reproduce the single shot to 1e-5."""
    torch = torch_gpu
    N = 700
    one, cache1 = _resident_replay(ctx, torch, [0, N], vva.F16)
    two, cache2 = _resident_replay(ctx, torch, [0, N // 2, N], vva.F16)
    four, cache4 = _resident_replay(ctx, torch, [0, N // 4, N // 2, 3 * N // 4, N], vva.F16)
    for c in (cache2, cache4):
        np.testing.assert_array_equal(c[0], cache1[0])
        np.testing.assert_array_equal(c[1], cache1[1])
    assert np.abs(two - one).max() < 1e-3
    assert np.abs(four - one).max() < 1e-3
    with ctx.schedule(prefill_splits=1):
        one1, _ = _resident_replay(ctx, torch, [0, N], vva.F16)
        two1, _ = _resident_replay(ctx, torch, [0, N // 2, N], vva.F16)
        four1, _ = _resident_replay(ctx, torch, [0, N // 4, N // 2, 3 * N // 4, N], vva.F16)
    assert np.abs(one1 - one).max() < 1e-3
    assert np.abs(two1 - one1).max() < 1e-5
    assert np.abs(four1 - one1).max() < 1e-5


def test_decode_after_prefill_equals_last_prefill_row(ctx, torch_gpu):
    torch = torch_gpu
    N = 1000
    full, _ = _resident_replay(ctx, torch, [0, N], vva.F16, seed=3)
    step, _ = _resident_replay(ctx, torch, [0, N - 1, N], vva.F16, seed=3)
    # different kernels (split-K fp32 P vs MFMA f16 P): the FA tolerance of
    # tests/test_qwen2_resident.cpp:478
    assert np.abs(step[0, N - 1] - full[0, N - 1]).max() < 1e-3


@pytest.mark.parametrize("t", [vva.F16, vva.Q8_0])
def test_chunk_over_a_128k_past(ctx, torch_gpu, t):
    """The last 512-token ASR chunk of a 128k-token window (7B heads): key
    splits merged in the launch (F16), and the converted f16 window of
    67 MB per operand plus the gated fallback (Q8_0).  Rows: the chunk's first
    and last 16 and 16 spread between."""
    torch = torch_gpu
    d, Hq, Hkv, T = 128, 28, 4, 512
    L = 131072
    past = L - T
    print(f"chunk over a 128k past type={t}", flush=True)
    kv = vva.KVCache(ctx, 1, Hkv, d, L, 1, t)
    fill_cache(kv, [L], seed=1280 + t)
    kv.set_len(0, past)
    rng = np.random.default_rng(1281)
    q = to_gpu(torch, rng.standard_normal((1, T, Hq, d)), vva.BF16)
    out = torch.full((1, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    ctx.attn(kv, 0, q, out, d ** -0.5)
    torch.cuda.synchronize()
    o = as_f32(torch, out)
    assert np.isfinite(o).all()
    rows = np.unique(np.concatenate([np.arange(16), np.arange(T - 16, T),
                                     np.linspace(16, T - 17, 16).astype(np.int64)])).astype(np.int32)
    q32 = as_f32(torch, q)
    ref = oracle_attn(q32, kv, 0, [0], [L], T, d ** -0.5, rows=rows)
    mx, mn = assert_close(o[0, rows], ref[0, rows], *TOL, what="128k-past chunk vs exact")
    print(f"  splits {ctx.last_decode_splits()}: vs exact max {mx:.2e} mean {mn:.2e}")
    kv.free()


def test_full_size_7b_prefill_row_subset(ctx, torch_gpu):
    """32768-token causal prefill, 28q/4kv, d=128, F16 cache (bf16 inputs)."""
    torch = torch_gpu
    d, Hq, Hkv, T = 128, 28, 4, 32768
    kv = vva.KVCache(ctx, 1, Hkv, d, T, 1, vva.F16)
    fill_cache(kv, [T], seed=77)
    kv.set_len(0, 0)
    rng = np.random.default_rng(78)
    q = to_gpu(torch, rng.standard_normal((1, T, Hq, d)), vva.BF16)
    out = torch.empty((1, T, Hq, d), dtype=torch.float32, device="cuda")
    ctx.attn(kv, 0, q, out, d ** -0.5)
    torch.cuda.synchronize()
    o = as_f32(torch, out)
    assert np.isfinite(o).all()
    rows = np.unique(np.concatenate([np.arange(128), np.arange(T - 128, T),
                                     np.linspace(128, T - 129, 64).astype(np.int64)])).astype(np.int32)
    q32 = as_f32(torch, q)
    ref = oracle_attn(q32, kv, 0, [0], [T], T, d ** -0.5, rows=rows)
    mx, mn = assert_close(o[0, rows], ref[0, rows], *TOL, what="32k subset vs exact")
    # ggml's CPU order: Q rounded to f16, per-key online softmax; with F16 V
    # the order's running V sum is kept in f16, whose own distance from the
    # exact result grows with the number of keys a row sees
    (gmx, gmn), (hmx, hmn) = check_ggml_order(o, q32, kv, 0, [0], [T], T, d ** -0.5, *TOL, rows=rows,
                                              what="32k subset")
    g16 = oracle_attn(q32, kv, 0, [0], [T], T, d ** -0.5, rows=rows, mode=vvo.GGML)
    smx, smn = err_stats(g16[0, rows], ref[0, rows])
    print(f"32k subset ({len(rows)} rows): vs exact max {mx:.2e} mean {mn:.2e}; vs ggml order max {gmx:.2e} "
          f"mean {gmn:.2e}; vs ggml order with F16 V sum max {hmx:.2e} mean {hmn:.2e}; that order vs exact "
          f"max {smx:.2e} mean {smn:.2e}")
    kv.free()


@pytest.mark.parametrize("t", [vva.F16, vva.BF16])
def test_full_size_1p5b_voice_clone_prefill(ctx, torch_gpu, t):
    """The 1.5B voice-cloning prefill at its configured size
    (src/vibevoice_tts.cpp:1199-1204): 4096 tokens in one causal shot, 12 q /
    2 kv heads, d = 128, bf16 Q/K/V N(0,1) roped (theta 1e6) and appended by
    vva_rope_append, then attention over the cache.  Every row is checked
    against both oracle modes."""
    torch = torch_gpu
    d, Hq, Hkv, T = 128, 12, 2, 4096
    print(f"1.5B prefill T={T} cache type {t}", flush=True)
    rng = np.random.default_rng(4096 + t)
    q = to_gpu(torch, rng.standard_normal((1, T, Hq, d)), vva.BF16)
    k = to_gpu(torch, rng.standard_normal((1, T, Hkv, d)), vva.BF16)
    v = to_gpu(torch, rng.standard_normal((1, T, Hkv, d)), vva.BF16)
    kv = vva.KVCache(ctx, 1, Hkv, d, T, 1, t)
    # RoPE(q) in the cache's type: the type attention rounds Q to anyway
    qr = torch.empty((1, T, Hq, d), dtype=torch.float16 if t == vva.F16 else torch.bfloat16, device="cuda")
    ctx.rope_append(kv, 0, q, k, v, torch.arange(T, dtype=torch.int32, device="cuda"), qr)
    out = torch.full((1, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    ctx.attn(kv, 0, qr, out, d ** -0.5)
    torch.cuda.synchronize()
    o, q32 = as_f32(torch, out), as_f32(torch, qr)
    ref = oracle_attn(q32, kv, 0, [0], [T], T, d ** -0.5)
    mx, mn = assert_close(o, ref, *TOL, what="1.5B T=4096 vs exact")
    (gmx, gmn), (hmx, hmn) = check_ggml_order(o, q32, kv, 0, [0], [T], T, d ** -0.5, *TOL, what="1.5B T=4096")
    print(f"  vs exact max {mx:.2e} mean {mn:.2e}; vs ggml order max {gmx:.2e} mean {gmn:.2e} "
          f"(F16 V sum: max {hmx:.2e} mean {hmn:.2e})")
    kv.free()


@pytest.mark.parametrize("t", [vva.F16, vva.BF16])
def test_prefill_repeated_score_jumps(ctx, torch_gpu, t):
    """Heavy-tailed logits: every query has 8 in dim 0 and the keys of 64-key
    tile j carry 2 sqrt(d) (j + 1) there, so each tile adds 16 nats to every
    row's scores and a row's running max jumps at every tile boundary it
    crosses (31 jumps for the last rows of a 2048-token prefill).  Every jump
    rescales O and the row sum; the result must match the exact oracle and
    stay finite."""
    torch = torch_gpu
    d, Hq, Hkv, T = 128, 28, 4, 2048
    rng = np.random.default_rng(21 + t)
    k = rng.standard_normal((T, Hkv, d)).astype(np.float32)
    k[:, :, 0] = (2.0 * d ** 0.5 * (np.arange(T) // 64 + 1))[:, None]
    v = rng.standard_normal((T, Hkv, d)).astype(np.float32)
    qn = rng.standard_normal((1, T, Hq, d))
    qn[..., 0] = 8.0
    kv = vva.KVCache(ctx, 1, Hkv, d, T, 1, t)
    kv.upload(0, 0, 0, k, v)
    kv.set_len(0, 0)
    q = to_gpu(torch, qn, t)
    out = torch.full((1, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    ctx.attn(kv, 0, q, out, d ** -0.5)
    torch.cuda.synchronize()
    o = as_f32(torch, out)
    assert np.isfinite(o).all()
    rows = np.unique(np.concatenate([np.arange(T - 256, T), np.arange(0, T, 37)])).astype(np.int32)
    q32 = as_f32(torch, q)
    ref = oracle_attn(q32, kv, 0, [0], [T], T, d ** -0.5, rows=rows)
    # jumps seen by the last row: tiles whose max score passes the running max by 10 nats
    kd = vvo.to_f32(kv.download(0, 0, T)[0].reshape(-1), t, T * Hkv * d).reshape(T, Hkv, d)
    s = (kd[:, 0] @ q32[0, T - 1, 0]) * d ** -0.5
    tile_max = s.reshape(-1, 64).max(axis=1)
    jumps = int(np.sum(tile_max[1:] > np.maximum.accumulate(tile_max)[:-1] + 10.0))
    mx, mn = assert_close(o[0, rows], ref[0, rows], *TOL, what="repeated score jumps")
    print(f"score jumps > 10 nats (last row, head 0): {jumps}; max {mx:.2e} mean {mn:.2e}")
    assert jumps >= 20
    kv.free()


def test_prefill_single_large_score_jump(ctx, torch_gpu):
    """Scores of later keys exceed the first tiles' by far more than 2^15 in
    the exp2 domain: the running max must be raised (O rescaled) without
    overflowing the f16 probabilities."""
    torch = torch_gpu
    d, Hq, Hkv, T = 128, 28, 4, 400
    rng = np.random.default_rng(11)
    k = rng.standard_normal((1, T, Hkv, d)) * 0.05
    k[:, 150:] *= 160.0                               # logits up to ~x60 larger after key 150
    v = rng.standard_normal((1, T, Hkv, d))
    kv = vva.KVCache(ctx, 1, Hkv, d, T, 1, vva.F16)
    kv.upload(0, 0, 0, k[0].astype(np.float32), v[0].astype(np.float32))
    kv.set_len(0, 0)
    q = to_gpu(torch, rng.standard_normal((1, T, Hq, d)), vva.F16)
    out = torch.full((1, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    ctx.attn(kv, 0, q, out, d ** -0.5)
    torch.cuda.synchronize()
    o = as_f32(torch, out)
    assert np.isfinite(o).all()
    ref = oracle_attn(as_f32(torch, q), kv, 0, [0], [T], T, d ** -0.5)
    assert_close(o, ref, *TOL, what="score jump")
    kv.free()


def _prefill_with_splits(ctx, torch, kv, q, splits, mask=None):
    d = kv.head_dim
    out = torch.full(tuple(q.shape[:3]) + (d,), float("nan"), dtype=torch.float32, device="cuda")
    with ctx.schedule(prefill_splits=splits):
        ctx.attn(kv, 0, q, out, d ** -0.5, mask=mask)
        torch.cuda.synchronize()
    return as_f32(torch, out), ctx.last_decode_splits()


def test_prefill_key_splits_do_not_change_result(ctx, torch_gpu):
    """A short chunk over a long past runs its keys in several workgroups per
    row tile (partials merged by log-sum-exp): the result must not depend on
    the split count beyond f16 rounding of P, and must match the oracle."""
    torch = torch_gpu
    d, Hq, Hkv, T, past = 128, 28, 4, 256, 5000
    L = past + T
    kv = vva.KVCache(ctx, 1, Hkv, d, L, 1, vva.F16)
    fill_cache(kv, [L], seed=21)
    kv.set_len(0, past)
    q = to_gpu(torch, np.random.default_rng(22).standard_normal((1, T, Hq, d)), vva.BF16)
    outs = []
    for n in (1, 2, 7, 32):
        o, used = _prefill_with_splits(ctx, torch, kv, q, n)
        assert used == n
        outs.append(o)
    for o in outs[1:]:
        assert np.isfinite(o).all()
        assert np.abs(o - outs[0]).max() < 2e-4
    ref = oracle_attn(as_f32(torch, q), kv, 0, [0], [L], T, d ** -0.5)
    assert_close(outs[2], ref, *TOL, what="7 key splits")
    kv.free()


@pytest.mark.parametrize("splits,masked", [(2, False), (3, False), (4, False), (4, True)])
def test_prefill_in_launch_merge_equals_merge_kernel(ctx, torch_gpu, splits, masked):
    """With at most four key splits per row tile, the last split of a row
    tile to finish merges the partials inside the prefill launch (a ticket
    per row tile); vva_attn_noalloc keeps the separate merge kernel.  Both
    combine the same partials in split order with the same arithmetic, so the
    outputs are equal bit for bit: two sequences of different lengths, causal
    or with an explicit mask that hides whole splits and whole rows.  Two
    calls in a row check that the tickets are back at zero after each."""
    torch = torch_gpu
    d, Hq, Hkv, T = 128, 28, 4, 256
    pasts = [3000, 1700]
    L = [p + T for p in pasts]
    print(f"in-launch merge splits={splits} masked={masked}", flush=True)
    kv = vva.KVCache(ctx, 1, Hkv, d, max(L), 2, vva.F16)
    fill_cache(kv, L, seed=40 + splits)
    for s, p in enumerate(pasts):
        kv.set_len(s, p)
    q = to_gpu(torch, np.random.default_rng(41).standard_normal((2, T, Hq, d)), vva.F16)
    mt = None
    if masked:
        Lm = max(L)
        m = np.where(np.arange(Lm)[None, :] > pasts[0] + np.arange(T)[:, None], -np.inf, 0.0).astype(np.float32)
        m[:, 200:2400] = -np.inf                      # whole splits with nothing visible
        m[7, :] = -np.inf                             # a row with no visible key -> 0
        mt = torch.from_numpy(vvo.f16_bits(m)[None].view(np.float16)).cuda()
    outs = []
    with ctx.schedule(prefill_splits=splits):
        for fn in (ctx.attn, ctx.attn, ctx.attn_noalloc):
            out = torch.full((2, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
            fn(kv, 0, q, out, d ** -0.5, mask=mt)
            torch.cuda.synchronize()
            assert ctx.last_decode_splits() == splits
            outs.append(as_f32(torch, out))
    assert np.isfinite(outs[0]).all()
    assert np.array_equal(outs[0], outs[1]), "second in-launch call differs"
    assert np.array_equal(outs[0], outs[2]), np.abs(outs[0] - outs[2]).max()
    if masked:
        assert not outs[0][:, 7].any()
    elif splits == 2:
        ref = oracle_attn(as_f32(torch, q), kv, 0, [0, 1], L, T, d ** -0.5)
        assert_close(outs[0], ref, *TOL, what=f"{splits} key splits, merged in the launch")
    kv.free()


def test_prefill_key_splits_explicit_mask(ctx, torch_gpu):
    torch = torch_gpu
    d, Hq, Hkv, T, past = 64, 14, 2, 40, 3000
    L = past + T
    kv = vva.KVCache(ctx, 1, Hkv, d, L, 1, vva.F16)
    fill_cache(kv, [L], seed=31)
    kv.set_len(0, past)
    m = np.where(np.arange(L)[None, :] > past + np.arange(T)[:, None], -np.inf, 0.0).astype(np.float32)
    m[:, 100:1900] = -np.inf                          # whole splits with nothing visible
    m[3, :] = -np.inf                                 # a row with no visible key -> 0
    m[5, :2990] = -np.inf                             # a row that sees only its last keys
    mbits = vvo.f16_bits(m)[None]
    q = to_gpu(torch, np.random.default_rng(32).standard_normal((1, T, Hq, d)), vva.F16)
    mt = torch.from_numpy(mbits.view(np.float16)).cuda()
    o, used = _prefill_with_splits(ctx, torch, kv, q, 12, mask=mt)
    assert used == 12
    ref = oracle_attn(as_f32(torch, q), kv, 0, [0], [L], T, d ** -0.5, mask=mbits)
    assert_close(o, ref, *TOL, what="masked, 12 key splits")
    assert not o[0, 3].any()
    kv.free()


def test_prefill_key_splits_score_jump(ctx, torch_gpu):
    """Logits jump by far more than 2^15 (exp2 domain) in the middle of a
    split: that split's workgroup restarts its key loop with a raised max."""
    torch = torch_gpu
    d, Hq, Hkv, T, past = 128, 28, 4, 64, 2000
    L = past + T
    rng = np.random.default_rng(41)
    k = rng.standard_normal((1, L, Hkv, d)) * 0.05
    k[:, 1200:] *= 160.0
    v = rng.standard_normal((1, L, Hkv, d))
    kv = vva.KVCache(ctx, 1, Hkv, d, L, 1, vva.F16)
    kv.upload(0, 0, 0, k[0].astype(np.float32), v[0].astype(np.float32))
    kv.set_len(0, past)
    q = to_gpu(torch, rng.standard_normal((1, T, Hq, d)), vva.F16)
    o, used = _prefill_with_splits(ctx, torch, kv, q, 6)
    assert used == 6
    assert np.isfinite(o).all()
    ref = oracle_attn(as_f32(torch, q), kv, 0, [0], [L], T, d ** -0.5)
    assert_close(o, ref, *TOL, what="score jump, 6 key splits")
    kv.free()


@pytest.mark.parametrize("t", [vva.BF16, vva.F32])
def test_prefill_v_at_the_f16_range_edge(ctx, torch_gpu, t):
    """P.V takes V as f16 for BF16 caches and, through the window's F16 cast
    (the reference's own cast before flash attention, src/qwen2.cpp:328-331),
    for F32 caches: V up to the f16 maximum 65504 must come through exactly.
    V * 2^14 with |V| < 4 reaches 65372; every product and sum then scales by
    the power of two, so the output must be exactly 2^14 times the unscaled
    one, and the unscaled one must match the oracle."""
    torch = torch_gpu
    d, Hq, Hkv, T = 128, 28, 4, 320
    rng = np.random.default_rng(31)
    k = rng.standard_normal((T, Hkv, d)).astype(np.float32)
    v = rng.standard_normal((T, Hkv, d))
    v = np.sign(v) * np.clip(np.abs(v), 2.0 ** -6, 3.99)          # no f16 subnormals at either scale
    v = v.astype(np.float32)
    q = to_gpu(torch, rng.standard_normal((1, T, Hq, d)), vva.F32)
    outs = []
    for scale in (1.0, 2.0 ** 14):
        kv = vva.KVCache(ctx, 1, Hkv, d, T, 1, t)
        kv.upload(0, 0, 0, k, (v * scale).astype(np.float32))
        kv.set_len(0, 0)
        out = torch.full((1, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
        ctx.attn(kv, 0, q, out, d ** -0.5)
        torch.cuda.synchronize()
        outs.append(as_f32(torch, out))
        if scale == 1.0:
            ref = oracle_attn(as_f32(torch, q), kv, 0, [0], [T], T, d ** -0.5)
            assert_close(outs[0], ref, *TOL, what="unscaled V")
        else:
            vmax = np.abs(vvo.to_f32(kv.download(0, 0, T)[1].reshape(-1), t, T * Hkv * d)).max()
            assert 6e4 < vmax <= 65504.0
        kv.free()
    assert np.isfinite(outs[1]).all()
    np.testing.assert_array_equal(outs[1], outs[0] * 2.0 ** 14)


@pytest.mark.parametrize("which", ["v", "k"])
def test_prefill_q8_0_window_beyond_the_f16_range(ctx, torch_gpu, which):
    """A Q8_0 prefill converts the window to f16 for the MFMA kernel; a block
    with |d q| > 65504 has no f16 value.  ggml dequantizes Q8_0 to fp32
    (src/qwen2.cpp:332-335), so the result must stay finite and match the
    oracle: the conversion flags the call and a gated fp32 kernel recomputes
    it from the Q8_0 cache.  "v": V * 2^16 (values to ~2.6e5; the output
    scales by exactly 2^16); "k": K * 2^16 with Q * 2^-16 (the scores keep
    their size), against the oracle on those inputs.  A 256-token chunk over
    a 300-token past at the 7B head shape."""
    torch = torch_gpu
    d, Hq, Hkv, T, past = 128, 28, 4, 256, 300
    L = past + T
    rng = np.random.default_rng(57)
    k = rng.standard_normal((L, Hkv, d)).astype(np.float32)
    v = rng.standard_normal((L, Hkv, d)).astype(np.float32)
    q = rng.standard_normal((1, T, Hq, d)).astype(np.float32)
    big = 2.0 ** 16
    if which == "v":
        v = v * big
    else:
        k, q = k * big, q / big
    kv = vva.KVCache(ctx, 1, Hkv, d, L, 1, vva.Q8_0)
    kv.upload(0, 0, 0, k, v)
    kv.set_len(0, past)
    qg = to_gpu(torch, q, vva.F32)
    out = torch.full((1, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    ctx.attn(kv, 0, qg, out, d ** -0.5)
    torch.cuda.synchronize()
    got = as_f32(torch, out)
    raw = kv.download(0, 0, L)[0 if which == "k" else 1].reshape(-1)
    vmax = np.abs(vvo.to_f32(raw, vva.Q8_0, L * Hkv * d)).max()
    assert vmax > 65504.0, vmax
    assert np.isfinite(got).all(), "non-finite output beyond the f16 range"
    ref = oracle_attn(as_f32(torch, qg), kv, 0, [0], [L], T, d ** -0.5)
    if which == "v":
        mx, mn = assert_close(got / big, ref / big, *TOL, what="V * 2^16, rescaled")
    else:
        mx, mn = assert_close(got, ref, *TOL, what="K * 2^16, Q * 2^-16")
    print(f"  {which} up to {vmax:.3g}: max {mx:.2e} mean {mn:.2e}")
    kv.free()
