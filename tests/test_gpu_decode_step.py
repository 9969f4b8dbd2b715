"""GPU parity of vva_decode_step: on F16 / BF16 caches decode_step.hip (RoPE +
append + split attention + in-kernel merge of the splits in one launch), on
Q8_0 caches the streamed decode kernel in step mode (RoPE + append +
attention, then its merge kernel).

Each step is checked three ways on the same inputs: the appended cache rows
must equal those of vva_rope_append bit for bit (same rotation, same
rounding); the output must match the unfused vva_rope_append + vva_attn pair
and the oracle (exact fp64 and ggml order with an F32 V sum) on the device's
own cache bytes, 2e-3 max-abs / 1e-3 mean-abs.  Consecutive steps reuse the
merge tickets, so a ticket left non-zero by a step would break the next one.
"""
import numpy as np
import pytest

import vva
import vvo
from gpu_util import as_f32, assert_close, fill_cache, oracle_attn, to_gpu

pytestmark = pytest.mark.gpu

TOL = (2e-3, 1e-3)

CASES = [
    # d, Hq, Hkv, cache type, lens before the step, input type
    (64, 14, 2, vva.F16, [1024, 1024], vva.F32),     # the 0.5B TTS CFG decode step
    (64, 14, 2, vva.F16, [1024, 300], vva.F32),      # ragged CFG streams
    (128, 12, 2, vva.BF16, [3999], vva.BF16),        # 1.5B heads
    (128, 28, 4, vva.F16, [90, 2000], vva.F16),      # one split for the first stream
    (128, 28, 4, vva.F16, [9000], vva.F32),          # past the fused kernel's window: the unfused path
    (64, 14, 2, vva.Q8_0, [700, 700], vva.F32),      # Q8_0 caches: the streamed kernel in step mode
    (128, 28, 4, vva.Q8_0, [3000, 2500], vva.F32),   # 7B heads (kv-head pairs), ragged CFG streams
    (128, 28, 4, vva.Q8_0, [32768, 32768], vva.F16), # the ASR transcript decode at full length
    (128, 12, 2, vva.Q8_0, [4100], vva.BF16),        # 1.5B heads, whole rows
    (64, 8, 1, vva.Q8_0, [500], vva.F32),            # one kv head
]


@pytest.mark.parametrize("d,Hq,Hkv,t,lens,it", CASES)
def test_decode_step_matches_unfused_and_oracle(ctx, torch_gpu, d, Hq, Hkv, t, lens, it):
    torch = torch_gpu
    B = len(lens)
    print(f"decode_step d={d} Hq={Hq} Hkv={Hkv} type={t} lens={lens}", flush=True)
    steps = 3
    a = vva.KVCache(ctx, 1, Hkv, d, max(lens) + steps + 1, B, t)
    u = vva.KVCache(ctx, 1, Hkv, d, max(lens) + steps + 1, B, t)
    fill_cache(a, lens, seed=sum(lens) + d)
    fill_cache(u, lens, seed=sum(lens) + d)
    rng = np.random.default_rng(d + t + B)
    for step in range(steps):
        L = [n + step for n in lens]
        q = to_gpu(torch, rng.standard_normal((B, 1, Hq, d)), it)
        k = to_gpu(torch, rng.standard_normal((B, 1, Hkv, d)), it)
        v = to_gpu(torch, rng.standard_normal((B, 1, Hkv, d)), it)
        pos = torch.tensor([[n] for n in L], dtype=torch.int32, device="cuda")
        qa = torch.empty((B, 1, Hq, d), dtype=torch.float32, device="cuda")
        qu = torch.empty_like(qa)
        oa = torch.full((B, 1, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
        ou = torch.full_like(oa, float("nan"))
        ctx.decode_step(a, 0, q, k, v, pos, qa, oa, d ** -0.5)
        splits = ctx.last_decode_splits()
        ctx.rope_append(u, 0, q, k, v, pos, qu)
        ctx.attn(u, 0, qu, ou, d ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(qa, qu), "rotated q differs"
        if t == vva.Q8_0:
            # the same streamed kernel on the same bytes: the new row patched
            # into its tile equals the row rope_append wrote
            assert torch.equal(oa, ou), "fused Q8_0 step differs from the unfused pair"
        for s in range(B):
            ka, va_ = a.download(0, s, L[s] + 1)
            ku, vu = u.download(0, s, L[s] + 1)
            np.testing.assert_array_equal(ka, ku)
            np.testing.assert_array_equal(va_, vu)
        got, unf = as_f32(torch, oa), as_f32(torch, ou)
        m1 = assert_close(got, unf, *TOL, what=f"step {step} vs unfused")
        Lk = [n + 1 for n in L]
        q32 = as_f32(torch, qa)
        ref = oracle_attn(q32, a, 0, range(B), Lk, 1, d ** -0.5)
        m2 = assert_close(got, ref, *TOL, what=f"step {step} vs exact")
        gg = oracle_attn(q32, a, 0, range(B), Lk, 1, d ** -0.5, mode=vvo.GGML_F32ACC)
        m3 = assert_close(got, gg, *TOL, what=f"step {step} vs ggml order")
        print(f"  step {step} splits {splits}: vs unfused max {m1[0]:.2e}; vs exact max {m2[0]:.2e} "
              f"mean {m2[1]:.2e}; vs ggml order max {m3[0]:.2e}")
        for s in range(B):
            a.set_len(s, L[s] + 1)
            u.set_len(s, L[s] + 1)
    a.free()
    u.free()


@pytest.mark.parametrize("lens,seq_ids", [([0, 17], None), ([0], None), ([5000, 33], [1, 0])])
def test_decode_step_q8_0_first_token_and_seq_ids(ctx, torch_gpu, lens, seq_ids):
    """Q8_0 step mode at its edges: an empty cache (the first token is the
    whole window), ragged streams, and sequences addressed through seq_ids
    in another order.  Bit for bit against the unfused pair."""
    torch = torch_gpu
    d, Hq, Hkv = 128, 28, 4
    B = len(lens)
    n_seq = max(B, 2)
    ids = seq_ids if seq_ids is not None else list(range(B))
    store = [0] * n_seq
    for b, s_ in enumerate(ids):
        store[s_] = lens[b]
    a = vva.KVCache(ctx, 1, Hkv, d, max(lens) + 4, n_seq, vva.Q8_0)
    u = vva.KVCache(ctx, 1, Hkv, d, max(lens) + 4, n_seq, vva.Q8_0)
    fill_cache(a, store, seed=77)
    fill_cache(u, store, seed=77)
    rng = np.random.default_rng(78)
    q = to_gpu(torch, rng.standard_normal((B, 1, Hq, d)), vva.F32)
    k = to_gpu(torch, rng.standard_normal((B, 1, Hkv, d)), vva.F32)
    v = to_gpu(torch, rng.standard_normal((B, 1, Hkv, d)), vva.F32)
    pos = torch.tensor([[n] for n in lens], dtype=torch.int32, device="cuda")
    qa = torch.empty((B, 1, Hq, d), dtype=torch.float32, device="cuda")
    qu = torch.empty_like(qa)
    oa = torch.full((B, 1, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    ou = torch.full_like(oa, float("nan"))
    ctx.decode_step(a, 0, q, k, v, pos, qa, oa, d ** -0.5, seq_ids=seq_ids)
    ctx.rope_append(u, 0, q, k, v, pos, qu, seq_ids=seq_ids)
    ctx.attn(u, 0, qu, ou, d ** -0.5, seq_ids=seq_ids)
    torch.cuda.synchronize()
    assert torch.equal(qa, qu)
    assert torch.equal(oa, ou)
    for b, s_ in enumerate(ids):
        ka, va_ = a.download(0, s_, lens[b] + 1)
        ku, vu = u.download(0, s_, lens[b] + 1)
        np.testing.assert_array_equal(ka, ku)
        np.testing.assert_array_equal(va_, vu)
    ref = oracle_attn(as_f32(torch, qa), a, 0, ids, [n + 1 for n in lens], 1, d ** -0.5)
    assert_close(as_f32(torch, oa), ref, *TOL, what="Q8_0 step edges")
    a.free()
    u.free()


def test_decode_step_graph_replays_match_eager(ctx, torch_gpu):
    """One captured step replayed three times, with eager work and
    synchronizations between the replays: every replay's output equals the
    eager call's (the in-kernel merge's tickets return to zero)."""
    torch = torch_gpu
    d, Hq, Hkv, B, L = 64, 14, 2, 2, 1024
    kv = vva.KVCache(ctx, 1, Hkv, d, L + 4, B, vva.F16)
    fill_cache(kv, [L, L], seed=5)
    rng = np.random.default_rng(6)
    q, k, v = (to_gpu(torch, rng.standard_normal((B, 1, h, d)), vva.F32) for h in (Hq, Hkv, Hkv))
    pos = torch.full((B, 1), L, dtype=torch.int32, device="cuda")
    qo = torch.empty((B, 1, Hq, d), dtype=torch.float32, device="cuda")
    out = torch.empty((B, 1, Hq, d), dtype=torch.float32, device="cuda")
    ctx.decode_step(kv, 0, q, k, v, pos, qo, out, d ** -0.5)      # sizes the workspace
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    default = torch.cuda.current_stream()
    try:
        with torch.cuda.graph(g):
            ctx.set_stream(torch.cuda.current_stream())
            ctx.decode_step(kv, 0, q, k, v, pos, qo, out, d ** -0.5)
    finally:
        ctx.set_stream(default)
    for _ in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        ctx.decode_step(kv, 0, q, k, v, pos, qo, out, d ** -0.5)   # eager call between replays
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    del g
    kv.free()


def test_decode_step_q8_v_beyond_the_f16_range(ctx, torch_gpu):
    """A 7B Q8_0 step whose V blocks reach d_v = 2^13 (|V| near 1e6, the
    new row's v as large): the streamed kernel raises the rows' exp2 base
    so its f16 P' stays finite.  Fused and unfused agree bit for bit and
    match the oracle within the tolerance scaled by the V scale."""
    torch = torch_gpu
    d, Hq, Hkv, lens, vs = 128, 28, 4, [3000, 2500], 2.0 ** 18
    B = len(lens)
    print(f"decode_step Q8_0 V scale 2^18 lens={lens}", flush=True)
    rng = np.random.default_rng(91)
    a = vva.KVCache(ctx, 1, Hkv, d, max(lens) + 4, B, vva.Q8_0)
    u = vva.KVCache(ctx, 1, Hkv, d, max(lens) + 4, B, vva.Q8_0)
    for s, n in enumerate(lens):
        kk = rng.standard_normal((n, Hkv, d)).astype(np.float32)
        vv = (np.clip(rng.standard_normal((n, Hkv, d)), -3.95, 3.95) * vs).astype(np.float32)
        for c in (a, u):
            c.upload(0, s, 0, kk, vv)
            c.set_len(s, n)
    q = to_gpu(torch, rng.standard_normal((B, 1, Hq, d)), vva.F32)
    k = to_gpu(torch, rng.standard_normal((B, 1, Hkv, d)), vva.F32)
    v = to_gpu(torch, rng.standard_normal((B, 1, Hkv, d)) * vs, vva.F32)
    pos = torch.tensor([[n] for n in lens], dtype=torch.int32, device="cuda")
    qa = torch.empty((B, 1, Hq, d), dtype=torch.float32, device="cuda")
    qu = torch.empty_like(qa)
    oa = torch.full((B, 1, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    ou = torch.full_like(oa, float("nan"))
    ctx.decode_step(a, 0, q, k, v, pos, qa, oa, d ** -0.5)
    ctx.rope_append(u, 0, q, k, v, pos, qu)
    ctx.attn(u, 0, qu, ou, d ** -0.5)
    torch.cuda.synchronize()
    got = as_f32(torch, oa)
    assert np.isfinite(got).all()
    assert torch.equal(oa, ou)
    ref = oracle_attn(as_f32(torch, qa), a, 0, range(B), [n + 1 for n in lens], 1, d ** -0.5)
    mx, mn = assert_close(got / vs, ref / vs, *TOL, what="Q8_0 step, V * 2^18, rescaled")
    print(f"  |out| up to {np.abs(got).max():.3g}; rescaled vs oracle max {mx:.2e} mean {mn:.2e}")
    a.free()
    u.free()
