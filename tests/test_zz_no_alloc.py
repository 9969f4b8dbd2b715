"""vva_attn_noalloc (split partials in the device's static scratch) against
vva_attn (partials in the context's workspace), through the C ABI.

Two calls in a row per path, the second with a smaller input, so the second
reads a scratch that still holds the first call's partials.  The same
kernels run with the same split counts, so decode outputs must be
bit-identical; prefill outputs agree to the path's tolerance (2e-3 max-abs
/ 1e-3 mean-abs for F16 / Q8_0 caches).  The prefill planner keeps the
no-alloc call's partials within the scratch (it may choose fewer key
splits); a forced split count whose partials exceed the scratch is refused
with VVA_ERR_INVALID_ARG before anything is enqueued.  Q8_0 caches, and F32
caches under flash-attention semantics, run the same window conversion and
MFMA prefill as vva_attn with the converted window in the scratch too; a
window too large for it is refused with VVA_ERR_NOT_IMPLEMENTED.  A call
captured in a HIP graph on a context that has never allocated a workspace
replays to the eager result, so the call allocates nothing.
"""
import numpy as np
import pytest

import vva
from gpu_util import as_f32, assert_close, fill_cache, to_gpu

pytestmark = pytest.mark.gpu

TOL = (2e-3, 1e-3)


def _both(ctx, torch, kv, q, scale):
    B, T, Hq, d = q.shape
    outs = []
    for fn in (ctx.attn, ctx.attn_noalloc):
        out = torch.full((B, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
        fn(kv, 0, q, out, scale)
        torch.cuda.synchronize()
        outs.append((as_f32(torch, out), ctx.last_decode_splits()))
    return outs


@pytest.mark.parametrize("lens", [[8193, 8193], [2049, 1500]])
def test_noalloc_decode_matches_attn(ctx, torch_gpu, lens):
    """7B-shaped CFG decode on a Q8_0 cache: split-K partials in the scratch."""
    torch = torch_gpu
    d, Hq, Hkv = 128, 28, 4
    print(f"noalloc decode lens={lens}", flush=True)
    kv = vva.KVCache(ctx, 1, Hkv, d, max(lens) + 8, 2, vva.Q8_0)
    fill_cache(kv, lens, seed=sum(lens))
    for s, n in enumerate(lens):
        kv.set_len(s, n - 1)
    rng = np.random.default_rng(lens[0])
    q = to_gpu(torch, rng.standard_normal((2, 1, Hq, d)), vva.F32)
    (a, sa), (b, sb) = _both(ctx, torch, kv, q, d ** -0.5)
    assert sa == sb and sa > 1, (sa, sb)
    assert np.array_equal(a, b), "noalloc decode: same kernels and splits, outputs must be bit-identical"
    print(f"  splits {sa}: bit-identical")
    kv.free()


@pytest.mark.parametrize("T,past", [(512, 3584), (128, 1000)])
def test_noalloc_prefill_key_splits_match_attn(ctx, torch_gpu, T, past):
    """A 512-token ASR chunk over a long past (key splits: partials in the
    scratch), then a smaller chunk."""
    torch = torch_gpu
    d, Hq, Hkv = 128, 28, 4
    L = past + T
    print(f"noalloc prefill T={T} past={past}", flush=True)
    kv = vva.KVCache(ctx, 1, Hkv, d, L, 1, vva.F16)
    fill_cache(kv, [L], seed=L)
    kv.set_len(0, past)
    rng = np.random.default_rng(T)
    q = to_gpu(torch, rng.standard_normal((1, T, Hq, d)), vva.F16)
    (a, sa), (b, sb) = _both(ctx, torch, kv, q, d ** -0.5)
    # the planner keeps the no-alloc call's partials within the scratch, so
    # its split count may be smaller: equal to the split-count tolerance
    assert sa > 1 and sb > 1, (sa, sb)
    mx, mn = assert_close(b, a, *TOL, what="noalloc prefill vs attn")
    print(f"  key splits {sa} / {sb}: max {mx:.2e} mean {mn:.2e}; bit-identical {np.array_equal(a, b)}")
    kv.free()


def test_noalloc_refuses_partials_beyond_the_scratch(ctx, torch_gpu):
    torch = torch_gpu
    d, Hq, Hkv, T = 128, 28, 4, 2048
    kv = vva.KVCache(ctx, 1, Hkv, d, T, 1, vva.F16)
    kv.set_len(0, 0)
    q = torch.zeros((1, T, Hq, d), dtype=torch.float16, device="cuda")
    out = torch.zeros((1, T, Hq, d), dtype=torch.float32, device="cuda")
    # 32 key splits x 2048 x 28 rows x 130 floats = 954 MB of partials
    with ctx.schedule(prefill_splits=32):
        with pytest.raises(vva.VvaError) as e:
            ctx.attn_noalloc(kv, 0, q, out, d ** -0.5)
    assert e.value.status == vva.ERR_INVALID_ARG
    assert "static scratch" in str(e.value)
    kv.free()


@pytest.mark.parametrize("kt,flash", [(vva.Q8_0, 1), (vva.F32, 1), (vva.F32, 0)])
def test_noalloc_converted_windows_match_attn(ctx, torch_gpu, kt, flash):
    """Prefill chunks over Q8_0 and F32 caches: the window converted to f16
    in the scratch (flash semantics) or the fp32 eager branch, two calls in
    a row, the second smaller."""
    torch = torch_gpu
    d, Hq, Hkv = 128, 28, 4
    print(f"noalloc converted window type={kt} flash={flash}", flush=True)
    ctx.set_flash_attn(flash)
    try:
        for T, past in [(256, 1792), (64, 300)]:
            L = past + T
            kv = vva.KVCache(ctx, 1, Hkv, d, L, 1, kt)
            fill_cache(kv, [L], seed=L + kt)
            kv.set_len(0, past)
            rng = np.random.default_rng(T + kt)
            q = to_gpu(torch, rng.standard_normal((1, T, Hq, d)), vva.F32 if kt == vva.F32 else vva.F16)
            (a, sa), (b, sb) = _both(ctx, torch, kv, q, d ** -0.5)
            tol = (1e-4, 1e-4) if (kt == vva.F32 and not flash) else TOL
            mx, mn = assert_close(b, a, *tol, what=f"noalloc {kt}/{flash} T={T} vs attn")
            print(f"  T={T} past={past} splits {sa}/{sb}: max {mx:.2e} mean {mn:.2e}")
            kv.free()
    finally:
        ctx.set_flash_attn(1)


def test_noalloc_refuses_windows_beyond_the_scratch(ctx, torch_gpu):
    """A 7B Q8_0 window of 40k keys converts to 80 MB of f16, more than the
    scratch: refused, nothing enqueued."""
    torch = torch_gpu
    d, Hq, Hkv, T, past = 128, 28, 4, 16, 40000
    kv = vva.KVCache(ctx, 1, Hkv, d, past + T, 1, vva.Q8_0)
    kv.set_len(0, past)
    q = torch.zeros((1, T, Hq, d), dtype=torch.float16, device="cuda")
    out = torch.zeros((1, T, Hq, d), dtype=torch.float32, device="cuda")
    with pytest.raises(vva.VvaError) as e:
        ctx.attn_noalloc(kv, 0, q, out, d ** -0.5)
    assert e.value.status == vva.ERR_NOT_IMPLEMENTED
    assert "static scratch" in str(e.value)
    kv.free()


@pytest.mark.parametrize("case", ["decode_q8", "prefill_f16"])
def test_noalloc_captured_on_a_fresh_context_replays(torch_gpu, case):
    """vva_attn_noalloc captured in a HIP graph on a new context (no
    workspace ever allocated: any growth would fail under capture), replayed
    three times with eager work in between, equals the eager call."""
    torch = torch_gpu
    d, Hq, Hkv = 128, 28, 4
    print(f"noalloc graph {case}", flush=True)
    c = vva.Context(0)
    try:
        if case == "decode_q8":
            lens, T, kt, qt = [4097, 4097], 1, vva.Q8_0, vva.F32
        else:
            lens, T, kt, qt = [1536], 512, vva.F16, vva.F16
        B = len(lens)
        kv = vva.KVCache(c, 1, Hkv, d, max(lens) + 8, B, kt)
        fill_cache(kv, lens, seed=T + 11)
        for s, n in enumerate(lens):
            kv.set_len(s, n - T)
        rng = np.random.default_rng(5)
        q = to_gpu(torch, rng.standard_normal((B, T, Hq, d)), qt)
        out = torch.empty((B, T, Hq, d), dtype=torch.float32, device="cuda")
        g = torch.cuda.CUDAGraph()
        default = torch.cuda.current_stream()
        try:
            with torch.cuda.graph(g):
                c.set_stream(torch.cuda.current_stream())
                c.attn_noalloc(kv, 0, q, out, d ** -0.5)
        finally:
            c.set_stream(default)
        ref = torch.empty_like(out)
        c.attn_noalloc(kv, 0, q, ref, d ** -0.5)
        torch.cuda.synchronize()
        ref_np = ref.cpu().numpy()
        for r in range(3):
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy(), ref_np), f"replay {r} differs from the eager call"
        kv.free()
    finally:
        c.close()
