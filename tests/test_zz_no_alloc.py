"""vva_attn_noalloc (split partials in the device's static scratch) against
vva_attn (partials in the context's workspace), through the C ABI.

Two calls in a row per path, the second with a smaller input, so the second
reads a scratch that still holds the first call's partials.  The same
kernels run with the same split counts, so the outputs must agree to the
path's tolerance (2e-3 max-abs / 1e-3 mean-abs for F16 / Q8_0 caches); the
test also reports whether they are bit-identical.  The prefill planner
keeps the no-alloc call's partials within the scratch (it may choose fewer
key splits); a forced split count whose partials exceed the scratch is
refused with VVA_ERR_INVALID_ARG before anything is enqueued.
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
    mx, mn = assert_close(b, a, *TOL, what="noalloc decode vs attn")
    print(f"  splits {sa}: max {mx:.2e} mean {mn:.2e}; bit-identical {np.array_equal(a, b)}")
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
