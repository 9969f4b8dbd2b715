"""HIP-graph capture of decode steps through the C ABI.

A decode step (per layer: fused RoPE + KV append, then single-token
attention) is captured with torch.cuda.graph on the context's stream and
replayed several times, with the program's own eager work (clearing the
outputs and the appended cache rows, reading them back) and synchronizations
between the replays.  Cache lengths are kernel arguments, so a replay
repeats the captured step at the same positions: every replay must write
the same cache rows and outputs as the eager step, bit for bit (same
kernels, same inputs).  Shapes: the TTS CFG decode of the 0.5B LM (B = 2,
14 q / 2 kv heads, d = 64, F16 caches at L = 1024: the register-streamed
decode and its merge) and the 7B ASR CFG decode on Q8_0 caches (the
LDS-streamed decode and its merge).
"""
import numpy as np
import pytest

import vva
from gpu_util import fill_cache, to_gpu

pytestmark = pytest.mark.gpu

CASES = [
    # d, Hq, Hkv, cache type, past length, layers
    (64, 14, 2, vva.F16, 1024, 3),
    (128, 28, 4, vva.Q8_0, 3000, 2),
]


@pytest.mark.parametrize("d,Hq,Hkv,kt,past,layers", CASES)
def test_decode_step_graph_replays(ctx, torch_gpu, d, Hq, Hkv, kt, past, layers):
    torch = torch_gpu
    print(f"graph decode d={d} Hq={Hq} Hkv={Hkv} type={kt} past={past} layers={layers}", flush=True)
    B = 2
    kv = vva.KVCache(ctx, layers, Hkv, d, past + 8, B, kt)
    fill_cache(kv, [past] * B, seed=past + d)
    rng = np.random.default_rng(7)
    q = to_gpu(torch, rng.standard_normal((B, 1, Hq, d)), vva.F32)
    k = to_gpu(torch, rng.standard_normal((B, 1, Hkv, d)), vva.F32)
    v = to_gpu(torch, rng.standard_normal((B, 1, Hkv, d)), vva.F32)
    pos = torch.full((1,), past, dtype=torch.int32, device="cuda")
    qr = [torch.empty_like(q) for _ in range(layers)]
    out = [torch.empty((B, 1, Hq, d), dtype=torch.float32, device="cuda") for _ in range(layers)]

    def step():
        for layer in range(layers):
            ctx.rope_append(kv, layer, q, k, v, pos, qr[layer])
            ctx.attn(kv, layer, qr[layer], out[layer], d ** -0.5)

    def new_rows():
        # the row each step appends, per (layer, seq); the lengths stay at past
        return [kv.download(layer, s, past + 1) for layer in range(layers) for s in range(B)]

    step()                                        # eager; also sizes the decode workspace
    torch.cuda.synchronize()
    ref_out = [o.cpu().numpy().copy() for o in out]
    ref_rows = new_rows()

    g = torch.cuda.CUDAGraph()
    default = torch.cuda.current_stream()
    try:
        with torch.cuda.graph(g):
            ctx.set_stream(torch.cuda.current_stream())
            step()
    finally:
        ctx.set_stream(default)

    blank = np.zeros((1, Hkv, d), np.float32)
    for r in range(3):
        for o in out:
            o.fill_(float("nan"))                 # eager work between replays
        for layer in range(layers):
            for s in range(B):
                kv.upload(layer, s, past, blank, blank)
        kv_len = [kv.get_len(s) for s in range(B)]
        assert kv_len == [past] * B
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for layer in range(layers):
            assert np.array_equal(out[layer].cpu().numpy(), ref_out[layer]), f"replay {r} layer {layer}"
        rows = new_rows()
        for a, b in zip(rows, ref_rows):
            assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]), f"replay {r}: appended rows"
        print(f"  replay {r}: outputs and appended rows equal the eager step", flush=True)
    del g
    kv.free()


def test_graph_replay_after_workspace_growth(torch_gpu):
    """A graph captured while the split workspace is small keeps working
    after a later eager call grows it: the outgrown workspace is retired,
    not freed, so the replays still write into live memory and reproduce
    the eager step bit for bit.  A fresh context, so the workspace starts
    at the small call's size."""
    torch = torch_gpu
    c = vva.Context(0)
    small = big = None
    try:
        d, Hq, Hkv, B, past = 64, 14, 2, 2, 1024
        small = vva.KVCache(c, 1, Hkv, d, past + 8, B, vva.F16)
        fill_cache(small, [past] * B, seed=77)
        rng = np.random.default_rng(78)
        q = to_gpu(torch, rng.standard_normal((B, 1, Hq, d)), vva.F32)
        out = torch.empty((B, 1, Hq, d), dtype=torch.float32, device="cuda")
        c.attn(small, 0, q, out, d ** -0.5)                # eager: sizes the workspace
        torch.cuda.synchronize()
        assert c.last_decode_splits() > 1
        ref = out.cpu().numpy().copy()

        g = torch.cuda.CUDAGraph()
        default = torch.cuda.current_stream()
        try:
            with torch.cuda.graph(g):
                c.set_stream(torch.cuda.current_stream())
                c.attn(small, 0, q, out, d ** -0.5)
        finally:
            c.set_stream(default)

        # a 7B-shaped Q8_0 decode over 4096 keys: many more split partials
        big = vva.KVCache(c, 1, 4, 128, 4104, B, vva.Q8_0)
        fill_cache(big, [4096] * B, seed=79)
        qb = to_gpu(torch, rng.standard_normal((B, 1, 28, 128)), vva.F32)
        ob = torch.empty((B, 1, 28, 128), dtype=torch.float32, device="cuda")
        c.attn(big, 0, qb, ob, 128 ** -0.5)
        torch.cuda.synchronize()
        assert c.last_decode_splits() > 9 and np.isfinite(ob.cpu().numpy()).all()

        for r in range(3):
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy(), ref), f"replay {r} after the workspace grew"
        print("  3 replays after the workspace grew equal the eager step", flush=True)
        del g
    finally:
        for kv in (small, big):
            if kv is not None:
                kv.free()
        c.close()


@pytest.mark.parametrize("kt", [vva.F16, vva.Q8_0])
def test_prefill_chunk_graph_replays(ctx, torch_gpu, kt):
    """An ASR chunk step (per layer: RoPE + append of 512 tokens, then the
    chunk's attention over a 2048-token past) captured and replayed three
    times with eager work between the replays.  The captured work holds the
    key-split prefill whose last split merges in the launch (its tickets
    must return to zero) and, on the Q8_0 cache, the window conversion to f16
    and the gated fp32 fallback (its gate closed: no value leaves the f16
    range).  Every replay's outputs equal the eager step's, bit for bit."""
    torch = torch_gpu
    d, Hq, Hkv, T, past, layers = 128, 28, 4, 512, 2048, 2
    print(f"graph chunk type={kt} T={T} past={past}", flush=True)
    kv = vva.KVCache(ctx, layers, Hkv, d, past + T, 1, kt)
    fill_cache(kv, [past], seed=4242 + kt)
    rng = np.random.default_rng(43)
    q = to_gpu(torch, rng.standard_normal((1, T, Hq, d)), vva.BF16)
    k = to_gpu(torch, rng.standard_normal((1, T, Hkv, d)), vva.BF16)
    v = to_gpu(torch, rng.standard_normal((1, T, Hkv, d)), vva.BF16)
    pos = torch.arange(past, past + T, dtype=torch.int32, device="cuda")
    qr = [torch.empty((1, T, Hq, d), dtype=torch.float16, device="cuda") for _ in range(layers)]
    out = [torch.empty((1, T, Hq, d), dtype=torch.float32, device="cuda") for _ in range(layers)]

    def step():
        for layer in range(layers):
            ctx.rope_append(kv, layer, q, k, v, pos, qr[layer])
            ctx.attn(kv, layer, qr[layer], out[layer], d ** -0.5)

    step()                                        # eager; sizes the workspace and settles the plan
    torch.cuda.synchronize()
    splits = ctx.last_decode_splits()
    ref_out = [o.cpu().numpy().copy() for o in out]
    g = torch.cuda.CUDAGraph()
    default = torch.cuda.current_stream()
    try:
        with torch.cuda.graph(g):
            ctx.set_stream(torch.cuda.current_stream())
            step()
    finally:
        ctx.set_stream(default)
    for r in range(3):
        for o in out:
            o.fill_(float("nan"))                 # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for layer in range(layers):
            assert np.array_equal(out[layer].cpu().numpy(), ref_out[layer]), f"replay {r} layer {layer}"
        print(f"  replay {r} ({splits} key splits): outputs equal the eager step", flush=True)
    del g
    kv.free()
