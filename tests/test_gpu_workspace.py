"""The context's split workspace grows geometrically.

A chunked prefill over a Q8_0 cache converts a window that grows by one
chunk per call into the workspace (the reference's ASR prefill runs 512-token
chunks, src/vibevoice_asr.cpp:542-652).  Every outgrown workspace is kept
until vva_destroy (a graph captured earlier may still write into it), so the
workspace at least doubles at each growth: the device memory a context holds
after the whole prefill stays within twice the largest call's need, instead
of the sum over all chunks.
"""
import numpy as np
import pytest

import vva

pytestmark = pytest.mark.gpu


def test_chunked_q8_prefill_workspace_stays_bounded(torch_gpu):
    torch = torch_gpu
    d, Hq, Hkv, chunk, n_chunks = 128, 28, 4, 512, 32
    L = chunk * n_chunks
    print(f"workspace growth: {n_chunks} chunks of {chunk}, Q8_0 7B heads", flush=True)
    c = vva.Context(0)
    try:
        kv = vva.KVCache(c, 1, Hkv, d, L, 1, vva.Q8_0)
        rng = np.random.default_rng(3)
        q = torch.from_numpy(rng.standard_normal((1, chunk, Hq, d)).astype(np.float32)).cuda().half()
        k = torch.from_numpy(rng.standard_normal((1, chunk, Hkv, d)).astype(np.float32)).cuda()
        v = torch.from_numpy(rng.standard_normal((1, chunk, Hkv, d)).astype(np.float32)).cuda()
        qr = torch.empty_like(q)
        out = torch.empty((1, chunk, Hq, d), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        for i in range(n_chunks):
            kv.set_len(0, i * chunk)
            pos = torch.arange(i * chunk, (i + 1) * chunk, dtype=torch.int32, device="cuda")
            c.rope_append(kv, 0, q, k, v, pos, qr)
            c.attn(kv, 0, qr, out, d ** -0.5)
        torch.cuda.synchronize()
        held = free0 - torch.cuda.mem_get_info()[0]
        # the last call's f16 window alone: K and V of L keys, 4 heads of 128
        window = 2 * L * Hkv * d * 2
        print(f"  held {held / 2**20:.1f} MiB after the prefill; last window {window / 2**20:.1f} MiB")
        assert np.isfinite(out.cpu().numpy()).all()
        # live workspace < 2x the need (power of two), retired ones sum to
        # less than the live one; the partials of a 512-token chunk add at
        # most ~30 MB to the need
        assert held <= 4 * (window + (32 << 20)), f"held {held} bytes"
        kv.free()
    finally:
        c.close()
