"""GPU parity of attention through the C ABI against the oracle.

The oracle runs on the exact bytes the GPU holds (cache rows downloaded
from the device) with Q rounded to K's dot type as ggml's CPU flash
attention does.  Tolerances (stated per test): 1e-4 max-abs for the F32
path, 2e-3 max-abs / 1e-3 mean-abs for F16 / BF16 / Q8_0 caches.  Each case
also reports the distance to the ggml-order oracle mode (per-key online
softmax, F16 running sum for F16 V).
"""

import numpy as np
import pytest

import vva
import vvo
from gpu_util import as_f32, assert_close, check_ggml_order, err_stats, fill_cache, oracle_attn, to_gpu

pytestmark = pytest.mark.gpu

TOL = {vva.F32: (1e-4, 1e-4), vva.F16: (2e-3, 1e-3), vva.BF16: (2e-3, 1e-3), vva.Q8_0: (2e-3, 1e-3)}


def run_attn(ctx, torch, kv, layer, T, B, Hq, q_type, seed, seqs=None, mask=None):
    rng = np.random.default_rng(seed)
    d = kv.head_dim
    q = to_gpu(torch, rng.standard_normal((B, T, Hq, d)), q_type)
    out = torch.full((B, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    mask_t = None
    if mask is not None:
        mask_t = torch.from_numpy(mask.view(np.float16)).to("cuda")
    ctx.attn(kv, layer, q, out, d ** -0.5, seq_ids=seqs, mask=mask_t)
    torch.cuda.synchronize()
    return as_f32(torch, q), as_f32(torch, out)


DECODE = [
    # d, Hq, Hkv, type, lens (per seq, incl. the new token), q_type
    (64, 14, 2, vva.F16, [1025, 1025], vva.F32),          # TTS CFG decode, 0.5B
    (64, 14, 2, vva.F16, [1224, 990], vva.F32),           # ragged CFG streams
    (128, 28, 4, vva.Q8_0, [4097, 3000], vva.F32),        # 7B Q8_0 decode
    (128, 28, 4, vva.Q8_0, [1], vva.F32),                 # first token
    (128, 12, 2, vva.BF16, [2049], vva.BF16),             # 1.5B
    (128, 28, 4, vva.F16, [17, 300], vva.F16),
    (64, 14, 2, vva.Q8_0, [777], vva.F32),
    (128, 28, 4, vva.F32, [513], vva.F32),                # F32 cache: VALU path
]


@pytest.mark.parametrize("d,Hq,Hkv,t,lens,q_type", DECODE)
def test_decode_matches_oracle(ctx, torch_gpu, d, Hq, Hkv, t, lens, q_type):
    torch = torch_gpu
    B = len(lens)
    print(f"decode d={d} Hq={Hq} Hkv={Hkv} type={t} lens={lens}", flush=True)
    kv = vva.KVCache(ctx, 1, Hkv, d, max(lens) + 4, B, t)
    fill_cache(kv, lens, seed=d + t + sum(lens))
    for s, n in enumerate(lens):
        kv.set_len(s, n - 1)                               # the last row is "the new token"
    q, out = run_attn(ctx, torch, kv, 0, 1, B, Hq, q_type, seed=7)
    ref = oracle_attn(q, kv, 0, range(B), lens, 1, d ** -0.5)
    mx, mn = assert_close(out, ref, *TOL[t], what="decode vs exact")
    (gmx, gmn), (hmx, hmn) = check_ggml_order(out, q, kv, 0, range(B), lens, 1, d ** -0.5, *TOL[t], what="decode")
    print(f"  vs exact max {mx:.2e} mean {mn:.2e}; vs ggml order max {gmx:.2e} mean {gmn:.2e} "
          f"(F16 V sum: max {hmx:.2e} mean {hmn:.2e}); splits {ctx.last_decode_splits()}")
    kv.free()


def test_decode_split_count_does_not_change_result(ctx, torch_gpu):
    torch = torch_gpu
    lens = [5000, 4321]
    kv = vva.KVCache(ctx, 1, 4, 128, 5008, 2, vva.Q8_0)
    fill_cache(kv, lens, seed=3)
    for s, n in enumerate(lens):
        kv.set_len(s, n - 1)
    outs = []
    for wgs in (2, 16, 100, 512):
        with ctx.schedule(decode_wgs=wgs):
            _, out = run_attn(ctx, torch, kv, 0, 1, 2, 28, vva.F32, seed=9)
        outs.append((ctx.last_decode_splits(), out))
    assert len({s for s, _ in outs}) == 4, [s for s, _ in outs]
    # each split has its own running max, so the f16 p * v products (2^-12
    # relative rounding per term) round differently: a few 1e-5 at most
    for s, o in outs[1:]:
        assert np.abs(o - outs[0][1]).max() < 2e-4, s
    kv.free()


def test_decode_explicit_mask(ctx, torch_gpu):
    torch = torch_gpu
    L = 700
    kv = vva.KVCache(ctx, 1, 2, 64, L, 1, vva.F16)
    fill_cache(kv, [L], seed=4)
    kv.set_len(0, L - 1)
    m = np.zeros((1, 1, L), np.float32)
    m[0, 0, 100:300] = -np.inf                             # a hole in the window
    mbits = vvo.f16_bits(m)
    q, out = run_attn(ctx, torch, kv, 0, 1, 1, 14, vva.F32, seed=5, mask=mbits)
    ref = oracle_attn(q, kv, 0, [0], [L], 1, 64 ** -0.5, mask=mbits)
    assert_close(out, ref, *TOL[vva.F16], what="masked decode")
    kv.free()


ROWS = [
    # d, Hq, Hkv, type, T, past  — VALU row kernel cases
    (64, 14, 2, vva.F32, 256, 0),        # 0.5B prefill (fp32 eager-equivalent)
    (128, 28, 4, vva.Q8_0, 64, 500),     # chunk into a Q8_0 cache (forced onto the row kernel)
    (128, 12, 2, vva.F32, 33, 7),
    (64, 14, 2, vva.F32, 100, 900),      # 0.5B TTS window past 1k: 16 key steps, the last partial
]


@pytest.mark.parametrize("d,Hq,Hkv,t,T,past", ROWS)
def test_row_kernel_prefill_matches_oracle(ctx, torch_gpu, d, Hq, Hkv, t, T, past):
    """F32 caches under the eager branch (vva_set_flash_attn(0): fp32
    throughout, 1e-4) and a Q8_0 chunk forced onto the row kernel."""
    torch = torch_gpu
    print(f"rows d={d} Hq={Hq} Hkv={Hkv} type={t} T={T} past={past}", flush=True)
    L = past + T
    kv = vva.KVCache(ctx, 1, Hkv, d, L, 1, t)
    fill_cache(kv, [L], seed=11, scale=1.0 if t != vva.F32 else 0.125)
    kv.set_len(0, past)
    ctx.set_flash_attn(False)
    if t == vva.Q8_0:
        ctx.set_attn_path(1)
    try:
        q, out = run_attn(ctx, torch, kv, 0, T, 1, Hq, vva.F32, seed=12)
    finally:
        ctx.set_flash_attn(True)
        ctx.set_attn_path(0)
    ref = oracle_attn(q, kv, 0, [0], [L], T, d ** -0.5)
    assert_close(out, ref, *TOL[t], what="row kernel")
    kv.free()


def test_row_kernel_f32_explicit_mask_ragged(ctx, torch_gpu):
    """The fp32 eager branch on F32 caches (the lane-per-key row kernel) over
    windows of several 64-key steps: two ragged sequences, an explicit F16
    mask with a hole covering one whole 64-key step and scattered holes, and
    a row with every key masked (its output is 0).  Tolerance 1e-4 (fp32)."""
    torch = torch_gpu
    d, Hq, Hkv, T = 128, 12, 2, 9
    lens = [700, 300]
    kv = vva.KVCache(ctx, 1, Hkv, d, max(lens), 2, vva.F32)
    fill_cache(kv, lens, seed=41, scale=0.125)
    for s_, L in enumerate(lens):
        kv.set_len(s_, L - T)
    rng = np.random.default_rng(42)
    m = np.where(rng.random((2, T, max(lens))) < 0.2, -np.inf, 0.0).astype(np.float32)
    m[0, :, 64:128] = -np.inf                               # one whole 64-key step
    m[1, 3, :] = -np.inf                                    # a row with nothing visible
    m[:, :, 5] = 0.0                                        # every other row sees key 5
    m[1, 3, 5] = -np.inf
    mbits = vvo.f16_bits(m)
    ctx.set_flash_attn(False)
    try:
        q, out = run_attn(ctx, torch, kv, 0, T, 2, Hq, vva.F32, seed=43, mask=mbits)
    finally:
        ctx.set_flash_attn(True)
    ref = oracle_attn(q, kv, 0, [0, 1], lens, T, d ** -0.5, mask=mbits)
    assert np.all(out[1, 3] == 0.0)
    mx, mn = assert_close(out, ref, *TOL[vva.F32], what="f32 rows, explicit mask")
    print(f"  f32 rows with mask: max {mx:.2e} mean {mn:.2e}")
    kv.free()


@pytest.mark.parametrize("t", [vva.Q8_0, vva.F32])
def test_converted_window_prefill_matches_oracle(ctx, torch_gpu, t):
    """A 512-token ASR chunk over a 32k past, 7B heads, on Q8_0 and F32
    caches: the window is converted to f16 on the device and prefilled on
    the MFMA kernel.  Q8_0: Q goes through a Q8_0 round trip (ggml's dot type
    for Q8_0 K), checked against both oracle orders on the cache bytes.  F32
    under the flash branch: the reference casts K/V to F16 first
    (src/qwen2.cpp:328-331), so the oracle sees the f16-rounded window.
    Rows: the chunk's first and last 16 and 32 spread between."""
    torch = torch_gpu
    d, Hq, Hkv, T, past = 128, 28, 4, 512, 32256
    L = past + T
    print(f"converted window type={t} T={T} past={past}", flush=True)
    kv = vva.KVCache(ctx, 1, Hkv, d, L, 1, t)
    fill_cache(kv, [L], seed=1717)
    kv.set_len(0, past)
    q, out = run_attn(ctx, torch, kv, 0, T, 1, Hq, vva.BF16, seed=1718)
    splits = ctx.last_decode_splits()
    rows = np.unique(np.concatenate([np.arange(16), np.arange(T - 16, T),
                                     np.linspace(16, T - 17, 32).astype(np.int64)])).astype(np.int32)
    if t == vva.Q8_0:
        ref = oracle_attn(q, kv, 0, [0], [L], T, d ** -0.5, rows=rows)
        mx, mn = assert_close(out[0, rows], ref[0, rows], *TOL[t], what="Q8_0 window vs exact")
        (gmx, gmn), _ = check_ggml_order(out, q, kv, 0, [0], [L], T, d ** -0.5, *TOL[t], rows=rows,
                                         what="Q8_0 window")
    else:
        kraw, vraw = kv.download(0, 0, L)
        k16 = vvo.from_f32(vvo.to_f32(kraw.reshape(-1), vvo.F32, L * Hkv * d), vvo.F16)
        v16 = vvo.from_f32(vvo.to_f32(vraw.reshape(-1), vvo.F32, L * Hkv * d), vvo.F16)
        args = dict(n_kv_heads=Hkv, scale=d ** -0.5, past=[past], rows=rows)
        ref = vvo.attn(q, [k16], [v16], vvo.F16, vvo.F16, [L], **args)
        mx, mn = assert_close(out[0, rows], ref[0, rows], *TOL[vva.F16], what="F32 window (F16 cast) vs exact")
        gg = vvo.attn(q, [k16], [v16], vvo.F16, vvo.F16, [L], mode=vvo.GGML_F32ACC, **args)
        gmx, gmn = assert_close(out[0, rows], gg[0, rows], *TOL[vva.F16], what="F32 window vs ggml order")
    print(f"  key splits {splits}: vs exact max {mx:.2e} mean {mn:.2e}; vs ggml order max {gmx:.2e} mean {gmn:.2e}")
    kv.free()


def test_forced_row_path_matches_decode(ctx, torch_gpu):
    torch = torch_gpu
    lens = [2000]
    kv = vva.KVCache(ctx, 1, 4, 128, 2000, 1, vva.F16)
    fill_cache(kv, lens, seed=21)
    kv.set_len(0, 1999)
    _, a = run_attn(ctx, torch, kv, 0, 1, 1, 28, vva.F32, seed=22)
    ctx.set_attn_path(1)
    try:
        _, b = run_attn(ctx, torch, kv, 0, 1, 1, 28, vva.F32, seed=22)
    finally:
        ctx.set_attn_path(0)
    # fp32 row kernel vs the split-K kernel's f16 p * v products
    assert np.abs(a - b).max() < 2e-4
    kv.free()


def test_flash_attn_ext_strided_head_major_kv(ctx, torch_gpu):
    """ggml_flash_attn_ext on tensors laid out [B][Hkv][L][d] (not the cache layout), no mask."""
    torch = torch_gpu
    rng = np.random.default_rng(31)
    B, Hq, Hkv, L, T, d = 2, 12, 2, 300, 1, 128
    q = to_gpu(torch, rng.standard_normal((B, Hq, T, d)), vva.F32)
    k = to_gpu(torch, rng.standard_normal((B, Hkv, L, d)), vva.F16)
    v = to_gpu(torch, rng.standard_normal((B, Hkv, L, d)), vva.F16)
    out = torch.empty((B, T, Hq, d), dtype=torch.float32, device="cuda")
    ctx.flash_attn_ext(q, k, v, out, d ** -0.5)
    torch.cuda.synchronize()
    q32 = as_f32(torch, q).transpose(0, 2, 1, 3)                  # [B, T, Hq, d]
    kc = [vvo.from_f32(as_f32(torch, k)[b].transpose(1, 0, 2), vvo.F16) for b in range(B)]
    vc = [vvo.from_f32(as_f32(torch, v)[b].transpose(1, 0, 2), vvo.F16) for b in range(B)]
    ref = vvo.attn(q32, kc, vc, 1, 1, [L] * B, n_kv_heads=Hkv, scale=d ** -0.5, mask_mode=vvo.MASK_NONE)
    assert_close(as_f32(torch, out), ref, *TOL[vva.F16], what="flash_attn_ext strided")


@pytest.mark.parametrize("t", [vva.Q8_0, vva.F32])
def test_flash_attn_ext_converted_strided_window(ctx, torch_gpu, t):
    """A multi-token call on K/V laid out [B][Hkv][L][d] (head-major, not the
    cache layout) of a type the MFMA prefill reads through the f16 window:
    Q8_0 rows in 34-byte blocks, and F32 rows starting 4 bytes past a 16-byte
    boundary (the conversion's 4-byte load path).  No mask (every key)."""
    torch = torch_gpu
    rng = np.random.default_rng(41)
    B, Hq, Hkv, L, T, d = 2, 28, 4, 700, 64, 128
    print(f"converted strided window type={t} B={B} L={L} T={T}", flush=True)
    q = to_gpu(torch, rng.standard_normal((B, Hq, T, d)), vva.F32)
    kf = rng.standard_normal((B, Hkv, L, d)).astype(np.float32)
    vf = rng.standard_normal((B, Hkv, L, d)).astype(np.float32)
    if t == vva.Q8_0:
        rb = d // 32 * vva.Q8_BLOCK_BYTES
        kb = vvo.from_f32(kf.reshape(-1), vvo.Q8_0).reshape(B, Hkv, L, rb)
        vb = vvo.from_f32(vf.reshape(-1), vvo.Q8_0).reshape(B, Hkv, L, rb)
        kg, vg = torch.from_numpy(kb).cuda(), torch.from_numpy(vb).cuda()
        ne, nb = [d, L, Hkv, B], [vva.Q8_BLOCK_BYTES, rb, L * rb, Hkv * L * rb]
        kt, vt = vva.view(kg, ne, nb, vva.Q8_0), vva.view(vg, ne, nb, vva.Q8_0)
        kc = [np.ascontiguousarray(kb[b].transpose(1, 0, 2)).reshape(-1) for b in range(B)]
        vc = [np.ascontiguousarray(vb[b].transpose(1, 0, 2)).reshape(-1) for b in range(B)]
        ct = vvo.Q8_0
    else:
        n = B * Hkv * L * d
        kflat = torch.from_numpy(np.concatenate([[0.0], kf.reshape(-1)]).astype(np.float32)).cuda()
        vflat = torch.from_numpy(np.concatenate([[0.0], vf.reshape(-1)]).astype(np.float32)).cuda()
        kg, vg = kflat[1:1 + n].view(B, Hkv, L, d), vflat[1:1 + n].view(B, Hkv, L, d)
        assert kg.data_ptr() % 16 == 4
        kt, vt = vva.view(kg), vva.view(vg)
        # the flash branch casts the window to F16, as the reference does
        kc = [vvo.from_f32(kf[b].transpose(1, 0, 2).reshape(-1), vvo.F16) for b in range(B)]
        vc = [vvo.from_f32(vf[b].transpose(1, 0, 2).reshape(-1), vvo.F16) for b in range(B)]
        ct = vvo.F16
    out = torch.full((B, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    ctx.flash_attn_ext(q, None, None, out, d ** -0.5, k_view=kt, v_view=vt)
    torch.cuda.synchronize()
    q32 = as_f32(torch, q).transpose(0, 2, 1, 3)                  # [B, T, Hq, d]
    ref = vvo.attn(q32, kc, vc, ct, ct, [L] * B, n_kv_heads=Hkv, scale=d ** -0.5, mask_mode=vvo.MASK_NONE)
    mx, mn = assert_close(as_f32(torch, out), ref, *TOL[vva.Q8_0 if t == vva.Q8_0 else vva.F16],
                          what="converted strided window")
    print(f"  max {mx:.2e} mean {mn:.2e}")


def test_unsupported_options_are_rejected(ctx, torch_gpu):
    torch = torch_gpu
    q = torch.zeros((1, 4, 1, 64), device="cuda")
    k = torch.zeros((1, 2, 8, 64), device="cuda", dtype=torch.float16)
    out = torch.zeros((1, 1, 4, 64), device="cuda")
    with pytest.raises(vva.VvaError) as e:
        st = ctx.lib.vva_flash_attn_ext(ctx.h, vva.ctypes.byref(vva.view(q)), vva.ctypes.byref(vva.view(k)),
                                        vva.ctypes.byref(vva.view(k)), None, 0.125, 1.0, 0.0,
                                        vva.ctypes.byref(vva.view(out)))
        ctx.check(st)
    assert e.value.status == vva.ERR_NOT_IMPLEMENTED


def test_empty_calls_are_rejected(ctx, torch_gpu):
    """Zero new tokens (ne[2] = 0; torch gives such tensors no storage) are
    argument errors, not silent no-ops, and leave the cache length alone."""
    torch = torch_gpu
    d, Hq, Hkv = 64, 14, 2
    kv = vva.KVCache(ctx, 1, Hkv, d, 16, 1, vva.F16)
    q = torch.zeros((1, 0, Hq, d), dtype=torch.float32, device="cuda")
    k = torch.zeros((1, 0, Hkv, d), dtype=torch.float32, device="cuda")
    out = torch.zeros((1, 0, Hq, d), dtype=torch.float32, device="cuda")
    pos = torch.zeros((0,), dtype=torch.int32, device="cuda")
    for call in (lambda: ctx.rope_append(kv, 0, q, k, k, pos, q), lambda: ctx.attn(kv, 0, q, out, d ** -0.5)):
        with pytest.raises(vva.VvaError) as err:
            call()
        assert err.value.status == vva.ERR_INVALID_ARG, err.value
    assert kv.get_len(0) == 0
    kv.free()


MASK_PATHS = [
    # d, Hq, Hkv, cache type, T, past, flash branch, q type — the kernel each reaches
    (128, 12, 2, vva.F32, 9, 600, False, vva.F32),     # fp32 eager rows (the reference's F32-mask branch)
    (128, 28, 4, vva.Q8_0, 1, 3000, True, vva.F32),    # streamed Q8_0 decode
    (64, 14, 2, vva.F16, 1, 1500, True, vva.F32),      # register-streamed decode
    (128, 28, 4, vva.F16, 64, 900, True, vva.F16),     # MFMA prefill
]


@pytest.mark.parametrize("d,Hq,Hkv,t,T,past,flash,qt", MASK_PATHS)
def test_f32_mask_equals_f16_mask(ctx, torch_gpu, d, Hq, Hkv, t, T, past, flash, qt):
    """An F32 mask (ggml_soft_max_ext's type, src/qwen2.hpp:34-37) holding
    the values of an F16 mask (0, -inf holes, a fully masked row and finite
    biases that f16 represents) gives the same output bit for bit on every
    kernel path; it also matches the oracle run with the F16 mask."""
    torch = torch_gpu
    print(f"f32 mask d={d} type={t} T={T} past={past} flash={flash}", flush=True)
    L = past + T
    kv = vva.KVCache(ctx, 1, Hkv, d, L, 1, t)
    fill_cache(kv, [L], seed=L + d)
    kv.set_len(0, past)
    rng = np.random.default_rng(L)
    m = np.where(rng.random((1, T, L)) < 0.15, -np.inf, 0.0).astype(np.float32)
    m += np.where(np.isfinite(m), np.round(rng.uniform(-2.0, 0.0, m.shape) * 64) / 64, 0.0).astype(np.float32)
    if T > 1:
        m[0, T - 1, :] = -np.inf                              # a row with nothing visible: output 0
    mbits = vvo.f16_bits(m)
    assert np.array_equal(mbits.view(np.float16).astype(np.float32), m)
    q = to_gpu(torch, rng.standard_normal((1, T, Hq, d)), qt)
    outs = []
    ctx.set_flash_attn(flash)
    try:
        for mt in (torch.from_numpy(mbits.view(np.float16)).cuda(), torch.from_numpy(m).cuda()):
            out = torch.full((1, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
            ctx.attn(kv, 0, q, out, d ** -0.5, mask=mt)
            torch.cuda.synchronize()
            outs.append(as_f32(torch, out))
    finally:
        ctx.set_flash_attn(True)
    assert np.array_equal(outs[0], outs[1]), "F32 mask result differs from the F16 mask's"
    ref = oracle_attn(as_f32(torch, q), kv, 0, [0], [L], T, d ** -0.5, mask=mbits)
    mx, mn = assert_close(outs[1], ref, *TOL[t], what="F32 mask vs oracle")
    print(f"  bit-equal to the F16 mask; vs oracle max {mx:.2e} mean {mn:.2e}")
    kv.free()


def test_f32_mask_beyond_f16_precision_eager_branch(ctx, torch_gpu):
    """The eager branch reads F32 mask entries at full precision: biases
    that f16 cannot hold (random fp32 in [-12, 0]) match an fp64 brute force
    softmax(scale q k^T + mask) v on the downloaded F32 cache, 1e-4."""
    torch = torch_gpu
    d, Hq, Hkv, T, past = 64, 14, 2, 5, 200
    L = past + T
    kv = vva.KVCache(ctx, 1, Hkv, d, L, 1, vva.F32)
    fill_cache(kv, [L], seed=9, scale=2.0)
    kv.set_len(0, past)
    rng = np.random.default_rng(10)
    m = rng.uniform(-12.0, 0.0, (1, T, L)).astype(np.float32)
    m[0, :, 17] = -np.inf
    q = to_gpu(torch, rng.standard_normal((1, T, Hq, d)), vva.F32)
    out = torch.full((1, T, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    ctx.set_flash_attn(False)
    try:
        ctx.attn(kv, 0, q, out, d ** -0.5, mask=torch.from_numpy(m).cuda())
        torch.cuda.synchronize()
    finally:
        ctx.set_flash_attn(True)
    k, v = kv.download(0, 0, L)                              # raw bytes of the F32 rows
    k = np.ascontiguousarray(k).view(np.float32).reshape(L, Hkv, d).astype(np.float64)
    v = np.ascontiguousarray(v).view(np.float32).reshape(L, Hkv, d).astype(np.float64)
    q64 = as_f32(torch, q).reshape(T, Hq, d).astype(np.float64)
    ref = np.zeros((T, Hq, d))
    g = Hq // Hkv
    for h in range(Hq):
        s = q64[:, h, :] @ k[:, h // g, :].T * d ** -0.5 + m[0].astype(np.float64)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        ref[:, h, :] = (p / p.sum(axis=1, keepdims=True)) @ v[:, h // g, :]
    got = as_f32(torch, out).reshape(T, Hq, d)
    mx, mn = assert_close(got, ref, 1e-4, 1e-4, what="eager branch, fp32 mask")
    # the f16-rounded mask moves the result by more than the tolerance: the
    # test would catch a kernel that rounds F32 mask entries to f16
    m16 = vvo.f16_bits(m).view(np.float16).astype(np.float64)
    ref16 = np.zeros_like(ref)
    for h in range(Hq):
        s = q64[:, h, :] @ k[:, h // g, :].T * d ** -0.5 + m16[0]
        p = np.exp(s - s.max(axis=1, keepdims=True))
        ref16[:, h, :] = (p / p.sum(axis=1, keepdims=True)) @ v[:, h // g, :]
    print(f"  vs fp64 max {mx:.2e}; the f16-rounded mask would be {np.abs(ref16 - ref).max():.2e} away")
    assert np.abs(ref16 - ref).max() > 1e-4
    kv.free()
