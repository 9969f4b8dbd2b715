"""GPU parity of the LDS-streamed Q8_0 decode kernel (decode_stream.hip).

Single-token attention over Q8_0 caches, through the C ABI, against the
oracle on the exact cache bytes the GPU holds (downloaded).  Tolerance: the
task's 2e-3 max-abs / 1e-3 mean-abs for Q8_0 caches, against both the exact
fp64 oracle and the ggml-order oracle (Q quantized to Q8_0, integer block
dots).  The cases cover every kv-head count the kernel takes (1, 2, 4, 8),
both head dims, splits whose first row is not 16-byte aligned in memory,
splits past a short sequence's end, explicit masks, each Q type, and the
register-streamed kernel (decode.hip) on the same bytes.
"""
import numpy as np
import pytest

import vva
import vvo
from gpu_util import as_f32, assert_close, err_stats, fill_cache, oracle_attn, to_gpu

pytestmark = pytest.mark.gpu

MAX_TOL, MEAN_TOL = 2e-3, 1e-3


def _decode(ctx, torch, kv, Hq, q_type, seed, mask=None, wgs=None, splits=None, q_scale=1.0):
    B = kv.n_seq
    rng = np.random.default_rng(seed)
    d = kv.head_dim
    q = to_gpu(torch, rng.standard_normal((B, 1, Hq, d)) * q_scale, q_type)
    out = torch.full((B, 1, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    mask_t = None if mask is None else torch.from_numpy(mask.view(np.float16)).to("cuda")
    with ctx.schedule(decode_wgs=wgs or 0, decode_splits=splits or 0):
        ctx.attn(kv, 0, q, out, d ** -0.5, mask=mask_t)
        torch.cuda.synchronize()
    return as_f32(torch, q), as_f32(torch, out), ctx.last_decode_splits()


def _cache(ctx, d, Hkv, lens, seed):
    kv = vva.KVCache(ctx, 1, Hkv, d, max(lens) + 8, len(lens), vva.Q8_0)
    fill_cache(kv, lens, seed=seed)
    for s, n in enumerate(lens):
        kv.set_len(s, n - 1)                   # the last row is "the new token"
    return kv


CASES = [
    # d, Hq, Hkv, lens (incl. the new token), q_type, workgroups (None = one per CU)
    (128, 28, 4, [8193, 8193], vva.F32, None),     # 7B CFG decode shape, shorter window
    (128, 28, 4, [33], vva.F32, None),             # one tile and one key
    (128, 28, 4, [4097, 40], vva.F16, None),       # second stream ends in its first split
    (128, 12, 2, [3001], vva.BF16, None),          # 1.5B heads: 64-key tiles
    (128, 8, 1, [2500, 1999], vva.F32, 37),        # one kv head: 136-byte rows, unaligned splits
    (128, 16, 8, [1777], vva.F32, None),           # eight kv heads: one wave each
    (64, 14, 2, [3333, 1025], vva.F32, 21),        # 0.5B heads: 136-byte rows, unaligned splits
    (64, 8, 4, [999], vva.F16, None),
    (64, 8, 1, [2222, 901], vva.F32, None),        # 0.5B-like d, one kv head: two key groups per wave
    (64, 16, 8, [1500], vva.BF16, 9),              # d = 64, eight kv heads
    (128, 28, 4, [700, 700], vva.F32, 1),          # one split: output written directly
    (128, 28, 4, [32769, 32769], vva.F32, None),   # the 7B CFG decode at full size: 32768 past + 1
    (128, 28, 4, [131073, 98305], vva.F32, None),  # the longest window the benchmark sweeps (128k past)
]


@pytest.mark.parametrize("d,Hq,Hkv,lens,q_type,wgs", CASES)
def test_stream_decode_matches_oracle(ctx, torch_gpu, d, Hq, Hkv, lens, q_type, wgs):
    torch = torch_gpu
    print(f"stream decode d={d} Hq={Hq} Hkv={Hkv} lens={lens} q={q_type} wgs={wgs}", flush=True)
    kv = _cache(ctx, d, Hkv, lens, seed=d + Hkv + sum(lens))
    q, out, splits = _decode(ctx, torch, kv, Hq, q_type, seed=5, wgs=wgs)
    ref = oracle_attn(q, kv, 0, range(len(lens)), lens, 1, d ** -0.5)
    mx, mn = assert_close(out, ref, MAX_TOL, MEAN_TOL, what="stream decode vs exact")
    gg = oracle_attn(q, kv, 0, range(len(lens)), lens, 1, d ** -0.5, mode=vvo.GGML)
    gmx, gmn = err_stats(out, gg)
    print(f"  splits {splits}: vs exact max {mx:.2e} mean {mn:.2e}; vs ggml-order max {gmx:.2e} mean {gmn:.2e}")
    assert gmx <= MAX_TOL and gmn <= MEAN_TOL
    kv.free()


def test_stream_decode_matches_register_kernel(ctx, torch_gpu):
    """Same bytes, same Q: the LDS-streamed and the register-streamed kernels
    differ only in where each split's running max sits (f16 p * d_v rounding)."""
    torch = torch_gpu
    lens = [6001, 5000]
    kv = _cache(ctx, 128, 4, lens, seed=77)
    _, a, sa = _decode(ctx, torch, kv, 28, vva.F32, seed=8)
    ctx.set_attn_path(2)
    try:
        _, b, sb = _decode(ctx, torch, kv, 28, vva.F32, seed=8)
    finally:
        ctx.set_attn_path(0)
    print(f"splits stream {sa}, register {sb}; max diff {np.abs(a - b).max():.2e}")
    assert np.abs(a - b).max() < 2e-4
    kv.free()


def test_stream_decode_split_count_does_not_change_result(ctx, torch_gpu):
    torch = torch_gpu
    lens = [5000, 4321]
    kv = _cache(ctx, 128, 4, lens, seed=3)
    outs = []
    for wgs in (2, 16, 100, 512):
        _, out, splits = _decode(ctx, torch, kv, 28, vva.F32, seed=9, wgs=wgs)
        outs.append((splits, out))
    assert len({s for s, _ in outs}) == 4, [s for s, _ in outs]
    for s, o in outs[1:]:
        assert np.abs(o - outs[0][1]).max() < 2e-4, s
    kv.free()


def test_stream_decode_explicit_mask(ctx, torch_gpu):
    torch = torch_gpu
    L = 2000
    kv = _cache(ctx, 128, 4, [L], seed=4)
    m = np.zeros((1, 1, L), np.float32)
    m[0, 0, 100:900] = -np.inf                 # a hole across several splits
    m[0, 0, 1500:1503] = -np.inf
    mbits = vvo.f16_bits(m)
    q, out, _ = _decode(ctx, torch, kv, 28, vva.F32, seed=6, mask=mbits)
    ref = oracle_attn(q, kv, 0, [0], [L], 1, 128 ** -0.5, mask=mbits)
    assert_close(out, ref, MAX_TOL, MEAN_TOL, what="masked stream decode")
    kv.free()


def test_stream_decode_consecutive_steps(ctx, torch_gpu):
    """Append-then-attend steps through rope_append, as the decode loop runs
    them: each step's output matches the oracle on the grown cache."""
    torch = torch_gpu
    d, Hq, Hkv, L0 = 128, 28, 4, 3000
    kv = vva.KVCache(ctx, 1, Hkv, d, L0 + 8, 2, vva.Q8_0)
    fill_cache(kv, [L0, L0], seed=12)
    rng = np.random.default_rng(13)
    for step in range(3):
        L = L0 + step
        q = to_gpu(torch, rng.standard_normal((2, 1, Hq, d)), vva.F32)
        k = to_gpu(torch, rng.standard_normal((2, 1, Hkv, d)), vva.F32)
        v = to_gpu(torch, rng.standard_normal((2, 1, Hkv, d)), vva.F32)
        pos = torch.full((1,), L, dtype=torch.int32, device="cuda")
        qr = torch.empty_like(q)
        ctx.rope_append(kv, 0, q, k, v, pos, qr)
        out = torch.empty_like(q)
        ctx.attn(kv, 0, qr, out, d ** -0.5)
        torch.cuda.synchronize()
        ref = oracle_attn(as_f32(torch, qr), kv, 0, [0, 1], [L + 1, L + 1], 1, d ** -0.5)
        assert_close(as_f32(torch, out), ref, MAX_TOL, MEAN_TOL, what=f"step {step}")
        for s in range(2):
            kv.set_len(s, L + 1)
    kv.free()



def _decode_splits(ctx, torch, kv, Hq, seed, splits):
    return _decode(ctx, torch, kv, Hq, vva.F32, seed=seed, splits=splits)


@pytest.mark.parametrize("d,Hq,Hkv,lens", [
    (128, 28, 4, [5000, 1234]),    # kv-head pairs gathered (272-byte slices), 64-key tiles
    (64, 14, 2, [3001, 77]),       # whole 136-byte rows, 128-key tiles
    (128, 8, 1, [2049, 2048]),     # 136-byte rows of one kv head
])
def test_stream_decode_round_robin_tiles(ctx, torch_gpu, d, Hq, Hkv, lens):
    """Split s takes tiles s, s + n, s + 2n, ... of its sequence.  Forced
    split counts from 1 (every tile in one workgroup) to far more splits than
    tiles (splits with no key at all, the short sequence's only partial tile
    in one split) give the oracle's result."""
    torch = torch_gpu
    kv = _cache(ctx, d, Hkv, lens, seed=d * Hkv + len(lens))
    for splits in (1, 3, 7, 64, 200, 1024):
        print(f"round-robin d={d} Hq={Hq} Hkv={Hkv} lens={lens} splits={splits}", flush=True)
        q, out, used = _decode_splits(ctx, torch, kv, Hq, seed=splits, splits=splits)
        assert used == splits
        ref = oracle_attn(q, kv, 0, range(len(lens)), lens, 1, d ** -0.5)
        assert_close(out, ref, MAX_TOL, MEAN_TOL, what=f"{splits} splits")
    kv.free()


def test_stream_decode_unaligned_window(ctx, torch_gpu):
    """ggml_flash_attn_ext over a window of a Q8_0 cache that starts 5 rows in
    (136-byte rows: 8 bytes past a 16-byte boundary), no mask: every tile is
    loaded from the 16-byte boundary below it."""
    torch = torch_gpu
    d, Hq, Hkv, r0, L = 64, 14, 2, 5, 3001
    kv = vva.KVCache(ctx, 1, Hkv, d, r0 + L + 8, 1, vva.Q8_0)
    fill_cache(kv, [r0 + L], seed=99)
    kview, vview = kv.views(0, 0)
    for t_ in (kview, vview):
        t_.data += r0 * t_.nb[2]
        t_.ne[1], t_.ne[2] = t_.ne[2], t_.ne[1]        # ne = [d, L, Hkv, 1]
        t_.nb[1], t_.nb[2] = t_.nb[2], t_.nb[1]
        t_.ne[1] = L
    assert (kview.data % 16) == 8
    rng = np.random.default_rng(98)
    q = to_gpu(torch, rng.standard_normal((1, 1, Hq, d)), vva.F32)
    out = torch.full((1, 1, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
    kraw, vraw = kv.download(0, 0, r0 + L)
    ref = vvo.attn(as_f32(torch, q), [kraw[r0:].reshape(-1)], [vraw[r0:].reshape(-1)], vva.Q8_0, vva.Q8_0,
                   [L], n_kv_heads=Hkv, scale=d ** -0.5, mask_mode=vvo.MASK_NONE)
    for splits in (5, 64):
        print(f"unaligned window splits={splits}", flush=True)
        with ctx.schedule(decode_splits=splits):
            ctx.flash_attn_ext(q.permute(0, 2, 1, 3), None, None, out, d ** -0.5, k_view=kview, v_view=vview)
            torch.cuda.synchronize()
        assert ctx.last_decode_splits() == splits
        assert_close(as_f32(torch, out), ref, MAX_TOL, MEAN_TOL, what=f"unaligned window, {splits} splits")
    kv.free()


def _tile_keys(d, Hkv):
    """Keys per LDS tile of the streamed kernel: 17,408 bytes of one operand
    over the kv heads a workgroup takes (a pair of them for d = 128 caches
    with 4 or 8 kv heads)."""
    heads = 2 if (d == 128 and Hkv >= 4) else Hkv
    return 17408 // (heads * (d // 32) * 34)


@pytest.mark.parametrize("d,Hq,Hkv,L", [
    (64, 14, 2, 4097),     # 0.5B heads: 128-key tiles, two slot pairs per wave per tile
    (64, 8, 1, 6001),      # one kv head: 256-key tiles, two slot pairs per wave per tile
    (128, 28, 4, 8193),    # 7B heads: 64-key tiles, one slot pair per wave per tile
])
def test_stream_decode_peaked_scores(ctx, torch_gpu, d, Hq, Hkv, L):
    """Peaked attention, where a running-max raise inside a tile is certain.

    Q is N(0,1) * 4 (scores spread ~4 nats), and in every 3rd tile a key is
    planted at 80 % of the tile (for d = 64, in the second slot pair of its
    wave) whose score for the first query head of each group is 23-27 nats,
    about 10 nats above every random score.  The split that meets it raises
    its running max after the tile's first slot pair has formed its p, the
    case where p formed on the old base must be rescaled too.  Checked
    against the ggml-order oracle (Q quantized to Q8_0 per block, as ggml
    does for Q8_0 K: the peaked softmax amplifies the Q rounding, so the
    exact-Q oracle is reported only) for several split counts, and against
    the register-streamed kernel on the same bytes."""
    torch = torch_gpu
    G = Hq // Hkv
    B = 2
    kv = _cache(ctx, d, Hkv, [L, L - 500], seed=d * 7 + Hkv)
    rng = np.random.default_rng(2024 + d + Hkv)
    q = (rng.standard_normal((B, 1, Hq, d)) * 4.0).astype(np.float32)
    TT = _tile_keys(d, Hkv)
    planted = 0
    for b in range(B):
        Lb = L if b == 0 else L - 500
        for t in range(0, (Lb - 1) // TT, 3):
            j = t * TT + (4 * TT) // 5
            if j >= Lb - 1:
                break
            target = 23.0 + 4.0 * rng.random()            # nats, for query head h * G
            k_row = np.empty((1, Hkv, d), np.float32)
            for h in range(Hkv):
                q0 = q[b, 0, h * G]
                k_row[0, h] = q0 * (target / (d ** -0.5 * float(q0 @ q0)))
            v_row = rng.standard_normal((1, Hkv, d)).astype(np.float32)
            kv.upload(0, b, j, k_row, v_row)
            planted += 1
    assert planted >= 6
    qg = torch.from_numpy(q).cuda()
    ggml_ref = None
    outs = {}
    for splits in (0, 3, 17, 64):
        out = torch.full((B, 1, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
        with ctx.schedule(decode_splits=splits):
            ctx.attn(kv, 0, qg, out, d ** -0.5)
            torch.cuda.synchronize()
        used = ctx.last_decode_splits()
        o = as_f32(torch, out)
        if ggml_ref is None:
            ggml_ref = oracle_attn(q, kv, 0, range(B), [L, L - 500], 1, d ** -0.5, mode=vvo.GGML)
            exact = oracle_attn(q, kv, 0, range(B), [L, L - 500], 1, d ** -0.5)
            emx, emn = err_stats(o, exact)
            print(f"  vs exact-Q oracle (reported): max {emx:.2e} mean {emn:.2e}")
        mx, mn = assert_close(o, ggml_ref, MAX_TOL, MEAN_TOL, what=f"peaked decode, {used} splits vs ggml-order")
        print(f"peaked d={d} Hq={Hq} Hkv={Hkv} L={L} planted={planted} splits={used}: max {mx:.2e} mean {mn:.2e}",
              flush=True)
        outs[used] = o
    ctx.set_attn_path(2)
    try:
        out = torch.full((B, 1, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
        ctx.attn(kv, 0, qg, out, d ** -0.5)
        torch.cuda.synchronize()
    finally:
        ctx.set_attn_path(0)
    reg = as_f32(torch, out)
    assert_close(reg, ggml_ref, MAX_TOL, MEAN_TOL, what="peaked decode, register kernel vs ggml-order")
    kv.free()


@pytest.mark.parametrize("vscale", [2.0 ** 13, 2.0 ** 16, 2.0 ** 20])
def test_stream_decode_v_beyond_the_f16_range(ctx, torch_gpu, vscale):
    """The streamed decode forms P' = p * d_v as an f16 MFMA operand with p
    <= 2^8 (the lazy running-max slack).  V blocks with d_v = amax / 127 <
    2^8 (|V| <= 32512) take the plain f16 product; a larger d_v raises the
    row's exp2 base so P' stays below 2^15, so any Q8_0 cache gives a finite
    result (ggml dequantizes Q8_0 V to fp32, src/qwen2.cpp:332-335).
    Scaling a Q8_0 block by a power of two keeps its codes and scales d by
    it, so the output divided by the scale must match the oracle of the
    unscaled cache.  V * 2^13 with |V| < 3.95 reaches 32358 (the plain path,
    at its edge); 2^16 and 2^20 reach 2.6e5 and 4.1e6 (d_v up to 32600)."""
    torch = torch_gpu
    d, Hq, Hkv, lens = 128, 28, 4, [6001, 6001]
    print(f"stream decode V scale 2^{int(np.log2(vscale))}", flush=True)
    rng = np.random.default_rng(41)
    caches, outs = [], []
    k = [rng.standard_normal((n, Hkv, d)).astype(np.float32) for n in lens]
    v = [np.clip(rng.standard_normal((n, Hkv, d)), -3.95, 3.95).astype(np.float32) for n in lens]
    q = to_gpu(torch, rng.standard_normal((len(lens), 1, Hq, d)), vva.F32)
    for scale in (1.0, vscale):
        kv = vva.KVCache(ctx, 1, Hkv, d, max(lens), len(lens), vva.Q8_0)
        for s, n in enumerate(lens):
            kv.upload(0, s, 0, k[s], (v[s] * scale).astype(np.float32))
            kv.set_len(s, n - 1)
        out = torch.full((len(lens), 1, Hq, d), float("nan"), dtype=torch.float32, device="cuda")
        ctx.attn(kv, 0, q, out, d ** -0.5)
        torch.cuda.synchronize()
        outs.append(as_f32(torch, out))
        caches.append(kv)
    vmax = max(np.abs(vvo.to_f32(caches[1].download(0, s, n)[1].reshape(-1), vva.Q8_0, n * Hkv * d)).max()
               for s, n in enumerate(lens))
    assert 3.2e4 * vscale / 2.0 ** 13 < vmax <= 32512.0 * vscale / 2.0 ** 13
    assert np.isfinite(outs[1]).all()
    ref = oracle_attn(as_f32(torch, q), caches[0], 0, range(len(lens)), lens, 1, d ** -0.5)
    assert_close(outs[0], ref, MAX_TOL, MEAN_TOL, what="unscaled V")
    mx, mn = assert_close(outs[1] / vscale, ref, MAX_TOL, MEAN_TOL, what="V scaled, rescaled back")
    print(f"  V up to {vmax:.0f}: rescaled output vs oracle max {mx:.2e} mean {mn:.2e}")
    for kv in caches:
        kv.free()
