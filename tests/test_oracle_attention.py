"""Pins the oracle's attention (both modes) before it is trusted as checker.

Checks, each independent of the oracle's code path:
  * the Hugging Face fp64 Qwen2 attention case (RoPE + repeat_kv + causal
    eager softmax; shape of tests/dump_qwen2_reference.py), tolerance 5e-5 as
    tests/test_qwen2_block.cpp:151;
  * a vectorised numpy fp64 softmax(QK^T)V brute force on tiny shapes for every
    cache type (the oracle is row-by-row two-pass / online);
  * invariants: causal row 0 returns V_0, Q = 0 returns the mean of the
    visible V rows, GQA equals MHA on repeated K/V, chunked prefill equals
    single-shot (tests/test_qwen2_resident.cpp paths B-D), decode equals the
    last prefill row, an explicit causal mask equals the implicit one, a row
    with no visible key is 0;
  * the ggml-order mode stays within the path's tolerances of the exact mode,
    and its F32-accumulator variant differs from it only through the F16
    running V sum.
"""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TYPES = {"f32": 0, "f16": 1, "q8_0": 8, "bf16": 30}


def make_cache(vvo, rows, type_):
    """rows: f32 [L, Hkv, d] -> raw cache bytes and the decoded f32 values."""
    raw = vvo.from_f32(rows, type_)
    dec = vvo.to_f32(raw, type_, rows.size).reshape(rows.shape)
    return raw, dec


def round_q(vvo, q, type_):
    """Q as ggml's FA feeds it to the K dot: rounded to K's vec-dot type."""
    if type_ == 0:
        return q.astype(np.float32)
    return vvo.to_f32(vvo.from_f32(q, type_), type_, q.size).reshape(q.shape)


def brute(q, kdec, vdec, past, scale, Hkv, mask=None):
    """numpy fp64 reference. q [T, Hq, d]; kdec/vdec [L, Hkv, d]; causal by past."""
    T, Hq, d = q.shape
    L = kdec.shape[0]
    g = Hq // Hkv
    out = np.zeros((T, Hq, d))
    for h in range(Hq):
        K = kdec[:, h // g].astype(np.float64)
        V = vdec[:, h // g].astype(np.float64)
        s = q[:, h].astype(np.float64) @ K.T * scale
        if mask is None:
            s = np.where(np.arange(L)[None, :] > past + np.arange(T)[:, None], -np.inf, s)
        else:
            s = s + mask
        m = s.max(axis=1, keepdims=True)
        ok = np.isfinite(m[:, 0])
        p = np.where(ok[:, None], np.exp(s - np.where(ok[:, None], m, 0)), 0)
        den = p.sum(axis=1, keepdims=True)
        out[:, h] = np.where(ok[:, None], (p @ V) / np.where(den == 0, 1, den), 0)
    return out


def test_matches_hf_fp64_golden_case(vvo):
    g = np.load(os.path.join(GOLDEN, "attn_seed1234.npz"))
    nh, nkv, hd, seq = 4, 2, 32, 64
    rng = np.random.default_rng(int(g["seed"]))
    q = rng.standard_normal((seq, nh, hd)).astype(np.float32)
    k = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    pos = np.arange(seq, dtype=np.int32)
    qr = vvo.rope(q[None], pos, float(g["theta"]))
    kr = vvo.rope(k[None], pos, float(g["theta"]))[0]
    for mode in (vvo.EXACT, vvo.GGML):
        out = vvo.attn(qr, [kr.view(np.uint8)], [v.view(np.uint8)], 0, 0, [seq], n_kv_heads=nkv,
                       scale=hd ** -0.5, mode=mode)[0]
        err = np.abs(out - g["expected"]).max()
        assert err < 5e-5, (mode, err)


@pytest.mark.parametrize("ktype", ["f32", "f16", "bf16", "q8_0"])
@pytest.mark.parametrize("T,past", [(1, 37), (7, 0), (5, 11)])
def test_exact_mode_matches_numpy_brute_force(vvo, ktype, T, past):
    rng = np.random.default_rng(hash((ktype, T, past)) % 2 ** 32)
    Hq, Hkv, d = 6, 2, 64
    L = past + T
    t = TYPES[ktype]
    q = rng.standard_normal((1, T, Hq, d)).astype(np.float32)
    kraw, kdec = make_cache(vvo, rng.standard_normal((L, Hkv, d)).astype(np.float32), t)
    vraw, vdec = make_cache(vvo, rng.standard_normal((L, Hkv, d)).astype(np.float32), t)
    scale = d ** -0.5
    out = vvo.attn(q, [kraw], [vraw], t, t, [L], n_kv_heads=Hkv, scale=scale)[0]
    ref = brute(round_q(vvo, q[0], t), kdec, vdec, past, scale, Hkv)
    assert np.abs(out - ref).max() < 1e-6


@pytest.mark.parametrize("ktype,tol", [("f32", 1e-5), ("f16", 2e-3), ("bf16", 1e-5), ("q8_0", 1e-5)])
def test_ggml_mode_within_tolerance_of_exact(vvo, ktype, tol):
    rng = np.random.default_rng(11)
    Hq, Hkv, d, T, past = 14, 2, 64, 3, 500
    t = TYPES[ktype]
    L = past + T
    q = rng.standard_normal((1, T, Hq, d)).astype(np.float32)
    kraw, _ = make_cache(vvo, rng.standard_normal((L, Hkv, d)).astype(np.float32), t)
    vraw, _ = make_cache(vvo, rng.standard_normal((L, Hkv, d)).astype(np.float32), t)
    ex = vvo.attn(q, [kraw], [vraw], t, t, [L], n_kv_heads=Hkv, scale=d ** -0.5, mode=vvo.EXACT)
    gg = vvo.attn(q, [kraw], [vraw], t, t, [L], n_kv_heads=Hkv, scale=d ** -0.5, mode=vvo.GGML)
    assert np.abs(ex - gg).max() < tol


@pytest.mark.parametrize("ktype", ["f32", "f16", "bf16", "q8_0"])
def test_ggml_f32acc_mode_isolates_the_f16_accumulator(vvo, ktype):
    """GGML_F32ACC is ggml's order with an F32 running V sum.  It equals GGML
    bit for bit unless V is F16; with F16 V it sits within fp32 rounding of
    the exact mode while GGML (F16 running sum) is far further away, so the
    two modes differ by the F16 accumulator and nothing else."""
    rng = np.random.default_rng(23)
    Hq, Hkv, d, T, past = 14, 2, 64, 4, 700
    t = TYPES[ktype]
    L = past + T
    q = rng.standard_normal((1, T, Hq, d)).astype(np.float32)
    kraw, _ = make_cache(vvo, rng.standard_normal((L, Hkv, d)).astype(np.float32), t)
    vraw, _ = make_cache(vvo, rng.standard_normal((L, Hkv, d)).astype(np.float32), t)
    args = dict(n_kv_heads=Hkv, scale=d ** -0.5)
    ex = vvo.attn(q, [kraw], [vraw], t, t, [L], mode=vvo.EXACT, **args)
    gg = vvo.attn(q, [kraw], [vraw], t, t, [L], mode=vvo.GGML, **args)
    g32 = vvo.attn(q, [kraw], [vraw], t, t, [L], mode=vvo.GGML_F32ACC, **args)
    if ktype != "f16":
        assert np.array_equal(gg, g32)
    else:
        e32 = np.abs(g32 - ex).max()
        e16 = np.abs(gg - ex).max()
        assert e32 < 2e-5, e32
        assert e16 > 20 * e32, (e16, e32)


def _rand_case(vvo, rng, T, past, Hq=4, Hkv=2, d=32, t=0):
    L = past + T
    q = rng.standard_normal((1, T, Hq, d)).astype(np.float32)
    k = rng.standard_normal((L, Hkv, d)).astype(np.float32)
    v = rng.standard_normal((L, Hkv, d)).astype(np.float32)
    return q, k, v


@pytest.mark.parametrize("mode", [0, 1])
def test_row0_returns_v0_and_zero_query_returns_mean(vvo, mode):
    rng = np.random.default_rng(12)
    q, k, v = _rand_case(vvo, rng, 9, 0)
    out = vvo.attn(q, [k.view(np.uint8)], [v.view(np.uint8)], 0, 0, [9], n_kv_heads=2, scale=0.2, mode=mode)[0]
    for h in range(4):
        np.testing.assert_allclose(out[0, h], v[0, h // 2], atol=1e-6)
    z = np.zeros_like(q)
    out = vvo.attn(z, [k.view(np.uint8)], [v.view(np.uint8)], 0, 0, [9], n_kv_heads=2, scale=0.2, mode=mode)[0]
    for t in range(9):
        for h in range(4):
            np.testing.assert_allclose(out[t, h], v[: t + 1, h // 2].mean(axis=0), atol=1e-6)


def test_gqa_equals_mha_on_repeated_kv(vvo):
    rng = np.random.default_rng(13)
    q, k, v = _rand_case(vvo, rng, 6, 4, Hq=6, Hkv=2)
    gqa = vvo.attn(q, [k.view(np.uint8)], [v.view(np.uint8)], 0, 0, [10], n_kv_heads=2, scale=0.3)
    kr = np.ascontiguousarray(np.repeat(k, 3, axis=1))
    vr = np.ascontiguousarray(np.repeat(v, 3, axis=1))
    mha = vvo.attn(q, [kr.view(np.uint8)], [vr.view(np.uint8)], 0, 0, [10], n_kv_heads=6, scale=0.3)
    np.testing.assert_allclose(gqa, mha, atol=1e-7)


@pytest.mark.parametrize("mode", [0, 1])
def test_chunked_prefill_and_decode_equal_single_shot(vvo, mode):
    rng = np.random.default_rng(14)
    N = 24
    q, k, v = _rand_case(vvo, rng, N, 0, t=1)
    kraw, vraw = vvo.from_f32(k, 1), vvo.from_f32(v, 1)
    full = vvo.attn(q, [kraw], [vraw], 1, 1, [N], n_kv_heads=2, scale=0.25, mode=mode)[0]
    bounds = [0, 5, 12, 18, N]                   # uneven chunks, as in path D
    for a, b in zip(bounds[:-1], bounds[1:]):
        part = vvo.attn(q[:, a:b], [kraw], [vraw], 1, 1, [b], n_kv_heads=2, scale=0.25, mode=mode)[0]
        np.testing.assert_array_equal(part, full[a:b])
    dec = vvo.attn(q[:, N - 1:], [kraw], [vraw], 1, 1, [N], n_kv_heads=2, scale=0.25, mode=mode)[0]
    np.testing.assert_array_equal(dec[0], full[N - 1])


def test_explicit_mask_equals_implicit_and_masked_row_is_zero(vvo):
    rng = np.random.default_rng(15)
    T, past = 5, 6
    L = T + past
    q, k, v = _rand_case(vvo, rng, T, past)
    causal = vvo.attn(q, [k.view(np.uint8)], [v.view(np.uint8)], 0, 0, [L], n_kv_heads=2, scale=0.3)
    m = np.where(np.arange(L)[None, :] > past + np.arange(T)[:, None], -np.inf, 0.0).astype(np.float32)
    mbits = vvo.f16_bits(m)[None]
    expl = vvo.attn(q, [k.view(np.uint8)], [v.view(np.uint8)], 0, 0, [L], n_kv_heads=2, scale=0.3,
                    mask_mode=vvo.MASK_EXPLICIT, mask=mbits)
    np.testing.assert_array_equal(causal, expl)
    m[2, :] = -np.inf                                     # row with no visible key
    for mode in (0, 1):
        out = vvo.attn(q, [k.view(np.uint8)], [v.view(np.uint8)], 0, 0, [L], n_kv_heads=2, scale=0.3,
                       mask_mode=vvo.MASK_EXPLICIT, mask=vvo.f16_bits(m)[None], mode=mode)
        assert not out[0, 2].any()


def test_ragged_batch_rows_are_independent(vvo):
    rng = np.random.default_rng(16)
    qa, ka, va = _rand_case(vvo, rng, 1, 30)
    qb, kb, vb = _rand_case(vvo, rng, 1, 9)
    both = vvo.attn(np.concatenate([qa, qb]), [ka.view(np.uint8), kb.view(np.uint8)],
                    [va.view(np.uint8), vb.view(np.uint8)], 0, 0, [31, 10], n_kv_heads=2, scale=0.3)
    a = vvo.attn(qa, [ka.view(np.uint8)], [va.view(np.uint8)], 0, 0, [31], n_kv_heads=2, scale=0.3)
    b = vvo.attn(qb, [kb.view(np.uint8)], [vb.view(np.uint8)], 0, 0, [10], n_kv_heads=2, scale=0.3)
    np.testing.assert_array_equal(both[0], a[0])
    np.testing.assert_array_equal(both[1], b[0])


def test_row_subset_matches_full(vvo):
    rng = np.random.default_rng(17)
    q, k, v = _rand_case(vvo, rng, 20, 3)
    full = vvo.attn(q, [k.view(np.uint8)], [v.view(np.uint8)], 0, 0, [23], n_kv_heads=2, scale=0.3)
    rows = np.array([0, 7, 19], dtype=np.int32)
    sub = vvo.attn(q, [k.view(np.uint8)], [v.view(np.uint8)], 0, 0, [23], n_kv_heads=2, scale=0.3, rows=rows)
    np.testing.assert_array_equal(sub[0, rows], full[0, rows])
    others = np.setdiff1d(np.arange(20), rows)
    assert not sub[0, others].any()


def test_planted_mistake_is_caught_by_brute_force(vvo):
    """A shifted causal boundary (j <= past + t + 1) must fail the brute-force check."""
    rng = np.random.default_rng(18)
    T, past = 6, 2
    q, k, v = _rand_case(vvo, rng, T, past)
    wrong = vvo.attn(q, [k.view(np.uint8)], [v.view(np.uint8)], 0, 0, [T + past], n_kv_heads=2, scale=0.3,
                     past=[past + 1])[0]
    ref = brute(q[0], k, v, past, 0.3, 2)
    assert np.abs(wrong[:-1] - ref[:-1]).max() > 1e-2


@pytest.mark.parametrize("mode_name", ["GGML", "GGML_F32ACC"])
def test_ggml_order_f16c_path_equals_scalar_path(vvo, mode_name):
    """The F16C conversions of F16 K rows and of the F16 running V sum give
    the scalar loops' values bit for bit (vcvtps2ph rounds to nearest even, as
    vvo_f32_to_f16 does).  Heavy-tailed scores force running-max rescales."""
    rng = np.random.default_rng(23)
    Hq, Hkv, d, T, past = 12, 2, 128, 9, 700
    L = past + T
    q = rng.standard_normal((1, T, Hq, d)).astype(np.float32)
    k = rng.standard_normal((L, Hkv, d)).astype(np.float32)
    k *= (1.0 + 3.0 * (np.arange(L) // 64))[:, None, None].astype(np.float32)
    kraw, _ = make_cache(vvo, k, TYPES["f16"])
    vraw, _ = make_cache(vvo, rng.standard_normal((L, Hkv, d)).astype(np.float32) * 40.0, TYPES["f16"])
    mode = getattr(vvo, mode_name)
    args = dict(n_kv_heads=Hkv, scale=d ** -0.5, mode=mode)
    fast = vvo.attn(q, [kraw], [vraw], 1, 1, [L], **args)
    vvo.set_simd(False)
    try:
        slow = vvo.attn(q, [kraw], [vraw], 1, 1, [L], **args)
    finally:
        vvo.set_simd(True)
    assert np.array_equal(fast.view(np.uint32), slow.view(np.uint32))
