"""Pins the oracle's conversions, Q8_0 blocks and RoPE.

Each check is independent of the oracle's own code: numpy's float16 and
torch's bfloat16 conversions (exhaustive / dense sweeps), closed-form Q8_0
blocks whose scale is an exact power of two, Hugging Face's fp64 RoPE on the
reference's RoPE test case (tests/dump_rope_reference.py defaults, tolerance
of tests/test_rope.cpp:97), and RoPE's group properties.
"""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ---------------------------------------------------------------- fp16 / bf16

def test_f16_to_f32_exhaustive(vvo):
    h = np.arange(65536, dtype=np.uint16)
    got = vvo.to_f32(h.view(np.uint8), vvo.F16, 65536)
    ref = h.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def _f16_edge_values():
    # every f16 value, the midpoints between neighbours and one f32 ulp either side
    h = np.arange(0, 0x7C00, dtype=np.uint16)
    v = h.view(np.float16).astype(np.float64)
    mid = ((v[:-1] + v[1:]) / 2).astype(np.float32)
    up = np.nextafter(mid, np.float32(np.inf))
    dn = np.nextafter(mid, np.float32(0))
    base = np.concatenate([v.astype(np.float32), mid, up, dn])
    specials = np.array([0.0, 65504.0, 65519.996, 65520.0, 65536.0, 1e30, np.inf, 2.0 ** -24,
                         2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -14, 5.9e-8], dtype=np.float32)
    base = np.concatenate([base, specials])
    return np.concatenate([base, -base])


def test_f32_to_f16_round_to_nearest_even(vvo):
    rng = np.random.default_rng(7)
    rand = (rng.standard_normal(500_000) * np.exp(rng.uniform(-30, 13, 500_000))).astype(np.float32)
    x = np.concatenate([_f16_edge_values(), rand])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    got = vvo.f16_bits(x)
    np.testing.assert_array_equal(got, ref)
    nan = vvo.f16_bits(np.array([np.nan], dtype=np.float32))
    assert (nan[0] & 0x7C00) == 0x7C00 and (nan[0] & 0x3FF) != 0


def test_f32_to_bf16_round_to_nearest_even(vvo):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(8)
    rand = (rng.standard_normal(500_000) * np.exp(rng.uniform(-80, 80, 500_000))).astype(np.float32)
    # exact ties: low 16 bits == 0x8000 with even and odd kept parts
    ties = (rng.integers(0, 2 ** 15, 20_000, dtype=np.uint32) << 16 | 0x8000).astype(np.uint32).view(np.float32)
    x = np.concatenate([rand, ties, np.array([0.0, -0.0, np.inf, -np.inf, 3.3895314e38], dtype=np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = vvo.bf16_bits(x)
    nan = np.isnan(x)
    np.testing.assert_array_equal(got[~nan], ref[~nan])
    # NaN stays a quiet NaN (payload is not compared: torch canonicalizes it)
    assert np.all((got[nan] & 0x7F80) == 0x7F80) and np.all((got[nan] & 0x0040) != 0)
    back = vvo.to_f32(vvo.from_f32(x[~nan], vvo.BF16), vvo.BF16, int((~nan).sum()))
    np.testing.assert_array_equal(back, torch.from_numpy(x[~nan]).to(torch.bfloat16).float().numpy())


# ---------------------------------------------------------------------- Q8_0

def _blocks(buf):
    b = buf.reshape(-1, 34)
    d = b[:, :2].copy().view(np.uint16)[:, 0]
    q = b[:, 2:].view(np.int8)
    return d, q


def test_q8_0_known_answer_power_of_two_scale(vvo):
    rng = np.random.default_rng(3)
    for k in range(-6, 7):
        codes = rng.integers(-127, 128, 32).astype(np.int32)
        codes[rng.integers(0, 32)] = 127 * (1 if rng.random() < 0.5 else -1)
        x = (codes * 2.0 ** k).astype(np.float32)          # amax = 127 * 2^k -> d = 2^k exactly
        buf = vvo.from_f32(x, vvo.Q8_0)
        d, q = _blocks(buf)
        assert d[0] == np.float16(2.0 ** k).view(np.uint16)
        np.testing.assert_array_equal(q[0], codes)
        np.testing.assert_array_equal(vvo.to_f32(buf, vvo.Q8_0, 32), x)


def test_q8_0_rounds_half_away_from_zero(vvo):
    x = np.zeros(32, dtype=np.float32)
    x[0] = 127.0                      # d = 1
    x[1], x[2], x[3], x[4] = 2.5, -2.5, 0.5, -1.5
    _, q = _blocks(vvo.from_f32(x, vvo.Q8_0))
    assert list(q[0, :5]) == [127, 3, -3, 1, -2]


def test_q8_0_error_bound_and_idempotence(vvo):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(32 * 4096) * np.exp(rng.uniform(-8, 8, 4096)).repeat(32)).astype(np.float32)
    buf = vvo.from_f32(x, vvo.Q8_0)
    y = vvo.to_f32(buf, vvo.Q8_0, x.size)
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    d = (amax / 127.0).repeat(32)
    # |x - c*fp16(d)| <= d/2 + 127*|d - fp16(d)|, and fp16 rounding of d is
    # relative 2^-11 for normal scales, absolute 2^-25 for subnormal ones
    bound = d * 0.5 + 127 * np.maximum(d * 2.0 ** -11, 2.0 ** -25)
    assert np.all(np.abs(x - y) <= bound * (1 + 1e-6))
    np.testing.assert_array_equal(vvo.from_f32(y, vvo.Q8_0), buf)
    zero = vvo.from_f32(np.zeros(32, np.float32), vvo.Q8_0)
    assert not zero.any()


# ---------------------------------------------------------------------- RoPE

def _golden_rope():
    g = np.load(os.path.join(GOLDEN, "rope_seed2025.npz"))
    seq, heads, dim = int(g["seq"]), int(g["heads"]), int(g["dim"])
    x = np.random.default_rng(int(g["seed"])).standard_normal((seq, heads, dim)).astype(np.float32)
    return x, g["rows"], g["expected"], float(g["theta"])


@pytest.mark.parametrize("mode", [0, 1])
def test_rope_matches_hf_fp64_reference_case(vvo, mode):
    x, rows, expected, theta = _golden_rope()
    y = vvo.rope(x[None], np.arange(x.shape[0], dtype=np.int32), theta, mode)[0]
    err = np.abs(y[rows] - expected).max()
    assert err < 5e-5, err                      # tests/test_rope.cpp:97


def test_rope_position_zero_is_identity(vvo):
    x = np.random.default_rng(1).standard_normal((2, 5, 3, 128)).astype(np.float32)
    y = vvo.rope(x, np.zeros((2, 5), np.int32))
    np.testing.assert_array_equal(y, x)


def test_rope_preserves_pair_norms(vvo):
    x = np.random.default_rng(2).standard_normal((1, 64, 4, 128)).astype(np.float32)
    pos = np.arange(0, 64 * 500, 500, dtype=np.int32)
    y = vvo.rope(x, pos)
    n0 = np.hypot(x[..., :64], x[..., 64:])
    n1 = np.hypot(y[..., :64], y[..., 64:])
    np.testing.assert_allclose(n1, n0, rtol=2e-6, atol=1e-6)


def test_rope_composition_matches_sum_of_positions(vvo):
    x = np.random.default_rng(5).standard_normal((1, 16, 2, 64)).astype(np.float32)
    p = np.arange(16, dtype=np.int32) * 37
    q = np.arange(16, dtype=np.int32) * 11 + 5
    two = vvo.rope(vvo.rope(x, p, mode=1), q, mode=1)
    one = vvo.rope(x, p + q, mode=1)
    np.testing.assert_allclose(two, one, atol=2e-5)


def test_rope_recurrence_drift_at_long_context(vvo):
    # ggml's fp32 theta recurrence (theta_{i+1} = theta_i * s) accumulates a
    # relative error of ~i * 2^-24 on angles of up to 3.3e4 rad at 32k
    # positions: ~1e-2 away from the exact pow form.  This is why the GPU
    # kernel reproduces the recurrence instead of using pow().
    x = np.random.default_rng(6).standard_normal((1, 8, 2, 128)).astype(np.float32)
    pos = np.arange(32760, 32768, dtype=np.int32)
    drift = np.abs(vvo.rope(x, pos, mode=0) - vvo.rope(x, pos, mode=1)).max()
    assert 1e-4 < drift < 3e-2
    near = np.abs(vvo.rope(x, pos - 32700, mode=0) - vvo.rope(x, pos - 32700, mode=1)).max()
    assert near < 5e-5
