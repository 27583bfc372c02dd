"""CPU pins of the shared numerics (include/lisa_numerics.h) through the
oracle, against double-precision math: ulp bounds for exp/exp2/log/rsqrt,
absolute bounds for sin/cos over the RoPE angle range, bf16 round-to-nearest-
even on constructed ties, and the activation formulas of gdn.metal:16-19 and
mlp.metal:11-16."""
import numpy as np

from _lisa import load_oracle

orc = load_oracle()


def ulp_err(got, want64):
    """Error in units of the f32 spacing at the exact value."""
    want32 = want64.astype(np.float32)
    spacing = np.spacing(np.abs(want32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - want64) / spacing


def grid(lo, hi, n=200001):
    return np.linspace(lo, hi, n, dtype=np.float64).astype(np.float32)


def test_exp_exp2_log_rsqrt_ulp():
    x = grid(-87.0, 88.0)
    assert ulp_err(orc.math("exp", x), np.exp(x.astype(np.float64))).max() <= 2.0
    x = grid(-125.0, 127.0)
    assert ulp_err(orc.math("exp2", x), np.exp2(x.astype(np.float64))).max() <= 2.0
    x = np.exp(grid(-80.0, 80.0).astype(np.float64)).astype(np.float32)
    x = x[x > 0]
    assert ulp_err(orc.math("log", x), np.log(x.astype(np.float64))).max() <= 2.0
    x = np.exp(grid(-60.0, 60.0).astype(np.float64)).astype(np.float32)
    # 1 / sqrt(x) from two correctly rounded operations: below 1.5 ulp
    assert ulp_err(orc.math("rsqrt", x), 1.0 / np.sqrt(x.astype(np.float64))).max() <= 1.5


def test_sincos_over_rope_range():
    """Angles are position * inv_freq with positions below 65536."""
    x = grid(-66000.0, 66000.0, 400001)
    x64 = x.astype(np.float64)
    assert np.max(np.abs(orc.math("sin", x) - np.sin(x64))) <= 2e-6
    assert np.max(np.abs(orc.math("cos", x) - np.cos(x64))) <= 2e-6
    small = grid(-8.0, 8.0)
    assert np.max(np.abs(orc.math("sin", small) - np.sin(small.astype(np.float64)))) <= 3e-7


def test_bf16_round_to_nearest_even():
    u = np.array([0x3F808000, 0x3F818000, 0x3F808001, 0x3F807FFF, 0x7F7FFFFF, 0xFF800000, 0x7FC00001,
                  0x00008000, 0x80018000], dtype=np.uint32)
    got = orc.math("bf16", u.view(np.float32)).view(np.uint32)
    want = np.array([0x3F800000, 0x3F820000, 0x3F810000, 0x3F800000, 0x7F800000, 0xFF800000, 0,
                     0x00000000, 0x80020000], dtype=np.uint32)
    for i in range(len(u)):
        if i == 6:
            assert np.isnan(got[i:i + 1].view(np.float32))[0]
        else:
            assert got[i] == want[i], hex(u[i])
    bits = orc.f32_to_bf16_bits(u[:4].view(np.float32))
    assert list(bits) == [0x3F80, 0x3F82, 0x3F81, 0x3F80]


def test_activations():
    x = grid(-30.0, 30.0)
    x64 = x.astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-x64))
    # the exp2 forms evaluate exp2(1.4427 * x): the rounded argument costs |x| * 2^-23 relative
    for fn, bound in (("sigmoid_exp", 4e-7), ("sigmoid_exp2", np.abs(x64) * 2.0**-23 + 4e-7)):
        assert np.all(np.abs(orc.math(fn, x) - sig) / np.maximum(sig, 1e-30) <= bound)
    for fn, bound in (("silu_exp", 4e-7), ("silu_exp2", np.abs(x64) * 2.0**-23 + 4e-7)):
        want = x64 * sig
        assert np.all(np.abs(orc.math(fn, x) - want) / np.maximum(np.abs(want), 1e-30) <= bound)
    # gdn.metal:16-19: softplus(x) = x above 20, log(1 + exp(x)) otherwise
    sp = orc.math("softplus", x)
    ref = np.where(x64 > 20.0, x64, np.log1p(np.exp(x64)))
    # log(1 + exp(x)) rounds 1 + exp(x): an absolute error of a few 2^-24
    assert np.all(np.abs(sp - ref) <= 2.4e-7 + 4e-7 * ref)
    assert np.array_equal(sp[x > 20.0], x[x > 20.0])


def test_rms_norm_matches_double():
    """norm.metal:10-47: y = bf16(x * rsqrt(mean(x^2) + 1e-6) * w)."""
    rng = np.random.default_rng(3)
    x = orc.f32_to_bf16_bits((rng.standard_normal(5120) * 3).astype(np.float32))
    w = orc.f32_to_bf16_bits(rng.uniform(0.9, 1.1, 5120).astype(np.float32))
    got = orc.bf16_bits_to_f32(orc.rms_norm(x, w))
    xf, wf = orc.bf16_bits_to_f32(x).astype(np.float64), orc.bf16_bits_to_f32(w).astype(np.float64)
    ref = xf / np.sqrt(np.mean(xf**2) + 1e-6) * wf
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-8 + 1e-30)


def test_rms_norm_tiles_matches_double():
    """The decode path's RMSNorm whose statistic is summed from per-8-row tile
    partials: the same closed form as norm.metal:10-47."""
    rng = np.random.default_rng(4)
    x = orc.f32_to_bf16_bits((rng.standard_normal(5120) * 3).astype(np.float32))
    w = orc.f32_to_bf16_bits(rng.uniform(0.9, 1.1, 5120).astype(np.float32))
    got = orc.bf16_bits_to_f32(orc.rms_norm_tiles(x, w))
    xf, wf = orc.bf16_bits_to_f32(x).astype(np.float64), orc.bf16_bits_to_f32(w).astype(np.float64)
    ref = xf / np.sqrt(np.mean(xf**2) + 1e-6) * wf
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-8 + 1e-30)
    # a different summation order than the single-launch statistic, same value to rounding
    other = orc.bf16_bits_to_f32(orc.rms_norm(x, w))
    assert np.max(np.abs(got - other) / np.maximum(np.abs(other), 1e-30)) <= 2.0**-7
