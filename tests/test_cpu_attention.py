"""CPU pins of the oracle's decode attention.

Split-K SDPA against a double-precision softmax at the reference's context
lengths {1, 16, 63, 64, 129, 1000} with its 1e-4 tolerance
(tests/attn_sliced.rs:132-191), the causal 3-row block equal to three single
rows (bit-exact), a context past 16384 where the reference's clamped merge is
wrong (attention.metal:611-641) and ours must still match the closed form,
and the q/k head norm + partial NeoX RoPE against double precision.
"""
import numpy as np
import pytest

from _lisa import load_oracle

orc = load_oracle()
QH, KVH, HD = 24, 4, 256


def bf(x):
    return orc.f32_to_bf16_bits(np.asarray(x, np.float32))


def fb(h):
    return orc.bf16_bits_to_f32(h)


def ref_sdpa(q, kc, vc, cap, pos):
    q = fb(q).reshape(QH, HD).astype(np.float64)
    K = fb(kc).reshape(KVH, cap, HD)[:, :pos + 1].astype(np.float64)
    V = fb(vc).reshape(KVH, cap, HD)[:, :pos + 1].astype(np.float64)
    out = np.empty((QH, HD))
    for h in range(QH):
        s = K[h // 6] @ q[h] / 16.0
        p = np.exp(s - s.max())
        out[h] = p @ V[h // 6] / p.sum()
    return out


def make_cache(rng, cap):
    return bf(rng.standard_normal(KVH * cap * HD)), bf(rng.standard_normal(KVH * cap * HD))


@pytest.mark.parametrize("ctx", [1, 16, 63, 64, 129, 1000])
def test_sdpa_matches_softmax(ctx):
    rng = np.random.default_rng(ctx)
    cap = ctx + 3
    kc, vc = make_cache(rng, cap)
    q = bf(rng.standard_normal(QH * HD))
    got = orc.sdpa(q, kc, vc, cap, ctx - 1, 1)[0]
    assert np.max(np.abs(got - ref_sdpa(q, kc, vc, cap, ctx - 1))) < 1e-4


def test_sdpa_block3_rows_equal_single_rows():
    rng = np.random.default_rng(3)
    cap, base = 200, 130
    kc, vc = make_cache(rng, cap)
    q3 = bf(rng.standard_normal(3 * QH * HD))
    got3 = orc.sdpa(q3, kc, vc, cap, base, 3)
    for t in range(3):
        one = orc.sdpa(q3[t * QH * HD:(t + 1) * QH * HD], kc, vc, cap, base + t, 1)[0]
        assert np.array_equal(got3[t].view(np.uint32), one.view(np.uint32))
        assert np.max(np.abs(got3[t] - ref_sdpa(q3[t * QH * HD:(t + 1) * QH * HD], kc, vc, cap, base + t))) < 1e-4


def test_sdpa_beyond_16k():
    """17000 keys = 266 slices: every slice must enter the merge."""
    rng = np.random.default_rng(17)
    ctx = 17000
    kc, vc = make_cache(rng, ctx)
    # put the decisive keys at the end of the context
    q = bf(rng.standard_normal(QH * HD))
    K = fb(kc).reshape(KVH, ctx, HD).copy()
    K[:, -8:] = fb(q).reshape(QH, HD)[::6][:, None, :] * 2.0
    kc = bf(K.reshape(-1))
    got = orc.sdpa(q, kc, vc, ctx, ctx - 1, 1)[0]
    assert np.max(np.abs(got - ref_sdpa(q, kc, vc, ctx, ctx - 1))) < 1e-4


@pytest.mark.parametrize("pos", [0, 1, 4095, 65535])
def test_head_norm_rope(pos):
    """attention.metal:118-155: n = x * rsqrt(mean(x^2)+1e-6) * w; dims j < 32
    rotate with their partner j + 32 by pos * 1e7^(-2j/64); dims >= 64 pass."""
    rng = np.random.default_rng(pos + 1)
    raw = (rng.standard_normal(HD) * 2).astype(np.float32)
    w = bf(rng.uniform(0.9, 1.1, HD))
    got = fb(orc.head_norm_rope(raw, w, pos)).astype(np.float64)
    x = fb(bf(raw)).astype(np.float64)
    n = x / np.sqrt(np.mean(x**2) + 1e-6) * fb(w)
    j = np.arange(32)
    ang = pos * (1.0 / 1e7 ** (2.0 * j / 64.0))
    want = n.copy()
    want[j] = n[j] * np.cos(ang) - n[j + 32] * np.sin(ang)
    want[j + 32] = n[j + 32] * np.cos(ang) + n[j] * np.sin(ang)
    tol = np.maximum(np.abs(want), np.max(np.abs(n)) * 2.0**-8) * 2.0**-7
    assert np.all(np.abs(got - want) <= tol)
