"""CPU pins of the oracle's small kernels against their closed forms: argmax
(the reference's KATs, tests/argmax.rs:60-92, and the lowest-index tie rule of
embed.metal:33-71), the q4 embedding row (embed.metal:6-28), the residual add
(norm.metal:50-57), SwiGLU (mlp.metal:6-17), the GDN gated RMSNorm
(gdn.metal:367-391) and the attention output gate (attention.metal:520-531)."""
import numpy as np

from _lisa import load_oracle

orc = load_oracle()


def bf(x):
    return orc.f32_to_bf16_bits(np.asarray(x, np.float32))


def fb(h):
    return orc.bf16_bits_to_f32(h)


def within_bf16(got_bits, ref64, ulps=1.0):
    """|got - ref| <= ulps * bf16 spacing at ref (one rounding of an exact value)."""
    got = fb(got_bits).astype(np.float64)
    spacing = np.maximum(np.abs(ref64), 1e-30) * 2.0**-8
    return np.all(np.abs(got - ref64) <= ulps * spacing)


def test_argmax_full_vocab_kat():
    n = 248320
    v = (np.sin(np.arange(n, dtype=np.float32) * np.float32(0.00137)) * np.float32(0.9)).astype(np.float32)
    v[123456] = 42.0
    assert orc.argmax(v) == 123456


def test_argmax_tail_kat():
    v = (np.cos(np.arange(1000, dtype=np.float32) * np.float32(0.0137)) * np.float32(0.5)).astype(np.float32)
    v[999] = 3.5
    assert orc.argmax(v) == 999


def test_argmax_ties_lowest_index():
    v = np.zeros(5000, np.float32)
    v[[17, 400, 4999]] = 7.0
    assert orc.argmax(v) == 17


def test_embed_row():
    rng = np.random.default_rng(1)
    vocab, hidden = 64, 5120
    w = rng.integers(0, 2**32, size=(vocab, hidden // 8), dtype=np.uint64).astype(np.uint32)
    s = bf(rng.uniform(0.005, 0.02, (vocab, hidden // 64)))
    b = bf(rng.uniform(-0.1, 0.1, (vocab, hidden // 64)))
    tok = 37
    got = orc.embed(w, s, b, tok, hidden)
    q = ((w[tok][:, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(-1).astype(np.float64)
    ref = q * np.repeat(fb(s[tok]), 64) + np.repeat(fb(b[tok]), 64)
    assert within_bf16(got, ref, 1.0)


def test_residual_add():
    rng = np.random.default_rng(2)
    x = bf(rng.standard_normal(5120) * 4)
    o = (rng.standard_normal(5120) * 2).astype(np.float32)
    ref = fb(x).astype(np.float64) + fb(bf(o)).astype(np.float64)
    assert within_bf16(orc.residual(x, o), ref, 1.0)


def test_silu_mul():
    rng = np.random.default_rng(3)
    g = (rng.standard_normal(17408) * 3).astype(np.float32)
    u = (rng.standard_normal(17408) * 3).astype(np.float32)
    gb, ub = fb(bf(g)).astype(np.float64), fb(bf(u)).astype(np.float64)
    ref = gb / (1.0 + np.exp(-gb)) * ub
    assert within_bf16(orc.silu_mul(g, u), ref, 1.01)


def test_gdn_gated_norm():
    """gated = bf16(bf16(y * rsqrt(mean(y^2) + eps) * w) * silu(bf16(z))) per value head."""
    rng = np.random.default_rng(4)
    VH, HD = 48, 128
    co = fb(bf(rng.standard_normal((1, 10240)))).astype(np.float32)
    z = (rng.standard_normal((1, VH * HD)) * 2).astype(np.float32)
    a = rng.standard_normal((1, VH)).astype(np.float32)
    b = rng.standard_normal((1, VH)).astype(np.float32)
    a_log, dt_bias, norm_w = bf(rng.uniform(-2, 0, VH)), bf(rng.uniform(-1, 1, VH)), bf(rng.uniform(0.9, 1.1, HD))
    s0 = (rng.standard_normal(VH * HD * HD) * 0.01).astype(np.float32)
    gated, _, y, _ = orc.gdn_recurrence(co, z, a, b, a_log, dt_bias, norm_w, s0, 1)
    y = y.reshape(VH, HD).astype(np.float64)
    n = y / np.sqrt(np.mean(y**2, axis=1, keepdims=True) + 1e-6) * fb(norm_w)
    n = fb(bf(n)).astype(np.float64)
    zz = fb(bf(z)).reshape(VH, HD).astype(np.float64)
    ref = n * zz / (1.0 + np.exp(-zz))
    got = fb(gated.reshape(VH, HD)).astype(np.float64)
    # n itself may sit one bf16 step away from the double-precision value
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-7 + np.abs(zz) * np.abs(n) * 2.0**-8 + 1e-30)


def test_attention_output_gate():
    """gated = bf16(sdpa(q, K, V) * sigmoid(bf16(gate))) with q/k normed and rotated."""
    rng = np.random.default_rng(5)
    cap, base = 80, 70
    q_proj = (rng.standard_normal((1, 12288)) * 2).astype(np.float32)
    k_raw = rng.standard_normal((1, 1024)).astype(np.float32)
    v_raw = rng.standard_normal((1, 1024)).astype(np.float32)
    qn, kn = bf(rng.uniform(0.9, 1.1, 256)), bf(rng.uniform(0.9, 1.1, 256))
    kc = bf(rng.standard_normal(4 * cap * 256))
    vc = bf(rng.standard_normal(4 * cap * 256))
    gated, kc2, vc2 = orc.attention(q_proj, k_raw, v_raw, qn, kn, kc, vc, cap, base, 1)
    # the new row was appended at position base
    for h in range(4):
        off = (h * cap + base) * 256
        assert np.array_equal(kc2[off:off + 256], orc.head_norm_rope(k_raw[0, h * 256:(h + 1) * 256], kn, base))
        assert np.array_equal(vc2[off:off + 256], bf(v_raw[0, h * 256:(h + 1) * 256]))
    query = np.concatenate([orc.head_norm_rope(q_proj[0, h * 512:h * 512 + 256], qn, base) for h in range(24)])
    o = orc.sdpa(query, kc2, vc2, cap, base, 1)[0].reshape(-1).astype(np.float64)
    g = np.concatenate([fb(bf(q_proj[0, h * 512 + 256:(h + 1) * 512])) for h in range(24)]).astype(np.float64)
    ref = o / (1.0 + np.exp(-g))
    assert within_bf16(gated[0], ref, 1.01)
