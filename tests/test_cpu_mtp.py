"""CPU pins of the oracle's MTP drafter step (orc_mtp_forward), which the GPU
drafter is compared with bit for bit.

The reference's drafter step (MtpRunner::forward_position_decode_device,
src/model/runner.rs:2711-2765) is: embed(token) -> RMSNorm(pre_fc_norm_embedding)
and RMSNorm(pre_fc_norm_hidden)(cond) into the contiguous fc input
[pre_fc | pre_fc_hidden] (runner.rs:2287-2291) -> q4 fc (5120 x 10240) ->
f32_to_bf16 -> one attention block on the drafter's own KV cache and one MLP,
each with its residual -> final norm -> the target's lm_head -> argmax.

Pins:
* the wiring of the fc input: zero scales and biases over the embedding half
  of fc make the step independent of the token; over the hidden half,
  independent of the conditioning hidden;
* the whole step composed here from the oracle's separately pinned kernel
  functions (embedding, RMSNorm, q4 linear, attention, residual, SwiGLU,
  argmax) in the reference's order equals orc_mtp_forward bit for bit, so a
  wrong norm gain, a dropped residual or a swapped half fails.
"""
import numpy as np
import pytest

from _lisa import load_oracle

orc = load_oracle()
H = 5120
LAYERS, VOCAB, CAP, SEED = 4, 2048, 64, 0x3171


def model():
    return orc.Model(LAYERS, VOCAB, CAP, SEED, with_mtp=True)


def mtp(m, kind, part=0, dtype=np.uint16):
    return m.tensor(orc.SCOPE_MTP, orc.T[kind], part, dtype)


def cond_row(seed):
    rng = np.random.default_rng(seed)
    return orc.f32_to_bf16_bits(rng.standard_normal(H).astype(np.float32))


def zero_fc_half(m, half):
    """fc is q4 [5120][10240]: groups 0..79 of a row read the embedding half,
    80..159 the hidden half; zero scale and bias make those weights 0."""
    s = mtp(m, "MTP_FC", 1).reshape(H, 160)
    b = mtp(m, "MTP_FC", 2).reshape(H, 160)
    sl = slice(0, 80) if half == 0 else slice(80, 160)
    s[:, sl] = 0
    b[:, sl] = 0


def step(m, token, cond):
    am, xn = m.mtp_forward(token, cond)
    m.mtp_trim(1)  # the next call runs at the same position on the same cache
    return am, xn


def test_embedding_half_zeroed_makes_step_token_independent():
    m = model()
    try:
        c = cond_row(1)
        a0, x0 = step(m, 3, c)
        a1, x1 = step(m, 1777, c)
        assert not np.array_equal(x0, x1)  # the token matters with the real weights
        zero_fc_half(m, 0)
        b0, y0 = step(m, 3, c)
        b1, y1 = step(m, 1777, c)
        assert b0 == b1 and np.array_equal(y0, y1)
        # and the conditioning hidden still matters
        _, y2 = step(m, 3, cond_row(2))
        assert not np.array_equal(y0, y2)
    finally:
        m.close()


def test_hidden_half_zeroed_makes_step_cond_independent():
    m = model()
    try:
        a0, x0 = step(m, 11, cond_row(3))
        a1, x1 = step(m, 11, cond_row(4))
        assert not np.array_equal(x0, x1)
        zero_fc_half(m, 1)
        b0, y0 = step(m, 11, cond_row(3))
        b1, y1 = step(m, 11, cond_row(4))
        assert b0 == b1 and np.array_equal(y0, y1)
        _, y2 = step(m, 12, cond_row(3))
        assert not np.array_equal(y0, y2)
    finally:
        m.close()


def compose_step(m, token, cond, position):
    """runner.rs:2711-2765 from the kernel functions, in the reference's order.
    The norms after a residual add sum their statistic from 8-row tile
    partials (the decode kernels' order, pinned in test_cpu_elementwise)."""
    emb = [m.tensor(0, orc.T["EMBED"], p, d) for p, d in ((0, np.uint32), (1, np.uint16), (2, np.uint16))]
    head = [m.tensor(0, orc.T["LM_HEAD"], p, d) for p, d in ((0, np.uint32), (1, np.uint16), (2, np.uint16))]

    def q4(kind, x, n, k, ksplit):
        w, s, b = mtp(m, kind, 0, np.uint32), mtp(m, kind, 1), mtp(m, kind, 2)
        return orc.q4_linear(x, w, s, b, n, k, 1, ksplit)[0]

    e = orc.embed(*emb, token)
    pre_fc = orc.rms_norm(e, mtp(m, "MTP_PRE_FC_EMB"))
    pre_fc_hidden = orc.rms_norm(cond, mtp(m, "MTP_PRE_FC_HID"))
    fc_in = np.concatenate([pre_fc, pre_fc_hidden])          # [pre_fc | pre_fc_hidden]
    fc_out = q4("MTP_FC", fc_in, H, 2 * H, 4)
    hidden = orc.f32_to_bf16_bits(fc_out)                     # encode_cast (f32_to_bf16, RNE)
    normalized = orc.rms_norm(hidden, mtp(m, "INPUT_NORM"))
    qp = q4("ATT_Q", normalized, 12288, H, 1)
    kr = q4("ATT_K", normalized, 1024, H, 1)
    vr = q4("ATT_V", normalized, 1024, H, 1)
    kc = mtp(m, "KEY_CACHE").copy()
    vc = mtp(m, "VALUE_CACHE").copy()
    gated, _, _ = orc.attention(qp, kr, vr, mtp(m, "ATT_Q_NORM"), mtp(m, "ATT_K_NORM"), kc, vc, CAP, position, 1)
    branch = q4("ATT_O", gated[0], H, 6144, 4)
    residual = orc.residual(hidden, branch)
    post = orc.rms_norm_tiles(residual, mtp(m, "POST_NORM"))
    g = q4("MLP_GATE", post, 17408, H, 1)
    u = q4("MLP_UP", post, 17408, H, 1)
    act = orc.silu_mul(g, u)
    down = q4("MLP_DOWN", act, H, 17408, 4)
    hidden2 = orc.residual(residual, down)
    final = orc.rms_norm_tiles(hidden2, mtp(m, "FINAL_NORM"))
    logits = orc.q4_linear(final, head[0], head[1], head[2], VOCAB, H, 1, 1)[0]
    return orc.argmax(logits), final


@pytest.mark.parametrize("position", [0, 5])
def test_step_equals_composition_of_kernel_functions(position):
    m = model()
    try:
        m.fill_state(position, 99)  # drafter KV rows [0, position) N(0, 1)
        c = cond_row(7)
        want_am, want_x = compose_step(m, 1234, c, position)
        am, xn = m.mtp_forward(1234, c)
        assert m.mtp_position == position + 1
        assert am == want_am
        assert np.array_equal(xn, want_x)
    finally:
        m.close()


def test_batched_drafter_agrees_with_sequential_steps():
    """MtpRunner::forward_position_batch (runner.rs:3486-3581) against the same
    positions one M=1 step at a time (forward_position_decode, :2618-2680):
    the batch rounds every dequantized weight to bf16 (gemm.metal:246-250), so
    the rows agree within that rounding; the argmax agrees at most positions."""
    rng = np.random.default_rng(12)
    n = 6
    tokens = rng.integers(0, VOCAB, n).astype(np.uint32)
    hiddens = rng.standard_normal((n, H)).astype(np.float32)
    m = model()
    try:
        m.fill_state(9, 99)
        bam, bxn = m.mtp_prefill(tokens, hiddens)
        assert m.mtp_position == 9 + n
        m.fill_state(9, 99)
        seq = [m.mtp_forward(int(tokens[t]), orc.f32_to_bf16_trunc(hiddens[t])) for t in range(n)]
    finally:
        m.close()
    sam = np.array([s[0] for s in seq])
    sxn = orc.bf16_bits_to_f32(np.stack([s[1] for s in seq])).astype(np.float64)
    bx = orc.bf16_bits_to_f32(bxn).astype(np.float64)
    assert np.mean(bam == sam) >= 5 / 6
    rel = np.sqrt(np.mean((bx - sxn) ** 2) / np.mean(sxn ** 2))
    assert 0 < rel < 2e-2, rel


def test_batched_drafter_wiring_of_fc_halves():
    """The batch builds the fc input as [pre_fc | pre_fc_hidden] too: with the
    embedding half of fc zeroed its rows do not depend on the tokens."""
    rng = np.random.default_rng(13)
    hiddens = rng.standard_normal((4, H)).astype(np.float32)
    m = model()
    try:
        zero_fc_half(m, 0)
        a0, x0 = m.mtp_prefill(np.array([1, 2, 3, 4], np.uint32), hiddens)
        m.mtp_trim(4)
        a1, x1 = m.mtp_prefill(np.array([900, 800, 700, 600], np.uint32), hiddens)
        assert np.array_equal(a0, a1) and np.array_equal(x0, x1)
    finally:
        m.close()
