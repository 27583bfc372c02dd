"""CPU pins of the oracle's gated-delta-net step.

Conv history: the reference's known-answer shift test (tests/gdn_state.rs:7-92)
for steps {1, 2, 3, 16} with its inputs, plus the conv itself against double
precision. Recurrence: the reference's invariant that a batched multi-step
call equals the same steps one at a time (tests/gdn_recurrence_state.rs:
70-173), and closed forms of the delta rule: with decay 1, beta 1 and one-hot
keys the state column of the key is overwritten by the value exactly; with a
zero key the state is only decayed.
"""
import numpy as np
import pytest

from _lisa import load_oracle

orc = load_oracle()
CONV, VH, HD, KEY = 10240, 48, 128, 2048


def bf(x):
    return orc.f32_to_bf16_bits(np.asarray(x, np.float32))


def fb(h):
    return orc.bf16_bits_to_f32(h)


@pytest.mark.parametrize("steps", [1, 2, 3, 16])
def test_conv_history_shift_kat(steps):
    """tests/gdn_state.rs:13-92: qkv = 10 + i*1e-4, old history = -3 + i*1e-4
    (stored with the host's truncating conversion); the new history is the
    last three of [old; RNE(qkv rows)]."""
    qkv = (10.0 + np.arange(steps * CONV, dtype=np.float64) * 0.0001).astype(np.float32).reshape(steps, CONV)
    old = (-3.0 + np.arange(3 * CONV, dtype=np.float64) * 0.0001).astype(np.float32)
    state = orc.f32_to_bf16_trunc(old)
    conv_w = bf(np.zeros(CONV * 4))
    _, new_state, _ = orc.gdn_conv(qkv, conv_w, state, steps)
    new_state = new_state.reshape(3, CONV)
    for slot in range(3):
        src = steps + slot
        for ch in (0, 17, CONV - 1):
            if src < 3:
                want = fb(orc.f32_to_bf16_trunc(old[src * CONV + ch]))
            else:
                want = fb(bf(qkv[src - 3, ch]))
            assert fb(new_state[slot, ch]) == want, (steps, slot, ch)


def test_conv_output_matches_double():
    """gdn.metal:163-170: out = bf16(silu(bf16(sum_tap hist * w)))."""
    rng = np.random.default_rng(8)
    m = 3
    qkv = rng.standard_normal((m, CONV)).astype(np.float32)
    conv_w = bf(rng.uniform(-0.5, 0.5, CONV * 4))
    state = bf(rng.standard_normal(3 * CONV))
    out, _, slots = orc.gdn_conv(qkv, conv_w, state, m, slots=True)
    hist = np.concatenate([fb(state).reshape(3, CONV), fb(bf(qkv))], axis=0).astype(np.float64)
    w = fb(conv_w).reshape(CONV, 4).astype(np.float64)
    for t in range(m):
        acc = sum(hist[t + tap] * w[:, tap] for tap in range(4))
        conv = fb(bf(acc))
        ref = conv / (1.0 + np.exp(-conv.astype(np.float64)))
        assert np.all(np.abs(out[t] - ref) <= np.abs(ref) * 2.0**-7 + 1e-6)
        # slot t holds the history after step t (rollback capture)
        assert np.array_equal(slots.reshape(m, 3, CONV)[t], bf(hist[t + 1:t + 4]))


def gdn_inputs(rng, m):
    conv_out = fb(bf(rng.standard_normal((m, CONV)))).astype(np.float32)
    z = rng.standard_normal((m, VH * HD)).astype(np.float32)
    a = rng.standard_normal((m, VH)).astype(np.float32)
    b = rng.standard_normal((m, VH)).astype(np.float32)
    a_log = bf(rng.uniform(-2.0, 0.0, VH))
    dt_bias = bf(rng.uniform(-1.0, 1.0, VH))
    norm_w = bf(rng.uniform(0.9, 1.1, HD))
    return conv_out, z, a, b, a_log, dt_bias, norm_w


def test_recurrence_batch_equals_single_steps():
    """tests/gdn_recurrence_state.rs:70-173: 16 steps in one call equal 16
    calls of one step, bit-exact for outputs and state."""
    rng = np.random.default_rng(16)
    m = 16
    co, z, a, b, alog, dtb, nw = gdn_inputs(rng, m)
    s0 = (rng.standard_normal(VH * HD * HD) * 0.01).astype(np.float32)
    g_all, s_all, y_all, _ = orc.gdn_recurrence(co, z, a, b, alog, dtb, nw, s0, m)
    s = s0
    for t in range(m):
        g, s, y, _ = orc.gdn_recurrence(co[t:t + 1], z[t:t + 1], a[t:t + 1], b[t:t + 1], alog, dtb, nw, s, 1)
        assert np.array_equal(g[0], g_all[t])
        assert np.array_equal(y[0].view(np.uint32), y_all[t].view(np.uint32))
    assert np.array_equal(s.view(np.uint32), s_all.view(np.uint32))


def delta_inputs(keys, values, query):
    """Rows t: one-hot key keys[t] for every key head, value values[t][h][v],
    one-hot query; gates chosen so decay == 1 and beta == 1."""
    m = len(keys)
    co = np.zeros((m, CONV), np.float32)
    for t in range(m):
        for kh in range(16):
            co[t, kh * HD + query] = 1.0
            co[t, KEY + kh * HD + keys[t]] = 1.0
        co[t, 2 * KEY:] = values[t].reshape(-1)
    z = np.ones((m, VH * HD), np.float32)
    a = np.zeros((m, VH), np.float32)
    b = np.full((m, VH), 100.0, np.float32)       # sigmoid -> 1
    a_log = bf(np.full(VH, -100.0))               # exp(-exp(-100) * dt) -> 1
    dt_bias = bf(np.zeros(VH))
    norm_w = bf(np.ones(HD))
    return co, z, a, b, a_log, dt_bias, norm_w


def test_delta_rule_one_hot_overwrite():
    rng = np.random.default_rng(21)
    # values with few significant bits so differences are exact
    vals = (rng.integers(-64, 64, size=(3, VH, HD)) / 8.0).astype(np.float32)
    keys = [5, 77, 5]
    co, z, a, b, alog, dtb, nw = delta_inputs(keys, vals, query=5)
    s0 = np.zeros(VH * HD * HD, np.float32)
    _, s, y, slots = orc.gdn_recurrence(co, z, a, b, alog, dtb, nw, s0, 3, slots=True)
    S = slots.reshape(3, VH, HD, HD)
    # step 0: column 5 <- v0, nothing else
    assert np.array_equal(S[0][:, :, 5], vals[0])
    assert np.count_nonzero(S[0]) == np.count_nonzero(vals[0])
    # step 1: column 77 <- v1, column 5 untouched
    assert np.array_equal(S[1][:, :, 77], vals[1])
    assert np.array_equal(S[1][:, :, 5], vals[0])
    # step 2: key 5 again: column 5 overwritten by v2
    assert np.array_equal(S[2][:, :, 5], vals[2])
    assert np.array_equal(S[2][:, :, 77], vals[1])
    assert np.array_equal(s.reshape(VH, HD, HD), S[2])
    # the query reads column 5 scaled by the normalized one-hot query,
    # 1/sqrt(128) up to two bf16 roundings
    qv = 1.0 / np.sqrt(128.0)
    for t, col in ((0, vals[0]), (1, vals[0]), (2, vals[2])):
        ref = col.reshape(-1) * qv
        assert np.all(np.abs(y[t] - ref) <= np.abs(ref) * 2.0**-7)


def test_zero_key_only_decays():
    """k = 0: the update term vanishes and S' = S * exp(-exp(A_log) * softplus(a + dt_bias))."""
    rng = np.random.default_rng(33)
    co, z, a, b, alog, dtb, nw = gdn_inputs(rng, 1)
    co[0, KEY:2 * KEY] = 0.0
    s0 = (rng.standard_normal(VH * HD * HD) * 0.01).astype(np.float32)
    _, s1, _, _ = orc.gdn_recurrence(co, z, a, b, alog, dtb, nw, s0, 1)
    arg = fb(bf(fb(bf(a[0])) + fb(dtb))).astype(np.float64)
    dt = fb(bf(np.where(arg > 20, arg, np.log1p(np.exp(arg)))))
    decay = np.exp(-np.exp(fb(alog).astype(np.float64)) * dt)
    want = s0.reshape(VH, -1).astype(np.float64) * decay[:, None]
    got = s1.reshape(VH, -1)
    assert np.all(np.abs(got - want) <= np.abs(want) * 4e-7 + 1e-30)


def test_value_heads_read_their_key_head():
    """gdn.metal:271: value head h reads key head h / 3 (value heads 3j, 3j+1,
    3j+2 share key head j). Every key head gets a different one-hot key
    column, so a wrong grouping (h % 16, or h / 3 of the wrong operand) writes
    another column; decay 1, beta 1 and a zero state make the update exact."""
    rng = np.random.default_rng(45)
    vals = (rng.integers(-64, 64, size=(1, VH, HD)) / 8.0).astype(np.float32)
    cols = [(7 * kh + 3) % HD for kh in range(16)]
    co, z, a, b, alog, dtb, nw = delta_inputs([0], vals, query=0)
    co[0, :2 * KEY] = 0.0
    for kh in range(16):
        co[0, kh * HD + cols[kh]] = 1.0            # query of key head kh
        co[0, KEY + kh * HD + cols[kh]] = 1.0      # key of key head kh
    s0 = np.zeros(VH * HD * HD, np.float32)
    _, s, y, _ = orc.gdn_recurrence(co, z, a, b, alog, dtb, nw, s0, 1)
    S = s.reshape(VH, HD, HD)
    for h in range(VH):
        col = cols[h // 3]
        assert np.array_equal(S[h][:, col], vals[0, h]), h
        assert np.count_nonzero(S[h]) == np.count_nonzero(vals[0, h]), h
        # the readout of head h uses the same key head's query
        ref = vals[0, h] / np.sqrt(128.0)
        assert np.all(np.abs(y[0, h * HD:(h + 1) * HD] - ref) <= np.abs(ref) * 2.0**-7), h


def test_beta_gate_against_double():
    """gdn.metal:196-204: beta = bf16(sigmoid(bf16 b)) at non-saturated b.
    From a zero state with decay 1 and a one-hot key, one step writes
    beta * v into the key's column, so the column pins beta (and its sign:
    sigmoid(-b) or 1 - beta would fail) against float64."""
    rng = np.random.default_rng(46)
    vals = (rng.integers(1, 64, size=(1, VH, HD)) / 8.0).astype(np.float32)
    co, z, a, b, alog, dtb, nw = delta_inputs([9], vals, query=9)
    b[0] = rng.uniform(-4.0, 4.0, VH).astype(np.float32)
    s0 = np.zeros(VH * HD * HD, np.float32)
    _, s, _, _ = orc.gdn_recurrence(co, z, a, b, alog, dtb, nw, s0, 1)
    S = s.reshape(VH, HD, HD)
    bb = fb(bf(b[0])).astype(np.float64)
    beta = 1.0 / (1.0 + np.exp(-bb))
    for h in range(VH):
        want = vals[0, h].astype(np.float64) * beta[h]
        got = S[h][:, 9].astype(np.float64)
        # beta is rounded to bf16 (relative 2^-9) and the product to f32
        assert np.all(np.abs(got - want) <= np.abs(want) * 2.0**-8), (h, b[0, h])
    assert np.unique(np.round(beta, 3)).size > 20  # the gates really span (0, 1)
