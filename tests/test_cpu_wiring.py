"""CPU pin of the target model's layer wiring in the oracle (orc_model_forward,
which the GPU decode step is compared with bit for bit).

The reference's M=1 step (QwenRunner::forward_token_decode,
src/model/runner.rs:555-591) is: embed -> for each layer: RMSNorm(input_norm)
-> the branch (GDN, runner.rs:1276-1425: qkv/z/a/b projections, causal conv,
gated-delta recurrence with the gated RMSNorm, out_proj; or attention,
runner.rs:1426-1592: q/k/v projections, head norms + RoPE + KV append, split-K
SDPA with the output gate, o_proj) -> residual -> RMSNorm(post_norm) -> MLP
(gate, up, SwiGLU, down, runner.rs:1248-1275) -> residual; then
RMSNorm(final_norm) -> lm_head -> argmax.

Here the step of a 4-layer model (GDN, GDN, GDN, attention) is composed from
the oracle's separately pinned kernel functions in that order and must equal
orc_model_forward bit for bit: its hidden after every layer stack, its
recurrent state, its conv history, its K/V append and its argmax. A swapped
norm gain, a dropped residual, the wrong state slice or the wrong projection
fails it, whichever recipe it hides in, because the composition shares no code
with orc_model_forward above the kernel functions.
"""
import numpy as np
import pytest

from _lisa import load_oracle

orc = load_oracle()
H = 5120
LAYERS, VOCAB, CAP, SEED = 4, 2048, 64, 0x51A7


def layer_t(m, layer, kind, part=0, dtype=np.uint16):
    return m.tensor(layer + 1, orc.T[kind], part, dtype)


def q4(m, layer, kind, x, n, k):
    """A q4 projection of the layer; the K split of the decode launches (one
    wave per tile at K = 5120, four waves per tile otherwise)."""
    w = layer_t(m, layer, kind, 0, np.uint32)
    s, b = layer_t(m, layer, kind, 1), layer_t(m, layer, kind, 2)
    return orc.q4_linear(x, w, s, b, n, k, 1, 1 if k == H else 4)[0]


def compose_step(m, token, position):
    """runner.rs:555-591 with the oracle's kernel functions. Returns the argmax,
    the hidden (bf16 bits) after the layer stack, and each layer's new state."""
    g = [m.tensor(0, orc.T["EMBED"], p, d) for p, d in ((0, np.uint32), (1, np.uint16), (2, np.uint16))]
    head = [m.tensor(0, orc.T["LM_HEAD"], p, d) for p, d in ((0, np.uint32), (1, np.uint16), (2, np.uint16))]
    hidden = orc.embed(*g, token)
    states = []
    for i in range(LAYERS):
        # the first layer's norm sums its statistic over 8-element chunks of
        # the embedding, every later one over 8-row tiles of the residual
        # (the decode kernels' order; both pinned in test_cpu_elementwise)
        norm = orc.rms_norm if i == 0 else orc.rms_norm_tiles
        x = norm(hidden, layer_t(m, i, "INPUT_NORM"))
        if not orc.layer_is_attention(i):
            qkv = q4(m, i, "GDN_QKV", x, 10240, H)
            z = q4(m, i, "GDN_Z", x, 6144, H)
            a = q4(m, i, "GDN_A", x, 48, H)
            b = q4(m, i, "GDN_B", x, 48, H)
            conv_out, conv_state, _ = orc.gdn_conv(qkv, layer_t(m, i, "GDN_CONV_W"),
                                                   layer_t(m, i, "CONV_STATE"), 1)
            gated, state, _, _ = orc.gdn_recurrence(conv_out, z, a, b, layer_t(m, i, "GDN_A_LOG"),
                                                    layer_t(m, i, "GDN_DT_BIAS"), layer_t(m, i, "GDN_NORM"),
                                                    layer_t(m, i, "GDN_STATE", 0, np.float32), 1)
            branch = q4(m, i, "GDN_OUT", gated[0], H, 6144)
            states.append((state, conv_state))
        else:
            qp = q4(m, i, "ATT_Q", x, 12288, H)
            kr = q4(m, i, "ATT_K", x, 1024, H)
            vr = q4(m, i, "ATT_V", x, 1024, H)
            gated, kc, vc = orc.attention(qp, kr, vr, layer_t(m, i, "ATT_Q_NORM"), layer_t(m, i, "ATT_K_NORM"),
                                          layer_t(m, i, "KEY_CACHE"), layer_t(m, i, "VALUE_CACHE"), CAP,
                                          position, 1)
            branch = q4(m, i, "ATT_O", gated[0], H, 6144)
            states.append((kc, vc))
        residual = orc.residual(hidden, branch)
        post = orc.rms_norm_tiles(residual, layer_t(m, i, "POST_NORM"))
        act = orc.silu_mul(q4(m, i, "MLP_GATE", post, 17408, H), q4(m, i, "MLP_UP", post, 17408, H))
        hidden = orc.residual(residual, q4(m, i, "MLP_DOWN", act, H, 17408))
    final = orc.rms_norm_tiles(hidden, m.tensor(0, orc.T["FINAL_NORM"], 0, np.uint16))
    logits = orc.q4_linear(final, head[0], head[1], head[2], VOCAB, H, 1, 1)[0]
    return orc.argmax(logits), hidden, states


def snapshot(m):
    """Copies of every layer's recurrent state and caches (the composition
    must start from the state the model's own step starts from)."""
    out = []
    for i in range(LAYERS):
        if orc.layer_is_attention(i):
            out.append((layer_t(m, i, "KEY_CACHE").copy(), layer_t(m, i, "VALUE_CACHE").copy()))
        else:
            out.append((layer_t(m, i, "GDN_STATE", 0, np.float32).copy(), layer_t(m, i, "CONV_STATE").copy()))
    return out


@pytest.mark.parametrize("position", [0, 9])
def test_step_equals_composition_of_kernel_functions(position):
    m = orc.Model(LAYERS, VOCAB, CAP, SEED)
    try:
        m.fill_state(position, 0x77)
        before = snapshot(m)
        want_am, want_h, want_states = compose_step(m, 1501, position)
        # the composition read the state without writing it
        assert all(np.array_equal(a, b) for s0, s1 in zip(before, snapshot(m)) for a, b in zip(s0, s1))
        am, hid = m.forward([1501])
        assert m.position == position + 1
        assert int(am[0]) == want_am
        assert np.array_equal(hid[0].view(np.uint32), orc.bf16_bits_to_f32(want_h).view(np.uint32))
        after = snapshot(m)
        for i, (got, want) in enumerate(zip(after, want_states)):
            for a, b in zip(got, want):
                assert np.array_equal(a.view(np.uint8), np.asarray(b).view(np.uint8)), f"layer {i} state"
        # the step changed every layer's state (GDN state and history, the K/V row)
        for i, (b0, a0) in enumerate(zip(before, after)):
            assert not all(np.array_equal(x, y) for x, y in zip(b0, a0)), f"layer {i} state unchanged"
    finally:
        m.close()


def test_composition_detects_a_swapped_norm_gain():
    """The pin is sensitive to the wiring: with layer 1's post_norm gains
    swapped for its input_norm gains the model's step no longer equals the
    composition made from the unswapped gains."""
    m = orc.Model(LAYERS, VOCAB, CAP, SEED)
    try:
        m.fill_state(4, 0x78)
        want_am, want_h, _ = compose_step(m, 77, 4)
        pn, inn = layer_t(m, 1, "POST_NORM"), layer_t(m, 1, "INPUT_NORM")
        saved = pn.copy()
        pn[:] = inn
        _, hid = m.forward([77])
        pn[:] = saved
        assert not np.array_equal(hid[0].view(np.uint32), orc.bf16_bits_to_f32(want_h).view(np.uint32))
    finally:
        m.close()
