"""The drafter's prompt side on the GPU against the CPU oracle (reduced-depth
model, real layer shapes): the host-hidden drafter step
(forward_position_decode, runner.rs:2618-2680) bit-exact; the batched drafter
(forward_position_batch, runner.rs:3486-3581) within the prefill GEMM's
tolerance; the (buffer, offset) addressing of forward_position_decode_device;
and prefill_prompt_from (speculative/mod.rs:237-311) against the same
orchestration composed from the oracle's target prefill and drafter batch,
followed by speculative decoding that emits the oracle's greedy stream."""
import numpy as np
import pytest

from _lisa import load_oracle, load_pkg

pytestmark = pytest.mark.gpu

LAYERS, VOCAB, CAP, SEED, CTX_SEED = 4, 4096, 512, 0x6D7, 0xC0DE


@pytest.fixture(scope="module")
def pair():
    pkg, orc = load_pkg(), load_oracle()
    r = pkg.Runner(layers=LAYERS, vocab=VOCAB, capacity=CAP, seed=SEED, with_mtp=True, use_graph=True)
    m = orc.Model(LAYERS, VOCAB, CAP, SEED, with_mtp=True)
    yield pkg, orc, r, m
    r.close()
    m.close()


def test_host_hidden_drafter_step_bit_exact(pair):
    pkg, orc, r, m = pair
    r.fill_state(33, CTX_SEED)
    m.fill_state(33, CTX_SEED)
    rng = np.random.default_rng(3)
    for tok in (5, 4000):
        h = rng.standard_normal(5120).astype(np.float32)
        am, xn = r.mtp_forward_position_decode(tok, h)
        wam, wxn = m.mtp_forward(tok, orc.f32_to_bf16_trunc(h))
        assert am == wam
        assert np.array_equal(xn, orc.bf16_bits_to_f32(wxn))
    assert r.mtp_position == m.mtp_position == 35


def test_reset_halves_are_independent(pair):
    """QwenRunner::reset_state (runner.rs:423-444) clears the target only and
    MtpRunner::reset_state (runner.rs:2508-2520) the drafter only, as
    src/cli/run.rs:74-82 and src/serve/mod.rs:209-234 call them."""
    pkg, orc, r, m = pair
    rng = np.random.default_rng(21)
    r.fill_state(33, CTX_SEED)
    m.fill_state(33, CTX_SEED)
    r.reset_state()
    assert (r.position, r.mtp_position) == (0, 33)
    # the drafter's K/V survived the target reset: its step attends rows 0..33
    h = rng.standard_normal(5120).astype(np.float32)
    am, xn = r.mtp_forward_position_decode(41, h)
    wam, wxn = m.mtp_forward(41, orc.f32_to_bf16_trunc(h))
    assert am == wam and np.array_equal(xn, orc.bf16_bits_to_f32(wxn))
    # the target restarts from zero state at position 0
    m.reset()
    tam, thid = r.forward_token_decode(7, want_hidden=True)
    wtam, wthid = m.forward([7])
    assert tam == int(wtam[0]) and np.array_equal(thid.view(np.uint32), wthid[0].view(np.uint32))
    assert (r.position, r.mtp_position) == (1, 34)
    r.mtp_reset_state()
    assert (r.position, r.mtp_position) == (1, 0)
    # the drafter restarts at position 0 (the oracle's drafter is at 0 after reset)
    h = rng.standard_normal(5120).astype(np.float32)
    am, xn = r.mtp_forward_position_decode(9, h)
    wam, wxn = m.mtp_forward(9, orc.f32_to_bf16_trunc(h))
    assert am == wam and np.array_equal(xn, orc.bf16_bits_to_f32(wxn))
    # and the target kept its state and position through the drafter reset
    tam, thid = r.forward_token_decode(8, want_hidden=True)
    wtam, wthid = m.forward([8])
    assert tam == int(wtam[0]) and np.array_equal(thid.view(np.uint32), wthid[0].view(np.uint32))
    assert (r.position, r.mtp_position, m.position, m.mtp_position) == (2, 1, 2, 1)


def test_device_addressing_equals_row_selection(pair):
    pkg, orc, r, m = pair
    r.fill_state(20, CTX_SEED)
    toks = [11, 22, 33]
    r.verify_block3(toks)  # target hidden rows 0..2 on the device
    r.commit_verified_prefix(3)
    ck = r.mtp_checkpoint_state()
    a = [r.mtp_forward(7, 0, row) for row in range(3)]
    a.append(r.mtp_forward(8, 1))
    xa = r.mtp_normalized()
    r.mtp_restore_state(ck)
    b = [r.mtp_forward_device(7, True, pkg.hidden_offset(row))[0] for row in range(3)]
    am, off = r.mtp_forward_device(8, False, pkg.normalized_offset())
    b.append(am)
    assert off == pkg.normalized_offset()
    assert a == b
    assert np.array_equal(r.mtp_normalized(), xa)
    r.free_mtp_checkpoint(ck)


@pytest.mark.parametrize("n,chunk", [(7, 0), (40, 16)])
def test_batched_drafter_matches_oracle(pair, n, chunk):
    pkg, orc, r, m = pair
    r.fill_state(30, CTX_SEED)
    m.fill_state(30, CTX_SEED)
    rng = np.random.default_rng(n)
    tokens = rng.integers(0, VOCAB, n).astype(np.uint32)
    hiddens = rng.standard_normal((n, 5120)).astype(np.float32)
    am, xn = r.mtp_forward_batch(tokens, hiddens, chunk=chunk)
    assert r.mtp_position == 30 + n
    wam, wxn = m.mtp_prefill(tokens, hiddens)
    w = orc.bf16_bits_to_f32(wxn).astype(np.float64)
    rel = np.sqrt(np.mean((xn - w) ** 2) / np.mean(w ** 2))
    assert rel < 1e-2, rel
    assert np.mean(am == wam) >= 0.9
    # and chunk-size invariant on the GPU
    r.fill_state(30, CTX_SEED)
    am2, xn2 = r.mtp_forward_batch(tokens, hiddens, chunk=5)
    assert np.array_equal(am, am2) and np.array_equal(xn.view(np.uint32), xn2.view(np.uint32))


def test_prefill_prompt_then_speculation(pair):
    pkg, orc, r, m = pair
    rng = np.random.default_rng(77)
    prompt = rng.integers(0, VOCAB, 24).astype(np.uint32)
    r.reset_state()
    r.mtp_reset_state()
    bonus, th, (seed_tok, seed_h) = r.prefill_prompt(prompt)
    assert r.position == r.mtp_position == len(prompt)
    # the same orchestration from the oracle's pieces
    m.reset()
    wam, wh = m.prefill(prompt, want_hidden=True)
    wb = int(wam[-1])
    mtoks = np.concatenate([prompt[1:], [wb]]).astype(np.uint32)
    mam, mxn = m.mtp_prefill(mtoks, wh)
    assert bonus == wb
    rel = np.sqrt(np.mean((th - wh[-1]) ** 2) / np.mean(wh[-1] ** 2))
    assert rel < 1e-2, rel
    assert seed_tok == int(mam[-1])
    # the drafter reads the target's prefill rows, which already carry the
    # GEMM summation-order difference above, through fc and one more layer
    ws = orc.bf16_bits_to_f32(mxn[-1]).astype(np.float64)
    assert np.sqrt(np.mean((seed_h - ws) ** 2) / np.mean(ws ** 2)) < 3e-2
    # short prompts take the M=1 path (fewer than 4 tokens)
    r.reset_state()
    r.mtp_reset_state()
    b3, th3, (s3, sh3) = r.prefill_prompt(prompt[:3])
    m.reset()
    seq = [m.forward([int(t)]) for t in prompt[:3]]
    assert b3 == int(seq[-1][0][0])
    assert np.array_equal(th3.view(np.uint32), seq[-1][1][0].view(np.uint32))
    # speculative decoding from the prompt state emits the target's greedy stream
    r.reset_state()
    r.mtp_reset_state()
    bonus, th, (seed_tok, seed_h) = r.prefill_prompt(prompt)
    ck = r.checkpoint_state()
    mck = r.mtp_checkpoint_state()
    truth = [bonus] + list(r.decode_greedy(bonus, 19))
    r.restore_state(ck)
    r.mtp_restore_state(mck)
    toks, st = r.generate_greedy_block3(bonus, th, seed_tok, seed_h, 20)
    assert [int(t) for t in toks] == truth
    r.free_checkpoint(ck)
    r.free_mtp_checkpoint(mck)
