"""GPU runner vs the CPU oracle on a reduced-depth model with the real layer
shapes: M=1 greedy decode (graph replay), M=3 verify + rollback, the MTP
drafter, and the speculative loop against sequential greedy decoding."""
import numpy as np
import pytest

from _lisa import load_oracle, load_pkg

pytestmark = pytest.mark.gpu

LAYERS, VOCAB, CAP, SEED, CTX_SEED = 4, 4096, 320, 0x5EED1, 0xC0FFEE


@pytest.fixture(scope="module")
def pair():
    pkg, orc = load_pkg(), load_oracle()
    r = pkg.Runner(layers=LAYERS, vocab=VOCAB, capacity=CAP, seed=SEED, with_mtp=True, use_graph=True)
    m = orc.Model(LAYERS, VOCAB, CAP, SEED, with_mtp=True)
    yield pkg, orc, r, m
    r.close()
    m.close()


def fresh(r, m, filled=64):
    r.fill_state(filled, CTX_SEED)
    m.fill_state(filled, CTX_SEED)
    assert r.position == m.position == filled


def test_decode_matches_oracle(pair):
    pkg, orc, r, m = pair
    fresh(r, m)
    tok = 17
    for _ in range(4):
        am, hid = r.forward_token_decode(tok, want_hidden=True)
        wam, whid = m.forward([tok])
        assert am == int(wam[0])
        assert np.array_equal(hid.view(np.uint32), whid[0].view(np.uint32))
        tok = am
    # device-side greedy loop (hipGraph replays, token fed back on device)
    got = r.decode_greedy(tok, 6)
    want = []
    for _ in range(6):
        wam, _ = m.forward([tok])
        tok = int(wam[0])
        want.append(tok)
    assert list(got) == want
    assert r.position == m.position


def test_logits_match_oracle(pair):
    pkg, orc, r, m = pair
    fresh(r, m, filled=10)
    am, hid, logits = r.forward_token_with_hidden(5)
    wam, whid, wlog = m.forward([5], want_logits=True)
    assert np.array_equal(logits.view(np.uint32), wlog[0].view(np.uint32))
    assert am == orc.argmax(wlog[0]) == int(wam[0])


@pytest.mark.parametrize("rows", [1, 2, 3])
def test_verify_commit_matches_oracle(pair, rows):
    """verify_block3 + commit_verified_prefix (runner.rs:866-944) against the
    oracle, then two more M=1 steps from the rolled-back state."""
    pkg, orc, r, m = pair
    fresh(r, m, filled=62)  # rows cross the 64-token slice boundary
    toks = [101, 2002, 303]
    am, hid = r.verify_block3(toks, want_hidden=True)
    wam, whid = m.forward(toks, capture=True)
    assert list(am) == list(wam)
    assert np.array_equal(hid.view(np.uint32), whid.view(np.uint32))
    r.commit_verified_prefix(rows)
    m.commit(rows)
    assert r.position == m.position == 62 + rows
    tok = int(am[rows - 1])
    for _ in range(2):
        a1, h1 = r.forward_token_decode(tok, want_hidden=True)
        w1, wh1 = m.forward([tok])
        assert a1 == int(w1[0])
        assert np.array_equal(h1.view(np.uint32), wh1[0].view(np.uint32))
        tok = a1


def test_commit_sequence_rotates_state_buffers(pair):
    """A run of verifications with commits of 1, 2, 1, 3, 2, 2 and 1 rows: a
    commit of one or two rows makes that row's slot buffer the live GDN/conv
    state (three rotating buffers, no copy), so the sequence visits every live
    buffer and every graph captured for one; after each commit the next
    verification, then the final M=1 steps, match the oracle bit for bit, and
    so does every GDN layer's state."""
    pkg, orc, r, m = pair
    fresh(r, m, filled=50)
    rng = np.random.default_rng(31)
    for rows in (1, 2, 1, 3, 2, 2, 1):
        toks = [int(t) for t in rng.integers(0, VOCAB, 3)]
        am, hid = r.verify_block3(toks, want_hidden=True)
        wam, whid = m.forward(toks, capture=True)
        assert list(am) == list(wam)
        assert np.array_equal(hid.view(np.uint32), whid.view(np.uint32))
        r.commit_verified_prefix(rows)
        m.commit(rows)
        assert r.position == m.position
    tok = 77
    for _ in range(3):
        a1, h1 = r.forward_token_decode(tok, want_hidden=True)
        w1, wh1 = m.forward([tok])
        assert a1 == int(w1[0]) and np.array_equal(h1.view(np.uint32), wh1[0].view(np.uint32))
        tok = a1
    for idx in range(LAYERS * 3 // 4):  # GDN layer idx is model layer idx + idx // 3
        scope = idx + idx // 3 + 1
        want = m.tensor(scope, orc.T["GDN_STATE"], 0, np.float32)
        assert np.array_equal(r.gdn_state(idx).view(np.uint32), want.view(np.uint32)), idx
        assert np.array_equal(r.conv_state(idx), m.tensor(scope, orc.T["CONV_STATE"], 0, np.uint16)), idx


def test_verify_row_equals_decode(pair):
    """runner_checkpoint.rs invariant: row t of an M=3 verify equals M=1
    decoding of the same tokens (bit-exact here: identical per-row order)."""
    pkg, orc, r, m = pair
    fresh(r, m, filled=40)
    ck = r.checkpoint_state()
    toks = [9, 99, 999]
    am3, h3 = r.verify_block3(toks, want_hidden=True)
    r.commit_verified_prefix(3)
    r.restore_state(ck)
    r.free_checkpoint(ck)
    assert r.position == 40
    for t in range(3):
        a1, h1 = r.forward_token_decode(toks[t], want_hidden=True)
        assert a1 == int(am3[t])
        assert np.array_equal(h1.view(np.uint32), h3[t].view(np.uint32))


def test_mtp_matches_oracle(pair):
    pkg, orc, r, m = pair
    fresh(r, m, filled=30)
    am, hid = r.forward_token_decode(11, want_hidden=True)
    wam, whid = m.forward([11])
    cond = orc.f32_to_bf16_trunc(whid[0])  # the bf16 hidden row the drafter reads
    d0 = r.mtp_forward(am, 0, 0)
    w0, wn0 = m.mtp_forward(int(wam[0]), cond)
    assert d0 == w0
    assert np.array_equal(r.mtp_normalized(), wn0)
    d1 = r.mtp_forward(d0, 1)
    w1, wn1 = m.mtp_forward(w0, wn0)
    assert d1 == w1
    assert np.array_equal(r.mtp_normalized(), wn1)
    assert r.mtp_position == m.mtp_position == 32
    r.mtp_trim_state(1)
    m.mtp_trim(1)
    assert r.mtp_position == m.mtp_position == 31


def test_speculative_equals_sequential(pair):
    """tests/speculative_loop.rs:32-82: the block-3 speculative stream equals
    sequential greedy decoding; drafts forced to a seeded Bernoulli(0.6)
    acceptance pattern so that 1, 2 and 3 accepted rows all occur."""
    pkg, orc, r, m = pair
    steps = 40
    fresh(r, m, filled=50)
    am, hid = r.forward_token_decode(7, want_hidden=True)
    truth = [am] + list(r.decode_greedy(am, steps - 1))
    fresh(r, m, filled=50)
    am2, hid2 = r.forward_token_decode(7, want_hidden=True)
    assert am2 == am
    seed_tok = r.mtp_forward(am2, 0, 0)
    seed_hidden = orc.bf16_bits_to_f32(r.mtp_normalized())
    toks, stats = r.generate_greedy_block3(am2, hid2, seed_tok, seed_hidden, steps, force_truth=truth,
                                           force_seed=1234, p_accept=0.6)
    assert list(toks) == truth
    assert stats["rounds"] > 3
    assert 0 < stats["accepted_drafts"] < stats["drafted_tokens"]


def test_restore_rejects_checkpoint_of_other_depth(pair):
    """A checkpoint holds the GDN/conv state of its runner's layers; restoring
    it into a runner of another depth must fail, not copy past the arenas."""
    pkg, orc, r, m = pair
    other = pkg.Runner(layers=2 * LAYERS, vocab=VOCAB, capacity=64, seed=SEED, use_graph=False)
    try:
        ck = other.checkpoint_state()
        with pytest.raises(pkg.LisaError) as err:
            r.restore_state(ck)
        assert err.value.code == -1  # LISA_E_ARG
        other.free_checkpoint(ck)
        ck = r.checkpoint_state()
        with pytest.raises(pkg.LisaError):
            other.restore_state(ck)
        r.free_checkpoint(ck)
    finally:
        other.close()


def test_mtp_checkpoint_restore(pair):
    """MtpRunner::checkpoint_state / restore_state (runner.rs:2382-2420): the
    drafter's KV rows and position come back. After the checkpoint, rows below
    the checkpoint position are overwritten by other steps; the same drafter
    step after the restore must reproduce the one taken before."""
    pkg, orc, r, m = pair
    fresh(r, m, filled=20)
    am = r.forward_token_decode(3)
    d0 = r.mtp_forward(am, 0, 0)
    ck = r.mtp_checkpoint_state()
    pos = r.mtp_position
    a1 = r.mtp_forward(d0, 0, 0)
    n1 = r.mtp_normalized()
    r.mtp_trim_state(2)            # back below the checkpoint position
    r.mtp_upload_cond(np.full(5120, 0x3F80, np.uint16))
    r.mtp_forward(77, 2)           # rewrites KV row pos - 1
    r.mtp_forward(78, 2)           # and row pos
    r.mtp_restore_state(ck)
    assert r.mtp_position == pos
    a2 = r.mtp_forward(d0, 0, 0)
    assert a2 == a1
    assert np.array_equal(r.mtp_normalized(), n1)
    r.free_mtp_checkpoint(ck)
    bad = r.mtp_checkpoint_state()
    r.free_mtp_checkpoint(bad)


def test_graph_buckets_follow_the_context():
    """The captured step launches attention slices for the live context
    (runner.rs:1498-1500) in buckets of 512 positions: greedy decoding across
    a bucket boundary switches graphs and still equals the oracle token for
    token, on a runner whose capacity is far above the context."""
    pkg, orc = load_pkg(), load_oracle()
    cap = 2100
    r = pkg.Runner(layers=LAYERS, vocab=VOCAB, capacity=cap, seed=SEED, use_graph=True)
    m = orc.Model(LAYERS, VOCAB, cap, SEED)
    try:
        r.fill_state(500, CTX_SEED)
        m.fill_state(500, CTX_SEED)
        got = r.decode_greedy(41, 30)  # positions 500..529: slice buckets 8 then 16
        tok, want = 41, []
        for _ in range(30):
            wam, _ = m.forward([tok])
            tok = int(wam[0])
            want.append(tok)
        assert list(got) == want
        am, h = r.forward_token_decode(tok, want_hidden=True)
        wam, wh = m.forward([tok])
        assert am == int(wam[0]) and np.array_equal(h.view(np.uint32), wh[0].view(np.uint32))
    finally:
        r.close()
        m.close()
