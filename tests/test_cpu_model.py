"""Model-level invariants of the oracle on a reduced-depth model (4 layers:
3 GDN + 1 attention, real widths, vocab 4096), CPU only.

tests/runner_checkpoint.rs:22-160: a 3-row verify pass computes the same rows
as three single-token steps, and committing r verified rows leaves exactly the
state r single steps leave (the next step is bit-identical)."""
import numpy as np
import pytest

from _lisa import load_oracle

orc = load_oracle()
LAYERS, VOCAB, CAP, SEED = 4, 4096, 96, 0x15A2026
CTX, CTX_SEED = 40, 0x4C1A


@pytest.fixture(scope="module")
def model():
    m = orc.Model(LAYERS, VOCAB, CAP, SEED)
    yield m
    m.close()


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def test_verify_rows_equal_single_steps(model):
    toks = [17, 2005, 4095]
    model.fill_state(CTX, CTX_SEED)
    singles = [model.forward([t]) for t in toks]
    model.fill_state(CTX, CTX_SEED)
    am3, h3 = model.forward(toks, capture=True)
    for t in range(3):
        assert am3[t] == singles[t][0][0]
        assert np.array_equal(bits(h3[t]), bits(singles[t][1][0]))


@pytest.mark.parametrize("rows", [1, 2, 3])
def test_commit_prefix_equals_sequential(model, rows):
    toks = [9, 123, 777]
    nxt = 55
    model.fill_state(CTX, CTX_SEED)
    for t in toks[:rows]:
        model.forward([t])
    want_am, want_h = model.forward([nxt])
    model.fill_state(CTX, CTX_SEED)
    model.forward(toks, capture=True)
    model.commit(rows)
    assert model.position == CTX + rows
    got_am, got_h = model.forward([nxt])
    assert got_am[0] == want_am[0]
    assert np.array_equal(bits(got_h), bits(want_h))


def test_forward_rejects_bad_input(model):
    model.fill_state(CTX, CTX_SEED)
    with pytest.raises(RuntimeError):
        model.forward([VOCAB])
    with pytest.raises(RuntimeError):
        model.commit(1)  # no verify pass pending
