"""A safetensors checkpoint in the reference's format and tensor names
(src/format/safetensor.rs; src/model/runner.rs:337-417, 2443-2502, 3769-3928)
loaded with lisa_runner_load decodes bit-exactly like the CPU oracle fed the
same tensors.

The oracle model's weights are first perturbed away from what the synthetic
generator of the same seed makes (layers' gate matrices exchanged, norm gains
and one MTP scale changed), so a loader that placed a tensor in the wrong
slot, dropped the interleaving of scales and biases, or fell back to generated
weights cannot pass."""
import numpy as np
import pytest

from _lisa import load_oracle, load_pkg
from _safetensors import mtp_spec, target_spec, tensors, write_snapshot

pytestmark = pytest.mark.gpu

LAYERS, VOCAB, CAP, SEED = 4, 4096, 160, 0x15A2026


@pytest.fixture(scope="module")
def loaded(tmp_path_factory):
    orc, pkg = load_oracle(), load_pkg()
    T = orc.T
    m = orc.Model(LAYERS, VOCAB, CAP, SEED, with_mtp=True)
    g0 = m.tensor(1, T["MLP_GATE"], 0, np.uint32)
    g1 = m.tensor(2, T["MLP_GATE"], 0, np.uint32)
    tmp = g0.copy()
    g0[:] = g1
    g1[:] = tmp
    fn = m.tensor(0, T["FINAL_NORM"], 0, np.uint16)
    fn[:] = fn[::-1].copy()
    s = m.tensor(orc.SCOPE_MTP, T["MTP_FC"], 1, np.uint16)
    s[: s.size // 2] = s[s.size // 2:].copy()
    d = tmp_path_factory.mktemp("ckpt")
    write_snapshot(d / "target", tensors(m, target_spec(LAYERS, VOCAB)), shards=3, order_seed=5,
                   extra={"vision_tower.blocks.0.attn.qkv.weight": np.zeros((8, 8), np.uint16)})
    write_snapshot(d / "mtp", tensors(m, mtp_spec()), shards=1)
    r = pkg.Runner.load(d / "target", d / "mtp", capacity=CAP, layers=LAYERS, vocab=VOCAB)
    yield pkg, orc, r, m, d
    r.close()
    m.close()


def test_loaded_runner_decodes_like_oracle(loaded):
    pkg, orc, r, m, _ = loaded
    r.fill_state(64, 7)
    m.fill_state(64, 7)
    tok = 123
    for step in range(12):
        am, hid = r.forward_token_decode(tok, want_hidden=True)
        wam, whid = m.forward([tok])
        assert am == int(wam[0]), step
        assert np.array_equal(hid.view(np.uint32), whid[0].view(np.uint32)), step
        tok = am
    # the same seed's generated weights give another model
    syn = pkg.Runner(layers=LAYERS, vocab=VOCAB, capacity=CAP, seed=SEED, use_graph=False)
    try:
        syn.fill_state(64, 7)
        r.fill_state(64, 7)
        _, h_syn = syn.forward_token_decode(123, want_hidden=True)
        _, h_ld = r.forward_token_decode(123, want_hidden=True)
        assert not np.array_equal(h_syn, h_ld)
    finally:
        syn.close()


def test_loaded_drafter_matches_oracle(loaded):
    pkg, orc, r, m, _ = loaded
    r.fill_state(40, 9)
    m.fill_state(40, 9)
    am, hid = r.forward_token_decode(11, want_hidden=True)
    wam, whid = m.forward([11])
    assert am == int(wam[0])
    d0 = r.mtp_forward(am, 0, 0)
    w0, wn0 = m.mtp_forward(int(wam[0]), orc.f32_to_bf16_trunc(whid[0]))
    assert d0 == w0
    assert np.array_equal(r.mtp_normalized(), wn0)
    d1 = r.mtp_forward(d0, 1)
    w1, wn1 = m.mtp_forward(w0, wn0)
    assert d1 == w1
    assert np.array_equal(r.mtp_normalized(), wn1)


def test_drafter_loaded_after_the_target(loaded):
    """QwenRunner::load then MtpRunner::load(&target, snapshot, capacity), the
    reference's two-step order (src/cli/run.rs:45-78)."""
    pkg, orc, _, m, d = loaded
    r = pkg.Runner.load(d / "target", capacity=CAP, layers=LAYERS, vocab=VOCAB)
    try:
        with pytest.raises(pkg.LisaError, match="without the MTP drafter"):
            r.mtp_forward(1, 2)
        with pytest.raises(pkg.LisaError, match="differs from the target"):
            r.load_mtp(d / "mtp", CAP + 64)
        r.load_mtp(d / "mtp", CAP)
        with pytest.raises(pkg.LisaError, match="already holds"):
            r.load_mtp(d / "mtp", CAP)
        r.fill_state(40, 9)
        m.fill_state(40, 9)
        am, hid = r.forward_token_decode(11, want_hidden=True)
        wam, whid = m.forward([11])
        assert am == int(wam[0])
        d0 = r.mtp_forward(am, 0, 0)
        w0, wn0 = m.mtp_forward(int(wam[0]), orc.f32_to_bf16_trunc(whid[0]))
        assert d0 == w0
        assert np.array_equal(r.mtp_normalized(), wn0)
        r.reset_state()
        assert r.position == 0 and r.mtp_position == 41  # the drafter kept its position
        r.mtp_reset_state()
        assert r.mtp_position == 0
    finally:
        r.close()


def test_load_errors_before_device_work(tmp_path):
    pkg = load_pkg()
    with pytest.raises(pkg.LisaError, match="KV capacity must be greater than zero"):
        pkg.Runner.load(tmp_path, capacity=0, layers=LAYERS, vocab=VOCAB)
    with pytest.raises(pkg.LisaError, match="no safetensors shards in"):
        pkg.Runner.load(tmp_path, capacity=CAP, layers=LAYERS, vocab=VOCAB)
