"""lisa_attention_decode (BASELINE config 2's attention core) through the C
ABI against the CPU oracle's attention (attention.metal:118-319, 520-641):
gated output and the appended K/V rows bit-exact, with the caller's workspace
and with the library's, at one and three rows and up to a 32k context."""
import numpy as np
import pytest

from _lisa import bf16, load_oracle, load_pkg

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    pkg, orc = load_pkg(), load_oracle()
    return pkg, orc, pkg.Device(0)


def case(pkg, orc, dev, m, pos, cap, seed, workspace):
    rng = np.random.default_rng(seed)
    q_proj = rng.standard_normal((m, 12288)).astype(np.float32)
    k_raw = rng.standard_normal((m, 1024)).astype(np.float32)
    v_raw = rng.standard_normal((m, 1024)).astype(np.float32)
    qn = bf16(rng.uniform(0.9, 1.1, 256).astype(np.float32))
    kn = bf16(rng.uniform(0.9, 1.1, 256).astype(np.float32))
    kc = np.zeros((4, cap, 256), np.uint16)
    vc = np.zeros((4, cap, 256), np.uint16)
    kc[:, :pos] = bf16(rng.standard_normal((4, pos, 256)).astype(np.float32))
    vc[:, :pos] = bf16(rng.standard_normal((4, pos, 256)).astype(np.float32))
    bufs = {k: dev.upload(v) for k, v in (("q", q_proj), ("k", k_raw), ("v", v_raw), ("qn", qn), ("kn", kn),
                                         ("kc", kc), ("vc", vc), ("pos", np.array([pos], np.uint32)))}
    gated = dev.buffer(m * 6144 * 2)
    a = pkg.AttnDecodeArgs(q_proj=bufs["q"].ptr, k_raw=bufs["k"].ptr, v_raw=bufs["v"].ptr, q_norm_w=bufs["qn"].ptr,
                           k_norm_w=bufs["kn"].ptr, key_cache=bufs["kc"].ptr, value_cache=bufs["vc"].ptr,
                           pos=bufs["pos"].ptr, gated=gated.ptr, capacity=cap, m_rows=m, max_pos=pos + m - 1)
    ws = None
    if workspace:
        ws = dev.buffer(int(pkg.lib().lisa_attention_workspace_bytes(m, pos + m - 1)))
    dev.attention_decode(a, ws)
    want, wkc, wvc = orc.attention(q_proj, k_raw, v_raw, qn, kn, kc.reshape(-1), vc.reshape(-1), cap, pos, m)
    assert np.array_equal(gated.read(np.uint16, m * 6144).reshape(m, 6144), want)
    assert np.array_equal(bufs["kc"].read(np.uint16, kc.size), wkc)
    assert np.array_equal(bufs["vc"].read(np.uint16, vc.size), wvc)


@pytest.mark.parametrize("m,pos,cap,workspace", [(1, 0, 64, True), (1, 4095, 4100, True), (3, 62, 200, False),
                                                 (1, 1000, 5000, False), (3, 16383, 16386, True),
                                                 (1, 32767, 32768, False)])
def test_attention_decode_matches_oracle(env, m, pos, cap, workspace):
    pkg, orc, dev = env
    case(pkg, orc, dev, m, pos, cap, 100 + m + pos, workspace)


def test_attention_decode_rejects_bad_arguments(env):
    pkg, orc, dev = env
    buf = dev.buffer(1 << 20)
    a = pkg.AttnDecodeArgs(q_proj=buf.ptr, k_raw=buf.ptr, v_raw=buf.ptr, q_norm_w=buf.ptr, k_norm_w=buf.ptr,
                           key_cache=buf.ptr, value_cache=buf.ptr, pos=buf.ptr, gated=buf.ptr, capacity=64, m_rows=2,
                           max_pos=5)
    with pytest.raises(pkg.LisaError):
        dev.attention_decode(a)
    a.m_rows, a.max_pos = 1, 64   # past the capacity
    with pytest.raises(pkg.LisaError):
        dev.attention_decode(a)
    a.max_pos = 63
    small = dev.buffer(16)
    with pytest.raises(pkg.LisaError):
        dev.attention_decode(a, small)  # workspace too small
