"""lisa_attention_decode_noalloc (the allocation-free variant) through the C
ABI against lisa_attention_decode on the same inputs: gated output and the
appended K/V rows bit-identical, on two calls in a row, the second with a
smaller input (fewer rows and a shorter context) than the first, so the
second reads a scratch that still holds the first call's partials; and a call
whose partials would not fit the fixed scratch is rejected before any launch."""
import numpy as np
import pytest

from _lisa import bf16, load_pkg

pytestmark = pytest.mark.gpu


def inputs(pkg, dev, m, pos, cap, seed):
    rng = np.random.default_rng(seed)
    host = {
        "q": rng.standard_normal((m, 12288)).astype(np.float32),
        "k": rng.standard_normal((m, 1024)).astype(np.float32),
        "v": rng.standard_normal((m, 1024)).astype(np.float32),
        "qn": bf16(rng.uniform(0.9, 1.1, 256).astype(np.float32)),
        "kn": bf16(rng.uniform(0.9, 1.1, 256).astype(np.float32)),
        "kc": bf16(rng.standard_normal((4, cap, 256)).astype(np.float32)),
        "vc": bf16(rng.standard_normal((4, cap, 256)).astype(np.float32)),
        "pos": np.array([pos], np.uint32),
    }

    def make():
        b = {k: dev.upload(v) for k, v in host.items()}
        b["gated"] = dev.buffer(m * 6144 * 2)
        a = pkg.AttnDecodeArgs(q_proj=b["q"].ptr, k_raw=b["k"].ptr, v_raw=b["v"].ptr, q_norm_w=b["qn"].ptr,
                               k_norm_w=b["kn"].ptr, key_cache=b["kc"].ptr, value_cache=b["vc"].ptr, pos=b["pos"].ptr,
                               gated=b["gated"].ptr, capacity=cap, m_rows=m, max_pos=pos + m - 1)
        return a, b

    return make, host["kc"].size


@pytest.mark.parametrize("first,second", [((3, 9000, 9100), (1, 700, 800)), ((1, 40000, 40960), (3, 130, 200))])
def test_noalloc_equals_allocating_entry_point(first, second):
    pkg = load_pkg()
    dev = pkg.Device(0)
    for i, (m, pos, cap) in enumerate((first, second)):
        make, n_cache = inputs(pkg, dev, m, pos, cap, 7 + i)
        a_ref, b_ref = make()
        a_new, b_new = make()
        dev.attention_decode(a_ref)           # library workspace (allocating)
        dev.attention_decode_noalloc(a_new)   # fixed scratch
        assert np.array_equal(b_new["gated"].read(np.uint16, m * 6144), b_ref["gated"].read(np.uint16, m * 6144)), i
        assert np.array_equal(b_new["kc"].read(np.uint16, n_cache), b_ref["kc"].read(np.uint16, n_cache)), i
        assert np.array_equal(b_new["vc"].read(np.uint16, n_cache), b_ref["vc"].read(np.uint16, n_cache)), i


def test_noalloc_rejects_partials_beyond_the_scratch():
    pkg = load_pkg()
    dev = pkg.Device(0)
    make, _ = inputs(pkg, dev, 3, 20000, 20100, 3)
    a, _ = make()
    assert pkg.lib().lisa_attention_workspace_bytes(3, 20002) > (16 << 20)
    with pytest.raises(pkg.LisaError) as err:
        dev.attention_decode_noalloc(a)
    assert err.value.code == -1 and "scratch" in str(err.value)
