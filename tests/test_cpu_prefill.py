"""CPU pins of the oracle's batched prefill (runner.rs:2129-2230).

The prefill q4 GEMM dequantizes each weight to bf16(fma(scale, q, bias))
(gemm.metal:238-266) and accumulates in f32 once per 8 consecutive k (the
order of the gfx950 bf16 MFMA): pinned by an exact-integer case (every sum
representable, compared bit for bit), by an independent numpy construction of
the bf16-rounded weights and of that accumulation order, and against the
double-precision sum within the order's rounding. The model-level prefill is pinned by
the reference's own contract: the recurrent state carries across chunks, so the
result does not depend on the chunk size, and each position's argmax equals the
sequential decode's (tests/batched_prefill.rs allows 5 % mismatches; this
synthetic model gives none)."""
import numpy as np
import pytest

from _lisa import f32, load_oracle, rand_q4

orc = load_oracle()


def test_gemm_exact_integer_case():
    rng = np.random.default_rng(1)
    M, N, K = 6, 40, 1024
    w = rng.integers(0, 2**32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    a = rng.integers(-4, 5, size=(M, K)).astype(np.float32)
    s = rng.choice(np.array([0.5, 1.0, 2.0], np.float32), size=(N, K // 64))
    b = rng.choice(np.array([-8.0, -4.0, 0.0, 1.0], np.float32), size=(N, K // 64))
    got = orc.q4_gemm(orc.f32_to_bf16_bits(a), w, orc.f32_to_bf16_bits(s), orc.f32_to_bf16_bits(b), N, K, M)
    q = ((w[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(N, K).astype(np.float64)
    wd = q * np.repeat(s, 64, axis=1) + np.repeat(b, 64, axis=1)
    assert np.array_equal(got.astype(np.float64), a.astype(np.float64) @ wd.T)


def test_gemm_bf16_dequant_then_blocked_f32_sum():
    rng = np.random.default_rng(2)
    M, N, K = 5, 64, 2048
    w, s, b = rand_q4(rng, N, K)
    a = orc.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    got = orc.q4_gemm(a, w, s, b, N, K, M)
    q = ((w[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(N, K).astype(np.float64)
    # fma(s, q, b) rounded once to f32 (exact in double first), then RNE to bf16
    wd = (q * np.repeat(f32(s), 64, axis=1) + np.repeat(f32(b), 64, axis=1)).astype(np.float32)
    wd = f32(orc.f32_to_bf16_bits(wd)).astype(np.float64)
    af = f32(a).astype(np.float64)
    acc = np.zeros((M, N), np.float32)
    for k0 in range(0, K, 8):  # acc = f32(acc + exact sum of 8 products)
        acc = (acc.astype(np.float64) + af[:, k0:k0 + 8] @ wd[:, k0:k0 + 8].T).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), acc.view(np.uint32))
    # within the rounding of K/8 f32 additions of the double-precision sum
    ref = af @ wd.T
    bound = (K / 8) * 2.0**-24 * (np.abs(af) @ np.abs(wd).T)
    assert np.all(np.abs(got - ref) <= bound)
    assert not np.array_equal(got, ref.astype(np.float32))  # the order is not one final rounding
    # and it is not the decode path's arithmetic (weights not rounded to bf16)
    exact = af @ (q * np.repeat(f32(s), 64, axis=1) + np.repeat(f32(b), 64, axis=1)).T
    assert not np.array_equal(got, exact.astype(np.float32))


@pytest.fixture(scope="module")
def model():
    m = orc.Model(4, 4096, 96, 0x15A2026)
    yield m
    m.close()


TOKENS = np.random.default_rng(7).integers(0, 4096, 16).astype(np.uint32)


def test_prefill_chunk_size_invariant(model):
    model.fill_state(40, 7)
    am1, h1 = model.prefill(TOKENS, chunk=0, want_hidden=True)
    assert model.position == 40 + len(TOKENS)
    model.fill_state(40, 7)
    am2, h2 = model.prefill(TOKENS, chunk=5, want_hidden=True)
    assert np.array_equal(am1, am2)
    assert np.array_equal(h1.view(np.uint32), h2.view(np.uint32))


def test_prefill_matches_sequential_decode(model):
    model.fill_state(40, 7)
    am, h = model.prefill(TOKENS, want_hidden=True)
    model.fill_state(40, 7)
    seq = [model.forward([t]) for t in TOKENS]
    seq_am = np.array([int(s[0][0]) for s in seq])
    seq_h = np.stack([s[1][0] for s in seq])
    assert np.mean(am == seq_am) >= 0.95
    # prefill GEMMs round every weight to bf16 (0.2 %), decode keeps exact nibble
    # products; through 4 layers the hidden rows differ by about 2 % rms
    rel = np.sqrt(np.mean((h - seq_h) ** 2) / np.mean(seq_h**2))
    assert rel < 5e-2


def test_prefill_rejects_bad_input(model):
    model.fill_state(40, 7)
    with pytest.raises(RuntimeError):
        model.prefill(np.array([4096], np.uint32))
    with pytest.raises(RuntimeError):
        model.prefill(np.zeros(60, np.uint32))  # capacity 96
