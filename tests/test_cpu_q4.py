"""CPU pins of the oracle's q4 linear (no GPU).

The reference's own known-answer tests (tests/qmv.rs:5-113 and :115-220) are
restated with their exact inputs and tolerance; the rest pins the arithmetic
with results the mathematics fixes: an exact-integer case where every partial
sum is representable (so any dropped term, swapped nibble or wrong group index
changes the answer), the closed form in double precision, power-of-two
homogeneity (bit-exact), and the row independence of the M=3 path.
"""
import numpy as np
import pytest

from _lisa import f32, load_oracle, rand_q4

orc = load_oracle()


def trunc_bf16(x):
    # src/format/dtype.rs:42-47: the reference's host conversion truncates
    return orc.f32_to_bf16_trunc(np.asarray(x, dtype=np.float32))


def dequant(w, s, b):
    n, k8 = w.shape
    q = ((w[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(n, k8 * 8)
    return q.astype(np.float64) * np.repeat(f32(s), 64, axis=1) + np.repeat(f32(b), 64, axis=1)


def kat_packed(n, k, a, c):
    idx = np.arange(n * k // 8, dtype=np.uint64)[:, None]
    nib = np.arange(8, dtype=np.uint64)[None, :]
    vals = (idx * a + nib * c) % 16
    return (vals << (4 * nib)).sum(axis=1).astype(np.uint32).reshape(n, k // 8)


def test_qmv_rs_tail_rows_kat():
    """tests/qmv.rs:5-113: N=19, K=128, nibble (i*3 + n*5) % 16, s=0.0125,
    b=-0.08, x=(k-63)*0.003, |y - ref| < 2e-4."""
    N, K = 19, 128
    x = trunc_bf16((np.arange(K, dtype=np.float32) - 63.0) * 0.003)
    w = kat_packed(N, K, 3, 5)
    s = np.full((N, K // 64), trunc_bf16(0.0125), np.uint16)
    b = np.full((N, K // 64), trunc_bf16(-0.08), np.uint16)
    for ksplit in (1, 4):
        got = orc.q4_linear(x[None, :], w, s, b, N, K, 1, ksplit)[0]
        want = dequant(w, s, b) @ f32(x).astype(np.float64)
        assert np.max(np.abs(got - want)) < 2e-4


def test_qmv_rs_wide3_kat():
    """tests/qmv.rs:115-220: M=3, N=19, K=128, nibble (i*7 + n*3) % 16,
    s=0.011, b=-0.075, x[r][k]=(k - 61 + 7r)*0.0025, |y - ref| < 2e-4."""
    M, N, K = 3, 19, 128
    r, c = np.meshgrid(np.arange(M), np.arange(K), indexing="ij")
    x = trunc_bf16(((c - 61.0 + r * 7.0) * 0.0025).astype(np.float32))
    w = kat_packed(N, K, 7, 3)
    s = np.full((N, K // 64), trunc_bf16(0.011), np.uint16)
    b = np.full((N, K // 64), trunc_bf16(-0.075), np.uint16)
    got = orc.q4_linear(x, w, s, b, N, K, M, 1)
    want = f32(x).astype(np.float64) @ dequant(w, s, b).T
    assert np.max(np.abs(got - want)) < 2e-4
    # tests/qmv.rs:222-348: row 0 of the wide path equals the M=1 path, bit-exact
    one = orc.q4_linear(x[:1], w, s, b, N, K, 1, 1)
    assert np.array_equal(got[0].view(np.uint32), one[0].view(np.uint32))


@pytest.mark.parametrize("K,ksplit", [(1024, 1), (1024, 4), (5120, 1), (6144, 4)])
def test_q4_exact_integer_case(K, ksplit):
    """Small-integer x, scales and biases: every partial sum is an exact
    binary fraction well inside f32, so the result must equal the exact dot
    product bit for bit. A dropped term, a nibble taken from the wrong half of
    a byte, a wrong group or a sign error all change it."""
    rng = np.random.default_rng(K + ksplit)
    N = 40
    w = rng.integers(0, 2**32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    x = rng.integers(-3, 4, size=(2, K)).astype(np.float32)
    s = rng.choice(np.array([0.5, 1.0, 2.0], np.float32), size=(N, K // 64))
    b = rng.choice(np.array([-1.0, -0.5, 0.0, 0.5, 1.0], np.float32), size=(N, K // 64))
    xb, sb, bb = orc.f32_to_bf16_bits(x), orc.f32_to_bf16_bits(s), orc.f32_to_bf16_bits(b)
    got = orc.q4_linear(xb, w, sb, bb, N, K, 2, ksplit)
    exact = x.astype(np.float64) @ dequant(w, sb, bb).T
    assert np.array_equal(got.astype(np.float64), exact)


@pytest.mark.parametrize("K,N,M,ksplit", [(5120, 64, 1, 1), (5120, 48, 3, 1), (17408, 24, 1, 4),
                                          (10240, 16, 1, 4), (6144, 40, 3, 4)])
def test_q4_closed_form(K, N, M, ksplit):
    """y = sum_k x_k (q s + b) in double precision (config-0 distributions)."""
    rng = np.random.default_rng(K * 7 + N + M)
    w, s, b = rand_q4(rng, N, K)
    x = orc.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    got = orc.q4_linear(x, w, s, b, N, K, M, ksplit)
    ref = f32(x).astype(np.float64) @ dequant(w, s, b).T
    scale = np.sqrt(np.mean(ref**2))
    assert np.max(np.abs(got - ref)) <= 1e-5 * scale + 1e-4


def test_q4_power_of_two_homogeneity():
    """Scaling x by 2^e scales every intermediate exactly: bit-exact 2^e * y.
    Pins that the 2^-24-scaled nibble chains and the scale-by-2^24 fold are
    pure power-of-two rescalings."""
    rng = np.random.default_rng(11)
    K, N = 5120, 32
    w, s, b = rand_q4(rng, N, K)
    x = rng.standard_normal((1, K)).astype(np.float32)
    xb = orc.f32_to_bf16_bits(x)
    base = orc.q4_linear(xb, w, s, b, N, K, 1, 1)
    for e in (-20, -3, 5, 30):
        xe = orc.f32_to_bf16_bits(f32(xb) * np.float32(2.0**e))
        got = orc.q4_linear(xe, w, s, b, N, K, 1, 1)
        assert np.array_equal(got.view(np.uint32), (base * np.float32(2.0**e)).view(np.uint32))


def test_q4_rows_independent_and_ksplit_consistent():
    """M=3 row m equals the M=1 result for row m (bit-exact); the two K
    partitions agree to rounding."""
    rng = np.random.default_rng(5)
    K, N = 6144, 24
    w, s, b = rand_q4(rng, N, K)
    x = orc.f32_to_bf16_bits(rng.standard_normal((3, K)).astype(np.float32))
    g3 = orc.q4_linear(x, w, s, b, N, K, 3, 4)
    for m in range(3):
        g1 = orc.q4_linear(x[m:m + 1], w, s, b, N, K, 1, 4)
        assert np.array_equal(g3[m].view(np.uint32), g1[0].view(np.uint32))
    g1s = orc.q4_linear(x, w, s, b, N, K, 3, 1)
    assert np.max(np.abs(g1s - g3)) <= 1e-5 * np.sqrt(np.mean(g3**2)) + 1e-5
