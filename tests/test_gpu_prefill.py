"""GPU batched prefill (runner.rs:2129-2230) against the CPU oracle.

The MFMA GEMM accumulates in the hardware's order, so it is compared with a
tolerance (bit-exact on an exact-integer case); every row kernel (embed,
RMSNorm, residual, SwiGLU, argmax, GDN conv and recurrence over rows,
attention rows) is bit-exact given the same inputs. The full prefill must not
depend on the chunk size (bit-exact on the GPU), must agree with the oracle's
prefill and with sequential GPU decoding, and decoding must continue from the
prefilled state."""
import numpy as np
import pytest

from _lisa import DevQ4, bf16, f32, load_oracle, load_pkg, rand_q4

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pkg():
    return load_pkg()


@pytest.fixture(scope="module")
def orc():
    return load_oracle()


@pytest.fixture(scope="module")
def dev(pkg):
    return pkg.Device(0)


GEMM_KERNELS = ["lisa_q4_gemm", "lisa_q4_gemm_wide", "lisa_q4_gemm_m128"]


def gemm(pkg, dev, a_bf16, q, m, kernel="lisa_q4_gemm"):
    out = dev.buffer(m * q.n * 4)
    ab = dev.upload(a_bf16)
    p = pkg.GemmParams(ab.ptr, q.wbuf.ptr, q.sbbuf.ptr, out.ptr, m, q.n, q.k, q.n)
    tm = pkg.GEMM_TILE_M_SMALL if kernel.endswith("_m128") else pkg.GEMM_TILE_M
    wide = kernel.endswith("_wide")
    tn = pkg.GEMM_TILE_N_WIDE if wide else pkg.GEMM_TILE_N
    dev.dispatch(kernel, p, ((q.n + tn - 1) // tn, (m + tm - 1) // tm), (pkg.GEMM_THREADS_WIDE if wide else 256,))
    return out.read(np.float32, m * q.n).reshape(m, q.n)


@pytest.mark.parametrize("kernel", GEMM_KERNELS)
@pytest.mark.parametrize("M,N,K", [(37, 200, 1024), (128, 512, 5120), (300, 48, 5120), (5, 256, 17408),
                                   (512, 384, 6144), (260, 300, 1024), (33, 96, 192), (9, 130, 64)])
def test_gemm_matches_oracle(pkg, orc, dev, M, N, K, kernel):
    rng = np.random.default_rng(M * 7 + N + K)
    w, s, b = rand_q4(rng, N, K)
    a = bf16(rng.standard_normal((M, K)).astype(np.float32))
    got = gemm(pkg, dev, a, DevQ4(dev, w, s, b), M, kernel)
    want = orc.q4_gemm(a, w, s, b, N, K, M)
    rms = np.sqrt(np.mean(want.astype(np.float64) ** 2))
    assert np.max(np.abs(got - want)) <= 1e-5 * np.sqrt(K / 64) * rms
    # the oracle accumulates in the MFMA's order (f32, once per 8 k): most
    # outputs are the same bits, the rest differ by the hardware's own rounding
    assert np.mean(got.view(np.uint32) == want.view(np.uint32)) >= 0.95


@pytest.mark.parametrize("kernel", GEMM_KERNELS)
@pytest.mark.parametrize("K", [2048, 192])  # an even and an odd number of 64-wide K steps
def test_gemm_exact_integer_case(pkg, orc, dev, kernel, K):
    rng = np.random.default_rng(3)
    M, N = 70, 130
    w = rng.integers(0, 2**32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    a = bf16(rng.integers(-4, 5, size=(M, K)).astype(np.float32))
    s = bf16(rng.choice(np.array([0.5, 1.0, 2.0], np.float32), size=(N, K // 64)))
    b = bf16(rng.choice(np.array([-8.0, -4.0, 0.0, 1.0], np.float32), size=(N, K // 64)))
    got = gemm(pkg, dev, a, DevQ4(dev, w, s, b), M, kernel)
    assert np.array_equal(got, orc.q4_gemm(a, w, s, b, N, K, M))


@pytest.mark.parametrize("M,N,K", [(2048, 48, 5120), (2048, 1024, 5120), (300, 130, 192), (37, 200, 1024)])
def test_gemm_m128_equals_256_row_tile(pkg, dev, M, N, K):
    """The 128-row tile (the small projections: GDN a/b, attention k/v) gives
    every output the same MFMA sequence as the 256-row tile: equal bits."""
    rng = np.random.default_rng(M + 3 * N + K)
    q = DevQ4(dev, *rand_q4(rng, N, K))
    a = bf16(rng.standard_normal((M, K)).astype(np.float32))
    got = gemm(pkg, dev, a, q, M, "lisa_q4_gemm_m128")
    ref = gemm(pkg, dev, a, q, M, "lisa_q4_gemm")
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("M,N,K", [(300, 600, 1024), (37, 256, 5120), (260, 130, 192)])
def test_gemm_swiglu_equals_separate_gemms(pkg, orc, dev, M, N, K):
    """lisa_q4_gemm_swiglu (the MLP's gate/up pair with the SwiGLU epilogue,
    gemm.metal:273-341) equals the eight-wave GEMM of gate and of up followed
    by bf16(silu(bf16 g) * bf16 u) (mlp.metal:11-16), bit for bit: the same
    MFMA sums, one launch, no f32 intermediates. Output columns past a
    128-wide tile and an odd number of K steps included."""
    rng = np.random.default_rng(M + N + K)
    gq, uq = DevQ4(dev, *rand_q4(rng, N, K)), DevQ4(dev, *rand_q4(rng, N, K))
    a = bf16(rng.standard_normal((M, K)).astype(np.float32))
    g = gemm(pkg, dev, a, gq, M, "lisa_q4_gemm_wide")
    u = gemm(pkg, dev, a, uq, M, "lisa_q4_gemm_wide")
    ab, act = dev.upload(a), dev.buffer(M * N * 2)
    p = pkg.GemmParams(a=ab.ptr, w=gq.wbuf.ptr, sb=gq.sbbuf.ptr, m=M, n=N, k=K, ldc=N, w2=uq.wbuf.ptr,
                       sb2=uq.sbbuf.ptr, act=act.ptr)
    dev.dispatch("lisa_q4_gemm_swiglu", p, ((N + 127) // 128, (M + pkg.GEMM_TILE_M - 1) // pkg.GEMM_TILE_M),
                 (pkg.GEMM_THREADS_WIDE,))
    assert np.array_equal(act.read(np.uint16, M * N).reshape(M, N), orc.silu_mul(g, u).reshape(M, N))


@pytest.mark.timeout(300)
def test_gemm_full_model_shapes(pkg, orc, dev):
    """The config-3 prefill's largest GEMMs at their real shapes against the
    oracle: the MLP down (2048 x 5120 x 17408) and the gate and up projections
    (2048 x 17408 x 5120) on the eight-wave 256-wide tile, each within the
    GEMM tolerance of the smaller shapes; and the gate/up pair with the
    SwiGLU epilogue (2 x 17408 interleaved outputs) bit-equal to
    bf16(silu(bf16 g) * bf16 u) of those two GEMMs' outputs."""
    rng = np.random.default_rng(2048)
    M, H, I = 2048, 5120, 17408

    def check(got, want, k):
        rms = np.sqrt(np.mean(want.astype(np.float64) ** 2))
        assert np.max(np.abs(got - want)) <= 1e-5 * np.sqrt(k / 64) * rms
        assert np.mean(got.view(np.uint32) == want.view(np.uint32)) >= 0.95

    a = bf16(rng.standard_normal((M, I)).astype(np.float32))
    dq = DevQ4(dev, *rand_q4(rng, H, I))
    check(gemm(pkg, dev, a, dq, M, "lisa_q4_gemm_wide"), orc.q4_gemm(a, dq.w, dq.s, dq.b, H, I, M), I)
    del dq, a

    x = bf16(rng.standard_normal((M, H)).astype(np.float32))
    gq, uq = DevQ4(dev, *rand_q4(rng, I, H)), DevQ4(dev, *rand_q4(rng, I, H))
    g = gemm(pkg, dev, x, gq, M, "lisa_q4_gemm_wide")
    check(g, orc.q4_gemm(x, gq.w, gq.s, gq.b, I, H, M), H)
    u = gemm(pkg, dev, x, uq, M, "lisa_q4_gemm_wide")
    check(u, orc.q4_gemm(x, uq.w, uq.s, uq.b, I, H, M), H)
    xb, act = dev.upload(x), dev.buffer(M * I * 2)
    p = pkg.GemmParams(a=xb.ptr, w=gq.wbuf.ptr, sb=gq.sbbuf.ptr, m=M, n=I, k=H, ldc=I, w2=uq.wbuf.ptr,
                       sb2=uq.sbbuf.ptr, act=act.ptr)
    dev.dispatch("lisa_q4_gemm_swiglu", p, ((I + 127) // 128, (M + pkg.GEMM_TILE_M - 1) // pkg.GEMM_TILE_M),
                 (pkg.GEMM_THREADS_WIDE,))
    assert np.array_equal(act.read(np.uint16, M * I), orc.silu_mul(g, u))


def rows(pkg, dev, p, gx, m):
    dev.dispatch("lisa_rows", p, (gx, m), (256,))


def test_rows_kernels_bit_exact(pkg, orc, dev):
    rng = np.random.default_rng(5)
    m, H = 9, 5120
    h = bf16((rng.standard_normal((m, H)) * 3).astype(np.float32))
    o = (rng.standard_normal((m, H)) * 2).astype(np.float32)
    w = bf16(rng.uniform(0.9, 1.1, H).astype(np.float32))
    hb, ob, wb = dev.upload(h), dev.upload(o), dev.upload(w)
    rb, xb = dev.buffer(m * H * 2), dev.buffer(m * H * 2)
    p = pkg.RowsParams(h_in=hb.ptr, o_in=ob.ptr, norm_w=wb.ptr, r_out=rb.ptr, x_out=xb.ptr, mode=pkg.ROWS_RESNORM)
    rows(pkg, dev, p, 1, m)
    r = np.stack([orc.residual(h[t], o[t]) for t in range(m)])
    assert np.array_equal(rb.read(np.uint16, m * H).reshape(m, H), r)
    assert np.array_equal(xb.read(np.uint16, m * H).reshape(m, H), np.stack([orc.rms_norm(r[t], w) for t in range(m)]))
    p = pkg.RowsParams(h_in=hb.ptr, norm_w=wb.ptr, x_out=xb.ptr, mode=pkg.ROWS_NORM)
    rows(pkg, dev, p, 1, m)
    assert np.array_equal(xb.read(np.uint16, m * H).reshape(m, H), np.stack([orc.rms_norm(h[t], w) for t in range(m)]))
    # SwiGLU rows
    W = 17408
    g = (rng.standard_normal((m, W)) * 3).astype(np.float32)
    u = (rng.standard_normal((m, W)) * 3).astype(np.float32)
    gb, ub, ab = dev.upload(g), dev.upload(u), dev.buffer(m * W * 2)
    rows(pkg, dev, pkg.RowsParams(g_in=gb.ptr, u_in=ub.ptr, act_out=ab.ptr, width=W, mode=pkg.ROWS_SILU), 9, m)
    assert np.array_equal(ab.read(np.uint16, m * W).reshape(m, W), orc.silu_mul(g, u).reshape(m, W))
    # argmax rows, ties to the lowest index
    V = 4096
    lg = rng.standard_normal((m, V)).astype(np.float32)
    lg[2, [10, 900]] = 9.0
    lb, amb = dev.upload(lg), dev.buffer(m * 4)
    rows(pkg, dev, pkg.RowsParams(logits=lb.ptr, argmax_out=amb.ptr, width=V, mode=pkg.ROWS_ARGMAX), 1, m)
    assert list(amb.read(np.uint32, m)) == [orc.argmax(lg[t]) for t in range(m)]
    # embedding rows
    vocab = 64
    ew = rng.integers(0, 2**32, size=(vocab, H // 8), dtype=np.uint64).astype(np.uint32)
    es = bf16(rng.uniform(0.005, 0.02, (vocab, H // 64)).astype(np.float32))
    eb = bf16(rng.uniform(-0.1, 0.1, (vocab, H // 64)).astype(np.float32))
    toks = np.array([3, 63, 0, 17, 17, 40, 1, 2, 5], np.uint32)
    tb, ewb, esb = dev.upload(toks), dev.upload(ew), dev.upload((es.astype(np.uint32) | (eb.astype(np.uint32) << 16)))
    rows(pkg, dev, pkg.RowsParams(tokens=tb.ptr, emb_w=ewb.ptr, emb_sb=esb.ptr, r_out=rb.ptr, mode=pkg.ROWS_EMBED), 1, m)
    assert np.array_equal(rb.read(np.uint16, m * H).reshape(m, H), np.stack([orc.embed(ew, es, eb, t) for t in toks]))


@pytest.mark.parametrize("m", [1, 2, 3, 64, 65, 150])
def test_gdn_conv_rows_bit_exact(pkg, orc, dev, m):
    """Row blocks of 64 in parallel; rows before 0 and the new state come from the
    carried conv state (m < 3 keeps part of the old state)."""
    rng = np.random.default_rng(60 + m)
    CV = 10240
    qkv = rng.standard_normal((m, CV)).astype(np.float32)
    conv_w = bf16(rng.uniform(-0.5, 0.5, CV * 4).astype(np.float32))
    state = bf16(rng.standard_normal(3 * CV).astype(np.float32))
    qb, cwb, sb, cob = dev.upload(qkv), dev.upload(conv_w), dev.upload(state), dev.buffer(m * CV * 4)
    dev.dispatch("lisa_gdn_conv_rows", pkg.ConvRowsParams(qb.ptr, cwb.ptr, sb.ptr, cob.ptr, m, 0), (40, (m + 63) // 64),
                 (256,))
    want_co, want_state, _ = orc.gdn_conv(qkv, conv_w, state, m)
    assert np.array_equal(cob.read(np.float32, m * CV).reshape(m, CV).view(np.uint32), want_co.view(np.uint32))
    assert np.array_equal(sb.read(np.uint16, 3 * CV), want_state)


@pytest.mark.parametrize("m", [40, 43, 5])  # whole, ragged and short blocks of the scan's eight-row staging
def test_gdn_rows_bit_exact(pkg, orc, dev, m):
    rng = np.random.default_rng(6 + m)
    CV, VH, HD = 10240, 48, 128
    qkv = rng.standard_normal((m, CV)).astype(np.float32)
    conv_w = bf16(rng.uniform(-0.5, 0.5, CV * 4).astype(np.float32))
    state = bf16(rng.standard_normal(3 * CV).astype(np.float32))
    qb, cwb, sb, cob = dev.upload(qkv), dev.upload(conv_w), dev.upload(state), dev.buffer(m * CV * 4)
    dev.dispatch("lisa_gdn_conv_rows", pkg.ConvRowsParams(qb.ptr, cwb.ptr, sb.ptr, cob.ptr, m, 0), (40, (m + 63) // 64), (256,))
    want_co, want_state, _ = orc.gdn_conv(qkv, conv_w, state, m)
    co = cob.read(np.float32, m * CV).reshape(m, CV)
    assert np.array_equal(co.view(np.uint32), want_co.view(np.uint32))
    assert np.array_equal(sb.read(np.uint16, 3 * CV), want_state)
    z = rng.standard_normal((m, VH * HD)).astype(np.float32)
    a = rng.standard_normal((m, VH)).astype(np.float32)
    b = rng.standard_normal((m, VH)).astype(np.float32)
    a_log, dt_bias = bf16(rng.uniform(-2, 0, VH).astype(np.float32)), bf16(rng.uniform(-1, 1, VH).astype(np.float32))
    nw = bf16(rng.uniform(0.9, 1.1, HD).astype(np.float32))
    s0 = (rng.standard_normal(VH * HD * HD) * 0.01).astype(np.float32)
    zb, ab_, bb, alb, dtb, nwb, stb = (dev.upload(x) for x in (z, a, b, a_log, dt_bias, nw, s0))
    gb = dev.buffer(m * VH * HD * 2)
    qkb, gtb, yb = dev.buffer(m * 2 * 2048 * 4), dev.buffer(m * VH * 2 * 4), dev.buffer(m * VH * HD * 4)
    inv = 1.0 / np.sqrt(np.float32(128))
    p = pkg.GdnParams(conv_out=cob.ptr, z=zb.ptr, a=ab_.ptr, b=bb.ptr, a_log=alb.ptr, dt_bias=dtb.ptr, norm_w=nwb.ptr,
                      state=stb.ptr, gated=gb.ptr, y_out=yb.ptr, q_scale=float(np.float32(inv * inv)),
                      k_scale=float(np.float32(inv)), m_rows=m, qk=qkb.ptr, gates=gtb.ptr)
    dev.dispatch("lisa_gdn_prep_rows", p, (m, 9), (256,))
    dev.dispatch("lisa_gdn_scan_rows", p, (VH, 8), (256,))
    dev.dispatch("lisa_gdn_out_rows", p, (m, VH), (128,))
    gated, st, y, _ = orc.gdn_recurrence(co, z, a, b, a_log, dt_bias, nw, s0, m)
    assert np.array_equal(gb.read(np.uint16, m * VH * HD).reshape(m, -1), gated)
    assert np.array_equal(stb.read(np.float32, VH * HD * HD).view(np.uint32), st.view(np.uint32))
    assert np.array_equal(yb.read(np.float32, m * VH * HD).reshape(m, -1).view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("m,cap,base", [(70, 200, 90), (33, 64, 0), (16, 300, 200)])
def test_attention_rows_bit_exact(pkg, orc, dev, m, cap, base):
    rng = np.random.default_rng(8 + m)
    q_proj = (rng.standard_normal((m, 12288)) * 2).astype(np.float32)
    k_raw = rng.standard_normal((m, 1024)).astype(np.float32)
    v_raw = rng.standard_normal((m, 1024)).astype(np.float32)
    qn, kn = bf16(rng.uniform(0.9, 1.1, 256).astype(np.float32)), bf16(rng.uniform(0.9, 1.1, 256).astype(np.float32))
    kc = bf16(rng.standard_normal(4 * cap * 256).astype(np.float32))
    vc = bf16(rng.standard_normal(4 * cap * 256).astype(np.float32))
    s_max = (cap + 63) // 64
    bufs = {n: dev.upload(x) for n, x in dict(q=q_proj, k=k_raw, v=v_raw, qn=qn, kn=kn, kc=kc, vc=vc,
                                              pos=np.array([base], np.uint32)).items()}
    query, gated = dev.buffer(m * 6144 * 4), dev.buffer(m * 6144 * 2)
    po, pml = dev.buffer(m * 24 * s_max * 256 * 4), dev.buffer(m * 24 * s_max * 2 * 4)
    p = pkg.AttnParams(q_proj=bufs["q"].ptr, k_raw=bufs["k"].ptr, v_raw=bufs["v"].ptr, q_norm_w=bufs["qn"].ptr,
                       k_norm_w=bufs["kn"].ptr, key_cache=bufs["kc"].ptr, value_cache=bufs["vc"].ptr, part_o=po.ptr,
                       part_ml=pml.ptr, pos=bufs["pos"].ptr, gated=gated.ptr, capacity=cap, s_max=s_max,
                       query=query.ptr, m_rows=m)
    dev.dispatch("lisa_attn_store_rows", p, (m, 7), (256,))
    rb = pkg.ATT_ROWS_PER_WG
    dev.dispatch("lisa_attn_partial_rows", p, ((base + m + 63) // 64, 4, (m + rb - 1) // rb), (pkg.ATT_ROWS_THREADS,))
    dev.dispatch("lisa_attn_merge_rows", p, (24, m), (256,))
    want, kc2, vc2 = orc.attention(q_proj, k_raw, v_raw, qn, kn, kc, vc, cap, base, m)
    assert np.array_equal(bufs["kc"].read(np.uint16, kc.size), kc2)
    assert np.array_equal(bufs["vc"].read(np.uint16, vc.size), vc2)
    assert np.array_equal(gated.read(np.uint16, m * 6144).reshape(m, 6144), want)


LAYERS, VOCAB, CAP, SEED, CTX_SEED = 4, 4096, 256, 0x5EED1, 0xC0FFEE


@pytest.fixture(scope="module")
def pair(pkg, orc):
    r = pkg.Runner(layers=LAYERS, vocab=VOCAB, capacity=CAP, seed=SEED, use_graph=True)
    m = orc.Model(LAYERS, VOCAB, CAP, SEED)
    yield r, m
    r.close()
    m.close()


PROMPT = np.random.default_rng(11).integers(0, VOCAB, 48).astype(np.uint32)


def test_prefill_model(pair):
    r, m = pair
    r.fill_state(40, CTX_SEED)
    am, h = r.forward_prefill(PROMPT, want_hidden=True)
    assert r.position == 40 + len(PROMPT)
    r.fill_state(40, CTX_SEED)
    am13, h13 = r.forward_prefill(PROMPT, chunk=13, want_hidden=True)
    assert np.array_equal(am, am13) and np.array_equal(h.view(np.uint32), h13.view(np.uint32))
    m.fill_state(40, CTX_SEED)
    wam, wh = m.prefill(PROMPT, want_hidden=True)
    assert np.mean(am == wam) >= 0.95
    rel = np.sqrt(np.mean((h - wh) ** 2) / np.mean(wh**2))
    assert rel < 1e-2, rel
    # decoding continues from the prefilled state (GDN, conv history, KV)
    tok = int(am[-1])
    gam, gh = r.forward_token_decode(tok, want_hidden=True)
    oam, oh = m.forward([tok])
    assert np.sqrt(np.mean((gh - oh[0]) ** 2) / np.mean(oh[0] ** 2)) < 1e-2
    # and agrees with sequential decoding of the prompt on the GPU
    r.fill_state(40, CTX_SEED)
    seq = [r.forward_token_decode(int(t)) for t in PROMPT]
    assert np.mean(am == np.array(seq)) >= 0.95
