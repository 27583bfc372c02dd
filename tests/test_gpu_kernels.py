"""GPU parity of the gfx950 kernels against the CPU oracle (bit-exact).

BASELINE configs 0 (one q4 GEMV), 1 (one GDN layer step) and 2 (one gated
attention layer at 4k and 32k context), plus the reference's own kernel
invariants (tests/qmv.rs: tail rows, fast == wide3 row 0, fused == separate;
tests/attn_sliced.rs: batch-3 row == standalone row; tests/gdn_recurrence_state.rs:
batched steps == single steps).
"""
import numpy as np
import pytest

from _lisa import DevQ4, bf16, f32, launch_qmv, load_oracle, load_pkg, rand_q4

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


def same_bits(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32 if a.dtype == np.float32 else a.dtype),
                                                  b.view(np.uint32 if b.dtype == np.float32 else b.dtype))


def run_linear(pkg, dev, q, x_bf16, M, K):
    out = dev.buffer(M * q.n * 4)
    xb = dev.upload(x_bf16)
    p = pkg.QmvParams()
    p.pro_mode = pkg.PRO_LOADX
    p.x_in = xb.ptr
    ks, _ = launch_qmv(pkg, dev, K, M, p, [(q, None, out.ptr, pkg.EPI_STORE)])
    return out.read(np.float32, M * q.n).reshape(M, q.n), ks


# ---------------------------------------------------------------- config 0
@pytest.mark.parametrize("M", [1, 3])
def test_qmv_config0_bitexact(pkg, orc, dev, M):
    """K=5120, N=17408, M=1 decode and M=3 verify."""
    rng = np.random.default_rng(20260 + M)
    K, N = 5120, 17408
    w, s, b = rand_q4(rng, N, K)
    x = bf16(rng.standard_normal((M, K)).astype(np.float32))
    q = DevQ4(dev, w, s, b)
    got, ks = run_linear(pkg, dev, q, x, M, K)
    want = orc.q4_linear(x, w, s, b, N, K, M, ks)
    assert ks == 1
    assert same_bits(got, want)
    # closed form in double precision: y = sum_k x_k (q s + b)
    qv = ((w[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(N, K).astype(np.float64)
    deq = qv * np.repeat(f32(s), 64, axis=1) + np.repeat(f32(b), 64, axis=1)
    ref = f32(x).astype(np.float64) @ deq.T
    scale = np.sqrt(np.mean(ref**2))
    assert np.max(np.abs(got - ref)) <= 1e-5 * scale + 1e-4


def test_qmv_wide3_row0_equals_fast(pkg, dev):
    """tests/qmv.rs:222-348: the M=3 kernel's row 0 equals the M=1 kernel."""
    rng = np.random.default_rng(7)
    K, N = 5120, 1024
    w, s, b = rand_q4(rng, N, K)
    q = DevQ4(dev, w, s, b)
    x3 = bf16(rng.standard_normal((3, K)).astype(np.float32))
    g1, _ = run_linear(pkg, dev, q, x3[:1], 1, K)
    g3, _ = run_linear(pkg, dev, q, x3, 3, K)
    assert same_bits(g3[0], g1[0])


@pytest.mark.parametrize("K,N,M", [(17408, 5120, 1), (17408, 5120, 3), (6144, 5120, 1), (6144, 5120, 3),
                                   (10240, 5120, 1)])
def test_qmv_ksplit_shapes(pkg, orc, dev, K, N, M):
    """The N=5120 projections (down, out_proj, o_proj, MTP fc) use the
    in-workgroup K split; K=17408 M=3 uses the bf16 LDS layout."""
    rng = np.random.default_rng(K + N + M)
    w, s, b = rand_q4(rng, N, K)
    x = bf16((rng.standard_normal((M, K)) * 3).astype(np.float32))
    q = DevQ4(dev, w, s, b)
    got, ks = run_linear(pkg, dev, q, x, M, K)
    assert ks == 4
    assert same_bits(got, orc.q4_linear(x, w, s, b, N, K, M, ks))


@pytest.mark.parametrize("M", [1, 3])
def test_qmv_tail_rows(pkg, orc, dev, M):
    """tests/qmv.rs:5-113 shape family: N=19 tail rows (K=1024 here)."""
    rng = np.random.default_rng(19)
    K, N = 1024, 19
    w, s, b = rand_q4(rng, N, K)
    x = bf16(rng.standard_normal((M, K)).astype(np.float32))
    got, ks = run_linear(pkg, dev, DevQ4(dev, w, s, b), x, M, K)
    assert same_bits(got, orc.q4_linear(x, w, s, b, N, K, M, ks))


def test_qmv_fused_equals_separate(pkg, orc, dev):
    """tests/qmv.rs:350-673: a multi-projection launch is bit-identical to
    single launches of the same ksplit (GDN in_proj shapes)."""
    rng = np.random.default_rng(4)
    K = 5120
    shapes = [10240, 6144, 48, 48]
    qs = [DevQ4(dev, *rand_q4(rng, n, K)) for n in shapes]
    x = bf16(rng.standard_normal((1, K)).astype(np.float32))
    xb = dev.upload(x)
    outs = [dev.buffer(n * 4) for n in shapes]
    p = pkg.QmvParams()
    p.pro_mode = pkg.PRO_LOADX
    p.x_in = xb.ptr
    ks, _ = launch_qmv(pkg, dev, K, 1, p, [(q, None, o.ptr, pkg.EPI_STORE) for q, o in zip(qs, outs)])
    assert ks == 1
    for q, o, n in zip(qs, outs, shapes):
        got = o.read(np.float32, n)
        assert same_bits(got, orc.q4_linear(x, q.w, q.s, q.b, n, K, 1, 1)[0])


@pytest.mark.parametrize("M", [1, 3])
def test_qmv_resnorm_gateup(pkg, orc, dev, M):
    """MLP first half: residual add + post RMSNorm prologue, gate/up pair with
    SwiGLU epilogue (norm.metal:10-57, mlp.metal:6-17)."""
    rng = np.random.default_rng(40 + M)
    K, N = 5120, 17408
    gw, gs, gb = rand_q4(rng, N, K)
    uw, us, ub = rand_q4(rng, N, K)
    h = bf16((rng.standard_normal((M, K)) * 4).astype(np.float32))
    o = (rng.standard_normal((M, K)) * 50).astype(np.float32)
    nw = bf16(rng.uniform(0.9, 1.1, K).astype(np.float32))
    hb, ob, nb = dev.upload(h), dev.upload(o), dev.upload(nw)
    rbuf, xbuf, act = dev.buffer(M * K * 2), dev.buffer(M * K * 2), dev.buffer(M * N * 2)
    p = pkg.QmvParams()
    p.pro_mode = pkg.PRO_RESNORM
    p.h_in, p.o_in, p.norm_w, p.r_out, p.x_out = hb.ptr, ob.ptr, nb.ptr, rbuf.ptr, xbuf.ptr
    qg, qu = DevQ4(dev, gw, gs, gb), DevQ4(dev, uw, us, ub)
    ks, _ = launch_qmv(pkg, dev, K, M, p, [(qg, qu, act.ptr, pkg.EPI_GATEUP)])
    r = np.stack([np.empty(K, np.uint16)] * M)
    x = np.stack([np.empty(K, np.uint16)] * M)
    L = orc.lib()
    for m in range(M):
        L.orc_residual(orc.p(h[m]), orc.p(o[m]), K, orc.p(r[m]))
        x[m] = orc.rms_norm(r[m], nw)
    assert np.array_equal(rbuf.read(np.uint16, M * K).reshape(M, K), r)
    assert np.array_equal(xbuf.read(np.uint16, M * K).reshape(M, K), x)
    g = orc.q4_linear(x, gw, gs, gb, N, K, M, ks)
    u = orc.q4_linear(x, uw, us, ub, N, K, M, ks)
    want = np.empty(M * N, np.uint16)
    L.orc_silu_mul(orc.p(g), orc.p(u), M * N, orc.p(want))
    assert np.array_equal(act.read(np.uint16, M * N), want)


@pytest.mark.parametrize("M", [1, 3])
def test_qmv_resid_then_prenorm_gateup(pkg, orc, dev, M):
    """The decode path's split residual: an out_proj-shaped launch (K=6144)
    adds its rows into the residual in place; the gate/up launch normalizes
    the updated rows with the per-8-row tile statistic (norm.metal:10-57,
    mlp.metal:6-17)."""
    rng = np.random.default_rng(70 + M)
    K, H, N = 6144, 5120, 17408
    ow, osc, ob = rand_q4(rng, H, K)
    gw, gs, gb = rand_q4(rng, N, H)
    uw, us, ub = rand_q4(rng, N, H)
    x = bf16(rng.standard_normal((M, K)).astype(np.float32))
    h = bf16((rng.standard_normal((M, H)) * 4).astype(np.float32))
    nw = bf16(rng.uniform(0.9, 1.1, H).astype(np.float32))
    xb, hb, nb = dev.upload(x), dev.upload(h), dev.upload(nw)
    p = pkg.QmvParams()
    p.pro_mode = pkg.PRO_LOADX
    p.x_in, p.h_in = xb.ptr, hb.ptr
    ks, _ = launch_qmv(pkg, dev, K, M, p, [(DevQ4(dev, ow, osc, ob), None, 0, pkg.EPI_RESID)])
    y = orc.q4_linear(x, ow, osc, ob, H, K, M, ks)
    r = np.stack([orc.residual(h[m], y[m]) for m in range(M)])
    assert np.array_equal(hb.read(np.uint16, M * H).reshape(M, H), r)
    act, xo = dev.buffer(M * N * 2), dev.buffer(M * H * 2)
    q = pkg.QmvParams()
    q.pro_mode = pkg.PRO_PRENORM
    q.h_in, q.norm_w, q.x_out = hb.ptr, nb.ptr, xo.ptr
    ks2, _ = launch_qmv(pkg, dev, H, M, q, [(DevQ4(dev, gw, gs, gb), DevQ4(dev, uw, us, ub), act.ptr, pkg.EPI_GATEUP)])
    xn = np.stack([orc.rms_norm_tiles(r[m], nw) for m in range(M)])
    assert np.array_equal(xo.read(np.uint16, M * H).reshape(M, H), xn)
    g = orc.q4_linear(xn, gw, gs, gb, N, H, M, ks2)
    u = orc.q4_linear(xn, uw, us, ub, N, H, M, ks2)
    assert np.array_equal(act.read(np.uint16, M * N), orc.silu_mul(g, u))


@pytest.mark.parametrize("M", [1, 3])
@pytest.mark.parametrize("N", [1001, 17408])
def test_qmv_wide_gateup_equals_four_wave(pkg, orc, dev, M, N):
    """The 16-wave MLP gate/up (17 tiles per workgroup, the 17th tile's five
    group iterations on waves 0..4, summed in iteration order by wave 15)
    against the four-wave kernel on the same inputs, bit for bit: at the
    model's 17408 rows (256 full workgroups) and at 1001 rows (a ragged last
    tile and a last workgroup of 13 tiles whose 17th is out of range); at
    1001 rows also against the oracle (mlp.metal:6-17)."""
    rng = np.random.default_rng(90 + M + N)
    H = 5120
    gw, gs, gb = rand_q4(rng, N, H)
    uw, us, ub = rand_q4(rng, N, H)
    h = bf16((rng.standard_normal((M, H)) * 4).astype(np.float32))
    nw = bf16(rng.uniform(0.9, 1.1, H).astype(np.float32))
    hb, nb = dev.upload(h), dev.upload(nw)
    qg, qu = DevQ4(dev, gw, gs, gb), DevQ4(dev, uw, us, ub)
    runs = []
    for wide in (True, False):
        act, xo = dev.buffer(M * N * 2), dev.buffer(M * H * 2)
        q = pkg.QmvParams()
        q.pro_mode = pkg.PRO_PRENORM
        q.h_in, q.norm_w, q.x_out = hb.ptr, nb.ptr, xo.ptr
        ks, grid = launch_qmv(pkg, dev, H, M, q, [(qg, qu, act.ptr, pkg.EPI_GATEUP)], wide=wide)
        runs.append((act.read(np.uint16, M * N), xo.read(np.uint16, M * H), grid, ks))
    tiles = (N + 3) // 4
    assert runs[0][2] == (tiles + pkg.QMV_WIDE_TILES - 1) // pkg.QMV_WIDE_TILES  # the wide launch ran
    assert runs[1][2] == (tiles + 3) // 4
    assert np.array_equal(runs[0][0], runs[1][0])
    assert np.array_equal(runs[0][1], runs[1][1])
    if N < 2048:
        xn = np.stack([orc.rms_norm_tiles(h[m], nw) for m in range(M)])
        assert np.array_equal(runs[0][1].reshape(M, H), xn)
        g = orc.q4_linear(xn, gw, gs, gb, N, H, M, runs[0][3])
        u = orc.q4_linear(xn, uw, us, ub, N, H, M, runs[0][3])
        assert np.array_equal(runs[0][0], orc.silu_mul(g, u))


@pytest.mark.parametrize("N", [17408, 17411, 18000])
def test_qmv_x_wide9_equals_four_wave(pkg, orc, dev, N):
    """The one-row plain-x launch of 2049..2304 tiles on nine-wave workgroups
    (x staged once per CU) against the four-wave kernel, bit for bit, and the
    oracle: the config-0 shape (2176 tiles, 242 workgroups, the last with 7
    tiles), a ragged last tile (17411 rows) and 2250 full tiles."""
    rng = np.random.default_rng(500 + N)
    K = 5120
    w, s, b = rand_q4(rng, N, K)
    q = DevQ4(dev, w, s, b)
    x = bf16(rng.standard_normal((1, K)).astype(np.float32))
    xb = dev.upload(x)
    runs = []
    for wide in (True, False):
        out = dev.buffer(N * 4)
        p = pkg.QmvParams()
        p.pro_mode = pkg.PRO_LOADX
        p.x_in = xb.ptr
        _, grid = launch_qmv(pkg, dev, K, 1, p, [(q, None, out.ptr, pkg.EPI_STORE)], wide=wide)
        runs.append((grid, out.read(np.float32, N)))
    tiles = (N + 7) // 8
    assert runs[0][0] == (tiles + pkg.QMV_X_WIDE_WAVES - 1) // pkg.QMV_X_WIDE_WAVES
    assert runs[1][0] == (tiles + 3) // 4
    assert same_bits(runs[0][1], runs[1][1])
    assert same_bits(runs[0][1], orc.q4_linear(x, w, s, b, N, K, 1, 1)[0])


@pytest.mark.parametrize("M", [1, 3])
@pytest.mark.parametrize("layer", ["gdn", "attn"])
def test_qmv_wide_inproj_equals_four_wave(pkg, orc, dev, M, layer):
    """The in-projection launches under PRENORM on one workgroup per CU, one
    tile per wave: GDN (qkv 10240 CONV + z 6144 rows = 2048 tiles = 256 x 8
    waves, with the a/b gate contributions) and attention (q 12288 + k 1024 +
    v 1024 = 1792 tiles = 256 x 7). Every output (projections, conv state and
    history slots, gate contributions) equals the four-wave kernel's bit for
    bit, and the projections and causal conv equal the oracle's
    (x = RMSNorm(h), gdn.metal:163-170)."""
    rng = np.random.default_rng(300 + M + (0 if layer == "gdn" else 7))
    K = 5120
    shapes = ([("qkv", 10240, pkg.EPI_CONV), ("z", 6144, pkg.EPI_STORE)] if layer == "gdn" else
              [("q", 12288, pkg.EPI_STORE), ("k", 1024, pkg.EPI_STORE), ("v", 1024, pkg.EPI_STORE)])
    mats = {n: rand_q4(rng, rows, K) for n, rows, _ in shapes}
    qd = {n: DevQ4(dev, *mats[n]) for n in mats}
    h = bf16((rng.standard_normal((M, K)) * 4).astype(np.float32))
    nw = bf16(rng.uniform(0.9, 1.1, K).astype(np.float32))
    hb, nb = dev.upload(h), dev.upload(nw)
    if layer == "gdn":
        gate = [DevQ4(dev, *rand_q4(rng, 48, K)) for _ in range(2)]
        conv_w = bf16(rng.uniform(-0.5, 0.5, 10240 * 4).astype(np.float32))
        conv_state = bf16(rng.standard_normal(3 * 10240).astype(np.float32))
        cwb = dev.upload(conv_w)
    runs = []
    for wide in (True, False):
        outs = {n: dev.buffer(M * rows * 4) for n, rows, _ in shapes}
        p = pkg.QmvParams()
        p.pro_mode = pkg.PRO_PRENORM
        p.h_in, p.norm_w = hb.ptr, nb.ptr
        if layer == "gdn":
            csb, cslot = dev.upload(conv_state), dev.upload(np.zeros(2 * 3 * 10240, np.uint16))
            gab = dev.upload(np.zeros(M * 48 * 192, np.float32))
            p.conv_w, p.conv_state, p.conv_slots, p.conv_slot_stride = cwb.ptr, csb.ptr, cslot.ptr, 3 * 10240
            p.capture = 1 if M == 3 else 0
            p.gate_a_w, p.gate_a_sb = gate[0].wbuf.ptr, gate[0].sbbuf.ptr
            p.gate_b_w, p.gate_b_sb = gate[1].wbuf.ptr, gate[1].sbbuf.ptr
            p.gate_ab = gab.ptr
        _, grid = launch_qmv(pkg, dev, K, M, p, [(qd[n], None, outs[n].ptr, kind) for n, _, kind in shapes], wide=wide)
        run = {n: outs[n].read(np.float32, M * rows).reshape(M, rows) for n, rows, _ in shapes}
        if layer == "gdn":
            run["conv_state"] = csb.read(np.uint16, 3 * 10240)
            run["conv_slots"] = cslot.read(np.uint16, 2 * 3 * 10240)
            run["gate_ab"] = gab.read(np.uint32, M * 48 * 192)
        runs.append((grid, run))
    tiles = sum(rows // 8 for _, rows, _ in shapes)
    assert runs[0][0] == pkg.QMV_WIDE_GROUPS and tiles == pkg.QMV_WIDE_GROUPS * (8 if layer == "gdn" else 7)
    assert runs[1][0] == tiles // 4
    for key, got in runs[0][1].items():
        assert np.array_equal(got.view(np.uint32) if got.dtype == np.float32 else got,
                              runs[1][1][key].view(np.uint32) if got.dtype == np.float32 else runs[1][1][key]), key
    wide = runs[0][1]
    x = np.stack([orc.rms_norm_tiles(h[m], nw) for m in range(M)])
    for n, rows, kind in shapes:
        y = orc.q4_linear(x, *mats[n], rows, K, M, 1)
        if kind == pkg.EPI_CONV:
            conv_out, cs_want, cslots = orc.gdn_conv(y, conv_w, conv_state, M, slots=True)
            assert same_bits(wide[n], conv_out)
            assert np.array_equal(wide["conv_state"], cs_want)
            if M == 3:
                assert np.array_equal(wide["conv_slots"], cslots[:2 * 3 * 10240])
        else:
            assert same_bits(wide[n], y), n


# ---------------------------------------------------------------- config 1
@pytest.mark.parametrize("M", [1, 3])
def test_gdn_layer_config1(pkg, orc, dev, M):
    """One GDN decode layer step: RMSNorm -> fused qkv/z/a/b q4 projections ->
    causal conv + SiLU (+history update) -> q/k RMSNorm, gates -> gated-delta
    recurrence on f32 [48,128,128] state -> gated RMSNorm -> q4 out_proj."""
    rng = np.random.default_rng(1000 + M)
    K = 5120
    hidden = bf16(rng.standard_normal((M, K)).astype(np.float32))
    in_norm = bf16(rng.uniform(0.9, 1.1, K).astype(np.float32))
    mats = {n: rand_q4(rng, rows, K) for n, rows in [("qkv", 10240), ("z", 6144), ("a", 48), ("b", 48)]}
    ow, osc, ob = rand_q4(rng, 5120, 6144)
    conv_w = bf16(rng.uniform(-0.5, 0.5, 10240 * 4).astype(np.float32))
    conv_state = bf16(rng.standard_normal(3 * 10240).astype(np.float32))
    a_log = bf16(rng.uniform(-2, 0, 48).astype(np.float32))
    dt_bias = bf16(rng.uniform(-1, 1, 48).astype(np.float32))
    gnorm = bf16(rng.uniform(0.9, 1.1, 128).astype(np.float32))
    state = (rng.standard_normal(48 * 128 * 128) * 0.01).astype(np.float32)

    # --- oracle
    x = np.stack([orc.rms_norm(hidden[m], in_norm) for m in range(M)])
    proj = {n: orc.q4_linear(x, *mats[n], mats[n][0].shape[0], K, M, 1) for n in mats}
    conv_out, cs_want, cslots = orc.gdn_conv(proj["qkv"], conv_w, conv_state, M, slots=True)
    gated, st_want, _, gslots = orc.gdn_recurrence(conv_out, proj["z"], proj["a"], proj["b"], a_log, dt_bias,
                                                   gnorm, state, M, slots=True)
    branch = orc.q4_linear(gated, ow, osc, ob, 5120, 6144, M, 4)

    # --- GPU
    qd = {n: DevQ4(dev, *mats[n]) for n in mats}
    hb, nb = dev.upload(hidden), dev.upload(in_norm)
    co, zb, ab, bb = dev.buffer(M * 10240 * 4), dev.buffer(M * 6144 * 4), dev.buffer(M * 48 * 4), dev.buffer(M * 48 * 4)
    cwb, csb = dev.upload(conv_w), dev.upload(conv_state)
    cslot = dev.buffer(2 * 3 * 10240 * 2)
    p = pkg.QmvParams()
    p.pro_mode = pkg.PRO_NORM
    p.h_in, p.norm_w = hb.ptr, nb.ptr
    p.conv_w, p.conv_state, p.conv_slots, p.conv_slot_stride = cwb.ptr, csb.ptr, cslot.ptr, 3 * 10240
    p.capture = 1 if M == 3 else 0
    # the decoder's in-projection: qkv and z tiles; a and b as per-group
    # contributions formed by the first 48 workgroups
    gab = dev.buffer(M * 48 * 192 * 4)  # LISA_GDN_GATE_FLOATS per (row, head)
    p.gate_a_w, p.gate_a_sb, p.gate_b_w, p.gate_b_sb = qd["a"].wbuf.ptr, qd["a"].sbbuf.ptr, qd["b"].wbuf.ptr, qd["b"].sbbuf.ptr
    p.gate_ab = gab.ptr
    launch_qmv(pkg, dev, K, M, p, [(qd["qkv"], None, co.ptr, pkg.EPI_CONV), (qd["z"], None, zb.ptr, pkg.EPI_STORE)])
    assert same_bits(co.read(np.float32, M * 10240).reshape(M, 10240), conv_out)
    assert same_bits(zb.read(np.float32, M * 6144).reshape(M, 6144), proj["z"])
    assert np.array_equal(csb.read(np.uint16, 3 * 10240), cs_want)
    # a and b as q4 tiles (the recurrence's raw a/b inputs)
    pab = pkg.QmvParams()
    pab.pro_mode = pkg.PRO_NORM
    pab.h_in, pab.norm_w = hb.ptr, nb.ptr
    launch_qmv(pkg, dev, K, M, pab, [(qd["a"], None, ab.ptr, pkg.EPI_STORE), (qd["b"], None, bb.ptr, pkg.EPI_STORE)])
    assert same_bits(ab.read(np.float32, M * 48).reshape(M, 48), proj["a"])
    assert same_bits(bb.read(np.float32, M * 48).reshape(M, 48), proj["b"])

    al, dtb, gn = dev.upload(a_log), dev.upload(dt_bias), dev.upload(gnorm)
    inv = np.float32(1.0) / np.sqrt(np.float32(128.0))
    oq, sink = DevQ4(dev, ow, osc, ob), dev.buffer(256)
    for source in ("contributions", "tiles"):
        stb = dev.upload(state)
        gslot = dev.buffer(2 * 48 * 128 * 128 * 4)
        gb = dev.buffer(M * 6144 * 2)
        g = pkg.GdnParams()
        g.conv_out, g.z = co.ptr, zb.ptr
        grid = 48
        if source == "contributions":
            g.gate_ab = gab.ptr
            # as the decoder launches it: 20 workgroups per XCD past the heads
            # prefetch the out_proj tiles (they compute nothing)
            g.pf_w, g.pf_sb, g.pf_sink = oq.wbuf.ptr, oq.sbbuf.ptr, sink.ptr
            g.pf_tiles, g.pf_k, grid = 5120 // 8, 6144, 48 + 8 * 20
        else:
            g.a, g.b = ab.ptr, bb.ptr
        g.a_log, g.dt_bias, g.norm_w = al.ptr, dtb.ptr, gn.ptr
        g.state, g.slots, g.slot_stride, g.gated = stb.ptr, gslot.ptr, 48 * 128 * 128, gb.ptr
        g.q_scale, g.k_scale = float(inv * inv), float(inv)
        g.capture = 1 if M == 3 else 0
        dev.dispatch(f"lisa_gdn_recurrence_m{M}", g, (grid,), (512,))
        assert np.array_equal(gb.read(np.uint16, M * 6144).reshape(M, 6144), gated), source
        assert same_bits(stb.read(np.float32, 48 * 128 * 128), st_want), source
    if M == 3:
        for t in range(2):
            assert same_bits(gslot.read(np.float32, 48 * 128 * 128, offset=t * 48 * 128 * 128 * 4),
                             gslots[t * 48 * 128 * 128:(t + 1) * 48 * 128 * 128])
            assert np.array_equal(cslot.read(np.uint16, 3 * 10240, offset=t * 3 * 10240 * 2),
                                  cslots[t * 3 * 10240:(t + 1) * 3 * 10240])

    outb = dev.buffer(M * 5120 * 4)
    po = pkg.QmvParams()
    po.pro_mode = pkg.PRO_LOADX
    po.x_in = gb.ptr
    launch_qmv(pkg, dev, 6144, M, po, [(oq, None, outb.ptr, pkg.EPI_STORE)])
    assert same_bits(outb.read(np.float32, M * 5120).reshape(M, 5120), branch)


def test_gdn_batch3_equals_three_single_steps(pkg, dev):
    """tests/gdn_recurrence_state.rs:70-173 on the HIP kernel: an M=3 dispatch
    equals three M=1 dispatches, output and state bit for bit."""
    rng = np.random.default_rng(5)
    conv = np.zeros((3, 10240), np.float32)
    conv[:, 4096:] = ((np.arange(3 * 6144).reshape(3, 6144) % 127) - 63) * 0.002
    conv[:, :4096] = f32(bf16(rng.standard_normal((3, 4096)).astype(np.float32)))
    z = rng.standard_normal((3, 6144)).astype(np.float32)
    a = rng.standard_normal((3, 48)).astype(np.float32)
    b = rng.standard_normal((3, 48)).astype(np.float32)
    a_log = bf16(rng.uniform(-2, 0, 48).astype(np.float32))
    dt = bf16(rng.uniform(-1, 1, 48).astype(np.float32))
    nw = bf16(rng.uniform(0.9, 1.1, 128).astype(np.float32))
    state0 = (rng.standard_normal(48 * 128 * 128) * 0.01).astype(np.float32)
    bufs = {k: dev.upload(v) for k, v in dict(a_log=a_log, dt=dt, nw=nw).items()}
    inv = np.float32(1.0) / np.sqrt(np.float32(128.0))

    def run(M, rows, state):
        stb = dev.upload(state)
        co, zb, ab, bb = (dev.upload(conv[rows]), dev.upload(z[rows]), dev.upload(a[rows]), dev.upload(b[rows]))
        gb = dev.buffer(M * 6144 * 2)
        g = pkg.GdnParams()
        g.conv_out, g.z, g.a, g.b = co.ptr, zb.ptr, ab.ptr, bb.ptr
        g.a_log, g.dt_bias, g.norm_w = bufs["a_log"].ptr, bufs["dt"].ptr, bufs["nw"].ptr
        g.state, g.gated = stb.ptr, gb.ptr
        g.q_scale, g.k_scale = float(inv * inv), float(inv)
        dev.dispatch(f"lisa_gdn_recurrence_m{M}", g, (48,), (512,))
        return gb.read(np.uint16, M * 6144), stb.read(np.float32, 48 * 128 * 128)

    g3, s3 = run(3, slice(0, 3), state0)
    st = state0
    singles = []
    for t in range(3):
        gt, st = run(1, slice(t, t + 1), st)
        singles.append(gt)
    assert np.array_equal(g3, np.concatenate(singles))
    assert same_bits(s3, st)


# ---------------------------------------------------------------- config 2
def attention_case(pkg, orc, dev, M, ctx, seed):
    rng = np.random.default_rng(seed)
    cap = ctx + 3
    base = ctx - 1 if M == 1 else ctx - 3  # the last row attends over ctx keys
    q_proj = (rng.standard_normal((M, 12288)) * 3).astype(np.float32)
    k_raw = (rng.standard_normal((M, 1024)) * 3).astype(np.float32)
    v_raw = rng.standard_normal((M, 1024)).astype(np.float32)
    qn = bf16(rng.uniform(0.9, 1.1, 256).astype(np.float32))
    kn = bf16(rng.uniform(0.9, 1.1, 256).astype(np.float32))
    kc = bf16(rng.standard_normal(4 * cap * 256).astype(np.float32))
    vc = bf16(rng.standard_normal(4 * cap * 256).astype(np.float32))
    want, kc_w, vc_w = orc.attention(q_proj, k_raw, v_raw, qn, kn, kc, vc, cap, base, M)

    s_max = (cap + 63) // 64
    bufs = dict(q=dev.upload(q_proj), k=dev.upload(k_raw), v=dev.upload(v_raw), qn=dev.upload(qn),
                kn=dev.upload(kn), kc=dev.upload(kc), vc=dev.upload(vc),
                po=dev.buffer(M * 24 * s_max * 256 * 4), pm=dev.buffer(M * 24 * s_max * 2 * 4),
                pos=dev.upload(np.array([base, 0, 0, 0], np.uint32)), g=dev.buffer(M * 6144 * 2))
    a = pkg.AttnParams()
    a.q_proj, a.k_raw, a.v_raw = bufs["q"].ptr, bufs["k"].ptr, bufs["v"].ptr
    a.q_norm_w, a.k_norm_w = bufs["qn"].ptr, bufs["kn"].ptr
    a.key_cache, a.value_cache = bufs["kc"].ptr, bufs["vc"].ptr
    a.part_o, a.part_ml, a.pos, a.gated = bufs["po"].ptr, bufs["pm"].ptr, bufs["pos"].ptr, bufs["g"].ptr
    a.capacity, a.s_max = cap, s_max
    dev.dispatch(f"lisa_attn_partial_m{M}", a, (s_max, 4), (pkg.ATT_PARTIAL_THREADS[M],))
    dev.dispatch(f"lisa_attn_merge_m{M}", a, (24, M), (256,))
    got = bufs["g"].read(np.uint16, M * 6144).reshape(M, 6144)
    return got, want, bufs["kc"].read(np.uint16, 4 * cap * 256), kc_w, bufs["vc"].read(np.uint16, 4 * cap * 256), vc_w


@pytest.mark.parametrize("M,ctx", [(1, 4096), (3, 4096), (1, 1), (3, 3), (1, 65), (1, 100), (3, 130), (1, 32768)])
def test_attention_config2(pkg, orc, dev, M, ctx):
    """Gated GQA decode attention: q/k RMSNorm + partial RoPE, KV append,
    split-K over 64-token slices, flash merge, sigmoid output gate; exact
    past 16k context (the reference's merge is wrong there)."""
    got, want, kc, kcw, vc, vcw = attention_case(pkg, orc, dev, M, ctx, 300 + ctx + M)
    assert np.array_equal(kc, kcw)
    assert np.array_equal(vc, vcw)
    assert np.array_equal(got, want)


def test_attention_batch3_row_equals_single(pkg, orc, dev):
    """tests/attn_sliced.rs:167-188: row 2 of a batch-3 dispatch equals the
    same row decoded alone, bit for bit (slices depend only on the row)."""
    ctx = 1000
    got3, _, kc3, _, vc3, _ = attention_case(pkg, orc, dev, 3, ctx, 77)
    # replay the same inputs as an M=1 dispatch of row 2 after rows 0,1 are cached
    rng = np.random.default_rng(77)
    cap = ctx + 3
    q_proj = (rng.standard_normal((3, 12288)) * 3).astype(np.float32)
    k_raw = (rng.standard_normal((3, 1024)) * 3).astype(np.float32)
    v_raw = rng.standard_normal((3, 1024)).astype(np.float32)
    qn = bf16(rng.uniform(0.9, 1.1, 256).astype(np.float32))
    kn = bf16(rng.uniform(0.9, 1.1, 256).astype(np.float32))
    s_max = (cap + 63) // 64
    bufs = dict(q=dev.upload(q_proj[2:]), k=dev.upload(k_raw[2:]), v=dev.upload(v_raw[2:]), qn=dev.upload(qn),
                kn=dev.upload(kn), kc=dev.upload(kc3), vc=dev.upload(vc3),
                po=dev.buffer(24 * s_max * 256 * 4), pm=dev.buffer(24 * s_max * 2 * 4),
                pos=dev.upload(np.array([ctx - 1, 0, 0, 0], np.uint32)), g=dev.buffer(6144 * 2))
    a = pkg.AttnParams()
    a.q_proj, a.k_raw, a.v_raw = bufs["q"].ptr, bufs["k"].ptr, bufs["v"].ptr
    a.q_norm_w, a.k_norm_w = bufs["qn"].ptr, bufs["kn"].ptr
    a.key_cache, a.value_cache = bufs["kc"].ptr, bufs["vc"].ptr
    a.part_o, a.part_ml, a.pos, a.gated = bufs["po"].ptr, bufs["pm"].ptr, bufs["pos"].ptr, bufs["g"].ptr
    a.capacity, a.s_max = cap, s_max
    dev.dispatch("lisa_attn_partial_m1", a, (s_max, 4), (pkg.ATT_PARTIAL_THREADS[1],))
    dev.dispatch("lisa_attn_merge_m1", a, (24, 1), (256,))
    assert np.array_equal(bufs["g"].read(np.uint16, 6144), got3[2])
