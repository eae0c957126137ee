"""Parity of the Q8 kernels (liblgx on gfx950) with the CPU oracle.

Integer results and every output of the canonical Q8 x Q8 schedule are
compared bit-for-bit; the binary32-activation GEMV within the north star's
1e-3 relative / 1e-4 absolute tolerance.  Inputs come from the oracle's seeded
SplitMix64 streams (config 0: seed 0, config 1: seed 1).
"""
import numpy as np
import pytest

import logicaffeine_amd as lgx

pytestmark = pytest.mark.gpu


def host(t):
    return t.cpu().numpy()


def u16(t):
    return host(t).view(np.uint16)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def config0(orc):
    qs, d = orc.gen_q8_matrix(0, 0, 4864, 896)
    x = orc.gen_normal_f32(0, 2, (896,))
    return qs, d, x


@pytest.fixture(scope="module")
def w0(ctx, orc):
    qs, d, x = config0(orc)
    return qs, d, x, ctx.q8_matrix(qs, d)


def test_repack_matches_oracle_and_round_trips(ctx, orc, w0):
    qs, d, _, W = w0
    assert np.array_equal(host(W.qs), orc.q8_repack_t16(qs))
    assert np.array_equal(u16(W.d), orc.q8_repack_s16(d, 4864, 896))
    bq, bd = ctx.unpack_t16(W.qs, W.d, 4864, 896)
    assert np.array_equal(host(bq), qs)
    assert np.array_equal(u16(bd), d)


@pytest.mark.parametrize("m,k", [(1, 896), (64, 8960), (7, 1536)])
def test_quantize_bit_exact(ctx, orc, m, k):
    x = orc.gen_normal_f32(1, 10 + m, (m, k))
    x[0, :32] = 0.0                      # zero block
    x[-1, 32:64] *= np.float32(1e-30)    # scales in the binary16 subnormal range
    x[-1, 64:96] *= np.float32(1e4)      # large block
    qs, d = ctx.quantize_q8_0(ctx.to_device(x))
    rq, rd = orc.quantize_q8_0(x)
    assert np.array_equal(host(qs), rq)
    assert np.array_equal(u16(d), rd)


def test_quantize_golden_edges(ctx, golden):
    qs, d = ctx.quantize_q8_0(ctx.to_device(golden["edge_x"]))
    assert np.array_equal(host(qs), golden["edge_q"])
    assert np.array_equal(u16(d), golden["edge_d"])


def test_q8_gemv_f32_config0_within_tolerance(ctx, orc, w0):
    qs, d, x, W = w0
    y = host(ctx.q8_gemv_f32(W, ctx.to_device(x)))
    ref = orc.q8_gemv_f32(qs, d, x)
    assert np.all(np.abs(y - ref) <= 1e-4 + 1e-3 * np.abs(ref))


def test_q8q8_gemv_config0_bit_exact(ctx, orc, w0):
    qs, d, x, W = w0
    xq, xd = orc.quantize_q8_0(x[None, :])
    y, s = ctx.q8q8_gemv(W, ctx.to_device(xq[0]), ctx.to_device(xd[0]), blockdots=True)
    assert np.array_equal(host(s), orc.q8_blockdots(qs, xq[0]))
    assert np.array_equal(host(y), orc.q8_gemm(qs, d, xq, xd)[0])


@pytest.mark.parametrize("n,k", [(1536, 8960), (8960, 1536), (32, 2112)])
def test_q8q8_gemv_multirange_bit_exact(ctx, orc, n, k):
    qs, d = orc.gen_q8_matrix(1, 20 + n, n, k)
    x = orc.gen_normal_f32(1, 30 + n, (1, k))
    xq, xd = orc.quantize_q8_0(x)
    W = ctx.q8_matrix(qs, d)
    y = ctx.q8q8_gemv(W, ctx.to_device(xq[0]), ctx.to_device(xd[0]))
    assert np.array_equal(host(y), orc.q8_gemm(qs, d, xq, xd)[0])


@pytest.fixture(scope="module")
def mlp1(ctx, orc):
    """Config 1 (Qwen2.5-1.5B MLP): gate [8960 x 1536] and down [1536 x 8960]."""
    out = {}
    for name, (n, k), stream in (("gate", (8960, 1536), 0), ("down", (1536, 8960), 4)):
        qs, d = orc.gen_q8_matrix(1, stream, n, k)
        out[name] = (qs, d, ctx.q8_matrix(qs, d))
    return out


@pytest.mark.parametrize("m", [1, 8, 32, 64, 100])
@pytest.mark.parametrize("which", ["gate", "down"])
def test_q8_gemm_config1_bit_exact(ctx, orc, mlp1, which, m):
    qs, d, W = mlp1[which]
    x = orc.gen_normal_f32(1, 100 + m, (m, W.k))
    xq, xd = orc.quantize_q8_0(x)
    y = ctx.q8_gemm(W, ctx.to_device(xq), ctx.to_device(xd))
    assert np.array_equal(host(y), orc.q8_gemm(qs, d, xq, xd))


def test_gemm_rows_equal_gemv(ctx, orc, mlp1):
    """Batch invariance across kernels: the MFMA GEMM row i is bit-identical to
    the dot4 GEMV of row i."""
    qs, d, W = mlp1["down"]
    x = orc.gen_normal_f32(1, 7, (5, W.k))
    xq, xd = orc.quantize_q8_0(x)
    gx, gd = ctx.to_device(xq), ctx.to_device(xd)
    y = host(ctx.q8_gemm(W, gx, gd))
    for i in range(5):
        yi = host(ctx.q8q8_gemv(W, gx[i], gd[i]))
        assert np.array_equal(y[i], yi)


def test_golden_fixtures(ctx, golden):
    for name in ("small", "ranges"):
        W = ctx.q8_matrix(golden[f"{name}_qs"], golden[f"{name}_d"])
        y = host(ctx.q8_gemm(W, ctx.to_device(golden[f"{name}_xq"]),
                             ctx.to_device(golden[f"{name}_xd"])))
        ref, absum = golden[f"{name}_y_q8q8"], golden[f"{name}_y_q8q8_abs"]
        assert np.all(np.abs(y - ref) <= 1e-5 * absum)
        yf = host(ctx.q8_gemv_f32(W, ctx.to_device(golden[f"{name}_x"][0])))
        rf = golden[f"{name}_y_f32"]
        assert np.all(np.abs(yf - rf) <= 1e-4 + 1e-3 * np.abs(rf))


def test_shape_errors_and_launch_count(ctx, orc):
    t = ctx.torch
    before = ctx.launch_count
    bad = t.zeros(17 * 64, dtype=t.int8, device=ctx.dev)
    dbad = t.zeros(17 * 2, dtype=t.int16, device=ctx.dev)
    with pytest.raises(lgx.LgxError) as ei:
        ctx.repack_t16(bad.view(17, 64), dbad.view(17, 2))
    assert ei.value.status_name == "LGX_INVALID_ARGUMENT"
    assert ctx.launch_count == before
    qs, d = orc.gen_q8_matrix(0, 50, 16, 64)
    W = ctx.q8_matrix(qs, d)
    assert ctx.launch_count == before + 2      # T16 quants + S16 scales
    ctx.torch.cuda.synchronize()
    assert W.n == 16 and ctx.arch == "gfx950"


def test_workspace_reuse_across_shapes(ctx, orc):
    """Regression: alternating multi-range shapes and batch sizes on one ctx
    reuse (and grow) its range-partials workspace; every call still equals the
    oracle, so no call reads partials another call left behind."""
    cases = []
    for n, k in ((1536, 8960), (8960, 1536), (32, 2112), (1536, 8960)):
        qs, d = orc.gen_q8_matrix(1, 60 + n + k, n, k)
        cases.append((qs, d, ctx.q8_matrix(qs, d)))
    for rep in range(2):
        for i, (qs, d, W) in enumerate(cases):
            m = (1, 3, 64, 70)[(i + rep) % 4]
            x = orc.gen_normal_f32(1, 200 + 10 * i + rep, (m, W.k))
            xq, xd = orc.quantize_q8_0(x)
            gx, gd = ctx.to_device(xq), ctx.to_device(xd)
            y = host(ctx.q8_gemm(W, gx, gd)) if m > 1 else host(ctx.q8q8_gemv(W, gx[0], gd[0]))[None]
            assert np.array_equal(y, orc.q8_gemm(qs, d, xq, xd)), (rep, i, m)


@pytest.mark.parametrize("n,k", [(4864, 896), (8960, 1536), (1536, 8960)])
def test_q8q8_gemv_fused_quantize_bit_exact(ctx, orc, n, k):
    """Fused Q8_0(x) prologue: the GEMV output and the emitted quants/scales
    equal the separate quantise + GEMV and the oracle bit-for-bit."""
    t = ctx.torch
    qs, d = orc.gen_q8_matrix(1, 40 + n, n, k)
    x = orc.gen_normal_f32(1, 50 + n, (1, k))
    x[0, 64:96] = 0.0
    xq, xd = orc.quantize_q8_0(x)
    W = ctx.q8_matrix(qs, d)
    gq = t.empty(k, dtype=t.int8, device=ctx.dev)
    gd = t.empty(k // 32, dtype=t.int16, device=ctx.dev)
    y = ctx.q8q8_gemv_quantize(W, ctx.to_device(x[0]), xq_out=gq, xd_out=gd)
    assert np.array_equal(host(gq), xq[0])
    assert np.array_equal(u16(gd), xd[0])
    assert np.array_equal(host(y), orc.q8_gemm(qs, d, xq, xd)[0])


def _ctx_with_env(**env):
    import os

    old = {k: os.environ.get(k) for k in env}
    os.environ.update({k: str(v) for k, v in env.items()})
    try:
        return lgx.Context(0)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.mark.parametrize("n,k", [(4864, 896), (1536, 8960), (272, 2112)])
def test_kernel_variants_agree(ctx, orc, n, k):
    """The whole-K workgroup GEMV, the per-(tile, range) v_dot4 and MFMA
    GEMVs and the MFMA GEMM at every m-tile width, with one or many row tiles
    per wave, all give the oracle's bits."""
    qs, d = orc.gen_q8_matrix(2, n + k, n, k)
    x = orc.gen_normal_f32(2, 7, (40, k))
    xq, xd = orc.quantize_q8_0(x)
    ref = orc.q8_gemm(qs, d, xq, xd)
    for c in (ctx, _ctx_with_env(LGX_GEMV="dot4"), _ctx_with_env(LGX_GEMV="split"),
              _ctx_with_env(LGX_GEMV="whole"), _ctx_with_env(LGX_GEMV_WGS=4),
              _ctx_with_env(LGX_GEMV_WGS=8), _ctx_with_env(LGX_GEMV_WGS=16),
              _ctx_with_env(LGX_WG_TARGET=3)):
        W = c.q8_matrix(qs, d)
        gx, gd = c.to_device(xq), c.to_device(xd)
        assert np.array_equal(host(c.q8q8_gemv(W, gx[0], gd[0])), ref[0])
        assert np.array_equal(host(c.q8q8_gemv_quantize(W, c.to_device(x[0]))), ref[0])
        for m in (1, 5, 16, 17, 32, 40):
            assert np.array_equal(host(c.q8_gemm(W, gx[:m].contiguous(), gd[:m].contiguous())),
                                  ref[:m]), m
        if c is not ctx:
            c.close()


@pytest.mark.parametrize("n,k,m", [
    (8960, 1536, 128),     # config-1 gate, one range group, whole tiles
    (1536, 8960, 200),     # config-1 down: 9 ranges = 3 groups, ragged m tile
    (272, 2112, 131),      # 17 row tiles (last workgroup tile mostly empty), 1-pair last range
    (4864, 896, 384),      # 3 m tiles
    (512, 18944, 130),     # 19 ranges = 5 groups (4, 4, 4, 4, 3)
    (64, 192, 129),        # 3 pairs: a half-filled last stage
])
def test_tiled_gemm_bit_exact(ctx, orc, n, k, m):
    """The large-M tiled product (T16 activations, group partials, tree over
    the groups) gives the oracle's bits."""
    qs, d = orc.gen_q8_matrix(3, n + k, n, k)
    x = orc.gen_normal_f32(3, m, (m, k))
    xq, xd = orc.quantize_q8_0(x)
    W = ctx.q8_matrix(qs, d)
    y = host(ctx.q8_gemm(W, ctx.to_device(xq), ctx.to_device(xd)))
    assert np.array_equal(y, orc.q8_gemm(qs, d, xq, xd))


@pytest.mark.parametrize("m,tiled_rows", [(1, 0), (16, 0), (64, 0), (140, 0), (64, 32)])
def test_special_scales_bit_exact(ctx, orc, m, tiled_rows):
    """Weight scales -0, the smallest binary16 denormal, the largest finite
    value, +inf (rows 3: its products are +-inf or NaN) and NaN, and
    activation scales that are denormal or zero, through the GEMV (m = 1),
    the streaming products and the tiled product (m = 140, and m = 64 forced
    through 32-row tiles): the outputs equal the oracle's, infinities and
    NaNs in the same places.  The scale of the other block of a pair never
    leaks into a block's scale product."""
    n, k = 256, 2048
    qs, d = orc.gen_q8_matrix(3, 9, n, k)
    d = d.copy()
    d[0, 0] = 0x8000                             # -0
    d[1, 1] = 0x0001                             # smallest denormal
    d[2, 2] = 0x7BFF                             # largest finite
    d[3, 3] = 0x7C00                             # +inf (its pair-mate, block 2, is finite)
    d[5, 4] = 0x7E00                             # NaN
    d[6, 17] = 0x0200                            # denormal
    x = orc.gen_normal_f32(3, 10, (m, k))
    xq, xd = orc.quantize_q8_0(x)
    xd = xd.copy()
    xd[0, 7] = 0x0001                            # denormal activation scale
    xd[m - 1, 8] = 0x0000                        # zero activation scale (nonzero quants)
    ref = orc.q8_gemm(qs, d, xq, xd)
    c = _ctx_with_env(LGX_GEMM_TILED_MIN=2, LGX_GEMM_TILED_ROWS=tiled_rows) if tiled_rows else ctx
    try:
        W = c.q8_matrix(qs, d)
        y = host(c.q8_gemm(W, c.to_device(xq), c.to_device(xd)))
    finally:
        if c is not ctx:
            c.close()
    assert np.isinf(ref[:, 3]).any() and np.isnan(ref[:, 5]).all()
    assert np.array_equal(y, ref, equal_nan=True)


@pytest.mark.parametrize("rows,grp", [(128, 0), (64, 0), (32, 0), (64, 1), (64, 2), (32, 4), (128, 1)])
def test_tiled_gemm_small_m_forced(ctx, orc, rows, grp):
    """LGX_GEMM_TILED_MIN=2 routes every m > 1 through the tiled product with
    128, 64 or 32 activation rows per workgroup and 1, 2 or 4 ranges per
    group (0: chosen by grid size): a ragged row tile, rows spanning
    workgroup tiles and 9 ranges (groups of 4 + 4 + 1, 2 + 2 + 2 + 2 + 1, or
    single ranges) agree with the oracle."""
    n, k = 1536, 8960
    qs, d = orc.gen_q8_matrix(3, 5, n, k)
    x = orc.gen_normal_f32(3, 6, (140, k))
    xq, xd = orc.quantize_q8_0(x)
    ref = orc.q8_gemm(qs, d, xq, xd)
    c = _ctx_with_env(LGX_GEMM_TILED_MIN=2, LGX_GEMM_TILED_ROWS=rows, LGX_GEMM_TILED_GRP=grp)
    try:
        W = c.q8_matrix(qs, d)
        gx, gd = c.to_device(xq), c.to_device(xd)
        for m in (2, 15, 17, 32, 33, 64, 140):
            assert np.array_equal(host(c.q8_gemm(W, gx[:m].contiguous(), gd[:m].contiguous())),
                                  ref[:m]), m
    finally:
        c.close()


@pytest.mark.parametrize("n,k", [(3584, 3584), (1024, 896), (512, 2112), (64, 192), (2048, 18944)])
@pytest.mark.parametrize("rows", [32, 64])
def test_tiled_gemm_stage_sizes_agree(orc, n, k, rows):
    """Grids of at most two workgroups per compute unit run in stages of 4
    pairs, larger ones in stages of 2 (LGX_TILED_S4=0: always 2).  Both
    stage sizes give the oracle's bits at 32 and 64 activation rows per
    workgroup: whole ranges (3584), a range of 14 pairs ending mid-stage
    (896), 33 pairs (2112), 3 pairs (192) and 19 ranges in groups (18944)."""
    qs, d = orc.gen_q8_matrix(5, n + k, n, k)
    x = orc.gen_normal_f32(5, rows, (64, k))
    xq, xd = orc.quantize_q8_0(x)
    ref = orc.q8_gemm(qs, d, xq, xd)
    for s4 in (1, 0):
        c = _ctx_with_env(LGX_GEMM_TILED_MIN=2, LGX_GEMM_TILED_ROWS=rows, LGX_TILED_S4=s4)
        try:
            W = c.q8_matrix(qs, d)
            gx, gd = c.to_device(xq), c.to_device(xd)
            for m in (33, 64):
                assert np.array_equal(host(c.q8_gemm(W, gx[:m].contiguous(), gd[:m].contiguous())),
                                      ref[:m]), (s4, m)
        finally:
            c.close()


@pytest.mark.parametrize("n,k", [(4864, 896), (1536, 8960)])
def test_partials_then_combine_equal_full_product(ctx, orc, n, k):
    """Range partials + lgx_q8_range_combine == the one-call product, and each
    partial is the oracle's chain of that range alone."""
    qs, d = orc.gen_q8_matrix(3, n + k, n, k)
    x = orc.gen_normal_f32(3, 1, (24, k))
    xq, xd = orc.quantize_q8_0(x)
    W = ctx.q8_matrix(qs, d)
    gx, gd = ctx.to_device(xq), ctx.to_device(xd)
    g = lgx.lib().lgx_q8_range_count(k)
    for m in (1, 24):
        part = ctx.q8_gemm_partials(W, gx[:m].contiguous(), gd[:m].contiguous())
        assert tuple(part.shape) == (g, m, n)
        y = host(ctx.range_combine(part))
        assert np.array_equal(y, orc.q8_gemm(qs, d, xq[:m], xd[:m]))
        # partial r alone = the product restricted to range r's 32 blocks
        r = g - 1
        lo, hi = 1024 * r, min(1024 * (r + 1), k)
        pr = orc.q8_gemm(np.ascontiguousarray(qs[:, lo:hi]), np.ascontiguousarray(d[:, lo // 32:hi // 32]),
                         np.ascontiguousarray(xq[:m, lo:hi]), np.ascontiguousarray(xd[:m, lo // 32:hi // 32]))
        assert np.array_equal(host(part[r]), pr)
    p1 = host(ctx.q8q8_gemv_quantize_partials(W, ctx.to_device(x[0])))
    assert np.array_equal(p1, host(ctx.q8_gemm_partials(W, gx[0:1], gd[0:1]))[:, 0, :])


def test_kernel_timing_window(ctx, orc):
    qs, d = orc.gen_q8_matrix(0, 90, 1536, 8960)
    W = ctx.q8_matrix(qs, d)
    x = ctx.to_device(orc.gen_normal_f32(0, 91, (8960,)))
    ctx.kernel_timing(True)
    for _ in range(3):
        ctx.q8q8_gemv_quantize(W, x)
    ctx.kernel_timing(False)
    ctx.q8q8_gemv_quantize(W, x)          # outside the window: not recorded
    stats = [ctx.kernel_stats(f"lgx_k_q8_gemv_grp{w}") for w in (4, 8, 16)]
    n, ms = sum(s[0] for s in stats), sum(s[1] for s in stats)
    assert n == 3 and 0.0 < ms < 100.0
    # the whole-K GEMV applies the range tree itself: no combine launches
    assert ctx.kernel_stats("lgx_k_q8_combine")[0] == 0
    assert ctx.kernel_stats("lgx_k_quantize_q8_0") == (0, 0.0)


def test_grouped_gemv_bit_exact(ctx, orc):
    """One launch over independent matrices of different shapes (config 1's
    gate/up/down, config 0, a 19-range K): each output equals its own
    fused-quantise GEMV and the oracle."""
    shapes = [(8960, 1536), (8960, 1536), (1536, 8960), (4864, 896), (512, 18944)]
    Ws, xs, refs = [], [], []
    for i, (n, k) in enumerate(shapes):
        qs, d = orc.gen_q8_matrix(4, 100 + i, n, k)
        x = orc.gen_normal_f32(4, 200 + i, (1, k))
        xq, xd = orc.quantize_q8_0(x)
        Ws.append(ctx.q8_matrix(qs, d))
        xs.append(ctx.to_device(x[0]))
        refs.append(orc.q8_gemm(qs, d, xq, xd)[0])
    before = ctx.launch_count
    ys = ctx.q8q8_gemv_quantize_group(Ws, xs)
    assert ctx.launch_count == before + 1
    for y, ref, W, x in zip(ys, refs, Ws, xs):
        assert np.array_equal(host(y), ref)
        assert np.array_equal(host(ctx.q8q8_gemv_quantize(W, x)), ref)
    c8 = _ctx_with_env(LGX_GEMV_WGS=8)          # eight-wave workgroups
    for (n, k), ref, i in zip(shapes, refs, range(len(shapes))):
        qs, d = orc.gen_q8_matrix(4, 100 + i, n, k)
        Ws[i] = c8.q8_matrix(qs, d)
        xs[i] = c8.to_device(orc.gen_normal_f32(4, 200 + i, (1, k))[0])
    for y, ref in zip(c8.q8q8_gemv_quantize_group(Ws, xs), refs):
        assert np.array_equal(host(y), ref)
    c8.close()


def test_grouped_gemv_long_k_and_errors(ctx, orc):
    """The longest K (32 ranges, two per wave) in a group; the whole-K variant
    rejects it for LDS, and single products then take the per-range path."""
    qs, d = orc.gen_q8_matrix(5, 1, 32, 32768)
    x = orc.gen_normal_f32(5, 2, (1, 32768))
    xq, xd = orc.quantize_q8_0(x)
    ref = orc.q8_gemm(qs, d, xq, xd)[0]
    W = ctx.q8_matrix(qs, d)
    gx = ctx.to_device(x[0])
    assert np.array_equal(host(ctx.q8q8_gemv_quantize_group([W], [gx])[0]), ref)
    with pytest.raises(lgx.LgxError):
        ctx.q8q8_gemv_quantize_group([W] * 9, [gx] * 9)
    cw = _ctx_with_env(LGX_GEMV="whole")
    Ww = cw.q8_matrix(qs, d)
    gw = cw.to_device(x[0])
    with pytest.raises(lgx.LgxError) as e:
        cw.q8q8_gemv_quantize_group([Ww], [gw])
    assert e.value.status_name == "LGX_UNSUPPORTED"
    assert np.array_equal(host(cw.q8q8_gemv_quantize(Ww, gw)), ref)
    assert np.array_equal(host(cw.q8q8_gemv(Ww, cw.to_device(xq[0]), cw.to_device(xd[0]))), ref)
    cw.close()


@pytest.mark.parametrize("n,k", [(37888, 3584), (3584, 18944), (152064, 3584)])
def test_q8_gemm_7b_shapes_m64_streaming_and_tiled(ctx, orc, n, k):
    """The config-4 (Qwen2.5-7B) products at the decode batch M = 64: the
    fused gate|up [37888 x 3584], down [3584 x 18944] (19 ranges) and the
    Q8_0 lm_head [152064 x 3584], the largest n in the system, through the
    streaming kernel and through the 32-row tiled product the 7B decode uses,
    against the oracle bit for bit."""
    m = 64
    qs, d = orc.gen_q8_matrix(4, 7000 + n % 1000 + k % 100, n, k)
    x = orc.gen_normal_f32(4, 7100 + n % 1000, (m, k))
    xq, xd = orc.quantize_q8_0(x)
    ref = orc.q8_gemm(qs, d, xq, xd)
    cs = _ctx_with_env(LGX_GEMM_TILED_MIN=100000)       # the streaming 64-row kernel
    for c in (ctx, cs):                                 # ctx: the tiled product (m >= 33)
        W = c.q8_matrix(qs, d)
        y = host(c.q8_gemm(W, c.to_device(xq), c.to_device(xd)))
        assert np.array_equal(y, ref), c is cs
        del W
    cs.close()


@pytest.mark.parametrize("m", [2, 8, 16, 17, 32, 33, 64, 100])
def test_grouped_gemm_bit_exact(ctx, orc, m):
    """lgx_q8_gemm_quantize_group: the quantisation of every activation
    matrix, the products and the range trees of several matrices in one
    launch up to 8 rows (lgx_k_q8_gemm_grpm16, where the device's LDS per
    workgroup holds every range's rows) or three (streaming 16-row kernels
    below 17 rows, tiled from 17), each output bit-identical to the oracle's
    Q8_0 + canonical product: config 1's gate / up / down, a single tile of
    one 64-column pair, a K of two ranges (the second partial), a ragged last
    row tile."""
    shapes = [(8960, 1536), (8960, 1536), (1536, 8960), (48, 64), (80, 1088)]
    Ws, xs, refs = [], [], []
    for i, (n, k) in enumerate(shapes):
        qs, d = orc.gen_q8_matrix(7, 300 + i, n, k)
        x = orc.gen_normal_f32(7, 400 + i + m, (m, k))
        xq, xd = orc.quantize_q8_0(x)
        Ws.append(ctx.q8_matrix(qs, d))
        xs.append(ctx.to_device(x))
        refs.append(orc.q8_gemm(qs, d, xq, xd))
    before = ctx.launch_count
    ys = ctx.q8_gemm_quantize_group(Ws, xs)
    assert ctx.launch_count - before in ((1, 2, 3) if m <= 8 else (2, 3))
    for i, (y, ref) in enumerate(zip(ys, refs)):
        assert np.array_equal(bits(host(y)), bits(ref)), (m, shapes[i])
    # a group of one and a repeat with other inputs (stale workspace)
    y1 = ctx.q8_gemm_quantize_group([Ws[4]], [xs[4]])[0]
    assert np.array_equal(bits(host(y1)), bits(refs[4]))
    x2 = orc.gen_normal_f32(7, 999, (m, 1536))
    xq2, xd2 = orc.quantize_q8_0(x2)
    qs0, d0 = orc.gen_q8_matrix(7, 300, 8960, 1536)
    y2 = ctx.q8_gemm_quantize_group([Ws[0]], [ctx.to_device(x2)])[0]
    assert np.array_equal(bits(host(y2)), bits(orc.q8_gemm(qs0, d0, xq2, xd2)))


@pytest.mark.parametrize("m", [2, 3, 5, 8])
def test_grouped_gemm_small_m_one_launch(ctx, orc, m):
    """2..8 rows of a group whose matrices have at most four ranges go
    through lgx_k_q8_gemm_grpm16 in one launch (the rows' Q8_0 staged per
    range in LDS, the rows as the MFMA's A operand, rows past m zeros, the
    tree over the ranges in the same workgroup): every output bit-identical
    to the oracle, and to the three-launch path (LGX_GEMM_GRPM=0)."""
    shapes = [(8960, 1536), (1536, 4096), (48, 64), (80, 1088), (160, 2112)]
    Ws, xs, refs = [], [], []
    for i, (n, k) in enumerate(shapes):
        qs, d = orc.gen_q8_matrix(8, 700 + i, n, k)
        x = orc.gen_normal_f32(8, 800 + i + m, (m, k))
        x[0, :32] = 0.0                          # a zero block: scale 0, quants 0
        xq, xd = orc.quantize_q8_0(x)
        Ws.append(ctx.q8_matrix(qs, d))
        xs.append(ctx.to_device(x))
        refs.append(orc.q8_gemm(qs, d, xq, xd))
    before = ctx.launch_count
    ys = ctx.q8_gemm_quantize_group(Ws, xs)
    assert ctx.launch_count - before == 1
    for i, (y, ref) in enumerate(zip(ys, refs)):
        assert np.array_equal(bits(host(y)), bits(ref)), (m, shapes[i])
    c3 = _ctx_with_env(LGX_GEMM_GRPM="0")
    Ws3 = [c3.q8_matrix(*orc.gen_q8_matrix(8, 700 + i, n, k)) for i, (n, k) in enumerate(shapes)]
    before = c3.launch_count
    ys3 = c3.q8_gemm_quantize_group(Ws3, [c3.to_device(host(x)) for x in xs])
    assert c3.launch_count - before in (2, 3)
    for y, y3 in zip(ys, ys3):
        assert np.array_equal(bits(host(y)), bits(host(y3)))
    del Ws3, ys3
    c3.close()


@pytest.mark.parametrize("m,env", [(160, {}), (64, dict(LGX_GEMM_TILED_ROWS="64"))],
                         ids=["tiled128-rows", "tiled64-rows"])
def test_grouped_gemm_other_kernel_forms(orc, m, env):
    """The grouped product's other tiled forms: 128-row tiles (m >= 128) and
    64-row tiles (forced), each output bit-identical to the oracle."""
    c = _ctx_with_env(**env)
    shapes = [(8960, 1536), (1536, 8960), (80, 1088)]
    Ws, xs, refs = [], [], []
    for i, (n, k) in enumerate(shapes):
        qs, d = orc.gen_q8_matrix(7, 500 + i, n, k)
        x = orc.gen_normal_f32(7, 600 + i + m, (m, k))
        xq, xd = orc.quantize_q8_0(x)
        Ws.append(c.q8_matrix(qs, d))
        xs.append(c.to_device(x))
        refs.append(orc.q8_gemm(qs, d, xq, xd))
    ys = c.q8_gemm_quantize_group(Ws, xs)
    for i, (y, ref) in enumerate(zip(ys, refs)):
        assert np.array_equal(bits(host(y)), bits(ref)), (m, shapes[i])
    del Ws, xs, ys
    c.close()


def test_grouped_gemm_m1_and_errors(ctx, orc):
    """m = 1 is the grouped GEMV; bad counts, row counts and shapes are
    refused before anything runs."""
    qs, d = orc.gen_q8_matrix(8, 1, 256, 512)
    x = orc.gen_normal_f32(8, 2, (1, 512))
    xq, xd = orc.quantize_q8_0(x)
    W = ctx.q8_matrix(qs, d)
    gx = ctx.to_device(x)
    before = ctx.launch_count
    y = ctx.q8_gemm_quantize_group([W], [gx])[0]
    assert ctx.launch_count == before + 1
    assert np.array_equal(bits(host(y)), bits(orc.q8_gemm(qs, d, xq, xd)))
    with pytest.raises(lgx.LgxError) as e:
        ctx.q8_gemm_quantize_group([W] * 9, [gx] * 9)
    assert e.value.status_name == "LGX_OUT_OF_BOUNDS"
    with pytest.raises(ValueError):
        ctx.q8_gemm_quantize_group([W], [ctx.to_device(orc.gen_normal_f32(8, 3, (2, 256)))])
