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
    back = ctx.unpack_t16(W.qs, 4864, 896)
    assert np.array_equal(host(back), qs)


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
    with pytest.raises(lgx.LgxError) as ei:
        ctx.repack_t16(bad.view(17, 64))
    assert ei.value.status_name == "LGX_INVALID_ARGUMENT"
    assert ctx.launch_count == before
    qs, d = orc.gen_q8_matrix(0, 50, 16, 64)
    W = ctx.q8_matrix(qs, d)
    assert ctx.launch_count == before + 1
    ctx.torch.cuda.synchronize()
    assert W.n == 16 and ctx.arch == "gfx950"
