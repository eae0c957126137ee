"""lgx_q8_gemm_noalloc against lgx_q8_gemm (and the oracle).

The allocation-free entry point keeps its intermediates in the library's
fixed device scratch array, so its results must equal lgx_q8_gemm's bit for
bit on every path: the M = 1 GEMV, the streaming M < 128 kernels with range
partials, and the tiled large-m product with its T16 activation copy and
group partials.  Each case runs two calls in a row on the shared scratch, the
second with a smaller input, so the second call cannot lean on a clean array.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _q8(ctx, orc, n, k, stream):
    qs, d = orc.gen_q8_matrix(7, stream, n, k)
    return qs, d, ctx.q8_matrix(qs, d)


def _acts(ctx, orc, m, k, stream):
    x = orc.gen_normal_f32(7, stream, (m, k))
    xq, xd = orc.quantize_q8_0(x)
    return xq, xd, ctx.to_device(xq), ctx.to_device(xd.view(np.int16))


def _bits(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("n,k,ms", [
    (1536, 8960, (40, 9)),      # streaming kernels, 9 range partials + combine
    (8960, 1536, (64, 1)),      # streaming, then the grouped M = 1 GEMV
    (8960, 1536, (200, 130)),   # tiled product (T16 copy; one group straight into y)
    (1536, 8960, (160, 128)),   # tiled product with group partials + combine
])
def test_noalloc_equals_q8_gemm_two_calls(ctx, orc, n, k, ms):
    t = ctx.torch
    qs, d, W = _q8(ctx, orc, n, k, 100 + n % 97 + k % 89)
    y = t.full((ms[0], n), float("nan"), dtype=t.float32, device=ctx.dev)
    for i, m in enumerate(ms):
        xq, xd, gq, gd = _acts(ctx, orc, m, k, 300 + 10 * i + m)
        want = ctx.q8_gemm(W, gq, gd)
        got = ctx.q8_gemm_noalloc(W, gq, gd, y[:m])
        t.cuda.synchronize()
        assert np.array_equal(_bits(got), _bits(want)), (n, k, m)
        if i == 0:
            assert np.array_equal(_bits(got), orc.q8_gemm(qs, d, xq, xd).view(np.uint32))


def test_noalloc_rejects_oversized_scratch_and_runs_untimed(ctx, orc):
    """A product whose partials exceed the scratch limit fails with
    LGX_OUT_OF_BOUNDS before launching; with per-kernel timing on, the
    no-alloc call still runs (untimed) and equals lgx_q8_gemm."""
    import logicaffeine_amd as lgx

    t = ctx.torch
    n = k = 8960                      # tiled product: 3 groups x 400 x 8960 x 4 B > 32 MiB
    W = ctx.q8_matrix(*orc.gen_q8_matrix(7, 501, n, k))
    m = 400
    gq = t.zeros((m, k), dtype=t.int8, device=ctx.dev)
    gd = t.zeros((m, k // 32), dtype=t.int16, device=ctx.dev)
    y = t.full((m, n), 7.0, dtype=t.float32, device=ctx.dev)
    before = ctx.launch_count
    with pytest.raises(lgx.LgxError) as e:
        ctx.q8_gemm_noalloc(W, gq, gd, y)
    assert e.value.status_name == "LGX_OUT_OF_BOUNDS"
    assert ctx.launch_count == before
    t.cuda.synchronize()
    assert bool((y == 7.0).all())
    qs, d, W2 = _q8(ctx, orc, 1536, 8960, 502)
    _, _, gq2, gd2 = _acts(ctx, orc, 24, 8960, 503)
    ctx.kernel_timing(True)
    try:
        got = ctx.q8_gemm_noalloc(W2, gq2, gd2, t.empty((24, 1536), dtype=t.float32, device=ctx.dev))
        assert ctx.kernel_stats("lgx_k_q8_gemm_mfma32") == (0, 0.0)
    finally:
        ctx.kernel_timing(False)
    want = ctx.q8_gemm(W2, gq2, gd2)
    t.cuda.synchronize()
    assert np.array_equal(_bits(got), _bits(want))
