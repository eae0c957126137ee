"""Parity of the decode-step glue kernels (embedding gather, RMSNorm + Q8_0,
RoPE + paged KV append, SwiGLU + Q8_0, binary16 lm_head, argmax) with the
CPU oracle, bit for bit, through their standalone C-ABI entry points.  The
same kernels run inside lgx_qwen_decode_step (checked in test_gpu_model)."""
import numpy as np
import pytest

import logicaffeine_amd as lgx

pytestmark = pytest.mark.gpu


def host(t):
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_embed_gathers_binary16_rows(ctx, orc):
    rng = np.random.default_rng(1)
    vocab, h = 1000, 256
    emb = orc.f32_to_f16(rng.standard_normal((vocab, h)).astype(np.float32))
    tok = np.array([0, 999, 17, 17, -5, 1000, 123456], np.int32)
    out = host(ctx.embed_f16(ctx.to_device(emb), ctx.to_device(tok)))
    want = orc.f16_to_f32(emb[np.clip(tok, 0, vocab - 1)])
    assert np.array_equal(bits(out), bits(want))


@pytest.mark.parametrize("m,n", [(1, 64), (3, 256), (5, 896), (32, 896), (96, 896), (64, 1024),
                                 (70, 960), (2, 1000), (65, 1000), (4, 3584), (2, 8192)])
def test_rmsnorm_quant_bit_exact(ctx, orc, m, n):
    rng = np.random.default_rng(n + m)
    x = (rng.standard_normal((m, n)) * rng.uniform(0.01, 30, size=(m, 1))).astype(np.float32)
    w = rng.uniform(0.5, 1.5, size=n).astype(np.float32)
    if m > 2:
        x[2] = 0.0   # zero row: y = 0, q = 0, d = 0
    q8 = n % 32 == 0
    y, xq, xd = ctx.rmsnorm_quant(ctx.to_device(x), ctx.to_device(w), 1e-6, y=True, q8=q8)
    ref = orc.rmsnorm(x, w, 1e-6)
    assert np.array_equal(bits(host(y)), bits(ref))
    if q8:
        rq, rd = orc.quantize_q8_0(ref)
        assert np.array_equal(host(xq), rq)
        assert np.array_equal(host(xd).view(np.uint16), rd)
        # Q8_0 only (no binary32 output) gives the same quants
        _, xq2, xd2 = ctx.rmsnorm_quant(ctx.to_device(x), ctx.to_device(w), 1e-6, y=False)
        assert np.array_equal(host(xq2), rq)
        assert np.array_equal(host(xd2).view(np.uint16), rd)


def _tree_rows(part):
    """Canonical pairwise tree over axis 0 of part[nr][m][n] (oracle)."""
    from oracle import oracle as orc

    nr, m, n = part.shape
    flat = part.reshape(nr, -1)
    return np.array([orc.tree_sum(flat[:, i].copy()) for i in range(flat.shape[1])],
                    np.float32).reshape(m, n)


@pytest.mark.parametrize("m,n,nr", [(3, 896, 1), (4, 896, 5), (80, 896, 5), (64, 896, 8), (66, 256, 8),
                                    (64, 1024, 3), (71, 64, 2), (64, 1000, 1), (2, 3584, 4), (5, 3584, 19),
                                    (2, 4096, 8), (2, 4096, 20), (2, 3584, 21), (1, 8192, 32),
                                    (2, 1000, 9), (1, 4096, 13), (3, 1000, 4), (2, 2048, 6),
                                    (2, 2052, 3)])
def test_add_rmsnorm_quant_bit_exact(ctx, orc, m, n, nr):
    """Residual form: h += tree of the range partials (one wave per row for
    64+ rows of n % 4 == 0, n <= 1024, nr <= 8; the float4-slot kernels for
    n <= 4096, nr <= 20, one slot per thread up to n = 2048 and nr = 8; the
    general kernel past those), written back, then the RMSNorm + Q8_0 of the
    new h."""
    rng = np.random.default_rng(m * 7 + n + nr)
    part = rng.standard_normal((nr, m, n)).astype(np.float32)
    h = (rng.standard_normal((m, n)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, size=n).astype(np.float32)
    hd = ctx.to_device(h)
    q8 = n % 32 == 0
    y, xq, xd = ctx.add_rmsnorm_quant(ctx.to_device(part), hd, ctx.to_device(w), 1e-6, q8=q8)
    h_ref = (h + _tree_rows(part)).astype(np.float32)
    assert np.array_equal(bits(host(hd)), bits(h_ref))
    ref = orc.rmsnorm(h_ref, w, 1e-6)
    assert np.array_equal(bits(host(y)), bits(ref))
    if q8:
        rq, rd = orc.quantize_q8_0(ref)
        assert np.array_equal(host(xq), rq)
        assert np.array_equal(host(xd).view(np.uint16), rd)


# a workgroup holds 256 rotation pairs of a row: d = 96 and 40 put parts of
# several heads (and the v heads' copies) in one workgroup, 32/8/128 fills
# 12 workgroups exactly
@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (28, 4, 128), (12, 2, 128), (4, 4, 64),
                                      (6, 2, 96), (3, 1, 40), (32, 8, 128)])
def test_rope_kv_append_bit_exact(ctx, orc, hq, hkv, d):
    rng = np.random.default_rng(hq * 1000 + d)
    B, max_seq = 5, 700
    maxp = -(-max_seq // 16)
    num_pages = B * maxp
    qn = (hq + 2 * hkv) * d
    qkv = rng.standard_normal((B, qn)).astype(np.float32)
    bias = (rng.standard_normal(qn) * 0.02).astype(np.float32)
    cos_t, sin_t = orc.rope_tables(max_seq, d, 1e6)
    pos = np.array([0, 1, 15, 16, 699], np.int32)
    pt = rng.permutation(num_pages).astype(np.int32).reshape(B, maxp)
    k0 = np.zeros((num_pages, hkv, 16, d), np.uint16)
    kp, vp = ctx.to_device(k0), ctx.to_device(k0)
    q = host(ctx.rope_kv_append(ctx.to_device(qkv), ctx.to_device(bias), ctx.to_device(cos_t),
                                ctx.to_device(sin_t), ctx.to_device(pos), ctx.to_device(pt),
                                kp, vp, hq, max_seq))
    kh, vh = host(kp).view(np.uint16), host(vp).view(np.uint16)
    kw, vw = k0.copy(), k0.copy()
    for b in range(B):
        r = (qkv[b] + bias).astype(np.float32)
        rot = orc.rope(r[:(hq + hkv) * d].reshape(hq + hkv, d), cos_t[pos[b]], sin_t[pos[b]])
        assert np.array_equal(bits(q[b]), bits(rot[:hq])), b
        page, slot = pt[b, pos[b] // 16], pos[b] % 16
        kw[page, :, slot] = orc.f32_to_f16(rot[hq:])
        vw[page, :, slot] = orc.f32_to_f16(r[(hq + hkv) * d:].reshape(hkv, d))
    assert np.array_equal(kh, kw)   # appended slots right, every other slot untouched
    assert np.array_equal(vh, vw)


def test_rope_without_bias_and_position_zero_is_identity(ctx, orc):
    rng = np.random.default_rng(7)
    hq, hkv, d, max_seq = 2, 1, 64, 32
    qkv = rng.standard_normal((1, (hq + 2 * hkv) * d)).astype(np.float32)
    cos_t, sin_t = orc.rope_tables(max_seq, d, 1e6)
    z = np.zeros((2, hkv, 16, d), np.uint16)
    q = host(ctx.rope_kv_append(ctx.to_device(qkv), None, ctx.to_device(cos_t),
                                ctx.to_device(sin_t), ctx.to_device(np.zeros(1, np.int32)),
                                ctx.to_device(np.array([[1, 0]], np.int32)), ctx.to_device(z),
                                ctx.to_device(z), hq, max_seq))
    assert np.array_equal(bits(q[0].reshape(-1)), bits(qkv[0, :hq * d]))


@pytest.mark.parametrize("m,inter", [(1, 64), (3, 512), (2, 4864), (4, 18944)])
def test_swiglu_quant_bit_exact(ctx, orc, m, inter):
    rng = np.random.default_rng(inter + m)
    gu = (rng.standard_normal((m, 2 * inter)) * 4).astype(np.float32)
    gu[0, :8] = [0.0, -0.0, 90.0, -90.0, 1e-30, -1e-30, 20.0, -20.0]
    y, xq, xd = ctx.swiglu_quant(ctx.to_device(gu))
    ref = orc.swiglu(gu)
    assert np.array_equal(bits(host(y)), bits(ref))
    rq, rd = orc.quantize_q8_0(ref)
    assert np.array_equal(host(xq), rq)
    assert np.array_equal(host(xd).view(np.uint16), rd)


@pytest.mark.parametrize("m,h,vocab", [(1, 64, 300), (5, 256, 1000), (64, 896, 2048),
                                       (70, 896, 1000), (3, 1536, 700), (65, 2048, 300),
                                       (2, 8192, 130)])
def test_lm_head_f16_bit_exact(ctx, orc, m, h, vocab):
    """Chains per 1024-column range and the pairwise tree over the ranges
    (h > 1024: range partials, then the tree) equal the oracle's logits."""
    rng = np.random.default_rng(m * h + vocab)
    x = rng.standard_normal((m, h)).astype(np.float32)
    E = orc.f32_to_f16((rng.standard_normal((vocab, h)) * 0.02).astype(np.float32))
    out = host(ctx.lm_head_f16(ctx.to_device(x), ctx.to_device(E)))
    assert np.array_equal(bits(out), bits(orc.lm_head_f16(x, E)))


@pytest.mark.parametrize("m,h,vocab", [(1, 64, 300), (5, 256, 1000), (17, 896, 2048),
                                       (64, 1024, 4160), (32, 896, 151936), (5, 1536, 1000),
                                       (20, 3072, 700), (2, 8192, 130)])
def test_lm_head_f16_t64_bit_exact(ctx, orc, m, h, vocab):
    """The T64 path (repacked embedding, activations in SGPRs) gives the
    oracle's logits bit for bit, including a ragged last row group and a
    partial last group of 16 activation rows."""
    rng = np.random.default_rng(m + h + vocab)
    x = rng.standard_normal((m, h)).astype(np.float32)
    E = orc.f32_to_f16((rng.standard_normal((vocab, h)) * 0.02).astype(np.float32))
    Et = ctx.f16_repack_t64(ctx.to_device(E))
    # the documented layout: unit (g, j), lane l = columns [8j, 8j+8) of row 64g + l
    g = -(-vocab // 64)
    Ep = np.zeros((g * 64, h), np.uint16)
    Ep[:vocab] = E
    want = Ep.reshape(g, 64, h // 8, 8).transpose(0, 2, 1, 3).reshape(-1)
    assert np.array_equal(host(Et).view(np.uint16), want)
    out = host(ctx.lm_head_f16_t64(ctx.to_device(x), Et, vocab))
    if vocab > 4096:                             # the oracle chain on a row sample
        rows = np.unique(np.r_[rng.integers(0, vocab, 3000), 0, vocab - 1])
        assert np.array_equal(bits(out[:, rows]), bits(orc.lm_head_f16(x, E[rows])))
    else:
        assert np.array_equal(bits(out), bits(orc.lm_head_f16(x, E)))


def test_lm_head_one_hot_selects_embedding_column(ctx, orc):
    rng = np.random.default_rng(3)
    h, vocab = 128, 512
    E = orc.f32_to_f16(rng.standard_normal((vocab, h)).astype(np.float32))
    x = np.zeros((2, h), np.float32)
    x[0, 5] = 1.0
    x[1, 127] = -2.0
    out = host(ctx.lm_head_f16(ctx.to_device(x), ctx.to_device(E)))
    Ef = orc.f16_to_f32(E)
    assert np.array_equal(out[0], Ef[:, 5])
    assert np.array_equal(out[1], -2.0 * Ef[:, 127])


def test_argmax_policy(ctx, orc):
    rng = np.random.default_rng(11)
    V = 151936
    x = rng.standard_normal((8, V)).astype(np.float32)
    x[1, 100] = x[1, 5000] = 50.0               # tie -> lower index
    x[2, :] = np.nan                            # all NaN -> 0
    x[3, :] = -np.inf
    x[3, 77] = np.nan                           # -inf everywhere, NaN skipped -> 0
    x[4, :] = 0.0
    x[4, 9] = -0.0                              # -0 == +0 -> first index 0
    x[5, 0] = np.nan
    x[5, 1] = 80.0                              # leading NaN skipped
    x[6, V - 1] = 1e30                          # last element
    out = host(ctx.argmax(ctx.to_device(x)))
    want = [orc.argmax(r) for r in x]
    assert list(out) == want
    assert want[1] == 100 and want[2] == 0 and want[4] == 0 and want[5] == 1 and want[6] == V - 1


def test_glue_argument_errors(ctx):
    t = ctx.torch
    x = t.zeros((2, 64), dtype=t.float32, device=ctx.dev)
    with pytest.raises(lgx.LgxError) as e:
        ctx.lm_head_f16(t.zeros((1, 8256), dtype=t.float32, device=ctx.dev),    # h > 8192
                        t.zeros((4, 8256), dtype=t.int16, device=ctx.dev))
    assert e.value.status_name == "LGX_UNSUPPORTED"
    with pytest.raises(lgx.LgxError) as e:          # m > 64 on the T64 path
        ctx.lm_head_f16_t64(t.zeros((65, 64), dtype=t.float32, device=ctx.dev),
                            t.zeros(64 * 64, dtype=t.int16, device=ctx.dev), 64)
    assert e.value.status_name == "LGX_UNSUPPORTED"
    with pytest.raises(lgx.LgxError):
        ctx.rmsnorm_quant(t.zeros((1, 8224), dtype=t.float32, device=ctx.dev), x[0], 1e-6)
    with pytest.raises(lgx.LgxError):
        ctx.swiglu_quant(t.zeros((1, 2 * 40), dtype=t.float32, device=ctx.dev))
