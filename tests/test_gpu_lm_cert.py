"""The certified greedy lm_head (lgx_lm_head_argmax_f16): binary16 MFMA logits
with an error bound, exact chains only for the rows within the bound of the
largest lower bound.  Its token must be the token of the full logits
(lgx_lm_head_f16_t64, bit-exact against the oracle in test_gpu_glue, followed
by lgx_argmax), for every x -- including rows taking the exact fallback
(zero, NaN, inf, out-of-range scale) and ties that overflow a slice's
candidate list.  The bound itself is checked against the exact logits."""
import numpy as np
import pytest

import logicaffeine_amd as lgx

pytestmark = pytest.mark.gpu

SLICE = 640          # vocabulary rows per certification workgroup


def host(t):
    return t.cpu().numpy()


def emb_device(ctx, vocab, h, seed, sigma=0.02):
    t = ctx.torch
    g = t.Generator(device=ctx.dev)
    g.manual_seed(seed)
    e = (t.randn((vocab, h), generator=g, device=ctx.dev) * sigma).to(t.float16)
    return e.view(t.int16).contiguous()


def x_rows(m, h, seed):
    """Rows over the scales the path meets, and the ones it hands to the
    exact fallback."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, h)).astype(np.float32)
    x *= rng.uniform(0.05, 20.0, size=(m, 1)).astype(np.float32)
    special = [
        lambda r: r,
        lambda r: np.where(np.arange(h) % 97 == 3, r * 300.0, r),   # outlier columns
        lambda r: r * 1e-10,                                        # small, certified
        lambda r: r * 1e15,                                         # large, certified
        lambda r: r * 1e-25,                                        # below 2^-60: exact rows
        lambda r: r * 1e30,                                         # above 2^60: exact rows
        lambda r: np.zeros_like(r),                                 # all logits 0: token 0
        lambda r: np.where(np.arange(h) == 7, np.nan, r),           # NaN: token 0
        lambda r: np.where(np.arange(h) == 9, np.inf, r),           # inf
    ]
    for i in range(min(m, len(special))):
        x[i] = special[i](x[i]).astype(np.float32)
    return x


def full_tokens(ctx, x_dev, emb_t64, vocab):
    return host(ctx.argmax(ctx.lm_head_f16_t64(x_dev, emb_t64, vocab)))


@pytest.mark.parametrize("m,h,vocab", [(1, 64, 300), (5, 256, 1000), (17, 896, 2048),
                                       (16, 960, 5003), (32, 1024, 7000), (32, 896, 151936)])
def test_certified_token_is_the_full_argmax(ctx, m, h, vocab):
    E = emb_device(ctx, vocab, h, seed=m + h + vocab)
    Et = ctx.f16_repack_t64(E)
    rc = ctx.lm_head_rowconst(E)
    for seed in range(3):
        x = ctx.to_device(x_rows(m, h, 100 * seed + m))
        got = host(ctx.lm_head_argmax_f16(x, E, Et, rc))
        want = full_tokens(ctx, x, Et, vocab)
        assert np.array_equal(got, want), (seed, np.nonzero(got != want))


def test_certified_token_small_vocab_against_oracle(ctx, orc):
    """The whole pick against the CPU oracle's chains and argmax."""
    rng = np.random.default_rng(8)
    m, h, vocab = 9, 128, 700
    E = orc.f32_to_f16((rng.standard_normal((vocab, h)) * 0.05).astype(np.float32))
    x = x_rows(m, h, 8)
    Ed = ctx.to_device(E)
    got = host(ctx.lm_head_argmax_f16(ctx.to_device(x), Ed, ctx.f16_repack_t64(Ed),
                                      ctx.lm_head_rowconst(Ed)))
    lg = orc.lm_head_f16(x, E)
    assert list(got) == [orc.argmax(r) for r in lg]


def test_bound_holds_with_margin(ctx):
    """|s z - T| <= eps for every (row, vocabulary row) of the certified rows
    (z the exact chain, s the row's power-of-two scale), with a wide margin:
    the bound allows an MFMA accumulation error 32x the sequential
    round-to-nearest one, over Cauchy-Schwarz."""
    m, h, vocab = 32, 896, 151936
    E = emb_device(ctx, vocab, h, seed=5)
    Et = ctx.f16_repack_t64(E)
    rc = ctx.lm_head_rowconst(E)
    x = x_rows(m, h, 77)
    xd = ctx.to_device(x)
    tok, bd = ctx.lm_head_argmax_f16(xd, E, Et, rc, bounds=True)
    z = host(ctx.lm_head_f16_t64(xd, Et, vocab)).astype(np.float64)
    bd = host(bd).astype(np.float64)
    worst = 0.0
    checked = 0
    for b in range(m):
        mx = float(np.max(np.abs(x[b])))
        if not np.all(np.isfinite(x[b])) or not (2.0 ** -60 <= mx <= 2.0 ** 60):
            continue                                 # exact rows: no bound used
        _, e = np.frexp(mx)
        s = 2.0 ** (15 - int(e))
        assert 2.0 ** 14 <= mx * s < 2.0 ** 15
        err = np.abs(s * z[b] - bd[b, :, 0])
        eps = bd[b, :, 1]
        assert np.all(err <= eps), (b, int(np.argmax(err - eps)))
        worst = max(worst, float(np.max(err / eps)))
        checked += 1
    assert checked >= 25
    print(f"bound check: {checked} rows, largest |s z - T| / eps = {worst:.3e}")
    assert worst < 0.25, worst


def test_ties_overflow_and_exact_slices(ctx, orc):
    """Duplicated vocabulary rows tie exactly: more than 8 of them in one
    slice overflow its list (every row of the slice gets the exact chain);
    the first maximum wins.  An embedding of identical rows ties everywhere
    (token 0)."""
    t = ctx.torch
    rng = np.random.default_rng(21)
    vocab, h = 5000, 256
    E = orc.f32_to_f16((rng.standard_normal((vocab, h)) * 0.02).astype(np.float32))
    src = 1300                                       # slice 2 = rows 1280..1919
    dup = list(range(1290, 1310)) + [2500, 4999]     # 20 copies in slice 2, two elsewhere
    for r in dup:
        E[r] = E[src]
    x = np.zeros((4, h), np.float32)
    x[0] = orc.f16_to_f32(E[src]) * 40.0             # aligned with the duplicated row
    x[1] = -x[0]
    x[2] = rng.standard_normal(h).astype(np.float32)
    x[3] = x[0]
    x[3, 0] += 1e-3
    Ed = ctx.to_device(E)
    Et = ctx.f16_repack_t64(Ed)
    rc = ctx.lm_head_rowconst(Ed)
    got = host(ctx.lm_head_argmax_f16(ctx.to_device(x), Ed, Et, rc))
    want = full_tokens(ctx, ctx.to_device(x), Et, vocab)
    assert list(got) == list(want)
    assert got[0] == 1290                            # the first of the tied maxima
    Eall = np.tile(E[src], (vocab, 1))
    Ed2 = ctx.to_device(Eall)
    got2 = host(ctx.lm_head_argmax_f16(ctx.to_device(x), Ed2, ctx.f16_repack_t64(Ed2),
                                       ctx.lm_head_rowconst(Ed2)))
    assert list(got2) == [0, 0, 0, 0]
    del t


def test_rowconst_bounds(ctx, orc):
    rng = np.random.default_rng(4)
    vocab, h = 300, 192
    E = orc.f32_to_f16((rng.standard_normal((vocab, h)) * 0.02).astype(np.float32))
    E[3, :40] = 0x0001                               # smallest subnormal
    E[4, 5] = 0x03ff                                 # largest subnormal
    E[5, 17] = 0x7c00                                # +inf
    E[6, 0] = 0x7e00                                 # NaN
    rc = host(ctx.lm_head_rowconst(ctx.to_device(E)))
    Ef = np.abs(orc.f16_to_f32(E).astype(np.float64))
    for v in range(vocab):
        if v in (5, 6):
            assert np.all(np.isinf(rc[v, :3]))
            continue
        s = Ef[v].sum()
        d = Ef[v][(E[v] & 0x7fff) < 0x0400].sum()
        for got, exact in ((rc[v, 0], s), (rc[v, 1], d)):
            assert float(got) >= exact
            assert float(got) == float(np.float32(exact)) or \
                float(got) == float(np.nextafter(np.float32(exact), np.float32(np.inf)))
        n2 = np.sqrt(np.sum(Ef[v] ** 2))             # the norm: above, by a few ulp at most
        assert n2 <= float(rc[v, 2]) <= n2 * (1 + 2.0 ** -21)
        assert rc[v, 3] == 0.0


def test_certified_argument_errors(ctx):
    t = ctx.torch
    E = t.zeros((100, 64), dtype=t.int16, device=ctx.dev)
    Et = ctx.f16_repack_t64(E)
    rc = ctx.lm_head_rowconst(E)
    with pytest.raises(lgx.LgxError) as e:
        ctx.lm_head_argmax_f16(t.zeros((33, 64), dtype=t.float32, device=ctx.dev), E, Et, rc)
    assert e.value.status_name == "LGX_UNSUPPORTED"
    with pytest.raises(lgx.LgxError) as e:
        ctx.lm_head_argmax_f16(t.zeros((2, 96), dtype=t.float32, device=ctx.dev),
                               t.zeros((100, 96), dtype=t.int16, device=ctx.dev), Et, rc)
    assert e.value.status_name == "LGX_UNSUPPORTED"


def test_certified_token_with_non_finite_embedding_rows(ctx, orc):
    """Embedding rows holding +inf, -inf or NaN at a column where x is
    nonzero but far below its largest entry (|x_k| < 2^-40 max|x|, so the
    binary16 copy of x holds 0 there and the MFMA forms 0 x inf = NaN): the
    exact chain gives +inf, -inf or NaN for those rows, and the certified
    token must still be the full logits' argmax (the +inf row when x_k > 0)."""
    rng = np.random.default_rng(11)
    m, h, vocab = 6, 256, 1300
    E = orc.f32_to_f16((rng.standard_normal((vocab, h)) * 0.05).astype(np.float32))
    k0, k1 = 5, 77
    E[101, k0] = 0x7c00            # +inf
    E[702, k0] = 0xfc00            # -inf
    E[903, k0] = 0x7e00            # NaN
    E[1250, k1] = 0x7c00           # +inf at another column
    x = rng.standard_normal((m, h)).astype(np.float32)
    x[0, k0] = 1e-30               # +inf row wins
    x[1, k0] = -1e-30              # row 101 -inf, row 702 +inf: 702 wins
    x[2, k0] = 0.0                 # 0 x inf = NaN: those rows are skipped
    x[3, k0] = 1e-30
    x[3, k1] = 1e-30               # two +inf rows: the first (101) wins
    x[4, k0] = 2.5                 # an ordinary value at the column
    x[5, k1] = -1e-30
    Ed = ctx.to_device(E)
    Et = ctx.f16_repack_t64(Ed)
    got = host(ctx.lm_head_argmax_f16(ctx.to_device(x), Ed, Et, ctx.lm_head_rowconst(Ed)))
    want = full_tokens(ctx, ctx.to_device(x), Et, vocab)
    lg = orc.lm_head_f16(x, E)
    assert list(want) == [orc.argmax(r) for r in lg]
    assert list(got) == list(want)
    assert got[0] == 101 and got[1] == 702 and got[3] == 101
