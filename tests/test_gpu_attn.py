"""Parity of the paged GQA decode attention kernels with the CPU oracle.

The canonical schedule (256-token chunks, sequential score and PV chains,
halving-tree sums, log-sum-exp merge in chunk order) is followed by both, so
outputs are compared bit-for-bit; the float64 golden fixture checks the
north star's 2e-3 tolerance."""
import numpy as np
import pytest

import logicaffeine_amd as lgx

pytestmark = pytest.mark.gpu


def host(t):
    return t.cpu().numpy()


def make_cache(B, hkv, d, lens, seed):
    rng = np.random.default_rng(seed)
    maxp = max(1, -(-max(lens) // 16))
    npages = B * maxp
    k = rng.standard_normal((npages, hkv, 16, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((npages, hkv, 16, d)).astype(np.float16).view(np.uint16)
    pt = rng.permutation(npages).astype(np.int32).reshape(B, maxp)
    return k, v, pt, maxp


def run(ctx, q, k, v, pt, lens, max_seq_len=None):
    lens = np.asarray(lens, np.int32)
    msl = int(max_seq_len or max(1, lens.max()))
    return host(ctx.gqa_decode_attn(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v),
                                    ctx.to_device(pt), ctx.to_device(lens), msl))


def test_golden_fixture(ctx, orc, golden):
    out = run(ctx, golden["attn_q"], golden["attn_k"], golden["attn_v"], golden["attn_pt"],
              golden["attn_lens"])
    ref = orc.gqa_decode_attn(golden["attn_q"], golden["attn_k"], golden["attn_v"],
                              golden["attn_pt"], golden["attn_lens"])
    assert np.array_equal(out, ref)
    f64 = golden["attn_out"]
    assert np.all(np.abs(out - f64) <= 2e-3 * (np.abs(f64) + 1e-2))


@pytest.mark.parametrize("L", [512, 4096, 32768])
def test_config2_uniform_bit_exact(ctx, orc, L):
    B, hq, hkv, d = 16, 12, 2, 128
    lens = [L] * B
    k, v, pt, _ = make_cache(B, hkv, d, lens, seed=L)
    q = orc.gen_normal_f32(2, 10 + L, (B, hq, d))
    out = run(ctx, q, k, v, pt, lens)
    assert np.array_equal(out, orc.gqa_decode_attn(q, k, v, pt, np.asarray(lens, np.int32)))


def test_config2_ragged_long_bit_exact(ctx, orc):
    """Config 2's ragged variant at its batch of 16: lengths uniform in
    [256, 32768], the first at the maximum."""
    B, hq, hkv, d = 16, 12, 2, 128
    lens = list(orc.gen_below_i32(2, 30, 32768 - 256 + 1, (B,)) + 256)
    lens[0] = 32768
    k, v, pt, _ = make_cache(B, hkv, d, lens, seed=3)
    q = orc.gen_normal_f32(2, 31, (B, hq, d))
    out = run(ctx, q, k, v, pt, lens)
    assert np.array_equal(out, orc.gqa_decode_attn(q, k, v, pt, np.asarray(lens, np.int32)))


@pytest.mark.parametrize("d,hq", [(64, 14), (128, 12)])
def test_very_long_context_merge_bit_exact(ctx, orc, d, hq):
    """Contexts past 64 Ki tokens (more than 256 chunks: the merge runs
    several LDS tiles, and more chunks than threads), next to a short one
    and an empty one in the same call."""
    B, hkv = 3, 2
    lens = [70000, 3000, 0]
    k, v, pt, _ = make_cache(B, hkv, d, lens, seed=d + 7)
    q = orc.gen_normal_f32(2, 40 + d, (B, hq, d))
    out = run(ctx, q, k, v, pt, lens)
    assert np.array_equal(out, orc.gqa_decode_attn(q, k, v, pt, np.asarray(lens, np.int32)))
    assert np.all(out[2] == 0.0)


@pytest.mark.parametrize("hq,hkv,d", [(2 * g, 2, d) for d in (64, 128) for g in range(1, 9)]
                         + [(28, 4, 128), (8, 8, 64), (8, 1, 128)])
def test_head_layouts_bit_exact(ctx, orc, hq, hkv, d):
    B = 5
    lens = [1, 16, 255, 257, 1500]
    k, v, pt, _ = make_cache(B, hkv, d, lens, seed=hq * d)
    q = orc.gen_normal_f32(3, hq + d, (B, hq, d))
    out = run(ctx, q, k, v, pt, lens)
    assert np.array_equal(out, orc.gqa_decode_attn(q, k, v, pt, np.asarray(lens, np.int32)))
    # single cached token: the output is that token's V row exactly
    for h in range(hq):
        assert np.array_equal(out[0, h], orc.f16_to_f32(v[pt[0, 0], h // (hq // hkv), 0]))


def test_lengths_clamped_to_max_seq_len(ctx, orc):
    B, hq, hkv, d = 3, 6, 2, 64
    lens = np.array([700, 100, 0], np.int32)
    k, v, pt, maxp = make_cache(B, hkv, d, [700, 700, 700], seed=9)
    q = orc.gen_normal_f32(3, 77, (B, hq, d))
    out = run(ctx, q, k, v, pt, lens, max_seq_len=300)
    ref = orc.gqa_decode_attn(q, k, v, pt, np.minimum(lens, 300))
    assert np.array_equal(out, ref)
    assert np.all(out[2] == 0.0)                      # empty sequence


def test_attention_argument_errors(ctx, orc):
    t = ctx.torch
    q = t.zeros((1, 6, 96), dtype=t.float32, device=ctx.dev)
    pages = t.zeros((4, 2, 16, 96), dtype=t.int16, device=ctx.dev)
    pt = t.zeros((1, 4), dtype=t.int32, device=ctx.dev)
    sl = t.ones(1, dtype=t.int32, device=ctx.dev)
    with pytest.raises(lgx.LgxError) as ei:
        ctx.gqa_decode_attn(q, pages, pages, pt, sl, 16)
    assert ei.value.status_name == "LGX_UNSUPPORTED"
    q = t.zeros((1, 6, 64), dtype=t.float32, device=ctx.dev)
    pages = t.zeros((4, 2, 16, 64), dtype=t.int16, device=ctx.dev)
    with pytest.raises(lgx.LgxError) as ei:
        ctx.gqa_decode_attn(q, pages, pages, pt, sl, 65)
    assert ei.value.status_name == "LGX_OUT_OF_BOUNDS"
    q3 = t.zeros((1, 6, 64), dtype=t.float32, device=ctx.dev)
    pages3 = t.zeros((4, 4, 16, 64), dtype=t.int16, device=ctx.dev)
    with pytest.raises(lgx.LgxError) as ei:                 # 6 / 4 heads
        ctx.gqa_decode_attn(q3, pages3, pages3, pt, sl, 16)
    assert ei.value.status_name == "LGX_INVALID_ARGUMENT"


# ---- prefill: several causal query rows per sequence ----

def prefill_ref(orc, q, k, v, pt, ctx_len, P):
    """Oracle: row b*P + j is a decode query of sequence b at length
    ctx_len[b] + j + 1 (the page table row repeated per query row)."""
    B = len(ctx_len)
    lens = np.array([ctx_len[b] + j + 1 for b in range(B) for j in range(P)], np.int32)
    ptr = np.repeat(pt, P, axis=0)
    return orc.gqa_decode_attn(q, k, v, ptr, lens)


@pytest.mark.parametrize("hq,hkv,d,ctx_len,P", [
    (14, 2, 64, [0, 37], 40),            # fresh sequence + short context, ragged row block
    (28, 4, 128, [0, 200], 72),          # rows cross the first chunk boundary
    (12, 2, 128, [500, 0, 255], 9),      # GQ 6; P not a multiple of the row block
    (8, 8, 64, [3], 257),                # GQ 1, rows spanning two chunks
    (8, 1, 128, [1000], 20),             # GQ 8
])
def test_prefill_attn_bit_exact(ctx, orc, hq, hkv, d, ctx_len, P):
    """Every prefill row equals the decode schedule at its own length."""
    B = len(ctx_len)
    lens_end = [c + P for c in ctx_len]
    k, v, pt, maxp = make_cache(B, hkv, d, lens_end, seed=hq * d + P)
    q = orc.gen_normal_f32(4, hq + d + P, (B * P, hq, d))
    msl = maxp * 16
    out = host(ctx.gqa_prefill_attn(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v),
                                    ctx.to_device(pt), ctx.to_device(np.asarray(ctx_len, np.int32)),
                                    P, msl))
    assert np.array_equal(out, prefill_ref(orc, q, k, v, pt, ctx_len, P))


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("g", range(1, 9))
def test_prefill_attn_head_groups_bit_exact(ctx, orc, g, d):
    """Every head-group size the prefill kernels are built for, with one
    fresh and one cached sequence whose rows cross a chunk boundary."""
    hkv, ctx_len, P = 2, [0, 230], 35
    B, hq = len(ctx_len), 2 * g
    k, v, pt, maxp = make_cache(B, hkv, d, [c + P for c in ctx_len], seed=g * d)
    q = orc.gen_normal_f32(5, g + d, (B * P, hq, d))
    out = host(ctx.gqa_prefill_attn(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v),
                                    ctx.to_device(pt), ctx.to_device(np.asarray(ctx_len, np.int32)),
                                    P, maxp * 16))
    assert np.array_equal(out, prefill_ref(orc, q, k, v, pt, ctx_len, P))


def test_prefill_attn_config4_shape_sampled(ctx, orc):
    """Config-4 head layout at a 4096-token context: 64 new rows after 4032
    cached tokens (17 chunks), checked on a sample of rows."""
    B, hq, hkv, d, P = 2, 28, 4, 128, 64
    ctx_len = [4032, 1111]
    k, v, pt, maxp = make_cache(B, hkv, d, [c + P for c in ctx_len], seed=77)
    q = orc.gen_normal_f32(4, 99, (B * P, hq, d))
    out = host(ctx.gqa_prefill_attn(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v),
                                    ctx.to_device(pt), ctx.to_device(np.asarray(ctx_len, np.int32)),
                                    P, maxp * 16))
    rows = [0, 1, 31, 63, 64, 100, 127]
    lens = np.array([ctx_len[r // P] + r % P + 1 for r in rows], np.int32)
    ref = orc.gqa_decode_attn(q[rows], k, v, pt[[r // P for r in rows]], lens)
    assert np.array_equal(out[rows], ref)


def test_repeated_calls_changing_lengths_bit_exact(ctx, orc):
    """Call after call with changing lengths (empty, one chunk, many chunks,
    ragged) on one ctx (its workspace reused), for d = 64 and 128: the
    oracle's bits each time, zeros for empty sequences."""
    for d, hq, hkv in ((64, 14, 2), (128, 28, 4)):
        for rep, lens in enumerate(([0, 1, 256, 257, 3000], [2049, 0, 5, 511, 4097],
                                    [7, 7, 7, 7, 7])):
            B = len(lens)
            k, v, pt, _ = make_cache(B, hkv, d, [4097] * B, seed=d + rep)
            q = orc.gen_normal_f32(5, 10 * d + rep, (B, hq, d))
            out = run(ctx, q, k, v, pt, lens, max_seq_len=4097)
            ref = orc.gqa_decode_attn(q, k, v, pt, np.asarray(lens, np.int32))
            assert np.array_equal(out, ref), (d, rep)
            assert np.all(out[np.asarray(lens) == 0] == 0.0)
