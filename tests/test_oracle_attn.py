"""Pin the oracle's paged GQA decode attention (no GPU).

References: an independent numpy float64 softmax attention (tests/golden),
closed forms (one token returns V exactly, equal scores give the mean,
constant V is returned), page-order invariance, and a planted mistake that
the tolerance check must reject."""
import numpy as np
import pytest

TOL = 2e-3   # attention tolerance of the north star (relative, with an absolute floor)


def close(a, b, tol=TOL):
    return np.all(np.abs(a - b) <= tol * (np.abs(b) + 1e-2))


def test_golden_attention(orc, golden):
    out = orc.gqa_decode_attn(golden["attn_q"], golden["attn_k"], golden["attn_v"],
                              golden["attn_pt"], golden["attn_lens"])
    ref = golden["attn_out"]
    assert close(out, ref)
    assert np.max(np.abs(out - ref)) < 1e-5          # far inside the tolerance


def test_planted_head_mapping_mistake_is_caught(orc, golden):
    # swap the two KV heads: the oracle then attends with the wrong group
    k = golden["attn_k"][:, ::-1].copy()
    v = golden["attn_v"][:, ::-1].copy()
    out = orc.gqa_decode_attn(golden["attn_q"], k, v, golden["attn_pt"], golden["attn_lens"])
    assert not close(out, golden["attn_out"])


def _cache(orc, B, hkv, d, maxp, seed=0):
    k = orc.gen_normal_f16(seed, 1, (B * maxp, hkv, 16, d))
    v = orc.gen_normal_f16(seed, 2, (B * maxp, hkv, 16, d))
    pt = orc.gen_page_table(seed, 3, B, maxp)
    return k, v, pt


def test_single_token_returns_v_exactly(orc):
    B, hq, hkv, d, maxp = 2, 6, 2, 128, 4
    k, v, pt = _cache(orc, B, hkv, d, maxp)
    q = orc.gen_normal_f32(0, 4, (B, hq, d))
    out = orc.gqa_decode_attn(q, k, v, pt, np.array([1, 1], np.int32))
    for b in range(B):
        for h in range(hq):
            assert np.array_equal(out[b, h], orc.f16_to_f32(v[pt[b, 0], h // 3, 0]))


def test_equal_scores_give_the_mean_and_constant_v(orc):
    B, hq, hkv, d, maxp = 1, 4, 1, 64, 40
    k, v, pt = _cache(orc, B, hkv, d, maxp, seed=5)
    q = np.zeros((B, hq, d), np.float32)            # all scores 0
    L = 600                                          # three chunks
    out = orc.gqa_decode_attn(q, k, v, pt, np.array([L], np.int32))
    dense = orc.paged_to_dense(v, pt, 0, L)[:, 0, :]
    mean = orc.f16_to_f32(dense).astype(np.float64).mean(0)
    assert np.allclose(out[0], mean[None, :], atol=1e-5)
    vc = v.copy()
    vc[:] = v[pt[0, 0], 0, 0]                        # every cached V row equal
    qr = orc.gen_normal_f32(5, 9, (B, hq, d))
    outc = orc.gqa_decode_attn(qr, k, vc, pt, np.array([L], np.int32))
    assert np.allclose(outc[0], orc.f16_to_f32(v[pt[0, 0], 0, 0])[None, :], rtol=1e-5, atol=1e-6)


def test_page_order_invariance(orc):
    """The same token rows under a different page permutation give the same
    bits (the page table only relocates rows)."""
    B, hq, hkv, d, maxp = 2, 6, 2, 64, 20
    k, v, pt = _cache(orc, B, hkv, d, maxp, seed=7)
    q = orc.gen_normal_f32(7, 4, (B, hq, d))
    lens = np.array([300, 77], np.int32)
    out1 = orc.gqa_decode_attn(q, k, v, pt, lens)
    perm = np.random.default_rng(0).permutation(B * maxp)
    inv = np.argsort(perm)
    k2, v2 = k[perm], v[perm]                        # page p moves to slot inv[p]
    pt2 = inv[pt].astype(np.int32)
    assert np.array_equal(orc.gqa_decode_attn(q, k2, v2, pt2, lens), out1)


def test_halving_sum_order(orc):
    p = np.zeros(256, np.float32)
    p[0], p[128], p[1] = 1e8, 1.0, -1e8
    # level s=128 pairs (0,128): 1e8+1 == 1e8; then (0,1): 0.  Left to right gives 1.
    assert orc.halving_sum(p) == 0.0
    assert orc.halving_sum(np.ones(256, np.float32)) == 256.0


def test_wide_path_matches_per_sequence_path(orc, golden):
    """Many (sequence, KV head) tasks take the oracle's vector path (AVX-512,
    when the host has it); one sequence at a time takes the scalar path.
    Same bits for ragged lengths (empty, one token, partial chunks, several
    chunks), d = 64 and 128 and group sizes 1 to 7; the golden fixture
    repeated over many sequences meets its float64 reference."""
    rng = np.random.default_rng(6)
    for hq, hkv, d in [(14, 2, 64), (28, 4, 128), (8, 8, 64), (12, 2, 128)]:
        B = max(8, 192 // hkv)
        lens = rng.integers(0, 700, size=B).astype(np.int32)
        lens[:4] = [0, 1, 256, 513]
        maxp = -(-int(lens.max()) // 16)
        k, v, pt = _cache(orc, B, hkv, d, maxp, seed=hq + d)
        q = orc.gen_normal_f32(9, hq + d, (B, hq, d))
        out = orc.gqa_decode_attn(q, k, v, pt, lens)
        for b in range(B):
            one = orc.gqa_decode_attn(q[b:b + 1], k, v, pt[b:b + 1], lens[b:b + 1])
            assert np.array_equal(out[b].view(np.uint32), one[0].view(np.uint32)), (hq, d, b)
    gB = golden["attn_q"].shape[0]
    reps = -(-96 // gB)
    q = np.tile(golden["attn_q"], (reps, 1, 1))
    pt = np.tile(golden["attn_pt"], (reps, 1))
    lens = np.tile(golden["attn_lens"], reps)
    out = orc.gqa_decode_attn(q, golden["attn_k"], golden["attn_v"], pt, lens)
    assert close(out, np.tile(golden["attn_out"], (reps, 1, 1)))
