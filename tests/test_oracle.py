"""Pin the CPU oracle (no GPU).

The reference has no implementation or vectors for this path, so each oracle
function is pinned by published vectors (SplitMix64), exhaustive comparison
with numpy (binary16), independent numpy restatements (tests/golden), closed
forms and invariants, and mutant checks showing those checks are
discriminating.
"""
import numpy as np
import pytest


# ---- SplitMix64 -----------------------------------------------------------

def test_splitmix64_published_vectors(orc):
    # Vigna's splitmix64.c, seed 1234567 (widely reproduced test vector)
    assert list(orc.splitmix64_seq(1234567, 5)) == [
        6457827717110365317, 3203168211198807973, 9817491932198370423,
        4593380528125082431, 16408922859458223821]
    # rand_xoshiro's SplitMix64 reference test, seed 1477776061723855037
    assert list(orc.splitmix64_seq(1477776061723855037, 3)) == [
        1985237415132408290, 2979275885539914483, 13511426838097143398]


def test_stream_indexing_matches_sequence(orc):
    base = int(orc.lib().orc_stream_base(7, 3))
    assert np.array_equal(orc.gen_u64(7, 3, 100), orc.splitmix64_seq(base, 100))
    assert not np.array_equal(orc.gen_u64(7, 3, 8), orc.gen_u64(7, 4, 8))
    assert not np.array_equal(orc.gen_u64(7, 3, 8), orc.gen_u64(8, 3, 8))


def test_generator_distributions(orc):
    q = orc.gen_i8(0, 0, (1 << 20,))
    assert q.min() == -127 and q.max() == 127
    assert abs(q.astype(np.float64).mean()) < 0.2
    counts = np.bincount(q.astype(np.int64) + 127, minlength=255)
    assert counts.min() > 0.9 * counts.mean() and counts.max() < 1.1 * counts.mean()
    z = orc.gen_normal_f32(0, 1, (1 << 20,))
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1) < 5e-3
    d = orc.f16_to_f32(orc.gen_q8_scales(0, 2, (1 << 18,))).astype(np.float64)
    assert d.min() >= 0
    assert abs(d.mean() / (0.02 * np.sqrt(2 / np.pi) / 127) - 1) < 0.01
    ids = orc.gen_below_i32(3, 0, 151936, (1 << 16,))
    assert ids.min() >= 0 and ids.max() < 151936


# ---- binary16 ---------------------------------------------------------------

def test_f16_decode_exhaustive(orc):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    a = orc.f16_to_f32(h)
    b = h.view(np.float16).astype(np.float32)
    same = (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))
    assert same.all()


def test_f16_encode_rne(orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(1 << 20).astype(np.float32)
    x *= np.exp2(rng.integers(-30, 18, x.size)).astype(np.float32)
    # boundaries: overflow threshold, subnormal range, ties, +-0
    specials = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e30, 2.0**-14,
                         2.0**-24, 2.0**-25, 2.0**-25 * 1.0000001, 2.0**-26, 1.5 * 2.0**-24,
                         2.5 * 2.0**-24, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, np.inf, -np.inf],
                        dtype=np.float32)
    x = np.concatenate([x, specials])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.f32_to_f16(x), ref)


# ---- exp / silu -------------------------------------------------------------

def test_expf_accuracy_and_special_values(orc):
    x = np.linspace(-87.33, 88.72, 400001, dtype=np.float32)
    y = orc.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    rel = np.abs(y - ref) / ref
    assert rel.max() < 2 * 2.0**-24
    assert np.all(np.diff(y) >= 0)  # monotone on a dense grid
    assert orc.expf(np.float32([0.0]))[0] == 1.0
    assert orc.expf(np.float32([-100.0]))[0] == 0.0
    assert np.isinf(orc.expf(np.float32([100.0]))[0])
    # a mutant with the ln2_lo correction term dropped is caught by this bound
    n = np.rint(x.astype(np.float64) * 1.4426950408889634)
    mutant = np.exp(x.astype(np.float64) - n * (0.693145751953125 - 0.6931471805599453)) / 1.0
    assert (np.abs(mutant - ref) / ref).max() > 2 * 2.0**-24


def test_silu(orc):
    g = np.float32([0.0, 1.0, -1.0, 5.0, -20.0, 30.0, -90.0, 100.0])
    s = orc.silu(g).astype(np.float64)
    gd = g.astype(np.float64)
    ref = gd / (1 + np.exp(-gd))
    assert s[0] == 0.0
    # exp saturates to +inf above 88.72, so silu(-90) is -0 instead of -7.4e-38
    np.testing.assert_allclose(s, ref, rtol=4 * 2.0**-24, atol=1e-36)


def test_tree_sum_order(orc):
    # pairwise: (1e8 + 1) + (-1e8 + 1) == 0 in binary32; left-to-right would give 1
    assert orc.tree_sum([1e8, 1.0, -1e8, 1.0]) == 0.0
    assert orc.tree_sum([1.0]) == 1.0
    # g = 3 is ((p0 + p1) + p2): (1 + 1e8) + (-1e8) = 0, p0 + (p1 + p2) would be 1
    assert orc.tree_sum([1.0, 1e8, -1e8]) == 0.0
    # g = 5 is ((p0+p1)+(p2+p3))+p4
    p = np.float32([3e7, 1.0, 1.0, -3e7, 0.5])
    exp = np.float32(np.float32(np.float32(p[0] + p[1]) + np.float32(p[2] + p[3])) + p[4])
    assert orc.tree_sum(p) == exp


# ---- Q8_0 -------------------------------------------------------------------

def test_quantize_golden_exact(orc, golden):
    for name in ("small", "ranges"):
        q, d = orc.quantize_q8_0(golden[f"{name}_x"])
        assert np.array_equal(q, golden[f"{name}_xq"])
        assert np.array_equal(d, golden[f"{name}_xd"])
    q, d = orc.quantize_q8_0(golden["edge_x"])
    assert np.array_equal(q, golden["edge_q"]) and np.array_equal(d, golden["edge_d"])
    assert np.all(q[0] == 0) and d[0] == 0          # zero block
    assert q[2, 7] == -127                           # absmax element -> -127


def test_quantize_closed_forms(orc):
    c = np.float32(0.731)
    x = (c * np.arange(32, dtype=np.float32))[None, :]
    q, d = orc.quantize_q8_0(x)
    i = np.arange(32)
    assert np.array_equal(q[0], np.floor(127 * i / 31 + 0.5).astype(np.int8))
    assert d[0, 0] == np.float16(np.float32(31 * c) / np.float32(127)).view(np.uint16)
    # sign symmetry
    qn, dn = orc.quantize_q8_0(-x)
    assert np.array_equal(qn, -q) and np.array_equal(dn, d)


def test_blockdots_exact(orc, golden):
    for name in ("small", "ranges"):
        s = orc.q8_blockdots(golden[f"{name}_qs"], golden[f"{name}_xq"][0])
        assert np.array_equal(s, golden[f"{name}_s"][0])
    # extremes: |s| = 32*127^2 fits int32
    w = np.full((16, 64), -127, np.int8)
    x = np.full(64, -127, np.int8)
    assert np.all(orc.q8_blockdots(w, x) == 32 * 127 * 127)


def _q8_bound_ok(y, ref, absum, tol=1e-5):
    return np.all(np.abs(y.astype(np.float64) - ref) <= tol * absum + 1e-30)


def test_q8_gemm_golden(orc, golden):
    for name in ("small", "ranges"):
        y = orc.q8_gemm(golden[f"{name}_qs"], golden[f"{name}_d"], golden[f"{name}_xq"],
                        golden[f"{name}_xd"])
        assert _q8_bound_ok(y, golden[f"{name}_y_q8q8"], golden[f"{name}_y_q8q8_abs"])


def test_q8_gemm_mutants_are_caught(orc, golden):
    """The bound above is discriminating: planted oracle mistakes fail it."""
    qs, d = golden["ranges_qs"], golden["ranges_d"]
    xq, xd = golden["ranges_xq"], golden["ranges_xd"]
    ref, absum = golden["ranges_y_q8q8"], golden["ranges_y_q8q8_abs"]
    mutants = {
        "scale index shifted by one block": (qs, np.roll(d, 1, axis=1), xq, xd),
        "last block dropped": (qs, np.concatenate([d[:, :-1], np.zeros_like(d[:, :1])], 1), xq, xd),
        "activation sign flipped": (qs, d, -xq, xd),
        "k-chunk order within block swapped": (
            qs.reshape(qs.shape[0], -1, 4, 8)[:, :, ::-1].reshape(qs.shape), d, xq, xd),
    }
    for what, (a, b, c, e) in mutants.items():
        y = orc.q8_gemm(a, b, c, e)
        assert not _q8_bound_ok(y, ref, absum), what


def test_q8_gemm_batch_invariance(orc, golden):
    qs, d = golden["ranges_qs"], golden["ranges_d"]
    xq, xd = golden["ranges_xq"], golden["ranges_xd"]
    y = orc.q8_gemm(qs, d, xq, xd)
    for i in range(xq.shape[0]):
        yi = orc.q8_gemm(qs, d, xq[i:i + 1], xd[i:i + 1])
        assert np.array_equal(y[i], yi[0])


def test_q8_gemm_one_hot_closed_form(orc):
    qs, d = orc.gen_q8_matrix(0, 0, 64, 2048)
    j = 1500
    xq = np.zeros(2048, np.int8)
    xq[j] = 1
    xd = np.zeros(64, np.uint16)
    xd[j // 32] = orc.f32_to_f16(np.float32([1.0]))[0]
    y = orc.q8_gemm(qs, d, xq, xd)[0]
    exp = qs[:, j].astype(np.float32) * orc.f16_to_f32(d[:, j // 32])
    assert np.array_equal(y, exp)


def test_q8_gemv_f32_golden(orc, golden):
    for name in ("small", "ranges"):
        y = orc.q8_gemv_f32(golden[f"{name}_qs"], golden[f"{name}_d"], golden[f"{name}_x"][0])
        assert _q8_bound_ok(y, golden[f"{name}_y_f32"], golden[f"{name}_y_f32_abs"], 1e-6)


def test_q8_gemv_f32_linearity_and_one_hot(orc):
    qs, d = orc.gen_q8_matrix(0, 0, 4864, 896)   # config 0 weights
    x = orc.gen_normal_f32(0, 2, (896,))
    e = np.zeros(896, np.float32)
    e[333] = 1.0
    y = orc.q8_gemv_f32(qs, d, e)
    assert np.array_equal(y, qs[:, 333].astype(np.float32) * orc.f16_to_f32(d[:, 333 // 32]))
    y1 = orc.q8_gemv_f32(qs, d, x).astype(np.float64)
    y2 = orc.q8_gemv_f32(qs, d, 2 * x).astype(np.float64)
    np.testing.assert_allclose(y2, 2 * y1, rtol=1e-6, atol=1e-9)


def test_t16_repack_round_trip_and_formula(orc):
    rng = np.random.default_rng(1)
    qs = rng.integers(-127, 128, size=(32, 128), dtype=np.int8)
    t = orc.q8_repack_t16(qs)
    assert np.array_equal(orc.q8_unpack_t16(t, 32, 128), qs)
    # explicit placement: row 17 (tile 1, r 1), k = 64*1 + 32 + 8*2 + 5 (pair 1, hi, c 2, j 5)
    k = 64 + 32 + 16 + 5
    unit = 1 * 2 + 1
    lane = 1 + 16 * 2
    assert t[unit * 1024 + lane * 16 + 8 + 5] == qs[17, k]


def test_s16_scale_layout_formula(orc):
    n, k = 32, 896                     # nb = 28 -> two half-ranges, the second padded
    d = np.arange(n * (k // 32), dtype=np.uint16).reshape(n, k // 32) + 1
    s = orc.q8_repack_s16(d, n, k)
    nh = 2
    assert s.size == (n // 16) * nh * 256
    # row 17 (tile 1, r 1), block 20 (half 1, j 4)
    assert s[((1 * nh + 1) * 16 + 1) * 16 + 4] == d[17, 20]
    # padding past nb is zero, and every scale appears exactly once
    assert s[((0 * nh + 1) * 16 + 3) * 16 + 12] == 0
    assert np.array_equal(np.sort(s[s != 0]), np.sort(d.ravel()))


def test_q8_gemm_wide_path_matches_row_path(orc, golden):
    """16+ activation rows take the oracle's vector path (AVX-512 VNNI, when
    the host has it); one row at a time takes the scalar path.  Both must give
    the same bits, scale specials (inf, NaN, -0, subnormal, max) included,
    and the wide path must meet the independent float64 golden bound."""
    rng = np.random.default_rng(5)
    for n, k, m in [(37, 96, 17), (100, 3584, 40), (16, 18944, 33), (5, 64, 300)]:
        qs = rng.integers(-128, 128, size=(n, k)).astype(np.int8)
        d = orc.f32_to_f16((np.abs(rng.standard_normal((n, k // 32))) * 0.02 / 127).astype(np.float32))
        xq = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
        xd = orc.f32_to_f16(rng.random((m, k // 32)).astype(np.float32))
        specials = np.array([0x7c00, 0xfc00, 0x7e00, 0x8000, 0x0001, 0x7bff], np.uint16)
        d.flat[rng.integers(0, d.size, 6)] = specials
        xd.flat[rng.integers(0, xd.size, 6)] = specials
        y = orc.q8_gemm(qs, d, xq, xd)
        rows = np.stack([orc.q8_gemm(qs, d, xq[i:i + 1], xd[i:i + 1])[0] for i in range(m)])
        assert np.array_equal(y.view(np.uint32), rows.view(np.uint32)), (n, k, m)
    qs, d = golden["ranges_qs"], golden["ranges_d"]
    reps = -(-16 // golden["ranges_xq"].shape[0])
    xq = np.tile(golden["ranges_xq"], (reps, 1))
    xd = np.tile(golden["ranges_xd"], (reps, 1))
    ref = np.tile(golden["ranges_y_q8q8"], (reps, 1))
    absum = np.tile(golden["ranges_y_q8q8_abs"], (reps, 1))
    assert _q8_bound_ok(orc.q8_gemm(qs, d, xq, xd), ref, absum)
