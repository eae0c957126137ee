"""The opt-in fast prefill (LGX_PREFILL_FAST): binary16 MFMA flash attention.

* lgx_gqa_prefill_attn_fast against the oracle's canonical attention within
  the attention tolerance 2e-3: per (query row, head), the largest deviation
  is at most 2e-3 of the largest magnitude in that canonical output vector.
  Cases: those of the exact kernel (fresh and cached sequences, row counts
  not a multiple of 16, every head group 1..8, d 64 and 128), config 4's head
  layout at a 4096-token context, closed forms (constant V gives V; a
  single cached token gives its V row exactly), and a cache whose slots past
  each sequence's length hold NaN keys and infinite values (the exact
  prefill and decode kernels on it stay bit-exact).
* A model prefilled in fast mode (binary16 GEMMs on dequantised weights,
  binary16 activations, the fast attention): the cache it leaves, loaded
  into the oracle, gives the device's next token, logits and last-position
  K/V bit for bit, and the greedy decode steps after it stay bit-exact (the
  decode step is exact given the cache).  The fast cache stays within a few
  percent (relative L2) of the exact prefill's at layer 0 and at the last
  layer.  The same on top of cached context of ragged lengths, and for a
  GGUF checkpoint with a Q8_0 embedding and norm weights != 1.
"""
import numpy as np
import pytest

import logicaffeine_amd as lgx
from test_gpu_attn import make_cache, prefill_ref

pytestmark = pytest.mark.gpu

TOL = 2e-3


def host(t):
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def fast(ctx, q, k, v, pt, ctx_len, P, msl):
    return host(ctx.gqa_prefill_attn(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v),
                                     ctx.to_device(pt),
                                     ctx.to_device(np.asarray(ctx_len, np.int32)), P, msl,
                                     fast=True))


def within(out, ref):
    """Per (row, head): max |out - ref| <= 2e-3 * max |ref|; returns the
    largest ratio seen."""
    err = np.abs(out.astype(np.float64) - ref).max(axis=-1)
    scale = np.abs(ref).max(axis=-1).astype(np.float64)
    assert np.all(np.isfinite(out))
    assert np.all(err <= TOL * scale), float((err / np.maximum(scale, 1e-30)).max())
    return float((err / np.maximum(scale, 1e-30)).max())


@pytest.mark.parametrize("hq,hkv,d,ctx_len,P", [
    (14, 2, 64, [0, 37], 40),
    (28, 4, 128, [0, 200], 72),
    (12, 2, 128, [500, 0, 255], 9),
    (8, 8, 64, [3], 257),
    (8, 1, 128, [1000], 20),
    (28, 4, 128, [0, 64, 63, 65], 129),   # tile boundaries of the 64-token loop
])
def test_fast_prefill_attn_within_tolerance(ctx, orc, hq, hkv, d, ctx_len, P):
    B = len(ctx_len)
    k, v, pt, maxp = make_cache(B, hkv, d, [c + P for c in ctx_len], seed=hq * d + P)
    q = orc.gen_normal_f32(4, hq + d + P, (B * P, hq, d))
    out = fast(ctx, q, k, v, pt, ctx_len, P, maxp * 16)
    r = within(out, prefill_ref(orc, q, k, v, pt, ctx_len, P))
    print(f"max error / max |ref| = {r:.2e}")


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("g", range(1, 9))
def test_fast_prefill_attn_head_groups(ctx, orc, g, d):
    hkv, ctx_len, P = 2, [0, 230], 35
    B, hq = len(ctx_len), 2 * g
    k, v, pt, maxp = make_cache(B, hkv, d, [c + P for c in ctx_len], seed=g * d)
    q = orc.gen_normal_f32(5, g + d, (B * P, hq, d))
    out = fast(ctx, q, k, v, pt, ctx_len, P, maxp * 16)
    within(out, prefill_ref(orc, q, k, v, pt, ctx_len, P))


def test_fast_prefill_attn_config4_shape_sampled(ctx, orc):
    """Config 4's heads (28 / 4 of 128): 64 new rows after 4032 cached tokens
    and 64 after 1111, sampled rows against the oracle."""
    B, hq, hkv, d, P = 2, 28, 4, 128, 64
    ctx_len = [4032, 1111]
    k, v, pt, maxp = make_cache(B, hkv, d, [c + P for c in ctx_len], seed=77)
    q = orc.gen_normal_f32(4, 99, (B * P, hq, d))
    out = fast(ctx, q, k, v, pt, ctx_len, P, maxp * 16)
    rows = [0, 1, 15, 16, 31, 63, 64, 100, 127]
    lens = np.array([ctx_len[r // P] + r % P + 1 for r in rows], np.int32)
    within(out[rows], orc.gqa_decode_attn(q[rows], k, v, pt[[r // P for r in rows]], lens))


def poison_past_lengths(k, v, pt, lens):
    """Every cache slot at or past its sequence's length: NaN in K, +-inf in
    V (the kernels read whole tiles and pages, and must not let those slots
    reach an attended output)."""
    k, v = k.copy(), v.copy()
    for b, n in enumerate(lens):
        for t in range(n, pt.shape[1] * 16):
            pg, sl = pt[b, t // 16], t % 16
            k[pg, :, sl, :] = 0x7E00
            v[pg, :, sl, :] = 0x7C00 if t % 2 else 0xFC00
    return k, v


@pytest.mark.parametrize("d", [64, 128])
def test_fast_prefill_attn_nonfinite_past_length(ctx, orc, d):
    """NaN keys and infinite values in every slot past a sequence's length
    (the last tile's rows past the block's last length, the rest of its
    pages): the fast outputs stay finite and within tolerance, and the exact
    prefill and decode kernels on the same cache stay bit-exact."""
    hq, hkv, P = 14, 2, 45
    ctx_len = [0, 70, 129]
    lens = [c + P for c in ctx_len]
    k, v, pt, maxp = make_cache(len(ctx_len), hkv, d, [n + 40 for n in lens], seed=91 + d)
    k, v = poison_past_lengths(k, v, pt, lens)
    q = orc.gen_normal_f32(7, d, (len(ctx_len) * P, hq, d))
    ref = prefill_ref(orc, q, k, v, pt, ctx_len, P)
    assert np.all(np.isfinite(ref))
    within(fast(ctx, q, k, v, pt, ctx_len, P, maxp * 16), ref)
    exact = host(ctx.gqa_prefill_attn(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v),
                                      ctx.to_device(pt), ctx.to_device(np.asarray(ctx_len, np.int32)),
                                      P, maxp * 16))
    assert np.array_equal(bits(exact), bits(ref))
    last = np.array([b * P + P - 1 for b in range(len(ctx_len))])
    dec = host(ctx.gqa_decode_attn(ctx.to_device(np.ascontiguousarray(q[last])), ctx.to_device(k),
                                   ctx.to_device(v), ctx.to_device(pt),
                                   ctx.to_device(np.asarray(lens, np.int32)), maxp * 16))
    assert np.array_equal(bits(dec), bits(ref[last]))


def test_fast_prefill_attn_closed_forms(ctx, orc):
    """Constant V rows: every output is that row (the weights normalise by
    their own sum); a fresh sequence's first query sees one token: its V."""
    B, hq, hkv, d, P = 2, 8, 2, 128, 50
    ctx_len = [0, 300]
    k, v, pt, maxp = make_cache(B, hkv, d, [c + P for c in ctx_len], seed=5)
    row = np.random.default_rng(6).standard_normal((hkv, d)).astype(np.float16)
    vc = np.broadcast_to(row.view(np.uint16)[None, :, None, :], v.shape).copy()
    q = orc.gen_normal_f32(6, 1, (B * P, hq, d))
    out = fast(ctx, q, k, vc, pt, ctx_len, P, maxp * 16)
    want = np.repeat(row.astype(np.float32), hq // hkv, axis=0)     # [hq][d]
    assert np.all(np.abs(out - want[None]) <= 2e-5 * np.abs(want[None]) + 1e-7)
    out = fast(ctx, q, k, v, pt, ctx_len, P, maxp * 16)
    first = orc.paged_to_dense(v, pt, 0, 1)[0].view(np.float16).astype(np.float32)
    assert np.array_equal(out[0], np.repeat(first, hq // hkv, axis=0))


def test_fast_prefill_attn_argument_errors(ctx):
    t = ctx.torch
    pt = t.zeros((1, 4), dtype=t.int32, device=ctx.dev)
    sl = t.zeros(1, dtype=t.int32, device=ctx.dev)
    for hq, hkv, d, status in ((4, 2, 96, "LGX_UNSUPPORTED"), (18, 2, 64, "LGX_UNSUPPORTED"),
                               (6, 4, 64, "LGX_INVALID_ARGUMENT")):
        q = t.zeros((3, hq, d), dtype=t.float32, device=ctx.dev)
        pages = t.zeros((4, hkv, 16, d), dtype=t.int16, device=ctx.dev)
        with pytest.raises(lgx.LgxError) as ei:
            ctx.gqa_prefill_attn(q, pages, pages, pt, sl, 3, 64, fast=True)
        assert ei.value.status_name == status, (hq, hkv, d)
    q = t.zeros((3, 4, 64), dtype=t.float32, device=ctx.dev)
    pages = t.zeros((4, 2, 16, 64), dtype=t.int16, device=ctx.dev)
    with pytest.raises(lgx.LgxError) as ei:                  # beyond the page table
        ctx.gqa_prefill_attn(q, pages, pages, pt, sl, 3, 65, fast=True)
    assert ei.value.status_name == "LGX_OUT_OF_BOUNDS"


@pytest.mark.parametrize("name,B,P,steps", [("tiny", 4, 300, 16), ("0.5b", 4, 600, 64)])
def test_fast_prefill_model_then_decode_bit_exact(ctx, name, B, P, steps):
    from oracle import oracle as orc

    cfg = dict(orc.qwen_config(name), max_batch=B, max_seq=P + steps)
    nl, V = cfg["n_layers"], cfg["vocab"]
    seed = 777
    prompt = np.random.default_rng(P).integers(0, V, size=(B, P)).astype(np.int32)
    gm = lgx.Model(ctx, cfg, seed)
    exact_l0 = None
    try:
        gm.prefill(ctx.to_device(prompt))
        exact_l0 = [[gm.kv_rows(0, w, b, P) for w in (0, 1)] for b in range(B)]
        exact_top = [gm.kv_rows(nl - 1, w, 0, P) for w in (0, 1)]
        gm.reset()
        gm.set_prefill_mode(True)
        tok = gm.prefill(ctx.to_device(prompt))
        nxt, lg_dev = host(tok), host(gm.logits(B))
        kv = [[[gm.kv_rows(layer, w, b, P) for w in (0, 1)] for b in range(B)]
              for layer in range(nl)]
    except Exception:
        gm.close()
        raise
    # the fast cache stays close to the exact one (layer 0: the binary16
    # qkv product against the exact Q8_0 one; the last layer: every layer's
    # rounding)
    def rel(a, e):
        a = a.view(np.float16).astype(np.float64)
        e = e.view(np.float16).astype(np.float64)
        return np.linalg.norm(a - e) / np.linalg.norm(e)

    for w in (0, 1):
        r0 = max(rel(kv[0][b][w], exact_l0[b][w]) for b in range(B))
        rl = rel(kv[nl - 1][0][w], exact_top[w])
        print(f"{'KV'[w]}: relative L2 distance fast vs exact: layer 0 {r0:.2e}, last layer {rl:.2e}")
        assert r0 <= 0.02 and rl <= 0.1, w
    om = orc.Model(cfg, seed)
    try:
        for layer in range(nl):
            for b in range(B):
                for w in (0, 1):
                    om.load_kv(layer, w, b, kv[layer][b][w][:P - 1])
        for b in range(B):
            om.set_seq_len(b, P - 1)
        ref, lg = om.step(np.arange(B), prompt[:, P - 1], want_logits=True)
        assert np.array_equal(nxt, ref)
        assert np.array_equal(bits(lg_dev), bits(lg))
        for layer in range(nl):
            for b in range(B):
                for w in (0, 1):
                    assert np.array_equal(om.kv(layer, w, b, P), kv[layer][b][w]), (layer, b, w)
        for s in range(steps):
            gm.decode_step(tok)
            ref, lg = om.step(np.arange(B), ref, want_logits=True)
            assert np.array_equal(host(tok), ref), f"step {s}"
            assert np.array_equal(bits(host(gm.logits(B))), bits(lg)), f"step {s}"
    finally:
        om.close()
        gm.close()


def _load_device_cache(gm, om, cfg, seqs, lens):
    """The device's cache of sequences `seqs` (first lens[i] positions) into
    oracle slots 0.. and their lengths."""
    nl = cfg["n_layers"]
    for slot, (b, L) in enumerate(zip(seqs, lens)):
        for layer in range(nl):
            for w in (0, 1):
                om.load_kv(layer, w, slot, gm.kv_rows(layer, w, b, L))
        om.set_seq_len(slot, L)


def test_fast_prefill_after_cached_context_ragged(ctx):
    """A fast prefill on top of cached context of different lengths (two
    sequences with 100 exact-prefilled positions, two fresh): the oracle,
    given the device's cache up to the last prompt position, reproduces the
    next tokens and logits, then 12 greedy steps, bit for bit."""
    from oracle import oracle as orc

    cfg = dict(orc.qwen_config("tiny"), max_seq=320)
    B, seed = cfg["max_batch"], 31
    rng = np.random.default_rng(8)
    p1 = rng.integers(0, cfg["vocab"], size=(2, 100)).astype(np.int32)
    p2 = rng.integers(0, cfg["vocab"], size=(B, 150)).astype(np.int32)
    gm = lgx.Model(ctx, cfg, seed)
    om = orc.Model(cfg, seed)
    try:
        gm.prefill(ctx.to_device(p1))                     # exact: sequences 0, 1
        gm.set_prefill_mode(True)
        tok = gm.prefill(ctx.to_device(p2))               # fast, on 100 / 100 / 0 / 0 cached
        nxt, lg_dev = host(tok), host(gm.logits(B))
        lens = [100 + 149, 100 + 149, 149, 149]
        _load_device_cache(gm, om, cfg, range(B), lens)
        ref, lg = om.step(np.arange(B), p2[:, -1], want_logits=True)
        assert np.array_equal(nxt, ref)
        assert np.array_equal(bits(lg_dev), bits(lg))
        for s in range(12):
            gm.decode_step(tok)
            ref, lg = om.step(np.arange(B), ref, want_logits=True)
            assert np.array_equal(host(tok), ref), s
            assert np.array_equal(bits(host(gm.logits(B))), bits(lg)), s
    finally:
        om.close()
        gm.close()


def test_fast_prefill_gguf_checkpoint_then_decode(ctx, tmp_path):
    """A checkpoint with a Q8_0 token embedding, norm weights != 1 and a
    tied hidden-1536 shape (two lm_head ranges) through the fast prefill:
    the device cache in the oracle (given the same tensors) reproduces the
    next tokens, logits and 10 greedy steps bit for bit."""
    from oracle import oracle as orc
    from tests import gguf_util as gg

    cfg = dict(orc.qwen_config("tiny"), eps=1e-5, theta=20000.0, hidden=1536, n_heads=12,
               n_kv=2, head_dim=128, inter=512, vocab=1008)
    t = gg.random_qwen2(cfg, 23, emb_q8=True)
    path = tmp_path / "model.gguf"
    gg.write_gguf(path, gg.qwen2_meta(cfg), gg.qwen2_tensors(cfg, t))
    gm = lgx.Model.load_gguf(ctx, str(path), cfg["max_batch"], cfg["max_seq"])
    om = orc.Model(gm.cfg, 0)
    try:
        gg.load_into_oracle(om, cfg, t)
        B, P = cfg["max_batch"], 90
        prompt = np.random.default_rng(5).integers(0, cfg["vocab"], size=(B, P)).astype(np.int32)
        gm.set_prefill_mode(True)
        tok = gm.prefill(ctx.to_device(prompt))
        nxt, lg_dev = host(tok), host(gm.logits(B))
        _load_device_cache(gm, om, gm.cfg, range(B), [P - 1] * B)
        ref, lg = om.step(np.arange(B), prompt[:, -1], want_logits=True)
        assert np.array_equal(nxt, ref)
        assert np.array_equal(bits(lg_dev), bits(lg))
        for s in range(10):
            gm.decode_step(tok)
            ref, lg = om.step(np.arange(B), ref, want_logits=True)
            assert np.array_equal(host(tok), ref), s
            assert np.array_equal(bits(host(gm.logits(B))), bits(lg)), s
    finally:
        om.close()
        gm.close()
