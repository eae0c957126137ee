"""The device Qwen2-shaped Q8_0 model against the CPU oracle model.

* Weights: the library generates every tensor from the seed on its own
  (host SplitMix64 streams -> upload -> device tile repack); the bytes must
  equal the oracle's tensors in the tile layouts.
* Decode: prefill (teacher forcing) and greedy decode steps give the same
  token ids, logits, final hidden rows and KV cache bits as the oracle's
  step, for tied (binary16 lm_head) and untied (Q8_0 lm_head) models, with
  ragged sequence lengths, page and 256-token chunk boundaries crossed.
* The 0.5B shape (24 layers, 896 hidden, 14/2 heads of 64, vocab 151936):
  token ids identical for 64 decode steps after a prompt.
"""
import numpy as np
import pytest

import logicaffeine_amd as lgx

pytestmark = pytest.mark.gpu


def host(t):
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def dev_array(gm, name, dtype, shape, layer=0):
    return gm.tensor_bytes(name, layer).view(dtype).reshape(shape)


def kv_dense(gm, cfg, layer, which, b, L):
    """Gather the first L cached tokens of sequence b from the device pages."""
    from oracle import oracle as orc

    maxp = -(-cfg["max_seq"] // 16)
    pages = dev_array(gm, "k_pages" if which == 0 else "v_pages", np.uint16,
                      (cfg["max_batch"] * maxp, cfg["n_kv"], 16, cfg["head_dim"]), layer)
    pt = dev_array(gm, "page_table", np.int32, (cfg["max_batch"], maxp))
    return orc.paged_to_dense(pages, pt, b, L)


@pytest.fixture(scope="module", params=["tiny", "tiny_untied"])
def pair(request, ctx):
    from oracle import oracle as orc

    cfg = orc.qwen_config(request.param)
    seed = 20261201
    gm = lgx.Model(ctx, cfg, seed)
    om = orc.Model(cfg, seed)
    yield cfg, gm, om
    gm.close()
    om.close()


def test_weights_match_oracle_generator(pair):
    from oracle import oracle as orc

    cfg, gm, om = pair
    H, I, d, hq, hkv = cfg["hidden"], cfg["inter"], cfg["head_dim"], cfg["n_heads"], cfg["n_kv"]
    qn = (hq + 2 * hkv) * d
    emb = dev_array(gm, "emb", np.uint16, (cfg["vocab"], H))
    assert np.array_equal(emb, om.tensor("emb"))
    mats = {"qkv": (qn, H), "o": (H, hq * d), "gu": (2 * I, H), "dn": (H, I)}
    if not cfg["tied"]:
        mats["lm"] = (cfg["vocab"], H)
    for layer in range(cfg["n_layers"]):
        for name, (n, k) in mats.items():
            if name == "lm" and layer > 0:
                continue
            qs, dd = om.tensor(name + "_q", layer), om.tensor(name + "_d", layer)
            assert np.array_equal(gm.tensor_bytes(name + "_q", layer).view(np.int8),
                                  orc.q8_repack_t16(qs)), (name, layer)
            assert np.array_equal(gm.tensor_bytes(name + "_d", layer).view(np.uint16),
                                  orc.q8_repack_s16(dd, n, k)), (name, layer)
        assert np.array_equal(dev_array(gm, "bias", np.float32, (qn,), layer).view(np.uint32),
                              bits(om.tensor("bias", layer)))
    pt = dev_array(gm, "page_table", np.int32, (-1,))
    assert sorted(pt.tolist()) == list(range(pt.size))        # a permutation of the pages


def test_prefill_then_decode_bit_exact(pair, ctx):
    cfg, gm, om = pair
    t = ctx.torch
    rng = np.random.default_rng(5)
    V, B = cfg["vocab"], cfg["max_batch"]
    gm.reset()
    # ragged lengths: sequences 0..1 get a 261-token prompt (two attention
    # chunks, page boundaries), then every sequence gets a 5-token prompt
    p1 = rng.integers(0, V, size=(2, 261)).astype(np.int32)
    nxt = host(gm.prefill(ctx.to_device(p1)))
    for p in range(p1.shape[1]):
        on, lg = om.step(np.arange(2), p1[:, p], want_logits=True)
    assert np.array_equal(nxt, on)
    assert np.array_equal(bits(host(gm.logits(2))), bits(lg))
    p2 = rng.integers(0, V, size=(B, 5)).astype(np.int32)
    nxt = host(gm.prefill(ctx.to_device(p2)))
    for p in range(p2.shape[1]):
        on, lg, hid = om.step(np.arange(B), p2[:, p], want_logits=True, want_hidden=True)
    assert np.array_equal(nxt, on)
    assert np.array_equal(bits(host(gm.logits(B))), bits(lg))
    assert np.array_equal(dev_array(gm, "hidden", np.float32, (B, cfg["hidden"])).view(np.uint32),
                          bits(hid))
    # greedy decode: the device feeds its own tokens back
    tok = t.from_numpy(nxt.copy()).to(ctx.dev)
    ref = on.copy()
    for s in range(12):
        gm.decode_step(tok)
        ref, lg = om.step(np.arange(B), ref, want_logits=True)
        got = host(tok)
        assert np.array_equal(got, ref), f"step {s}"
        assert np.array_equal(bits(host(gm.logits(B))), bits(lg)), f"step {s}"
    lens = dev_array(gm, "seq_len", np.int32, (B,))
    assert [int(x) for x in lens] == [om.seq_len(b) for b in range(B)] == [278, 278, 17, 17]
    for layer in range(cfg["n_layers"]):
        for b in range(B):
            for which in (0, 1):
                got = kv_dense(gm, cfg, layer, which, b, int(lens[b]))
                assert np.array_equal(got, om.kv(layer, which, b, int(lens[b]))), (layer, b, which)


@pytest.mark.parametrize("chunk,env", [(48, {}), (16, {}), (48, dict(LGX_TILED_SWIGLU="0"))])
def test_chunked_prefill_equals_oracle(chunk, env):
    """The batched prefill in several chunks (positions per chunk forced
    small: chunk boundaries inside and across 256-token attention chunks,
    ragged starting lengths) leaves the oracle's tokens, logits and KV bits,
    with SwiGLU + Q8_0 inside the gate|up product (default) or in a kernel of
    its own."""
    from oracle import oracle as orc

    c = _ctx_with(dict(env, LGX_PREFILL_CHUNK=str(chunk)))
    cfg = orc.qwen_config("tiny_untied")
    gm = lgx.Model(c, cfg, 31)
    om = orc.Model(cfg, 31)
    rng = np.random.default_rng(chunk)
    B = cfg["max_batch"]
    p1 = rng.integers(0, cfg["vocab"], size=(1, 70)).astype(np.int32)
    nxt = host(gm.prefill(c.to_device(p1)))
    for p in range(p1.shape[1]):
        on = om.step(np.arange(1), p1[:, p])
    assert np.array_equal(nxt, on)
    p2 = rng.integers(0, cfg["vocab"], size=(B, 221)).astype(np.int32)
    nxt = host(gm.prefill(c.to_device(p2)))
    for p in range(p2.shape[1]):
        on, lg = om.step(np.arange(B), p2[:, p], want_logits=True)
    assert np.array_equal(nxt, on)
    assert np.array_equal(bits(host(gm.logits(B))), bits(lg))
    lens = dev_array(gm, "seq_len", np.int32, (B,))
    assert [int(x) for x in lens] == [291, 221, 221, 221]
    for layer in range(cfg["n_layers"]):
        for b in range(B):
            for which in (0, 1):
                got = kv_dense(gm, cfg, layer, which, b, int(lens[b]))
                assert np.array_equal(got, om.kv(layer, which, b, int(lens[b]))), (layer, b, which)
    # a prompt past max_seq is an error, not a silent clamp
    with pytest.raises(lgx.LgxError):
        gm.prefill(c.to_device(rng.integers(0, 10, size=(B, 100)).astype(np.int32)))
    gm.close()
    om.close()
    c.close()


@pytest.mark.parametrize("env", [{}, dict(LGX_TILED_SWIGLU="0")])
@pytest.mark.parametrize("name", ["tiny", "tiny_untied"])
def test_wide_batch_decode_bit_exact(name, env):
    """Batches of 33 or more sequences take the tiled products, whose
    activations the norms, attention merge and SwiGLU write in T16 tiles:
    40 sequences (a ragged last row tile) prefilled and decoded agree with
    the oracle in tokens, logits and KV bits, graph replays included.  The
    gate|up product runs SwiGLU + Q8_0 in its own workgroups (default) or
    leaves its outputs to the SwiGLU kernel (LGX_TILED_SWIGLU=0)."""
    from oracle import oracle as orc

    ctx = _ctx_with(env)
    cfg = dict(orc.qwen_config(name), max_batch=40, max_seq=64)
    gm = lgx.Model(ctx, cfg, 5)
    om = orc.Model(cfg, 5)
    rng = np.random.default_rng(11)
    B, P = 40, 21
    prompt = rng.integers(0, cfg["vocab"], size=(B, P)).astype(np.int32)
    tok = gm.prefill(ctx.to_device(prompt))
    for p in range(P):
        ref, lg = om.step(np.arange(B), prompt[:, p], want_logits=True)
    assert np.array_equal(host(tok), ref)
    assert np.array_equal(bits(host(gm.logits(B))), bits(lg))
    for s in range(3):
        gm.decode_step(tok)
        ref, lg = om.step(np.arange(B), ref, want_logits=True)
        assert np.array_equal(host(tok), ref), s
        assert np.array_equal(bits(host(gm.logits(B))), bits(lg)), s
    hist = ctx.torch.empty((3, B), dtype=ctx.torch.int32, device=ctx.dev)
    gm.generate(tok, 3, hist)
    for s in range(3):
        ref = om.step(np.arange(B), ref)
        assert np.array_equal(host(hist[s]), ref), s
    L = P + 6
    for layer in range(cfg["n_layers"]):
        for b in (0, 17, 39):
            for which in (0, 1):
                assert np.array_equal(kv_dense(gm, cfg, layer, which, b, L),
                                      om.kv(layer, which, b, L)), (layer, b, which)
    gm.close()
    om.close()
    ctx.close()


def test_decode_uses_only_first_B_sequences(pair, ctx):
    """A step over B < max_batch leaves the other sequences' state alone."""
    cfg, gm, om = pair
    B = cfg["max_batch"]
    gm.reset()
    tok = ctx.to_device(np.arange(B, dtype=np.int32) + 3)
    gm.decode_step(tok)
    before = dev_array(gm, "seq_len", np.int32, (B,)).copy()
    t1 = ctx.to_device(np.array([7], np.int32))
    gm.decode_step(t1)
    after = dev_array(gm, "seq_len", np.int32, (B,))
    assert list(before) == [1] * B
    assert list(after) == [2] + [1] * (B - 1)


def test_model_argument_errors(ctx):
    from oracle import oracle as orc

    cfg = dict(orc.qwen_config("tiny"))
    for bad in (dict(head_dim=96), dict(n_heads=20, n_kv=2), dict(hidden=16384),
                dict(hidden=200)):
        with pytest.raises(lgx.LgxError):
            lgx.Model(ctx, dict(cfg, **bad), 1)
    gm = lgx.Model(ctx, cfg, 1)
    with pytest.raises(lgx.LgxError) as e:
        gm.decode_step(ctx.to_device(np.zeros(cfg["max_batch"] + 1, np.int32)))
    assert e.value.status_name == "LGX_OUT_OF_BOUNDS"
    gm.close()


def test_qwen_0_5b_shape_token_identity_64_steps(ctx):
    from oracle import oracle as orc

    cfg = dict(orc.qwen_config("0.5b"), max_batch=4, max_seq=128)
    seed = 77
    gm = lgx.Model(ctx, cfg, seed)
    om = orc.Model(cfg, seed)
    rng = np.random.default_rng(9)
    B, P = 4, 24
    prompt = rng.integers(0, cfg["vocab"], size=(B, P)).astype(np.int32)
    tok = gm.prefill(ctx.to_device(prompt))
    for p in range(P):
        ref = om.step(np.arange(B), prompt[:, p])
    assert np.array_equal(host(tok), ref)
    got_seq, ref_seq = [], []
    for _ in range(64):
        gm.decode_step(tok)
        ref = om.step(np.arange(B), ref)
        got_seq.append(host(tok))
        ref_seq.append(ref)
    assert np.array_equal(np.stack(got_seq), np.stack(ref_seq))
    # the random model does not collapse to one token (the check is not vacuous)
    assert len(np.unique(np.stack(ref_seq))) > 8
    gm.close()
    om.close()


@pytest.mark.parametrize("name", ["tiny", "tiny_untied"])
def test_generate_graph_replays_match_eager_and_oracle(name, ctx):
    """lgx_qwen_generate replays one recorded decode step.  Every replay is
    checked against the eager step of a second model and the oracle, with
    eager steps, reads and synchronisations of the same model between the
    replays; then a multi-step call with history, a second recording for a
    smaller batch on a side stream, and the argument errors."""
    from oracle import oracle as orc

    t = ctx.torch
    cfg = orc.qwen_config(name)
    seed = 4242
    B, V = cfg["max_batch"], cfg["vocab"]
    gg, ge, om = lgx.Model(ctx, cfg, seed), lgx.Model(ctx, cfg, seed), orc.Model(cfg, seed)
    rng = np.random.default_rng(13)
    prompt = rng.integers(0, V, size=(B, 3)).astype(np.int32)
    tg = gg.prefill(ctx.to_device(prompt))
    te = ge.prefill(ctx.to_device(prompt))
    for p in range(prompt.shape[1]):
        ref = om.step(np.arange(B), prompt[:, p])
    assert np.array_equal(host(tg), ref)
    for s in range(8):
        if s % 3 == 2:
            gg.decode_step(tg)                  # eager work between the replays
        else:
            gg.generate(tg, 1)
        ge.decode_step(te)
        ref, lg = om.step(np.arange(B), ref, want_logits=True)
        t.cuda.synchronize()
        assert np.array_equal(host(tg), ref), f"step {s}"
        assert np.array_equal(host(te), ref), f"step {s}"
        assert np.array_equal(bits(host(gg.logits(B))), bits(lg)), f"step {s}"
    # several replays in one call, with every step's tokens kept
    hist = t.full((5, B), -1, dtype=t.int32, device=ctx.dev)
    gg.generate(tg, 5, hist)
    refs = []
    for _ in range(5):
        ref, lg = om.step(np.arange(B), ref, want_logits=True)
        refs.append(ref)
    assert np.array_equal(host(hist), np.stack(refs))
    assert np.array_equal(host(tg), ref)
    assert np.array_equal(bits(host(gg.logits(B))), bits(lg))
    # a second recording (smaller batch, other tokens tensor) on a side stream
    side = t.cuda.Stream(ctx.dev)
    t1 = tg[:1].clone()
    side.wait_stream(t.cuda.current_stream(ctx.dev))
    with t.cuda.stream(side):
        gg.generate(t1, 2)
    side.synchronize()
    r1 = ref[:1]
    for _ in range(2):
        r1 = om.step(np.arange(1), r1)
    assert np.array_equal(host(t1), r1)
    lens = dev_array(gg, "seq_len", np.int32, (B,))
    assert [int(x) for x in lens] == [om.seq_len(b) for b in range(B)]
    assert int(lens[0]) == int(lens[1]) + 2
    gg.generate(tg, 0)                              # no-op
    with pytest.raises(lgx.LgxError) as e:
        gg.generate(tg, -1)
    assert e.value.status_name == "LGX_INVALID_ARGUMENT"
    with pytest.raises(lgx.LgxError) as e:
        gg.generate(ctx.to_device(np.zeros(B + 1, np.int32)), 1)
    assert e.value.status_name == "LGX_OUT_OF_BOUNDS"
    for m in (gg, ge, om):
        m.close()


@pytest.mark.parametrize("env", [dict(LGX_GEMV_WGS="8"), dict(LGX_GEMV="whole", LGX_GEMV_WGS="8")])
def test_single_sequence_decode_eight_wave_gemv(env):
    """M = 1 decode steps with the eight-wave GEMV workgroups forced (the
    grouped per-range kernels over Q8_0 and binary32 activations, then the
    whole-K kernel) give the oracle's tokens."""
    import os

    from oracle import oracle as orc

    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        c = lgx.Context(0)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k)
            else:
                os.environ[k] = v
    cfg = orc.qwen_config("tiny_untied")
    gm = lgx.Model(c, cfg, 41)
    om = orc.Model(cfg, 41)
    tok = np.array([5], np.int32)
    dtok = c.to_device(tok)
    for step in range(6):
        gm.decode_step(dtok)
        tok = om.step(np.arange(1), tok)
        assert np.array_equal(host(dtok), tok), step
    gm.close()
    om.close()
    c.close()


def test_ctx_destroy_refused_while_a_model_lives():
    """lgx_ctx_destroy of a ctx that a live model still uses fails (the model
    would read the freed ctx); after lgx_model_destroy it succeeds.
    Context.close() closes its live models first."""
    from oracle import oracle as orc

    c = lgx.Context(0)
    gm = lgx.Model(c, orc.qwen_config("tiny"), 3)
    st = lgx.lib().lgx_ctx_destroy(c.handle)
    assert lgx.STATUS_NAMES[st] == "LGX_INVALID_ARGUMENT"
    assert b"destroy them first" in lgx.lib().lgx_last_error()
    gm.decode_step(c.to_device(np.array([1], np.int32)))    # the model still works
    gm.close()
    assert lgx.lib().lgx_ctx_destroy(c.handle) == 0
    c.handle = None
    c2 = lgx.Context(0)
    gm2 = lgx.Model(c2, orc.qwen_config("tiny"), 3)
    c2.close()                                  # closes gm2, then the ctx
    assert gm2.handle is None and c2.handle is None


def test_max_seq_bound_on_every_path():
    """A call that would grow a sequence past max_seq fails with
    LGX_OUT_OF_BOUNDS before launching anything, on every path: decode step,
    generate, one-token prefill, batched prefill and serial prefill; the
    device lengths stay unchanged, and calls that end exactly at max_seq
    succeed."""
    import os

    from oracle import oracle as orc

    cfg = dict(orc.qwen_config("tiny"), max_seq=40)
    B = cfg["max_batch"]
    old = os.environ.get("LGX_PREFILL")
    os.environ["LGX_PREFILL"] = "serial"
    try:
        cs = lgx.Context(0)
    finally:
        if old is None:
            os.environ.pop("LGX_PREFILL")
        else:
            os.environ["LGX_PREFILL"] = old
    c = lgx.Context(0)
    rng = np.random.default_rng(3)

    def lens(gm):
        return [int(x) for x in dev_array(gm, "seq_len", np.int32, (B,))]

    def refused(fn):
        with pytest.raises(lgx.LgxError) as e:
            fn()
        assert e.value.status_name == "LGX_OUT_OF_BOUNDS"

    for cc in (c, cs):
        gm = lgx.Model(cc, cfg, 9)
        prompt = cc.to_device(rng.integers(0, cfg["vocab"], size=(B, 37)).astype(np.int32))
        tok = gm.prefill(prompt)                                 # 37
        gm.decode_step(tok)                                      # 38
        refused(lambda: gm.generate(tok, 3))                     # 41 > 40
        gm.generate(tok, 2)                                      # 40 == max_seq
        assert lens(gm) == [40] * B
        refused(lambda: gm.decode_step(tok))
        refused(lambda: gm.decode_step(tok[:1]))
        refused(lambda: gm.generate(tok, 1))
        refused(lambda: gm.prefill(prompt[:, :1].contiguous()))  # the one-token path
        refused(lambda: gm.prefill(prompt[:, :2].contiguous()))
        assert lens(gm) == [40] * B
        gm.reset()
        gm.prefill(prompt[:1, :1].contiguous())                  # seq 0 only: 1
        p40 = cc.to_device(rng.integers(0, cfg["vocab"], size=(B, 40)).astype(np.int32))
        refused(lambda: gm.prefill(p40))                         # seq 0 would reach 41
        assert lens(gm) == [1] + [0] * (B - 1)
        gm.prefill(p40[:1, :39].contiguous())                   # 1 + 39 == max_seq
        assert lens(gm) == [40] + [0] * (B - 1)
        gm.close()
    cs.close()
    c.close()


def _ctx_with(env):
    import os

    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return lgx.Context(0)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k)
            else:
                os.environ[k] = v


@pytest.mark.parametrize("env", [{}, dict(LGX_FUSE_SWIGLU_COLS="64"), dict(LGX_DECODE_FUSE="0"),
                                 dict(LGX_LM_CERT="0")])
@pytest.mark.parametrize("name", ["tiny", "tiny_untied"])
def test_fused_decode_consumers_bit_exact(name, env):
    """Decode batches of 2..32 rows run RoPE + KV append inside the qkv
    product's workgroups (one per head and 16-row m-group), SwiGLU + Q8_0
    inside the gate|up product's (32 or 64 columns each) and, from one row,
    the attention-side residual + RMSNorm + Q8_0 inside the qkv product's
    (one per sequence and 128 columns, the residual alternating between two
    buffers) and the attention merge inside the o_proj product's (one per
    sequence and eight row tiles); with the fusion off they run as kernels
    of their own.  Every form leaves the oracle's
    tokens, logits, hidden state and KV bits: 24 rows (a second, partial
    m-group), 3 rows, and one row (the grouped GEMV), graph replays
    included."""
    from oracle import oracle as orc

    c = _ctx_with(env)
    cfg = dict(orc.qwen_config(name), max_batch=24, max_seq=64)
    gm = lgx.Model(c, cfg, 77)
    om = orc.Model(cfg, 77)
    rng = np.random.default_rng(5)
    B = 24
    tok = rng.integers(0, cfg["vocab"], size=B).astype(np.int32)
    ref = tok.copy()
    dtok = c.to_device(tok)
    for s in range(4):
        gm.decode_step(dtok)
        ref, lg = om.step(np.arange(B), ref, want_logits=True)
        assert np.array_equal(host(dtok), ref), s
        assert np.array_equal(bits(host(gm.logits(B))), bits(lg)), s
    hist = c.torch.empty((3, B), dtype=c.torch.int32, device=c.dev)
    gm.generate(dtok, 3, hist)
    for s in range(3):
        ref = om.step(np.arange(B), ref)
        assert np.array_equal(host(hist[s]), ref), s
    for nb in (3, 1):
        t = c.to_device(ref[:nb].copy())
        for s in range(2):
            gm.decode_step(t)
            r, lg, hid = om.step(np.arange(nb), (ref[:nb] if s == 0 else r), want_logits=True,
                                 want_hidden=True)
            assert np.array_equal(host(t), r), (nb, s)
            assert np.array_equal(bits(host(gm.logits(nb))), bits(lg)), (nb, s)
            assert np.array_equal(bits(dev_array(gm, "hidden", np.float32, (B, cfg["hidden"]))[:nb]),
                                  bits(hid)), (nb, s)
    lens = [int(x) for x in dev_array(gm, "seq_len", np.int32, (B,))]
    assert lens == [11, 9, 9] + [7] * 21
    for layer in range(cfg["n_layers"]):
        for b in (0, 2, 5, 23):
            for which in (0, 1):
                assert np.array_equal(kv_dense(gm, cfg, layer, which, b, lens[b]),
                                      om.kv(layer, which, b, lens[b])), (layer, b, which)
    gm.close()
    om.close()
    c.close()


@pytest.mark.parametrize("hidden", [1536, 2048])
def test_tied_model_hidden_above_1024(ctx, hidden):
    """A tied binary16 embedding with hidden > 1024 (the Qwen2.5-1.5B / 3B
    widths): the lm_head runs one chain per 1024-column range and the
    argmax, the seeded draw and the logits entry point apply the pairwise
    tree over them (the certified pick covers hidden <= 1024 only).  Tokens
    and logits equal the oracle's through prefill, greedy decode, graph
    replays and sampled decode."""
    from oracle import oracle as orc

    cfg = dict(orc.qwen_config("tiny"), n_layers=2, hidden=hidden, inter=512, n_heads=hidden // 128,
               n_kv=2, head_dim=128, vocab=1000, tied=1, max_batch=4, max_seq=64)
    gm = lgx.Model(ctx, cfg, 17)
    om = orc.Model(cfg, 17)
    rng = np.random.default_rng(hidden)
    B, P = 4, 9
    prompt = rng.integers(0, cfg["vocab"], size=(B, P)).astype(np.int32)
    tok = gm.prefill(ctx.to_device(prompt))
    ref, lg = om.prefill(np.arange(B), prompt, want_logits=True)
    assert np.array_equal(host(tok), ref)
    assert np.array_equal(bits(host(gm.logits(B))), bits(lg))
    for s in range(4):
        gm.decode_step(tok)
        ref, lg = om.step(np.arange(B), ref, want_logits=True)
        assert np.array_equal(host(tok), ref), s
        assert np.array_equal(bits(host(gm.logits(B))), bits(lg)), s
    hist = ctx.torch.empty((3, B), dtype=ctx.torch.int32, device=ctx.dev)
    gm.generate(tok, 3, hist)
    for s in range(3):
        ref = om.step(np.arange(B), ref)
        assert np.array_equal(host(hist[s]), ref), s
    gm.set_sampling(0.8, top_k=20, top_p=0.9, seed=5)
    om.set_sampling(0.8, top_k=20, top_p=0.9, seed=5)
    for s in range(4):
        gm.decode_step(tok)
        ref = om.step(np.arange(B), ref)
        assert np.array_equal(host(tok), ref), ("sampled", s)
    gm.close()
    om.close()


@pytest.mark.parametrize("fuse", ["1", "0"])
@pytest.mark.parametrize("shape", [
    dict(hidden=512, inter=1024, n_heads=6, n_kv=2, head_dim=64, tied=1),     # hq*d = 384 != H, gq 3
    dict(hidden=384, inter=768, n_heads=2, n_kv=1, head_dim=128, tied=0),     # d = 128, hq*d = 256
], ids=["h512-gq3-d64", "h384-gq2-d128"])
def test_fused_decode_other_shapes_multi_chunk(shape, fuse):
    """The decode step's per-sequence fused kernels (residual + RMSNorm +
    Q8_0 inside the qkv product, the attention merge inside o_proj) on
    shapes where the attention width hq * d differs from the hidden size and
    the head groups are 3 or 2, with ragged contexts across three 256-token
    chunks and every batch size from 1 to 5 rows; LGX_DECODE_FUSE=0 runs the
    separate kernels.  Tokens, logits, hidden rows and the KV cache equal the
    oracle's bit for bit."""
    from oracle import oracle as orc

    c = _ctx_with(dict(LGX_DECODE_FUSE=fuse))
    cfg = dict(orc.qwen_config("tiny"), n_layers=2, vocab=1024, max_batch=5, max_seq=600, **shape)
    gm = lgx.Model(c, cfg, 91)
    om = orc.Model(cfg, 91)
    rng = np.random.default_rng(17)
    lens = [530, 300, 257, 40, 3]
    # ragged contexts: sequence b takes lens[b] prompt tokens through
    # teacher-forced decode steps of sequences 0..nb-1 (lens descending)
    prompts = [rng.integers(0, cfg["vocab"], size=L).astype(np.int32) for L in lens]
    P = max(lens)
    for p in range(P):
        nb = sum(1 for L in lens if L > p)     # lens are descending: sequences 0..nb-1
        tok = np.array([prompts[b][p] for b in range(nb)], np.int32)
        dtok = c.to_device(tok)
        gm.decode_step(dtok)
        om.step(np.arange(nb), tok)
    ref = None
    for nb in (5, 4, 3, 2, 1):
        tok = rng.integers(0, cfg["vocab"], size=nb).astype(np.int32)
        dtok = c.to_device(tok)
        gm.decode_step(dtok)
        ref, lg, hid = om.step(np.arange(nb), tok, want_logits=True, want_hidden=True)
        assert np.array_equal(host(dtok), ref), nb
        assert np.array_equal(bits(host(gm.logits(nb))), bits(lg)), nb
        assert np.array_equal(bits(dev_array(gm, "hidden", np.float32, (5, cfg["hidden"]))[:nb]),
                              bits(hid)), nb
    lens2 = [int(x) for x in dev_array(gm, "seq_len", np.int32, (5,))]
    for layer in range(cfg["n_layers"]):
        for b in range(5):
            for which in (0, 1):
                assert np.array_equal(kv_dense(gm, cfg, layer, which, b, lens2[b]),
                                      om.kv(layer, which, b, lens2[b])), (layer, b, which)
    gm.close()
    om.close()
    c.close()
