"""Models loaded from Q8_0 GGUF checkpoints, against the oracle given the
same tensors.

* A checkpoint of random tensors (norm weights != 1, biases, tied binary16
  or untied Q8_0 lm_head) written by tests/gguf_util.py: the device tensors
  equal the file's (repacked), and prefill + greedy decode give the oracle's
  tokens and logits bit for bit.
* The seeded random-init model exported to GGUF and loaded back decodes
  exactly as lgx_model_create of that seed.
* Truncated and misshapen files fail with their status before anything is
  built.
"""
import numpy as np
import pytest

import logicaffeine_amd as lgx
from tests import gguf_util as gg

pytestmark = pytest.mark.gpu


def host(t):
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _cfg(name, **kw):
    from oracle import oracle as orc

    return dict(orc.qwen_config(name), **kw)


H1536 = dict(hidden=1536, n_heads=12, n_kv=2, head_dim=128, inter=512)


@pytest.mark.parametrize("name,emb_q8,kw", [
    ("tiny", False, {}), ("tiny_untied", False, {}),
    ("tiny", True, dict(vocab=1008)), ("tiny_untied", True, {}),
    ("tiny", False, H1536), ("tiny", True, dict(H1536, vocab=1008))],
    ids=["tied", "untied", "tied-q8emb", "untied-q8emb", "tied-h1536", "tied-h1536-q8emb"])
def test_loaded_checkpoint_decodes_like_oracle(ctx, tmp_path, name, emb_q8, kw):
    """Binary16 or Q8_0 token_embd (llama.cpp's Q8_0 files store it as
    Q8_0: the gather dequantises, a tied model's lm_head is the Q8 product
    with it), hidden <= 1024 and 1536 (two ranges in the tied binary16
    lm_head)."""
    from oracle import oracle as orc

    cfg = _cfg(name, eps=1e-5, theta=20000.0, **kw)
    t = gg.random_qwen2(cfg, 17, emb_q8=emb_q8)
    path = tmp_path / "model.gguf"
    gg.write_gguf(path, gg.qwen2_meta(cfg), gg.qwen2_tensors(cfg, t))
    gm = lgx.Model.load_gguf(ctx, str(path), cfg["max_batch"], cfg["max_seq"])
    for key in ("n_layers", "hidden", "inter", "n_heads", "n_kv", "head_dim", "vocab", "tied"):
        assert gm.cfg[key] == cfg[key], key
    # device tensors are the file's, in the tile layouts
    H, I = cfg["hidden"], cfg["inter"]
    for l in range(cfg["n_layers"]):
        for nm, (n, k) in (("qkv", ((cfg["n_heads"] + 2 * cfg["n_kv"]) * cfg["head_dim"], H)),
                           ("gu", (2 * I, H)), ("dn", (H, I))):
            assert np.array_equal(gm.tensor_bytes(nm + "_q", l).view(np.int8),
                                  orc.q8_repack_t16(t[(nm + "_q", l)]))
            assert np.array_equal(gm.tensor_bytes(nm + "_d", l).view(np.uint16),
                                  orc.q8_repack_s16(t[(nm + "_d", l)], n, k))
        for nm in ("attn_norm", "ffn_norm"):
            assert np.array_equal(gm.tensor_bytes(nm, l).view(np.float32), t[(nm, l)])
    assert np.array_equal(gm.tensor_bytes("out_norm").view(np.float32), t["out_norm"])
    if emb_q8:
        V = cfg["vocab"]
        assert np.array_equal(gm.tensor_bytes("emb_q").view(np.int8), orc.q8_repack_t16(t["emb_q"]))
        assert np.array_equal(gm.tensor_bytes("emb_d").view(np.uint16),
                              orc.q8_repack_s16(t["emb_d"], V, H))
        with pytest.raises(lgx.LgxError):
            gm.tensor_bytes("emb")
    om = orc.Model(gm.cfg, 0)
    gg.load_into_oracle(om, cfg, t)
    B = cfg["max_batch"]
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, cfg["vocab"], size=(B, 19)).astype(np.int32)
    tok = gm.prefill(ctx.to_device(prompt))
    ref, lg = om.prefill(np.arange(B), prompt, want_logits=True)
    assert np.array_equal(host(tok), ref)
    assert np.array_equal(bits(host(gm.logits(B))), bits(lg))
    seen, prev = set(), bits(lg).copy()
    for s in range(10):
        gm.decode_step(tok)
        ref, lg = om.step(np.arange(B), ref, want_logits=True)
        assert np.array_equal(host(tok), ref), s
        assert np.array_equal(bits(host(gm.logits(B))), bits(lg)), s
        assert not np.array_equal(bits(lg), prev)         # the state moves every step
        prev = bits(lg).copy()
        seen |= set(ref.tolist())
    assert len(seen) >= 4
    gm.close()
    om.close()


def test_seeded_model_round_trips_through_gguf(ctx, tmp_path):
    from oracle import oracle as orc

    cfg = _cfg("tiny_untied")
    seed = 909
    om = orc.Model(cfg, seed)
    t = {"emb": om.tensor("emb"), "lm_q": om.tensor("lm_q"), "lm_d": om.tensor("lm_d"),
         "out_norm": np.ones(cfg["hidden"], np.float32)}
    for l in range(cfg["n_layers"]):
        for nm in ("qkv_q", "qkv_d", "o_q", "o_d", "gu_q", "gu_d", "dn_q", "dn_d", "bias"):
            t[(nm, l)] = om.tensor(nm, l)
        t[("attn_norm", l)] = np.ones(cfg["hidden"], np.float32)
        t[("ffn_norm", l)] = np.ones(cfg["hidden"], np.float32)
    om.close()
    path = tmp_path / "seeded.gguf"
    gg.write_gguf(path, gg.qwen2_meta(cfg), gg.qwen2_tensors(cfg, t))
    ga = lgx.Model.load_gguf(ctx, str(path), cfg["max_batch"], cfg["max_seq"])
    gb = lgx.Model(ctx, cfg, seed)
    prompt = ctx.to_device(np.arange(4 * 7, dtype=np.int32).reshape(4, 7) * 13 % cfg["vocab"])
    ta, tb = ga.prefill(prompt), gb.prefill(prompt)
    for _ in range(6):
        ga.decode_step(ta)
        gb.decode_step(tb)
        assert np.array_equal(host(ta), host(tb))
        assert np.array_equal(bits(host(ga.logits(4))), bits(host(gb.logits(4))))
    ga.close()
    gb.close()


def test_truncated_and_misshapen_files(ctx, tmp_path):
    cfg = _cfg("tiny")
    t = gg.random_qwen2(cfg, 5)
    p = tmp_path / "cut.gguf"
    gg.write_gguf(p, gg.qwen2_meta(cfg), gg.qwen2_tensors(cfg, t))
    raw = p.read_bytes()
    p.write_bytes(raw[:len(raw) - 4096])              # tensor data cut short
    with pytest.raises(lgx.LgxError) as e:
        lgx.Model.load_gguf(ctx, str(p), 4, 64)
    assert e.value.status_name == "LGX_MODULE_LOAD_FAILED"
    tens = gg.qwen2_tensors(cfg, t)
    i = [n for n, _, _ in tens].index("blk.1.ffn_down.weight")
    qs, d = tens[i][2]
    tens[i] = (tens[i][0], gg.GGML_Q8_0, (qs[:-16], d[:-16]))
    gg.write_gguf(p, gg.qwen2_meta(cfg), tens)
    with pytest.raises(lgx.LgxError) as e:
        lgx.Model.load_gguf(ctx, str(p), 4, 64)
    assert e.value.status_name == "LGX_INVALID_ARGUMENT"
    tens = [x for x in gg.qwen2_tensors(cfg, t) if x[0] != "blk.0.attn_k.bias"]
    gg.write_gguf(p, gg.qwen2_meta(cfg), tens)
    with pytest.raises(lgx.LgxError) as e:
        lgx.Model.load_gguf(ctx, str(p), 4, 64)
    assert e.value.status_name == "LGX_INVALID_ARGUMENT"
