"""The benchmark-shaped models at their benchmark batch and context, against
the CPU oracle on sampled sequences.

Decode sequences are independent in every kernel (products, norms and
attention work per row, and the products are batch-invariant), so the
oracle steps a few sampled slots while the device runs the whole batch; each
sampled slot must match its device sequence bit for bit in tokens and logits
at every step.  The oracle prefills its slots with orc_model_prefill, which
the CPU tests pin bit for bit to repeated oracle steps.

* Config 4 (Qwen2.5-7B shape, Q8_0 lm_head of 152064 x 3584): batch 64, so
  every product runs through the tiled kernels (gate|up 37888 x 3584, down
  3584 x 18944, the lm_head); two sequences carry a 320-token prompt (two
  256-token attention chunks and their merge), the others 20 tokens; 64
  greedy steps.  The 4096-token prompt of the benchmark is shortened here so
  that the oracle finishes in seconds; the chunk merge it exercises is the
  same one.
* Config 3 (Qwen2.5-0.5B shape, tied binary16 lm_head): batch 32, the full
  2048-token prompts (8 attention chunks merged), the 32-row streaming
  products (lgx_k_q8_gemm_mfma32), 64 greedy steps.
"""
import numpy as np
import pytest

import logicaffeine_amd as lgx

pytestmark = pytest.mark.gpu


def host(t):
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _kv_dense(gm, cfg, layer, which, b, L):
    from oracle import oracle as orc

    maxp = -(-cfg["max_seq"] // 16)
    pages = gm.tensor_bytes("k_pages" if which == 0 else "v_pages", layer).view(np.uint16).reshape(
        cfg["max_batch"] * maxp, cfg["n_kv"], 16, cfg["head_dim"])
    pt = gm.tensor_bytes("page_table", 0).view(np.int32).reshape(cfg["max_batch"], maxp)
    return orc.paged_to_dense(pages, pt, b, L)


def _decode_and_compare(gm, om, tok, seqs, ref, steps):
    """`steps` greedy steps of the whole device batch; the oracle steps slots
    0..len(seqs)-1 standing for device sequences `seqs`.  Returns the
    oracle's token history and the number of steps whose logits differ from
    the previous step's (the state keeps evolving, so the bit-exact logit
    comparison is not a comparison of one repeated vector)."""
    B = tok.numel()
    hist = []
    changed, prev = 0, None
    for s in range(steps):
        gm.decode_step(tok)
        ref, lg = om.step(np.arange(len(seqs)), ref, want_logits=True)
        got = host(tok)
        assert np.array_equal(got[seqs], ref), f"step {s}: tokens {got[seqs]} vs {ref}"
        glg = host(gm.logits(B))
        assert np.array_equal(bits(glg[seqs]), bits(lg)), f"step {s}: logits differ"
        hist.append(ref.copy())
        changed += prev is not None and not np.array_equal(bits(lg), prev)
        prev = bits(lg).copy()
    return np.stack(hist), changed


def test_config4_7b_shape_batch64_token_identity(ctx):
    from oracle import oracle as orc

    cfg = dict(orc.qwen_config("7b"), max_batch=64, max_seq=400)
    seed = 4
    B, V = 64, cfg["vocab"]
    seqs = [0, 63]                       # a long-prompt sequence and the last row tile's
    gm = lgx.Model(ctx, cfg, seed)
    om = orc.Model(dict(cfg, max_batch=len(seqs)), seed)
    rng = np.random.default_rng(44)
    p_long = rng.integers(0, V, size=(2, 300)).astype(np.int32)
    p_short = rng.integers(0, V, size=(B, 20)).astype(np.int32)
    gm.prefill(ctx.to_device(p_long))                 # sequences 0, 1: 300 tokens
    tok = gm.prefill(ctx.to_device(p_short))          # all 64: + 20
    om.prefill([0], p_long[:1])
    ref, lg = om.prefill([0, 1], p_short[seqs], want_logits=True)
    assert np.array_equal(host(tok)[seqs], ref)
    assert np.array_equal(bits(host(gm.logits(B))[seqs]), bits(lg))
    hist, changed = _decode_and_compare(gm, om, tok, seqs, ref, 64)
    assert len(np.unique(hist)) > 16                  # the check is not vacuous
    assert changed == 63
    lens = gm.tensor_bytes("seq_len", 0).view(np.int32)
    assert int(lens[0]) == 384 and int(lens[63]) == 84 and int(lens[5]) == 84
    for layer in (0, cfg["n_layers"] - 1):
        for which in (0, 1):
            assert np.array_equal(_kv_dense(gm, cfg, layer, which, 0, 384),
                                  om.kv(layer, which, 0, 384)), (layer, which)
    gm.close()
    om.close()


def test_config3_05b_shape_batch32_context2048_token_identity(ctx):
    from oracle import oracle as orc

    cfg = orc.qwen_config("0.5b")                     # max_batch 32, max_seq 2048 + 64
    seed = 3
    B, P, V = cfg["max_batch"], 2048, cfg["vocab"]
    seqs = [0, 31]
    gm = lgx.Model(ctx, cfg, seed)
    om = orc.Model(dict(cfg, max_batch=len(seqs)), seed)
    rng = np.random.default_rng(33)
    prompt = rng.integers(0, V, size=(B, P)).astype(np.int32)
    tok = gm.prefill(ctx.to_device(prompt))
    ref, lg = om.prefill([0, 1], prompt[seqs], want_logits=True)
    assert np.array_equal(host(tok)[seqs], ref)
    assert np.array_equal(bits(host(gm.logits(B))[seqs]), bits(lg))
    hist, changed = _decode_and_compare(gm, om, tok, seqs, ref, 64)
    # after 2048 random prompt tokens the random model settles on a few
    # tokens; the logits still change at every step, and they are the ones
    # compared bit for bit
    assert len(np.unique(hist)) >= 2
    assert changed == 63
    assert int(gm.tensor_bytes("seq_len", 0).view(np.int32)[31]) == P + 64
    for layer in (0, cfg["n_layers"] - 1):
        for which in (0, 1):
            assert np.array_equal(_kv_dense(gm, cfg, layer, which, 31, P + 64),
                                  om.kv(layer, which, 1, P + 64)), (layer, which)
    gm.close()
    om.close()
