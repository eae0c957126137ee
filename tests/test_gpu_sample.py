"""Seeded top-k / top-p sampling on the device against the CPU oracle.

lgx_sample and the model's sampled decode (lgx_model_set_sampling) must draw
the oracle's token ids bit for bit: the same candidate order (ties, NaN,
-0), the same binary32 weights and prefix sums, the same SplitMix64 draw.
"""
import numpy as np
import pytest

import logicaffeine_amd as lgx

pytestmark = pytest.mark.gpu


def host(t):
    return t.cpu().numpy()


def _logits(rng, m, V):
    x = (rng.standard_normal((m, V)) * 2.5).astype(np.float32)
    x[0, :] = 1.25                                   # all equal: lowest indices win
    x[1, ::7] = np.nan                               # NaN never a candidate
    x[2, :] = np.nan                                 # no candidate at all: 0
    x[3, 5:9] = 40.0                                 # a tie at the top
    x[3, 100] = -0.0
    x[4, :] = -np.inf
    x[4, 17] = 0.0                                   # -inf weights are zero
    x[5, V - 1] = 30.0                               # the maximum in the last slice
    return x


@pytest.mark.parametrize("V", [152064, 4096, 4097, 1000])
@pytest.mark.parametrize("top_k,top_p,temp", [(1, 1.0, 1.0), (40, 0.95, 0.8), (64, 1.0, 1.7),
                                              (7, 0.3, 0.6), (64, 0.999, 1.0)])
def test_sample_bit_exact(ctx, orc, V, top_k, top_p, temp):
    rng = np.random.default_rng(V + top_k)
    m = 64
    x = _logits(rng, m, V)
    pos = rng.integers(0, 5000, size=m).astype(np.int32)
    seed = 20261202 + top_k
    got = host(ctx.sample(ctx.to_device(x), ctx.to_device(pos), top_k, top_p, temp, seed))
    want = orc.sample(x, top_k, top_p, temp, seed, np.arange(m), pos)
    assert np.array_equal(got, want)
    assert got[2] == 0 and got[4] == 17
    if top_k == 1:
        assert got[0] == 0 and got[3] == 5 and got[5] == V - 1


def test_sample_argument_errors(ctx):
    x = ctx.to_device(np.zeros((2, 100), np.float32))
    pos = ctx.to_device(np.zeros(2, np.int32))
    for k, p, t in ((0, 1.0, 1.0), (65, 1.0, 1.0), (5, 0.0, 1.0), (5, 1.5, 1.0), (5, 1.0, 0.0),
                    (5, 1.0, -1.0), (5, 1.0, float("inf"))):
        with pytest.raises(lgx.LgxError) as e:
            ctx.sample(x, pos, k, p, t, 1)
        assert e.value.status_name == "LGX_INVALID_ARGUMENT", (k, p, t)


@pytest.mark.parametrize("name", ["tiny", "tiny_untied"])
def test_model_sampled_decode_bit_exact(ctx, name):
    """Sampled prefill, eager steps and graph replays give the oracle model's
    sampled tokens (stream = sequence, draw index = consumed position); back
    to greedy with temperature 0."""
    from oracle import oracle as orc

    cfg = orc.qwen_config(name)
    seed = 77
    B, V = cfg["max_batch"], cfg["vocab"]
    gm, om = lgx.Model(ctx, cfg, seed), orc.Model(cfg, seed)
    gm.set_sampling(0.9, 40, 0.95, 123)
    om.set_sampling(0.9, 40, 0.95, 123)
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, V, size=(B, 9)).astype(np.int32)
    tok = gm.prefill(ctx.to_device(prompt))
    ref = om.prefill(np.arange(B), prompt)
    assert np.array_equal(host(tok), ref)
    seen = set(ref.tolist())
    for s in range(10):
        gm.decode_step(tok)
        ref = om.step(np.arange(B), ref)
        assert np.array_equal(host(tok), ref), s
        seen |= set(ref.tolist())
    hist = ctx.torch.empty((6, B), dtype=ctx.torch.int32, device=ctx.dev)
    gm.generate(tok, 6, hist)
    for s in range(6):
        ref = om.step(np.arange(B), ref)
        assert np.array_equal(host(hist[s]), ref), s
    assert len(seen) > 8
    # another setting drops the recorded graph; greedy again with 0
    gm.set_sampling(1.3, 5, 0.7, 9)
    om.set_sampling(1.3, 5, 0.7, 9)
    gm.generate(tok, 3, hist[:3])
    for s in range(3):
        ref = om.step(np.arange(B), ref)
        assert np.array_equal(host(hist[s]), ref), s
    gm.set_sampling(0.0)
    om.set_sampling(0.0)
    for s in range(3):
        gm.decode_step(tok)
        ref, lg = om.step(np.arange(B), ref, want_logits=True)
        assert np.array_equal(host(tok), ref)
        assert np.array_equal(ref, [orc.argmax(r) for r in lg])
    with pytest.raises(lgx.LgxError):
        gm.set_sampling(1.0, 0, 1.0, 1)
    gm.close()
    om.close()
