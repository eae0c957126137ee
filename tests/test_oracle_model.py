"""Pin the oracle's decode-step glue and Qwen2-shaped model (no GPU).

The glue functions are checked against float64 numpy and closed forms; the
model step against an independent numpy forward of the same architecture
(float64 arithmetic, the GGML Q8_0 rule for activation quantisation) within
a tolerance, plus a planted architecture mistake that the comparison must
reject, and batch / slot invariance of the oracle itself."""
import numpy as np
import pytest


def test_rmsnorm(orc):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 896)).astype(np.float32) * 3
    y = orc.rmsnorm(x)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-6)
    assert np.allclose(y, ref, rtol=3e-6, atol=1e-7)
    # scale invariance and constant rows
    assert np.allclose(orc.rmsnorm(4 * x), y, rtol=1e-6, atol=1e-6)
    c = np.full((1, 3584), -2.5, np.float32)
    assert np.allclose(orc.rmsnorm(c), -1.0, atol=1e-6)


def test_rope_properties(orc):
    cos_t, sin_t = orc.rope_tables(4096, 128, 1e6)
    assert np.all(cos_t[0] == 1.0) and np.all(sin_t[0] == 0.0)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 128)).astype(np.float32)
    assert np.array_equal(orc.rope(x, cos_t[0], sin_t[0]), x)          # position 0
    y = orc.rope(x, cos_t[777], sin_t[777])
    assert np.allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=1e-5)
    # rotate-half pairing (i, i + d/2) with angle p * theta^(-2i/d)
    i = 5
    ang = 777 * 1e6 ** (-2 * i / 128)
    ref_i = x[0, i] * np.cos(ang) - x[0, i + 64] * np.sin(ang)
    assert abs(y[0, i] - ref_i) < 1e-5
    # relative position: <R_p q, R_s k> depends only on p - s
    q, k = x[0:1], x[1:2]
    d1 = np.dot(orc.rope(q, cos_t[100], sin_t[100])[0], orc.rope(k, cos_t[90], sin_t[90])[0])
    d2 = np.dot(orc.rope(q, cos_t[2010], sin_t[2010])[0], orc.rope(k, cos_t[2000], sin_t[2000])[0])
    assert abs(d1 - d2) < 1e-3


def test_swiglu_and_argmax(orc):
    rng = np.random.default_rng(2)
    gu = rng.standard_normal((3, 2 * 64)).astype(np.float32) * 4
    a = orc.swiglu(gu).astype(np.float64)
    g, u = gu[:, :64].astype(np.float64), gu[:, 64:].astype(np.float64)
    assert np.allclose(a, g / (1 + np.exp(-g)) * u, rtol=1e-6, atol=1e-7)
    z = np.zeros((1, 8), np.float32)
    assert np.all(orc.swiglu(z) == 0.0)
    v = np.array([1.0, 3.0, -1.0, 3.0, 2.0], np.float32)
    assert orc.argmax(v) == 1                          # ties -> lowest index
    assert orc.argmax(np.array([-0.0, 0.0], np.float32)) == 0
    assert orc.argmax(np.array([np.nan, 1.0, 1.0], np.float32)) == 1


def test_lm_head_f16(orc):
    rng = np.random.default_rng(3)
    E = (rng.standard_normal((300, 2100)) * 0.02).astype(np.float16)
    x = rng.standard_normal((2, 2100)).astype(np.float32)
    out = orc.lm_head_f16(x, E.view(np.uint16))
    ref = x.astype(np.float64) @ E.astype(np.float64).T
    assert np.allclose(out, ref, rtol=1e-5, atol=1e-5)
    e = np.zeros((1, 2100), np.float32)
    e[0, 1500] = 1.0
    assert np.array_equal(orc.lm_head_f16(e, E.view(np.uint16))[0],
                          E[:, 1500].astype(np.float32))


# ---- independent numpy forward of the model ---------------------------------

def _q8_np(x):
    """GGML Q8_0 rule in binary32 numpy arithmetic -> dequantised float64."""
    xb = x.astype(np.float32).reshape(-1, 32)
    amax = np.abs(xb).max(1).astype(np.float32)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    v = (xb * idv[:, None]).astype(np.float32).astype(np.float64)
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -127, 127)
    return (q * d.astype(np.float16).astype(np.float64)[:, None]).reshape(x.shape)


class NumpyQwen:
    def __init__(self, orc, m, rope_pairing="half"):
        c = m.cfg
        self.c, self.pairing = c, rope_pairing
        self.E = m.tensor("emb").view(np.float16).astype(np.float64)

        def deq(q, d):
            return (q.astype(np.float64).reshape(q.shape[0], -1, 32) *
                    d.view(np.float16).astype(np.float64)[:, :, None]).reshape(q.shape)

        self.L = []
        for l in range(c["n_layers"]):
            self.L.append(dict(
                qkv=deq(m.tensor("qkv_q", l), m.tensor("qkv_d", l)),
                o=deq(m.tensor("o_q", l), m.tensor("o_d", l)),
                gu=deq(m.tensor("gu_q", l), m.tensor("gu_d", l)),
                dn=deq(m.tensor("dn_q", l), m.tensor("dn_d", l)),
                b=m.tensor("bias", l).astype(np.float64)))
        self.lm = None if c["tied"] else deq(m.tensor("lm_q"), m.tensor("lm_d"))
        self.kv = [[[], []] for _ in range(c["n_layers"])]

    def rope(self, x, pos):
        d = self.c["head_dim"]
        i = np.arange(d // 2)
        ang = pos * self.c["theta"] ** (-2.0 * i / d)
        cs, sn = np.cos(ang), np.sin(ang)
        if self.pairing == "half":
            a, b = x[..., :d // 2], x[..., d // 2:]
            return np.concatenate([a * cs - b * sn, b * cs + a * sn], -1)
        a, b = x[..., 0::2], x[..., 1::2]                  # planted mistake: interleaved
        out = np.empty_like(x)
        out[..., 0::2], out[..., 1::2] = a * cs - b * sn, b * cs + a * sn
        return out

    def step(self, tok):
        c = self.c
        H, d, hq, hkv = c["hidden"], c["head_dim"], c["n_heads"], c["n_kv"]
        pos = len(self.kv[0][0])
        h = self.E[tok].copy()

        def norm(v):
            return v / np.sqrt((v * v).mean() + c["eps"])

        for l, W in enumerate(self.L):
            qkv = W["qkv"] @ _q8_np(norm(h)) + W["b"]
            q = self.rope(qkv[:hq * d].reshape(hq, d), pos)
            k = self.rope(qkv[hq * d:(hq + hkv) * d].reshape(hkv, d), pos)
            v = qkv[(hq + hkv) * d:].reshape(hkv, d)
            self.kv[l][0].append(k.astype(np.float16).astype(np.float64))
            self.kv[l][1].append(v.astype(np.float16).astype(np.float64))
            K, V = np.stack(self.kv[l][0]), np.stack(self.kv[l][1])
            o = np.empty((hq, d))
            for hh in range(hq):
                g = hh // (hq // hkv)
                s = K[:, g] @ q[hh] / np.sqrt(d)
                w = np.exp(s - s.max())
                o[hh] = (w[:, None] * V[:, g]).sum(0) / w.sum()
            h = h + W["o"] @ _q8_np(o.ravel())
            gu = W["gu"] @ _q8_np(norm(h))
            g, u = gu[:c["inter"]], gu[c["inter"]:]
            h = h + W["dn"] @ _q8_np(g / (1 + np.exp(-g)) * u)
        xn = norm(h)
        return (self.E @ xn) if c["tied"] else (self.lm @ _q8_np(xn))


@pytest.mark.parametrize("name", ["tiny", "tiny_untied"])
def test_model_against_numpy_forward(orc, name):
    m = orc.Model(orc.qwen_config(name), seed=11)
    ref = NumpyQwen(orc, m)
    bad = NumpyQwen(orc, m, rope_pairing="interleaved")
    toks = [17]
    for step in range(6):
        nxt, logits = m.step([0], [toks[-1]], want_logits=True)
        r = ref.step(toks[-1])
        rb = bad.step(toks[-1])
        scale = np.abs(r).max()
        # measured: ~5e-7 of the logit scale for the oracle, ~1e-2 for the mutant
        assert np.max(np.abs(logits[0] - r)) < 1e-3 * scale, step
        if step >= 1:                                      # pairing matters from pos 1 on
            assert np.max(np.abs(logits[0] - rb)) > 3e-3 * scale, step
        toks.append(int(nxt[0]))
    m.close()


def test_model_batch_and_slot_invariance(orc):
    """Sequences are independent: stepping slots together or one at a time
    (in any slot order) gives identical tokens and logits."""
    cfg = orc.qwen_config("tiny")
    a, b = orc.Model(cfg, 5), orc.Model(cfg, 5)
    ta = np.array([3, 9, 27, 81], np.int32)
    tb = ta.copy()
    for step in range(8):
        na, la = a.step([0, 1, 2, 3], ta, want_logits=True)
        nb = np.empty(4, np.int32)
        lb = np.empty_like(la)
        for s in (2, 0, 3, 1):
            n1, l1 = b.step([s], tb[s:s + 1], want_logits=True)
            nb[s], lb[s] = n1[0], l1[0]
        assert np.array_equal(na, nb) and np.array_equal(la, lb)
        ta, tb = na, nb
    assert a.seq_len(0) == 8
    a.close()
    b.close()


@pytest.mark.parametrize("name", ["tiny", "tiny_untied"])
def test_prefill_equals_repeated_steps(orc, name):
    """orc_model_prefill (all positions of a chunk per layer at once) equals
    P calls of the already-pinned step bit for bit: next tokens, logits,
    hidden rows and every cached K/V row, over two chunks per slot with
    ragged start lengths, a 256-token attention-chunk boundary crossed
    inside a chunk, and slots passed out of order."""
    cfg = orc.qwen_config(name)
    seed = 606
    a, b = orc.Model(cfg, seed), orc.Model(cfg, seed)
    rng = np.random.default_rng(7)
    V = cfg["vocab"]
    slots = np.array([2, 0], np.int32)
    # chunk 1: slot 2 gets 250 tokens, slot 0 gets 250 (then both cross 256)
    for P in (250, 19):
        toks = rng.integers(0, V, size=(2, P)).astype(np.int32)
        na, la, ha = a.prefill(slots, toks, want_logits=True, want_hidden=True)
        for p in range(P):
            nb, lb, hb = b.step(slots, toks[:, p], want_logits=True, want_hidden=True)
        assert np.array_equal(na, nb)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        assert np.array_equal(ha.view(np.uint32), hb.view(np.uint32))
    # a third slot starting later, alone
    toks = rng.integers(0, V, size=(1, 7)).astype(np.int32)
    assert np.array_equal(a.prefill([1], toks), [b.step([1], toks[:, p]) for p in range(7)][-1])
    for s in (0, 1, 2, 3):
        assert a.seq_len(s) == b.seq_len(s)
    for layer in range(cfg["n_layers"]):
        for s in (0, 1, 2):
            n = a.seq_len(s)
            for which in (0, 1):
                assert np.array_equal(a.kv(layer, which, s, n), b.kv(layer, which, s, n))
    a.close()
    b.close()


def test_load_kv_round_trip_and_decode(orc):
    """A cache copied out of one model (kv) and loaded into another
    (load_kv + set_seq_len) decodes exactly as the model that made it."""
    cfg = orc.qwen_config("tiny")
    a, b = orc.Model(cfg, 9), orc.Model(cfg, 9)
    rng = np.random.default_rng(8)
    toks = rng.integers(0, cfg["vocab"], size=(1, 40)).astype(np.int32)
    nxt = a.prefill([3], toks)
    for layer in range(cfg["n_layers"]):
        for which in (0, 1):
            rows = a.kv(layer, which, 3, 40)
            b.load_kv(layer, which, 1, rows)
            assert np.array_equal(b.kv(layer, which, 1, 40), rows)
    b.set_seq_len(1, 40)
    ta, tb = nxt.copy(), nxt.copy()
    for _ in range(5):
        ta, la = a.step([3], ta, want_logits=True)
        tb, lb = b.step([1], tb, want_logits=True)
        assert np.array_equal(ta, tb)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    a.close()
    b.close()


def test_q8_embedding_gather_and_tied_head(orc):
    """orc_model_set_emb_q8: the gather is f32(d) * q per element (checked on
    the hidden rows of a zero-layer-like comparison: the same model with the
    binary16 embedding set to a Q8_0 matrix whose dequantised values are
    binary16-exact gives the same hidden rows), and the tied model's logits
    with a Q8_0 embedding equal an untied model's whose lm_head is that
    matrix."""
    import numpy as np

    cfg_t = dict(orc.qwen_config("tiny"), vocab=1008, max_batch=2, max_seq=32)
    cfg_u = dict(cfg_t, tied=0)
    rng = np.random.default_rng(4)
    V, H = cfg_t["vocab"], cfg_t["hidden"]
    # quants times power-of-two scales: f32(d) * q is exact in binary16 too
    qs = rng.integers(-127, 128, size=(V, H), dtype=np.int8)
    d = orc.f32_to_f16(np.full((V, H // 32), 2.0 ** -14, np.float32))
    emb16 = orc.f32_to_f16(qs.astype(np.float32) * np.float32(2.0 ** -14))
    a = orc.Model(cfg_t, 9)
    b = orc.Model(cfg_t, 9)
    a.set_emb_q8(qs, d)
    b.set_tensor("emb", 0, emb16)
    toks = np.array([3, 999], np.int32)
    _, ha = a.step([0, 1], toks, want_hidden=True)
    _, hb = b.step([0, 1], toks, want_hidden=True)
    assert np.array_equal(ha.view(np.uint32), hb.view(np.uint32))
    # tied Q8_0 head == untied head with the same matrix (general scales)
    d2 = orc.f32_to_f16((np.abs(rng.standard_normal((V, H // 32))) * 0.02 / 127).astype(np.float32))
    t = orc.Model(cfg_t, 9)
    u = orc.Model(cfg_u, 9)
    t.set_emb_q8(qs, d2)
    u.set_emb_q8(qs, d2)
    u.set_tensor("lm_q", 0, qs)
    u.set_tensor("lm_d", 0, d2)
    nt, lt = t.step([0, 1], toks, want_logits=True)
    nu, lu = u.step([0, 1], toks, want_logits=True)
    assert np.array_equal(lt.view(np.uint32), lu.view(np.uint32)) and np.array_equal(nt, nu)
    for m in (a, b, t, u):
        m.close()
