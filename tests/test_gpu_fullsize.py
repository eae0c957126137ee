"""The benchmarked workloads at their full size, against the CPU oracle.

* Config 4 exactly as bench.py runs it: the Qwen2.5-7B-shaped model at batch
  64 with 4096-token prompts, so the prefill runs 32 chunks of 64 x 128 =
  8192 rows through the tiled products (gate|up 37888 x 3584 with the fused
  SwiGLU, down 3584 x 18944, qkv, o_proj) and the causal prefill attention up
  to 4095 cached tokens, then 64 greedy decode steps at contexts 4096..4159.
  Sequence 0 (the first row tiles of every chunk) is prefilled by the oracle
  on its own, all 4096 positions, independently of the device: its K/V rows
  at every layer, the prefill's next token and logits must equal the
  device's bit for bit.  Sequence 63 (the last row tiles) is checked position
  by position at sampled positions: the oracle, given the device's cache of
  that sequence up to position p, steps position p, and its K/V at p (every
  layer) must equal the device's -- the same operations the device's batched
  prefill applies to that row.  Both sequences then decode 64 steps in the
  oracle beside the device batch, tokens and logits compared at every step.
* Config 4 through the opt-in fast prefill: the caches of sequences 0 and 63
  loaded into the oracle give the device's next token, logits and last K/V
  row bit for bit, and 64 greedy steps after it stay bit-exact.
* The tiled product through the lgx_q8_gemm entry point at M = 8192 (one
  prefill chunk) for the 7B gate|up and down shapes, sampled rows against
  the oracle (rows are independent in the canonical product).
"""
import time

import numpy as np
import pytest

import logicaffeine_amd as lgx

pytestmark = pytest.mark.gpu


def host(t):
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _log(msg, t0):
    print(f"[fullsize {time.perf_counter() - t0:7.1f} s] {msg}", flush=True)


@pytest.mark.timeout(900)
def test_config4_bench_workload_prompt4096_batch64(ctx):
    from oracle import oracle as orc

    t0 = time.perf_counter()
    P, B, steps, seed = 4096, 64, 64, 4
    cfg = dict(orc.qwen_config("7b"), max_batch=B, max_seq=P + steps)
    V, nl = cfg["vocab"], cfg["n_layers"]
    rng = np.random.default_rng(4096)
    prompt = rng.integers(0, V, size=(B, P)).astype(np.int32)
    gm = lgx.Model(ctx, cfg, seed)
    tok = gm.prefill(ctx.to_device(prompt))
    dev_next = host(tok)
    dev_logits = host(gm.logits(B))
    lens = gm.tensor_bytes("seq_len", 0).view(np.int32)
    assert np.all(lens[:B] == P)
    _log("device prefill done", t0)

    om = orc.Model(dict(cfg, max_batch=2), seed)
    _log("oracle model built", t0)
    # sequence 0: the oracle's own prefill of all 4096 positions
    ref0, lg0 = om.prefill([0], prompt[:1], want_logits=True)
    _log("oracle prefill of sequence 0 done", t0)
    assert int(dev_next[0]) == int(ref0[0])
    assert np.array_equal(bits(dev_logits[0]), bits(lg0[0]))
    pt = gm.tensor_bytes("page_table").view(np.int32).reshape(B, -1)
    for layer in range(nl):
        for which in (0, 1):
            got = gm.kv_rows(layer, which, 0, P, page_table=pt)
            assert np.array_equal(got, om.kv(layer, which, 0, P)), (layer, which)
    _log("sequence 0: K/V of all 28 layers x 4096 positions equal", t0)

    # sequence 63 in oracle slot 1: the device's cache, then position-by-
    # position steps at sampled positions (ascending, so the positions the
    # oracle rewrites are ones already found equal)
    dev63 = [[gm.kv_rows(layer, which, 63, P, page_table=pt) for which in (0, 1)]
             for layer in range(nl)]
    for layer in range(nl):
        om.load_kv(layer, 0, 1, dev63[layer][0])
        om.load_kv(layer, 1, 1, dev63[layer][1])
    sampled = sorted(set([0, 1, 15, 16, 127, 128, 255, 256, 1023, 2047, 2048, 3000, 3071,
                          3072, 4094] + list(rng.integers(1, P - 1, size=9))))
    for p in sampled:
        om.set_seq_len(1, int(p))
        om.step([1], prompt[63, p:p + 1])
        for layer in range(nl):
            for which in (0, 1):
                row = om.kv(layer, which, 1, int(p) + 1)[p]
                assert np.array_equal(row, dev63[layer][which][p]), (int(p), layer, which)
    om.set_seq_len(1, P - 1)
    ref63, lg63 = om.step([1], prompt[63, P - 1:P], want_logits=True)
    assert int(dev_next[63]) == int(ref63[0])
    assert np.array_equal(bits(dev_logits[63]), bits(lg63[0]))
    for layer in (0, nl - 1):
        for which in (0, 1):
            assert np.array_equal(om.kv(layer, which, 1, P), dev63[layer][which]), (layer, which)
    _log(f"sequence 63: {len(sampled) + 1} sampled positions equal at every layer", t0)
    del dev63

    # 64 greedy steps of the device batch; the oracle steps both sequences
    ref = np.array([ref0[0], ref63[0]], np.int32)
    seqs = [0, 63]
    hist, changed, prev = [], 0, None
    for s in range(steps):
        gm.decode_step(tok)
        ref, lg = om.step([0, 1], ref, want_logits=True)
        got = host(tok)
        assert np.array_equal(got[seqs], ref), f"step {s}: tokens {got[seqs]} vs {ref}"
        assert np.array_equal(bits(host(gm.logits(B))[seqs]), bits(lg)), f"step {s}: logits"
        hist.append(ref.copy())
        changed += prev is not None and not np.array_equal(bits(lg), prev)
        prev = bits(lg).copy()
    _log(f"{steps} decode steps equal in tokens and logits", t0)
    # after 4096 random prompt tokens the random model cycles through a
    # dozen tokens; the logits change at every step and are compared bit
    # for bit
    assert len(np.unique(np.stack(hist))) >= 8
    assert changed == steps - 1
    for layer in (0, nl - 1):
        for which in (0, 1):
            assert np.array_equal(gm.kv_rows(layer, which, 0, P + steps, page_table=pt),
                                  om.kv(layer, which, 0, P + steps)), (layer, which)
    gm.close()
    om.close()


@pytest.mark.timeout(900)
def test_config4_fast_prefill_then_64_decode_steps_bit_exact(ctx):
    """Config 4 through the opt-in fast prefill (binary16 GEMMs and flash
    attention): sequences 0 and 63's caches (positions 0..4094, all 28
    layers), loaded into the oracle, give the device's next token, logits and
    last-position K/V bit for bit, then 64 greedy steps of both, tokens and
    logits, bit for bit."""
    from oracle import oracle as orc

    t0 = time.perf_counter()
    P, B, steps, seed = 4096, 64, 64, 4
    cfg = dict(orc.qwen_config("7b"), max_batch=B, max_seq=P + steps)
    V, nl = cfg["vocab"], cfg["n_layers"]
    rng = np.random.default_rng(4097)
    prompt = rng.integers(0, V, size=(B, P)).astype(np.int32)
    gm = lgx.Model(ctx, cfg, seed)
    gm.set_prefill_mode(True)
    tok = gm.prefill(ctx.to_device(prompt))
    dev_next = host(tok)
    dev_logits = host(gm.logits(B))
    pt = gm.tensor_bytes("page_table").view(np.int32).reshape(B, -1)
    _log("device fast prefill done", t0)
    seqs = [0, 63]
    kv = {b: [[gm.kv_rows(layer, w, b, P, page_table=pt) for w in (0, 1)] for layer in range(nl)]
          for b in seqs}
    om = orc.Model(dict(cfg, max_batch=2), seed)
    for slot, b in enumerate(seqs):
        for layer in range(nl):
            for w in (0, 1):
                om.load_kv(layer, w, slot, kv[b][layer][w][:P - 1])
        om.set_seq_len(slot, P - 1)
    ref, lg = om.step([0, 1], prompt[seqs, P - 1], want_logits=True)
    assert np.array_equal(dev_next[seqs], ref)
    assert np.array_equal(bits(dev_logits[seqs]), bits(lg))
    for slot, b in enumerate(seqs):
        for layer in range(nl):
            for w in (0, 1):
                assert np.array_equal(om.kv(layer, w, slot, P)[P - 1], kv[b][layer][w][P - 1]), (b, layer, w)
    _log("last prompt position equal at every layer", t0)
    del kv
    hist = []
    for s in range(steps):
        gm.decode_step(tok)
        ref, lg = om.step([0, 1], ref, want_logits=True)
        got = host(tok)
        assert np.array_equal(got[seqs], ref), f"step {s}: tokens {got[seqs]} vs {ref}"
        assert np.array_equal(bits(host(gm.logits(B))[seqs]), bits(lg)), f"step {s}: logits"
        hist.append(ref.copy())
    assert len(np.unique(np.stack(hist))) >= 8
    _log(f"{steps} decode steps equal in tokens and logits", t0)
    gm.close()
    om.close()


@pytest.mark.parametrize("n,k", [(37888, 3584), (3584, 18944)])
def test_q8_gemm_7b_shapes_m8192_sampled_rows(ctx, orc, n, k):
    m = 8192
    rng = np.random.default_rng(n + k)
    qs, d = orc.gen_q8_matrix(4, 9000 + k % 1000, n, k)
    xq = rng.integers(-127, 128, size=(m, k)).astype(np.int8)
    xd = orc.f32_to_f16((np.abs(rng.standard_normal((m, k // 32))) * 0.01).astype(np.float32))
    W = ctx.q8_matrix(qs, d)
    y = ctx.q8_gemm(W, ctx.to_device(xq), ctx.to_device(xd))
    rows = np.unique(np.concatenate([np.arange(16), rng.integers(16, m - 16, size=32),
                                     np.arange(m - 16, m)]))
    got = host(y[ctx.to_device(rows.astype(np.int64))])
    ref = orc.q8_gemm(qs, d, xq[rows], xd[rows])
    assert np.array_equal(bits(got), bits(ref))
