"""Generate the committed golden fixtures for the Q8 path.

The reference (LOGOS 0.10.1) holds no vectors for this path (it has no GEMV,
attention or LLM code), so the fixtures are computed here with numpy from the
public definitions, independently of the C oracle:

* inputs come from numpy's PCG64 generator (not the oracle's SplitMix64);
* Q8_0 activation quantisation is restated with numpy binary32 arithmetic
  (GGML rule: d = amax/127, id = 1/d, q = round-half-away(x*id)), so the
  expected quants and scale bits are exact;
* block dot products are exact int64;
* GEMV / GEMM outputs are float64 sums of exact terms, checked against the
  oracle's binary32 canonical schedule with an error bound.

Run: python tests/golden/gen_golden.py   (writes q8_golden.npz beside itself)
"""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def quantize_q8_0_np(x: np.ndarray):
    """GGML Q8_0 reference rule in binary32 numpy arithmetic."""
    m, k = x.shape
    xb = x.reshape(m, k // 32, 32).astype(np.float32)
    amax = np.max(np.abs(xb), axis=2).astype(np.float32)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    v = (xb * idv[:, :, None]).astype(np.float32).astype(np.float64)
    q = np.sign(v) * np.floor(np.abs(v) + 0.5)
    q = np.clip(q, -127, 127).astype(np.int8).reshape(m, k)
    return q, d.astype(np.float16).view(np.uint16)


def case(rng, n, k, m):
    nb = k // 32
    qs = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    d = (np.abs(rng.normal(0.0, 0.02, size=(n, nb))) / 127.0).astype(np.float16)
    x = rng.standard_normal((m, k)).astype(np.float32)
    xq, xd = quantize_q8_0_np(x)
    s = np.einsum("nbi,mbi->mnb", qs.reshape(n, nb, 32).astype(np.int64),
                  xq.reshape(m, nb, 32).astype(np.int64))
    dw = d.astype(np.float64)
    dx = xd.view(np.float16).astype(np.float64)
    terms = s.astype(np.float64) * dw[None, :, :] * dx[:, None, :]
    y_q8q8 = terms.sum(axis=2)
    y_q8q8_abs = np.abs(terms).sum(axis=2)
    # binary32-activation GEMV of x[0]
    t32 = (qs.reshape(n, nb, 32).astype(np.float64) *
           x[0].reshape(nb, 32).astype(np.float64)[None]).sum(axis=2) * dw
    y_f32 = t32.sum(axis=1)
    y_f32_abs = (np.abs(qs.reshape(n, nb, 32).astype(np.float64) *
                        x[0].reshape(nb, 32).astype(np.float64)[None]).sum(axis=2) * dw).sum(axis=1)
    return dict(qs=qs, d=d.view(np.uint16), x=x, xq=xq, xd=xd, s=s.astype(np.int32),
                y_q8q8=y_q8q8, y_q8q8_abs=y_q8q8_abs, y_f32=y_f32, y_f32_abs=y_f32_abs)


def attn_case(rng, B, hq, hkv, d, lens, maxp):
    """Paged fp16 KV cache with a random page table, float64 softmax attention."""
    npages = B * maxp
    k = rng.standard_normal((npages, hkv, 16, d)).astype(np.float16)
    v = rng.standard_normal((npages, hkv, 16, d)).astype(np.float16)
    pt = rng.permutation(npages).astype(np.int32).reshape(B, maxp)
    q = rng.standard_normal((B, hq, d)).astype(np.float32)
    out = np.zeros((B, hq, d))
    gq = hq // hkv
    for b in range(B):
        L = lens[b]
        kk = np.stack([k[pt[b, t // 16], :, t % 16, :] for t in range(L)]).astype(np.float64)
        vv = np.stack([v[pt[b, t // 16], :, t % 16, :] for t in range(L)]).astype(np.float64)
        for h in range(hq):
            g = h // gq
            sc = kk[:, g, :] @ q[b, h].astype(np.float64) / np.sqrt(d)
            w = np.exp(sc - sc.max())
            out[b, h] = (w[:, None] * vv[:, g, :]).sum(0) / w.sum()
    return dict(q=q, k=k.view(np.uint16), v=v.view(np.uint16), pt=pt,
                lens=np.asarray(lens, np.int32), out=out)


def main():
    rng = np.random.default_rng(20261201)
    out = {}
    # single range (6 blocks) and three ranges (66 blocks = 32 + 32 + 2)
    for name, (n, k, m) in {"small": (48, 192, 3), "ranges": (32, 2112, 2)}.items():
        for key, v in case(rng, n, k, m).items():
            out[f"{name}_{key}"] = v
    # quantiser edge cases: zero block, ramp, one dominant element, tiny values
    e = np.zeros((4, 32), np.float32)
    e[1] = np.arange(32, dtype=np.float32) * np.float32(0.37)
    e[2] = np.float32(1e-3)
    e[2, 7] = np.float32(-5.0)
    e[3] = np.float32(3e-7) * np.arange(-16, 16, dtype=np.float32)
    eq, ed = quantize_q8_0_np(e)
    out.update(edge_x=e, edge_q=eq, edge_d=ed)
    for key, val in attn_case(rng, 3, 6, 2, 64, [1, 300, 700], 48).items():
        out[f"attn_{key}"] = val
    path = os.path.join(HERE, "q8_golden.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
