"""Writer of small GGUF files for the loader tests (test infrastructure).

The GGUF container as the llama.cpp project publishes it: little-endian
"GGUF", version u32, tensor count u64, metadata count u64; metadata entries
(key string, value type u32, value); tensor infos (name, n_dims u32, dims
u64 with dims[0] the row length, ggml type u32, offset u64 into the data
section); zero padding to the alignment; the tensor data, each tensor at an
aligned offset.  Strings are a u64 byte count and the bytes.  A Q8_0 row is
blocks of (binary16 scale, 32 int8 quants).
"""
import struct

import numpy as np

T_U32, T_I32, T_F32, T_STRING, T_ARRAY, T_U64 = 4, 5, 6, 8, 9, 10
GGML_F32, GGML_F16, GGML_Q8_0 = 0, 1, 8


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v) -> bytes:
    if vtype == T_U32:
        return struct.pack("<I", v)
    if vtype == T_I32:
        return struct.pack("<i", v)
    if vtype == T_U64:
        return struct.pack("<Q", v)
    if vtype == T_F32:
        return struct.pack("<f", v)
    if vtype == T_STRING:
        return _s(v)
    if vtype == T_ARRAY:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, x) for x in items)
    raise ValueError(vtype)


def q8_rows(qs: np.ndarray, d: np.ndarray) -> bytes:
    """Row-major quants [n][k] int8 + scales [n][k/32] (binary16 bits) ->
    Q8_0 blocks."""
    n, k = qs.shape
    blk = np.empty((n, k // 32, 34), np.uint8)
    blk[:, :, 0:2] = np.ascontiguousarray(d, np.uint16).reshape(n, k // 32, 1).view(np.uint8)
    blk[:, :, 2:] = np.ascontiguousarray(qs, np.int8).reshape(n, k // 32, 32).view(np.uint8)
    return blk.tobytes()


def write_gguf(path, meta, tensors, alignment=32, version=3, magic=b"GGUF"):
    """meta: [(key, value type, value)]; tensors: [(name, ggml type, data)]
    with data a float32 / uint16 (binary16) array or (qs, d) for Q8_0."""
    blobs, infos = [], []
    off = 0
    for name, gtype, data in tensors:
        if gtype == GGML_Q8_0:
            qs, d = data
            rows, cols = qs.shape
            dims = [cols, rows]
            raw = q8_rows(qs, d)
        else:
            arr = np.ascontiguousarray(data, np.float32 if gtype == GGML_F32 else np.uint16)
            dims = [arr.shape[0]] if arr.ndim == 1 else [arr.shape[1], arr.shape[0]]
            raw = arr.tobytes()
        off = (off + alignment - 1) // alignment * alignment
        infos.append(_s(name) + struct.pack("<I", len(dims)) +
                     b"".join(struct.pack("<Q", x) for x in dims) + struct.pack("<IQ", gtype, off))
        blobs.append((off, raw))
        off += len(raw)
    head = magic + struct.pack("<IQQ", version, len(tensors), len(meta))
    head += b"".join(_s(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in meta)
    head += b"".join(infos)
    pad = (len(head) + alignment - 1) // alignment * alignment - len(head)
    data = bytearray(off)
    for o, raw in blobs:
        data[o:o + len(raw)] = raw
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad + bytes(data))


def qwen2_meta(cfg, alignment=None, extra=()):
    m = [("general.architecture", T_STRING, "qwen2"),
         ("qwen2.block_count", T_U32, cfg["n_layers"]),
         ("qwen2.embedding_length", T_U32, cfg["hidden"]),
         ("qwen2.feed_forward_length", T_U32, cfg["inter"]),
         ("qwen2.attention.head_count", T_U32, cfg["n_heads"]),
         ("qwen2.attention.head_count_kv", T_U32, cfg["n_kv"]),
         ("qwen2.attention.key_length", T_U32, cfg["head_dim"]),
         ("qwen2.attention.value_length", T_U32, cfg["head_dim"]),
         ("qwen2.attention.layer_norm_rms_epsilon", T_F32, cfg["eps"]),
         ("qwen2.rope.freq_base", T_F32, cfg["theta"]),
         ("tokenizer.ggml.tokens", T_ARRAY, (T_STRING, ["<a>", "bb", "c"])),
         ("tokenizer.ggml.token_type", T_ARRAY, (T_I32, [1, 2, 3]))]
    if alignment:
        m.append(("general.alignment", T_U32, alignment))
    return m + list(extra)


def qwen2_tensors(cfg, t):
    """GGUF tensor list of a Qwen2 model from a dict of arrays (the oracle's
    names: emb, lm_q/lm_d, per layer qkv_q/qkv_d (rows q | k | v), o, gu
    (rows gate | up), dn, bias and the norm weights)."""
    H, I, d = cfg["hidden"], cfg["inter"], cfg["head_dim"]
    qd, kd = cfg["n_heads"] * d, cfg["n_kv"] * d
    emb = ("token_embd.weight", GGML_Q8_0, (t["emb_q"], t["emb_d"])) if "emb_q" in t else \
        ("token_embd.weight", GGML_F16, t["emb"])
    out = [emb, ("output_norm.weight", GGML_F32, t["out_norm"])]
    if not cfg["tied"]:
        out.append(("output.weight", GGML_Q8_0, (t["lm_q"], t["lm_d"])))
    for l in range(cfg["n_layers"]):
        b = f"blk.{l}."
        qq, qdd = t[("qkv_q", l)], t[("qkv_d", l)]
        gq, gd = t[("gu_q", l)], t[("gu_d", l)]
        bias = t[("bias", l)]
        out += [
            (b + "attn_norm.weight", GGML_F32, t[("attn_norm", l)]),
            (b + "attn_q.weight", GGML_Q8_0, (qq[:qd], qdd[:qd])),
            (b + "attn_k.weight", GGML_Q8_0, (qq[qd:qd + kd], qdd[qd:qd + kd])),
            (b + "attn_v.weight", GGML_Q8_0, (qq[qd + kd:], qdd[qd + kd:])),
            (b + "attn_q.bias", GGML_F32, bias[:qd]),
            (b + "attn_k.bias", GGML_F32, bias[qd:qd + kd]),
            (b + "attn_v.bias", GGML_F32, bias[qd + kd:]),
            (b + "attn_output.weight", GGML_Q8_0, (t[("o_q", l)], t[("o_d", l)])),
            (b + "ffn_norm.weight", GGML_F32, t[("ffn_norm", l)]),
            (b + "ffn_gate.weight", GGML_Q8_0, (gq[:I], gd[:I])),
            (b + "ffn_up.weight", GGML_Q8_0, (gq[I:], gd[I:])),
            (b + "ffn_down.weight", GGML_Q8_0, (t[("dn_q", l)], t[("dn_d", l)])),
        ]
    return out


def random_qwen2(cfg, seed, emb_q8=False):
    """Random tensors of a Qwen2 model (numpy PCG64): Q8_0 quants and scales,
    biases, norm weights in [0.5, 1.5), a binary16 embedding (or, emb_q8, a
    Q8_0 one as llama.cpp's Q8_0 files store token_embd)."""
    rng = np.random.default_rng(seed)
    H, I, d, V = cfg["hidden"], cfg["inter"], cfg["head_dim"], cfg["vocab"]
    qn = (cfg["n_heads"] + 2 * cfg["n_kv"]) * d

    def q8(n, k):
        qs = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        dd = (np.abs(rng.normal(0, 0.02, size=(n, k // 32))) / 127).astype(np.float16)
        return qs, dd.view(np.uint16)

    t = {"emb": rng.normal(0, 0.002, size=(V, H)).astype(np.float16).view(np.uint16),
         "out_norm": rng.uniform(0.5, 1.5, H).astype(np.float32)}
    if emb_q8:
        t["emb_q"], t["emb_d"] = q8(V, H)
    if not cfg["tied"]:
        t["lm_q"], t["lm_d"] = q8(V, H)
    for l in range(cfg["n_layers"]):
        t[("qkv_q", l)], t[("qkv_d", l)] = q8(qn, H)
        t[("o_q", l)], t[("o_d", l)] = q8(H, cfg["n_heads"] * d)
        t[("gu_q", l)], t[("gu_d", l)] = q8(2 * I, H)
        t[("dn_q", l)], t[("dn_d", l)] = q8(H, I)
        t[("bias", l)] = rng.normal(0, 0.02, qn).astype(np.float32)
        t[("attn_norm", l)] = rng.uniform(0.5, 1.5, H).astype(np.float32)
        t[("ffn_norm", l)] = rng.uniform(0.5, 1.5, H).astype(np.float32)
    return t


def load_into_oracle(om, cfg, t):
    """Set the oracle model's tensors to the dict `t` (random_qwen2 layout)."""
    om.set_tensor("emb", 0, t["emb"])
    if "emb_q" in t:
        om.set_emb_q8(t["emb_q"], t["emb_d"])
    om.set_tensor("out_norm", 0, t["out_norm"])
    if not cfg["tied"]:
        om.set_tensor("lm_q", 0, t["lm_q"])
        om.set_tensor("lm_d", 0, t["lm_d"])
    for l in range(cfg["n_layers"]):
        for name in ("qkv_q", "qkv_d", "o_q", "o_d", "gu_q", "gu_d", "dn_q", "dn_d", "bias",
                     "attn_norm", "ffn_norm"):
            om.set_tensor(name, l, t[(name, l)])
