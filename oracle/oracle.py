"""ctypes view of the CPU oracle (liblgx_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg, always as the checker.  The product package
``logicaffeine_amd`` never imports this module.

The arithmetic lives in ``lgx_oracle.c``; this file only marshals numpy arrays.
The reference (LOGOS 0.10.1) has no implementation of this path (no GPU
back-end, no tensor types), so each function is pinned by the checks listed in
``lgx_oracle.h`` rather than by reference vectors.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liblgx_oracle.so")
_lib = None

Q8_RANGE_BLOCKS = 32

_P = C.c_void_p
_I64 = C.c_int64
_I32 = C.c_int32
_U64 = C.c_uint64


def build() -> str:
    """Compile the oracle with its Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        sigs = {
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f32_to_f16_array": (None, [_P, _P, _I64]),
            "orc_f16_to_f32_array": (None, [_P, _P, _I64]),
            "orc_expf": (C.c_float, [C.c_float]),
            "orc_silu": (C.c_float, [C.c_float]),
            "orc_expf_array": (None, [_P, _P, _I64]),
            "orc_stream_base": (_U64, [_U64, _U64]),
            "orc_gen_u64": (None, [_U64, _U64, _P, _I64]),
            "orc_splitmix64_seq": (None, [_U64, _P, _I64]),
            "orc_gen_i8": (None, [_U64, _U64, _P, _I64]),
            "orc_gen_normal_f32": (None, [_U64, _U64, C.c_double, _P, _I64]),
            "orc_gen_normal_f16": (None, [_U64, _U64, C.c_double, _P, _I64]),
            "orc_gen_q8_scales": (None, [_U64, _U64, _P, _I64]),
            "orc_gen_below_i32": (None, [_U64, _U64, C.c_uint32, _P, _I64]),
            "orc_quantize_q8_0": (None, [_P, _I64, _I32, _P, _P]),
            "orc_q8_repack_t16": (None, [_P, _I32, _I32, _P]),
            "orc_q8_unpack_t16": (None, [_P, _I32, _I32, _P]),
            "orc_q8_s16_count": (_I64, [_I32, _I32]),
            "orc_q8_repack_s16": (None, [_P, _I32, _I32, _P]),
            "orc_q8_gemv_f32": (None, [_P, _P, _I32, _I32, _P, _P]),
            "orc_q8_blockdots": (None, [_P, _I32, _I32, _P, _P]),
            "orc_q8_gemm": (None, [_P, _P, _I32, _I32, _P, _P, _I32, _P]),
            "orc_tree_sum": (C.c_float, [_P, _I32]),
            "orc_halving_sum": (C.c_float, [_P, _I32]),
            "orc_gqa_decode_attn": (None, [_P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32,
                                           C.c_float, _P]),
            "orc_gen_page_table": (None, [_U64, _U64, _I32, _I32, _P]),
            "orc_rmsnorm": (None, [_P, _P, _I32, _I32, C.c_float, _P]),
            "orc_rope_tables": (None, [_I32, _I32, C.c_double, _P, _P]),
            "orc_rope": (None, [_P, _I32, _I32, _P, _P]),
            "orc_swiglu": (None, [_P, _I32, _I32, _P]),
            "orc_argmax": (_I32, [_P, _I32]),
            "orc_lm_head_f16": (None, [_P, _I32, _P, _I32, _I32, _P]),
            "orc_model_create": (_P, [_P, _U64]),
            "orc_model_destroy": (None, [_P]),
            "orc_model_seq_len": (_I32, [_P, _I32]),
            "orc_model_tensor": (_P, [_P, _I32, _I32]),
            "orc_model_kv": (None, [_P, _I32, _I32, _I32, _I32, _P]),
            "orc_model_step": (None, [_P, _I32, _P, _P, _P, _P, _P]),
            "orc_model_prefill": (None, [_P, _I32, _P, _I32, _P, _P, _P, _P]),
            "orc_model_load_kv": (None, [_P, _I32, _I32, _I32, _I32, _P]),
            "orc_model_set_seq_len": (None, [_P, _I32, _I32]),
            "orc_model_set_sampling": (None, [_P, C.c_float, _I32, C.c_float, C.c_uint64]),
            "orc_set_threads": (None, [_I32]),
            "orc_model_set_tensor": (None, [_P, _I32, _I32, _P]),
            "orc_model_set_emb_q8": (None, [_P, _P, _P]),
            "orc_max_threads": (_I32, []),
            "orc_sample": (None, [_P, _I32, _I32, _I32, C.c_float, C.c_float, C.c_uint64, _P,
                                  _P, _P]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- scalar formats -------------------------------------------------------

def f32_to_f16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


def expf(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.float32)
    lib().orc_expf_array(_ptr(x), _ptr(out), x.size)
    return out


def silu(x) -> np.ndarray:
    x = _c(x, np.float32).ravel()
    return np.array([lib().orc_silu(float(v)) for v in x], np.float32)


def tree_sum(p) -> np.float32:
    p = _c(p, np.float32).copy()
    return np.float32(lib().orc_tree_sum(_ptr(p), p.size))


# ---- generators -----------------------------------------------------------

def gen_u64(seed: int, stream: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint64)
    lib().orc_gen_u64(seed, stream, _ptr(out), n)
    return out


def splitmix64_seq(state: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint64)
    lib().orc_splitmix64_seq(state, _ptr(out), n)
    return out


def gen_i8(seed: int, stream: int, shape) -> np.ndarray:
    out = np.empty(shape, np.int8)
    lib().orc_gen_i8(seed, stream, _ptr(out), out.size)
    return out


def gen_normal_f32(seed: int, stream: int, shape, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(shape, np.float32)
    lib().orc_gen_normal_f32(seed, stream, sigma, _ptr(out), out.size)
    return out


def gen_normal_f16(seed: int, stream: int, shape, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(shape, np.uint16)
    lib().orc_gen_normal_f16(seed, stream, sigma, _ptr(out), out.size)
    return out


def gen_q8_scales(seed: int, stream: int, shape) -> np.ndarray:
    out = np.empty(shape, np.uint16)
    lib().orc_gen_q8_scales(seed, stream, _ptr(out), out.size)
    return out


def gen_below_i32(seed: int, stream: int, bound: int, shape) -> np.ndarray:
    out = np.empty(shape, np.int32)
    lib().orc_gen_below_i32(seed, stream, bound, _ptr(out), out.size)
    return out


def gen_q8_matrix(seed: int, stream: int, n: int, k: int):
    """Config-0 style weights: int8 U[-127,127] and d = |N(0,0.02)|/127 (f16)."""
    qs = gen_i8(seed, stream, (n, k))
    d = gen_q8_scales(seed, stream + 1, (n, k // 32))
    return qs, d


# ---- Q8_0 -----------------------------------------------------------------

def quantize_q8_0(x):
    x = _c(x, np.float32)
    m, k = x.shape
    qs = np.empty((m, k), np.int8)
    d = np.empty((m, k // 32), np.uint16)
    lib().orc_quantize_q8_0(_ptr(x), m, k, _ptr(qs), _ptr(d))
    return qs, d


def q8_repack_t16(qs):
    qs = _c(qs, np.int8)
    n, k = qs.shape
    out = np.empty(n * k, np.int8)
    lib().orc_q8_repack_t16(_ptr(qs), n, k, _ptr(out))
    return out


def q8_unpack_t16(t16, n: int, k: int):
    t16 = _c(t16, np.int8)
    out = np.empty((n, k), np.int8)
    lib().orc_q8_unpack_t16(_ptr(t16), n, k, _ptr(out))
    return out


def q8_repack_s16(d, n: int, k: int):
    d = _c(d, np.uint16)
    out = np.empty(lib().orc_q8_s16_count(n, k), np.uint16)
    lib().orc_q8_repack_s16(_ptr(d), n, k, _ptr(out))
    return out


def q8_gemv_f32(qs, d, x):
    qs = _c(qs, np.int8)
    d = _c(d, np.uint16)
    x = _c(x, np.float32)
    n, k = qs.shape
    y = np.empty(n, np.float32)
    lib().orc_q8_gemv_f32(_ptr(qs), _ptr(d), n, k, _ptr(x), _ptr(y))
    return y


def q8_blockdots(qs, xq):
    qs = _c(qs, np.int8)
    xq = _c(xq, np.int8)
    n, k = qs.shape
    s = np.empty((n, k // 32), np.int32)
    lib().orc_q8_blockdots(_ptr(qs), n, k, _ptr(xq), _ptr(s))
    return s


def q8_gemm(qs, d, xq, xd):
    """Y[m][n] with the canonical range/tree schedule."""
    qs = _c(qs, np.int8)
    d = _c(d, np.uint16)
    xq = _c(xq, np.int8)
    xd = _c(xd, np.uint16)
    n, k = qs.shape
    if xq.ndim == 1:
        xq = xq.reshape(1, k)
        xd = xd.reshape(1, k // 32)
    m = xq.shape[0]
    y = np.empty((m, n), np.float32)
    lib().orc_q8_gemm(_ptr(qs), _ptr(d), n, k, _ptr(xq), _ptr(xd), m, _ptr(y))
    return y


# ---- paged KV cache + attention --------------------------------------------

PAGE = 16
ATTN_CHUNK = 256


def attn_scale(d: int) -> np.float32:
    return np.float32(1.0 / np.sqrt(np.float64(d)))


def halving_sum(p) -> np.float32:
    p = _c(p, np.float32).copy()
    return np.float32(lib().orc_halving_sum(_ptr(p), p.size))


def gen_page_table(seed: int, stream: int, B: int, maxp: int) -> np.ndarray:
    out = np.empty((B, maxp), np.int32)
    lib().orc_gen_page_table(seed, stream, B, maxp, _ptr(out))
    return out


def gqa_decode_attn(q, kpages, vpages, page_table, seq_len, scale=None):
    """q [B][hq][d] f32; k/v pages [P][hkv][16][d] f16 bits; page_table [B][maxp]."""
    q = _c(q, np.float32)
    kpages = _c(kpages, np.uint16)
    vpages = _c(vpages, np.uint16)
    page_table = _c(page_table, np.int32)
    seq_len = _c(seq_len, np.int32)
    B, hq, d = q.shape
    hkv = kpages.shape[1]
    maxp = page_table.shape[1]
    scale = attn_scale(d) if scale is None else np.float32(scale)
    out = np.empty((B, hq, d), np.float32)
    lib().orc_gqa_decode_attn(_ptr(q), _ptr(kpages), _ptr(vpages), _ptr(page_table),
                              _ptr(seq_len), B, hq, hkv, d, maxp, float(scale), _ptr(out))
    return out


def paged_to_dense(pages, page_table, b, L):
    """[L][hkv][d] view of sequence b's cached rows (test helper)."""
    rows = [pages[page_table[b, t // PAGE], :, t % PAGE, :] for t in range(L)]
    return np.stack(rows) if rows else np.zeros((0,) + pages.shape[1:2] + pages.shape[3:], pages.dtype)


# ---- decode-step glue -------------------------------------------------------

def rmsnorm(x, w=None, eps=1e-6):
    x = _c(x, np.float32)
    m, h = x.shape
    w = np.ones(h, np.float32) if w is None else _c(w, np.float32)
    y = np.empty_like(x)
    lib().orc_rmsnorm(_ptr(x), _ptr(w), m, h, eps, _ptr(y))
    return y


def rope_tables(max_seq: int, d: int, theta: float = 1e6):
    c = np.empty((max_seq, d // 2), np.float32)
    s = np.empty((max_seq, d // 2), np.float32)
    lib().orc_rope_tables(max_seq, d, theta, _ptr(c), _ptr(s))
    return c, s


def rope(x, cos_row, sin_row):
    """x [nheads][d] rotated in a copy."""
    x = _c(x, np.float32).copy()
    nh, d = x.shape
    cr, sr = _c(cos_row, np.float32), _c(sin_row, np.float32)
    lib().orc_rope(_ptr(x), nh, d, _ptr(cr), _ptr(sr))
    return x


def swiglu(gu):
    gu = _c(gu, np.float32)
    m, n2 = gu.shape
    a = np.empty((m, n2 // 2), np.float32)
    lib().orc_swiglu(_ptr(gu), m, n2 // 2, _ptr(a))
    return a


def argmax(x) -> int:
    x = _c(x, np.float32)
    return int(lib().orc_argmax(_ptr(x), x.size))


def lm_head_f16(x, E):
    x = _c(x, np.float32)
    E = _c(E, np.uint16)
    m, h = x.shape
    V = E.shape[0]
    out = np.empty((m, V), np.float32)
    lib().orc_lm_head_f16(_ptr(x), m, _ptr(E), V, h, _ptr(out))
    return out


def set_threads(n: int) -> None:
    """OpenMP threads of later oracle calls."""
    lib().orc_set_threads(n)


def max_threads() -> int:
    return int(lib().orc_max_threads())


def sample(logits, top_k: int, top_p: float, temperature: float, seed: int, streams, pos):
    """Seeded top-k / top-p draw per row of logits [m][vocab] (the rule of
    lgx_sample); row i uses SplitMix64 stream streams[i] at index pos[i]."""
    logits = _c(logits, np.float32)
    m, vocab = logits.shape
    streams = _c(np.broadcast_to(np.asarray(streams, np.int32), (m,)), np.int32)
    pos = _c(np.broadcast_to(np.asarray(pos, np.int32), (m,)), np.int32)
    out = np.empty(m, np.int32)
    lib().orc_sample(_ptr(logits), m, vocab, top_k, top_p, temperature, seed, _ptr(streams),
                     _ptr(pos), _ptr(out))
    return out


# ---- random-init Qwen2-shaped model ------------------------------------------

class QwenConfigC(C.Structure):
    _fields_ = [("n_layers", _I32), ("hidden", _I32), ("inter", _I32), ("n_heads", _I32),
                ("n_kv", _I32), ("head_dim", _I32), ("vocab", _I32), ("tied", _I32),
                ("max_batch", _I32), ("max_seq", _I32), ("eps", C.c_float),
                ("theta", C.c_double), ("emb_sigma", C.c_double)]


TENSORS = {"emb": 0, "lm_q": 1, "lm_d": 2, "qkv_q": 3, "qkv_d": 4, "o_q": 5, "o_d": 6,
           "gu_q": 7, "gu_d": 8, "dn_q": 9, "dn_d": 10, "bias": 11, "attn_norm": 12,
           "ffn_norm": 13, "out_norm": 14}


class Model:
    """The oracle's random-init Qwen2-shaped Q8_0 model (C implementation)."""

    def __init__(self, cfg: dict, seed: int):
        self.cfg = dict(cfg)
        self.c = QwenConfigC(**{k: cfg[k] for k, _ in QwenConfigC._fields_})
        self.h = lib().orc_model_create(C.byref(self.c), seed)

    def close(self):
        if self.h:
            lib().orc_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def seq_len(self, slot: int) -> int:
        return int(lib().orc_model_seq_len(self.h, slot))

    def tensor(self, name: str, layer: int = 0) -> np.ndarray:
        c = self.cfg
        H, I, d = c["hidden"], c["inter"], c["head_dim"]
        qn = (c["n_heads"] + 2 * c["n_kv"]) * d
        shapes = {"emb": ((c["vocab"], H), np.uint16), "lm_q": ((c["vocab"], H), np.int8),
                  "lm_d": ((c["vocab"], H // 32), np.uint16), "qkv_q": ((qn, H), np.int8),
                  "qkv_d": ((qn, H // 32), np.uint16), "o_q": ((H, c["n_heads"] * d), np.int8),
                  "o_d": ((H, c["n_heads"] * d // 32), np.uint16), "gu_q": ((2 * I, H), np.int8),
                  "gu_d": ((2 * I, H // 32), np.uint16), "dn_q": ((H, I), np.int8),
                  "dn_d": ((H, I // 32), np.uint16), "bias": ((qn,), np.float32)}
        shape, dt = shapes[name]
        ptr = lib().orc_model_tensor(self.h, layer, TENSORS[name])
        n = int(np.prod(shape)) * np.dtype(dt).itemsize
        return np.frombuffer(C.string_at(ptr, n), dtype=dt).reshape(shape).copy()

    def set_tensor(self, name: str, layer: int, data) -> None:
        """Replace a tensor (the shapes and dtypes of tensor()) -- e.g. a
        checkpoint's weights."""
        want = self.tensor(name, layer) if name in self._shaped() else None
        arr = np.ascontiguousarray(data)
        if want is not None:
            assert arr.shape == want.shape and arr.dtype == want.dtype, (name, arr.shape, arr.dtype)
        lib().orc_model_set_tensor(self.h, layer, TENSORS[name], arr.ctypes.data_as(C.c_void_p))

    def set_emb_q8(self, qs, d) -> None:
        """A Q8_0 embedding (row-major quants [vocab][hidden] int8, scales
        [vocab][hidden/32] binary16 bits): gathered as f32(d) * q, and the
        tied lm_head becomes the Q8 product with it."""
        c = self.cfg
        qs = _c(qs, np.int8)
        d = _c(d, np.uint16)
        assert qs.shape == (c["vocab"], c["hidden"]) and d.shape == (c["vocab"], c["hidden"] // 32)
        lib().orc_model_set_emb_q8(self.h, _ptr(qs), _ptr(d))

    @staticmethod
    def _shaped():
        return ("emb", "lm_q", "lm_d", "qkv_q", "qkv_d", "o_q", "o_d", "gu_q", "gu_d", "dn_q",
                "dn_d", "bias")

    def kv(self, layer: int, which: int, slot: int, n: int) -> np.ndarray:
        c = self.cfg
        out = np.empty((n, c["n_kv"], c["head_dim"]), np.uint16)
        lib().orc_model_kv(self.h, layer, which, slot, n, _ptr(out))
        return out

    def step(self, slots, tokens, want_logits=False, want_hidden=False):
        slots = _c(slots, np.int32)
        tokens = _c(tokens, np.int32)
        B = slots.size
        nxt = np.empty(B, np.int32)
        hid = np.empty((B, self.cfg["hidden"]), np.float32) if want_hidden else None
        lg = np.empty((B, self.cfg["vocab"]), np.float32) if want_logits else None
        lib().orc_model_step(self.h, B, _ptr(slots), _ptr(tokens), _ptr(nxt),
                             _ptr(hid) if hid is not None else None,
                             _ptr(lg) if lg is not None else None)
        out = [nxt]
        if want_logits:
            out.append(lg)
        if want_hidden:
            out.append(hid)
        return out[0] if len(out) == 1 else tuple(out)

    def prefill(self, slots, tokens, want_logits=False, want_hidden=False):
        """Teacher-forced prefill: tokens [nseq][P] for `slots`, all P
        positions of every slot per layer in one batched pass; returns what
        the P-th step call would (next tokens, logits, hidden rows)."""
        slots = _c(slots, np.int32)
        tokens = _c(tokens, np.int32)
        nseq, P = tokens.shape
        assert slots.size == nseq
        nxt = np.empty(nseq, np.int32)
        hid = np.empty((nseq, self.cfg["hidden"]), np.float32) if want_hidden else None
        lg = np.empty((nseq, self.cfg["vocab"]), np.float32) if want_logits else None
        lib().orc_model_prefill(self.h, nseq, _ptr(slots), P, _ptr(tokens), _ptr(nxt),
                                _ptr(hid) if hid is not None else None,
                                _ptr(lg) if lg is not None else None)
        out = [nxt]
        if want_logits:
            out.append(lg)
        if want_hidden:
            out.append(hid)
        return out[0] if len(out) == 1 else tuple(out)

    def load_kv(self, layer: int, which: int, slot: int, rows) -> None:
        """Write cached K (which 0) or V (1) rows [n][n_kv][head_dim] binary16
        of `slot`, tokens 0..n-1 (the inverse of kv())."""
        rows = _c(rows, np.uint16)
        lib().orc_model_load_kv(self.h, layer, which, slot, rows.shape[0], _ptr(rows))

    def set_seq_len(self, slot: int, n: int) -> None:
        lib().orc_model_set_seq_len(self.h, slot, n)

    def set_sampling(self, temperature: float, top_k: int = 1, top_p: float = 1.0,
                     seed: int = 0) -> None:
        """Seeded top-k / top-p token choice (temperature 0: greedy); stream =
        slot, draw index = the consumed position."""
        lib().orc_model_set_sampling(self.h, temperature, top_k, top_p, seed)


EMB_SIGMA = 0.002


def qwen_config(name: str) -> dict:
    """Shapes of BASELINE configs 3 and 4 and a tiny test model."""
    base = dict(eps=1e-6, theta=1e6, emb_sigma=EMB_SIGMA)
    if name == "0.5b":
        return dict(base, n_layers=24, hidden=896, inter=4864, n_heads=14, n_kv=2, head_dim=64,
                    vocab=151936, tied=1, max_batch=32, max_seq=2048 + 64)
    if name == "7b":
        return dict(base, n_layers=28, hidden=3584, inter=18944, n_heads=28, n_kv=4,
                    head_dim=128, vocab=152064, tied=0, max_batch=64, max_seq=4096 + 64)
    if name == "tiny":
        return dict(base, n_layers=2, hidden=256, inter=512, n_heads=4, n_kv=2, head_dim=64,
                    vocab=1000, tied=1, max_batch=4, max_seq=320)
    if name == "tiny_untied":
        return dict(base, n_layers=2, hidden=256, inter=512, n_heads=4, n_kv=1, head_dim=128,
                    vocab=1024, tied=0, max_batch=4, max_seq=320)
    raise KeyError(name)
