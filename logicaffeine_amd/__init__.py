"""logicaffeine_amd -- Python view of liblgx, the MI355X back-end of the Q8
LLM-decode hot path.

Every compute call goes through the C ABI in ``include/lgx.h`` (liblgx.so ->
hipModuleLaunchKernel on lgx_kernels.hsaco).  There is no CPU or PyTorch
fallback: if the library or its code object is missing, :class:`Context`
raises.  torch is used only for device memory and the current stream.

The loader mirrors the reference's AOT tier (load a built module, resolve its
``extern "C"`` symbols, keep it alive, count calls;
crates/logicaffeine_compile/src/vm/aot_tier.rs:86-111), and errors surface as
:class:`LgxError` carrying the ``lgx_status`` and ``lgx_last_error()`` text
(crates/logicaffeine_compile/src/codegen/ffi.rs:196-258).
"""
from __future__ import annotations

import ctypes as C
import os
import weakref

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblgx.so")
HSACO_PATH = os.path.join(HERE, "lgx_kernels.hsaco")

Q8_ROWMAJOR = 0
Q8_T16 = 1
Q8_RANGE_BLOCKS = 32

STATUS_NAMES = {
    0: "LGX_OK", 1: "LGX_ERROR", 2: "LGX_INVALID_ARGUMENT", 3: "LGX_NULL_POINTER",
    4: "LGX_OUT_OF_BOUNDS", 5: "LGX_MODULE_LOAD_FAILED", 6: "LGX_INVALID_HANDLE",
    8: "LGX_INTERNAL_PANIC", 9: "LGX_OUT_OF_MEMORY", 10: "LGX_HIP_ERROR",
    11: "LGX_NO_DEVICE", 12: "LGX_UNSUPPORTED",
}

# Exported symbols and their C signatures (include/lgx.h).
_P = C.c_void_p
_I32 = C.c_int32
SIGNATURES = {
    "lgx_abi_version": (C.c_uint32, []),
    "lgx_version": (C.c_char_p, []),
    "lgx_last_error": (C.c_char_p, []),
    "lgx_clear_error": (None, []),
    "lgx_ctx_create": (C.c_int, [_I32, C.c_char_p, C.POINTER(_P)]),
    "lgx_ctx_destroy": (C.c_int, [_P]),
    "lgx_ctx_launch_count": (C.c_uint64, [_P]),
    "lgx_ctx_arch": (C.c_char_p, [_P]),
    "lgx_ctx_set_kernel_timing": (C.c_int, [_P, _I32]),
    "lgx_ctx_kernel_stats": (C.c_int, [_P, C.c_char_p, C.POINTER(C.c_uint64),
                                       C.POINTER(C.c_double)]),
    "lgx_q8_scale_count": (C.c_size_t, [_I32, _I32]),
    "lgx_q8_repack_t16": (C.c_int, [_P, _P, _P, _I32, _I32, _P, _P, _P]),
    "lgx_q8_unpack_t16": (C.c_int, [_P, _P, _P, _I32, _I32, _P, _P, _P]),
    "lgx_quantize_q8_0": (C.c_int, [_P, _P, _I32, _I32, _P, _P, _P]),
    "lgx_q8_gemv_f32": (C.c_int, [_P, _P, _P, _P, _P]),
    "lgx_q8q8_gemv": (C.c_int, [_P, _P, _P, _P, _P, _P, _P]),
    "lgx_q8_gemm": (C.c_int, [_P, _P, _P, _P, _I32, _P, _P]),
    "lgx_q8_gemm_noalloc": (C.c_int, [_P, _P, _P, _P, _I32, _P, _P]),
    "lgx_q8q8_gemv_quantize": (C.c_int, [_P, _P, _P, _P, _P, _P, _P]),
    "lgx_q8q8_gemv_quantize_group": (C.c_int, [_P, _I32, _P, _P, _P, _P]),
    "lgx_q8_gemm_quantize_group": (C.c_int, [_P, _I32, _P, _P, _I32, _P, _P]),
    "lgx_q8_range_count": (_I32, [_I32]),
    "lgx_q8q8_gemv_quantize_partials": (C.c_int, [_P, _P, _P, _P, _P, _P, _P]),
    "lgx_q8_gemm_partials": (C.c_int, [_P, _P, _P, _P, _I32, _P, _P]),
    "lgx_q8_range_combine": (C.c_int, [_P, _P, _I32, C.c_int64, _P, _P]),
    "lgx_gqa_decode_attn": (C.c_int, [_P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32,
                                      _I32, _I32, _P, _P]),
    "lgx_gqa_prefill_attn": (C.c_int, [_P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32,
                                       _I32, _I32, _I32, _P, _P]),
    "lgx_gqa_prefill_attn_fast": (C.c_int, [_P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32,
                                            _I32, _I32, _I32, _I32, _P, _P]),
    "lgx_embed_f16": (C.c_int, [_P, _P, _P, _I32, _I32, _I32, _P, _P]),
    "lgx_rmsnorm_quant": (C.c_int, [_P, _P, _P, _I32, _I32, C.c_float, _P, _P, _P, _P]),
    "lgx_add_rmsnorm_quant": (C.c_int, [_P, _P, _I32, _P, _P, _I32, _I32, C.c_float, _P, _P, _P,
                                        _P]),
    "lgx_rope_kv_append": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32,
                                     _I32, _I32, _I32, _I32, _P]),
    "lgx_swiglu_quant": (C.c_int, [_P, _P, _I32, _I32, _P, _P, _P, _P]),
    "lgx_lm_head_f16": (C.c_int, [_P, _P, _P, _I32, _I32, _I32, _P, _P]),
    "lgx_f16_t64_count": (C.c_int64, [_I32, _I32]),
    "lgx_f16_repack_t64": (C.c_int, [_P, _P, _I32, _I32, _P, _P]),
    "lgx_lm_head_f16_t64": (C.c_int, [_P, _P, _P, _I32, _I32, _I32, _P, _P]),
    "lgx_lm_head_rowconst": (C.c_int, [_P, _P, _I32, _I32, _P, _P]),
    "lgx_lm_head_argmax_f16": (C.c_int, [_P, _P, _P, _P, _P, _I32, _I32, _I32, _P, _P, _P]),
    "lgx_argmax": (C.c_int, [_P, _P, _I32, _I32, _P, _P]),
    "lgx_sample": (C.c_int, [_P, _P, _I32, _I32, _I32, C.c_float, C.c_float, C.c_uint64, _P, _P,
                             _P]),
    "lgx_model_set_sampling": (C.c_int, [_P, C.c_float, _I32, C.c_float, C.c_uint64]),
    "lgx_model_set_prefill_mode": (C.c_int, [_P, _I32]),
    "lgx_model_create": (C.c_int, [_P, _P, C.c_uint64, C.POINTER(_P)]),
    "lgx_gguf_config": (C.c_int, [C.c_char_p, _I32, _I32, _P]),
    "lgx_model_load_gguf": (C.c_int, [_P, C.c_char_p, _I32, _I32, C.POINTER(_P)]),
    "lgx_model_config": (C.c_int, [_P, _P]),
    "lgx_model_destroy": (C.c_int, [_P]),
    "lgx_model_reset": (C.c_int, [_P, _P]),
    "lgx_qwen_decode_step": (C.c_int, [_P, _I32, _P, _P]),
    "lgx_qwen_prefill": (C.c_int, [_P, _I32, _I32, _P, _P, _P]),
    "lgx_qwen_generate": (C.c_int, [_P, _I32, _P, _I32, _P, _P]),
    "lgx_model_tensor": (C.c_int, [_P, _I32, _I32, C.POINTER(_P), C.POINTER(C.c_size_t)]),
    "lgx_qwen_logits": (C.c_int, [_P, _I32, _P, _P]),
}

# Model shapes of the decode benchmarks (random-init Qwen2.5-0.5B / -7B shaped
# Q8_0 models): keys as lgx.Model's cfg.
QWEN_SHAPES = {
    "0.5b": dict(n_layers=24, hidden=896, inter=4864, n_heads=14, n_kv=2, head_dim=64,
                 vocab=151936, tied=1),
    "7b": dict(n_layers=28, hidden=3584, inter=18944, n_heads=28, n_kv=4, head_dim=128,
               vocab=152064, tied=0),
}


def qwen_shape(name: str, max_batch: int, max_seq: int, emb_sigma: float = 0.002) -> dict:
    """cfg dict for lgx.Model: shape `name` with RMSNorm eps 1e-6, RoPE theta 1e6."""
    return dict(QWEN_SHAPES[name], max_batch=max_batch, max_seq=max_seq, eps=1e-6, theta=1e6,
                emb_sigma=emb_sigma)


def decode_step_bytes(cfg: dict, B: int, context: float) -> float:
    """Algorithmic HBM bytes of one greedy decode step of B sequences whose
    attention spans `context` cached tokens on average (the new token
    included): Q8_0 weights (1.0625 B/weight), the lm_head (binary16 tied
    embedding or Q8_0), the K/V cache read and the new K/V rows written."""
    H, I, d = cfg["hidden"], cfg["inter"], cfg["head_dim"]
    hq, hkv, L, V = cfg["n_heads"], cfg["n_kv"], cfg["n_layers"], cfg["vocab"]
    per_layer = ((hq + 2 * hkv) * d * H + H * hq * d + 2 * I * H + H * I) * 1.0625
    lm = V * H * (2.0 if cfg["tied"] else 1.0625)
    kv_row = L * hkv * d * 2 * 2                    # K and V, binary16, all layers
    return L * per_layer + lm + B * context * kv_row + B * kv_row


# Non-packed binary32 VALU lane operations per second of MI355X: 256 CUs x 4
# SIMDs x 16 lanes x 2.4 GHz (the published 157.3 TFLOP/s counts an FMA as
# two flops and packed FP32, which this build does not use).
VALU_LANE_OPS_PEAK = 256 * 4 * 16 * 2.4e9


def prefill_int8_ops(cfg: dict, B: int, P: int) -> float:
    """int8 MFMA operations (2 per multiply-add) of the Q8_0 products of the
    prefill of B prompts of P tokens: rows B x (P - 1) through the batched
    chunks (the last layer of a chunk runs its QKV product only), the last
    position of every prompt through the decode step, and the untied lm_head
    for those B rows (the tied lm_head is a binary16 VALU chain)."""
    H, I, d = cfg["hidden"], cfg["inter"], cfg["head_dim"]
    hq, hkv, L, V = cfg["n_heads"], cfg["n_kv"], cfg["n_layers"], cfg["vocab"]
    qkv = (hq + 2 * hkv) * d * H
    full = qkv + H * hq * d + 2 * I * H + H * I
    rows = B * (P - 1)
    macs = rows * ((L - 1) * full + qkv) + B * L * full
    if not cfg["tied"]:
        macs += B * V * H
    return 2.0 * macs


def prefill_fast_flops(cfg: dict, B: int, P: int) -> tuple:
    """MFMA work of the fast prefill of B prompts of P tokens: (binary16
    flops, int8 operations).  binary16: the GEMMs of the batched rows
    B x (P - 1) (2 per multiply-add; the last layer of a chunk runs its qkv
    GEMM only) and the causal attention of layers 0 .. L - 2 (2 d per query
    head and attended token for the scores, 2 d for PV; the row at position
    p attends p + 1 tokens).  int8: the last position of every prompt
    through the exact decode step (and the untied Q8_0 lm_head)."""
    H, I, d = cfg["hidden"], cfg["inter"], cfg["head_dim"]
    hq, hkv, L, V = cfg["n_heads"], cfg["n_kv"], cfg["n_layers"], cfg["vocab"]
    qkv = (hq + 2 * hkv) * d * H
    full = qkv + H * hq * d + 2 * I * H + H * I
    rows = B * (P - 1)
    gemm = 2.0 * rows * ((L - 1) * full + qkv)
    att_rows = B * (P - 1) * P / 2.0
    attn = 4.0 * d * hq * att_rows * (L - 1)
    int8 = 2.0 * B * (L * full + (0 if cfg["tied"] else V * H))
    return gemm + attn, int8


def prefill_valu_ops(cfg: dict, B: int, P: int) -> float:
    """Essential VALU lane operations of the canonical prefill of B prompts of
    P tokens (rows B x (P - 1) through the batched chunks, the last position
    through the decode step): 2 per (row, output, 32-block) of every Q8_0
    product (cvt of the int32 block dot, chain FMA; the scale products come
    from a rank-1 f16 MFMA) and 1 per attention FMA (score chain over d and PV
    chain over the attended tokens, per query head).  The last layer of a
    batched chunk stops after its KV append (QKV product only)."""
    H, I, d = cfg["hidden"], cfg["inter"], cfg["head_dim"]
    hq, hkv, L, V = cfg["n_heads"], cfg["n_kv"], cfg["n_layers"], cfg["vocab"]
    qkv = (hq + 2 * hkv) * d * H / 32
    full = qkv + (H * hq * d + 2 * I * H + H * I) / 32
    rows = B * (P - 1)
    gemm = 2.0 * (rows * ((L - 1) * full + qkv) + B * L * full)
    gemm += B * V * H * (1.0 if cfg["tied"] else 3.0 / 32)
    # attention: row at position p attends p + 1 tokens (2d FMAs per head each)
    att_rows = B * (P - 1) * P / 2.0            # sum over p < P - 1 of (p + 1)
    attn = 2.0 * d * hq * (att_rows * (L - 1) + B * P * L)
    return gemm + attn


# Tensor ids of lgx_model_tensor.
MODEL_TENSORS = {"emb": 0, "lm_q": 1, "lm_d": 2, "qkv_q": 3, "qkv_d": 4, "o_q": 5, "o_d": 6,
                 "gu_q": 7, "gu_d": 8, "dn_q": 9, "dn_d": 10, "bias": 11, "k_pages": 12,
                 "v_pages": 13, "page_table": 14, "seq_len": 15, "hidden": 16,
                 "attn_norm": 17, "ffn_norm": 18, "out_norm": 19, "emb_q": 20, "emb_d": 21}


class LgxError(RuntimeError):
    def __init__(self, status: int, message: str):
        self.status = status
        self.status_name = STATUS_NAMES.get(status, str(status))
        super().__init__(f"{self.status_name}: {message}")


class Q8MatrixC(C.Structure):
    _fields_ = [("qs", _P), ("d", _P), ("n", _I32), ("k", _I32), ("layout", _I32)]


class QwenConfigC(C.Structure):
    """lgx_qwen_config."""
    _fields_ = [("n_layers", _I32), ("hidden", _I32), ("intermediate", _I32),
                ("n_heads", _I32), ("n_kv_heads", _I32), ("head_dim", _I32), ("vocab", _I32),
                ("tied_embedding", _I32), ("max_batch", _I32), ("max_seq", _I32),
                ("rms_eps", C.c_float), ("rope_theta", C.c_double), ("emb_sigma", C.c_double)]


_lib = None


def lib() -> C.CDLL:
    """Load liblgx.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m logicaffeine_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(status: int) -> None:
    if status != 0:
        msg = lib().lgx_last_error()
        raise LgxError(status, msg.decode(errors="replace") if msg else "(no message)")


def _stream(torch, device):
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


class Q8Matrix:
    """A Q8_0 weight matrix resident on the device in the tile layouts.

    ``qs`` is an int8 device tensor (T16 order, n*k bytes); ``d`` an int16
    device tensor holding the binary16 scale bits in S16 order
    (lgx_q8_scale_count(n, k) elements)."""

    def __init__(self, qs, d, n: int, k: int):
        self.qs, self.d, self.n, self.k = qs, d, n, k
        self._c = Q8MatrixC(qs.data_ptr(), d.data_ptr(), n, k, Q8_T16)

    @property
    def cstruct(self):
        return C.byref(self._c)

    @property
    def nbytes(self) -> int:
        return self.qs.numel() + 2 * self.d.numel()


class Context:
    """One lgx_ctx: the loaded code object on one device."""

    def __init__(self, device: int = 0, hsaco: str | None = None):
        import torch

        self.torch = torch
        self.device = device
        self.dev = torch.device("cuda", device)
        h = C.c_void_p()
        _check(lib().lgx_ctx_create(device, hsaco.encode() if hsaco else None, C.byref(h)))
        self.handle = h
        self._models = weakref.WeakSet()   # live Models built on this ctx

    def close(self) -> None:
        """Destroy the ctx; Models still open on it are closed first
        (lgx_ctx_destroy refuses a ctx that live models still use)."""
        if self.handle:
            for m in list(self._models):
                m.close()
            _check(lib().lgx_ctx_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def launch_count(self) -> int:
        return int(lib().lgx_ctx_launch_count(self.handle))

    @property
    def arch(self) -> str:
        return lib().lgx_ctx_arch(self.handle).decode()

    def _s(self):
        return _stream(self.torch, self.dev)

    def kernel_timing(self, enable: bool) -> None:
        """Time every launch by its own dispatch (fresh window when enabled)."""
        _check(lib().lgx_ctx_set_kernel_timing(self.handle, 1 if enable else 0))

    def kernel_stats(self, kernel_name: str):
        """(launch count, total ms) of `kernel_name` in the timing window."""
        n, ms = C.c_uint64(), C.c_double()
        _check(lib().lgx_ctx_kernel_stats(self.handle, kernel_name.encode(), C.byref(n),
                                          C.byref(ms)))
        return int(n.value), float(ms.value)

    # ---- layout ----------------------------------------------------------
    def repack_t16(self, qs_rowmajor, d_rowmajor):
        """Row-major quants [n][k] + scales [n][k/32] -> (T16 quants, S16 scales)."""
        t = self.torch
        n, k = qs_rowmajor.shape
        out = t.empty(n * k, dtype=t.int8, device=self.dev)
        dout = t.empty(max(1, lib().lgx_q8_scale_count(n, k)), dtype=t.int16, device=self.dev)
        _check(lib().lgx_q8_repack_t16(self.handle, qs_rowmajor.data_ptr(), d_rowmajor.data_ptr(),
                                       n, k, out.data_ptr(), dout.data_ptr(), self._s()))
        return out, dout

    def unpack_t16(self, qs_t16, d_s16, n: int, k: int):
        t = self.torch
        out = t.empty((n, k), dtype=t.int8, device=self.dev)
        dout = t.empty((n, k // 32), dtype=t.int16, device=self.dev)
        _check(lib().lgx_q8_unpack_t16(self.handle, qs_t16.data_ptr(), d_s16.data_ptr(), n, k,
                                       out.data_ptr(), dout.data_ptr(), self._s()))
        return out, dout

    def to_device(self, a, dtype=None):
        """numpy array or tensor -> contiguous device tensor (uint16 data is
        carried as int16 bit patterns)."""
        t = self.torch
        if not isinstance(a, t.Tensor):
            import numpy as np

            a = np.ascontiguousarray(a)
            if a.dtype == np.uint16:
                a = a.view(np.int16)
            a = t.from_numpy(a)
        elif a.dtype == t.uint16:
            a = a.view(t.int16)
        if dtype is not None and a.dtype != dtype:
            a = a.to(dtype)
        return a.to(self.dev).contiguous()

    def q8_matrix(self, qs_rowmajor, d) -> Q8Matrix:
        """Upload (if host) and repack row-major quants + binary16 scale bits."""
        t = self.torch
        qs = self.to_device(qs_rowmajor, t.int8)
        dd = self.to_device(d, t.int16)
        n, k = qs.shape
        qt, ds = self.repack_t16(qs, dd)
        return Q8Matrix(qt, ds, n, k)

    # ---- Q8_0 ------------------------------------------------------------
    def quantize_q8_0(self, x, qs=None, d=None):
        t = self.torch
        m, k = x.shape
        qs = t.empty((m, k), dtype=t.int8, device=self.dev) if qs is None else qs
        d = t.empty((m, k // 32), dtype=t.int16, device=self.dev) if d is None else d
        _check(lib().lgx_quantize_q8_0(self.handle, x.data_ptr(), m, k, qs.data_ptr(),
                                       d.data_ptr(), self._s()))
        return qs, d

    def q8_gemv_f32(self, W: Q8Matrix, x, y=None):
        y = self.torch.empty(W.n, dtype=self.torch.float32, device=self.dev) if y is None else y
        _check(lib().lgx_q8_gemv_f32(self.handle, W.cstruct, x.data_ptr(), y.data_ptr(),
                                     self._s()))
        return y

    def q8q8_gemv(self, W: Q8Matrix, xq, xd, y=None, blockdots: bool = False):
        t = self.torch
        y = t.empty(W.n, dtype=t.float32, device=self.dev) if y is None else y
        dbg = t.empty((W.n, W.k // 32), dtype=t.int32, device=self.dev) if blockdots else None
        _check(lib().lgx_q8q8_gemv(self.handle, W.cstruct, xq.data_ptr(), xd.data_ptr(),
                                   y.data_ptr(), dbg.data_ptr() if dbg is not None else None,
                                   self._s()))
        return (y, dbg) if blockdots else y

    def q8q8_gemv_quantize(self, W: Q8Matrix, x, y=None, xq_out=None, xd_out=None):
        """y = W Q8_0(x) with the quantisation fused into the GEMV."""
        t = self.torch
        y = t.empty(W.n, dtype=t.float32, device=self.dev) if y is None else y
        _check(lib().lgx_q8q8_gemv_quantize(
            self.handle, W.cstruct, x.data_ptr(), y.data_ptr(),
            xq_out.data_ptr() if xq_out is not None else None,
            xd_out.data_ptr() if xd_out is not None else None, self._s()))
        return y

    def q8q8_gemv_quantize_group(self, Ws, xs, ys=None):
        """ys[i] = Ws[i] Q8_0(xs[i]) for up to 8 matrices in one launch."""
        t = self.torch
        n = len(Ws)
        ys = [t.empty(W.n, dtype=t.float32, device=self.dev) for W in Ws] if ys is None else ys
        arr = (Q8MatrixC * n)(*[W._c for W in Ws])
        xp = (C.c_void_p * n)(*[x.data_ptr() for x in xs])
        yp = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
        _check(lib().lgx_q8q8_gemv_quantize_group(self.handle, n, arr, xp, yp, self._s()))
        return ys

    def q8_gemm_quantize_group(self, Ws, xs, ys=None):
        """ys[i] = Q8_0(xs[i]) Ws[i]^T for up to 8 matrices (xs[i]: [m][k_i]
        binary32, the same m for all) in three launches."""
        t = self.torch
        n = len(Ws)
        m = xs[0].shape[0] if xs[0].dim() == 2 else 1
        for x, W in zip(xs, Ws):
            if (x.shape[0] if x.dim() == 2 else 1) != m or x.shape[-1] != W.k or not x.is_contiguous():
                raise ValueError("every x must be a contiguous [m][k] of its matrix")
        ys = [t.empty((m, W.n), dtype=t.float32, device=self.dev) for W in Ws] if ys is None else ys
        arr = (Q8MatrixC * n)(*[W._c for W in Ws])
        xp = (C.c_void_p * n)(*[x.data_ptr() for x in xs])
        yp = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
        _check(lib().lgx_q8_gemm_quantize_group(self.handle, n, arr, xp, m, yp, self._s()))
        return ys

    def q8q8_gemv_quantize_partials(self, W: Q8Matrix, x, part=None):
        t = self.torch
        g = lib().lgx_q8_range_count(W.k)
        part = t.empty((g, W.n), dtype=t.float32, device=self.dev) if part is None else part
        _check(lib().lgx_q8q8_gemv_quantize_partials(self.handle, W.cstruct, x.data_ptr(),
                                                     part.data_ptr(), None, None, self._s()))
        return part

    def q8_gemm_partials(self, W: Q8Matrix, xq, xd, part=None):
        t = self.torch
        m = xq.shape[0] if xq.dim() == 2 else 1
        g = lib().lgx_q8_range_count(W.k)
        part = t.empty((g, m, W.n), dtype=t.float32, device=self.dev) if part is None else part
        _check(lib().lgx_q8_gemm_partials(self.handle, W.cstruct, xq.data_ptr(), xd.data_ptr(), m,
                                          part.data_ptr(), self._s()))
        return part

    def range_combine(self, part, y=None):
        t = self.torch
        g = part.shape[0]
        count = part[0].numel()
        y = t.empty(part.shape[1:], dtype=t.float32, device=self.dev) if y is None else y
        _check(lib().lgx_q8_range_combine(self.handle, part.data_ptr(), g, count, y.data_ptr(),
                                          self._s()))
        return y

    def gqa_decode_attn(self, q, kpages, vpages, page_table, seq_len, max_seq_len: int,
                        out=None):
        """q [B][hq][d] f32; pages [P][hkv][16][d] (int16 bit patterns of binary16)."""
        t = self.torch
        B, hq, d = q.shape
        num_pages, hkv = kpages.shape[0], kpages.shape[1]
        maxp = page_table.shape[1]
        out = t.empty((B, hq, d), dtype=t.float32, device=self.dev) if out is None else out
        _check(lib().lgx_gqa_decode_attn(self.handle, q.data_ptr(), kpages.data_ptr(),
                                         vpages.data_ptr(), page_table.data_ptr(),
                                         seq_len.data_ptr(), B, hq, hkv, d, maxp, num_pages,
                                         max_seq_len, out.data_ptr(), self._s()))
        return out

    def gqa_prefill_attn(self, q, kpages, vpages, page_table, seq_len, P: int, max_seq_len: int,
                         out=None, fast: bool = False):
        """q [B*P][hq][d] f32: row b*P + j is the query at position seq_len[b] + j
        (causal over the first seq_len[b] + j + 1 cached tokens).  fast: the
        binary16 MFMA flash attention (within 2e-3 of the canonical result)."""
        t = self.torch
        rows, hq, d = q.shape
        B = seq_len.numel()
        if rows != B * P:
            raise ValueError(f"q has {rows} rows, expected B*P = {B * P}")
        num_pages, hkv = kpages.shape[0], kpages.shape[1]
        maxp = page_table.shape[1]
        out = t.empty((rows, hq, d), dtype=t.float32, device=self.dev) if out is None else out
        fn = lib().lgx_gqa_prefill_attn_fast if fast else lib().lgx_gqa_prefill_attn
        _check(fn(self.handle, q.data_ptr(), kpages.data_ptr(), vpages.data_ptr(),
                  page_table.data_ptr(), seq_len.data_ptr(), B, P, hq, hkv, d, maxp, num_pages,
                  max_seq_len, out.data_ptr(), self._s()))
        return out

    def q8_gemm(self, W: Q8Matrix, xq, xd, y=None):
        t = self.torch
        m = xq.shape[0]
        y = t.empty((m, W.n), dtype=t.float32, device=self.dev) if y is None else y
        _check(lib().lgx_q8_gemm(self.handle, W.cstruct, xq.data_ptr(), xd.data_ptr(), m,
                                 y.data_ptr(), self._s()))
        return y

    def q8_gemm_noalloc(self, W: Q8Matrix, xq, xd, y):
        """lgx_q8_gemm_noalloc: the same product into the caller's y, with the
        library's fixed device scratch instead of any allocation."""
        m = xq.shape[0]
        _check(lib().lgx_q8_gemm_noalloc(self.handle, W.cstruct, xq.data_ptr(), xd.data_ptr(), m,
                                         y.data_ptr(), self._s()))
        return y

    # ---- decode-step glue ------------------------------------------------
    def embed_f16(self, emb, tokens, out=None):
        t = self.torch
        vocab, h = emb.shape
        m = tokens.numel()
        out = t.empty((m, h), dtype=t.float32, device=self.dev) if out is None else out
        _check(lib().lgx_embed_f16(self.handle, emb.data_ptr(), tokens.data_ptr(), m, h, vocab,
                                   out.data_ptr(), self._s()))
        return out

    def rmsnorm_quant(self, x, w, eps: float, y: bool = True, q8: bool = True):
        """(y, xq, xd) of RMSNorm(x) * w; unrequested outputs are None."""
        t = self.torch
        m, n = x.shape
        yo = t.empty((m, n), dtype=t.float32, device=self.dev) if y else None
        xq = t.empty((m, n), dtype=t.int8, device=self.dev) if q8 else None
        xd = t.empty((m, n // 32), dtype=t.int16, device=self.dev) if q8 else None
        _check(lib().lgx_rmsnorm_quant(self.handle, x.data_ptr(), w.data_ptr(), m, n, eps,
                                       _ptr_or_none(yo), _ptr_or_none(xq), _ptr_or_none(xd),
                                       self._s()))
        return yo, xq, xd

    def add_rmsnorm_quant(self, part, h, w, eps: float, y: bool = True, q8: bool = True):
        """h += tree(part) in place; then (y, xq, xd) of RMSNorm(h) * w."""
        t = self.torch
        nr, m, n = part.shape
        yo = t.empty((m, n), dtype=t.float32, device=self.dev) if y else None
        xq = t.empty((m, n), dtype=t.int8, device=self.dev) if q8 else None
        xd = t.empty((m, n // 32), dtype=t.int16, device=self.dev) if q8 else None
        _check(lib().lgx_add_rmsnorm_quant(self.handle, part.data_ptr(), nr, h.data_ptr(),
                                           w.data_ptr(), m, n, eps, _ptr_or_none(yo),
                                           _ptr_or_none(xq), _ptr_or_none(xd), self._s()))
        return yo, xq, xd

    def rope_kv_append(self, qkv, bias, cos_t, sin_t, seq_len, page_table, kpages, vpages,
                       hq: int, max_seq: int, q_out=None):
        t = self.torch
        B = qkv.shape[0]
        num_pages, hkv, _, d = kpages.shape
        maxp = page_table.shape[1]
        q_out = t.empty((B, hq, d), dtype=t.float32, device=self.dev) if q_out is None else q_out
        _check(lib().lgx_rope_kv_append(
            self.handle, qkv.data_ptr(), _ptr_or_none(bias), cos_t.data_ptr(), sin_t.data_ptr(),
            seq_len.data_ptr(), page_table.data_ptr(), kpages.data_ptr(), vpages.data_ptr(),
            q_out.data_ptr(), B, hq, hkv, d, maxp, num_pages, max_seq, self._s()))
        return q_out

    def swiglu_quant(self, gu, y: bool = True, q8: bool = True):
        t = self.torch
        m, i2 = gu.shape
        inter = i2 // 2
        yo = t.empty((m, inter), dtype=t.float32, device=self.dev) if y else None
        xq = t.empty((m, inter), dtype=t.int8, device=self.dev) if q8 else None
        xd = t.empty((m, inter // 32), dtype=t.int16, device=self.dev) if q8 else None
        _check(lib().lgx_swiglu_quant(self.handle, gu.data_ptr(), m, inter, _ptr_or_none(yo),
                                      _ptr_or_none(xq), _ptr_or_none(xd), self._s()))
        return yo, xq, xd

    def lm_head_f16(self, x, emb, out=None):
        t = self.torch
        m, h = x.shape
        vocab = emb.shape[0]
        out = t.empty((m, vocab), dtype=t.float32, device=self.dev) if out is None else out
        _check(lib().lgx_lm_head_f16(self.handle, x.data_ptr(), emb.data_ptr(), m, h, vocab,
                                     out.data_ptr(), self._s()))
        return out

    def f16_repack_t64(self, emb):
        """binary16 rows (int16/uint16 bits, [rows][h]) -> T64 order (flat)."""
        t = self.torch
        rows, h = emb.shape
        out = t.empty(int(lib().lgx_f16_t64_count(rows, h)), dtype=t.int16, device=self.dev)
        _check(lib().lgx_f16_repack_t64(self.handle, emb.data_ptr(), rows, h, out.data_ptr(),
                                        self._s()))
        return out

    def lm_head_f16_t64(self, x, emb_t64, vocab, out=None):
        t = self.torch
        m, h = x.shape
        out = t.empty((m, vocab), dtype=t.float32, device=self.dev) if out is None else out
        _check(lib().lgx_lm_head_f16_t64(self.handle, x.data_ptr(), emb_t64.data_ptr(), m, h,
                                         vocab, out.data_ptr(), self._s()))
        return out

    def lm_head_rowconst(self, emb):
        """Per-row constants of a binary16 embedding (int16 bits [vocab][h]) for
        lm_head_argmax_f16: float32 [vocab][4]."""
        t = self.torch
        vocab, h = emb.shape
        out = t.empty((vocab, 4), dtype=t.float32, device=self.dev)
        _check(lib().lgx_lm_head_rowconst(self.handle, emb.data_ptr(), vocab, h, out.data_ptr(),
                                          self._s()))
        return out

    def lm_head_argmax_f16(self, x, emb, emb_t64, rowc, out=None, bounds: bool = False):
        """Certified greedy token of the tied lm_head (the token of
        argmax(lm_head_f16(x, emb))); with bounds=True also the [m][vocab][2]
        scaled approximations and their bounds."""
        t = self.torch
        m, h = x.shape
        vocab = emb.shape[0]
        out = t.empty(m, dtype=t.int32, device=self.dev) if out is None else out
        bd = t.empty((m, vocab, 2), dtype=t.float32, device=self.dev) if bounds else None
        _check(lib().lgx_lm_head_argmax_f16(self.handle, x.data_ptr(), emb.data_ptr(),
                                            emb_t64.data_ptr(), rowc.data_ptr(), m, h, vocab,
                                            out.data_ptr(), bd.data_ptr() if bd is not None else None,
                                            self._s()))
        return (out, bd) if bounds else out

    def argmax(self, logits, out=None):
        t = self.torch
        m, vocab = logits.shape
        out = t.empty(m, dtype=t.int32, device=self.dev) if out is None else out
        _check(lib().lgx_argmax(self.handle, logits.data_ptr(), m, vocab, out.data_ptr(),
                                self._s()))
        return out

    def sample(self, logits, positions, top_k: int, top_p: float, temperature: float, seed: int,
               out=None):
        """lgx_sample: seeded top-k / top-p draw per row of logits [m][vocab];
        positions (device int32 [m]) are the draw indices of the rows' streams."""
        t = self.torch
        m, vocab = logits.shape
        out = t.empty(m, dtype=t.int32, device=self.dev) if out is None else out
        _check(lib().lgx_sample(self.handle, logits.data_ptr(), m, vocab, top_k, top_p,
                                temperature, seed, positions.data_ptr(), out.data_ptr(),
                                self._s()))
        return out


def _ptr_or_none(tensor):
    return tensor.data_ptr() if tensor is not None else None


class Model:
    """lgx_model: the seeded random-init Qwen2-shaped Q8_0 model on one device.

    ``cfg`` uses the oracle's keys (n_layers, hidden, inter, n_heads, n_kv,
    head_dim, vocab, tied, max_batch, max_seq, eps, theta, emb_sigma)."""

    def __init__(self, ctx: Context, cfg: dict, seed: int, _handle=None):
        self.ctx = ctx
        self.cfg = dict(cfg)
        self.c = QwenConfigC(cfg["n_layers"], cfg["hidden"], cfg["inter"], cfg["n_heads"],
                             cfg["n_kv"], cfg["head_dim"], cfg["vocab"], cfg["tied"],
                             cfg["max_batch"], cfg["max_seq"], cfg["eps"], cfg["theta"],
                             cfg["emb_sigma"])
        if _handle is None:
            h = C.c_void_p()
            _check(lib().lgx_model_create(ctx.handle, C.byref(self.c), seed, C.byref(h)))
            _handle = h
        self.handle = _handle
        ctx._models.add(self)

    @classmethod
    def load_gguf(cls, ctx: Context, path: str, max_batch: int, max_seq: int) -> "Model":
        """lgx_model_load_gguf: the model of a Qwen2 Q8_0 GGUF file."""
        h = C.c_void_p()
        _check(lib().lgx_model_load_gguf(ctx.handle, path.encode(), max_batch, max_seq,
                                         C.byref(h)))
        c = QwenConfigC()
        _check(lib().lgx_model_config(h, C.byref(c)))
        return cls(ctx, _cfg_dict(c), 0, _handle=h)

    def close(self) -> None:
        if self.handle:
            _check(lib().lgx_model_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self) -> None:
        _check(lib().lgx_model_reset(self.handle, self.ctx._s()))

    def set_sampling(self, temperature: float, top_k: int = 1, top_p: float = 1.0,
                     seed: int = 0) -> None:
        """Seeded top-k / top-p token choice for later steps (temperature 0:
        greedy)."""
        _check(lib().lgx_model_set_sampling(self.handle, temperature, top_k, top_p, seed))

    def set_prefill_mode(self, fast: bool) -> None:
        """fast: later prefills run in binary16 (LGX_PREFILL_FAST: binary16
        GEMMs and flash attention, the last position exact); the call does the
        mode's one-time work (binary16 weights, GEMM plans) and synchronises.
        Otherwise the exact canonical schedule."""
        _check(lib().lgx_model_set_prefill_mode(self.handle, 1 if fast else 0))

    def decode_step(self, tokens) -> None:
        """tokens: device int32 [B], replaced in place by the next tokens."""
        _check(lib().lgx_qwen_decode_step(self.handle, tokens.numel(), tokens.data_ptr(),
                                          self.ctx._s()))

    def generate(self, tokens, nsteps: int, history=None) -> None:
        """nsteps decode steps replayed from a recorded HIP graph; tokens
        (device int32 [B]) ends as the last step's next tokens and history
        (device int32 [nsteps][B], optional) receives every step's."""
        _check(lib().lgx_qwen_generate(self.handle, tokens.numel(), tokens.data_ptr(), nsteps,
                                       0 if history is None else history.data_ptr(),
                                       self.ctx._s()))

    def prefill(self, prompt, next_tokens=None):
        """prompt: device int32 [B][P]; returns the device int32 [B] next tokens."""
        t = self.ctx.torch
        B, P = prompt.shape
        nxt = t.empty(B, dtype=t.int32, device=self.ctx.dev) if next_tokens is None else next_tokens
        _check(lib().lgx_qwen_prefill(self.handle, B, P, prompt.data_ptr(), nxt.data_ptr(),
                                      self.ctx._s()))
        return nxt

    def logits(self, B: int):
        t = self.ctx.torch
        out = t.empty((B, self.cfg["vocab"]), dtype=t.float32, device=self.ctx.dev)
        _check(lib().lgx_qwen_logits(self.handle, B, out.data_ptr(), self.ctx._s()))
        return out

    def tensor_ptr(self, name: str, layer: int = 0):
        """(device pointer, bytes) of a model tensor."""
        p, n = C.c_void_p(), C.c_size_t()
        _check(lib().lgx_model_tensor(self.handle, layer, MODEL_TENSORS[name], C.byref(p),
                                      C.byref(n)))
        return int(p.value or 0), int(n.value)

    def tensor_bytes(self, name: str, layer: int = 0):
        """Host copy (numpy uint8) of a model tensor's bytes."""
        import numpy as np

        t = self.ctx.torch
        p, n = self.tensor_ptr(name, layer)
        t.cuda.current_stream(self.ctx.dev).synchronize()
        out = np.empty(n, np.uint8)
        _check_hip(C.CDLL("libamdhip64.so").hipMemcpy(
            out.ctypes.data_as(C.c_void_p), C.c_void_p(p), C.c_size_t(n), 2))
        return out


    def kv_rows(self, layer: int, which: int, b: int, n: int, page_table=None):
        """Host copy of the first n cached K (which 0) or V (1) rows of
        sequence b at `layer`: binary16 [n][n_kv][head_dim] (gathered page by
        page through the model's page table)."""
        import numpy as np

        cfg = self.cfg
        hkv, d = cfg["n_kv"], cfg["head_dim"]
        maxp = -(-cfg["max_seq"] // 16)
        if page_table is None:
            page_table = self.tensor_bytes("page_table").view(np.int32).reshape(
                cfg["max_batch"], maxp)
        p, _ = self.tensor_ptr("k_pages" if which == 0 else "v_pages", layer)
        page_bytes = hkv * 16 * d * 2
        npg = -(-n // 16)
        buf = np.empty((npg, hkv, 16, d), np.uint16)
        hip = C.CDLL("libamdhip64.so")
        self.ctx.torch.cuda.current_stream(self.ctx.dev).synchronize()
        for i in range(npg):
            _check_hip(hip.hipMemcpy(buf[i].ctypes.data_as(C.c_void_p),
                                     C.c_void_p(p + int(page_table[b, i]) * page_bytes),
                                     C.c_size_t(page_bytes), 2))
        return np.ascontiguousarray(buf.transpose(0, 2, 1, 3).reshape(npg * 16, hkv, d)[:n])


def _cfg_dict(c) -> dict:
    return dict(n_layers=c.n_layers, hidden=c.hidden, inter=c.intermediate, n_heads=c.n_heads,
                n_kv=c.n_kv_heads, head_dim=c.head_dim, vocab=c.vocab, tied=c.tied_embedding,
                max_batch=c.max_batch, max_seq=c.max_seq, eps=c.rms_eps, theta=c.rope_theta,
                emb_sigma=c.emb_sigma)


def gguf_config(path: str, max_batch: int, max_seq: int) -> dict:
    """lgx_gguf_config: the model shape of a Qwen2 GGUF file (host only)."""
    c = QwenConfigC()
    _check(lib().lgx_gguf_config(path.encode(), max_batch, max_seq, C.byref(c)))
    return _cfg_dict(c)


def _check_hip(err: int) -> None:
    if err != 0:
        raise LgxError(10, f"hipMemcpy failed with hipError {err}")
