"""The GGUF reader on the host (no GPU): the test writer against the byte
layout the format fixes, the model shape lgx_gguf_config derives, and the
errors of malformed files."""
import struct

import numpy as np
import pytest

import logicaffeine_amd as lgx
from tests import gguf_util as gg


def test_writer_byte_layout(tmp_path):
    """A one-entry, one-tensor file byte for byte as the format lays it out."""
    p = tmp_path / "min.gguf"
    gg.write_gguf(p, [("a", gg.T_U32, 7)], [("t", gg.GGML_F32, np.array([1.5, -2.0], np.float32))])
    b = p.read_bytes()
    want = (b"GGUF" + struct.pack("<IQQ", 3, 1, 1) +
            struct.pack("<Q", 1) + b"a" + struct.pack("<II", 4, 7) +
            struct.pack("<Q", 1) + b"t" + struct.pack("<IQIQ", 1, 2, 0, 0))
    assert b[:len(want)] == want
    assert len(b) % 32 == 8 and b[-8:] == struct.pack("<ff", 1.5, -2.0)
    # a Q8_0 row: the scale bits then the 32 quants, per block
    qs = np.arange(64, dtype=np.int8).reshape(1, 64) - 30
    d = np.array([[0x3C00, 0x8001]], np.uint16)
    raw = gg.q8_rows(qs, d)
    assert raw[:2] == b"\x00\x3c" and raw[34:36] == b"\x01\x80"
    assert raw[2:34] == qs[0, :32].tobytes() and raw[36:] == qs[0, 32:].tobytes()


def _tiny(tied=True):
    from oracle import oracle as orc

    return dict(orc.qwen_config("tiny" if tied else "tiny_untied"), eps=1e-5, theta=50000.0)


@pytest.mark.parametrize("tied", [True, False])
def test_config_from_file(tmp_path, tied):
    cfg = _tiny(tied)
    p = tmp_path / "m.gguf"
    gg.write_gguf(p, gg.qwen2_meta(cfg, alignment=64),
                  gg.qwen2_tensors(cfg, gg.random_qwen2(cfg, 1)), alignment=64)
    got = lgx.gguf_config(str(p), 3, 99)
    for key in ("n_layers", "hidden", "inter", "n_heads", "n_kv", "head_dim", "vocab", "tied"):
        assert got[key] == cfg[key], key
    assert got["max_batch"] == 3 and got["max_seq"] == 99
    assert got["eps"] == np.float32(1e-5) and got["theta"] == 50000.0


def _err(path, *args):
    with pytest.raises(lgx.LgxError) as e:
        lgx.gguf_config(str(path), *(args or (1, 16)))
    return e.value.status_name


def test_malformed_files(tmp_path):
    cfg = _tiny()
    t = gg.random_qwen2(cfg, 2)
    meta = gg.qwen2_meta(cfg)
    assert _err(tmp_path / "absent.gguf") == "LGX_MODULE_LOAD_FAILED"
    p = tmp_path / "bad.gguf"
    gg.write_gguf(p, meta, gg.qwen2_tensors(cfg, t), magic=b"GGUX")
    assert _err(p) == "LGX_MODULE_LOAD_FAILED"
    gg.write_gguf(p, meta, gg.qwen2_tensors(cfg, t), version=1)
    assert _err(p) == "LGX_UNSUPPORTED"
    gg.write_gguf(p, meta, gg.qwen2_tensors(cfg, t))
    p.write_bytes(p.read_bytes()[:200])                      # cut inside the metadata
    assert _err(p) == "LGX_MODULE_LOAD_FAILED"
    llama = [("general.architecture", gg.T_STRING, "llama")] + meta[1:]
    gg.write_gguf(p, llama, gg.qwen2_tensors(cfg, t))
    assert _err(p) == "LGX_UNSUPPORTED"
    no_layers = [m for m in meta if m[0] != "qwen2.block_count"]
    gg.write_gguf(p, no_layers, gg.qwen2_tensors(cfg, t))
    assert _err(p) == "LGX_INVALID_ARGUMENT"
    tq = gg.random_qwen2(dict(cfg, vocab=1008), 2, emb_q8=True)     # a Q8_0 token_embd is read
    gg.write_gguf(p, gg.qwen2_meta(dict(cfg, vocab=1008)), gg.qwen2_tensors(dict(cfg, vocab=1008), tq))
    assert lgx.gguf_config(str(p), 1, 16)["vocab"] == 1008
    tens = gg.qwen2_tensors(cfg, t)
    tens[0] = ("token_embd.weight", gg.GGML_F32, np.zeros((cfg["vocab"], cfg["hidden"]), np.float32))
    gg.write_gguf(p, meta, tens)
    assert _err(p) == "LGX_UNSUPPORTED"
    gg.write_gguf(p, meta, gg.qwen2_tensors(cfg, t))
    assert _err(p, 0, 16) == "LGX_INVALID_ARGUMENT"


def _patch_info(p, name, ndims, field, value):
    """Overwrite a field of tensor `name`'s info in file p: "dim0" or
    "offset" (little-endian u64)."""
    b = bytearray(p.read_bytes())
    key = struct.pack("<Q", len(name)) + name.encode()
    at = b.find(key) + len(key) + 4                      # after n_dims
    pos = at if field == "dim0" else at + 8 * ndims + 4
    b[pos:pos + 8] = struct.pack("<Q", value)
    p.write_bytes(bytes(b))


def test_corrupt_tensor_extents(tmp_path):
    """Offsets or dims that would overflow the size arithmetic are refused
    when the file is opened, before any tensor is read."""
    cfg = _tiny()
    t = gg.random_qwen2(cfg, 3)
    meta = gg.qwen2_meta(cfg)
    p = tmp_path / "c.gguf"
    for field, value in [("offset", 2**64 - 16), ("offset", 2**63), ("dim0", 2**62),
                         ("dim0", 0), ("offset", 10**9)]:
        gg.write_gguf(p, meta, gg.qwen2_tensors(cfg, t))
        assert lgx.gguf_config(str(p), 1, 16)["hidden"] == cfg["hidden"]
        _patch_info(p, "output_norm.weight", 1, field, value)
        assert _err(p) == "LGX_MODULE_LOAD_FAILED", (field, value)
    # a shape number past int32 in the metadata
    big = [(k, gg.T_U64 if k == "qwen2.embedding_length" else ty,
            2**40 if k == "qwen2.embedding_length" else v) for k, ty, v in meta]
    gg.write_gguf(p, big, gg.qwen2_tensors(cfg, t))
    assert _err(p) == "LGX_INVALID_ARGUMENT"


def test_non_text_names_in_errors(tmp_path):
    """Names read from a damaged file reach the error message as printable
    text: a tensor name of raw bytes with impossible dims gives
    LGX_MODULE_LOAD_FAILED and a message the binding decodes."""
    cfg = _tiny()
    t = gg.random_qwen2(cfg, 2)
    p = tmp_path / "names.gguf"
    gg.write_gguf(p, gg.qwen2_meta(cfg), gg.qwen2_tensors(cfg, t))
    name = "token_embd.weight"
    _patch_info(p, name, 2, "dim0", 0)                      # a zero dimension: invalid dims
    b = bytearray(p.read_bytes())
    at = b.find(name.encode())
    b[at:at + 5] = b"\xff\xfe\x80\x01\x7f"                   # not UTF-8, not printable
    p.write_bytes(bytes(b))
    with pytest.raises(lgx.LgxError) as e:
        lgx.gguf_config(str(p), 1, 16)
    assert e.value.status_name == "LGX_MODULE_LOAD_FAILED"
    assert "tensor ?????_embd.weight has invalid dims" in str(e.value)
