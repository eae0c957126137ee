"""The C-ABI library loads and exports every symbol include/lgx.h declares;
error paths that need no device (no compute calls are made here)."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lgx.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(lgx_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    import logicaffeine_amd as lgx

    L = lgx.lib()
    names = declared_functions()
    assert len(names) >= 14
    for n in names:
        assert hasattr(L, n), f"liblgx.so does not export {n}"
    # the Python mirror binds exactly the declared surface
    assert sorted(lgx.SIGNATURES) == names


def test_abi_version_and_status_values():
    import logicaffeine_amd as lgx

    src = open(HEADER).read()
    assert int(re.search(r"LGX_ABI_VERSION (\d+)u", src).group(1)) == lgx.lib().lgx_abi_version()
    block = re.search(r"typedef enum lgx_status \{(.*?)\} lgx_status;", src, re.S).group(1)
    enum = dict((name, int(v)) for name, v in re.findall(r"(LGX_[A-Z_]+) = (\d+)", block))
    assert {v: k for k, v in enum.items()} == lgx.STATUS_NAMES
    # model tensor ids
    tids = dict((name[6:].lower(), int(v))
                for name, v in re.findall(r"(LGX_T_[A-Z_]+) = (\d+)", src))
    tids["dn_q"], tids["dn_d"] = tids.pop("down_q"), tids.pop("down_d")
    tids["bias"] = tids.pop("qkv_bias")
    assert tids == lgx.MODEL_TENSORS
    # LogosStatus values carried over (codegen/ffi.rs:196-209)
    assert enum["LGX_OK"] == 0 and enum["LGX_NULL_POINTER"] == 3
    assert enum["LGX_OUT_OF_BOUNDS"] == 4 and enum["LGX_INVALID_HANDLE"] == 6
    assert enum["LGX_OUT_OF_MEMORY"] == 9


def test_invalid_handle_and_null_pointer_paths():
    import logicaffeine_amd as lgx

    L = lgx.lib()
    L.lgx_clear_error()
    assert L.lgx_last_error() is None
    assert L.lgx_ctx_launch_count(None) == 0
    assert L.lgx_ctx_arch(None) is None
    assert L.lgx_ctx_create(0, None, None) == 3
    assert b"NULL" in L.lgx_last_error()
    bogus = C.c_void_p(0)
    assert L.lgx_ctx_destroy(bogus) == 6
    assert L.lgx_quantize_q8_0(bogus, None, 1, 32, None, None, None) == 6
    assert L.lgx_q8_gemm(bogus, None, None, None, 1, None, None) == 6
    assert L.lgx_q8_gemm_noalloc(bogus, None, None, None, 1, None, None) == 6
    assert L.lgx_q8q8_gemv(bogus, None, None, None, None, None, None) == 6
    assert L.lgx_q8_gemv_f32(bogus, None, None, None, None) == 6
    assert L.lgx_q8_repack_t16(bogus, None, None, 16, 64, None, None, None) == 6
    assert L.lgx_q8_unpack_t16(bogus, None, None, 16, 64, None, None, None) == 6
    assert b"invalid lgx_ctx" in L.lgx_last_error()
    L.lgx_clear_error()
    assert L.lgx_last_error() is None


def test_scale_count_matches_oracle_layout():
    import logicaffeine_amd as lgx
    from oracle import oracle as orc

    L = lgx.lib()
    for n, k in ((16, 64), (4864, 896), (8960, 1536), (3584, 18944), (32, 2112)):
        assert L.lgx_q8_scale_count(n, k) == orc.lib().orc_q8_s16_count(n, k)
    assert L.lgx_q8_scale_count(17, 64) == 0 and L.lgx_q8_scale_count(16, 32) == 0


def test_ctx_create_without_device_fails_loudly():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present; covered by the gpu tests")
    import logicaffeine_amd as lgx

    with pytest.raises(lgx.LgxError) as ei:
        lgx.lib()  # loads
        h = C.c_void_p()
        lgx._check(lgx.lib().lgx_ctx_create(0, None, C.byref(h)))
    assert ei.value.status_name == "LGX_NO_DEVICE"


def test_missing_code_object_is_a_load_error(tmp_path):
    """With a device present a bad path gives LGX_MODULE_LOAD_FAILED; without
    one the device check comes first.  Either way: an error, no fallback."""
    import logicaffeine_amd as lgx

    h = C.c_void_p()
    st = lgx.lib().lgx_ctx_create(0, str(tmp_path / "nope.hsaco").encode(), C.byref(h))
    assert st in (5, 11)
    assert h.value is None


def test_every_host_kernel_exists_in_code_object():
    """The launcher resolves kernels by name (hipModuleGetFunction); every
    name in its table must be a kernel symbol of the built lgx_kernels.hsaco."""
    import subprocess

    import logicaffeine_amd as lgx

    src = open(os.path.join(ROOT, "logicaffeine_amd", "csrc", "lgx_internal.h")).read()
    table = src[src.index("kKernelNames[] = {"):]
    table = table[:table.index("};")]
    names = re.findall(r'"(lgx_k_[a-z0-9_]+)"', table)
    # the count against the kernel enum is a static_assert in lgx_internal.h
    assert len(names) == len(set(names)) > 20
    readelf = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib", "llvm", "bin",
                           "llvm-readelf")
    syms = subprocess.run([readelf, "-sW", lgx.HSACO_PATH], capture_output=True,
                          text=True, check=True).stdout
    defined = set(line.split()[-1] for line in syms.splitlines() if " FUNC " in line)
    for n in names:
        assert n in defined, f"{n} missing from {lgx.HSACO_PATH}"
