"""The Rust binding (crates/foundry-attn-hip) cannot be compiled here (no Rust
toolchain), so its #[repr(C)] structs are checked against the C header by
proxy: field for field, in order and type, against the ctypes mirrors that
test_abi_cpu.py compiles against the header with gcc.  Every fa_* function
the crate declares must be one the library exports."""
import ctypes
import os
import re

import pytest

from conftest import ROOT
from foundry_attn import _abi
from foundry_attn._abi import lib

CRATE = os.path.join(ROOT, "crates", "foundry-attn-hip")
FFI = os.path.join(CRATE, "src", "ffi.rs")

RUST_TO_CTYPES = {
    "i32": ctypes.c_int32, "f32": ctypes.c_float, "i64": ctypes.c_int64, "f64": ctypes.c_double,
    "usize": ctypes.c_size_t, "fa_strides": _abi.Strides,
}


def rust_structs():
    src = re.sub(r"//.*", "", open(FFI).read())
    out = {}
    for name, body in re.findall(r"pub struct (\w+)\s*\{(.*?)\}", src, flags=re.S):
        fields = re.findall(r"pub (\w+):\s*([^,]+),", body)
        out[name] = [(f, t.strip()) for f, t in fields]
    return out


def ctype_of(rust_type: str):
    if rust_type.startswith("*"):
        return ctypes.c_void_p
    return RUST_TO_CTYPES[rust_type]


@pytest.mark.parametrize("rust_name,mirror", [
    ("fa_strides", _abi.Strides),
    ("fa_attn_fwd_args", _abi.AttnFwdArgs),
    ("fa_attn_bwd_args", _abi.AttnBwdArgs),
    ("fa_ln_mod_args", _abi.LnModArgs),
    ("fa_ln_mod_bwd_args", _abi.LnModBwdArgs),
])
def test_rust_structs_match_the_header(rust_name, mirror):
    fields = rust_structs()[rust_name]
    assert [f for f, _ in fields] == [f for f, _ in mirror._fields_], rust_name
    for (f, rt), (_, ct) in zip(fields, mirror._fields_):
        if rt == "fa_ln_mod_args":
            assert ct is _abi.LnModArgs, f
            continue
        want = ctype_of(rt)
        assert ctypes.sizeof(want) == ctypes.sizeof(ct), (rust_name, f, rt)
        if want is not ctypes.c_void_p:
            assert want is ct or (want is ctypes.c_size_t and ct is ctypes.c_size_t), (rust_name, f, rt, ct)


def test_rust_declares_only_exported_functions():
    src = open(FFI).read()
    declared = set(re.findall(r"pub fn (fa_\w+)\(", src))
    assert {"fa_attn_fwd", "fa_attn_bwd", "fa_attn_fwd_workspace_size", "fa_attn_bwd_workspace_size",
            "fa_last_error", "fa_version"} <= declared
    assert declared <= set(_abi.EXPORTED), declared - set(_abi.EXPORTED)
    for name in declared:
        assert hasattr(lib(), name), name


def test_rust_op_keeps_the_reference_surface():
    """Unit struct `AttnBwd`, the reference's name, the cpu_fwd offset-0 guard
    (lib.rs:167-172), and a bwd that takes the saved LSE out of the slot before
    any other work and regenerates it without calling itself."""
    src = open(os.path.join(CRATE, "src", "lib.rs")).read()
    assert re.search(r"pub struct AttnBwd;", src)
    assert 'pub const OP_NAME: &str = "foundry-attn-bwd";' in src
    assert "cpu_fwd requires contiguous offset-0 inputs" in src
    body = src[src.index("fn bwd("):]
    assert "self.bwd(" not in body and "apply_op3" not in body
    assert body.index("take_lse(&key)") < body.index("launch_fwd(")
    # every HIP runtime call goes through the checked wrapper, except hipFree in Drop
    for call in re.findall(r"ffi::(hip\w+)\(", src):
        assert call in ("hipMalloc", "hipMemcpy", "hipDeviceSynchronize", "hipFree", "hipGetErrorString"), call
    for path in ("lib.rs", "block.rs"):
        text = open(os.path.join(CRATE, "src", path)).read()
        for m in re.finditer(r"ffi::hip(Malloc|Memcpy|DeviceSynchronize)\(", text):
            # inside a hip(...) wrapper: no statement boundary since its opening
            opened = text.rfind("hip(", 0, m.start())
            assert opened >= 0 and ";" not in text[opened:m.start()], (path, text[m.start() - 80:m.end()])
