"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, validates arguments before any device work, and reports
NO_DEVICE cleanly where no GPU is visible.  No kernel is launched here."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT, gpu_available
from foundry_attn import _abi
from foundry_attn._abi import lib

HEADER = os.path.join(ROOT, "include", "foundry_attn.h")
BLOCK_HEADER = os.path.join(ROOT, "include", "foundry_block.h")


def header_functions():
    names = set()
    for h in (HEADER, BLOCK_HEADER):
        src = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(fa_[a-z0-9_]+)\s*\(", src))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    L = lib()
    declared = header_functions()
    assert set(declared) == set(_abi.EXPORTED), declared
    for name in declared:
        assert hasattr(L, name), name


def test_version_and_name():
    assert lib().fa_version() == 2
    # CustomOp3::name of the reference op (lib.rs:154-156)
    assert lib().fa_op_name() == b"foundry-attn-bwd"


def test_struct_layouts_match_header(tmp_path):
    """Compile the header with gcc and compare every field offset and struct
    size with the ctypes mirrors."""
    import shutil
    import subprocess
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    structs = {"fa_strides": _abi.Strides, "fa_attn_fwd_args": _abi.AttnFwdArgs,
               "fa_attn_bwd_args": _abi.AttnBwdArgs, "fa_qk_prologue_args": _abi.QkPrologueArgs,
               "fa_qk_prologue_bwd_args": _abi.QkPrologueBwdArgs, "fa_lora_args": _abi.LoraArgs,
               "fa_lora_bwd_args": _abi.LoraBwdArgs, "fa_ln_mod_args": _abi.LnModArgs,
               "fa_ln_mod_bwd_args": _abi.LnModBwdArgs, "fa_rows_args": _abi.RowsArgs,
               "fa_adamw_args": _abi.AdamwArgs, "fa_swiglu_args": _abi.SwigluArgs,
               "fa_swiglu_bwd_args": _abi.SwigluBwdArgs, "fa_lora_down_args": _abi.LoraDownArgs,
               "fa_lora_up_args": _abi.LoraUpArgs, "fa_lora_grad_args": _abi.LoraGradArgs,
               "fa_gated_ln_mod_args": _abi.GatedLnModArgs, "fa_ln_mod_bwd_gate_args": _abi.LnModBwdGateArgs,
               "fa_gemm_args": _abi.GemmArgs}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{BLOCK_HEADER}"', "int main(void){"]
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    for line in out.splitlines():
        cname, what, val = line.split()
        py = structs[cname]
        want = ctypes.sizeof(py) if what == "size" else getattr(py, what).offset
        assert int(val) == want, (cname, what, val, want)


def _fwd_args(**kw):
    fake = 1 << 20  # aligned non-null placeholder; validation fails before any use
    a = _abi.AttnFwdArgs(dtype=0, batch=1, seq=128, heads=2, head_dim=128, scale=0.088,
                         q=fake, k=fake, v=fake, o=fake, lse=fake,
                         q_stride=_abi.Strides(128 * 256, 256, 128),
                         k_stride=_abi.Strides(128 * 256, 256, 128),
                         v_stride=_abi.Strides(128 * 256, 256, 128),
                         o_stride=_abi.Strides(128 * 256, 256, 128))
    for k_, v_ in kw.items():
        setattr(a, k_, v_)
    return a


@pytest.mark.parametrize("field,value,code", [
    ("head_dim", 96, _abi.FA_ERR_UNSUPPORTED),
    ("head_dim", 0, _abi.FA_ERR_UNSUPPORTED),
    ("seq", 0, _abi.FA_ERR_INVALID_ARG),
    ("batch", -1, _abi.FA_ERR_INVALID_ARG),
    ("scale", 0.0, _abi.FA_ERR_INVALID_ARG),
    ("scale", float("nan"), _abi.FA_ERR_INVALID_ARG),
    ("dtype", 7, _abi.FA_ERR_INVALID_ARG),
    ("q", None, _abi.FA_ERR_INVALID_ARG),
    ("lse", None, _abi.FA_ERR_INVALID_ARG),
    ("k", (1 << 20) + 2, _abi.FA_ERR_INVALID_ARG),          # misaligned bf16 base
    ("q_stride", _abi.Strides(8, 252, 128), _abi.FA_ERR_INVALID_ARG),  # not 16-B rows
])
def test_fwd_validation_errors(field, value, code):
    a = _fwd_args(**{field: value})
    assert lib().fa_attn_fwd(ctypes.byref(a), None) == code
    assert len(lib().fa_last_error()) > 0


def test_null_args_pointer():
    assert lib().fa_attn_fwd(None, None) == _abi.FA_ERR_INVALID_ARG
    assert lib().fa_attn_bwd(None, None) == _abi.FA_ERR_INVALID_ARG


def test_bwd_workspace_size_and_validation():
    fake = 1 << 20
    st = _abi.Strides(128 * 256, 256, 128)
    a = _abi.AttnBwdArgs(dtype=0, batch=2, seq=100, heads=3, head_dim=128, scale=0.1,
                         q=fake, k=fake, v=fake, o=fake, dout=fake, lse=fake, dq=fake, dk=fake,
                         dv=fake, q_stride=st, k_stride=st, v_stride=st, o_stride=st,
                         do_stride=st, dq_stride=st, dk_stride=st, dv_stride=st)
    need = lib().fa_attn_bwd_workspace_size(ctypes.byref(a))
    assert need >= 2 * 3 * 100 * 4 and need % 256 == 0
    a.workspace, a.workspace_bytes = fake, need - 256
    assert lib().fa_attn_bwd(ctypes.byref(a), None) == _abi.FA_ERR_INVALID_ARG
    assert b"workspace" in lib().fa_last_error()
    # 4-wave shapes and f32 have no stored-dS path: the full size is the least
    assert lib().fa_attn_bwd_min_workspace_size(ctypes.byref(a)) == need
    # an 8-wave bf16 shape (44 heads x 5 tiles: 220 workgroups) adds the dS
    # blocks, [heads][S rounded up to 32][S rounded up to 256] bf16, and
    # accepts any workspace of at least the minimum
    b = _abi.AttnBwdArgs.from_buffer_copy(a)
    b.batch, b.seq, b.heads = 1, 1100, 44
    full = lib().fa_attn_bwd_workspace_size(ctypes.byref(b))
    least = lib().fa_attn_bwd_min_workspace_size(ctypes.byref(b))
    assert least == 2 * ((44 * 1100 * 4 + 255) // 256 * 256)
    assert full - least == (44 * 1120 * 1280 * 2 + 255) // 256 * 256
    b.dtype = 1
    assert lib().fa_attn_bwd_workspace_size(ctypes.byref(b)) == lib().fa_attn_bwd_min_workspace_size(ctypes.byref(b))
    b.dtype = 0
    # past 16 GiB of dS (here 8 x 44 heads at S 8192: 47 GiB) no dS is asked for
    big = _abi.AttnBwdArgs.from_buffer_copy(b)
    big.batch, big.seq = 8, 8192
    assert lib().fa_attn_bwd_workspace_size(ctypes.byref(big)) == lib().fa_attn_bwd_min_workspace_size(ctypes.byref(big))
    ok_dev = _abi.FA_OK if gpu_available() else _abi.FA_ERR_NO_DEVICE
    st2 = _abi.Strides(128 * 44 * 1100, 128 * 44, 128)
    for f in ("q_stride", "k_stride", "v_stride", "o_stride", "do_stride", "dq_stride", "dk_stride", "dv_stride"):
        setattr(b, f, st2)
    b.workspace, b.workspace_bytes = fake, least - 256
    assert lib().fa_attn_bwd(ctypes.byref(b), None) == _abi.FA_ERR_INVALID_ARG
    if not gpu_available():
        b.workspace_bytes = least
        assert lib().fa_attn_bwd(ctypes.byref(b), None) == ok_dev


def test_bwd_noalloc_validates_before_device_work():
    """fa_attn_bwd_noalloc refuses a workspace and shapes past its fixed
    scratch before touching the device; a valid call without a GPU reports
    NO_DEVICE."""
    fake = 1 << 20
    st = _abi.Strides(128 * 256, 256, 128)
    mk = lambda **kw: _abi.AttnBwdArgs(**{**dict(dtype=0, batch=2, seq=100, heads=3, head_dim=128, scale=0.1,
                                                 q=fake, k=fake, v=fake, o=fake, dout=fake, lse=fake,
                                                 dq=fake, dk=fake, dv=fake, q_stride=st, k_stride=st,
                                                 v_stride=st, o_stride=st, do_stride=st, dq_stride=st,
                                                 dk_stride=st, dv_stride=st), **kw})
    assert lib().fa_attn_bwd_noalloc(None, None) == _abi.FA_ERR_INVALID_ARG
    a = mk(workspace=fake, workspace_bytes=4096)
    assert lib().fa_attn_bwd_noalloc(ctypes.byref(a), None) == _abi.FA_ERR_INVALID_ARG
    assert b"no workspace" in lib().fa_last_error()
    # one row past the scratch: (2^21 + 1) rows as B=1, H=1, S=2^21+1 (f32 needs
    # no 2 GiB buffer-view check)
    a = mk(dtype=1, batch=1, heads=1, seq=(1 << 21) + 1)
    assert lib().fa_attn_bwd_noalloc(ctypes.byref(a), None) == _abi.FA_ERR_INVALID_ARG
    assert b"2097152 rows" in lib().fa_last_error()
    if not gpu_available():
        a = mk(dtype=1, batch=1, heads=1, seq=1 << 21)
        assert lib().fa_attn_bwd_noalloc(ctypes.byref(a), None) == _abi.FA_ERR_NO_DEVICE


@pytest.mark.skipif(gpu_available(), reason="checks the GPU-less error path")
def test_valid_call_without_device_reports_no_device():
    a = _fwd_args()
    assert lib().fa_attn_fwd(ctypes.byref(a), None) == _abi.FA_ERR_NO_DEVICE
    assert lib().fa_init(0) == _abi.FA_ERR_NO_DEVICE


def test_prologue_validation():
    fake = 1 << 20
    st = _abi.Strides(0, 3072, 128)
    ax = (ctypes.c_int32 * 8)(16, 56, 50, 0, 0, 0, 0, 0)
    a = _abi.QkPrologueArgs(dtype=0, batch=1, tokens=4, heads=24, head_dim=128, eps=1e-6, x=fake,
                            x_stride=st, weight=fake, cos=fake, sin=fake, n_axes=3, axes=ax,
                            y=fake, y_stride=st, y_seq_offset=0)
    assert lib().fa_qk_prologue_fwd(ctypes.byref(a), None) == _abi.FA_ERR_INVALID_ARG
    assert b"sum" in lib().fa_last_error()
    a.axes[2] = 55  # odd width
    assert lib().fa_qk_prologue_fwd(ctypes.byref(a), None) == _abi.FA_ERR_INVALID_ARG
    a.axes[2] = 56
    a.tokens, a.heads = 1 << 26, 32  # tokens * heads = 2^31 rows per batch item
    assert lib().fa_qk_prologue_fwd(ctypes.byref(a), None) == _abi.FA_ERR_UNSUPPORTED
    # the kernels address a batch item's rows in 32 bits from 24-bit products
    a.tokens, a.heads = 4, 24
    a.x_stride = _abi.Strides(0, 1 << 24, 128)  # token stride of 2^24 elements
    assert lib().fa_qk_prologue_fwd(ctypes.byref(a), None) == _abi.FA_ERR_UNSUPPORTED
    assert b"2^24" in lib().fa_last_error()
    a.x_stride = st
    a.tokens, a.y_stride = 1 << 20, _abi.Strides(0, 3072, 128)  # (2^20 - 1) * 3072 + ... >= 2^31
    assert lib().fa_qk_prologue_fwd(ctypes.byref(a), None) == _abi.FA_ERR_UNSUPPORTED
    assert b"2^31" in lib().fa_last_error()
    # a row's token and head come from 24-bit products and an f32 quotient
    # exact for heads <= 1024: 2^24 + 1 tokens of stride 64 span only ~2^30
    # elements, and 1025 heads of stride 128 fit too, yet both are refused
    a.tokens, a.heads = (1 << 24) + 1, 1
    a.x_stride = a.y_stride = _abi.Strides(0, 64, 64)
    a.head_dim, a.axes[0], a.axes[1], a.axes[2] = 64, 16, 24, 24
    assert lib().fa_qk_prologue_fwd(ctypes.byref(a), None) == _abi.FA_ERR_UNSUPPORTED
    assert b"2^24" in lib().fa_last_error()
    a.tokens, a.heads = 4, 1025
    a.x_stride = a.y_stride = _abi.Strides(0, 1025 * 64, 64)
    assert lib().fa_qk_prologue_fwd(ctypes.byref(a), None) == _abi.FA_ERR_UNSUPPORTED
    assert b"1024" in lib().fa_last_error()
    a.head_dim, a.axes[0], a.axes[1], a.axes[2] = 128, 16, 56, 56
    a.x_stride = a.y_stride = st
    a.tokens, a.heads = 4, 24
    b = _abi.QkPrologueBwdArgs(fwd=a, dy=fake, dx=fake, dx_stride=_abi.Strides(0, 3072, 1 << 24))
    assert lib().fa_qk_prologue_bwd(ctypes.byref(b), None) == _abi.FA_ERR_UNSUPPORTED
    assert b"dx" in lib().fa_last_error()


def test_prologue_multi_validation():
    """fa_qk_prologue_{fwd,bwd}_multi check the count, each segment, matching
    dtype / head_dim and overlapping output rows before any device work."""
    fake = 1 << 20
    st = _abi.Strides(0, 3072, 128)
    ax = (ctypes.c_int32 * 8)(16, 56, 56, 0, 0, 0, 0, 0)
    mk = lambda **kw: _abi.QkPrologueArgs(**{**dict(dtype=0, batch=1, tokens=4, heads=24, head_dim=128, eps=1e-6,
                                                    x=fake, x_stride=st, weight=fake, cos=fake, sin=fake, n_axes=3,
                                                    axes=ax, y=fake, y_stride=st, y_seq_offset=0), **kw})
    L = lib()
    arr = (_abi.QkPrologueArgs * 5)(mk(), mk(), mk(), mk(), mk())
    assert L.fa_qk_prologue_fwd_multi(arr, 0, None) == _abi.FA_ERR_INVALID_ARG
    assert L.fa_qk_prologue_fwd_multi(arr, 5, None) == _abi.FA_ERR_INVALID_ARG
    # same y, same strides, rows 0..4 twice
    arr = (_abi.QkPrologueArgs * 2)(mk(), mk())
    assert L.fa_qk_prologue_fwd_multi(arr, 2, None) == _abi.FA_ERR_INVALID_ARG
    assert b"overlapping" in L.fa_last_error()
    arr = (_abi.QkPrologueArgs * 2)(mk(), mk(y_seq_offset=4, head_dim=64,
                                              axes=(ctypes.c_int32 * 8)(16, 24, 24, 0, 0, 0, 0, 0)))
    assert L.fa_qk_prologue_fwd_multi(arr, 2, None) == _abi.FA_ERR_INVALID_ARG
    assert b"head_dim" in L.fa_last_error()
    arr = (_abi.QkPrologueArgs * 2)(mk(), mk(y_seq_offset=4, n_axes=9))
    assert L.fa_qk_prologue_fwd_multi(arr, 2, None) == _abi.FA_ERR_INVALID_ARG
    b = (_abi.QkPrologueBwdArgs * 2)(_abi.QkPrologueBwdArgs(fwd=mk(), dy=fake, dx=fake, dx_stride=st),
                                     _abi.QkPrologueBwdArgs(fwd=mk(y_seq_offset=4), dy=fake, dx=fake, dx_stride=st))
    assert L.fa_qk_prologue_bwd_multi(b, 2, None) == _abi.FA_ERR_INVALID_ARG
    assert b"dx" in L.fa_last_error()
    if not gpu_available():
        arr = (_abi.QkPrologueArgs * 2)(mk(), mk(y_seq_offset=4))
        assert L.fa_qk_prologue_fwd_multi(arr, 2, None) == _abi.FA_ERR_NO_DEVICE


def test_lora_validation():
    fake = 1 << 20
    a = _abi.LoraArgs(dtype=0, tokens=8, in_features=3072, out_features=9216, rank=64, scale=1.0,
                      x=fake, ldx=3072, a=fake, b=fake, u=fake, y=fake, ldy=9216)
    assert lib().fa_lora_fwd(ctypes.byref(a), None) == _abi.FA_ERR_UNSUPPORTED
    a.rank = 16
    a.in_features = 3000  # not a multiple of 16
    assert lib().fa_lora_fwd(ctypes.byref(a), None) == _abi.FA_ERR_UNSUPPORTED


@pytest.mark.parametrize("bf16", [False, True])
def test_rope_tables_host_matches_oracle(bf16):
    """fa_rope_tables_host is host code: it runs here and must equal the
    oracle's rope_tables_dtype restatement bit for bit."""
    import oracle
    from foundry_attn.configs import C2
    pos = np.ascontiguousarray(C2.positions()[::37])
    n = pos.shape[0]
    code = _abi.FA_DTYPE_BF16 if bf16 else _abi.FA_DTYPE_F32
    dt = np.uint16 if bf16 else np.float32
    cos = np.empty((n, 128), dt)
    sin = np.empty((n, 128), dt)
    ax = (ctypes.c_int32 * 3)(16, 56, 56)
    assert lib().fa_rope_tables_host(pos.ctypes.data, n, 3, ctypes.addressof(ax), 1e4, code,
                                     cos.ctypes.data, sin.ctypes.data) == 0
    if bf16:
        cos = (cos.astype(np.uint32) << 16).view(np.float32)
        sin = (sin.astype(np.uint32) << 16).view(np.float32)
    oc, os_ = oracle.rope_tables(pos, [16, 56, 56], 1e4, bf16=bf16)
    np.testing.assert_array_equal(cos, oc)
    np.testing.assert_array_equal(sin, os_)


# ----- block ops (include/foundry_block.h) ----------------------------------

_FAKE = 1 << 20  # aligned non-null placeholder; validation fails before any use


def _status_name(st):
    return _abi.STATUS_NAMES[st]


def test_fused_gated_ln_mod_validates_before_device_work():
    """fa_gated_ln_mod_fwd and fa_ln_mod_bwd_gate check the layer-norm
    arguments as their plain forms do, plus the gate, the branch and the
    extra outputs, before touching a device."""
    L = lib()
    ok_dev = _abi.FA_OK if gpu_available() else _abi.FA_ERR_NO_DEVICE
    ln = _abi.LnModArgs(dtype=0, rows=4, cols=3072, eps=1e-6, x=_FAKE, ldx=3072, shift=_FAKE, scale=_FAKE,
                        y=_FAKE, ldy=3072)
    fw = _abi.GatedLnModArgs(ln=ln, g=_FAKE, b=_FAKE, ldb=3072, sum=_FAKE, ldsum=3072)
    if not gpu_available():
        assert L.fa_gated_ln_mod_fwd(ctypes.byref(fw), None) == ok_dev
        fw2 = _abi.GatedLnModArgs.from_buffer_copy(fw)
        fw2.sum2, fw2.ldsum2 = _FAKE, 3072
        assert L.fa_gated_ln_mod_fwd(ctypes.byref(fw2), None) == ok_dev
    for field, val in (("g", 0), ("g", _FAKE + 2), ("b", 0), ("ldb", 3071), ("sum", 0), ("ldsum", 3000),
                       ("sum2", _FAKE + 8)):
        bad = _abi.GatedLnModArgs.from_buffer_copy(fw)
        setattr(bad, field, val)
        if field == "sum2":
            bad.ldsum2 = 3072
        assert L.fa_gated_ln_mod_fwd(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG, field
    bad = _abi.GatedLnModArgs.from_buffer_copy(fw)
    bad.ln.cols = 3070
    assert L.fa_gated_ln_mod_fwd(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG
    bad = _abi.GatedLnModArgs.from_buffer_copy(fw)
    bad.ln.mean = _FAKE
    assert L.fa_gated_ln_mod_fwd(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG

    stats = _abi.LnModArgs.from_buffer_copy(ln)
    stats.mean, stats.rstd = _FAKE, _FAKE + 256
    bw = _abi.LnModBwdGateArgs(bwd=_abi.LnModBwdArgs(fwd=stats, dy=_FAKE, lddy=3072, dx=_FAKE, lddx=3072),
                               g=_FAKE, gdx=_FAKE, ldgdx=3072)
    if not gpu_available():
        assert L.fa_ln_mod_bwd_gate(ctypes.byref(bw), None) == ok_dev
    for field, val in (("g", 0), ("gdx", 0), ("gdx", _FAKE + 4), ("ldgdx", 3071)):
        bad = _abi.LnModBwdGateArgs.from_buffer_copy(bw)
        setattr(bad, field, val)
        assert L.fa_ln_mod_bwd_gate(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG, field
    bad = _abi.LnModBwdGateArgs.from_buffer_copy(bw)
    bad.bwd.fwd.mean = 0
    assert L.fa_ln_mod_bwd_gate(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG
    assert b"mean and rstd" in L.fa_last_error()


def test_block_ops_validate_before_device_work():
    L = lib()
    ok_dev = _abi.FA_OK if gpu_available() else _abi.FA_ERR_NO_DEVICE
    ln = _abi.LnModArgs(dtype=0, rows=4, cols=3072, eps=1e-6, x=_FAKE, ldx=3072, shift=_FAKE, scale=_FAKE,
                        y=_FAKE, ldy=3072)
    if not gpu_available():
        assert L.fa_ln_mod_fwd(ctypes.byref(ln), None) == ok_dev
    for field, val in (("cols", 3070), ("cols", 8192), ("eps", 0.0), ("ldx", 3071), ("rows", 0),
                       ("dtype", 7), ("x", 0), ("shift", _FAKE + 4)):
        bad = _abi.LnModArgs.from_buffer_copy(ln)
        setattr(bad, field, val)
        assert L.fa_ln_mod_fwd(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG, field
    # mean without rstd
    bad = _abi.LnModArgs.from_buffer_copy(ln)
    bad.mean = _FAKE
    assert L.fa_ln_mod_fwd(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG
    # the backward needs the forward's statistics
    bw = _abi.LnModBwdArgs(fwd=ln, dy=_FAKE, lddy=3072, dx=_FAKE, lddx=3072)
    assert L.fa_ln_mod_bwd(ctypes.byref(bw), None) == _abi.FA_ERR_INVALID_ARG
    assert b"mean and rstd" in L.fa_last_error()

    rows = _abi.RowsArgs(dtype=0, rows=4, cols=64, x=0, ldx=64, g=_FAKE, b=_FAKE, ldb=64, y=_FAKE, ldy=64)
    if not gpu_available():
        for fn in ("fa_gated_residual", "fa_gelu_fwd", "fa_silu"):
            assert getattr(L, fn)(ctypes.byref(rows), None) == ok_dev, fn
    # gelu_bwd needs the upstream gradient x
    assert L.fa_gelu_bwd(ctypes.byref(rows), None) == _abi.FA_ERR_INVALID_ARG
    bad = _abi.RowsArgs.from_buffer_copy(rows)
    bad.g = 0
    assert L.fa_gated_residual(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG
    bad = _abi.RowsArgs.from_buffer_copy(rows)
    bad.ldb = 60
    assert L.fa_gelu_fwd(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG

    ad = _abi.AdamwArgs(dtype=0, n=1000, param=_FAKE, grad=_FAKE, m=_FAKE, v=_FAKE, lr=1e-3, beta1=0.9,
                        beta2=0.999, eps=1e-8, step=1)
    if not gpu_available():
        assert L.fa_adamw_step(ctypes.byref(ad), None) == ok_dev
    for field, val in (("step", 0), ("beta1", 1.0), ("beta2", -0.1), ("eps", 0.0), ("n", 0), ("grad", 0),
                       ("m", _FAKE + 2)):
        bad = _abi.AdamwArgs.from_buffer_copy(ad)
        setattr(bad, field, val)
        assert L.fa_adamw_step(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG, field
    # several tensors of one step: the hyperparameters and dtype must agree
    arr = (_abi.AdamwArgs * 3)(ad, ad, ad)
    if not gpu_available():
        assert L.fa_adamw_step_many(arr, 3, None) == ok_dev
    assert L.fa_adamw_step_many(arr, 0, None) == _abi.FA_ERR_INVALID_ARG
    assert L.fa_adamw_step_many(None, 3, None) == _abi.FA_ERR_INVALID_ARG
    for field, val in (("step", 2), ("lr", 2e-3), ("beta2", 0.99), ("eps", 1e-6), ("dtype", 1), ("n", 0)):
        bad = (_abi.AdamwArgs * 3)(ad, ad, ad)
        setattr(bad[2], field, val)
        assert L.fa_adamw_step_many(bad, 3, None) == _abi.FA_ERR_INVALID_ARG, field
        assert b"tensor 2" in L.fa_last_error() or field == "n", field



def test_swiglu_validate_before_device_work():
    L = lib()
    ok_dev = _abi.FA_OK if gpu_available() else _abi.FA_ERR_NO_DEVICE
    sw = _abi.SwigluArgs(dtype=0, rows=4, cols=9216, gate=_FAKE, ldgate=27648, up=_FAKE + 18432,
                         ldup=27648, y=_FAKE, ldy=12288)
    if not gpu_available():
        assert L.fa_swiglu_fwd(ctypes.byref(sw), None) == ok_dev
    for field, val in (("cols", 9212), ("rows", 0), ("dtype", 3), ("gate", 0), ("up", _FAKE + 2),
                       ("ldgate", 9000), ("ldy", 12290), ("y", 0)):
        bad = _abi.SwigluArgs.from_buffer_copy(sw)
        setattr(bad, field, val)
        assert L.fa_swiglu_fwd(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG, field
    bw = _abi.SwigluBwdArgs(fwd=sw, dy=_FAKE, lddy=9216, dgate=_FAKE, lddgate=27648, dup=_FAKE,
                            lddup=27648)
    if not gpu_available():
        assert L.fa_swiglu_bwd(ctypes.byref(bw), None) == ok_dev
    for field, val in (("dy", 0), ("dgate", _FAKE + 8), ("lddup", 100)):
        bad = _abi.SwigluBwdArgs.from_buffer_copy(bw)
        setattr(bad, field, val)
        assert L.fa_swiglu_bwd(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG, field


def test_lora_pieces_validate_before_device_work():
    L = lib()
    ok_dev = _abi.FA_OK if gpu_available() else _abi.FA_ERR_NO_DEVICE
    dn = _abi.LoraDownArgs(dtype=0, tokens=64, in_features=3072, rank=16, scale=1.0, x=_FAKE, ldx=3136, a=_FAKE,
                           u=_FAKE + 6144, ldu=3136)
    if not gpu_available():
        assert L.fa_lora_down(ctypes.byref(dn), None) == ok_dev
    for field, val, code in (("dtype", 1, _abi.FA_ERR_UNSUPPORTED), ("rank", 65, _abi.FA_ERR_INVALID_ARG),
                             ("in_features", 3080, _abi.FA_ERR_UNSUPPORTED), ("ldu", 8, _abi.FA_ERR_INVALID_ARG),
                             ("x", _FAKE + 2, _abi.FA_ERR_INVALID_ARG), ("u", _FAKE + 1, _abi.FA_ERR_INVALID_ARG)):
        bad = _abi.LoraDownArgs.from_buffer_copy(dn)
        setattr(bad, field, val)
        assert L.fa_lora_down(ctypes.byref(bad), None) == code, field
    # a workgroup addresses up to 64 rows of x with 32-bit offsets: 64 rows
    # spanning 4 GiB are refused, 16 rows of the same stride are not
    bad = _abi.LoraDownArgs.from_buffer_copy(dn)
    bad.ldx = 1 << 26
    assert L.fa_lora_down(ctypes.byref(bad), None) == _abi.FA_ERR_UNSUPPORTED
    assert b"4 GiB" in L.fa_last_error()
    if not gpu_available():
        bad.tokens = 16
        assert L.fa_lora_down(ctypes.byref(bad), None) == ok_dev
    up = _abi.LoraUpArgs(dtype=0, tokens=64, out_features=3072, rank=16, scale=1.0, u=_FAKE, ldu=3136, b=_FAKE,
                         y=_FAKE, ldy=3136)
    if not gpu_available():
        assert L.fa_lora_up(ctypes.byref(up), None) == ok_dev
    bad = _abi.LoraUpArgs.from_buffer_copy(up)
    bad.ldy = 3000
    assert L.fa_lora_up(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG
    gr = _abi.LoraGradArgs(dtype=0, tokens=64, features=3072, rank=16, scale=1.0, u=_FAKE, ldu=3136, x=_FAKE,
                           ldx=3072, grad=_FAKE, transpose=0, workspace=0, workspace_bytes=0)
    assert L.fa_lora_grad_workspace_size(ctypes.byref(gr)) > 0
    assert L.fa_lora_grad(ctypes.byref(gr), None) == _abi.FA_ERR_INVALID_ARG  # no workspace
    assert b"workspace" in L.fa_last_error()
    # the grouped form: one workspace for all products
    arr = (_abi.LoraGradArgs * 3)(*[_abi.LoraGradArgs.from_buffer_copy(gr) for _ in range(3)])
    arr[1].rank, arr[2].transpose = 48, 1
    need = L.fa_lora_grad_many_workspace_size(arr, 3)
    assert need > L.fa_lora_grad_workspace_size(ctypes.byref(gr))
    assert L.fa_lora_grad_many(arr, 3, None, 0, None) == _abi.FA_ERR_INVALID_ARG
    assert b"workspace" in L.fa_last_error()
    assert L.fa_lora_grad_many(arr, 3, _FAKE, need - 256, None) == _abi.FA_ERR_INVALID_ARG
    assert L.fa_lora_grad_many(arr, 0, _FAKE, need, None) == _abi.FA_ERR_INVALID_ARG
    # products may differ in token count: a longer one needs more workspace
    arr[2].tokens = 4096
    assert L.fa_lora_grad_many_workspace_size(arr, 3) > need
    arr[2].tokens = 0
    assert L.fa_lora_grad_many_workspace_size(arr, 3) == 0
    assert L.fa_lora_grad_many(arr, 3, _FAKE, need, None) == _abi.FA_ERR_INVALID_ARG
    assert b"tokens" in L.fa_last_error()
    arr[2].tokens, arr[1].rank = 64, 65
    assert L.fa_lora_grad_many(arr, 3, _FAKE, need, None) == _abi.FA_ERR_INVALID_ARG
    # an x whose rows span 4 GiB or more is refused before any launch
    arr[1].rank, arr[0].tokens, arr[0].ldx = 16, 1 << 20, 4096
    assert L.fa_lora_grad_many(arr, 3, _FAKE, 1 << 40, None) == _abi.FA_ERR_UNSUPPORTED
    assert b"4 GiB" in L.fa_last_error()


def test_copy2d_many_validates_before_device_work():
    """fa_copy2d_many refuses bad views before touching a device."""
    L = _abi.lib()
    good = _abi.Copy2dArgs(dtype=0, rows=16, cols=3072, src=_FAKE, src_rs=3072, src_cs=1, dst=_FAKE + 4096,
                           dst_rs=1, dst_cs=16)
    assert L.fa_copy2d_many(None, 1, None) == _abi.FA_ERR_INVALID_ARG
    arr = (_abi.Copy2dArgs * 2)(good, good)
    assert L.fa_copy2d_many(arr, 0, None) == _abi.FA_ERR_INVALID_ARG
    for field, val in (("dtype", 7), ("rows", 0), ("cols", -1), ("src_rs", -1), ("dst_cs", -2), ("src", 0),
                       ("dst", _FAKE + 1)):
        bad = _abi.Copy2dArgs.from_buffer_copy(good)
        setattr(bad, field, val)
        arr = (_abi.Copy2dArgs * 2)(good, bad)
        assert L.fa_copy2d_many(arr, 2, None) == _abi.FA_ERR_INVALID_ARG, field
        assert b"view 1" in L.fa_last_error(), field
    mixed = _abi.Copy2dArgs.from_buffer_copy(good)
    mixed.dtype = 1
    arr = (_abi.Copy2dArgs * 2)(good, mixed)
    assert L.fa_copy2d_many(arr, 2, None) == _abi.FA_ERR_INVALID_ARG


def test_public_headers_are_plain_c():
    """include/*.h compile as C99 on their own (no C++ or HIP types cross the
    boundary), as a Rust bindgen or cgo consumer would read them."""
    import subprocess
    inc = os.path.join(ROOT, "include")
    for h in ("foundry_attn.h", "foundry_block.h"):
        src = f'#include "{h}"\nint main(void) {{ return 0; }}\n'
        r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", "-fsyntax-only",
                            "-I", inc, "-x", "c", "-"], input=src, capture_output=True, text=True)
        assert r.returncode == 0, (h, r.stderr)


def test_gemm_validation():
    """fa_gemm_bf16 refuses shapes off its 256 x 256 x 64 tiles, bad views,
    unknown epilogues and a missing GELU input before any device work."""
    fake = 1 << 20
    a = _abi.GemmArgs(epilogue=0, m=512, n=256, k=128, a=fake, lda=128, b=fake, ldb=128, c=fake, ldc=256,
                      c2=0, ldc2=0, aux=0, ldaux=0)
    for field, value in (("m", 300), ("n", 128), ("k", 96), ("k", 0)):
        bad = _abi.GemmArgs.from_buffer_copy(a)
        setattr(bad, field, value)
        assert lib().fa_gemm_bf16(ctypes.byref(bad), None) == _abi.FA_ERR_UNSUPPORTED, field
    bad = _abi.GemmArgs.from_buffer_copy(a)
    bad.epilogue = 3
    assert lib().fa_gemm_bf16(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG
    bad = _abi.GemmArgs.from_buffer_copy(a)
    bad.lda = 64  # < k
    assert lib().fa_gemm_bf16(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG
    bad = _abi.GemmArgs.from_buffer_copy(a)
    bad.a = fake + 2  # not 16-byte aligned
    assert lib().fa_gemm_bf16(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG
    bad = _abi.GemmArgs.from_buffer_copy(a)
    bad.epilogue = _abi.FA_GEMM_DGELU  # no aux
    assert lib().fa_gemm_bf16(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG
    bad = _abi.GemmArgs.from_buffer_copy(a)
    bad.epilogue = _abi.FA_GEMM_GELU  # no c2
    assert lib().fa_gemm_bf16(ctypes.byref(bad), None) == _abi.FA_ERR_INVALID_ARG
    bad = _abi.GemmArgs.from_buffer_copy(a)
    bad.lda = bad.ldb = 1 << 23  # a 256-row block spans >= 2^31 bytes
    assert lib().fa_gemm_bf16(ctypes.byref(bad), None) == _abi.FA_ERR_UNSUPPORTED
    assert b"2^31" in lib().fa_last_error()
