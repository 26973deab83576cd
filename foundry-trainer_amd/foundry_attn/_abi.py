"""ctypes view of include/foundry_attn.h (libfoundry_attn.so).

The structures below are field-for-field copies of the C header; tests check
that every symbol the header declares is exported.  Loading fails loudly: if
the shared library is missing there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_PKG_DIR), "libfoundry_attn.so")

FA_OK, FA_ERR_INVALID_ARG, FA_ERR_UNSUPPORTED, FA_ERR_NO_DEVICE, FA_ERR_LOAD_FAILED, FA_ERR_HIP = range(6)
STATUS_NAMES = {0: "OK", 1: "INVALID_ARG", 2: "UNSUPPORTED", 3: "NO_DEVICE", 4: "LOAD_FAILED",
                5: "HIP_ERROR"}
FA_DTYPE_BF16, FA_DTYPE_F32 = 0, 1
FA_BWD_ALL, FA_BWD_PREPASS, FA_BWD_DKDV, FA_BWD_DQ = 0, 1, 2, 3
FA_MAX_ROPE_AXES = 8

EXPORTED = [
    "fa_version", "fa_last_error", "fa_op_name", "fa_init",
    "fa_attn_fwd", "fa_attn_fwd_workspace_size", "fa_attn_bwd_workspace_size", "fa_attn_bwd_min_workspace_size",
    "fa_attn_bwd",
    "fa_attn_bwd_phase", "fa_attn_bwd_noalloc",
    "fa_qk_prologue_fwd", "fa_qk_prologue_bwd", "fa_rope_tables_host",
    "fa_qk_prologue_fwd_multi", "fa_qk_prologue_bwd_multi",
    "fa_lora_fwd", "fa_lora_bwd_workspace_size", "fa_lora_bwd",
    # include/foundry_block.h
    "fa_ln_mod_fwd", "fa_ln_mod_bwd", "fa_gated_residual", "fa_gelu_fwd", "fa_gelu_bwd", "fa_silu",
    "fa_swiglu_fwd", "fa_swiglu_bwd", "fa_adamw_step", "fa_adamw_step_many", "fa_copy2d_many",
    "fa_lora_down", "fa_lora_up", "fa_lora_grad", "fa_lora_grad_workspace_size",
    "fa_lora_grad_many", "fa_lora_grad_many_workspace_size",
    "fa_gated_ln_mod_fwd", "fa_ln_mod_bwd_gate", "fa_gemm_bf16",
]


class FoundryAttnError(RuntimeError):
    """A non-OK fa_status, with the library's thread-local message."""

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")


class Strides(ctypes.Structure):
    _fields_ = [("b", ctypes.c_int64), ("s", ctypes.c_int64), ("h", ctypes.c_int64)]


class AttnFwdArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("batch", ctypes.c_int32), ("seq", ctypes.c_int32),
        ("heads", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("scale", ctypes.c_float),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("lse", ctypes.c_void_p), ("key_keep", ctypes.c_void_p),
        ("q_stride", Strides), ("k_stride", Strides), ("v_stride", Strides), ("o_stride", Strides),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
    ]


class AttnBwdArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("batch", ctypes.c_int32), ("seq", ctypes.c_int32),
        ("heads", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("scale", ctypes.c_float),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("dout", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("key_keep", ctypes.c_void_p),
        ("dq", ctypes.c_void_p), ("dk", ctypes.c_void_p), ("dv", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("q_stride", Strides), ("k_stride", Strides), ("v_stride", Strides), ("o_stride", Strides),
        ("do_stride", Strides), ("dq_stride", Strides), ("dk_stride", Strides),
        ("dv_stride", Strides),
    ]


class QkPrologueArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("batch", ctypes.c_int32), ("tokens", ctypes.c_int32),
        ("heads", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("eps", ctypes.c_float),
        ("x", ctypes.c_void_p), ("x_stride", Strides),
        ("weight", ctypes.c_void_p), ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p),
        ("n_axes", ctypes.c_int32), ("axes", ctypes.c_int32 * FA_MAX_ROPE_AXES),
        ("y", ctypes.c_void_p), ("y_stride", Strides), ("y_seq_offset", ctypes.c_int32),
    ]


class QkPrologueBwdArgs(ctypes.Structure):
    _fields_ = [("fwd", QkPrologueArgs), ("dy", ctypes.c_void_p), ("dx", ctypes.c_void_p),
                ("dx_stride", Strides)]


class LoraArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("tokens", ctypes.c_int32), ("in_features", ctypes.c_int32),
        ("out_features", ctypes.c_int32), ("rank", ctypes.c_int32), ("scale", ctypes.c_float),
        ("x", ctypes.c_void_p), ("ldx", ctypes.c_int64), ("a", ctypes.c_void_p),
        ("b", ctypes.c_void_p), ("u", ctypes.c_void_p), ("y", ctypes.c_void_p),
        ("ldy", ctypes.c_int64),
    ]


class LoraBwdArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", LoraArgs), ("dy", ctypes.c_void_p), ("ldy", ctypes.c_int64),
        ("da", ctypes.c_void_p), ("db", ctypes.c_void_p), ("dx", ctypes.c_void_p),
        ("ldx", ctypes.c_int64), ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class LnModArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("rows", ctypes.c_int32), ("cols", ctypes.c_int32),
        ("eps", ctypes.c_float), ("x", ctypes.c_void_p), ("ldx", ctypes.c_int64),
        ("shift", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("y", ctypes.c_void_p),
        ("ldy", ctypes.c_int64), ("mean", ctypes.c_void_p), ("rstd", ctypes.c_void_p),
    ]


class LnModBwdArgs(ctypes.Structure):
    _fields_ = [("fwd", LnModArgs), ("dy", ctypes.c_void_p), ("lddy", ctypes.c_int64),
                ("dres", ctypes.c_void_p), ("ldres", ctypes.c_int64), ("dx", ctypes.c_void_p),
                ("lddx", ctypes.c_int64)]


class GatedLnModArgs(ctypes.Structure):
    _fields_ = [("ln", LnModArgs), ("g", ctypes.c_void_p), ("b", ctypes.c_void_p), ("ldb", ctypes.c_int64),
                ("sum", ctypes.c_void_p), ("ldsum", ctypes.c_int64), ("sum2", ctypes.c_void_p),
                ("ldsum2", ctypes.c_int64)]


class LnModBwdGateArgs(ctypes.Structure):
    _fields_ = [("bwd", LnModBwdArgs), ("g", ctypes.c_void_p), ("gdx", ctypes.c_void_p), ("ldgdx", ctypes.c_int64)]


class RowsArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("rows", ctypes.c_int32), ("cols", ctypes.c_int32),
        ("x", ctypes.c_void_p), ("ldx", ctypes.c_int64), ("g", ctypes.c_void_p),
        ("b", ctypes.c_void_p), ("ldb", ctypes.c_int64), ("y", ctypes.c_void_p), ("ldy", ctypes.c_int64),
    ]


class LoraDownArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("tokens", ctypes.c_int32), ("in_features", ctypes.c_int32),
        ("rank", ctypes.c_int32), ("scale", ctypes.c_float), ("x", ctypes.c_void_p), ("ldx", ctypes.c_int64),
        ("a", ctypes.c_void_p), ("u", ctypes.c_void_p), ("ldu", ctypes.c_int64),
    ]


class LoraUpArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("tokens", ctypes.c_int32), ("out_features", ctypes.c_int32),
        ("rank", ctypes.c_int32), ("scale", ctypes.c_float), ("u", ctypes.c_void_p), ("ldu", ctypes.c_int64),
        ("b", ctypes.c_void_p), ("y", ctypes.c_void_p), ("ldy", ctypes.c_int64),
    ]


class LoraGradArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("tokens", ctypes.c_int32), ("features", ctypes.c_int32),
        ("rank", ctypes.c_int32), ("scale", ctypes.c_float), ("u", ctypes.c_void_p), ("ldu", ctypes.c_int64),
        ("x", ctypes.c_void_p), ("ldx", ctypes.c_int64), ("grad", ctypes.c_void_p), ("transpose", ctypes.c_int32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
    ]


class SwigluArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("rows", ctypes.c_int32), ("cols", ctypes.c_int32),
        ("gate", ctypes.c_void_p), ("ldgate", ctypes.c_int64), ("up", ctypes.c_void_p),
        ("ldup", ctypes.c_int64), ("y", ctypes.c_void_p), ("ldy", ctypes.c_int64),
    ]


class SwigluBwdArgs(ctypes.Structure):
    _fields_ = [("fwd", SwigluArgs), ("dy", ctypes.c_void_p), ("lddy", ctypes.c_int64),
                ("dgate", ctypes.c_void_p), ("lddgate", ctypes.c_int64), ("dup", ctypes.c_void_p),
                ("lddup", ctypes.c_int64)]


class AdamwArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("n", ctypes.c_int64), ("param", ctypes.c_void_p),
        ("grad", ctypes.c_void_p), ("m", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("lr", ctypes.c_double), ("beta1", ctypes.c_double), ("beta2", ctypes.c_double),
        ("eps", ctypes.c_double), ("step", ctypes.c_int32),
    ]


class Copy2dArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("rows", ctypes.c_int32), ("cols", ctypes.c_int32),
        ("src", ctypes.c_void_p), ("src_rs", ctypes.c_int64), ("src_cs", ctypes.c_int64),
        ("dst", ctypes.c_void_p), ("dst_rs", ctypes.c_int64), ("dst_cs", ctypes.c_int64),
    ]


FA_GEMM_PLAIN, FA_GEMM_GELU, FA_GEMM_DGELU = 0, 1, 2


class GemmArgs(ctypes.Structure):
    _fields_ = [
        ("epilogue", ctypes.c_int32), ("m", ctypes.c_int32), ("n", ctypes.c_int32), ("k", ctypes.c_int32),
        ("a", ctypes.c_void_p), ("lda", ctypes.c_int64), ("b", ctypes.c_void_p), ("ldb", ctypes.c_int64),
        ("c", ctypes.c_void_p), ("ldc", ctypes.c_int64), ("c2", ctypes.c_void_p), ("ldc2", ctypes.c_int64),
        ("aux", ctypes.c_void_p), ("ldaux", ctypes.c_int64),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    """Load libfoundry_attn.so (built by `make -C foundry-trainer_amd`)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FoundryAttnError(FA_ERR_LOAD_FAILED,
                               f"{LIB_PATH} is missing; build it with __graft_entry__.build() "
                               "or `make -C foundry-trainer_amd`")
    L = ctypes.CDLL(LIB_PATH)
    L.fa_version.restype = ctypes.c_int
    L.fa_last_error.restype = ctypes.c_char_p
    L.fa_op_name.restype = ctypes.c_char_p
    L.fa_init.restype = ctypes.c_int
    L.fa_init.argtypes = [ctypes.c_int]
    for name, st in (("fa_attn_fwd", AttnFwdArgs), ("fa_attn_bwd", AttnBwdArgs),
                     ("fa_attn_bwd_noalloc", AttnBwdArgs),
                     ("fa_qk_prologue_fwd", QkPrologueArgs),
                     ("fa_qk_prologue_bwd", QkPrologueBwdArgs),
                     ("fa_lora_fwd", LoraArgs), ("fa_lora_bwd", LoraBwdArgs)):
        fn = getattr(L, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.POINTER(st), ctypes.c_void_p]
    L.fa_qk_prologue_fwd_multi.restype = ctypes.c_int
    L.fa_qk_prologue_fwd_multi.argtypes = [ctypes.POINTER(QkPrologueArgs), ctypes.c_int32, ctypes.c_void_p]
    L.fa_qk_prologue_bwd_multi.restype = ctypes.c_int
    L.fa_qk_prologue_bwd_multi.argtypes = [ctypes.POINTER(QkPrologueBwdArgs), ctypes.c_int32, ctypes.c_void_p]
    L.fa_adamw_step_many.restype = ctypes.c_int
    L.fa_adamw_step_many.argtypes = [ctypes.POINTER(AdamwArgs), ctypes.c_int32, ctypes.c_void_p]
    L.fa_copy2d_many.restype = ctypes.c_int
    L.fa_copy2d_many.argtypes = [ctypes.POINTER(Copy2dArgs), ctypes.c_int32, ctypes.c_void_p]
    L.fa_attn_bwd_phase.restype = ctypes.c_int
    L.fa_attn_bwd_phase.argtypes = [ctypes.POINTER(AttnBwdArgs), ctypes.c_int32, ctypes.c_void_p]
    L.fa_attn_fwd_workspace_size.restype = ctypes.c_size_t
    L.fa_attn_fwd_workspace_size.argtypes = [ctypes.POINTER(AttnFwdArgs)]
    L.fa_attn_bwd_workspace_size.restype = ctypes.c_size_t
    L.fa_attn_bwd_workspace_size.argtypes = [ctypes.POINTER(AttnBwdArgs)]
    L.fa_attn_bwd_min_workspace_size.restype = ctypes.c_size_t
    L.fa_attn_bwd_min_workspace_size.argtypes = [ctypes.POINTER(AttnBwdArgs)]
    L.fa_lora_bwd_workspace_size.restype = ctypes.c_size_t
    L.fa_lora_bwd_workspace_size.argtypes = [ctypes.POINTER(LoraBwdArgs)]
    for name, st in (("fa_ln_mod_fwd", LnModArgs), ("fa_ln_mod_bwd", LnModBwdArgs),
                     ("fa_gated_ln_mod_fwd", GatedLnModArgs), ("fa_ln_mod_bwd_gate", LnModBwdGateArgs),
                     ("fa_gated_residual", RowsArgs), ("fa_gelu_fwd", RowsArgs),
                     ("fa_gelu_bwd", RowsArgs), ("fa_silu", RowsArgs), ("fa_adamw_step", AdamwArgs),
                     ("fa_swiglu_fwd", SwigluArgs), ("fa_swiglu_bwd", SwigluBwdArgs),
                     ("fa_lora_down", LoraDownArgs), ("fa_lora_up", LoraUpArgs), ("fa_lora_grad", LoraGradArgs),
                     ("fa_gemm_bf16", GemmArgs)):
        fn = getattr(L, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.POINTER(st), ctypes.c_void_p]
    L.fa_lora_grad_workspace_size.restype = ctypes.c_size_t
    L.fa_lora_grad_workspace_size.argtypes = [ctypes.POINTER(LoraGradArgs)]
    L.fa_lora_grad_many.restype = ctypes.c_int
    L.fa_lora_grad_many.argtypes = [ctypes.POINTER(LoraGradArgs), ctypes.c_int32, ctypes.c_void_p, ctypes.c_size_t,
                                    ctypes.c_void_p]
    L.fa_lora_grad_many_workspace_size.restype = ctypes.c_size_t
    L.fa_lora_grad_many_workspace_size.argtypes = [ctypes.POINTER(LoraGradArgs), ctypes.c_int32]
    L.fa_rope_tables_host.restype = ctypes.c_int
    L.fa_rope_tables_host.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                      ctypes.c_void_p, ctypes.c_float, ctypes.c_int32,
                                      ctypes.c_void_p, ctypes.c_void_p]
    _lib = L
    return L


def check(status: int) -> None:
    if status != FA_OK:
        raise FoundryAttnError(status, lib().fa_last_error().decode(errors="replace"))
