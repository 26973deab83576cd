//! Declarations of `include/foundry_attn.h` (the attention part of the C ABI
//! of libfoundry_attn.so) and the few HIP runtime calls the op needs.  The
//! structs are field-for-field copies of the header's; the Python mirror
//! (`foundry_attn/_abi.py`) is checked against the header by a compiled
//! offsetof test, and these follow the same order and types.
#![allow(non_camel_case_types, dead_code)]

use std::os::raw::{c_char, c_int, c_void};

pub type fa_status = c_int;
pub const FA_OK: fa_status = 0;
pub const FA_ERR_INVALID_ARG: fa_status = 1;
pub const FA_ERR_UNSUPPORTED: fa_status = 2;
pub const FA_ERR_NO_DEVICE: fa_status = 3;
pub const FA_ERR_LOAD_FAILED: fa_status = 4;
pub const FA_ERR_HIP: fa_status = 5;

pub const FA_DTYPE_BF16: i32 = 0;
pub const FA_DTYPE_F32: i32 = 1;
pub const FA_ABI_VERSION: c_int = 2;

/// Element strides of a [B, S, H, D] view; the D stride is 1.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct fa_strides {
    pub b: i64,
    pub s: i64,
    pub h: i64,
}

#[repr(C)]
pub struct fa_attn_fwd_args {
    pub dtype: i32,
    pub batch: i32,
    pub seq: i32,
    pub heads: i32,
    pub head_dim: i32,
    pub scale: f32,
    pub q: *const c_void,
    pub k: *const c_void,
    pub v: *const c_void,
    pub o: *mut c_void,
    pub lse: *mut f32,
    pub key_keep: *const u8,
    pub q_stride: fa_strides,
    pub k_stride: fa_strides,
    pub v_stride: fa_strides,
    pub o_stride: fa_strides,
    pub workspace: *mut c_void,
    pub workspace_bytes: usize,
}

#[repr(C)]
pub struct fa_attn_bwd_args {
    pub dtype: i32,
    pub batch: i32,
    pub seq: i32,
    pub heads: i32,
    pub head_dim: i32,
    pub scale: f32,
    pub q: *const c_void,
    pub k: *const c_void,
    pub v: *const c_void,
    pub o: *const c_void,
    pub dout: *const c_void,
    pub lse: *const f32,
    pub key_keep: *const u8,
    pub dq: *mut c_void,
    pub dk: *mut c_void,
    pub dv: *mut c_void,
    pub workspace: *mut c_void,
    pub workspace_bytes: usize,
    pub q_stride: fa_strides,
    pub k_stride: fa_strides,
    pub v_stride: fa_strides,
    pub o_stride: fa_strides,
    pub do_stride: fa_strides,
    pub dq_stride: fa_strides,
    pub dk_stride: fa_strides,
    pub dv_stride: fa_strides,
}

extern "C" {
    pub fn fa_version() -> c_int;
    pub fn fa_last_error() -> *const c_char;
    pub fn fa_op_name() -> *const c_char;
    pub fn fa_init(device: c_int) -> fa_status;
    pub fn fa_attn_fwd(args: *const fa_attn_fwd_args, stream: *mut c_void) -> fa_status;
    pub fn fa_attn_fwd_workspace_size(args: *const fa_attn_fwd_args) -> usize;
    pub fn fa_attn_bwd_workspace_size(args: *const fa_attn_bwd_args) -> usize;
    pub fn fa_attn_bwd_min_workspace_size(args: *const fa_attn_bwd_args) -> usize;
    pub fn fa_attn_bwd(args: *const fa_attn_bwd_args, stream: *mut c_void) -> fa_status;
    pub fn fa_attn_bwd_noalloc(args: *const fa_attn_bwd_args, stream: *mut c_void) -> fa_status;
}

// HIP runtime (libamdhip64): hipError_t is a C enum, hipSuccess = 0.
pub type hipError_t = c_int;
pub const HIP_SUCCESS: hipError_t = 0;
pub const HIP_MEMCPY_HOST_TO_DEVICE: c_int = 1;
pub const HIP_MEMCPY_DEVICE_TO_HOST: c_int = 2;

extern "C" {
    pub fn hipMalloc(ptr: *mut *mut c_void, bytes: usize) -> hipError_t;
    pub fn hipFree(ptr: *mut c_void) -> hipError_t;
    pub fn hipMemcpy(dst: *mut c_void, src: *const c_void, bytes: usize, kind: c_int) -> hipError_t;
    pub fn hipDeviceSynchronize() -> hipError_t;
    pub fn hipGetErrorString(e: hipError_t) -> *const c_char;
}

// include/foundry_block.h: the LayerNorm-modulation op (the other block ops
// bind the same way).
#[repr(C)]
pub struct fa_ln_mod_args {
    pub dtype: i32,
    pub rows: i32,
    pub cols: i32,
    pub eps: f32,
    pub x: *const c_void,
    pub ldx: i64,
    pub shift: *const c_void,
    pub scale: *const c_void,
    pub y: *mut c_void,
    pub ldy: i64,
    pub mean: *mut f32,
    pub rstd: *mut f32,
}

#[repr(C)]
pub struct fa_ln_mod_bwd_args {
    pub fwd: fa_ln_mod_args,
    pub dy: *const c_void,
    pub lddy: i64,
    pub dres: *const c_void,
    pub ldres: i64,
    pub dx: *mut c_void,
    pub lddx: i64,
}

extern "C" {
    pub fn fa_ln_mod_fwd(args: *const fa_ln_mod_args, stream: *mut c_void) -> fa_status;
    pub fn fa_ln_mod_bwd(args: *const fa_ln_mod_bwd_args, stream: *mut c_void) -> fa_status;
}
