"""TEST INFRASTRUCTURE ONLY — numpy/ctypes front end of the CPU oracle.

Wraps ``oracle/liboracle.so`` (the plain-C restatement of foundry-spike's
Candle CPU path, crates/foundry-spike/src/lib.rs:45-287; see oracle.h for the
per-function citations).  Only tests/, ``__graft_entry__.smoke()`` and
bench.py's ``cpu_baseline`` leg may import this module, and only as the
checker or the timed CPU baseline; the product path never does.

All arrays are float32 numpy arrays; attention tensors are [B, S, H, D] and
LSE is [B, H, S].  ``bf16=True`` emulates the reference's bf16 run (inputs are
rounded to bf16 here first, then the restatement rounds at the reference's
cast points).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i32p = ctypes.POINTER(ctypes.c_int)


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (gcc + OpenMP)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "all", "-C", _HERE], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_bf16_round.restype = ctypes.c_float
        L.oracle_bf16_round.argtypes = [ctypes.c_float]
        L.oracle_round_bf16_inplace.argtypes = [_f32p, ctypes.c_long]
        L.oracle_attn_fwd.restype = ctypes.c_int
        L.oracle_attn_fwd.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p] + [ctypes.c_int] * 4 + [
            ctypes.c_float, _u8p] + [ctypes.c_int] * 4
        L.oracle_attn_bwd.restype = ctypes.c_int
        L.oracle_attn_bwd.argtypes = [_f32p] * 7 + [ctypes.c_int] * 4 + [ctypes.c_float, _u8p] + [
            ctypes.c_int] * 4
        L.oracle_rms_norm.argtypes = [_f32p, _f32p, _f32p, ctypes.c_long, ctypes.c_int,
                                      ctypes.c_float, ctypes.c_int]
        L.oracle_rope_tables.restype = ctypes.c_int
        L.oracle_rope_tables.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _i32p, ctypes.c_float,
                                         _f32p, _f32p, ctypes.c_int]
        L.oracle_apply_rope.restype = ctypes.c_int
        L.oracle_apply_rope.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_long, ctypes.c_int,
                                        ctypes.c_int, _i32p, ctypes.c_int]
        L.oracle_qk_prologue_bwd.restype = ctypes.c_int
        L.oracle_qk_prologue_bwd.argtypes = [_f32p] * 6 + [ctypes.c_long, ctypes.c_int,
                                                           ctypes.c_int, _i32p, ctypes.c_float]
        L.oracle_linear_lora.argtypes = [_f32p] * 6 + [ctypes.c_int] * 4 + [
            ctypes.c_float, ctypes.c_int, ctypes.c_int]
        L.oracle_linear_lora_bwd.argtypes = [_f32p] * 8 + [ctypes.c_int] * 4 + [
            ctypes.c_float, ctypes.c_int, ctypes.c_int]
        L.oracle_ln_mod_fwd.argtypes = [_f32p, ctypes.c_long, ctypes.c_int, _f32p, _f32p, ctypes.c_float,
                                        ctypes.c_int, _f32p, _f32p, _f32p]
        L.oracle_ln_mod_bwd.argtypes = [_f32p, _f32p, ctypes.c_long, ctypes.c_int, _f32p, _f32p, _f32p,
                                        _f32p, ctypes.c_int, _f32p]
        L.oracle_gated_residual.argtypes = [_f32p, _f32p, _f32p, ctypes.c_long, ctypes.c_int, ctypes.c_int,
                                            _f32p]
        L.oracle_gelu_fwd.argtypes = [_f32p, ctypes.c_long, ctypes.c_int, _f32p]
        L.oracle_gelu_bwd.argtypes = [_f32p, _f32p, ctypes.c_long, ctypes.c_int, _f32p]
        L.oracle_silu.argtypes = [_f32p, ctypes.c_long, ctypes.c_int, _f32p]
        L.oracle_swiglu_fwd.argtypes = [_f32p, _f32p, ctypes.c_long, ctypes.c_int, _f32p]
        L.oracle_swiglu_bwd.argtypes = [_f32p, _f32p, _f32p, ctypes.c_long, ctypes.c_int, _f32p, _f32p]
        L.oracle_adamw_step.argtypes = [_f32p] * 4 + [ctypes.c_long] + [ctypes.c_double] * 4 + [
            ctypes.c_int, ctypes.c_int]
        _lib = L
    return _lib


def _c(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return None if a is None else a.ctypes.data_as(_f32p)


def default_threads() -> int:
    return max(1, len(os.sched_getaffinity(0)))


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even), kept as float32."""
    a = np.array(a, dtype=np.float32, copy=True)
    u = a.view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + np.uint32(0x7FFF) + ((u >> 16) & 1)) & np.uint32(0xFFFF0000)
    u[:] = np.where(nan, u, r)
    return a


def _mask(key_keep, B, S):
    if key_keep is None:
        return None, None
    m = np.ascontiguousarray(key_keep, dtype=np.uint8).reshape(B, S)
    return m, m.ctypes.data_as(_u8p)


def attn_fwd(q, k, v, scale=None, key_keep=None, bf16=False, heads=None, nthreads=None):
    """O [B,S,H,D], LSE [B,H,S] of softmax(q k^T * scale) v (lib.rs:131-149)."""
    q, k, v = _c(q), _c(k), _c(v)
    if bf16:
        q, k, v = bf16_round(q), bf16_round(k), bf16_round(v)
    B, S, H, D = q.shape
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    h0, h1 = (0, H) if heads is None else heads
    o = np.zeros_like(q)
    lse = np.zeros((B, H, S), np.float32)
    m, mp = _mask(key_keep, B, S)
    rc = lib().oracle_attn_fwd(_p(q), _p(k), _p(v), _p(o), _p(lse), B, S, H, D, float(scale), mp,
                               int(bf16), h0, h1, nthreads or default_threads())
    if rc:
        raise RuntimeError(f"oracle_attn_fwd failed rc={rc}")
    return o, lse


def attn_bwd(q, k, v, dout, scale=None, key_keep=None, bf16=False, heads=None, nthreads=None):
    """dQ, dK, dV [B,S,H,D] of the reference backward (lib.rs:216-263)."""
    q, k, v, dout = _c(q), _c(k), _c(v), _c(dout)
    if bf16:
        q, k, v, dout = bf16_round(q), bf16_round(k), bf16_round(v), bf16_round(dout)
    B, S, H, D = q.shape
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    h0, h1 = (0, H) if heads is None else heads
    dq, dk, dv = np.zeros_like(q), np.zeros_like(q), np.zeros_like(q)
    m, mp = _mask(key_keep, B, S)
    rc = lib().oracle_attn_bwd(_p(q), _p(k), _p(v), _p(dout), _p(dq), _p(dk), _p(dv), B, S, H, D,
                               float(scale), mp, int(bf16), h0, h1, nthreads or default_threads())
    if rc:
        raise RuntimeError(f"oracle_attn_bwd failed rc={rc}")
    return dq, dk, dv


def rms_norm(x, w, eps=1e-6, bf16=False):
    """lib.rs:45-58 over the last dim."""
    x, w = _c(x), _c(w)
    D = x.shape[-1]
    y = np.empty_like(x)
    lib().oracle_rms_norm(_p(x), _p(w), _p(y), x.size // D, D, float(eps), int(bf16))
    return y


def _axes(axes):
    a = (ctypes.c_int * len(axes))(*[int(t) for t in axes])
    return a


def rope_tables(positions, axes, theta, bf16=False):
    """lib.rs:77-105: cos, sin [n_pos, sum(axes)] from positions [n_pos, n_axes]."""
    pos = _c(positions)
    n, na = pos.shape
    if na != len(axes):
        raise ValueError("positions/axes mismatch")
    D = int(sum(axes))
    cos = np.empty((n, D), np.float32)
    sin = np.empty((n, D), np.float32)
    rc = lib().oracle_rope_tables(_p(pos), n, na, _axes(axes), float(theta), _p(cos), _p(sin),
                                  int(bf16))
    if rc:
        raise ValueError("bad rope axes")
    return cos, sin


def apply_rope(x, cos, sin, axes, bf16=False):
    """lib.rs:122-129: x [S, H, D], cos/sin [S, D]."""
    x, cos, sin = _c(x), _c(cos), _c(sin)
    S, H, D = x.shape
    y = np.empty_like(x)
    rc = lib().oracle_apply_rope(_p(x), _p(cos), _p(sin), _p(y), S, H, len(axes), _axes(axes),
                                 int(bf16))
    if rc:
        raise ValueError("bad rope args")
    return y


def qk_prologue_bwd(x, w, cos, sin, dy, axes, eps=1e-6):
    """Chain rule through apply_rope(rms_norm(x, w)) in f32; x, dy [S, H, D]."""
    x, w, cos, sin, dy = _c(x), _c(w), _c(cos), _c(sin), _c(dy)
    S, H, D = x.shape
    dx = np.empty_like(x)
    rc = lib().oracle_qk_prologue_bwd(_p(x), _p(w), _p(cos), _p(sin), _p(dy), _p(dx), S, H,
                                      len(axes), _axes(axes), float(eps))
    if rc:
        raise ValueError("bad prologue args")
    return dx


def linear_lora(x, W, bias=None, A=None, Bm=None, scale=1.0, bf16=False, nthreads=None):
    """lib.rs:270-287: y = x W^T (+b) + scale (x A^T) B^T."""
    x, W = _c(x), _c(W)
    bias = None if bias is None else _c(bias)
    A = None if A is None else _c(A)
    Bm = None if Bm is None else _c(Bm)
    N, in_f = x.shape
    out_f = W.shape[0]
    r = 0 if A is None else A.shape[0]
    y = np.empty((N, out_f), np.float32)
    lib().oracle_linear_lora(_p(x), _p(W), _p(bias), _p(A), _p(Bm), _p(y), N, in_f, out_f, r,
                             float(scale), int(bf16), nthreads or default_threads())
    return y


def linear_lora_bwd(x, W, A, Bm, dy, scale=1.0, bf16=False, want_dx=True, nthreads=None):
    """Chain rule through linear_scaled: returns (dx | None, dA, dB)."""
    x, W, A, Bm, dy = _c(x), _c(W), _c(A), _c(Bm), _c(dy)
    N, in_f = x.shape
    out_f, r = Bm.shape
    dx = np.empty((N, in_f), np.float32) if want_dx else None
    dA = np.empty((r, in_f), np.float32)
    dB = np.empty((out_f, r), np.float32)
    lib().oracle_linear_lora_bwd(_p(x), _p(W), _p(A), _p(Bm), _p(dy), _p(dx), _p(dA), _p(dB), N,
                                 in_f, out_f, r, float(scale), int(bf16),
                                 nthreads or default_threads())
    return dx, dA, dB


# ----- double-stream block ops (block_oracle.c) -------------------------------

def ln_mod_fwd(x, shift, scale, eps=1e-6, bf16=False):
    """layer_norm_mod (lib.rs:60-71) over the rows of x [N, C]; returns
    y, mean [N], rstd [N]."""
    x = _c(x)
    N, C = x.shape
    y = np.empty_like(x)
    mean = np.empty(N, np.float32)
    rstd = np.empty(N, np.float32)
    lib().oracle_ln_mod_fwd(_p(x), N, C, _p(_c(shift)), _p(_c(scale)), eps, int(bf16), _p(y), _p(mean),
                            _p(rstd))
    return y, mean, rstd


def ln_mod_bwd(x, dy, scale, mean, rstd, dres=None, bf16=False):
    x, dy = _c(x), _c(dy)
    N, C = x.shape
    dx = np.empty_like(x)
    lib().oracle_ln_mod_bwd(_p(x), _p(dy), N, C, _p(_c(scale)), _p(_c(mean)), _p(_c(rstd)),
                            None if dres is None else _p(_c(dres)), int(bf16), _p(dx))
    return dx


def gated_residual(x, g, b, bf16=False):
    b = _c(b)
    N, C = b.shape
    y = np.empty_like(b)
    lib().oracle_gated_residual(None if x is None else _p(_c(x)), _p(_c(g)), _p(b), N, C, int(bf16), _p(y))
    return y


def gelu_fwd(b, bf16=False):
    b = _c(b)
    y = np.empty_like(b)
    lib().oracle_gelu_fwd(_p(b), b.size, int(bf16), _p(y))
    return y


def gelu_bwd(dy, b, bf16=False):
    b, dy = _c(b), _c(dy)
    y = np.empty_like(b)
    lib().oracle_gelu_bwd(_p(dy), _p(b), b.size, int(bf16), _p(y))
    return y


def silu(b, bf16=False):
    b = _c(b)
    y = np.empty_like(b)
    lib().oracle_silu(_p(b), b.size, int(bf16), _p(y))
    return y


def swiglu_fwd(gate, up, bf16=False):
    """silu(gate) * up (lib.rs:293-297)."""
    g, u = _c(gate), _c(up)
    y = np.empty_like(g)
    lib().oracle_swiglu_fwd(_p(g), _p(u), g.size, int(bf16), _p(y))
    return y


def swiglu_bwd(dy, gate, up, bf16=False):
    """(dgate, dup) of silu(gate) * up."""
    g, u, d = _c(gate), _c(up), _c(dy)
    dg, du = np.empty_like(g), np.empty_like(g)
    lib().oracle_swiglu_bwd(_p(d), _p(g), _p(u), g.size, int(bf16), _p(dg), _p(du))
    return dg, du


def adamw_step(param, grad, m, v, step, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, bf16=False):
    """adamw_step (lib.rs:477-510); returns the updated (param, m, v)."""
    p, g = _c(param).copy(), _c(grad)
    m, v = _c(m).copy(), _c(v).copy()
    lib().oracle_adamw_step(_p(p), _p(g), _p(m), _p(v), p.size, lr, beta1, beta2, eps, int(step), int(bf16))
    return p, m, v

