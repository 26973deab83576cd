"""PyTorch-facing host layer over the C ABI.

Mirrors foundry-spike's op surface so callers (and the parity tests) read like
the reference's own code:

  AttnBwd            the CustomOp3 (crates/foundry-spike/src/lib.rs:151-264):
                     name(), fwd() in place of cuda_fwd/cpu_fwd, bwd()
  attention          autograd wrapper: q.apply_op3(k, v, AttnBwd) (lib.rs:366)
  rope_tables        rope_tables_dtype (lib.rs:77-105)
  qk_prologue        apply_rope(rms_norm(x, w)) written into the joint buffer
                     (lib.rs:45-58, 122-129, 363-365)
  lora_fwd/lora_bwd  the adapter term of linear_scaled (lib.rs:270-287)

Every call goes through libfoundry_attn.so on the tensors' HIP device and the
current torch stream.  Tensors are [B, S, H, D] (or the reference's per-sample
(S, H, D), treated as B = 1) with a contiguous head dim.  PyTorch only supplies
device memory and streams here; all arithmetic is in the HIP kernels.
"""
from __future__ import annotations

import ctypes
import math
import weakref
from typing import Optional, Sequence, Tuple

import numpy as np
import torch

from . import _abi
from ._abi import FoundryAttnError, check, lib

_DTYPES = {torch.bfloat16: _abi.FA_DTYPE_BF16, torch.float32: _abi.FA_DTYPE_F32}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise FoundryAttnError(_abi.FA_ERR_UNSUPPORTED, f"dtype {t.dtype} (bf16 and f32 only)")


def _as4(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dim() == 3:
        t = t.unsqueeze(0)
    if t.dim() != 4:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, f"{name} must be (S,H,D) or (B,S,H,D)")
    if not t.is_cuda:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, f"{name} must be a device tensor")
    if t.stride(3) != 1:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, f"{name} must have a contiguous head dim")
    return t


def _strides(t: torch.Tensor) -> _abi.Strides:
    return _abi.Strides(t.stride(0), t.stride(1), t.stride(2))


def _stream(t: torch.Tensor) -> int:
    """torch's current stream on t's device, which must be the current
    device: the library launches on the current HIP device (and sizes split
    workspaces for it), so a tensor elsewhere is refused rather than read
    from the wrong GPU."""
    cur = torch.cuda.current_device()
    if t.device.index != cur:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG,
                               f"{t.device} is not the current device cuda:{cur}; the library launches on the "
                               f"current device: call inside `with torch.cuda.device({t.device})`")
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _keep(key_keep: Optional[torch.Tensor], B: int, S: int, dev) -> Optional[torch.Tensor]:
    if key_keep is None:
        return None
    kk = key_keep.to(device=dev, dtype=torch.uint8).reshape(B, S).contiguous()
    return kk


def attn_fwd(q, k, v, scale: Optional[float] = None, key_keep=None, out=None, lse=None,
             workspace: Optional[torch.Tensor] = None, split: bool = True):
    """O, LSE of softmax(q k^T * scale) v via fa_attn_fwd.

    q, k, v: (B,S,H,D) or (S,H,D) device tensors, bf16 or f32.  scale defaults
    to 1/sqrt(D) (the reference hard-codes 1/sqrt(128), lib.rs:138).
    key_keep: optional (B,S) bool/uint8 mask, False = key excluded.
    split: pass a workspace so that a grid too small for the GPU (few heads,
    fa_attn_fwd_workspace_size > 0) splits each tile's keys; `workspace` is
    used when large enough, else one is allocated.  split=False runs the
    unsplit kernel.
    Returns o (same shape as q) and lse (B,H,S) float32.
    """
    squeeze = q.dim() == 3
    q4, k4, v4 = _as4(q, "q"), _as4(k, "k"), _as4(v, "v")
    B, S, H, D = q4.shape
    if k4.shape != q4.shape or v4.shape != q4.shape:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "q, k, v shapes differ")
    if not (k4.dtype == v4.dtype == q4.dtype) or not (k4.device == v4.device == q4.device):
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "q, k, v dtypes or devices differ")
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    o4 = torch.empty_like(q4, memory_format=torch.contiguous_format) if out is None else _as4(out, "out")
    lse_t = torch.empty((B, H, S), dtype=torch.float32, device=q4.device) if lse is None else lse
    if o4.shape != q4.shape or o4.dtype != q4.dtype or o4.device != q4.device:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "out does not match q")
    if lse_t.shape != (B, H, S) or lse_t.dtype != torch.float32 or not lse_t.is_contiguous() \
            or lse_t.device != q4.device:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "lse must be contiguous float32 (B,H,S)")
    kk = _keep(key_keep, B, S, q4.device)
    a = _abi.AttnFwdArgs(dtype=_dtype_code(q4), batch=B, seq=S, heads=H, head_dim=D, scale=scale,
                         q=_ptr(q4), k=_ptr(k4), v=_ptr(v4), o=_ptr(o4), lse=_ptr(lse_t),
                         key_keep=_ptr(kk), q_stride=_strides(q4), k_stride=_strides(k4),
                         v_stride=_strides(v4), o_stride=_strides(o4))
    need = lib().fa_attn_fwd_workspace_size(ctypes.byref(a)) if split else 0
    if need:
        if workspace is None or workspace.numel() * workspace.element_size() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=q4.device)
        a.workspace = workspace.data_ptr()
        a.workspace_bytes = workspace.numel() * workspace.element_size()
    check(lib().fa_attn_fwd(ctypes.byref(a), _stream(q4)))
    return (o4[0] if squeeze else o4), lse_t


def attn_bwd_workspace_bytes(B: int, S: int, H: int, D: int, dtype=torch.bfloat16, minimum: bool = False) -> int:
    """Backward workspace bytes for (B, S, H, D) on the current device: the
    full size (dQ reads the dK/dV kernel's stored dS where that path applies)
    or, with minimum, the least fa_attn_bwd accepts (dQ recomputes S and dP).
    Both give the same bits."""
    ba = _abi.AttnBwdArgs(dtype=_dtype_code(torch.empty(0, dtype=dtype)), batch=B, seq=S, heads=H, head_dim=D)
    f = lib().fa_attn_bwd_min_workspace_size if minimum else lib().fa_attn_bwd_workspace_size
    return int(f(ctypes.byref(ba)))


def attn_workspace_bytes(q) -> Tuple[int, int]:
    """(forward, backward) workspace bytes the library asks for q's shape
    (B,S,H,D) or (S,H,D) and dtype on its device: the forward's is 0 unless
    the shape splits (fa_attn_fwd_workspace_size)."""
    q4 = _as4(q, "q")
    B, S, H, D = q4.shape
    with torch.cuda.device(q4.device):
        fa = _abi.AttnFwdArgs(dtype=_dtype_code(q4), batch=B, seq=S, heads=H, head_dim=D)
        ba = _abi.AttnBwdArgs(dtype=_dtype_code(q4), batch=B, seq=S, heads=H, head_dim=D)
        return (int(lib().fa_attn_fwd_workspace_size(ctypes.byref(fa))),
                int(lib().fa_attn_bwd_workspace_size(ctypes.byref(ba))))


def attn_bwd(q, k, v, o, dout, lse, scale: Optional[float] = None, key_keep=None,
             workspace: Optional[torch.Tensor] = None, phases=None, out=None):
    """dq, dk, dv via fa_attn_bwd (P recomputed from the saved LSE).

    phases: None runs the whole backward in one call; otherwise an iterable of
    (phase, stream_or_None) pairs issued in order through fa_attn_bwd_phase
    (FA_BWD_PREPASS must come first), e.g. to time the launches separately.
    out: optional (dq, dk, dv) tensors to write into.
    """
    squeeze = q.dim() == 3
    q4, k4, v4 = _as4(q, "q"), _as4(k, "k"), _as4(v, "v")
    o4, do4 = _as4(o, "o"), _as4(dout, "dout")
    B, S, H, D = q4.shape
    for name, t in (("k", k4), ("v", v4), ("o", o4), ("dout", do4)):
        if t.shape != q4.shape or t.dtype != q4.dtype or t.device != q4.device:
            raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, f"{name} does not match q")
    if lse.shape != (B, H, S) or lse.dtype != torch.float32 or lse.device != q4.device:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "lse must be float32 (B,H,S) on q's device")
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    if out is None:
        dq = torch.empty_like(q4, memory_format=torch.contiguous_format)
        dk = torch.empty_like(k4, memory_format=torch.contiguous_format)
        dv = torch.empty_like(v4, memory_format=torch.contiguous_format)
    else:
        dq, dk, dv = (_as4(t, "out") for t in out)
        for t in (dq, dk, dv):
            if t.shape != q4.shape or t.dtype != q4.dtype or t.device != q4.device:
                raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "out grads do not match q")
    kk = _keep(key_keep, B, S, q4.device)
    # the launch reads lse asynchronously: a contiguous copy must stay alive
    # (and out of the caching allocator) until it has been enqueued, or the
    # workspace allocated below could reuse its block
    lse_c = lse.contiguous()
    a = _abi.AttnBwdArgs(dtype=_dtype_code(q4), batch=B, seq=S, heads=H, head_dim=D, scale=scale,
                         q=_ptr(q4), k=_ptr(k4), v=_ptr(v4), o=_ptr(o4), dout=_ptr(do4),
                         lse=_ptr(lse_c), key_keep=_ptr(kk), dq=_ptr(dq), dk=_ptr(dk),
                         dv=_ptr(dv), q_stride=_strides(q4), k_stride=_strides(k4),
                         v_stride=_strides(v4), o_stride=_strides(o4), do_stride=_strides(do4),
                         dq_stride=_strides(dq), dk_stride=_strides(dk), dv_stride=_strides(dv))
    # a given workspace of at least the minimum is used as it is (below the
    # full size: dQ recomputes S and dP); none gets the full size (dQ reads
    # the dK/dV kernel's stored dS)
    need = lib().fa_attn_bwd_workspace_size(ctypes.byref(a))
    least = lib().fa_attn_bwd_min_workspace_size(ctypes.byref(a))
    if workspace is None or workspace.numel() * workspace.element_size() < least:
        if workspace is not None and phases is not None:
            # separate phase calls share the pre-pass rows through it
            raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG,
                                   f"workspace of {workspace.numel() * workspace.element_size()} bytes is "
                                   f"smaller than the {least} these shapes need")
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=q4.device)
    a.workspace = workspace.data_ptr()
    a.workspace_bytes = workspace.numel() * workspace.element_size()
    if phases is None:
        check(lib().fa_attn_bwd(ctypes.byref(a), _stream(q4)))
    else:
        for ph, st in phases:
            sp = _stream(q4) if st is None else st.cuda_stream
            check(lib().fa_attn_bwd_phase(ctypes.byref(a), int(ph), sp))
    del lse_c, kk  # enqueued: the stream orders any reuse of their blocks
    if squeeze:
        return dq[0], dk[0], dv[0]
    return dq, dk, dv


class AttnBwd:
    """Host mirror of foundry-spike's `AttnBwd` CustomOp3 (lib.rs:151-264).

    `fwd` takes the place of `cuda_fwd` (lib.rs:189-214) and `cpu_fwd`
    (lib.rs:158-187); `bwd` keeps the reference signature
    (q, k, v, res, grad_res) -> (dq, dk, dv) (lib.rs:216-263).  The forward's
    LSE is kept for the call that produced `res`: `bwd` reuses it only when
    it is handed that very `res` object and the same q, k, v (same storage,
    shape and strides), none of them modified since (tensor versions).
    Otherwise the forward is rerun to regenerate it, as the reference's
    backward recomputes its probabilities from q and k.  The slot is
    released once a backward has used it.

    Host (CPU) tensors take the `cpu_fwd` route as the Rust shim does: they
    must be contiguous with storage offset 0, as `cpu_fwd` requires
    (lib.rs:167-172); they are staged to the current GPU, the HIP kernels run
    there, and the results come back as host tensors (no CPU computation
    path exists).
    """

    def __init__(self, scale: Optional[float] = None, key_keep=None):
        self.scale = scale
        self.key_keep = key_keep
        self._saved = None  # (weakref to res, identity keys of q, k, v, res, lse on the device)

    @staticmethod
    def name() -> str:
        return lib().fa_op_name().decode()

    @staticmethod
    def _key(t: torch.Tensor):
        return (t.device, t.data_ptr(), tuple(t.shape), t.stride(), t._version)

    @staticmethod
    def _staged(*ts):
        dev = torch.device("cuda", torch.cuda.current_device())
        return tuple(t.to(dev) for t in ts)

    def fwd(self, q, k, v):
        host = not q.is_cuda
        if host:
            for name, t in (("q", q), ("k", k), ("v", v)):
                if t.is_cuda or not t.is_contiguous() or t.storage_offset() != 0:
                    raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG,
                                           f"cpu_fwd requires contiguous offset-0 host inputs ({name})")
            keys = tuple(self._key(t) for t in (q, k, v))
            q, k, v = self._staged(q, k, v)
        else:
            keys = tuple(self._key(t) for t in (q, k, v))
        o, lse = attn_fwd(q, k, v, self.scale, self.key_keep)
        if host:
            o = o.cpu()
        self._saved = (weakref.ref(o), keys + (self._key(o),), lse)
        return o

    def _saved_lse(self, q, k, v, res):
        if self._saved is None:
            return None
        ref, keys, lse = self._saved
        if ref() is not res or keys != tuple(self._key(t) for t in (q, k, v, res)):
            return None
        return lse

    def bwd(self, q, k, v, res, grad_res):
        lse = self._saved_lse(q, k, v, res)
        self._saved = None
        host = not q.is_cuda
        if host:
            q, k, v, res, grad_res = self._staged(q, k, v, res, grad_res)
        if lse is None:
            _, lse = attn_fwd(q, k, v, self.scale, self.key_keep)
        grads = attn_bwd(q, k, v, res, grad_res, lse, self.scale, self.key_keep)
        return tuple(g.cpu() for g in grads) if host else grads


class _AttentionFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, scale, key_keep):
        o, lse = attn_fwd(q, k, v, scale, key_keep)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.scale, ctx.key_keep = scale, key_keep
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = attn_bwd(q, k, v, o, do.contiguous(), lse, ctx.scale, ctx.key_keep)
        return dq, dk, dv, None, None


def attention(q, k, v, scale: Optional[float] = None, key_keep=None):
    """Differentiable joint attention: the analogue of q.apply_op3(&k, &v, AttnBwd)."""
    return _AttentionFn.apply(q, k, v, scale, key_keep)


# ---------------------------------------------------------------------------
# QK prologue
# ---------------------------------------------------------------------------
def rope_tables(positions, axes: Sequence[int], theta: float, dtype=torch.bfloat16,
                device="cuda") -> Tuple[torch.Tensor, torch.Tensor]:
    """cos, sin (n_pos, sum(axes)) exactly as rope_tables_dtype (lib.rs:77-105)."""
    pos = np.ascontiguousarray(np.asarray(positions, dtype=np.float32))
    n_pos, n_axes = pos.shape
    D = int(sum(axes))
    code = _DTYPES[dtype]
    np_dt = np.uint16 if code == _abi.FA_DTYPE_BF16 else np.float32
    cos = np.empty((n_pos, D), np_dt)
    sin = np.empty((n_pos, D), np_dt)
    ax = (ctypes.c_int32 * len(axes))(*[int(a) for a in axes])
    check(lib().fa_rope_tables_host(pos.ctypes.data, n_pos, n_axes, ctypes.addressof(ax),
                                    float(theta), code, cos.ctypes.data, sin.ctypes.data))
    if code == _abi.FA_DTYPE_BF16:
        c = torch.from_numpy(cos.view(np.int16)).view(torch.bfloat16)
        s = torch.from_numpy(sin.view(np.int16)).view(torch.bfloat16)
    else:
        c, s = torch.from_numpy(cos), torch.from_numpy(sin)
    return c.to(device), s.to(device)


def _prologue_args(x4, weight, cos, sin, axes, eps, y4, seq_offset) -> _abi.QkPrologueArgs:
    B, T, H, D = x4.shape
    if len(axes) > _abi.FA_MAX_ROPE_AXES:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "too many rope axes")
    ax = (ctypes.c_int32 * _abi.FA_MAX_ROPE_AXES)(*([int(a) for a in axes] +
                                                    [0] * (_abi.FA_MAX_ROPE_AXES - len(axes))))
    for name, t in (("weight", weight), ("cos", cos), ("sin", sin)):
        if t.dtype != x4.dtype or not t.is_contiguous() or t.device != x4.device:
            raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG,
                                   f"{name} must be a contiguous {x4.dtype} tensor on {x4.device}")
    if cos.shape != (T, D) or sin.shape != (T, D) or weight.shape != (D,):
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "weight/cos/sin shapes do not match x")
    return _abi.QkPrologueArgs(dtype=_dtype_code(x4), batch=B, tokens=T, heads=H, head_dim=D,
                               eps=float(eps), x=_ptr(x4), x_stride=_strides(x4),
                               weight=_ptr(weight), cos=_ptr(cos), sin=_ptr(sin),
                               n_axes=len(axes), axes=ax, y=_ptr(y4), y_stride=_strides(y4),
                               y_seq_offset=int(seq_offset))


def _prologue_fwd_args(x, weight, cos, sin, axes, eps, out, seq_offset):
    x4 = _as4(x, "x")
    B, T, H, D = x4.shape
    y4 = torch.empty((B, T, H, D), dtype=x4.dtype, device=x4.device) if out is None else _as4(out, "out")
    if y4.shape[0] != B or y4.shape[2:] != (H, D) or seq_offset + T > y4.shape[1] \
            or y4.dtype != x4.dtype or y4.device != x4.device or seq_offset < 0:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "out does not fit x at seq_offset")
    return _prologue_args(x4, weight, cos, sin, axes, eps, y4, seq_offset), x4, y4


def qk_prologue(x, weight, cos, sin, axes: Sequence[int], eps: float = 1e-6,
                out: Optional[torch.Tensor] = None, seq_offset: int = 0):
    """apply_rope(rms_norm(x, weight, eps), cos, sin) written to out[:, seq_offset:+T].

    x: (B,T,H,D) or (T,H,D) linear output (any row strides); out: the joint
    (B,S,H,D) buffer (allocated as (B,T,H,D) if None).  Returns out.
    """
    a, x4, y4 = _prologue_fwd_args(x, weight, cos, sin, axes, eps, out, seq_offset)
    check(lib().fa_qk_prologue_fwd(ctypes.byref(a), _stream(x4)))
    if out is None and x.dim() == 3:
        return y4[0]
    return out if out is not None else y4


def qk_prologue_multi(segments, eps: float = 1e-6):
    """Several qk_prologue calls in one launch (fa_qk_prologue_fwd_multi).

    segments: up to 4 tuples (x, weight, cos, sin, axes, out, seq_offset)
    sharing dtype and head_dim, e.g. Q and K of a block's txt and img
    streams; `out` is required.  Same results as the separate calls."""
    segs = [_prologue_fwd_args(x, w, c, s_, ax, eps, out, off) for (x, w, c, s_, ax, out, off) in segments]
    if not 1 <= len(segs) <= 4:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "1..4 segments")
    arr = (_abi.QkPrologueArgs * len(segs))(*[a for a, _, _ in segs])
    check(lib().fa_qk_prologue_fwd_multi(arr, len(segs), _stream(segs[0][1])))


def _prologue_bwd_args(x, weight, cos, sin, axes, dy, seq_offset, eps, dx):
    x4, dy4 = _as4(x, "x"), _as4(dy, "dy")
    B, T, H, D = x4.shape
    if dy4.shape[0] != B or dy4.shape[2:] != (H, D) or seq_offset + T > dy4.shape[1] \
            or dy4.dtype != x4.dtype or dy4.device != x4.device:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "dy does not fit x at seq_offset")
    if dx is None:
        dx = torch.empty(x4.shape, dtype=x4.dtype, device=x4.device)
    else:
        dx = _as4(dx, "dx")
        if dx.shape != x4.shape or dx.dtype != x4.dtype or dx.device != x4.device:
            raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "dx must match x")
    a = _abi.QkPrologueBwdArgs(fwd=_prologue_args(x4, weight, cos, sin, axes, eps, dy4, seq_offset),
                               dy=_ptr(dy4), dx=_ptr(dx), dx_stride=_strides(dx))
    return a, x4, dx


def qk_prologue_bwd(x, weight, cos, sin, axes: Sequence[int], dy, seq_offset: int = 0,
                    eps: float = 1e-6, dx: Optional[torch.Tensor] = None):
    """Gradient wrt x of qk_prologue, given dy wrt the joint buffer; written to
    `dx` (a view shaped like x, any row strides) when given."""
    a, x4, dx = _prologue_bwd_args(x, weight, cos, sin, axes, dy, seq_offset, eps, dx)
    check(lib().fa_qk_prologue_bwd(ctypes.byref(a), _stream(x4)))
    return dx[0] if x.dim() == 3 else dx


def qk_prologue_bwd_multi(segments, eps: float = 1e-6):
    """Several qk_prologue_bwd calls in one launch (fa_qk_prologue_bwd_multi).

    segments: up to 4 tuples (x, weight, cos, sin, axes, dy, seq_offset, dx)
    sharing dtype and head_dim; `dx` is required.  Same results as the
    separate calls."""
    segs = [_prologue_bwd_args(x, w, c, s_, ax, dy, off, eps, dx) for (x, w, c, s_, ax, dy, off, dx) in segments]
    if not 1 <= len(segs) <= 4:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "1..4 segments")
    arr = (_abi.QkPrologueBwdArgs * len(segs))(*[a for a, _, _ in segs])
    check(lib().fa_qk_prologue_bwd_multi(arr, len(segs), _stream(segs[0][1])))


# ---------------------------------------------------------------------------
# LoRA
# ---------------------------------------------------------------------------
def _lora_args(x, a, b, y, scale, u) -> _abi.LoraArgs:
    if x.dim() != 2 or a.dim() != 2 or b.dim() != 2:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "x, lora_a, lora_b must be 2-D")
    N, K = x.shape
    r = a.shape[0]
    M = b.shape[0]
    if a.shape != (r, K) or b.shape != (M, r):
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "lora_a must be [r,K], lora_b [M,r]")
    if x.stride(1) != 1 or not a.is_contiguous() or not b.is_contiguous():
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "x rows, lora_a, lora_b must be contiguous")
    if not (a.dtype == b.dtype == x.dtype) or not (a.device == b.device == x.device):
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "x, lora_a, lora_b dtypes/devices differ")
    if u.shape != (N, r) or u.dtype != torch.float32 or not u.is_contiguous():
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "u must be contiguous float32 [N, r]")
    if y is not None and (y.shape != (N, M) or y.stride(1) != 1 or y.dtype != x.dtype
                          or y.device != x.device):
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "y must be [N, M] with contiguous rows")
    return _abi.LoraArgs(dtype=_dtype_code(x), tokens=N, in_features=K, out_features=M, rank=r,
                         scale=float(scale), x=_ptr(x), ldx=x.stride(0), a=_ptr(a), b=_ptr(b),
                         u=_ptr(u), y=_ptr(y), ldy=0 if y is None else y.stride(0))


def lora_fwd(x, a, b, y, scale: float):
    """y += scale * (x a^T) b^T in place; returns u = x a^T (f32) for the backward."""
    u = torch.empty((x.shape[0], a.shape[0]), dtype=torch.float32, device=x.device)
    args = _lora_args(x, a, b, y, scale, u)
    check(lib().fa_lora_fwd(ctypes.byref(args), _stream(x)))
    return u


def lora_bwd(x, a, b, u, dy, scale: float, dx: Optional[torch.Tensor] = None):
    """(dA, dB) in f32 for the adapter term; dx += scale (dy b) a when given."""
    r, K = a.shape
    M = b.shape[0]
    N = x.shape[0]
    if dy.shape != (N, M) or dy.stride(1) != 1 or dy.dtype != x.dtype or dy.device != x.device:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "dy must be [N, M] with contiguous rows")
    if dx is not None and (dx.shape != (N, K) or dx.stride(1) != 1 or dx.dtype != x.dtype
                           or dx.device != x.device):
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "dx must be [N, K] with contiguous rows")
    da = torch.empty((r, K), dtype=torch.float32, device=x.device)
    db = torch.empty((M, r), dtype=torch.float32, device=x.device)
    args = _abi.LoraBwdArgs(fwd=_lora_args(x, a, b, None, scale, u), dy=_ptr(dy), ldy=dy.stride(0),
                            da=_ptr(da), db=_ptr(db), dx=_ptr(dx),
                            ldx=0 if dx is None else dx.stride(0))
    need = lib().fa_lora_bwd_workspace_size(ctypes.byref(args))
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=x.device)
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    check(lib().fa_lora_bwd(ctypes.byref(args), _stream(x)))
    return da, db


# ---------------------------------------------------------------------------
# adapter pieces around a base GEMM that carries the adapter (bf16)
# ---------------------------------------------------------------------------
def _rank_view(t: torch.Tensor, N: int, r: int, name: str, dev) -> torch.Tensor:
    if t.dim() != 2 or t.shape != (N, r) or t.stride(1) != 1 or t.dtype != torch.bfloat16 \
            or t.device != dev:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG,
                               f"{name} must be a bf16 [{N}, {r}] view with unit column stride on {dev}")
    return t


def _rows(t: torch.Tensor, name: str, dtype=None, dev=None) -> torch.Tensor:
    """A 2-D row view with unit column stride (the kernels read whole rows)."""
    if t.dim() != 2 or t.stride(1) != 1:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, f"{name} must be 2-D with unit column stride")
    if (dtype is not None and t.dtype != dtype) or (dev is not None and t.device != dev):
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, f"{name} must be {dtype} on {dev}")
    return t


def _factor(t: torch.Tensor, shape, name: str, like: torch.Tensor) -> torch.Tensor:
    if tuple(t.shape) != tuple(shape) or t.dtype != like.dtype or t.device != like.device:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG,
                               f"{name} must be {like.dtype} {list(shape)} on {like.device}")
    return t.contiguous()


def lora_down(x, a, scale: float, out: torch.Tensor):
    """out = scale * x a^T, bf16, into a [N, r] view (e.g. the extra K-columns
    of a GEMM operand).  x [N, K] bf16 rows, a [r, K]."""
    x = _rows(x, "x", torch.bfloat16)
    N, K = x.shape
    if a.dim() != 2:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "lora_a must be 2-D [r, K]")
    r = a.shape[0]
    a_c = _factor(a, (r, K), "lora_a", x)
    _rank_view(out, N, r, "out", x.device)
    args = _abi.LoraDownArgs(dtype=_dtype_code(x), tokens=N, in_features=K, rank=r, scale=float(scale),
                             x=_ptr(x), ldx=x.stride(0), a=_ptr(a_c), u=_ptr(out), ldu=out.stride(0))
    check(lib().fa_lora_down(ctypes.byref(args), _stream(x)))
    return out


def lora_up(u, b, y, scale: float):
    """y += scale * u b^T in place; u a bf16 [N, r] view, b [M, r], y [N, M]
    bf16 rows."""
    y = _rows(y, "y", torch.bfloat16)
    N, M = y.shape
    if b.dim() != 2:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "lora_b must be 2-D [M, r]")
    r = b.shape[1]
    b_c = _factor(b, (M, r), "lora_b", y)
    _rank_view(u, N, r, "u", y.device)
    args = _abi.LoraUpArgs(dtype=_dtype_code(y), tokens=N, out_features=M, rank=r, scale=float(scale),
                           u=_ptr(u), ldu=u.stride(0), b=_ptr(b_c), y=_ptr(y), ldy=y.stride(0))
    check(lib().fa_lora_up(ctypes.byref(args), _stream(y)))
    return y


def _lora_grad_args(u, x, scale: float, transpose: bool, out: Optional[torch.Tensor]):
    """Validated LoraGradArgs (no workspace yet) and the f32 output tensor."""
    x = _rows(x, "x", torch.bfloat16)
    N, C = x.shape
    if u.dim() != 2:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "u must be 2-D [N, r]")
    r = u.shape[1]
    _rank_view(u, N, r, "u", x.device)
    shape = (C, r) if transpose else (r, C)
    if out is None:
        g = torch.empty(shape, dtype=torch.float32, device=x.device)
    else:
        if tuple(out.shape) != shape or out.dtype != torch.float32 or not out.is_contiguous() \
                or out.device != x.device:
            raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG,
                                   f"out must be a contiguous float32 {list(shape)} tensor on {x.device}")
        g = out
    args = _abi.LoraGradArgs(dtype=_dtype_code(x), tokens=N, features=C, rank=r, scale=float(scale), u=_ptr(u),
                             ldu=u.stride(0), x=_ptr(x), ldx=x.stride(0), grad=_ptr(g), transpose=int(transpose))
    return args, g


def lora_grad(u, x, scale: float, transpose: bool, out: Optional[torch.Tensor] = None):
    """f32 scale * u^T x: [r, C] (lora_a layout) or, with transpose, [C, r]
    (lora_b layout).  u a bf16 [N, r] view, x [N, C] bf16 rows; `out`, when
    given, a contiguous f32 tensor of that shape on x's device."""
    args, g = _lora_grad_args(u, x, scale, transpose, out)
    need = lib().fa_lora_grad_workspace_size(ctypes.byref(args))
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=g.device)
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    check(lib().fa_lora_grad(ctypes.byref(args), _stream(g)))
    return g


def lora_grad_many(items):
    """Several lora_grad products, each of its own token count, in one set of
    launches: items are (u, x, scale, transpose) or (u, x, scale, transpose,
    out); the results (same bits as separate lora_grad calls) come back in
    order."""
    if not items:
        return []
    built = [_lora_grad_args(*it[:4], it[4] if len(it) > 4 else None) for it in items]
    dev = built[0][1].device
    if any(g.device != dev for _, g in built):
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "all products must be on one device")
    arr = (_abi.LoraGradArgs * len(built))(*[a for a, _ in built])
    need = lib().fa_lora_grad_many_workspace_size(arr, len(built))
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
    check(lib().fa_lora_grad_many(arr, len(built), ws.data_ptr(), ws.numel(), _stream(built[0][1])))
    return [g for _, g in built]
