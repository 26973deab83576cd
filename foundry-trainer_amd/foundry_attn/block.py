"""foundry-spike's double-stream LoRA block on the MI355X path (config c4).

Mirrors ``double_block`` (crates/foundry-spike/src/bin/throughput.rs:480-574)
and one training step of it (Session::step, throughput.rs:784-803: forward,
backward, adamw_step on the LoRA factors), with the c4 choices:
  - both streams' q, k, v and out projections carry LoRA (the reference's
    klein run trains the image stream only, throughput.rs:424-428);
  - the MLP is tanh-GELU with hidden 4 * dim (the reference block uses
    SwiGLU, lib.rs:293-297);
  - the upstream gradient is a given dY per stream (the seed trick,
    attn_backward.rs:220-222) instead of the MSE loss;
  - the frozen linears have no bias.
The same class also replays the reference's own double block
(crates/foundry-spike/src/lib.rs:301-392, the fixture block of
tools/fixtures/gen_block.py:199-240): frozen linears with biases, a SwiGLU
MLP (mlp="swiglu", lib.rs:293-297), LoRA on only some projections (the
fixture adapts the image stream's to_q and to_v), one modulation linear
shared by both streams, and the caller's RoPE positions.

Compute path: the memory-bound ops (layer_norm_mod and its backward, gated
residuals, GELU, the fused QK-RMSNorm + RoPE prologue, the LoRA adapters,
AdamW) and the joint attention run as libfoundry_attn.so kernels; the frozen
base linears are plain library GEMMs (torch.mm -> hipBLASLt), bf16 in, f32
accumulation, bf16 out.  In bf16 the adapters ride in those GEMMs as extra
K or N columns (DoubleBlockLoRA's fold options, SingleBlockLoRA's fused
adapters), and GraphedTrainStep captures either block's forward and
backward in one HIP graph.

With want_dx=False the backward forms exactly the gradients Candle's
autograd needs for the LoRA factors: nothing flows into the first
layer_norm_mod (its output feeds only frozen weights and the adapters), so no
dX is formed for the frozen qkv projection.  want_dx=True also forms the
block-input gradient, as a block inside a stack needs.
"""
from __future__ import annotations

import contextlib
import ctypes
import math
from dataclasses import dataclass, field
from typing import Dict, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _abi, gemm_tuning
from ._abi import FoundryAttnError, check, lib
from .ops import (_dtype_code, _ptr, _stream, attn_bwd, attn_bwd_workspace_bytes, attn_fwd, lora_bwd, lora_down,
                  lora_fwd, lora_grad,
                  lora_grad_many,
                  lora_up, qk_prologue_bwd_multi, qk_prologue_multi, rope_tables)


# ---------------------------------------------------------------------------
# block ops (include/foundry_block.h)
# ---------------------------------------------------------------------------
def _rows(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dim() != 2 or t.stride(1) != 1:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, f"{name} must be 2-D with contiguous rows")
    return t


def _vec(t: torch.Tensor, C: int, like: torch.Tensor, name: str) -> torch.Tensor:
    if t.shape != (C,) or not t.is_contiguous() or t.dtype != like.dtype or t.device != like.device:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, f"{name} must be a contiguous [{C}] {like.dtype}")
    return t


def _like(out: Optional[torch.Tensor], ref: torch.Tensor, name: str = "out") -> torch.Tensor:
    if out is None:
        return torch.empty_like(ref, memory_format=torch.contiguous_format)
    _rows(out, name)
    if out.shape != ref.shape or out.dtype != ref.dtype or out.device != ref.device:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, f"{name} must match {tuple(ref.shape)} {ref.dtype}")
    return out


def ln_mod_fwd(x, shift, scale, eps: float = 1e-6, out=None, stats: bool = False):
    """layer_norm_mod (lib.rs:60-71) over the rows of x [N, C]:
    y = (1 + scale) * LN(x) + shift.  With stats=True also returns the f32
    row mean and rstd the backward needs: (y, mean, rstd)."""
    x = _rows(x, "x")
    N, C = x.shape
    y = _like(out, x)
    mean = rstd = None
    if stats:
        mean = torch.empty(N, dtype=torch.float32, device=x.device)
        rstd = torch.empty(N, dtype=torch.float32, device=x.device)
    a = _abi.LnModArgs(dtype=_dtype_code(x), rows=N, cols=C, eps=float(eps), x=_ptr(x), ldx=x.stride(0),
                       shift=_ptr(_vec(shift, C, x, "shift")), scale=_ptr(_vec(scale, C, x, "scale")),
                       y=_ptr(y), ldy=y.stride(0), mean=_ptr(mean), rstd=_ptr(rstd))
    check(lib().fa_ln_mod_fwd(ctypes.byref(a), _stream(x)))
    return (y, mean, rstd) if stats else y


def ln_mod_bwd(x, dy, scale, mean, rstd, eps: float = 1e-6, dres=None, out=None):
    """dx = dres + d/dx layer_norm_mod(x)^T dy (shift / scale frozen)."""
    x, dy = _rows(x, "x"), _rows(dy, "dy")
    N, C = x.shape
    dx = _like(out, x)
    if dres is not None:
        _rows(dres, "dres")
    fwd = _abi.LnModArgs(dtype=_dtype_code(x), rows=N, cols=C, eps=float(eps), x=_ptr(x), ldx=x.stride(0),
                         shift=_ptr(_vec(scale, C, x, "scale")), scale=_ptr(_vec(scale, C, x, "scale")),
                         mean=_ptr(mean), rstd=_ptr(rstd))
    a = _abi.LnModBwdArgs(fwd=fwd, dy=_ptr(dy), lddy=dy.stride(0), dres=_ptr(dres),
                          ldres=0 if dres is None else dres.stride(0), dx=_ptr(dx), lddx=dx.stride(0))
    check(lib().fa_ln_mod_bwd(ctypes.byref(a), _stream(x)))
    return dx


def gated_ln_mod_fwd(x, g, b, shift, scale, eps: float = 1e-6, out=None, sum_out=None, sum_copy=None):
    """The gated residual s = x + g * b and layer_norm_mod(s) in one pass
    (throughput.rs:552-566): returns (s, y, mean, rstd), the bits of
    gated_residual followed by ln_mod_fwd(stats=True) on its output.
    sum_copy, when given, receives a second copy of s."""
    x = _rows(x, "x")
    N, C = x.shape
    b = _like(b, x, "b")
    s = _like(sum_out, x, "sum_out")
    y = _like(out, x)
    if sum_copy is not None:
        _like(sum_copy, x, "sum_copy")
    mean = torch.empty(N, dtype=torch.float32, device=x.device)
    rstd = torch.empty(N, dtype=torch.float32, device=x.device)
    ln = _abi.LnModArgs(dtype=_dtype_code(x), rows=N, cols=C, eps=float(eps), x=_ptr(x), ldx=x.stride(0),
                        shift=_ptr(_vec(shift, C, x, "shift")), scale=_ptr(_vec(scale, C, x, "scale")),
                        y=_ptr(y), ldy=y.stride(0), mean=_ptr(mean), rstd=_ptr(rstd))
    a = _abi.GatedLnModArgs(ln=ln, g=_ptr(_vec(g, C, x, "g")), b=_ptr(b), ldb=b.stride(0), sum=_ptr(s),
                            ldsum=s.stride(0), sum2=_ptr(sum_copy),
                            ldsum2=0 if sum_copy is None else sum_copy.stride(0))
    check(lib().fa_gated_ln_mod_fwd(ctypes.byref(a), _stream(x)))
    return s, y, mean, rstd


def ln_mod_bwd_gate(x, dy, scale, mean, rstd, g, eps: float = 1e-6, dres=None, out=None, gated_out=None):
    """ln_mod_bwd's dx and g * dx in one pass: returns (dx, g * dx), the bits
    of ln_mod_bwd followed by gated_residual(None, g, dx)."""
    x, dy = _rows(x, "x"), _rows(dy, "dy")
    N, C = x.shape
    dx = _like(out, x)
    gdx = _like(gated_out, x, "gated_out")
    if dres is not None:
        _rows(dres, "dres")
    fwd = _abi.LnModArgs(dtype=_dtype_code(x), rows=N, cols=C, eps=float(eps), x=_ptr(x), ldx=x.stride(0),
                         shift=_ptr(_vec(scale, C, x, "scale")), scale=_ptr(_vec(scale, C, x, "scale")),
                         mean=_ptr(mean), rstd=_ptr(rstd))
    bw = _abi.LnModBwdArgs(fwd=fwd, dy=_ptr(dy), lddy=dy.stride(0), dres=_ptr(dres),
                           ldres=0 if dres is None else dres.stride(0), dx=_ptr(dx), lddx=dx.stride(0))
    a = _abi.LnModBwdGateArgs(bwd=bw, g=_ptr(_vec(g, C, x, "g")), gdx=_ptr(gdx), ldgdx=gdx.stride(0))
    check(lib().fa_ln_mod_bwd_gate(ctypes.byref(a), _stream(x)))
    return dx, gdx


def _rows_op(fn, x, g, b, out):
    b = _rows(b, "b")
    N, C = b.shape
    y = _like(out, b)
    if x is not None:
        _rows(x, "x")
    a = _abi.RowsArgs(dtype=_dtype_code(b), rows=N, cols=C, x=_ptr(x), ldx=0 if x is None else x.stride(0),
                      g=_ptr(g), b=_ptr(b), ldb=b.stride(0), y=_ptr(y), ldy=y.stride(0))
    check(getattr(lib(), fn)(ctypes.byref(a), _stream(b)))
    return y


def gated_residual(x, g, b, out=None):
    """y = x + g * b (g [C] broadcast over rows); x None gives g * b."""
    return _rows_op("fa_gated_residual", x, _vec(g, b.shape[1], b, "g"), b, out)


def gelu(b, out=None):
    """tanh-GELU, elementwise."""
    return _rows_op("fa_gelu_fwd", None, None, b, out)


def gelu_bwd(dy, b, out=None):
    """dy * gelu'(b); out may be dy itself."""
    return _rows_op("fa_gelu_bwd", dy, None, b, out)


def silu(b, out=None):
    return _rows_op("fa_silu", None, None, b, out)


def gemm(a, w, epilogue: str = "plain", out=None, act_out=None, pre=None):
    """a [M, K] @ w[N, K]^T in bf16 with f32 accumulation (fa_gemm_bf16), one
    launch with a fused epilogue:
      "plain": returns bf16(a w^T);
      "gelu":  returns (pre, act), pre = bf16(a w^T), act = bf16(gelu(pre));
      "dgelu": returns bf16(bf16(a w^T) * gelu'(pre)) for the saved `pre`.
    M and N multiples of 256, K of 64; bf16 row views."""
    epi = {"plain": _abi.FA_GEMM_PLAIN, "gelu": _abi.FA_GEMM_GELU, "dgelu": _abi.FA_GEMM_DGELU}[epilogue]
    a, w = _rows(a, "a"), _rows(w, "w")
    M, K = a.shape
    N = w.shape[0]
    if w.shape[1] != K or a.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise ValueError("gemm: a [M, K] and w [N, K] must be bf16 with the same K")
    c = out if out is not None else torch.empty((M, N), dtype=a.dtype, device=a.device)
    c2 = None
    if epi == _abi.FA_GEMM_GELU:
        c2 = act_out if act_out is not None else torch.empty_like(c)
    if epi == _abi.FA_GEMM_DGELU and pre is None:
        raise ValueError("gemm: the dgelu epilogue needs the saved pre-activation")
    args = _abi.GemmArgs(epilogue=epi, m=M, n=N, k=K, a=_ptr(a), lda=a.stride(0), b=_ptr(w), ldb=w.stride(0),
                         c=_ptr(c), ldc=c.stride(0), c2=_ptr(c2), ldc2=0 if c2 is None else c2.stride(0),
                         aux=_ptr(pre), ldaux=0 if pre is None else pre.stride(0))
    check(lib().fa_gemm_bf16(ctypes.byref(args), _stream(a)))
    return (c, c2) if epi == _abi.FA_GEMM_GELU else c


def _same_rows(t: torch.Tensor, ref: torch.Tensor, name: str) -> torch.Tensor:
    _rows(t, name)
    if t.shape != ref.shape or t.dtype != ref.dtype or t.device != ref.device:
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, f"{name} must match {tuple(ref.shape)} {ref.dtype}")
    return t


def _swiglu_args(gate, up):
    gate = _rows(gate, "gate")
    _same_rows(up, gate, "up")
    N, C = gate.shape
    return _abi.SwigluArgs(dtype=_dtype_code(gate), rows=N, cols=C, gate=_ptr(gate), ldgate=gate.stride(0),
                           up=_ptr(up), ldup=up.stride(0))


def swiglu(gate, up, out=None):
    """silu(gate) * up (the activation of swiglu, lib.rs:293-297); gate and up
    may be column slices of one fused projection output."""
    a = _swiglu_args(gate, up)
    y = _like(out, gate)
    a.y, a.ldy = _ptr(y), y.stride(0)
    check(lib().fa_swiglu_fwd(ctypes.byref(a), _stream(gate)))
    return y


def swiglu_bwd(dy, gate, up, dgate=None, dup=None):
    """(dgate, dup) of silu(gate) * up for the upstream gradient dy."""
    fwd = _swiglu_args(gate, up)
    _same_rows(dy, gate, "dy")
    dg, du = _like(dgate, gate, "dgate"), _like(dup, gate, "dup")
    a = _abi.SwigluBwdArgs(fwd=fwd, dy=_ptr(dy), lddy=dy.stride(0), dgate=_ptr(dg), lddgate=dg.stride(0),
                           dup=_ptr(du), lddup=du.stride(0))
    check(lib().fa_swiglu_bwd(ctypes.byref(a), _stream(gate)))
    return dg, du


def adamw_step(param, grad, m, v, step: int, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8):
    """adamw_step (lib.rs:477-510) in place on param (bf16/f32) with f32 grad,
    m, v of the same number of elements."""
    n = param.numel()
    for name, t in (("grad", grad), ("m", m), ("v", v)):
        if t.numel() != n or t.dtype != torch.float32 or not t.is_contiguous() or t.device != param.device:
            raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, f"{name} must be contiguous float32 like param")
    if not param.is_contiguous():
        raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "param must be contiguous")
    a = _abi.AdamwArgs(dtype=_dtype_code(param), n=n, param=_ptr(param), grad=_ptr(grad), m=_ptr(m),
                       v=_ptr(v), lr=float(lr), beta1=float(betas[0]), beta2=float(betas[1]), eps=float(eps),
                       step=int(step))
    check(lib().fa_adamw_step(ctypes.byref(a), _stream(param)))


def adamw_step_many(items, step: int, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8):
    """adamw_step over several (param, grad, m, v) of one step in one call
    (fa_adamw_step_many: up to 32 tensors per launch, the bits of separate
    adamw_step calls).  The params share a dtype and a device."""
    items = list(items)
    if not items:
        return
    arr = (_abi.AdamwArgs * len(items))()
    for i, (param, grad, m, v) in enumerate(items):
        n = param.numel()
        for name, t in (("grad", grad), ("m", m), ("v", v)):
            if t.numel() != n or t.dtype != torch.float32 or not t.is_contiguous() or t.device != param.device:
                raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, f"{name} must be contiguous float32 like param")
        if not param.is_contiguous() or param.device != items[0][0].device:
            raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "params must be contiguous on one device")
        arr[i] = _abi.AdamwArgs(dtype=_dtype_code(param), n=n, param=_ptr(param), grad=_ptr(grad), m=_ptr(m),
                                v=_ptr(v), lr=float(lr), beta1=float(betas[0]), beta2=float(betas[1]),
                                eps=float(eps), step=int(step))
    check(lib().fa_adamw_step_many(arr, len(items), _stream(items[0][0])))


def _set_mod(old, parts):
    """New modulation parts, written into the old tensors when their shapes
    match (a captured GraphedTrainStep reads those addresses)."""
    parts = [t.contiguous() for t in parts]
    if len(old) == len(parts) and all(o.shape == p.shape and o.dtype == p.dtype for o, p in zip(old, parts)):
        for o, p in zip(old, parts):
            o.copy_(p)
        return old
    return tuple(parts)


def copy2d_many(pairs):
    """dst.copy_(src) for several (src, dst) pairs of 2-D views of one dtype
    (any strides, no overlaps) in one launch per 32 views (fa_copy2d_many)."""
    pairs = list(pairs)
    if not pairs:
        return
    dev = pairs[0][1].device
    if dev.type == "cpu":
        # a block built in host memory only to read or write adapter files
        # (its compute ops refuse host tensors): plain host copies
        for src, dst in pairs:
            dst.copy_(src)
        return
    arr = (_abi.Copy2dArgs * len(pairs))()
    for i, (src, dst) in enumerate(pairs):
        if src.dim() != 2 or src.shape != dst.shape or src.dtype != dst.dtype or src.device != dev \
                or dst.device != dev:
            raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "copy2d_many: pairs of equal-shape 2-D views "
                                                            "of one dtype on one device")
        arr[i] = _abi.Copy2dArgs(dtype=_dtype_code(src), rows=src.shape[0], cols=src.shape[1], src=_ptr(src),
                                 src_rs=src.stride(0), src_cs=src.stride(1), dst=_ptr(dst), dst_rs=dst.stride(0),
                                 dst_cs=dst.stride(1))
    check(lib().fa_copy2d_many(arr, len(pairs), _stream(pairs[0][1])))


# ---------------------------------------------------------------------------
# the block
# ---------------------------------------------------------------------------
LORA_TARGETS = ("q", "k", "v", "out")
QKV = ("q", "k", "v")
STREAMS = ("txt", "img")  # joint order: txt first (throughput.rs:545-547)
# Host issue order of the two streams' ops between the joint attention calls:
# img's rows (8x txt's at c4) are the critical path, so its launches go first
# and the GPU starts on them while the host issues txt's on the side stream.
# Under HIP-graph capture there is no host issue time to hide, and the graph
# dispatches its nodes in capture order: txt's short ops go first there, so
# that img's long GEMMs do not hold every CU while txt's wait (measured at c4:
# about 30 us per replay).
ISSUE_ORDER = ("img", "txt")
CAPTURE_ORDER = ("txt", "img")


@dataclass
class StreamWeights:
    """Frozen weights of one stream (torch tensors, compute dtype) and its
    LoRA factors with their AdamW moments.

    MLP: tanh-GELU (the block's mlp="gelu"): w1 [F, C], w2 [C, F];
    SwiGLU (mlp="swiglu", lib.rs:293-297): w1 [2M, C] = gate rows then up
    rows, w2 [C, M] = down.  Biases are optional (None: no bias, as klein's
    linears; the reference fixture has one on every linear).  LoRA factors
    exist only for the targets in lora_a / lora_b."""
    w_qkv: torch.Tensor   # [3C, C]: to_q, to_k, to_v stacked
    w_out: torch.Tensor   # [C, C]
    w1: torch.Tensor      # [F, C] (gelu) or [2M, C] (swiglu: gate | up)
    w2: torch.Tensor      # [C, F] (gelu) or [C, M] (swiglu: down)
    q_norm: torch.Tensor  # [D]
    k_norm: torch.Tensor  # [D]
    w_mod: torch.Tensor   # [6C, C]: shift1, scale1, gate1, shift2, scale2, gate2
    lora_a: Dict[str, torch.Tensor] = field(default_factory=dict)  # [r, in]
    lora_b: Dict[str, torch.Tensor] = field(default_factory=dict)  # [out, r]
    m: Dict[str, torch.Tensor] = field(default_factory=dict)
    v: Dict[str, torch.Tensor] = field(default_factory=dict)
    mod: Tuple[torch.Tensor, ...] = ()
    b_qkv: Optional[torch.Tensor] = None  # [3C]
    b_out: Optional[torch.Tensor] = None  # [C]
    b1: Optional[torch.Tensor] = None     # [F] or [2M]
    b2: Optional[torch.Tensor] = None     # [C]
    b_mod: Optional[torch.Tensor] = None  # [6C]


def _linear(x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor], out: torch.Tensor) -> torch.Tensor:
    """out = x w^T (+ b): one library GEMM, the bias in its epilogue."""
    if b is None:
        return torch.mm(x, w.t(), out=out)
    return torch.addmm(b, x, w.t(), out=out)


class DoubleBlockLoRA:
    """One double-stream block with LoRA on q/k/v/out of both streams.

    heads * head_dim = dim; img tokens lie on an (img_rows, img_cols) grid,
    txt tokens get positions (l, 0, 0), img tokens (0, r, c)
    (throughput.rs:724-748).

    batch_qkv_adapters (bf16, 3r <= 64): the q, k and v adapters of a stream
    read the same h, so their A factors are stacked into one [3r, C] tensor
    (lora_a[t] become row views of it) and every product that contracts or
    expands over h runs once at rank 3r -- s u = s h A^T, dh += s t A_qkv
    and dA = s t^T h.  The block-diagonal ones (the three up projections and
    t_j = dy_j B_j) ride in the qkv GEMMs with fold_qkv_adapters (see
    __init__), or stay per adapter without; the dB_j are formed with dA in
    one grouped launch set.  u and t are rounded to bf16 as the reference's
    bf16 matmuls round them.
    """

    def __init__(self, weights: Dict[str, StreamWeights], heads: int, head_dim: int, txt_tokens: int,
                 img_rows: int, img_cols: int, axes: Sequence[int] = (16, 56, 56), theta: float = 1e4,
                 lora_scale: float = 1.0, eps: float = 1e-6, overlap_streams: bool = True,
                 tuned_gemms: bool = True, batch_qkv_adapters: bool = True, mlp: str = "gelu",
                 positions: Optional[np.ndarray] = None, dx_weights_t: bool = True,
                 fold_qkv_adapters: bool = True, fold_mlp_gate: bool = True, fused_gelu=False):
        """positions: [S, n_axes] RoPE position ids of the joint sequence (txt
        rows first); None gives txt (l, 0, 0), img (0, r, c).

        dx_weights_t: keep a transposed copy of each frozen linear weight, so
        that the backward's dX = dY W reads W with the contraction dimension
        contiguous, the operand layout the library GEMMs run fastest on (the
        forward's x W^T already reads it that way).  Costs one more copy of
        the frozen weights (12 C^2 values per stream for the GELU MLP); call
        refresh_frozen() after changing a frozen weight.

        fold_qkv_adapters (with the batched q/k/v adapters): the three
        adapters ride in the frozen qkv GEMM, as ADAPTER_PAD extra columns of
        its weight [W_qkv | B_blk | 0], B_blk [3C, 3r] block-diagonal with
        B_q, B_k, B_v.  Forward: [h | s u | 0] [W_qkv | B_blk | 0]^T = h W_qkv^T
        + s u_j B_j^T for each of q, k, v, in one GEMM (no separate up
        projections).  Backward with the input gradient: dY [W_qkv | B_blk | 0]
        = [dY W_qkv | t | 0], t_j = dY_j B_j, in one GEMM (no separate
        t_j products).  Each output is one f32 sum rounded once, where the
        unfolded path rounds the base product and the adapter sum apart.
        With out adapters on both streams the out projection folds the same
        way: a [W_out; A_out; 0]^T = [out | u | 0] (then out += s u B_out^T),
        and [dout | s dout B_out | 0] [W_out; A_out; 0] = dout W_out + du A_out
        gives dO.

        fold_mlp_gate (no MLP output bias): the MLP's gate g2 (a per-channel
        modulation, fixed by set_conditioning) scales the rows of W2 once,
        W2g = diag(g2) W2.  Then y = x1 + act W2g^T is one GEMM with x1 as its
        accumulator input, and the backward's dact = (g2 * dy) W2 = dy W2g
        needs no separate g2 * dy pass.

        fused_gelu (GELU MLP, bf16, no W1 bias, token and MLP widths multiples
        of 256): W1's forward and W2's dX product run as this library's GEMM
        (fa_gemm_bf16) with the GELU and GELU-gradient epilogues, in place of
        the library GEMM followed by a separate GELU / GELU-backward pass.
        The backward's operand is W2's (or W2g's) transposed copy, so it also
        needs dx_weights_t.  True fuses both streams; an iterable of stream
        names ("img", "txt") fuses only those."""
        if mlp not in ("gelu", "swiglu"):
            raise ValueError(f"mlp must be 'gelu' or 'swiglu', not {mlp!r}")
        self.w = weights
        self.mlp = mlp
        self.H, self.D = heads, head_dim
        self.C = heads * head_dim
        self.T, self.I = txt_tokens, img_rows * img_cols
        self.S = self.T + self.I
        self.axes = tuple(int(a) for a in axes)
        self.lora_scale = float(lora_scale)
        self.eps = float(eps)
        self.attn_scale = 1.0 / math.sqrt(head_dim)
        ref = weights["img"].w_qkv
        self.dtype, self.device = ref.dtype, ref.device
        # capture: None, or a dict the forward and backward fill with copies
        # of their intermediates (for replaying a fixture's activations)
        self.capture: Optional[Dict[str, torch.Tensor]] = None
        if positions is None:
            pos = np.zeros((self.S, 3), np.float32)
            pos[:self.T, 0] = np.arange(self.T)
            rr, cc = np.meshgrid(np.arange(img_rows), np.arange(img_cols), indexing="ij")
            pos[self.T:, 1] = rr.ravel()
            pos[self.T:, 2] = cc.ravel()
        else:
            pos = np.asarray(positions, np.float32)
            if pos.shape != (self.S, len(self.axes)):
                raise ValueError(f"positions must be [{self.S}, {len(self.axes)}], got {pos.shape}")
        cos, sin = rope_tables(pos, self.axes, theta, dtype=self.dtype, device=self.device)
        self.rope = {"txt": (cos[:self.T].contiguous(), sin[:self.T].contiguous()),
                     "img": (cos[self.T:].contiguous(), sin[self.T:].contiguous())}
        self.offset = {"txt": 0, "img": self.T}
        self.rows = {"txt": self.T, "img": self.I}
        self.step_count = 0
        self._buf = None
        self._side = torch.cuda.Stream(device=self.device) if overlap_streams else None
        self._wt = {name: {} for name in STREAMS} if dx_weights_t else None
        self._fold_g2 = fold_mlp_gate and all(weights[name].b2 is None for name in STREAMS)
        self._w2g, self._w2g_t = {}, {}
        self._fused_gelu = ({"img", "txt"} if fused_gelu is True else set(fused_gelu) if fused_gelu else set())
        if tuned_gemms and self.dtype == torch.bfloat16:
            gemm_tuning.enable()
        ranks = {int(a.shape[0]) for w in weights.values() for a in w.lora_a.values()}
        if len(ranks) > 1:
            raise ValueError(f"LoRA factors of one block share a rank, got {sorted(ranks)}")
        self.rank = ranks.pop() if ranks else 0
        full_qkv = all(t in weights[name].lora_a for name in STREAMS for t in QKV)
        self._batched = (batch_qkv_adapters and full_qkv and self.dtype == torch.bfloat16
                         and 3 * self.rank <= 64)
        if self._batched:
            r = self.rank
            self._a_qkv, self._a_qkv_t, self._b_qkv, self._b_qkv_t, self._b_t = {}, {}, {}, {}, {}
            for name in STREAMS:
                w = weights[name]
                # A_q|A_k|A_v as one [3r, C] tensor and B_q|B_k|B_v as one
                # [3, C, r] tensor; lora_a[t] / lora_b[t] are views of them
                # (AdamW updates the stacks in place)
                a = torch.cat([w.lora_a[t] for t in QKV]).contiguous()
                b = torch.stack([w.lora_b[t] for t in QKV]).contiguous()
                for j, t in enumerate(QKV):
                    w.lora_a[t] = a[j * r:(j + 1) * r]
                    w.lora_b[t] = b[j]
                self._a_qkv[name], self._b_qkv[name] = a, b
                self._a_qkv_t[name] = torch.empty((a.shape[1], 3 * r), dtype=a.dtype, device=a.device)
                bt = torch.empty((3, r, b.shape[1]), dtype=a.dtype, device=a.device)
                self._b_qkv_t[name] = bt
                self._b_t[name] = {t: bt[j] for j, t in enumerate(QKV)}
        self._fold = self._batched and fold_qkv_adapters and 3 * self.rank <= ADAPTER_PAD
        if self._fold:
            C, r, P = self.C, self.rank, ADAPTER_PAD
            kw = dict(dtype=self.dtype, device=self.device)
            self._qkv_ext, self._qkv_ext_t, self._bview, self._bview_t = {}, {}, {}, {}
            for name in STREAMS:
                ext = torch.zeros((3 * C, C + P), **kw)  # [W_qkv | B_blk | 0]
                self._qkv_ext[name] = ext
                # B_j [C, r] at rows jC.., columns C + jr..: one strided [3, C, r] view
                self._bview[name] = ext.as_strided((3, C, r), (C * (C + P) + r, C + P, 1), C)
                if self._wt is not None:  # its transpose [C + P, 3C], the backward's operand
                    ext_t = torch.zeros((C + P, 3 * C), **kw)
                    self._qkv_ext_t[name] = ext_t
                    self._bview_t[name] = ext_t.as_strided((3, C, r), (3 * C * r + C, 1, 3 * C), 3 * C * C)
        self._fold_out = self._fold and all("out" in weights[name].lora_a for name in STREAMS)
        if self._fold_out:
            C, r, P = self.C, self.rank, ADAPTER_PAD
            kw = dict(dtype=self.dtype, device=self.device)
            self._out_ext, self._out_ext_t, self._b_out_t, self._b_out_ext = {}, {}, {}, {}
            for name in STREAMS:
                self._out_ext[name] = torch.zeros((C + P, C), **kw)   # [W_out; A_out; 0]
                if self._wt is not None:
                    self._out_ext_t[name] = torch.zeros((C, C + P), **kw)
                self._b_out_t[name] = torch.empty((r, C), **kw)       # B_out^T: du = s dout B_out
                self._b_out_ext[name] = None if weights[name].b_out is None else torch.zeros(C + P, **kw)
        self.refresh_frozen()
        if self._batched:
            self.refresh_adapters()

    def refresh_frozen(self) -> None:
        """Re-derive, in place, every operand formed from the frozen weights:
        the extended (adapter-carrying) GEMM operands, the gate-folded W2g,
        and the transposed copies the backward reads (with dx_weights_t)."""
        C = self.C
        self._refresh_w2g()
        for name in STREAMS:
            w = self.w[name]
            if self._fold:
                self._qkv_ext[name][:, :C].copy_(w.w_qkv)
                if self._wt is not None:
                    self._qkv_ext_t[name][:C].copy_(w.w_qkv.t())
            if self._fold_out:
                self._out_ext[name][:C].copy_(w.w_out)
                if self._wt is not None:
                    self._out_ext_t[name][:, :C].copy_(w.w_out.t())
                if w.b_out is not None:
                    self._b_out_ext[name][:C].copy_(w.b_out)
        if self._wt is None:
            return
        folded = (("w_qkv",) if self._fold else ()) + (("w_out",) if self._fold_out else ()) + \
            (("w2",) if self._fold_g2 else ())
        for name in STREAMS:
            w = self.w[name]
            for key in (k for k in ("w_qkv", "w_out", "w1", "w2") if k not in folded):
                src = getattr(w, key)
                dst = self._wt[name].get(key)
                if dst is None or dst.shape != (src.shape[1], src.shape[0]):
                    self._wt[name][key] = src.t().contiguous()
                else:
                    dst.copy_(src.t())

    def _refresh_w2g(self) -> None:
        """W2g = diag(g2) W2 per stream (and its transpose with dx_weights_t),
        once the modulation is known; rounded once from the f32 product."""
        if not self._fold_g2:
            return
        for name in STREAMS:
            w = self.w[name]
            if len(w.mod) < 6:
                continue
            w2g = (w.w2.float() * w.mod[5].float()[:, None]).to(self.dtype)
            if name in self._w2g and self._w2g[name].shape == w2g.shape:
                self._w2g[name].copy_(w2g)  # in place: a captured step reads this address
            else:
                self._w2g[name] = w2g
            if self._wt is not None:
                if name in self._w2g_t and self._w2g_t[name].shape == (w2g.shape[1], w2g.shape[0]):
                    self._w2g_t[name].copy_(w2g.t())
                else:
                    self._w2g_t[name] = w2g.t().contiguous()

    def _gelu_fused(self, name: str, backward: bool) -> bool:
        """Whether stream `name`'s MLP runs W1 (forward) or W2's dX product
        (backward) as fa_gemm_bf16 with the GELU epilogue."""
        w = self.w[name]
        ok = (name in self._fused_gelu and self.mlp == "gelu" and self.dtype == torch.bfloat16 and w.b1 is None
              and self.rows[name] % 256 == 0 and w.w1.shape[0] % 256 == 0 and self.C % 64 == 0)
        return ok and (not backward or self._wt is not None)

    def _dx_weight(self, name: str, key: str) -> torch.Tensor:
        """W of stream `name` as the right operand of dX = dY W."""
        if self._wt is None:
            return getattr(self.w[name], key)
        return self._wt[name][key].t()

    def refresh_adapters(self) -> None:
        """Re-derive what the batched adapter products read from the LoRA
        factors: the stacked A_qkv and B_qkv, A_qkv^T (for dh += s t A_qkv),
        the B_j^T (for t_j = dy_j B_j) and, with folded adapters, the factor
        columns of the qkv and out GEMM operands (and their transposes) -- in
        one fa_copy2d_many launch for both streams.
        apply_adamw calls it; call it after changing lora_a / lora_b any other
        way (loading a LoRA file: a tensor assigned to lora_a[t] or lora_b[t]
        is copied into its stack and replaced by its view)."""
        if not self._batched:
            return
        r = self.rank
        pairs = []
        for name in STREAMS:
            w, a, b = self.w[name], self._a_qkv[name], self._b_qkv[name]
            for j, t in enumerate(QKV):
                view = a[j * r:(j + 1) * r]
                if w.lora_a[t].data_ptr() != view.data_ptr():
                    view.copy_(w.lora_a[t])
                    w.lora_a[t] = view
                if w.lora_b[t].data_ptr() != b[j].data_ptr():
                    b[j].copy_(w.lora_b[t])
                    w.lora_b[t] = b[j]
            pairs.append((a.t(), self._a_qkv_t[name]))
            for j in range(len(QKV)):
                pairs.append((b[j].t(), self._b_qkv_t[name][j]))
                if self._fold:
                    pairs.append((b[j], self._bview[name][j]))
                    if self._wt is not None:
                        pairs.append((b[j], self._bview_t[name][j]))
            if self._fold_out:
                C = self.C
                pairs.append((w.lora_a["out"], self._out_ext[name][C:C + r]))
                if self._wt is not None:
                    pairs.append((w.lora_a["out"].t(), self._out_ext_t[name][:, C:C + r]))
                pairs.append((w.lora_b["out"].t(), self._b_out_t[name]))
        copy2d_many(pairs)  # one launch for every derived operand of both streams

    # -- conditioning: computed once per run (throughput.rs:936-938) -------
    def set_conditioning(self, c: torch.Tensor) -> None:
        """Modulation parts chunk6(silu(c) W_mod^T) per stream."""
        sc = silu(c.reshape(1, -1))
        for name in STREAMS:
            w = self.w[name]
            m = torch.empty((1, w.w_mod.shape[0]), dtype=self.dtype, device=self.device)
            _linear(sc, w.w_mod, w.b_mod, m)
            w.mod = _set_mod(w.mod, m.reshape(-1).split(self.C))
        self._refresh_w2g()

    def _buffers(self):
        if self._buf is None:
            C, S, H, D = self.C, self.S, self.H, self.D
            F = self.w["img"].w1.shape[0]        # pre-activation width (gelu F, swiglu 2M)
            FA = self.w["img"].w2.shape[1]       # activation width (gelu F, swiglu M)
            R = max(3 * self.rank, 1)
            kw = dict(dtype=self.dtype, device=self.device)
            b = {"qkv": torch.empty((S, 3 * C), **kw), "dqkv": torch.empty((S, 3 * C), **kw),
                 "q": torch.empty((1, S, H, D), **kw), "k": torch.empty((1, S, H, D), **kw),
                 "o": torch.empty((1, S, H, D), **kw), "do": torch.empty((1, S, H, D), **kw),
                 "dq": torch.empty((1, S, H, D), **kw), "dk": torch.empty((1, S, H, D), **kw),
                 "lse": torch.empty((1, H, S), dtype=torch.float32, device=self.device),
                 "ws": torch.empty(attn_bwd_workspace_bytes(1, S, H, D, self.dtype), dtype=torch.uint8,
                                  device=self.device)}
            for name in STREAMS:
                n = self.rows[name]
                for key, width in (("h", C), ("out", C), ("x1", C), ("h2", C), ("y", C), ("t1", C),
                                   ("t2", C), ("dx1", C), ("dx", C), ("pre", F), ("act", FA), ("dact", FA),
                                   ("dpre", F), ("mlp", C), ("su", R), ("tq", R)):
                    b[f"{key}.{name}"] = torch.empty((n, width), **kw)
                if self._fold:
                    # [h | s u | 0]: the padding columns stay zero
                    b[f"hx.{name}"] = torch.zeros((n, C + ADAPTER_PAD), **kw)
                    b[f"dhx.{name}"] = torch.empty((n, C + ADAPTER_PAD), **kw)
                if self._fold_out:
                    b[f"ox.{name}"] = torch.empty((n, C + ADAPTER_PAD), **kw)   # [out | u | 0]
                    b[f"dox.{name}"] = torch.zeros((n, C + ADAPTER_PAD), **kw)  # [dout | du | 0]
            self._buf = b
        return self._buf

    def forward(self, x: Dict[str, torch.Tensor], keep_attention: bool = False):
        """Block outputs y[stream] only (the detached forward of a checkpointed
        stack).  keep_attention also returns copies of the joint attention
        output and its LSE, (O, LSE), which forward_backward can reuse."""
        y, att = self._run(x, None, False, None, keep_attention)
        return (y, att) if keep_attention else y

    def forward_backward(self, x: Dict[str, torch.Tensor], dy: Dict[str, torch.Tensor], want_dx: bool = False,
                         attention=None):
        """Block outputs y[stream] and the f32 LoRA gradients
        grads[(stream, target)] = (dA, dB) for upstream gradients dy.

        want_dx=False forms what one block's LoRA factors need (Candle's
        autograd stops at the first layer_norm_mod, whose input tracks no
        variable); want_dx=True also forms the input gradients of a block
        inside a stack (dX through the frozen qkv projection and the first
        layer_norm_mod), returned as grads[(stream, "x")].  attention: the
        (O, LSE) a forward(keep_attention=True) of the same x returned; the
        attention forward is then skipped (the backward takes P from the LSE)."""
        return self._run(x, dy, want_dx, attention, False)

    # -- txt / img overlap ----------------------------------------------
    # Between the joint attention calls the two streams touch disjoint rows
    # of the joint buffers, so the txt stream's ops run on a second HIP
    # stream (default priority) beside the img stream's, joined by events.
    def _fork(self):
        if self._side is not None:
            self._side.wait_stream(torch.cuda.current_stream(self.device))

    def _join(self):
        if self._side is not None:
            torch.cuda.current_stream(self.device).wait_stream(self._side)

    def _on(self, name):
        if self._side is not None and name == "txt":
            return torch.cuda.stream(self._side)
        return contextlib.nullcontext()

    def _qkv_phase(self, name, x, saved):
        """layer_norm_mod -> frozen fused qkv + three adapters (the prologue of
        all four Q / K segments follows in one launch, _prologue_fwd)."""
        B, C, H, D, s = self._buf, self.C, self.H, self.D, self.lora_scale
        w, off, n = self.w[name], self.offset[name], self.rows[name]
        rows = B["qkv"][off:off + n]
        if self._fold:
            hx, r = B[f"hx.{name}"], self.rank
            h, mean1, rstd1 = ln_mod_fwd(x[name], w.mod[0], w.mod[1], self.eps, out=hx[:, :C], stats=True)
            saved[(name, "ln1")] = (mean1, rstd1)
            lora_down(h, self._a_qkv[name], s, out=hx[:, C:C + 3 * r])  # s h A_qkv^T
            _linear(hx, self._qkv_ext[name], w.b_qkv, rows)
            if self.capture is not None:
                self.capture[f"{name}_norm1"] = h.clone()
            return
        h, mean1, rstd1 = ln_mod_fwd(x[name], w.mod[0], w.mod[1], self.eps, out=B[f"h.{name}"], stats=True)
        saved[(name, "ln1")] = (mean1, rstd1)
        _linear(h, w.w_qkv, w.b_qkv, rows)
        if self._batched:
            r = self.rank
            su = lora_down(h, self._a_qkv[name], s, out=B[f"su.{name}"])  # [n, 3r] = s h A_qkv^T
            for j, t in enumerate(QKV):
                lora_up(su[:, j * r:(j + 1) * r], w.lora_b[t], rows[:, j * C:(j + 1) * C], 1.0)
        else:
            for j, t in enumerate(QKV):
                if t in w.lora_a:
                    saved[(name, t)] = lora_fwd(h, w.lora_a[t], w.lora_b[t], rows[:, j * C:(j + 1) * C], s)
        if self.capture is not None:
            self.capture[f"{name}_norm1"] = h.clone()

    def _prologue_segments(self, bwd: bool):
        """Q and K of both streams as the four segments of one fused
        RMSNorm + RoPE launch (forward: into the joint Q / K buffers;
        backward: dQ / dK of the joint buffers into the dqkv rows)."""
        B, C, H, D = self._buf, self.C, self.H, self.D
        segs = []
        for name in STREAMS:
            w, off, n = self.w[name], self.offset[name], self.rows[name]
            rows, drows = B["qkv"][off:off + n], B["dqkv"][off:off + n]
            cos, sin = self.rope[name]
            for j, (wn, dst, grad) in enumerate(((w.q_norm, "q", "dq"), (w.k_norm, "k", "dk"))):
                x = rows[:, j * C:(j + 1) * C].view(1, n, H, D)
                if bwd:
                    segs.append((x, wn, cos, sin, self.axes, B[grad], off,
                                 drows[:, j * C:(j + 1) * C].view(1, n, H, D)))
                else:
                    segs.append((x, wn, cos, sin, self.axes, B[dst], off))
        return segs

    def _prologue_fwd(self):
        B = self._buf
        qk_prologue_multi(self._prologue_segments(False), self.eps)
        if self.capture is not None:
            for name in STREAMS:
                off, n = self.offset[name], self.rows[name]
                self.capture[f"{name}.q"] = B["q"][0, off:off + n].clone()
                self.capture[f"{name}.k"] = B["k"][0, off:off + n].clone()

    def _out_phase(self, name, x, dy, o_t, y, saved, grads):
        """Out projection, gated residuals, MLP; with dy, the backward down to dO."""
        B, C, s = self._buf, self.C, self.lora_scale
        w, off, n = self.w[name], self.offset[name], self.rows[name]
        sh2, sc2, g1, g2 = w.mod[3], w.mod[4], w.mod[2], w.mod[5]
        a = o_t[0, off:off + n].reshape(n, C)
        if self._fold_out:
            ox, r = B[f"ox.{name}"], self.rank
            _linear(a, self._out_ext[name], self._b_out_ext[name], ox)  # [out | u | 0]
            out, u_out = ox[:, :C], ox[:, C:C + r]
            lora_up(u_out, w.lora_b["out"], out, s)
        else:
            out = _linear(a, w.w_out, w.b_out, B[f"out.{name}"])
            u_out = lora_fwd(a, w.lora_a["out"], w.lora_b["out"], out, s) if "out" in w.lora_a else None
        # the gated residual and the second layer norm in one pass; with the
        # MLP gate folded into W2, x1 also lands in y, which the W2 GEMM then
        # accumulates into in place (no separate copy of x1)
        yb = B[f"y.{name}"]
        x1, h2, mean2, rstd2 = gated_ln_mod_fwd(x[name], g1, out, sh2, sc2, self.eps, out=B[f"h2.{name}"],
                                                sum_out=B[f"x1.{name}"], sum_copy=yb if self._fold_g2 else None)
        M = w.w2.shape[1]
        if self._gelu_fused(name, backward=False):
            pre, act = gemm(h2, w.w1, "gelu", out=B[f"pre.{name}"], act_out=B[f"act.{name}"])
        else:
            pre = _linear(h2, w.w1, w.b1, B[f"pre.{name}"])
            if self.mlp == "swiglu":
                act = swiglu(pre[:, :M], pre[:, M:], out=B[f"act.{name}"])
            else:
                act = gelu(pre, out=B[f"act.{name}"])
        if self._fold_g2:
            y[name] = yb.addmm_(act, self._w2g[name].t())  # x1 + act W2g^T
        else:
            mlp = _linear(act, w.w2, w.b2, B[f"mlp.{name}"])
            y[name] = gated_residual(x1, g2, mlp, out=B[f"y.{name}"])
        if self.capture is not None:
            self.capture[f"{name}_post_attn"] = x1.clone()
            self.capture[f"{name}_out"] = y[name].clone()
        if dy is None:
            return
        # backward: y = x1 + g2 * mlp(h2), h2 = ln_mod(x1), x1 = x + g1 * out(a)
        dmlp = dy[name] if self._fold_g2 else gated_residual(None, g2, dy[name], out=B[f"t1.{name}"])
        if self._gelu_fused(name, backward=True):
            # dpre = (dmlp W2) * gelu'(pre) in one GEMM; W2 (W2g) as [F, C]
            w2t = self._w2g_t[name] if self._fold_g2 else self._wt[name]["w2"]
            dpre = gemm(dmlp, w2t, "dgelu", out=B[f"dact.{name}"], pre=pre)
        else:
            if self._fold_g2:  # (g2 * dy) W2 = dy W2g
                w2g = self._w2g[name] if self._wt is None else self._w2g_t[name].t()
                dact = torch.mm(dmlp, w2g, out=B[f"dact.{name}"])
            else:
                dact = torch.mm(dmlp, self._dx_weight(name, "w2"), out=B[f"dact.{name}"])
            if self.mlp == "swiglu":
                dpre = B[f"dpre.{name}"]
                swiglu_bwd(dact, pre[:, :M], pre[:, M:], dgate=dpre[:, :M], dup=dpre[:, M:])
            else:
                dpre = gelu_bwd(dact, pre, out=dact)
        dh2 = torch.mm(dpre, self._dx_weight(name, "w1"), out=B[f"t2.{name}"])
        # dx1 and dout = g1 * dx1 (the out projection's gradient) in one pass
        dox = B[f"dox.{name}"] if self._fold_out else None
        dx1, dout = ln_mod_bwd_gate(x1, dh2, sc2, mean2, rstd2, g1, self.eps, dres=dy[name], out=B[f"dx1.{name}"],
                                    gated_out=dox[:, :C] if self._fold_out else B[f"t1.{name}"])
        do_rows = B["do"][0, off:off + n].reshape(n, C)
        if self._fold_out:
            r = self.rank
            du = lora_down(dout, self._b_out_t[name], s, out=dox[:, C:C + r])  # s dout B_out
            rhs = self._out_ext_t[name].t() if self._wt is not None else self._out_ext[name]
            torch.mm(dox, rhs, out=do_rows)  # dout W_out + du A_out
            # dA_out = du^T a, dB_out = s dout^T u: formed with the step's other
            # factor gradients (_grad_pending)
            self._grad_pending.append(([(du, a, 1.0, False), (u_out, dout, s, True)],
                                       lambda res, name=name: grads.__setitem__((name, "out"), tuple(res))))
            return
        torch.mm(dout, self._dx_weight(name, "w_out"), out=do_rows)
        if u_out is not None:
            saved[(name, "out", "grad")] = lora_bwd(a, w.lora_a["out"], w.lora_b["out"], u_out, dout, s,
                                                    dx=do_rows)

    def _qkv_bwd_phase(self, name, x, want_dx, saved, grads):
        """The three adapters' gradients and the input gradient (the prologue
        backward of all four segments ran before, in one launch)."""
        B, C, H, D, s = self._buf, self.C, self.H, self.D, self.lora_scale
        w, off, n = self.w[name], self.offset[name], self.rows[name]
        drows = B["dqkv"][off:off + n]
        r = self.rank
        if self._fold:
            hx = B[f"hx.{name}"]
            h, su = hx[:, :C], hx[:, C:C + 3 * r]
        else:
            h, su = B[f"h.{name}"], B[f"su.{name}"]
        if self._fold and want_dx:
            # dY [W_qkv | B_blk | 0] = [dh | t | 0]
            dhx = B[f"dhx.{name}"]
            rhs = self._qkv_ext_t[name].t() if self._wt is not None else self._qkv_ext[name]
            torch.mm(drows, rhs, out=dhx)
            dh, tq = dhx[:, :C], dhx[:, C:C + 3 * r]
        else:
            dh = torch.mm(drows, self._dx_weight(name, "w_qkv"), out=B[f"t2.{name}"]) if want_dx else None
            tq = B[f"tq.{name}"] if self._batched else None
        if self._batched:
            if not (self._fold and want_dx):
                for j, t in enumerate(QKV):  # t_j = dy_j B_j
                    lora_down(drows[:, j * C:(j + 1) * C], self._b_t[name][t], 1.0, out=tq[:, j * r:(j + 1) * r])
            if dh is not None:
                lora_up(tq, self._a_qkv_t[name], dh, s)  # dh += s t A_qkv
            # dA_qkv [3r, C] = s t^T h and dB_j = dy_j^T (s u_j)
            def place(res, name=name):
                da, *dbs = res
                for j, t in enumerate(QKV):
                    grads[(name, t)] = (da[j * r:(j + 1) * r], dbs[j])
            self._grad_pending.append(([(tq, h, s, False)] +
                                       [(su[:, j * r:(j + 1) * r], drows[:, j * C:(j + 1) * C], 1.0, True)
                                        for j in range(len(QKV))], place))
        else:
            for j, t in enumerate(QKV):
                if t in w.lora_a:
                    grads[(name, t)] = lora_bwd(h, w.lora_a[t], w.lora_b[t], saved[(name, t)],
                                                drows[:, j * C:(j + 1) * C], s, dx=dh)
        if (name, "out", "grad") in saved:
            grads[(name, "out")] = saved[(name, "out", "grad")]
        if want_dx:
            mean1, rstd1 = saved[(name, "ln1")]
            grads[(name, "x")] = ln_mod_bwd(x[name], dh, w.mod[1], mean1, rstd1, self.eps,
                                            dres=B[f"dx1.{name}"], out=B[f"dx.{name}"])

    def _run(self, x, dy, want_dx, attention, keep_attention):
        B = self._buffers()
        C, S, H, D = self.C, self.S, self.H, self.D
        main = torch.cuda.current_stream(self.device)
        saved, y, grads = {}, {}, {}
        self._grad_pending = []
        order = CAPTURE_ORDER if torch.cuda.is_current_stream_capturing() else ISSUE_ORDER
        self._fork()
        for name in order:
            with self._on(name):
                self._qkv_phase(name, x, saved)
        self._join()
        self._prologue_fwd()
        v = B["qkv"][:, 2 * C:].view(1, S, H, D)
        if attention is None:
            o_t, lse_t = attn_fwd(B["q"], B["k"], v, self.attn_scale, None, out=B["o"], lse=B["lse"])
        else:
            o_t, lse_t = attention
        kept = (o_t.clone(), lse_t.clone()) if keep_attention else None
        if self.capture is not None:
            self.capture["attn_in.q"], self.capture["attn_in.k"] = B["q"][0].clone(), B["k"][0].clone()
            self.capture["attn_in.v"], self.capture["attn"] = v[0].clone(), o_t[0].clone()
        self._fork()
        for name in order:
            with self._on(name):
                self._out_phase(name, x, dy, o_t, y, saved, grads)
        self._join()
        if dy is None:
            return y, kept
        dv = B["dqkv"][:, 2 * C:].view(1, S, H, D)
        attn_bwd(B["q"], B["k"], v, o_t, B["do"], lse_t, self.attn_scale, None, workspace=B["ws"],
                 out=(B["dq"], B["dk"], dv))
        if self.capture is not None:
            for key, t in (("grad_attn.out", B["do"]), ("grad_attn.q", B["dq"]), ("grad_attn.k", B["dk"]),
                           ("grad_attn.v", dv)):
                self.capture[key] = t[0].clone()
        qk_prologue_bwd_multi(self._prologue_segments(True), self.eps)
        self._fork()
        for name in order:
            with self._on(name):
                self._qkv_bwd_phase(name, x, want_dx, saved, grads)
        self._join()
        if self._grad_pending:
            # The LoRA factor gradients of both streams (q/k/v and out) in one
            # fa_lora_grad_many call: their inputs stay in the step's buffers,
            # and only AdamW reads the results.
            items = [it for its, _ in self._grad_pending for it in its]
            res = lora_grad_many(items)
            k = 0
            for its, place in self._grad_pending:
                place(res[k:k + len(its)])
                k += len(its)
        if self._side is not None:
            # tensors made on the side stream and consumed on this one
            for key, g in grads.items():
                if key[0] == "txt" and key[1] != "x":
                    for t in g:
                        t.record_stream(main)
        return y, grads

    def apply_adamw(self, grads, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8) -> None:
        """One AdamW step of every LoRA factor (adamw_step, lib.rs:477-510),
        all factors in one fa_adamw_step_many call."""
        self.step_count += 1
        items = []
        for (name, t), g in grads.items():
            if t == "x":
                continue
            da, db = g
            w = self.w[name]
            items.append((w.lora_a[t], da, w.m[f"{t}.a"], w.v[f"{t}.a"]))
            items.append((w.lora_b[t], db, w.m[f"{t}.b"], w.v[f"{t}.b"]))
        adamw_step_many(items, self.step_count, lr, betas, eps)
        self.refresh_adapters()

    def train_step(self, x, dy, lr: float = 1e-3, want_dx: bool = False):
        """One LoRA block step: forward, backward, AdamW (the unit of the
        'LoRA block steps/s' metric)."""
        y, grads = self.forward_backward(x, dy, want_dx=want_dx)
        self.apply_adamw(grads, lr)
        return y, grads


def random_block(dim: int, heads: int, txt_tokens: int, img_rows: int, img_cols: int, mlp_ratio: int = 4,
                 rank: int = 16, alpha: float = 16.0, dtype=torch.bfloat16, device="cuda", seed: int = 20261028,
                 axes=(16, 56, 56), theta: float = 1e4, **block_kw) -> DoubleBlockLoRA:
    """c4-style random init: base W ~ N(0, 0.02) frozen, LoRA A ~ N(0, 1/r)
    (PEFT "gaussian"), B ~ N(0, 1e-3), QK-norm scales 1 + N(0, 0.02),
    modulation W ~ N(0, 0.02).  block_kw go to DoubleBlockLoRA."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    C, F = dim, mlp_ratio * dim
    D = dim // heads

    def rn(*shape, std):
        return (torch.randn(*shape, generator=g) * std).to(dtype=dtype, device=device)

    ws = {}
    for name in STREAMS:
        w = StreamWeights(w_qkv=rn(3 * C, C, std=0.02), w_out=rn(C, C, std=0.02), w1=rn(F, C, std=0.02),
                          w2=rn(C, F, std=0.02), q_norm=(1 + rn(D, std=0.02).float()).to(dtype),
                          k_norm=(1 + rn(D, std=0.02).float()).to(dtype), w_mod=rn(6 * C, C, std=0.02))
        for t in LORA_TARGETS:
            w.lora_a[t] = rn(rank, C, std=1.0 / rank)
            w.lora_b[t] = rn(C, rank, std=1e-3)
            for part, shape in (("a", (rank, C)), ("b", (C, rank))):
                w.m[f"{t}.{part}"] = torch.zeros(shape, dtype=torch.float32, device=device)
                w.v[f"{t}.{part}"] = torch.zeros(shape, dtype=torch.float32, device=device)
        ws[name] = w
    return DoubleBlockLoRA(ws, heads, D, txt_tokens, img_rows, img_cols, axes=axes, theta=theta,
                           lora_scale=alpha / rank, **block_kw)


# ---------------------------------------------------------------------------
# single-stream block (the real klein layout)
# ---------------------------------------------------------------------------
SINGLE_LORA_TARGETS = ("to_in", "to_out")
ADAPTER_PAD = 64  # extra GEMM columns that carry a folded adapter (rank <= 64, K stays a multiple of 64)


@dataclass
class SingleWeights:
    """Frozen weights of one single-stream block and its LoRA factors."""
    w_in: torch.Tensor    # [3C + 2M, C]: Q, K, V, SwiGLU gate, SwiGLU up
    w_out: torch.Tensor   # [C, C + M]: over cat(attention, activated MLP)
    q_norm: torch.Tensor  # [D]
    k_norm: torch.Tensor  # [D]
    w_mod: torch.Tensor   # [3C, C]: shift, scale, gate
    lora_a: Dict[str, torch.Tensor] = field(default_factory=dict)
    lora_b: Dict[str, torch.Tensor] = field(default_factory=dict)
    m: Dict[str, torch.Tensor] = field(default_factory=dict)
    v: Dict[str, torch.Tensor] = field(default_factory=dict)
    mod: Tuple[torch.Tensor, ...] = ()


def klein_positions(txt_tokens: int, img_rows: int, img_cols: int) -> np.ndarray:
    """Joint position ids, txt first: txt (0, 0, 0, l), img (0, h, w, 0)
    (throughput.rs:724-748, axes T, H, W, L)."""
    pos = np.zeros((txt_tokens + img_rows * img_cols, 4), np.float32)
    pos[:txt_tokens, 3] = np.arange(txt_tokens)
    rr, cc = np.meshgrid(np.arange(img_rows), np.arange(img_cols), indexing="ij")
    pos[txt_tokens:, 1] = rr.ravel()
    pos[txt_tokens:, 2] = cc.ravel()
    return pos


class SingleBlockLoRA:
    """One single-stream block (single_block, throughput.rs:584-629) with LoRA
    on its fused in-projection and out-projection:

        nh = layer_norm_mod(x, shift, scale)
        [q | k | v | gate | up] = to_in(nh)            (C, C, C, M, M columns)
        attn = attention(rope(rms(q)), rope(rms(k)), v)
        y = x + g * to_out(cat(attn, silu(gate) * up))

    The fused projection output is one [S, 3C + 2M] buffer: the prologue,
    the attention and the SwiGLU read their column slices in place, and the
    attention output and the activation are written straight into the two
    column slices of the [S, C + M] out-projection input (the reference's
    narrow / cat become strides).  Default RoPE: the real klein assignment,
    axes (32, 32, 32, 32), theta 2000 (RESEARCH.md:47, 79 in the reference).
    """

    def __init__(self, weights: SingleWeights, heads: int, head_dim: int, txt_tokens: int, img_rows: int,
                 img_cols: int, axes: Sequence[int] = (32, 32, 32, 32), theta: float = 2000.0,
                 lora_scale: float = 1.0, eps: float = 1e-6, fuse_adapters: bool = True,
                 tuned_gemms: bool = True, dx_weights_t: bool = True):
        """dx_weights_t (with fused adapters): keep transposed copies of the two
        adapter-carrying GEMM operands, so that the backward's dX products read
        them with the contraction dimension contiguous (as the forward does)."""
        self.w = weights
        self.H, self.D = heads, head_dim
        self.C = heads * head_dim
        self.M = (weights.w_in.shape[0] - 3 * self.C) // 2
        if weights.w_in.shape != (3 * self.C + 2 * self.M, self.C) or \
                weights.w_out.shape != (self.C, self.C + self.M):
            raise FoundryAttnError(_abi.FA_ERR_INVALID_ARG, "w_in must be [3C+2M, C] and w_out [C, C+M]")
        self.S = txt_tokens + img_rows * img_cols
        self.axes = tuple(int(a) for a in axes)
        self.lora_scale = float(lora_scale)
        self.eps = float(eps)
        self.attn_scale = 1.0 / math.sqrt(head_dim)
        self.dtype, self.device = weights.w_in.dtype, weights.w_in.device
        self.cos, self.sin = rope_tables(klein_positions(txt_tokens, img_rows, img_cols), self.axes, theta,
                                         dtype=self.dtype, device=self.device)
        self.step_count = 0
        self._buf = None
        if tuned_gemms and self.dtype == torch.bfloat16:
            gemm_tuning.enable()
        self.r = weights.lora_a["to_in"].shape[0]
        # bf16: the adapters ride in the frozen GEMMs (ADAPTER_PAD extra K or N
        # columns: r of them the adapter's, the rest zero)
        self.fused = fuse_adapters and self.dtype == torch.bfloat16 and self.r <= ADAPTER_PAD
        if self.fused:
            C, M, P = self.C, self.M, ADAPTER_PAD
            kw = dict(dtype=self.dtype, device=self.device)
            self.w_in_ext = torch.zeros((3 * C + 2 * M, C + P), **kw)   # [W_in | B_in | 0]
            self.w_in_ext[:, :C] = weights.w_in
            self.w_out_ext = torch.zeros((C + P, C + M), **kw)          # [W_out; A_out; 0]
            self.w_out_ext[:C] = weights.w_out
            self.a_in_t = torch.empty((C, self.r), **kw)    # A_in^T: the dx term's "B"
            self.b_out_t = torch.empty((self.r, C), **kw)   # B_out^T: du_out = s dout B_out
            # [C + P, 3C + 2M] and [C + M, C + P]: the dX products' right operands, transposed
            self.w_in_ext_t = self.w_in_ext.t().contiguous() if dx_weights_t else None
            self.w_out_ext_t = self.w_out_ext.t().contiguous() if dx_weights_t else None
            self.refresh_adapters()

    def refresh_adapters(self) -> None:
        """Copy the trainable factors into the GEMM operands that carry them.
        apply_adamw calls it; call it after changing lora_a / lora_b any other
        way (loading a LoRA file)."""
        if not self.fused:
            return
        C, r, w = self.C, self.r, self.w
        # copied in place, one launch: a captured step (GraphedTrainStep) reads these addresses
        pairs = [(w.lora_b["to_in"], self.w_in_ext[:, C:C + r]), (w.lora_a["to_out"], self.w_out_ext[C:C + r]),
                 (w.lora_a["to_in"].t(), self.a_in_t), (w.lora_b["to_out"].t(), self.b_out_t)]
        if self.w_in_ext_t is not None:
            pairs += [(w.lora_b["to_in"].t(), self.w_in_ext_t[C:C + r]),
                      (w.lora_a["to_out"].t(), self.w_out_ext_t[:, C:C + r])]
        copy2d_many(pairs)

    def set_conditioning(self, c: torch.Tensor) -> None:
        """Modulation parts chunk3(silu(c) W_mod^T) (the Mod3 of throughput.rs:284-288)."""
        m = torch.mm(silu(c.reshape(1, -1)), self.w.w_mod.t()).reshape(-1)
        self.w.mod = _set_mod(self.w.mod, m.split(self.C))

    def _buffers(self):
        if self._buf is None:
            C, M, S, H, D = self.C, self.M, self.S, self.H, self.D
            kw = dict(dtype=self.dtype, device=self.device)
            self._buf = {
                "nh": torch.empty((S, C), **kw), "fused": torch.empty((S, 3 * C + 2 * M), **kw),
                "dfused": torch.empty((S, 3 * C + 2 * M), **kw), "joined": torch.empty((S, C + M), **kw),
                "djoined": torch.empty((S, C + M), **kw), "out": torch.empty((S, C), **kw),
                "y": torch.empty((S, C), **kw), "dout": torch.empty((S, C), **kw),
                "dnh": torch.empty((S, C), **kw), "dx": torch.empty((S, C), **kw),
                "q": torch.empty((1, S, H, D), **kw), "k": torch.empty((1, S, H, D), **kw),
                "dq": torch.empty((1, S, H, D), **kw), "dk": torch.empty((1, S, H, D), **kw),
                "lse": torch.empty((1, H, S), dtype=torch.float32, device=self.device),
                "ws": torch.empty(attn_bwd_workspace_bytes(1, S, H, D, self.dtype), dtype=torch.uint8,
                                  device=self.device)}
            if self.fused:
                P = ADAPTER_PAD
                for key in ("nh_ext", "out_ext", "dout_ext", "dnh_ext"):  # padding columns stay zero
                    self._buf[key] = torch.zeros((S, C + P), **kw)
                self._buf["t_in"] = torch.zeros((S, self.r), **kw)
        return self._buf

    def _heads(self, t: torch.Tensor) -> torch.Tensor:
        """[S, C] column slice (any row stride) as a (1, S, H, D) view."""
        return t.as_strided((1, self.S, self.H, self.D), (self.S * t.stride(0), t.stride(0), self.D, 1))

    def forward(self, x: torch.Tensor, keep_attention: bool = False):
        """Block output y only; keep_attention also returns copies of the
        attention output and its LSE, (O, LSE), for forward_backward."""
        y, att = self._run(x, None, False, None, keep_attention)
        return (y, att) if keep_attention else y

    def forward_backward(self, x: torch.Tensor, dy: torch.Tensor, want_dx: bool = True, attention=None):
        """Block output y and the f32 LoRA gradients grads[target] = (dA, dB);
        with want_dx (a block inside a stack) also grads["x"] = dL/dx.
        attention: (O, LSE) from forward(keep_attention=True) of the same x;
        the attention forward is then skipped."""
        return self._run(x, dy, want_dx, attention, False)

    def _run(self, x, dy, want_dx, attention, keep_attention):
        B = self._buffers()
        C, M = self.C, self.M
        s = self.lora_scale
        w = self.w
        sh, sc, g = w.mod
        fused, dfused, joined, djoined = B["fused"], B["dfused"], B["joined"], B["djoined"]
        F = self.fused
        r = self.r
        if F:
            # [nh | s u_in | 0] [W_in | B_in | 0]^T = nh W_in^T + s u_in B_in^T
            nh_ext = B["nh_ext"]
            nh, mean, rstd = ln_mod_fwd(x, sh, sc, self.eps, out=nh_ext[:, :C], stats=True)
            su_in = lora_down(nh, w.lora_a["to_in"], s, out=nh_ext[:, C:C + r])
            torch.mm(nh_ext, self.w_in_ext.t(), out=fused)
        else:
            nh, mean, rstd = ln_mod_fwd(x, sh, sc, self.eps, out=B["nh"], stats=True)
            torch.mm(nh, w.w_in.t(), out=fused)
            u_in = lora_fwd(nh, w.lora_a["to_in"], w.lora_b["to_in"], fused, s)
        q_raw, k_raw, v = self._heads(fused[:, :C]), self._heads(fused[:, C:2 * C]), self._heads(fused[:, 2 * C:3 * C])
        qk_prologue_multi([(q_raw, w.q_norm, self.cos, self.sin, self.axes, B["q"], 0),
                           (k_raw, w.k_norm, self.cos, self.sin, self.axes, B["k"], 0)], self.eps)
        o = self._heads(joined[:, :C])
        if attention is None:
            _, lse = attn_fwd(B["q"], B["k"], v, self.attn_scale, None, out=o, lse=B["lse"])
        else:
            o.copy_(attention[0])
            lse = attention[1]
        kept = (o.clone(memory_format=torch.contiguous_format), lse.clone()) if keep_attention else None
        gate, up = fused[:, 3 * C:3 * C + M], fused[:, 3 * C + M:]
        swiglu(gate, up, out=joined[:, C:])
        if F:
            # joined [W_out; A_out; 0]^T = [out | u_out | 0]; then out += s u_out B_out^T
            out_ext = B["out_ext"]
            torch.mm(joined, self.w_out_ext.t(), out=out_ext)
            out, u_out = out_ext[:, :C], out_ext[:, C:C + r]
            lora_up(u_out, w.lora_b["to_out"], out, s)
        else:
            out = torch.mm(joined, w.w_out.t(), out=B["out"])
            u_out = lora_fwd(joined, w.lora_a["to_out"], w.lora_b["to_out"], out, s)
        y = gated_residual(x, g, out, out=B["y"])
        if dy is None:
            return y, kept
        # backward: y = x + g * to_out(joined)
        if F:
            # [dout | s dout B_out | 0] [W_out; A_out; 0] = dout W_out + du_out A_out
            dout_ext = B["dout_ext"]
            dout = gated_residual(None, g, dy, out=dout_ext[:, :C])
            du_out = lora_down(dout, self.b_out_t, s, out=dout_ext[:, C:C + r])
            torch.mm(dout_ext, self.w_out_ext if self.w_out_ext_t is None else self.w_out_ext_t.t(), out=djoined)
            # dA_out = du_out^T joined, dB_out = s dout^T u_out: formed with
            # to_in's in one fa_lora_grad_many call at the end (the inputs are
            # not written again)
            out_items = [(du_out, joined, 1.0, False), (u_out, dout, s, True)]
            grads = {}
        else:
            dout = gated_residual(None, g, dy, out=B["dout"])
            torch.mm(dout, w.w_out, out=djoined)
            grads = {"to_out": lora_bwd(joined, w.lora_a["to_out"], w.lora_b["to_out"], u_out, dout, s,
                                        dx=djoined)}
        swiglu_bwd(djoined[:, C:], gate, up, dgate=dfused[:, 3 * C:3 * C + M], dup=dfused[:, 3 * C + M:])
        attn_bwd(B["q"], B["k"], v, o, self._heads(djoined[:, :C]), lse, self.attn_scale, None,
                 workspace=B["ws"], out=(B["dq"], B["dk"], self._heads(dfused[:, 2 * C:3 * C])))
        qk_prologue_bwd_multi([(q_raw, w.q_norm, self.cos, self.sin, self.axes, B["dq"], 0,
                                self._heads(dfused[:, :C])),
                               (k_raw, w.k_norm, self.cos, self.sin, self.axes, B["dk"], 0,
                                self._heads(dfused[:, C:2 * C]))], self.eps)
        if F:
            if want_dx:
                # dfused [W_in | B_in | 0] = [dfused W_in | dfused B_in | 0]
                dnh_ext = B["dnh_ext"]
                torch.mm(dfused, self.w_in_ext if self.w_in_ext_t is None else self.w_in_ext_t.t(), out=dnh_ext)
                dnh, t_in = dnh_ext[:, :C], dnh_ext[:, C:C + r]
                lora_up(t_in, self.a_in_t, dnh, s)  # + s (dfused B_in) A_in
            else:
                dnh = None
                t_in = lora_down(dfused, w.lora_b["to_in"].t().contiguous(), 1.0, out=B["t_in"])
            res = lora_grad_many(out_items + [(t_in, nh, s, False), (su_in, dfused, 1.0, True)])
            grads["to_out"], grads["to_in"] = tuple(res[:2]), tuple(res[2:])
        else:
            dnh = torch.mm(dfused, w.w_in, out=B["dnh"]) if want_dx else None
            grads["to_in"] = lora_bwd(nh, w.lora_a["to_in"], w.lora_b["to_in"], u_in, dfused, s, dx=dnh)
        if want_dx:
            grads["x"] = ln_mod_bwd(x, dnh, sc, mean, rstd, self.eps, dres=dy, out=B["dx"])
        return y, grads

    def apply_adamw(self, grads, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8) -> None:
        self.step_count += 1
        w = self.w
        items = []
        for t in SINGLE_LORA_TARGETS:
            da, db = grads[t]
            items.append((w.lora_a[t], da, w.m[f"{t}.a"], w.v[f"{t}.a"]))
            items.append((w.lora_b[t], db, w.m[f"{t}.b"], w.v[f"{t}.b"]))
        adamw_step_many(items, self.step_count, lr, betas, eps)
        self.refresh_adapters()

    def train_step(self, x, dy, lr: float = 1e-3, want_dx: bool = True):
        y, grads = self.forward_backward(x, dy, want_dx=want_dx)
        self.apply_adamw(grads, lr)
        return y, grads


def random_single_block(dim: int, heads: int, txt_tokens: int, img_rows: int, img_cols: int,
                        mlp_ratio: int = 3, rank: int = 16, alpha: float = 16.0, dtype=torch.bfloat16,
                        device="cuda", seed: int = 20261029, axes=(32, 32, 32, 32),
                        theta: float = 2000.0) -> SingleBlockLoRA:
    """Random init as random_block: base W ~ N(0, 0.02) frozen, LoRA A ~
    N(0, 1/r), B ~ N(0, 1e-3), QK-norm scales 1 + N(0, 0.02)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    C, M = dim, mlp_ratio * dim
    D = dim // heads

    def rn(*shape, std):
        return (torch.randn(*shape, generator=g) * std).to(dtype=dtype, device=device)

    w = SingleWeights(w_in=rn(3 * C + 2 * M, C, std=0.02), w_out=rn(C, C + M, std=0.02),
                      q_norm=(1 + rn(D, std=0.02).float()).to(dtype), k_norm=(1 + rn(D, std=0.02).float()).to(dtype),
                      w_mod=rn(3 * C, C, std=0.02))
    for t, (fin, fout) in (("to_in", (C, 3 * C + 2 * M)), ("to_out", (C + M, C))):
        w.lora_a[t] = rn(rank, fin, std=1.0 / rank)
        w.lora_b[t] = rn(fout, rank, std=1e-3)
        for part, shape in (("a", (rank, fin)), ("b", (fout, rank))):
            w.m[f"{t}.{part}"] = torch.zeros(shape, dtype=torch.float32, device=device)
            w.v[f"{t}.{part}"] = torch.zeros(shape, dtype=torch.float32, device=device)
    return SingleBlockLoRA(w, heads, D, txt_tokens, img_rows, img_cols, axes=axes, theta=theta,
                           lora_scale=alpha / rank)


class GraphedTrainStep:
    """train_step of a DoubleBlockLoRA or SingleBlockLoRA with its forward +
    backward captured once into a HIP graph: one graph launch per step instead
    of the ~115 (double) / ~35 (single) host launches, and the txt / img stream
    fork and joins kept as graph edges.

    - The graph reads the input tensors given here (x and dy): copy each
      step's data into them (x["img"].copy_(...)) before the call.
    - Its outputs (y, grads) are tensors of the graph's memory pool,
      overwritten by the next call.
    - AdamW and the adapter refresh run eagerly after each replay: their bias
      corrections change with the step count.  They update the LoRA factors
      in place, at the addresses the graph reads; so do set_conditioning,
      refresh_adapters and refresh_frozen.
    - The captured ops record no memset: the step's kernels and hipBLASLt
      GEMMs write every element they later read.
    """

    def __init__(self, block, x, dy, want_dx: bool = True, warmup: int = 2):
        self.block, self.x, self.dy = block, x, dy
        cur = torch.cuda.current_stream(block.device)
        side = torch.cuda.Stream(device=block.device)
        side.wait_stream(cur)
        with torch.cuda.stream(side):  # the block's buffers and GEMM handles, outside the capture
            for _ in range(max(1, warmup)):
                block.forward_backward(x, dy, want_dx=want_dx)
        cur.wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.y, self.grads = block.forward_backward(x, dy, want_dx=want_dx)

    def __call__(self, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8):
        """One training step on the current contents of x and dy: (y, grads)."""
        self.graph.replay()
        self.block.apply_adamw(self.grads, lr, betas, eps)
        return self.y, self.grads
