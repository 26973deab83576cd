"""fa_attn_bwd_noalloc (the backward entry point that allocates nothing and
keeps its scratch in a fixed per-device array) against fa_attn_bwd, through
the C ABI, on several calls in a row with shrinking inputs.

Shapes fa_attn_bwd does not split must match it bit for bit (same kernels,
same order of arithmetic; the no-allocation call only runs them in order on
one stream).  A shape fa_attn_bwd splits runs unsplit here, so it is held to
the bf16 gate of the exact gradients (max-abs 2e-2, rel-L2 1e-2) instead."""
import ctypes
import math

import numpy as np
import pytest
import torch

from foundry_attn import _abi, ops
from foundry_attn._abi import check, lib
from helpers import BF16_MAX_ABS, BF16_REL_L2, max_abs, rel_l2

pytestmark = pytest.mark.gpu


def _inputs(B, S, H, D, dtype, seed, device):
    g = torch.Generator(device="cpu").manual_seed(seed)
    mk = lambda: torch.randn((B, S, H, D), generator=g).to(device=device, dtype=dtype)
    return mk(), mk(), mk(), mk()


def _noalloc_args(q, k, v, o, do, lse, keep, scale, dq, dk, dv):
    B, S, H, D = q.shape
    return _abi.AttnBwdArgs(dtype=ops._dtype_code(q), batch=B, seq=S, heads=H, head_dim=D, scale=scale,
                         q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), o=o.data_ptr(),
                         dout=do.data_ptr(), lse=lse.data_ptr(),
                         key_keep=0 if keep is None else keep.data_ptr(),
                         dq=dq.data_ptr(), dk=dk.data_ptr(), dv=dv.data_ptr(),
                         q_stride=ops._strides(q), k_stride=ops._strides(k), v_stride=ops._strides(v),
                         o_stride=ops._strides(o), do_stride=ops._strides(do),
                         dq_stride=ops._strides(dq), dk_stride=ops._strides(dk),
                         dv_stride=ops._strides(dv))


def _noalloc_call(q, k, v, o, do, lse, keep, scale):
    """dq, dk, dv from fa_attn_bwd_noalloc (outputs come from the caller)."""
    dq, dk, dv = (torch.empty_like(t) for t in (q, k, v))
    a = _noalloc_args(q, k, v, o, do, lse, keep, scale, dq, dk, dv)
    check(lib().fa_attn_bwd_noalloc(ctypes.byref(a), torch.cuda.current_stream().cuda_stream))
    return dq, dk, dv


# (B, S, H, D, dtype, masked, split by fa_attn_bwd), largest first: each later
# call finds the earlier calls' rows still in the shared scratch
CASES = [
    (1, 4608, 24, 128, torch.bfloat16, False, False),  # c2 shape, 8-wave kernels
    (2, 700, 3, 64, torch.bfloat16, True, False),      # 4-wave kernels, key mask
    (1, 256, 4, 64, torch.float32, False, False),      # c1 shape, f32 kernels
    (1, 4608, 3, 128, torch.bfloat16, True, True),     # 8-way Ulysses shard: split
    (1, 200, 2, 128, torch.bfloat16, True, False),     # small, masked
]


def test_noalloc_matches_fa_attn_bwd(device):
    for i, (B, S, H, D, dt, masked, split) in enumerate(CASES):
        print(f"noalloc case {i}: B={B} S={S} H={H} D={D} {dt} masked={masked}", flush=True)
        q, k, v, do = _inputs(B, S, H, D, dt, 100 + i, device)
        keep = None
        if masked:
            keep = torch.ones((B, S), dtype=torch.uint8)
            keep[:, S // 7: S // 7 + S // 5] = 0
            keep = keep.to(device)
        scale = 1.0 / math.sqrt(D)
        o, lse = ops.attn_fwd(q, k, v, key_keep=keep, split=False)
        want = ops.attn_bwd(q, k, v, o, do, lse, key_keep=keep)
        assert (ops.attn_workspace_bytes(q)[0] > 0) == split, "split policy changed for this case"
        got = _noalloc_call(q, k, v, o, do, lse, keep, scale)
        torch.cuda.synchronize()
        for name, g_, w_ in zip(("dq", "dk", "dv"), got, want):
            assert torch.isfinite(g_.float()).all(), (i, name)
            if split:
                g64, w64 = g_.float().cpu().numpy(), w_.float().cpu().numpy()
                assert max_abs(g64, w64) <= BF16_MAX_ABS, (i, name, max_abs(g64, w64))
                assert rel_l2(g64, w64) <= BF16_REL_L2, (i, name, rel_l2(g64, w64))
            else:
                assert torch.equal(g_, w_), (i, name, (g_.float() - w_.float()).abs().max().item())


def test_noalloc_rejects_rows_past_scratch(device):
    """One row past the fixed scratch is refused before any launch."""
    q = torch.zeros((1, 8, 1, 64), dtype=torch.float32, device=device)
    a = _abi.AttnBwdArgs(dtype=_abi.FA_DTYPE_F32, batch=1, seq=(1 << 21) + 1, heads=1, head_dim=64,
                         scale=0.125, q=q.data_ptr(), k=q.data_ptr(), v=q.data_ptr(), o=q.data_ptr(),
                         dout=q.data_ptr(), lse=q.data_ptr(), dq=q.data_ptr(), dk=q.data_ptr(),
                         dv=q.data_ptr(), q_stride=_abi.Strides(0, 64, 64), k_stride=_abi.Strides(0, 64, 64),
                         v_stride=_abi.Strides(0, 64, 64), o_stride=_abi.Strides(0, 64, 64),
                         do_stride=_abi.Strides(0, 64, 64), dq_stride=_abi.Strides(0, 64, 64),
                         dk_stride=_abi.Strides(0, 64, 64), dv_stride=_abi.Strides(0, 64, 64))
    assert lib().fa_attn_bwd_noalloc(ctypes.byref(a), None) == _abi.FA_ERR_INVALID_ARG
    assert b"2097152 rows" in lib().fa_last_error()


def test_noalloc_replays_under_graph_capture(device):
    """fa_attn_bwd_noalloc captured in a HIP graph, after fa_init on the
    device (the first call's device query and scratch lookup stay outside the
    capture): four replays, each after eager work that overwrites the outputs
    with NaN and the shared scratch with another call's rows, all give the
    eager call's bits."""
    assert lib().fa_init(torch.cuda.current_device()) == _abi.FA_OK
    B, S, H, D = 1, 1000, 4, 128
    q, k, v, do = _inputs(B, S, H, D, torch.bfloat16, 300, device)
    keep = torch.ones((B, S), dtype=torch.uint8)
    keep[:, 100:260] = 0
    keep = keep.to(device)
    scale = 1.0 / math.sqrt(D)
    o, lse = ops.attn_fwd(q, k, v, key_keep=keep, split=False)
    want = _noalloc_call(q, k, v, o, do, lse, keep, scale)
    other = _inputs(1, 600, 3, 64, torch.bfloat16, 301, device)
    o2, lse2 = ops.attn_fwd(*other[:3], split=False)
    out = tuple(torch.empty_like(t) for t in (q, k, v))
    a = _noalloc_args(q, k, v, o, do, lse, keep, scale, *out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        check(lib().fa_attn_bwd_noalloc(ctypes.byref(a), torch.cuda.current_stream().cuda_stream))
    for rep in range(4):
        for t in out:
            t.fill_(float("nan"))
        _noalloc_call(*other[:3], o2, other[3], lse2, None, 0.125)  # rewrites the scratch rows
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name, got, w in zip(("dq", "dk", "dv"), out, want):
            assert torch.equal(got, w), (rep, name)
