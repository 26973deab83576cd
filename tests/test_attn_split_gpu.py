"""GPU parity of the range-split attention kernels (grids too small for the
GPU: one GPU's share of the heads under sequence parallelism).

When B x H x ceil(S/256) workgroups would leave at least half of the CUs idle
(S >= 1024), the forward and dQ cut each tile's keys, and dK/dV each tile's
queries, into ranges run by separate workgroups; f32 partials are merged
(forward: through their LSEs) or summed in a fixed order.  Gates as for the
unsplit kernels: bf16 max-abs <= 2e-2 and rel-L2 <= 1e-2 against the CPU
oracle, LSE max-abs <= 2e-3; the same gates between the split and the
unsplit forward.
"""
import ctypes
import dataclasses

import numpy as np
import pytest
import torch

from foundry_attn import _abi, attn_bwd, attn_fwd, attn_workspace_bytes, lib
from foundry_attn.configs import C2, C5
from helpers import BF16_MAX_ABS, BF16_REL_L2, attn_inputs, rel_l2
from test_attn_gpu import compare, dev, host, run_gpu

pytestmark = pytest.mark.gpu


def _splits(B, S, H, D, dtype=torch.bfloat16):
    q = torch.empty(B, S, H, D, dtype=dtype, device="cuda")
    return attn_workspace_bytes(q)


def test_split_policy_and_workspace_sizes():
    """Split shapes ask for a forward workspace and a larger backward one;
    full grids, short sequences and f32 ask for none beyond the pre-pass rows,
    except the stored dS blocks of 8-wave bf16 grids (c2: [24 heads][4608
    keys][4608 queries] bf16)."""
    def base(B, S, H):
        r = (B * H * S * 4 + 255) // 256 * 256
        return 2 * r

    def ds(B, S, H):
        return (B * H * ((S + 31) // 32 * 32) * ((S + 255) // 256 * 256) * 2 + 255) // 256 * 256

    fwd, bwd = _splits(1, 4608, 3, 128)  # one GPU's share of c2 over 8 GPUs
    assert fwd > 0 and bwd > base(1, 4608, 3)
    # 3 heads x 18 tiles on 256 CUs: 4 ranges -> f32 partials of 4 x O (+ LSEs)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    split = min(cus // 54, 36 // 4, 16)
    assert fwd == (split * 3 * 4608 * 128 * 4 + 255) // 256 * 256 + (split * 3 * 4608 * 4 + 255) // 256 * 256
    assert bwd == base(1, 4608, 3) + 3 * ((split * 3 * 4608 * 128 * 4 + 255) // 256 * 256)
    f, b = _splits(1, 4608, 24, 128)
    assert f == 0 and b == base(1, 4608, 24) + ds(1, 4608, 24)
    for shape in ((4, 1536, 24, 128), (1, 900, 2, 128)):  # 4-wave grids: no stored dS
        f, b = _splits(*shape)
        assert f == 0 and b == base(shape[0], shape[1], shape[2]), shape
    f, b = _splits(1, 4608, 3, 128, torch.float32)
    assert f == 0 and b == base(1, 4608, 3)


@pytest.mark.parametrize("B,S,H,D,masked", [(1, 2048, 2, 128, False), (1, 2048, 2, 128, True),
                                            (1, 1400, 2, 64, False), (2, 1500, 1, 128, True)],
                         ids=["s2048", "s2048_masked", "s1400_d64", "b2_s1500_masked"])
def test_split_parity_vs_oracle(B, S, H, D, masked):
    """Ragged and masked split shapes against the oracle on every head."""
    assert _splits(B, S, H, D)[0] > 0, "shape does not split"
    rng = np.random.default_rng(11)
    from oracle import bf16_round
    q, k, v, do = (bf16_round(rng.standard_normal((B, S, H, D), dtype=np.float32)) for _ in range(4))
    keep = None
    if masked:
        keep = np.ones((B, S), np.uint8)
        keep[0, 77:512] = 0  # a padded text segment, as in c5
        if B > 1:
            keep[1, S - 300:] = 0
    scale = 1.0 / np.sqrt(D)
    g = run_gpu(q, k, v, do, torch.bfloat16, scale, keep)
    compare(g, q, k, v, do, scale, keep, True, (0, H))


@pytest.fixture(scope="module")
def shard_run():
    """c2's inputs (RMSNorm + axial RoPE) at 3 heads: the per-GPU attention
    of c2 under 8-way sequence (Ulysses) parallelism."""
    cfg = dataclasses.replace(C2, heads=3)
    x = attn_inputs(cfg)
    g = run_gpu(x["q"], x["k"], x["v"], x["do"], torch.bfloat16, cfg.scale)
    return cfg, x, g


def test_ulysses_shard_parity(shard_run):
    """All 3 heads of the shard against the oracle."""
    cfg, x, g = shard_run
    assert _splits(1, cfg.seq, cfg.heads, cfg.head_dim)[0] > 0
    compare(g, x["q"], x["k"], x["v"], x["do"], cfg.scale, None, True, (0, cfg.heads))


def test_ulysses_shard_properties(shard_run):
    """All 3 heads at S = 4608: sum_j dK_j = 0, sum_j dV_j = sum_i dO_i."""
    cfg, x, g = shard_run
    sk = np.abs(g["dk"].astype(np.float64).sum(1))
    assert np.all(sk <= 1e-3 * np.abs(g["dk"]).sum(1) + 1e-6)
    assert rel_l2(g["dv"].astype(np.float64).sum(1), x["do"].astype(np.float64).sum(1)) <= 1e-2
    for n in ("o", "lse", "dq", "dk", "dv"):
        assert np.all(np.isfinite(g[n])), n


@pytest.mark.parametrize("cfg_name", ["c2_h3", "c5_h1"])
def test_split_forward_matches_unsplit(cfg_name):
    """The same inputs through the split and the unsplit forward, within the
    bf16 gates (c5 at one head: key-padding mask, B = 2, all rows checked).
    The two are not bit-identical: each key range rounds P to bf16 against
    its own exp2 reference, noise of the size each path shows against the
    oracle (O rel-L2 ~3e-3)."""
    cfg = dataclasses.replace(C2, heads=3) if cfg_name == "c2_h3" else dataclasses.replace(C5, heads=1)
    B, S, H, D = cfg.batch, cfg.seq, cfg.heads, cfg.head_dim
    assert _splits(B, S, H, D)[0] > 0
    torch.manual_seed(4)
    q, k, v = (torch.randn(B, S, H, D, device="cuda").to(torch.bfloat16) for _ in range(3))
    keep = None if cfg.key_keep() is None else dev(cfg.key_keep(), torch.uint8)
    o_s, l_s = attn_fwd(q, k, v, cfg.scale, keep)
    o_u, l_u = attn_fwd(q, k, v, cfg.scale, keep, split=False)
    torch.cuda.synchronize()
    a, b = host(o_s), host(o_u)
    ma, rl = float(np.max(np.abs(a - b))), rel_l2(a, b)
    print(f"  O split vs unsplit: max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
    assert ma <= BF16_MAX_ABS and rl <= BF16_REL_L2
    ls, lu = host(l_s), host(l_u)
    assert np.array_equal(np.isfinite(ls), np.isfinite(lu))
    fin = np.isfinite(lu)
    assert np.max(np.abs(ls[fin] - lu[fin])) <= 2e-3


def test_split_results_are_repeatable():
    """Fixed-order partial sums: two runs give the same bits."""
    torch.manual_seed(8)
    q, k, v, do = (torch.randn(1, 2048, 2, 128, device="cuda").to(torch.bfloat16) for _ in range(4))
    runs = []
    for _ in range(2):
        o, lse = attn_fwd(q, k, v)
        runs.append((o, lse) + tuple(attn_bwd(q, k, v, o, do, lse)))
    torch.cuda.synchronize()
    for a, b in zip(*runs):
        assert torch.equal(a, b)


def test_forward_workspace_too_small_is_refused():
    """A non-NULL forward workspace smaller than fa_attn_fwd_workspace_size is
    FA_ERR_INVALID_ARG with a message; NULL runs the unsplit kernel."""
    B, S, H, D = 1, 2048, 2, 128
    q, k, v = (torch.randn(B, S, H, D, device="cuda").to(torch.bfloat16) for _ in range(3))
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, device="cuda")
    need = _splits(B, S, H, D)[0]
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    st = lambda t: _abi.Strides(t.stride(0), t.stride(1), t.stride(2))
    a = _abi.AttnFwdArgs(dtype=_abi.FA_DTYPE_BF16, batch=B, seq=S, heads=H, head_dim=D, scale=D ** -0.5,
                         q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), o=o.data_ptr(), lse=lse.data_ptr(),
                         key_keep=None, q_stride=st(q), k_stride=st(k), v_stride=st(v), o_stride=st(o),
                         workspace=ws.data_ptr(), workspace_bytes=need - 256)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib().fa_attn_fwd(ctypes.byref(a), stream) == _abi.FA_ERR_INVALID_ARG
    assert b"smaller" in lib().fa_last_error()
    a.workspace_bytes = need
    assert lib().fa_attn_fwd(ctypes.byref(a), stream) == _abi.FA_OK
    o_null = torch.empty_like(q)
    a.workspace, a.workspace_bytes, a.o = None, 0, o_null.data_ptr()
    assert lib().fa_attn_fwd(ctypes.byref(a), stream) == _abi.FA_OK
    ref, _ = attn_fwd(q, k, v, split=False)
    torch.cuda.synchronize()
    assert torch.equal(o_null, ref)


@pytest.mark.parametrize("seed", [1, 2, 3, 4, 5, 6])
def test_split_random_shapes(seed):
    """Seeded random split shapes (B 1-2, H 1-3, ragged S 1024-3000, D 64 or
    128, half of them with a random key mask that keeps every batch item's
    first key) against the oracle on one head."""
    rng = np.random.default_rng(100 + seed)
    B, H = int(rng.integers(1, 3)), int(rng.integers(1, 4))
    S, D = int(rng.integers(1024, 3001)), int(rng.choice([64, 128]))
    print(f"  B={B} S={S} H={H} D={D}", flush=True)
    assert _splits(B, S, H, D)[0] > 0, "shape does not split"
    from oracle import bf16_round
    q, k, v, do = (bf16_round(rng.standard_normal((B, S, H, D), dtype=np.float32)) for _ in range(4))
    keep = None
    if seed % 2:
        keep = (rng.random((B, S)) > 0.3).astype(np.uint8)
        keep[:, 0] = 1
    scale = 1.0 / np.sqrt(D)
    g = run_gpu(q, k, v, do, torch.bfloat16, scale, keep)
    h = int(rng.integers(0, H))
    compare(g, q, k, v, do, scale, keep, True, (h, h + 1))
