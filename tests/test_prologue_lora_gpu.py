"""GPU parity of the fused QK prologue and the LoRA kernels (through the C
ABI) against the oracle and the reference's fixtures."""
import numpy as np
import pytest
import torch

import oracle
from foundry_attn import lora_bwd, lora_fwd, qk_prologue, qk_prologue_bwd, rope_tables
from foundry_attn.configs import C2
from helpers import BF16_MAX_ABS, BF16_REL_L2, load_golden, max_abs, rel_l2

pytestmark = pytest.mark.gpu


def dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device="cuda", dtype=dtype)


def host(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_prologue_fwd_joint_buffer_matches_oracle(dtype):
    """c2 shapes: txt stream (512 tokens) at joint offset 0 and img stream
    (64x64) at offset 512, each RMSNormed and roped into one joint buffer."""
    bf = dtype == "bf16"
    tdt = torch.bfloat16 if bf else torch.float32
    rng = np.random.default_rng(4)
    H, D, T_txt = C2.heads, C2.head_dim, C2.txt_len
    T_img = C2.seq - T_txt
    rnd = oracle.bf16_round if bf else (lambda a: a.astype(np.float32))
    xt = rnd(rng.standard_normal((1, T_txt, H, D)).astype(np.float32))
    xi = rnd(rng.standard_normal((1, T_img, H, D)).astype(np.float32) * 3)
    w = rnd(1 + 0.02 * rng.standard_normal(D).astype(np.float32))
    pos = C2.positions()
    cos, sin = oracle.rope_tables(pos, C2.axes, C2.theta, bf16=bf)
    want = np.concatenate(
        [oracle.apply_rope(oracle.rms_norm(xt[0], w, bf16=bf), cos[:T_txt], sin[:T_txt], C2.axes, bf16=bf),
         oracle.apply_rope(oracle.rms_norm(xi[0], w, bf16=bf), cos[T_txt:], sin[T_txt:], C2.axes, bf16=bf)])
    tc, ts = rope_tables(pos, C2.axes, C2.theta, dtype=tdt)
    assert np.array_equal(host(tc), cos) and np.array_equal(host(ts), sin)
    joint = torch.empty((1, C2.seq, H, D), dtype=tdt, device="cuda")
    tw = dev(w, tdt)
    qk_prologue(dev(xt, tdt), tw, tc[:T_txt].contiguous(), ts[:T_txt].contiguous(), C2.axes,
                out=joint, seq_offset=0)
    qk_prologue(dev(xi, tdt), tw, tc[T_txt:].contiguous(), ts[T_txt:].contiguous(), C2.axes,
                out=joint, seq_offset=T_txt)
    got = host(joint)[0]
    if bf:
        # same cast points as the reference; the RMS statistic summed in another
        # order can move a normalised input by one bf16 ulp, which moves the
        # rotated output by at most ~2 ulp of the row's largest input
        row_max = np.abs(want).max(-1, keepdims=True)
        assert np.mean(got != want) < 1e-3
        assert np.all(np.abs(got - want) <= row_max * 2.0 ** -6)
        assert max_abs(got, want) <= BF16_MAX_ABS and rel_l2(got, want) <= 1e-3
    else:
        assert rel_l2(got, want) <= 1e-6


def test_prologue_fixture_replay():
    """double.q of the reference fixture: linear (oracle, host) -> fused
    RMSNorm + RoPE kernel, bf16 and fp32."""
    axes = [32, 32, 32, 32]
    rows, cols = np.arange(16) // 4, np.arange(16) % 4
    z = np.zeros(16)
    pos = np.stack([rows, cols, z, z], -1).astype(np.float32)
    for tag, tdt in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
        f = load_golden(tag)
        bf = tag == "bf16"
        W = lambda p: f.get(f"weights/double.img.to_q.{p}")
        h = oracle.linear_lora(f["double.img_norm1"], W("weight"), W("bias"), W("lora_a"),
                               W("lora_b"), scale=2.0, bf16=bf).reshape(1, 16, 2, 128)
        tc, ts = rope_tables(pos, axes, 1e4, dtype=tdt)
        y = qk_prologue(dev(h, tdt), dev(f["weights/double.img_q_norm.weight"], tdt), tc, ts, axes)
        rl = rel_l2(host(y)[0], f["double.q"])
        print(f"  {tag}: rel_l2={rl:.3e}", flush=True)
        assert rl <= (1e-6 if not bf else 2e-3)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("H,D,axes", [(4, 128, None), (6, 128, None), (3, 128, None), (8, 64, None),
                                      (5, 64, None), (4, 128, (22, 54, 52)), (3, 128, (22, 54, 52))],
                         ids=["h4", "h6", "h3_odd", "h8_d64", "h5_d64_odd", "h4_odd_halves", "h3_odd_halves"])
def test_prologue_fwd_strided_matches_oracle(dtype, H, D, axes):
    """A strided input view (a q slice of a packed qkv buffer).  Head counts
    that are multiples of 4 give each lane 4 adjacent heads of one token
    (one cos / sin load; 128-row workgroups at D = 64), even ones 2, and odd
    ones rows of different tokens.  Axis halves that are all multiples of 4
    (the default axes) read rotate-half partners 4 at a time; (22, 54, 52)
    has halves 11, 27, 26 and reads them one by one."""
    bf = dtype == "bf16"
    tdt = torch.bfloat16 if bf else torch.float32
    rng = np.random.default_rng(12)
    T = 301
    rnd = oracle.bf16_round if bf else (lambda a: a.astype(np.float32))
    qkv = rnd(rng.standard_normal((1, T, 3, H, D)).astype(np.float32) * 2)
    w = rnd(1 + 0.02 * rng.standard_normal(D).astype(np.float32))
    pos = np.stack([np.zeros(T), np.arange(T) // 20, np.arange(T) % 20], -1).astype(np.float32)
    axes = list(axes) if axes else [16, 56, 56] if D == 128 else [16, 24, 24]
    cos, sin = oracle.rope_tables(pos, axes, 1e4, bf16=bf)
    want = oracle.apply_rope(oracle.rms_norm(qkv[0, :, 0], w, bf16=bf), cos, sin, axes, bf16=bf)
    x = dev(qkv, tdt)[:, :, 0]  # token stride 3*H*D, head stride D
    out = torch.full((1, T + 7, H, D), float("nan"), dtype=tdt, device="cuda")
    qk_prologue(x, dev(w, tdt), dev(cos, tdt), dev(sin, tdt), axes, out=out, seq_offset=7)
    got = host(out)[0]
    assert np.all(np.isnan(got[:7]))
    got = got[7:]
    if bf:
        assert np.mean(got != want) < 1e-3
        assert max_abs(got, want) <= BF16_MAX_ABS and rel_l2(got, want) <= 1e-3
    else:
        assert rel_l2(got, want) <= 1e-6


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("H,axes", [(4, (16, 56, 56)), (3, (16, 56, 56)), (4, (22, 54, 52))],
                         ids=["even_heads", "odd_heads", "odd_halves"])
def test_prologue_bwd_matches_oracle(dtype, H, axes):
    bf = dtype == "bf16"
    tdt = torch.bfloat16 if bf else torch.float32
    rng = np.random.default_rng(8)
    T, D = 300, 128
    rnd = oracle.bf16_round if bf else (lambda a: a.astype(np.float32))
    x = rnd(rng.standard_normal((T, H, D)).astype(np.float32))
    w = rnd(1 + 0.02 * rng.standard_normal(D).astype(np.float32))
    pos = np.stack([np.zeros(T), np.arange(T) // 20, np.arange(T) % 20], -1).astype(np.float32)
    axes = list(axes)
    cos, sin = oracle.rope_tables(pos, axes, 1e4, bf16=bf)
    dy_joint = rnd(rng.standard_normal((1, T + 50, H, D)).astype(np.float32))
    want = oracle.qk_prologue_bwd(x, w, cos, sin, dy_joint[0, 50:], axes)
    dx = qk_prologue_bwd(dev(x, tdt), dev(w, tdt), dev(cos, tdt), dev(sin, tdt), axes,
                         dev(dy_joint, tdt), seq_offset=50)
    got = host(dx)
    if bf:
        assert max_abs(got, want) <= BF16_MAX_ABS and rel_l2(got, want) <= BF16_REL_L2
    else:
        assert rel_l2(got, want) <= 1e-5


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_lora_fwd_bwd_match_oracle(dtype):
    bf = dtype == "bf16"
    tdt = torch.bfloat16 if bf else torch.float32
    rng = np.random.default_rng(3)
    N, K, M, r, s = 600, 256, 384, 16, 1.0
    rnd = oracle.bf16_round if bf else (lambda a: a.astype(np.float32))
    x = rnd(rng.standard_normal((N, K)).astype(np.float32))
    Wb = rnd(0.02 * rng.standard_normal((M, K)).astype(np.float32))
    A = rnd(rng.standard_normal((r, K)).astype(np.float32) / r)
    B = rnd(0.05 * rng.standard_normal((M, r)).astype(np.float32))
    dy = rnd(rng.standard_normal((N, M)).astype(np.float32))
    base = oracle.linear_lora(x, Wb, bf16=bf)
    want = oracle.linear_lora(x, Wb, None, A, B, scale=s, bf16=bf)
    y = dev(base, tdt)
    u = lora_fwd(dev(x, tdt), dev(A, tdt), dev(B, tdt), y, s)
    got = host(y)
    if bf:
        assert max_abs(got, want) <= BF16_MAX_ABS and rel_l2(got, want) <= BF16_REL_L2
    else:
        assert rel_l2(got, want) <= 1e-5
    np.testing.assert_allclose(host(u), x.astype(np.float64) @ A.T.astype(np.float64),
                               rtol=1e-4, atol=1e-3)
    dx_base = np.zeros((N, K), np.float32)
    dx = dev(dx_base, tdt)
    dA, dB = lora_bwd(dev(x, tdt), dev(A, tdt), dev(B, tdt), u, dev(dy, tdt), s, dx=dx)
    _, wA, wB = oracle.linear_lora_bwd(x, Wb, A, B, dy, scale=s, bf16=False, want_dx=False)
    # adapter share of dx: s * (dy B) A
    want_dx = (s * (dy.astype(np.float64) @ B) @ A).astype(np.float32)
    tol = 1e-2 if bf else 1e-5
    assert rel_l2(host(dA), wA) <= tol and rel_l2(host(dB), wB) <= tol
    assert rel_l2(host(dx), want_dx) <= tol


def test_lora_grads_fixture_replay():
    """LoRA dA/dB of double.img.to_v from the reference fixture (PyTorch
    autograd), seeded with the fixture's dL/dv (fp32)."""
    f = load_golden("fp32")
    x = f["double.img_norm1"]
    W = lambda p: f[f"weights/double.img.to_v.{p}"]
    dy = f["grad/attn/double.v"][8:].reshape(16, 256)
    y = dev(np.zeros((16, 256), np.float32), torch.float32)
    u = lora_fwd(dev(x, torch.float32), dev(W("lora_a"), torch.float32),
                 dev(W("lora_b"), torch.float32), y, 2.0)
    dA, dB = lora_bwd(dev(x, torch.float32), dev(W("lora_a"), torch.float32),
                      dev(W("lora_b"), torch.float32), u, dev(dy, torch.float32), 2.0)
    assert rel_l2(host(dA), f["grad/double.img.to_v.lora_a"]) <= 1e-5
    assert rel_l2(host(dB), f["grad/double.img.to_v.lora_b"]) <= 1e-5


@pytest.mark.parametrize("r", [4, 12, 32])
def test_lora_bf16_ranks_ragged(r):
    """bf16 adapters at ranks that are and are not multiples of 8, a token
    count that is not a multiple of 32, and B held at a 2-byte offset (the
    scalar-load path of the expand kernel)."""
    rng = np.random.default_rng(100 + r)
    N, K, M, s = 333, 192, 320, 0.5
    rnd = oracle.bf16_round
    x = rnd(rng.standard_normal((N, K)).astype(np.float32))
    Wb = rnd(0.02 * rng.standard_normal((M, K)).astype(np.float32))
    A = rnd(rng.standard_normal((r, K)).astype(np.float32) / r)
    B = rnd(0.05 * rng.standard_normal((M, r)).astype(np.float32))
    dy = rnd(rng.standard_normal((N, M)).astype(np.float32))
    base = oracle.linear_lora(x, Wb, bf16=True)
    want = oracle.linear_lora(x, Wb, None, A, B, scale=s, bf16=True)
    Bbuf = torch.zeros(M * r + 1, dtype=torch.bfloat16, device="cuda")
    Bv = Bbuf[1:].view(M, r)
    Bv.copy_(dev(B, torch.bfloat16))
    y = dev(base, torch.bfloat16)
    u = lora_fwd(dev(x, torch.bfloat16), dev(A, torch.bfloat16), Bv, y, s)
    got = host(y)
    assert max_abs(got, want) <= BF16_MAX_ABS and rel_l2(got, want) <= BF16_REL_L2
    np.testing.assert_allclose(host(u), x.astype(np.float64) @ A.T.astype(np.float64),
                               rtol=1e-4, atol=1e-3)
    dx = dev(np.zeros((N, K), np.float32), torch.bfloat16)
    dA, dB = lora_bwd(dev(x, torch.bfloat16), dev(A, torch.bfloat16), Bv, u,
                      dev(dy, torch.bfloat16), s, dx=dx)
    _, wA, wB = oracle.linear_lora_bwd(x, Wb, A, B, dy, scale=s, bf16=False, want_dx=False)
    want_dx = (s * (dy.astype(np.float64) @ B) @ A).astype(np.float32)
    assert rel_l2(host(dA), wA) <= 1e-2 and rel_l2(host(dB), wB) <= 1e-2
    assert rel_l2(host(dx), want_dx) <= 1e-2


@pytest.mark.parametrize("K", [16, 208, 3088])
@pytest.mark.parametrize("r", [16, 33, 48, 64])
def test_lora_down_k_tails(K, r):
    """fa_lora_down where K is not a multiple of 32 (the last 32-wide k-step
    is half, its upper 16 columns zeroed in the operand), where some waves of
    a workgroup have no k-step (K = 16, 208), and where a wave's k-steps run
    over several LDS stages with a remainder (K = 3088); ranks over 1 to 4
    16-column tiles, and a token count that is not a multiple of 16.  Against
    the f64 product of the same bf16 values, rounded to bf16 as the kernel
    writes it."""
    from foundry_attn.ops import lora_down
    rng = np.random.default_rng(300 + K + r)
    N, s = 333, 0.5
    rnd = oracle.bf16_round
    x = rnd(rng.standard_normal((N, K)).astype(np.float32))
    A = rnd(rng.standard_normal((r, K)).astype(np.float32) / np.sqrt(K))
    bf = torch.bfloat16
    # x with columns past K holding large values: a wrongly read column shows
    xe = torch.full((N, K + 48), 1e4, dtype=bf, device="cuda")
    xe[:, :K] = dev(x, bf)
    u = lora_down(xe[:, :K], dev(A, bf), s, out=torch.empty((N, r), dtype=bf, device="cuda"))
    want = (s * (x.astype(np.float64) @ A.T.astype(np.float64))).astype(np.float32)
    got = host(u)
    peak = np.abs(want).max()
    assert max_abs(got, want) <= 2 ** -7 * peak + 1e-6 and rel_l2(got, want) <= 4e-3, (K, r)


@pytest.mark.parametrize("N", [4096, 4613, 9219])
@pytest.mark.parametrize("r", [16, 48])
def test_lora_down_slab_counts(N, r):
    """Token counts whose rowdot launches take one, two and four 16-row slabs
    per workgroup on a 256-CU device (4096: 256 workgroups of one slab; 4613:
    two slabs, the last workgroup ragged; 9219: four slabs, three of the last
    workgroup's slabs wholly past N).  At rank 16 the f32-output rowdot of
    fa_lora_fwd (its u) goes through the same choice.  Against the f64 product
    of the same bf16 values."""
    from foundry_attn.ops import lora_down, lora_fwd
    rng = np.random.default_rng(900 + N + r)
    K, s = 208, 0.5
    rnd = oracle.bf16_round
    x = rnd(rng.standard_normal((N, K)).astype(np.float32))
    A = rnd(rng.standard_normal((r, K)).astype(np.float32) / np.sqrt(K))
    bf = torch.bfloat16
    xe = torch.full((N, K + 48), 1e4, dtype=bf, device="cuda")
    xe[:, :K] = dev(x, bf)
    u = lora_down(xe[:, :K], dev(A, bf), s, out=torch.empty((N, r), dtype=bf, device="cuda"))
    want = x.astype(np.float64) @ A.T.astype(np.float64)
    got = host(u)
    assert max_abs(got, s * want) <= 2 ** -7 * np.abs(s * want).max() + 1e-6 and rel_l2(got, s * want) <= 4e-3
    if r <= 32:
        M = 32
        B = rnd(0.05 * rng.standard_normal((M, r)).astype(np.float32))
        y = torch.zeros((N, M), dtype=bf, device="cuda")
        uf = lora_fwd(xe[:, :K], dev(A, bf), dev(B, bf), y, s)
        np.testing.assert_allclose(host(uf), want, rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("r", [1, 16, 17, 48, 64])
@pytest.mark.parametrize("y_aligned", [True, False])
def test_lora_up_rank_steps_and_y_alignment(r, y_aligned):
    """fa_lora_up over one to four 16-wide rank steps (the kernel's rank-step
    count is a template argument chosen per call), a token count that is not a
    multiple of 32, a column count that leaves idle waves in the last
    workgroup, and y either 16-byte aligned (16-byte loads and stores, loaded
    before the product) or at a 2-byte offset (the element path).  Against y
    plus the f64 product of the same bf16 values."""
    from foundry_attn.ops import lora_up
    rng = np.random.default_rng(700 + r)
    N, M, s = 77, 336, 0.75
    rnd = oracle.bf16_round
    u = rnd(rng.standard_normal((N, r)).astype(np.float32))
    B = rnd(0.05 * rng.standard_normal((M, r)).astype(np.float32))
    y0 = rnd(rng.standard_normal((N, M)).astype(np.float32))
    bf = torch.bfloat16
    ldy = M + 24 if y_aligned else M + 1
    yb = torch.zeros(N * ldy + 8, dtype=bf, device="cuda")
    yv = yb[(0 if y_aligned else 1):][:N * ldy].view(N, ldy)[:, :M]
    yv.copy_(dev(y0, bf))
    lora_up(dev(u, bf), dev(B, bf), yv, s)
    want = y0.astype(np.float64) + s * (u.astype(np.float64) @ B.T.astype(np.float64))
    got = host(yv)
    assert max_abs(got, want) <= 2 ** -7 * np.abs(want).max() + 1e-6 and rel_l2(got, want) <= 4e-3, (r, y_aligned)
    # columns between rows (the row padding) are untouched
    pad = yb[(0 if y_aligned else 1):][:N * ldy].view(N, ldy)[:, M:]
    assert float(pad.abs().max()) == 0.0


@pytest.mark.parametrize("r", [4, 16, 32, 40, 48, 64])
def test_lora_pieces_strided_views(r):
    """fa_lora_down / fa_lora_up / fa_lora_grad on the rank-column views a
    GEMM that carries the adapter uses: u lives in extra columns of wider
    buffers.  Checked against f64 products of the same bf16 values, and the
    fused product [x | s u] [W | B]^T against x W^T + s u B^T."""
    from foundry_attn.ops import lora_down, lora_grad, lora_up
    rng = np.random.default_rng(200 + r)
    N, K, M, s, pad = 333, 256, 384, 0.75, 80
    rnd = oracle.bf16_round
    x = rnd(rng.standard_normal((N, K)).astype(np.float32))
    A = rnd(rng.standard_normal((r, K)).astype(np.float32) / r)
    B = rnd(0.05 * rng.standard_normal((M, r)).astype(np.float32))
    dy = rnd(rng.standard_normal((N, M)).astype(np.float32))
    bf = torch.bfloat16
    xe = torch.zeros(N, K + pad, dtype=bf, device="cuda")
    xe[:, :K] = dev(x, bf)
    u = lora_down(xe[:, :K], dev(A, bf), s, out=xe[:, K:K + r])
    want_u = rnd((s * (x.astype(np.float64) @ A.T.astype(np.float64))).astype(np.float32))
    got_u = host(u)
    assert max_abs(got_u, want_u) <= 2 ** -7 * np.abs(want_u).max() and rel_l2(got_u, want_u) <= 4e-3
    assert float(xe[:, K + r:].abs().max()) == 0.0  # padding untouched
    # y += s' u B^T into a strided y view
    ye = torch.zeros(N, M + 32, dtype=bf, device="cuda")
    y0 = rnd(rng.standard_normal((N, M)).astype(np.float32))
    ye[:, :M] = dev(y0, bf)
    lora_up(xe[:, K:K + r], dev(B, bf), ye[:, :M], 2.0)
    want_y = y0 + 2.0 * (got_u.astype(np.float64) @ B.T.astype(np.float64))
    assert rel_l2(host(ye[:, :M]), want_y) <= 1e-2 and max_abs(host(ye[:, :M]), want_y) <= 2e-2 * np.abs(want_y).max()
    assert float(ye[:, M:].abs().max()) == 0.0
    # grads: dA-style [r, K] and dB-style [M, r]
    gA = lora_grad(xe[:, K:K + r], xe[:, :K], 1.5, transpose=False)
    np.testing.assert_allclose(host(gA), 1.5 * got_u.astype(np.float64).T @ x, rtol=1e-4, atol=1e-3)
    gB = lora_grad(xe[:, K:K + r], dev(dy, bf), 0.5, transpose=True)
    np.testing.assert_allclose(host(gB), 0.5 * dy.astype(np.float64).T @ got_u, rtol=1e-4, atol=1e-3)
    # the fused product carries the adapter term
    We = torch.zeros(M, K + pad, dtype=bf, device="cuda")
    We[:, :K] = dev(rnd(0.02 * rng.standard_normal((M, K)).astype(np.float32)), bf)
    We[:, K:K + r] = dev(B, bf)
    fused = host(torch.mm(xe, We.t()))
    ref = host(torch.mm(xe[:, :K], We[:, :K].t()).float() + torch.mm(xe[:, K:K + r].float(), We[:, K:K + r].t().float()))
    assert rel_l2(fused, ref) <= 1e-2


def test_lora_grad_many_matches_separate_calls():
    """fa_lora_grad_many: eighteen products of several token counts (1 to
    4096; ranks 4..64, so one- and two-accumulator products, dA and dB
    layouts, strided u and x views, a partial last column tile, two sets of
    launches) give the bits of separate fa_lora_grad calls, with U staged or
    read directly, and three of them match f64 products of the same values."""
    from foundry_attn.ops import lora_grad, lora_grad_many
    rng = np.random.default_rng(321)
    bf = torch.bfloat16
    rnd = oracle.bf16_round
    items = []
    for k, (N, r, C, tr) in enumerate([(300, 4, 256, False), (300, 16, 384, True), (64, 40, 128, False),
                                        (300, 48, 3072, True), (517, 64, 256, False), (1, 12, 512, True),
                                        (300, 33, 256, True), (4096, 16, 3072, False), (77, 8, 128, False),
                                        (300, 64, 384, True), (300, 20, 208, True), (512, 48, 3072, False),
                                        (512, 16, 3072, True), (4096, 48, 1024, False), (130, 16, 128, True),
                                        (300, 4, 256, True), (1000, 32, 640, False), (63, 64, 128, True)]):
        ue = torch.zeros(N, r + 8, dtype=bf, device="cuda")
        ue[:, 3:3 + r] = dev(rnd(rng.standard_normal((N, r)).astype(np.float32)), bf)
        xe = torch.zeros(N, C + 16, dtype=bf, device="cuda")
        xe[:, :C] = dev(rnd(rng.standard_normal((N, C)).astype(np.float32)), bf)
        items.append((ue[:, 3:3 + r], xe[:, :C], 0.5 + 0.25 * k, tr))
    many = lora_grad_many(items)
    one = [lora_grad(*it) for it in items]
    # The views above start 6 bytes into their rows, so the colsum reads a
    # staged U^T.  The same values in 16-byte aligned rows (every product
    # aligned) take the direct path, U read by DMA inside the colsum kernel
    # with no staging launch: the same bits.
    aligned = []
    for u, x, sc, tr in items:
        buf = torch.zeros(u.shape[0], 72, dtype=bf, device="cuda")
        buf[:, :u.shape[1]] = u
        aligned.append((buf[:, :u.shape[1]], x, sc, tr))
    direct = lora_grad_many(aligned)
    torch.cuda.synchronize()
    for k, (a, b) in enumerate(zip(many, one)):
        assert a.shape == b.shape and torch.equal(a, b), k
    for k, (a, b) in enumerate(zip(direct, many)):
        assert torch.equal(a, b), k
    for k in (3, 10, 12):  # C = 3072, C = 208 (a partial last column tile), 512 tokens
        u, x, sc, tr = items[k]
        want = sc * host(x).astype(np.float64).T @ host(u).astype(np.float64)  # [C, r]
        np.testing.assert_allclose(host(many[k]), want, rtol=1e-4, atol=1e-3)
        np.testing.assert_allclose(host(direct[k]), want, rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_prologue_multi_matches_separate_calls(dtype):
    """fa_qk_prologue_fwd_multi / _bwd_multi: the block's four segments (Q
    and K of the txt and img streams, different norm weights, tables and joint
    offsets) in one launch give the bits of four separate calls."""
    from foundry_attn import qk_prologue_bwd_multi, qk_prologue_multi
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    g = torch.Generator(device="cpu").manual_seed(11)
    T_txt, T_img, H, D = 77, 300, 6, 128
    S = T_txt + T_img
    axes = [16, 56, 56]
    pos = np.zeros((S, 3), np.float32)
    pos[:T_txt, 0] = np.arange(T_txt)
    pos[T_txt:, 1] = np.arange(T_img) // 20
    pos[T_txt:, 2] = np.arange(T_img) % 20
    cos, sin = rope_tables(pos, axes, 1e4, dtype=tdt)
    r = lambda *sh: torch.randn(*sh, generator=g).to(device="cuda", dtype=tdt)
    x = {(n, t): r(1, T, H, D) for n, T in (("txt", T_txt), ("img", T_img)) for t in "qk"}
    w = {t: (1 + 0.02 * torch.randn(D, generator=g)).to(device="cuda", dtype=tdt) for t in "qk"}
    off = {"txt": 0, "img": T_txt}
    tab = {"txt": (cos[:T_txt].contiguous(), sin[:T_txt].contiguous()),
           "img": (cos[T_txt:].contiguous(), sin[T_txt:].contiguous())}
    sep = {t: torch.full((1, S, H, D), float("nan"), dtype=tdt, device="cuda") for t in "qk"}
    one = {t: torch.full((1, S, H, D), float("nan"), dtype=tdt, device="cuda") for t in "qk"}
    segs = []
    for (n, t), xv in x.items():
        qk_prologue(xv, w[t], *tab[n], axes, out=sep[t], seq_offset=off[n])
        segs.append((xv, w[t], *tab[n], axes, one[t], off[n]))
    qk_prologue_multi(segs)
    torch.cuda.synchronize()
    for t in "qk":
        assert torch.equal(sep[t], one[t]), t
    dy = {t: r(1, S, H, D) for t in "qk"}
    dsep = {k: torch.empty_like(v) for k, v in x.items()}
    done = {k: torch.empty_like(v) for k, v in x.items()}
    bsegs = []
    for (n, t), xv in x.items():
        qk_prologue_bwd(xv, w[t], *tab[n], axes, dy[t], seq_offset=off[n], dx=dsep[(n, t)])
        bsegs.append((xv, w[t], *tab[n], axes, dy[t], off[n], done[(n, t)]))
    qk_prologue_bwd_multi(bsegs)
    torch.cuda.synchronize()
    for k in x:
        assert torch.equal(dsep[k], done[k]), k


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_prologue_bwd_multi_c2_shape_matches_oracle(dtype):
    """The backward the double block runs, at c2's shape: Q and K of the txt
    (512 tokens) and img (64 x 64) streams, H = 24, D = 128, in one
    fa_qk_prologue_bwd_multi launch.  x is the q or k slice of each stream's
    packed [T, 3, H, D] projection output and dx is written into the same
    slice of a packed gradient buffer (the block's strides); dy is the joint
    [1, 4608, H, D] gradient read at each stream's offset.  Every segment
    against the oracle's chain rule."""
    from foundry_attn import qk_prologue_bwd_multi
    bf = dtype == "bf16"
    tdt = torch.bfloat16 if bf else torch.float32
    rnd = oracle.bf16_round if bf else (lambda a: a.astype(np.float32))
    rng = np.random.default_rng(24)
    H, D, T_txt, S = C2.heads, C2.head_dim, C2.txt_len, C2.seq
    lens = {"txt": T_txt, "img": S - T_txt}
    off = {"txt": 0, "img": T_txt}
    pos = C2.positions()
    cos, sin = oracle.rope_tables(pos, C2.axes, C2.theta, bf16=bf)
    tc, ts = rope_tables(pos, C2.axes, C2.theta, dtype=tdt)
    tab = {n: (tc[off[n]:off[n] + lens[n]].contiguous(), ts[off[n]:off[n] + lens[n]].contiguous()) for n in lens}
    qkv = {n: rnd(rng.standard_normal((lens[n], 3, H, D)).astype(np.float32)) for n in lens}
    w = {t: rnd(1 + 0.02 * rng.standard_normal(D).astype(np.float32)) for t in "qk"}
    dy = {t: rnd(rng.standard_normal((1, S, H, D)).astype(np.float32)) for t in "qk"}
    tqkv = {n: dev(a, tdt) for n, a in qkv.items()}
    tdq = {n: torch.full(a.shape, float("nan"), dtype=tdt, device="cuda") for n, a in qkv.items()}
    tw, tdy = {t: dev(a, tdt) for t, a in w.items()}, {t: dev(a, tdt) for t, a in dy.items()}
    segs = []
    for i, t in enumerate("qk"):
        for n in ("txt", "img"):
            segs.append((tqkv[n][None, :, i], tw[t], *tab[n], C2.axes, tdy[t], off[n], tdq[n][None, :, i]))
    qk_prologue_bwd_multi(segs)
    torch.cuda.synchronize()
    for i, t in enumerate("qk"):
        for n in ("txt", "img"):
            want = oracle.qk_prologue_bwd(qkv[n][:, i], w[t], cos[off[n]:off[n] + lens[n]],
                                          sin[off[n]:off[n] + lens[n]], dy[t][0, off[n]:off[n] + lens[n]],
                                          C2.axes)
            got = host(tdq[n][:, i])
            r, m = rel_l2(got, want), max_abs(got, want)
            print(f"  d{t}.{n}: rel_l2={r:.2e} max_abs={m:.2e}", flush=True)
            if bf:
                assert r <= BF16_REL_L2 and m <= BF16_MAX_ABS * max(1.0, float(np.abs(want).max())), (t, n)
            else:
                assert r <= 1e-5, (t, n)
    for n in lens:  # the v slices were never written
        assert torch.isnan(tdq[n][:, 2]).all(), n
