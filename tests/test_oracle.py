"""Pins the CPU oracle (oracle/) before anything is checked against it.

Sources of truth, none of them the oracle's own formula:
  - the reference's golden fixtures (PyTorch CPU, fp32 and bf16 runs,
    tools/fixtures/block_*.safetensors; subset in tests/golden/):
    attention O/dQ/dK/dV, the QK prologue outputs, the LoRA linear output and
    the LoRA gradients (which also pin the prologue backward);
  - library routines (scipy logsumexp) and finite differences of an
    independent float64 forward;
  - exact invariants of softmax attention.
A planted mistake (in a float64 mutant, on the CPU) is shown to fail the same
fixture bounds, so the bounds discriminate.
"""
import numpy as np
import pytest
from scipy.special import logsumexp

import oracle
from helpers import load_golden, rel_l2

AXES4 = [32, 32, 32, 32]


def _fixture_positions():
    # tools/fixtures/gen_block.py:311-320: img (row, col, 0, 0) on a 4x4 grid,
    # txt (index, 0, 0, 0); the single block uses img-then-txt (fixture quirk).
    g = 4
    rows, cols = np.arange(16) // g, np.arange(16) % g
    z = np.zeros(16)
    pos_img = np.stack([rows, cols, z, z], -1).astype(np.float32)
    pos_txt = np.stack([np.arange(8), np.zeros(8), np.zeros(8), np.zeros(8)], -1).astype(np.float32)
    return pos_img, pos_txt, np.concatenate([pos_img, pos_txt])


@pytest.fixture(scope="module", params=["fp32", "bf16"])
def golden(request):
    return request.param, load_golden(request.param)


@pytest.mark.parametrize("blk", ["double", "single"])
def test_attention_matches_reference_fixture(golden, blk):
    tag, f = golden
    bf = tag == "bf16"
    q, k, v, out = (f[f"attn_in/{blk}.{n}"][None] for n in ("q", "k", "v", "attn"))
    o, lse = oracle.attn_fwd(q, k, v, bf16=bf)
    dq, dk, dv = oracle.attn_bwd(q, k, v, f[f"grad/attn/{blk}.out"][None], bf16=bf)
    tol = 1e-5 if not bf else 1e-6
    assert rel_l2(o, out) < tol
    assert rel_l2(dk, f[f"grad/attn/{blk}.k"][None]) < tol
    assert rel_l2(dv, f[f"grad/attn/{blk}.v"][None]) < tol
    # bf16 dQ: one bf16 rounding of an f32 GEMM may differ in accumulation order
    assert rel_l2(dq, f[f"grad/attn/{blk}.q"][None]) < (1e-5 if not bf else 1e-3)


def _lin(f, name, x, bf):
    w = lambda p: f.get(f"weights/{name}.{p}")
    return oracle.linear_lora(x, w("weight"), w("bias"), w("lora_a"), w("lora_b"), scale=2.0, bf16=bf)


def test_prologue_and_lora_match_reference_fixture(golden):
    tag, f = golden
    bf = tag == "bf16"
    tol = 1e-5 if not bf else 1e-6
    pos_img, pos_txt, pos_all = _fixture_positions()
    ci, si = oracle.rope_tables(pos_img, AXES4, 1e4, bf16=bf)
    ct, st = oracle.rope_tables(pos_txt, AXES4, 1e4, bf16=bf)
    ca, sa = oracle.rope_tables(pos_all, AXES4, 1e4, bf16=bf)
    ih, th = f["double.img_norm1"], f["double.txt_norm1"]

    def qk(lin, x, norm, c, s, n):
        h = _lin(f, lin, x, bf).reshape(n, 2, 128)
        return oracle.apply_rope(oracle.rms_norm(h, f[f"weights/{norm}.weight"], bf16=bf), c, s,
                                 AXES4, bf16=bf)

    qi = qk("double.img.to_q", ih, "double.img_q_norm", ci, si, 16)
    ki = qk("double.img.to_k", ih, "double.img_k_norm", ci, si, 16)
    qt = qk("double.txt.to_q", th, "double.txt_q_norm", ct, st, 8)
    kt = qk("double.txt.to_k", th, "double.txt_k_norm", ct, st, 8)
    assert rel_l2(qi, f["double.q"]) < tol
    assert rel_l2(ki, f["double.k"]) < tol
    # joint assembly: txt first, then img (lib.rs:363-365)
    assert rel_l2(np.concatenate([qt, qi]), f["attn_in/double.q"]) < tol
    assert rel_l2(np.concatenate([kt, ki]), f["attn_in/double.k"]) < tol
    # LoRA linear forward (to_v carries LoRA, scale 2): the img half of the joint v
    vi = _lin(f, "double.img.to_v", ih, bf).reshape(16, 2, 128)
    assert rel_l2(vi, f["attn_in/double.v"][8:]) < tol
    qkv = _lin(f, "single.to_qkv", f["single.norm1"], bf).reshape(24, 3, 2, 128)
    sq = oracle.apply_rope(oracle.rms_norm(qkv[:, 0], f["weights/single.q_norm.weight"], bf16=bf),
                           ca, sa, AXES4, bf16=bf)
    assert rel_l2(sq, f["single.q"]) < tol


def test_lora_and_prologue_backward_match_reference_gradients():
    """grad/{lora} in the fixture is PyTorch autograd through the whole block;
    the LoRA factors only feed one linear, so dL/d(lora) is a function of the
    attention input gradients — through the prologue backward for q/k."""
    f = load_golden("fp32")
    pos_img, _, pos_all = _fixture_positions()
    ci, si = oracle.rope_tables(pos_img, AXES4, 1e4)
    ca, sa = oracle.rope_tables(pos_all, AXES4, 1e4)
    W = lambda n, p: f[f"weights/{n}.{p}"]
    ih = f["double.img_norm1"]
    # to_v: dL/dv_img is the img half of grad/attn/double.v
    _, dA, dB = oracle.linear_lora_bwd(ih, W("double.img.to_v", "weight"),
                                       W("double.img.to_v", "lora_a"),
                                       W("double.img.to_v", "lora_b"),
                                       f["grad/attn/double.v"][8:].reshape(16, 256), scale=2.0,
                                       want_dx=False)
    assert rel_l2(dA, f["grad/double.img.to_v.lora_a"]) < 1e-5
    assert rel_l2(dB, f["grad/double.img.to_v.lora_b"]) < 1e-5
    # to_q: through RoPE + RMSNorm backward
    hq = _lin(f, "double.img.to_q", ih, False).reshape(16, 2, 128)
    dq = oracle.qk_prologue_bwd(hq, W("double.img_q_norm", "weight"), ci, si,
                                f["grad/attn/double.q"][8:], AXES4)
    _, dA, dB = oracle.linear_lora_bwd(ih, W("double.img.to_q", "weight"),
                                       W("double.img.to_q", "lora_a"),
                                       W("double.img.to_q", "lora_b"), dq.reshape(16, 256),
                                       scale=2.0, want_dx=False)
    assert rel_l2(dA, f["grad/double.img.to_q.lora_a"]) < 1e-5
    assert rel_l2(dB, f["grad/double.img.to_q.lora_b"]) < 1e-5
    # single.to_qkv: q, k through the prologue backward, v direct
    x = f["single.norm1"]
    qkv = _lin(f, "single.to_qkv", x, False).reshape(24, 3, 2, 128)
    dqq = oracle.qk_prologue_bwd(qkv[:, 0], W("single.q_norm", "weight"), ca, sa,
                                 f["grad/attn/single.q"], AXES4)
    dkk = oracle.qk_prologue_bwd(qkv[:, 1], W("single.k_norm", "weight"), ca, sa,
                                 f["grad/attn/single.k"], AXES4)
    dqkv = np.stack([dqq, dkk, f["grad/attn/single.v"]], 1).reshape(24, 768)
    _, dA, dB = oracle.linear_lora_bwd(x, W("single.to_qkv", "weight"),
                                       W("single.to_qkv", "lora_a"), W("single.to_qkv", "lora_b"),
                                       dqkv, scale=2.0, want_dx=False)
    assert rel_l2(dA, f["grad/single.to_qkv.lora_a"]) < 1e-5
    assert rel_l2(dB, f["grad/single.to_qkv.lora_b"]) < 1e-5


# ---- independent float64 forward, used only for finite differences --------
def _f64_forward(q, k, v, scale, keep=None):
    s = np.einsum("bihd,bjhd->bhij", q, k) * scale
    if keep is not None:
        s = np.where(keep[:, None, None, :] > 0, s, -np.inf)
    lse = logsumexp(s, axis=-1)
    p = np.exp(s - lse[..., None])
    return np.einsum("bhij,bjhd->bihd", p, v), lse


def _case(B=1, S=13, H=2, D=64, seed=0, masked=False):
    rng = np.random.default_rng(seed)
    q, k, v, do = (rng.standard_normal((B, S, H, D)).astype(np.float32) for _ in range(4))
    keep = None
    if masked:
        keep = (rng.random((B, S)) > 0.3).astype(np.uint8)
        keep[:, 0] = 1
    return q, k, v, do, keep


def test_lse_matches_scipy_logsumexp():
    q, k, v, do, keep = _case(B=2, S=29, H=3, D=64, masked=True)
    scale = 0.125
    _, lse = oracle.attn_fwd(q, k, v, scale=scale, key_keep=keep)
    s = np.einsum("bihd,bjhd->bhij", q.astype(np.float64), k.astype(np.float64)) * scale
    s = np.where(keep[:, None, None, :] > 0, s, -np.inf)
    np.testing.assert_allclose(lse, logsumexp(s, axis=-1), rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("masked", [False, True])
def test_gradients_match_finite_differences(masked):
    q, k, v, do, keep = _case(B=1, S=7, H=1, D=64, seed=3, masked=masked)
    scale = 0.2
    dq, dk, dv = oracle.attn_bwd(q, k, v, do, scale=scale, key_keep=keep)
    q64, k64, v64, do64 = (a.astype(np.float64) for a in (q, k, v, do))
    loss = lambda q_, k_, v_: float(np.sum(_f64_forward(q_, k_, v_, scale, keep)[0] * do64))
    rng = np.random.default_rng(11)
    eps = 1e-5
    for name, x, g in (("q", q64, dq), ("k", k64, dk), ("v", v64, dv)):
        for _ in range(6):
            idx = tuple(rng.integers(0, n) for n in x.shape)
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            args_p = {"q": (xp, k64, v64), "k": (q64, xp, v64), "v": (q64, k64, xp)}[name]
            args_m = {"q": (xm, k64, v64), "k": (q64, xm, v64), "v": (q64, k64, xm)}[name]
            fd = (loss(*args_p) - loss(*args_m)) / (2 * eps)
            assert abs(fd - g[idx]) < 1e-4 * (1 + abs(fd)), (name, idx, fd, g[idx])


def test_invariants():
    q, k, v, do, _ = _case(B=2, S=40, H=3, D=64, seed=5)
    scale = 1 / 8
    # uniform V rows -> O equals that row; V = 1 -> O = 1 (rows of P sum to 1)
    vu = np.broadcast_to(v[:, :1], v.shape).copy()
    o, _ = oracle.attn_fwd(q, k, vu, scale=scale)
    np.testing.assert_allclose(o, vu, rtol=1e-5, atol=1e-5)
    # a single kept key -> O = V of that key, LSE = its scaled score
    keep = np.zeros((2, 40), np.uint8)
    keep[:, 17] = 1
    o, lse = oracle.attn_fwd(q, k, v, scale=scale, key_keep=keep)
    np.testing.assert_allclose(o, np.broadcast_to(v[:, 17:18], v.shape), rtol=1e-6, atol=1e-6)
    s17 = np.einsum("bihd,bhd->bhi", q, k[:, 17]) * scale
    np.testing.assert_allclose(lse, s17, rtol=1e-5, atol=1e-5)
    # sum_j dK_j = 0 and sum_j dV_j = sum_i dO_i per (b, h)
    dq, dk, dv = oracle.attn_bwd(q, k, v, do, scale=scale)
    assert np.abs(dk.sum(1)).max() < 1e-4 * np.abs(dk).max()
    np.testing.assert_allclose(dv.sum(1), do.sum(1), rtol=1e-4, atol=1e-4)
    # key/value permutation equivariance
    perm = np.random.default_rng(2).permutation(40)
    o1, _ = oracle.attn_fwd(q, k, v, scale=scale)
    o2, _ = oracle.attn_fwd(q, k[:, perm], v[:, perm], scale=scale)
    np.testing.assert_allclose(o1, o2, rtol=1e-5, atol=1e-5)
    dq2, dk2, dv2 = oracle.attn_bwd(q, k[:, perm], v[:, perm], do, scale=scale)
    np.testing.assert_allclose(dk2, dk[:, perm], rtol=1e-4, atol=1e-5)
    # shifting every key by the same vector leaves O and dQ unchanged
    shift = np.random.default_rng(4).standard_normal((1, 1, 3, 64)).astype(np.float32)
    o3, _ = oracle.attn_fwd(q, k + shift, v, scale=scale)
    dq3, _, _ = oracle.attn_bwd(q, k + shift, v, do, scale=scale)
    np.testing.assert_allclose(o3, o1, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(dq3, dq, rtol=1e-3, atol=1e-4)


def test_mask_equals_unpadded_attention():
    q, k, v, do, keep = _case(B=1, S=50, H=2, D=64, seed=9, masked=True)
    scale = 0.1
    o, lse = oracle.attn_fwd(q, k, v, scale=scale, key_keep=keep)
    dq, dk, dv = oracle.attn_bwd(q, k, v, do, scale=scale, key_keep=keep)
    idx = np.flatnonzero(keep[0])
    ks, vs = k[:, idx], v[:, idx]
    # unpadded: queries attend over the kept keys only (q rows are all kept)
    s = np.einsum("bihd,bjhd->bhij", q, ks) * scale
    p = np.exp(s - logsumexp(s, axis=-1)[..., None])
    np.testing.assert_allclose(o, np.einsum("bhij,bjhd->bihd", p, vs), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(lse, logsumexp(s, axis=-1), rtol=1e-5, atol=1e-5)
    masked = np.flatnonzero(keep[0] == 0)
    assert np.all(dk[:, masked] == 0) and np.all(dv[:, masked] == 0)


def test_fully_masked_row_gives_zero_and_minus_inf():
    q, k, v, do, _ = _case(B=1, S=9, H=1, D=64)
    keep = np.zeros((1, 9), np.uint8)
    o, lse = oracle.attn_fwd(q, k, v, key_keep=keep)
    assert np.all(o == 0) and np.all(np.isneginf(lse))
    dq, dk, dv = oracle.attn_bwd(q, k, v, do, key_keep=keep)
    assert not np.any(dq) and not np.any(dk) and not np.any(dv)


def test_rope_tables_invariants():
    pos = np.array([[0, 0, 0], [3, 5, 7]], np.float32)
    cos, sin = oracle.rope_tables(pos, [16, 56, 56], 1e4)
    assert np.all(cos[0] == 1) and np.all(sin[0] == 0)
    np.testing.assert_allclose(cos ** 2 + sin ** 2, 1, atol=1e-6)
    # position 0 is the identity rotation; rotation preserves pair norms (f32)
    x = np.random.default_rng(0).standard_normal((2, 4, 128)).astype(np.float32)
    y = oracle.apply_rope(x, cos, sin, [16, 56, 56])
    np.testing.assert_array_equal(y[0], x[0])
    off = 0
    for w in (16, 56, 56):
        h = w // 2
        nx = x[1, :, off:off + h] ** 2 + x[1, :, off + h:off + w] ** 2
        ny = y[1, :, off:off + h] ** 2 + y[1, :, off + h:off + w] ** 2
        np.testing.assert_allclose(ny, nx, rtol=1e-5, atol=1e-6)
        off += w


def test_planted_mistakes_fail_fixture_bounds():
    """A float64 restatement with a planted mistake misses the fixture by far
    more than the bounds used above, so those bounds detect such mistakes."""
    f = load_golden("fp32")
    q, k, v = (f[f"attn_in/double.{n}"][None].astype(np.float64) for n in ("q", "k", "v"))
    do = f["grad/attn/double.out"][None].astype(np.float64)
    scale = 1 / np.sqrt(128)

    def grads(sign_rowsum=1.0, transpose_scores=False):
        s = np.einsum("bihd,bjhd->bhij", q, k) * scale
        if transpose_scores:
            s = np.swapaxes(s, -1, -2)
        p = np.exp(s - logsumexp(s, axis=-1)[..., None])
        dp = np.einsum("bihd,bjhd->bhij", do, v)
        ds = p * (dp - sign_rowsum * np.sum(dp * p, -1, keepdims=True)) * scale
        return np.einsum("bhij,bjhd->bihd", ds, k)

    good = grads()
    assert rel_l2(good, f["grad/attn/double.q"][None]) < 1e-5
    assert rel_l2(grads(sign_rowsum=-1.0), f["grad/attn/double.q"][None]) > 1e-1
    assert rel_l2(grads(transpose_scores=True), f["grad/attn/double.q"][None]) > 1e-1
