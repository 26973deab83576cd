"""CPU checks of the block-op oracle (oracle/block_oracle.c) against the
reference fixture and closed forms, before it is trusted as the GPU checker.

Pins:
  layer_norm_mod + modulation parts   double.img_norm1 / double.txt_norm1
      = layer_norm_mod(inputs/*, shift1, scale1), (shift1, scale1, gate1, ...)
      = chunk6(silu(temb) W_mod^T + b_mod)        (gen_block.py:199-208)
  gated residual                       double.img_post_attn
      = inputs/img + gate1 * (attn_img W_out^T + b_out)   (gen_block.py:235)
  AdamW                                opt1/* = one step from weights/* with grad/*
  tanh-GELU, SiLU                      torch's CPU reference forms
  gradients (ln_mod_bwd, gelu_bwd)     central finite differences
Each pin has a planted mistake that must fail it.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import load_block_golden, rel_l2


def mod_parts(f, bf16):
    c = oracle.silu(f["inputs/temb"][None, :], bf16=bf16)[0]
    m = f["weights/double.mod.weight"] @ c + f["weights/double.mod.bias"]
    if bf16:
        m = oracle.bf16_round(m)
    return np.split(m.astype(np.float32), 6)


@pytest.mark.parametrize("tag,tol", [("fp32", 2e-6), ("bf16", 1e-2)])
def test_ln_mod_and_mod_parts_match_fixture(tag, tol):
    f = load_block_golden(tag)
    bf = tag == "bf16"
    sh1, sc1 = mod_parts(f, bf)[:2]
    for stream in ("img", "txt"):
        y, _, _ = oracle.ln_mod_fwd(f[f"inputs/{stream}"], sh1, sc1, 1e-6, bf16=bf)
        r = rel_l2(y, f[f"double.{stream}_norm1"])
        print(tag, stream, r)
        assert r <= tol
    # planted mistake: scale instead of (1 + scale)
    y_bad, _, _ = oracle.ln_mod_fwd(f["inputs/img"], sh1, sc1 - 1.0, 1e-6, bf16=bf)
    assert rel_l2(y_bad, f["double.img_norm1"]) > 10 * tol


@pytest.mark.parametrize("tag,tol", [("fp32", 2e-6), ("bf16", 1e-2)])
def test_gated_residual_matches_fixture(tag, tol):
    f = load_block_golden(tag)
    bf = tag == "bf16"
    g1 = mod_parts(f, bf)[2]
    a = f["double.attn_img"].reshape(f["double.attn_img"].shape[0], -1)
    out = a @ f["weights/double.img.to_out.weight"].T + f["weights/double.img.to_out.bias"]
    if bf:
        out = oracle.bf16_round(out.astype(np.float32))
    y = oracle.gated_residual(f["inputs/img"], g1, out, bf16=bf)
    r = rel_l2(y, f["double.img_post_attn"])
    print(tag, r)
    assert r <= tol
    # planted mistake: the second gate instead of the first.  The gated branch
    # is ~1% of the result's norm, so only the fp32 fixture resolves it.
    if not bf:
        y_bad = oracle.gated_residual(f["inputs/img"], mod_parts(f, bf)[5], out, bf16=bf)
        assert rel_l2(y_bad, f["double.img_post_attn"]) > 1000 * tol


def test_adamw_step1_matches_fixture():
    """torch.optim.AdamW (the fixture) and adamw_step (lib.rs:477-510) round
    differently, so the bound is a few f32 ulps of the step size."""
    f = load_block_golden("fp32")
    names = sorted(k[len("opt1/"):] for k in f if k.startswith("opt1/"))
    assert len(names) == 6
    for nm in names:
        p0, g = f[f"weights/{nm}"], f[f"grad/{nm}"]
        z = np.zeros_like(p0)
        p1, m1, v1 = oracle.adamw_step(p0, g, z, z, step=1, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8)
        want = f[f"opt1/{nm}"]
        err = np.abs(p1 - want).max()
        print(nm, err)
        assert err <= 2e-9 + 1e-6 * np.abs(want).max()
        np.testing.assert_allclose(m1, 0.1 * g, rtol=1e-6, atol=0)
        np.testing.assert_allclose(v1, 0.001 * g * g, rtol=1e-5, atol=1e-30)
        # planted mistake: no bias correction moves the step by 10x
        p_bad = p0 - 1e-3 * (0.1 * g) / (np.sqrt(0.001 * g * g) + 1e-8)
        assert np.abs(p_bad - want).max() > 100 * max(err, 1e-9)


def test_adamw_ten_steps_closed_form():
    """With a constant gradient the moments have closed forms
    m_t = (1 - b1^t) g, v_t = (1 - b2^t) g^2, so every bias-corrected step is
    lr * g / (|g| + eps)."""
    rng = np.random.default_rng(3)
    g = rng.standard_normal(1000).astype(np.float32)
    p = rng.standard_normal(1000).astype(np.float32)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    p0 = p.copy()
    for t in range(1, 11):
        p, m, v = oracle.adamw_step(p, g, m, v, step=t)
    np.testing.assert_allclose(m, (1 - 0.9 ** 10) * g, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(p, p0 - 10 * 1e-3 * g / (np.abs(g) + 1e-8), rtol=0, atol=2e-6)


def test_gelu_and_silu_match_torch_forms():
    x = np.linspace(-8, 8, 4001, dtype=np.float32)
    want = torch.nn.functional.gelu(torch.from_numpy(x).double(), approximate="tanh").numpy()
    np.testing.assert_allclose(oracle.gelu_fwd(x), want, rtol=1e-6, atol=1e-7)
    ws = torch.nn.functional.silu(torch.from_numpy(x).double()).numpy()
    np.testing.assert_allclose(oracle.silu(x), ws, rtol=1e-6, atol=1e-7)
    # planted mistake: exact (erf) GELU differs from the tanh form by ~1e-3
    erf = torch.nn.functional.gelu(torch.from_numpy(x).double()).numpy()
    assert np.abs(erf - want).max() > 1e-4


def test_gelu_bwd_finite_difference():
    x = np.linspace(-6, 6, 241).astype(np.float64)
    h = 1e-3
    fd = (oracle.gelu_fwd((x + h).astype(np.float32)).astype(np.float64)
          - oracle.gelu_fwd((x - h).astype(np.float32)).astype(np.float64)) / (2 * h)
    d = oracle.gelu_bwd(np.ones_like(x, dtype=np.float32), x.astype(np.float32))
    np.testing.assert_allclose(d, fd, atol=3e-3)


def test_ln_mod_bwd_finite_difference():
    rng = np.random.default_rng(5)
    N, C = 3, 32
    x = rng.standard_normal((N, C)).astype(np.float32)
    sh = rng.standard_normal(C).astype(np.float32) * 0.1
    sc = rng.standard_normal(C).astype(np.float32) * 0.1
    dy = rng.standard_normal((N, C)).astype(np.float32)
    dres = rng.standard_normal((N, C)).astype(np.float32)
    _, mean, rstd = oracle.ln_mod_fwd(x, sh, sc, 1e-6)
    dx = oracle.ln_mod_bwd(x, dy, sc, mean, rstd, dres=dres)

    def loss(xx):
        y, _, _ = oracle.ln_mod_fwd(xx.astype(np.float32), sh, sc, 1e-6)
        return float((y.astype(np.float64) * dy).sum())

    h = 1e-2
    fd = np.zeros_like(x, dtype=np.float64)
    for i in range(N):
        for j in range(C):
            e = np.zeros_like(x)
            e[i, j] = h
            fd[i, j] = (loss(x + e) - loss(x - e)) / (2 * h)
    np.testing.assert_allclose(dx - dres, fd, atol=2e-3)
    # gradient of a normalised row sums to zero over the row (the part from dy)
    assert np.abs((dx - dres).sum(1)).max() < 1e-4
