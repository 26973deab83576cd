"""GPU parity of the double-stream LoRA block (config c4's unit) against the
CPU oracle.  Every block op goes through libfoundry_attn.so; the frozen base
linears are library GEMMs.  Gates: the ops at bf16 max-abs / rel-L2 from the
attention gates (2e-2 / 1e-2), f32 rel-L2 1e-4 (ln-mod backward 1e-3); the
whole block step (outputs, input gradients, LoRA gradients) at the same gate
as attention: bf16 rel-L2 <= 1e-2 with max-abs <= 2e-2 x max(1, peak), f32
rel-L2 <= 1e-4 (the reference's fp32 policy, docs/TESTING.md:15)."""
import numpy as np
import pytest
import torch

import block_ref  # noqa: E402  (oracle/ on sys.path via conftest)
import oracle
from block_case import make_case, make_single_case, oracle_mods, single_oracle_mods
from foundry_attn import block as fb
from helpers import check_gate, max_abs, rel_l2

pytestmark = pytest.mark.gpu


def dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device="cuda", dtype=dtype)


def host(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("C", [256, 3072, 4096])
def test_block_ops_match_oracle(dtype, C):
    bf = dtype == torch.bfloat16
    rng = np.random.default_rng(C)
    rnd = (lambda a: oracle.bf16_round(a.astype(np.float32))) if bf else (lambda a: a.astype(np.float32))
    N = 300
    x, dy, dres, b = (rnd(rng.standard_normal((N, C))) for _ in range(4))
    sh, sc, g = (rnd(0.1 * rng.standard_normal(C)) for _ in range(3))
    tol = (2e-2, 1e-2) if bf else (None, 1e-4)

    def chk(name, got, want, rel=None):
        r = rel_l2(got, want)
        print(f"  {name} C={C} {dtype}: rel_l2={r:.2e} max_abs={max_abs(got, want):.2e}", flush=True)
        assert r <= (rel or tol[1]), (name, r)
        if bf:
            assert max_abs(got, want) <= tol[0] * max(1.0, float(np.abs(want).max())), name

    y, mean, rstd = fb.ln_mod_fwd(dev(x, dtype), dev(sh, dtype), dev(sc, dtype), 1e-6, stats=True)
    wy, wmean, wrstd = oracle.ln_mod_fwd(x, sh, sc, 1e-6, bf16=bf)
    chk("ln_mod_fwd", host(y), wy)
    np.testing.assert_allclose(host(mean), wmean, rtol=0, atol=1e-5)
    np.testing.assert_allclose(host(rstd), wrstd, rtol=1e-5)
    dx = fb.ln_mod_bwd(dev(x, dtype), dev(dy, dtype), dev(sc, dtype), mean, rstd, 1e-6, dres=dev(dres, dtype))
    chk("ln_mod_bwd", host(dx), oracle.ln_mod_bwd(x, dy, sc, wmean, wrstd, dres=dres, bf16=bf),
        None if bf else 1e-3)
    chk("gated_residual", host(fb.gated_residual(dev(x, dtype), dev(g, dtype), dev(b, dtype))),
        oracle.gated_residual(x, g, b, bf16=bf))
    chk("gated_branch", host(fb.gated_residual(None, dev(g, dtype), dev(b, dtype))),
        oracle.gated_residual(None, g, b, bf16=bf))
    chk("gelu", host(fb.gelu(dev(b, dtype))), oracle.gelu_fwd(b, bf16=bf))
    chk("gelu_bwd", host(fb.gelu_bwd(dev(dy, dtype), dev(b, dtype))), oracle.gelu_bwd(dy, b, bf16=bf))
    chk("silu", host(fb.silu(dev(b, dtype))), oracle.silu(b, bf16=bf))
    # in-place gelu_bwd (out aliases the upstream gradient), as the block uses it
    t = dev(dy, dtype)
    fb.gelu_bwd(t, dev(b, dtype), out=t)
    chk("gelu_bwd_inplace", host(t), oracle.gelu_bwd(dy, b, bf16=bf))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("C", [256, 3072, 4096])
def test_fused_gated_ln_mod_matches_separate_ops(dtype, C):
    """gated_ln_mod_fwd gives the bits of gated_residual followed by
    ln_mod_fwd, and ln_mod_bwd_gate those of ln_mod_bwd followed by
    gated_residual(None, g, dx): on row views with padded strides (the double
    block's [dout | du | 0] operand), with the sum written in place over x,
    and against the oracle."""
    bf = dtype == torch.bfloat16
    rng = np.random.default_rng(7 + C)
    rnd = (lambda a: oracle.bf16_round(a.astype(np.float32))) if bf else (lambda a: a.astype(np.float32))
    N = 300
    x, b, dy, dres = (rnd(rng.standard_normal((N, C))) for _ in range(4))
    sh, sc, g = (rnd(0.1 * rng.standard_normal(C)) for _ in range(3))
    X, DY, DRES = dev(x, dtype), dev(dy, dtype), dev(dres, dtype)
    SH, SC, G = dev(sh, dtype), dev(sc, dtype), dev(g, dtype)
    wide = torch.zeros((N, C + 64), dtype=dtype, device="cuda")
    wide[:, :C] = dev(b, dtype)
    Bv = wide[:, :C]  # a strided branch view

    s_ref = fb.gated_residual(X, G, Bv)
    y_ref, m_ref, r_ref = fb.ln_mod_fwd(s_ref, SH, SC, 1e-6, stats=True)
    copy = torch.full((N, C + 64), 7.0, dtype=dtype, device="cuda")
    s, y, m, r = fb.gated_ln_mod_fwd(X, G, Bv, SH, SC, 1e-6, sum_copy=copy[:, :C])
    torch.cuda.synchronize()
    for name, got, want in (("sum", s, s_ref), ("y", y, y_ref), ("mean", m, m_ref), ("rstd", r, r_ref),
                            ("sum_copy", copy[:, :C], s_ref)):
        assert torch.equal(got, want), name
    assert bool((copy[:, C:] == 7.0).all()), "sum_copy wrote past its view"
    inplace = X.clone()
    s2, y2, _, _ = fb.gated_ln_mod_fwd(inplace, G, Bv, SH, SC, 1e-6, sum_out=inplace)
    torch.cuda.synchronize()
    assert torch.equal(inplace, s_ref) and torch.equal(y2, y_ref)
    ws = oracle.gated_residual(x, g, b, bf16=bf)
    wy, _, _ = oracle.ln_mod_fwd(ws, sh, sc, 1e-6, bf16=bf)
    tol = 2e-2 if bf else 1e-4
    assert rel_l2(host(y), wy) <= tol

    dx_ref = fb.ln_mod_bwd(s_ref, DY, SC, m_ref, r_ref, 1e-6, dres=DRES)
    gd_ref = fb.gated_residual(None, G, dx_ref)
    gwide = torch.full((N, C + 64), 7.0, dtype=dtype, device="cuda")
    dx, gd = fb.ln_mod_bwd_gate(s, DY, SC, m, r, G, 1e-6, dres=DRES, gated_out=gwide[:, :C])
    torch.cuda.synchronize()
    assert torch.equal(dx, dx_ref) and torch.equal(gd, gd_ref)
    assert bool((gwide[:, C:] == 7.0).all()), "gated_out wrote past its view"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_swiglu_fused_views_match_oracle(dtype):
    """silu(gate) * up and its gradients with gate and up read as column
    slices of one fused projection output [N, 3C + 2M] (the single block's
    layout) and the results written into column slices of wider buffers."""
    bf = dtype == torch.bfloat16
    rng = np.random.default_rng(7)
    rnd = (lambda a: oracle.bf16_round(a.astype(np.float32))) if bf else (lambda a: a.astype(np.float32))
    N, C, M = 333, 256, 768
    fused = rnd(2.0 * rng.standard_normal((N, 3 * C + 2 * M)))
    gate, up = fused[:, 3 * C:3 * C + M], fused[:, 3 * C + M:]
    dy = rnd(rng.standard_normal((N, M)))
    tf = dev(fused, dtype)
    tg, tu = tf[:, 3 * C:3 * C + M], tf[:, 3 * C + M:]
    joined = torch.zeros(N, C + M, dtype=dtype, device="cuda")
    y = fb.swiglu(tg, tu, out=joined[:, C:])
    assert y.data_ptr() == joined[:, C:].data_ptr()
    wy = oracle.swiglu_fwd(gate, up, bf16=bf)
    dfused = torch.zeros_like(tf)
    dg, du = fb.swiglu_bwd(dev(dy, dtype), tg, tu, dgate=dfused[:, 3 * C:3 * C + M], dup=dfused[:, 3 * C + M:])
    wdg, wdu = oracle.swiglu_bwd(dy, gate, up, bf16=bf)
    for name, got, want in (("swiglu", host(joined[:, C:]), wy), ("dgate", host(dg), wdg), ("dup", host(du), wdu)):
        r = rel_l2(got, want)
        print(f"  {name} {dtype}: rel_l2={r:.2e} max_abs={max_abs(got, want):.2e}", flush=True)
        if bf:
            assert r <= 1e-2 and max_abs(got, want) <= 2e-2 * max(1.0, float(np.abs(want).max())), name
        else:
            assert r <= 1e-5, name
    # nothing outside the slices was written
    assert float(joined[:, :C].abs().max()) == 0.0
    assert float(dfused[:, :3 * C].abs().max()) == 0.0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_adamw_matches_oracle_over_steps(dtype):
    bf = dtype == torch.bfloat16
    rng = np.random.default_rng(1)
    n = 70001
    p = rng.standard_normal(n).astype(np.float32) * 0.05
    if bf:
        p = oracle.bf16_round(p)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    tp, tm, tv = dev(p, dtype), dev(m, torch.float32), dev(v, torch.float32)
    for step in range(1, 6):
        g = rng.standard_normal(n).astype(np.float32) * 10.0 ** rng.uniform(-6, 0)
        fb.adamw_step(tp, dev(g, torch.float32), tm, tv, step)
        p, m, v = oracle.adamw_step(p, g, m, v, step, bf16=bf)
    torch.cuda.synchronize()
    # same operation order: f32 moments agree to the last bits, the parameter
    # to one bf16 ulp where a rounding tie flips
    np.testing.assert_allclose(host(tm), m, rtol=1e-6, atol=1e-12)
    np.testing.assert_allclose(host(tv), v, rtol=1e-6, atol=1e-20)
    if bf:
        assert np.mean(host(tp) != p) < 1e-3
        assert max_abs(host(tp), p) <= 2 ** -8 * float(np.abs(p).max())
    else:
        np.testing.assert_allclose(host(tp), p, rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_adamw_many_matches_separate_steps(dtype):
    """fa_adamw_step_many over 40 tensors (two launches of up to 32; sizes
    from 7 elements to more than 1024 x 256, which strides) gives the bits of
    40 separate fa_adamw_step calls, over two steps."""
    torch.manual_seed(9)
    sizes = [7, 256, 257, 49152, 300000] + [1000 + 97 * i for i in range(35)]
    mk = lambda n: (torch.randn(n, device="cuda").to(dtype), torch.randn(n, device="cuda"),
                    torch.zeros(n, device="cuda"), torch.zeros(n, device="cuda"))
    many = [mk(n) for n in sizes]
    one = [tuple(t.clone() for t in item) for item in many]
    for step in (1, 2):
        grads = [torch.randn(n, device="cuda") for n in sizes]
        fb.adamw_step_many([(p, g, m, v) for (p, _, m, v), g in zip(many, grads)], step, lr=3e-3)
        for (p, _, m, v), g in zip(one, grads):
            fb.adamw_step(p, g, m, v, step, lr=3e-3)
    torch.cuda.synchronize()
    for a, b in zip(many, one):
        for x, y in zip(a[::2] + a[3:], b[::2] + b[3:]):
            assert torch.equal(x, y)


def device_block(case, dtype, **kw):
    ws = {}
    for name in ("txt", "img"):
        w = case["W"][name]
        sw = fb.StreamWeights(w_qkv=dev(w["w_qkv"], dtype), w_out=dev(w["w_out"], dtype),
                              w1=dev(w["w1"], dtype), w2=dev(w["w2"], dtype), q_norm=dev(w["q_norm"], dtype),
                              k_norm=dev(w["k_norm"], dtype), w_mod=dev(w["w_mod"], dtype))
        for t in fb.LORA_TARGETS:
            sw.lora_a[t] = dev(w["lora_a"][t], dtype)
            sw.lora_b[t] = dev(w["lora_b"][t], dtype)
            for part, P in (("a", w["lora_a"][t]), ("b", w["lora_b"][t])):
                sw.m[f"{t}.{part}"] = torch.zeros(P.shape, dtype=torch.float32, device="cuda")
                sw.v[f"{t}.{part}"] = torch.zeros(P.shape, dtype=torch.float32, device="cuda")
        ws[name] = sw
    blk = fb.DoubleBlockLoRA(ws, case["H"], case["D"], case["T"], case["rows"], case["cols"], axes=case["axes"],
                             lora_scale=case["scale"], **kw)
    blk.set_conditioning(dev(case["c"], dtype))
    return blk


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("want_dx", [False, True])
def test_block_step_matches_oracle(dtype, want_dx):
    bf = dtype == torch.bfloat16
    case = oracle_mods(make_case(C=256, H=2, T=16, rows=4, cols=8, r=4, bf16=bf, seed=5))
    blk = device_block(case, dtype)
    for name in ("txt", "img"):  # the device modulation parts equal the oracle's
        for i in range(6):
            r = rel_l2(host(blk.w[name].mod[i]), case["W"][name]["mod"][i])
            assert r <= (1e-2 if bf else 1e-5), (name, i, r)
    x = {k: dev(v, dtype) for k, v in case["x"].items()}
    dy = {k: dev(v, dtype) for k, v in case["dy"].items()}
    y, grads = blk.train_step(x, dy, want_dx=want_dx)
    torch.cuda.synchronize()
    wy, wgrads, wupd = block_ref.block_step(case["x"], case["dy"], case["W"], case["H"], case["D"], case["cos"],
                                            case["sin"], case["axes"], case["scale"], bf16=bf, want_dx=want_dx)
    for name in ("txt", "img"):
        check_gate(f"y.{name}", host(y[name]), wy[name], bf)
        if want_dx:
            check_gate(f"dx.{name}", host(grads[(name, "x")]), wgrads[(name, "x")], bf)
    for key, g in wgrads.items():
        if key[1] == "x":
            continue
        wa, wb = g
        da, db = grads[key]
        check_gate(f"grad {key} dA", host(da), wa, bf)
        check_gate(f"grad {key} dB", host(db), wb, bf)
        a1, b1 = wupd[key]
        w = blk.w[key[0]]
        # one AdamW step moves each factor by ~lr * sign(g): compare the step
        step_a = host(w.lora_a[key[1]]) - case["W"][key[0]]["lora_a"][key[1]]
        step_b = host(w.lora_b[key[1]]) - case["W"][key[0]]["lora_b"][key[1]]
        wa1 = a1 - case["W"][key[0]]["lora_a"][key[1]]
        wb1 = b1 - case["W"][key[0]]["lora_b"][key[1]]
        agree = np.mean(np.sign(step_a) == np.sign(wa1)), np.mean(np.sign(step_b) == np.sign(wb1))
        print(f"  update {key}: sign agreement {agree[0]:.4f} {agree[1]:.4f}", flush=True)
        assert min(agree) >= (0.97 if bf else 0.999), key


def test_fused_gelu_block_matches_oracle():
    """fused_gelu: W1 and W2's dX product as fa_gemm_bf16 with the GELU /
    GELU-gradient epilogues.  Widths multiples of 256 (512 tokens, MLP 1024)
    so that both streams take the fused path; against the oracle, and against
    the same block with the library GEMM and separate GELU passes."""
    case = oracle_mods(make_case(C=256, H=2, T=256, rows=16, cols=16, r=4, bf16=True, seed=9))
    x = {k: dev(v, torch.bfloat16) for k, v in case["x"].items()}
    dy = {k: dev(v, torch.bfloat16) for k, v in case["dy"].items()}
    out = {}
    for fused in (False, True):
        blk = device_block(case, torch.bfloat16, fused_gelu=fused)
        assert all(blk._gelu_fused(n, b) == fused for n in ("txt", "img") for b in (False, True))
        y, grads = blk.forward_backward(x, dy, want_dx=True)
        torch.cuda.synchronize()
        out[fused] = _flat(y, grads)
    wy, wgrads, _ = block_ref.block_step(case["x"], case["dy"], case["W"], case["H"], case["D"], case["cos"],
                                         case["sin"], case["axes"], case["scale"], bf16=True, want_dx=True)
    for name in ("txt", "img"):
        check_gate(f"y.{name}", host(out[True][("y", name)]), wy[name], True)
        check_gate(f"dx.{name}", host(out[True][((name, "x"), 0)]), wgrads[(name, "x")], True)
    for key, g in wgrads.items():
        if key[1] != "x":
            check_gate(f"grad {key} dA", host(out[True][(key, 0)]), g[0], True)
            check_gate(f"grad {key} dB", host(out[True][(key, 1)]), g[1], True)
    for k, t in out[False].items():
        check_gate(f"fused vs library {k}", host(out[True][k]), host(t), True)


def test_refresh_adapters_after_changing_factors():
    """LoRA factors changed outside apply_adamw -- a new tensor assigned to
    lora_a[t] (as a LoRA-file loader would), an in-place copy into
    lora_b[t] -- followed by refresh_adapters() give the bits of blocks built
    from the changed factors: the double block (q/k/v adapters stacked, their
    transposes cached) and the single block (adapters carried by its GEMMs)."""
    import copy
    bf = torch.bfloat16
    rng = np.random.default_rng(77)
    rnd = oracle.bf16_round
    case = oracle_mods(make_case(C=256, H=2, T=16, rows=4, cols=8, r=4, bf16=True, seed=7))
    case2 = copy.deepcopy(case)
    blk = device_block(case, bf)
    for name in ("txt", "img"):
        W2 = case2["W"][name]
        W2["lora_a"]["q"] = rnd(rng.standard_normal(W2["lora_a"]["q"].shape).astype(np.float32) / 4)
        W2["lora_b"]["k"] = rnd(0.05 * rng.standard_normal(W2["lora_b"]["k"].shape).astype(np.float32))
        blk.w[name].lora_a["q"] = dev(W2["lora_a"]["q"], bf)
        blk.w[name].lora_b["k"].copy_(dev(W2["lora_b"]["k"], bf))
    blk.refresh_adapters()
    ref = device_block(case2, bf)
    x = {k: dev(v, bf) for k, v in case["x"].items()}
    dy = {k: dev(v, bf) for k, v in case["dy"].items()}
    (y1, g1), (y2, g2) = (b.forward_backward(x, dy, want_dx=True) for b in (blk, ref))
    torch.cuda.synchronize()
    for name in ("txt", "img"):
        assert torch.equal(y1[name], y2[name]), name
    assert g1.keys() == g2.keys()
    for key in g1:
        parts = (g1[key],) if key[1] == "x" else g1[key]
        want = (g2[key],) if key[1] == "x" else g2[key]
        for a, b in zip(parts, want):
            assert torch.equal(a, b), key

    sc = single_oracle_mods(make_single_case(C=256, H=2, T=40, rows=8, cols=12, r=4, bf16=True, seed=9))
    sc2 = copy.deepcopy(sc)
    sblk = device_single_block(sc, bf)
    sc2["W"]["lora_a"]["to_out"] = rnd(rng.standard_normal(sc["W"]["lora_a"]["to_out"].shape).astype(np.float32) / 4)
    sc2["W"]["lora_b"]["to_in"] = rnd(0.05 * rng.standard_normal(sc["W"]["lora_b"]["to_in"].shape).astype(np.float32))
    sblk.w.lora_a["to_out"].copy_(dev(sc2["W"]["lora_a"]["to_out"], bf))
    sblk.w.lora_b["to_in"].copy_(dev(sc2["W"]["lora_b"]["to_in"], bf))
    sblk.refresh_adapters()
    sref = device_single_block(sc2, bf)
    (y1, g1), (y2, g2) = (b.forward_backward(dev(sc["x"], bf), dev(sc["dy"], bf), want_dx=True) for b in (sblk, sref))
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert g1.keys() == g2.keys()
    for key in g1:
        parts = (g1[key],) if key == "x" else g1[key]
        want = (g2[key],) if key == "x" else g2[key]
        for a, b in zip(parts, want):
            assert torch.equal(a, b), key


@pytest.mark.parametrize("dx_weights_t", [False, True], ids=["strided_dx", "transposed_dx"])
def test_refresh_frozen_after_changing_weights(dx_weights_t):
    """Frozen weights changed in place (w_qkv, w_out, w1, w2 of both streams)
    followed by refresh_frozen() give the bits of a block built from the
    changed weights: the adapter-carrying qkv / out operands, the gate-folded
    W2g = diag(g2) W2 and (with dx_weights_t) the transposed copies all follow
    the new weights."""
    import copy
    bf = torch.bfloat16
    rng = np.random.default_rng(78)
    case = oracle_mods(make_case(C=256, H=2, T=16, rows=4, cols=8, r=4, bf16=True, seed=8))
    case2 = copy.deepcopy(case)
    blk = device_block(case, bf, dx_weights_t=dx_weights_t)
    assert blk._fold_g2
    for name in ("txt", "img"):
        for key in ("w_qkv", "w_out", "w1", "w2"):
            W = case2["W"][name][key]
            case2["W"][name][key] = oracle.bf16_round(W + 0.02 * rng.standard_normal(W.shape).astype(np.float32))
            getattr(blk.w[name], key).copy_(dev(case2["W"][name][key], bf))
    blk.refresh_frozen()
    ref = device_block(case2, bf, dx_weights_t=dx_weights_t)
    x = {k: dev(v, bf) for k, v in case["x"].items()}
    dy = {k: dev(v, bf) for k, v in case["dy"].items()}
    (y1, g1), (y2, g2) = (b.forward_backward(x, dy, want_dx=True) for b in (blk, ref))
    torch.cuda.synchronize()
    for name in ("txt", "img"):
        assert torch.equal(y1[name], y2[name]), name
    assert g1.keys() == g2.keys()
    for key in g1:
        parts = (g1[key],) if key[1] == "x" else g1[key]
        want = (g2[key],) if key[1] == "x" else g2[key]
        for a, b in zip(parts, want):
            assert torch.equal(a, b), key


def test_c4_block_step_properties():
    """The full c4 block (4096 img + 512 txt tokens, dim 3072): one step gives
    finite outputs, nonzero finite LoRA gradients that repeat bit for bit, and
    an AdamW update of every factor."""
    from foundry_attn.configs import C4
    rows = int(C4.img_tokens ** 0.5)
    blk = fb.random_block(C4.hidden, C4.heads, C4.txt_tokens, rows, C4.img_tokens // rows, C4.mlp_ratio,
                          C4.lora_rank, C4.lora_alpha)
    g = torch.Generator(device="cuda").manual_seed(4)
    blk.set_conditioning(torch.randn(C4.hidden, device="cuda", generator=g).to(torch.bfloat16))
    x = {"img": torch.randn(C4.img_tokens, C4.hidden, device="cuda", generator=g).to(torch.bfloat16),
         "txt": torch.randn(C4.txt_tokens, C4.hidden, device="cuda", generator=g).to(torch.bfloat16)}
    dy = {k: torch.randn(v.shape, device="cuda", generator=g).to(torch.bfloat16) for k, v in x.items()}
    y1, g1 = blk.forward_backward(x, dy)
    y1 = {k: v.clone() for k, v in y1.items()}
    g1 = {k: (a.clone(), b.clone()) for k, (a, b) in g1.items()}
    y2, g2 = blk.forward_backward(x, dy)
    torch.cuda.synchronize()
    for k in y1:
        assert torch.isfinite(y1[k].float()).all() and torch.equal(y1[k], y2[k]), k
    assert len(g1) == 8
    for k, (da, db) in g1.items():
        assert torch.isfinite(da).all() and torch.isfinite(db).all(), k
        assert float(da.abs().max()) > 0 and float(db.abs().max()) > 0, k
        assert torch.equal(da, g2[k][0]) and torch.equal(db, g2[k][1]), k
    before = {k: (blk.w[k[0]].lora_a[k[1]].clone(), blk.w[k[0]].lora_b[k[1]].clone()) for k in g1}
    blk.apply_adamw(g1)
    torch.cuda.synchronize()
    for k, (a0, b0) in before.items():
        assert not torch.equal(a0, blk.w[k[0]].lora_a[k[1]]), k
        assert not torch.equal(b0, blk.w[k[0]].lora_b[k[1]]), k


def test_c4_full_size_step_matches_oracle():
    """Config c4 at full size (img 4096 = 64 x 64 + txt 512 tokens, dim 3072,
    24 x 128 heads, MLP 4x, LoRA r16 alpha 16 on q/k/v/out of both streams,
    A ~ N(0, 1/r^2), B ~ N(0, 1e-3^2)): one bf16 block step with the
    block-input gradient against the composed CPU restatement (block_ref) of
    the reference's bf16 algorithm, as the reference's block test compares
    its gradients (block_backward.rs:34-136).

    Gate: both block outputs, both dX and the v / out adapters' dA / dB at the
    bf16 gate (rel-L2 <= 1e-2, max-abs <= 2e-2 x max(1, peak)).  The q and k
    adapters' gradients sit at the bf16 noise floor of this shape and are
    held to rel-L2 <= 1.5e-2 instead: q and k are RMS-normalised, so the
    scores have a standard deviation near 11 and the softmax amplifies a
    one-ulp difference in q or k, and the kernels round dS to bf16 for the
    dQ / dK MFMAs where the reference runs those two products in f32.  The
    reference's own bf16 algorithm is as far from exact: every tensor is also
    compared with the same restatement run in f32, where the bf16 restatement
    measures 0.46-0.88e-2 rel-L2 and this path 0.46-1.22e-2 (seed 41).  This
    path must stay within 1.5e-2 of the f32 result for every tensor."""
    import copy
    case = make_case(C=3072, H=24, T=512, rows=64, cols=64, r=16, alpha=16.0, bf16=True, seed=41)
    for name in ("txt", "img"):
        for t in fb.LORA_TARGETS:
            b = case["W"][name]["lora_b"][t]
            case["W"][name]["lora_b"][t] = oracle.bf16_round(b * (1e-3 / 0.02))
    case = oracle_mods(case)
    blk = device_block(case, torch.bfloat16)
    x = {k: dev(v, torch.bfloat16) for k, v in case["x"].items()}
    dy = {k: dev(v, torch.bfloat16) for k, v in case["dy"].items()}
    y, grads = blk.forward_backward(x, dy, want_dx=True)
    torch.cuda.synchronize()
    y = {k: host(v) for k, v in y.items()}
    grads = {k: (host(v) if k[1] == "x" else tuple(host(t) for t in v)) for k, v in grads.items()}
    wy, wgrads, _ = block_ref.block_step(case["x"], case["dy"], case["W"], case["H"], case["D"], case["cos"],
                                         case["sin"], case["axes"], case["scale"], bf16=True, want_dx=True)
    # the same restatement in f32 on the same (bf16-valued) inputs
    c32 = copy.deepcopy(case)
    c32["bf16"] = False
    c32 = oracle_mods(c32)
    T, I = case["T"], case["rows"] * case["cols"]
    pos = np.zeros((T + I, 3), np.float32)
    pos[:T, 0] = np.arange(T)
    rr, cc = np.meshgrid(np.arange(case["rows"]), np.arange(case["cols"]), indexing="ij")
    pos[T:, 1], pos[T:, 2] = rr.ravel(), cc.ravel()
    cos, sin = oracle.rope_tables(pos, case["axes"], 1e4, bf16=False)
    fy, fgrads, _ = block_ref.block_step(c32["x"], c32["dy"], c32["W"], c32["H"], c32["D"],
                                         {"txt": cos[:T], "img": cos[T:]}, {"txt": sin[:T], "img": sin[T:]},
                                         c32["axes"], c32["scale"], bf16=False, want_dx=True)

    def both(label, got, want, want32, noise_floor=False):
        r32, o32 = rel_l2(got, want32), rel_l2(want, want32)
        print(f"  {label}: vs f32 restatement {r32:.2e} (bf16 restatement vs f32: {o32:.2e})", flush=True)
        assert r32 <= 1.5e-2, (label, r32)
        if not noise_floor:
            check_gate(label, got, want, True)
            return
        r, m = rel_l2(got, want), max_abs(got, want)
        print(f"  {label}: rel_l2={r:.2e} max_abs={m:.2e} (q/k adapter: rel-L2 gate 1.5e-2)", flush=True)
        assert r <= 1.5e-2 and m <= 2e-2 * max(1.0, float(np.abs(want).max())), (label, r, m)

    for name in ("txt", "img"):
        both(f"y.{name}", y[name], wy[name], fy[name])
        both(f"dx.{name}", grads[(name, "x")], wgrads[(name, "x")], fgrads[(name, "x")])
    n_adapters = 0
    for key, g in wgrads.items():
        if key[1] == "x":
            continue
        (wa, wb), (da, db), (fa_, fb_) = g, grads[key], fgrads[key]
        floor = key[1] in ("q", "k")
        both(f"grad {key} dA", da, wa, fa_, floor)
        both(f"grad {key} dB", db, wb, fb_, floor)
        n_adapters += 1
    assert n_adapters == 8


def device_single_block(case, dtype):
    W = case["W"]
    w = fb.SingleWeights(w_in=dev(W["w_in"], dtype), w_out=dev(W["w_out"], dtype), q_norm=dev(W["q_norm"], dtype),
                         k_norm=dev(W["k_norm"], dtype), w_mod=dev(W["w_mod"], dtype))
    for t in fb.SINGLE_LORA_TARGETS:
        w.lora_a[t], w.lora_b[t] = dev(W["lora_a"][t], dtype), dev(W["lora_b"][t], dtype)
        for part, arr in (("a", W["lora_a"][t]), ("b", W["lora_b"][t])):
            w.m[f"{t}.{part}"] = torch.zeros(arr.shape, dtype=torch.float32, device="cuda")
            w.v[f"{t}.{part}"] = torch.zeros(arr.shape, dtype=torch.float32, device="cuda")
    blk = fb.SingleBlockLoRA(w, case["H"], case["D"], case["T"], case["rows"], case["cols"], axes=case["axes"],
                             theta=case["theta"], lora_scale=case["scale"])
    blk.set_conditioning(dev(case["c"], dtype))
    return blk


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_single_block_step_matches_oracle(dtype):
    """The single-stream klein block (fused to_in -> q/k/v + SwiGLU, fused
    to_out over cat(attention, activation), one gate), LoRA on both fused
    projections, klein RoPE (axes 32 x 4, theta 2000, txt (0,0,0,l), img
    (0,h,w,0)); one train step with the input gradient, against the oracle
    restatement."""
    bf = dtype == torch.bfloat16
    case = single_oracle_mods(make_single_case(C=256, H=2, T=40, rows=8, cols=12, r=4, bf16=bf, seed=9))
    blk = device_single_block(case, dtype)
    for i in range(3):
        r = rel_l2(host(blk.w.mod[i]), case["W"]["mod"][i])
        assert r <= (1e-2 if bf else 1e-5), (i, r)
    np.testing.assert_array_equal(host(blk.cos), case["cos"])
    y, grads = blk.train_step(dev(case["x"], dtype), dev(case["dy"], dtype))
    torch.cuda.synchronize()
    wy, wgrads, wupd, wdx = block_ref.single_block_step(case["x"], case["dy"], case["W"], case["H"], case["D"],
                                                        case["cos"], case["sin"], case["axes"], case["scale"],
                                                        bf16=bf)
    for name, got, want in (("y", host(y), wy), ("dx", host(grads["x"]), wdx)):
        check_gate(name, got, want, bf)
    for t in fb.SINGLE_LORA_TARGETS:
        (da, db), (wa, wb) = grads[t], wgrads[t]
        check_gate(f"grad {t} dA", host(da), wa, bf)
        check_gate(f"grad {t} dB", host(db), wb, bf)
        a1, b1 = wupd[t]
        step_a = host(blk.w.lora_a[t]) - case["W"]["lora_a"][t]
        step_b = host(blk.w.lora_b[t]) - case["W"]["lora_b"][t]
        agree = (np.mean(np.sign(step_a) == np.sign(a1 - case["W"]["lora_a"][t])),
                 np.mean(np.sign(step_b) == np.sign(b1 - case["W"]["lora_b"][t])))
        print(f"  update {t}: sign agreement {agree[0]:.4f} {agree[1]:.4f}", flush=True)
        assert min(agree) >= (0.97 if bf else 0.999), t


def test_klein_single_block_step_properties():
    """The single block at klein size (dim 3072, 24 heads, MLP 3 x dim, 512 txt
    + 4096 img tokens): finite outputs and gradients, bit-for-bit repeatable,
    nonzero LoRA gradients."""
    from foundry_attn.configs import C4
    rows = int(C4.img_tokens ** 0.5)
    blk = fb.random_single_block(C4.hidden, C4.heads, C4.txt_tokens, rows, C4.img_tokens // rows,
                                 rank=C4.lora_rank, alpha=C4.lora_alpha)
    g = torch.Generator(device="cuda").manual_seed(6)
    blk.set_conditioning(torch.randn(C4.hidden, device="cuda", generator=g).to(torch.bfloat16))
    S = C4.txt_tokens + C4.img_tokens
    x = torch.randn(S, C4.hidden, device="cuda", generator=g).to(torch.bfloat16)
    dy = torch.randn(S, C4.hidden, device="cuda", generator=g).to(torch.bfloat16)
    y1, g1 = blk.forward_backward(x, dy)
    y1 = y1.clone()
    g1 = {k: (tuple(t.clone() for t in v) if isinstance(v, tuple) else v.clone()) for k, v in g1.items()}
    y2, g2 = blk.forward_backward(x, dy)
    torch.cuda.synchronize()
    assert torch.isfinite(y1.float()).all() and torch.equal(y1, y2)
    assert torch.isfinite(g1["x"].float()).all() and torch.equal(g1["x"], g2["x"])
    for t in fb.SINGLE_LORA_TARGETS:
        for a, b in zip(g1[t], g2[t]):
            assert torch.isfinite(a).all() and float(a.abs().max()) > 0 and torch.equal(a, b), t


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_copy2d_many_matches_torch_copies(dtype):
    """fa_copy2d_many over 40 views (two launches): transposed sources,
    strided destinations inside wider buffers, column blocks -- every
    destination equals torch's copy_, and the bytes around it are untouched."""
    g = torch.Generator(device="cuda").manual_seed(5)
    pairs, want, bufs = [], [], []
    for i in range(40):
        r, c = 1 + (7 * i) % 48, 16 + (37 * i) % 300
        src = torch.randn(c, r, device="cuda", generator=g).to(dtype).t() if i % 3 == 0 else \
            torch.randn(r, c, device="cuda", generator=g).to(dtype)
        buf = torch.full((r + 3, c + 9), -7.0, device="cuda", dtype=dtype)
        dst = buf[1:1 + r, 4:4 + c] if i % 2 else buf[:c, :r].t() if c + 3 <= r else buf[2:2 + r, :c]
        ref = buf.clone()
        ref_dst = ref[1:1 + r, 4:4 + c] if i % 2 else ref[:c, :r].t() if c + 3 <= r else ref[2:2 + r, :c]
        ref_dst.copy_(src)
        pairs.append((src, dst))
        want.append(ref)
        bufs.append(buf)
    fb.copy2d_many(pairs)
    torch.cuda.synchronize()
    for i, (b, w) in enumerate(zip(bufs, want)):
        assert torch.equal(b, w), i


def _flat(y, grads):
    """Copies of a block step's outputs as a name -> tensor dict."""
    out = {}
    for k, v in (y.items() if isinstance(y, dict) else [("y", y)]):
        out[("y", k)] = v.clone()
    for k, v in grads.items():
        for i, t in enumerate(v if isinstance(v, tuple) else (v,)):
            out[(k, i)] = t.clone()
    return out


@pytest.mark.parametrize("kind", ["double", "single"])
def test_graphed_train_step_replays_match_eager(kind):
    """GraphedTrainStep (forward + backward captured in one HIP graph): four
    replays with an AdamW step between them (the LoRA factors and the
    adapter operands the graph reads change every step; before the last, the
    conditioning changes too) each give the bits of an eager forward_backward
    on the same state, run right after the replay with a synchronisation
    between; calling the step replays and applies AdamW."""
    bf = torch.bfloat16
    if kind == "double":
        case = oracle_mods(make_case(C=256, H=2, T=16, rows=4, cols=8, r=4, bf16=True, seed=5))
        blk = device_block(case, bf)
        x = {k: dev(v, bf) for k, v in case["x"].items()}
        dy = {k: dev(v, bf) for k, v in case["dy"].items()}
    else:
        sc = single_oracle_mods(make_single_case(C=256, H=2, T=40, rows=8, cols=12, r=4, bf16=True, seed=9))
        blk = device_single_block(sc, bf)
        x, dy = dev(sc["x"], bf), dev(sc["dy"], bf)
    c = case["c"] if kind == "double" else sc["c"]
    gs = fb.GraphedTrainStep(blk, x, dy, want_dx=True)
    for i in range(4):
        if i == 3:  # new conditioning: the modulation (and diag(g2) W2) change in place
            blk.set_conditioning(dev(0.5 * c, bf))
        gs.graph.replay()
        torch.cuda.synchronize()
        got = _flat(gs.y, gs.grads)
        want = _flat(*blk.forward_backward(x, dy, want_dx=True))
        torch.cuda.synchronize()
        assert got.keys() == want.keys()
        for k in got:
            assert torch.equal(got[k], want[k]), (i, k)
        grads = {k: v for k, v in gs.grads.items()}
        blk.apply_adamw(grads)
    before = blk.step_count
    a_before = (blk.w["img"] if kind == "double" else blk.w).lora_a["q" if kind == "double" else "to_in"].clone()
    gs()
    torch.cuda.synchronize()
    assert blk.step_count == before + 1
    a_after = (blk.w["img"] if kind == "double" else blk.w).lora_a["q" if kind == "double" else "to_in"]
    assert not torch.equal(a_before, a_after)


def test_tuned_gemm_file_loads_and_tuned_shapes_stay_accurate():
    """The packaged TunableOp file (solutions measured on MI355X for the block
    GEMM shapes) loads read-only on this image, and a tuned shape (the txt
    stream's fused qkv projection, 512 x 3072 -> 9216) still agrees with an
    f32 product."""
    from foundry_attn import gemm_tuning
    assert gemm_tuning.enable(), "TunableOp refused the packaged file (library versions differ?)"
    assert torch.cuda.tunable.is_enabled() and not torch.cuda.tunable.tuning_is_enabled()
    g = torch.Generator(device="cuda").manual_seed(8)
    a = torch.randn(512, 3072, device="cuda", generator=g).to(torch.bfloat16)
    w = (0.02 * torch.randn(9216, 3072, device="cuda", generator=g)).to(torch.bfloat16)
    got = torch.mm(a, w.t()).float()
    ref = torch.mm(a.float(), w.float().t())
    assert float((got - ref).norm() / ref.norm()) <= 1e-2
