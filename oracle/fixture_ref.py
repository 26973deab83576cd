"""TEST INFRASTRUCTURE ONLY — CPU restatement of the reference fixture's
whole pipeline, forward and backward, composed from the oracle's pieces.

What it restates (erikerikerik/foundry-trainer tools/fixtures/gen_block.py):
  DoubleBlock.forward   gen_block.py:199-240  (LN-mod, q/k/v linears with LoRA
                        on img to_q / to_v, QK RMSNorm + RoPE, joint attention
                        txt-then-img, gated out-projection, LN-mod, SwiGLU MLP,
                        gated residual)
  SingleBlock.forward   gen_block.py:265-288  (LN-mod, fused to_qkv with LoRA,
                        RMSNorm + RoPE on the img-then-txt table, attention,
                        SwiGLU MLP, x + g_at * attn + g_mlp * mlp)
  run                   gen_block.py:300-360  (joint = cat(txt, img) into the
                        single block, MSE loss on both outputs, backward)
The Rust reference's blocks (crates/foundry-spike/src/lib.rs:301-450) are
the same graph at the same fixture sizes.

The backward is the chain rule in reverse op order, written out here (no
autograd), through the oracle's backward pieces: ln_mod_bwd, swiglu_bwd,
attn_bwd, qk_prologue_bwd, linear_lora_bwd, gated_residual.  With bf16=True
every op result is rounded to bf16; PyTorch's bf16 rounding sequence is not
reproduced op for op, so bf16 agreement is approximate.

`mutate` plants one mistake in the composition (for tests that check the
fixture comparison catches it): "swiglu_swap" exchanges the SwiGLU input
gradients, "ln_drop_proj" drops the n * mean(dn * n) term of the LN-mod
gradient.  Only tests/ import this module.
"""
from __future__ import annotations

import numpy as np

import oracle

DIM, HEADS, HEAD_DIM = 256, 2, 128
AXES = (32, 32, 32, 32)
THETA = 1e4
GRID, TXT = 4, 8
LORA_SCALE = 8.0 / 4  # alpha / rank
EPS = 1e-6
LORA_LINEARS = ("double.img.to_q", "double.img.to_v", "single.to_qkv")


def _r(a, bf16):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return oracle.bf16_round(a) if bf16 else a


def positions():
    """img (row, col, 0, 0) over the 4x4 grid; txt (l, 0, 0, 0) (gen_block.py:311-314)."""
    n = GRID * GRID
    pos_img = np.zeros((n, 4), np.float32)
    pos_img[:, 0] = np.arange(n) // GRID
    pos_img[:, 1] = np.arange(n) % GRID
    pos_txt = np.zeros((TXT, 4), np.float32)
    pos_txt[:, 0] = np.arange(TXT)
    return pos_img, pos_txt


def _ln_bwd_drop_proj(x, dy, scale, mean, rstd, dres):
    n = (x.astype(np.float64) - mean[:, None]) * rstd[:, None]
    dn = dy.astype(np.float64) * (1.0 + scale.astype(np.float64))
    dx = rstd[:, None] * (dn - dn.mean(axis=1, keepdims=True))
    return (dx + dres).astype(np.float32)


def pipeline(f, bf16=False, mutate=None):
    """f: name -> float32 array (fixture weights and inputs, bf16-valued for
    bf16).  Returns (acts, grads): acts has the fixture's activation names,
    grads has grad/inputs/{img,txt}, grad/<lora linear>.lora_{a,b} and the
    double block's output gradients grad/double.{txt,img}_out."""
    C, H, D = DIM, HEADS, HEAD_DIM
    r = lambda a: _r(a, bf16)
    W = lambda name: f[f"weights/{name}.weight"]

    def lin(x, name, lora=False):
        if lora:
            return oracle.linear_lora(x, W(name), f[f"weights/{name}.bias"], f[f"weights/{name}.lora_a"],
                                      f[f"weights/{name}.lora_b"], scale=LORA_SCALE, bf16=bf16)
        return oracle.linear_lora(x, W(name), f[f"weights/{name}.bias"], bf16=bf16)

    def swiglu_bwd(d, g, u):
        dg, du = oracle.swiglu_bwd(d, g, u, bf16=bf16)
        return (du, dg) if mutate == "swiglu_swap" else (dg, du)

    def ln_bwd(x, dy, scale, mean, rstd, dres):
        if mutate == "ln_drop_proj":
            return r(_ln_bwd_drop_proj(x, dy, scale, mean, rstd, dres))
        return oracle.ln_mod_bwd(x, dy, scale, mean, rstd, dres=dres, bf16=bf16)

    def mlp_fwd(h, prefix):
        gp, up = lin(h, f"{prefix}.gate"), lin(h, f"{prefix}.up")
        act = oracle.swiglu_fwd(gp, up, bf16=bf16)
        return lin(act, f"{prefix}.down"), (gp, up)

    def mlp_bwd(dmlp, prefix, saved):
        gp, up = saved
        dact = r(dmlp @ W(f"{prefix}.down"))
        dg, du = swiglu_bwd(dact, gp, up)
        return r(r(dg @ W(f"{prefix}.gate")) + r(du @ W(f"{prefix}.up")))

    def prologue(x_raw, wname, cos, sin):
        n = x_raw.shape[0]
        return oracle.apply_rope(oracle.rms_norm(x_raw.reshape(n, H, D), f[f"weights/{wname}.weight"], EPS,
                                                 bf16=bf16), cos, sin, list(AXES), bf16=bf16)

    def prologue_bwd(x_raw, wname, cos, sin, dy):
        n = x_raw.shape[0]
        return r(oracle.qk_prologue_bwd(x_raw.reshape(n, H, D), f[f"weights/{wname}.weight"], cos, sin,
                                        np.ascontiguousarray(dy), list(AXES), EPS).reshape(n, C))

    pos_img, pos_txt = positions()
    cos_i, sin_i = oracle.rope_tables(pos_img, list(AXES), THETA, bf16=bf16)
    cos_t, sin_t = oracle.rope_tables(pos_txt, list(AXES), THETA, bf16=bf16)
    cos_a, sin_a = oracle.rope_tables(np.concatenate([pos_img, pos_txt]), list(AXES), THETA, bf16=bf16)
    tables = {"txt": (cos_t, sin_t), "img": (cos_i, sin_i)}

    acts = {}
    st = oracle.silu(f["inputs/temb"].reshape(1, -1), bf16=bf16)
    mod = lin(st, "double.mod").reshape(-1)
    sh1, sc1, g1, sh2, sc2, g2 = (mod[i * C:(i + 1) * C].copy() for i in range(6))

    # ---- double block forward
    x_in = {"txt": f["inputs/txt"], "img": f["inputs/img"]}
    sv = {}
    for name in ("txt", "img"):
        x = x_in[name]
        h, m1, rs1 = oracle.ln_mod_fwd(x, sh1, sc1, EPS, bf16=bf16)
        acts[f"double.{name}_norm1"] = h
        lora = name == "img"
        q_raw = lin(h, f"double.{name}.to_q", lora)
        k_raw = lin(h, f"double.{name}.to_k")
        v = lin(h, f"double.{name}.to_v", lora)
        cos, sin = tables[name]
        sv[name] = dict(h=h, m1=m1, rs1=rs1, q_raw=q_raw, k_raw=k_raw,
                        q=prologue(q_raw, f"double.{name}_q_norm", cos, sin),
                        k=prologue(k_raw, f"double.{name}_k_norm", cos, sin),
                        v=v.reshape(-1, H, D))
    acts["double.q"], acts["double.k"] = sv["img"]["q"], sv["img"]["k"]
    Q = np.concatenate([sv["txt"]["q"], sv["img"]["q"]])[None]
    K = np.concatenate([sv["txt"]["k"], sv["img"]["k"]])[None]
    V = np.concatenate([sv["txt"]["v"], sv["img"]["v"]])[None]
    O = oracle.attn_fwd(Q, K, V, bf16=bf16)[0][0]
    off = {"txt": 0, "img": TXT}
    x2 = {}
    for name in ("txt", "img"):
        s = sv[name]
        n = x_in[name].shape[0]
        a = np.ascontiguousarray(O[off[name]:off[name] + n].reshape(n, C))
        x1 = oracle.gated_residual(x_in[name], g1, lin(a, f"double.{name}.to_out"), bf16=bf16)
        h2, m2, rs2 = oracle.ln_mod_fwd(x1, sh2, sc2, EPS, bf16=bf16)
        mlp, saved = mlp_fwd(h2, f"double.{name}.mlp")
        x2[name] = oracle.gated_residual(x1, g2, mlp, bf16=bf16)
        s.update(a=a, x1=x1, h2=h2, m2=m2, rs2=rs2, mlp_saved=saved)
    acts["double.attn_img"] = sv["img"]["a"]
    acts["double.img_post_attn"] = sv["img"]["x1"]
    acts["double.img_out"], acts["double.txt_out"] = x2["img"], x2["txt"]

    # ---- single block forward
    joint = np.concatenate([x2["txt"], x2["img"]])
    smod = lin(st, "single.mod").reshape(-1)
    ssh1, ssc1, g_at, _, _, g_mlp = (smod[i * C:(i + 1) * C].copy() for i in range(6))
    nh, ms, rss = oracle.ln_mod_fwd(joint, ssh1, ssc1, EPS, bf16=bf16)
    acts["single.norm1"] = nh
    qkv = lin(nh, "single.to_qkv", True)
    sq_raw, sk_raw = np.ascontiguousarray(qkv[:, :C]), np.ascontiguousarray(qkv[:, C:2 * C])
    sq = prologue(sq_raw, "single.q_norm", cos_a, sin_a)
    sk = prologue(sk_raw, "single.k_norm", cos_a, sin_a)
    sv_ = np.ascontiguousarray(qkv[:, 2 * C:]).reshape(-1, H, D)
    acts["single.q"], acts["single.k"] = sq, sk
    sattn = oracle.attn_fwd(sq[None], sk[None], sv_[None], bf16=bf16)[0][0].reshape(-1, C)
    acts["single.attn"] = sattn
    smlp, ssaved = mlp_fwd(nh, "single.mlp")
    acts["single.mlp"] = smlp
    out = oracle.gated_residual(oracle.gated_residual(joint, g_at, sattn, bf16=bf16), g_mlp, smlp, bf16=bf16)
    acts["single.out"] = out
    acts["output/txt"], acts["output/img"] = out[:TXT], out[TXT:]
    t_img, t_txt = f["inputs/target_img"], f["inputs/target_txt"]
    di, dt = out[TXT:].astype(np.float64) - t_img, out[:TXT].astype(np.float64) - t_txt
    acts["loss"] = np.float32(np.mean(di * di) + np.mean(dt * dt))

    # ---- backward: MSE, single block
    grads = {}
    dout = r(np.concatenate([2.0 * dt / dt.size, 2.0 * di / di.size]))
    dattn = oracle.gated_residual(None, g_at, dout, bf16=bf16)
    dmlp = oracle.gated_residual(None, g_mlp, dout, bf16=bf16)
    dnh_mlp = mlp_bwd(dmlp, "single.mlp", ssaved)
    dq, dk, dv = oracle.attn_bwd(sq[None], sk[None], sv_[None], dattn.reshape(-1, H, D)[None], bf16=bf16)
    dqkv = np.concatenate([prologue_bwd(sq_raw, "single.q_norm", cos_a, sin_a, dq[0]),
                           prologue_bwd(sk_raw, "single.k_norm", cos_a, sin_a, dk[0]),
                           dv[0].reshape(-1, C)], axis=1)
    dnh_at, dA, dB = oracle.linear_lora_bwd(nh, W("single.to_qkv"), f["weights/single.to_qkv.lora_a"],
                                            f["weights/single.to_qkv.lora_b"], dqkv, LORA_SCALE, bf16=bf16)
    grads["grad/single.to_qkv.lora_a"], grads["grad/single.to_qkv.lora_b"] = dA, dB
    djoint = ln_bwd(joint, r(dnh_at + dnh_mlp), ssc1, ms, rss, dout)

    # ---- double block backward
    dx2 = {"txt": np.ascontiguousarray(djoint[:TXT]), "img": np.ascontiguousarray(djoint[TXT:])}
    # the gradient at the double block's outputs (not a fixture tensor: it
    # lets a block be checked on its own from here down)
    grads["grad/double.txt_out"], grads["grad/double.img_out"] = dx2["txt"], dx2["img"]
    dx1, dO = {}, []
    for name in ("txt", "img"):
        s = sv[name]
        dmlp = oracle.gated_residual(None, g2, dx2[name], bf16=bf16)
        dh2 = mlp_bwd(dmlp, f"double.{name}.mlp", s["mlp_saved"])
        dx1[name] = ln_bwd(s["x1"], dh2, sc2, s["m2"], s["rs2"], dx2[name])
        dlin = oracle.gated_residual(None, g1, dx1[name], bf16=bf16)
        dO.append(r(dlin @ W(f"double.{name}.to_out")).reshape(-1, H, D))
    dq, dk, dv = oracle.attn_bwd(Q, K, V, np.concatenate(dO)[None], bf16=bf16)
    for name in ("txt", "img"):
        s = sv[name]
        n = x_in[name].shape[0]
        cos, sin = tables[name]
        o = off[name]
        dq_raw = prologue_bwd(s["q_raw"], f"double.{name}_q_norm", cos, sin, dq[0, o:o + n])
        dk_raw = prologue_bwd(s["k_raw"], f"double.{name}_k_norm", cos, sin, dk[0, o:o + n])
        dvn = np.ascontiguousarray(dv[0, o:o + n].reshape(n, C))
        dh = r(dk_raw @ W(f"double.{name}.to_k"))
        for t, d in (("to_q", dq_raw), ("to_v", dvn)):
            lname = f"double.{name}.{t}"
            if name == "img":
                dxt, dA, dB = oracle.linear_lora_bwd(s["h"], W(lname), f[f"weights/{lname}.lora_a"],
                                                     f[f"weights/{lname}.lora_b"], d, LORA_SCALE, bf16=bf16)
                grads[f"grad/{lname}.lora_a"], grads[f"grad/{lname}.lora_b"] = dA, dB
            else:
                dxt = r(d @ W(lname))
            dh = r(dh + dxt)
        grads[f"grad/inputs/{name}"] = ln_bwd(x_in[name], dh, sc1, s["m1"], s["rs1"], dx1[name])
    return acts, grads
