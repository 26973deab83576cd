"""TEST INFRASTRUCTURE ONLY — CPU restatement of one double-stream LoRA
block step (forward, backward to the LoRA factors, AdamW), composed from the
oracle's pinned pieces:
  layer_norm_mod / its gradient, gated residual, tanh-GELU   block_oracle.c
  rms_norm + apply_rope, and the prologue gradient           attn_oracle.c
  attention fwd / bwd                                        attn_oracle.c
  linear_scaled (+ LoRA) and its gradient                    oracle_gemm.c
  adamw_step                                                 block_oracle.c
plus numpy matmuls for the frozen linears.  The wiring follows
crates/foundry-spike/src/bin/throughput.rs:480-574 with the c4 choices
(LoRA on q/k/v/out of both streams, tanh-GELU MLP, no bias, dY given).
bf16=True rounds every op output to bf16, as the device path stores it.
Only tests/ import this module.
"""
from __future__ import annotations

import numpy as np

import oracle

STREAMS = ("txt", "img")


def _r(a, bf16):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return oracle.bf16_round(a) if bf16 else a


def mod_parts(c, w_mod, C, bf16):
    sc = oracle.silu(c.reshape(1, -1), bf16=bf16)
    m = _r(sc @ w_mod.T, bf16).reshape(-1)
    return [m[i * C:(i + 1) * C].copy() for i in range(6)]


def block_step(x, dy, W, heads, head_dim, cos, sin, axes, lora_scale, bf16, eps=1e-6, lr=1e-3):
    """x, dy: {stream: [n, C]}; W: {stream: dict of numpy weights:
    w_qkv, w_out, w1, w2, q_norm, k_norm, mod (6 vectors), lora_a / lora_b
    {q,k,v,out}}; cos / sin: {stream: [n, D]} rope tables.
    Returns (y, grads, updated) with grads[(stream, t)] = (dA, dB) and
    updated[(stream, t)] = (A', B') after one AdamW step from zero moments."""
    H, D = heads, head_dim
    C = H * D
    s = lora_scale
    T = x["txt"].shape[0]
    n_of = {k: v.shape[0] for k, v in x.items()}
    q_j, k_j, v_j, h_s, qkv_s = [], [], [], {}, {}
    for name in STREAMS:
        w, n = W[name], n_of[name]
        h = oracle.ln_mod_fwd(x[name], w["mod"][0], w["mod"][1], eps, bf16=bf16)[0]
        h_s[name] = h
        parts = []
        for j, t in enumerate(("q", "k", "v")):
            Wt = w["w_qkv"][j * C:(j + 1) * C]
            base = _r(h @ Wt.T, bf16)
            u = h @ w["lora_a"][t].T
            parts.append(_r(base + s * (u @ w["lora_b"][t].T), bf16))
        qkv_s[name] = parts
        q = oracle.apply_rope(oracle.rms_norm(parts[0].reshape(n, H, D), w["q_norm"], eps, bf16=bf16),
                              cos[name], sin[name], axes, bf16=bf16)
        k = oracle.apply_rope(oracle.rms_norm(parts[1].reshape(n, H, D), w["k_norm"], eps, bf16=bf16),
                              cos[name], sin[name], axes, bf16=bf16)
        q_j.append(q)
        k_j.append(k)
        v_j.append(parts[2].reshape(n, H, D))
    Q = np.concatenate(q_j)[None]
    K = np.concatenate(k_j)[None]
    V = np.concatenate(v_j)[None]
    scale = 1.0 / np.sqrt(D)
    O, _ = oracle.attn_fwd(Q, K, V, scale=scale, bf16=bf16)
    y, dO_parts, grads = {}, {}, {}
    for name in STREAMS:
        w, n = W[name], n_of[name]
        off = 0 if name == "txt" else T
        a = np.ascontiguousarray(O[0, off:off + n].reshape(n, C))
        base = _r(a @ w["w_out"].T, bf16)
        out = _r(base + s * ((a @ w["lora_a"]["out"].T) @ w["lora_b"]["out"].T), bf16)
        sh1, sc1, g1, sh2, sc2, g2 = w["mod"]
        x1 = oracle.gated_residual(x[name], g1, out, bf16=bf16)
        h2, mean2, rstd2 = oracle.ln_mod_fwd(x1, sh2, sc2, eps, bf16=bf16)
        pre = _r(h2 @ w["w1"].T, bf16)
        act = oracle.gelu_fwd(pre, bf16=bf16)
        mlp = _r(act @ w["w2"].T, bf16)
        y[name] = oracle.gated_residual(x1, g2, mlp, bf16=bf16)
        dmlp = oracle.gated_residual(None, g2, dy[name], bf16=bf16)
        dact = oracle.gelu_bwd(_r(dmlp @ w["w2"], bf16), pre, bf16=bf16)
        dh2 = _r(dact @ w["w1"], bf16)
        dx1 = oracle.ln_mod_bwd(x1, dh2, sc2, mean2, rstd2, dres=dy[name], bf16=bf16)
        dout = oracle.gated_residual(None, g1, dx1, bf16=bf16)
        _, dA, dB = oracle.linear_lora_bwd(a, w["w_out"], w["lora_a"]["out"], w["lora_b"]["out"], dout, s,
                                           bf16=False, want_dx=False)
        grads[(name, "out")] = (dA, dB)
        dpart = dout @ w["w_out"] + s * ((dout @ w["lora_b"]["out"]) @ w["lora_a"]["out"])
        dO_parts[name] = _r(dpart, bf16).reshape(n, H, D)
    dO = np.concatenate([dO_parts["txt"], dO_parts["img"]])[None]
    dq, dk, dv = oracle.attn_bwd(Q, K, V, dO, scale=scale, bf16=bf16)
    for name in STREAMS:
        w, n = W[name], n_of[name]
        off = 0 if name == "txt" else T
        parts = qkv_s[name]
        dq_raw = oracle.qk_prologue_bwd(parts[0].reshape(n, H, D), w["q_norm"], cos[name], sin[name],
                                        dq[0, off:off + n], axes, eps)
        dk_raw = oracle.qk_prologue_bwd(parts[1].reshape(n, H, D), w["k_norm"], cos[name], sin[name],
                                        dk[0, off:off + n], axes, eps)
        dqkv = [_r(dq_raw.reshape(n, C), bf16), _r(dk_raw.reshape(n, C), bf16),
                np.ascontiguousarray(dv[0, off:off + n].reshape(n, C))]
        for j, t in enumerate(("q", "k", "v")):
            _, dA, dB = oracle.linear_lora_bwd(h_s[name], w["w_qkv"][j * C:(j + 1) * C], w["lora_a"][t],
                                               w["lora_b"][t], dqkv[j], s, bf16=False, want_dx=False)
            grads[(name, t)] = (dA, dB)
    updated = {}
    for key, (dA, dB) in grads.items():
        name, t = key
        w = W[name]
        z_a, z_b = np.zeros_like(dA), np.zeros_like(dB)
        A1 = oracle.adamw_step(w["lora_a"][t], dA, z_a, z_a, step=1, lr=lr, bf16=bf16)[0]
        B1 = oracle.adamw_step(w["lora_b"][t], dB, z_b, z_b, step=1, lr=lr, bf16=bf16)[0]
        updated[key] = (A1, B1)
    return y, grads, updated
