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


def block_step(x, dy, W, heads, head_dim, cos, sin, axes, lora_scale, bf16, eps=1e-6, lr=1e-3, want_dx=False):
    """x, dy: {stream: [n, C]}; W: {stream: dict of numpy weights:
    w_qkv, w_out, w1, w2, q_norm, k_norm, mod (6 vectors), lora_a / lora_b
    {q,k,v,out}}; cos / sin: {stream: [n, D]} rope tables.
    Returns (y, grads, updated) with grads[(stream, t)] = (dA, dB) and
    updated[(stream, t)] = (A', B') after one AdamW step from zero moments;
    want_dx adds grads[(stream, "x")], the input gradient of a block inside a
    stack (through the frozen qkv projection and the first layer_norm_mod)."""
    H, D = heads, head_dim
    C = H * D
    s = lora_scale
    T = x["txt"].shape[0]
    n_of = {k: v.shape[0] for k, v in x.items()}
    q_j, k_j, v_j, h_s, qkv_s, ln1, dx1_s = [], [], [], {}, {}, {}, {}
    for name in STREAMS:
        w, n = W[name], n_of[name]
        h, mean1, rstd1 = oracle.ln_mod_fwd(x[name], w["mod"][0], w["mod"][1], eps, bf16=bf16)
        h_s[name] = h
        ln1[name] = (mean1, rstd1)
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
        dx1_s[name] = dx1
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
        dh = np.zeros((n, C), np.float64)
        for j, t in enumerate(("q", "k", "v")):
            Wj = w["w_qkv"][j * C:(j + 1) * C]
            _, dA, dB = oracle.linear_lora_bwd(h_s[name], Wj, w["lora_a"][t],
                                               w["lora_b"][t], dqkv[j], s, bf16=False, want_dx=False)
            grads[(name, t)] = (dA, dB)
            dh += dqkv[j] @ Wj + s * ((dqkv[j] @ w["lora_b"][t]) @ w["lora_a"][t])
        if want_dx:
            mean1, rstd1 = ln1[name]
            grads[(name, "x")] = oracle.ln_mod_bwd(x[name], _r(dh, bf16), w["mod"][1], mean1, rstd1,
                                                   dres=dx1_s[name], bf16=bf16)
    updated = {}
    for key, g in grads.items():
        name, t = key
        if t == "x":
            continue
        dA, dB = g
        w = W[name]
        z_a, z_b = np.zeros_like(dA), np.zeros_like(dB)
        A1 = oracle.adamw_step(w["lora_a"][t], dA, z_a, z_a, step=1, lr=lr, bf16=bf16)[0]
        B1 = oracle.adamw_step(w["lora_b"][t], dB, z_b, z_b, step=1, lr=lr, bf16=bf16)[0]
        updated[key] = (A1, B1)
    return y, grads, updated


def single_block_step(x, dy, W, heads, head_dim, cos, sin, axes, lora_scale, bf16, eps=1e-6, lr=1e-3,
                      want_dx=True):
    """One single-stream block step (throughput.rs:584-629) with LoRA on the
    fused to_in and to_out projections, restated from the oracle's pieces:
    layer_norm_mod -> to_in (+LoRA) -> [q|k|v|gate|up] -> rms_norm + rope on
    q, k -> attention; silu(gate) * up; to_out(cat(attn, act)) (+LoRA) ->
    x + g * out; then the backward and one AdamW step.

    x, dy [S, C]; W: w_in [3C+2M, C], w_out [C, C+M], q_norm, k_norm, mod
    (shift, scale, gate), lora_a / lora_b {to_in, to_out}; cos / sin [S, D].
    Returns (y, grads, updated, dx) with grads[t] = (dA, dB) (f32) and dx
    None unless want_dx."""
    H, D = heads, head_dim
    C = H * D
    M = (W["w_in"].shape[0] - 3 * C) // 2
    S = x.shape[0]
    s = lora_scale
    sh, sc, g = W["mod"]
    A, Bm = W["lora_a"], W["lora_b"]
    nh, mean, rstd = oracle.ln_mod_fwd(x, sh, sc, eps, bf16=bf16)
    fused = oracle.linear_lora(nh, W["w_in"], None, A["to_in"], Bm["to_in"], scale=s, bf16=bf16)
    q_raw = np.ascontiguousarray(fused[:, :C]).reshape(S, H, D)
    k_raw = np.ascontiguousarray(fused[:, C:2 * C]).reshape(S, H, D)
    v = np.ascontiguousarray(fused[:, 2 * C:3 * C]).reshape(S, H, D)
    gate, up = np.ascontiguousarray(fused[:, 3 * C:3 * C + M]), np.ascontiguousarray(fused[:, 3 * C + M:])
    q = oracle.apply_rope(oracle.rms_norm(q_raw, W["q_norm"], eps, bf16=bf16), cos, sin, axes, bf16=bf16)
    k = oracle.apply_rope(oracle.rms_norm(k_raw, W["k_norm"], eps, bf16=bf16), cos, sin, axes, bf16=bf16)
    scale = 1.0 / np.sqrt(D)
    O = oracle.attn_fwd(q[None], k[None], v[None], scale=scale, bf16=bf16)[0][0].reshape(S, C)
    act = oracle.swiglu_fwd(gate, up, bf16=bf16)
    joined = np.ascontiguousarray(np.concatenate([O, act], axis=1))
    out = oracle.linear_lora(joined, W["w_out"], None, A["to_out"], Bm["to_out"], scale=s, bf16=bf16)
    y = oracle.gated_residual(x, g, out, bf16=bf16)
    # backward
    grads = {}
    dout = oracle.gated_residual(None, g, dy, bf16=bf16)
    _, dA, dB = oracle.linear_lora_bwd(joined, W["w_out"], A["to_out"], Bm["to_out"], dout, s, bf16=False,
                                       want_dx=False)
    grads["to_out"] = (dA, dB)
    djoined = _r(dout @ W["w_out"] + s * ((dout @ Bm["to_out"]) @ A["to_out"]), bf16)
    dgate, dup = oracle.swiglu_bwd(np.ascontiguousarray(djoined[:, C:]), gate, up, bf16=bf16)
    dq, dk, dv = oracle.attn_bwd(q[None], k[None], v[None], np.ascontiguousarray(djoined[:, :C]).reshape(1, S, H, D),
                                 scale=scale, bf16=bf16)
    dq_raw = _r(oracle.qk_prologue_bwd(q_raw, W["q_norm"], cos, sin, dq[0], axes, eps).reshape(S, C), bf16)
    dk_raw = _r(oracle.qk_prologue_bwd(k_raw, W["k_norm"], cos, sin, dk[0], axes, eps).reshape(S, C), bf16)
    dfused = np.ascontiguousarray(np.concatenate([dq_raw, dk_raw, dv[0].reshape(S, C), dgate, dup], axis=1))
    _, dA, dB = oracle.linear_lora_bwd(nh, W["w_in"], A["to_in"], Bm["to_in"], dfused, s, bf16=False,
                                       want_dx=False)
    grads["to_in"] = (dA, dB)
    dx = None
    if want_dx:
        dnh = _r(dfused @ W["w_in"] + s * ((dfused @ Bm["to_in"]) @ A["to_in"]), bf16)
        dx = oracle.ln_mod_bwd(x, dnh, sc, mean, rstd, dres=dy, bf16=bf16)
    updated = {}
    for t, (dA, dB) in grads.items():
        z_a, z_b = np.zeros_like(dA), np.zeros_like(dB)
        updated[t] = (oracle.adamw_step(A[t], dA, z_a, z_a, step=1, lr=lr, bf16=bf16)[0],
                      oracle.adamw_step(Bm[t], dB, z_b, z_b, step=1, lr=lr, bf16=bf16)[0])
    return y, grads, updated, dx
