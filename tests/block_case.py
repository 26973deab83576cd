"""Shared construction of small double-block cases for the block tests:
numpy weights for the oracle (oracle/block_ref.py) and the same values as a
DoubleBlockLoRA for the device path."""
import numpy as np

import oracle


def make_case(C=256, H=2, T=16, rows=4, cols=8, F=None, r=4, alpha=8.0, seed=11, bf16=True):
    rng = np.random.default_rng(seed)
    D = C // H
    F = F or 4 * C
    rnd = (lambda a: oracle.bf16_round(a.astype(np.float32))) if bf16 else (lambda a: a.astype(np.float32))
    n_of = {"txt": T, "img": rows * cols}
    W, x, dy = {}, {}, {}
    for name in ("txt", "img"):
        w = {"w_qkv": rnd(rng.standard_normal((3 * C, C)) * 0.02),
             "w_out": rnd(rng.standard_normal((C, C)) * 0.02),
             "w1": rnd(rng.standard_normal((F, C)) * 0.02),
             "w2": rnd(rng.standard_normal((C, F)) * 0.02),
             "q_norm": rnd(1 + 0.02 * rng.standard_normal(D)),
             "k_norm": rnd(1 + 0.02 * rng.standard_normal(D)),
             "w_mod": rnd(rng.standard_normal((6 * C, C)) * 0.02),
             "lora_a": {}, "lora_b": {}}
        for t in ("q", "k", "v", "out"):
            w["lora_a"][t] = rnd(rng.standard_normal((r, C)) / r)
            w["lora_b"][t] = rnd(rng.standard_normal((C, r)) * 0.02)
        W[name] = w
        x[name] = rnd(rng.standard_normal((n_of[name], C)))
        dy[name] = rnd(rng.standard_normal((n_of[name], C)))
    c = rnd(rng.standard_normal(C))
    pos = np.zeros((T + rows * cols, 3), np.float32)
    pos[:T, 0] = np.arange(T)
    rr, cc = np.meshgrid(np.arange(rows), np.arange(cols), indexing="ij")
    pos[T:, 1], pos[T:, 2] = rr.ravel(), cc.ravel()
    axes = (16, 56, 56) if D == 128 else (D // 4, D // 4, D // 2)
    cos, sin = oracle.rope_tables(pos, axes, 1e4, bf16=bf16)
    return dict(C=C, H=H, D=D, T=T, rows=rows, cols=cols, F=F, r=r, scale=alpha / r, W=W, x=x, dy=dy, c=c,
                axes=axes, cos={"txt": cos[:T], "img": cos[T:]}, sin={"txt": sin[:T], "img": sin[T:]},
                bf16=bf16)


def oracle_mods(case):
    import block_ref
    for name in ("txt", "img"):
        case["W"][name]["mod"] = block_ref.mod_parts(case["c"], case["W"][name]["w_mod"], case["C"],
                                                     case["bf16"])
    return case


def make_single_case(C=256, H=2, T=40, rows=8, cols=12, ratio=3, r=4, alpha=8.0, seed=9, bf16=True):
    """A small single-stream block: fused to_in [3C + 2M, C], to_out [C, C + M]
    (M = ratio * C), LoRA on both, klein RoPE (axes 32 x 4 for D = 128,
    theta 2000, txt (0, 0, 0, l), img (0, h, w, 0), txt first)."""
    rng = np.random.default_rng(seed)
    D = C // H
    M = ratio * C
    rnd = (lambda a: oracle.bf16_round(a.astype(np.float32))) if bf16 else (lambda a: a.astype(np.float32))
    S = T + rows * cols
    W = {"w_in": rnd(rng.standard_normal((3 * C + 2 * M, C)) * 0.02),
         "w_out": rnd(rng.standard_normal((C, C + M)) * 0.02),
         "q_norm": rnd(1 + 0.02 * rng.standard_normal(D)),
         "k_norm": rnd(1 + 0.02 * rng.standard_normal(D)),
         "w_mod": rnd(rng.standard_normal((3 * C, C)) * 0.02),
         "lora_a": {}, "lora_b": {}}
    for t, (fin, fout) in (("to_in", (C, 3 * C + 2 * M)), ("to_out", (C + M, C))):
        W["lora_a"][t] = rnd(rng.standard_normal((r, fin)) / r)
        W["lora_b"][t] = rnd(rng.standard_normal((fout, r)) * 0.02)
    x, dy, c = rnd(rng.standard_normal((S, C))), rnd(rng.standard_normal((S, C))), rnd(rng.standard_normal(C))
    pos = np.zeros((S, 4), np.float32)
    pos[:T, 3] = np.arange(T)
    rr, cc = np.meshgrid(np.arange(rows), np.arange(cols), indexing="ij")
    pos[T:, 1], pos[T:, 2] = rr.ravel(), cc.ravel()
    axes = (32, 32, 32, 32) if D == 128 else (D // 4,) * 4
    theta = 2000.0
    cos, sin = oracle.rope_tables(pos, axes, theta, bf16=bf16)
    return dict(C=C, H=H, D=D, T=T, rows=rows, cols=cols, M=M, r=r, scale=alpha / r, W=W, x=x, dy=dy, c=c,
                axes=axes, theta=theta, cos=cos, sin=sin, bf16=bf16)


def single_oracle_mods(case):
    """Mod3 parts chunk3(silu(c) W_mod^T) (throughput.rs:284-288)."""
    C = case["C"]
    sc = oracle.silu(case["c"].reshape(1, -1), bf16=case["bf16"])
    m = sc @ case["W"]["w_mod"].T
    m = (oracle.bf16_round(m.astype(np.float32)) if case["bf16"] else m.astype(np.float32)).reshape(-1)
    case["W"]["mod"] = [m[i * C:(i + 1) * C].copy() for i in range(3)]
    return case
