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
