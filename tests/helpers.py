"""Shared test utilities: comparators, golden fixtures, seeded config inputs."""
from __future__ import annotations

import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")

# bf16 gate: max-abs 2e-2 and rel-L2 1e-2; f32 gate: rel-L2 1e-4
BF16_MAX_ABS = 2e-2
BF16_REL_L2 = 1e-2
F32_REL_L2 = 1e-4


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-30))


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def check_gate(label: str, got, want, bf16: bool) -> None:
    """The north-star gate for one tensor: bf16 rel-L2 <= 1e-2 and max-abs
    <= 2e-2 x max(1, max|want|) (bf16's spacing is relative, so above unit
    magnitude the bound scales with the tensor's peak); f32 rel-L2 <= 1e-4.
    Prints the measured values, peak-relative max-abs included."""
    r, m = rel_l2(got, want), max_abs(got, want)
    peak = float(np.max(np.abs(np.asarray(want, np.float64)))) if np.size(want) else 0.0
    print(f"  {label}: rel_l2={r:.2e} max_abs={m:.2e} max_abs/peak={m / (peak + 1e-30):.2e}", flush=True)
    if bf16:
        assert r <= BF16_REL_L2, (label, r)
        assert m <= BF16_MAX_ABS * max(1.0, peak), (label, m, peak)
    else:
        assert r <= F32_REL_L2, (label, r)


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-30))


def load_golden(tag: str) -> dict:
    """The reference fixture subset as float32 numpy arrays (bf16 values are exact)."""
    from safetensors.torch import load_file
    return {k: v.float().numpy() for k, v in
            load_file(os.path.join(GOLDEN, f"attn_fixture_{tag}.safetensors")).items()}


def load_block_golden(tag: str) -> dict:
    """The reference fixture's block subset (block_fixture_{tag}) as float32 numpy."""
    from safetensors.torch import load_file
    return {k: v.float().numpy() for k, v in
            load_file(os.path.join(GOLDEN, f"block_fixture_{tag}.safetensors")).items()}


def load_pipeline_golden(tag: str) -> dict:
    """Everything the reference fixture's whole pipeline touches, as float32
    numpy: the attention, block and pipeline subsets merged.  For bf16 the
    weights are the bf16 casts of the fp32 ones (what the reference fixture
    holds, checked when the subsets were extracted) and the activations,
    gradients and targets come from the bf16 files."""
    from safetensors.torch import load_file
    f = {}
    for name in ("attn", "block", "pipeline"):
        f.update({k: v.float().numpy() for k, v in
                  load_file(os.path.join(GOLDEN, f"{name}_fixture_fp32.safetensors")).items()})
    if tag == "bf16":
        f = {k: (bf16_round(v) if k.startswith(("weights/", "inputs/")) else v) for k, v in f.items()}
        for name in ("attn", "block", "pipeline"):
            f.update({k: v.float().numpy() for k, v in
                      load_file(os.path.join(GOLDEN, f"{name}_fixture_bf16.safetensors")).items()})
    return f


def bf16_round(a):
    import oracle
    return oracle.bf16_round(a)


def attn_inputs(cfg, seed: int = 20261028):
    """Seeded q, k, v, dO [B,S,H,D] float32 (bf16-valued for bf16 configs).

    For RoPE configs, raw Q/K ~ N(0,1) go through the oracle's RMSNorm
    (w = 1 + N(0, 0.02), separate for Q and K) and RoPE (cfg.axes, cfg.theta)
    with the reference's bf16 cast points; V, dO ~ N(0,1).  For c5, dO is
    zeroed on padded query rows.
    """
    import oracle
    rng = np.random.default_rng(seed)
    B, S, H, D = cfg.batch, cfg.seq, cfg.heads, cfg.head_dim
    bf = cfg.dtype == "bf16"
    rnd = (lambda a: oracle.bf16_round(a)) if bf else (lambda a: a.astype(np.float32))
    q = rnd(rng.standard_normal((B, S, H, D), dtype=np.float32))
    k = rnd(rng.standard_normal((B, S, H, D), dtype=np.float32))
    v = rnd(rng.standard_normal((B, S, H, D), dtype=np.float32))
    do = rnd(rng.standard_normal((B, S, H, D), dtype=np.float32))
    extra = {}
    if cfg.rope:
        wq = rnd(1.0 + 0.02 * rng.standard_normal(D, dtype=np.float32))
        wk = rnd(1.0 + 0.02 * rng.standard_normal(D, dtype=np.float32))
        cos, sin = oracle.rope_tables(cfg.positions(), cfg.axes, cfg.theta, bf16=bf)
        raw_q, raw_k = q, k
        qn = np.empty_like(q)
        kn = np.empty_like(k)
        for b in range(B):
            qn[b] = oracle.apply_rope(oracle.rms_norm(q[b], wq, bf16=bf), cos, sin, cfg.axes, bf16=bf)
            kn[b] = oracle.apply_rope(oracle.rms_norm(k[b], wk, bf16=bf), cos, sin, cfg.axes, bf16=bf)
        q, k = qn, kn
        extra = dict(raw_q=raw_q, raw_k=raw_k, wq=wq, wk=wk, cos=cos, sin=sin)
    keep = cfg.key_keep()
    if keep is not None:
        do = do * keep[:, :, None, None]
    return dict(q=q, k=k, v=v, do=do, keep=keep, **extra)
