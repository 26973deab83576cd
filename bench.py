#!/usr/bin/env python3
"""Benchmark of the attention hot path on one MI355X.

Workload ("c2"): FLUX-style joint attention at
1024 px — B=1, H=24, D=128, S=4608 (512 txt + 64x64 img tokens), bf16.
Raw Q/K ~ N(0,1) are QK-RMSNormed (scale 1+N(0,0.02)) and axial-roped (axes
16/56/56, theta 1e4) by the fused prologue kernel once, outside the timed
region; V, dO ~ N(0,1).  One step = attention forward (O + LSE) + backward
(dQ, dK, dV) through libfoundry_attn.so, inputs resident in HBM.

value = 14*B*H*S^2*D / step time (forward 4*B*H*S^2*D, backward 2.5x that).

Before the W warm-up steps the GPU runs the step untimed for --settle-s
seconds (default 0.3): MI355X ramps its clocks over the first ~100 ms of
work, and the driver's short warm-up would otherwise time part of that ramp.
The timed region is exactly K steps either way.

Prints ONE JSON line.  Besides the contract fields it carries:
  roofline      for the kernel with the largest share of the step time
                (HIP events on the launch stream, averaged over the timed steps)
  cpu_baseline  the CPU oracle (restatement of the reference's Candle CPU path,
                materialised f32 scores, 5-GEMM backward) timed on this host
                on a bounded sample of the same workload, with the host's
                logical, physical and usable (affinity) core counts
  kernels       per-kernel times and rates
  configs       the same measurement at c3 (B4 S1536) and c5 (B2 S6656,
                key-padding mask): step, forward, backward and per-kernel rates
  ulysses_shards  fwd+bwd at one GPU's share of the heads (H/2, H/4, H/8) at
                the full sequence, the per-GPU attention of 2-, 4- and 8-way
                sequence parallelism
--only-headline runs the c2 measurement alone (no other section), so that a
profiler trace of the run holds only c2 attention dispatches.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "foundry-trainer_amd"))

METRIC = "attn fwd+bwd TFLOP/s (% bf16 MFMA peak) at S=4608,D=128; LoRA block steps/s"  # block: rec["block"]
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
# HBM bytes per launch of each attention kernel, per config: the table in
# profiles/attn_traffic.md, made from rocprofv3 FETCH_SIZE and WRITE_SIZE runs
# of this script (--only-headline --config <c> --calib-copy-mib 256), scaled
# by what the same counters read for that 256 MiB copy.  A kernel or config
# the table does not hold reports traffic null.
TRAFFIC_TABLE = os.path.join(ROOT, "profiles", "attn_traffic.md")


def load_traffic(path: str = TRAFFIC_TABLE) -> dict:
    """{(config, kernel): HBM bytes per launch} from the table rows
    `| config | kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes | ...`."""
    out = {}
    if not os.path.exists(path):
        return out
    with open(path) as f:
        for line in f:
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 5 and cells[0] in ("c2", "c3", "c5") and cells[4].isdigit():
                out[(cells[0], cells[1])] = int(cells[4])
    return out


TRAFFIC = load_traffic()


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2", choices=["c2", "c3", "c5"])
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="bound on the CPU baseline sample (0 = skip)")
    ap.add_argument("--block-steps", type=int, default=30,
                    help="timed c4 LoRA block steps (0 = skip the block measurement); the block "
                         "sections warm up for a third as many steps (at least 2)")
    ap.add_argument("--settle-s", type=float, default=0.3,
                    help="untimed seconds of steps before the warm-up steps (clock ramp)")
    ap.add_argument("--only-headline", action="store_true",
                    help="measure the --config attention step only (for profiler runs)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="first run one device-to-device copy of this many MiB: the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE to HBM bytes")
    return ap.parse_args()


def make_inputs(cfg, torch, fa):
    g = torch.Generator(device="cuda").manual_seed(20261028)
    B, S, H, D = cfg.batch, cfg.seq, cfg.heads, cfg.head_dim
    bf = torch.bfloat16
    rq = torch.randn((B, S, H, D), device="cuda", generator=g).to(bf)
    rk = torch.randn((B, S, H, D), device="cuda", generator=g).to(bf)
    v = torch.randn((B, S, H, D), device="cuda", generator=g).to(bf)
    do = torch.randn((B, S, H, D), device="cuda", generator=g).to(bf)
    wq = (1 + 0.02 * torch.randn(D, device="cuda", generator=g)).to(bf)
    wk = (1 + 0.02 * torch.randn(D, device="cuda", generator=g)).to(bf)
    cos, sin = fa.rope_tables(cfg.positions(), cfg.axes, cfg.theta, dtype=bf)
    q = torch.empty_like(rq)
    k = torch.empty_like(rk)
    fa.qk_prologue(rq, wq, cos, sin, cfg.axes, out=q)
    fa.qk_prologue(rk, wk, cos, sin, cfg.axes, out=k)
    keep = None
    if cfg.key_keep() is not None:
        keep = torch.from_numpy(cfg.key_keep()).to("cuda")
        do = do * keep[:, :, None, None].to(bf)
    return q, k, v, do, keep


def _time_steps(torch, step, steps: int, warmup: int):
    """Wall and GPU-event seconds per call of step() over `steps` timed calls."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps, e0.elapsed_time(e1) * 1e-3 / steps


def _event_ms(torch, fn, n: int = 20) -> float:
    """Mean HIP-event time (ms) of fn() on torch's current stream, the stream
    the ABI launches on, after warm-up."""
    for _ in range(3):
        fn()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n


def _graph_ms(torch, fn, reps: int = 20, replays: int = 5) -> float:
    """Mean time (ms) of fn() from HIP-event timing of replays of a HIP graph
    that holds `reps` calls: the kernel's own duration, without the host's
    per-call time (for these 10-30 us kernels a Python call costs about as
    much).  fn must allocate nothing; the ABI launches on torch's current
    stream, which the capture redirects."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            for _ in range(reps):
                fn()
    torch.cuda.current_stream().wait_stream(side)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (reps * replays)
    del g
    return ms


def box_reference(torch):
    """Rates of two library operations on this box, measured right after the
    headline (clocks already up), so that runs on different boxes of the pool
    can be compared: an 8192^3 bf16 torch.mm and a 1 GiB device-to-device
    copy, each over 10 timed calls after 3 warm-up calls."""
    n = 8192
    a = torch.randn((n, n), device="cuda", dtype=torch.bfloat16)
    b = torch.randn((n, n), device="cuda", dtype=torch.bfloat16)
    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    gemm_ms = _event_ms(torch, lambda: torch.mm(a, b), 10)
    copy_ms = _event_ms(torch, lambda: dst.copy_(src), 10)
    del a, b, src, dst
    torch.cuda.empty_cache()
    return {"bf16_gemm_8192_tflops": round(2 * n ** 3 / (gemm_ms * 1e-3) / 1e12, 1),
            "copy_1gib_gbs": round(2 * (1 << 30) / (copy_ms * 1e-3) / 1e9, 1),
            "note": "library GEMM and device copy rates on this box, for comparing runs across boxes; "
                    "not part of the metric"}


def memory_bound_bench(torch, fa, cfg):
    """Achieved HBM rates of the memory-bound kernels around the attention,
    from algorithmic bytes (each tensor read or written once) over HIP-event
    time: the QK-RMSNorm + RoPE prologue of Q and K at the attention config's
    shape in one fused launch, as the blocks run it (forward reads x, writes
    the joint buffer; backward reads x and dy, writes dx; both read the
    per-token cos/sin rows and the weights), and the LoRA down / up pieces at
    the c4 img stream's shape (x [4096, 3072], r = 16: down reads x and A,
    writes u; up reads u and B and updates y in place), and the stream's
    q/k/v adapter gradients in one grouped call, and every factor gradient of
    a c4 step (both streams) in the one call the block makes."""
    from foundry_attn.configs import C4
    g = torch.Generator(device="cuda").manual_seed(7)
    bf = torch.bfloat16
    B, S, H, D = cfg.batch, cfg.seq, cfg.heads, cfg.head_dim
    xs = [torch.randn((B, S, H, D), device="cuda", generator=g).to(bf) for _ in range(2)]
    dys = [torch.randn((B, S, H, D), device="cuda", generator=g).to(bf) for _ in range(2)]
    ws = [(1 + 0.02 * torch.randn(D, device="cuda", generator=g)).to(bf) for _ in range(2)]
    cos, sin = fa.rope_tables(cfg.positions(), cfg.axes, cfg.theta, dtype=bf)
    ys, dxs = [torch.empty_like(x) for x in xs], [torch.empty_like(x) for x in xs]
    fwd_segs = [(xs[i], ws[i], cos, sin, cfg.axes, ys[i], 0) for i in range(2)]
    bwd_segs = [(xs[i], ws[i], cos, sin, cfg.axes, dys[i], 0, dxs[i]) for i in range(2)]
    row = B * S * H * D * 2
    tables = 2 * (2 * S * D * 2 + D * 2)  # each segment reads the tables and its weight
    N, C, r = C4.img_tokens, C4.hidden, C4.lora_rank
    lx = torch.randn((N, C), device="cuda", generator=g).to(bf)
    la = (torch.randn((r, C), device="cuda", generator=g) / r).to(bf)
    lb = (1e-3 * torch.randn((C, r), device="cuda", generator=g)).to(bf)
    lu = torch.empty((N, r), device="cuda", dtype=bf)
    ly = torch.randn((N, C), device="cuda", generator=g).to(bf)
    # the c4 stream's q/k/v adapter gradients in one fa_lora_grad_many call:
    # dA_qkv [3r, C] = t^T h and dB_j [C, r] = dy_j^T su_j (j = q, k, v)
    gh = torch.randn((N, C), device="cuda", generator=g).to(bf)
    gdy = [torch.randn((N, C), device="cuda", generator=g).to(bf) for _ in range(3)]
    gt = torch.randn((N, 3 * r), device="cuda", generator=g).to(bf)
    gsu = [torch.randn((N, r), device="cuda", generator=g).to(bf) for _ in range(3)]
    gout = [torch.empty((3 * r, C), device="cuda")] + [torch.empty((C, r), device="cuda") for _ in range(3)]
    gitems = [(gt, gh, 1.0, False, gout[0])] + [(gsu[j], gdy[j], 1.0, True, gout[1 + j]) for j in range(3)]
    gbytes = 4 * N * C * 2 + N * 6 * r * 2 + 6 * r * C * 4
    # every LoRA factor gradient of a c4 double-block step in one call, as
    # the block forms them: per stream (img N rows, txt T rows) the q/k/v
    # group above plus the out adapter's pair (dA_out = du^T a, dB_out =
    # dout^T u), 12 products
    T = C4.txt_tokens
    sitems, sbytes = [], 0
    for rows, qkv in ((N, gitems), (T, None)):
        if qkv is None:
            th = torch.randn((rows, C), device="cuda", generator=g).to(bf)
            qkv = [(torch.randn((rows, 3 * r), device="cuda", generator=g).to(bf), th, 1.0, False)] + \
                  [(torch.randn((rows, r), device="cuda", generator=g).to(bf),
                    torch.randn((rows, C), device="cuda", generator=g).to(bf), 1.0, True) for _ in range(3)]
        sa_ = torch.randn((rows, C), device="cuda", generator=g).to(bf)
        sdo = torch.randn((rows, C), device="cuda", generator=g).to(bf)
        sdu = torch.randn((rows, r), device="cuda", generator=g).to(bf)
        su = torch.randn((rows, r), device="cuda", generator=g).to(bf)
        sitems += [it[:4] for it in qkv] + [(sdu, sa_, 1.0, False), (su, sdo, 1.0, True)]
        sbytes += 6 * rows * C * 2 + 8 * rows * r * 2 + 8 * r * C * 4
    cases = {
        "qk_prologue_fwd": (lambda: fa.qk_prologue_multi(fwd_segs), 4 * row + tables),
        "qk_prologue_bwd": (lambda: fa.qk_prologue_bwd_multi(bwd_segs), 6 * row + tables),
        "lora_down": (lambda: fa.lora_down(lx, la, 1.0, out=lu), N * C * 2 + r * C * 2 + N * r * 2),
        "lora_up": (lambda: fa.lora_up(lu, lb, ly, 1.0), 2 * N * C * 2 + N * r * 2 + C * r * 2),
        "lora_grad_qkv": (lambda: fa.lora_grad_many(gitems), gbytes),
        "lora_grad_step": (lambda: fa.lora_grad_many(sitems), sbytes),
    }
    out = {}
    for name, (fn, nbytes) in cases.items():
        ms = _graph_ms(torch, fn)
        eager = _event_ms(torch, fn)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"ms": round(ms, 4), "bytes": nbytes, "gbs": round(gbs, 1),
                     "pct_of_hbm_peak": round(100 * gbs / PEAK_HBM_GBS, 2), "eager_ms": round(eager, 4)}
    out["shapes"] = (f"prologue: Q and K in one launch, each B={B} S={S} H={H} D={D} bf16; "
                     f"lora: N={N} C={C} r={r} bf16; lora_grad_qkv: dA [{3 * r}, {C}] and three dB [{C}, {r}] "
                     f"in one call (reads h and three dy, f32 grads); lora_grad_step: the c4 step's 12 factor "
                     f"gradients (q/k/v and out of the img ({N} rows) and txt ({T} rows) streams) in one call")
    out["timing"] = ("ms: HIP events over 5 replays of a HIP graph of 20 calls (kernel time); "
                     "eager_ms: HIP events over 20 eager calls, which includes the host's per-call time")
    return out


def gemm_bench(torch):
    """This build's bf16 GEMM (fa_gemm_bf16) against the tuned library GEMM
    at the c4 block's W1 shape ([4096, 3072] x [12288, 3072]^T), plain and
    with the fused GELU epilogue against the library GEMM followed by the
    GELU kernel: HIP events over 20 calls after 3."""
    from foundry_attn import block as fb
    from foundry_attn import gemm_tuning
    gemm_tuning.enable()
    g = torch.Generator(device="cuda").manual_seed(11)
    M, N, K = 4096, 12288, 3072
    a = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    w = (0.02 * torch.randn((N, K), device="cuda", generator=g)).to(torch.bfloat16)
    c = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)
    act = torch.empty_like(c)
    lib_ms = _event_ms(torch, lambda: torch.mm(a, w.t(), out=c))
    lib_gelu_ms = _event_ms(torch, lambda: (torch.mm(a, w.t(), out=c), fb.gelu(c, out=act)))
    own_ms = _event_ms(torch, lambda: fb.gemm(a, w, out=c))
    own_gelu_ms = _event_ms(torch, lambda: fb.gemm(a, w, "gelu", out=c, act_out=act))
    tf = lambda ms: round(2 * M * N * K / (ms * 1e-3) / 1e12, 1)
    del a, w, c, act
    return {"shape": f"M={M} N={N} K={K} bf16 (c4 W1)",
            "library_ms": round(lib_ms, 4), "library_tflops": tf(lib_ms),
            "own_ms": round(own_ms, 4), "own_tflops": tf(own_ms),
            "library_plus_gelu_ms": round(lib_gelu_ms, 4), "own_fused_gelu_ms": round(own_gelu_ms, 4),
            "note": "the blocks keep the library GEMM: this GEMM is slower than the tuned library solution "
                    "by more than the separate GELU pass costs"}


def shard_bench(torch, fa, cfg):
    """Attention fwd+bwd at one GPU's share of cfg's heads under P-way
    sequence (Ulysses) parallelism, P = 2, 4, 8: the same kernels at
    H = heads / P and the full sequence (what one GPU runs between the two
    all-to-alls).  Small grids take the range-split kernels; `split` is the
    number of key/query ranges per tile (1 = unsplit)."""
    import dataclasses
    out = {}
    for p in (2, 4, 8):
        if cfg.heads % p:
            continue
        c = dataclasses.replace(cfg, heads=cfg.heads // p)
        q, k, v, do, keep = make_inputs(c, torch, fa)
        o = torch.empty_like(q)
        lse = torch.empty((c.batch, c.heads, c.seq), dtype=torch.float32, device="cuda")
        fws, bws = fa.attn_workspace_bytes(q)
        wf = torch.empty(max(fws, 256), dtype=torch.uint8, device="cuda")
        wb = torch.empty(bws, dtype=torch.uint8, device="cuda")
        grads = tuple(torch.empty_like(q) for _ in range(3))
        fwd = lambda: fa.attn_fwd(q, k, v, c.scale, keep, out=o, lse=lse, workspace=wf)
        bwd = lambda: fa.attn_bwd(q, k, v, o, do, lse, c.scale, keep, workspace=wb, out=grads)
        for _ in range(20):
            fwd()
            bwd()
        f_ms, b_ms = _event_ms(torch, fwd), _event_ms(torch, bwd)
        tf = lambda fl, ms: round(fl / (ms * 1e-3) / 1e12, 2)
        out[f"{p}_gpus"] = {
            # the forward workspace holds split x (O rows in f32 + their LSEs)
            "heads": c.heads, "split": round(fws / (c.batch * c.heads * c.seq * (c.head_dim + 1) * 4)) or 1,
            "fwd_ms": round(f_ms, 4), "bwd_ms": round(b_ms, 4),
            "fwd_tflops": tf(c.fwd_flops(), f_ms), "bwd_tflops": tf(c.bwd_flops(), b_ms),
            "tflops": tf(c.fwd_flops() + c.bwd_flops(), f_ms + b_ms),
            "pct_of_peak": round(100 * tf(c.fwd_flops() + c.bwd_flops(), f_ms + b_ms) / PEAK_BF16_TFLOPS, 2)}
        del q, k, v, do, o, lse, wf, wb, grads
    return out


def _lora_flops(N, r, fin, fout):
    """x A^T, u B^T forward; dB, du, dA, dx backward: 6 skinny GEMMs of 2 N r (in or out)."""
    return 6 * N * r * (fin + fout)


def block_bench(torch, steps: int, warmup: int):
    """c4: one double-stream LoRA block training step per step, as a block
    inside a stack: forward, backward to the LoRA factors and to the block
    input (dX through every frozen linear and both layer_norm_mods), AdamW.
    img 4096 + txt 512 tokens, dim 3072, 24 x 128 heads, MLP 4x tanh-GELU,
    LoRA r16 on q/k/v/out of both streams; synthetic N(0,1) inputs,
    conditioning and dY; random-init weights."""
    from foundry_attn import block as fb
    from foundry_attn.configs import C4
    rows = int(round(C4.img_tokens ** 0.5))
    blk = fb.random_block(C4.hidden, C4.heads, C4.txt_tokens, rows, C4.img_tokens // rows, C4.mlp_ratio,
                          C4.lora_rank, C4.lora_alpha)
    g = torch.Generator(device="cuda").manual_seed(20261028)
    blk.set_conditioning(torch.randn(C4.hidden, device="cuda", generator=g).to(torch.bfloat16))
    x = {"img": torch.randn(C4.img_tokens, C4.hidden, device="cuda", generator=g).to(torch.bfloat16),
         "txt": torch.randn(C4.txt_tokens, C4.hidden, device="cuda", generator=g).to(torch.bfloat16)}
    dy = {k: torch.randn(v.shape, device="cuda", generator=g).to(torch.bfloat16) for k, v in x.items()}
    e_wall, e_gpu = _time_steps(torch, lambda: blk.train_step(x, dy, want_dx=True), steps, warmup)
    wall, gpu = _time_steps(torch, fb.GraphedTrainStep(blk, x, dy, want_dx=True), steps, warmup)
    N, C, F, H, D, r = (C4.img_tokens + C4.txt_tokens, C4.hidden, C4.mlp_ratio * C4.hidden, C4.heads,
                        C4.head_dim, C4.lora_rank)
    gemm = 2 * (2 * N * C * 3 * C + 2 * N * C * C + 2 * 2 * N * C * F)  # forward + dX of every linear
    attn = 14 * H * N * N * D
    lora = 4 * _lora_flops(N, r, C, C)
    flops = gemm + attn + lora
    return {"workload": "c4: double-stream LoRA block step (fwd + bwd incl. block-input dX + AdamW), "
                        "img 4096 + txt 512 tokens, dim 3072, 24x128 heads, MLP 4x tanh-GELU, LoRA r16 on "
                        "q/k/v/out of both streams",
            "steps": steps, "warmup": warmup, "steps_per_s": round(1.0 / wall, 2),
            "ms_per_step": round(wall * 1e3, 3), "gpu_ms_per_step": round(gpu * 1e3, 3),
            "tflops": round(flops / wall / 1e12, 1), "step_tflop": round(flops / 1e12, 3),
            "eager_ms_per_step": round(e_wall * 1e3, 3), "timing": _GRAPH_STEP_NOTE}


_GRAPH_STEP_NOTE = ("ms_per_step: one HIP-graph replay per step (forward + backward captured once by "
                    "block.GraphedTrainStep) plus the eager AdamW launch and adapter refresh, the same kernels "
                    "as the op-by-op step timed in eager_ms_per_step")


def single_block_bench(torch, steps: int, warmup: int):
    """The single-stream klein block step (fused to_in 3072 -> 27648 with
    LoRA, QK-RMSNorm + klein RoPE, joint attention over 4608 tokens, SwiGLU
    3x, fused to_out 12288 -> 3072 with LoRA, one gate), backward including
    the block-input dX, AdamW on the LoRA factors (r16)."""
    from foundry_attn import block as fb
    from foundry_attn.configs import C4
    rows = int(round(C4.img_tokens ** 0.5))
    blk = fb.random_single_block(C4.hidden, C4.heads, C4.txt_tokens, rows, C4.img_tokens // rows,
                                 rank=C4.lora_rank, alpha=C4.lora_alpha)
    g = torch.Generator(device="cuda").manual_seed(20261029)
    blk.set_conditioning(torch.randn(C4.hidden, device="cuda", generator=g).to(torch.bfloat16))
    N = C4.img_tokens + C4.txt_tokens
    x = torch.randn(N, C4.hidden, device="cuda", generator=g).to(torch.bfloat16)
    dy = torch.randn(N, C4.hidden, device="cuda", generator=g).to(torch.bfloat16)
    e_wall, e_gpu = _time_steps(torch, lambda: blk.train_step(x, dy, want_dx=True), steps, warmup)
    wall, gpu = _time_steps(torch, fb.GraphedTrainStep(blk, x, dy, want_dx=True), steps, warmup)
    C, M, H, D, r = C4.hidden, blk.M, C4.heads, C4.head_dim, C4.lora_rank
    gemm = 2 * (2 * N * C * (3 * C + 2 * M) + 2 * N * (C + M) * C)
    attn = 14 * H * N * N * D
    lora = _lora_flops(N, r, C, 3 * C + 2 * M) + _lora_flops(N, r, C + M, C)
    flops = gemm + attn + lora
    return {"workload": "single-stream klein block step (fwd + bwd incl. block-input dX + AdamW), 4608 joint "
                        "tokens, dim 3072, 24x128 heads, SwiGLU 3x, LoRA r16 on to_in and to_out",
            "steps": steps, "warmup": warmup, "steps_per_s": round(1.0 / wall, 2),
            "ms_per_step": round(wall * 1e3, 3), "gpu_ms_per_step": round(gpu * 1e3, 3),
            "tflops": round(flops / wall / 1e12, 1), "step_tflop": round(flops / 1e12, 3),
            "eager_ms_per_step": round(e_wall * 1e3, 3), "timing": _GRAPH_STEP_NOTE}


def stack_bench(torch, steps: int, warmup: int):
    """A checkpointed klein stack step (checkpointed_backward, lib.rs:541-638):
    the c4 double block, cat, the single block, split; MSE seed, recompute and
    backward stage by stage, AdamW.  Timed twice: recomputing each attention
    forward (the reference's scheme) and reusing the saved attention output
    and LSE."""
    from foundry_attn import block as fb
    from foundry_attn import checkpoint as ck
    from foundry_attn.configs import C4
    rows = int(round(C4.img_tokens ** 0.5))
    dbl = fb.random_block(C4.hidden, C4.heads, C4.txt_tokens, rows, C4.img_tokens // rows, C4.mlp_ratio,
                          C4.lora_rank, C4.lora_alpha)
    sgl = fb.random_single_block(C4.hidden, C4.heads, C4.txt_tokens, rows, C4.img_tokens // rows,
                                 rank=C4.lora_rank, alpha=C4.lora_alpha)
    g = torch.Generator(device="cuda").manual_seed(20261030)
    c = torch.randn(C4.hidden, device="cuda", generator=g).to(torch.bfloat16)
    dbl.set_conditioning(c)
    sgl.set_conditioning(c)
    stages = [ck.DoubleStage(dbl), ck.JoinStage(C4.txt_tokens), ck.SingleStage(sgl), ck.SplitStage(C4.txt_tokens)]
    mk = lambda n: torch.randn(n, C4.hidden, device="cuda", generator=g).to(torch.bfloat16)
    inputs = [mk(C4.txt_tokens), mk(C4.img_tokens)]
    seed = ck.mse_seed([mk(C4.txt_tokens), mk(C4.img_tokens)])
    out = {"workload": "checkpointed klein stack step: c4 double block -> cat -> single block -> split, MSE "
                       "seed, recompute + backward per stage, AdamW; 4608 tokens, dim 3072",
           "steps": steps, "warmup": warmup}
    for save in (False, True):
        def step():
            _, _, grads = ck.checkpointed_step(stages, inputs, seed, save_attention=save)
            ck.apply_adamw(stages, grads)
        wall, gpu = _time_steps(torch, step, steps, warmup)
        key = "saved_attention" if save else "recompute_attention"
        out[key] = {"steps_per_s": round(1.0 / wall, 2), "ms_per_step": round(wall * 1e3, 3),
                    "gpu_ms_per_step": round(gpu * 1e3, 3)}
    return out


def host_cores():
    """(logical CPUs, physical cores, CPUs this process may run on, CPU model)
    from os.cpu_count (nproc --all), /proc/cpuinfo's distinct (physical id,
    core id) pairs (lscpu's core count) and the scheduler affinity."""
    model, pairs, phys, core = "", set(), None, None
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "model name" and not model:
                model = val
            elif key == "physical id":
                phys = val
            elif key == "core id":
                core = val
            elif not key and phys is not None and core is not None:
                pairs.add((phys, core))
                phys = core = None
        if phys is not None and core is not None:
            pairs.add((phys, core))
    except OSError:
        pass
    return os.cpu_count() or 0, len(pairs) or None, len(os.sched_getaffinity(0)), model


def cpu_baseline(cfg, budget_s: float):
    """The oracle (port of the reference's Candle CPU path) on whole heads of
    the same workload, f32 arithmetic on bf16-valued inputs, one OpenMP thread
    per CPU this process may use (the box's share of the host: its
    scheduler affinity)."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    nproc, physical, affinity, cpu_model = host_cores()
    threads = affinity
    rng = np.random.default_rng(0)
    B, S, D = 1, cfg.seq, cfg.head_dim
    mk = lambda: oracle.bf16_round(rng.standard_normal((B, S, 1, D)).astype(np.float32))
    q, k, v, do = mk(), mk(), mk(), mk()
    heads, t = 0, 0.0
    while t < budget_s and heads < cfg.heads * cfg.batch:
        t0 = time.perf_counter()
        oracle.attn_fwd(q, k, v, scale=cfg.scale, bf16=True, nthreads=threads)
        oracle.attn_bwd(q, k, v, do, scale=cfg.scale, bf16=True, nthreads=threads)
        t += time.perf_counter() - t0
        heads += 1
    flops = 14.0 * S * S * D * heads
    return {"value": round(flops / t / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"{heads} head(s) of {cfg.name} (S={S}, D={D}) fwd+bwd, oracle "
                      f"(materialised f32 scores, 5-GEMM backward), {t:.1f} s on {cpu_model}, "
                      f"{threads} OpenMP threads",
            "ms_per_head": round(1e3 * t / heads, 1),
            "host": {"nproc": nproc, "physical_cores": physical, "affinity_cpus": affinity,
                     "threads_used": threads, "cpu_model": cpu_model}}


def attention_bench(torch, fa, cfg, steps: int, warmup: int, settle_s: float):
    """Time `steps` fwd+bwd steps of cfg through the ABI (after settle_s
    seconds of untimed steps and `warmup` warm-up steps), then time each
    launch with HIP events in a separate pass over the same number of steps.
    Returns the step time (ms) and the per-kernel means (ms)."""
    q, k, v, do, keep = make_inputs(cfg, torch, fa)
    lse = torch.empty((cfg.batch, cfg.heads, cfg.seq), dtype=torch.float32, device="cuda")
    o = torch.empty_like(q)
    # the full backward workspace: dQ reads the stored dS where that path applies
    ws = torch.empty(max(fa.attn_workspace_bytes(q)[1], 256), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()
    grads = (torch.empty_like(q), torch.empty_like(q), torch.empty_like(q))
    ph = [(fa._abi.FA_BWD_PREPASS, None), (fa._abi.FA_BWD_DKDV, None), (fa._abi.FA_BWD_DQ, None)]

    def step(ev=None):
        """One fwd+bwd.  With `ev`, HIP events bracket each launch on the
        launch stream (the ABI launches on torch's current stream)."""
        if ev is None:
            fa.attn_fwd(q, k, v, cfg.scale, keep, out=o, lse=lse)
            fa.attn_bwd(q, k, v, o, do, lse, cfg.scale, keep, workspace=ws, out=grads)
            return
        ev[0].record(stream)
        fa.attn_fwd(q, k, v, cfg.scale, keep, out=o, lse=lse)
        ev[1].record(stream)
        for i, p_ in enumerate(ph):
            fa.attn_bwd(q, k, v, o, do, lse, cfg.scale, keep, workspace=ws, out=grads, phases=[p_])
            ev[2 + i].record(stream)

    t_end = time.perf_counter() + settle_s
    while time.perf_counter() < t_end:
        for _ in range(8):
            step()
        torch.cuda.synchronize()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(steps)]
    for e in evs:
        step(e)
    torch.cuda.synchronize()
    names = ["attn_fwd", "attn_bwd_prepass", "attn_bwd_dkdv", "attn_bwd_dq"]
    kms = {nm: sum(e[i].elapsed_time(e[i + 1]) for e in evs) / len(evs) for i, nm in enumerate(names)}
    return 1e3 * wall / steps, kms, keep is not None


def attention_record(cfg, ms: float, kms: dict) -> dict:
    """Rates of one attention measurement: the fwd+bwd step, the forward and
    the three backward launches (algorithmic FLOPs per launch: forward 2G,
    dK/dV 4G -- the S recompute, dP, dV, dK --, dQ 1G; G = 2*B*H*S_q*S_kv*D)."""
    B, H, S, D = cfg.batch, cfg.heads, cfg.seq, cfg.head_dim
    unit = cfg.fwd_flops() / 2.0
    kflops = {"attn_fwd": 2 * unit, "attn_bwd_dkdv": 4 * unit, "attn_bwd_dq": 1 * unit}
    pre_bytes = 2 * B * S * H * D * 2 + 3 * B * H * S * 4  # read O, dO, LSE; write delta, lse2
    tf = lambda fl, t: fl / (t * 1e-3) / 1e12
    pct = lambda x: round(100 * x / PEAK_BF16_TFLOPS, 2)
    kernels = {}
    for nm, t in kms.items():
        if nm in kflops:
            kernels[nm] = {"ms": round(t, 4), "tflops": round(tf(kflops[nm], t), 2),
                           "pct_of_peak": pct(tf(kflops[nm], t))}
            # the HBM rate from the counter table's bytes per launch (dQ from
            # the stored dS is HBM-bound)
            hbm = TRAFFIC.get((cfg.name, nm))
            if hbm:
                kernels[nm]["hbm_gbs"] = round(hbm / (t * 1e-3) / 1e9, 1)
        else:
            gbs = pre_bytes / (t * 1e-3) / 1e9
            kernels[nm] = {"ms": round(t, 4), "gbs": round(gbs, 1), "pct_of_hbm_peak": round(100 * gbs / PEAK_HBM_GBS, 2)}
    bwd_ms = kms["attn_bwd_prepass"] + kms["attn_bwd_dkdv"] + kms["attn_bwd_dq"]
    value = tf(cfg.fwd_flops() + cfg.bwd_flops(), ms)
    dominant = max(kflops, key=lambda nm: kms[nm])
    return {
        "value": value, "ms": ms, "kernels": kernels, "dominant": dominant,
        "dominant_tflops": tf(kflops[dominant], kms[dominant]),
        "fwd": {"ms": round(kms["attn_fwd"], 4), "tflops": round(tf(cfg.fwd_flops(), kms["attn_fwd"]), 2),
                "pct_of_peak": pct(tf(cfg.fwd_flops(), kms["attn_fwd"]))},
        "bwd": {"ms": round(bwd_ms, 4), "tflops": round(tf(cfg.bwd_flops(), bwd_ms), 2),
                "pct_of_peak": pct(tf(cfg.bwd_flops(), bwd_ms))},
    }


def roofline(cfg, r: dict) -> dict:
    """The roofline record of one attention measurement: its dominant
    kernel's algorithmic rate against the bf16 MFMA peak, and that kernel's
    HBM bytes per launch from the counter table (null when not measured)."""
    dom_tf = r["dominant_tflops"]
    return {"bound": "mfma", "kernel": r["dominant"], "achieved": round(dom_tf, 2), "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(dom_tf / PEAK_BF16_TFLOPS, 4),
            "traffic": TRAFFIC.get((cfg.name, r["dominant"]))}


def configs_bench(torch, fa, steps: int, warmup: int, settle_s: float):
    """c3 and c5 measured as the
    headline is: step time over `steps` timed fwd+bwd steps, then per-launch
    HIP events."""
    from foundry_attn.configs import CONFIGS
    out = {}
    for name in ("c3", "c5"):
        cfg = CONFIGS[name]
        ms, kms, masked = attention_bench(torch, fa, cfg, steps, warmup, settle_s)
        r = attention_record(cfg, ms, kms)
        out[name] = {"workload": f"B={cfg.batch} H={cfg.heads} S={cfg.seq} ({cfg.txt_len} txt + "
                                 f"{cfg.img_rows}x{cfg.img_cols} img) D={cfg.head_dim} bf16"
                                 + (", key-padding mask (FLOPs count kept keys)" if masked else ""),
                     "ms_per_step": round(ms, 4), "tflops": round(r["value"], 2),
                     "pct_of_peak": round(100 * r["value"] / PEAK_BF16_TFLOPS, 2),
                     "fwd": r["fwd"], "bwd": r["bwd"], "roofline": roofline(cfg, r), "kernels": r["kernels"]}
        torch.cuda.empty_cache()
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build is single-GPU; --gpus {args.gpus} is not supported "
              "(the attention path would shard over heads, one process per GPU, with an all-to-all "
              "before and after attention; only one GPU's share is measured here)",
              file=sys.stderr)
        return 2
    import torch
    import foundry_attn as fa
    from foundry_attn.configs import CONFIGS

    cfg = CONFIGS[args.config]
    torch.cuda.set_device(0)
    if args.calib_copy_mib > 0:
        src = torch.ones(args.calib_copy_mib << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    ms, kms, masked = attention_bench(torch, fa, cfg, args.steps, args.warmup, args.settle_s)
    r = attention_record(cfg, ms, kms)
    value = r["value"]
    rec = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) Q/K/V/dO; Q/K RMSNormed + axial RoPE by the prologue kernel)",
        "config": {"workload": f"{cfg.name}: joint attention fwd+bwd, B={cfg.batch} H={cfg.heads} "
                               f"S={cfg.seq} ({cfg.txt_len} txt + {cfg.img_rows}x{cfg.img_cols} img) "
                               f"D={cfg.head_dim} bf16" + (", key-padding mask" if masked else ""),
                   "batch": cfg.batch, "heads": cfg.heads, "seq_len": cfg.seq,
                   "head_dim": cfg.head_dim, "parallelism": "single GPU"},
        "pct_of_peak": round(100 * value / PEAK_BF16_TFLOPS, 2),
        "fwd": r["fwd"],
        "bwd": r["bwd"],
        "roofline": roofline(cfg, r),
        "kernels": r["kernels"],
    }
    if not args.only_headline:
        rec["box_reference"] = box_reference(torch)
        rec["configs"] = configs_bench(torch, fa, args.steps, args.warmup, args.settle_s)
        rec["memory_bound"] = memory_bound_bench(torch, fa, cfg)
        rec["ulysses_shards"] = shard_bench(torch, fa, cfg)
        rec["gemm_mlp"] = gemm_bench(torch)
        if args.block_steps > 0:
            rec["block"] = block_bench(torch, args.block_steps, max(2, args.block_steps // 3))
            rec["single_block"] = single_block_bench(torch, args.block_steps, max(2, args.block_steps // 3))
            rec["checkpointed_stack"] = stack_bench(torch, args.block_steps, max(2, args.block_steps // 3))
    rec["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds) if args.cpu_seconds > 0 and not args.only_headline \
        else None
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
