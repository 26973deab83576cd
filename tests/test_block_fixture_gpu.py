"""The reference's own double block (crates/foundry-spike/src/lib.rs:301-392;
tools/fixtures/gen_block.py:199-240) replayed on the HIP path with the
reference fixture's weights and inputs, fp32 and bf16.

The block is DoubleBlockLoRA configured as the fixture's: dim 256, 2 heads
x 128, txt 8 + img 16 (4 x 4) tokens, biases on every linear, SwiGLU MLP
(hidden 512), LoRA (rank 4, scale 2.0) on the image stream's to_q and to_v
only, one modulation linear for both streams, RoPE axes [32] x 4 with
theta 1e4 at the fixture's positions (img (row, col, 0, 0), txt (l, 0, 0, 0),
gen_block.py:311-314).

Forward: every activation the fixture holds for the block is compared --
double.{img,txt}_norm1, double.q / double.k, attn_in/double.{q,k,v,attn},
double.attn_img, double.img_post_attn, double.{img,txt}_out.
Backward: the block runs its own backward from the gradient at its outputs
(which the fixture does not hold: the oracle's restatement of the single
block and the MSE seed after it supplies it, gen_block.py:300-360) and is
compared at grad/attn/double.{out,q,k,v}, grad/double.img.to_{q,v}.lora_{a,b}
and grad/inputs/{img,txt}; then one AdamW step against opt1/*.

Gates: for bf16, the reference's cos >= 0.999 (lib.rs:28-29) with the
north-star rel-L2 <= 1e-2 (tighter than the reference's 2e-2); for fp32,
rel-L2 <= 1e-4 (the reference's fp32 policy, docs/TESTING.md:15) and
cos >= 0.99999."""
import numpy as np
import pytest
import torch

import fixture_ref
from foundry_attn import block as fb
from helpers import cosine, load_pipeline_golden, rel_l2

pytestmark = pytest.mark.gpu

GATES = {"fp32": (0.99999, 1e-4), "bf16": (0.999, 1e-2)}


def build(f, dtype, device):
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(device=device, dtype=dtype)
    W = lambda n: f[f"weights/{n}.weight"]
    Bv = lambda n: f[f"weights/{n}.bias"]
    ws = {}
    for name in ("txt", "img"):
        p = f"double.{name}"
        sw = fb.StreamWeights(
            w_qkv=dev(np.concatenate([W(f"{p}.to_q"), W(f"{p}.to_k"), W(f"{p}.to_v")])),
            w_out=dev(W(f"{p}.to_out")),
            w1=dev(np.concatenate([W(f"{p}.mlp.gate"), W(f"{p}.mlp.up")])),
            w2=dev(W(f"{p}.mlp.down")),
            q_norm=dev(f[f"weights/{p}_q_norm.weight"]), k_norm=dev(f[f"weights/{p}_k_norm.weight"]),
            w_mod=dev(W("double.mod")), b_mod=dev(Bv("double.mod")),
            b_qkv=dev(np.concatenate([Bv(f"{p}.to_q"), Bv(f"{p}.to_k"), Bv(f"{p}.to_v")])),
            b_out=dev(Bv(f"{p}.to_out")),
            b1=dev(np.concatenate([Bv(f"{p}.mlp.gate"), Bv(f"{p}.mlp.up")])),
            b2=dev(Bv(f"{p}.mlp.down")))
        if name == "img":
            for t in ("q", "v"):
                sw.lora_a[t] = dev(f[f"weights/{p}.to_{t}.lora_a"])
                sw.lora_b[t] = dev(f[f"weights/{p}.to_{t}.lora_b"])
                for part, ref in (("a", sw.lora_a[t]), ("b", sw.lora_b[t])):
                    sw.m[f"{t}.{part}"] = torch.zeros(ref.shape, dtype=torch.float32, device=device)
                    sw.v[f"{t}.{part}"] = torch.zeros(ref.shape, dtype=torch.float32, device=device)
        ws[name] = sw
    pos_img, pos_txt = fixture_ref.positions()
    blk = fb.DoubleBlockLoRA(ws, fixture_ref.HEADS, fixture_ref.HEAD_DIM, fixture_ref.TXT, fixture_ref.GRID,
                             fixture_ref.GRID, axes=fixture_ref.AXES, theta=fixture_ref.THETA,
                             lora_scale=fixture_ref.LORA_SCALE, eps=fixture_ref.EPS, mlp="swiglu",
                             positions=np.concatenate([pos_txt, pos_img]), overlap_streams=False,
                             tuned_gemms=False)
    blk.set_conditioning(dev(f["inputs/temb"]))
    return blk, dev


def host(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("tag", ["fp32", "bf16"])
def test_fixture_double_block_on_hip(tag, device):
    f = load_pipeline_golden(tag)
    dtype = torch.float32 if tag == "fp32" else torch.bfloat16
    cos_min, rel_max = GATES[tag]
    blk, dev = build(f, dtype, device)
    blk.capture = {}
    x = {"txt": dev(f["inputs/txt"]), "img": dev(f["inputs/img"])}
    _, og = fixture_ref.pipeline(f, bf16=tag == "bf16")
    dy = {"txt": dev(og["grad/double.txt_out"]), "img": dev(og["grad/double.img_out"])}
    y, grads = blk.forward_backward(x, dy, want_dx=True)
    torch.cuda.synchronize()
    T = fixture_ref.TXT
    cap = blk.capture
    got = {
        "double.img_norm1": cap["img_norm1"], "double.txt_norm1": cap["txt_norm1"],
        "double.q": cap["img.q"], "double.k": cap["img.k"],
        "attn_in/double.q": cap["attn_in.q"], "attn_in/double.k": cap["attn_in.k"],
        "attn_in/double.v": cap["attn_in.v"], "attn_in/double.attn": cap["attn"],
        "double.attn_img": cap["attn"][T:], "double.img_post_attn": cap["img_post_attn"],
        "double.img_out": y["img"], "double.txt_out": y["txt"],
        "grad/attn/double.out": cap["grad_attn.out"], "grad/attn/double.q": cap["grad_attn.q"],
        "grad/attn/double.k": cap["grad_attn.k"], "grad/attn/double.v": cap["grad_attn.v"],
        "grad/double.img.to_q.lora_a": grads[("img", "q")][0], "grad/double.img.to_q.lora_b": grads[("img", "q")][1],
        "grad/double.img.to_v.lora_a": grads[("img", "v")][0], "grad/double.img.to_v.lora_b": grads[("img", "v")][1],
        "grad/inputs/img": grads[("img", "x")], "grad/inputs/txt": grads[("txt", "x")],
    }
    # only the image stream's to_q / to_v carry LoRA
    assert sorted(k for k in grads if k[1] != "x") == [("img", "q"), ("img", "v")]
    report = []
    for key, g in got.items():
        want = f[key].astype(np.float64)
        a = host(g).reshape(want.shape)
        c, r = cosine(a, want), rel_l2(a, want)
        report.append(f"{key}: cos {c:.6f} rel-L2 {r:.2e}")
        assert np.isfinite(a).all(), key
        assert c >= cos_min and r <= rel_max, "\n".join(report)
    print("\n".join(report))

    # one AdamW step from the reference's initial factors (lr 1e-3, betas
    # (0.9, 0.999), eps 1e-8: the fixture's opt1/* step)
    blk.apply_adamw(grads, lr=1e-3, betas=(0.9, 0.999), eps=1e-8)
    torch.cuda.synchronize()
    for t in ("q", "v"):
        for part, got_t in (("a", blk.w["img"].lora_a[t]), ("b", blk.w["img"].lora_b[t])):
            key = f"opt1/double.img.to_{t}.lora_{part}"
            want = f[key].astype(np.float64)
            a = host(got_t)
            c, r = cosine(a, want), rel_l2(a, want)
            assert c >= cos_min and r <= rel_max, (key, c, r)


def test_fixture_block_needs_matching_positions(device):
    """positions of the wrong shape are refused before any device work."""
    f = load_pipeline_golden("fp32")
    with pytest.raises(ValueError):
        blk, _ = build(f, torch.float32, device)
        fb.DoubleBlockLoRA(blk.w, 2, 128, 8, 4, 4, axes=(32,) * 4, mlp="swiglu",
                           positions=np.zeros((23, 4), np.float32), overlap_streams=False, tuned_gemms=False)
