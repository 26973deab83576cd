"""LoRA adapter files (foundry_attn/lora_file.py), on the CPU: the diffusers
layout the klein trainer writes (docs/RESEARCH.md:87-97 and its section
3.1: `transformer.<module>.lora_A.weight` [rank, in], `.lora_B.weight`
[out, rank], bf16, alpha in the PEFT metadata) and the reference harness's
own weight keys (throughput.rs:1078-1093), saved from and loaded into tiny
blocks built on the CPU (no kernel runs)."""
import json

import pytest
import torch
from safetensors import safe_open

from foundry_attn import block as fb
from foundry_attn import lora_file as lf

C, H, R = 64, 2, 4


def double_block(seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    bf = torch.bfloat16
    ws = {}
    for name in fb.STREAMS:
        z = lambda *s: torch.zeros(*s, dtype=bf)
        w = fb.StreamWeights(w_qkv=z(3 * C, C), w_out=z(C, C), w1=z(4 * C, C), w2=z(C, 4 * C),
                             q_norm=torch.ones(C // H, dtype=bf), k_norm=torch.ones(C // H, dtype=bf), w_mod=z(6 * C, C))
        for t in fb.LORA_TARGETS:
            w.lora_a[t] = torch.randn(R, C, generator=g).to(bf)
            w.lora_b[t] = torch.randn(C, R, generator=g).to(bf)
        ws[name] = w
    return fb.DoubleBlockLoRA(ws, H, C // H, 4, 2, 4, lora_scale=scale, overlap_streams=False)


def single_block(seed, scale=1.0):
    return fb.random_single_block(C, H, 4, 2, 4, rank=R, alpha=scale * R, device="cpu", seed=seed)


def stack(seed, scale=1.0):
    return [double_block(seed, scale), double_block(seed + 1, scale)], [single_block(seed + 2, scale),
                                                                        single_block(seed + 3, scale)]


def factors(doubles, singles):
    out = {}
    for i, b in enumerate(doubles):
        for s in fb.STREAMS:
            for t in fb.LORA_TARGETS:
                out[("d", i, s, t)] = (b.w[s].lora_a[t].clone(), b.w[s].lora_b[t].clone())
    for i, b in enumerate(singles):
        for t in fb.SINGLE_LORA_TARGETS:
            out[("s", i, t)] = (b.w.lora_a[t].clone(), b.w.lora_b[t].clone())
    return out


def test_diffusers_layout_keys_shapes_metadata(tmp_path):
    d, s = stack(1)
    path = str(tmp_path / "pytorch_lora_weights.safetensors")
    lf.save_lora(path, d, s)
    with safe_open(path, framework="pt") as f:
        keys = set(f.keys())
        meta = f.metadata()
        shapes = {k: tuple(f.get_slice(k).get_shape()) for k in keys}
        dtypes = {f.get_slice(k).get_dtype() for k in keys}
    want = set()
    for i in range(2):
        for mod in ("attn.to_q", "attn.to_k", "attn.to_v", "attn.to_out.0", "attn.add_q_proj", "attn.add_k_proj",
                    "attn.add_v_proj", "attn.to_add_out"):
            want |= {f"transformer.transformer_blocks.{i}.{mod}.lora_A.weight",
                     f"transformer.transformer_blocks.{i}.{mod}.lora_B.weight"}
        for mod in ("attn.to_qkv_mlp_proj", "attn.to_out"):
            want |= {f"transformer.single_transformer_blocks.{i}.{mod}.lora_A.weight",
                     f"transformer.single_transformer_blocks.{i}.{mod}.lora_B.weight"}
    assert keys == want
    assert dtypes == {"BF16"}
    M = 3 * C
    assert shapes["transformer.transformer_blocks.0.attn.to_q.lora_A.weight"] == (R, C)
    assert shapes["transformer.transformer_blocks.0.attn.to_out.0.lora_B.weight"] == (C, R)
    assert shapes["transformer.single_transformer_blocks.1.attn.to_qkv_mlp_proj.lora_A.weight"] == (R, C)
    assert shapes["transformer.single_transformer_blocks.1.attn.to_qkv_mlp_proj.lora_B.weight"] == (3 * C + 2 * M, R)
    assert shapes["transformer.single_transformer_blocks.0.attn.to_out.lora_A.weight"] == (R, C + M)
    assert shapes["transformer.single_transformer_blocks.0.attn.to_out.lora_B.weight"] == (C, R)
    assert meta["format"] == "pt"
    peft = json.loads(meta["lora_adapter_metadata"])
    assert peft["transformer.r"] == R and peft["transformer.lora_alpha"] == R
    assert peft["transformer.init_lora_weights"] == "gaussian"
    assert peft["transformer.use_rslora"] is False and peft["transformer.use_dora"] is False
    assert "attn.to_qkv_mlp_proj" in peft["transformer.target_modules"]
    assert lf.read_metadata(path) == (R, float(R))


@pytest.mark.parametrize("layout", ["diffusers", "foundry"])
def test_round_trip_restores_every_factor(tmp_path, layout):
    src_d, src_s = stack(10)
    path = str(tmp_path / f"lora_{layout}.safetensors")
    lf.save_lora(path, src_d, src_s, layout=layout)
    dst_d, dst_s = stack(20)
    assert not torch.equal(dst_d[0].w["img"].lora_a["q"], src_d[0].w["img"].lora_a["q"])
    rep = lf.load_lora(path, dst_d, dst_s, layout=layout, strict=True)
    assert rep["missing"] == [] and len(rep["loaded"]) == 2 * (2 * 8 + 2 * 2)
    want, got = factors(src_d, src_s), factors(dst_d, dst_s)
    for k in want:
        assert torch.equal(want[k][0], got[k][0]) and torch.equal(want[k][1], got[k][1]), k
    # the double block's stacked q/k/v factors are views that moved with the
    # load, and the cached transposes were refreshed
    for b in dst_d:
        for s in fb.STREAMS:
            stack_a = torch.cat([b.w[s].lora_a[t] for t in fb.QKV])
            assert torch.equal(b._a_qkv[s], stack_a)
            assert torch.equal(b._a_qkv_t[s], stack_a.t())
            for t in fb.QKV:
                assert torch.equal(b._b_t[s][t], b.w[s].lora_b[t].t())
    # the single block's GEMM operands carry the loaded factors
    for b in dst_s:
        assert torch.equal(b.w_in_ext[:, C:C + R], b.w.lora_b["to_in"])
        assert torch.equal(b.w_out_ext[C:C + R], b.w.lora_a["to_out"])


def test_foundry_layout_key_names(tmp_path):
    d, s = stack(3)
    keys = set(lf.lora_state_dict(d, s, layout="foundry"))
    assert "weights/double.0.img.to_q.lora_a" in keys and "weights/double.1.txt.to_out.lora_b" in keys
    assert "weights/single.1.to_in.lora_b" in keys and "weights/single.0.to_out.lora_a" in keys
    assert len(keys) == 2 * (2 * 8 + 2 * 2)


def test_image_stream_file_leaves_text_factors(tmp_path):
    """The klein trainer adapts only the double blocks' image stream: such a
    file loads into blocks that also adapt the text stream, which keeps its
    factors; strict=True refuses it."""
    src_d, src_s = stack(30)
    path = str(tmp_path / "img_only.safetensors")
    lf.save_lora(path, src_d, src_s, streams=("img",))
    dst_d, dst_s = stack(40)
    before = factors(dst_d, dst_s)
    rep = lf.load_lora(path, dst_d, dst_s)
    assert len(rep["missing"]) == 2 * 8 and all("add_" in k or "to_add_out" in k for k in rep["missing"])
    after = factors(dst_d, dst_s)
    for k in before:
        if k[0] == "d" and k[2] == "txt":
            assert torch.equal(before[k][0], after[k][0]) and torch.equal(before[k][1], after[k][1])
        else:
            want = factors(src_d, src_s)[k]
            assert torch.equal(want[0], after[k][0]) and torch.equal(want[1], after[k][1])
    with pytest.raises(ValueError, match="missing"):
        lf.load_lora(path, *stack(41), strict=True)


def test_errors_and_scale_adoption(tmp_path):
    src_d, src_s = stack(50, scale=2.0)  # alpha = 2 * rank
    path = str(tmp_path / "scaled.safetensors")
    meta = lf.save_lora(path, src_d, src_s)
    assert json.loads(meta["lora_adapter_metadata"])["transformer.lora_alpha"] == 2.0 * R
    dst_d, dst_s = stack(60, scale=1.0)
    rep = lf.load_lora(path, dst_d, dst_s)
    assert rep["scale"] == 2.0 and all(b.lora_scale == 2.0 for b in dst_d + dst_s)
    # a key with no slot (a third double block) and a shape mismatch are errors
    with pytest.raises(ValueError, match="no LoRA slot"):
        lf.load_lora(path, dst_d[:1], dst_s)
    single_path = str(tmp_path / "singles.safetensors")
    lf.save_lora(single_path, [], src_s)
    wide = fb.random_single_block(2 * C, H, 4, 2, 4, rank=R, device="cpu", seed=70)
    with pytest.raises(ValueError, match="shape"):
        lf.load_lora(single_path, [], [wide, wide])
    with pytest.raises(ValueError, match="layout"):
        lf.lora_state_dict(dst_d, dst_s, layout="kohya")
