"""fa_gemm_bf16 (this build's bf16 GEMM with fused epilogues) on the GPU.

Plain product: against the exact product of the bf16 inputs (f64 on the
host) rounded to bf16 -- f32 accumulation over K moves a result by far less
than a bf16 ulp, so only results within an ulp of a rounding boundary may
differ, by one ulp -- and against torch.mm at the c4 MLP shape.  The GELU and
GELU-gradient epilogues against the standalone kernels they replace
(fa_gelu_fwd on the plain product, fa_gelu_bwd on it), bit for bit: the same
formula applied to the same rounded product."""
import numpy as np
import pytest
import torch

from foundry_attn import block as fb

pytestmark = pytest.mark.gpu


def _rand(shape, std, g):
    return (std * torch.randn(shape, generator=g)).to(torch.bfloat16).to("cuda")


@pytest.mark.parametrize("M,N,K", [(256, 256, 64), (512, 768, 192), (768, 512, 3072)])
def test_gemm_matches_exact_product(M, N, K):
    g = torch.Generator().manual_seed(M + N + K)
    a, w = _rand((M, K), 1.0, g), _rand((N, K), 0.05, g)
    c = fb.gemm(a, w)
    torch.cuda.synchronize()
    an, wn = a.double().cpu().numpy(), w.double().cpu().numpy()
    exact = an @ wn.T
    want = torch.from_numpy(exact).to(torch.bfloat16).float().numpy()
    got = c.float().cpu().numpy()
    # one bf16 ulp of the result (at most |x| 2^-7) plus the f32 summation
    # error bound K 2^-24 sum_k |a_k w_k|, which dominates near cancellation
    bound = np.abs(want) * 2.0 ** -7 + K * 2.0 ** -24 * (np.abs(an) @ np.abs(wn).T)
    diff = np.abs(got - want)
    frac = float(np.mean(got != want))
    print(f"  M{M} N{N} K{K}: differing {frac:.2e}, max diff / bound {float(np.max(diff / bound)):.2f}", flush=True)
    assert np.all(diff <= bound)
    assert frac < 1e-2


def test_gemm_c4_mlp_shape_matches_torch():
    """W1 of the c4 block: [4096, 3072] x [12288, 3072]^T."""
    g = torch.Generator().manual_seed(4)
    a, w = _rand((4096, 3072), 1.0, g), _rand((12288, 3072), 0.02, g)
    c = fb.gemm(a, w)
    ref = torch.mm(a, w.t())
    torch.cuda.synchronize()
    d = (c.float() - ref.float()).abs()
    rel = float((c.float() - ref.float()).norm() / ref.float().norm())
    print(f"  vs torch.mm: rel_l2 {rel:.2e}, max {float(d.max()):.2e}, identical {bool(torch.equal(c, ref))}",
          flush=True)
    assert rel <= 1e-3 and float(d.max()) <= 2.0 ** -7 * float(ref.float().abs().max())


@pytest.mark.parametrize("M,N,K", [(512, 768, 192), (4096, 12288, 3072)])
def test_gelu_epilogues_match_separate_kernels(M, N, K):
    g = torch.Generator().manual_seed(7)
    x, w1 = _rand((M, K), 1.0, g), _rand((N, K), 0.05, g)
    pre, act = fb.gemm(x, w1, "gelu")
    plain = fb.gemm(x, w1)
    act_sep = fb.gelu(plain)
    # the GELU gradient after W2's dX product: dy [M, K'] x W2g_t [N, K']^T
    dy, w2t = _rand((M, 256), 1.0, g), _rand((N, 256), 0.05, g)
    dpre = fb.gemm(dy, w2t, "dgelu", pre=pre)
    dact = fb.gemm(dy, w2t)
    dpre_sep = fb.gelu_bwd(dact, pre)
    torch.cuda.synchronize()
    assert torch.equal(pre, plain)
    assert torch.equal(act, act_sep)
    assert torch.equal(dpre, dpre_sep)


def test_gemm_strided_views():
    """Operands and output as column slices of wider buffers (row strides
    larger than the extents)."""
    g = torch.Generator().manual_seed(9)
    abuf, wbuf = _rand((512, 448), 1.0, g), _rand((256, 320), 0.05, g)
    a, w = abuf[:, 64:64 + 256], wbuf[:, :256]
    out = torch.full((512, 512), float("nan"), dtype=torch.bfloat16, device="cuda")
    c = fb.gemm(a, w, out=out[:, 128:384])
    torch.cuda.synchronize()
    assert torch.equal(c, fb.gemm(a.contiguous(), w.contiguous()))
    assert torch.isnan(out[:, :128].float()).all() and torch.isnan(out[:, 384:].float()).all()
