"""GPU parity of the HIP attention path against the CPU oracle.

Every compute call goes through libfoundry_attn.so (the C ABI) on cuda:0.
Gates (from the north star): bf16 max-abs <= 2e-2 and rel-L2 <= 1e-2 for O,
dQ, dK, dV; f32 rel-L2 <= 1e-4.  LSE is f32 in both paths: max-abs <= 2e-3
for bf16 inputs, rel 1e-5 for f32.  Config-size cases compare the oracle on a
subset of heads (heads are independent) and check size-independent
properties on all heads.  The config-size cases (c2, c3, c5) compare every
(batch, head) pair with the oracle: an indexing mistake tied to the XCD
remap or to a tile's position in the grid would show on some heads only.
"""
import numpy as np
import pytest
import torch

import oracle
from foundry_attn import attention, attn_bwd, attn_fwd, attn_workspace_bytes, AttnBwd
from foundry_attn.configs import C1, C2, C3, C5
from helpers import (BF16_MAX_ABS, BF16_REL_L2, F32_REL_L2, attn_inputs, load_golden, max_abs,
                     rel_l2)

pytestmark = pytest.mark.gpu


def dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device="cuda", dtype=dtype)


def host(t):
    return t.float().cpu().numpy()


def run_gpu(q, k, v, do, dtype, scale, keep=None):
    tq, tk, tv, tdo = (dev(a, dtype) for a in (q, k, v, do))
    tkeep = None if keep is None else dev(keep, torch.uint8)
    o, lse = attn_fwd(tq, tk, tv, scale, tkeep)
    dq, dk, dv = attn_bwd(tq, tk, tv, o, tdo, lse, scale, tkeep)
    torch.cuda.synchronize()
    return {n: host(t) for n, t in dict(o=o, lse=lse, dq=dq, dk=dk, dv=dv).items()}


def _zero_reference(want) -> bool:
    # e.g. dQ at S = 1 is exactly zero: rel-L2 is undefined there, so the
    # check falls back to an absolute bound
    return float(np.abs(want).max(initial=0.0)) < 1e-6


def check_bf16(name, got, want):
    ma, rl = max_abs(got, want), rel_l2(got, want)
    print(f"  {name}: max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
    if _zero_reference(want):
        assert ma <= 1e-5, (name, ma)
        return
    assert ma <= BF16_MAX_ABS and rl <= BF16_REL_L2, (name, ma, rl)


def check_f32(name, got, want):
    rl = rel_l2(got, want)
    print(f"  {name}: rel_l2={rl:.3e}", flush=True)
    if _zero_reference(want):
        assert max_abs(got, want) <= 1e-5, (name, max_abs(got, want))
        return
    assert rl <= F32_REL_L2, (name, rl)


def compare(g, q, k, v, do, scale, keep, bf16, heads):
    h0, h1 = heads
    o, lse = oracle.attn_fwd(q, k, v, scale=scale, key_keep=keep, bf16=bf16, heads=heads)
    dq, dk, dv = oracle.attn_bwd(q, k, v, do, scale=scale, key_keep=keep, bf16=bf16, heads=heads)
    sl = (slice(None), slice(None), slice(h0, h1))
    chk = check_bf16 if bf16 else check_f32
    for name, got, want in (("O", g["o"][sl], o[sl]), ("dQ", g["dq"][sl], dq[sl]),
                            ("dK", g["dk"][sl], dk[sl]), ("dV", g["dv"][sl], dv[sl])):
        chk(name, got, want)
    gl, wl = g["lse"][:, h0:h1], lse[:, h0:h1]
    fin = np.isfinite(wl)
    assert np.array_equal(np.isfinite(gl), fin)
    if bf16:
        assert max_abs(gl[fin], wl[fin]) <= 2e-3
    else:
        np.testing.assert_allclose(gl[fin], wl[fin], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("tag", ["fp32", "bf16"])
@pytest.mark.parametrize("blk", ["double", "single"])
def test_reference_fixture_replay(tag, blk):
    """The reference's own attention test (attn_backward.rs:203-233): fixture
    q/k/v (S=24, H=2, D=128) through fwd, fixture dO through bwd."""
    f = load_golden(tag)
    dt = torch.float32 if tag == "fp32" else torch.bfloat16
    q, k, v, out = (f[f"attn_in/{blk}.{n}"] for n in ("q", "k", "v", "attn"))
    do = f[f"grad/attn/{blk}.out"]
    g = run_gpu(q[None], k[None], v[None], do[None], dt, 1 / np.sqrt(128))
    want = dict(o=out, dq=f[f"grad/attn/{blk}.q"], dk=f[f"grad/attn/{blk}.k"],
                dv=f[f"grad/attn/{blk}.v"])
    for n, w in want.items():
        rl = rel_l2(g[n][0], w)
        print(f"  {tag} {blk} {n}: rel_l2={rl:.3e}", flush=True)
        # the fixture dO is ~1e-4 in magnitude, so rel-L2 is the binding check
        assert rl <= (F32_REL_L2 if tag == "fp32" else BF16_REL_L2), (n, rl)


def test_c1_f32_parity():
    c = C1
    x = attn_inputs(c)
    g = run_gpu(x["q"], x["k"], x["v"], x["do"], torch.float32, c.scale)
    compare(g, x["q"], x["k"], x["v"], x["do"], c.scale, None, False, (0, c.heads))


@pytest.fixture(scope="module")
def c2_run():
    x = attn_inputs(C2)
    g = run_gpu(x["q"], x["k"], x["v"], x["do"], torch.bfloat16, C2.scale)
    return x, g


def test_c2_bf16_parity(c2_run):
    """All 24 heads of c2 against the oracle."""
    x, g = c2_run
    compare(g, x["q"], x["k"], x["v"], x["do"], C2.scale, None, True, (0, C2.heads))


def test_c2_full_size_properties(c2_run):
    """Size-independent checks on all 24 heads at S=4608."""
    x, g = c2_run
    # sum_j dK_j = 0 per (b, h): softmax rows sum to one
    sk = np.abs(g["dk"].astype(np.float64).sum(1))
    assert np.all(sk <= 1e-3 * np.abs(g["dk"]).sum(1) + 1e-6)
    # sum_j dV_j = sum_i dO_i per (b, h)
    sv = g["dv"].astype(np.float64).sum(1)
    so = x["do"].astype(np.float64).sum(1)
    assert rel_l2(sv, so) <= 1e-2
    # LSE >= max scaled score of the row >= LSE - ln(S): LSE = m + ln(sum_j
    # exp(s_j - m)) with the sum between 1 (the max term) and S.  The scores
    # are recomputed here in f64 from the bf16 inputs; 1e-3 covers the
    # kernel's f32 rounding of LSE (|LSE| < 40 here).
    assert np.all(np.isfinite(g["lse"]))
    S = C2.seq
    for h in range(C2.heads):
        qh = x["q"][0, :, h, :].astype(np.float64)
        kh = x["k"][0, :, h, :].astype(np.float64)
        m = (qh @ kh.T).max(axis=1) * C2.scale
        lse = g["lse"][0, h].astype(np.float64)
        assert np.all(lse >= m - 1e-3), (h, float((m - lse).max()))
        assert np.all(m >= lse - np.log(S) - 1e-3), (h, float((lse - np.log(S) - m).max()))
    assert np.all(np.isfinite(g["o"])) and np.all(np.isfinite(g["dq"]))


def test_c3_batched_parity():
    c = C3
    x = attn_inputs(c)
    g = run_gpu(x["q"], x["k"], x["v"], x["do"], torch.bfloat16, c.scale)
    compare(g, x["q"], x["k"], x["v"], x["do"], c.scale, None, True, (0, c.heads))


def test_c5_masked_parity():
    c = C5
    x = attn_inputs(c)
    g = run_gpu(x["q"], x["k"], x["v"], x["do"], torch.bfloat16, c.scale, x["keep"])
    compare(g, x["q"], x["k"], x["v"], x["do"], c.scale, x["keep"], True, (0, c.heads))
    # padded keys receive no gradient; padded query rows (dO = 0) give dQ = 0
    pad = x["keep"] == 0
    for b in range(c.batch):
        assert not np.any(g["dk"][b][pad[b]]) and not np.any(g["dv"][b][pad[b]])
        assert not np.any(g["dq"][b][pad[b]])


@pytest.mark.parametrize("S", [1, 2, 63, 65, 129, 200])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_ragged_shapes(S, D, dtype):
    rng = np.random.default_rng(S * 7 + D)
    bf = dtype == "bf16"
    mk = lambda: (oracle.bf16_round if bf else np.float32)(
        rng.standard_normal((2, S, 3, D)).astype(np.float32))
    q, k, v, do = mk(), mk(), mk(), mk()
    scale = 0.9 / np.sqrt(D)
    keep = (rng.random((2, S)) > 0.25).astype(np.uint8)
    keep[:, 0] = 1
    g = run_gpu(q, k, v, do, torch.bfloat16 if bf else torch.float32, scale, keep)
    compare(g, q, k, v, do, scale, keep, bf, (0, 3))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fully_masked_batch_item(dtype):
    rng = np.random.default_rng(1)
    q, k, v, do = (rng.standard_normal((2, 80, 2, 64)).astype(np.float32) for _ in range(4))
    if dtype == torch.bfloat16:
        q, k, v, do = (oracle.bf16_round(a) for a in (q, k, v, do))
    keep = np.ones((2, 80), np.uint8)
    keep[1] = 0
    g = run_gpu(q, k, v, do, dtype, 0.125, keep)
    assert np.all(g["o"][1] == 0) and np.all(np.isneginf(g["lse"][1]))
    assert not np.any(g["dq"][1]) and not np.any(g["dk"][1]) and not np.any(g["dv"][1])
    compare(g, q, k, v, do, 0.125, keep, dtype == torch.bfloat16, (0, 2))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("H", [2, 6, 8], ids=["split", "four_wave", "eight_wave"])
def test_dead_key_blocks_are_skipped(H, D):
    """Masks whose excluded keys fill whole key blocks, which the kernels do
    not stream (forward: 64-key blocks; dQ: 128-key groups; dK/dV: a
    workgroup whose keys are all excluded).  B4 S3000 (47 forward blocks, so
    the live-block words cross a 32-block boundary): a dead prefix (first
    live block is block 10), a dead suffix (the last 31 blocks), every third
    64-key block live, and one kept key (the last).  H picks the grid: 2 the
    range-split kernels, 6 the 4-wave and 8 the 8-wave ones."""
    from foundry_attn import attn_workspace_bytes
    B, S = 4, 3000
    rng = np.random.default_rng(H * 100 + D)
    mk = lambda: oracle.bf16_round(rng.standard_normal((B, S, H, D)).astype(np.float32))
    q, k, v, do = mk(), mk(), mk(), mk()
    keep = np.ones((B, S), np.uint8)
    keep[0, :700] = 0
    keep[1, 1000:] = 0
    keep[2] = ((np.arange(S) // 64) % 3 == 0).astype(np.uint8)
    keep[3] = 0
    keep[3, S - 1] = 1
    fwd_ws = attn_workspace_bytes(torch.empty(B, S, H, D, dtype=torch.bfloat16, device="cuda"))[0]
    assert (fwd_ws > 0) == (H == 2), "split policy changed for this case"
    scale = D ** -0.5
    g = run_gpu(q, k, v, do, torch.bfloat16, scale, keep)
    compare(g, q, k, v, do, scale, keep, True, (0, 2))
    pad = keep == 0
    for b in range(B):
        assert not np.any(g["dk"][b][pad[b]]) and not np.any(g["dv"][b][pad[b]]), b
    assert np.all(np.isfinite(g["o"])) and np.all(np.isfinite(g["lse"]))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("masked", [False, True])
def test_wide_tiles_partial_last_tile(D, masked):
    """B=1, H=40, S=1400 runs the 8-wave (256-row) forward and dK/dV kernels
    (and dQ at D = 128): 240 workgroups fill most of the chip, so the
    workgroup-shape rule picks them, and 1400 = 5*256 + 120 leaves a partial
    last tile of queries and of keys.  The backward then runs its three
    launches in order.  Checked against the oracle on three heads."""
    rng = np.random.default_rng(40 + D + masked)
    B, S, H = 1, 1400, 40
    q, k, v, do = (oracle.bf16_round(rng.standard_normal((B, S, H, D)).astype(np.float32)) for _ in range(4))
    keep = None
    if masked:
        keep = (rng.random((B, S)) > 0.2).astype(np.uint8)
        keep[:, :8] = 1
    g = run_gpu(q, k, v, do, torch.bfloat16, D ** -0.5, keep)
    compare(g, q, k, v, do, D ** -0.5, keep, True, (0, 2))
    compare(g, q, k, v, do, D ** -0.5, keep, True, (39, 40))


@pytest.mark.parametrize("shape", [(2, 2), (1, 44)], ids=["4wave", "8wave"])
@pytest.mark.parametrize("case", ["growing", "overflow", "masked_prefix"])
def test_softmax_reference_moves(case, shape):
    """Scores that make the bf16 forward move its lazy exp2 reference:
    - growing: key scales rise along the sequence, so later blocks' P would
      exceed the stale reference by many orders of magnitude;
    - overflow: the same with logits of magnitude ~200, so P against a stale
      reference is inf and must be caught;
    - masked_prefix: rows whose first key blocks are all masked have no
      reference until a kept key appears, and every kept score is below -99
      (P against a zero reference would underflow to 0).
    S = 640 with B x H = 2 x 2 runs the 4-wave kernels, 1 x 44 the 8-wave
    ones (132 workgroups), both with a partial last tile.
    Near one-hot rows give |O| up to ~4.5, where one bf16 ulp (2^-5) exceeds
    the 2e-2 max-abs gate: O is held to rel-L2 <= 1e-2 and, element-wise, to
    max(2e-2, one bf16 ulp of the oracle's value).  The backward (unchanged
    kernels fed this LSE) is held to rel-L2, as its magnitudes scale with the
    keys.  Two heads are compared."""
    rng = np.random.default_rng({"growing": 31, "overflow": 32, "masked_prefix": 33}[case])
    (B, H), S, D = shape, 640, 128
    q, k, v, do = (rng.standard_normal((B, S, H, D)).astype(np.float32) for _ in range(4))
    scale, keep = D ** -0.5, None
    if case in ("growing", "overflow"):
        k *= (1.0 + np.arange(S, dtype=np.float32) / 16.0)[None, :, None, None]
        if case == "overflow":
            q *= 3.0
    else:
        q, k, scale = np.abs(q), -np.abs(k), 24.0 * D ** -0.5
        keep = np.ones((B, S), np.uint8)
        keep[0, :320] = 0
        if B > 1:
            keep[1, :130] = 0
    q, k, v, do = (oracle.bf16_round(a) for a in (q, k, v, do))
    g = run_gpu(q, k, v, do, torch.bfloat16, scale, keep)
    hs = (0, 2)
    sl = (slice(None), slice(None), slice(*hs))
    o, lse = oracle.attn_fwd(q, k, v, scale=scale, key_keep=keep, bf16=True, heads=hs)
    o, go = o[sl], g["o"][sl]
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(o), 2.0 ** -126))) - 7)
    err = np.abs(go.astype(np.float64) - o)
    print(f"  O: max_abs={err.max():.3e} max_ulps={(err / ulp).max():.2f} rel_l2={rel_l2(go, o):.3e}",
          flush=True)
    assert np.all(err <= np.maximum(BF16_MAX_ABS, ulp)) and rel_l2(go, o) <= BF16_REL_L2
    gl, wl = g["lse"][:, hs[0]:hs[1]], lse[:, hs[0]:hs[1]]
    assert max_abs(gl, wl) <= 2e-3 * max(1.0, float(np.abs(wl).max()) / 64.0)
    dq, dk, dv = oracle.attn_bwd(q, k, v, do, scale=scale, key_keep=keep, bf16=True, heads=hs)
    for name, got, want in (("dQ", g["dq"], dq), ("dK", g["dk"], dk), ("dV", g["dv"], dv)):
        rl = rel_l2(got[sl], want[sl])
        print(f"  {name}: rel_l2={rl:.3e}", flush=True)
        assert rl <= BF16_REL_L2, (name, rl)


def test_bitwise_repeatable():
    """The reference's determinism gate (docs/TESTING.md:19) as a kernel
    property: three runs give identical bits."""
    x = attn_inputs(C3)
    runs = [run_gpu(x["q"], x["k"], x["v"], x["do"], torch.bfloat16, C3.scale) for _ in range(3)]
    for r in runs[1:]:
        for n in ("o", "lse", "dq", "dk", "dv"):
            assert np.array_equal(r[n], runs[0][n], equal_nan=True), n


def test_strided_views_match_contiguous():
    """q/k/v as views into one fused [B, S, 3, H, D] buffer (Candle Layout
    strides pass straight through the ABI)."""
    torch.manual_seed(0)
    qkv = torch.randn(2, 300, 3, 4, 128, device="cuda").to(torch.bfloat16)
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    o1, l1 = attn_fwd(q, k, v)
    o2, l2 = attn_fwd(q.contiguous(), k.contiguous(), v.contiguous())
    do = torch.randn_like(o1)
    g1 = attn_bwd(q, k, v, o1, do, l1)
    g2 = attn_bwd(q.contiguous(), k.contiguous(), v.contiguous(), o2, do, l2)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def test_custom_op_surface_and_autograd():
    """AttnBwd keeps the reference's CustomOp3 surface: name(), fwd, and
    bwd(q, k, v, res, grad_res); the autograd wrapper gives the same grads."""
    op = AttnBwd()
    assert op.name() == "foundry-attn-bwd"
    torch.manual_seed(1)
    q, k, v = (torch.randn(96, 2, 128, device="cuda").to(torch.bfloat16) for _ in range(3))
    res = op.fwd(q, k, v)
    gres = torch.randn_like(res)
    dq, dk, dv = op.bwd(q, k, v, res, gres)
    # a fresh instance has no saved LSE and regenerates it: same bits
    dq2, dk2, dv2 = AttnBwd().bwd(q, k, v, res, gres)
    assert torch.equal(dq, dq2) and torch.equal(dk, dk2) and torch.equal(dv, dv2)
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = attention(qa, ka, va)
    out.backward(gres)
    torch.cuda.synchronize()
    assert torch.equal(out, res)
    assert torch.equal(qa.grad, dq) and torch.equal(ka.grad, dk) and torch.equal(va.grad, dv)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_custom_op_host_tensors_take_the_cpu_fwd_route(dtype):
    """Host (CPU) tensors through AttnBwd -- the reference's cpu_fwd path
    (lib.rs:158-187) -- are staged to the GPU, run by the same kernels and
    returned as host tensors: bit-identical to the device call (the reference
    f32 CPU case c1's shape)."""
    torch.manual_seed(2)
    q, k, v, g = (torch.randn(256, 4, 64).to(dtype) for _ in range(4))
    op = AttnBwd()
    res = op.fwd(q, k, v)
    assert res.device.type == "cpu" and res.dtype == dtype
    grads = op.bwd(q, k, v, res, g)
    assert all(t.device.type == "cpu" for t in grads)
    dev_op = AttnBwd()
    dres = dev_op.fwd(q.cuda(), k.cuda(), v.cuda())
    dgrads = dev_op.bwd(q.cuda(), k.cuda(), v.cuda(), dres, g.cuda())
    torch.cuda.synchronize()
    assert torch.equal(res, dres.cpu())
    for a, b in zip(grads, dgrads):
        assert torch.equal(a, b.cpu())
    # a fresh instance regenerates the LSE from the host inputs: same bits
    fresh = AttnBwd().bwd(q, k, v, res, g)
    for a, b in zip(grads, fresh):
        assert torch.equal(a, b)


def _op_run(q, k, v, do, route, fresh):
    """q.apply_op3(k, v, AttnBwd) then the op's backward seeded with do, as
    the reference's acceptance run drives it (attn_backward.rs:203-233).
    route "host" hands host tensors to the op (the cpu_fwd slot), "device"
    device tensors (the cuda_fwd slot).  fresh: the backward runs on a new
    op instance, so it regenerates the LSE instead of reusing the forward's."""
    if route == "device":
        q, k, v, do = (t.cuda() for t in (q, k, v, do))
    op = AttnBwd()
    res = op.fwd(q, k, v)
    grads = (AttnBwd() if fresh else op).bwd(q, k, v, res, do)
    torch.cuda.synchronize()
    for t in (res,) + tuple(grads):
        assert t.device.type == ("cuda" if route == "device" else "cpu") and t.dtype == q.dtype
    return host(res), tuple(host(t) for t in grads)


@pytest.mark.parametrize("fresh", [False, True], ids=["saved_lse", "regenerated_lse"])
@pytest.mark.parametrize("route", ["device", "host"])
@pytest.mark.parametrize("tag", ["fp32", "bf16"])
@pytest.mark.parametrize("blk", ["double", "single"])
def test_op_surface_fixture_replay(blk, tag, route, fresh):
    """The reference fixture through the AttnBwd op surface on both routes:
    O against the fixture's attn_in/*.attn and the oracle, dQ/dK/dV against
    grad/attn/* and the oracle (rel-L2, the binding check at the fixture's
    tiny dO; plus max-abs against the oracle)."""
    f = load_golden(tag)
    dt = torch.float32 if tag == "fp32" else torch.bfloat16
    arrs = [f[f"attn_in/{blk}.{n}"] for n in ("q", "k", "v")] + [f[f"grad/attn/{blk}.out"]]
    q, k, v, do = (torch.from_numpy(a).to(dt) for a in arrs)
    o, (dq, dk, dv) = _op_run(q, k, v, do, route, fresh)
    bf = tag == "bf16"
    wo, _ = oracle.attn_fwd(*(a[None] for a in arrs[:3]), bf16=bf)
    wq, wk, wv = oracle.attn_bwd(*(a[None] for a in arrs), bf16=bf)
    gate = BF16_REL_L2 if bf else F32_REL_L2
    for n, got, fix, orc in (("O", o, f[f"attn_in/{blk}.attn"], wo[0]), ("dQ", dq, f[f"grad/attn/{blk}.q"], wq[0]),
                             ("dK", dk, f[f"grad/attn/{blk}.k"], wk[0]), ("dV", dv, f[f"grad/attn/{blk}.v"], wv[0])):
        rf, ro = rel_l2(got, fix), rel_l2(got, orc)
        print(f"  {n}: rel_l2 fixture={rf:.3e} oracle={ro:.3e}", flush=True)
        assert rf <= gate and ro <= gate, (n, rf, ro)
        if bf:
            assert max_abs(got, orc) <= BF16_MAX_ABS, n


@pytest.mark.parametrize("fresh", [False, True], ids=["saved_lse", "regenerated_lse"])
@pytest.mark.parametrize("route", ["device", "host"])
def test_op_surface_c1_against_oracle(route, fresh):
    """Config c1 (f32, S=256 = 64 txt + 192 img, H=4, D=64, the reference's
    CPU-runnable case) through AttnBwd on both routes, against the oracle at
    the f32 gate; the op's default scale is 1/sqrt(D) = 1/8."""
    x = attn_inputs(C1)
    q, k, v, do = (torch.from_numpy(np.ascontiguousarray(x[n][0])) for n in ("q", "k", "v", "do"))
    o, grads = _op_run(q, k, v, do, route, fresh)
    wo, _ = oracle.attn_fwd(x["q"], x["k"], x["v"], scale=C1.scale)
    wgrads = oracle.attn_bwd(x["q"], x["k"], x["v"], x["do"], scale=C1.scale)
    check_f32("O", o, wo[0])
    for n, got, want in zip(("dQ", "dK", "dV"), grads, wgrads):
        check_f32(n, got, want[0])


def test_attn_bwd_noncontiguous_lse():
    """A strided LSE view gives the bits of its contiguous copy (the host
    layer's copy stays alive until the launch is enqueued, so the workspace
    cannot take its memory)."""
    torch.manual_seed(5)
    q, k, v, do = (torch.randn(1, 700, 3, 128, device="cuda").to(torch.bfloat16) for _ in range(4))
    o, lse = attn_fwd(q, k, v)
    wide = torch.full((1, 3, 2 * 700), float("nan"), device="cuda")
    wide[..., ::2] = lse
    lse_view = wide[..., ::2]
    assert not lse_view.is_contiguous()
    for _ in range(3):
        want = attn_bwd(q, k, v, o, do, lse)
        got = attn_bwd(q, k, v, o, do, lse_view)
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b)


@pytest.mark.parametrize("B,S,H,D", [(2, 700, 3, 128), (1, 1100, 44, 128), (1, 1100, 44, 64),
                                     (1, 2048, 2, 128), (1, 1400, 2, 64)],
                         ids=["4wave", "8wave", "8wave_d64", "split", "split_d64"])
def test_backward_phases_match_single_call(B, S, H, D):
    """fa_attn_bwd_phase: pre-pass, dK/dV and dQ issued separately (one
    stream, then dK/dV and dQ on two streams) give the one-call bits.  With
    8-wave kernels the one call (full workspace) is the pre-pass, dK/dV
    storing dS, then dQ from it; its phases on two streams run dQ after dK/dV.
    With the minimum workspace dQ recomputes S and dP (and, in one call, also
    does the pre-pass for its queries, in the pre-pass's order), so dK/dV and
    dQ may run side by side -- with the same bits.  A split call adds the
    reduce, and its phases reduce their own partials."""
    from foundry_attn import _abi
    from foundry_attn.ops import attn_bwd_workspace_bytes
    torch.manual_seed(3)
    q, k, v, do = (torch.randn(B, S, H, D, device="cuda").to(torch.bfloat16) for _ in range(4))
    keep = torch.ones(B, S, dtype=torch.uint8, device="cuda")
    keep[0, 100:300] = 0
    o, lse = attn_fwd(q, k, v, key_keep=keep)
    ref = attn_bwd(q, k, v, o, do, lse, key_keep=keep)
    seq = attn_bwd(q, k, v, o, do, lse, key_keep=keep,
                   phases=[(_abi.FA_BWD_PREPASS, None), (_abi.FA_BWD_DKDV, None),
                           (_abi.FA_BWD_DQ, None)])
    cur = torch.cuda.current_stream()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()  # default priority
    full = torch.empty(attn_workspace_bytes(q)[1], dtype=torch.uint8, device="cuda")
    out_f = tuple(torch.empty_like(q) for _ in range(3))
    attn_bwd(q, k, v, o, do, lse, key_keep=keep, workspace=full, out=out_f,
             phases=[(_abi.FA_BWD_PREPASS, None)])
    s1.wait_stream(cur)
    attn_bwd(q, k, v, o, do, lse, key_keep=keep, workspace=full, out=out_f,
             phases=[(_abi.FA_BWD_DKDV, s1)])
    s2.wait_stream(s1)
    attn_bwd(q, k, v, o, do, lse, key_keep=keep, workspace=full, out=out_f,
             phases=[(_abi.FA_BWD_DQ, s2)])
    cur.wait_stream(s2)
    ws = torch.empty(attn_bwd_workspace_bytes(B, S, H, D, minimum=True), dtype=torch.uint8, device="cuda")
    out = tuple(torch.empty_like(q) for _ in range(3))
    attn_bwd(q, k, v, o, do, lse, key_keep=keep, workspace=ws, out=out,
             phases=[(_abi.FA_BWD_PREPASS, None)])
    s1.wait_stream(cur)
    s2.wait_stream(cur)
    attn_bwd(q, k, v, o, do, lse, key_keep=keep, workspace=ws, out=out,
             phases=[(_abi.FA_BWD_DKDV, s1)])
    attn_bwd(q, k, v, o, do, lse, key_keep=keep, workspace=ws, out=out,
             phases=[(_abi.FA_BWD_DQ, s2)])
    cur.wait_stream(s1)
    cur.wait_stream(s2)
    torch.cuda.synchronize()
    for a, b, c, f in zip(ref, seq, out, out_f):
        assert torch.equal(a, b) and torch.equal(a, c) and torch.equal(a, f)


@pytest.mark.parametrize("B,S,H,D,masked", [(1, 1100, 44, 128, False), (1, 1037, 44, 128, True),
                                            (1, 1100, 44, 64, True), (1, 4608, 24, 128, False)],
                         ids=["8wave", "ragged_masked", "d64_masked", "c2"])
def test_stored_ds_backward_matches_recompute(B, S, H, D, masked):
    """With the full workspace the 8-wave backward stores dS from dK/dV and
    forms dQ = dS K from it; with the minimum one dQ recomputes S and dP.
    Both multiply the same bf16 dS by K in the same key order, so the
    gradients are bit-identical -- including a key count that is not a
    multiple of 32 or 64 (the last key tile and query block partly past S),
    excluded keys (stored as zero dS), fully masked rows, and D = 64."""
    from foundry_attn.ops import attn_bwd_workspace_bytes
    torch.manual_seed(5)
    q, k, v, do = (torch.randn(B, S, H, D, device="cuda").to(torch.bfloat16) for _ in range(4))
    keep = None
    if masked:
        keep = torch.ones(B, S, dtype=torch.uint8, device="cuda")
        keep[0, 37:301] = 0
        keep[-1, S - 50:] = 0
    o, lse = attn_fwd(q, k, v, key_keep=keep)
    full_b, least_b = attn_bwd_workspace_bytes(B, S, H, D), attn_bwd_workspace_bytes(B, S, H, D, minimum=True)
    assert full_b > least_b
    res = []
    for nbytes in (least_b, full_b, full_b):
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        out = tuple(torch.empty_like(q) for _ in range(3))
        attn_bwd(q, k, v, o, do, lse, key_keep=keep, workspace=ws, out=out)
        torch.cuda.synchronize()
        res.append(out)
        del ws
    for name, a, b, c in zip(("dq", "dk", "dv"), *res):
        assert torch.equal(a, b), name
        assert torch.equal(b, c), name  # repeatable


@pytest.mark.parametrize("S,H", [(700, 4), (1100, 44), (1100, 4)], ids=["forked", "in_order", "split"])
def test_one_call_backward_is_ordered_on_the_caller_stream(S, H):
    """fa_attn_bwd runs dQ on a library side stream and joins it back (S =
    700, H = 4: the 4-wave kernels), runs its launches in order (H = 44: 220
    workgroups, 8-wave), or splits and reduces in order (S = 1100, H = 4: 20
    8-wave workgroups): either way, work queued on the caller's stream right
    after the call (a copy of dq, and a second call reusing the same
    workspace with other inputs) sees finished results."""
    torch.manual_seed(5)
    mk = lambda: torch.randn(1, S, H, 128, device="cuda").to(torch.bfloat16)
    q1, k1, v1, do1, q2, k2, v2, do2 = (mk() for _ in range(8))
    o1, l1 = attn_fwd(q1, k1, v1)
    o2, l2 = attn_fwd(q2, k2, v2)
    ref1 = attn_bwd(q1, k1, v1, o1, do1, l1)
    ref2 = attn_bwd(q2, k2, v2, o2, do2, l2)
    torch.cuda.synchronize()
    ws = torch.empty(attn_workspace_bytes(q1)[1], dtype=torch.uint8, device="cuda")
    out1 = tuple(torch.empty_like(q1) for _ in range(3))
    out2 = tuple(torch.empty_like(q1) for _ in range(3))
    s = torch.cuda.Stream()  # default priority
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        attn_bwd(q1, k1, v1, o1, do1, l1, workspace=ws, out=out1)
        snap = out1[0].clone()
        attn_bwd(q2, k2, v2, o2, do2, l2, workspace=ws, out=out2)
    torch.cuda.synchronize()
    assert torch.equal(snap, ref1[0])
    for a, b in zip(out1, ref1):
        assert torch.equal(a, b)
    for a, b in zip(out2, ref2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("S,H", [(900, 3), (900, 40), (2048, 2)], ids=["forked", "in_order", "split"])
def test_backward_from_two_host_threads(S, H):
    """Each host thread gets its own side stream and events (H = 3 forks dQ;
    H = 40, 160 workgroups of the 8-wave kernels, runs in order; S = 2048,
    H = 2 splits, each call with its own workspace): two threads calling
    fa_attn_fwd / fa_attn_bwd at once give the single-threaded bits."""
    import threading
    torch.manual_seed(6)
    cases = []
    for _ in range(2):
        q, k, v, do = (torch.randn(1, S, H, 128, device="cuda").to(torch.bfloat16) for _ in range(4))
        o, lse = attn_fwd(q, k, v)
        cases.append((q, k, v, o, do, lse))
    refs = [(c[3], c[5]) + tuple(attn_bwd(*c)) for c in cases]
    torch.cuda.synchronize()
    results, errors = {}, []

    def work(i):
        try:
            q, k, v, _, do, _ = cases[i]
            st = torch.cuda.Stream()
            st.wait_stream(torch.cuda.default_stream())
            with torch.cuda.stream(st):
                for _ in range(3):
                    o, lse = attn_fwd(q, k, v)
                    r = (o, lse) + tuple(attn_bwd(q, k, v, o, do, lse))
            st.synchronize()
            results[i] = r
        except Exception as e:  # surfaced below
            errors.append(e)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i in range(2):
        for a, b in zip(results[i], refs[i]):
            assert torch.equal(a, b), i
