"""Host-side argument checks of the PyTorch-facing layer (no GPU needed).

Every case below must be refused with FoundryAttnError before anything is
launched: the C ABI only sees pointers and leading dimensions, so a short
factor or a wrong-shaped output would otherwise become an out-of-bounds
device access.  The tensors are host tensors; each check fires before the
call would look for a device.
"""
import pytest
import torch

from foundry_attn import AttnBwd, FoundryAttnError, lora_down, lora_grad, lora_up

bf = torch.bfloat16


def _x(N=64, K=128, dtype=bf):
    return torch.zeros(N, K, dtype=dtype)


@pytest.mark.parametrize("case", ["a_short_k", "a_dtype", "a_1d", "x_col_stride", "x_dtype",
                                  "out_shape", "out_dtype", "out_col_stride"])
def test_lora_down_rejects(case):
    x, a, out = _x(), torch.zeros(16, 128, dtype=bf), torch.zeros(64, 16, dtype=bf)
    if case == "a_short_k":
        a = torch.zeros(16, 96, dtype=bf)
    elif case == "a_dtype":
        a = torch.zeros(16, 128, dtype=torch.float32)
    elif case == "a_1d":
        a = torch.zeros(128, dtype=bf)
    elif case == "x_col_stride":
        x = torch.zeros(128, 64, dtype=bf).t()
    elif case == "x_dtype":
        x = _x(dtype=torch.float32)
    elif case == "out_shape":
        out = torch.zeros(64, 8, dtype=bf)
    elif case == "out_dtype":
        out = torch.zeros(64, 16, dtype=torch.float32)
    else:
        out = torch.zeros(16, 64, dtype=bf).t()
    with pytest.raises(FoundryAttnError):
        lora_down(x, a, 1.0, out)


@pytest.mark.parametrize("case", ["b_short_m", "b_rank", "b_dtype", "u_shape", "y_col_stride", "y_dtype"])
def test_lora_up_rejects(case):
    u, b, y = torch.zeros(64, 16, dtype=bf), torch.zeros(128, 16, dtype=bf), _x()
    if case == "b_short_m":
        b = torch.zeros(96, 16, dtype=bf)
    elif case == "b_rank":
        b = torch.zeros(128, 8, dtype=bf)
    elif case == "b_dtype":
        b = torch.zeros(128, 16, dtype=torch.float32)
    elif case == "u_shape":
        u = torch.zeros(32, 16, dtype=bf)
    elif case == "y_col_stride":
        y = torch.zeros(128, 64, dtype=bf).t()
    else:
        y = _x(dtype=torch.float32)
    with pytest.raises(FoundryAttnError):
        lora_up(u, b, y, 1.0)


@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("case", ["out_shape", "out_dtype", "out_noncontig", "x_col_stride", "u_rows", "u_dtype"])
def test_lora_grad_rejects(case, transpose):
    u, x = torch.zeros(64, 16, dtype=bf), _x()
    shape = (128, 16) if transpose else (16, 128)
    out = torch.zeros(shape, dtype=torch.float32)
    if case == "out_shape":
        out = torch.zeros(shape[::-1], dtype=torch.float32)
    elif case == "out_dtype":
        out = torch.zeros(shape, dtype=bf)
    elif case == "out_noncontig":
        out = torch.zeros(shape[1], shape[0], dtype=torch.float32).t()
    elif case == "x_col_stride":
        x = torch.zeros(128, 64, dtype=bf).t()
    elif case == "u_rows":
        u = torch.zeros(32, 16, dtype=bf)
    else:
        u = torch.zeros(64, 16, dtype=torch.float32)
    with pytest.raises(FoundryAttnError):
        lora_grad(u, x, 1.0, transpose, out=out)


@pytest.mark.parametrize("case", ["transposed", "offset", "sliced_heads"])
def test_cpu_fwd_route_requires_contiguous_offset0(case):
    """The host route mirrors cpu_fwd's guard (lib.rs:167-172): a host input
    that is not contiguous from storage offset 0 is refused, not staged."""
    q = torch.zeros(32, 2, 64)
    if case == "transposed":
        bad = torch.zeros(2, 32, 64).transpose(0, 1)
    elif case == "offset":
        bad = torch.zeros(33, 2, 64)[1:]
    else:
        bad = torch.zeros(32, 4, 64)[:, :2]
    for args in ((bad, q, q), (q, bad, q), (q, q, bad)):
        with pytest.raises(FoundryAttnError, match="contiguous offset-0"):
            AttnBwd().fwd(*args)


def test_saved_lse_is_keyed_on_the_forward_call():
    """The LSE slot of AttnBwd is reused only for the res object the forward
    returned, with q, k, v unchanged; anything else regenerates it."""
    op = AttnBwd()
    q, k, v = (torch.randn(16, 2, 64) for _ in range(3))
    res = torch.randn(16, 2, 64)
    lse = torch.zeros(1, 2, 16)
    import weakref
    op._saved = (weakref.ref(res), tuple(op._key(t) for t in (q, k, v, res)), lse)
    assert op._saved_lse(q, k, v, res) is lse
    other = res.clone()
    assert op._saved_lse(q, k, v, other) is None          # a different res object
    assert op._saved_lse(q, k.clone(), v, res) is None    # different storage for k
    q.add_(1.0)                                           # q modified in place
    assert op._saved_lse(q, k, v, res) is None


@pytest.mark.parametrize("case", ["b_shape", "b_dtype", "g_len", "shift_dtype", "sum_shape", "copy_col_stride",
                                  "x_col_stride"])
def test_gated_ln_mod_fwd_rejects(case):
    """The fused gated residual + layer_norm_mod refuses views that do not
    match x before anything is launched."""
    from foundry_attn import block as fb
    x, b = _x(), _x()
    g, sh, sc = (torch.zeros(128, dtype=bf) for _ in range(3))
    kw = {}
    if case == "b_shape":
        b = _x(K=96)
    elif case == "b_dtype":
        b = _x(dtype=torch.float32)
    elif case == "g_len":
        g = torch.zeros(96, dtype=bf)
    elif case == "shift_dtype":
        sh = torch.zeros(128, dtype=torch.float32)
    elif case == "sum_shape":
        kw["sum_out"] = _x(N=32)
    elif case == "copy_col_stride":
        kw["sum_copy"] = torch.zeros(128, 64, dtype=bf).t()
    else:
        x = torch.zeros(128, 64, dtype=bf).t()
    with pytest.raises(FoundryAttnError):
        fb.gated_ln_mod_fwd(x, g, b, sh, sc, 1e-6, **kw)


@pytest.mark.parametrize("case", ["gated_out_shape", "gated_out_dtype", "g_len", "dy_col_stride"])
def test_ln_mod_bwd_gate_rejects(case):
    from foundry_attn import block as fb
    x, dy = _x(), _x()
    sc, g = torch.zeros(128, dtype=bf), torch.zeros(128, dtype=bf)
    mean, rstd = torch.zeros(64), torch.ones(64)
    kw = {}
    if case == "gated_out_shape":
        kw["gated_out"] = _x(K=64)
    elif case == "gated_out_dtype":
        kw["gated_out"] = _x(dtype=torch.float32)
    elif case == "g_len":
        g = torch.zeros(64, dtype=bf)
    else:
        dy = torch.zeros(128, 64, dtype=bf).t()
    with pytest.raises(FoundryAttnError):
        fb.ln_mod_bwd_gate(x, dy, sc, mean, rstd, g, 1e-6, **kw)
