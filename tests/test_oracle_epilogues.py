"""Pins the oracle's epilogues (oracle/epilogues.py) with library routines and
RoPE identities."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oa
from oracle import epilogues as oe

D64 = torch.float64


def _r(*shape, seed=0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=D64)


def test_layernorm_equals_torch():
    x, w, b = _r(50, 768, seed=1), _r(768, seed=2), _r(768, seed=3)
    torch.testing.assert_close(oe.layernorm(x, w, b, 1e-5, dtype=D64), F.layer_norm(x, (768,), w, b, 1e-5))
    torch.testing.assert_close(oe.layernorm(x, None, None, 1e-5, dtype=D64), F.layer_norm(x, (768,), eps=1e-5))


def test_rmsnorm_equals_transformers_t5_layernorm():
    from transformers.models.t5.modeling_t5 import T5LayerNorm
    x, w = _r(20, 1024, seed=4).float(), _r(1024, seed=5).float()
    m = T5LayerNorm(1024, eps=1e-6)
    with torch.no_grad():
        m.weight.copy_(w)
    torch.testing.assert_close(oe.rmsnorm(x, w, 1e-6), m(x))


@pytest.mark.parametrize("act,ref", [("gelu_erf", lambda a: F.gelu(a)),
                                     ("gelu_tanh", lambda a: F.gelu(a, approximate="tanh")),
                                     ("silu", F.silu), ("relu", F.relu)])
def test_glu_equals_torch_activations(act, ref):
    a, b = _r(100, 64, seed=6) * 3, _r(100, 64, seed=7)
    torch.testing.assert_close(oe.glu(a, b, act, dtype=D64), ref(a) * b)


def test_rope_identities():
    x = _r(1, 50, 3, 64, seed=8)
    cos, sin = oa.rope_cos_sin(torch.arange(50), 10000.0)
    y = oe.rope_table(x, cos[None].double(), sin[None].double(), dtype=D64)
    torch.testing.assert_close(y[:, 0], x[:, 0])                      # position 0
    n_x = x[..., :32] ** 2 + x[..., 32:] ** 2
    n_y = y[..., :32] ** 2 + y[..., 32:] ** 2
    torch.testing.assert_close(n_x, n_y)                              # pair norms
    # <rope(q, p), rope(k, p')> depends only on p - p'
    q, k = _r(64, seed=9), _r(64, seed=10)
    qs = q.expand(1, 50, 1, 64)
    ks = k.expand(1, 50, 1, 64)
    cq = oe.rope_table(qs, cos[None].double(), sin[None].double(), dtype=D64)[0, :, 0]
    ck = oe.rope_table(ks, cos[None].double(), sin[None].double(), dtype=D64)[0, :, 0]
    for d in (0, 3, 11):
        vals = torch.stack([cq[p + d] @ ck[p] for p in range(0, 50 - d)])
        assert float(vals.max() - vals.min()) < 1e-4 * float(vals.abs().max() + 1)


def _rope_sign_flipped(x, cos, sin, dtype=torch.float64):
    """A plausible mistake: rotate_half with the wrong sign (a rotation by -theta)."""
    x, cos, sin = x.to(dtype), cos.to(dtype), sin.to(dtype)
    h = x.shape[-1] // 2
    rot = torch.cat((x[..., h:], -x[..., :h]), dim=-1)
    return x * cos.unsqueeze(2) + rot * sin.unsqueeze(2)


def _rope_checks(fn):
    """Checks that pin a RoPE implementation f(x [B,S,H,64], cos, sin [B,S,64]):
    (1) the closed form: the pair (x[f], x[f + 32]) read as the complex number
    x[f] + i x[f + 32] is multiplied by e^{i pos inv_freq[f]} (RoPE's
    definition, non-interleaved halves); (2) transformers' ModernBERT
    apply_rotary_pos_emb; (3) the brute-force-pinned oracle.attention.apply_rope."""
    from transformers.models.modernbert.modeling_modernbert import apply_rotary_pos_emb
    g = torch.Generator().manual_seed(11)
    B, S, H = 2, 37, 3
    x = torch.randn(B, S, H, 64, generator=g, dtype=D64)
    pos = torch.randint(0, 4000, (B, S), generator=g)
    inv = 1.0 / (160000.0 ** (torch.arange(0, 64, 2, dtype=torch.int64).float() / 64))
    ang = (pos.float()[..., None] * inv).double()          # fp32 angles, as HF forms them
    cos = torch.cat((ang.cos(), ang.cos()), -1)
    sin = torch.cat((ang.sin(), ang.sin()), -1)
    got = fn(x, cos, sin)
    z = torch.complex(x[..., :32], x[..., 32:]) * torch.polar(torch.ones_like(ang), ang)[:, :, None]
    want = torch.cat((z.real, z.imag), -1)
    ok = [torch.allclose(got, want, rtol=0, atol=1e-12)]
    qh, _ = apply_rotary_pos_emb(x.float(), x.float(), cos.float(), sin.float(), unsqueeze_dim=2)
    ok.append(torch.allclose(got.float(), qh, rtol=0, atol=1e-5))
    ok.append(torch.allclose(got, oa.apply_rope(x, cos, sin), rtol=0, atol=1e-12))
    return ok


def test_rope_table_pinned_by_closed_form_and_transformers():
    assert _rope_checks(lambda x, c, s: oe.rope_table(x, c, s, dtype=D64)) == [True, True, True]
    # the [B, 1, S, D] table layout the reference also accepts
    x = _r(2, 9, 2, 64, seed=12)
    c, s = _r(2, 9, 64, seed=13), _r(2, 9, 64, seed=14)
    torch.testing.assert_close(oe.rope_table(x, c[:, None], s[:, None], dtype=D64),
                               oe.rope_table(x, c, s, dtype=D64))


def test_rope_checks_reject_sign_flip():
    """Negative control: the sign-flipped rotation passes the identities of
    test_rope_identities (norms, position 0, relative dependence) but fails
    every check that pins rope_table."""
    assert _rope_checks(_rope_sign_flipped) == [False, False, False]
    x = _r(1, 50, 3, 64, seed=8)
    cos, sin = oa.rope_cos_sin(torch.arange(50), 10000.0)
    y = _rope_sign_flipped(x, cos[None].double(), sin[None].double())
    torch.testing.assert_close(y[:, 0], x[:, 0])
    torch.testing.assert_close(x[..., :32] ** 2 + x[..., 32:] ** 2, y[..., :32] ** 2 + y[..., 32:] ** 2)


def test_residual_add_equals_torch_add():
    """kernels/fused_dropout_residual.py:50-51 (inference): residual + input,
    in the oracle's dtype, element for element."""
    x, r = _r(30, 768, seed=15), _r(30, 768, seed=16)
    assert torch.equal(oe.residual_add(x, r, dtype=D64), torch.add(r, x))
    xb, rb = x.to(torch.bfloat16), r.to(torch.bfloat16)
    assert torch.equal(oe.residual_add(xb, rb), torch.add(rb.float(), xb.float()))


# ------------------------------------------------------------------ ColBERT head
def test_colbert_head_matches_library_routines():
    """LayerNorm -> Linear -> L2 normalise equals F.layer_norm, F.linear and
    F.normalize (eps 1e-8 is the reference's clamp) composed."""
    import torch.nn.functional as F
    from oracle import epilogues as oep
    g = torch.Generator().manual_seed(31)
    x = torch.randn(50, 256, generator=g, dtype=torch.float64)
    r = torch.randn(50, 256, generator=g, dtype=torch.float64)
    lw = 1 + 0.1 * torch.randn(256, generator=g, dtype=torch.float64)
    w = torch.randn(64, 256, generator=g, dtype=torch.float64) * 0.05
    b = torch.randn(64, generator=g, dtype=torch.float64) * 0.01
    got = oep.colbert_head(x, [(w, b, None, False)], lw, None, 1e-5, residual=r, dtype=torch.float64)
    want = F.normalize(F.linear(F.layer_norm(x + r, (256,), lw, None, 1e-5), w, b), dim=-1, eps=1e-8)
    torch.testing.assert_close(got, want, rtol=0, atol=1e-12)
    torch.testing.assert_close(got.norm(dim=-1), torch.ones(50, dtype=torch.float64))


def test_colbert_head_residual_stack_and_zero_rows():
    """The PyLate residual Dense stack (widths 256 -> 512 -> 256 -> 64, residual
    projections where widths differ, identity where equal), and an all-zero
    projected row stays zero (the norm is clamped at 1e-8, not divided by 0)."""
    import torch.nn.functional as F
    from oracle import epilogues as oep
    g = torch.Generator().manual_seed(32)
    x = torch.randn(20, 256, generator=g, dtype=torch.float64)
    w1, r1 = torch.randn(512, 256, generator=g, dtype=torch.float64) * 0.05, \
        torch.randn(512, 256, generator=g, dtype=torch.float64) * 0.05
    w2 = torch.randn(256, 512, generator=g, dtype=torch.float64) * 0.05
    r2 = torch.randn(256, 512, generator=g, dtype=torch.float64) * 0.05
    w3 = torch.randn(64, 256, generator=g, dtype=torch.float64) * 0.05
    layers = [(w1, None, r1, True), (w2, None, r2, True), (w3, None, None, False)]
    got = oep.colbert_head(x, layers, layer_norm=False, dtype=torch.float64)
    h = F.linear(x, w1) + F.linear(x, r1)
    h = F.linear(h, w2) + F.linear(h, r2)
    want = F.normalize(F.linear(h, w3), dim=-1, eps=1e-8)
    torch.testing.assert_close(got, want, rtol=0, atol=1e-12)
    # same width: the residual is the input itself
    sq = torch.randn(256, 256, generator=g, dtype=torch.float64) * 0.05
    y = oep.residual_dense(x, sq, None, None, True, dtype=torch.float64)
    torch.testing.assert_close(y, F.linear(x, sq) + x)
    z = oep.colbert_head(torch.zeros(3, 256, dtype=torch.float64), [(w3, None, None, False)],
                         layer_norm=False, dtype=torch.float64)
    assert torch.equal(z, torch.zeros(3, 64, dtype=torch.float64))


# ------------------------------------------------ DeBERTa dense + residual + LN
def test_dense_residual_layernorm_matches_torch_modules():
    """LayerNorm(dense(h) + input) built from torch.nn.Linear and
    torch.nn.LayerNorm (DebertaV2SelfOutput's modules, eps 1e-7) in float64;
    unit-gamma rows have mean 0 and variance 1; dropping the bias or the
    residual fails."""
    from oracle import epilogues as oep
    g = torch.Generator().manual_seed(41)
    x = torch.randn(40, 512, generator=g, dtype=D64)
    res = torch.randn(40, 256, generator=g, dtype=D64)
    lin = torch.nn.Linear(512, 256).double()
    ln = torch.nn.LayerNorm(256, eps=1e-7).double()
    with torch.no_grad():
        lin.weight.copy_(torch.randn(256, 512, generator=g, dtype=D64) * 0.05)
        lin.bias.copy_(torch.randn(256, generator=g, dtype=D64))
        ln.weight.copy_(1 + 0.1 * torch.randn(256, generator=g, dtype=D64))
        ln.bias.copy_(0.1 * torch.randn(256, generator=g, dtype=D64))
        want = ln(lin(x) + res)
    got = oep.dense_residual_layernorm(x, lin.weight, lin.bias, res, ln.weight, ln.bias, 1e-7,
                                       dtype=D64)
    torch.testing.assert_close(got, want, rtol=0, atol=1e-12)
    unit = oep.dense_residual_layernorm(x, lin.weight, lin.bias, res, eps=0.0, dtype=D64)
    torch.testing.assert_close(unit.mean(-1), torch.zeros(40, dtype=D64), rtol=0, atol=1e-12)
    torch.testing.assert_close(unit.var(-1, unbiased=False), torch.ones(40, dtype=D64), rtol=0, atol=1e-10)
    no_bias = oep.dense_residual_layernorm(x, lin.weight, None, res, ln.weight, ln.bias, 1e-7, dtype=D64)
    no_res = oep.layernorm(lin(x).detach(), ln.weight, ln.bias, 1e-7, dtype=D64)
    assert (no_bias - want).abs().max() > 1e-2 and (no_res - want).abs().max() > 1e-2
    # round_dtype rounds the projection once: equal to the unrounded form on
    # inputs whose projection is exactly representable in bf16
    xi = torch.randint(-2, 3, (8, 64), generator=g).to(D64)
    wi = torch.randint(-2, 3, (256, 64), generator=g).to(D64)
    ri = torch.randn(8, 256, generator=g, dtype=D64)
    torch.testing.assert_close(
        oep.dense_residual_layernorm(xi, wi, None, ri, round_dtype=torch.bfloat16, dtype=D64),
        oep.dense_residual_layernorm(xi, wi, None, ri, dtype=D64), rtol=0, atol=0)
