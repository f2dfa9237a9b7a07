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
