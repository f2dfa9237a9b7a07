"""GPU parity of the fused GLU projection (vfk_glu_linear_fwd) against a
float64 reference of the same composition: the projection x W^T followed by
act(input) * gate (oracle.epilogues.glu), i.e. modernbert_encoder.py:157-178
up to Wo. Inputs are scaled so that the projections are O(1); the bound is one
16-bit rounding of the output plus fp32 accumulation, which a missing K slice,
a swapped token or feature block, or a wrong activation exceeds by orders of
magnitude."""
import pytest
import torch

from _tol import assert_elem_close, cosine
from oracle import epilogues as oe

pytestmark = pytest.mark.gpu

ACTS = [("gelu", "gelu_erf"), ("gelu_new", "gelu_tanh"), ("silu", "silu")]


def _inputs(M, K, I, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (torch.randn(2 * I, K, generator=g) / K ** 0.5).to(dtype)
    return x, w


def _ref(x, w, act):
    y = x.double() @ w.double().T
    I = w.shape[0] // 2
    return oe.glu(y[:, :I], y[:, I:], act, dtype=torch.float64)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K,I", [(1000, 768, 1152), (257, 128, 200), (1, 64, 8),
                                   (300, 1024, 64), (513, 192, 136)])
@pytest.mark.parametrize("act", ACTS, ids=[a[0] for a in ACTS])
def test_glu_linear_matches_reference(dev, dtype, M, K, I, act):
    from kernels.fused_glu_mlp import glu_linear
    x, w = _inputs(M, K, I, dtype, M + K + I)
    got = glu_linear(x.to(dev), w.to(dev), act[0])
    assert got.shape == (M, I) and got.dtype == dtype
    assert_elem_close(got, _ref(x, w, act[1]), dtype, f"glu_linear {M}x{K}x{I} {act[0]}")


def test_glu_linear_strided_rows_and_out(dev):
    """x and out as column slices of wider tensors (row strides K + 64 and
    I + 32), batch dims flattened, and the result written into `out`."""
    from kernels.fused_glu_mlp import glu_linear
    M, K, I = 700, 256, 96
    x, w = _inputs(M, K, I, torch.bfloat16, 5)
    xw = torch.zeros(M, K + 64, dtype=torch.bfloat16)
    xw[:, :K] = x
    xd = xw.to(dev)[:, :K]
    ow = torch.full((M, I + 32), 7.0, dtype=torch.bfloat16, device=dev)
    glu_linear(xd, w.to(dev), "gelu", out=ow[:, :I])
    assert_elem_close(ow[:, :I], _ref(x, w, "gelu_erf"), torch.bfloat16, "strided")
    assert (ow[:, I:] == 7.0).all(), "columns past I were written"
    y3 = glu_linear(x.view(7, 100, K).to(dev), w.to(dev), "gelu")
    assert y3.shape == (7, 100, I)
    assert_elem_close(y3.view(M, I), _ref(x, w, "gelu_erf"), torch.bfloat16, "3-d input")


def test_glu_linear_matches_unfused_path(dev):
    """Against F.linear + fused_gelu_mul_dropout (the layer's unfused path):
    the two differ only by where the projection is rounded to bf16. The
    unfused path rounds twice (projection, then product), which puts a few
    elements past a one-rounding bound, so it is held to the cosine only."""
    import torch.nn.functional as F
    from kernels.fused_glu_mlp import fused_gelu_mul_dropout, glu_linear
    M, K, I = 4096, 768, 1152
    x, w = _inputs(M, K, I, torch.bfloat16, 9)
    xd, wd = x.to(dev), w.to(dev)
    got = glu_linear(xd, wd, "gelu")
    y = F.linear(xd, wd)
    unf = fused_gelu_mul_dropout(y[:, :I], y[:, I:], "gelu")
    want = _ref(x, w, "gelu_erf")
    assert_elem_close(got, want, torch.bfloat16, "fused")
    assert cosine(unf.cpu(), want) >= 0.9999
    # the fused result is at least as close to the float64 reference
    e_f = (got.double().cpu() - want).abs().mean().item()
    e_u = (unf.double().cpu() - want).abs().mean().item()
    assert e_f <= e_u * 1.05, (e_f, e_u)


def test_glu_linear_modernbert_config5_shape(dev):
    """The ModernBERT-base MLP projection of the 256-sequence pack: x
    [163 736, 768], Wi [2304, 768], bf16. Rows checked: 384 sampled rows, the
    first and the last token tile (a partial tile of 152 rows)."""
    from kernels.fused_glu_mlp import glu_linear
    M, K, I = 163736, 768, 1152
    g = torch.Generator().manual_seed(11)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(2 * I, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    got = glu_linear(x.to(dev), w.to(dev), "gelu").cpu()
    rows = torch.cat([torch.arange(256), torch.randint(256, M - 256, (384,), generator=g),
                      torch.arange(M - 256, M)])
    want = _ref(x[rows], w, "gelu_erf")
    assert_elem_close(got[rows], want, torch.bfloat16, "config-5 rows")
    assert torch.isfinite(got.float()).all()
    assert cosine(got[rows], want) >= 0.9999
