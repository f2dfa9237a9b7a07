"""GPU parity of the dense + bias + residual + LayerNorm kernel
(dense_add_layernorm, vfk_dense_residual_layernorm_fwd) against the oracle's
DeBERTa post-LN output block (oracle.epilogues.dense_residual_layernorm,
deberta_v2_encoder.py:504-508, :563-567) with the projection rounded to the
storage type once, as the unfused Linear writes it.

Tolerance, per element: the kernel and the oracle round the projection y at
the same point, but their fp32 sums differ in order, so a rounded y may differ
by one unit in the last place (2^-7 |y| for bf16, 2^-10 for fp16); that moves
the output by rstd |gamma| times as much, plus at most as much again through
the row mean; the output itself is rounded once (2^-8 |out| for bf16, 2^-11
for fp16). The bound is the sum of those terms plus 1e-3, and the cosine
over the whole output must be >= 0.9999."""
import pytest
import torch

from _tol import cosine
from oracle import epilogues as oe

pytestmark = pytest.mark.gpu

ULP = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}


def _ops():
    from kernels import dense_layernorm as dl
    return dl


def _inputs(M, N, K, dtype, seed, bias=True, affine=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(dtype)
    b = (0.5 * torch.randn(N, generator=g)).to(dtype) if bias else None
    r = torch.randn(M, N, generator=g).to(dtype)
    lw = (1 + 0.2 * torch.randn(N, generator=g)).to(dtype) if affine else None
    lb = (0.1 * torch.randn(N, generator=g)).to(dtype) if affine else None
    return x, w, b, r, lw, lb


def _check(got, x, w, b, r, lw, lb, eps, dtype, what, scale=1.0):
    """got [M, N] against the oracle on the same (CPU) inputs."""
    got = got.detach().float().cpu()
    want = oe.dense_residual_layernorm(x, w, b, r, lw, lb, eps, round_dtype=dtype)
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    y = oe.residual_dense(x, w, b)                           # unrounded projection
    v = y.to(dtype).float() + r.float()
    rstd = 1.0 / torch.sqrt(v.var(-1, unbiased=False, keepdim=True) + eps)
    gam = lw.float().abs() if lw is not None else torch.ones(w.shape[0])
    u = ULP[dtype]
    flip = rstd * gam * u * (y.abs() + y.abs().mean(-1, keepdim=True))
    lim = scale * (flip + (u / 2) * want.abs() + 1e-3)
    err = (got - want).abs()
    assert bool((err <= lim).all()), f"{what}: worst excess {(err - lim).max().item():.3e}, " \
                                     f"max-abs {err.max().item():.3e}"
    c = cosine(got, want)
    assert c >= 0.9999, f"{what}: cos {c:.6f}"


@pytest.mark.parametrize("N,K", [(256, 64), (768, 768), (1024, 4096)])
def test_pack_weight_layout(dev, N, K):
    """packed[f][s][c + 32 h][i] = w[32 f + c][16 s + 8 h + i], bit for bit,
    also from a weight with padded rows."""
    g = torch.Generator().manual_seed(N + K)
    w = torch.randn(N, K + 64, generator=g).to(torch.bfloat16)[:, :K]
    got = _ops().pack_dense_weight(w.to(dev)).cpu()
    want = w.reshape(N // 32, 32, K // 16, 2, 8).permute(0, 2, 3, 1, 4).reshape(N // 32, K // 16, 64, 8)
    assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("N", [256, 512, 768, 1024])
@pytest.mark.parametrize("M", [1, 63, 64, 65, 200])
def test_matches_oracle(dev, dtype, N, M):
    x, w, b, r, lw, lb = _inputs(M, N, 768, dtype, 100 + N + M)
    got = _ops().dense_add_layernorm(x.to(dev), w.to(dev), b.to(dev), r.to(dev), lw.to(dev),
                                     lb.to(dev), 1e-7)
    torch.cuda.synchronize()
    _check(got, x, w, b, r, lw, lb, 1e-7, dtype, f"{dtype} M={M} N={N}")


@pytest.mark.parametrize("K", [64, 128, 192, 1024, 3072, 4096])
def test_reduction_lengths(dev, K):
    """The K loop at its shortest (one 64-wide slice: only the peeled last
    step), odd numbers of slices, and the FFN-output widths."""
    dtype = torch.bfloat16
    x, w, b, r, lw, lb = _inputs(130, 1024, K, dtype, 7 + K)
    got = _ops().dense_add_layernorm(x.to(dev), w.to(dev), b.to(dev), r.to(dev), lw.to(dev),
                                     lb.to(dev), 1e-7)
    torch.cuda.synchronize()
    _check(got, x, w, b, r, lw, lb, 1e-7, dtype, f"K={K}")


@pytest.mark.parametrize("bias,affine", [(False, False), (False, True), (True, False)])
def test_optional_parameters(dev, bias, affine):
    dtype = torch.bfloat16
    x, w, b, r, lw, lb = _inputs(100, 768, 768, dtype, 21, bias=bias, affine=affine)
    mv = lambda t: t.to(dev) if t is not None else None
    got = _ops().dense_add_layernorm(x.to(dev), w.to(dev), mv(b), r.to(dev), mv(lw), mv(lb), 1e-5)
    torch.cuda.synchronize()
    _check(got, x, w, b, r, lw, lb, 1e-5, dtype, f"bias={bias} affine={affine}")


def test_in_place_strided_and_3d(dev):
    """out = the residual (updated in place); x rows with a padded stride;
    [B, L, K] inputs; the module form with the reference's parameter names."""
    dtype = torch.bfloat16
    x, w, b, r, lw, lb = _inputs(3 * 70, 1024, 1024, dtype, 33)
    xs = torch.zeros(3 * 70, 1024 + 64, dtype=dtype)
    xs[:, :1024] = x
    xd = xs.to(dev)[:, :1024]
    rd = r.to(dev).clone()
    out = _ops().dense_add_layernorm(xd, w.to(dev), b.to(dev), rd, lw.to(dev), lb.to(dev), 1e-7,
                                     out=rd)
    torch.cuda.synchronize()
    assert out.data_ptr() == rd.data_ptr()
    _check(rd, x, w, b, r, lw, lb, 1e-7, dtype, "in place")
    m = _ops().SelfOutput(1024, 1024, eps=1e-7, dtype=dtype, device=dev)
    with torch.no_grad():
        m.dense.weight.copy_(w)
        m.dense.bias.copy_(b)
        m.LayerNorm.weight.copy_(lw)
        m.LayerNorm.bias.copy_(lb)
        got = m(x.view(3, 70, 1024).to(dev), r.view(3, 70, 1024).to(dev))
    torch.cuda.synchronize()
    assert got.shape == (3, 70, 1024)
    _check(got.view(-1, 1024), x, w, b, r, lw, lb, 1e-7, dtype, "module")


@pytest.mark.parametrize("K", [1024, 4096])
def test_deberta_large_size_against_unfused(dev, K):
    """DeBERTa-v3-large's two post-LN blocks at B=32, L=512 (16 384 rows,
    hidden 1024; K = 1024 after attention, 4096 after the FFN): against the
    unfused F.linear + fused_add_layernorm on every row, and against the
    oracle on a sample of rows."""
    import torch.nn.functional as F
    from kernels.fused_layernorm import fused_add_layernorm
    dtype = torch.bfloat16
    M, N = 16384, 1024
    x, w, b, r, lw, lb = _inputs(M, N, K, dtype, 55 + K)
    xd, wd, bd, rd, lwd, lbd = (t.to(dev) for t in (x, w, b, r, lw, lb))
    got = _ops().dense_add_layernorm(xd, wd, bd, rd, lwd, lbd, 1e-7)
    ref = fused_add_layernorm(F.linear(xd, wd, bd), rd, lwd, lbd, 1e-7, return_sum=False)
    torch.cuda.synchronize()
    d = (got.float() - ref.float()).abs()
    assert d.max().item() < 0.15 and d.mean().item() < 2e-3, (d.max().item(), d.mean().item())
    assert cosine(got.float().cpu(), ref.float().cpu()) >= 0.9999
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(5))[:256]
    _check(got[rows.to(dev)], x[rows], w, b, r[rows], lw, lb, 1e-7, dtype, f"K={K} sample")


@pytest.mark.parametrize("in_place", [False, True])
def test_residual_sum_output(dev, in_place):
    """return_sum: the sum round(x W^T) + residual, rounded once, beside the
    normalised rows (ModernBERT's pre-LN stream: Wo, residual add, next
    LayerNorm without bias); in place over the residual when asked."""
    dtype = torch.bfloat16
    x, w, _, r, lw, _ = _inputs(300, 768, 1152, dtype, 77, bias=False)
    rd = r.to(dev).clone()
    got, s = _ops().dense_add_layernorm(x.to(dev), w.to(dev), None, rd, lw.to(dev), None, 1e-5,
                                        return_sum=True, residual_out=rd if in_place else None)
    torch.cuda.synchronize()
    if in_place:
        assert s.data_ptr() == rd.data_ptr()
    _check(got, x, w, None, r, lw, None, 1e-5, dtype, "normalised")
    y = oe.residual_dense(x, w)
    want = y.to(dtype).float() + r.float()
    err = (s.float().cpu() - want).abs()
    lim = ULP[dtype] * y.abs() + (ULP[dtype] / 2) * want.abs() + 1e-3
    assert bool((err <= lim).all()), (err - lim).max().item()
