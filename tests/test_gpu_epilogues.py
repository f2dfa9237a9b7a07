"""GPU parity of the memory-bound epilogues against the oracle (fp32, CPU)."""
import pytest
import torch

from _tol import assert_elem_close
from oracle import epilogues as oe

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _rand(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(4096, 768), (333, 1024), (17, 1000), (5, 8192), (64, 24)])
@pytest.mark.parametrize("affine", ["none", "w", "wb"])
def test_layernorm(dev, dtype, shape, affine):
    from kernels.fused_layernorm import FusedLayerNorm, fused_layernorm
    x = _rand(shape, dtype, 1)
    n = shape[-1]
    w = _rand((n,), dtype, 2) if affine != "none" else None
    b = _rand((n,), dtype, 3) if affine == "wb" else None
    want = oe.layernorm(x, w, b, 1e-5)
    got = fused_layernorm(x.to(dev), n, None if w is None else w.to(dev),
                          None if b is None else b.to(dev), 1e-5)
    assert_elem_close(got, want, dtype, f"layernorm {shape} {affine}")
    if affine == "wb":
        mod = FusedLayerNorm(n, eps=1e-5, dtype=dtype, device=dev)
        with torch.no_grad():
            mod.weight.copy_(w)
            mod.bias.copy_(b)
        assert_elem_close(mod(x.to(dev)), want, dtype, "FusedLayerNorm module")


@pytest.mark.parametrize("dtype", DTYPES)
def test_layernorm_residual_fused(dev, dtype):
    from kernels.fused_layernorm import fused_add_layernorm
    x = _rand((1000, 768), dtype, 4)
    r = _rand((1000, 768), dtype, 5)
    w = _rand((768,), dtype, 6)
    y, s = fused_add_layernorm(x.to(dev), r.to(dev), w.to(dev), None, 1e-5)
    ssum = (x.float() + r.float())
    assert_elem_close(s, ssum, dtype, "residual sum")
    # the norm sees the sum as computed (rounded to dtype when stored)
    assert_elem_close(y, oe.layernorm(ssum, w, None, 1e-5), dtype, "add+LN")


def test_layernorm_state_dict_compat(dev):
    from kernels.fused_layernorm import FusedLayerNorm
    ref = torch.nn.LayerNorm(768, eps=1e-5, bias=False)
    mod = FusedLayerNorm(768, eps=1e-5, bias=False)
    mod.load_state_dict(ref.state_dict())
    assert set(mod.state_dict()) == {"weight"}


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(2048, 1024), (7, 1000)])
def test_rmsnorm(dev, dtype, shape):
    from kernels.rms_norm import RMSNorm
    x = _rand(shape, dtype, 7)
    mod = RMSNorm(shape[-1], eps=1e-6, dtype=dtype, device=dev)
    w = _rand((shape[-1],), dtype, 8)
    with torch.no_grad():
        mod.weight.copy_(w)
    assert_elem_close(mod(x.to(dev)), oe.rmsnorm(x, w, 1e-6), dtype, "rmsnorm")
    r = _rand(shape, dtype, 9)
    y, s = mod(x.to(dev), r.to(dev))
    assert_elem_close(y, oe.rmsnorm(x.float() + r.float(), w, 1e-6), dtype, "add+rms")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("act", ["gelu", "gelu_pytorch_tanh", "silu"])
def test_glu_chunked(dev, dtype, act):
    """ModernBERT MLP: act(input) * gate on the two chunk() halves of Wi's output."""
    from kernels.fused_glu_mlp import fused_gelu_mul_dropout
    x = _rand((1500, 2 * 1152), dtype, 10, 2.0).to(dev)
    a, b = x.chunk(2, dim=-1)
    got = fused_gelu_mul_dropout(a, b, act_fn=act)
    name = {"gelu": "gelu_erf", "gelu_pytorch_tanh": "gelu_tanh", "silu": "silu"}[act]
    want = oe.glu(a.cpu(), b.cpu(), name)
    assert_elem_close(got, want, dtype, f"glu {act}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("act", ["gelu", "gelu_new", "gelu_accurate", "relu", "silu"])
def test_ff_fused(dev, dtype, act):
    from kernels.ff_fused import fused_gelu_mul_dropout
    gate = _rand((3, 77, 2816), dtype, 11, 2.0)
    up = _rand((3, 77, 2816), dtype, 12)
    got = fused_gelu_mul_dropout(gate.to(dev), up.to(dev), act_fn=act)
    assert got.shape == gate.shape
    name = {"gelu": "gelu_tanh", "gelu_new": "gelu_tanh", "gelu_accurate": "gelu_erf",
            "relu": "relu", "silu": "silu"}[act]
    assert_elem_close(got, oe.glu(gate, up, name), dtype, f"ff_fused {act}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_residual(dev, dtype):
    from kernels.fused_dropout_residual import fused_dropout_residual
    x = _rand((1, 4001, 768), dtype, 13)
    r = _rand((1, 4001, 768), dtype, 14)
    got = fused_dropout_residual(x.to(dev), r.to(dev), 0.1, training=False)
    assert_elem_close(got, oe.residual_add(x, r), dtype, "residual")
    # odd sizes take the scalar path
    x2, r2 = _rand((3, 5), dtype, 15), _rand((3, 5), dtype, 16)
    assert_elem_close(fused_dropout_residual(x2.to(dev), r2.to(dev)), oe.residual_add(x2, r2),
                      dtype, "residual odd")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("cos_rank", [3, 4])
def test_rope_table(dev, dtype, cos_rank):
    from kernels.fused_rope_global import fused_rope_global_apply
    from kernels.fused_rope_local import fused_rope_local_apply
    from oracle.attention import rope_cos_sin
    B, S, H, D = 2, 300, 12, 64
    q = _rand((B, S, H, D), dtype, 17)
    k = _rand((B, S, H, D), dtype, 18)
    cos, sin = rope_cos_sin(torch.arange(S), 160000.0, D)
    cos = cos.to(dtype)[None].expand(B, S, D)
    sin = sin.to(dtype)[None].expand(B, S, D)
    if cos_rank == 4:
        cos, sin = cos[:, None], sin[:, None]
    for fn in (fused_rope_global_apply, fused_rope_local_apply):
        gq, gk = fn(q.to(dev), k.to(dev), cos.to(dev), sin.to(dev))
        assert_elem_close(gq, oe.rope_table(q, cos, sin), dtype, "rope q")
        assert_elem_close(gk, oe.rope_table(k, cos, sin), dtype, "rope k")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_fp32_tables_used_at_fp32(dev, dtype):
    """16-bit q/k with fp32 cos/sin (the reference's Triton kernel promotes
    the mixed product to fp32): the tables are not rounded to q's dtype first,
    so the result is the fp32 rotation rounded once. q and k have different
    head counts (7 and 5, not multiples of the kernel's head slots), and
    D = 64 runs the unit-layout kernel; test_rope_head_dim_32_general_kernel
    covers the general one."""
    from kernels.fused_rope_global import fused_rope_global_apply
    from oracle.attention import rope_cos_sin
    B, S, D = 2, 333, 64
    q = _rand((B, S, 7, D), dtype, 21)
    k = _rand((B, S, 5, D), dtype, 22)
    cos, sin = rope_cos_sin(torch.arange(S) * 7 + 3, 160000.0, D)   # fp32, large angles
    gq, gk = fused_rope_global_apply(q.to(dev), k.to(dev), cos.to(dev), sin.to(dev))
    for got, x, name in ((gq, q, "q"), (gk, k, "k")):
        want = oe.rope_table(x, cos[None], sin[None])                  # fp32 tables, fp32 math
        assert got.dtype == dtype
        assert_elem_close(got, want, dtype, f"rope fp32-table {name}")
        # the output is the fp32 result (products rounded separately, then
        # the add) rounded once: it equals the oracle rounded to q's dtype at
        # every element; tables rounded to q's dtype first would change about
        # a quarter of them
        got_c = got.cpu()
        exact = (got_c == want.to(dtype)).float().mean().item()
        lossy = oe.rope_table(x, cos[None].to(dtype), sin[None].to(dtype)).to(dtype)
        lossy_exact = (lossy == want.to(dtype)).float().mean().item()
        print(f"rope {dtype} {name}: {exact:.5f} of elements equal the rounded fp32 result "
              f"(tables rounded first: {lossy_exact:.5f})")
        assert exact == 1.0 and lossy_exact < 0.9, (exact, lossy_exact)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_head_dim_32_general_kernel(dev, dtype):
    """D = 32 (4 chunks of 8 per head: outside the unit layout) through the
    general kernel, fp32 tables, q and k of 3 and 9 heads: every element
    equals the oracle's fp32 result rounded once."""
    from kernels.fused_rope_global import fused_rope_global_apply
    from oracle.attention import rope_cos_sin
    B, S, D = 3, 97, 32
    q = _rand((B, S, 3, D), dtype, 23)
    k = _rand((B, S, 9, D), dtype, 24)
    cos, sin = rope_cos_sin(torch.arange(S) * 5 + 1, 10000.0, D)
    gq, gk = fused_rope_global_apply(q.to(dev), k.to(dev), cos.to(dev), sin.to(dev))
    for got, x in ((gq, q), (gk, k)):
        want = oe.rope_table(x, cos[None], sin[None]).to(dtype)
        assert torch.equal(got.cpu(), want)


def test_rope_fp32(dev):
    from kernels.fused_rope_global import fused_rope_global_apply
    from oracle.attention import rope_cos_sin
    q = _rand((1, 257, 12, 64), torch.float32, 23)
    k = _rand((1, 257, 12, 64), torch.float32, 24)
    cos, sin = rope_cos_sin(torch.arange(257), 10000.0, 64)
    gq, gk = fused_rope_global_apply(q.to(dev), k.to(dev), cos.to(dev), sin.to(dev))
    assert_elem_close(gq, oe.rope_table(q, cos[None], sin[None]), torch.float32, "rope f32 q")
    assert_elem_close(gk, oe.rope_table(k, cos[None], sin[None]), torch.float32, "rope f32 k")


def test_rope_strided_qkv_view(dev):
    """q/k as strided views of a fused [B,S,3,H,D] projection (no copies)."""
    from kernels.fused_rope_global import fused_rope_apply
    from oracle.attention import rope_cos_sin
    qkv = _rand((1, 500, 3, 12, 64), torch.bfloat16, 19)
    q = qkv[:, :, 0]
    cos, sin = rope_cos_sin(torch.arange(500), 10000.0, 64)
    cos, sin = cos.bfloat16()[None], sin.bfloat16()[None]
    got = fused_rope_apply(qkv.to(dev)[:, :, 0], cos.to(dev), sin.to(dev))
    assert_elem_close(got, oe.rope_table(q, cos, sin), torch.bfloat16, "rope view")


# ------------------------------------------------------------------ ColBERT head
def _colbert_rows_close(got, want, what):
    """Unit-norm embeddings of 16-bit LayerNorm outputs projected over D terms:
    each row within cosine 0.9999 of the fp32 oracle and every entry within
    4e-3 (entries are ~1/sqrt(N) ~ 0.09; one bf16 rounding of the normalised
    hidden row, the product sum and the output each contribute < 1e-3)."""
    from _tol import cosine
    got = got.float().cpu()
    assert torch.isfinite(got).all(), what
    err = (got - want).abs().max().item()
    worst = min(cosine(got[i], want[i]) for i in range(0, got.shape[0], max(1, got.shape[0] // 64)))
    assert err <= 4e-3 and worst >= 0.9999, (what, err, worst)
    torch.testing.assert_close(got.norm(dim=-1), torch.ones(got.shape[0]), atol=5e-3, rtol=0)


@pytest.mark.parametrize("pack", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,D,N", [(1000, 768, 128), (1, 768, 128), (33, 1024, 96), (64, 256, 32)])
def test_colbert_head_with_final_layernorm(dev, dtype, T, D, N, pack):
    """ModernBERT final LayerNorm (weight, no bias, eps 1e-5) of x + residual,
    projection [N, D] without bias, L2 normalisation; the LayerNorm output
    that comes back equals the LayerNorm oracle. Both weight layouts: operand
    order (packed) and [N, D] rows."""
    from kernels.colbert_head import colbert_head
    x, r = _rand((T, D), dtype, 41), _rand((T, D), dtype, 42)
    lw = (1 + 0.1 * _rand((D,), torch.float32, 43)).to(dtype)
    w = _rand((N, D), dtype, 44, 0.05)
    want = oe.colbert_head(x, [(w, None, None, False)], lw, None, 1e-5, residual=r)
    got, h = colbert_head(x.to(dev), w.to(dev), None, lw.to(dev), None, 1e-5, residual=r.to(dev),
                          return_hidden=True, pack=pack)
    _colbert_rows_close(got, want, f"colbert {dtype} {T}x{D}->{N} pack={pack}")
    assert_elem_close(h, oe.layernorm(x.float() + r.float(), lw, None, 1e-5), dtype,
                      f"colbert hidden {dtype}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,D,N,res,ln,lnb,bias", [
    (1000, 768, 128, True, True, False, False), (1, 768, 128, True, True, False, False),
    (33, 1024, 96, True, True, True, True), (64, 256, 32, False, True, False, False),
    (300, 384, 64, False, False, False, True), (129, 2048, 128, True, True, True, False),
    (257, 640, 128, True, False, False, False)])
def test_colbert_head_folded(dev, dtype, T, D, N, res, ln, lnb, bias):
    """The folded form (LayerNorm weight multiplied into the projection, the
    raw rows projected; taken whenever the LayerNorm output is not returned):
    with and without residual, LayerNorm weight and bias, projection bias;
    token counts around the 128-token workgroup; hidden sizes up to 2048."""
    from kernels.colbert_head import colbert_head
    x = _rand((T, D), dtype, 141)
    r = _rand((T, D), dtype, 142) if res else None
    lw = (1 + 0.1 * _rand((D,), torch.float32, 143)).to(dtype) if ln else None
    lb = (0.1 * _rand((D,), torch.float32, 144)).to(dtype) if lnb else None
    w = _rand((N, D), dtype, 145, 0.05)
    b = _rand((N,), dtype, 146, 0.1) if bias else None
    want = oe.colbert_head(x, [(w, b, None, False)], lw, lb, 1e-5, residual=r,
                           layer_norm=ln)
    d = lambda t: None if t is None else t.to(dev)
    got = colbert_head(x.to(dev), w.to(dev), d(b), d(lw), d(lb), 1e-5, residual=d(r))
    _colbert_rows_close(got, want, f"folded {dtype} {T}x{D}->{N} res={res} ln={ln}")


def test_colbert_head_folded_rows_far_from_zero_mean(dev):
    """Rows whose mean is 30 standard deviations from zero: the folded form
    subtracts mu G from the raw projection, which its shifted statistics keep
    exact enough. The LayerNorm input is the residual sum rounded to bf16 (as
    the encoder's is; its spacing near 30 is 1/8), so the oracle takes that
    rounded sum."""
    from kernels.colbert_head import colbert_head
    T, D, N = 500, 768, 128
    x = (_rand((T, D), torch.float32, 151) + 30.0).bfloat16()
    r = (0.5 * _rand((T, D), torch.float32, 152)).bfloat16()
    lw = (1 + 0.1 * _rand((D,), torch.float32, 153)).bfloat16()
    w = _rand((N, D), torch.bfloat16, 154, 0.05)
    u = (x.float() + r.float()).bfloat16()
    want = oe.colbert_head(u, [(w, None, None, False)], lw, None, 1e-5)
    got = colbert_head(x.to(dev), w.to(dev), None, lw.to(dev), None, 1e-5, residual=r.to(dev))
    _colbert_rows_close(got, want, "folded, mean 30")


def test_colbert_head_folded_multi_chunk(dev):
    """Token counts past 128 x the workgroups the device holds at once: each
    workgroup then runs several 128-token chunks through one pipeline (the
    next chunk's first slices load during a chunk's outputs), the last one
    partial. Every 97th row against the oracle; every row equal, bit for bit,
    to the same rows run in a call of their own (a row's result does not
    depend on how the rows are split among workgroups)."""
    from kernels.colbert_head import colbert_head
    T, D, N = 131149, 768, 128
    x = _rand((T, D), torch.bfloat16, 171)
    r = _rand((T, D), torch.bfloat16, 172)
    lw = (1 + 0.1 * _rand((D,), torch.float32, 173)).bfloat16()
    w = _rand((N, D), torch.bfloat16, 174, 0.05)
    xd, rd, lwd, wd = x.to(dev), r.to(dev), lw.to(dev), w.to(dev)
    got = colbert_head(xd, wd, None, lwd, None, 1e-5, residual=rd)
    idx = torch.arange(0, T, 97)
    want = oe.colbert_head(x[idx], [(w, None, None, False)], lw, None, 1e-5, residual=r[idx])
    _colbert_rows_close(got[idx.to(dev)], want, "folded, several chunks per workgroup")
    for a, b in ((0, 1000), (T - 777, T), (65536, 65536 + 300)):
        part = colbert_head(xd[a:b], wd, None, lwd, None, 1e-5, residual=rd[a:b])
        assert torch.equal(part, got[a:b]), (a, b)


def test_colbert_head_refolds_an_updated_norm_weight(dev):
    """The folded weight follows the LayerNorm weight it was made from: an
    in-place update of it is seen by the next call."""
    from kernels.colbert_head import colbert_head
    x = _rand((200, 768), torch.bfloat16, 161)
    w = _rand((128, 768), torch.bfloat16, 162, 0.05)
    lw = (1 + 0.1 * _rand((768,), torch.float32, 163)).bfloat16()
    wd, lwd = w.to(dev), lw.to(dev)
    got1 = colbert_head(x.to(dev), wd, None, lwd)
    _colbert_rows_close(got1, oe.colbert_head(x, [(w, None, None, False)], lw, None, 1e-5), "before")
    lwd.mul_(torch.linspace(0.5, 1.5, 768, device=dev).bfloat16())
    got2 = colbert_head(x.to(dev), wd, None, lwd)
    _colbert_rows_close(got2, oe.colbert_head(x, [(w, None, None, False)], lwd.cpu(), None, 1e-5),
                        "after")


def test_colbert_head_repacks_an_updated_weight(dev):
    """The packed copy is cached per weight tensor and version: an in-place
    update of the weight is seen by the next call."""
    from kernels.colbert_head import colbert_head
    x = _rand((100, 768), torch.bfloat16, 61)
    w = _rand((128, 768), torch.bfloat16, 62, 0.05)
    wd = w.to(dev)
    got1 = colbert_head(x.to(dev), wd)
    _colbert_rows_close(got1, oe.colbert_head(x, [(w, None, None, False)], layer_norm=False), "before")
    delta = _rand((128, 768), torch.bfloat16, 63, 0.05)
    wd.add_(delta.to(dev))
    w2 = wd.cpu()
    got2 = colbert_head(x.to(dev), wd)
    _colbert_rows_close(got2, oe.colbert_head(x, [(w2, None, None, False)], layer_norm=False), "after")


def test_colbert_head_projection_only_with_bias(dev):
    """No LayerNorm (rows projected as given), a bias, and a strided input view."""
    from kernels.colbert_head import colbert_head
    base = _rand((300, 2 * 512), torch.bfloat16, 45)
    x = base[:, 512:]  # row stride 1024
    w = _rand((64, 512), torch.bfloat16, 46, 0.05)
    b = _rand((64,), torch.bfloat16, 47, 0.1)
    want = oe.colbert_head(x, [(w, b, None, False)], layer_norm=False)
    got = colbert_head(x.to(dev), w.to(dev), b.to(dev))
    _colbert_rows_close(got, want, "colbert projection only")


def test_colbert_project_residual_stack(dev):
    """A PyLate stack like the LateOn checkpoint's (768 -> 1536 + residual,
    1536 -> 768 + residual, 768 -> 128): GEMMs, then the fused last layer."""
    from kernels.colbert_head import colbert_project
    g = lambda shape, seed: _rand(shape, torch.bfloat16, seed, 0.03)
    layers = [(g((1536, 768), 51), None, g((1536, 768), 52), True),
              (g((768, 1536), 53), None, g((768, 1536), 54), True),
              (g((128, 768), 55), None, None, False)]
    x = _rand((257, 768), torch.bfloat16, 56)
    want = oe.colbert_head(x, layers, layer_norm=False)
    got = colbert_project(x.to(dev), [tuple(None if t is None else (t.to(dev) if torch.is_tensor(t) else t)
                                            for t in l) for l in layers])
    from _tol import cosine
    got = got.float().cpu()
    # the intermediate GEMM outputs are rounded to bf16 twice per layer
    assert min(cosine(got[i], want[i]) for i in range(257)) >= 0.9995
    torch.testing.assert_close(got.norm(dim=-1), torch.ones(257), atol=5e-3, rtol=0)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 40), (torch.bfloat16, 72),
                                     (torch.bfloat16, 36), (torch.float16, 40),
                                     (torch.float32, 36)])
@pytest.mark.parametrize("table", ["fp32", "same"])
def test_rope_head_dims_outside_chunking(dev, dtype, D, table):
    """Head dims the one-launch q/k kernel does not chunk (D not a multiple of
    16 in 16 bits, of 8 in fp32) still work as in the reference, which takes
    any even D: the drop-ins route them through the general kernel. q as a
    strided view of a fused projection, k contiguous; fp32 tables are used at
    fp32, tables in the input's dtype as given. Every element equals the
    oracle's fp32 result rounded once."""
    from kernels.fused_rope_global import fused_rope_apply, fused_rope_global_apply
    from kernels.fused_rope_local import fused_rope_local_apply
    from oracle.attention import rope_cos_sin
    B, S = 2, 131
    qkv = _rand((B, S, 3, 5, D), dtype, 31)
    k = _rand((B, S, 7, D), dtype, 32)
    cos, sin = rope_cos_sin(torch.arange(S) * 3 + 2, 10000.0, D)
    if table == "same":
        cos, sin = cos.to(dtype), sin.to(dtype)
    q = qkv[:, :, 0]
    for fn in (fused_rope_global_apply, fused_rope_local_apply):
        gq, gk = fn(qkv.to(dev)[:, :, 0], k.to(dev), cos.to(dev), sin.to(dev))
        for got, x in ((gq, q), (gk, k)):
            want = oe.rope_table(x, cos[None], sin[None]).to(dtype)
            assert got.is_contiguous() and got.shape == x.shape
            assert torch.equal(got.cpu(), want), f"{fn.__name__} {dtype} D={D} {table}"
    one = fused_rope_apply(k.to(dev), cos[None].to(dev), sin[None].to(dev))
    assert torch.equal(one.cpu(), oe.rope_table(k, cos[None], sin[None]).to(dtype))


def test_packed_weights_under_inference_mode(dev):
    """Weights built under torch.inference_mode() (as a model loaded and run
    by vLLM has them) through the packed-weight paths, called inside
    inference mode twice: colbert_head (pack=True) and SelfOutput."""
    from kernels.colbert_head import colbert_head
    from kernels.dense_layernorm import SelfOutput
    from oracle.epilogues import dense_residual_layernorm
    from _tol import cosine
    x = _rand((200, 768), torch.bfloat16, 71)
    w = _rand((128, 768), torch.bfloat16, 72, 0.05)
    with torch.inference_mode():
        wd = w.to(dev)
        mod = SelfOutput(768, 768, eps=1e-7, dtype=torch.bfloat16, device=dev)
        mod.dense.weight.copy_(_rand((768, 768), torch.bfloat16, 73, 768 ** -0.5).to(dev))
        mod.dense.bias.copy_(_rand((768,), torch.bfloat16, 74, 0.5).to(dev))
    assert wd.is_inference()
    want = oe.colbert_head(x, [(w, None, None, False)], layer_norm=False)
    r = _rand((200, 768), torch.bfloat16, 75)
    for _ in range(2):
        with torch.inference_mode():
            got = colbert_head(x.to(dev), wd)
            y = mod(x.to(dev), r.to(dev))
        _colbert_rows_close(got, want, "colbert head, inference-mode weight")
        ref = dense_residual_layernorm(x, mod.dense.weight.cpu(), mod.dense.bias.cpu(), r,
                                       mod.LayerNorm.weight.cpu(), mod.LayerNorm.bias.cpu(), 1e-7,
                                       round_dtype=torch.bfloat16)
        err = (y.float().cpu() - ref).abs().max().item()
        assert err <= 6e-2 and cosine(y.float().cpu(), ref) >= 0.9999, err
