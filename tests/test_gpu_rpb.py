"""GPU parity of T5 relative-position-bias attention (flash_attention_rpb_final)
against the oracle restatement of the reference's eager path."""
import pytest
import torch

import workloads
from _tol import assert_attn_close
from oracle import attention as oa
from oracle import buckets as ob

pytestmark = pytest.mark.gpu


def _rpb():
    from kernels.flash_attention_rpb import flash_attention_rpb_final
    return flash_attention_rpb_final


def test_config1_fp32(dev):
    """Config 1 (the CPU plumbing check) on the GPU in fp32."""
    c = workloads.config1()
    want = oa.rpb_attention(c.q, c.k, c.v, c.table, 32, 128, False, c.mask, 1.0)
    got = _rpb()(c.q.to(dev), c.k.to(dev), c.v.to(dev), c.table.to(dev), 32, 128, False,
                 padding_mask=c.mask.to(dev), softmax_scale=1.0)
    assert got.dtype == torch.float32 and got.shape == c.q.shape
    assert_attn_close(got, want, "cfg1 fp32", max_abs=1e-4, cos=0.999999)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_config1_16bit(dev, dtype):
    c = workloads.config1()
    q, k, v = (t.to(dtype) for t in (c.q, c.k, c.v))
    mask = c.mask.clamp(min=torch.finfo(dtype).min).to(dtype)
    want = oa.rpb_attention(q, k, v, c.table, 32, 128, False, mask, 1.0)
    got = _rpb()(q.to(dev), k.to(dev), v.to(dev), c.table.to(dev), 32, 128, False,
                 padding_mask=mask.to(dev))
    assert got.dtype == dtype
    assert_attn_close(got, want, f"cfg1 {dtype}")


def test_config4_attention_all_sequences(dev):
    """Config 4 (mT5-large, B = 32, L = 768, lengths U{512..768}): q, k, v
    projected from the config's hidden states and Wq / Wk / Wv, the config's
    [32, 16] table and [B, 1, 1, L] key mask; every valid row of all 32
    sequences against the oracle (four batch rows per oracle call)."""
    c = workloads.config4(device=dev)
    B, L, D = c.hidden.shape
    H = c.table.shape[1]
    q, k, v = ((c.hidden @ w).view(B, L, H, 64).transpose(1, 2) for w in (c.wq, c.wk, c.wv))
    got = _rpb()(q, k, v, c.table, 32, 128, False, padding_mask=c.mask).cpu()
    table, mask = c.table.cpu(), c.mask.cpu()
    worst = 0.0
    for b0 in range(0, B, 4):
        sl = slice(b0, b0 + 4)
        want = oa.rpb_attention(q[sl].cpu(), k[sl].cpu(), v[sl].cpu(), table, 32, 128, False,
                                mask[sl], 1.0)
        for i in range(want.shape[0]):
            n = int(c.lengths[b0 + i])
            err, _ = assert_attn_close(got[b0 + i, :, :n], want[i, :, :n], f"cfg4 batch {b0 + i}")
            worst = max(worst, err)
    print(f"config 4: {B} sequences, max-abs {worst:.3e}")


def test_config4_full_size_properties(dev):
    """All 32 x 768 rows at full size: V = 1 gives 1 on every row, and a
    batch permutation permutes the output (size-independent checks)."""
    c = workloads.config4(device=dev)
    B, L = c.hidden.shape[:2]
    g = torch.Generator().manual_seed(44)
    q = (torch.randn(B, 16, L, 64, generator=g) * 0.64).bfloat16().to(dev)
    k = (torch.randn(B, 16, L, 64, generator=g) * 0.64).bfloat16().to(dev)
    ones = torch.ones(B, 16, L, 64, dtype=torch.bfloat16, device=dev)
    out = _rpb()(q, k, ones, c.table, 32, 128, False, padding_mask=c.mask)
    assert torch.allclose(out.float(), torch.ones_like(out, dtype=torch.float32), atol=1e-2)
    v = torch.randn(B, 16, L, 64, generator=g).bfloat16().to(dev)
    o1 = _rpb()(q, k, v, c.table, 32, 128, False, padding_mask=c.mask)
    perm = torch.randperm(B, generator=g).to(dev)
    o2 = _rpb()(q[perm], k[perm], v[perm], c.table, 32, 128, False, padding_mask=c.mask[perm])
    assert torch.equal(o1[perm], o2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_causal_decoder(dev, dtype):
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(2, 4, 200, 64, generator=g).to(dtype) for _ in range(3))
    table = torch.randn(32, 4, generator=g) * 0.1
    want = oa.rpb_attention(q, k, v, table, 32, 128, True, None, 0.125)
    got = _rpb()(q.to(dev), k.to(dev), v.to(dev), table.to(dev), 32, 128, True,
                 softmax_scale=0.125)
    assert_attn_close(got, want, f"causal {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_no_table_full_mask_cross_lengths(dev, dtype):
    """rpb_table=None, a per-query 4-D mask, Lq != Lk."""
    g = torch.Generator().manual_seed(6)
    q = torch.randn(2, 3, 130, 64, generator=g).to(dtype)
    k = torch.randn(2, 3, 70, 64, generator=g).to(dtype)
    v = torch.randn(2, 3, 70, 64, generator=g).to(dtype)
    mask = torch.randn(2, 1, 130, 70, generator=g).to(dtype)
    want = oa.rpb_attention(q, k, v, None, 32, 128, False, mask, 0.125)
    got = _rpb()(q.to(dev), k.to(dev), v.to(dev), None, 32, 128, False,
                 padding_mask=mask.to(dev), softmax_scale=0.125)
    assert_attn_close(got, want, f"no-table {dtype}")


def test_strided_inputs(dev):
    """[B, L, H, D] projections viewed as [B, H, L, D] (transpose, no copy)."""
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 300, 3, 8, 64, generator=g).bfloat16()
    q, k, v = (x[:, :, i].transpose(1, 2) for i in range(3))
    table = torch.randn(32, 8, generator=g) * 0.1
    want = oa.rpb_attention(q, k, v, table, 32, 128, False, None, 0.3)
    xd = x.to(dev)
    qd, kd, vd = (xd[:, :, i].transpose(1, 2) for i in range(3))
    got = _rpb()(qd, kd, vd, table.to(dev), 32, 128, False, softmax_scale=0.3)
    assert_attn_close(got, want, "strided")


@pytest.mark.parametrize("case", ["overflow", "underflow", "mixed"])
@pytest.mark.parametrize("masked", [False, True])
def test_fixed_pass_fallback(dev, case, masked):
    """The bf16 kernel first takes p = exp2(c s) without a running max, and
    runs a workgroup again with it where a row sum or output is not finite or
    below 2^-64. Cases that need the second run: scores that overflow 2^127
    (q = k, |q|^2 ~ 1000), scores all far below 0 (a table of -300), and a
    batch where only the second row's items overflow; with and without a key
    mask (the two kernels that take the first pass)."""
    g = torch.Generator().manual_seed(11)
    B, H, L = 2, 3, 200
    q = torch.randn(B, H, L, 64, generator=g) * 0.5
    k = torch.randn(B, H, L, 64, generator=g) * 0.5
    v = torch.randn(B, H, L, 64, generator=g)
    table = torch.randn(32, H, generator=g) * 0.1
    if case == "overflow":
        q = torch.randn(B, H, L, 64, generator=g) * 4.0
        k = q.clone()
    elif case == "underflow":
        table = torch.full((32, H), -300.0)
    else:
        q[1] = torch.randn(H, L, 64, generator=g) * 4.0
        k[1] = q[1]
    q, k, v = (t.bfloat16() for t in (q, k, v))
    mask = None
    if masked:
        mask = torch.zeros(B, 1, 1, L)
        mask[:, :, :, 170:] = torch.finfo(torch.float32).min
    want = oa.rpb_attention(q, k, v, table, 32, 128, False, mask, 1.0)
    got = _rpb()(q.to(dev), k.to(dev), v.to(dev), table.to(dev), 32, 128, False,
                 padding_mask=None if mask is None else mask.to(dev))
    assert torch.isfinite(got.float()).all(), f"{case}: non-finite output"
    assert_attn_close(got, want, f"fallback {case} masked={masked}")


def test_all_keys_masked_row_is_uniform(dev):
    """A batch row whose keys are all masked averages V uniformly, as the
    reference's finite additive mask does."""
    g = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(2, 2, 96, 64, generator=g).bfloat16() for _ in range(3))
    mask = torch.zeros(2, 1, 1, 96)
    mask[1] = torch.finfo(torch.float32).min
    want = oa.rpb_attention(q, k, v, None, 32, 128, False, mask, 1.0)
    got = _rpb()(q.to(dev), k.to(dev), v.to(dev), None, 32, 128, False,
                 padding_mask=mask.to(dev))
    assert_attn_close(got, want, "all-masked")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("bidirectional", [True, False])
def test_device_buckets_exact(dev, dtype, bidirectional):
    """Recovers the device's bucket of every (query, key) pair: q = k = 0, V
    one-hot per key and a table with a single hot bucket give
    out[q, j] > 0 exactly when bucket(j - q) is the hot bucket."""
    Lq, Lk, H = 256, 64, 1
    want = ob.t5_bucket_matrix(Lq, Lk, bidirectional, 32, 128)
    z = torch.zeros(1, H, Lq, 64, dtype=dtype, device=dev)
    zk = torch.zeros(1, H, Lk, 64, dtype=dtype, device=dev)
    v = torch.eye(64, dtype=dtype, device=dev)[None, None]
    for hot in range(32):
        table = torch.zeros(32, H, device=dev)
        table[hot] = 80.0
        out = _rpb()(z, zk, v, table, 32, 128, not bidirectional)
        member = (want == hot)
        if not bidirectional:
            member &= torch.arange(Lk)[None, :] <= torch.arange(Lq)[:, None]
        rows = member.any(dim=1)
        got = out[0, 0].float().cpu() > 1e-3
        assert torch.equal(got[rows], member[rows]), f"bucket {hot}"


@pytest.mark.parametrize("lens", [[768, 512, 700, 601], [1, 130, 0, 257, 64]])
def test_varlen_matches_padded_call_and_oracle(dev, lens):
    """flash_attention_rpb_varlen on packed [T, H, 64] rows (a view of a fused
    [T, 3, H, 64] projection, so strided) against the padded call with the
    reference's [B, 1, 1, L] key mask on the same sequences: the kernel runs
    the same tiles in the same order and masked keys contribute exact zeros,
    so the valid rows are equal bit for bit; and against the oracle at the
    attention tolerance. Includes an empty and a one-token sequence and
    lengths that are not tile multiples."""
    from kernels.flash_attention_rpb import flash_attention_rpb_varlen
    g = torch.Generator().manual_seed(sum(lens))
    B, H, L = len(lens), 16, max(lens)
    T = sum(lens)
    qkv = (torch.randn(T, 3, H, 64, generator=g) * 0.64).bfloat16()
    table = (torch.randn(32, H, generator=g) * 0.1).bfloat16()
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    pad = torch.zeros(B, L, 3, H, 64, dtype=torch.bfloat16)
    for b in range(B):
        pad[b, :lens[b]] = qkv[int(cu[b]):int(cu[b + 1])]
    q, k, v = (pad[:, :, i].transpose(1, 2) for i in range(3))      # [B, H, L, 64]
    keep = (torch.arange(L)[None] < torch.tensor(lens)[:, None]).bfloat16()
    mask = ((1.0 - keep) * torch.finfo(torch.bfloat16).min)[:, None, None, :]
    print(f"rpb varlen lens {lens}", flush=True)
    qd = qkv.to(dev)
    got = flash_attention_rpb_varlen(qd[:, 0], qd[:, 1], qd[:, 2], cu.to(dev), L, table.to(dev),
                                     32, 128).cpu()
    padded = _rpb()(q.contiguous().to(dev), k.contiguous().to(dev), v.contiguous().to(dev),
                    table.to(dev), 32, 128, False, padding_mask=mask.to(dev)).cpu()
    want = oa.rpb_attention(q, k, v, table, 32, 128, False, mask, 1.0)
    for b in range(B):
        a, e = int(cu[b]), int(cu[b + 1])
        if e == a:
            continue
        gb = got[a:e].transpose(0, 1)                                 # [H, n, 64]
        assert torch.equal(gb, padded[b, :, :e - a]), f"sequence {b}"
        assert_attn_close(gb, want[b, :, :e - a], f"varlen seq {b}")
