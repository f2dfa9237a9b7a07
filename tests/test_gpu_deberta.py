"""GPU parity of DeBERTa disentangled attention (gather form = the reference
interface, fused form = in-kernel c2p/p2c) against the oracle."""
import math

import pytest
import torch

import workloads
from _tol import assert_attn_close
from oracle import attention as oa

pytestmark = pytest.mark.gpu
SM = 1.0 / math.sqrt(192)


def _k():
    from kernels import flash_deberta_attention as m
    return m


def _case(B, H, L, S, dtype, seed, lens=None, scale=0.8):
    g = torch.Generator().manual_seed(seed)
    q, k, v = ((torch.randn(B, H, L, 64, generator=g) * scale).to(dtype) for _ in range(3))
    kr = (torch.randn(H, 2 * S, 64, generator=g) * scale).to(dtype)
    qr = (torch.randn(H, 2 * S, 64, generator=g) * scale).to(dtype)
    if lens is None:
        lens = torch.randint(1, L + 1, (B,), generator=g)
    return q, k, v, kr, qr, torch.as_tensor(lens, dtype=torch.int32)


def _valid_rows(out, lens):
    return [out[b, :, :int(n)] for b, n in enumerate(lens)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("log_bucket", [True, False])
def test_gather_small(dev, dtype, log_bucket):
    q, k, v, kr, qr, lens = _case(2, 3, 200, 64, dtype, 1, lens=[200, 77])
    pk, pq = oa.deberta_position_projections(q, k, kr, qr)
    pk, pq = pk.to(dtype), pq.to(dtype)
    want = oa.deberta_flash_attention(q, k, v, lens, pk, pq, SM, 64, 128, log_bucket)
    got = _k().flash_deberta_attention(q.to(dev), k.to(dev), v.to(dev), lens.to(dev), pk.to(dev),
                                       pq.to(dev), False, SM, 64, 128, log_bucket)
    assert_attn_close(got, want, f"gather {dtype} log={log_bucket}")
    assert torch.all(got[1, :, 77:] == 0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gather_causal_and_partial_projections(dev, dtype):
    q, k, v, kr, qr, lens = _case(2, 2, 150, 32, dtype, 2, lens=[150, 150])
    pk, pq = oa.deberta_position_projections(q, k, kr, qr)
    pk = pk.to(dtype)
    want = oa.deberta_flash_attention(q, k, v, None, pk, None, SM, 32, 64, True, causal=True)
    got = _k().flash_deberta_attention(q.to(dev), k.to(dev), v.to(dev), None, pk.to(dev), None,
                                       True, SM, 32, 64, True)
    assert_attn_close(got, want, f"causal c2p-only {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_fused_small(dev, dtype):
    for lens in ([200, 77, 1, 64], [129, 128, 65, 190]):
        q, k, v, kr, qr, ln = _case(4, 2, 200, 256, dtype, 3, lens=lens)
        pk, pq = oa.deberta_position_projections(q, k, kr, qr)
        want = oa.deberta_flash_attention(q, k, v, ln, pk, pq, SM, 256, 512, True)
        got = _k().flash_deberta_attention_fused(q.to(dev), k.to(dev), v.to(dev), ln.to(dev),
                                                 kr.to(dev), qr.to(dev), SM, 256, 512, True)
        for b, n in enumerate(lens):
            assert_attn_close(got[b, :, :n], want[b, :, :n], f"fused {dtype} lens={lens} b={b}")
        assert torch.all(got[2, :, lens[2]:] == 0)


def test_fused_config3_all_sequences(dev):
    """DeBERTa-v3-large at config 3 (B = 32, L = 512, 256 buckets,
    max_relative_positions 512): every valid row of all 32 sequences of the
    fused kernel against the oracle (four batch rows per oracle call), rows
    past each length zero."""
    c = workloads.config3(device=dev)
    got = _k().flash_deberta_attention_fused(c.q, c.k, c.v, c.lengths, c.key_rel, c.query_rel,
                                             c.sm_scale, 256, 512, True).cpu()
    q, k, v, kr, qr = (t.cpu() for t in (c.q, c.k, c.v, c.key_rel, c.query_rel))
    lens = c.lengths.cpu()
    worst = 0.0
    for b0 in range(0, q.shape[0], 4):
        sl = slice(b0, b0 + 4)
        pk, pq = oa.deberta_position_projections(q[sl], k[sl], kr, qr)
        want = oa.deberta_flash_attention(q[sl], k[sl], v[sl], lens[sl], pk, pq, c.sm_scale,
                                          256, 512, True)
        for i in range(want.shape[0]):
            n = int(lens[b0 + i])
            err, _ = assert_attn_close(got[b0 + i, :, :n], want[i, :, :n], f"cfg3 b={b0 + i}")
            worst = max(worst, err)
            assert torch.all(got[b0 + i, :, n:] == 0)
    print(f"config 3 fused: {q.shape[0]} sequences, max-abs {worst:.3e}")


def test_fused_equals_gather_full_config3(dev):
    """All of config 3: the fused kernel and the gather kernel fed with the
    device-computed projections agree (size-independent consistency)."""
    c = workloads.config3(device=dev)
    pk = torch.matmul(c.q, c.key_rel.unsqueeze(0).transpose(-1, -2).contiguous())
    pq = torch.matmul(c.k, c.query_rel.unsqueeze(0).transpose(-1, -2).contiguous())
    a = _k().flash_deberta_attention(c.q, c.k, c.v, c.lengths, pk, pq, False, c.sm_scale, 256, 512, True)
    b = _k().flash_deberta_attention_fused(c.q, c.k, c.v, c.lengths, c.key_rel, c.query_rel,
                                           c.sm_scale, 256, 512, True)
    for i, n in enumerate(c.lengths.tolist()):
        assert_attn_close(b[i, :, :n], a[i, :, :n], f"fused vs gather b={i}")
        assert torch.all(b[i, :, n:] == 0) and torch.all(a[i, :, n:] == 0)


def test_zero_length_rows(dev):
    q, k, v, kr, qr, lens = _case(2, 2, 70, 64, torch.bfloat16, 5, lens=[0, 70])
    got = _k().flash_deberta_attention_fused(q.to(dev), k.to(dev), v.to(dev), lens.to(dev),
                                             kr.to(dev), qr.to(dev), SM, 64, 128, True)
    assert torch.all(got[0] == 0)
    pk, pq = oa.deberta_position_projections(q, k, kr, qr)
    want = oa.deberta_flash_attention(q, k, v, lens, pk, pq, SM, 64, 128, True)
    assert_attn_close(got[1], want[1], "zero-length batch row")


@pytest.mark.parametrize("which", ["c2p", "p2c", "none"])
def test_fused_partial_projections_linear_buckets(dev, which):
    """One or neither position projection, linear buckets clamped at +-S
    (L = 200 > S = 64)."""
    q, k, v, kr, qr, lens = _case(3, 2, 200, 64, torch.bfloat16, 7, lens=[200, 130, 63])
    pk, pq = oa.deberta_position_projections(q, k, kr, qr)
    pk = pk if which == "c2p" else None
    pq = pq if which == "p2c" else None
    want = oa.deberta_flash_attention(q, k, v, lens, pk, pq, SM, 64, 128, False)
    got = _k().flash_deberta_attention_fused(
        q.to(dev), k.to(dev), v.to(dev), lens.to(dev), kr.to(dev) if which == "c2p" else None,
        qr.to(dev) if which == "p2c" else None, SM, 64, 128, False)
    for b, n in enumerate(lens.tolist()):
        assert_attn_close(got[b, :, :n], want[b, :, :n], f"fused {which} b={b}")
        assert torch.all(got[b, :, n:] == 0)


def test_fused_strided_views_and_out(dev):
    """q/k/v as head-transposed views of one [B, L, 3, H, 64] projection,
    key_rel / query_rel as views of one [2S, 2, H, 64] projection, and the
    output written in place into a [B, L, H, 64] buffer."""
    B, L, H, S = 2, 150, 3, 64
    g = torch.Generator().manual_seed(8)
    qkv = (torch.randn(B, L, 3, H, 64, generator=g) * 0.8).to(torch.bfloat16)
    rel = (torch.randn(2 * S, 2, H, 64, generator=g) * 0.8).to(torch.bfloat16)
    lens = torch.tensor([150, 91], dtype=torch.int32)
    qd, reld = qkv.to(dev), rel.to(dev)
    buf = torch.full((B, L, H, 64), float("nan"), dtype=torch.bfloat16, device=dev)
    got = _k().flash_deberta_attention_fused(
        qd[:, :, 0].transpose(1, 2), qd[:, :, 1].transpose(1, 2), qd[:, :, 2].transpose(1, 2),
        lens.to(dev), reld[:, 1].transpose(0, 1), reld[:, 0].transpose(0, 1), SM, S, 128, True,
        out=buf.transpose(1, 2))
    assert got.data_ptr() == buf.data_ptr()
    q, k, v = (qkv[:, :, i].transpose(1, 2).contiguous() for i in range(3))
    kr, qr = rel[:, 1].transpose(0, 1).contiguous(), rel[:, 0].transpose(0, 1).contiguous()
    pk, pq = oa.deberta_position_projections(q, k, kr, qr)
    want = oa.deberta_flash_attention(q, k, v, lens, pk, pq, SM, S, 128, True)
    for b, n in enumerate(lens.tolist()):
        assert_attn_close(got[b, :, :n], want[b, :, :n], f"strided b={b}")
        assert torch.all(buf[b, n:] == 0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("log_bucket", [True, False])
def test_gather_staged_vs_oracle(dev, dtype, log_bucket):
    """Row-contiguous pos tensors with 2S >= 136 take the LDS-staged gather:
    partial query and key tiles (L = 300), a short sequence, windows clamped at
    both ends of the 2S columns (S = 128 < L)."""
    q, k, v, kr, qr, lens = _case(2, 3, 300, 128, dtype, 6, lens=[300, 77])
    pk, pq = oa.deberta_position_projections(q, k, kr, qr)
    pk, pq = pk.to(dtype), pq.to(dtype)
    want = oa.deberta_flash_attention(q, k, v, lens, pk, pq, SM, 128, 256, log_bucket)
    print(f"deberta staged gather {dtype} log={log_bucket}", flush=True)
    got = _k().flash_deberta_attention(q.to(dev), k.to(dev), v.to(dev), lens.to(dev), pk.to(dev),
                                       pq.to(dev), False, SM, 128, 256, log_bucket)
    assert_attn_close(got[0], want[0], f"staged {dtype} log={log_bucket} b=0")
    assert_attn_close(got[1, :, :77], want[1, :, :77], f"staged {dtype} log={log_bucket} b=1")
    assert torch.all(got[1, :, 77:] == 0)


@pytest.mark.parametrize("which", ["both", "c2p", "p2c"])
def test_gather_staged_equals_unstaged(dev, which):
    """The staged and the per-score gather read the same bias values in the
    same order: bit-equal outputs, with both pos tensors or only one of them
    (pos_att_type c2p or p2c alone). Pos tensors viewed out of [.., 2S + 1]
    buffers (row stride not a multiple of 8) take the per-score gather."""
    q, k, v, kr, qr, lens = _case(3, 2, 384, 256, torch.bfloat16, 7, lens=[384, 200, 5])
    pk, pq = oa.deberta_position_projections(q, k, kr, qr)
    pk, pq = pk.bfloat16().to(dev), pq.bfloat16().to(dev)
    wide = lambda t: torch.cat([t, t[..., :1]], -1)[..., :t.shape[-1]]
    pk_w, pq_w = wide(pk), wide(pq)
    assert pk_w.stride(2) % 8 != 0
    args = (q.to(dev), k.to(dev), v.to(dev), lens.to(dev))
    if which == "c2p":
        pq = pq_w = None
    if which == "p2c":
        pk = pk_w = None
    print(f"deberta staged vs unstaged ({which})", flush=True)
    a = _k().flash_deberta_attention(*args, pk, pq, False, SM, 256, 512, True)
    b = _k().flash_deberta_attention(*args, pk_w, pq_w, False, SM, 256, 512, True)
    assert torch.equal(a, b)


def test_gather_staged_causal(dev):
    q, k, v, kr, qr, lens = _case(2, 2, 260, 96, torch.bfloat16, 8, lens=[260, 260])
    pk, pq = oa.deberta_position_projections(q, k, kr, qr)
    pk, pq = pk.bfloat16(), pq.bfloat16()
    want = oa.deberta_flash_attention(q, k, v, None, pk, pq, SM, 96, 192, True, causal=True)
    print("deberta staged causal", flush=True)
    got = _k().flash_deberta_attention(q.to(dev), k.to(dev), v.to(dev), None, pk.to(dev),
                                       pq.to(dev), True, SM, 96, 192, True)
    assert_attn_close(got, want, "staged causal")


def test_gather_staged_c2p_only_vs_oracle(dev):
    q, k, v, kr, qr, lens = _case(2, 2, 200, 128, torch.bfloat16, 9, lens=[200, 131])
    pk, _ = oa.deberta_position_projections(q, k, kr, qr)
    pk = pk.bfloat16()
    want = oa.deberta_flash_attention(q, k, v, lens, pk, None, SM, 128, 256, True)
    print("deberta staged c2p only", flush=True)
    got = _k().flash_deberta_attention(q.to(dev), k.to(dev), v.to(dev), lens.to(dev), pk.to(dev),
                                       None, False, SM, 128, 256, True)
    assert_attn_close(got[0], want[0], "staged c2p-only b=0")
    assert_attn_close(got[1, :, :131], want[1, :, :131], "staged c2p-only b=1")


@pytest.mark.parametrize("log_bucket", [True, False])
def test_fused_varlen_equals_padded_call(dev, log_bucket):
    """flash_deberta_attention_varlen on packed [T, H, 64] rows (strided views
    of a [T, 3, H, 64] projection) against the padded fused call with
    seq_lengths on the same sequences: the kernel runs the same tiles in the
    same order, so every valid row is equal bit for bit; and against the
    oracle at the attention tolerance. Lengths 512, 1, 0, 300 and 130 cover
    one-token and empty sequences and partial tiles."""
    lens = [512, 1, 0, 300, 130]
    B, H, S, L = len(lens), 4, 256, max(lens)
    q, k, v, kr, qr, ln = _case(B, H, L, S, torch.bfloat16, 77, lens=lens)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    qkv = torch.stack([torch.cat([t[b, :, :n].transpose(0, 1) for b, n in enumerate(lens)])
                       for t in (q, k, v)], 1)                      # [T, 3, H, 64]
    print(f"deberta varlen log={log_bucket} lens {lens}", flush=True)
    qd = qkv.to(dev)
    got = _k().flash_deberta_attention_varlen(qd[:, 0], qd[:, 1], qd[:, 2], cu.to(dev), L, kr.to(dev),
                                              qr.to(dev), SM, S, 512, log_bucket).cpu()
    pad = _k().flash_deberta_attention_fused(q.to(dev), k.to(dev), v.to(dev), ln.to(dev), kr.to(dev),
                                             qr.to(dev), SM, S, 512, log_bucket).cpu()
    pk, pq = oa.deberta_position_projections(q, k, kr, qr)
    want = oa.deberta_flash_attention(q, k, v, ln, pk, pq, SM, S, 512, log_bucket)
    for b, n in enumerate(lens):
        if n == 0:
            continue
        a = int(cu[b])
        gb = got[a:a + n].transpose(0, 1)
        assert torch.equal(gb, pad[b, :, :n]), f"sequence {b}"
        assert_attn_close(gb, want[b, :, :n], f"varlen b={b}")


@pytest.mark.parametrize("present", ["both", "key", "query"])
def test_rel_chunk_major_kernel_equals_torch_layout(dev, present):
    """vfk_deberta_rel_chunk_major (the calls' one-launch conversion) writes
    exactly rel_chunk_major's layout, from strided views of one [2S, 2, H,
    64] projection with extra rows past 2S, bit for bit."""
    from kernels import _lib
    S, H = 256, 16
    g = torch.Generator().manual_seed(12)
    pr = torch.randn(2 * S + 8, 2, H, 64, generator=g).to(torch.bfloat16).to(dev)
    qrel, krel = pr[:, 0].transpose(0, 1), pr[:, 1].transpose(0, 1)   # [H, 2S + 8, 64] views
    kr = krel if present != "query" else None
    qr = qrel if present != "key" else None
    out = [torch.full((H, 8, 2 * S, 8), 7.0, dtype=torch.bfloat16, device=dev) if t is not None else None
           for t in (kr, qr)]
    _lib.on_device("vfk_deberta_rel_chunk_major", dev, _lib.ref(_lib.desc(kr)), _lib.ref(_lib.desc(out[0])),
                   _lib.ref(_lib.desc(qr)), _lib.ref(_lib.desc(out[1])), S)
    for t, o in zip((kr, qr), out):
        if t is not None:
            assert torch.equal(o, _k().rel_chunk_major(t, S))


@pytest.mark.parametrize("which", ["both", "c2p", "p2c"])
@pytest.mark.parametrize("log_bucket", [True, False])
def test_chunk_major_tables_equal_row_tables(dev, which, log_bucket):
    """The fused kernels read key_rel / query_rel either as [H, 2S, 64] rows
    or in the chunk-major layout [H, 8, 2S, 8]: the same products in the same
    order, so the outputs are equal bit for bit (padded and packed calls),
    including windows that run past the table's last row."""
    lens = [300, 77, 512]
    B, H, S, L = len(lens), 3, 256, max(lens)
    q, k, v, kr, qr, ln = _case(B, H, L, S, torch.bfloat16, 91, lens=lens)
    kr = kr if which != "p2c" else None
    qr = qr if which != "c2p" else None
    mv = lambda t: t.to(dev) if t is not None else None
    print(f"deberta chunk-major {which} log={log_bucket}", flush=True)
    rows = _k().flash_deberta_attention_fused(q.to(dev), k.to(dev), v.to(dev), ln.to(dev), mv(kr), mv(qr),
                                              SM, S, 512, log_bucket, chunk_major=False)
    cm = lambda t: _k().rel_chunk_major(t.to(dev), S) if t is not None else None
    chunk = _k().flash_deberta_attention_fused(q.to(dev), k.to(dev), v.to(dev), ln.to(dev), cm(kr), cm(qr),
                                               SM, S, 512, log_bucket)
    assert torch.equal(rows, chunk)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    qkv = torch.stack([torch.cat([t[b, :, :n].transpose(0, 1) for b, n in enumerate(lens)])
                       for t in (q, k, v)], 1).to(dev)
    vr = _k().flash_deberta_attention_varlen(qkv[:, 0], qkv[:, 1], qkv[:, 2], cu.to(dev), L, mv(kr), mv(qr),
                                             SM, S, 512, log_bucket, chunk_major=False)
    vc = _k().flash_deberta_attention_varlen(qkv[:, 0], qkv[:, 1], qkv[:, 2], cu.to(dev), L, cm(kr), cm(qr),
                                             SM, S, 512, log_bucket)
    assert torch.equal(vr, vc)
