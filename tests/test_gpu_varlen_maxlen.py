"""Packed sequences longer than the max_seqlen a caller passes.

The varlen entry points (ModernBERT varlen attention, RPB varlen, DeBERTa
varlen) size their grids and tables by max_seqlen. A sequence longer than it
is cut there: its first max_seqlen rows attend among themselves, and its rows
past max_seqlen are written as zeros (never left as whatever torch.empty
held). The other sequences of the pack are unaffected. Each case checks the
kept rows against the oracle on the cut pack, the cut rows for exact zeros,
and the output buffer starts as NaN so that an unwritten row shows.
"""
import math

import pytest
import torch

from _tol import assert_attn_close
from oracle import attention as oa

pytestmark = pytest.mark.gpu

LENS = [300, 517, 64, 401]
MAXLEN = 400


def _pack(H, seed, scale=0.7, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    T = sum(LENS)
    qkv = (torch.randn(T, 3, H, 64, generator=g) * scale).to(dtype)
    cu = torch.tensor([0] + torch.tensor(LENS).cumsum(0).tolist(), dtype=torch.int32)
    return qkv, cu


def _cut(qkv, cu):
    """The pack with every sequence cut at MAXLEN rows, and its cu_seqlens."""
    rows, lens = [], []
    for b in range(len(LENS)):
        a = int(cu[b])
        n = min(LENS[b], MAXLEN)
        rows.append(qkv[a:a + n])
        lens.append(n)
    cut_cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    return torch.cat(rows), cut_cu


def _check(got, want_cut, cu, cut_cu, what):
    got = got.cpu()
    for b in range(len(LENS)):
        a, n = int(cu[b]), min(LENS[b], MAXLEN)
        ca = int(cut_cu[b])
        assert_attn_close(got[a:a + n], want_cut[ca:ca + n], f"{what} seq {b}")
        if LENS[b] > MAXLEN:
            assert torch.all(got[a + n:a + LENS[b]] == 0), f"{what} seq {b}: rows past max_seqlen"


@pytest.mark.parametrize("window,theta,dtype", [(-1, 160000.0, torch.bfloat16),
                                                (64, 10000.0, torch.bfloat16),
                                                (-1, 0.0, torch.bfloat16),
                                                (64, 10000.0, torch.float32)])
def test_modernbert_varlen_cut_at_max_seqlen(dev, window, theta, dtype):
    from kernels.varlen_attention import varlen_rope_attention
    qkv, cu = _pack(12, 41, dtype=dtype)
    out = torch.full(qkv[:, 0].shape, float("nan"), dtype=dtype, device=dev)
    qd = qkv.to(dev)
    got = varlen_rope_attention(qd[:, 0], qd[:, 1], qd[:, 2], cu.to(dev), MAXLEN, window=window,
                                rope_theta=theta, softmax_scale=0.125, out=out)
    cut, cut_cu = _cut(qkv, cu)
    want = oa.varlen_attention(cut[:, 0], cut[:, 1], cut[:, 2], cut_cu, window=window,
                               rope_theta=theta, softmax_scale=0.125)
    _check(got, want, cu, cut_cu, f"varlen w={window} theta={theta} {dtype}")


@pytest.mark.parametrize("H", [1, 3, 16, 20, 24])
@pytest.mark.parametrize("window,theta", [(-1, 160000.0), (64, 10000.0)])
def test_modernbert_varlen_head_counts(dev, H, window, theta):
    """Head counts other than 12 through the K pre-pass's head groups: 4 head
    pairs per block for 16, 6 for the others, two groups for 16, 20 (the
    second clamped at the last head) and 24, one partly filled group for 1 and
    3; the cut rows of every head are zeroed by its group's blocks."""
    from kernels.varlen_attention import varlen_rope_attention
    qkv, cu = _pack(H, 60 + H)
    out = torch.full(qkv[:, 0].shape, float("nan"), dtype=qkv.dtype, device=dev)
    qd = qkv.to(dev)
    print(f"head counts H={H} window={window}", flush=True)
    got = varlen_rope_attention(qd[:, 0], qd[:, 1], qd[:, 2], cu.to(dev), MAXLEN, window=window,
                                rope_theta=theta, softmax_scale=0.125, out=out)
    cut, cut_cu = _cut(qkv, cu)
    want = oa.varlen_attention(cut[:, 0], cut[:, 1], cut[:, 2], cut_cu, window=window,
                               rope_theta=theta, softmax_scale=0.125)
    _check(got, want, cu, cut_cu, f"varlen H={H} w={window}")


def test_rpb_varlen_cut_at_max_seqlen(dev):
    from kernels.flash_attention_rpb import flash_attention_rpb_varlen
    H = 8
    qkv, cu = _pack(H, 42)
    table = (torch.randn(32, H, generator=torch.Generator().manual_seed(43)) * 0.1).bfloat16()
    qd = qkv.to(dev)
    got = flash_attention_rpb_varlen(qd[:, 0], qd[:, 1], qd[:, 2], cu.to(dev), MAXLEN,
                                     table.to(dev), 32, 128)
    cut, cut_cu = _cut(qkv, cu)
    want = torch.empty(cut.shape[0], H, 64)
    for b in range(len(LENS)):
        a, e = int(cut_cu[b]), int(cut_cu[b + 1])
        q, k, v = (cut[a:e, i].transpose(0, 1)[None] for i in range(3))   # [1, H, n, 64]
        want[a:e] = oa.rpb_attention(q, k, v, table, 32, 128, False)[0].transpose(0, 1)
    _check(got, want, cu, cut_cu, "rpb varlen")


def test_deberta_varlen_cut_at_max_seqlen(dev):
    from kernels.flash_deberta_attention import flash_deberta_attention_varlen
    H, S = 4, 256
    qkv, cu = _pack(H, 44, scale=0.8)
    g = torch.Generator().manual_seed(45)
    kr = (torch.randn(H, 2 * S, 64, generator=g) * 0.8).bfloat16()
    qr = (torch.randn(H, 2 * S, 64, generator=g) * 0.8).bfloat16()
    sm = 1.0 / math.sqrt(192)
    qd = qkv.to(dev)
    got = flash_deberta_attention_varlen(qd[:, 0], qd[:, 1], qd[:, 2], cu.to(dev), MAXLEN,
                                         kr.to(dev), qr.to(dev), sm, S, 512, True)
    cut, cut_cu = _cut(qkv, cu)
    want = torch.empty(cut.shape[0], H, 64)
    for b in range(len(LENS)):
        a, e = int(cut_cu[b]), int(cut_cu[b + 1])
        q, k, v = (cut[a:e, i].transpose(0, 1)[None] for i in range(3))
        pk, pq = oa.deberta_position_projections(q, k, kr, qr)
        want[a:e] = oa.deberta_flash_attention(q, k, v, None, pk, pq, sm, S, 512, True)[0].transpose(0, 1)
    _check(got, want, cu, cut_cu, "deberta varlen")
