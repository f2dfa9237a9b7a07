"""The DeBERTa drop-in fed exactly what the reference's models build.

models/deberta_v2/deberta_v2_encoder.py:246-328 (`_flash_forward`, v2/v3) and
models/deberta/deberta_encoder.py:246-307 (v1) build the inputs of
`flash_deberta_attention` from the layer's projections: q/k/v as head views
[B, H, L, 64] of the [B, L, H*64] projection outputs (not contiguous),
pos_key = q @ key_proj(rel_emb)^T and pos_query = k @ query_proj(rel_emb)^T
as batched matmul outputs [B, H, L, 2S], seq_lengths from row 0 of the
[B, 1, L, L] mask that `get_attention_mask` (deberta_v2_encoder.py:776-782)
makes, and the bucket settings of the layer. These tests rebuild those
tensors the same way and check every valid row of the kernel's output
against the oracle (max-abs <= 2e-2, cosine >= 0.9999 against fp32), and
that rows past each length are zero.

The one departure from the callers: the transposed right operand of each
bf16 batched matmul is made contiguous first (a batched bf16 product over a
transposed view is avoided on this GPU); the product is the same.
"""
import math

import pytest
import torch
import torch.nn.functional as F

import workloads
from _tol import assert_attn_close
from oracle import attention as oa

pytestmark = pytest.mark.gpu


def _heads(x, H):
    """(B, L, H*64) -> (B, H, L, 64) view, as `_transpose_4d` / `transpose_for_scores`."""
    return x.view(*x.shape[:-1], H, -1).permute(0, 2, 1, 3)


def _mask_seq_lengths(lens, L, dev):
    """get_attention_mask of a 2-D 0/1 mask, then `_flash_forward`'s
    seq_lengths = attention_mask[:, 0, 0, :].sum(-1).int()."""
    m2 = (torch.arange(L)[None, :] < lens[:, None]).to(torch.int64).to(dev)
    ext = m2.unsqueeze(1).unsqueeze(2)
    mask4 = ext * ext.squeeze(-2).unsqueeze(-1)
    return mask4[:, 0, 0, :].sum(dim=-1).int()


def _check_rows(got, q, k, v, lens, pk, pq, sm, pb, mrd, log, what):
    """Oracle on CPU, four batch rows at a time; returns the largest max-abs."""
    worst = 0.0
    B = got.shape[0]
    for b0 in range(0, B, 4):
        sl = slice(b0, min(B, b0 + 4))
        cpu = lambda t: None if t is None else t[sl].cpu()
        want = oa.deberta_flash_attention(cpu(q), cpu(k), cpu(v), lens[sl], cpu(pk), cpu(pq),
                                          sm, pb, mrd, log)
        g = got[sl].cpu()
        for i, n in enumerate(lens[sl].tolist()):
            err, _ = assert_attn_close(g[i, :, :n], want[i, :, :n], f"{what} b={b0 + i}")
            worst = max(worst, err)
            assert torch.all(g[i, :, n:] == 0), f"{what} b={b0 + i}: rows past the length"
    return worst


def test_v2_flash_forward_call_config3(dev):
    """DeBERTa-v3-large at config 3 (B = 32, L = 512, lengths U{256..512},
    256 log buckets, max_relative_positions 512, share_att_key, c2p|p2c):
    all 32 sequences."""
    from kernels.flash_deberta_attention import HAS_TRITON, flash_deberta_attention
    assert HAS_TRITON
    bf = torch.bfloat16
    hidden, lens = workloads.config3_hidden()
    B, L, Dm = hidden.shape
    H = 16
    g = torch.Generator().manual_seed(3301)
    Wq, Wk, Wv = (torch.randn(Dm, Dm, generator=g) * 0.02 for _ in range(3))
    bq, bk, bv = (torch.randn(Dm, generator=g) * 0.02 for _ in range(3))
    rel_w = torch.randn(512, Dm, generator=g) * 0.02
    d = lambda t: t.to(dev, bf)
    x = d(hidden)
    # the layer's projections (vLLM QKV linears with bias): [B, L, H*64]
    q_out, k_out, v_out = (F.linear(x, d(W), d(b)) for W, b in ((Wq, bq), (Wk, bk), (Wv, bv)))
    query_layer, key_layer, value_layer = (_heads(t, H) for t in (q_out, k_out, v_out))
    assert not query_layer.is_contiguous()
    # rel_embeddings = LayerNorm(rel_embeddings.weight) (norm_rel_ebd), then [0 : 2 att_span]
    rel_emb = F.layer_norm(d(rel_w), (Dm,), eps=1e-7)[0:512, :].unsqueeze(0)
    att_span = 256
    pos_key_layer = _heads(F.linear(rel_emb, d(Wk), d(bk)), H)     # (1, H, 2S, 64)
    pos_query_layer = _heads(F.linear(rel_emb, d(Wq), d(bq)), H)
    pos_key = torch.matmul(query_layer, pos_key_layer.transpose(-1, -2).contiguous())
    pos_query = torch.matmul(key_layer, pos_query_layer.transpose(-1, -2).to(bf).contiguous())
    assert pos_key.shape == (B, H, L, 2 * att_span)
    seq_lengths = _mask_seq_lengths(lens, L, dev)
    assert torch.equal(seq_lengths.cpu(), lens.int())
    sm_scale = 1.0 / (64 * 3) ** 0.5
    out = flash_deberta_attention(
        q=query_layer, k=key_layer, v=value_layer, seq_lengths=seq_lengths,
        pos_key=pos_key, pos_query=pos_query, causal=False, sm_scale=sm_scale,
        position_buckets=256, max_relative_distance=512, use_log_bucket=True)
    assert out.shape == (B, H, L, 64) and out.dtype == bf
    worst = _check_rows(out, query_layer, key_layer, value_layer, lens, pos_key, pos_query,
                        sm_scale, 256, 512, True, "v2 _flash_forward cfg3")
    print(f"v2 _flash_forward config 3, 32 sequences: max-abs {worst:.3e}")


@pytest.mark.parametrize("pos_att", [("c2p", "p2c"), ("c2p",), ("p2c",)])
def test_v1_flash_forward_call(dev, pos_att):
    """DeBERTa v1 (base widths: hidden 768, 12 heads): in_proj chunks as q/k/v
    views, q_bias / v_bias added, att_span = min(L, max_relative_positions),
    the relative table's middle 2 att_span rows, linear positions
    (use_log_bucket=False, position_buckets = att_span), and either position
    term alone as pos_att_type allows."""
    from kernels.flash_deberta_attention import HAS_TRITON, flash_deberta_attention
    assert HAS_TRITON
    bf = torch.bfloat16
    B, L, Dm, H, max_rel = 4, 320, 768, 12, 512
    lens = torch.tensor([320, 301, 64, 17])
    g = torch.Generator().manual_seed(3302)
    hidden = torch.randn(B, L, Dm, generator=g)
    W_in = torch.randn(3 * Dm, Dm, generator=g) * 0.02
    q_bias, v_bias = (torch.randn(Dm, generator=g) * 0.02 for _ in range(2))
    W_pos = torch.randn(Dm, Dm, generator=g) * 0.02
    W_posq = torch.randn(Dm, Dm, generator=g) * 0.02
    b_posq = torch.randn(Dm, generator=g) * 0.02
    rel_w = torch.randn(2 * max_rel, Dm, generator=g) * 0.02
    d = lambda t: t.to(dev, bf)
    qp = F.linear(d(hidden), d(W_in))
    query_layer, key_layer, value_layer = _heads(qp, H).chunk(3, dim=-1)
    query_layer = query_layer + _heads(d(q_bias)[None, None, :], H)
    value_layer = value_layer + _heads(d(v_bias)[None, None, :], H)
    assert not key_layer.is_contiguous()
    att_span = min(L, max_rel)
    rel_emb = d(rel_w)[max_rel - att_span: max_rel + att_span, :].unsqueeze(0)
    sm_scale = 1.0 / (64 * (1 + len(pos_att))) ** 0.5
    pos_key = pos_query = None
    if "c2p" in pos_att:
        pk_layer = _heads(F.linear(rel_emb, d(W_pos)), H)
        pos_key = torch.matmul(query_layer, pk_layer.transpose(-1, -2).contiguous())
    if "p2c" in pos_att:
        pq_layer = _heads(F.linear(rel_emb, d(W_posq), d(b_posq)), H)
        pos_query = torch.matmul(key_layer, pq_layer.transpose(-1, -2).to(bf).contiguous())
    seq_lengths = _mask_seq_lengths(lens, L, dev)
    out = flash_deberta_attention(
        q=query_layer, k=key_layer, v=value_layer, seq_lengths=seq_lengths,
        pos_key=pos_key, pos_query=pos_query, causal=False, sm_scale=sm_scale,
        position_buckets=att_span, max_relative_distance=max_rel, use_log_bucket=False)
    worst = _check_rows(out, query_layer, key_layer, value_layer, lens, pos_key, pos_query,
                        sm_scale, att_span, max_rel, False, f"v1 _flash_forward {pos_att}")
    print(f"v1 _flash_forward {pos_att}: max-abs {worst:.3e}")
