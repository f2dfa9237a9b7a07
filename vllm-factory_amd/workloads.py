"""Seeded synthetic workloads of the encoder-attention benchmark configurations.

Every generator draws from torch.Generator().manual_seed(1000 + config id) on
the CPU (so CPU and GPU consumers see identical values) and returns CPU
tensors; callers move them to the device. Sizes follow the five benchmark
configurations:

  1  mT5-style RPB attention, B=2, L=256, H=8, d=64, fp32, keys 192..255 of
     sequence 2 masked, 32 buckets / max_distance 128, table ~ N(0, 0.1)
  2  ModernBERT-base attention, 64 packed sequences, lengths U{512..768},
     hidden ~ N(0,1) -> LayerNorm(1e-5) -> Wqkv [768, 2304] ~ N(0, 0.02), bf16
  3  DeBERTa-v3-large disentangled attention, B=32, L=512, lengths
     U{256..512}, 16 heads, 256 buckets, max_relative_positions 512, bf16
  4  mT5-large RPB attention + RMSNorm + gated-GELU FFN, B=32, L=768,
     lengths U{512..768}, d_model 1024, 16 heads, d_ff 2816, bf16
  5  ModernBERT-base encoder, 22 layers, 256 packed sequences U{512..768}
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch


def gen(cfg_id: int) -> torch.Generator:
    return torch.Generator().manual_seed(1000 + cfg_id)


def _lengths(g: torch.Generator, n: int, lo: int, hi: int) -> torch.Tensor:
    return torch.randint(lo, hi + 1, (n,), generator=g, dtype=torch.int64)


def cu_from_lengths(lengths: torch.Tensor) -> torch.Tensor:
    cu = torch.zeros(lengths.numel() + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lengths, 0).to(torch.int32)
    return cu


# ---------------------------------------------------------------------------
# config 1
# ---------------------------------------------------------------------------
@dataclass
class RpbCase:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    table: torch.Tensor
    mask: Optional[torch.Tensor]   # additive [B, 1, 1, L]
    lengths: torch.Tensor          # valid keys per batch row
    num_buckets: int = 32
    max_distance: int = 128
    scale: float = 1.0


def config1() -> RpbCase:
    g = gen(1)
    B, L, H, D = 2, 256, 8, 64
    q = torch.randn(B, H, L, D, generator=g)
    k = torch.randn(B, H, L, D, generator=g)
    v = torch.randn(B, H, L, D, generator=g)
    table = torch.randn(32, H, generator=g) * 0.1
    lengths = torch.tensor([256, 192])
    keep = (torch.arange(L)[None, :] < lengths[:, None]).float()
    mask = ((1.0 - keep) * torch.finfo(torch.float32).min)[:, None, None, :]
    return RpbCase(q, k, v, table, mask, lengths)


# ---------------------------------------------------------------------------
# config 2
# ---------------------------------------------------------------------------
@dataclass
class VarlenCase:
    qkv: torch.Tensor          # [T, 3, H, 64] (view of the fused projection)
    cu_seqlens: torch.Tensor   # int32 [n + 1]
    lengths: torch.Tensor
    max_seqlen: int
    hidden: int = 768
    heads: int = 12


def config2(num_seqs: int = 64, device="cpu", dtype=torch.bfloat16) -> VarlenCase:
    """hidden ~ N(0,1) -> LayerNorm (w=1, no bias, eps 1e-5) -> Wqkv ~ N(0, 0.02).
    The projection runs on `device` in fp32 and is then cast to `dtype`."""
    g = gen(2)
    lengths = _lengths(g, 64, 512, 768)[:num_seqs]
    T = int(lengths.sum())
    hidden = torch.randn(T, 768, generator=g)
    w = torch.randn(768, 2304, generator=g) * 0.02
    x = torch.nn.functional.layer_norm(hidden.to(device), (768,), eps=1e-5)
    qkv = (x @ w.to(device)).to(dtype).view(T, 3, 12, 64)
    return VarlenCase(qkv, cu_from_lengths(lengths).to(device), lengths, int(lengths.max()))


# ---------------------------------------------------------------------------
# config 3
# ---------------------------------------------------------------------------
@dataclass
class DebertaCase:
    q: torch.Tensor         # [B, H, L, 64]
    k: torch.Tensor
    v: torch.Tensor
    key_rel: torch.Tensor   # [H, 2S, 64] = key_proj(LN(rel)) per head
    query_rel: torch.Tensor
    lengths: torch.Tensor   # int32 [B]
    position_buckets: int = 256
    max_relative_positions: int = 512

    @property
    def sm_scale(self) -> float:
        return 1.0 / math.sqrt(64 * 3)


def config3(batch: int = 32, device="cpu", dtype=torch.bfloat16) -> DebertaCase:
    """hidden ~ N(0,1); Wq/Wk/Wv [1024,1024] ~ N(0,0.02) with bias ~ N(0,0.02);
    rel table [512,1024] ~ N(0,0.02) -> LayerNorm -> shared key/query projections."""
    g = gen(3)
    B, L, Hd, H = 32, 512, 1024, 16
    lengths = _lengths(g, B, 256, 512)[:batch]
    hidden = torch.randn(B, L, Hd, generator=g)[:batch]
    Wq, Wk, Wv = (torch.randn(Hd, Hd, generator=g) * 0.02 for _ in range(3))
    bq, bk, bv = (torch.randn(Hd, generator=g) * 0.02 for _ in range(3))
    rel = torch.randn(512, Hd, generator=g) * 0.02
    hidden, rel = hidden.to(device), rel.to(device)
    Wq, Wk, Wv, bq, bk, bv = (t.to(device) for t in (Wq, Wk, Wv, bq, bk, bv))
    rel = torch.nn.functional.layer_norm(rel, (Hd,), eps=1e-7)

    def heads(x):  # [..., L, 1024] -> [..., H, L, 64]
        return x.view(*x.shape[:-1], H, 64).transpose(-2, -3)

    q = heads(hidden @ Wq + bq).to(dtype).contiguous()
    k = heads(hidden @ Wk + bk).to(dtype).contiguous()
    v = heads(hidden @ Wv + bv).to(dtype).contiguous()
    key_rel = heads(rel @ Wk + bk).to(dtype).contiguous()     # [H, 512, 64]
    query_rel = heads(rel @ Wq + bq).to(dtype).contiguous()
    return DebertaCase(q, k, v, key_rel, query_rel, lengths.to(torch.int32).to(device))


def config3_hidden(batch: int = 32):
    """The config-3 layer input: (hidden [B, 512, 1024] ~ N(0, 1), lengths
    int32 [B]), the same draws config3 starts from. Layer weights:
    encoders.deberta.random_weights."""
    g = gen(3)
    lengths = _lengths(g, 32, 256, 512)[:batch]
    hidden = torch.randn(32, 512, 1024, generator=g)[:batch]
    return hidden, lengths.to(torch.int32)


# ---------------------------------------------------------------------------
# config 4
# ---------------------------------------------------------------------------
@dataclass
class Mt5Case:
    hidden: torch.Tensor      # [B, L, 1024]
    lengths: torch.Tensor
    mask: torch.Tensor        # additive [B, 1, 1, L] in the model dtype
    table: torch.Tensor       # [32, 16]
    wq: torch.Tensor
    wk: torch.Tensor
    wv: torch.Tensor
    wo: torch.Tensor
    wi0: torch.Tensor
    wi1: torch.Tensor
    wff_o: torch.Tensor
    ln1: torch.Tensor
    ln2: torch.Tensor


def config4(batch: int = 32, device="cpu", dtype=torch.bfloat16) -> Mt5Case:
    g = gen(4)
    B, L, Dm, H, F = 32, 768, 1024, 16, 2816
    lengths = _lengths(g, B, 512, 768)[:batch]
    hidden = torch.randn(B, L, Dm, generator=g)[:batch]
    table = torch.randn(32, H, generator=g) * 0.1
    ws = [torch.randn(Dm, Dm, generator=g) * 0.02 for _ in range(4)]
    wi0 = torch.randn(Dm, F, generator=g) * 0.02
    wi1 = torch.randn(Dm, F, generator=g) * 0.02
    wff_o = torch.randn(F, Dm, generator=g) * 0.02
    keep = (torch.arange(L)[None, :] < lengths[:, None]).to(dtype)
    mask = ((1.0 - keep) * torch.finfo(dtype).min)[:, None, None, :]
    cv = lambda t: t.to(device=device, dtype=dtype)
    return Mt5Case(cv(hidden), lengths, mask.to(device), cv(table), *(cv(w) for w in ws),
                   cv(wi0), cv(wi1), cv(wff_o),
                   torch.ones(Dm, device=device, dtype=dtype),
                   torch.ones(Dm, device=device, dtype=dtype))


def attention_flops_dense(lengths_q, lengths_k=None, heads: int = 1, d: int = 64) -> float:
    """4 * d * H * sum(len_q * len_k): QK^T and PV over valid pairs only."""
    lk = lengths_q if lengths_k is None else lengths_k
    return float(4 * d * heads * sum(int(a) * int(b) for a, b in zip(lengths_q, lk)))


def window_pairs(n: int, w: int) -> int:
    """Number of (i, j) in [0, n)^2 with |i - j| <= w."""
    if w < 0 or w >= n:
        return n * n
    # full band: n rows * (2w+1) minus the two triangles cut at the borders
    return n * (2 * w + 1) - w * (w + 1)


# ---------------------------------------------------------------------------
# config 5
# ---------------------------------------------------------------------------
@dataclass
class EncoderCase:
    ids: torch.Tensor          # [T] int64 token ids, U{0..vocab-1}
    cu_seqlens: torch.Tensor   # int32 [n + 1]
    lengths: torch.Tensor
    max_seqlen: int


def config5(num_seqs: int = 256, lo: int = 512, hi: int = 768, vocab: int = 50368) -> EncoderCase:
    """ModernBERT-base encoder input: packed sequences with lengths U{lo..hi}
    and token ids uniform over the vocabulary (ids equal to 50284 are the
    reference's masked keys). Weights: encoders.modernbert.random_weights."""
    g = gen(5)
    lengths = _lengths(g, num_seqs, lo, hi)
    T = int(lengths.sum())
    ids = torch.randint(0, vocab, (T,), generator=g, dtype=torch.int64)
    return EncoderCase(ids, cu_from_lengths(lengths), lengths, int(lengths.max()))


# ---------------------------------------------------------------------------
# GLiNER pooler input (the requests of configs 3 / 5 as GLiNER prompts)
# ---------------------------------------------------------------------------
@dataclass
class GlinerRequests:
    ids: torch.Tensor           # [T] int64
    words_mask: torch.Tensor    # [T] int64, word id + 1 on text subtokens, else 0
    cu_seqlens: torch.Tensor    # int32 [n + 1]
    text_lengths: list          # words per request
    ent_token_id: int


def gliner_requests(num_seqs: int = 256, lo: int = 512, hi: int = 768, max_labels: int = 25,
                    ent_token_id: int = 128001, seed: int = 7) -> GlinerRequests:
    """Packed GLiNER requests in the prompt layout of poolers/gliner.py's
    callers: per request, U{1..max_labels} labels, each a class token followed
    by 1-3 label tokens, one separator, then words of 1-3 subtokens each until
    the request's length U{lo..hi} is reached (the last word may be cut)."""
    g = torch.Generator().manual_seed(1000 + seed)
    lengths = _lengths(g, num_seqs, lo, hi)
    ids, wm, tls = [], [], []
    for n in lengths.tolist():
        labels = int(torch.randint(1, max_labels + 1, (1,), generator=g))
        lab_len = torch.randint(1, 4, (labels,), generator=g).tolist()
        prompt = []
        for k in lab_len:
            prompt += [ent_token_id] + [500 + k] * k
        prompt = (prompt + [3])[:n]
        text = n - len(prompt)
        sub = torch.randint(1, 4, (text + 1,), generator=g).tolist()
        mask, w = [], 0
        while len(mask) < text:
            w += 1
            mask += [w] * sub[w - 1]
        mask = mask[:text]
        ids += prompt + torch.randint(1000, 120000, (text,), generator=g).tolist()
        wm += [0] * len(prompt) + mask
        tls.append(w)
    return GlinerRequests(torch.tensor(ids, dtype=torch.int64), torch.tensor(wm, dtype=torch.int64),
                          cu_from_lengths(lengths), tls, ent_token_id)
