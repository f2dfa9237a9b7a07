"""Pins the oracle's attention restatements (oracle/attention.py) with library
routines, brute-force loops, the reference's second (bmm) formulation of the
DeBERTa bias, invariants and the committed golden vectors."""
import math
import os

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oa
from oracle import buckets as ob

GOLD = os.path.join(os.path.dirname(__file__), "golden")
D64 = torch.float64


def _r(*shape, seed=0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=D64)


# ------------------------------------------------------------------ T5 RPB
def test_rpb_no_bias_equals_sdpa():
    q, k, v = _r(2, 3, 50, 64, seed=1), _r(2, 3, 50, 64, seed=2), _r(2, 3, 50, 64, seed=3)
    got = oa.rpb_attention(q, k, v, None, 32, 128, False, None, 0.2, dtype=D64)
    want = F.scaled_dot_product_attention(q, k, v, scale=0.2)
    torch.testing.assert_close(got, want)


def test_rpb_bias_equals_sdpa_with_dense_bias():
    q, k, v = _r(2, 3, 50, 64, seed=4), _r(2, 3, 50, 64, seed=5), _r(2, 3, 50, 64, seed=6)
    table = _r(32, 3, seed=7)
    bias = table[ob.t5_bucket_matrix(50, 50, True, 32, 128)].permute(2, 0, 1)[None]
    mask = torch.zeros(2, 1, 1, 50, dtype=D64)
    mask[1, ..., 40:] = torch.finfo(torch.float32).min
    got = oa.rpb_attention(q, k, v, table, 32, 128, False, mask, 1.0, dtype=D64)
    want = F.scaled_dot_product_attention(q, k, v, attn_mask=bias + mask, scale=1.0)
    torch.testing.assert_close(got, want)


@pytest.mark.parametrize("causal", [False, True])
def test_rpb_brute_force(causal):
    B, H, Lq, Lk = 1, 2, 6, 9
    q, k, v = _r(B, H, Lq, 64, seed=8), _r(B, H, Lk, 64, seed=9), _r(B, H, Lk, 64, seed=10)
    table = _r(32, H, seed=11) * 3
    mask = _r(B, 1, 1, Lk, seed=12)
    got = oa.rpb_attention(q, k, v, table, 32, 128, causal, mask, 0.7, dtype=D64)
    want = torch.zeros_like(got)
    for h in range(H):
        for i in range(Lq):
            sc = []
            for j in range(Lk):
                rel = j - i
                if causal:
                    bkt = 0 if rel >= 0 else (-rel if -rel < 16 else None)
                    if bkt is None:
                        bkt = int(ob.t5_relative_position_bucket(torch.tensor([rel]), False, 32, 128))
                else:
                    bkt = int(ob.t5_relative_position_bucket(torch.tensor([rel]), True, 32, 128))
                s = float(q[0, h, i] @ k[0, h, j]) * 0.7 + float(table[bkt, h]) + float(mask[0, 0, 0, j])
                sc.append(-math.inf if (causal and j > i) else s)
            m = max(sc)
            p = [math.exp(s - m) for s in sc]
            z = sum(p)
            want[0, h, i] = sum(p[j] / z * v[0, h, j] for j in range(Lk))
    torch.testing.assert_close(got, want)


# ------------------------------------------------------------------ DeBERTa
def test_deberta_zero_projections_is_plain_attention():
    q, k, v = _r(2, 2, 30, 64, seed=13), _r(2, 2, 30, 64, seed=14), _r(2, 2, 30, 64, seed=15)
    z = torch.zeros(2, 2, 30, 512, dtype=D64)
    sm = 1 / math.sqrt(192)
    got = oa.deberta_flash_attention(q, k, v, None, z, z, sm, 256, 512, True, dtype=D64)
    torch.testing.assert_close(got, F.scaled_dot_product_attention(q, k, v, scale=sm))


def test_deberta_brute_force_log_buckets():
    """Tiny sizes with mid = 4 so the log branch is exercised (|q - k| up to 11)."""
    B, H, L, S, MAXP = 1, 1, 12, 8, 16
    q, k, v = _r(B, H, L, 64, seed=16), _r(B, H, L, 64, seed=17), _r(B, H, L, 64, seed=18)
    pk, pq = _r(B, H, L, 2 * S, seed=19), _r(B, H, L, 2 * S, seed=20)
    lens = torch.tensor([10], dtype=torch.int32)
    got = oa.deberta_flash_attention(q, k, v, lens, pk, pq, 0.3, S, MAXP, True, dtype=D64)

    def bucket(rel):
        mid = S // 2
        a = abs(rel)
        if a <= mid:
            return rel
        val = math.ceil(math.log(a / mid) / math.log((MAXP - 1) / mid) * (mid - 1)) + mid
        return val if rel > 0 else -val

    want = torch.zeros_like(got)
    for i in range(10):
        sc = []
        for j in range(10):
            c = min(max(bucket(i - j) + S, 0), 2 * S - 1)
            s = (float(q[0, 0, i] @ k[0, 0, j]) + float(pk[0, 0, i, c]) + float(pq[0, 0, j, c])) * 0.3
            sc.append(s)
        m = max(sc)
        p = [math.exp(s - m) for s in sc]
        z = sum(p)
        want[0, 0, i] = sum(p[j] / z * v[0, 0, j] for j in range(10))
    torch.testing.assert_close(got, want)   # rows >= 10 are zero in both


def test_deberta_gather_matches_bmm_formulation():
    """Gather formulation (flash_deberta_attention.py:420-433) == the model's bmm
    formulation (deberta_v2_encoder.py:447-487: c2p from Q Kr^T, p2c from
    K Qr^T gathered with -r_pos then transposed), incl. the 1/scale division."""
    B, H, L, S = 2, 3, 40, 256
    q, k, v = _r(B, H, L, 64, seed=21), _r(B, H, L, 64, seed=22), _r(B, H, L, 64, seed=23)
    key_rel, query_rel = _r(H, 2 * S, 64, seed=24) * 0.3, _r(H, 2 * S, 64, seed=25) * 0.3
    pk, pq = oa.deberta_position_projections(q, k, key_rel, query_rel, dtype=D64)
    sm = 1 / math.sqrt(64 * 3)
    got = oa.deberta_flash_attention(q, k, v, None, pk, pq, sm, S, 512, True, zero_padded_rows=False,
                                     dtype=D64)
    # bmm formulation, (B*H, L, D) layout
    rel = ob.build_relative_position_v2(L, L, S, 512)
    qb, kb = q.reshape(B * H, L, 64), k.reshape(B * H, L, 64)
    scale = math.sqrt(64 * 3)
    scores = torch.bmm(qb, kb.transpose(-1, -2) / scale)
    pkl = key_rel.repeat(B, 1, 1)
    pql = query_rel.repeat(B, 1, 1)
    c2p = torch.bmm(qb, pkl.transpose(-1, -2))
    c2p = torch.gather(c2p, -1, torch.clamp(rel + S, 0, 2 * S - 1).expand(B * H, L, L))
    p2c = torch.bmm(kb, pql.transpose(-1, -2))
    p2c = torch.gather(p2c, -1, torch.clamp(-rel + S, 0, 2 * S - 1).expand(B * H, L, L)).transpose(-1, -2)
    scores = scores + c2p / scale + p2c / scale
    want = torch.bmm(torch.softmax(scores, -1), v.reshape(B * H, L, 64)).view(B, H, L, 64)
    torch.testing.assert_close(got, want)


# ------------------------------------------------------------------ varlen
def test_varlen_single_sequence_equals_sdpa():
    n = 70
    q, k, v = _r(n, 4, 64, seed=26), _r(n, 4, 64, seed=27), _r(n, 4, 64, seed=28)
    got = oa.varlen_attention(q, k, v, torch.tensor([0, n]), -1, 0.0, None, 0.125, dtype=D64)
    want = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1),
                                          scale=0.125).transpose(0, 1)
    torch.testing.assert_close(got, want)


def test_varlen_wide_window_is_global():
    lens = [3, 40, 17]
    T = sum(lens)
    cu = torch.tensor([0, 3, 43, 60])
    q, k, v = _r(T, 2, 64, seed=29), _r(T, 2, 64, seed=30), _r(T, 2, 64, seed=31)
    a = oa.varlen_attention(q, k, v, cu, 40, 10000.0, None, 0.125, dtype=D64)
    b = oa.varlen_attention(q, k, v, cu, -1, 10000.0, None, 0.125, dtype=D64)
    torch.testing.assert_close(a, b)


def test_varlen_brute_force():
    """Window, key mask and RoPE by explicit loops (rotation written per pair)."""
    n, w, theta = 9, 2, 10000.0
    q, k, v = _r(n, 1, 64, seed=32), _r(n, 1, 64, seed=33), _r(n, 1, 64, seed=34)
    kv = torch.tensor([1, 1, 0, 1, 1, 1, 0, 1, 1], dtype=torch.bool)
    got = oa.varlen_attention(q, k, v, torch.tensor([0, n]), w, theta, kv, 0.125, dtype=D64)

    def rot(x, p):
        y = x.clone()
        for f in range(32):
            ang = p * (1.0 / theta ** (2 * f / 64))
            c, s = math.cos(ang), math.sin(ang)
            y[f] = x[f] * c - x[f + 32] * s
            y[f + 32] = x[f + 32] * c + x[f] * s
        return y

    want = torch.zeros_like(got)
    for i in range(n):
        qi = rot(q[i, 0], i)
        js = [j for j in range(n) if abs(i - j) <= w and kv[j]]
        sc = [float(qi @ rot(k[j, 0], j)) * 0.125 for j in js]
        m = max(sc)
        p = [math.exp(s - m) for s in sc]
        z = sum(p)
        want[i, 0] = sum(pp / z * v[j, 0] for pp, j in zip(p, js))
    torch.testing.assert_close(got, want, atol=1e-6, rtol=1e-6)


def test_varlen_pack_order_equivariance():
    lens = [7, 30, 12]
    cu = torch.tensor([0, 7, 37, 49])
    q, k, v = _r(49, 2, 64, seed=35), _r(49, 2, 64, seed=36), _r(49, 2, 64, seed=37)
    a = oa.varlen_attention(q, k, v, cu, 4, 10000.0, None, 0.125, dtype=D64)
    idx = torch.cat([torch.arange(37, 49), torch.arange(0, 7), torch.arange(7, 37)])
    cu2 = torch.tensor([0, 12, 19, 49])
    b = oa.varlen_attention(q[idx], k[idx], v[idx], cu2, 4, 10000.0, None, 0.125, dtype=D64)
    torch.testing.assert_close(a[idx], b)


def test_rope_matches_transformers_rotary():
    """The oracle's cos/sin tables equal transformers' ModernBertRotaryEmbedding
    (the module the reference calls at modernbert_encoder.py:236-242)."""
    from transformers import ModernBertConfig
    from transformers.models.modernbert.modeling_modernbert import ModernBertRotaryEmbedding
    cfg = ModernBertConfig(hidden_size=768, num_attention_heads=12)
    pos = torch.arange(800)[None]
    x = torch.zeros(1, 800, 12, 64)
    rot = ModernBertRotaryEmbedding(cfg)
    for theta, kind in ((160000.0, "full_attention"), (10000.0, "sliding_attention")):
        cos, sin = rot(x, pos, layer_type=kind)
        c2, s2 = oa.rope_cos_sin(torch.arange(800), theta)
        assert torch.equal(cos[0].float(), c2) and torch.equal(sin[0].float(), s2)


# ------------------------------------------------------------------ golden
def test_golden_attention_vectors():
    g = torch.load(os.path.join(GOLD, "attention_small.pt"), weights_only=True)
    r = g["rpb"]
    got = oa.rpb_attention(r["q"], r["k"], r["v"], r["table"], 32, 128, False, r["mask"], 1.0, dtype=D64)
    torch.testing.assert_close(got.float(), r["out"], atol=1e-6, rtol=1e-6)
    d = g["deberta"]
    got = oa.deberta_flash_attention(d["q"], d["k"], d["v"], d["seq_lengths"], d["pos_key"],
                                     d["pos_query"], 0.1, 16, 32, True, dtype=D64)
    torch.testing.assert_close(got.float(), d["out"], atol=1e-6, rtol=1e-6)
    vl = g["varlen"]
    got = oa.varlen_attention(vl["q"], vl["k"], vl["v"], vl["cu_seqlens"], 16, 10000.0,
                              vl["key_valid"], 0.125, dtype=D64)
    torch.testing.assert_close(got.float(), vl["out"], atol=1e-6, rtol=1e-6)
