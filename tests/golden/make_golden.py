"""Writes the committed golden fixtures of tests/golden/ from the oracle.

The bucket tables cover every relative position the benchmark configurations
meet (|rel| <= 767, plus margin); the attention vectors are small seeded
inputs with their oracle outputs in fp64. Regenerate with
    python tests/golden/make_golden.py
and review the diff: these files freeze the oracle's behaviour, which the
oracle tests pin independently (exact arithmetic, transformers, brute force).
"""
import json
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention as oa  # noqa: E402
from oracle import buckets as ob  # noqa: E402


def buckets():
    cases = []
    for bidir in (True, False):
        for nb, md in ((32, 128), (32, 64), (64, 256)):
            rel = torch.arange(-1024, 1025)
            cases.append(dict(bidirectional=bidir, num_buckets=nb, max_distance=md, rel_min=-1024,
                              bucket=ob.t5_relative_position_bucket(rel, bidir, nb, md).tolist()))
    with open(os.path.join(HERE, "t5_buckets.json"), "w") as f:
        json.dump({"source": "models/mt5/mt5_encoder.py:124-148 (fp32 eager formula)",
                   "cases": cases}, f)
    cases = []
    for bs, mp in ((256, 512), (256, 1024), (128, 512)):
        rel = torch.arange(-1024, 1025)
        cases.append(dict(bucket_size=bs, max_position=mp, rel_min=-1024,
                          bucket=ob.make_log_bucket_position(rel, bs, mp).long().tolist()))
    with open(os.path.join(HERE, "deberta_buckets.json"), "w") as f:
        json.dump({"source": "models/deberta_v2/deberta_v2_encoder.py:70-89 (fp32 eager formula)",
                   "cases": cases}, f)


def attention():
    g = torch.Generator().manual_seed(2024)
    d = torch.float64
    out = {}

    def r(*shape):  # fp32 values, kept in fp64 for the oracle
        return torch.randn(*shape, generator=g).to(d)

    # T5 RPB, bidirectional, key padding mask
    q, k, v = (r(1, 2, 40, 64) for _ in range(3))
    table = r(32, 2) * 0.5
    mask = torch.zeros(1, 1, 1, 40, dtype=d)
    mask[..., 33:] = torch.finfo(torch.float32).min
    out["rpb"] = dict(q=q, k=k, v=v, table=table, mask=mask,
                      out=oa.rpb_attention(q, k, v, table, 32, 128, False, mask, 1.0, dtype=d))
    # DeBERTa disentangled with log buckets active at small L (mid = 8)
    B, H, L, S = 2, 1, 40, 16
    q, k, v = (r(B, H, L, 64) for _ in range(3))
    pk = r(B, H, L, 2 * S)
    pq = r(B, H, L, 2 * S)
    lens = torch.tensor([40, 27], dtype=torch.int32)
    out["deberta"] = dict(q=q, k=k, v=v, pos_key=pk, pos_query=pq, seq_lengths=lens,
                          out=oa.deberta_flash_attention(q, k, v, lens, pk, pq, 0.1, S, 32, True,
                                                         dtype=d))
    # ModernBERT varlen local attention with RoPE and a key mask
    lens = [5, 33, 40]
    T = sum(lens)
    q, k, v = (r(T, 1, 64) for _ in range(3))
    cu = torch.tensor([0, 5, 38, 78], dtype=torch.int32)
    kvalid = torch.rand(T, generator=g) > 0.2
    out["varlen"] = dict(q=q, k=k, v=v, cu_seqlens=cu, key_valid=kvalid,
                         out=oa.varlen_attention(q, k, v, cu, 16, 10000.0, kvalid, 0.125, dtype=d))
    # store fp32 (inputs are exactly fp32 values; outputs rounded once)
    out = {k1: {k2: (t.float() if t.is_floating_point() else t) for k2, t in c.items()}
           for k1, c in out.items()}
    torch.save(out, os.path.join(HERE, "attention_small.pt"))


if __name__ == "__main__":
    buckets()
    attention()
    print("golden fixtures written")
