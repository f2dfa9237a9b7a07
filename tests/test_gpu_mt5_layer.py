"""mT5-large encoder layer (config 4 shapes) on the GPU against the fp32
oracle restatement, on two of the config-4 batch rows (L = 768, right-padded).

Tolerance: the layer output is x + attention + FFN with x ~ N(0, 1); the GPU
path rounds each intermediate to bf16, so max-abs 6e-2 (a few bf16 roundings
of values up to ~5) and cosine 0.9999, on valid (unpadded) rows."""
import pytest
import torch

import workloads
from _tol import cosine

pytestmark = pytest.mark.gpu


def test_mt5_layer_matches_oracle():
    from encoders.mt5 import mt5_layer_forward
    from oracle import encoders as oe
    c = workloads.config4(batch=2)
    dev = torch.device("cuda:0")
    ws = (c.wq, c.wk, c.wv, c.wo, c.wi0, c.wi1, c.wff_o, c.ln1, c.ln2, c.table)
    got = mt5_layer_forward(c.hidden.to(dev), *(w.to(dev) for w in ws), c.mask.to(dev))
    want = oe.mt5_layer(c.hidden, *ws, c.mask)
    got = got.float().cpu()
    for b in range(2):
        n = int(c.lengths[b])
        err = (got[b, :n] - want[b, :n]).abs().max().item()
        cs = cosine(got[b, :n], want[b, :n])
        print(f"row {b} (len {n}): max-abs {err:.3e} cosine {cs:.6f}")
        assert err <= 6e-2 and cs >= 0.9999, (b, err, cs)


def test_mt5_flat_stream_routed_per_sequence():
    """The GLiNER flat call (plugins/mt5_gliner/model.py:169-201) routed per
    sequence: two layers on the packed valid rows of three config-4 rows equal
    the padded-batch forward with the reference's key mask, row for row
    (same kernels on the same padded batch)."""
    from encoders.mt5 import mt5_encoder_flat, mt5_layer_forward
    c = workloads.config4(batch=3)
    dev = torch.device("cuda:0")
    lens = [int(n) for n in c.lengths]
    L = max(lens)
    xb = c.hidden[:, :L].clone()
    for b, n in enumerate(lens):
        xb[b, n:] = 0
    xb = xb.to(dev)
    lw = tuple(w.to(dev) for w in (c.wq, c.wk, c.wv, c.wo, c.wi0, c.wi1, c.wff_o, c.ln1, c.ln2))
    table = c.table.to(dev)
    flat = torch.cat([xb[b, :n] for b, n in enumerate(lens)])
    pos = torch.cat([torch.arange(n) for n in lens]).to(dev)
    got = mt5_encoder_flat(flat, pos, [lw, lw], table)
    valid = torch.arange(L, device=dev)[None, :] < torch.tensor(lens, device=dev)[:, None]
    mask = ((~valid).to(xb.dtype) * torch.finfo(xb.dtype).min).view(3, 1, 1, L)
    want_b = mt5_layer_forward(mt5_layer_forward(xb, *lw, table, mask), *lw, table, mask)
    want = torch.cat([want_b[b, :n] for b, n in enumerate(lens)])
    assert torch.equal(got, want)
