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


def test_mt5_encoder_stack_matches_oracle():
    """mt5_encoder_forward (models/mt5/mt5_encoder.py:524-599): two layers with
    their own weights, the layer-0 bias table shared, the reference's key mask
    built from an attention_mask of ones and zeros, then the final RMSNorm, on
    two config-4 batch rows. The final RMSNorm rescales rows to unit RMS
    (values up to ~5), so the bound is the per-layer one: max-abs 6e-2,
    cosine 0.9999 on valid rows."""
    from encoders.mt5 import mt5_encoder_forward
    from oracle import encoders as oe
    c = workloads.config4(batch=2)
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(1404)
    base = (c.wq, c.wk, c.wv, c.wo, c.wi0, c.wi1, c.wff_o, c.ln1, c.ln2)
    second = tuple((w.float() + 0.01 * torch.randn(w.shape, generator=g)).to(w.dtype) for w in base)
    layers = [base, second]
    lnf = (1.0 + 0.1 * torch.randn(1024, generator=g)).bfloat16()
    L = c.hidden.shape[1]
    keep = (torch.arange(L)[None, :] < c.lengths[:, None]).long()
    got = mt5_encoder_forward(None, keep.to(dev), [tuple(w.to(dev) for w in lw) for lw in layers],
                              c.table.to(dev), lnf.to(dev), inputs_embeds=c.hidden.to(dev))
    want = oe.mt5_encoder(c.hidden, layers, c.table, lnf, c.mask)
    got = got.float().cpu()
    for b in range(2):
        n = int(c.lengths[b])
        err = (got[b, :n] - want[b, :n]).abs().max().item()
        cs = cosine(got[b, :n], want[b, :n])
        print(f"2 layers + final RMSNorm, row {b} (len {n}): max-abs {err:.3e} cosine {cs:.6f}")
        assert err <= 6e-2 and cs >= 0.9999, (b, err, cs)


def test_mt5_flat_stream_routed_per_sequence():
    """The GLiNER flat call (plugins/mt5_gliner/model.py:169-201) routed per
    sequence: two layers on the packed rows of three config-4 rows (varlen RPB
    attention, no padding) against the padded-batch forward with the
    reference's key mask, on the valid rows. The GEMMs run on a different row
    count, so the bound is 2 bf16 steps of the output scale; and against the
    fp32 oracle at the layer tolerance (6e-2, cosine 0.9999)."""
    from encoders.mt5 import mt5_encoder_flat, mt5_layer_forward
    from oracle import encoders as oe
    c = workloads.config4(batch=3)
    dev = torch.device("cuda:0")
    lens = [int(n) for n in c.lengths]
    L = max(lens)
    xb = c.hidden[:, :L].clone()
    for b, n in enumerate(lens):
        xb[b, n:] = 0
    xbd = xb.to(dev)
    ws = (c.wq, c.wk, c.wv, c.wo, c.wi0, c.wi1, c.wff_o, c.ln1, c.ln2)
    lw = tuple(w.to(dev) for w in ws)
    table = c.table.to(dev)
    flat = torch.cat([xbd[b, :n] for b, n in enumerate(lens)])
    pos = torch.cat([torch.arange(n) for n in lens]).to(dev)
    got = mt5_encoder_flat(flat, pos, [lw, lw], table).float().cpu()
    valid = torch.arange(L, device=dev)[None, :] < torch.tensor(lens, device=dev)[:, None]
    mask = ((~valid).to(xb.dtype) * torch.finfo(xb.dtype).min).view(3, 1, 1, L)
    want_b = mt5_layer_forward(mt5_layer_forward(xbd, *lw, table, mask), *lw, table, mask).float().cpu()
    cmask = ((~valid.cpu()).to(xb.dtype) * torch.finfo(xb.dtype).min).view(3, 1, 1, L)
    ref = oe.mt5_layer(oe.mt5_layer(xb, *ws, c.table, cmask), *ws, c.table, cmask)
    a = 0
    for b, n in enumerate(lens):
        g_, w_ = got[a:a + n], want_b[b, :n]
        dp = (g_ - w_).abs().max().item()
        err = (g_ - ref[b, :n]).abs().max().item()
        cs = cosine(g_, ref[b, :n])
        print(f"flat row {b} (len {n}): vs padded {dp:.3e}; vs oracle {err:.3e} cosine {cs:.6f}")
        assert dp <= 2 * 2.0 ** -7 * w_.abs().max().item(), (b, dp)
        assert err <= 6e-2 and cs >= 0.9999, (b, err, cs)
        a += n


def test_mt5_layer_packed_matches_oracle_and_padded_layer():
    """mt5_layer_packed on the packed valid rows of three config-4 batch rows
    against the fp32 oracle layer (bound as for the padded layer: max-abs
    6e-2, cosine 0.9999) and against the padded layer's valid rows (same
    kernels on fewer rows: the GEMMs may pick other tilings for the smaller
    row count, so within 2 bf16 steps of the output scale)."""
    from encoders.mt5 import mt5_layer_forward, mt5_layer_packed
    from kernels.packing import unpad_packed
    from oracle import encoders as oe
    c = workloads.config4(batch=3)
    dev = torch.device("cuda:0")
    ws = (c.wq, c.wk, c.wv, c.wo, c.wi0, c.wi1, c.wff_o, c.ln1, c.ln2, c.table)
    wd = tuple(w.to(dev) for w in ws)
    lens = c.lengths.tolist()
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device=dev)
    L = c.hidden.shape[1]
    x = c.hidden.to(dev)
    mask = c.mask.to(dev)
    xf = unpad_packed(x, cu, int(cu[-1]))
    got = mt5_layer_packed(xf, cu, L, *wd, mask).float().cpu()
    pad = unpad_packed(mt5_layer_forward(x, *wd, mask), cu, int(cu[-1])).float().cpu()
    want = oe.mt5_layer(c.hidden, *ws, c.mask)
    for b, n in enumerate(lens):
        a, e = int(cu[b]), int(cu[b + 1])
        err = (got[a:e] - want[b, :n]).abs().max().item()
        cs = cosine(got[a:e], want[b, :n])
        dp = (got[a:e] - pad[a:e]).abs().max().item()
        print(f"packed row {b} (len {n}): max-abs {err:.3e} cosine {cs:.6f}; vs padded {dp:.3e}")
        assert err <= 6e-2 and cs >= 0.9999, (b, err, cs)
        assert dp <= 2 * 2.0 ** -7 * pad[a:e].abs().max().item(), (b, dp)


def test_mt5_layer_packed_fused_glu_matches_oracle():
    """mt5_layer_packed with the gated FF as one GLU projection kernel
    (wi_glu = stack_glu_weight(wi0, wi1)) against the fp32 oracle layer, same
    bound as the unfused packed layer."""
    from encoders.mt5 import mt5_layer_packed, stack_glu_weight
    from kernels.packing import unpad_packed
    from oracle import encoders as oe
    c = workloads.config4(batch=3)
    dev = torch.device("cuda:0")
    ws = (c.wq, c.wk, c.wv, c.wo, c.wi0, c.wi1, c.wff_o, c.ln1, c.ln2, c.table)
    wd = tuple(w.to(dev) for w in ws)
    lens = c.lengths.tolist()
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device=dev)
    L = c.hidden.shape[1]
    xf = unpad_packed(c.hidden.to(dev), cu, int(cu[-1]))
    wg = stack_glu_weight(wd[4], wd[5])
    assert wg is not None and wg.shape == (2 * c.wi0.shape[1], c.wi0.shape[0])
    got = mt5_layer_packed(xf, cu, L, *wd, None, wi_glu=wg).float().cpu()
    want = oe.mt5_layer(c.hidden, *ws, c.mask)
    for b, n in enumerate(lens):
        a, e = int(cu[b]), int(cu[b + 1])
        err = (got[a:e] - want[b, :n]).abs().max().item()
        cs = cosine(got[a:e], want[b, :n])
        print(f"fused-FF packed row {b} (len {n}): max-abs {err:.3e} cosine {cs:.6f}")
        assert err <= 6e-2 and cs >= 0.9999, (b, err, cs)
