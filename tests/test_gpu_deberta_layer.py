"""DeBERTa-v3-large encoder layers (config 3 shapes: hidden 1024, 16 heads,
intermediate 4096, 256 log buckets, max_relative_positions 512) on the GPU
against the fp32 oracle restatement, on config-3 batch rows (L = 512,
right-padded).

Tolerance: each layer ends in a LayerNorm (outputs O(1), up to ~5); the GPU
path rounds every intermediate to bf16 (relative 2^-8), so max-abs 6e-2 per
layer stack and cosine 0.9999, on valid rows. Padded rows are checked to be
finite (their values are defined by the reference's zeroed attention rows)."""
import pytest
import torch

import workloads
from _tol import cosine

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("batch,layers", [(3, 1), (2, 2)])
def test_deberta_layers_match_oracle(batch, layers):
    from encoders.deberta import deberta_forward, random_weights
    from oracle import encoders as oe
    hidden, lens = workloads.config3_hidden(batch)
    w = random_weights(num_layers=layers, dtype=torch.bfloat16)
    dev = torch.device("cuda:0")
    got = deberta_forward(hidden.to(dev, torch.bfloat16), lens.to(dev), w.to(dev)).float().cpu()
    want = oe.deberta_encoder(hidden.to(torch.bfloat16).float(), lens, w)
    assert torch.isfinite(got).all()
    for b in range(batch):
        n = int(lens[b])
        err = (got[b, :n] - want[b, :n]).abs().max().item()
        cs = cosine(got[b, :n], want[b, :n])
        print(f"layers {layers} row {b} (len {n}): max-abs {err:.3e} cosine {cs:.6f}")
        assert err <= 6e-2 and cs >= 0.9999, (b, err, cs)


def test_deberta_layer_dense_ln_paths_agree_and_match_oracle():
    """DeBERTa-v3-base widths (hidden 768, 12 heads, intermediate 3072), where
    the attention output's dense + residual + LayerNorm runs as one kernel by
    default: that path and the GEMM + LayerNorm pass (fuse_dense_ln=False)
    both match the oracle on the valid rows of the padded layer, and the
    packed layer's two paths agree with each other."""
    from encoders.deberta import (deberta_layer_forward, deberta_layer_packed,
                                  deberta_rel_embeddings, random_weights)
    from kernels.packing import unpad_packed
    from oracle import encoders as oe
    _, lens = workloads.config3_hidden(3)
    hidden = torch.randn(3, 512, 768, generator=torch.Generator().manual_seed(71))
    w = random_weights(num_layers=1, hidden=768, heads=12, inter=3072, dtype=torch.bfloat16)
    dev = torch.device("cuda:0")
    wd = w.to(dev)
    x, sl = hidden.to(dev, torch.bfloat16), lens.to(dev)
    rel = deberta_rel_embeddings(wd)
    want = oe.deberta_encoder(hidden.to(torch.bfloat16).float(), lens, w)
    outs = {}
    for fuse in (True, False):
        got = deberta_layer_forward(x, sl, rel, wd.layers[0], wd, fuse_dense_ln=fuse).float().cpu()
        for b in range(3):
            n = int(lens[b])
            err = (got[b, :n] - want[b, :n]).abs().max().item()
            cs = cosine(got[b, :n], want[b, :n])
            assert err <= 6e-2 and cs >= 0.9999, (fuse, b, err, cs)
        cu = torch.cat([lens.new_zeros(1), lens.cumsum(0)]).to(device=dev, dtype=torch.int32)
        xf = unpad_packed(x, cu, int(lens.sum()))
        outs[fuse] = deberta_layer_packed(xf, cu, x.shape[1], rel, wd.layers[0], wd,
                                          fuse_dense_ln=fuse).float().cpu()
    from kernels import weight_pack
    assert id(wd.layers[0].wo) in weight_pack._CACHE
    d = (outs[True] - outs[False]).abs()
    assert d.max().item() <= 6e-2 and cosine(outs[True], outs[False]) >= 0.9999, d.max().item()


def test_deberta_layer_wide_bucket_steps_match_oracle():
    """position_buckets 256 with max_relative_positions 256: the log bucket
    moves by 2 per unit of distance in places, so the layer takes the
    reference interface (materialised pos_key / pos_query, per-score gather)
    instead of the fused kernel; the output still matches the oracle."""
    from encoders.deberta import deberta_forward, random_weights
    from kernels.flash_deberta_attention import unit_steps
    from oracle import encoders as oe
    assert not unit_steps(256, 256, True, 512)
    hidden, lens = workloads.config3_hidden(2)
    w = random_weights(num_layers=1, dtype=torch.bfloat16)
    w.max_relative_positions = 256
    dev = torch.device("cuda:0")
    got = deberta_forward(hidden.to(dev, torch.bfloat16), lens.to(dev), w.to(dev)).float().cpu()
    want = oe.deberta_encoder(hidden.to(torch.bfloat16).float(), lens, w)
    for b in range(2):
        n = int(lens[b])
        err = (got[b, :n] - want[b, :n]).abs().max().item()
        cs = cosine(got[b, :n], want[b, :n])
        print(f"wide steps row {b} (len {n}): max-abs {err:.3e} cosine {cs:.6f}")
        assert err <= 6e-2 and cs >= 0.9999, (b, err, cs)


def test_activation_gelu_matches_oracle():
    """vfk_act_fwd on a strided [rows, n] view (DeBERTa's intermediate GELU)."""
    from kernels.activation import activation
    from oracle.epilogues import gelu_erf, gelu_tanh
    g = torch.Generator().manual_seed(9)
    x = (torch.randn(301, 4100, generator=g) * 3).to(torch.bfloat16)
    dev = torch.device("cuda:0")
    xd = x.to(dev)[:, 2:4098]
    for name, ref in (("gelu", gelu_erf), ("gelu_new", gelu_tanh)):
        got = activation(xd, name).float().cpu()
        want = ref(x[:, 2:4098].float())
        # one bf16 rounding of the result (relative 2^-8 of |y| <= ~10)
        assert (got - want).abs().max().item() <= 2 ** -8 * want.abs().max().item(), name


def test_deberta_flat_call_matches_padded_batch_and_oracle():
    """The GLiNER plugins' flat call (plugins/deberta_gliner/model.py:166-202)
    on the packed rows (varlen attention, no padding) against the valid rows
    of the padded forward (the GEMMs run on another row count: within 2 bf16
    steps of the output scale) and against the fp32 oracle at the layer
    tolerance (6e-2, cosine 0.9999)."""
    from encoders.deberta import deberta_forward, deberta_forward_flat, random_weights
    from oracle import encoders as oe
    hidden, lens = workloads.config3_hidden(3)
    wc = random_weights(num_layers=2, dtype=torch.bfloat16)
    w = wc.to(torch.device("cuda:0"))
    dev = torch.device("cuda:0")
    xb = hidden.to(dev, torch.bfloat16)
    L = int(lens.max())
    xb = xb[:, :L].contiguous()     # the flat call pads to the longest sequence, with zeros
    for b, n in enumerate(lens):
        xb[b, int(n):] = 0
    flat = torch.cat([xb[b, :int(n)] for b, n in enumerate(lens)])
    pos = torch.cat([torch.arange(int(n)) for n in lens]).to(dev)
    got = deberta_forward_flat(flat, pos, w).float().cpu()
    want_b = deberta_forward(xb, lens.to(dev, torch.int32), w).float().cpu()
    ref = oe.deberta_encoder(xb.float().cpu(), lens, wc)
    a = 0
    for b, n in enumerate(lens.tolist()):
        g_, w_ = got[a:a + n], want_b[b, :n]
        dp = (g_ - w_).abs().max().item()
        err = (g_ - ref[b, :n]).abs().max().item()
        cs = cosine(g_, ref[b, :n])
        print(f"flat row {b} (len {n}): vs padded {dp:.3e}; vs oracle {err:.3e} cosine {cs:.6f}")
        assert dp <= 2 * 2.0 ** -7 * w_.abs().max().item(), (b, dp)
        assert err <= 6e-2 and cs >= 0.9999, (b, err, cs)
        a += n


@pytest.mark.parametrize("layers,max_rel", [(1, 512), (2, 128)])
def test_deberta_v1_layers_match_oracle(layers, max_rel):
    """DeBERTa v1 (deberta-base shapes: hidden 768, 12 heads, GELU 3072) with
    linear relative positions: att_span = min(L, max_rel) = 512 uses the whole
    relative table; max_rel 128 < L clamps at +-128. Valid rows only."""
    import encoders.deberta as ed
    from oracle import encoders as oe
    B, L = 3, 512
    g = torch.Generator().manual_seed(1013 + max_rel)
    lens = torch.tensor([512, 300, 129], dtype=torch.int32)
    x = torch.randn(B, L, 768, generator=g)
    w = ed.random_weights_v1(num_layers=layers, max_relative_positions=max_rel, dtype=torch.bfloat16)
    dev = torch.device("cuda:0")
    got = ed.deberta_v1_forward(x.to(dev, torch.bfloat16), lens.to(dev), w.to(dev)).float().cpu()
    want = x.to(torch.bfloat16).float()
    for lw in w.layers:
        want = oe.deberta_v1_layer(want, lens, w.rel_emb.float(),
                                   ed.DebertaV1LayerWeights(*(getattr(lw, f).float() for f in
                                                              ed.DebertaV1LayerWeights.__dataclass_fields__)),
                                   12, max_rel, w.eps)
    assert torch.isfinite(got).all()
    for b in range(B):
        n = int(lens[b])
        err = (got[b, :n] - want[b, :n]).abs().max().item()
        cs = cosine(got[b, :n], want[b, :n])
        print(f"v1 layers {layers} max_rel {max_rel} row {b} (len {n}): max-abs {err:.3e} cosine {cs:.6f}")
        assert err <= 6e-2 and cs >= 0.9999, (b, err, cs)
