"""Pins oracle/encoders.py against an independent implementation:
transformers' ModernBertModel with the same random weights, run one sequence
at a time on a reduced configuration (hidden 128 = 2 heads of 64, 4 layers
with global layers 0 and 3, sliding window +-8 so short sequences exercise
it). No GPU is used."""
import pytest
import torch

from oracle import encoders as oe


def _small_weights(seed=7):
    import encoders.modernbert as em
    return em.random_weights(num_layers=4, hidden=128, heads=2, inter=192, vocab=500, seed=seed,
                             std=0.05, dtype=torch.float32)


def _hf_model(w, window):
    from transformers import ModernBertConfig, ModernBertModel
    cfg = ModernBertConfig(vocab_size=w.emb.shape[0], hidden_size=w.hidden, intermediate_size=w.inter,
                           num_hidden_layers=len(w.layers), num_attention_heads=w.heads,
                           local_attention=2 * window, global_attn_every_n_layers=3,
                           hidden_activation="gelu", norm_eps=w.eps, norm_bias=False,
                           attention_bias=False, mlp_bias=False, pad_token_id=0)
    cfg._attn_implementation = "eager"
    m = ModernBertModel(cfg).eval()
    sd = {"embeddings.tok_embeddings.weight": w.emb, "embeddings.norm.weight": w.emb_norm,
          "final_norm.weight": w.final_norm}
    for i, lw in enumerate(w.layers):
        p = f"layers.{i}."
        sd[p + "attn.Wqkv.weight"] = lw.wqkv
        sd[p + "attn.Wo.weight"] = lw.wo
        sd[p + "mlp.Wi.weight"] = lw.wi
        sd[p + "mlp.Wo.weight"] = lw.wo_mlp
        sd[p + "mlp_norm.weight"] = lw.mlp_norm
        if lw.attn_norm is not None:
            sd[p + "attn_norm.weight"] = lw.attn_norm
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all("rotary" in k or "inv_freq" in k for k in missing), missing
    return m


def test_modernbert_oracle_matches_transformers():
    w = _small_weights()
    w.window = 8
    lens = [40, 23, 17]
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(1, 500, (sum(lens),), generator=g)
    cu = torch.tensor([0, 40, 63, 80], dtype=torch.int32)
    got = oe.modernbert_encoder(ids, cu, w, dtype=torch.float64)
    m = _hf_model(w, 8).double()
    for s in range(len(lens)):
        a, b = int(cu[s]), int(cu[s + 1])
        with torch.no_grad():
            want = m(input_ids=ids[a:b][None]).last_hidden_state[0]
        # agreement to fp32 rounding of HF's float32 rotary tables; a wrong
        # window, theta, sign or norm placement differs by O(1e-2) or more
        torch.testing.assert_close(got[a:b], want, rtol=0, atol=1e-6)


def test_modernbert_oracle_mask_token_hides_key():
    # a token with id 50284 is never seen as a key (modernbert_encoder.py:456-460):
    # every other row is independent of that token's embedding
    import encoders.modernbert as em
    w = em.random_weights(num_layers=3, hidden=128, heads=2, inter=192, vocab=50368, seed=9,
                          std=0.05, dtype=torch.float32)
    ids = torch.randint(0, 50000, (30,), generator=torch.Generator().manual_seed(4))
    ids[11] = oe.MASK_TOKEN_ID
    cu = torch.tensor([0, 30], dtype=torch.int32)
    a = oe.modernbert_encoder(ids, cu, w, dtype=torch.float64)
    w.emb = w.emb.clone()
    w.emb[oe.MASK_TOKEN_ID] = torch.randn(128, generator=torch.Generator().manual_seed(5))
    b = oe.modernbert_encoder(ids, cu, w, dtype=torch.float64)
    others = torch.arange(30) != 11
    torch.testing.assert_close(a[others], b[others], rtol=0, atol=1e-12)
    assert (a[11] - b[11]).abs().max() > 1e-3  # the token's own row does change


def test_mt5_layer_oracle_matches_transformers():
    # one MT5EncoderModel block (layer 0 owns the relative-attention bias) on
    # inputs_embeds, then its final RMSNorm; weights shared with the oracle
    from transformers import MT5Config, MT5EncoderModel
    g = torch.Generator().manual_seed(11)
    B, L, D, H, F = 2, 40, 128, 2, 192
    cfg = MT5Config(vocab_size=64, d_model=D, d_kv=64, d_ff=F, num_layers=1, num_heads=H,
                    relative_attention_num_buckets=32, relative_attention_max_distance=128,
                    feed_forward_proj="gated-gelu", layer_norm_epsilon=1e-6, dropout_rate=0.0)
    m = MT5EncoderModel(cfg).eval().double()
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    wq, wk, wv, wo = (r(D, D) * 0.08 for _ in range(4))
    wi0, wi1, wff = r(D, F) * 0.08, r(D, F) * 0.08, r(F, D) * 0.08
    ln1, ln2, lnf = 1 + 0.1 * r(D), 1 + 0.1 * r(D), 1 + 0.1 * r(D)
    table = r(32, H) * 0.5
    blk = m.encoder.block[0]
    sa, ff = blk.layer[0], blk.layer[1]
    with torch.no_grad():
        sa.SelfAttention.q.weight.copy_(wq.t()); sa.SelfAttention.k.weight.copy_(wk.t())
        sa.SelfAttention.v.weight.copy_(wv.t()); sa.SelfAttention.o.weight.copy_(wo.t())
        sa.SelfAttention.relative_attention_bias.weight.copy_(table)
        sa.layer_norm.weight.copy_(ln1)
        ff.DenseReluDense.wi_0.weight.copy_(wi0.t()); ff.DenseReluDense.wi_1.weight.copy_(wi1.t())
        ff.DenseReluDense.wo.weight.copy_(wff.t()); ff.layer_norm.weight.copy_(ln2)
        m.encoder.final_layer_norm.weight.copy_(lnf)
    x = r(B, L, D)
    keep = torch.ones(B, L, dtype=torch.float64)
    keep[1, 29:] = 0
    with torch.no_grad():
        want = m(inputs_embeds=x, attention_mask=keep).last_hidden_state
    mask = ((1.0 - keep) * torch.finfo(torch.float64).min)[:, None, None, :]
    got = oe.mt5_layer(x, wq, wk, wv, wo, wi0, wi1, wff, ln1, ln2, table, mask, dtype=torch.float64)
    got = oe.rmsnorm(got, lnf, 1e-6, torch.float64)
    # transformers' T5LayerNorm takes the variance in fp32 even for fp64
    # models (~1e-7 relative); a wrong bucket, mask, norm or gate is >= 1e-3
    torch.testing.assert_close(got, want, rtol=0, atol=1e-5)


def test_mt5_encoder_stack_oracle_matches_transformers():
    """Two MT5EncoderModel blocks (layer 1 reuses layer 0's relative-attention
    bias, as the reference passes one table to every layer) and the final
    RMSNorm against oracle.encoders.mt5_encoder with the same weights."""
    from transformers import MT5Config, MT5EncoderModel
    g = torch.Generator().manual_seed(12)
    B, L, D, H, F = 2, 36, 128, 2, 192
    cfg = MT5Config(vocab_size=64, d_model=D, d_kv=64, d_ff=F, num_layers=2, num_heads=H,
                    relative_attention_num_buckets=32, relative_attention_max_distance=128,
                    feed_forward_proj="gated-gelu", layer_norm_epsilon=1e-6, dropout_rate=0.0)
    m = MT5EncoderModel(cfg).eval().double()
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    table = r(32, H) * 0.5
    layers = []
    for i in range(2):
        wq, wk, wv, wo = (r(D, D) * 0.08 for _ in range(4))
        wi0, wi1, wff = r(D, F) * 0.08, r(D, F) * 0.08, r(F, D) * 0.08
        ln1, ln2 = 1 + 0.1 * r(D), 1 + 0.1 * r(D)
        layers.append((wq, wk, wv, wo, wi0, wi1, wff, ln1, ln2))
        sa, ff = m.encoder.block[i].layer[0], m.encoder.block[i].layer[1]
        with torch.no_grad():
            sa.SelfAttention.q.weight.copy_(wq.t()); sa.SelfAttention.k.weight.copy_(wk.t())
            sa.SelfAttention.v.weight.copy_(wv.t()); sa.SelfAttention.o.weight.copy_(wo.t())
            if i == 0:
                sa.SelfAttention.relative_attention_bias.weight.copy_(table)
            sa.layer_norm.weight.copy_(ln1)
            ff.DenseReluDense.wi_0.weight.copy_(wi0.t()); ff.DenseReluDense.wi_1.weight.copy_(wi1.t())
            ff.DenseReluDense.wo.weight.copy_(wff.t()); ff.layer_norm.weight.copy_(ln2)
    assert not m.encoder.block[1].layer[0].SelfAttention.has_relative_attention_bias
    lnf = 1 + 0.1 * r(D)
    with torch.no_grad():
        m.encoder.final_layer_norm.weight.copy_(lnf)
    x = r(B, L, D)
    keep = torch.ones(B, L, dtype=torch.float64)
    keep[0, 30:] = 0
    with torch.no_grad():
        want = m(inputs_embeds=x, attention_mask=keep).last_hidden_state
    mask = ((1.0 - keep) * torch.finfo(torch.float64).min)[:, None, None, :]
    got = oe.mt5_encoder(x, layers, table, lnf, mask, dtype=torch.float64)
    torch.testing.assert_close(got, want, rtol=0, atol=1e-5)
    # dropping the final RMSNorm or the second layer is far outside that bound
    assert (oe.mt5_encoder(x, layers[:1], table, lnf, mask, dtype=torch.float64) - want).abs().max() > 1e-2


def _deberta_small(seed=11):
    import encoders.deberta as ed
    return ed.random_weights(num_layers=3, hidden=128, heads=2, inter=256, position_buckets=16,
                             seed=seed, std=0.05, dtype=torch.float64)


def _hf_deberta(w):
    from transformers import DebertaV2Config
    from transformers.models.deberta_v2.modeling_deberta_v2 import DebertaV2Encoder
    cfg = DebertaV2Config(hidden_size=w.hidden, num_attention_heads=w.heads,
                          intermediate_size=w.inter, num_hidden_layers=len(w.layers),
                          relative_attention=True, position_buckets=w.position_buckets,
                          max_relative_positions=w.max_relative_positions,
                          pos_att_type=["p2c", "c2p"], share_att_key=True,
                          norm_rel_ebd="layer_norm", layer_norm_eps=w.eps, hidden_act="gelu",
                          hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0)
    m = DebertaV2Encoder(cfg).double().eval()
    sd = {"rel_embeddings.weight": w.rel_emb, "LayerNorm.weight": w.rel_ln_w,
          "LayerNorm.bias": w.rel_ln_b}
    for i, lw in enumerate(w.layers):
        p = f"layer.{i}."
        for name, wt, b in zip(("query_proj", "key_proj", "value_proj"), lw.wqkv.chunk(3),
                               lw.bqkv.chunk(3)):
            sd[p + f"attention.self.{name}.weight"] = wt
            sd[p + f"attention.self.{name}.bias"] = b
        sd.update({p + "attention.output.dense.weight": lw.wo, p + "attention.output.dense.bias": lw.bo,
                   p + "attention.output.LayerNorm.weight": lw.ln1_w,
                   p + "attention.output.LayerNorm.bias": lw.ln1_b,
                   p + "intermediate.dense.weight": lw.wi, p + "intermediate.dense.bias": lw.bi,
                   p + "output.dense.weight": lw.wo2, p + "output.dense.bias": lw.bo2,
                   p + "output.LayerNorm.weight": lw.ln2_w, p + "output.LayerNorm.bias": lw.ln2_b})
    m.load_state_dict(sd, strict=True)
    return m


def test_deberta_oracle_matches_transformers():
    """3 layers, 16 position buckets, max_relative_positions 64, L = 80 > 64 so
    both the log buckets and the clamp at +-2S are exercised; padded rows of
    the batch are ignored (the reference's kernel zeroes them, transformers
    does not)."""
    w = _deberta_small()
    w.max_relative_positions = 64
    lens = torch.tensor([80, 50, 33], dtype=torch.int32)
    B, L = 3, 80
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, L, w.hidden, generator=g, dtype=torch.float64)
    got = oe.deberta_encoder(x, lens, w, dtype=torch.float64)
    m = _hf_deberta(w)
    mask = (torch.arange(L)[None, :] < lens[:, None].long()).long()
    with torch.no_grad():
        want = m(x, mask, output_hidden_states=False).last_hidden_state
    for b in range(B):
        n = int(lens[b])
        # float64 throughout except transformers' scale sqrt(d * 3), taken in
        # float32 (relative error ~3e-8); a missing c2p/p2c term, a wrong
        # bucket or clamp differs by O(1e-2)
        torch.testing.assert_close(got[b, :n], want[b, :n], rtol=0, atol=1e-8)


def test_deberta_oracle_padding_invariance():
    """Valid rows do not depend on what the padded rows hold."""
    w = _deberta_small(seed=12)
    lens = torch.tensor([40, 21], dtype=torch.int32)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 48, w.hidden, generator=g, dtype=torch.float64)
    y = x.clone()
    y[0, 40:] = 7.0
    y[1, 21:] = -3.0
    a = oe.deberta_encoder(x, lens, w, dtype=torch.float64)
    b = oe.deberta_encoder(y, lens, w, dtype=torch.float64)
    torch.testing.assert_close(a[0, :40], b[0, :40], rtol=0, atol=1e-12)
    torch.testing.assert_close(a[1, :21], b[1, :21], rtol=0, atol=1e-12)


def _hf_deberta_v1(w):
    from transformers import DebertaConfig
    from transformers.models.deberta.modeling_deberta import DebertaEncoder
    cfg = DebertaConfig(hidden_size=w.hidden, num_attention_heads=w.heads,
                        intermediate_size=w.inter, num_hidden_layers=len(w.layers),
                        relative_attention=True, max_relative_positions=w.max_relative_positions,
                        pos_att_type=["c2p", "p2c"], layer_norm_eps=w.eps, hidden_act="gelu",
                        hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0)
    m = DebertaEncoder(cfg).double().eval()
    sd = {"rel_embeddings.weight": w.rel_emb}
    for i, lw in enumerate(w.layers):
        p = f"layer.{i}."
        sd.update({p + "attention.self.in_proj.weight": lw.in_proj,
                   p + "attention.self.q_bias": lw.q_bias, p + "attention.self.v_bias": lw.v_bias,
                   p + "attention.self.pos_proj.weight": lw.pos_proj,
                   p + "attention.self.pos_q_proj.weight": lw.pos_q_proj,
                   p + "attention.self.pos_q_proj.bias": lw.pos_q_bias,
                   p + "attention.output.dense.weight": lw.wo, p + "attention.output.dense.bias": lw.bo,
                   p + "attention.output.LayerNorm.weight": lw.ln1_w,
                   p + "attention.output.LayerNorm.bias": lw.ln1_b,
                   p + "intermediate.dense.weight": lw.wi, p + "intermediate.dense.bias": lw.bi,
                   p + "output.dense.weight": lw.wo2, p + "output.dense.bias": lw.bo2,
                   p + "output.LayerNorm.weight": lw.ln2_w, p + "output.LayerNorm.bias": lw.ln2_b})
    m.load_state_dict(sd, strict=True)
    return m


@pytest.mark.parametrize("L,max_rel", [(80, 64), (40, 64)])
def test_deberta_v1_oracle_matches_transformers(L, max_rel):
    """transformers' DeBERTa v1 DebertaEncoder with the same weights: linear
    positions, att_span = min(L, max_rel) (L = 80 > 64 clamps at +-S; L = 40
    slices the middle of the relative table). Padded query rows are ignored
    (transformers' 2-D mask hides every key of them, the flash path zeroes
    them)."""
    import encoders.deberta as ed
    w = ed.random_weights_v1(num_layers=2, hidden=128, heads=2, inter=256,
                             max_relative_positions=max_rel, seed=21, std=0.05,
                             dtype=torch.float64)
    lens = torch.tensor([L, L // 2 + 3, 17], dtype=torch.int32)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(3, L, w.hidden, generator=g, dtype=torch.float64)
    got = x
    for lw in w.layers:
        got = oe.deberta_v1_layer(got, lens, w.rel_emb, lw, w.heads, max_rel, w.eps, torch.float64)
    m = _hf_deberta_v1(w)
    mask = (torch.arange(L)[None, :] < lens[:, None].long()).long()
    with torch.no_grad():
        want = m(x, mask, output_hidden_states=False).last_hidden_state
    for b in range(3):
        n = int(lens[b])
        # transformers' v1 DebertaLayerNorm normalises in float32 (.float())
        # even in a float64 model, so outputs agree to ~1e-6; a missing c2p/p2c
        # term, a wrong clamp or span slice differs by O(1e-2)
        torch.testing.assert_close(got[b, :n], want[b, :n], rtol=0, atol=5e-6)


def test_mt5_fused_layer_weights_cached():
    """encoders.mt5.fused_layer_weights builds the q|k|v concatenation and the
    stacked GLU weight once per weight set (same objects on the next call,
    also for weights made under inference mode), rebuilds after an in-place
    update, and equals the plain torch constructions."""
    from encoders.mt5 import fused_layer_weights, stack_glu_weight
    g = torch.Generator().manual_seed(5)
    D, F_ = 128, 192
    mk = lambda *s: (torch.randn(*s, generator=g) * 0.02).bfloat16()
    lw = [mk(D, D), mk(D, D), mk(D, D), mk(D, D), mk(D, F_), mk(D, F_), mk(F_, D), None, None]
    a = fused_layer_weights(lw)
    assert torch.equal(a[0], torch.cat(lw[:3], 1))
    assert torch.equal(a[1], torch.cat((lw[4].t(), lw[5].t()), 0))
    assert torch.equal(a[1], stack_glu_weight(lw[4], lw[5]))
    b = fused_layer_weights(lw)
    assert b[0] is a[0] and b[1] is a[1]
    lw[1].add_(1.0)
    c = fused_layer_weights(lw)
    assert c[0] is not a[0] and torch.equal(c[0], torch.cat(lw[:3], 1))
    with torch.inference_mode():
        li = [t.clone() if t is not None else None for t in lw]
        d = fused_layer_weights(li)
        e = fused_layer_weights(li)
    assert d[0] is e[0] and torch.equal(d[0], c[0])
