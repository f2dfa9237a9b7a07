"""MI355X (gfx950) kernels behind the reference's `kernels/` call signatures.

Modules mirror the reference package one-to-one (same module and function
names, argument order, defaults and return conventions), so a caller that
does `from kernels.flash_attention_rpb import flash_attention_rpb_final`
with `vllm-factory_amd/` on sys.path gets the HIP implementation:

    flash_attention_rpb      -> flash_attention_rpb_final
    flash_deberta_attention  -> flash_deberta_attention, clear_config_cache
    fused_rope_global        -> fused_rope_apply, fused_rope_global_apply
    fused_rope_local         -> fused_rope_local_apply
    fused_layernorm          -> FusedLayerNorm, fused_layernorm
    fused_glu_mlp            -> fused_gelu_mul_dropout   ('gelu' = erf)
    ff_fused                 -> fused_gelu_mul_dropout   ('gelu' = tanh)
    fused_dropout_residual   -> fused_dropout_residual

plus ops with no reference kernel: varlen_attention.varlen_rope_attention
(ModernBERT packed local/global attention), packing (sequence boundaries from
flat position ids and flat <-> padded row copies, on the device),
rms_norm.RMSNorm, flash_deberta_attention.flash_deberta_attention_fused,
colbert_head (final LayerNorm + ColBERT projection + L2 normalisation), and
gliner_pooler (the GLiNER span pooler's prompt and word gathers for a whole
packed batch).
"""
