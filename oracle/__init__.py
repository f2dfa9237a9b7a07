"""CPU oracle for the encoder-attention hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU in PyTorch/numpy, the reference's *eager*
PyTorch path for every function on the hot path (vllm-factory: the mT5, DeBERTa-v2
and ModernBERT encoder layers and the kernels/ ops they call). Each function
cites the reference file:line it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
it, and only as the checker (or the timed CPU baseline). The product path in
vllm-factory_amd/ never imports, calls or falls back to anything here.

Modules:
  buckets    T5 and DeBERTa relative-position buckets (fp32 formulas)
  attention  RPB, disentangled and varlen local/global RoPE attention
  epilogues  LayerNorm, RMSNorm, GELU variants, RoPE tables, residual add
  encoders   layer-level restatements (ModernBERT, mT5, DeBERTa-v2)

How each function is pinned (golden vectors, closed forms, library routines,
brute force) is stated in its docstring and checked in tests/test_oracle_*.py.
"""
