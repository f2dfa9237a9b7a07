#!/usr/bin/env python3
"""Benchmark of the encoder-attention hot path on one MI355X.

Headline (one JSON line): ModernBERT-base attention on a varlen pack of 64
sequences with lengths U{512..768} (bf16, 12 heads, d 64). One step = one
global layer (RoPE theta 160000, full attention within each sequence) plus one
local layer (RoPE theta 10000, window +-64), both with RoPE applied in the
kernel. `value` = algorithmic attention TFLOP/s over valid pairs only:
sum_s 4*d*H*len_s^2 (global) + 4*d*H*#{|i-j| <= 64} (local).

Extra figures in the same line: per-kernel roofline of the dominant kernel,
the T5 RPB attention at mT5-large shapes, the DeBERTa disentangled attention,
the memory-bound epilogues in GB/s, the end-to-end tokens/s of the full
22-layer ModernBERT-base encoder over 256 packed sequences, and the CPU
oracle timed on the host.

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--no-cpu]
                       [--only headline|traffic|SECTION[,SECTION...]]
SECTION names the extra figures to run after the headline (rpb, deberta,
epilogues, glu_linear, qkv_rope, dense_ln, mt5_layer, deberta_layer,
deberta_v1_layer, encoder); the default runs all of them.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "vllm-factory_amd"))

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
SETTLE_S = 0.5              # busy time before the headline's warmup steps (clock ramp)


def _events(torch):
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


class KernelTimer:
    """Per-launch HIP-event timing on the current stream (the one the kernels use)."""

    def __init__(self, torch):
        self.torch = torch
        self.ms = {}

    def run(self, name, fn):
        s, e = _events(self.torch)
        s.record()
        out = fn()
        e.record()
        self.ms.setdefault(name, []).append((s, e))
        return out

    def avg_ms(self, name):
        ev = self.ms[name]
        return sum(s.elapsed_time(e) for s, e in ev) / len(ev)

    def reset(self):
        self.ms = {}


def traffic_workload(torch):
    """Workload of the FETCH_SIZE / WRITE_SIZE counter runs (--only traffic):
    three plain copies of a 512 MiB bf16 tensor (calibration: known bytes,
    larger than the last-level cache), then three calls each of the config-2
    global and local attention, the config-4 RPB attention, the config-3 fused
    DeBERTa attention and the config-5 ColBERT head."""
    import workloads
    from kernels.colbert_head import colbert_head
    from kernels.flash_attention_rpb import flash_attention_rpb_final
    from kernels.flash_deberta_attention import flash_deberta_attention_fused
    from kernels.varlen_attention import varlen_rope_attention

    dev = torch.device("cuda:0")
    x = torch.empty(256 * 1024 * 1024, dtype=torch.bfloat16, device=dev).normal_()
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    del x, y
    c = workloads.config2(device=dev)
    q, k, v = c.qkv[:, 0], c.qkv[:, 1], c.qkv[:, 2]
    out = torch.empty_like(q)
    for _ in range(3):
        varlen_rope_attention(q, k, v, c.cu_seqlens, c.max_seqlen, -1, 160000.0, 0.125, out=out)
        varlen_rope_attention(q, k, v, c.cu_seqlens, c.max_seqlen, 64, 10000.0, 0.125, out=out)
    del c, q, k, v, out
    c4 = workloads.config4(device=dev)
    B, L = c4.hidden.shape[:2]
    g = torch.Generator().manual_seed(1004)
    q4, k4, v4 = ((torch.randn(B, 16, L, 64, generator=g) * 0.64).bfloat16().to(dev) for _ in range(3))
    for _ in range(3):
        flash_attention_rpb_final(q4, k4, v4, c4.table, 32, 128, False, padding_mask=c4.mask)
    del c4, q4, k4, v4
    c3 = workloads.config3(device=dev)
    for _ in range(3):
        flash_deberta_attention_fused(c3.q, c3.k, c3.v, c3.lengths, c3.key_rel, c3.query_rel,
                                      c3.sm_scale, 256, 512, True)
    del c3
    T5 = 163736
    pend = torch.randn(T5, 768, generator=g).bfloat16().to(dev)
    resid = torch.randn(T5, 768, generator=g).bfloat16().to(dev)
    lnw = torch.ones(768, dtype=torch.bfloat16, device=dev)
    proj = (torch.randn(128, 768, generator=g) * 0.03).bfloat16().to(dev)
    for _ in range(3):
        colbert_head(pend, proj, None, lnw, None, 1e-5, residual=resid)
    torch.cuda.synchronize()
    print("traffic workload done", file=sys.stderr)


def measured_traffic(name):
    """HBM bytes per launch recorded by the rocprofv3 FETCH_SIZE / WRITE_SIZE
    runs summarised in profiles/<name> (line 'traffic_bytes_per_launch = N'),
    or None when that summary is absent."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch"):
                return int(line.split("=")[1])
    except OSError:
        pass
    return None


def settle(torch, fn, seconds, max_calls=1 << 30):
    """Runs fn back to back for about `seconds` of GPU time. The
    MI355X raises its clock over tens of milliseconds of load: measured on one
    box, the headline read 345-356 TFLOP/s after 5 warmup steps, 396-397 after
    50 and 405-407 after 200. Timing starts from that steady state; the
    warmup steps asked for still run after it."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(4):
        fn()
    torch.cuda.synchronize()
    per = max((time.perf_counter() - t0) / 4, 1e-5)
    # the calls are queued without a sync in between, so the GPU never idles
    for _ in range(min(int(seconds / per) + 1, max_calls)):
        fn()
    torch.cuda.synchronize()


def device_ms(torch, fn, n):
    """Average device time of fn over n back-to-back calls: a spin kernel first
    holds the stream so that all n launches are queued before the start event
    fires, which keeps host launch overhead out of short kernels' figures.
    The clock is settled first (about 0.1 s of queued calls, at most 2000)."""
    settle(torch, fn, 0.1, 2000)
    torch.cuda.synchronize()
    torch.cuda._sleep(20_000_000)  # ~10 ms of spinning at MI355X clocks
    s, e = _events(torch)
    s.record()
    for _ in range(n):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / n


def headline(torch, args):
    import workloads
    from kernels.varlen_attention import varlen_rope_attention

    dev = torch.device("cuda:0")
    c = workloads.config2(device=dev)
    q, k, v = c.qkv[:, 0], c.qkv[:, 1], c.qkv[:, 2]
    lens = c.lengths.tolist()
    H, d = 12, 64
    fl_global = sum(4 * d * H * n * n for n in lens)
    fl_local = sum(4 * d * H * workloads.window_pairs(n, 64) for n in lens)
    out_g = torch.empty_like(q)
    out_l = torch.empty_like(q)
    timer = KernelTimer(torch)

    def step():
        timer.run("global", lambda: varlen_rope_attention(q, k, v, c.cu_seqlens, c.max_seqlen, -1,
                                                           160000.0, 0.125, out=out_g))
        timer.run("local", lambda: varlen_rope_attention(q, k, v, c.cu_seqlens, c.max_seqlen, 64,
                                                          10000.0, 0.125, out=out_l))

    settle(torch, step, SETTLE_S)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    timer.reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    g_ms, l_ms = timer.avg_ms("global"), timer.avg_ms("local")
    value = (fl_global + fl_local) / (ms_step * 1e-3) / 1e12
    g_tf = fl_global / (g_ms * 1e-3) / 1e12
    l_tf = fl_local / (l_ms * 1e-3) / 1e12
    return dict(
        value=value, ms_per_step=ms_step, tokens=int(sum(lens)),
        roofline=dict(bound="mfma",
                      kernel="global attention call: rope_k_pack_kernel + varlen_fwd_kernel "
                             "(RoPE theta 160000)",
                      achieved=g_tf, peak=PEAK_BF16_TFLOPS, unit="TFLOP/s", frac=g_tf / PEAK_BF16_TFLOPS,
                      traffic=measured_traffic("varlen_global_traffic_config2.md"),
                      flops_per_launch=fl_global, avg_launch_ms=g_ms),
        kernels=dict(
            global_attn=dict(ms=g_ms, tflops=g_tf, gflop=fl_global / 1e9, frac=g_tf / PEAK_BF16_TFLOPS),
            local_attn=dict(ms=l_ms, tflops=l_tf, gflop=fl_local / 1e9, frac=l_tf / PEAK_BF16_TFLOPS),
        ),
    ), c


def rpb_config4(torch, args):
    """mT5-large RPB attention at config 4 shapes (B=32, L=768, lens U{512..768})."""
    import workloads
    from kernels.flash_attention_rpb import flash_attention_rpb_final

    dev = torch.device("cuda:0")
    c = workloads.config4(device=dev)
    B, L = c.hidden.shape[:2]
    g = torch.Generator().manual_seed(1004)
    q, k, v = ((torch.randn(B, 16, L, 64, generator=g) * 0.64).bfloat16().to(dev) for _ in range(3))
    lens = c.lengths.tolist()
    flops = sum(4 * 64 * 16 * n * n for n in lens)
    fn = lambda: flash_attention_rpb_final(q, k, v, c.table, 32, 128, False, padding_mask=c.mask)
    for _ in range(args.warmup):
        fn()
    ms = device_ms(torch, fn, args.steps)
    tf = flops / (ms * 1e-3) / 1e12
    # the same sequences packed (no padding): [T, 3, H, 64] rows of a fused
    # projection, the varlen RPB kernel
    from kernels.flash_attention_rpb import flash_attention_rpb_varlen
    cu = torch.tensor([0] + c.lengths.cumsum(0).tolist(), dtype=torch.int32, device=dev)
    qkv = torch.stack([torch.cat([t[b, :, :n].transpose(0, 1) for b, n in enumerate(lens)])
                       for t in (q, k, v)], 1).contiguous()
    fv = lambda: flash_attention_rpb_varlen(qkv[:, 0], qkv[:, 1], qkv[:, 2], cu, L, c.table, 32, 128)
    for _ in range(args.warmup):
        fv()
    vms = device_ms(torch, fv, args.steps)
    return dict(ms=ms, tflops=tf, gflop=flops / 1e9, frac=tf / PEAK_BF16_TFLOPS,
                note="queries and keys of padded rows excluded from the FLOP count",
                varlen_ms=vms, varlen_tflops=flops / (vms * 1e-3) / 1e12,
                varlen_note="the same sequences packed as [T, 3, 16, 64] rows, no mask")


def deberta_config3(torch, args):
    """DeBERTa-v3-large disentangled attention, config 3 (B=32, L=512, lens U{256..512}).
    Primary FLOP count includes the c2p/p2c projections over valid rows:
    sum_b H * (4 d len_b^2 + 4 d len_b 2S); the core-only count is also given."""
    import workloads
    from kernels.flash_deberta_attention import (flash_deberta_attention, flash_deberta_attention_fused,
                                                 rel_chunk_major)

    dev = torch.device("cuda:0")
    c = workloads.config3(device=dev)
    lens = c.lengths.tolist()
    H, d, S = 16, 64, 256
    core = sum(4 * d * H * n * n for n in lens)
    proj = sum(4 * d * H * n * 2 * S for n in lens)
    fused = lambda: flash_deberta_attention_fused(c.q, c.k, c.v, c.lengths, c.key_rel, c.query_rel,
                                                  c.sm_scale, 256, 512, True)
    kcm, qcm = rel_chunk_major(c.key_rel, S), rel_chunk_major(c.query_rel, S)
    fused_cm = lambda: flash_deberta_attention_fused(c.q, c.k, c.v, c.lengths, kcm, qcm,
                                                     c.sm_scale, 256, 512, True)
    pk = torch.matmul(c.q, c.key_rel.unsqueeze(0).transpose(-1, -2).contiguous())
    pq = torch.matmul(c.k, c.query_rel.unsqueeze(0).transpose(-1, -2).contiguous())
    gather = lambda: flash_deberta_attention(c.q, c.k, c.v, c.lengths, pk, pq, False, c.sm_scale,
                                             256, 512, True)
    times = {}
    for name, fn in (("fused", fused), ("fused_cm", fused_cm), ("gather", gather)):
        for _ in range(args.warmup):
            fn()
        times[name] = device_ms(torch, fn, args.steps)
    fm, gm = times["fused"], times["gather"]
    tf = (core + proj) / (fm * 1e-3) / 1e12
    return dict(fused_ms=fm, tflops=tf, frac=tf / PEAK_BF16_TFLOPS, gflop=(core + proj) / 1e9,
                core_gflop=core / 1e9, core_only_tflops=core / (fm * 1e-3) / 1e12,
                chunk_major_tables_ms=times["fused_cm"],
                note="fused_ms: the call on [H, 512, 64] key_rel / query_rel, converted to the "
                     "kernel's chunk-major layout inside the call; chunk_major_tables_ms: tables "
                     "already chunk-major, as the encoder layers produce them",
                gather_ms=gm, gather_note="reference interface: pos_key/pos_query [B,H,L,512] "
                                          "precomputed outside the timed region")


def epilogue_bench(torch, args, c2):
    import workloads
    from kernels.fused_layernorm import fused_layernorm
    from kernels.fused_rope_global import fused_rope_global_apply
    from kernels.rms_norm import rms_norm
    from kernels.ff_fused import fused_gelu_mul_dropout as ffg

    dev = torch.device("cuda:0")
    T = c2.qkv.shape[0]
    res = {}

    def bench(name, fn, nbytes):
        for _ in range(args.warmup):
            fn()
        ms = device_ms(torch, fn, args.steps)
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = dict(ms=ms, gbs=gbs, mb=nbytes / 1e6, frac=gbs / PEAK_HBM_GBS)

    # RoPE (table form, the drop-in kernel): q, k [1, T, 12, 64] bf16, cos/sin [1, T, 64]
    q = c2.qkv[:, 0].contiguous().view(1, T, 12, 64)
    k = c2.qkv[:, 1].contiguous().view(1, T, 12, 64)
    pos = torch.cat([torch.arange(int(n)) for n in c2.lengths]).to(dev)
    inv = 1.0 / (160000.0 ** (torch.arange(0, 64, 2, device=dev).float() / 64))
    fr = pos.float()[:, None] * inv[None]
    emb = torch.cat([fr, fr], -1)
    cos, sin = emb.cos().bfloat16()[None], emb.sin().bfloat16()[None]
    bench("rope_qk", lambda: fused_rope_global_apply(q, k, cos, sin), 4 * T * 768 * 2 + 2 * T * 64 * 2)
    res["rope_qk"]["launches"] = 1
    # LayerNorm [T, 768] bf16, no bias (ModernBERT)
    g = torch.Generator().manual_seed(1002)
    x = torch.randn(T, 768, generator=g).bfloat16().to(dev)
    w = torch.ones(768, dtype=torch.bfloat16, device=dev)
    bench("layernorm", lambda: fused_layernorm(x, 768, w, None, 1e-5), 2 * T * 768 * 2)
    # mT5 RMSNorm and gated-GELU at config 4 sizes on the packed valid rows
    # (20 280 of the 24 576 padded rows), as the packed mT5 layer runs them
    c4 = workloads.config4(device=dev)
    tv = int(c4.lengths.sum())
    keep = (torch.arange(c4.hidden.shape[1], device=dev)[None, :] < c4.lengths.to(dev)[:, None])
    h = c4.hidden[keep].contiguous()
    bench("rmsnorm", lambda: rms_norm(h, c4.ln1, 1e-6), 2 * tv * 1024 * 2)
    gate = torch.randn(tv, 2816, generator=g).bfloat16().to(dev)
    up = torch.randn(tv, 2816, generator=g).bfloat16().to(dev)
    bench("gated_gelu", lambda: ffg(gate, up, "gelu_new"), 3 * tv * 2816 * 2)
    res["rmsnorm"]["rows"] = res["gated_gelu"]["rows"] = tv
    del c4, gate, up, h
    # flat <-> padded rows of the DeBERTa-v3-large GLiNER flat call at config 3
    # sizes: 32 sequences U{256..512} of 1024 bf16 hidden values
    from kernels.packing import pad_packed, unpad_packed
    hid, lens3 = workloads.config3_hidden(32)
    cu3 = workloads.cu_from_lengths(lens3.long()).to(dev)
    T3, L3 = int(lens3.sum()), int(lens3.max())
    flat = torch.cat([hid[b, :int(n)] for b, n in enumerate(lens3)]).bfloat16().to(dev)
    padded, _ = pad_packed(flat, cu3, 32, L3)
    row = 1024 * 2
    bench("pad_rows", lambda: pad_packed(flat, cu3, 32, L3), (T3 + 32 * L3) * row)
    bench("unpad_rows", lambda: unpad_packed(padded, cu3, T3), 2 * T3 * row)
    del hid, flat, padded
    # ColBERT head at config 5 size: last residual add + final LayerNorm +
    # projection 768 -> 128 + L2 norm, fused vs the unfused composition
    # (LayerNorm kernel, hipBLASLt GEMM, torch normalize)
    import torch.nn.functional as F
    from kernels.colbert_head import colbert_head
    from kernels.fused_layernorm import fused_add_layernorm
    T5 = 163736
    pend = torch.randn(T5, 768, generator=g).bfloat16().to(dev)
    resid = torch.randn(T5, 768, generator=g).bfloat16().to(dev)
    lnw = torch.ones(768, dtype=torch.bfloat16, device=dev)
    proj = (torch.randn(128, 768, generator=g) * 0.03).bfloat16().to(dev)
    hb = (2 * T5 * 768 + T5 * 128) * 2
    bench("colbert_head", lambda: colbert_head(pend, proj, None, lnw, None, 1e-5, residual=resid), hb)

    def unfused():
        h, _ = fused_add_layernorm(pend, resid, lnw, None, 1e-5)
        return F.normalize(F.linear(h, proj), dim=-1, eps=1e-8)
    bench("colbert_head_unfused", unfused, hb)
    del pend, resid
    # GLiNER pooler front-end over 256 packed prompt + text requests of
    # U{512..768} tokens, bf16 768: class-token compaction, first-subtoken
    # word index, prompt rows and word rows. The whole call includes its one
    # read-back; the word-row gather, which moves most of the bytes, is also
    # timed alone.
    from kernels import _lib
    from kernels.gliner_pooler import gliner_reps_packed
    gr = workloads.gliner_requests()
    Tg = gr.ids.numel()
    hg = torch.randn(Tg, 768, generator=g).bfloat16().to(dev)
    ids_g, wm_g, cu_g = gr.ids.to(dev), gr.words_mask.to(dev), gr.cu_seqlens.to(dev)
    pe, pe_cu, we, we_cu = gliner_reps_packed(hg, ids_g, wm_g, cu_g, gr.text_lengths,
                                              gr.ent_token_id)
    C, W = pe.shape[0], we.shape[0]
    row = 768 * 2
    bench("gliner_reps", lambda: gliner_reps_packed(hg, ids_g, wm_g, cu_g, gr.text_lengths,
                                                     gr.ent_token_id),
          16 * Tg + 2 * (C + W) * row)
    wcu = we_cu.to(device=dev, dtype=torch.int32)
    src = torch.zeros(W, dtype=torch.int32, device=dev)
    _lib.on_device("vfk_gliner_word_index", dev, wm_g.data_ptr(), Tg, cu_g.data_ptr(),
                   cu_g.numel() - 1, wcu.data_ptr(), src.data_ptr(), None)
    bench("gliner_word_index", lambda: _lib.on_device(
        "vfk_gliner_word_index", dev, wm_g.data_ptr(), Tg, cu_g.data_ptr(), cu_g.numel() - 1,
        wcu.data_ptr(), src.data_ptr(), None), 8 * Tg + 4 * W)
    bench("gliner_word_rows", lambda: _lib.on_device(
        "vfk_gliner_word_rows", dev, hg.data_ptr(), row, Tg, src.data_ptr(), W, we.data_ptr()),
        4 * W + 2 * W * row)
    res["gliner_reps"].update(tokens=Tg, class_rows=C, word_rows=W)
    # SpanMarkerV0 pair rows for the same 256 requests: default spans of
    # width 12 over each request's word rows, relu(cat(start[i], end[j]))
    # written as [S, 1536] bf16 (the projections are random rows here)
    from kernels.gliner_pooler import default_spans, gliner_span_rows
    lens_w = [int(t) for t in gr.text_lengths]
    sp = [default_spans(n, n, 12) for n in lens_w]
    s_idx = torch.cat([x[0] for x in sp]).to(dev)
    s_mask = torch.cat([x[1] for x in sp]).to(dev)
    row_cu = we_cu.to(device=dev, dtype=torch.int32)
    span_cu = torch.tensor([0] + torch.tensor([x[0].shape[0] for x in sp]).cumsum(0).tolist(),
                           dtype=torch.int32, device=dev)
    S = int(span_cu[-1])
    st_rep = torch.randn(W, 768, generator=g).bfloat16().to(dev)
    en_rep = torch.randn(W, 768, generator=g).bfloat16().to(dev)
    bench("gliner_span_rows", lambda: gliner_span_rows(st_rep, en_rep, row_cu, s_idx, s_mask, span_cu),
          S * (2 * row + 24) + 2 * W * row)
    res["gliner_span_rows"].update(spans=S)
    # the marker's out_project first layer (Linear(1536, 3072) + ReLU) on all
    # spans: pair rows then the [S, 1536] x [1536, 3072] GEMM, against the
    # split form (relu(start) W1a^T and relu(end) W1b^T per word row, then
    # relu(a[i] + b[j] + b1) per span); both end with [S, 3072] bf16
    from kernels.activation import activation
    from kernels.gliner_pooler import gliner_span_hidden
    w1 = (torch.randn(3072, 1536, generator=g) * 0.02).bfloat16().to(dev)
    b1 = (torch.randn(3072, generator=g) * 0.02).bfloat16().to(dev)
    w1a, w1b = w1[:, :768].contiguous(), w1[:, 768:].contiguous()

    def pair_linear():
        return torch.relu_(torch.addmm(b1, gliner_span_rows(st_rep, en_rep, row_cu, s_idx, s_mask, span_cu),
                                       w1.t()))

    def split_linear():
        a = torch.matmul(activation(st_rep, "relu"), w1a.t())
        b = torch.matmul(activation(en_rep, "relu"), w1b.t())
        return gliner_span_hidden(a, b, b1, row_cu, s_idx, s_mask, span_cu)
    ha = torch.matmul(activation(st_rep, "relu"), w1a.t())
    hb = torch.matmul(activation(en_rep, "relu"), w1b.t())
    bench("gliner_span_hidden", lambda: gliner_span_hidden(ha, hb, b1, row_cu, s_idx, s_mask, span_cu),
          S * (3072 * 2 + 24) + 2 * W * 3072 * 2)
    res["gliner_span_hidden"].update(spans=S, note="bytes: output rows, index lists and a, b read once")
    del ha, hb
    for name, fn in (("span_first_layer_pair_rows", pair_linear), ("span_first_layer_split", split_linear)):
        for _ in range(max(1, args.warmup // 5)):
            fn()
        res[name] = dict(ms=device_ms(torch, fn, max(2, args.steps // 10)), spans=S)
    res["span_first_layer_split"]["speedup"] = (res["span_first_layer_pair_rows"]["ms"]
                                                / res["span_first_layer_split"]["ms"])
    hid = split_linear()
    ref = pair_linear()
    res["span_first_layer_split"]["max_abs_vs_pair"] = (hid.float() - ref.float()).abs().max().item()
    del hid, ref
    return res


def encoder_config5(torch, args):
    """Full ModernBERT-base encoder forward (22 layers, random-init bf16 weights)
    over 256 packed sequences U{512..768}: end-to-end tokens/s and sequences/s."""
    import workloads
    from encoders.modernbert import modernbert_forward, random_weights

    dev = torch.device("cuda:0")
    c = workloads.config5()
    w = random_weights().to(dev)
    ids, cu = c.ids.to(dev), c.cu_seqlens.to(dev)
    fn = lambda: modernbert_forward(ids, cu, c.max_seqlen, w)
    for _ in range(max(2, args.warmup // 5)):
        fn()
    torch.cuda.synchronize()
    n = max(3, args.steps // 10)
    t0 = time.perf_counter()
    for _ in range(n):
        fn()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / n
    T = int(c.lengths.sum())
    del w
    # sequence boundaries from the flat position ids (the reference's input),
    # on the device: 4 small launches, int64 positions in, cu_seqlens out
    from kernels.varlen_attention import seq_metadata
    pos = torch.cat([torch.arange(int(n)) for n in c.lengths]).to(dev)
    for _ in range(args.warmup):
        seq_metadata(pos)
    meta_ms = device_ms(torch, lambda: seq_metadata(pos), args.steps)
    return dict(ms_per_forward=ms, tokens_per_s=T / (ms * 1e-3),
                sequences_per_s=len(c.lengths) / (ms * 1e-3), tokens=T, layers=22,
                seq_metadata_us=meta_ms * 1e3,
                note="wall clock per forward (embeddings to final LayerNorm), GEMMs via torch/hipBLASLt")


def glu_linear_config5(torch, args):
    """ModernBERT-base MLP projection over the 256-sequence pack (x [163 736,
    768] bf16, Wi [2304, 768]): the fused GLU projection (vfk_glu_linear_fwd,
    act(x W_in^T) * (x W_gate^T) in one MFMA kernel) against the unfused path
    (hipBLASLt F.linear, then the GELU-gate kernel) and the plain GEMM."""
    import torch.nn.functional as F
    from kernels.fused_glu_mlp import fused_gelu_mul_dropout, glu_linear

    dev = torch.device("cuda:0")
    M, K, I = 163736, 768, 1152
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(2 * I, K, device=dev, generator=g) * 0.036).to(torch.bfloat16)
    out = torch.empty(M, I, device=dev, dtype=torch.bfloat16)
    fused = lambda: glu_linear(x, w, "gelu", out=out)

    def unfused():
        y = F.linear(x, w)
        return fused_gelu_mul_dropout(y[:, :I], y[:, I:], "gelu")

    gemm = lambda: F.linear(x, w)
    # interleaved rounds, best of 3 per path: the first kernels of a process
    # run before the clock has settled
    res = {}
    for _ in range(3):
        for name, fn in (("fused", fused), ("unfused", unfused), ("gemm_only", gemm)):
            for _ in range(args.warmup):
                fn()
            ms = device_ms(torch, fn, args.steps)
            res[name] = min(res.get(name, ms), ms)
    flop = 2.0 * M * K * 2 * I
    return dict(fused_ms=res["fused"], unfused_ms=res["unfused"], hipblaslt_gemm_ms=res["gemm_only"],
                gflop=flop / 1e9, fused_tflops=flop / (res["fused"] * 1e-3) / 1e12,
                fused_frac=flop / (res["fused"] * 1e-3) / 2.5e15,
                note="fused: one kernel writes [M, 1152]; unfused: [M, 2304] projection + GELU-gate pass")


def dense_ln_config3(torch, args):
    """DeBERTa post-LN output block at the config-3 batch shape (32 x 512 =
    16 384 rows): LayerNorm(x W^T + b + residual) as one kernel
    (dense_add_layernorm, packed weight) against hipBLASLt F.linear plus the
    residual + LayerNorm pass, at the attention output's square projection of
    DeBERTa-base (768) and -large (1024) and the -large FFN output (K 4096)."""
    import torch.nn.functional as F
    from kernels.dense_layernorm import dense_add_layernorm, pack_dense_weight
    from kernels.fused_layernorm import fused_add_layernorm

    dev = torch.device("cuda:0")
    M = 32 * 512
    out = {}
    for tag, N, K in (("base_attn_out", 768, 768), ("large_attn_out", 1024, 1024),
                      ("large_ffn_out", 1024, 4096)):
        g = torch.Generator(device=dev).manual_seed(N + K)
        x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
        w = (torch.randn(N, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
        b = (0.1 * torch.randn(N, device=dev, generator=g)).to(torch.bfloat16)
        r = torch.randn(M, N, device=dev, generator=g).to(torch.bfloat16)
        lw = torch.ones(N, device=dev, dtype=torch.bfloat16)
        lb = torch.zeros(N, device=dev, dtype=torch.bfloat16)
        wp = pack_dense_weight(w)
        o = torch.empty_like(r)
        fused = lambda: dense_add_layernorm(x, None, b, r, lw, lb, 1e-7, out=o, packed_weight=wp)
        unfused = lambda: fused_add_layernorm(F.linear(x, w, b), r, lw, lb, 1e-7, return_sum=False)
        res = {}
        for _ in range(3):
            for name, fn in (("fused", fused), ("unfused", unfused)):
                for _ in range(args.warmup):
                    fn()
                ms = device_ms(torch, fn, args.steps)
                res[name] = min(res.get(name, ms), ms)
        flop = 2.0 * M * N * K
        out[tag] = dict(N=N, K=K, fused_ms=res["fused"], unfused_ms=res["unfused"],
                        fused_tflops=flop / (res["fused"] * 1e-3) / 1e12,
                        fused_frac=flop / (res["fused"] * 1e-3) / 2.5e15)
    out["note"] = ("fused: vfk_dense_residual_layernorm_fwd (the [M, N] projection never written); "
                   "unfused: hipBLASLt GEMM with bias, then the residual + LayerNorm pass; "
                   "best of 3 interleaved rounds")
    return out


def qkv_rope_config5(torch, args):
    """ModernBERT-base attention block input side over the 256-sequence pack
    (x [163 736, 768] bf16, Wqkv [2304, 768], token-50284 key mask): the fused
    q | k | v projection with the k rotation in the GEMM epilogue plus the
    attention over its rotated k (qkv_rope_projection +
    varlen_rope_attention_krot), against hipBLASLt F.linear plus the attention
    call with its k pre-pass (varlen_rope_attention); global and local layers,
    and the two projections alone."""
    import math
    import torch.nn.functional as F

    import workloads
    from kernels.varlen_attention import (qkv_rope_projection, token_positions,
                                          varlen_rope_attention, varlen_rope_attention_krot)

    dev = torch.device("cuda:0")
    c = workloads.config5()
    cu = c.cu_seqlens.to(dev)
    M, K, H = int(c.ids.numel()), 768, 12
    g = torch.Generator(device=dev).manual_seed(4)
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(3 * K, K, device=dev, generator=g) * 0.036).to(torch.bfloat16)
    key_valid = (c.ids != 50284).to(dev)
    pos = token_positions(cu, M)
    scale = 1.0 / math.sqrt(64)
    res = {}
    for name, window, theta in (("global", -1, 160000.0), ("local", 64, 10000.0)):
        def fused():
            r = qkv_rope_projection(x, w, H, pos, c.max_seqlen, theta, scale)
            return varlen_rope_attention_krot(r, cu, c.max_seqlen, window, key_valid)

        def unfused():
            qkv = F.linear(x, w).view(M, 3, H, 64)
            return varlen_rope_attention(qkv[:, 0], qkv[:, 1], qkv[:, 2], cu, c.max_seqlen, window,
                                         theta, scale, key_valid)
        for _ in range(2):
            for tag, fn in (("fused", fused), ("unfused", unfused)):
                for _ in range(args.warmup):
                    fn()
                ms = device_ms(torch, fn, args.steps)
                key = f"{name}_{tag}_ms"
                res[key] = min(res.get(key, ms), ms)
    proj = lambda: qkv_rope_projection(x, w, H, pos, c.max_seqlen, 160000.0, scale)
    gemm = lambda: F.linear(x, w)
    for _ in range(2):
        for tag, fn in (("projection_fused_ms", proj), ("projection_hipblaslt_ms", gemm)):
            for _ in range(args.warmup):
                fn()
            ms = device_ms(torch, fn, args.steps)
            res[tag] = min(res.get(tag, ms), ms)
    flop = 2.0 * M * K * 3 * K
    res.update(gflop_projection=flop / 1e9,
               projection_fused_tflops=flop / (res["projection_fused_ms"] * 1e-3) / 1e12,
               note="fused: projection writes q, v and the rotated k, attention reads the rotated "
                    "k; unfused: [M, 2304] projection, then k pre-pass + attention")
    return res


def mt5_layer_config4(torch, args):
    """One mT5-large encoder layer (RMSNorm, RPB attention, gated-GELU FFN) at
    config 4 (B=32, L=768, lengths U{512..768}); tokens/s over valid tokens."""
    import workloads
    from encoders.mt5 import mt5_layer_forward

    dev = torch.device("cuda:0")
    c = workloads.config4(device=dev)
    ws = (c.wq, c.wk, c.wv, c.wo, c.wi0, c.wi1, c.wff_o, c.ln1, c.ln2, c.table)
    from encoders.mt5 import mt5_layer_packed
    from kernels.packing import unpad_packed
    fn = lambda: mt5_layer_forward(c.hidden, *ws, c.mask)
    tv = int(c.lengths.sum())
    cu = torch.cat([c.lengths.new_zeros(1), c.lengths.cumsum(0)]).to(device=dev, dtype=torch.int32)
    xf = unpad_packed(c.hidden, cu, tv)
    wqkv = torch.cat((c.wq, c.wk, c.wv), 1)
    L = c.hidden.shape[1]
    fp = lambda: mt5_layer_packed(xf, cu, L, *ws, c.mask, wqkv=wqkv)
    from encoders.mt5 import stack_glu_weight
    wg = stack_glu_weight(c.wi0, c.wi1)
    ff = lambda: mt5_layer_packed(xf, cu, L, *ws, c.mask, wqkv=wqkv, wi_glu=wg)
    res = {}
    for name, f in (("padded", fn), ("packed", fp), ("packed_glu", ff)):
        for _ in range(args.warmup):
            f()
        res[name] = device_ms(torch, f, args.steps)
    ms = res["packed_glu"]
    return dict(ms_per_layer=ms, valid_tokens_per_s=tv / (ms * 1e-3), valid_tokens=tv,
                padded_tokens=int(c.hidden.shape[0] * c.hidden.shape[1]),
                padded_layer_ms=res["padded"], packed_unfused_ff_ms=res["packed"],
                note="ms_per_layer: the layer on the packed valid rows (mt5_layer_packed) with the "
                     "gated FF as one GLU projection kernel; packed_unfused_ff_ms: the same with "
                     "two GEMMs + the gelu_new gate pass; padded_layer_ms: the padded batch")


def deberta_layer_config3(torch, args):
    """One DeBERTa-v3-large encoder layer (projections, disentangled attention,
    LayerNorms, GELU FFN) at config 3 (B=32, L=512, lengths U{256..512});
    tokens/s over valid tokens."""
    import workloads
    from encoders.deberta import deberta_layer_forward, deberta_rel_embeddings, random_weights

    dev = torch.device("cuda:0")
    hidden, lens = workloads.config3_hidden()
    x, sl = hidden.to(dev, torch.bfloat16), lens.to(dev)
    w = random_weights(num_layers=1).to(dev)
    rel = deberta_rel_embeddings(w)
    from encoders.deberta import deberta_layer_packed
    from kernels.packing import unpad_packed
    fn = lambda: deberta_layer_forward(x, sl, rel, w.layers[0], w)
    tv = int(lens.sum())
    cu = torch.cat([lens.new_zeros(1), lens.cumsum(0)]).to(device=dev, dtype=torch.int32)
    xf = unpad_packed(x, cu, tv)
    L = x.shape[1]
    fp = lambda: deberta_layer_packed(xf, cu, L, rel, w.layers[0], w)
    res = {}
    for name, f in (("padded", fn), ("packed", fp)):
        for _ in range(args.warmup):
            f()
        res[name] = device_ms(torch, f, args.steps)
    ms = res["packed"]
    return dict(ms_per_layer=ms, valid_tokens_per_s=tv / (ms * 1e-3), valid_tokens=tv,
                padded_tokens=int(x.shape[0] * x.shape[1]), padded_layer_ms=res["padded"],
                note="ms_per_layer: the layer on the packed valid rows (deberta_layer_packed, "
                     "varlen attention); padded_layer_ms: the same layer over the padded batch")


def deberta_v1_layer_config3(torch, args):
    """One DeBERTa v1 (deberta-base: hidden 768, 12 heads, GELU 3072, linear
    relative positions, max_relative_positions 512) encoder layer on the
    config-3 batch shape (B=32, L=512, lengths U{256..512}); tokens/s over
    valid tokens."""
    import workloads
    from encoders.deberta import deberta_v1_layer_forward, random_weights_v1

    dev = torch.device("cuda:0")
    _, lens = workloads.config3_hidden()
    g = torch.Generator().manual_seed(1013)
    x = torch.randn(32, 512, 768, generator=g).to(dev, torch.bfloat16)
    sl = lens.to(dev)
    w = random_weights_v1(num_layers=1).to(dev)
    fn = lambda: deberta_v1_layer_forward(x, sl, w.layers[0], w)
    fu = lambda: deberta_v1_layer_forward(x, sl, w.layers[0], w, fuse_dense_ln=False)
    res = {}
    for name, f in (("fused", fn), ("unfused", fu)):
        for _ in range(args.warmup):
            f()
        res[name] = device_ms(torch, f, args.steps)
    ms = res["fused"]
    tv = int(lens.sum())
    return dict(ms_per_layer=ms, valid_tokens_per_s=tv / (ms * 1e-3), valid_tokens=tv,
                padded_tokens=32 * 512, unfused_dense_ln_ms=res["unfused"],
                note="unfused_dense_ln_ms: the attention output's dense + residual + LayerNorm "
                     "as GEMM + LayerNorm pass instead of one kernel")


def cpu_baseline(torch, c2, min_seconds=10.0):
    """The oracle (CPU restatement of the reference's eager path, fp32) on the
    host cores: global + local attention over the config-2 sequences, cycling
    through them until about min_seconds of CPU work are done, reported as
    TFLOP/s of the same algorithmic count."""
    sys.path.insert(0, ROOT)
    import workloads
    from oracle import attention as oa

    # every core this process may run on (the host's CPUs minus any affinity
    # restriction the box places on the job)
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    model = ""
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    qkv = c2.qkv.float().cpu()
    cu = c2.cu_seqlens.cpu().tolist()
    lens = c2.lengths.tolist()
    flops = 0
    done = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < min_seconds:
        s = done % len(lens)
        a, b = cu[s], cu[s + 1]
        sub = qkv[a:b]
        cus = torch.tensor([0, b - a], dtype=torch.int32)
        oa.varlen_attention(sub[:, 0], sub[:, 1], sub[:, 2], cus, -1, 160000.0, None, 0.125)
        oa.varlen_attention(sub[:, 0], sub[:, 1], sub[:, 2], cus, 64, 10000.0, None, 0.125)
        n = b - a
        flops += 4 * 64 * 12 * (n * n + workloads.window_pairs(n, 64))
        done += 1
    dt = time.perf_counter() - t0
    return dict(value=flops / dt / 1e12, unit="TFLOP/s", cores=threads, kind="port",
                host_cpus=os.cpu_count(), cpu_model=model, dtype="fp32",
                sample=f"{done} sequence-layer pairs cycling over the {len(lens)} config-2 sequences "
                       f"(global + local layer each), fp32 oracle, per-sequence dense softmax, "
                       f"{dt:.1f} s")


def _progress(what):
    print(f"[bench] {what} done", file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="", help="'headline' to skip the extra figures; 'traffic' "
                    "runs only the workload of the HBM-traffic counter runs; a comma list of "
                    "sections runs the headline and those")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the path is "
              "data-parallel with no exchange step: N GPUs each run the same kernels on their "
              "share of sequences)", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.only == "traffic":
        traffic_workload(torch)
        return
    head, c2 = headline(torch, args)
    _progress("headline")
    extra = {}
    sections = (("rpb", "rpb_mt5_large_config4", lambda: rpb_config4(torch, args)),
                ("deberta", "deberta_v3_large_config3", lambda: deberta_config3(torch, args)),
                ("epilogues", "epilogues", lambda: epilogue_bench(torch, args, c2)),
                ("glu_linear", "glu_linear_modernbert_config5", lambda: glu_linear_config5(torch, args)),
                ("qkv_rope", "qkv_rope_modernbert_config5", lambda: qkv_rope_config5(torch, args)),
                ("dense_ln", "dense_ln_deberta_config3", lambda: dense_ln_config3(torch, args)),
                ("mt5_layer", "mt5_large_layer_config4", lambda: mt5_layer_config4(torch, args)),
                ("deberta_layer", "deberta_v3_large_layer_config3",
                 lambda: deberta_layer_config3(torch, args)),
                ("deberta_v1_layer", "deberta_v1_base_layer_config3",
                 lambda: deberta_v1_layer_config3(torch, args)),
                ("encoder", "modernbert_encoder_config5", lambda: encoder_config5(torch, args)))
    wanted = None if not args.only else set(args.only.split(","))
    unknown = (wanted or set()) - {s[0] for s in sections} - {"headline"}
    if unknown:
        print(f"unknown sections {sorted(unknown)}", file=sys.stderr)
        sys.exit(2)
    for short, key, fn in sections:
        if wanted is None or short in wanted:
            extra[key] = fn()
            _progress(key)
    line = {
        "metric": "encoder attn TFLOP/s + % bf16 MFMA peak at L=512-768; end-to-end tokens/s",
        "value": head["value"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded, random-init Wqkv ~ N(0,0.02))",
        "config": {"workload": "ModernBERT-base attention, 64 varlen-packed sequences U{512..768} "
                               "(T=%d), 12 heads x 64, global (RoPE 160000) + local +-64 (RoPE 10000)"
                               % head["tokens"],
                   "global_batch": 64, "seq_len": "512-768", "parallelism": "none (1 GPU)",
                   "settle_s": SETTLE_S},
        "roofline": head["roofline"],
        "kernels": head["kernels"],
        "extra": extra,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(torch, c2)
        _progress("cpu_baseline")
    print(json.dumps(line))


if __name__ == "__main__":
    main()
