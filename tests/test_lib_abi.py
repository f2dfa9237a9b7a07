"""The C ABI library loads on a CPU-only host, exports every symbol that
include/vfk.h declares, and its host-side bucket helpers are bit-exact with
the oracle. No GPU compute is issued here."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from oracle import buckets as ob

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    src = open(os.path.join(ROOT, "include", "vfk.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(vfk_[a-z0-9_]+)\s*\(", src)))


def test_header_symbols_exported():
    from kernels import _lib
    lib = _lib.load()
    syms = _declared_symbols()
    assert len(syms) >= 13
    for s in syms:
        assert hasattr(lib, s), s
    assert set(syms) <= set(_lib._SIGNATURES) | {"vfk_last_error"}


def test_abi_version():
    from kernels import _lib
    assert _lib.load().vfk_abi_version() == 19


def _host_t5(rel, bidirectional, nb, md):
    from kernels import _lib
    rel = np.ascontiguousarray(rel, dtype=np.int64)
    out = np.zeros(rel.shape, dtype=np.int32)
    _lib.call("vfk_t5_bucket", rel.ctypes.data, out.ctypes.data, rel.size,
              int(bidirectional), nb, md)
    return out


def _host_deb(rel, bs, mp):
    from kernels import _lib
    rel = np.ascontiguousarray(rel, dtype=np.int64)
    out = np.zeros(rel.shape, dtype=np.int32)
    _lib.call("vfk_deberta_bucket", rel.ctypes.data, out.ctypes.data, rel.size, bs, mp)
    return out


@pytest.mark.parametrize("bidirectional", [True, False])
@pytest.mark.parametrize("nb,md", [(32, 128), (32, 64), (64, 256), (16, 100), (128, 1024)])
def test_t5_host_bucket_matches_oracle(bidirectional, nb, md):
    # full [L, L] matrix like the reference evaluates it
    L = 1200
    want = ob.t5_bucket_matrix(L, L, bidirectional, nb, md).numpy()
    rel = (np.arange(L)[None, :] - np.arange(L)[:, None]).astype(np.int64)
    got = _host_t5(rel, bidirectional, nb, md)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("bs,mp", [(256, 512), (256, 1024), (128, 512), (64, 256)])
def test_deberta_host_bucket_matches_oracle(bs, mp):
    L = 1100
    want = ob.build_relative_position_v2(L, L, bs, mp)[0].numpy()
    rel = (np.arange(L)[:, None] - np.arange(L)[None, :]).astype(np.int64)
    got = _host_deb(rel, bs, mp)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("pb,mrp", [(256, 512), (256, 1024), (128, 512), (64, 128), (256, 256),
                                    (256, 300), (128, 128), (64, 64)])
def test_deberta_unit_steps_matches_oracle(pb, mrp):
    """vfk_deberta_unit_steps reports whether the clamped index
    clamp(bucket(d) + S, 0, 2S - 1) moves by at most 1 per unit of d, as the
    oracle's bucket matrix shows it (256/256, 256/300 and 128/128 jump by 2)."""
    from kernels import _lib
    L = 1100
    S = pb
    c = torch.clamp(ob.build_relative_position_v2(L, L, pb, mrp)[0][0] + S, 0, 2 * S - 1)
    want = int((c[:-1] - c[1:]).abs().max() <= 1)  # row 0: d = -j, consecutive keys
    assert _lib.load().vfk_deberta_unit_steps(pb, mrp, 1, L) == want
    assert _lib.load().vfk_deberta_unit_steps(pb, mrp, 0, L) == 1   # linear positions
    if (pb, mrp) in ((256, 256), (256, 300), (128, 128)):
        assert want == 0


def test_noalloc_meta_rejects_sizes_above_its_array():
    """vfk_varlen_meta_noalloc checks total_tokens against its built-in array
    before any HIP call, so the rejection runs without a GPU."""
    from kernels import _lib
    lib = _lib.load()
    rc = lib.vfk_varlen_meta_noalloc(None, 8, 16384 * 1024 + 1, 0, None, None, None)
    assert rc == -2
    assert b"above the 16777216" in lib.vfk_last_error()


def test_invalid_arguments_raise():
    from kernels import _lib
    # num_buckets too small for the T5 formula: rejected, nothing launched
    rel = np.zeros(4, dtype=np.int64)
    out = np.zeros(4, dtype=np.int32)
    with pytest.raises(NotImplementedError):
        _lib.call("vfk_t5_bucket", rel.ctypes.data, out.ctypes.data, 4, 1, 2, 128)
    with pytest.raises(ValueError):
        _lib.call("vfk_t5_bucket", None, None, 4, 1, 32, 128)


def test_product_rejects_cpu_tensors():
    from kernels.flash_attention_rpb import flash_attention_rpb_final
    from kernels.fused_layernorm import fused_layernorm
    q = torch.randn(1, 1, 8, 64)
    with pytest.raises(RuntimeError, match="GPU only"):
        flash_attention_rpb_final(q, q, q, None, 32, 128, False)
    with pytest.raises(RuntimeError, match="GPU only"):
        fused_layernorm(torch.randn(4, 8), 8)


def test_varlen_workspace_bytes():
    from kernels import _lib
    lib = _lib.load()
    # rotated K rounded up to 256 bytes, then four fp32 norms per (head, sequence, key tile)
    kr = (40265 * 12 * 64 * 2 + 255) // 256 * 256
    assert lib.vfk_varlen_attn_workspace_bytes(_lib.BF16, 40265, 12, 1, 64, 768) == kr + 12 * 64 * 12 * 16
    assert lib.vfk_varlen_attn_workspace_bytes(_lib.F16, 7, 3, 1, 2, 5) == 7 * 3 * 128 + 256 - 7 * 3 * 128 % 256 + 3 * 2 * 1 * 16
    assert lib.vfk_varlen_attn_workspace_bytes(_lib.BF16, 40265, 12, 0, 64, 768) == 0
    assert lib.vfk_varlen_attn_workspace_bytes(_lib.F32, 40265, 12, 1, 64, 768) == 0


def test_packing_argument_checks():
    """Rejected before any HIP call, so these run without a GPU."""
    from kernels import _lib
    from kernels.packing import pad_packed, seq_metadata
    lib = _lib.load()
    assert lib.vfk_varlen_meta_workspace_bytes(1) == 4
    assert lib.vfk_varlen_meta_workspace_bytes(1024) == 4
    assert lib.vfk_varlen_meta_workspace_bytes(163736) == 160 * 4
    assert lib.vfk_varlen_meta_workspace_bytes(0) == 0
    meta = lambda *a: _lib.call("vfk_varlen_meta", *a)
    with pytest.raises(ValueError, match="NULL"):
        meta(None, 8, 10, 0, None, None, None, 0, None)
    fake = 1 << 20  # never dereferenced: every case below fails its host checks
    with pytest.raises(ValueError, match="int32 or int64"):
        meta(fake, 2, 10, 0, fake, fake, fake, 4, None)
    with pytest.raises(ValueError, match="rule"):
        meta(fake, 8, 10, 2, fake, fake, fake, 4, None)
    with pytest.raises(ValueError, match="total_tokens"):
        meta(fake, 8, 0, 0, fake, fake, fake, 4, None)
    with pytest.raises(ValueError, match="workspace"):
        meta(fake, 8, 5000, 1, fake, fake, fake, 16, None)
    pad = lambda *a: _lib.call("vfk_pad_rows", *a)
    with pytest.raises(ValueError, match="NULL"):
        pad(None, 16, fake, 2, 8, 2, 0, fake, None, None)
    with pytest.raises(ValueError, match="num_seqs"):
        pad(fake, 16, fake, 70000, 8, 2, 0, fake, None, None)
    with pytest.raises(ValueError, match="2\\^31"):
        pad(fake, 1 << 20, fake, 2, 4096, 2, 0, fake, None, None)
    with pytest.raises(ValueError, match="elem_bytes"):
        pad(fake, 6, fake, 2, 8, 4, 0, fake, None, None)
    with pytest.raises(ValueError, match="elem_bytes must be"):
        pad(fake, 16, fake, 2, 8, 3, 0, fake, None, None)
    with pytest.raises(ValueError, match="max_len"):
        _lib.call("vfk_unpad_rows", fake, 16, fake, 2, 0, fake, None)
    with pytest.raises(RuntimeError, match="GPU only"):
        seq_metadata(torch.arange(5))
    with pytest.raises(ValueError, match="rule"):
        seq_metadata(torch.arange(5), "other")
    with pytest.raises(RuntimeError, match="GPU only"):
        pad_packed(torch.arange(5), torch.tensor([0, 5]), 1, 5)


def test_gliner_front_end_argument_checks():
    """Rejected before any HIP call, so these run without a GPU."""
    from kernels import _lib
    from kernels.gliner_pooler import gliner_reps_packed
    lib = _lib.load()
    assert lib.vfk_gliner_class_workspace_bytes(2048) == 8
    fake = 1 << 20  # never dereferenced: every case below fails its host checks
    cls = lambda *a: _lib.call("vfk_gliner_class_index", *a)
    with pytest.raises(ValueError, match="NULL"):
        cls(None, 10, 5, 0, fake, 1, fake, fake, fake, None, fake, 4, None)
    with pytest.raises(ValueError, match="total_tokens"):
        cls(fake, 0, 5, 0, fake, 1, fake, fake, fake, None, fake, 4, None)
    with pytest.raises(ValueError, match="num_seqs"):
        cls(fake, 10, 5, 0, fake, 0, fake, fake, fake, None, fake, 4, None)
    with pytest.raises(ValueError, match="workspace"):
        cls(fake, 5000, 5, 0, fake, 1, fake, fake, fake, None, fake, 8, None)
    pr = lambda *a: _lib.call("vfk_gliner_prompt_rows", *a)
    with pytest.raises(ValueError, match="multiple of 16"):
        pr(fake, 24, 10, fake, fake, 0, 4, fake, None)
    with pytest.raises(ValueError, match="aligned"):
        pr(fake + 8, 32, 10, fake, fake, 0, 4, fake, None)
    with pytest.raises(ValueError, match="sizes"):
        pr(fake, 32, 0, fake, fake, 0, 4, fake, None)
    wi = lambda *a: _lib.call("vfk_gliner_word_index", *a)
    with pytest.raises(ValueError, match="NULL"):
        wi(None, 10, fake, 1, fake, fake, None, None)
    with pytest.raises(ValueError, match="sizes"):
        wi(fake, 10, fake, 0, fake, fake, None, None)
    wr = lambda *a: _lib.call("vfk_gliner_word_rows", *a)
    with pytest.raises(ValueError, match="NULL"):
        wr(fake, 32, 10, None, 4, fake, None)
    with pytest.raises(ValueError, match="sizes"):
        wr(fake, 32, 10, fake, -1, fake, None)
    with pytest.raises(RuntimeError, match="GPU only"):
        gliner_reps_packed(torch.zeros(4, 8), torch.zeros(4), torch.zeros(4), torch.tensor([0, 4]),
                           [1], 5)


def test_qkv_rope_argument_checks():
    """The fused q|k|v projection and the attention over its rotated k reject
    bad arguments before any HIP call (CPU tensors serve as descriptors and
    are never dereferenced)."""
    from kernels import _lib
    lib = _lib.load()
    kr = (100 * 12 * 128 + 255) // 256 * 256
    assert lib.vfk_qkv_rope_workspace_bytes(100, 12) == kr + 12 * 4 * 4
    assert lib.vfk_qkv_rope_workspace_bytes(0, 12) == 0
    T, H, K = 100, 12, 768
    bf = torch.bfloat16
    x, w = torch.zeros(T, K, dtype=bf), torch.zeros(3 * H * 64, K, dtype=bf)
    q, v = torch.zeros(T, H, 64, dtype=bf), torch.zeros(T, H, 64, dtype=bf)
    d = lambda t: _lib.ref(_lib.desc(t))
    fake = 1 << 20
    ws = lib.vfk_qkv_rope_workspace_bytes(T, H)
    proj = lambda *a: _lib.call("vfk_qkv_rope_linear_fwd", *a)
    with pytest.raises(ValueError, match="w must be"):
        proj(d(x), d(torch.zeros(3 * H * 64 + 64, K, dtype=bf)), fake, fake, 512, H, 0.125, d(q), d(v),
             fake, ws, None)
    with pytest.raises(NotImplementedError, match="multiple of 64"):
        proj(d(torch.zeros(T, 96, dtype=bf)), d(torch.zeros(3 * H * 64, 96, dtype=bf)), fake, fake,
             512, H, 0.125, d(q), d(v), fake, ws, None)
    with pytest.raises(NotImplementedError, match="bf16 or fp16"):
        proj(d(x.float()), d(w.float()), fake, fake, 512, H, 0.125, d(q.float()), d(v.float()), fake,
             ws, None)
    with pytest.raises(ValueError, match="positions"):
        proj(d(x), d(w), None, fake, 512, H, 0.125, d(q), d(v), fake, ws, None)
    with pytest.raises(ValueError, match="rope table"):
        proj(d(x), d(w), fake, None, 512, H, 0.125, d(q), d(v), fake, ws, None)
    with pytest.raises(ValueError, match="workspace"):
        proj(d(x), d(w), fake, fake, 512, H, 0.125, d(q), d(v), fake, ws - 4, None)
    with pytest.raises(ValueError, match="q_out / v_out"):
        proj(d(x), d(w), fake, fake, 512, H, 0.125, d(torch.zeros(T, H - 1, 64, dtype=bf)), d(v), fake,
             ws, None)
    att = lambda *a: _lib.call("vfk_varlen_attn_krot_fwd", *a)
    o = torch.zeros(T, H, 64, dtype=bf)
    with pytest.raises(NotImplementedError, match="bf16 or fp16"):
        att(d(q.float()), d(v.float()), fake, ws, fake, 2, 64, -1, fake, 512, None, 0.125,
            d(o.float()), None)
    with pytest.raises(ValueError, match="krot"):
        att(d(q), d(v), fake, ws - 4, fake, 2, 64, -1, fake, 512, None, 0.125, d(o), None)
    with pytest.raises(ValueError, match="rope table"):
        att(d(q), d(v), fake, ws, fake, 2, 64, -1, None, 512, None, 0.125, d(o), None)
    with pytest.raises(ValueError, match="rope table"):
        att(d(q), d(v), fake, ws, fake, 2, 640, -1, fake, 512, None, 0.125, d(o), None)
    with pytest.raises(ValueError, match="cu_seqlens"):
        att(d(q), d(v), fake, ws, None, 2, 64, -1, fake, 512, None, 0.125, d(o), None)


def test_dense_layernorm_argument_checks():
    """The dense + residual + LayerNorm entry point rejects unsupported widths,
    reduction lengths, dtypes, parameter shapes and an output overlapping x
    before any HIP call (CPU tensors serve as descriptors, never read)."""
    from kernels import _lib
    bf = torch.bfloat16
    M, N, K = 100, 1024, 1024
    x, w = torch.zeros(M, K, dtype=bf), torch.zeros(N // 32, K // 16, 64, 8, dtype=bf)
    r, o, p = torch.zeros(M, N, dtype=bf), torch.zeros(M, N, dtype=bf), torch.zeros(N, dtype=bf)
    d = lambda t: _lib.ref(_lib.desc(t))
    g = lambda *a: _lib.call("vfk_dense_residual_layernorm_fwd", *a, None)
    f = lambda *a: g(*a, None)
    with pytest.raises(NotImplementedError, match="N must be"):
        f(d(x), d(torch.zeros(20, K // 16, 64, 8, dtype=bf)), None, d(torch.zeros(M, 640, dtype=bf)),
          None, None, 1e-7, d(torch.zeros(M, 640, dtype=bf)))
    with pytest.raises(NotImplementedError, match="multiple of 64"):
        f(d(torch.zeros(M, 96, dtype=bf)), d(torch.zeros(N // 32, 6, 64, 8, dtype=bf)), None, d(r),
          None, None, 1e-7, d(o))
    with pytest.raises(NotImplementedError, match="bf16 or fp16"):
        f(d(x.float()), d(w.float()), None, d(r.float()), None, None, 1e-7, d(o.float()))
    with pytest.raises(ValueError, match="share one dtype"):
        f(d(x), d(w.half()), None, d(r), None, None, 1e-7, d(o))
    with pytest.raises(ValueError, match="w_packed must be"):
        f(d(x), d(torch.zeros(N // 32, K // 16 + 4, 64, 8, dtype=bf)), None, d(r), None, None, 1e-7, d(o))
    with pytest.raises(ValueError, match="expected 4 dims"):
        f(d(x), d(torch.zeros(N, K, dtype=bf)), None, d(r), None, None, 1e-7, d(o))
    pk = lambda *a: _lib.call("vfk_pack_weight_mfma32", *a, None)
    with pytest.raises(ValueError, match="packed must be"):
        pk(d(torch.zeros(N, K, dtype=bf)), d(torch.zeros(N // 32, K // 16, 64, 4, dtype=bf)))
    with pytest.raises(NotImplementedError, match="multiple of 32"):
        pk(d(torch.zeros(N + 16, K, dtype=bf)), d(torch.zeros(N // 32, K // 16, 64, 8, dtype=bf)))
    with pytest.raises(ValueError, match="residual and out"):
        f(d(x), d(w), None, d(r[:50]), None, None, 1e-7, d(o))
    with pytest.raises(ValueError, match="ln_weight"):
        f(d(x), d(w), None, d(r), d(torch.zeros(N - 8, dtype=bf)), None, 1e-7, d(o))
    with pytest.raises(ValueError, match="bias"):
        f(d(x), d(w), d(p.float()), d(r), None, None, 1e-7, d(o))
    big = torch.zeros(M, N + K, dtype=bf)
    with pytest.raises(ValueError, match="output overlaps"):
        f(d(big[:, :K]), d(w), None, d(r), None, None, 1e-7, d(big[:, K:]))
    with pytest.raises(ValueError, match="output overlaps"):
        g(d(big[:, :K]), d(w), None, d(r), None, None, 1e-7, d(o), d(big[:, K:]))
    with pytest.raises(ValueError, match="out and residual_out overlap"):
        g(d(x), d(w), None, d(r), None, None, 1e-7, d(o), d(o))
    with pytest.raises(ValueError, match="residual_out must be"):
        g(d(x), d(w), None, d(r), None, None, 1e-7, d(o), d(torch.zeros(M, N, dtype=torch.float16)))
    with pytest.raises(ValueError, match="eps"):
        f(d(x), d(w), None, d(r), None, None, -1.0, d(o))
    # M = 0 returns before any launch
    d0 = lambda t: _lib.ref(_lib.desc(t, shape=[0, t.shape[1]]))
    f(d0(x), d(w), d(p), d0(r), d(p), d(p), 1e-7, d0(o))


def test_rel_chunk_major_layout_and_checks():
    """rel_chunk_major: out[h][c][r][i] = rel[h][r][8 c + i] for r < 2S (a
    torch view-and-copy, checked on the CPU); the fused entry point rejects
    mixed layouts, a wrong chunk-major shape and chunk-major fp32 tables
    before any HIP call."""
    from kernels import _lib
    from kernels.flash_deberta_attention import rel_chunk_major
    rel = torch.arange(3 * 600 * 64, dtype=torch.float32).view(3, 600, 64)
    cm = rel_chunk_major(rel, 256)
    assert cm.shape == (3, 8, 512, 8) and cm.is_contiguous()
    for h, c, r, i in [(0, 0, 0, 0), (2, 7, 511, 7), (1, 3, 200, 5)]:
        assert cm[h, c, r, i] == rel[h, r, 8 * c + i]
    assert rel_chunk_major(cm, 256) is cm
    bf = torch.bfloat16
    B, H, L = 2, 3, 64
    q = torch.zeros(B, H, L, 64, dtype=bf)
    d = lambda t: _lib.ref(_lib.desc(t))
    fake = 1 << 20
    f = lambda kr, qr, qq=q: _lib.call("vfk_deberta_fused_fwd", d(qq), d(qq), d(qq), fake, kr, qr,
                                       0.07, 256, 512, 1, d(qq), None)
    rows = torch.zeros(H, 512, 64, dtype=bf)
    cmt = torch.zeros(H, 8, 512, 8, dtype=bf)
    with pytest.raises(ValueError, match="one layout"):
        f(d(rows), d(cmt))
    with pytest.raises(ValueError, match="chunk-major"):
        f(d(torch.zeros(H, 8, 500, 8, dtype=bf)), None)
    with pytest.raises(NotImplementedError, match="16-bit"):
        f(d(cmt.float()), None, q.float())


def test_deberta_flash_flag_is_set():
    """The reference's DeBERTa v2 and v1 models take their flash path only when
    `HAS_TRITON` imported from kernels.flash_deberta_attention is true
    (models/deberta_v2/deberta_v2_encoder.py:39-42, :201, :230;
    models/deberta/deberta_encoder.py:35-38, :202, :227): the same import
    here must give a true flag and the kernel entry point."""
    from kernels.flash_deberta_attention import HAS_TRITON, flash_deberta_attention
    assert HAS_TRITON is True
    assert callable(flash_deberta_attention)


def test_packed_weight_cache_with_inference_tensors(monkeypatch):
    """packed_weight on a weight made under torch.inference_mode() (no version
    counter) packs once and reuses the copy, also when called inside
    inference mode; an ordinary weight re-packs after an in-place update; a
    new tensor object packs again. The pack itself is a stand-in here (the
    real one needs the GPU): only the cache logic is under test."""
    from kernels import weight_pack as wp
    calls = []

    def fake_pack(w):
        calls.append(w)
        return w.clone()

    monkeypatch.setattr(wp, "pack_weight", fake_pack)
    wp.clear_cache()
    with torch.inference_mode():
        w_inf = torch.randn(64, 32)
    assert w_inf.is_inference()
    a = wp.packed_weight(w_inf)
    with torch.inference_mode():
        b = wp.packed_weight(w_inf)
    assert a is b and len(calls) == 1
    w = torch.randn(64, 32)
    c = wp.packed_weight(w)
    assert wp.packed_weight(w) is c and len(calls) == 2
    w.add_(1.0)
    d = wp.packed_weight(w)
    assert d is not c and len(calls) == 3 and torch.equal(d, w)
    with torch.inference_mode():
        tmp = w_inf * 2            # a per-call temporary: its own entry
        e = wp.packed_weight(tmp)
    assert len(calls) == 4 and torch.equal(e, w_inf * 2)
    wp.clear_cache()
    wp.packed_weight(w_inf)
    assert len(calls) == 5
    wp.clear_cache()
