"""GPU parity of the ModernBERT packed local/global RoPE attention against the
oracle's per-sequence restatement of the reference's SDPA + dense masks."""
import pytest
import torch

import workloads
from _tol import assert_attn_close
from oracle import attention as oa

pytestmark = pytest.mark.gpu

LENGTHS = [1, 5, 63, 64, 65, 127, 128, 129, 200, 300, 700]


def _vl():
    from kernels.varlen_attention import varlen_rope_attention
    return varlen_rope_attention


def _pack(lengths, dtype, seed, H=12):
    g = torch.Generator().manual_seed(seed)
    T = sum(lengths)
    qkv = (torch.randn(T, 3, H, 64, generator=g) * 0.8).to(dtype)
    cu = workloads.cu_from_lengths(torch.tensor(lengths))
    return qkv, cu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("window,theta", [(-1, 160000.0), (64, 10000.0), (-1, 0.0), (5, 10000.0)])
def test_varlen_small_packs(dev, dtype, window, theta):
    qkv, cu = _pack(LENGTHS, dtype, 1)
    q, k, v = qkv[:, 0], qkv[:, 1], qkv[:, 2]
    want = oa.varlen_attention(q, k, v, cu, window, theta, None, 0.125)
    qd = qkv.to(dev)
    got = _vl()(qd[:, 0], qd[:, 1], qd[:, 2], cu.to(dev), max(LENGTHS), window, theta, 0.125)
    assert_attn_close(got, want, f"varlen {dtype} w={window} theta={theta}")


@pytest.mark.parametrize("window", [-1, 64])
def test_varlen_key_valid_mask(dev, window):
    qkv, cu = _pack(LENGTHS, torch.bfloat16, 2)
    T = qkv.shape[0]
    g = torch.Generator().manual_seed(3)
    key_valid = torch.rand(T, generator=g) > 0.1
    q, k, v = qkv[:, 0], qkv[:, 1], qkv[:, 2]
    want = oa.varlen_attention(q, k, v, cu, window, 160000.0, key_valid, 0.125)
    qd = qkv.to(dev)
    got = _vl()(qd[:, 0], qd[:, 1], qd[:, 2], cu.to(dev), max(LENGTHS), window, 160000.0, 0.125,
                key_valid=key_valid.to(dev))
    assert_attn_close(got, want, f"key_valid w={window}")


@pytest.mark.parametrize("window,theta", [(-1, 160000.0), (64, 10000.0)])
def test_config2_all_sequences(dev, window, theta):
    """Config 2 (64 sequences, 512..768 tokens, T = 40 265), the benchmark's
    own pack: every sequence against the oracle run on it alone."""
    c = workloads.config2(device=dev)
    qkv = c.qkv
    got = _vl()(qkv[:, 0], qkv[:, 1], qkv[:, 2], c.cu_seqlens, c.max_seqlen, window, theta,
                0.125).cpu()
    cu = c.cu_seqlens.cpu()
    worst = 0.0
    for s in range(len(cu) - 1):
        a, b = int(cu[s]), int(cu[s + 1])
        sub = qkv[a:b].cpu()
        want = oa.varlen_attention(sub[:, 0], sub[:, 1], sub[:, 2],
                                   torch.tensor([0, b - a], dtype=torch.int32), window, theta, None, 0.125)
        err, _ = assert_attn_close(got[a:b], want, f"cfg2 seq {s} w={window}")
        worst = max(worst, err)
    print(f"config 2 window={window}: {len(cu) - 1} sequences, max-abs {worst:.3e}")


def test_config2_full_properties(dev):
    """Whole config 2: V = 1 -> 1; permuting the packing order permutes rows."""
    c = workloads.config2(device=dev)
    q, k = c.qkv[:, 0], c.qkv[:, 1]
    ones = torch.ones_like(c.qkv[:, 2])
    for window in (-1, 64):
        o = _vl()(q, k, ones, c.cu_seqlens, c.max_seqlen, window, 160000.0, 0.125)
        assert torch.allclose(o.float(), torch.ones_like(o, dtype=torch.float32), atol=1e-2)
    # reverse the sequence order of the pack
    cu = c.cu_seqlens.cpu().tolist()
    n = len(cu) - 1
    order = list(range(n))[::-1]
    idx = torch.cat([torch.arange(cu[s], cu[s + 1]) for s in order]).to(dev)
    lens = torch.tensor([cu[s + 1] - cu[s] for s in order])
    cu2 = workloads.cu_from_lengths(lens).to(dev)
    v = c.qkv[:, 2]
    o1 = _vl()(q, k, v, c.cu_seqlens, c.max_seqlen, 64, 10000.0, 0.125)
    o2 = _vl()(q[idx], k[idx], v[idx], cu2, c.max_seqlen, 64, 10000.0, 0.125)
    assert torch.equal(o1[idx], o2)


def test_rope_table_matches_hf(dev):
    """vfk_rope_table == the HF rotary tables (fp32), up to one ulp of sin/cos."""
    from kernels.varlen_attention import rope_table
    for theta in (160000.0, 10000.0):
        t = rope_table(theta, 800, dev).cpu()
        c, s = oa.rope_cos_sin(torch.arange(t.shape[0]), theta)   # cat(f, f): [n, 64]
        torch.testing.assert_close(t[..., 0], c[:, :32], atol=2e-7, rtol=0)
        torch.testing.assert_close(t[..., 1], s[:, :32], atol=2e-7, rtol=0)


@pytest.mark.parametrize("window", [-1, 64])
def test_varlen_large_scores(dev, window):
    """Scores spread over ~+-12 (log2 units) with key norms growing along each
    sequence, so the running reference max of a row moves more than once. At
    this spread bf16-rounded rotated q/k alone (the reference model's own
    rounding) already miss the fp32 oracle by ~1e-2, so larger spreads are
    not a meaningful bf16 parity case."""
    lengths = [700, 300, 129, 64]
    g = torch.Generator().manual_seed(11)
    T = sum(lengths)
    q = torch.randn(T, 12, 64, generator=g)
    k = torch.randn(T, 12, 64, generator=g)
    cu = workloads.cu_from_lengths(torch.tensor(lengths))
    for s in range(len(lengths)):   # key norms grow along each sequence
        a, b = int(cu[s]), int(cu[s + 1])
        k[a:b] *= torch.linspace(0.3, 1.5, b - a)[:, None, None]
    v = torch.randn(T, 12, 64, generator=g)
    q, k, v = (t.bfloat16() for t in (q, k, v))
    want = oa.varlen_attention(q, k, v, cu, window, 160000.0, None, 0.125)
    got = _vl()(q.to(dev), k.to(dev), v.to(dev), cu.to(dev), max(lengths), window, 160000.0, 0.125)
    assert_attn_close(got, want, f"large scores w={window}")


def test_varlen_from_positions_drives_attention(dev):
    """Attention on cu_seqlens derived from position ids on the device equals
    the oracle on the lengths the positions were built from."""
    from kernels.varlen_attention import varlen_from_positions
    qkv, cu = _pack(LENGTHS, torch.bfloat16, 5)
    pos = torch.cat([torch.arange(n) for n in LENGTHS]).to(dev)
    got_cu, mx = varlen_from_positions(pos)
    assert mx == max(LENGTHS) and torch.equal(got_cu.cpu(), cu)
    qd = qkv.to(dev)
    got = _vl()(qd[:, 0], qd[:, 1], qd[:, 2], got_cu, mx, 64, 10000.0, 0.125)
    want = oa.varlen_attention(qkv[:, 0], qkv[:, 1], qkv[:, 2], cu, 64, 10000.0, None, 0.125)
    assert_attn_close(got, want, "varlen from positions")
    with pytest.raises(ValueError, match="count up from 0"):
        varlen_from_positions(torch.tensor([0, 1, 2, 5, 6], device=dev))


@pytest.mark.parametrize("window", [-1, 64])
def test_varlen_zero_length_sequences(dev, window):
    """cu_seqlens with empty sequences (repeated offsets, also first and last):
    their query tiles exit at once and the other sequences are unaffected."""
    lengths = [0, 130, 0, 0, 65, 1, 0]
    qkv, cu = _pack(lengths, torch.bfloat16, 21)
    q, k, v = qkv[:, 0], qkv[:, 1], qkv[:, 2]
    want = oa.varlen_attention(q, k, v, cu, window, 10000.0, None, 0.125)
    qd = qkv.to(dev)
    got = _vl()(qd[:, 0], qd[:, 1], qd[:, 2], cu.to(dev), max(lengths), window, 10000.0, 0.125)
    assert_attn_close(got, want, f"zero-length sequences w={window}")


@pytest.mark.parametrize("window", [-1, 64])
def test_varlen_bound_fallback_and_fast_waves(dev, window):
    """Both softmax paths in one workgroup. With RoPE every wave bounds its
    scores by |q| * max|k| over its key tiles before the loop: within
    log2(kPMax) it takes p = exp2(score) directly, otherwise the online
    softmax with a running max. Sequence 0 holds one key with 100x the norm of
    the others (masked by key_valid, so it cannot change any output but it
    sets the bound), which sends its normal rows to the running-max path,
    while its rows 32..63 (q scaled by 1e-3) stay under the bound; sequence 1
    is ordinary."""
    lengths = [300, 200]
    g = torch.Generator().manual_seed(12)
    T = sum(lengths)
    q = torch.randn(T, 12, 64, generator=g) * 0.8
    k = torch.randn(T, 12, 64, generator=g) * 0.8
    v = torch.randn(T, 12, 64, generator=g)
    q[32:64] *= 1e-3
    k[5] *= 100.0
    key_valid = torch.ones(T, dtype=torch.bool)
    key_valid[5] = False
    cu = workloads.cu_from_lengths(torch.tensor(lengths))
    q, k, v = (t.bfloat16() for t in (q, k, v))
    want = oa.varlen_attention(q, k, v, cu, window, 160000.0, key_valid, 0.125)
    got = _vl()(q.to(dev), k.to(dev), v.to(dev), cu.to(dev), max(lengths), window, 160000.0, 0.125,
                key_valid=key_valid.to(dev))
    assert_attn_close(got, want, f"bound fallback w={window}")


@pytest.mark.parametrize("window", [64, 5])
@pytest.mark.parametrize("masked", [False, True])
def test_local_many_sequences(dev, window, masked):
    """Sliding-window attention over a pack of 160 sequences (lengths 1..700,
    among them 1, 129 and 700 rows): every sequence is checked against the
    oracle, with and without a key_valid mask."""
    g = torch.Generator().manual_seed(40 + window)
    lengths = torch.randint(1, 701, (160,), generator=g).tolist()
    lengths[:4] = [1, 700, 129, 384]
    qkv, cu = _pack(lengths, torch.bfloat16, 41)
    T = qkv.shape[0]
    key_valid = (torch.rand(T, generator=g) > 0.1) if masked else None
    q, k, v = qkv[:, 0], qkv[:, 1], qkv[:, 2]
    want = oa.varlen_attention(q, k, v, cu, window, 10000.0, key_valid, 0.125)
    qd = qkv.to(dev)
    got = _vl()(qd[:, 0], qd[:, 1], qd[:, 2], cu.to(dev), max(lengths), window, 10000.0, 0.125,
                key_valid=None if key_valid is None else key_valid.to(dev))
    assert_attn_close(got, want, f"local pack w={window} masked={masked}")
