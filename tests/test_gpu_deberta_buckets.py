"""Bit-exact recovery of the DeBERTa device index c(i - j) for every
(query, key) pair, from the three bf16 kernels: the staged reference-interface
gather, the per-score gather (taken for pos tensors without unit column
stride, and for bucket functions whose steps exceed 1) and the fused in-kernel
c2p / p2c form. The probe inputs (tests/_deb_probe.py, pinned on the oracle by
tests/test_oracle_deb_probe.py) make the output show, per hot index value and
key block, which keys of the block have c(i - j) == hot; the test compares
that with clamp(build_relative_position_v2 + S, 0, 2S - 1)
(models/deberta_v2/deberta_v2_encoder.py:70-103,
kernels/flash_deberta_attention.py:249-268)."""
import pytest
import torch

import _deb_probe as dp

pytestmark = pytest.mark.gpu

CHUNK = 64  # hot index values per launch (one per head)


def _kern():
    from kernels import flash_deberta_attention as m
    return m


def _run(form, q, k, v, a, b, pb, mrp, log):
    m = _kern()
    if form == "fused":
        return m.flash_deberta_attention_fused(q, k, v, None, a, b, 1.0, pb, mrp, log)
    if form == "per_score":
        # pos tensors with column stride 2: the staged kernel needs unit stride
        def strided(t):
            if t is None:
                return None
            base = torch.zeros(t.shape[1], t.shape[-1], 2, dtype=t.dtype, device=t.device)
            base[..., 0] = t[0, :, 0]
            return base[..., 0][None, :, None, :].expand(t.shape)
        a, b = strided(a), strided(b)
        assert a is None or a.stride(-1) == 2
        assert b is None or b.stride(-1) == 2
    return m.flash_deberta_attention(q, k, v, None, a, b, False, 1.0, pb, mrp, log)


def _sweep(dev, N, pb, mrp, log, form, mode):
    S = pb
    c = dp.c_matrix(N, S, pb, mrp, log).to(dev)
    for ref in (N - 1, 0):
        J = dp.blocks_for(N, ref)
        for h0 in range(0, 2 * S, CHUNK):
            hots = list(range(h0, min(h0 + CHUNK, 2 * S)))
            q, k, v, a, b = dp.inputs(N, J, ref, hots, S, mode,
                                      "fused" if form == "fused" else "gather", device=dev)
            out = _run(form, q, k, v, a, b, pb, mrp, log)
            dp.check(out, c, J, ref, hots, f"{form} {mode} N={N} log={log} ref={ref} hots {h0}+")


@pytest.mark.parametrize("form", ["staged", "per_score", "fused"])
@pytest.mark.parametrize("mode", ["c2p", "p2c"])
@pytest.mark.parametrize("N,log", [(512, True), (1024, True), (1024, False)])
def test_device_index_exact(dev, N, log, form, mode):
    print(f"deberta index probe: {form} {mode} N={N} log={log}", flush=True)
    _sweep(dev, N, 256, 512, log, form, mode)


@pytest.mark.parametrize("form", ["staged", "per_score"])
@pytest.mark.parametrize("mode", ["c2p", "p2c"])
def test_device_index_exact_wide_steps(dev, form, mode):
    """position_buckets 256 with max_relative_positions 256: the log bucket
    advances by 2 per unit of distance in places, so the gather entry point
    takes its per-score kernel whatever the pos layout; the indices still
    match the oracle bit for bit."""
    from kernels import _lib
    assert _lib.load().vfk_deberta_unit_steps(256, 256, 1, 512) == 0
    print(f"deberta index probe (wide steps): {form} {mode}", flush=True)
    _sweep(dev, 512, 256, 256, True, form, mode)


def test_fused_rejects_wide_steps(dev):
    q = torch.zeros(1, 1, 512, 64, dtype=torch.bfloat16, device=dev)
    rel = torch.zeros(1, 512, 64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(NotImplementedError, match="bucket steps above 1"):
        _kern().flash_deberta_attention_fused(q, q, q, None, rel, rel, 1.0, 256, 256, True)
