"""The DeBERTa index probe (tests/_deb_probe.py) run through the oracle's
attention: decoding the oracle's own output gives back the oracle's index
matrix for every (query, key) pair, in both bucket modes, both position terms
and both input forms, and a planted index mistake is caught. This pins the
probe before the GPU test trusts it on the device kernels."""
import pytest
import torch

import _deb_probe as dp
from oracle import attention as oa

D64 = torch.float64


def _oracle_out(q, k, v, a, b, form, mode, S, pb, mrp, log, c_override=None):
    if form == "fused":
        pk = torch.matmul(q, a.transpose(-1, -2).unsqueeze(0)) if a is not None else None
        pq = torch.matmul(k, b.transpose(-1, -2).unsqueeze(0)) if b is not None else None
    else:
        pk, pq = a, b
    if c_override is None:
        return oa.deberta_flash_attention(q, k, v, None, pk, pq, 1.0, pb, mrp, log, dtype=D64)
    # same attention with a given index matrix (a planted mistake)
    s = torch.matmul(q, k.transpose(-1, -2))
    B, H, N, _ = q.shape
    idx = c_override[None, None].expand(B, H, N, N)
    if pk is not None:
        s = s + torch.gather(pk, -1, idx)
    if pq is not None:
        s = s + torch.gather(pq, -1, idx.transpose(-1, -2)).transpose(-1, -2)
    return torch.matmul(torch.softmax(s, -1), v)


@pytest.mark.parametrize("log", [True, False])
@pytest.mark.parametrize("mode", ["c2p", "p2c"])
@pytest.mark.parametrize("form", ["gather", "fused"])
def test_probe_recovers_oracle_index(log, mode, form):
    N, S, pb, mrp, width = 70, 16, 16, 40, 10
    c = dp.c_matrix(N, S, pb, mrp, log)
    hots = list(range(2 * S))
    for ref in (N - 1, 0):
        J = dp.blocks_for(N, ref, width)
        q, k, v, a, b = dp.inputs(N, J, ref, hots, S, mode, form, dtype=D64)
        out = _oracle_out(q, k, v, a, b, form, mode, S, pb, mrp, log)
        dp.check(out, c, J, ref, hots, f"oracle {form} {mode} log={log} ref={ref}")


def test_probe_covers_every_pair():
    """Each (row, key) pair is decided in at least one of the two launches:
    the rows a reference key skips for a hot value are never skipped by the
    other reference key for the same value."""
    for N, S, pb, mrp in ((70, 16, 16, 40), (512, 256, 256, 512), (1024, 256, 256, 512)):
        c = dp.c_matrix(N, S, pb, mrp, True)
        both = c[:, N - 1] == c[:, 0]
        assert not both.any()


def test_probe_catches_planted_index_mistake():
    """Saturated indices moved by one (2S - 2 instead of 2S - 1), the hazard
    at |i - j| >= max_relative_positions - 1, are reported."""
    N, S, pb, mrp, width = 70, 16, 16, 40, 10
    c = dp.c_matrix(N, S, pb, mrp, True)
    assert (c == 2 * S - 1).any()
    bad_c = torch.where(c == 2 * S - 1, torch.full_like(c, 2 * S - 2), c)
    hots = list(range(2 * S))
    ref = N - 1
    J = dp.blocks_for(N, ref, width)
    q, k, v, a, b = dp.inputs(N, J, ref, hots, S, "c2p", "gather", dtype=D64)
    out = _oracle_out(q, k, v, a, b, "gather", "c2p", S, pb, mrp, True, c_override=bad_c)
    with pytest.raises(AssertionError, match="device index differs"):
        dp.check(out, c, J, ref, hots, "planted")
    # the sign hazard at one column: c(d) for d = -1 taken as c(+1)
    bad_c = c.clone()
    r = torch.arange(N - 1)
    bad_c[r, r + 1] = c[r + 1, r]
    out = _oracle_out(q, k, v, a, b, "gather", "c2p", S, pb, mrp, True, c_override=bad_c)
    with pytest.raises(AssertionError, match="device index differs"):
        dp.check(out, c, J, ref, hots, "planted sign")
