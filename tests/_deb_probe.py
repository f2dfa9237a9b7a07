"""Inputs that make DeBERTa attention reveal its clamped relative index
c(i - j) = clamp(bucket(i - j) + S, 0, 2S - 1) for every (query, key) pair.

One launch asks, for a set of "hot" index values (one per head) and a set of
key blocks (one per batch row), which keys j of the block have
c(i - j) == hot for each query row i:

  * q_i = 64 e_0 for every row; k_j[0] is 0 for the block's keys, 0.5 for one
    reference key r outside every block and -2 for all other keys, so the
    content score q.k is 0 / 32 / -128;
  * the position term adds 64 exactly when c(i - j) == hot (c2p: pos_key or
    key_rel one-hot at the hot index; p2c: pos_query or query_rel one-hot,
    with k_j[1] = 1 carrying it in the fused form);
  * v_j = e_w for the w-th key of the block, e_63 for r, 0 otherwise.

Scores are then 64 (block key, hot), 32 (r, not hot), <= 0 (block key, not
hot) and <= -64 (other keys). A row whose block holds n >= 1 hot keys puts
weight 1/n on each of them (the rest is below e^-32); a row with none puts
all weight on dim 63. Rows where r itself is hot are skipped (the launch with
the other reference key covers them: c(i) != c(i - N + 1) for every row when
N > 1, so r = N - 1 and r = 0 never both fail).

`decode` turns an output [B, H, N, 64] into the membership it shows; `expect`
computes the membership the oracle's c matrix implies. Equal booleans for
every (hot, block, row, key) pin the device index bit-exactly.
"""
from __future__ import annotations

import torch

from oracle import buckets as ob

BIG = 64.0


def c_matrix(N: int, S: int, position_buckets: int, max_relative: int, log: bool) -> torch.Tensor:
    """clamp(build_relative_position_v2(N, N) + S, 0, 2S - 1) as int64 [N, N]
    (models/deberta_v2/deberta_v2_encoder.py:92-103; the clamp of
    kernels/flash_deberta_attention.py:249-268)."""
    if log:
        rel = ob.build_relative_position_v2(N, N, position_buckets, max_relative)[0]
    else:
        rel = ob.build_relative_position_v2(N, N)[0]
    return torch.clamp(rel + S, 0, 2 * S - 1)


def blocks_for(N: int, ref: int, width: int = 62) -> torch.Tensor:
    """Key blocks [nb, width] over every key except ref (-1 pads the last)."""
    keys = [j for j in range(N) if j != ref]
    nb = (len(keys) + width - 1) // width
    J = torch.full((nb, width), -1, dtype=torch.long)
    for b in range(nb):
        part = keys[b * width:(b + 1) * width]
        J[b, :len(part)] = torch.tensor(part)
    return J


def inputs(N: int, J: torch.Tensor, ref: int, hots, S: int, mode: str, form: str,
           dtype=torch.bfloat16, device="cpu"):
    """q, k, v [nb, H, N, 64] and either (pos_key, pos_query) [nb, H, N, 2S]
    broadcast views (form 'gather') or (key_rel, query_rel) [H, 2S, 64]
    (form 'fused'); mode 'c2p' or 'p2c' selects which term carries the mark."""
    nb, width = J.shape
    H = len(hots)
    hot = torch.as_tensor(hots, dtype=torch.long)
    q = torch.zeros(nb, H, N, 64, device=device)
    q[..., 0] = BIG
    k = torch.zeros(nb, H, N, 64, device=device)
    k[..., 0] = -2.0
    v = torch.zeros(nb, H, N, 64, device=device)
    bi, wi = (J >= 0).nonzero(as_tuple=True)
    jj = J[bi, wi]
    bi, wi, jj = bi.to(device), wi.to(device), jj.to(device)
    k[bi, :, jj, 0] = 0.0
    v[bi, :, jj, wi] = 1.0
    k[:, :, ref, 0] = 0.5
    v[:, :, ref, 63] = 1.0
    onehot = torch.zeros(H, 2 * S, device=device)
    onehot[torch.arange(H, device=device), hot.to(device)] = 1.0
    a, b_ = None, None
    if form == "gather":
        mark = (BIG * onehot).to(dtype)[None, :, None, :].expand(nb, H, N, 2 * S)
        a, b_ = (mark, None) if mode == "c2p" else (None, mark)
    else:
        rel = torch.zeros(H, 2 * S, 64, device=device)
        if mode == "c2p":
            rel[..., 0] = onehot            # q.key_rel[c] = 64 [c == hot]
            a = rel
        else:
            rel[..., 1] = BIG * onehot      # k.query_rel[c] = 64 [c == hot]
            k[..., 1] = 1.0
            b_ = rel
        a = a.to(dtype) if a is not None else None
        b_ = b_.to(dtype) if b_ is not None else None
    q, k, v = (t.to(dtype) for t in (q, k, v))
    return q, k, v, a, b_


def expect(c: torch.Tensor, J: torch.Tensor, ref: int, hots):
    """(member [nb, H, N, width], any [nb, H, N], skip [H, N]) from the
    oracle's index matrix c [N, N]."""
    hot = torch.as_tensor(hots, dtype=c.dtype, device=c.device)
    Jc = J.clamp(min=0).to(c.device)
    sel = c[:, Jc]                                       # [N, nb, width]
    member = (sel.permute(1, 0, 2)[:, None] == hot[None, :, None, None]) & (J >= 0).to(c.device)[:, None, None, :]
    skip = c[:, ref][None, :] == hot[:, None]            # [H, N]
    return member, member.any(-1), skip


def decode(out: torch.Tensor, width: int):
    """(member, ref_weight) as the output shows them."""
    o = out.float()
    return o[..., :width] > 1e-3, o[..., 63] > 0.5


def check(out: torch.Tensor, c: torch.Tensor, J: torch.Tensor, ref: int, hots, what: str):
    member, anyhot, skip = expect(c, J, ref, hots)
    got_m, got_r = decode(out, J.shape[1])
    keep = ~skip[None, :, :, None]
    bad = (got_m != member) & keep
    bad_r = (got_r != ~anyhot) & ~skip[None]
    if bad.any() or bad_r.any():
        idx = bad.nonzero()[:1].tolist() or bad_r.nonzero()[:1].tolist()
        raise AssertionError(f"{what}: device index differs from the oracle at "
                             f"(block, head, row[, key slot]) {idx}; "
                             f"{int(bad.sum())} key and {int(bad_r.sum())} row mismatches")
    # every hot key carries the weight 1 / n of its row (within 16-bit rounding)
    n = member.sum(-1, keepdim=True).clamp(min=1).float()
    w = out[..., :J.shape[1]].float()
    err = ((w - 1.0 / n).abs() * member * keep).max()
    assert float(err) <= 1e-2, f"{what}: hot-key weight off by {float(err)}"
