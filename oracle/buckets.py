"""Relative-position buckets (oracle; test infrastructure only).

Both functions evaluate the reference's eager formula with the same tensor
ops in the same dtype (fp32 on the CPU), over whole [Lq, Lk] matrices like the
reference does.

Pinned by (tests/test_oracle_buckets.py):
  * closed forms: |rel| < max_exact -> |rel| (T5), |rel| <= mid -> rel
    (DeBERTa); saturation at num_buckets//2 - 1 (T5) for |rel| >= max_distance;
  * exact arithmetic away from rounding points (fractions + math.log in fp64);
  * the independent third-party implementations in transformers
    (models/t5/modeling_t5.py `_relative_position_bucket`,
    models/deberta_v2/modeling_deberta_v2.py `make_log_bucket_position`);
  * invariants: Toeplitz, monotone, odd symmetry (DeBERTa), sign offset (T5);
  * the committed golden tables tests/golden/*_buckets_*.json.
"""
from __future__ import annotations

import torch


def t5_relative_position_bucket(relative_position: torch.Tensor, bidirectional: bool,
                                num_buckets: int, max_distance: int) -> torch.Tensor:
    """models/mt5/mt5_encoder.py:124-148 (T5RelativePositionBias._relative_position_bucket).

    relative_position = memory - context = key - query (mt5_encoder.py:157).
    """
    relative_buckets = 0
    if bidirectional:
        num_buckets //= 2
        relative_buckets += (relative_position > 0).to(torch.long) * num_buckets
        relative_position = torch.abs(relative_position)
    else:
        relative_position = -torch.min(relative_position, torch.zeros_like(relative_position))
    max_exact = num_buckets // 2
    is_small = relative_position < max_exact
    relative_position_if_large = max_exact + (
        torch.log(relative_position.float() / max_exact)
        / torch.log(torch.tensor(max_distance / max_exact))
        * (num_buckets - max_exact)
    ).to(torch.long)
    relative_position_if_large = torch.min(
        relative_position_if_large,
        torch.full_like(relative_position_if_large, num_buckets - 1),
    )
    return torch.where(is_small, relative_position, relative_position_if_large) + relative_buckets


def t5_bucket_matrix(q_len: int, k_len: int, bidirectional: bool, num_buckets: int,
                     max_distance: int) -> torch.Tensor:
    """mt5_encoder.py:150-159: the [q_len, k_len] bucket matrix of key - query."""
    context_position = torch.arange(q_len, dtype=torch.long)[:, None]
    memory_position = torch.arange(k_len, dtype=torch.long)[None, :]
    return t5_relative_position_bucket(memory_position - context_position, bidirectional,
                                       num_buckets, max_distance)


def make_log_bucket_position(relative_pos: torch.Tensor, bucket_size: int,
                             max_position: int) -> torch.Tensor:
    """models/deberta_v2/deberta_v2_encoder.py:70-89 (make_log_bucket_position).

    relative_pos = query - key (deberta_v2_encoder.py:99). Returns fp32.
    """
    sign = torch.sign(relative_pos)
    mid = bucket_size // 2
    abs_pos = torch.where(
        (relative_pos < mid) & (relative_pos > -mid),
        torch.tensor(mid - 1).type_as(relative_pos),
        torch.abs(relative_pos),
    )
    log_pos = (
        torch.ceil(
            torch.log(abs_pos / mid) / torch.log(torch.tensor((max_position - 1) / mid)) * (mid - 1)
        )
        + mid
    )
    return torch.where(abs_pos <= mid, relative_pos.type_as(log_pos), log_pos * sign)


def build_relative_position_v2(query_size: int, key_size: int, bucket_size: int = -1,
                               max_position: int = -1) -> torch.Tensor:
    """deberta_v2_encoder.py:92-103: [1, q, k] long tensor of (log-)bucketed q - k."""
    q_ids = torch.arange(query_size, dtype=torch.long)
    k_ids = torch.arange(key_size, dtype=torch.long)
    rel = q_ids[:, None] - k_ids[None, :]
    if bucket_size > 0 and max_position > 0:
        rel = make_log_bucket_position(rel, bucket_size, max_position)
    return rel.to(torch.long).unsqueeze(0)
