"""CPU oracle of the packed-stream plumbing — TEST INFRASTRUCTURE ONLY.

Restates how the reference finds sequences in vLLM's flat position ids and
re-pads them for a padded encoder:
  * seq_metadata: models/modernbert/modernbert_encoder.py:505-513 (rule
    "reset") and plugins/deberta_gliner/model.py:166-170 (rule "zero");
  * gliner_batch / gliner_unbatch: plugins/deberta_gliner/model.py:171-200;
  * gliner_reps / gliner_reps_packed: the prompt and word gathers of the
    GLiNER span pooler, poolers/gliner.py:313-347 (_extract_gliner_reps) per
    request of the flat stream (poolers/gliner.py:201, :219-255);
  * gliner_default_spans / gliner_span_rows: the pooler's default span list
    (poolers/gliner.py:270-283) and SpanMarkerV0's start/end pair rows
    (:131-145 with extract_elements :40-45); gliner_fit_length (_fit_length
    :299-311) and gliner_out_project (the marker's out_project, :141-144).
Pinned in tests/test_oracle_packing.py by construction (positions built from
known lengths; hidden rows that encode their own index), hand cases, a
pairwise brute force and round trips.
"""
from __future__ import annotations

import torch


def seq_metadata(position_ids: torch.Tensor, rule: str = "reset"):
    """Sequence boundaries of a packed stream from its flat position ids.

    rule "reset" (modernbert_encoder.py:505-513, _build_seq_block_mask):
    token 0 starts a sequence and so does every token with pos[i] <= pos[i-1];
    segment ids are the cumsum of those starts. rule "zero"
    (deberta_gliner/model.py:168, starts = (pos == 0).nonzero()): every token
    at position 0 starts one; token 0 is taken as a start as well (the
    reference's start list begins at the first zero).

    Returns (cu_seqlens int32 [n + 1], n, longest length, bad) where bad counts
    the breaks in the run of positions: a sequence start whose position is not
    0, or a token inside a sequence whose position is not its predecessor's + 1.
    bad == 0 exactly when every position equals the token's offset in its
    sequence (the position the varlen attention uses for RoPE)."""
    pos = position_ids.reshape(-1).to(torch.int64)
    T = pos.numel()
    starts = torch.zeros(T, dtype=torch.bool)
    starts[0] = True
    if T > 1:
        starts[1:] = pos[1:] <= pos[:-1] if rule == "reset" else pos[1:] == 0
    idx = torch.nonzero(starts).flatten()
    cu = torch.cat([idx, torch.tensor([T])]).to(torch.int32)
    lens = cu[1:] - cu[:-1]
    bad = int((starts & (pos != 0)).sum()) + int((~starts[1:] & (pos[1:] != pos[:-1] + 1)).sum())
    return cu, int(idx.numel()), int(lens.max()), bad


def gliner_batch(input_ids: torch.Tensor, positions: torch.Tensor, pad_id: int = 0):
    """The padded batch of plugins/deberta_gliner/model.py:166-191, written as
    its per-row loop: starts at position 0, rows padded with pad_id (ids) and 0
    (positions), attention mask 1 on valid tokens. Returns (batched_ids,
    batched_positions, attention_mask, lengths)."""
    pos = positions
    starts = (pos == 0).nonzero(as_tuple=False).flatten().tolist()
    ends = starts[1:] + [input_ids.shape[0]]
    lengths = [e - s for s, e in zip(starts, ends)]
    max_len = max(lengths)
    ids = input_ids.new_full((len(lengths), max_len), pad_id)
    bpos = pos.new_zeros((len(lengths), max_len))
    mask = torch.zeros((len(lengths), max_len), dtype=torch.long)
    for row, (s, e, n) in enumerate(zip(starts, ends, lengths)):
        ids[row, :n] = input_ids[s:e]
        bpos[row, :n] = pos[s:e]
        mask[row, :n] = 1
    return ids, bpos, mask, lengths


def gliner_unbatch(encoded: torch.Tensor, lengths):
    """torch.cat of the valid rows, plugins/deberta_gliner/model.py:197-200."""
    return torch.cat([encoded[row, :n] for row, n in enumerate(lengths)], dim=0)


def gliner_reps(tok: torch.Tensor, iid: torch.Tensor, wmask: torch.Tensor, true_len: int,
                ent_token_id: int, embed_ent_token: bool = True):
    """_extract_gliner_reps of poolers/gliner.py:313-347 for one request.

    pe: rows of tok at the class tokens (iid == ent_token_id), shifted by one
    row when the class token itself is not embedded (:317-319); a shifted
    index past the request raises IndexError like index_select. we [true_len,
    H]: for the tokens with wmask > 0 in order, word id w = wmask - 1 takes the
    token's row when w differs from the previous such token's (first-subtoken
    pooling, :333-341); other rows stay zero. Returns (pe [C, H], we [true_len,
    H]); the reference's leading batch dim of 1 and its all-ones masks are
    left out."""
    H = tok.shape[-1]
    class_pos = [i for i, v in enumerate(iid.tolist()) if v == ent_token_id]
    if not embed_ent_token:
        class_pos = [i + 1 for i in class_pos]
    if any(i >= tok.shape[0] for i in class_pos):
        raise IndexError("class token position past the end of the request")
    pe = tok[class_pos] if class_pos else tok.new_zeros(0, H)
    we = tok.new_zeros(true_len, H)
    prev = None
    for p, w in enumerate(wmask.tolist()):
        if w <= 0:
            continue
        if w - 1 != prev:
            if w - 1 >= true_len:
                raise IndexError(f"word id {w} past text length {true_len}")
            we[w - 1] = tok[p]
        prev = w - 1
    return pe, we


def gliner_reps_packed(hidden: torch.Tensor, input_ids: torch.Tensor, words_mask: torch.Tensor,
                       cu_seqlens, text_lengths, ent_token_id: int, embed_ent_token: bool = True):
    """gliner_reps over each request of a packed stream (split_hidden_states
    at poolers/gliner.py:201, then the per-request loop :219-255). Returns
    the lists of per-request pe and we."""
    cu = [int(c) for c in cu_seqlens]
    pes, wes = [], []
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        pe, we = gliner_reps(hidden[a:b], input_ids[a:b], words_mask[a:b], int(text_lengths[s]),
                             ent_token_id, embed_ent_token)
        pes.append(pe)
        wes.append(we)
    return pes, wes


def gliner_span_rows(start_rep: torch.Tensor, end_rep: torch.Tensor, span_idx: torch.Tensor,
                     span_mask: torch.Tensor) -> torch.Tensor:
    """SpanMarkerV0's pair rows for one request (poolers/gliner.py:131-145,
    extract_elements :40-45, indices masked at :285): span s takes start row
    i and end row j, i, j = span_idx[s] * span_mask[s] clamped to [0, L - 1],
    written as an explicit loop; out[s] = relu(cat(start[i], end[j]))."""
    L = start_rep.shape[0]
    rows = []
    for (a, b), m in zip(span_idx.tolist(), span_mask.tolist()):
        a, b = a * int(m), b * int(m)        # span_idx * span_mask.unsqueeze(-1), :286
        i, j = min(max(a, 0), L - 1), min(max(b, 0), L - 1)
        rows.append(torch.cat([start_rep[i], end_rep[j]]))
    if not rows:
        return start_rep.new_zeros(0, 2 * start_rep.shape[1])
    return torch.relu(torch.stack(rows))


def gliner_fit_length(we: torch.Tensor, target_len: int) -> torch.Tensor:
    """_fit_length of poolers/gliner.py:299-311 for one request's word rows
    [L, D]: the first target_len rows, or all rows followed by zero rows up to
    target_len (applied at :285-286 with target_W = span_idx.size(1) //
    max_width)."""
    L = we.shape[0]
    if L >= target_len:
        return we[:target_len]
    return torch.cat([we, we.new_zeros(target_len - L, we.shape[1])])


def gliner_out_project(pair_rows: torch.Tensor, w1: torch.Tensor, b1, w2: torch.Tensor,
                       b2) -> torch.Tensor:
    """SpanMarkerV0's out_project (poolers/gliner.py:141-144) in eval mode on
    its pair rows: create_projection_layer (:26-37) is Linear(2D, 4D), ReLU,
    Dropout (identity), Linear(4D, D); fp32."""
    h = pair_rows.float() @ w1.float().t()
    if b1 is not None:
        h = h + b1.float()
    h = torch.relu(h)
    out = h @ w2.float().t()
    return out + b2.float() if b2 is not None else out


def gliner_default_spans(block_len: int, true_len: int, max_width: int):
    """The pooler's default spans (poolers/gliner.py:270-283) as a loop: for
    every start word i < block_len and width k < max_width, span (i, i + k),
    valid when both ends are < true_len."""
    idx, mask = [], []
    for i in range(block_len):
        for k in range(max_width):
            idx.append([i, i + k])
            mask.append(int(i < true_len and i + k < true_len))
    return torch.tensor(idx, dtype=torch.int64).reshape(-1, 2), torch.tensor(mask, dtype=torch.int64)
