"""GLiNER span pooler front-end on the device: the prompt (class-token) and
word gathers of poolers/gliner.py:313-347 (_extract_gliner_reps) for every
request of a packed stream at once.

The reference splits the flat hidden stream per request (poolers/gliner.py:
201, split_hidden_states) and, in a Python loop over requests (:219-255),
finds the class tokens with nonzero(), index_selects their rows, and writes
the first subtoken of each word into a zero [text_length, H] block. Here
the whole batch takes five launches of index work and two row gathers.

Two index passes (class-token compaction with per-request offsets; the first
subtoken of every word, as a source index per word row) run before the one
read-back: the class counts that set pe's shape, as the reference reads them
with numel() per request, and the status words that turn the reference's
IndexErrors into IndexErrors here. Two row passes then write every output
row once.
"""
from __future__ import annotations

from typing import List, Sequence, Tuple

import torch

from . import _lib


def _stream_i64(x, dev, T: int, name: str) -> torch.Tensor:
    """A tensor or list of ids as contiguous int64 on the device (the
    reference's _to_tensor(..., dtype=torch.long), poolers/gliner.py:349-357)."""
    x = torch.as_tensor(x).reshape(-1)
    if x.numel() != T:
        raise ValueError(f"{name} has {x.numel()} entries, the hidden stream {T} rows")
    return x.to(device=dev, dtype=torch.int64).contiguous()


def gliner_reps_packed(hidden: torch.Tensor, input_ids: torch.Tensor, words_mask: torch.Tensor,
                       cu_seqlens: torch.Tensor, text_lengths: Sequence[int], ent_token_id: int,
                       embed_ent_token: bool = True):
    """Prompt and word representations of every request of a packed stream.

    hidden [T, H] (any dtype, H * itemsize a multiple of 16), input_ids and
    words_mask [T] (tensors of any integer dtype, on any device, or lists;
    cast to int64 as the reference's _to_tensor does),
    cu_seqlens int32 [n + 1] on the device (request s owns rows cu[s] ..
    cu[s + 1] - 1), text_lengths: n word counts (the reference's
    text_lengths). Returns (pe [C, H], pe_cu int64 [n + 1] on the host, we
    [W, H], we_cu int64 [n + 1] on the host): request s's prompt rows are
    pe[pe_cu[s]:pe_cu[s + 1]] and its word rows we[we_cu[s]:we_cu[s + 1]],
    exactly the reference's pe[0] and we[0]. Raises IndexError where the
    reference's index_select or indexed write would."""
    dev = _lib.require_gpu(hidden)
    if hidden.dim() != 2:
        raise ValueError("hidden must be [T, H]")
    hidden = hidden.contiguous()
    if hidden.data_ptr() % 16:
        hidden = hidden.clone()
    T, H = hidden.shape
    row_bytes = H * hidden.element_size()
    if T == 0 or row_bytes % 16:
        raise ValueError("hidden must have rows and a row size that is a multiple of 16 bytes")
    ids = _stream_i64(input_ids, dev, T, "input_ids")
    wm = _stream_i64(words_mask, dev, T, "words_mask")
    cu = cu_seqlens.to(device=dev, dtype=torch.int32).contiguous()
    n = cu.numel() - 1
    if n < 1 or len(text_lengths) != n:
        raise ValueError("need one text length per request of cu_seqlens")
    tl = torch.tensor([int(t) for t in text_lengths], dtype=torch.int64)
    if (tl < 0).any():
        raise ValueError("text_lengths must be non-negative")
    we_cu = torch.cat([torch.zeros(1, dtype=torch.int64), tl.cumsum(0)])
    W = int(we_cu[-1])
    if W >= 2**31 - 1:
        raise ValueError("too many word rows for int32 offsets")
    lib = _lib.load()

    # Index passes: class tokens (compaction + per-request offsets) and the
    # first subtoken of every word; both flag the reference's IndexErrors in
    # aux[n + 1:], read back with the class offsets in one copy.
    class_idx = torch.empty(T + 1, dtype=torch.int32, device=dev)
    aux = torch.zeros(n + 5, dtype=torch.int32, device=dev)
    class_cu, status = aux[:n + 1], aux[n + 1:n + 3]
    aux[n + 3:] = cu[[0, n]]  # endpoints, checked with the same read-back
    meta = torch.empty(4, dtype=torch.int32, device=dev)
    ws_bytes = int(lib.vfk_gliner_class_workspace_bytes(T))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    shift = 0 if embed_ent_token else 1
    _lib.on_device("vfk_gliner_class_index", dev, ids.data_ptr(), T, int(ent_token_id), shift,
                   cu.data_ptr(), n, class_idx.data_ptr(), class_cu.data_ptr(), meta.data_ptr(),
                   status.data_ptr(), ws.data_ptr(), ws_bytes)
    word_src = torch.zeros(max(W, 1), dtype=torch.int32, device=dev)
    if W:
        wcu = we_cu.to(device=dev, dtype=torch.int32)
        _lib.on_device("vfk_gliner_word_index", dev, wm.data_ptr(), T, cu.data_ptr(), n,
                       wcu.data_ptr(), word_src.data_ptr(), status.data_ptr() + 4)
    host = aux.cpu()
    if int(host[n + 3]) != 0 or int(host[n + 4]) != T:
        raise ValueError(f"cu_seqlens must run from 0 to the {T} hidden rows, got "
                         f"{int(host[n + 3])} .. {int(host[n + 4])}")
    if host[n + 1]:
        raise IndexError("index out of range: a shifted class token lies past its request")
    if host[n + 2]:
        raise IndexError("index out of range: a word id exceeds its request's text length")
    pe_cu = host[:n + 1].to(torch.int64)
    C = int(pe_cu[-1])

    # Row passes: every output row written once (word rows with no token as
    # zeros), no fill of the outputs beforehand.
    pe = torch.empty(C, H, dtype=hidden.dtype, device=dev)
    if C:
        _lib.on_device("vfk_gliner_prompt_rows", dev, hidden.data_ptr(), row_bytes, T,
                       class_idx.data_ptr(), meta.data_ptr(), shift, C, pe.data_ptr())
    we = torch.empty(W, H, dtype=hidden.dtype, device=dev)
    if W:
        _lib.on_device("vfk_gliner_word_rows", dev, hidden.data_ptr(), row_bytes, T,
                       word_src.data_ptr(), W, we.data_ptr())
    return pe, pe_cu, we, we_cu


def extract_gliner_reps(hidden: torch.Tensor, input_ids: torch.Tensor, words_mask: torch.Tensor,
                        cu_seqlens: torch.Tensor, text_lengths: Sequence[int], ent_token_id: int,
                        embed_ent_token: bool = True
                        ) -> List[Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]]:
    """Per-request outputs of the reference's _extract_gliner_reps
    (poolers/gliner.py:313-347): a list of (pe [1, C, H], pe_mask long [1, C]
    of ones, we [1, text_length, H], we_mask long [1, text_length] of ones),
    all views or small tensors over one batched device gather."""
    pe, pe_cu, we, we_cu = gliner_reps_packed(hidden, input_ids, words_mask, cu_seqlens,
                                              text_lengths, ent_token_id, embed_ent_token)
    out = []
    dev = pe.device
    for s in range(pe_cu.numel() - 1):
        a, b = int(pe_cu[s]), int(pe_cu[s + 1])
        c, d = int(we_cu[s]), int(we_cu[s + 1])
        out.append((pe[a:b].unsqueeze(0), torch.ones(1, b - a, dtype=torch.long, device=dev),
                    we[c:d].unsqueeze(0), torch.ones(1, d - c, dtype=torch.long, device=dev)))
    return out


def default_spans(block_len: int, true_len: int, max_width: int):
    """The pooler's default span list for one request (poolers/gliner.py:
    270-283): span (i, i + k) for every start i < block_len and width
    k < max_width, valid where both ends are < true_len. Returns (span_idx
    int64 [block_len * max_width, 2], span_mask int64 [block_len * max_width])
    on the CPU."""
    starts = torch.arange(block_len).repeat_interleave(max_width)
    widths = torch.arange(max_width).repeat(block_len)
    idx = torch.stack([starts, starts + widths], dim=-1)
    mask = ((idx[:, 0] < true_len) & (idx[:, 1] < true_len)).to(torch.int64)
    return idx, mask


def gliner_span_rows(start_rep: torch.Tensor, end_rep: torch.Tensor, row_cu: torch.Tensor,
                     span_idx: torch.Tensor, span_mask: torch.Tensor,
                     span_cu: torch.Tensor) -> torch.Tensor:
    """SpanMarkerV0's pair rows for every request of a packed batch at once:
    relu(cat(start_rep[i], end_rep[j])) per span (poolers/gliner.py:131-145,
    extract_elements :40-45, the masked indices of :285).

    start_rep / end_rep [W, D] (bf16, fp16 or fp32; the project_start /
    project_end outputs over the requests' word rows, request r owning rows
    row_cu[r] .. row_cu[r + 1] - 1), span_idx [S, 2] request-local word
    indices and span_mask [S] (any integer or bool dtype), span_cu [n + 1]
    (request r owns spans span_cu[r] .. span_cu[r + 1] - 1). Returns
    [S, 2 * D]; for request r it equals the reference's cat(...).relu()
    rows before out_project."""
    dev = _lib.require_gpu(start_rep, end_rep)
    if start_rep.dim() != 2 or start_rep.shape != end_rep.shape or start_rep.dtype != end_rep.dtype:
        raise ValueError("start_rep and end_rep must be [W, D] of one dtype")
    codes = {torch.bfloat16: 1, torch.float16: 2, torch.float32: 0}
    if start_rep.dtype not in codes:
        raise ValueError("start_rep must be bf16, fp16 or fp32")

    def rows(t):
        t = t.contiguous()
        return t if t.data_ptr() % 16 == 0 else t.clone()
    sr, er = rows(start_rep), rows(end_rep)
    W, D = sr.shape
    row_bytes = D * sr.element_size()
    if row_bytes % 16:
        raise ValueError("row size must be a multiple of 16 bytes")
    idx = torch.as_tensor(span_idx).to(device=dev, dtype=torch.int64).reshape(-1, 2).contiguous()
    S = idx.shape[0]
    mask = torch.as_tensor(span_mask).to(device=dev, dtype=torch.int64).reshape(-1).contiguous()
    if mask.numel() != S:
        raise ValueError("span_mask must have one entry per span")
    rcu = torch.as_tensor(row_cu).to(device=dev, dtype=torch.int32).contiguous()
    scu = torch.as_tensor(span_cu).to(device=dev, dtype=torch.int32).contiguous()
    n = rcu.numel() - 1
    if n < 1 or scu.numel() != n + 1:
        raise ValueError("row_cu and span_cu need one entry per request plus one")
    out = torch.empty(S, 2 * D, dtype=sr.dtype, device=dev)
    if S:
        _lib.on_device("vfk_gliner_span_rows", dev, sr.data_ptr(), er.data_ptr(), row_bytes, W,
                       codes[sr.dtype], rcu.data_ptr(), n, idx.data_ptr(), mask.data_ptr(),
                       scu.data_ptr(), S, out.data_ptr())
    return out
