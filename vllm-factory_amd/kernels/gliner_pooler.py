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
    aux[n + 3:].copy_(cu[::n])  # endpoints cu[0], cu[n], checked with the same read-back
    meta = torch.empty(4, dtype=torch.int32, device=dev)
    ws_bytes = int(lib.vfk_gliner_class_workspace_bytes(T))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    shift = 0 if embed_ent_token else 1
    _lib.on_device("vfk_gliner_class_index", dev, ids.data_ptr(), T, int(ent_token_id), shift,
                   cu.data_ptr(), n, class_idx.data_ptr(), class_cu.data_ptr(), meta.data_ptr(),
                   status.data_ptr(), ws.data_ptr(), ws_bytes)
    word_src = torch.zeros(max(W, 1), dtype=torch.int32, device=dev)
    if W:
        # from pinned memory: the copy does not wait for the kernels above
        wcu = we_cu.to(torch.int32).pin_memory().to(dev, non_blocking=True)
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


def fit_word_rows(we: torch.Tensor, we_cu: Sequence[int], target_rows: Sequence[int]):
    """The reference's per-request _fit_length (poolers/gliner.py:285-286,
    :299-311) over packed word rows: request r's rows we[we_cu[r]:we_cu[r+1]]
    are cut to target_rows[r] or padded with zero rows to it (target_W =
    span_idx.size(1) // max_width for its span list). Returns (rows
    [sum(target_rows), H], row_cu int32 [n + 1] on the device), the rows that
    the span marker's project_start / project_end take."""
    dev = _lib.require_gpu(we)
    cu = [int(x) for x in we_cu]
    tw = [int(x) for x in target_rows]
    if len(cu) != len(tw) + 1 or any(t < 0 for t in tw):
        raise ValueError("we_cu needs one entry per request plus one; target_rows >= 0")
    src = []
    for r, t in enumerate(tw):
        n = cu[r + 1] - cu[r]
        src.append(torch.arange(cu[r], cu[r] + min(n, t)))
        src.append(torch.full((max(t - n, 0),), we.shape[0], dtype=torch.int64))  # zero row
    src = torch.cat(src).to(dev) if src else torch.zeros(0, dtype=torch.int64, device=dev)
    padded = torch.cat([we, we.new_zeros(1, we.shape[1])])
    row_cu = torch.tensor([0] + list(torch.tensor(tw).cumsum(0).tolist()), dtype=torch.int32, device=dev)
    return padded.index_select(0, src), row_cu


_SPAN_DT = {torch.bfloat16: 1, torch.float16: 2, torch.float32: 0}


def _span_args(x: torch.Tensor, y: torch.Tensor, row_cu, span_idx, span_mask, span_cu):
    """Shared checks of the span ops: x, y [W, N] rows of one dtype, the
    index lists on x's device. Returns (x, y, idx, mask, row_cu, span_cu)."""
    dev = _lib.require_gpu(x, y)
    if x.dim() != 2 or x.shape != y.shape or x.dtype != y.dtype:
        raise ValueError("the two row sets must be [W, N] of one dtype")
    if x.dtype not in _SPAN_DT:
        raise ValueError("rows must be bf16, fp16 or fp32")

    def rows(t):
        t = t.contiguous()
        return t if t.data_ptr() % 16 == 0 else t.clone()
    x, y = rows(x), rows(y)
    if (x.shape[1] * x.element_size()) % 16:
        raise ValueError("row size must be a multiple of 16 bytes")
    idx = torch.as_tensor(span_idx).to(device=dev, dtype=torch.int64).reshape(-1, 2).contiguous()
    mask = torch.as_tensor(span_mask).to(device=dev, dtype=torch.int64).reshape(-1).contiguous()
    if mask.numel() != idx.shape[0]:
        raise ValueError("span_mask must have one entry per span")
    rcu = torch.as_tensor(row_cu).to(device=dev, dtype=torch.int32).contiguous()
    scu = torch.as_tensor(span_cu).to(device=dev, dtype=torch.int32).contiguous()
    if rcu.numel() < 2 or scu.numel() != rcu.numel():
        raise ValueError("row_cu and span_cu need one entry per request plus one")
    return x, y, idx, mask, rcu, scu


def gliner_span_rows(start_rep: torch.Tensor, end_rep: torch.Tensor, row_cu: torch.Tensor,
                     span_idx: torch.Tensor, span_mask: torch.Tensor,
                     span_cu: torch.Tensor) -> torch.Tensor:
    """SpanMarkerV0's pair rows for every request of a packed batch at once:
    relu(cat(start_rep[i], end_rep[j])) per span (poolers/gliner.py:131-145,
    extract_elements :40-45, the masked indices of :285).

    start_rep / end_rep [W, D] (bf16, fp16 or fp32): project_start /
    project_end over each request's fitted word rows (fit_word_rows), request
    r owning rows row_cu[r] .. row_cu[r + 1] - 1; span_idx [S, 2]
    request-local word indices, span_mask [S] (any integer or bool dtype;
    the indices are multiplied by its value, as the reference does), span_cu
    [n + 1] (request r owns spans span_cu[r] .. span_cu[r + 1] - 1). Returns
    [S, 2 * D]; for request r it equals the reference's cat(...).relu() rows
    before out_project."""
    sr, er, idx, mask, rcu, scu = _span_args(start_rep, end_rep, row_cu, span_idx, span_mask, span_cu)
    W, D = sr.shape
    S = idx.shape[0]
    out = torch.empty(S, 2 * D, dtype=sr.dtype, device=sr.device)
    if S:
        _lib.on_device("vfk_gliner_span_rows", sr.device, sr.data_ptr(), er.data_ptr(),
                       D * sr.element_size(), W, _SPAN_DT[sr.dtype], rcu.data_ptr(), rcu.numel() - 1,
                       idx.data_ptr(), mask.data_ptr(), scu.data_ptr(), S, out.data_ptr())
    return out


def gliner_span_hidden(a: torch.Tensor, b: torch.Tensor, bias, row_cu: torch.Tensor,
                       span_idx: torch.Tensor, span_mask: torch.Tensor,
                       span_cu: torch.Tensor) -> torch.Tensor:
    """relu(a[i] + b[j] + bias) per span: the first layer (Linear + ReLU) of
    SpanMarkerV0's out_project without the pair rows, for a = relu(start_rep)
    W1[:, :D]^T and b = relu(end_rep) W1[:, D:]^T (per word row) and bias =
    b1 (or None). Rows, spans and masks as in gliner_span_rows. Returns
    [S, N] of a's dtype, summed in fp32 and rounded once."""
    a, b, idx, mask, rcu, scu = _span_args(a, b, row_cu, span_idx, span_mask, span_cu)
    W, N = a.shape
    S = idx.shape[0]
    bp = None
    if bias is not None:
        bias = bias.to(device=a.device, dtype=a.dtype).reshape(-1).contiguous()
        if bias.numel() != N:
            raise ValueError("bias must have one entry per column")
        if bias.data_ptr() % 16:
            bias = bias.clone()
        bp = bias.data_ptr()
    out = torch.empty(S, N, dtype=a.dtype, device=a.device)
    if S:
        _lib.on_device("vfk_gliner_span_hidden", a.device, a.data_ptr(), b.data_ptr(), bp,
                       N * a.element_size(), W, _SPAN_DT[a.dtype], rcu.data_ptr(), rcu.numel() - 1,
                       idx.data_ptr(), mask.data_ptr(), scu.data_ptr(), S, out.data_ptr())
    return out


def span_marker_forward(start_rep: torch.Tensor, end_rep: torch.Tensor, row_cu: torch.Tensor,
                        span_idx: torch.Tensor, span_mask: torch.Tensor, span_cu: torch.Tensor,
                        w1: torch.Tensor, b1, w2: torch.Tensor, b2) -> torch.Tensor:
    """SpanMarkerV0's out_project over every span of a packed batch
    (poolers/gliner.py:141-144, create_projection_layer :26-37 in eval mode:
    Linear(2D, 4D), ReLU, Linear(4D, D)) without the [S, 2D] pair rows. The
    ReLU of cat(start[i], end[j]) acts on each half, so the first Linear
    splits: relu(start) W1[:, :D]^T and relu(end) W1[:, D:]^T are formed once
    per word row (W rows instead of S spans), gliner_span_hidden adds them per
    span with b1 and applies the ReLU, and the second Linear follows. w1
    [4D, 2D], w2 [D, 4D] (nn.Linear weights). Returns [S, D], the rows that
    the reference views as [B, L, max_width, D]."""
    D = start_rep.shape[1]
    if w1.shape[1] != 2 * D:
        raise ValueError("w1 must be [4D, 2D] for start/end rows of width D")
    from .activation import activation
    w1a = w1[:, :D].contiguous()
    w1b = w1[:, D:].contiguous()
    a = torch.matmul(activation(start_rep, "relu"), w1a.t())
    b = torch.matmul(activation(end_rep, "relu"), w1b.t())
    h = gliner_span_hidden(a, b, b1, row_cu, span_idx, span_mask, span_cu)
    if b2 is None:
        return torch.matmul(h, w2.t())
    return torch.addmm(b2.to(h.dtype), h, w2.t())
