"""GPU parity of the GLiNER pooler front-end gathers (kernels/gliner_pooler.py)
against the oracle (oracle/packing.py gliner_reps_packed, the per-request
_extract_gliner_reps of poolers/gliner.py:313-347). Row gathers: bit-exact."""
import pytest
import torch

import workloads
from oracle import packing as op
from _tol import cosine

pytestmark = pytest.mark.gpu

E = 128001


def _check(hidden, ids, wm, cu, tls, embed=True):
    from kernels.gliner_pooler import extract_gliner_reps, gliner_reps_packed
    print(f"gliner reps: T={hidden.shape[0]} H={hidden.shape[1]} {hidden.dtype} "
          f"n={cu.numel() - 1} embed={embed}", flush=True)
    want_pe, want_we = op.gliner_reps_packed(hidden, ids, wm, cu.tolist(), tls, E, embed)
    dev = "cuda"
    pe, pe_cu, we, we_cu = gliner_reps_packed(hidden.to(dev), ids.to(dev), wm.to(dev), cu.to(dev),
                                              tls, E, embed)
    torch.cuda.synchronize()
    assert pe_cu.tolist() == [0] + torch.tensor([p.shape[0] for p in want_pe]).cumsum(0).tolist()
    assert we_cu.tolist() == [0] + torch.tensor([int(t) for t in tls]).cumsum(0).tolist()
    assert torch.equal(pe.cpu(), torch.cat(want_pe))
    assert torch.equal(we.cpu(), torch.cat(want_we))
    reps = extract_gliner_reps(hidden.to(dev), ids.to(dev), wm.to(dev), cu.to(dev), tls, E, embed)
    assert len(reps) == len(want_pe)
    for (p, pm, w, wmk), wp, ww in zip(reps, want_pe, want_we):
        assert p.shape == (1,) + tuple(wp.shape) and w.shape == (1,) + tuple(ww.shape)
        assert torch.equal(p[0].cpu(), wp) and torch.equal(w[0].cpu(), ww)
        assert pm.shape == (1, wp.shape[0]) and bool((pm == 1).all())
        assert wmk.shape == (1, ww.shape[0]) and bool((wmk == 1).all())


@pytest.mark.parametrize("embed", [True, False])
@pytest.mark.parametrize("dtype, H", [(torch.bfloat16, 768), (torch.float32, 1024),
                                      (torch.float16, 8)])
def test_gliner_reps_requests(embed, dtype, H):
    r = workloads.gliner_requests(24, 120, 300)
    g = torch.Generator().manual_seed(H)
    hidden = torch.randn(r.ids.numel(), H, generator=g).to(dtype)
    _check(hidden, r.ids, r.words_mask, r.cu_seqlens, r.text_lengths, embed)


def test_gliner_reps_full_batch():
    """256 requests of 512-768 tokens (the config-5 stream size), bf16 768."""
    r = workloads.gliner_requests()
    hidden = torch.randn(r.ids.numel(), 768, generator=torch.Generator().manual_seed(1)).bfloat16()
    _check(hidden, r.ids, r.words_mask, r.cu_seqlens, r.text_lengths)


def test_gliner_reps_edge_requests():
    """No class tokens, no words, a zero gap inside a word run (the keep rule
    looks past it), words that never appear (zero rows), more text length
    than words, a one-token request, and a long prompt-free run (the
    look-back crosses many 64-token steps)."""
    reqs = [
        ([5, 6, 7], [0, 0, 0], 0),
        ([E, 9, 3, 11, 12, 13, 14], [0, 0, 0, 1, 0, 1, 2], 2),
        ([E, 9, E, 8, 3, 11, 12], [0, 0, 0, 0, 0, 2, 2], 4),
        ([E], [0], 0),
        ([3] + [11] * 300, [0] * 150 + [1] * 50 + [0] * 100 + [1], 1),
        ([E, 4, 3] + [11] * 130, [0, 0, 0] + [k // 2 + 1 for k in range(130)], 65),
    ]
    ids = torch.tensor(sum((q[0] for q in reqs), []))
    wm = torch.tensor(sum((q[1] for q in reqs), []))
    cu = torch.tensor([0] + torch.tensor([len(q[0]) for q in reqs]).cumsum(0).tolist(),
                      dtype=torch.int32)
    tls = [q[2] for q in reqs]
    hidden = torch.randn(ids.numel(), 64, generator=torch.Generator().manual_seed(2)).bfloat16()
    _check(hidden, ids, wm, cu, tls, embed=True)


def test_gliner_reps_errors():
    """IndexError where the reference's index_select / indexed write raise."""
    from kernels.gliner_pooler import gliner_reps_packed
    hidden = torch.randn(6, 64, device="cuda").bfloat16()
    ids = torch.tensor([E, 3, 11, 3, 11, E], device="cuda")   # request 1 ends on a class token
    cu = torch.tensor([0, 3, 6], dtype=torch.int32, device="cuda")
    wm = torch.tensor([0, 0, 1, 0, 1, 0], device="cuda")
    print("gliner reps: errors", flush=True)
    gliner_reps_packed(hidden, ids, wm, cu, [1, 1], E, True)
    with pytest.raises(IndexError, match="class token"):
        gliner_reps_packed(hidden, ids, wm, cu, [1, 1], E, False)
    with pytest.raises(IndexError, match="word id"):
        gliner_reps_packed(hidden, ids, wm, cu, [1, 0], E, True)
    with pytest.raises(ValueError, match="cu_seqlens"):
        gliner_reps_packed(hidden, ids, wm, torch.tensor([0, 3, 5], dtype=torch.int32,
                                                         device="cuda"), [1, 1], E, True)


def test_gliner_reps_list_and_int32_inputs():
    """input_ids / words_mask as host lists or int32 tensors, as the
    reference's _to_tensor accepts them: same rows as int64 device tensors."""
    from kernels.gliner_pooler import gliner_reps_packed
    r = workloads.gliner_requests(6, 120, 200)
    hidden = torch.randn(r.ids.numel(), 64, generator=torch.Generator().manual_seed(4)).bfloat16()
    h, cu = hidden.to("cuda"), r.cu_seqlens.to("cuda")
    print("gliner reps: list / int32 inputs", flush=True)
    base = gliner_reps_packed(h, r.ids.to("cuda"), r.words_mask.to("cuda"), cu, r.text_lengths, E)
    for ids, wm in ((r.ids.tolist(), r.words_mask.tolist()),
                    (r.ids.int(), r.words_mask.int().to("cuda"))):
        got = gliner_reps_packed(h, ids, wm, cu, r.text_lengths, E)
        assert torch.equal(got[0], base[0]) and torch.equal(got[2], base[2])
        assert torch.equal(got[1], base[1]) and torch.equal(got[3], base[3])


def _span_batch(dtype, D, seed):
    g = torch.Generator().manual_seed(seed)
    lens = [int(x) for x in torch.randint(1, 40, (7,), generator=g)]
    W = sum(lens)
    start = torch.randn(W, D, generator=g).to(dtype)
    end = torch.randn(W, D, generator=g).to(dtype)
    idxs, masks, counts = [], [], []
    for r, L in enumerate(lens):
        if r % 2 == 0:   # the pooler's default spans, text shorter than the block
            i, m = op.gliner_default_spans(L, max(L - 3, 0), 12)
        else:            # caller-given spans: out-of-range indices, random masks
            S = int(torch.randint(0, 60, (1,), generator=g))
            i = torch.randint(-5, L + 5, (S, 2), generator=g)
            m = torch.randint(0, 3, (S,), generator=g)   # mask values multiply the indices
        idxs.append(i)
        masks.append(m)
        counts.append(i.shape[0])
    cu = lambda c: torch.tensor([0] + torch.tensor(c).cumsum(0).tolist(), dtype=torch.int32)
    return start, end, lens, idxs, masks, cu(lens), cu(counts)


@pytest.mark.parametrize("dtype, D", [(torch.bfloat16, 768), (torch.float32, 1024),
                                      (torch.float16, 8)])
def test_gliner_span_rows(dtype, D):
    from kernels.gliner_pooler import gliner_span_rows
    start, end, lens, idxs, masks, row_cu, span_cu = _span_batch(dtype, D, D)
    print(f"gliner span rows {dtype} D={D} spans={int(span_cu[-1])}", flush=True)
    got = gliner_span_rows(start.cuda(), end.cuda(), row_cu.cuda(), torch.cat(idxs).cuda(),
                           torch.cat(masks).cuda(), span_cu.cuda()).cpu()
    for r in range(len(lens)):
        a, b = int(row_cu[r]), int(row_cu[r + 1])
        want = op.gliner_span_rows(start[a:b], end[a:b], idxs[r], masks[r])
        assert torch.equal(got[int(span_cu[r]):int(span_cu[r + 1])], want), f"request {r}"


@pytest.mark.parametrize("dtype, D", [(torch.bfloat16, 768), (torch.float32, 1000),
                                      (torch.float16, 24)])
@pytest.mark.parametrize("lead", [0, 5])
def test_gliner_span_rows_default_span_lists(dtype, D, lead):
    """Default span lists only (waves of 48 spans then cover 4 starts x 12
    widths, the kernel's one-load-per-row form), and the same after a
    caller-given request of `lead` spans (waves straddle starts): bit for bit
    against the oracle's pair rows."""
    from kernels.gliner_pooler import gliner_span_rows
    g = torch.Generator().manual_seed(61 + D + lead)
    lens = [int(x) for x in torch.randint(1, 45, (9,), generator=g)]
    idxs, masks = [], []
    if lead:
        lens = [6] + lens
        idxs.append(torch.randint(0, 6, (lead, 2), generator=g))
        masks.append(torch.ones(lead, dtype=torch.int64))
    for L in lens[1 if lead else 0:]:
        i, m = op.gliner_default_spans(L, L, 12)
        idxs.append(i)
        masks.append(m)
    cu = lambda c: torch.tensor([0] + torch.tensor(c).cumsum(0).tolist(), dtype=torch.int32)
    row_cu, span_cu = cu(lens), cu([i.shape[0] for i in idxs])
    W = sum(lens)
    start = torch.randn(W, D, generator=g).to(dtype)
    end = torch.randn(W, D, generator=g).to(dtype)
    print(f"gliner span rows default lists {dtype} D={D} lead={lead} spans={int(span_cu[-1])}",
          flush=True)
    got = gliner_span_rows(start.cuda(), end.cuda(), row_cu.cuda(), torch.cat(idxs).cuda(),
                           torch.cat(masks).cuda(), span_cu.cuda()).cpu()
    want = torch.cat([op.gliner_span_rows(start[a:b], end[a:b], i, m)
                      for a, b, i, m in zip(row_cu[:-1].tolist(), row_cu[1:].tolist(), idxs, masks)])
    assert torch.equal(got, want)


def test_gliner_span_rows_special_values():
    """ReLU on the bits: negatives (-0 and -inf included) become +0, NaN and
    +inf pass; an empty request gives zero rows."""
    from kernels.gliner_pooler import gliner_span_rows
    vals = torch.tensor([float("nan"), -0.0, float("-inf"), float("inf"), -2.5, 3.0, 0.0, -1e-30])
    start = vals.repeat(1, 1).bfloat16()
    end = (-vals).repeat(1, 1).bfloat16()
    print("gliner span rows special values", flush=True)
    out = gliner_span_rows(start.cuda(), end.cuda(), torch.tensor([0, 1, 1]), torch.tensor([[0, 0], [0, 0]]),
                           torch.tensor([1, 1]), torch.tensor([0, 1, 2])).cpu()
    want = torch.tensor([float("nan"), 0.0, 0.0, float("inf"), 0.0, 3.0, 0.0, 0.0,
                         float("nan"), 0.0, float("inf"), 0.0, 2.5, 0.0, 0.0, 1e-30]).bfloat16()
    got0 = out[0].float()
    assert torch.isnan(got0[0]) and torch.isnan(got0[8])
    assert torch.equal(out[0, 1:8].view(torch.int16), want[1:8].view(torch.int16))
    assert torch.equal(out[0, 9:].view(torch.int16), want[9:].view(torch.int16))
    assert torch.all(out[1] == 0) and not torch.any(torch.signbit(out[1].float()))


def _span_sources(lens, idxs, masks):
    """(i, j) source rows of every span (global row numbers), read back from
    the oracle's pair rows of rows that encode their own index."""
    src, base = [], 0
    for L, i, m in zip(lens, idxs, masks):
        enc = (torch.arange(L, dtype=torch.float64) + 1).unsqueeze(1)
        rows = op.gliner_span_rows(enc, enc, i, m)
        src.append(rows.long() - 1 + base)
        base += L
    return torch.cat(src)


@pytest.mark.parametrize("dtype, N", [(torch.bfloat16, 3072), (torch.float32, 256),
                                      (torch.float16, 24)])
def test_gliner_span_hidden_matches_gathered_sum(dtype, N):
    """relu(a[i] + b[j] + bias) per span, bit for bit against the same fp32
    sum in that order over the oracle's source rows (mask values of 0, 1, 2,
    clamped indices, default and caller-given span lists)."""
    from kernels.gliner_pooler import gliner_span_hidden
    _, _, lens, idxs, masks, row_cu, span_cu = _span_batch(dtype, 8, 100 + N)
    W = sum(lens)
    g = torch.Generator().manual_seed(N)
    a = torch.randn(W, N, generator=g).to(dtype)
    b = torch.randn(W, N, generator=g).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    print(f"gliner span hidden {dtype} N={N} spans={int(span_cu[-1])}", flush=True)
    got = gliner_span_hidden(a.cuda(), b.cuda(), bias.cuda(), row_cu.cuda(), torch.cat(idxs).cuda(),
                             torch.cat(masks).cuda(), span_cu.cuda()).cpu()
    src = _span_sources(lens, idxs, masks)
    want = torch.relu((a.float()[src[:, 0]] + b.float()[src[:, 1]]) + bias.float()).to(dtype)
    assert torch.equal(got, want)
    nob = gliner_span_hidden(a.cuda(), b.cuda(), None, row_cu.cuda(), torch.cat(idxs).cuda(),
                             torch.cat(masks).cuda(), span_cu.cuda()).cpu()
    assert torch.equal(nob, torch.relu(a.float()[src[:, 0]] + b.float()[src[:, 1]]).to(dtype))


@pytest.mark.parametrize("dtype, N", [(torch.bfloat16, 3072), (torch.float32, 1000),
                                      (torch.float16, 24)])
@pytest.mark.parametrize("lead", [0, 5])
def test_gliner_span_hidden_default_span_lists(dtype, N, lead):
    """Default span lists only (every wave of 12 spans then shares one start
    row, the kernel's one-load-per-start form), and the same lists after a
    caller-given request of `lead` spans, so that the waves straddle two
    starts; bit for bit against the fp32 sum over the oracle's rows, with and
    without bias."""
    from kernels.gliner_pooler import gliner_span_hidden
    g = torch.Generator().manual_seed(31 + N + lead)
    lens = [int(x) for x in torch.randint(1, 40, (9,), generator=g)]
    idxs, masks = [], []
    if lead:
        lens = [6] + lens
        idxs.append(torch.randint(0, 6, (lead, 2), generator=g))
        masks.append(torch.ones(lead, dtype=torch.int64))
    for L in lens[1 if lead else 0:]:
        i, m = op.gliner_default_spans(L, L, 12)
        idxs.append(i)
        masks.append(m)
    cu = lambda c: torch.tensor([0] + torch.tensor(c).cumsum(0).tolist(), dtype=torch.int32)
    row_cu, span_cu = cu(lens), cu([i.shape[0] for i in idxs])
    W = sum(lens)
    a = torch.randn(W, N, generator=g).to(dtype)
    b = torch.randn(W, N, generator=g).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    print(f"gliner span hidden default lists {dtype} N={N} lead={lead} spans={int(span_cu[-1])}",
          flush=True)
    src = _span_sources(lens, idxs, masks)
    args = (row_cu.cuda(), torch.cat(idxs).cuda(), torch.cat(masks).cuda(), span_cu.cuda())
    got = gliner_span_hidden(a.cuda(), b.cuda(), bias.cuda(), *args).cpu()
    want = torch.relu((a.float()[src[:, 0]] + b.float()[src[:, 1]]) + bias.float()).to(dtype)
    assert torch.equal(got, want)
    nob = gliner_span_hidden(a.cuda(), b.cuda(), None, *args).cpu()
    assert torch.equal(nob, torch.relu(a.float()[src[:, 0]] + b.float()[src[:, 1]]).to(dtype))


def test_gliner_span_hidden_request_without_rows():
    """A request with no rows gives relu(bias) for each of its spans."""
    from kernels.gliner_pooler import gliner_span_hidden
    a = torch.randn(3, 16).bfloat16()
    bias = torch.linspace(-1, 1, 16).bfloat16()
    out = gliner_span_hidden(a.cuda(), a.cuda(), bias.cuda(), torch.tensor([0, 3, 3]),
                             torch.tensor([[0, 1], [1, 1], [0, 0]]), torch.tensor([1, 1, 1]),
                             torch.tensor([0, 2, 3])).cpu()
    assert torch.equal(out[2], torch.relu(bias.float()).bfloat16())
    assert torch.equal(out[0], torch.relu(a[0].float() + a[1].float() + bias.float()).bfloat16())


def test_fit_word_rows_matches_oracle():
    """Per-request _fit_length over packed word rows: cut, kept and padded."""
    from kernels.gliner_pooler import fit_word_rows
    g = torch.Generator().manual_seed(9)
    lens, targets = [5, 3, 0, 7], [3, 3, 4, 9]
    we = torch.randn(sum(lens), 8, generator=g).bfloat16()
    cu = [0] + torch.tensor(lens).cumsum(0).tolist()
    rows, row_cu = fit_word_rows(we.cuda(), cu, targets)
    assert row_cu.cpu().tolist() == [0, 3, 6, 10, 19]
    want = torch.cat([op.gliner_fit_length(we[cu[r]:cu[r + 1]], t) for r, t in enumerate(targets)])
    assert torch.equal(rows.cpu(), want)


def test_span_marker_forward_matches_oracle():
    """SpanMarkerV0's out_project over every span of a packed batch with the
    first Linear split per word row, against the oracle's composition
    (pair rows, then Linear(2D, 4D), ReLU, Linear(4D, D) in fp32) on the same
    bf16 rows and weights. Two requests take caller span lists whose width
    count differs from their text length, fitted by fit_word_rows as the
    reference's _fit_length does. The GPU path rounds a, b, the hidden
    layer and the output to bf16: max-abs error bounded by 2e-2 of the
    output scale, cosine 0.9999."""
    from kernels.gliner_pooler import default_spans, fit_word_rows, span_marker_forward
    g = torch.Generator().manual_seed(77)
    D, K = 64, 12
    lens = [9, 14, 6, 11]
    targets = [9, 10, 6, 13]                 # requests 1 and 3 fitted (cut, padded)
    we = torch.randn(sum(lens), D, generator=g).bfloat16()
    cu = [0] + torch.tensor(lens).cumsum(0).tolist()
    idxs, masks = [], []
    for r, (L, t) in enumerate(zip(lens, targets)):
        i, m = default_spans(t, min(L, t), K)
        if r == 3:
            m = m * 2                        # mask value 2: indices doubled
        idxs.append(i)
        masks.append(m)
    span_cu = torch.tensor([0] + torch.tensor([x.shape[0] for x in idxs]).cumsum(0).tolist(),
                           dtype=torch.int32)
    fitted, row_cu = fit_word_rows(we.cuda(), cu, targets)
    # start/end projections stand in as two random linear maps of the rows
    ps = (torch.randn(D, D, generator=g) / D ** 0.5).bfloat16()
    pe_ = (torch.randn(D, D, generator=g) / D ** 0.5).bfloat16()
    start = fitted @ ps.cuda()
    end = fitted @ pe_.cuda()
    w1 = (torch.randn(4 * D, 2 * D, generator=g) / (2 * D) ** 0.5).bfloat16()
    b1 = (0.1 * torch.randn(4 * D, generator=g)).bfloat16()
    w2 = (torch.randn(D, 4 * D, generator=g) / (4 * D) ** 0.5).bfloat16()
    b2 = (0.1 * torch.randn(D, generator=g)).bfloat16()
    got = span_marker_forward(start, end, row_cu, torch.cat(idxs).cuda(), torch.cat(masks).cuda(),
                              span_cu.cuda(), w1.cuda(), b1.cuda(), w2.cuda(), b2.cuda()).float().cpu()
    sc, ec, rc = start.cpu(), end.cpu(), row_cu.cpu().tolist()
    want = torch.cat([op.gliner_out_project(op.gliner_span_rows(sc[rc[r]:rc[r + 1]].float(),
                                                                ec[rc[r]:rc[r + 1]].float(), idxs[r], masks[r]),
                                            w1, b1, w2, b2) for r in range(len(lens))])
    assert got.shape == want.shape
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    cs = cosine(got, want)
    print(f"span marker: max-abs {err:.3e} (scale {scale:.3f}) cosine {cs:.6f}", flush=True)
    assert err <= 2e-2 * scale and cs >= 0.9999, (err, scale, cs)
