"""Pins the oracle's packed-stream plumbing (oracle/packing.py): positions
built from known lengths, hand cases, a pairwise brute force of the segment
rule, the reference's dense-mask formulation of ModernBERT attention, and the
GLiNER re-padding loop's round trip."""
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oa
from oracle import packing as op

D64 = torch.float64


def _r(*shape, seed=0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=D64)


# ------------------------------------------------------- packed-sequence metadata
def _positions(lens):
    return torch.cat([torch.arange(n) for n in lens])


@pytest.mark.parametrize("lens", [[1], [5], [1, 1, 1], [3, 1, 4, 1, 5], [700, 300, 129, 64],
                                  [2] * 50])
def test_seq_metadata_recovers_lengths(lens):
    """Positions built from known lengths give those lengths back (a '<' for
    '<=' merges the runs of length 1; an off-by-one shifts every start)."""
    cu, n, mx, bad = op.seq_metadata(_positions(lens))
    assert cu.tolist() == [0] + torch.tensor(lens).cumsum(0).tolist()
    assert (n, mx, bad) == (len(lens), max(lens), 0)


@pytest.mark.parametrize("pos, cu, bad", [
    ([0, 1, 2, 5, 6], [0, 5], 1),        # no reset: one sequence, one gap
    ([0, 1, 2, 1, 2], [0, 3, 5], 1),     # reset to 1: a sequence that does not start at 0
    ([3, 4, 0, 0, 1], [0, 2, 3, 5], 1),  # first sequence starts at 3
    ([0, 0, 0], [0, 1, 2, 3], 0),        # equal positions are resets
    ([7], [0, 1], 1),
    ([3, 4, 5, 9, 10, 0, 1, 1, 2, 7], [0, 5, 7, 10], 4),
])
def test_seq_metadata_hand_cases(pos, cu, bad):
    got_cu, n, mx, got_bad = op.seq_metadata(torch.tensor(pos))
    assert got_cu.tolist() == cu and got_bad == bad and n == len(cu) - 1
    assert mx == max(b - a for a, b in zip(cu[:-1], cu[1:]))


@pytest.mark.parametrize("seed", range(6))
def test_seq_metadata_bad_is_zero_iff_positions_are_offsets(seed):
    """bad == 0 exactly when each token's position is its index minus the
    start of its sequence (checked on random streams, some built valid)."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, 9, (40,), generator=g).tolist()
    pos = _positions(lens)
    if seed % 2:
        i = int(torch.randint(0, pos.numel(), (1,), generator=g))
        pos[i] += int(torch.randint(1, 3, (1,), generator=g))
    cu, _, _, bad = op.seq_metadata(pos)
    offset = torch.cat([torch.arange(int(b - a)) for a, b in zip(cu[:-1], cu[1:])])
    assert (bad == 0) == bool(torch.equal(pos, offset)), (seed, bad)
    assert (bad == 0) == (seed % 2 == 0)


def test_seq_metadata_pairwise_brute_force():
    """Tokens i < j share a sequence iff no reset lies in (i, j]: the
    reference's segment-id equality written as a pairwise loop."""
    g = torch.Generator().manual_seed(3)
    pos = torch.randint(0, 6, (60,), generator=g)
    cu, _, _, _ = op.seq_metadata(pos)
    seg = torch.zeros(60, dtype=torch.int64)
    for s in range(len(cu) - 1):
        seg[cu[s]:cu[s + 1]] = s
    for i in range(60):
        for j in range(i, 60):
            same = all(pos[t] > pos[t - 1] for t in range(i + 1, j + 1))
            assert (seg[i] == seg[j]) == same, (i, j)


def test_seq_metadata_drives_varlen_like_dense_masks():
    """The reference's own formulation at modernbert_encoder.py:236-255 and
    :491-550 (RoPE by position id, one SDPA over the whole stream with the
    block-diagonal and sliding-window masks) equals the per-sequence varlen
    oracle run on the cu_seqlens the metadata derives."""
    lens, w, theta = [9, 1, 23, 14], 4, 10000.0
    pos = _positions(lens)
    T = pos.numel()
    q, k, v = _r(T, 2, 64, seed=40), _r(T, 2, 64, seed=41), _r(T, 2, 64, seed=42)
    cu, _, _, _ = op.seq_metadata(pos)
    starts = torch.zeros(T, dtype=torch.bool)
    starts[0] = True
    starts[1:] = pos[1:] <= pos[:-1]
    seg = starts.cumsum(0)
    cos, sin = oa.rope_cos_sin(pos, theta)
    qr, kr = oa.apply_rope(q, cos.to(D64), sin.to(D64)), oa.apply_rope(k, cos.to(D64), sin.to(D64))
    for window in (-1, w):
        vis = seg[:, None] == seg[None, :]
        if window >= 0:
            idx = torch.arange(T)
            vis &= (idx[:, None] - idx[None, :]).abs() <= window
        want = F.scaled_dot_product_attention(qr.transpose(0, 1), kr.transpose(0, 1),
                                              v.transpose(0, 1), attn_mask=vis,
                                              scale=0.125).transpose(0, 1)
        got = oa.varlen_attention(q, k, v, cu, window, theta, None, 0.125, dtype=D64)
        torch.testing.assert_close(got, want)


# ------------------------------------------------------- rule "zero" (GLiNER plugins)
@pytest.mark.parametrize("pos, reset_cu, zero_cu", [
    ([0, 1, 2, 0, 1], [0, 3, 5], [0, 3, 5]),            # well-formed: the rules agree
    ([0, 1, 1, 2, 0], [0, 2, 4, 5], [0, 4, 5]),         # a repeat resets only under "reset"
    ([0, 5, 3, 4], [0, 2, 4], [0, 4]),                  # a decrease resets only under "reset"
    ([0, 0, 0], [0, 1, 2, 3], [0, 1, 2, 3]),
])
def test_seq_metadata_rules(pos, reset_cu, zero_cu):
    assert op.seq_metadata(torch.tensor(pos), "reset")[0].tolist() == reset_cu
    assert op.seq_metadata(torch.tensor(pos), "zero")[0].tolist() == zero_cu


@pytest.mark.parametrize("lens", [[1], [4, 1, 7], [300, 2, 129], [1] * 20])
def test_gliner_batch_matches_known_lengths(lens):
    """The loop restatement puts sequence b's ids in row b, pad_id after it,
    and its lengths agree with the metadata's cu_seqlens under rule "zero"."""
    g = torch.Generator().manual_seed(len(lens))
    pos = torch.cat([torch.arange(n) for n in lens])
    ids = torch.randint(1, 1000, (pos.numel(),), generator=g)
    bids, bpos, mask, got_lens = op.gliner_batch(ids, pos, pad_id=-7)
    assert got_lens == lens
    cu, n, mx, bad = op.seq_metadata(pos, "zero")
    assert (n, mx, bad) == (len(lens), max(lens), 0)
    assert cu.tolist() == [0] + torch.tensor(lens).cumsum(0).tolist()
    for b, L in enumerate(lens):
        a = int(cu[b])
        assert torch.equal(bids[b, :L], ids[a:a + L])
        assert bool((bids[b, L:] == -7).all()) and bool((bpos[b, L:] == 0).all())
        assert torch.equal(bpos[b, :L], torch.arange(L))
        assert mask[b].tolist() == [1] * L + [0] * (mx - L)
    # round trip: the valid rows, concatenated, are the flat stream again
    assert torch.equal(op.gliner_unbatch(bids, got_lens), ids)
    h = torch.randn(pos.numel(), 3, generator=g)
    hb = torch.zeros(len(lens), mx, 3)
    for b, L in enumerate(lens):
        hb[b, :L] = h[int(cu[b]):int(cu[b]) + L]
    assert torch.equal(op.gliner_unbatch(hb, got_lens), h)


# ------------------------------------------------------- GLiNER prompt / word gathers
E = 99  # class token id


def _index_rows(T, H=4):
    """Hidden rows that hold their own index: a gathered row names its source."""
    return torch.arange(T, dtype=D64).unsqueeze(1).repeat(1, H)


def _src(rows):
    return rows[:, 0].long().tolist()


@pytest.mark.parametrize("embed, pe_src", [(True, [1, 3]), (False, [2, 4])])
def test_gliner_reps_hand_case(embed, pe_src):
    """Prompt '<x> E a E b <sep>' then three subtokens of two words: word 0
    spans tokens 6-7 (first subtoken 6, not the last one, 7) and word 1 is
    token 8; the class rows move one token right when the class token itself
    is not embedded."""
    ids = torch.tensor([5, E, 7, E, 8, 3, 11, 12, 13])
    wm = torch.tensor([0, 0, 0, 0, 0, 0, 1, 1, 2])
    pe, we = op.gliner_reps(_index_rows(9), ids, wm, 2, E, embed)
    assert _src(pe) == pe_src
    assert _src(we) == [6, 8]


def test_gliner_reps_keep_rule_skips_zero_gaps():
    """The first-subtoken rule compares with the previous token whose mask is
    positive, across zeros: mask [1, 0, 1, 2] keeps token 0 for word 0."""
    _, we = op.gliner_reps(_index_rows(4), torch.zeros(4, dtype=torch.long),
                           torch.tensor([1, 0, 1, 2]), 2, E)
    assert _src(we) == [0, 3]


def test_gliner_reps_unwritten_words_stay_zero():
    h = _index_rows(5) + 1.0
    _, we = op.gliner_reps(h, torch.zeros(5, dtype=torch.long), torch.tensor([0, 2, 2, 4, 0]), 5, E)
    assert we[:, 0].tolist() == [0.0, 2.0, 0.0, 4.0, 0.0]


def test_gliner_reps_errors():
    """The reference's index_select / indexed write raise on these."""
    with pytest.raises(IndexError):
        op.gliner_reps(_index_rows(3), torch.tensor([0, 1, E]), torch.zeros(3, dtype=torch.long),
                       0, E, embed_ent_token=False)
    with pytest.raises(IndexError):
        op.gliner_reps(_index_rows(3), torch.zeros(3, dtype=torch.long), torch.tensor([1, 2, 3]),
                       2, E)


def test_gliner_reps_by_construction():
    """Requests built from word subtoken counts: word k's row must be the token
    at prompt_len + (subtokens of words 0..k-1), the class rows the E positions,
    in a packed stream of several requests."""
    g = torch.Generator().manual_seed(3)
    ids, wms, cu, tls, want_pe, want_we = [], [], [0], [], [], []
    for r in range(6):
        n_cls = int(torch.randint(0, 5, (1,), generator=g))
        counts = torch.randint(1, 4, (int(torch.randint(0, 12, (1,), generator=g)),), generator=g)
        prompt = []
        for _ in range(n_cls):
            want_pe.append(cu[-1] + len(prompt))
            prompt += [E, 7]
        prompt += [3]
        start = cu[-1] + len(prompt)
        firsts = (torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)[:-1]]) + start).tolist()
        want_we += firsts
        mask = [0] * len(prompt) + [k + 1 for k, c in enumerate(counts.tolist()) for _ in range(c)]
        ids += prompt + [11] * int(counts.sum())
        wms += mask
        cu.append(cu[-1] + len(mask))
        tls.append(len(counts))
    h = _index_rows(cu[-1])
    pes, wes = op.gliner_reps_packed(h, torch.tensor(ids), torch.tensor(wms), cu, tls, E)
    assert sum((_src(p) for p in pes), []) == want_pe
    assert sum((_src(w) for w in wes), []) == want_we


def test_gliner_default_spans_hand_case():
    idx, mask = op.gliner_default_spans(3, 2, 2)
    assert idx.tolist() == [[0, 0], [0, 1], [1, 1], [1, 2], [2, 2], [2, 3]]
    assert mask.tolist() == [1, 1, 1, 0, 0, 0]


def test_gliner_default_spans_mirror():
    """The device-side helper's torch construction equals the loop."""
    from kernels.gliner_pooler import default_spans
    for L, T, K in [(5, 3, 4), (1, 1, 12), (7, 7, 3), (4, 0, 2), (0, 0, 3)]:
        a, b = default_spans(L, T, K), op.gliner_default_spans(L, T, K)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_gliner_span_rows_sources_and_relu():
    """Start rows hold i + 1 and end rows 100 + j, so each output names its
    sources: a masked span takes rows (0, 0), indices clamp into [0, L - 1],
    and negative values leave the ReLU as zeros."""
    L = 4
    start = (torch.arange(L, dtype=D64) + 1).unsqueeze(1).repeat(1, 2)
    end = (torch.arange(L, dtype=D64) + 100).unsqueeze(1).repeat(1, 2)
    idx = torch.tensor([[1, 2], [3, 3], [2, 3], [-3, 99]])
    out = op.gliner_span_rows(start, end, idx, torch.tensor([1, 1, 0, 1]))
    assert out[:, 0].tolist() == [2.0, 4.0, 1.0, 1.0]
    assert out[:, 2].tolist() == [102.0, 103.0, 100.0, 103.0]
    neg = op.gliner_span_rows(-start, end, idx[:1], torch.tensor([1]))
    assert neg[0].tolist() == [0.0, 0.0, 102.0, 102.0]


def test_gliner_span_rows_multiply_by_mask_value():
    """The reference multiplies the indices by the mask value (:286): a mask
    of 2 doubles them before the clamp, 0 sends both to row 0."""
    L = 4
    start = (torch.arange(L, dtype=D64) + 1).unsqueeze(1)
    end = (torch.arange(L, dtype=D64) + 100).unsqueeze(1)
    idx = torch.tensor([[1, 1], [1, 2], [2, 0]])
    out = op.gliner_span_rows(start, end, idx, torch.tensor([2, 2, 0]))
    assert out[:, 0].tolist() == [3.0, 3.0, 1.0]       # rows 2, 2, 0
    assert out[:, 1].tolist() == [102.0, 103.0, 100.0]  # rows 2, min(4, 3), 0


def test_gliner_fit_length_pads_and_cuts():
    we = torch.arange(6, dtype=D64).view(3, 2) + 1
    assert torch.equal(op.gliner_fit_length(we, 3), we)
    assert torch.equal(op.gliner_fit_length(we, 2), we[:2])
    padded = op.gliner_fit_length(we, 5)
    assert torch.equal(padded[:3], we) and torch.equal(padded[3:], torch.zeros(2, 2, dtype=D64))


def test_gliner_out_project_selection_weights():
    """With W1 = [I_2D; 0] (b1 = 0) and W2 = [I_D, I_D, 0, 0], out_project of
    the pair rows is relu(start[i]) + relu(end[j]) in closed form; a bias b1
    of -inf on the start half leaves only the end rows, and b2 shifts all."""
    g = torch.Generator().manual_seed(5)
    D, L = 3, 5
    start = torch.randn(L, D, generator=g, dtype=D64)
    end = torch.randn(L, D, generator=g, dtype=D64)
    idx = torch.tensor([[0, 4], [2, 1], [3, 3]])
    mask = torch.tensor([1, 1, 1])
    pair = op.gliner_span_rows(start, end, idx, mask)
    w1 = torch.cat([torch.eye(2 * D, dtype=D64), torch.zeros(2 * D, 2 * D, dtype=D64)])
    w2 = torch.cat([torch.eye(D, dtype=D64), torch.eye(D, dtype=D64), torch.zeros(D, 2 * D, dtype=D64)], 1)
    out = op.gliner_out_project(pair, w1, None, w2, None)
    want = torch.stack([torch.relu(start[i]) + torch.relu(end[j]) for i, j in idx.tolist()])
    torch.testing.assert_close(out, want.float(), rtol=1e-6, atol=1e-6)
    b1 = torch.cat([torch.full((D,), -1e30, dtype=D64), torch.zeros(3 * D, dtype=D64)])
    b2 = torch.full((D,), 0.5, dtype=D64)
    out2 = op.gliner_out_project(pair, w1, b1, w2, b2)
    want2 = torch.stack([torch.relu(end[j]) + 0.5 for _, j in idx.tolist()])
    torch.testing.assert_close(out2, want2.float(), rtol=1e-6, atol=1e-6)
