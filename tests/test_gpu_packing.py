"""GPU parity of the packed-stream plumbing (kernels/packing.py) against the
oracle (oracle/packing.py): sequence metadata from flat position ids under
both boundary rules, flat <-> padded row copies, and the GLiNER batch built
from a flat call. All of it is integer / byte work: bit-exact."""
import pytest
import torch

import workloads
from oracle import packing as op

pytestmark = pytest.mark.gpu


def _meta_case(name):
    g = torch.Generator().manual_seed(sum(map(ord, name)))
    if name == "one_token":
        return torch.tensor([0])
    if name == "one_sequence":
        return torch.arange(777)
    if name == "all_length_one":          # 5000 resets: every block full of starts
        return torch.zeros(5000, dtype=torch.int64)
    if name == "pairs":
        return torch.arange(2).repeat(3000)
    if name == "config5":                 # 256 sequences of U{512..768}, 163 736 tokens
        lens = workloads.config5().lengths
        return torch.cat([torch.arange(int(n)) for n in lens])
    if name == "many_blocks":             # > 1024 scan blocks: the scan's carry loop
        lens = torch.randint(1, 3000, (900,), generator=g)
        return torch.cat([torch.arange(int(n)) for n in lens])
    if name == "no_restart":              # gaps, repeats, a non-zero first position
        return torch.tensor([3, 4, 5, 9, 10, 0, 1, 1, 2, 7] * 300)
    if name == "random":
        return torch.randint(0, 40, (20000,), generator=g)
    raise KeyError(name)


META_CASES = ["one_token", "one_sequence", "all_length_one", "pairs", "config5", "many_blocks",
              "no_restart", "random"]


@pytest.mark.parametrize("rule", ["reset", "zero"])
@pytest.mark.parametrize("pos_dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("name", META_CASES)
def test_seq_metadata_matches_oracle(dev, name, pos_dtype, rule):
    """Bit-exact cu_seqlens, count, longest length and break count."""
    from kernels.packing import seq_metadata
    pos = _meta_case(name).to(pos_dtype)
    cu, n, mx, bad = op.seq_metadata(pos, rule)
    print(f"seq_metadata case {name} T={pos.numel()} {pos_dtype} rule={rule}", flush=True)
    got_cu, meta = seq_metadata(pos.to(dev)[None], rule)   # the reference's [1, T] layout
    meta = meta.cpu().tolist()
    assert meta == [n, mx, bad, pos.numel()], (meta, [n, mx, bad])
    assert torch.equal(got_cu[:n + 1].cpu(), cu)


def test_seq_metadata_repeat_calls_reset_counters(dev):
    """The maximum and the break count start from zero on every call."""
    from kernels.packing import seq_metadata
    _, meta1 = seq_metadata(_meta_case("no_restart").to(dev))
    _, meta2 = seq_metadata(torch.arange(10, device=dev))
    assert meta1.cpu().tolist()[2] > 0
    assert meta2.cpu().tolist() == [1, 10, 0, 10]


def _rows(T, shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    if dtype.is_floating_point:
        return torch.randn((T,) + shape, generator=g).to(dtype)
    return torch.randint(0, 250, (T,) + shape, generator=g, dtype=dtype)


@pytest.mark.parametrize("shape,dtype", [
    ((1024,), torch.bfloat16),     # DeBERTa-v3-large hidden rows: 16-byte units
    ((), torch.int64),             # token ids: 8-byte units
    ((3,), torch.float16),         # 6-byte rows: 2-byte units
    ((5,), torch.uint8),           # 5-byte rows: 1-byte units
    ((12, 64), torch.float32),
])
@pytest.mark.parametrize("lens", [[1], [512, 256, 300, 511], [1, 1, 7, 1], [4000, 3]])
def test_pad_unpad_match_oracle(dev, shape, dtype, lens):
    from kernels.packing import pad_packed, unpad_packed
    T = sum(lens)
    x = _rows(T, shape, dtype, len(lens))
    cu = workloads.cu_from_lengths(torch.tensor(lens))
    print(f"pad/unpad case {shape} {dtype} lens={lens[:4]}", flush=True)
    fill = 7 if not dtype.is_floating_point else -2.5
    padded, slen = pad_packed(x.to(dev), cu.to(dev), len(lens), max(lens), fill)
    want = torch.full((len(lens), max(lens)) + shape, fill, dtype=dtype)
    for b, n in enumerate(lens):
        want[b, :n] = x[int(cu[b]):int(cu[b]) + n]
    assert torch.equal(padded.cpu(), want)
    assert slen.cpu().tolist() == lens
    back = unpad_packed(padded, cu.to(dev), T)
    assert torch.equal(back.cpu(), op.gliner_unbatch(want, lens))
    assert torch.equal(back.cpu(), x)


def test_pad_cuts_at_max_len_and_unpad_skips_padding(dev):
    """max_len below a length cuts that sequence; unpad never reads padding
    (poisoned here) and leaves flat rows past the cut untouched."""
    from kernels.packing import pad_packed, unpad_packed
    lens = [10, 3]
    x = _rows(13, (8,), torch.float32, 3).to(dev)
    cu = workloads.cu_from_lengths(torch.tensor(lens)).to(dev)
    padded, _ = pad_packed(x, cu, 2, 6)
    assert torch.equal(padded[0], x[:6]) and torch.equal(padded[1, :3], x[10:13])
    poisoned = padded.clone()
    poisoned[1, 3:] = float("nan")
    out = unpad_packed(poisoned, cu, 13)   # rows 6..9 are past the cut: not written
    assert torch.equal(out[:6], x[:6]) and torch.equal(out[10:], x[10:])


@pytest.mark.parametrize("lens", [[7], [300, 2, 129, 1], [1] * 33])
def test_batch_from_flat_matches_gliner_loop(dev, lens):
    """batch_from_flat equals the reference's re-padding loop (restated in the
    oracle) on ids, positions, mask and lengths."""
    from kernels.packing import batch_from_flat
    g = torch.Generator().manual_seed(sum(lens))
    pos = torch.cat([torch.arange(n) for n in lens])
    ids = torch.randint(1, 128000, (pos.numel(),), generator=g)
    want = op.gliner_batch(ids, pos, pad_id=0)
    got = batch_from_flat(ids.to(dev), pos.to(dev), pad_id=0)
    for a, b in zip(got[:3], want[:3]):
        assert torch.equal(a.cpu(), b)
    assert got[4].cpu().tolist() == want[3]


def test_pad_unpad_zero_length_sequences(dev):
    """Empty sequences get a padded block of fill only (their flat rows need
    not exist, even at the end of the stream) and write nothing back."""
    from kernels.packing import pad_packed, unpad_packed
    lens = [0, 3, 0, 2, 0]
    cu = workloads.cu_from_lengths(torch.tensor(lens))
    x = _rows(5, (16,), torch.bfloat16, 9)
    padded, slen = pad_packed(x.to(dev), cu.to(dev), 5, 4, -1.0)
    want = torch.full((5, 4, 16), -1.0, dtype=torch.bfloat16)
    want[1, :3] = x[:3]
    want[3, :2] = x[3:5]
    assert torch.equal(padded.cpu(), want)
    assert slen.cpu().tolist() == lens
    assert torch.equal(unpad_packed(padded, cu.to(dev), 5).cpu(), x)
