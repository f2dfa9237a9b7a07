"""Pins the oracle's bucket functions (oracle/buckets.py) independently of the
formula they restate: closed forms, exact arithmetic, transformers' own
implementations, invariants and the committed golden tables."""
import json
import math
import os
from fractions import Fraction

import pytest
import torch

from oracle import buckets as ob

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _t5_exact(rel: int, bidirectional: bool, nb: int, md: int) -> int:
    """T5 bucket in exact arithmetic (log ratios as exact rationals where they
    are powers of the base, fp64 elsewhere with a margin check)."""
    off = 0
    if bidirectional:
        nb //= 2
        off = nb if rel > 0 else 0
        a = abs(rel)
    else:
        a = max(-rel, 0)
    me = nb // 2
    if a < me:
        return a + off
    val = math.log(a / me) / math.log(md / me) * (nb - me)
    near = round(val)
    if abs(val - near) < 1e-9:
        val = near  # exact ratio of logs (a/me a power of md/me's root)
    return min(me + int(math.floor(val)), nb - 1) + off


@pytest.mark.parametrize("bidirectional", [True, False])
@pytest.mark.parametrize("nb,md", [(32, 128), (32, 64), (64, 256), (128, 1024)])
def test_t5_bucket_exact_math(bidirectional, nb, md):
    rel = torch.arange(-1500, 1501)
    got = ob.t5_relative_position_bucket(rel, bidirectional, nb, md).tolist()
    want = [_t5_exact(int(r), bidirectional, nb, md) for r in rel]
    assert got == want


def test_t5_bucket_closed_forms():
    rel = torch.arange(-3000, 3001)
    b = ob.t5_relative_position_bucket(rel, True, 32, 128)
    a = rel.abs()
    small = a < 8
    assert torch.equal(b[small], a[small] + 16 * (rel[small] > 0))
    big = a >= 128
    assert torch.equal(b[big], 15 + 16 * (rel[big] > 0))
    # the rounding points named in the survey: |rel| = 16, 32, 64
    for r, v in ((16, 10), (32, 12), (64, 14), (-16, 10), (-64, 14)):
        assert int(ob.t5_relative_position_bucket(torch.tensor([r]), True, 32, 128)) == v + (16 if r > 0 else 0)


@pytest.mark.parametrize("bidirectional", [True, False])
@pytest.mark.parametrize("nb,md", [(32, 128), (32, 64), (64, 256), (16, 100), (128, 1024)])
def test_t5_bucket_matches_transformers(bidirectional, nb, md):
    from transformers.models.t5.modeling_t5 import T5Attention
    rel = torch.arange(-2000, 2001)[None, :]
    a = ob.t5_relative_position_bucket(rel, bidirectional, nb, md)
    b = T5Attention._relative_position_bucket(rel, bidirectional, nb, md)
    assert torch.equal(a, b)


def test_t5_bucket_matrix_is_toeplitz_and_monotone():
    m = ob.t5_bucket_matrix(300, 400, True, 32, 128)
    for d in range(-299, 400):
        assert torch.unique(torch.diagonal(m, d)).numel() == 1
    r = torch.arange(0, 2000)
    b = ob.t5_relative_position_bucket(r, True, 32, 128)
    assert bool((b[1:] >= b[:-1]).all())
    bn = ob.t5_relative_position_bucket(-r, True, 32, 128)
    assert bool((bn[1:] >= bn[:-1]).all())


def _deb_exact(rel: int, bs: int, mp: int) -> int:
    mid = bs // 2
    a = abs(rel)
    if a <= mid:
        return rel
    val = math.log(a / mid) / math.log((mp - 1) / mid) * (mid - 1)
    near = round(val)
    if abs(val - near) < 1e-9:
        val = near
    v = mid + int(math.ceil(val))
    return v if rel > 0 else -v


@pytest.mark.parametrize("bs,mp", [(256, 512), (256, 1024), (128, 512), (64, 256)])
def test_deberta_bucket_exact_math(bs, mp):
    rel = torch.arange(-1200, 1201)
    got = ob.make_log_bucket_position(rel, bs, mp).long().tolist()
    assert got == [_deb_exact(int(r), bs, mp) for r in rel]


def test_deberta_bucket_closed_forms_and_symmetry():
    rel = torch.arange(-2000, 2001)
    b = ob.make_log_bucket_position(rel, 256, 512)
    assert b.dtype == torch.float32
    small = rel.abs() <= 128
    assert torch.equal(b[small].long(), rel[small])
    assert torch.equal(b, -b.flip(0))                 # odd symmetry
    assert bool((b[1:] >= b[:-1]).all())              # monotone
    assert int(ob.make_log_bucket_position(torch.tensor([511]), 256, 512)) == 255
    assert int(ob.make_log_bucket_position(torch.tensor([-511]), 256, 512)) == -255
    assert int(ob.make_log_bucket_position(torch.tensor([129]), 256, 512)) == 129


@pytest.mark.parametrize("bs,mp", [(256, 512), (256, 1024), (128, 512), (64, 256)])
def test_deberta_bucket_matches_transformers(bs, mp):
    from transformers.models.deberta_v2 import modeling_deberta_v2 as md
    rel = torch.arange(-1100, 1101)
    assert torch.equal(ob.make_log_bucket_position(rel, bs, mp), md.make_log_bucket_position(rel, bs, mp))


def test_golden_bucket_tables():
    with open(os.path.join(GOLD, "t5_buckets.json")) as f:
        t5 = json.load(f)
    for case in t5["cases"]:
        rel = torch.arange(case["rel_min"], case["rel_min"] + len(case["bucket"]))
        got = ob.t5_relative_position_bucket(rel, case["bidirectional"], case["num_buckets"],
                                             case["max_distance"])
        assert got.tolist() == case["bucket"]
    with open(os.path.join(GOLD, "deberta_buckets.json")) as f:
        deb = json.load(f)
    for case in deb["cases"]:
        rel = torch.arange(case["rel_min"], case["rel_min"] + len(case["bucket"]))
        got = ob.make_log_bucket_position(rel, case["bucket_size"], case["max_position"]).long()
        assert got.tolist() == case["bucket"]
