"""vfk_varlen_meta_noalloc (the metadata entry point with no workspace and no
allocation) against vfk_varlen_meta with a caller workspace, both through the
C-ABI, on two calls in a row where the second has fewer tokens (the shared
device array then holds the first call's counts, which must not leak into the
second), plus the size limit and the oracle on a third case. Bit-exact:
integer work."""
import pytest
import torch

import workloads

pytestmark = pytest.mark.gpu


def _positions(lens):
    return torch.cat([torch.arange(int(n)) for n in lens])


def _meta_call(fn, pos, rule, dev):
    from kernels import _lib
    T = pos.numel()
    cu = torch.full((T + 1,), -7, dtype=torch.int32, device=dev)
    meta = torch.full((4,), -7, dtype=torch.int32, device=dev)
    if fn == "vfk_varlen_meta":
        ws_bytes = int(_lib.load().vfk_varlen_meta_workspace_bytes(T))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        _lib.on_device(fn, dev, pos.data_ptr(), pos.element_size(), T, rule, cu.data_ptr(),
                       meta.data_ptr(), ws.data_ptr(), ws_bytes)
    else:
        _lib.on_device(fn, dev, pos.data_ptr(), pos.element_size(), T, rule, cu.data_ptr(),
                       meta.data_ptr())
    torch.cuda.synchronize(dev)
    m = meta.cpu().tolist()
    return cu[:m[0] + 1].cpu(), m


@pytest.mark.parametrize("rule", [0, 1])
def test_noalloc_meta_matches_workspace_entry_point(rule):
    dev = torch.device("cuda:0")
    first = _positions(workloads.config5().lengths).to(dev)         # 163 736 tokens, 160 blocks
    g = torch.Generator().manual_seed(77)
    second = _positions(torch.randint(1, 900, (40,), generator=g)).to(torch.int32).to(dev)
    for pos in (first, second):
        print(f"no-alloc meta: T={pos.numel()} {pos.dtype} rule={rule}", flush=True)
        want_cu, want_m = _meta_call("vfk_varlen_meta", pos, rule, dev)
        got_cu, got_m = _meta_call("vfk_varlen_meta_noalloc", pos, rule, dev)
        assert got_m == want_m, (got_m, want_m)
        assert torch.equal(got_cu, want_cu)


def test_noalloc_meta_matches_oracle_and_limit():
    from kernels import _lib
    from oracle import packing as op
    dev = torch.device("cuda:0")
    pos = torch.tensor([3, 4, 5, 9, 10, 0, 1, 1, 2, 7] * 300)
    cu, n, mx, bad = op.seq_metadata(pos, "reset")
    got_cu, got_m = _meta_call("vfk_varlen_meta_noalloc", pos.to(dev), 0, dev)
    assert got_m == [n, mx, bad, pos.numel()]
    assert torch.equal(got_cu, cu.to(torch.int32))
    too_many = (16384 * 1024) + 1
    rc = _lib.load().vfk_varlen_meta_noalloc(pos.to(dev).data_ptr(), 8, too_many, 0, 0, 0, None)
    assert rc == -2
    assert b"above" in _lib.load().vfk_last_error()
