"""GPU parity of the K pre-pass of vfk_varlen_attn_fwd (RoPE): the workspace
it leaves behind, read back through the C-ABI.

The attention reads K rotated, multiplied by softmax_scale * log2(e) and laid
out head-major [H][T][64], and four partial key-norm maxima per (head,
sequence, 64-key tile), one per 16 rows, that bound its scores. The rotated
rows are checked against the oracle's rotary step (apply_rope, the HF
formula) within one rounding to 16 bits; the maxima against the norms of the
stored rows themselves, and the slots of a live tile that lie past the
sequence end must be exactly 0 (the workspace is filled with NaN bytes
first, so a slot the pass forgot shows up). Head counts 12 (six head pairs
per block), 16 (four) and 3 (clamped head loads) and sequence lengths that
end inside every 16-row group of a tile are covered."""
import math

import pytest
import torch

import workloads
from oracle import attention as oa

pytestmark = pytest.mark.gpu

SCALE = 0.125


def _close16(got, want, what):
    # one rounding to 16 bits (2^-8 relative covers bf16) plus fp32 sum order
    err = (got - want).abs()
    lim = want.abs() * 2.0 ** -8 + 2e-3
    assert bool((err <= lim).all()), f"{what}: worst excess {(err - lim).max().item():.3e}"


@pytest.mark.parametrize("H", [12, 16, 3])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prepass_workspace(dev, H, dtype):
    from kernels import _lib
    from kernels.varlen_attention import rope_table
    lengths = [1, 5, 16, 17, 31, 33, 48, 63, 64, 65, 100, 127, 128, 129, 200, 300]
    T = sum(lengths)
    nseq = len(lengths)
    maxlen = max(lengths)
    theta = 160000.0
    g = torch.Generator().manual_seed(100 + H)
    qkv = torch.randn(T, 3, H, 64, generator=g).to(dtype).to(dev)
    q, k, v = qkv[:, 0], qkv[:, 1], qkv[:, 2]
    cu = workloads.cu_from_lengths(torch.tensor(lengths)).to(dev)
    lib = _lib.load()
    ws_bytes = int(lib.vfk_varlen_attn_workspace_bytes(_lib.dtype_code(dtype), T, H, 1, nseq, maxlen))
    ws = torch.full((ws_bytes,), 0xFF, dtype=torch.uint8, device=dev)  # NaN in every float slot
    tab = rope_table(theta, maxlen, dev)
    out = torch.empty(T, H, 64, dtype=dtype, device=dev)
    print(f"prepass workspace H={H} {dtype} T={T}", flush=True)
    _lib.on_device("vfk_varlen_attn_fwd", dev, _lib.ref(_lib.desc(q)), _lib.ref(_lib.desc(k)),
                   _lib.ref(_lib.desc(v)), cu.data_ptr(), nseq, maxlen, -1, tab.data_ptr(),
                   int(tab.shape[0]), None, float(SCALE), ws.data_ptr(), ws_bytes,
                   _lib.ref(_lib.desc(out)))
    torch.cuda.synchronize()
    w = ws.cpu()
    kb = T * H * 64 * 2
    kr_bytes = (kb + 255) // 256 * 256
    kr = w[:kb].view(dtype).view(H, T, 64).permute(1, 0, 2).float()  # [T, H, 64]
    nkt = (maxlen + 63) // 64
    kmax = w[kr_bytes:kr_bytes + H * nseq * nkt * 16].view(torch.float32).view(H, nseq, nkt, 4)

    pos = torch.cat([torch.arange(n) for n in lengths])
    cos, sin = oa.rope_cos_sin(pos, theta)
    want = oa.apply_rope(k.float().cpu(), cos, sin) * (SCALE * math.log2(math.e))
    _close16(kr, want, f"rotated k H={H} {dtype}")

    norms = kr.double().norm(dim=-1)  # [T, H], of the stored rows
    starts = [0] + torch.tensor(lengths).cumsum(0).tolist()
    for s, n in enumerate(lengths):
        for kt in range((n + 63) // 64):          # live tiles only
            for g4 in range(4):
                r0 = kt * 64 + 16 * g4
                got = kmax[:, s, kt, g4].double()
                if r0 >= n:
                    assert bool((got == 0).all()), f"slot past the end: seq {s} tile {kt} group {g4}"
                else:
                    rows = norms[starts[s] + r0:starts[s] + min(r0 + 16, n)]  # [rows, H]
                    assert torch.allclose(got, rows.amax(dim=0), rtol=1e-5, atol=1e-6), \
                        f"key-norm max: seq {s} tile {kt} group {g4}"
