"""Parity criteria shared by the GPU tests.

Attention outputs: max-abs <= 2e-2 and cosine >= 0.9999 against the fp32
oracle, on valid rows only (the tolerance stated for this path). Memory-bound
epilogues with 16-bit outputs: the same cosine and a max-abs bound scaled by
the output magnitude (one 16-bit rounding of a value of size |y| is
|y| * 2^-8 at most for bf16).
"""
import torch

ATTN_MAX_ABS = 2e-2
ATTN_COS = 0.9999


def cosine(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.double().flatten()
    b = b.double().flatten()
    den = a.norm() * b.norm()
    if den == 0:
        return 1.0 if a.norm() == b.norm() else 0.0
    return float((a @ b) / den)


def assert_attn_close(got: torch.Tensor, want: torch.Tensor, what: str = "",
                      max_abs: float = ATTN_MAX_ABS, cos: float = ATTN_COS):
    got = got.detach().float().cpu()
    want = want.detach().float().cpu()
    assert got.shape == want.shape, (got.shape, want.shape)
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    err = (got - want).abs().max().item()
    c = cosine(got, want)
    assert err <= max_abs and c >= cos, f"{what}: max-abs {err:.3e} (<= {max_abs}), cos {c:.6f} (>= {cos})"
    return err, c


def assert_elem_close(got: torch.Tensor, want: torch.Tensor, dtype: torch.dtype, what: str = ""):
    got = got.detach().float().cpu()
    want = want.detach().float().cpu()
    assert got.shape == want.shape, (got.shape, want.shape)
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    if dtype == torch.float32:
        atol, rtol = 1e-5, 1e-5
    elif dtype == torch.bfloat16:
        atol, rtol = 1e-2, 2 ** -7
    else:
        atol, rtol = 2e-3, 2 ** -9
    torch.testing.assert_close(got, want, atol=atol, rtol=rtol, msg=lambda m: f"{what}: {m}")
    assert cosine(got, want) >= 0.9999, what
