"""Comparison helpers shared by the GPU parity tests."""

import torch


def bf16_ulp_diff(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in bf16 units-in-the-last-place between two bf16 tensors (same sign side)."""
    ai = a.detach().cpu().contiguous().view(torch.int16).to(torch.int32)
    bi = b.detach().cpu().contiguous().view(torch.int16).to(torch.int32)
    # Map sign-magnitude bit patterns onto a monotone integer line.
    ai = torch.where(ai < 0, -(ai & 0x7FFF), ai)
    bi = torch.where(bi < 0, -(bi & 0x7FFF), bi)
    return (ai - bi).abs()


def assert_bf16_close_ulp(got, want, max_ulp=1, max_frac=1e-3, name=""):
    """All elements within ``max_ulp`` bf16 ulps and at most ``max_frac`` of them differing."""
    d = bf16_ulp_diff(got, want)
    frac = float((d > 0).float().mean())
    assert int(d.max()) <= max_ulp, f"{name}: max ulp diff {int(d.max())} > {max_ulp}"
    assert frac <= max_frac, f"{name}: {frac:.2e} of elements differ (> {max_frac})"


def assert_close(got, want, atol, rtol, name=""):
    g, w = got.detach().float().cpu(), want.detach().float().cpu()
    diff = (g - w).abs()
    ok = diff <= atol + rtol * w.abs()
    assert bool(ok.all()), f"{name}: max abs diff {float(diff.max()):.4g} (atol {atol}, rtol {rtol})"
