"""Shared numerics helpers for the parity tests."""
import torch


def bf(x):
    """Round to bf16 values (kept as fp32): the inputs both sides see."""
    return x.to(torch.bfloat16).float()


def metrics(got, ref):
    """(cosine, relative L2, max abs err) of got vs ref, in float64."""
    g = got.double().reshape(-1).cpu()
    r = ref.double().reshape(-1).cpu()
    cos = float(torch.nn.functional.cosine_similarity(g, r, dim=0))
    rel = float((g - r).norm() / r.norm().clamp_min(1e-30))
    return cos, rel, float((g - r).abs().max())


def assert_close(got, ref, cos_min=0.999, rel_max=1e-2, label=""):
    cos, rel, mx = metrics(got, ref)
    assert torch.isfinite(got.float()).all(), f"{label}: non-finite output"
    assert cos >= cos_min and rel <= rel_max, f"{label}: cos={cos:.6f} relL2={rel:.3e} maxabs={mx:.3e}"
    return cos, rel


def gen(seed):
    return torch.Generator().manual_seed(seed)


def randn(shape, seed, scale=1.0):
    return torch.randn(shape, generator=gen(seed)) * scale
