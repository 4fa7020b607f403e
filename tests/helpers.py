"""Shared helpers for the test suite (input generators, error metrics)."""
import torch
import torch.nn.functional as F


def randn_pair(n, d, seed=0, dtype=torch.float32):
    """Config 1-3 generator: i.i.d. randn(0,1) image and text features."""
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(n, d, generator=g)
    b = torch.randn(n, d, generator=g)
    return a.to(dtype), b.to(dtype)


def correlated_pair(n, d, seed=0, dtype=torch.bfloat16):
    """Config 4-5 generator: image = normalize(randn), text = normalize(image +
    0.5 randn), fp32 math, then cast (diagonal-dominant similarity)."""
    g = torch.Generator().manual_seed(seed)
    img = F.normalize(torch.randn(n, d, generator=g), dim=1)
    txt = F.normalize(img + 0.5 * torch.randn(n, d, generator=g), dim=1)
    return img.to(dtype), txt.to(dtype)


def rel_err(a, ref):
    a, ref = float(a), float(ref)
    if ref == 0.0:
        return abs(a)
    return abs(a - ref) / abs(ref)


def max_rel(g, ref):
    """max|g - ref| / max|ref| (the north-star gradient metric)."""
    g = g.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = ref.abs().max().item()
    num = (g - ref).abs().max().item()
    return num if den == 0.0 else num / den


TOL = {
    torch.float32: dict(loss=1e-4, grad=1e-3),
    torch.bfloat16: dict(loss=1e-2, grad=1e-2),
}
