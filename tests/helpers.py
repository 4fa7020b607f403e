"""Shared helpers for the test suite (input generators, error metrics)."""
import contextlib

import numpy as np
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
    torch.float16: dict(loss=1e-2, grad=1e-2),
}


def ref_fp64(a, b, t, lit, normalized, chunk):
    """Loss and input gradients of the dense definition, fp64 on the GPU.

    a: rows of S (image for CLIP, text for LiT); b: columns."""
    x = a.double()
    y = b.double()
    xh = x if normalized else F.normalize(x, dim=1)
    yh = y if normalized else F.normalize(y, dim=1)
    n = x.shape[0]
    r = torch.zeros(n, dtype=torch.float64, device=x.device)
    c = torch.zeros(n, dtype=torch.float64, device=x.device)
    for i0 in range(0, n, chunk):
        e = torch.exp((xh[i0:i0 + chunk] @ yh.T - 1.0) / t)
        r[i0:i0 + chunk] = e.sum(dim=1)
        if not lit:
            c += e.sum(dim=0)
        del e
    tdiag = ((xh * yh).sum(dim=1) - 1.0) / t
    loss = (torch.log(r) - tdiag).mean()
    if not lit:
        loss = 0.5 * (loss + (torch.log(c) - tdiag).mean())
    # G = (E/R_i + E/C_j)/(2 N t) - I/(N t)   (LiT: E/R_i/(N t) - I/(N t))
    dxh = torch.zeros_like(xh)
    dyh = None if lit else torch.zeros_like(yh)
    s = 1.0 / (n * t) if lit else 1.0 / (2 * n * t)
    for i0 in range(0, n, chunk):
        e = torch.exp((xh[i0:i0 + chunk] @ yh.T - 1.0) / t)
        g = e / r[i0:i0 + chunk, None]
        if not lit:
            g += e / c[None, :]
        del e
        g *= s
        dxh[i0:i0 + chunk] = g @ yh
        if not lit:
            dyh += g.T @ xh[i0:i0 + chunk]
        del g
    dxh -= yh / (n * t)
    if not lit:
        dyh -= xh / (n * t)

    def norm_bwd(v, dvh):
        if normalized:
            return dvh
        nrm = v.norm(dim=1, keepdim=True).clamp_min(1e-12)
        vh = v / nrm
        return (dvh - vh * (vh * dvh).sum(dim=1, keepdim=True)) / nrm

    return loss, norm_bwd(x, dxh), (None if lit else norm_bwd(y, dyh))


@contextlib.contextmanager
def matmul_precision(p):
    """torch.set_float32_matmul_precision(p) within the block."""
    old = torch.get_float32_matmul_precision()
    torch.set_float32_matmul_precision(p)
    try:
        yield
    finally:
        torch.set_float32_matmul_precision(old)


def bf16_rne(v: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (finite inputs)."""
    u = v.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def split_rows(x: np.ndarray, order: int) -> np.ndarray:
    """bf16 copies of fp32 rows as the bf16-product modes lay them out, each
    segment d rounded up to 8 wide with zero padding: [hi | lo | hi] (order
    0, x side of bf16x3), [hi | hi | lo] (order 1, y side) or [hi] (order 2,
    plain bf16 products)."""
    n, d = x.shape
    dp = (d + 7) // 8 * 8
    hi = np.zeros((n, dp), np.uint16)
    lo = np.zeros((n, dp), np.uint16)
    hi[:, :d] = bf16_rne(x)
    lo[:, :d] = bf16_rne(x - bf16_to_f32(hi[:, :d]))
    return np.concatenate({0: [hi, lo, hi], 1: [hi, hi, lo], 2: [hi]}[order], axis=1)
