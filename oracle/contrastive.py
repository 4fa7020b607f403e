"""fp64 CPU restatement of the reference's CLIP / LiT loss (test infrastructure).

Follows the reference's algorithm step by step, densely (no tiling):

* fixed-max exponentials E_ij = exp((S_ij - 1)/T)          clip_loss.py:56, :115
* row / column sums R_i = sum_j E_ij, C_j = sum_i E_ij       clip_loss.py:59-64
* loss = -mean_i [ln(e^{(S_ii-1)/T}/R_i) + ln(e^{(S_ii-1)/T}/C_i)] / 2
                                                             clip_loss.py:206-211
  (LiT: -mean_i ln(e^{(S_ii-1)/T}/R_i)                       lit_loss.py:199-203)
* G = (E/R_i + E/C_j) * s/(2N) - I * s/N, s = 1/T (Stable: sqrt(N/T))
                                                             clip_loss.py:121-124, :235-236, :299
  (LiT: G = E/R_i * s/N - I * s/N                            lit_loss.py:118-120, :227)
* dX^ = G Y^, dY^ = G^T X^, times grad_output                clip_loss.py:148-149, :252-254
* x^ = x / max(||x||, 1e-12) (F.normalize, dim=1)            clip_loss.py:266-268

Unlike the reference's masked Triton tiles (clip_loss.py:41-50, which add
e^{-1/T} for every padded tile slot to valid rows' sums when N % 128 != 0),
sums here run over exactly the N valid entries, which is the loss definition.
Test infrastructure only; see ``oracle/__init__.py``.
"""
from __future__ import annotations

import math

import torch

EPS = 1e-12
F64 = torch.float64


def _f64(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to(device="cpu", dtype=F64)


def normalize(x: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """x / max(||x||_2, eps) row-wise (F.normalize(dim=1), clip_loss.py:267)."""
    x = _f64(x)
    return x / x.norm(dim=1, keepdim=True).clamp_min(eps)


def normalize_backward(x: torch.Tensor, dxh: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """Backward of ``normalize``: (dxh - xh<xh, dxh>)/||x|| where ||x|| > eps,
    dxh/eps where the norm is clamped."""
    x, dxh = _f64(x), _f64(dxh)
    nrm = x.norm(dim=1, keepdim=True)
    xh = x / nrm.clamp_min(eps)
    proj = dxh - xh * (xh * dxh).sum(dim=1, keepdim=True)
    return torch.where(nrm > eps, proj / nrm.clamp_min(eps), dxh / eps)


def similarity_sums(xh: torch.Tensor, yh: torch.Tensor, temperature: float):
    """S = xh yh^T, E = exp((S-1)/T), R = row sums, C = column sums."""
    xh, yh = _f64(xh), _f64(yh)
    s = xh @ yh.T
    e = torch.exp((s - 1.0) / temperature)
    return s, e, e.sum(dim=1), e.sum(dim=0)


def clip_forward(xh: torch.Tensor, yh: torch.Tensor, temperature: float) -> torch.Tensor:
    """CLIP loss on normalised features (fp64 0-d tensor)."""
    s, e, r, c = similarity_sums(xh, yh, temperature)
    sv = (torch.diagonal(s) - 1.0) / temperature
    logits = (sv - torch.log(r)) + (sv - torch.log(c))
    return -logits.mean() / 2.0


def lit_forward(xh: torch.Tensor, yh: torch.Tensor, temperature: float) -> torch.Tensor:
    """LiT loss on normalised features, xh = text rows (fp64 0-d tensor)."""
    s, e, r, _ = similarity_sums(xh, yh, temperature)
    sv = (torch.diagonal(s) - 1.0) / temperature
    return -(sv - torch.log(r)).mean()


def _grad_scale(n: int, temperature: float, stable: bool) -> float:
    return math.sqrt(n / temperature) if stable else 1.0 / temperature


def clip_backward(xh, yh, temperature, stable=False, grad_output=1.0):
    """(dX^, dY^) of the CLIP loss w.r.t. the normalised features."""
    xh, yh = _f64(xh), _f64(yh)
    n = xh.shape[0]
    _, e, r, c = similarity_sums(xh, yh, temperature)
    gs = _grad_scale(n, temperature, stable)
    g = (e / r[:, None] + e / c[None, :]) * (gs / (2 * n)) - torch.eye(n, dtype=F64) * (gs / n)
    return (g @ yh) * grad_output, (g.T @ xh) * grad_output


def lit_backward(xh, yh, temperature, stable=False, grad_output=1.0):
    """dX^ (text) of the LiT loss; the image side gets no gradient."""
    xh, yh = _f64(xh), _f64(yh)
    n = xh.shape[0]
    _, e, r, _ = similarity_sums(xh, yh, temperature)
    gs = _grad_scale(n, temperature, stable)
    g = e / r[:, None] * (gs / n) - torch.eye(n, dtype=F64) * (gs / n)
    return (g @ yh) * grad_output


def clip_loss_and_grads(image, text, temperature=0.07, normalized_inputs=False, stable=False, grad_output=1.0):
    """Full CLIP module (clip_loss.py:259-273): loss, d image, d text in fp64."""
    img, txt = _f64(image), _f64(text)
    xh = img if normalized_inputs else normalize(img)
    yh = txt if normalized_inputs else normalize(txt)
    loss = clip_forward(xh, yh, temperature)
    dxh, dyh = clip_backward(xh, yh, temperature, stable, grad_output)
    if normalized_inputs:
        return loss, dxh, dyh
    return loss, normalize_backward(img, dxh), normalize_backward(txt, dyh)


def lit_loss_and_grads(text, image, temperature=0.07, normalized_inputs=False, stable=False, grad_output=1.0):
    """Full LiT module (lit_loss.py:250-263): loss, d text in fp64."""
    txt, img = _f64(text), _f64(image)
    xh = txt if normalized_inputs else normalize(txt)
    yh = img if normalized_inputs else normalize(img)
    loss = lit_forward(xh, yh, temperature)
    dxh = lit_backward(xh, yh, temperature, stable, grad_output)
    return loss, (dxh if normalized_inputs else normalize_backward(txt, dxh))


# ------------------------------------------------------------ chunked helpers
# For N too large for dense N x N fp64: exact values on a subset of rows or
# columns, from the full other side.

def row_sums(xh, yh, temperature, rows, exclude_diag=False, chunk=4096):
    """R_i (optionally without the i == j term) for i in ``rows``."""
    xh, yh = _f64(xh), _f64(yh)
    rows = torch.as_tensor(rows, dtype=torch.long)
    xr = xh[rows]
    out = torch.zeros(len(rows), dtype=F64)
    for j0 in range(0, yh.shape[0], chunk):
        e = torch.exp((xr @ yh[j0:j0 + chunk].T - 1.0) / temperature)
        if exclude_diag:
            cols = torch.arange(j0, min(j0 + chunk, yh.shape[0]))
            e = e * (rows[:, None] != cols[None, :])
        out += e.sum(dim=1)
    return out


def col_sums(xh, yh, temperature, cols, exclude_diag=False, chunk=4096):
    """C_j (optionally without the i == j term) for j in ``cols``."""
    return row_sums(yh, xh, temperature, cols, exclude_diag, chunk)


def grad_rows(xh, yh, temperature, rows, r_full, c_full=None, stable=False, grad_output=1.0, chunk=4096):
    """Rows ``rows`` of dX^ given the full sum vectors R (and C for CLIP;
    LiT when c_full is None)."""
    xh, yh = _f64(xh), _f64(yh)
    n = xh.shape[0]
    rows = torch.as_tensor(rows, dtype=torch.long)
    r_full = _f64(r_full)
    gs = _grad_scale(n, temperature, stable)
    xr = xh[rows]
    out = torch.zeros(len(rows), xh.shape[1], dtype=F64)
    for j0 in range(0, n, chunk):
        yj = yh[j0:j0 + chunk]
        e = torch.exp((xr @ yj.T - 1.0) / temperature)
        if c_full is None:
            g = e / r_full[rows][:, None] * (gs / n)
        else:
            g = (e / r_full[rows][:, None] + e / _f64(c_full)[j0:j0 + chunk][None, :]) * (gs / (2 * n))
        out += g @ yj
    diag = (gs / n) * yh[rows]
    return (out - diag) * grad_output
