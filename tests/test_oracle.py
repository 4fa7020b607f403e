"""Pins the CPU oracle (oracle/contrastive.py) independently of its own
formulas: library cross-entropy + autograd, finite differences, pure-Python
brute force, closed forms and invariants.  CPU only."""
import math
import random

import pytest
import torch
import torch.nn.functional as F

import oracle

F64 = torch.float64


def _inputs(n, d, seed=0, dtype=F64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, d, generator=g, dtype=dtype), torch.randn(n, d, generator=g, dtype=dtype)


# ---------------------------------------------------------------- library route
def lib_clip(img, txt, t, normalized=False):
    """0.5*(CE(S/T) + CE(S^T/T)) with F.normalize and F.cross_entropy."""
    xh = img if normalized else F.normalize(img, dim=1)
    yh = txt if normalized else F.normalize(txt, dim=1)
    s = xh @ yh.T / t
    lab = torch.arange(img.shape[0])
    return 0.5 * (F.cross_entropy(s, lab) + F.cross_entropy(s.T, lab))


def lib_lit(txt, img, t, normalized=False):
    xh = txt if normalized else F.normalize(txt, dim=1)
    yh = img if normalized else F.normalize(img, dim=1)
    s = xh @ yh.T / t
    return F.cross_entropy(s, torch.arange(txt.shape[0]))


@pytest.mark.parametrize("n,d,t", [(1, 4, 0.07), (7, 5, 0.07), (64, 16, 0.07), (130, 33, 0.05), (40, 8, 0.5)])
@pytest.mark.parametrize("normalized", [False, True])
def test_clip_matches_library_route(n, d, t, normalized):
    img, txt = _inputs(n, d, seed=n * 31 + d)
    if normalized:
        img, txt = F.normalize(img, dim=1), F.normalize(txt, dim=1)
    a = img.clone().requires_grad_(True)
    b = txt.clone().requires_grad_(True)
    ref = lib_clip(a, b, t, normalized)
    ref.backward()
    loss, di, dt = oracle.clip_loss_and_grads(img, txt, t, normalized_inputs=normalized)
    assert torch.allclose(loss, ref.detach(), rtol=1e-12, atol=1e-12)
    assert torch.allclose(di, a.grad, rtol=1e-10, atol=1e-13)
    assert torch.allclose(dt, b.grad, rtol=1e-10, atol=1e-13)


@pytest.mark.parametrize("n,d,t", [(1, 4, 0.07), (9, 6, 0.07), (100, 32, 0.05)])
@pytest.mark.parametrize("normalized", [False, True])
def test_lit_matches_library_route(n, d, t, normalized):
    txt, img = _inputs(n, d, seed=7 * n + d)
    if normalized:
        img, txt = F.normalize(img, dim=1), F.normalize(txt, dim=1)
    a = txt.clone().requires_grad_(True)
    b = img.clone().requires_grad_(True)
    ref = lib_lit(a, b, t, normalized)
    ref.backward()
    loss, dx = oracle.lit_loss_and_grads(txt, img, t, normalized_inputs=normalized)
    assert torch.allclose(loss, ref.detach(), rtol=1e-12, atol=1e-12)
    assert torch.allclose(dx, a.grad, rtol=1e-10, atol=1e-13)


# ---------------------------------------------------------------- finite differences
class _ClipFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, y, t):
        ctx.save_for_backward(x, y)
        ctx.t = t
        return oracle.clip_forward(x, y, t)

    @staticmethod
    def backward(ctx, g):
        x, y = ctx.saved_tensors
        dx, dy = oracle.clip_backward(x, y, ctx.t, grad_output=g)
        return dx, dy, None


class _LitFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, y, t):
        ctx.save_for_backward(x, y)
        ctx.t = t
        return oracle.lit_forward(x, y, t)

    @staticmethod
    def backward(ctx, g):
        x, y = ctx.saved_tensors
        return oracle.lit_backward(x, y, ctx.t, grad_output=g), None, None


def test_clip_backward_gradcheck():
    x, y = _inputs(6, 5, seed=3)
    x = F.normalize(x, dim=1).requires_grad_(True)
    y = F.normalize(y, dim=1).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b: _ClipFn.apply(a, b, 0.3), (x, y), eps=1e-6, atol=1e-7)


def test_lit_backward_gradcheck():
    x, y = _inputs(5, 4, seed=4)
    x = F.normalize(x, dim=1).requires_grad_(True)
    y = F.normalize(y, dim=1)
    assert torch.autograd.gradcheck(lambda a: _LitFn.apply(a, y, 0.25), (x,), eps=1e-6, atol=1e-7)


def test_normalize_backward_matches_autograd_incl_clamped_rows():
    x, _ = _inputs(6, 7, seed=5)
    x[2] = 0.0                       # ||x|| = 0 < eps: clamped
    x[4] *= 1e-14                    # tiny but non-zero: clamped
    dxh = torch.randn(6, 7, dtype=F64, generator=torch.Generator().manual_seed(9))
    a = x.clone().requires_grad_(True)
    F.normalize(a, dim=1).backward(dxh)
    assert torch.allclose(oracle.normalize(x), F.normalize(x, dim=1), rtol=0, atol=0)
    assert torch.allclose(oracle.normalize_backward(x, dxh), a.grad, rtol=1e-12, atol=0)


# ---------------------------------------------------------------- brute force (pure Python)
def _py_clip_loss(X, Y, t):
    n = len(X)
    nx = [math.sqrt(sum(v * v for v in r)) for r in X]
    ny = [math.sqrt(sum(v * v for v in r)) for r in Y]
    xh = [[v / max(nx[i], 1e-12) for v in X[i]] for i in range(n)]
    yh = [[v / max(ny[i], 1e-12) for v in Y[i]] for i in range(n)]
    s = [[sum(a * b for a, b in zip(xh[i], yh[j])) / t for j in range(n)] for i in range(n)]
    row = sum(-(s[i][i] - math.log(sum(math.exp(s[i][j]) for j in range(n)))) for i in range(n)) / n
    col = sum(-(s[j][j] - math.log(sum(math.exp(s[i][j]) for i in range(n)))) for j in range(n)) / n
    return 0.5 * (row + col), row


def test_brute_force_loss_and_central_differences():
    rnd = random.Random(11)
    n, d, t = 4, 3, 0.2
    X = [[rnd.gauss(0, 1) for _ in range(d)] for _ in range(n)]
    Y = [[rnd.gauss(0, 1) for _ in range(d)] for _ in range(n)]
    clip, lit = _py_clip_loss(X, Y, t)
    loss, dx, dy = oracle.clip_loss_and_grads(torch.tensor(X, dtype=F64), torch.tensor(Y, dtype=F64), t)
    lloss, ldx = oracle.lit_loss_and_grads(torch.tensor(X, dtype=F64), torch.tensor(Y, dtype=F64), t)
    assert abs(loss.item() - clip) < 1e-12
    assert abs(lloss.item() - lit) < 1e-12
    h = 1e-6
    for i in range(n):
        for k in range(d):
            Xp = [r[:] for r in X]
            Xm = [r[:] for r in X]
            Xp[i][k] += h
            Xm[i][k] -= h
            (cp, lp), (cm, lm) = _py_clip_loss(Xp, Y, t), _py_clip_loss(Xm, Y, t)
            assert abs((cp - cm) / (2 * h) - dx[i, k].item()) < 1e-7
            assert abs((lp - lm) / (2 * h) - ldx[i, k].item()) < 1e-7
            Yp = [r[:] for r in Y]
            Ym = [r[:] for r in Y]
            Yp[i][k] += h
            Ym[i][k] -= h
            dyk = (_py_clip_loss(X, Yp, t)[0] - _py_clip_loss(X, Ym, t)[0]) / (2 * h)
            assert abs(dyk - dy[i, k].item()) < 1e-7


# ---------------------------------------------------------------- closed forms
def test_known_answers():
    t = 0.07
    x, y = _inputs(1, 8, seed=1)
    loss, dx, dy = oracle.clip_loss_and_grads(x, y, t)
    assert loss.item() == 0.0 and dx.abs().max() == 0 and dy.abs().max() == 0
    # identical unit rows -> every logit equal -> ln N, zero gradient
    n = 9
    v = F.normalize(torch.randn(1, 5, dtype=F64), dim=1).repeat(n, 1)
    loss, dx, dy = oracle.clip_loss_and_grads(v, v, t, normalized_inputs=True)
    assert abs(loss.item() - math.log(n)) < 1e-12
    lloss, ldx = oracle.lit_loss_and_grads(v, v, t, normalized_inputs=True)
    assert abs(lloss.item() - math.log(n)) < 1e-12
    # orthonormal one-hot rows: S = I -> ln(1 + (N-1) e^{-1/T})
    n = 6
    eye = torch.eye(n, 8, dtype=F64)
    loss, _, _ = oracle.clip_loss_and_grads(eye, eye, t, normalized_inputs=True)
    assert abs(loss.item() - math.log1p((n - 1) * math.exp(-1 / t))) < 1e-14


# ---------------------------------------------------------------- invariants
def test_invariants():
    t, n = 0.07, 20
    x, y = _inputs(n, 12, seed=2)
    loss, dx, dy = oracle.clip_loss_and_grads(x, y, t)
    loss2, dx2, dy2 = oracle.clip_loss_and_grads(y, x, t)
    assert torch.allclose(loss, loss2, rtol=1e-13) and torch.allclose(dx, dy2) and torch.allclose(dy, dx2)
    # scale invariance of the normalised loss: gradient orthogonal to each row
    assert (dx * x).sum(dim=1).abs().max() < 1e-14
    # Stable: same loss, gradients times sqrt(N T)
    sl, sdx, sdy = oracle.clip_loss_and_grads(x, y, t, stable=True)
    assert torch.allclose(sl, loss) and torch.allclose(sdx, dx * math.sqrt(n * t), rtol=1e-12)
    # grad_output linearity
    _, gdx, _ = oracle.clip_loss_and_grads(x, y, t, grad_output=-2.5)
    assert torch.allclose(gdx, -2.5 * dx, rtol=1e-13)
    # CLIP = mean of the two LiT directions
    l1, _ = oracle.lit_loss_and_grads(x, y, t)
    l2, _ = oracle.lit_loss_and_grads(y, x, t)
    assert abs(loss.item() - 0.5 * (l1.item() + l2.item())) < 1e-13
    # a wrong-sign or dropped diagonal term breaks the zero-sum of the gradient matrix rows:
    # sum_i dX^_i . ... instead check the row-stochastic identity sum_j G_ij = 0 for LiT
    xh, yh = oracle.normalize(x), oracle.normalize(y)
    _, e, r, _ = oracle.similarity_sums(xh, yh, t)
    g = e / r[:, None] / (n * t) - torch.eye(n, dtype=F64) / (n * t)
    assert torch.allclose(oracle.lit_backward(xh, yh, t), g @ yh)
    assert g.sum(dim=1).abs().max() < 1e-15


def test_chunked_helpers_match_dense():
    t, n = 0.05, 300
    x, y = _inputs(n, 16, seed=8)
    xh, yh = oracle.normalize(x), oracle.normalize(y)
    _, e, r, c = oracle.similarity_sums(xh, yh, t)
    rows = [0, 5, 128, 299]
    assert torch.allclose(oracle.row_sums(xh, yh, t, rows, chunk=97), r[rows])
    assert torch.allclose(oracle.col_sums(xh, yh, t, rows, chunk=64), c[rows])
    off = oracle.row_sums(xh, yh, t, rows, exclude_diag=True, chunk=50)
    assert torch.allclose(off, r[rows] - torch.diagonal(e)[rows])
    dxh, _ = oracle.clip_backward(xh, yh, t)
    assert torch.allclose(oracle.grad_rows(xh, yh, t, rows, r, c, chunk=77), dxh[rows], rtol=1e-12, atol=1e-16)
    ldx = oracle.lit_backward(xh, yh, t, stable=True)
    assert torch.allclose(oracle.grad_rows(xh, yh, t, rows, r, None, stable=True, chunk=33), ldx[rows],
                          rtol=1e-12, atol=1e-16)


def test_reference_padding_quirk_is_not_followed():
    """The reference's masked tiles add e^{-1/T} per padded slot to R_i when
    N % 128 != 0 (clip_loss.py:41-64).  The oracle sums exactly N terms."""
    t, n = 0.07, 10
    x, y = _inputs(n, 4, seed=12)
    xh, yh = oracle.normalize(x), oracle.normalize(y)
    _, e, r, _ = oracle.similarity_sums(xh, yh, t)
    assert torch.allclose(r, e.sum(dim=1))
    padded = r + (128 - n) * math.exp(-1 / t)
    assert (padded - r).min() > 0


@pytest.mark.parametrize("path", ["clip", "lit"])
def test_golden_fixtures(path):
    import glob
    import os
    import numpy as np
    here = os.path.join(os.path.dirname(__file__), "golden")
    files = sorted(glob.glob(os.path.join(here, f"{path}_*.npz")))
    assert files, "golden fixtures missing; run tests/golden/make_golden.py"
    for f in files:
        z = np.load(f)
        t = float(z["temperature"])
        normed = bool(z["normalized_inputs"])
        stable = bool(z["stable"])
        a, b = torch.from_numpy(z["a"]), torch.from_numpy(z["b"])
        if path == "clip":
            loss, da, db = oracle.clip_loss_and_grads(a, b, t, normed, stable)
            assert torch.allclose(db, torch.from_numpy(z["db"]), rtol=1e-9, atol=1e-15), f
        else:
            loss, da = oracle.lit_loss_and_grads(a, b, t, normed, stable)
        assert abs(loss.item() - float(z["loss"])) <= 1e-11 * max(1.0, abs(float(z["loss"]))), f
        assert torch.allclose(da, torch.from_numpy(z["da"]), rtol=1e-9, atol=1e-15), f


def test_cpu_baseline_matches_oracle():
    """The dense fp32 CPU baseline timed by bench.py computes the same loss."""
    from oracle.cpu_baseline import dense_step
    a, b = _inputs(96, 40, seed=77, dtype=torch.float32)
    loss, da, db = dense_step(a, b, 0.07, lit=False, normalized_inputs=False)
    rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.07)
    assert abs(loss.item() - rl.item()) < 1e-5 * rl.item()
    assert torch.allclose(da.double(), rda, rtol=1e-3, atol=1e-6 * rda.abs().max().item())
    assert torch.allclose(db.double(), rdb, rtol=1e-3, atol=1e-6 * rdb.abs().max().item())
    loss, dt, none = dense_step(a, b, 0.05, lit=True, normalized_inputs=False)
    rl, rdt = oracle.lit_loss_and_grads(a, b, 0.05)
    assert none is None and abs(loss.item() - rl.item()) < 1e-5 * rl.item()
    assert torch.allclose(dt.double(), rdt, rtol=1e-3, atol=1e-6 * rdt.abs().max().item())


@pytest.mark.parametrize("lit", [False, True])
@pytest.mark.parametrize("normalized", [False, True])
def test_fullsize_reference_matches_oracle(lit, normalized):
    """The chunked fp64 reference used at full size on the GPU (tests/helpers.py
    ref_fp64) agrees with the oracle, chunk boundaries included."""
    from helpers import ref_fp64
    x, y = _inputs(150, 24, seed=31 + lit + 2 * normalized)
    if normalized:
        x, y = F.normalize(x, dim=1), F.normalize(y, dim=1)
    loss, dx, dy = ref_fp64(x, y, 0.05, lit, normalized, chunk=64)
    if lit:
        rl, rdx = oracle.lit_loss_and_grads(x, y, 0.05, normalized_inputs=normalized)
        assert dy is None
    else:
        rl, rdx, rdy = oracle.clip_loss_and_grads(x, y, 0.05, normalized_inputs=normalized)
        assert torch.allclose(dy, rdy, rtol=1e-10, atol=1e-14)
    assert abs(loss.item() - rl.item()) < 1e-12 * abs(rl.item())
    assert torch.allclose(dx, rdx, rtol=1e-10, atol=1e-14)
