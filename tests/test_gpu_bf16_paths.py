"""GPU parity of the bf16 code paths, against the fp64 CPU oracle on the same
bf16-rounded inputs (tolerance 1e-2 on loss and gradient max-rel).

bf16 inputs with 16-byte aligned rows (D and the row stride multiples of 8) run
on the direct-to-LDS core (128 x 256 forward tiles); other layouts on the
register-staged 128 x 128 core.  The backward always keeps only the transposed
gradient matrix: the y-side contraction reads it K-major, the x-side one (the
only side LiT has) through transposing LDS loads.  Blocks are multiples of 256
rows, so N = 1300 / 2300 / 2500 give two or three blocks with a short last one.
"""
import pytest
import torch

import oracle
from helpers import correlated_pair, max_rel, randn_pair, rel_err
from memoryefficientclip_amd import _lib
from memoryefficientclip_amd.clip_loss import MemoryEfficientCLIPLoss
from memoryefficientclip_amd.lit_loss import MemoryEfficientLiTLoss

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-2


def say(*a):
    print(*a, flush=True)


def grads_of(module, a, b, grad_b=True):
    ga = a.to(DEV).requires_grad_(True)
    gb = b.to(DEV).requires_grad_(grad_b)
    loss = module(ga, gb)
    loss.backward()
    torch.cuda.synchronize()
    return loss.detach().cpu(), ga.grad.cpu(), (gb.grad.cpu() if grad_b else None)


def check(name, loss, ref, pairs):
    msg = f"{name}: loss {float(loss):.6f} ref {float(ref):.6f} rel {rel_err(loss, ref):.2e}"
    errs = [max_rel(g, r) for _, g, r in pairs]
    msg += "".join(f" | {n} {e:.2e}" for (n, _, _), e in zip(pairs, errs))
    say(msg)
    assert rel_err(loss, ref) <= TOL, msg
    assert all(e <= TOL for e in errs), msg


def test_blocking_of_these_shapes():
    # the shapes below really exercise several backward blocks with a short last one
    for n, d in [(1300, 72), (2300, 96), (2500, 72), (2300, 64)]:
        bs, nb = _lib.grad_blocking(n, d, _lib.DTYPE_BF16)
        assert nb >= 2 and nb * bs > n, (n, d, bs, nb)


@pytest.mark.parametrize("n,d,normed", [(2300, 96, False), (2500, 72, True), (1300, 200, False)])
def test_bf16_clip_multiblock(n, d, normed):
    if normed:
        a, b = correlated_pair(n, d, seed=n + d)
    else:
        a, b = randn_pair(n, d, seed=n + d, dtype=torch.bfloat16)
    say(f"bf16 CLIP n={n} d={d} normalized_inputs={normed}")
    loss, da, db = grads_of(MemoryEfficientCLIPLoss(0.07, normed), a, b)
    rl, rda, rdb = oracle.clip_loss_and_grads(a.float(), b.float(), 0.07, normalized_inputs=normed)
    check(f"bf16 clip n={n} d={d}", loss, rl, [("d_img", da, rda), ("d_txt", db, rdb)])


@pytest.mark.parametrize("n,d,normed", [(2300, 64, False), (1300, 72, True), (777, 1152, False)])
def test_bf16_lit(n, d, normed):
    if normed:
        txt, img = correlated_pair(n, d, seed=7 * n + d)
    else:
        txt, img = randn_pair(n, d, seed=7 * n + d, dtype=torch.bfloat16)
    say(f"bf16 LiT n={n} d={d} normalized_inputs={normed} (image frozen)")
    loss, dt, _ = grads_of(MemoryEfficientLiTLoss(0.07, normed), txt, img, grad_b=False)
    rl, rdt = oracle.lit_loss_and_grads(txt.float(), img.float(), 0.07, normalized_inputs=normed)
    check(f"bf16 lit n={n} d={d}", loss, rl, [("d_text", dt, rdt)])


@pytest.mark.parametrize("width,off,label", [(136, 8, "16-byte aligned rows (direct-to-LDS core)"),
                                              (101, 3, "unaligned rows (register-staged core)")])
def test_bf16_row_strided(width, off, label):
    n, d = 1300, 96
    a, b = randn_pair(n, d, seed=99, dtype=torch.bfloat16)
    wa = torch.zeros(n, width, dtype=torch.bfloat16)
    wb = torch.zeros(n, width, dtype=torch.bfloat16)
    wa[:, off:off + d] = a
    wb[:, off:off + d] = b
    ga = wa.to(DEV)[:, off:off + d].requires_grad_(True)
    gb = wb.to(DEV)[:, off:off + d].requires_grad_(True)
    say(f"bf16 row-strided n={n} d={d} ld={width}: {label}")
    loss = MemoryEfficientCLIPLoss(0.07)(ga, gb)
    loss.backward()
    rl, rda, rdb = oracle.clip_loss_and_grads(a.float(), b.float(), 0.07)
    check(f"bf16 strided ld={width}", loss.detach().cpu(), rl,
          [("d_img", ga.grad.cpu(), rda), ("d_txt", gb.grad.cpu(), rdb)])


@pytest.mark.parametrize("mode", [_lib.MODE_CLIP, _lib.MODE_LIT])
def test_bf16_contractions_through_abi(mode):
    """mec_grad on bf16 inputs against the oracle's off-diagonal contractions
    (the gradient matrix is rounded to bf16 before its MFMAs)."""
    n, d, t = 1300, 72, 0.07
    a, b = randn_pair(n, d, seed=5 + mode, dtype=torch.bfloat16)
    x, y = a.to(DEV), b.to(DEV)
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    ws = torch.empty(lib.mec_workspace_floats(n), device=DEV)
    loss = torch.empty((), device=DEV)
    say(f"bf16 ABI contractions mode={mode} n={n} d={d}")
    _lib.call("mec_forward", x.data_ptr(), d, y.data_ptr(), d, n, d, _lib.DTYPE_BF16, mode, 1, t, ws.data_ptr(),
              loss.data_ptr(), st)
    nbytes = lib.mec_grad_scratch_bytes(n, d, _lib.DTYPE_BF16)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    acc_x = torch.empty(n, d, device=DEV)
    acc_y = torch.empty(n, d, device=DEV) if mode == _lib.MODE_CLIP else None
    _lib.call("mec_grad", x.data_ptr(), d, y.data_ptr(), d, n, d, _lib.DTYPE_BF16, mode, 1, t, ws.data_ptr(),
              scratch.data_ptr(), nbytes, acc_x.data_ptr(), None if acc_y is None else acc_y.data_ptr(), st)
    torch.cuda.synchronize()
    xh, yh = oracle.normalize(a.float()), oracle.normalize(b.float())
    s, e, r, c = oracle.similarity_sums(xh, yh, t)
    off = 1.0 - torch.eye(n, dtype=torch.float64)
    gp = e * (1 / r)[:, None] * off
    if mode == _lib.MODE_CLIP:
        gp = gp + e * (1 / c)[None, :] * off
        ey = max_rel(acc_y.cpu(), gp.T @ xh)
        say(f"  acc_y max-rel {ey:.2e}")
        assert ey < TOL
    ex = max_rel(acc_x.cpu(), gp @ yh)
    say(f"  acc_x max-rel {ex:.2e}")
    assert ex < TOL
