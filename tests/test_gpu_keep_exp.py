"""GPU parity of the kept-exponential path (MEC_FLAG_KEEP_EXP: small fp32
problems keep E = exp((S-1)/T) from the forward for the backward).

The modules take this path by themselves for fp32 inputs with 16-byte rows and
n <= 2048; MEC_KEEP_EXP=0 turns it off, which the comparisons with the
recomputing path use.  Checked here: the loss and both gradients against the
fp64 CPU oracle (fp32 tolerances: loss rel 1e-4, gradient max-rel 1e-3) on
ragged n and d, CLIP and LiT, fused normalisation on and off, the Stable
variants, grad_output scaling and a frozen tower; agreement with the
recomputing path; bitwise reproducibility without the deterministic flag, and
the same bits with it; a second backward of the same graph; and the C ABI's three backward entry
points on one kept workspace.
"""
import ctypes

import pytest
import torch

import oracle
from helpers import TOL, max_rel, randn_pair, rel_err
from memoryefficientclip_amd import _lib
from memoryefficientclip_amd.clip_loss import (
    MemoryEfficientCLIPLoss,
    MemoryEfficientCLIPLossNormed,
    StableMemoryEfficientCLIPLoss,
)
from memoryefficientclip_amd.lit_loss import MemoryEfficientLiTLoss, MemoryEfficientLiTLossNormed

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
F32 = TOL[torch.float32]


def say(*a):
    print(*a, flush=True)


def fwd_bwd(module, a, b, grad_a=True, grad_b=True, grad_scale=None):
    ga = a.to(DEV).requires_grad_(grad_a)
    gb = b.to(DEV).requires_grad_(grad_b)
    loss = module(ga, gb)
    kept = bool(loss.grad_fn.mec[5] & _lib.FLAG_KEEP_EXP)
    (loss if grad_scale is None else loss * grad_scale).backward()
    torch.cuda.synchronize()
    return (loss.detach().cpu(), ga.grad.cpu() if grad_a else None, gb.grad.cpu() if grad_b else None, kept)


def check(name, loss, ref_loss, grads):
    le = rel_err(loss, ref_loss)
    errs = [(g, max_rel(v, r)) for g, v, r in grads]
    say(f"{name}: loss rel {le:.2e} " + " ".join(f"{g} {e:.2e}" for g, e in errs))
    assert le <= F32["loss"] or (float(ref_loss) == 0.0 and abs(float(loss)) < 1e-6)
    for g, e in errs:
        assert e <= F32["grad"], (name, g, e)


SHAPES = [(1024, 512), (1000, 384), (65, 36), (1, 8), (2048, 64), (2048, 512), (130, 1028), (777, 4)]


@pytest.mark.parametrize("n,d", SHAPES)
def test_keep_clip_parity(n, d):
    a, b = randn_pair(n, d, seed=n + d)
    loss, da, db, kept = fwd_bwd(MemoryEfficientCLIPLoss(0.07), a, b)
    assert kept
    rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.07)
    check(f"clip keep n={n} d={d}", loss, rl, [("da", da, rda), ("db", db, rdb)])


@pytest.mark.parametrize("n,d", [(1024, 512), (1000, 384), (65, 36), (1, 8)])
def test_keep_lit_parity(n, d):
    txt, img = randn_pair(n, d, seed=3 * n + d)
    loss, dt, _, kept = fwd_bwd(MemoryEfficientLiTLoss(0.07), txt, img, grad_b=False)
    assert kept
    rl, rdt = oracle.lit_loss_and_grads(txt, img, 0.07)
    check(f"lit keep n={n} d={d}", loss, rl, [("dtext", dt, rdt)])


def test_keep_normed_stable_grad_output_frozen():
    n, d = 700, 256
    a, b = randn_pair(n, d, seed=11)
    an = torch.nn.functional.normalize(a, dim=1)
    bn = torch.nn.functional.normalize(b, dim=1)
    loss, da, db, kept = fwd_bwd(lambda u, v: MemoryEfficientCLIPLossNormed.apply(u, v, 0.05), an, bn,
                                 grad_scale=-1.5)
    assert kept
    rl, rda, rdb = oracle.clip_loss_and_grads(an, bn, 0.05, normalized_inputs=True, grad_output=-1.5)
    check("clip normed g=-1.5", loss, rl, [("da", da, rda), ("db", db, rdb)])
    loss, da, db, kept = fwd_bwd(StableMemoryEfficientCLIPLoss(0.07), a, b)
    assert kept
    rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.07, stable=True)
    check("clip stable", loss, rl, [("da", da, rda), ("db", db, rdb)])
    loss, dt, _, kept = fwd_bwd(lambda u, v: MemoryEfficientLiTLossNormed.apply(u, v, 0.07), an, bn, grad_b=False)
    assert kept
    rl, rdt = oracle.lit_loss_and_grads(an, bn, 0.07, normalized_inputs=True)
    check("lit normed", loss, rl, [("dtext", dt, rdt)])
    # frozen text tower: the x side alone
    loss, da, _, kept = fwd_bwd(MemoryEfficientCLIPLoss(0.07), a, b, grad_b=False)
    assert kept
    rl, rda, _ = oracle.clip_loss_and_grads(a, b, 0.07)
    check("clip frozen text", loss, rl, [("da", da, rda)])


def test_keep_zero_rows_and_frozen_image():
    """A zero row on each side (F.normalize clamps its norm: the gradient is
    dx^ / eps, no projection) and the y side alone (frozen image tower)."""
    n, d = 300, 64
    a, b = randn_pair(n, d, seed=13)
    a[5] = 0.0
    b[17] = 0.0
    loss, da, db, kept = fwd_bwd(MemoryEfficientCLIPLoss(0.07), a, b)
    assert kept
    rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.07)
    rest = [i for i in range(n) if i not in (5, 17)]
    check("clip zero rows (other rows)", loss, rl, [("da", da[rest], rda[rest]), ("db", db[rest], rdb[rest])])
    check("clip zero rows (those rows)", loss, rl, [("da", da[5], rda[5]), ("db", db[17], rdb[17])])
    loss, _, db, kept = fwd_bwd(MemoryEfficientCLIPLoss(0.07), a, b, grad_a=False)
    assert kept
    check("clip frozen image (other rows)", loss, rl, [("db", db[rest], rdb[rest])])


@pytest.mark.parametrize("lit", [False, True])
def test_keep_row_strided_views(lit):
    """Column slices of wider tensors (row stride 300 > d = 288, 16-byte
    rows): the kept path reads the inputs, and the fused backward its
    epilogue's own and other-side values, at the row stride."""
    n, d, ld = 500, 288, 300
    wa, wb = randn_pair(n, ld, seed=17)
    a, b = wa[:, :d], wb[:, :d]
    ga = wa.to(DEV)[:, :d].requires_grad_(True)
    gb = wb.to(DEV)[:, :d].requires_grad_(not lit)
    assert ga.stride(0) == ld and gb.stride(0) == ld
    mod = MemoryEfficientLiTLoss(0.07) if lit else MemoryEfficientCLIPLoss(0.07)
    loss = mod(ga, gb)
    assert loss.grad_fn.mec[0] == ld and loss.grad_fn.mec[5] & _lib.FLAG_KEEP_EXP
    loss.backward()
    torch.cuda.synchronize()
    if lit:
        rl, rda = oracle.lit_loss_and_grads(a, b, 0.07)
        check("lit keep strided", loss.detach().cpu(), rl, [("dtext", ga.grad.cpu(), rda)])
    else:
        rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.07)
        check("clip keep strided", loss.detach().cpu(), rl, [("da", ga.grad.cpu(), rda), ("db", gb.grad.cpu(), rdb)])


@pytest.mark.parametrize("lit", [False, True])
def test_keep_matches_recomputing_path(monkeypatch, lit):
    n, d = 1000, 512
    a, b = randn_pair(n, d, seed=5)
    mod = MemoryEfficientLiTLoss(0.07) if lit else MemoryEfficientCLIPLoss(0.07)
    l1, da1, db1, kept = fwd_bwd(mod, a, b, grad_b=not lit)
    assert kept
    monkeypatch.setenv("MEC_KEEP_EXP", "0")
    l0, da0, db0, kept0 = fwd_bwd(mod, a, b, grad_b=not lit)
    assert not kept0
    le, ge = rel_err(l1, l0), max_rel(da1, da0)
    if not lit:
        ge = max(ge, max_rel(db1, db0))
    say(f"keep vs recompute (lit={lit}): loss rel {le:.2e}, grad max-rel {ge:.2e}")
    assert le <= 1e-5 and ge <= 1e-4


def test_keep_is_bitwise_reproducible_and_second_backward():
    n, d = 900, 320
    a, b = randn_pair(n, d, seed=9)
    outs = []
    for _ in range(2):
        ga = a.to(DEV).requires_grad_(True)
        gb = b.to(DEV).requires_grad_(True)
        loss = MemoryEfficientCLIPLoss(0.07)(ga, gb)
        g1 = torch.autograd.grad(loss, (ga, gb), retain_graph=True)
        g2 = torch.autograd.grad(loss, (ga, gb))  # a second backward of the same graph
        torch.cuda.synchronize()
        assert torch.equal(g1[0], g2[0]) and torch.equal(g1[1], g2[1])
        outs.append((loss.detach().cpu(), g1[0].cpu(), g1[1].cpu()))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1]) and torch.equal(outs[0][2], outs[1][2])


def test_keep_under_deterministic_algorithms():
    """With torch.use_deterministic_algorithms(True) the module still keeps
    the matrix (the flag and MEC_FLAG_DETERMINISTIC together), and the result
    is bitwise the one without: every sum of the kept path is in a fixed
    order either way."""
    n, d = 700, 128
    a, b = randn_pair(n, d, seed=17)
    plain = fwd_bwd(MemoryEfficientCLIPLoss(0.07), a, b)
    prev = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True)
    try:
        det = fwd_bwd(MemoryEfficientCLIPLoss(0.07), a, b)
    finally:
        torch.use_deterministic_algorithms(prev)
    assert plain[3] and det[3]
    for u, v in zip(plain[:3], det[:3]):
        assert torch.equal(u, v)
    rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.07)
    check("keep, deterministic", det[0], rl, [("dx", det[1], rda), ("dy", det[2], rdb)])


@pytest.mark.parametrize("case", ["nan", "overflow"])
def test_keep_non_finite_loss(monkeypatch, case):
    """A NaN input gives a NaN loss, and rows far outside the unit sphere
    under normalized_inputs=True (cos >> 1: exp overflows in fp32) an
    infinite one, on the kept path as on the recomputing path (the kept
    finalize's fixed-point loss word carries both as flag bits)."""
    n, d = 300, 64
    a, b = randn_pair(n, d, seed=31)
    if case == "nan":
        a[7, 5] = float("nan")
        mod = MemoryEfficientCLIPLoss(0.07)
    else:
        # every row near one direction at norm 3: the off-diagonal cos are
        # about 9, and exp((cos - 1) / T) overflows in the tiles' fp32 sums
        u = torch.nn.functional.normalize(a[:1], dim=1)
        a = 3.0 * torch.nn.functional.normalize(u + 0.01 * a, dim=1)
        b = 3.0 * torch.nn.functional.normalize(u + 0.01 * b, dim=1)
        mod = MemoryEfficientCLIPLoss(0.07, normalized_inputs=True)
    kept = fwd_bwd(mod, a, b)
    monkeypatch.setenv("MEC_KEEP_EXP", "0")
    rec = fwd_bwd(mod, a, b)
    assert kept[3] and not rec[3]
    say(f"{case}: kept loss {float(kept[0])}, recomputing {float(rec[0])}")
    if case == "nan":
        assert torch.isnan(kept[0]) and torch.isnan(rec[0])
    else:
        assert torch.isinf(kept[0]) and kept[0] > 0 and not torch.isfinite(rec[0])


def test_keep_c_abi_entry_points():
    """mec_forward with the flag, then mec_backward (no scratch), mec_grad +
    mec_postpass and mec_backward_noalloc on the same kept workspace.
    mec_backward and mec_backward_noalloc run the same fused launch
    (identical gradients); mec_grad + mec_postpass forms the normalisation
    backward's dot products over the features instead of from the finalize's
    block sums (agreement to fp32 rounding); all three match the oracle."""
    lib = _lib.load()
    n, d, t = 513, 200, 0.07
    a, b = randn_pair(n, d, seed=21)
    x, y = a.to(DEV), b.to(DEV)
    assert lib.mec_keep_exp_supported(x.data_ptr(), d, y.data_ptr(), d, n, d, _lib.DTYPE_F32) == 1
    mode = _lib.MODE_CLIP | _lib.FLAG_KEEP_EXP
    ws = torch.empty(lib.mec_workspace_floats_mode(n, d, _lib.DTYPE_F32, mode), dtype=torch.float32, device=DEV)
    loss = torch.empty((), dtype=torch.float32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    _lib.call("mec_forward", x.data_ptr(), d, y.data_ptr(), d, n, d, _lib.DTYPE_F32, mode, 1, t, ws.data_ptr(),
              loss.data_ptr(), stream)
    assert lib.mec_grad_scratch_bytes_for(n, d, _lib.DTYPE_F32, mode, _lib.SIDE_X | _lib.SIDE_Y) == 0
    res = []
    for how in ("backward", "grad+postpass", "noalloc"):
        ax = torch.empty(n, d, device=DEV)
        ay = torch.empty(n, d, device=DEV)
        if how == "backward":
            _lib.call("mec_backward", x.data_ptr(), d, y.data_ptr(), d, n, d, 0, mode, 1, t, 1.0 / t, ws.data_ptr(),
                      None, None, 0, ax.data_ptr(), ay.data_ptr(), ax.data_ptr(), ay.data_ptr(), stream)
        elif how == "grad+postpass":
            _lib.call("mec_grad", x.data_ptr(), d, y.data_ptr(), d, n, d, 0, mode, 1, t, ws.data_ptr(), None, 0,
                      ax.data_ptr(), ay.data_ptr(), stream)
            _lib.call("mec_postpass", x.data_ptr(), d, y.data_ptr(), d, n, d, 0, mode, 1, 1.0 / t, ws.data_ptr(),
                      None, ax.data_ptr(), ay.data_ptr(), ax.data_ptr(), ay.data_ptr(), stream)
        else:
            _lib.call("mec_backward_noalloc", x.data_ptr(), d, y.data_ptr(), d, n, d, 0, mode, 1, t, 1.0 / t,
                      ws.data_ptr(), None, ax.data_ptr(), ay.data_ptr(), ax.data_ptr(), ay.data_ptr(), stream)
        torch.cuda.synchronize()
        res.append((ax.cpu(), ay.cpu()))
    assert torch.equal(res[2][0], res[0][0]) and torch.equal(res[2][1], res[0][1])
    fe = max(max_rel(res[1][0], res[0][0]), max_rel(res[1][1], res[0][1]))
    say(f"fused vs grad + postpass: max-rel {fe:.2e}")
    assert fe <= 1e-5
    rl, rda, rdb = oracle.clip_loss_and_grads(a, b, t)
    check("c abi keep", loss.cpu(), rl, [("dx", res[0][0], rda), ("dy", res[0][1], rdb)])
    check("c abi keep, grad + postpass", loss.cpu(), rl, [("dx", res[1][0], rda), ("dy", res[1][1], rdb)])
    # the one-stage entry points refuse the flag
    plan = _lib.backward_plan(n, d, _lib.DTYPE_F32, mode)
    assert (plan.num_blocks, plan.scratch_bytes, plan.contract_tile_rows) == (1, 0, 64)
    rc = lib.mec_grad_step(x.data_ptr(), d, y.data_ptr(), d, n, d, 0, mode, 1, t, ws.data_ptr(), 0, None, 0,
                           ctypes.c_void_p(ws.data_ptr()), None, stream)
    assert rc == _lib.MEC_ERR_INVALID and "MEC_FLAG_KEEP_EXP" in _lib.last_error()
