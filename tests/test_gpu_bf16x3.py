"""The bf16x3 mode for fp32 inputs (torch.set_float32_matmul_precision("high")):
every product of the similarity GEMMs and the gradient contractions is formed
as hi*hi + lo*hi + hi*lo from bf16 terms on the bf16 MFMA.

* The split copies of x and y that mec_prepass writes into the workspace are
  checked bit for bit against a numpy restatement of the split (round to
  nearest even, lo = bf16(v - hi)) of the rows, normalized first (x_i rx_i
  in fp32, rx as the pre-pass wrote it) when normalize is set.
* Loss and gradients are held to the fp32 tolerances (loss rel 1e-4,
  gradient max-rel 1e-3) against the fp64 CPU oracle at small sizes and
  against the dense fp64 definition on the GPU (PyTorch fp64 GEMMs, none of
  this package's kernels) at the benchmark's fp32 sizes.
* The mode really runs: its gradients differ from the IEEE fp32 path's.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from helpers import TOL, matmul_precision, max_rel, randn_pair, ref_fp64, rel_err, split_rows
from memoryefficientclip_amd import _lib
from memoryefficientclip_amd.clip_loss import MemoryEfficientCLIPLoss, StableMemoryEfficientCLIPLoss
from memoryefficientclip_amd.lit_loss import MemoryEfficientLiTLoss, StableMemoryEfficientLiTLoss

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
F32 = TOL[torch.float32]


def say(*a):
    print(*a, flush=True)


def run(module, a, b, grad_b=True):
    ga = a.to(DEV).requires_grad_(True)
    gb = b.to(DEV).requires_grad_(grad_b)
    loss = module(ga, gb)
    loss.backward()
    torch.cuda.synchronize()
    return loss.detach().cpu(), ga.grad.cpu(), (gb.grad.cpu() if grad_b else None)


@pytest.mark.parametrize("norm", [1, 0], ids=["normalize", "raw"])
@pytest.mark.parametrize("n,d,ld", [(300, 96, 96), (77, 3, 5), (1000, 130, 136)])
def test_split_copies_are_exact(n, d, ld, norm):
    """k_split3 output read back from the workspace, bit for bit."""
    g = torch.Generator().manual_seed(n + d)
    xw = torch.randn(n, ld, generator=g) * torch.exp(torch.randn(n, ld, generator=g))  # wide dynamic range
    yw = torch.randn(n, ld, generator=g)
    x, y = xw.to(DEV), yw.to(DEV)
    dt = _lib.DTYPE_F32_BF16X3
    lib = _lib.load()
    nf = lib.mec_workspace_floats_for(n, d, dt)
    ws = torch.zeros(nf, dtype=torch.float32, device=DEV)
    say(f"split n={n} d={d} ld={ld} normalize={norm}")
    _lib.call("mec_prepass", x.data_ptr(), ld, y.data_ptr(), ld, n, d, dt, norm, ws.data_ptr(),
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    off = (lib.mec_workspace_floats(n) + 3) // 4 * 4
    dp = (d + 7) // 8 * 8
    raw = ws[off:].cpu().numpy().view(np.uint16)
    assert raw.size == 2 * n * 3 * dp
    a3 = raw[: n * 3 * dp].reshape(n, 3 * dp)
    b3 = raw[n * 3 * dp:].reshape(n, 3 * dp)
    rx = ws[:n].cpu().numpy()[:, None]
    ry = ws[n:2 * n].cpu().numpy()[:, None]
    if not norm:
        assert np.all(rx == 1) and np.all(ry == 1)
    np.testing.assert_array_equal(a3, split_rows(xw[:, :d].numpy() * rx, 0))
    np.testing.assert_array_equal(b3, split_rows(yw[:, :d].numpy() * ry, 1))
    # the norms and the diagonal come from the fp32 inputs, as in the fp32 mode
    ws32 = torch.zeros(lib.mec_workspace_floats(n), dtype=torch.float32, device=DEV)
    _lib.call("mec_prepass", x.data_ptr(), ld, y.data_ptr(), ld, n, d, _lib.DTYPE_F32, norm, ws32.data_ptr(),
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(ws[: 3 * n].cpu(), ws32[: 3 * n].cpu())


CASES = [
    # (mode, n, d, normalized_inputs, stable, temperature)
    ("clip", 300, 96, False, False, 0.07),
    ("clip", 1000, 3, False, False, 0.07),
    ("clip", 2300, 128, True, False, 0.05),
    ("clip", 4133, 520, False, True, 0.07),
    ("lit", 777, 200, False, False, 0.07),
    ("lit", 2600, 264, True, True, 0.1),
]


@pytest.mark.parametrize("mode,n,d,normed,stable,t", CASES, ids=[f"{c[0]}-{c[1]}x{c[2]}" for c in CASES])
def test_parity_against_the_oracle(mode, n, d, normed, stable, t):
    lit = mode == "lit"
    a, b = randn_pair(n, d, seed=n + 7 * d)
    if normed:
        a = torch.nn.functional.normalize(a, dim=1)
        b = torch.nn.functional.normalize(b, dim=1)
    if lit:
        cls = StableMemoryEfficientLiTLoss if stable else MemoryEfficientLiTLoss
    else:
        cls = StableMemoryEfficientCLIPLoss if stable else MemoryEfficientCLIPLoss
    mod = cls(t, normalized_inputs=normed)
    say(f"bf16x3 {mode} n={n} d={d} normed={normed} stable={stable} T={t}")
    with matmul_precision("high"):
        loss, da, db = run(mod, a, b, grad_b=not lit)
    if lit:
        rl, rda = oracle.lit_loss_and_grads(a, b, t, normalized_inputs=normed, stable=stable)
        grads = [("d_text", da, rda)]
    else:
        rl, rda, rdb = oracle.clip_loss_and_grads(a, b, t, normalized_inputs=normed, stable=stable)
        grads = [("d_img", da, rda), ("d_txt", db, rdb)]
    le = rel_err(loss, rl)
    ge = {name: max_rel(g, r) for name, g, r in grads}
    say(f"  loss rel {le:.2e}, grads {ge}")
    assert le <= F32["loss"] and all(e <= F32["grad"] for e in ge.values())


@pytest.mark.parametrize("n,d", [(1, 1), (2, 5), (3, 1), (257, 9)])
def test_tiny_shapes(n, d):
    a, b = randn_pair(n, d, seed=31 * n + d)
    say(f"bf16x3 tiny n={n} d={d}")
    with matmul_precision("high"):
        loss, da, db = run(MemoryEfficientCLIPLoss(0.07), a, b)
    rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.07)
    assert abs(float(loss) - float(rl)) <= max(F32["loss"] * abs(float(rl)), 1e-6)
    assert max_rel(da, rda) <= F32["grad"] and max_rel(db, rdb) <= F32["grad"]


def test_frozen_tower_and_grad_output():
    """CLIP with the text tower frozen (only the x side is contracted) and a
    loss scaled by a non-unit grad_output."""
    n, d = 1300, 72
    a, b = randn_pair(n, d, seed=77)
    ga = a.to(DEV).requires_grad_(True)
    gb = b.to(DEV)
    say(f"bf16x3 frozen text tower, grad_output -1.5, n={n} d={d}")
    with matmul_precision("high"):
        loss = MemoryEfficientCLIPLoss(0.07)(ga, gb)
        (loss * -1.5).backward()
    torch.cuda.synchronize()
    rl, rda, _ = oracle.clip_loss_and_grads(a, b, 0.07, grad_output=-1.5)
    assert rel_err(loss.detach().cpu(), rl) <= F32["loss"]
    assert max_rel(ga.grad.cpu(), rda) <= F32["grad"]


def test_mode_differs_from_ieee_and_strided_inputs():
    """Row-strided inputs are read in place; the result differs from the IEEE
    path's (the bf16 products ran) by less than the fp32 tolerance."""
    n, d = 1500, 256
    a, b = randn_pair(n, d, seed=5)
    wa = torch.zeros(n, d + 40)
    wa[:, 7:7 + d] = a
    ga = wa.to(DEV)[:, 7:7 + d]
    say(f"bf16x3 vs ieee, strided n={n} d={d}")
    ieee = run(MemoryEfficientCLIPLoss(0.07), ga.detach().clone(), b)
    with matmul_precision("high"):
        x3 = run(MemoryEfficientCLIPLoss(0.07), ga, b)
    assert rel_err(x3[0], ieee[0]) <= F32["loss"]
    for g3, gi in zip(x3[1:], ieee[1:]):
        e = max_rel(g3, gi)
        say(f"  grad max-rel vs ieee {e:.2e}")
        assert 0.0 < e <= F32["grad"]


def test_deterministic_mode_is_bitwise_repeatable():
    n, d = 2100, 200
    a, b = randn_pair(n, d, seed=9)
    say(f"bf16x3 deterministic n={n} d={d}")
    prev = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True)
    try:
        with matmul_precision("high"):
            r1 = run(MemoryEfficientCLIPLoss(0.07), a, b)
            r2 = run(MemoryEfficientCLIPLoss(0.07), a, b)
    finally:
        torch.use_deterministic_algorithms(prev)
    for u, v in zip(r1, r2):
        assert torch.equal(u, v)
    rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.07)
    assert rel_err(r1[0], rl) <= F32["loss"] and max_rel(r1[1], rda) <= F32["grad"]


@pytest.mark.parametrize("mode", ["clip", "lit"])
def test_full_size(mode):
    """The benchmark's fp32 shape (configs 2 and 3) against the dense fp64
    definition on the GPU."""
    n, d, t = 32768, 1152, 0.07
    lit = mode == "lit"
    a, b = randn_pair(n, d, seed=0)
    say(f"bf16x3 full size {mode} n={n} d={d}")
    mod = MemoryEfficientLiTLoss(t) if lit else MemoryEfficientCLIPLoss(t)
    with matmul_precision("high"):
        loss, da, db = run(mod, a, b, grad_b=not lit)
    rl, rda, rdb = ref_fp64(a.to(DEV), b.to(DEV), t, lit, False, 4096)
    le = rel_err(loss, rl.item())
    ea = max_rel(da, rda)
    eb = 0.0 if lit else max_rel(db, rdb)
    say(f"  loss {float(loss):.7f} ref {rl.item():.7f} rel {le:.2e}; grads {ea:.2e} {eb:.2e}")
    assert math.isfinite(float(loss))
    assert le <= F32["loss"] and ea <= F32["grad"] and eb <= F32["grad"]
