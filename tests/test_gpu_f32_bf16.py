"""fp32 inputs under torch.set_float32_matmul_precision("medium"): the
similarity GEMMs and the contractions multiply bf16-rounded values (fp32
accumulate), PyTorch's meaning of "medium"; the norms, the diagonal and the
post-pass stay fp32.

* The bf16 copies that mec_prepass writes are checked bit for bit against a
  numpy round-to-nearest-even restatement (of x_i rx_i when normalize is
  set).
* Loss and gradients are held to the bf16 tolerances (1e-2) against the fp64
  CPU oracle, and at the benchmark's fp32 shape against the dense fp64
  definition on the GPU.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import TOL, matmul_precision, max_rel, randn_pair, ref_fp64, rel_err, split_rows
from memoryefficientclip_amd import _lib
from memoryefficientclip_amd.clip_loss import MemoryEfficientCLIPLoss, StableMemoryEfficientCLIPLoss
from memoryefficientclip_amd.lit_loss import MemoryEfficientLiTLoss

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
BF16 = TOL[torch.bfloat16]


def say(*a):
    print(*a, flush=True)


def run(module, a, b, grad_b=True):
    ga = a.to(DEV).requires_grad_(True)
    gb = b.to(DEV).requires_grad_(grad_b)
    with matmul_precision("medium"):
        loss = module(ga, gb)
        loss.backward()
    torch.cuda.synchronize()
    return loss.detach().cpu(), ga.grad.cpu(), (gb.grad.cpu() if grad_b else None)


@pytest.mark.parametrize("norm", [1, 0], ids=["normalize", "raw"])
@pytest.mark.parametrize("n,d,ld", [(300, 96, 96), (77, 3, 5)])
def test_bf16_copies_are_exact(n, d, ld, norm):
    g = torch.Generator().manual_seed(n + d)
    xw = torch.randn(n, ld, generator=g) * torch.exp(torch.randn(n, ld, generator=g))
    yw = torch.randn(n, ld, generator=g)
    x, y = xw.to(DEV), yw.to(DEV)
    dt = _lib.DTYPE_F32_BF16
    lib = _lib.load()
    ws = torch.zeros(lib.mec_workspace_floats_for(n, d, dt), dtype=torch.float32, device=DEV)
    say(f"bf16 copies n={n} d={d} ld={ld} normalize={norm}")
    _lib.call("mec_prepass", x.data_ptr(), ld, y.data_ptr(), ld, n, d, dt, norm, ws.data_ptr(),
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    off = (lib.mec_workspace_floats(n) + 3) // 4 * 4
    dp = (d + 7) // 8 * 8
    raw = ws[off:].cpu().numpy().view(np.uint16)
    assert raw.size == 2 * n * dp
    # normalize: the copies are of x_i rx_i (fp32 product, rx as the pre-pass wrote it)
    rx = ws[:n].cpu().numpy()[:, None]
    ry = ws[n:2 * n].cpu().numpy()[:, None]
    if not norm:
        assert np.all(rx == 1) and np.all(ry == 1)
    np.testing.assert_array_equal(raw[: n * dp].reshape(n, dp), split_rows(xw[:, :d].numpy() * rx, 2))
    np.testing.assert_array_equal(raw[n * dp:].reshape(n, dp), split_rows(yw[:, :d].numpy() * ry, 2))


CASES = [
    # (mode, n, d, normalized_inputs, stable, temperature)
    ("clip", 300, 96, False, False, 0.07),
    ("clip", 1000, 3, False, False, 0.07),
    ("clip", 2300, 130, True, True, 0.05),
    ("lit", 777, 200, False, False, 0.07),
    ("clip", 1, 1, False, False, 0.07),
]


@pytest.mark.parametrize("mode,n,d,normed,stable,t", CASES, ids=[f"{c[0]}-{c[1]}x{c[2]}" for c in CASES])
def test_parity_against_the_oracle(mode, n, d, normed, stable, t):
    lit = mode == "lit"
    a, b = randn_pair(n, d, seed=n + 3 * d)
    if normed:
        a = torch.nn.functional.normalize(a, dim=1)
        b = torch.nn.functional.normalize(b, dim=1)
    mod = (MemoryEfficientLiTLoss if lit else StableMemoryEfficientCLIPLoss if stable else MemoryEfficientCLIPLoss)(
        t, normalized_inputs=normed)
    say(f"fp32/bf16 {mode} n={n} d={d} normed={normed} stable={stable} T={t}")
    loss, da, db = run(mod, a, b, grad_b=not lit)
    if lit:
        rl, rda = oracle.lit_loss_and_grads(a, b, t, normalized_inputs=normed)
        grads = [(da, rda)]
    else:
        rl, rda, rdb = oracle.clip_loss_and_grads(a, b, t, normalized_inputs=normed, stable=stable)
        grads = [(da, rda), (db, rdb)]
    le = abs(float(loss) - float(rl)) if float(rl) == 0.0 else rel_err(loss, rl)
    ge = [max_rel(g, r) for g, r in grads]
    say(f"  loss rel {le:.2e}, grads {['%.2e' % e for e in ge]}")
    assert le <= BF16["loss"] and all(e <= BF16["grad"] for e in ge)


def test_strided_and_differs_from_bf16x3():
    n, d = 1500, 256
    a, b = randn_pair(n, d, seed=5)
    wa = torch.zeros(n, d + 40)
    wa[:, 7:7 + d] = a
    ga = wa.to(DEV)[:, 7:7 + d]
    say(f"fp32/bf16 strided n={n} d={d}")
    lm, dam, dbm = run(MemoryEfficientCLIPLoss(0.07), ga, b)
    with matmul_precision("high"):
        gx = a.to(DEV).requires_grad_(True)
        gy = b.to(DEV).requires_grad_(True)
        lh = MemoryEfficientCLIPLoss(0.07)(gx, gy)
        lh.backward()
    rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.07)
    assert rel_err(lm, rl) <= BF16["loss"] and max_rel(dam, rda) <= BF16["grad"] and max_rel(dbm, rdb) <= BF16["grad"]
    # bf16 products are a coarser computation than the three-term form
    e_m, e_h = max_rel(dam, rda), max_rel(gx.grad.cpu(), rda)
    say(f"  grad max-rel: medium {e_m:.2e}, high {e_h:.2e}")
    assert e_h < e_m


def test_full_size():
    n, d, t = 32768, 1152, 0.07
    a, b = randn_pair(n, d, seed=0)
    say(f"fp32/bf16 full size clip n={n} d={d}")
    loss, da, db = run(MemoryEfficientCLIPLoss(t), a, b)
    rl, rda, rdb = ref_fp64(a.to(DEV), b.to(DEV), t, False, False, 4096)
    le, ea, eb = rel_err(loss, rl.item()), max_rel(da, rda), max_rel(db, rdb)
    say(f"  loss {float(loss):.7f} ref {rl.item():.7f} rel {le:.2e}; grads {ea:.2e} {eb:.2e}")
    assert le <= BF16["loss"] and ea <= BF16["grad"] and eb <= BF16["grad"]
