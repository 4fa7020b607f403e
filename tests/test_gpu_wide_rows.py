"""Rows wider than the post-pass register cache (D > 2048 features: the
normalisation backward reads each row twice) and at its edge (D = 2048,
held in registers), through the modules, against the fp64 oracle."""
import pytest
import torch

import oracle
from helpers import TOL, max_rel, randn_pair, rel_err
from memoryefficientclip_amd import MemoryEfficientCLIPLoss, MemoryEfficientLiTLoss

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

CASES = [
    # (dtype, mode, n, d)
    (torch.float32, "clip", 300, 2100),
    (torch.float32, "lit", 257, 2048),
    (torch.bfloat16, "clip", 500, 2304),
    (torch.float16, "lit", 130, 2049),
]


@pytest.mark.parametrize("dtype,mode,n,d", CASES, ids=[f"{c[1]}-{c[2]}x{c[3]}-{str(c[0])[6:]}" for c in CASES])
def test_wide_rows(dtype, mode, n, d):
    lit = mode == "lit"
    a, b = randn_pair(n, d, seed=n + d, dtype=dtype)
    print(f"wide rows {mode} n={n} d={d} {dtype}", flush=True)
    ga = a.to(DEV).requires_grad_(True)
    gb = b.to(DEV).requires_grad_(not lit)
    mod = MemoryEfficientLiTLoss(0.07) if lit else MemoryEfficientCLIPLoss(0.07)
    loss = mod(ga, gb)
    (loss * 1.5).backward()
    torch.cuda.synchronize()
    tol = TOL[dtype]
    if lit:
        rl, rda = oracle.lit_loss_and_grads(a.float(), b.float(), 0.07, grad_output=1.5)
        grads = [(ga.grad, rda)]
    else:
        rl, rda, rdb = oracle.clip_loss_and_grads(a.float(), b.float(), 0.07, grad_output=1.5)
        grads = [(ga.grad, rda), (gb.grad, rdb)]
    le = rel_err(loss.detach().cpu(), rl)
    ge = [max_rel(g.float().cpu(), r) for g, r in grads]
    print(f"  loss rel {le:.2e}, grads {ge}", flush=True)
    assert le <= tol["loss"] and all(e <= tol["grad"] for e in ge)
