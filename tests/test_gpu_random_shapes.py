"""Randomised GPU parity sweep: shapes, dtypes (fp32, bf16, fp16, and fp32
under float32 matmul precision "high", "f32x3"), modes and layouts drawn from
a fixed seed, each checked against the fp64 CPU oracle on the same
(dtype-rounded) inputs at the task's tolerances.  It covers the
masking of ragged tiles and short last backward blocks, D that is or is not a
multiple of the 16-byte vector, row strides (both 16-bit cores), frozen towers
and grad_output != 1.
"""
import random

import pytest
import torch

import oracle
from helpers import TOL, max_rel, rel_err
from memoryefficientclip_amd import MemoryEfficientCLIPLoss, MemoryEfficientLiTLoss

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def draw_cases(seed=20261201, count=20, dtypes=("f32", "bf16", "f16")):
    rng = random.Random(seed)
    cases = []
    for k in range(count):
        n = rng.choice([1, 2, rng.randint(3, 300), rng.randint(300, 1200), rng.randint(1200, 2600)])
        d = rng.choice([rng.randint(1, 40), 8 * rng.randint(1, 48), rng.randint(41, 400)])
        dtype = rng.choice(list(dtypes))
        mode = rng.choice(["clip", "lit"])
        normed = rng.random() < 0.3
        pad = rng.choice([0, 0, 8, 3])           # extra row stride (0 = contiguous)
        go = rng.choice([1.0, 1.0, -0.5, 2.0])  # grad_output
        temp = rng.choice([0.07, 0.05, 0.1])
        cases.append((k, n, d, dtype, mode, normed, pad, go, temp))
    return cases


CASES = (draw_cases() + [(20 + c[0],) + c[1:] for c in draw_cases(seed=777, count=8, dtypes=("f32x3",))]
         + [(100 + c[0],) + c[1:] for c in draw_cases(seed=101, count=30)])


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(v) for v in c[:6]))
def test_random_case(case):
    k, n, d, dt, mode, normed, pad, go, temp = case
    torch_dt = {"f32": torch.float32, "f32x3": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dt]
    g = torch.Generator().manual_seed(1000 + k)
    a = torch.randn(n, d, generator=g)
    b = torch.randn(n, d, generator=g)
    if normed:
        a = torch.nn.functional.normalize(a, dim=1)
        b = torch.nn.functional.normalize(a + 0.5 * b, dim=1)
    a, b = a.to(torch_dt), b.to(torch_dt)
    wa = torch.zeros(n, d + pad, dtype=torch_dt)
    wb = torch.zeros(n, d + pad, dtype=torch_dt)
    wa[:, pad:pad + d] = a
    wb[:, pad:pad + d] = b
    ga = wa.to(DEV)[:, pad:pad + d].requires_grad_(True)
    gb = wb.to(DEV)[:, pad:pad + d].requires_grad_(mode == "clip")
    print(f"case {case}", flush=True)
    old_precision = torch.get_float32_matmul_precision()
    torch.set_float32_matmul_precision("high" if dt == "f32x3" else "highest")
    try:
        if mode == "clip":
            loss = MemoryEfficientCLIPLoss(temp, normed)(ga, gb)
        else:
            loss = MemoryEfficientLiTLoss(temp, normed)(ga, gb)
        (loss * go).backward()
        torch.cuda.synchronize()
    finally:
        torch.set_float32_matmul_precision(old_precision)
    tol = TOL[torch_dt]
    if mode == "clip":
        rl, rda, rdb = oracle.clip_loss_and_grads(a.float(), b.float(), temp, normalized_inputs=normed, grad_output=go)
        pairs = [(ga.grad.cpu(), rda), (gb.grad.cpu(), rdb)]
    else:
        rl, rda = oracle.lit_loss_and_grads(a.float(), b.float(), temp, normalized_inputs=normed, grad_output=go)
        pairs = [(ga.grad.cpu(), rda)]
    lv = loss.detach().cpu()
    le = rel_err(lv, rl) if float(rl) != 0.0 else abs(float(lv))
    ge = [max_rel(x, r) for x, r in pairs]
    print(f"  loss {float(lv):.6f} ref {float(rl):.6f} rel {le:.2e} grads {['%.2e' % e for e in ge]}", flush=True)
    assert le <= tol["loss"] or abs(float(lv) - float(rl)) < 1e-6
    assert all(e <= tol["grad"] for e in ge)
