"""GPU parity of the 16-bit contraction tiles 384 features wide (256 x 384
tiles, 8 waves of 128 x 96 on the rolling operand schedule, the
gradient-matrix operand in four half-chunk LDS stages).

MEC_WIDE_CONTRACT=1 forces them for every 16-bit contraction, =0 the 256 x
256 tiles (with the narrow tiles where those apply).  Every output element
sums the same products in the same k order in both tile shapes, so the
gradients are bitwise equal; both agree with the fp64 CPU oracle within the
16-bit tolerance.  The runs use torch.use_deterministic_algorithms, so that
the forward sums (atomic for unnormalized 16-bit inputs otherwise) are
bitwise reproducible too.  The shapes cover D below, at and between
multiples of 384 (the last feature tile partly empty), ragged N with a
short last block, and several k-chunks per tile.  The contraction's k runs
over a block's rows in chunks of 64 of two half-chunks each: the shapes end
k within the first half of the last chunk (N = 513, 1300, 20, 150), within
the second (N = 1000, 700, 40, 100), on a chunk boundary (N = 1024), and
cover one, two and three chunks in all (N = 20 and 40, 100, 150).
"""
import os

import pytest
import torch

import oracle
from helpers import TOL, matmul_precision, max_rel, randn_pair, rel_err
from memoryefficientclip_amd.clip_loss import MemoryEfficientCLIPLoss
from memoryefficientclip_amd.lit_loss import MemoryEfficientLiTLoss

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(*a):
    print(*a, flush=True)


def run(module, a, b, grad_b, env):
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    det = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True)
    try:
        ga = a.to(DEV).requires_grad_(True)
        gb = b.to(DEV).requires_grad_(grad_b)
        loss = module(ga, gb)
        loss.backward()
        torch.cuda.synchronize()
        return loss.detach().cpu(), ga.grad.cpu(), (gb.grad.cpu() if grad_b else None)
    finally:
        torch.use_deterministic_algorithms(det)
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


SHAPES = [(1024, 300, False), (1000, 384, True), (2048, 100, False), (1300, 1152, True), (700, 768, False),
          (1024, 385, False), (513, 1000, True), (3000, 64, False), (20, 768, True), (40, 300, False),
          (100, 1152, False), (150, 384, True)]


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("lit", [False, True], ids=["clip", "lit"])
@pytest.mark.parametrize("n,d,normed", SHAPES)
def test_wide_contraction_tiles(dt, lit, n, d, normed):
    a, b = randn_pair(n, d, seed=5 * n + d, dtype=dt)
    if normed:
        a = torch.nn.functional.normalize(a.float(), dim=1).to(dt)
        b = torch.nn.functional.normalize(b.float(), dim=1).to(dt)
    kind = "LiT" if lit else "CLIP"
    mod = (MemoryEfficientLiTLoss if lit else MemoryEfficientCLIPLoss)(0.1, normalized_inputs=normed)
    say(f"{dt} {kind} n={n} d={d} normalized={normed}: 384- vs 256-wide contraction tiles")
    l_w, da_w, db_w = run(mod, a, b, not lit, {"MEC_WIDE_CONTRACT": "1"})
    l_s, da_s, db_s = run(mod, a, b, not lit, {"MEC_WIDE_CONTRACT": "0"})
    assert torch.equal(l_w, l_s)
    assert torch.equal(da_w, da_s)
    if not lit:
        assert torch.equal(db_w, db_s)
    af, bf = a.float(), b.float()
    if lit:
        rl, rda = oracle.lit_loss_and_grads(af, bf, 0.1, normalized_inputs=normed)
        pairs = [(da_w, rda)]
    else:
        rl, rda, rdb = oracle.clip_loss_and_grads(af, bf, 0.1, normalized_inputs=normed)
        pairs = [(da_w, rda), (db_w, rdb)]
    errs = [max_rel(g.float(), r) for g, r in pairs]
    tol = TOL[dt]
    say(f"  loss rel {rel_err(l_w, rl):.2e}; grads {['%.2e' % e for e in errs]}")
    assert rel_err(l_w, rl) <= tol["loss"]
    assert all(e <= tol["grad"] for e in errs)


@pytest.mark.parametrize("prec,tol", [("high", TOL[torch.float32]), ("medium", TOL[torch.bfloat16])],
                         ids=["bf16x3", "bf16-products"])
@pytest.mark.parametrize("lit", [False, True], ids=["clip", "lit"])
@pytest.mark.parametrize("n,d", [(1024, 300), (1300, 1152)])
def test_wide_contraction_tiles_fp32_split(prec, tol, lit, n, d):
    """fp32 inputs under matmul precision "high" (bf16x3: three passes over
    hi / lo planes into one accumulator) and "medium" (bf16 products) run
    the same contraction kernel on their bf16 copies."""
    a, b = randn_pair(n, d, seed=13 * n + d)
    kind = "LiT" if lit else "CLIP"
    mod = (MemoryEfficientLiTLoss if lit else MemoryEfficientCLIPLoss)(0.1)
    say(f"fp32 ({prec}) {kind} n={n} d={d}: 384- vs 256-wide contraction tiles")
    with matmul_precision(prec):
        l_w, da_w, db_w = run(mod, a, b, not lit, {"MEC_WIDE_CONTRACT": "1"})
        l_s, da_s, db_s = run(mod, a, b, not lit, {"MEC_WIDE_CONTRACT": "0"})
    assert torch.equal(l_w, l_s) and torch.equal(da_w, da_s)
    if not lit:
        assert torch.equal(db_w, db_s)
    if lit:
        rl, rda = oracle.lit_loss_and_grads(a, b, 0.1)
        pairs = [(da_w, rda)]
    else:
        rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.1)
        pairs = [(da_w, rda), (db_w, rdb)]
    errs = [max_rel(g, r) for g, r in pairs]
    say(f"  loss rel {rel_err(l_w, rl):.2e}; grads {['%.2e' % e for e in errs]}")
    assert rel_err(l_w, rl) <= tol["loss"]
    assert all(e <= tol["grad"] for e in errs)
