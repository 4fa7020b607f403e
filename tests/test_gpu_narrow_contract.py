"""GPU parity of the 16-bit contraction tiles for a last feature column of at
most 128 features (D % 256 in [1, 128], the block's 256-row tiles in pairs):
512 x 128 tiles, one per pair of row tiles, instead of half-empty 256 x 256
tiles.

MEC_NARROW_CONTRACT=1 forces the narrow tiles wherever the shape allows
them (by default they run only with blocks of at most 4096 rows and when they
save a round of workgroups), =0 the wide tiles alone.  Every output element
sums the same products in the same k order in both tile shapes, so the
gradients are bitwise equal; both agree with the fp64 CPU oracle within the
16-bit tolerance.  The runs use torch.use_deterministic_algorithms, so
that the forward sums (atomic for unnormalized 16-bit inputs otherwise) are
bitwise reproducible too.  The shapes cover D below 256 (narrow tiles only),
ragged N, an odd number of row tiles per block (the wide tiles then cover
the last column, as before) and a remainder of 129 features (no narrow
tiles).
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


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("lit", [False, True], ids=["clip", "lit"])
@pytest.mark.parametrize("n,d,normed", [(1024, 300, False), (1000, 384, True), (2048, 100, False),
                                        (1300, 1152, True), (700, 300, False), (1024, 385, False)])
def test_narrow_contraction_tiles(dt, lit, n, d, normed):
    a, b = randn_pair(n, d, seed=7 * n + d, dtype=dt)
    if normed:
        a = torch.nn.functional.normalize(a.float(), dim=1).to(dt)
        b = torch.nn.functional.normalize(b.float(), dim=1).to(dt)
    kind = "LiT" if lit else "CLIP"
    mod = (MemoryEfficientLiTLoss if lit else MemoryEfficientCLIPLoss)(0.1, normalized_inputs=normed)
    say(f"{dt} {kind} n={n} d={d} normalized={normed}: narrow vs wide contraction tiles")
    l_n, da_n, db_n = run(mod, a, b, not lit, {"MEC_NARROW_CONTRACT": "1"})
    l_w, da_w, db_w = run(mod, a, b, not lit, {"MEC_NARROW_CONTRACT": "0"})
    assert torch.equal(l_n, l_w)
    assert torch.equal(da_n, da_w)
    if not lit:
        assert torch.equal(db_n, db_w)
    af, bf = a.float(), b.float()
    if lit:
        rl, rda = oracle.lit_loss_and_grads(af, bf, 0.1, normalized_inputs=normed)
        pairs = [(da_n, rda)]
    else:
        rl, rda, rdb = oracle.clip_loss_and_grads(af, bf, 0.1, normalized_inputs=normed)
        pairs = [(da_n, rda), (db_n, rdb)]
    errs = [max_rel(g.float(), r) for g, r in pairs]
    tol = TOL[dt]
    say(f"  loss rel {rel_err(l_n, rl):.2e}; grads {['%.2e' % e for e in errs]}")
    assert rel_err(l_n, rl) <= tol["loss"]
    assert all(e <= tol["grad"] for e in errs)


@pytest.mark.parametrize("prec,tol", [("high", TOL[torch.float32]), ("medium", TOL[torch.bfloat16])],
                         ids=["bf16x3", "bf16-products"])
@pytest.mark.parametrize("lit", [False, True], ids=["clip", "lit"])
@pytest.mark.parametrize("n,d", [(1024, 300), (2048, 100)])
def test_narrow_contraction_tiles_fp32_split(prec, tol, lit, n, d):
    """fp32 inputs under matmul precision "high" (bf16x3: three passes over
    hi / lo planes) and "medium" (bf16 products) run the same contraction
    kernel on their bf16 copies."""
    a, b = randn_pair(n, d, seed=11 * n + d)
    kind = "LiT" if lit else "CLIP"
    mod = (MemoryEfficientLiTLoss if lit else MemoryEfficientCLIPLoss)(0.1)
    say(f"fp32 ({prec}) {kind} n={n} d={d}: narrow vs wide contraction tiles")
    with matmul_precision(prec):
        l_n, da_n, db_n = run(mod, a, b, not lit, {"MEC_NARROW_CONTRACT": "1"})
        l_w, da_w, db_w = run(mod, a, b, not lit, {"MEC_NARROW_CONTRACT": "0"})
    assert torch.equal(l_n, l_w) and torch.equal(da_n, da_w)
    if not lit:
        assert torch.equal(db_n, db_w)
    if lit:
        rl, rda = oracle.lit_loss_and_grads(a, b, 0.1)
        pairs = [(da_n, rda)]
    else:
        rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.1)
        pairs = [(da_n, rda), (db_n, rdb)]
    errs = [max_rel(g, r) for g, r in pairs]
    say(f"  loss rel {rel_err(l_n, rl):.2e}; grads {['%.2e' % e for e in errs]}")
    assert rel_err(l_n, rl) <= tol["loss"]
    assert all(e <= tol["grad"] for e in errs)
