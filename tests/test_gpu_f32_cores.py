"""GPU parity of the fp32 core choices, against the fp64 CPU oracle.

fp32 inputs whose rows are 16-byte aligned (base, d and the row stride
multiples of 4 floats) run the forward and gradient-matrix tiles on the
direct-to-LDS core, and the contractions read the raw input rows with 16-byte
load lanes; other layouts run the forward and gradient-matrix tiles on the
register-staged core and the contractions with 4-byte load lanes.  Both are
checked against the oracle and against each other, and a row stride past the
direct core's 32-bit panel range takes the second path too.

Up to N = 2816 the direct-to-LDS kernels run 64 x 64 tiles (a 128 x 128
grid would leave CUs idle), above it where a launch's 128 x 128 grid would be
small for its K or fill its rounds of CUs poorly (the forward and each
backward step choose on their own); MEC_F32_SMALL_TILES=0 / 1 forces either
tile size, so both are checked on both sides of those bounds, with the kept
similarity matrix (which takes over at N <= 2048) turned off.
"""
import os

import pytest
import torch

import oracle
from helpers import max_rel, randn_pair, rel_err
from memoryefficientclip_amd.clip_loss import MemoryEfficientCLIPLoss
from memoryefficientclip_amd.lit_loss import MemoryEfficientLiTLoss

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL_LOSS, TOL_GRAD = 1e-4, 1e-3


def say(*a):
    print(*a, flush=True)


def run(module, a, b, grad_b=True):
    ga = a.to(DEV).requires_grad_(True)
    gb = b.to(DEV).requires_grad_(grad_b)
    loss = module(ga, gb)
    loss.backward()
    torch.cuda.synchronize()
    return loss.detach().cpu(), ga.grad.cpu(), (gb.grad.cpu() if grad_b else None)


def strided(t, ld):
    """A GPU copy of t [n, d] with row stride ld (ld >= d)."""
    n, d = t.shape
    flat = torch.zeros(n * ld, device=DEV)
    g = flat.as_strided((n, d), (ld, 1))
    g.copy_(t.to(DEV))
    return g


@pytest.mark.parametrize("lit", [False, True], ids=["clip", "lit"])
@pytest.mark.parametrize("n,d,ld", [(2300, 96, 97), (700, 130, 130), (4500, 64, 66)])
def test_f32_unaligned_rows(lit, n, d, ld):
    """Rows that are not 16-byte vectors (an odd row stride, d % 4 != 0):
    register-staged gradient-matrix tiles, 4-byte load lanes for the
    contractions' raw-input operand; against the oracle, and against the
    same values in aligned rows (16-byte lanes, direct-to-LDS tiles).  The
    shapes cover two backward blocks with a short last one (2300 rows at
    d = 96), one block, and the 128 x 128 tiles (4500 rows)."""
    a, b = randn_pair(n, d, seed=31 + n)
    mod = MemoryEfficientLiTLoss(0.07) if lit else MemoryEfficientCLIPLoss(0.07)
    say(f"fp32 {'LiT' if lit else 'CLIP'} n={n} d={d}: row stride {ld} vs aligned rows")
    l_al, da_al, db_al = run(mod, a, b, grad_b=not lit)
    ga = strided(a, ld).requires_grad_(True)
    gb = strided(b, ld).requires_grad_(not lit)
    loss = mod(ga, gb)
    loss.backward()
    torch.cuda.synchronize()
    l_un, da_un = loss.detach().cpu(), ga.grad.cpu()
    db_un = None if lit else gb.grad.cpu()
    if lit:
        rl, rda = oracle.lit_loss_and_grads(a, b, 0.07)
        pairs = [(da_al, rda), (da_un, rda)]
    else:
        rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.07)
        pairs = [(da_al, rda), (db_al, rdb), (da_un, rda), (db_un, rdb)]
    errs = [max_rel(g, r) for g, r in pairs]
    say(f"  loss rel {rel_err(l_al, rl):.2e} / {rel_err(l_un, rl):.2e}; grads {['%.2e' % e for e in errs]}")
    assert rel_err(l_al, rl) <= TOL_LOSS and rel_err(l_un, rl) <= TOL_LOSS
    assert all(e <= TOL_GRAD for e in errs)
    # the two cores sum the same products in different orders
    assert max_rel(da_al, da_un) < 1e-5


def test_f32_row_stride_beyond_the_direct_core_range():
    """A row stride of 2^23 floats puts a 128-row panel past the direct-to-LDS
    core's 2^31-byte range: the forward and gradient-matrix tiles then run on
    the register-staged core."""
    n, d, ld = 300, 64, 1 << 23
    a, b = randn_pair(n, d, seed=37)
    flat_a = torch.zeros((n - 1) * ld + d, device=DEV)
    flat_b = torch.zeros((n - 1) * ld + d, device=DEV)
    ga = flat_a.as_strided((n, d), (ld, 1))
    gb = flat_b.as_strided((n, d), (ld, 1))
    ga.copy_(a.to(DEV))
    gb.copy_(b.to(DEV))
    ga.requires_grad_(True)
    gb.requires_grad_(True)
    say(f"fp32 CLIP n={n} d={d} row stride {ld}")
    loss = MemoryEfficientCLIPLoss(0.07)(ga, gb)
    loss.backward()
    rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.07)
    ea, eb = max_rel(ga.grad.cpu(), rda), max_rel(gb.grad.cpu(), rdb)
    say(f"  loss rel {rel_err(loss.detach().cpu(), rl):.2e} grads {ea:.2e} {eb:.2e}")
    assert rel_err(loss.detach().cpu(), rl) <= TOL_LOSS
    assert ea <= TOL_GRAD and eb <= TOL_GRAD


def run_env(env, module, a, b, grad_b=True):
    """run() with the environment variables `env` set for the call."""
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return run(module, a, b, grad_b)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


@pytest.mark.parametrize("lit", [False, True], ids=["clip", "lit"])
@pytest.mark.parametrize("n,d", [(1024, 512), (1000, 130), (2900, 72), (63, 8), (4096, 128), (5120, 516)])
def test_f32_small_and_large_tiles(lit, n, d):
    """64 x 64 and 128 x 128 direct-to-LDS tiles (forward sums,
    gradient-matrix tiles, contractions) of the recomputing path agree with
    the oracle and with each other, below the 2816-row bound (where 64 x 64 is
    the default: config 1's shape, a ragged N, a tiny N) and above it (n =
    2900; 4096 with 1024-row backward blocks and 5120 with a poorly filled
    last round, where the backward's default is 64 x 64 again)."""
    a, b = randn_pair(n, d, seed=41 + n)
    mod = MemoryEfficientLiTLoss(0.07) if lit else MemoryEfficientCLIPLoss(0.07)
    say(f"fp32 {'LiT' if lit else 'CLIP'} n={n} d={d}: 64 x 64 vs 128 x 128 tiles")
    l_s, da_s, db_s = run_env({"MEC_F32_SMALL_TILES": "1", "MEC_KEEP_EXP": "0"}, mod, a, b, grad_b=not lit)
    l_l, da_l, db_l = run_env({"MEC_F32_SMALL_TILES": "0", "MEC_KEEP_EXP": "0"}, mod, a, b, grad_b=not lit)
    if lit:
        rl, rda = oracle.lit_loss_and_grads(a, b, 0.07)
        pairs = [(da_s, rda), (da_l, rda)]
    else:
        rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.07)
        pairs = [(da_s, rda), (db_s, rdb), (da_l, rda), (db_l, rdb)]
    errs = [max_rel(g, r) for g, r in pairs]
    say(f"  loss rel {rel_err(l_s, rl):.2e} / {rel_err(l_l, rl):.2e}; grads {['%.2e' % e for e in errs]}")
    assert rel_err(l_s, rl) <= TOL_LOSS and rel_err(l_l, rl) <= TOL_LOSS
    assert all(e <= TOL_GRAD for e in errs)
    # the same products summed in a different order
    assert rel_err(l_s, l_l) < 1e-5 and max_rel(da_s, da_l) < 1e-5


@pytest.mark.parametrize("n,d", [(4096, 128), (3072, 512), (6144, 64)])
def test_f32_default_tile_choice(n, d):
    """The default choice, where forward and backward differ: 128 x 128
    forward tiles with 64 x 64 backward tiles (n = 4096, 6144 at small D),
    64 x 64 for both (n = 3072, D = 512); against the oracle."""
    a, b = randn_pair(n, d, seed=43 + n)
    say(f"fp32 CLIP n={n} d={d}: default tiles")
    l, da, db = run_env({}, MemoryEfficientCLIPLoss(0.07), a, b)
    rl, rda, rdb = oracle.clip_loss_and_grads(a, b, 0.07)
    errs = [max_rel(da, rda), max_rel(db, rdb)]
    say(f"  loss rel {rel_err(l, rl):.2e}; grads {['%.2e' % e for e in errs]}")
    assert rel_err(l, rl) <= TOL_LOSS and all(e <= TOL_GRAD for e in errs)
