"""Parity at the benchmark's full sizes (all five configurations).

The fp64 CPU oracle cannot evaluate N = 32768..262144 in seconds, so the
reference here is the same dense definition evaluated with PyTorch's fp64
GEMMs on the GPU, chunked over rows (an independent library route: cuBLAS-
style fp64 matmul, exp, log, sums; none of this package's kernels).  It
follows the loss and gradient definition of the reference (clip_loss.py:
206-211, 235-249; lit_loss.py:199-203, 227-241) and F.normalize's backward.

Size-independent properties are checked on the same outputs:
* with the normalisation fused, each input row's gradient is orthogonal to the
  row (the loss is invariant to rescaling a row);
* CLIP is symmetric: swapping image and text swaps the gradients.

Tolerances: fp32 loss rel 1e-4 / gradient max-rel 1e-3, bf16 1e-2.
"""
import math

import pytest
import torch

from helpers import TOL, correlated_pair, max_rel, randn_pair, ref_fp64, rel_err
from memoryefficientclip_amd import MemoryEfficientCLIPLoss, MemoryEfficientLiTLoss

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# name -> (mode, n, d, dtype, normalized_inputs, temperature, generator); the
# benchmark table, same generators as bench.py, seed 0
CONFIGS = {
    "c1_clip_1024x512_f32": ("clip", 1024, 512, torch.float32, False, 0.07, "randn"),
    "c2_clip_32768x1152_f32": ("clip", 32768, 1152, torch.float32, False, 0.07, "randn"),
    "c3_lit_32768x1152_f32": ("lit", 32768, 1152, torch.float32, False, 0.07, "randn"),
    "c4_clip_65536x768_bf16": ("clip", 65536, 768, torch.bfloat16, True, 0.07, "correlated"),
    "c5_clip_262144x1152_bf16": ("clip", 262144, 1152, torch.bfloat16, True, 0.05, "correlated"),
}


def say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("name", list(CONFIGS))
def test_full_size_against_fp64(name):
    mode, n, d, dtype, normalized, t, gen = CONFIGS[name]
    lit = mode == "lit"
    say(f"full-size {name}: n={n} d={d} {dtype} normalized_inputs={normalized} T={t}")
    a, b = randn_pair(n, d, seed=0) if gen == "randn" else correlated_pair(n, d, seed=0, dtype=torch.float32)
    ga = a.to(DEV, dtype).requires_grad_(True)
    gb = b.to(DEV, dtype).requires_grad_(not lit)
    del a, b
    mod = (MemoryEfficientLiTLoss if lit else MemoryEfficientCLIPLoss)(t, normalized)
    loss = mod(ga, gb)
    loss.backward()
    torch.cuda.synchronize()
    chunk = max(256, min(n, (1 << 28) // n))  # ~2 GiB of fp64 per S chunk
    ref_loss, ref_da, ref_db = ref_fp64(ga.detach(), gb.detach(), t, lit, normalized, chunk)
    tol = TOL[dtype]
    le = rel_err(loss.item(), ref_loss.item())
    ea = max_rel(ga.grad, ref_da)
    msg = f"{name}: loss {loss.item():.7f} ref {ref_loss.item():.7f} rel {le:.2e} | d_a max-rel {ea:.2e}"
    eb = 0.0
    if not lit:
        eb = max_rel(gb.grad, ref_db)
        msg += f" | d_b max-rel {eb:.2e}"
    say(msg)
    assert le <= tol["loss"] and ea <= tol["grad"] and eb <= tol["grad"], msg
    if not normalized:
        # the gradient through the normalisation is orthogonal to each input row
        x = ga.detach().double()
        gx = ga.grad.double()
        cos = ((gx * x).sum(dim=1).abs() / (gx.norm(dim=1) * x.norm(dim=1)).clamp_min(1e-30)).max().item()
        say(f"{name}: max |cos(grad_i, x_i)| = {cos:.2e}")
        assert cos < 10 * tol["grad"], cos


def test_full_size_clip_symmetry():
    """CLIP(x, y) == CLIP(y, x) with the gradients swapped, at the headline shape."""
    n, d = 32768, 1152
    a, b = randn_pair(n, d, seed=5)
    say(f"symmetry n={n} d={d}")
    mod = MemoryEfficientCLIPLoss(0.07)
    outs = []
    for p, q in [(a, b), (b, a)]:
        gp = p.to(DEV).requires_grad_(True)
        gq = q.to(DEV).requires_grad_(True)
        loss = mod(gp, gq)
        loss.backward()
        outs.append((loss.item(), gp.grad, gq.grad))
    (l1, da1, db1), (l2, da2, db2) = outs
    say(f"symmetry: loss {l1:.7f} vs {l2:.7f}; grads {max_rel(da1, db2):.2e}, {max_rel(db1, da2):.2e}")
    assert rel_err(l1, l2) < 1e-5
    assert max_rel(da1, db2) < 1e-4 and max_rel(db1, da2) < 1e-4
    assert math.isfinite(l1)


@pytest.mark.parametrize("lit", [False, True], ids=["clip", "lit"])
def test_stable_variant_at_config5_scale(lit):
    """The Stable modules at config 5's shape (N = 262144, D = 1152, bf16,
    normalized inputs, T = 0.05), the scale the reference's docstring claims
    for them ("300k+ works just fine", clip_loss.py:380, lit_loss.py:369):
    the same loss as the standard module, and gradients sqrt(N T) times the
    standard ones (grad scale sqrt(N/T) in place of 1/T, clip_loss.py:299,
    lit_loss.py:289).  Both gradients are rounded to bf16 (unit roundoff
    2^-8), so they may differ by 2^-7 of an element: bar 1e-2 of the largest."""
    from memoryefficientclip_amd import StableMemoryEfficientCLIPLoss, StableMemoryEfficientLiTLoss
    n, d, t = 262144, 1152, 0.05
    a, b = correlated_pair(n, d, seed=0, dtype=torch.float32)
    say(f"Stable {'LiT' if lit else 'CLIP'} at n={n} d={d} bf16 T={t}")
    out = []
    for cls in ((MemoryEfficientLiTLoss, StableMemoryEfficientLiTLoss) if lit else
                (MemoryEfficientCLIPLoss, StableMemoryEfficientCLIPLoss)):
        ga = a.to(DEV, torch.bfloat16).requires_grad_(True)
        gb = b.to(DEV, torch.bfloat16).requires_grad_(not lit)
        loss = cls(t, True)(ga, gb)
        loss.backward()
        torch.cuda.synchronize()
        out.append((loss.item(), ga.grad.float(), None if lit else gb.grad.float()))
        del ga, gb
    (l0, da0, db0), (l1, da1, db1) = out
    s = math.sqrt(n * t)
    le = rel_err(l1, l0)
    ea = max_rel(da1, s * da0)
    eb = 0.0 if lit else max_rel(db1, s * db0)
    say(f"  loss {l0:.6f} vs {l1:.6f} (rel {le:.1e}); grads vs sqrt(N T) x standard: {ea:.2e} {eb:.2e}")
    assert le < 1e-6 and ea < 1e-2 and eb < 1e-2
    assert da1.abs().max() > 100 * da0.abs().max()  # the scale is applied (sqrt(N T) = 114.5)
