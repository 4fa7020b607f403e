"""GPU tests of the deterministic forward (MEC_FLAG_DETERMINISTIC, enabled from
Python by torch.use_deterministic_algorithms(True)).

The default forward adds each tile's row and column sums into the workspace
with relaxed fp32 atomics (as the reference does, clip_loss.py:63-64), so the
loss may differ in its last bits between runs.  The deterministic forward
walks the tile grid in P x Q blocks (one workgroup each, tiles in order),
keeps one row partial per column block and one column partial per row block,
and adds those partials in a fixed order.  Checked here:

* the sums and the loss agree with the fp64 oracle, and with the atomic path;
* repeated runs are bitwise identical (sums, loss, and through the module the
  gradients);
* shapes with fewer tiles than blocks (the block counts clamp to the tile
  counts), blocks of uneven tile counts (6000 rows: 47 fp32 tiles over 32 row
  blocks), ragged N, all three dtypes, both modes, fused normalisation on and
  off.
"""
import pytest
import torch

import oracle
from helpers import max_rel, randn_pair, rel_err
from memoryefficientclip_amd import _lib
from memoryefficientclip_amd.clip_loss import MemoryEfficientCLIPLoss
from memoryefficientclip_amd.lit_loss import MemoryEfficientLiTLoss

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ABI = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16}
WS_ROW_OFF, WS_COL_OFF = 3, 4


def say(*a):
    print(*a, flush=True)


def forward_abi(x, y, n, d, dt, mode, normalize, t):
    lib = _lib.load()
    ws = torch.empty(lib.mec_workspace_floats(n), device=DEV)
    loss = torch.empty((), device=DEV)
    _lib.call("mec_forward", x.data_ptr(), d, y.data_ptr(), d, n, d, dt, mode, normalize, t, ws.data_ptr(),
              loss.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    sums = ws[:8 * n].view(8, n)
    return loss.cpu(), sums[WS_ROW_OFF].cpu().clone(), sums[WS_COL_OFF].cpu().clone()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("mode", [_lib.MODE_CLIP, _lib.MODE_LIT], ids=["clip", "lit"])
@pytest.mark.parametrize("n,d,normalize", [(1, 8, 1), (2, 24, 1), (300, 64, 0), (777, 37, 1), (2500, 96, 1),
                                           (6000, 40, 1)])
def test_deterministic_sums(n, d, normalize, mode, dtype):
    a, b = randn_pair(n, d, seed=n + 7 * d)
    if not normalize:  # the kernels take the inputs as unit rows
        a, b = torch.nn.functional.normalize(a, dim=1), torch.nn.functional.normalize(b, dim=1)
    a, b = a.to(dtype), b.to(dtype)
    x, y = a.to(DEV), b.to(DEV)
    dt = ABI[dtype]
    t = 0.07
    say(f"deterministic forward {dtype} mode={mode} n={n} d={d} normalize={normalize}")
    flag = mode | _lib.FLAG_DETERMINISTIC
    l1, r1, c1 = forward_abi(x, y, n, d, dt, flag, normalize, t)
    l2, r2, c2 = forward_abi(x, y, n, d, dt, flag, normalize, t)
    la, ra, ca = forward_abi(x, y, n, d, dt, mode, normalize, t)
    # bitwise reproducible
    assert torch.equal(l1, l2) and torch.equal(r1, r2)
    if mode == _lib.MODE_CLIP:
        assert torch.equal(c1, c2)
    # the oracle's off-diagonal sums on the same (dtype-rounded) inputs
    xh = oracle.normalize(a.float()) if normalize else a.double()
    yh = oracle.normalize(b.float()) if normalize else b.double()
    s, e, r, c = oracle.similarity_sums(xh, yh, t)
    de = torch.diagonal(e)
    ref_r, ref_c = r - de, c - de
    if n > 1:
        er = max_rel(r1, ref_r)
        ec = max_rel(c1, ref_c) if mode == _lib.MODE_CLIP else 0.0
        say(f"  sums max-rel vs oracle: rows {er:.2e} cols {ec:.2e}; vs atomic path rows {max_rel(r1, ra):.2e}")
        assert er < 1e-4 and ec < 1e-4
        assert max_rel(r1, ra) < 1e-5
        if mode == _lib.MODE_CLIP:
            assert max_rel(c1, ca) < 1e-5
    else:
        assert float(r1[0]) == 0.0
    ref_loss = (oracle.clip_forward if mode == _lib.MODE_CLIP else oracle.lit_forward)(xh, yh, t)
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    assert rel_err(l1, ref_loss) <= tol or abs(float(l1) - float(ref_loss)) < 1e-6
    assert rel_err(l1, la) < 1e-5 or abs(float(l1) - float(la)) < 1e-6


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("lit", [False, True], ids=["clip", "lit"])
def test_module_bitwise_reproducible_under_torch_deterministic(dtype, lit):
    n, d = 3000, 128
    a, b = randn_pair(n, d, seed=5, dtype=dtype)
    prev = torch.are_deterministic_algorithms_enabled()
    prev_warn = torch.is_deterministic_algorithms_warn_only_enabled()
    say(f"module under torch.use_deterministic_algorithms(True): {dtype} {'LiT' if lit else 'CLIP'} n={n} d={d}")
    runs = []
    try:
        torch.use_deterministic_algorithms(True, warn_only=True)
        for _ in range(3):
            ga = a.to(DEV).requires_grad_(True)
            gb = b.to(DEV).requires_grad_(not lit)
            mod = MemoryEfficientLiTLoss(0.07) if lit else MemoryEfficientCLIPLoss(0.07)
            loss = mod(ga, gb)
            loss.backward()
            torch.cuda.synchronize()
            runs.append((loss.detach().cpu(), ga.grad.cpu(), None if lit else gb.grad.cpu()))
    finally:
        torch.use_deterministic_algorithms(prev, warn_only=prev_warn)
    for other in runs[1:]:
        assert torch.equal(runs[0][0], other[0])
        assert torch.equal(runs[0][1], other[1])
        if not lit:
            assert torch.equal(runs[0][2], other[2])
    if lit:
        rl, rda = oracle.lit_loss_and_grads(a.float(), b.float(), 0.07)
        pairs = [(runs[0][1], rda)]
    else:
        rl, rda, rdb = oracle.clip_loss_and_grads(a.float(), b.float(), 0.07)
        pairs = [(runs[0][1], rda), (runs[0][2], rdb)]
    tol = (1e-4, 1e-3) if dtype == torch.float32 else (1e-2, 1e-2)
    errs = [max_rel(g, r) for g, r in pairs]
    say(f"  loss rel {rel_err(runs[0][0], rl):.2e}, grads {['%.2e' % e for e in errs]}")
    assert rel_err(runs[0][0], rl) <= tol[0]
    assert all(e <= tol[1] for e in errs)
