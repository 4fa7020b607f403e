"""The 16-bit forward on pre-normalised inputs runs k_sumexp_det with chained
tiles: the tile grid is cut into P x Q blocks (at most 32 x 16), one
workgroup walks each block's tiles in order (row tiles outer), and the last
k-chunk of each tile loads the first chunk of the next.  Row sums stay in a
register across a block's column tiles; column sums are added to the row
block's partial after every tile.  These shapes give blocks of one and of
several row and column tiles, uneven block sizes, ragged edges, and k-loops of
one chunk (D <= 64, where the first chunk is also the last) and of several.

* The row and column sums (workspace slots 3 and 4 after mec_sumexp) against
  the fp64 oracle's off-diagonal sums on the same bf16/fp16-rounded inputs.
  A tile visited twice or missed would move the sums of its 256 rows by about
  256 / N of their value, far above the 1e-4 allowed.  The sums are the same
  with and without MEC_FLAG_DETERMINISTIC (one kernel serves both) and
  bitwise identical run to run.
* Loss and gradients through the module against the fp64 oracle at the
  16-bit tolerances.
"""
import pytest
import torch

import oracle
from helpers import TOL, max_rel, rel_err
from memoryefficientclip_amd import _lib
from memoryefficientclip_amd.clip_loss import MemoryEfficientCLIPLoss
from memoryefficientclip_amd.lit_loss import MemoryEfficientLiTLoss

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
WS_ROW_OFF, WS_COL_OFF = 3, 4

CASES = [
    # (dtype, mode, n, d)
    (torch.bfloat16, "clip", 5000, 40),    # 20 x 20 tiles, one k-chunk: blocks of 1 x 1-2 tiles
    (torch.bfloat16, "lit", 4700, 200),    # 19 x 19 tiles, ragged, 4 chunks
    (torch.float16, "clip", 6000, 128),    # 24 x 24 tiles
    (torch.bfloat16, "clip", 8192, 64),    # 32 x 32 tiles, exact edges: blocks of 1 x 2 tiles
    (torch.bfloat16, "clip", 4400, 264),   # last chunk partial
    (torch.bfloat16, "clip", 12000, 40),   # 47 x 47 tiles: blocks of 1-2 x 2-3 tiles, uneven
    (torch.bfloat16, "lit", 12000, 72),    # the same, row sums only
]


def say(*a):
    print(*a, flush=True)


def normed_pair(n, d, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    a = torch.nn.functional.normalize(torch.randn(n, d, generator=g), dim=1)
    b = torch.nn.functional.normalize(a + 0.5 * torch.randn(n, d, generator=g), dim=1)
    return a.to(dtype), b.to(dtype)


def sums(x, y, dtype_code, mode):
    n, d = x.shape
    lib = _lib.load()
    ws = torch.zeros(lib.mec_workspace_floats(n), dtype=torch.float32, device=DEV)
    s = torch.cuda.current_stream().cuda_stream
    _lib.call("mec_prepass", x.data_ptr(), d, y.data_ptr(), d, n, d, dtype_code, 0, ws.data_ptr(), s)
    _lib.call("mec_sumexp", x.data_ptr(), d, y.data_ptr(), d, n, d, dtype_code, mode, 0, 0.07, ws.data_ptr(), s)
    torch.cuda.synchronize()
    return ws[WS_ROW_OFF * n:(WS_ROW_OFF + 1) * n].cpu(), ws[WS_COL_OFF * n:(WS_COL_OFF + 1) * n].cpu()


@pytest.mark.parametrize("dtype,mode,n,d", CASES, ids=[f"{c[1]}-{c[2]}x{c[3]}-{str(c[0])[6:]}" for c in CASES])
def test_chained_sums_against_the_oracle(dtype, mode, n, d):
    a, b = normed_pair(n, d, seed=n + d, dtype=dtype)
    x, y = a.to(DEV), b.to(DEV)
    code = _lib.DTYPE_BF16 if dtype == torch.bfloat16 else _lib.DTYPE_F16
    m = _lib.MODE_LIT if mode == "lit" else _lib.MODE_CLIP
    say(f"chained sums {mode} n={n} d={d} {dtype}")
    r1, c1 = sums(x, y, code, m)
    r2, c2 = sums(x, y, code, m)
    r_det, c_det = sums(x, y, code, m | _lib.FLAG_DETERMINISTIC)
    assert torch.equal(r1, r2) and torch.equal(r1, r_det)
    _, e, r, c = oracle.similarity_sums(a.double(), b.double(), 0.07)
    de = torch.diagonal(e)
    er = max_rel(r1, r - de)
    say(f"  row sums max-rel vs oracle {er:.2e}")
    assert er <= 1e-4
    if mode == "clip":
        assert torch.equal(c1, c2) and torch.equal(c1, c_det)
        ec = max_rel(c1, c - de)
        say(f"  column sums max-rel vs oracle {ec:.2e}")
        assert ec <= 1e-4


@pytest.mark.parametrize("dtype,mode,n,d", CASES, ids=[f"{c[1]}-{c[2]}x{c[3]}-{str(c[0])[6:]}" for c in CASES])
def test_chained_forward_against_the_oracle(dtype, mode, n, d):
    a, b = normed_pair(n, d, seed=7 * n + d, dtype=dtype)
    lit = mode == "lit"
    say(f"chained forward + backward {mode} n={n} d={d} {dtype}")
    ga = a.to(DEV).requires_grad_(True)
    gb = b.to(DEV).requires_grad_(not lit)
    mod = MemoryEfficientLiTLoss(0.07, normalized_inputs=True) if lit else MemoryEfficientCLIPLoss(0.07, True)
    loss = mod(ga, gb)
    loss.backward()
    torch.cuda.synchronize()
    tol = TOL[dtype]
    if lit:
        rl, rda = oracle.lit_loss_and_grads(a.float(), b.float(), 0.07, normalized_inputs=True)
        grads = [(ga.grad, rda)]
    else:
        rl, rda, rdb = oracle.clip_loss_and_grads(a.float(), b.float(), 0.07, normalized_inputs=True)
        grads = [(ga.grad, rda), (gb.grad, rdb)]
    le = rel_err(loss.detach().cpu(), rl)
    ge = [max_rel(g.float().cpu(), r) for g, r in grads]
    say(f"  loss rel {le:.2e}, grads {ge}")
    assert le <= tol["loss"] and all(e <= tol["grad"] for e in ge)
