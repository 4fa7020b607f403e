"""GPU parity of the 16-bit (bf16 and fp16) code paths, against the fp64 CPU
oracle on the same dtype-rounded inputs (tolerance 1e-2 on loss and gradient
max-rel).

16-bit inputs with 16-byte aligned rows (D and the row stride multiples of 8)
run on the direct-to-LDS core (256 x 256 forward tiles); other layouts on the
register-staged 128 x 128 core.  The backward always keeps only the transposed
gradient matrix: the y-side contraction reads it K-major, the x-side one (the
only side LiT has) through transposing LDS loads.  fp16 stores that matrix
scaled by 2^14, since its typical entries (~1/N) are fp16 subnormals from
N ~ 2^14 on.  Blocks are multiples of 256 rows, so N = 1300 / 2300 / 2500 give
two or three blocks with a short last one.
"""
import pytest
import torch

import oracle
from helpers import correlated_pair, max_rel, randn_pair, ref_fp64, rel_err
from memoryefficientclip_amd import _lib
from memoryefficientclip_amd.clip_loss import MemoryEfficientCLIPLoss
from memoryefficientclip_amd.lit_loss import MemoryEfficientLiTLoss

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-2
DTYPES = [torch.bfloat16, torch.float16]
ABI_DTYPE = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16}


def say(*a):
    print(*a, flush=True)


def grads_of(module, a, b, grad_b=True):
    ga = a.to(DEV).requires_grad_(True)
    gb = b.to(DEV).requires_grad_(grad_b)
    loss = module(ga, gb)
    loss.backward()
    torch.cuda.synchronize()
    return loss.detach().cpu(), ga.grad.cpu(), (gb.grad.cpu() if grad_b else None)


def check(name, loss, ref, pairs):
    msg = f"{name}: loss {float(loss):.6f} ref {float(ref):.6f} rel {rel_err(loss, ref):.2e}"
    errs = [max_rel(g, r) for _, g, r in pairs]
    msg += "".join(f" | {n} {e:.2e}" for (n, _, _), e in zip(pairs, errs))
    say(msg)
    assert rel_err(loss, ref) <= TOL, msg
    assert all(e <= TOL for e in errs), msg


def test_blocking_of_these_shapes():
    # the shapes below really exercise several backward blocks with a short last one
    for dt in ABI_DTYPE.values():
        for n, d in [(1300, 72), (2300, 96), (2500, 72), (2300, 64)]:
            bs, nb = _lib.grad_blocking(n, d, dt)
            assert nb >= 2 and nb * bs > n, (n, d, bs, nb)


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "f16"])
@pytest.mark.parametrize("n,d,normed", [(2300, 96, False), (2500, 72, True), (1300, 200, False)])
def test_16bit_clip_multiblock(n, d, normed, dtype):
    if normed:
        a, b = correlated_pair(n, d, seed=n + d, dtype=dtype)
    else:
        a, b = randn_pair(n, d, seed=n + d, dtype=dtype)
    say(f"{dtype} CLIP n={n} d={d} normalized_inputs={normed}")
    loss, da, db = grads_of(MemoryEfficientCLIPLoss(0.07, normed), a, b)
    rl, rda, rdb = oracle.clip_loss_and_grads(a.float(), b.float(), 0.07, normalized_inputs=normed)
    check(f"{dtype} clip n={n} d={d}", loss, rl, [("d_img", da, rda), ("d_txt", db, rdb)])
    assert da.dtype == dtype and db.dtype == dtype


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "f16"])
@pytest.mark.parametrize("n,d,normed", [(2300, 64, False), (1300, 72, True), (777, 1152, False)])
def test_16bit_lit(n, d, normed, dtype):
    if normed:
        txt, img = correlated_pair(n, d, seed=7 * n + d, dtype=dtype)
    else:
        txt, img = randn_pair(n, d, seed=7 * n + d, dtype=dtype)
    say(f"{dtype} LiT n={n} d={d} normalized_inputs={normed} (image frozen)")
    loss, dt, _ = grads_of(MemoryEfficientLiTLoss(0.07, normed), txt, img, grad_b=False)
    rl, rdt = oracle.lit_loss_and_grads(txt.float(), img.float(), 0.07, normalized_inputs=normed)
    check(f"{dtype} lit n={n} d={d}", loss, rl, [("d_text", dt, rdt)])


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "f16"])
@pytest.mark.parametrize("width,off,label", [(136, 8, "16-byte aligned rows (direct-to-LDS core)"),
                                              (101, 3, "unaligned rows (register-staged core)")])
def test_16bit_row_strided(width, off, label, dtype):
    n, d = 1300, 96
    a, b = randn_pair(n, d, seed=99, dtype=dtype)
    wa = torch.zeros(n, width, dtype=dtype)
    wb = torch.zeros(n, width, dtype=dtype)
    wa[:, off:off + d] = a
    wb[:, off:off + d] = b
    ga = wa.to(DEV)[:, off:off + d].requires_grad_(True)
    gb = wb.to(DEV)[:, off:off + d].requires_grad_(True)
    say(f"{dtype} row-strided n={n} d={d} ld={width}: {label}")
    loss = MemoryEfficientCLIPLoss(0.07)(ga, gb)
    loss.backward()
    rl, rda, rdb = oracle.clip_loss_and_grads(a.float(), b.float(), 0.07)
    check(f"{dtype} strided ld={width}", loss.detach().cpu(), rl,
          [("d_img", ga.grad.cpu(), rda), ("d_txt", gb.grad.cpu(), rdb)])


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "f16"])
@pytest.mark.parametrize("mode", [_lib.MODE_CLIP, _lib.MODE_LIT])
def test_16bit_contractions_through_abi(mode, dtype):
    """mec_grad on 16-bit inputs against the oracle's off-diagonal contractions
    (the gradient matrix is rounded to the input dtype before its MFMAs)."""
    n, d, t = 1300, 72, 0.07
    a, b = randn_pair(n, d, seed=5 + mode, dtype=dtype)
    x, y = a.to(DEV), b.to(DEV)
    dt = ABI_DTYPE[dtype]
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    ws = torch.empty(lib.mec_workspace_floats(n), device=DEV)
    loss = torch.empty((), device=DEV)
    say(f"{dtype} ABI contractions mode={mode} n={n} d={d}")
    _lib.call("mec_forward", x.data_ptr(), d, y.data_ptr(), d, n, d, dt, mode, 1, t, ws.data_ptr(),
              loss.data_ptr(), st)
    nbytes = lib.mec_grad_scratch_bytes(n, d, dt)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    acc_x = torch.empty(n, d, device=DEV)
    acc_y = torch.empty(n, d, device=DEV) if mode == _lib.MODE_CLIP else None
    _lib.call("mec_grad", x.data_ptr(), d, y.data_ptr(), d, n, d, dt, mode, 1, t, ws.data_ptr(),
              scratch.data_ptr(), nbytes, acc_x.data_ptr(), None if acc_y is None else acc_y.data_ptr(), st)
    torch.cuda.synchronize()
    xh, yh = oracle.normalize(a.float()), oracle.normalize(b.float())
    s, e, r, c = oracle.similarity_sums(xh, yh, t)
    off = 1.0 - torch.eye(n, dtype=torch.float64)
    gp = e * (1 / r)[:, None] * off
    if mode == _lib.MODE_CLIP:
        gp = gp + e * (1 / c)[None, :] * off
        ey = max_rel(acc_y.cpu(), gp.T @ xh)
        say(f"  acc_y max-rel {ey:.2e}")
        assert ey < TOL
    ex = max_rel(acc_x.cpu(), gp @ yh)
    say(f"  acc_x max-rel {ex:.2e}")
    assert ex < TOL


def test_f16_clip_large_n():
    """fp16 CLIP at N = 20000 against the dense definition in fp64, chunked
    over rows on the GPU (the same fp16-rounded inputs)."""
    n, d, t = 20000, 64, 0.07
    a, b = correlated_pair(n, d, seed=11, dtype=torch.float16)
    say(f"fp16 CLIP n={n} d={d}")
    loss, da, db = grads_of(MemoryEfficientCLIPLoss(t, True), a, b)
    rl, rda, rdb = ref_fp64(a.to(DEV), b.to(DEV), t, False, True, 4096)
    check(f"fp16 clip n={n}", loss, rl.cpu(), [("d_img", da, rda.cpu()), ("d_txt", db, rdb.cpu())])


def test_f16_tiny_gradient_matrix_entries():
    """fp16 with y_i = x_i, D = 512 and T = 0.05: E_ii = 1 dominates every row
    and column sum, and the typical off-diagonal gradient-matrix entry
    E_ij (1/R_i + 1/C_j) is ~4e-9, below half the smallest fp16 subnormal
    (3e-8).  Stored unscaled, most entries would flush to zero (rounding G' to
    fp16 this way gives a max-rel error of 0.71 on the contraction, emulated
    on the CPU); the 2^14 storage scale keeps them normal (1.2e-4)."""
    n, d, t = 4096, 512, 0.05
    g = torch.Generator().manual_seed(21)
    a = torch.nn.functional.normalize(torch.randn(n, d, generator=g), dim=1).to(torch.float16)
    x = a.to(DEV)
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    ws = torch.empty(lib.mec_workspace_floats(n), device=DEV)
    loss = torch.empty((), device=DEV)
    say(f"fp16 ABI contractions, y = x, T = {t}, n={n} d={d}")
    _lib.call("mec_forward", x.data_ptr(), d, x.data_ptr(), d, n, d, _lib.DTYPE_F16, _lib.MODE_CLIP, 0, t,
              ws.data_ptr(), loss.data_ptr(), st)
    nbytes = lib.mec_grad_scratch_bytes(n, d, _lib.DTYPE_F16)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    acc_x = torch.empty(n, d, device=DEV)
    acc_y = torch.empty(n, d, device=DEV)
    _lib.call("mec_grad", x.data_ptr(), d, x.data_ptr(), d, n, d, _lib.DTYPE_F16, _lib.MODE_CLIP, 0, t,
              ws.data_ptr(), scratch.data_ptr(), nbytes, acc_x.data_ptr(), acc_y.data_ptr(), st)
    torch.cuda.synchronize()
    xh = a.double()
    s, e, r, c = oracle.similarity_sums(xh, xh, t)
    offd = ~torch.eye(n, dtype=torch.bool)
    gp = (e * (1 / r)[:, None] + e * (1 / c)[None, :]) * offd
    med = float(gp[offd].median())
    assert med < 1.5e-8, "the case must put the typical entry below the fp16 subnormal range"
    ex, ey = max_rel(acc_x.cpu(), gp @ xh), max_rel(acc_y.cpu(), gp.T @ xh)
    say(f"  median entry {med:.2e}; acc_x max-rel {ex:.2e} acc_y max-rel {ey:.2e}")
    assert ex < TOL and ey < TOL


def test_bf16_large_d_caps_the_block_size():
    """D = 4352: the ~8D-row block target (34816 rows) would make a transposed
    gradient-matrix block exceed the direct-to-LDS core's 2^31-byte operand
    range; the blocking caps it (here: two blocks of 16640 rows).  Reference:
    the dense definition in fp64, chunked over rows on the GPU."""
    n, d, t = 33000, 4352, 0.07
    bs, nb = _lib.grad_blocking(n, d, _lib.DTYPE_BF16)
    assert bs <= 32512 and nb >= 2, (bs, nb)
    a, b = correlated_pair(n, d, seed=17, dtype=torch.bfloat16)
    say(f"bf16 CLIP n={n} d={d} blocks {nb} x {bs}")
    loss, da, db = grads_of(MemoryEfficientCLIPLoss(t, True), a, b)
    rl, rda, rdb = ref_fp64(a.to(DEV), b.to(DEV), t, False, True, 2048)
    check(f"bf16 clip n={n} d={d}", loss, rl.cpu(), [("d_img", da, rda.cpu()), ("d_txt", db, rdb.cpu())])


def test_bf16_row_stride_beyond_the_direct_core_range():
    """A row stride of 2^23 elements puts a 256-row panel past the direct-to-LDS
    core's 2^31-byte range: such inputs run on the register-staged core."""
    n, d, ld = 300, 64, 1 << 23
    # rows of width d at stride ld inside one flat buffer per input (5 GB each)
    a, b = randn_pair(n, d, seed=23, dtype=torch.bfloat16)
    flat_a = torch.zeros((n - 1) * ld + d, dtype=torch.bfloat16, device=DEV)
    flat_b = torch.zeros((n - 1) * ld + d, dtype=torch.bfloat16, device=DEV)
    ga = flat_a.as_strided((n, d), (ld, 1))
    gb = flat_b.as_strided((n, d), (ld, 1))
    ga.copy_(a.to(DEV))
    gb.copy_(b.to(DEV))
    ga.requires_grad_(True)
    gb.requires_grad_(True)
    say(f"bf16 CLIP n={n} d={d} row stride {ld}")
    loss = MemoryEfficientCLIPLoss(0.07)(ga, gb)
    loss.backward()
    rl, rda, rdb = oracle.clip_loss_and_grads(a.float(), b.float(), 0.07)
    check(f"bf16 stride {ld}", loss.detach().cpu(), rl,
          [("d_img", ga.grad.cpu(), rda), ("d_txt", gb.grad.cpu(), rdb)])
