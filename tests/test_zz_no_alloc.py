"""mec_backward_noalloc (no caller scratch, no allocation: the scratch is a
file-scope device array) against mec_backward with caller scratch, through
the C ABI, on two calls in a row where the second has a smaller input (the
array keeps the first call's contents).  Every dtype family and both modes;
one shape where the array is too small for mec_backward's blocking, so the
no-allocation path takes shorter blocks (results then differ by rounding)."""
import pytest
import torch

from helpers import correlated_pair, max_rel, randn_pair, rel_err
from memoryefficientclip_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TDT = {_lib.DTYPE_F32: torch.float32, _lib.DTYPE_BF16: torch.bfloat16, _lib.DTYPE_F16: torch.float16}


def say(*a):
    print(*a, flush=True)


def backward_pair(a, b, dt, mode, normalize, t):
    """Forward once, then (dx, dy) from mec_backward and from mec_backward_noalloc."""
    x, y = a.to(DEV), b.to(DEV)
    n, d = x.shape
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    ws = torch.empty(lib.mec_workspace_floats_for(n, d, dt), device=DEV)
    loss = torch.empty((), device=DEV)
    _lib.call("mec_forward", x.data_ptr(), d, y.data_ptr(), d, n, d, dt, mode, normalize, t, ws.data_ptr(),
              loss.data_ptr(), st)
    clip = mode == _lib.MODE_CLIP
    fp32_data = dt in (_lib.DTYPE_F32, _lib.DTYPE_F32_BF16X3, _lib.DTYPE_F32_BF16)
    out = []
    for noalloc in (False, True):
        acc_x = torch.empty(n, d, device=DEV)
        acc_y = torch.empty(n, d, device=DEV) if clip else None
        if fp32_data:
            dx, dy = acc_x, acc_y
        else:
            dx = torch.empty(n, d, dtype=x.dtype, device=DEV)
            dy = torch.empty(n, d, dtype=x.dtype, device=DEV) if clip else None

        def p(v):
            return None if v is None else v.data_ptr()

        if noalloc:
            _lib.call("mec_backward_noalloc", x.data_ptr(), d, y.data_ptr(), d, n, d, dt, mode, normalize, t,
                      1.0 / t, ws.data_ptr(), None, p(acc_x), p(acc_y), p(dx), p(dy), st)
        else:
            nbytes = lib.mec_grad_scratch_bytes(n, d, dt)
            scratch = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
            _lib.call("mec_backward", x.data_ptr(), d, y.data_ptr(), d, n, d, dt, mode, normalize, t, 1.0 / t,
                      ws.data_ptr(), None, scratch.data_ptr(), nbytes, p(acc_x), p(acc_y), p(dx), p(dy), st)
        out.append((dx, dy))
    torch.cuda.synchronize()
    return out


CASES = [  # (dtype code, mode, normalize, generator)
    (_lib.DTYPE_F32, _lib.MODE_CLIP, 1, randn_pair),
    (_lib.DTYPE_F32, _lib.MODE_LIT, 1, randn_pair),
    (_lib.DTYPE_BF16, _lib.MODE_CLIP, 0, correlated_pair),
    (_lib.DTYPE_F16, _lib.MODE_CLIP, 1, randn_pair),
    (_lib.DTYPE_F32_BF16X3, _lib.MODE_CLIP, 1, randn_pair),
]


@pytest.mark.parametrize("dt,mode,normalize,gen", CASES, ids=["f32-clip", "f32-lit", "bf16-clip", "f16-clip",
                                                              "bf16x3-clip"])
def test_noalloc_matches_backward_twice(dt, mode, normalize, gen):
    for n, d, seed in [(3000, 256, 1), (1100, 72, 2)]:  # the second call is smaller
        tdt = TDT.get(dt, torch.float32)
        a, b = gen(n, d, seed=seed, dtype=tdt)
        say(f"noalloc dtype={dt} mode={mode} normalize={normalize} n={n} d={d}")
        (rx, ry), (gx, gy) = backward_pair(a, b, dt, mode, normalize, 0.07)
        ex = max_rel(gx.float(), rx.float())
        ey = 0.0 if ry is None else max_rel(gy.float(), ry.float())
        say(f"  vs mec_backward: dx max-rel {ex:.2e}, dy max-rel {ey:.2e}")
        # the same blocking (mec_backward's fits the array) and a deterministic
        # backward: the same numbers
        assert ex == 0.0 and ey == 0.0


def test_noalloc_shorter_blocks_when_the_array_is_small():
    """fp32, n = 16384, d = 2048: mec_backward's scratch (two 8192-row
    blocks, double-buffered: 1.07 GB) exceeds the 256 MiB array, so the
    no-allocation path runs 2048-row blocks; the gradients agree to fp32
    rounding (bar: 1e-3)."""
    n, d, t = 16384, 2048, 0.07
    bs, nb = _lib.grad_blocking(n, d, _lib.DTYPE_F32)
    assert _lib.load().mec_grad_scratch_bytes(n, d, _lib.DTYPE_F32) > _lib.NOALLOC_SCRATCH_BYTES and bs == 8192
    assert _lib.backward_plan(n, d, _lib.DTYPE_F32).noalloc_block_rows == 2048
    a, b = randn_pair(n, d, seed=3)
    say(f"noalloc f32 CLIP n={n} d={d}: default blocks {nb} x {bs}")
    (rx, ry), (gx, gy) = backward_pair(a, b, _lib.DTYPE_F32, _lib.MODE_CLIP, 1, t)
    ex, ey = max_rel(gx, rx), max_rel(gy, ry)
    say(f"  vs mec_backward: dx max-rel {ex:.2e}, dy max-rel {ey:.2e}")
    assert ex < 1e-5 and ey < 1e-5
    # and the smaller problem after it, back on the default blocking
    a, b = randn_pair(1000, 64, seed=4)
    (rx, ry), (gx, gy) = backward_pair(a, b, _lib.DTYPE_F32, _lib.MODE_CLIP, 1, t)
    assert max_rel(gx, rx) == 0.0 and max_rel(gy, ry) == 0.0
