"""Host side of the contrastive-loss hot path: argument checks, buffer
allocation and the calls into the HIP library (``include/mec.h``).

This mirrors the glue of the reference's autograd Functions
(``clip_loss.py:159-256``, ``lit_loss.py:151-247``): the same inputs, the same
0-d fp32 loss, the same gradients.  Differences by design:

* the loss epilogue, the gradient initialisation and ``grad_output`` scaling
  run in HIP kernels (no PyTorch epilogue ops, no host sync on
  ``grad_output != 1``, ``clip_loss.py:252``);
* the optional L2 normalisation is fused (``normalize=True``) instead of
  running ``F.normalize`` (``clip_loss.py:266-268``) as separate PyTorch ops;
* any N >= 1 and D >= 1 is accepted, with exact masking of ragged tiles, and
  inputs with a row stride are read in place (no ``.contiguous()`` copy);
* under ``torch.use_deterministic_algorithms(True)`` the loss and gradients
  are bitwise reproducible (the reference's relaxed atomics are not,
  ``clip_loss.py:63-64,155-156``);
* fp32 inputs follow ``torch.get_float32_matmul_precision()``: "highest" (the
  default) multiplies in IEEE fp32 on the fp32 MFMA; "high" forms each product
  from bf16 terms (hi*hi + lo*hi + hi*lo, about 16 significant bits per
  operand) on the bf16 MFMA and keeps the fp32 tolerances; "medium" multiplies
  bf16-rounded values (the bf16 tolerances).  These are PyTorch's meanings of
  the three settings.  The reference's fp32 dot products are TF32 on NVIDIA
  (``tl.dot`` without ``input_precision``, ``clip_loss.py:53,113,148-149``).
"""
from __future__ import annotations

import math

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16}


def check_inputs(x: torch.Tensor, y: torch.Tensor) -> None:
    """Argument checks; AssertionError where the reference asserts
    (``clip_loss.py:166-167``), TypeError/ValueError for the rest."""
    if not (isinstance(x, torch.Tensor) and isinstance(y, torch.Tensor)):
        raise TypeError("features must be torch.Tensor")
    if not (x.is_cuda and y.is_cuda):
        raise AssertionError("MemoryEfficientCLIP: inputs must be GPU tensors (x.is_cuda and y.is_cuda)")
    if x.shape != y.shape:
        raise AssertionError(f"MemoryEfficientCLIP: shape mismatch {tuple(x.shape)} vs {tuple(y.shape)}")
    if x.dim() != 2:
        raise ValueError(f"features must be 2-D [batch, dim], got {x.dim()}-D")
    if x.shape[0] < 1 or x.shape[1] < 1:
        raise ValueError("features must have batch >= 1 and dim >= 1")
    if x.dtype != y.dtype:
        raise TypeError(f"dtype mismatch {x.dtype} vs {y.dtype}")
    if x.dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {x.dtype}; supported: float32, bfloat16, float16")
    if x.device != y.device:
        raise ValueError(f"inputs on different devices {x.device} vs {y.device}")


def _rows(t: torch.Tensor) -> tuple[torch.Tensor, int]:
    """Tensor with unit column stride and its row stride (elements)."""
    if t.stride(1) != 1 or t.stride(0) < t.shape[1]:
        t = t.contiguous()
    return t, t.stride(0)


# the current stream's handle without building a torch.cuda.Stream object
# (about 2 us of host time per call at N = 1024, where the step is host-bound)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(index: int) -> int:
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


class _on_device:
    """Make device `index` current for the C-ABI calls (which launch on the
    current device), restoring the previous one; nothing to do, and no
    device switch, in the common case where it already is."""

    __slots__ = ("index", "prev")

    def __init__(self, index: int):
        self.index = index
        self.prev = -1

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.index:
            self.prev = cur
            torch.cuda.set_device(self.index)
        return self

    def __exit__(self, *exc):
        if self.prev >= 0:
            torch.cuda.set_device(self.prev)
        return False


def refuse_graph_capture() -> None:
    """Raise instead of enqueueing work into a CUDA/HIP graph capture.

    Capturing a step that calls this loss ended in a host segmentation fault
    inside ``torch.cuda.graph``'s ``capture_end`` on the MI355X box, with no
    cause found in this library's launches; a clear error is better than a
    crashed training process."""
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("MemoryEfficientCLIP: the fused loss does not support CUDA/HIP graph capture; "
                           "call it outside the captured region")


def compute_dtype(dtype: torch.dtype) -> int:
    """C-ABI dtype code for inputs of `dtype` under the current
    ``torch.get_float32_matmul_precision()`` (fp32 only: "high" selects the
    three-term bf16 products, "medium" plain bf16 products)."""
    code = _DTYPES[dtype]
    if code == _lib.DTYPE_F32:
        p = torch.get_float32_matmul_precision()
        if p == "high":
            return _lib.DTYPE_F32_BF16X3
        if p == "medium":
            return _lib.DTYPE_F32_BF16
    return code


def forward(ctx, x: torch.Tensor, y: torch.Tensor, temperature: float, mode: int, normalize: bool,
            stable: bool) -> torch.Tensor:
    check_inputs(x, y)
    refuse_graph_capture()
    temperature = float(temperature)
    if not (temperature > 0.0 and math.isfinite(temperature)):
        raise ValueError(f"temperature must be finite and > 0, got {temperature}")
    x, ldx = _rows(x)
    y, ldy = _rows(y)
    n, d = x.shape
    dev = x.device
    di = x.get_device()
    dt = compute_dtype(x.dtype)
    lib = _lib.load()
    # small fp32 problems keep the similarity matrix for the backward (three
    # launches per step instead of six, no gradient scratch), when a gradient
    # will be asked for
    if (ctx.needs_input_grad[0] or ctx.needs_input_grad[1]) and \
            lib.mec_keep_exp_supported(x.data_ptr(), ldx, y.data_ptr(), ldy, n, d, dt):
        mode |= _lib.FLAG_KEEP_EXP
    ws = torch.empty(lib.mec_workspace_floats_mode(n, d, dt, mode), dtype=torch.float32, device=dev)
    loss = torch.empty((), dtype=torch.float32, device=dev)
    # under torch.use_deterministic_algorithms(True) the forward sums are
    # formed without atomics (the backward is deterministic either way)
    fmode = mode | (_lib.FLAG_DETERMINISTIC if torch.are_deterministic_algorithms_enabled() else 0)
    with _on_device(di):
        _lib.call("mec_forward", x.data_ptr(), ldx, y.data_ptr(), ldy, n, d, dt, fmode, int(normalize),
                  temperature, ws.data_ptr(), loss.data_ptr(), _stream(di))
    ctx.save_for_backward(x, y, ws)
    ctx.mec = (ldx, ldy, n, d, dt, mode, bool(normalize), temperature,
               math.sqrt(n / temperature) if stable else 1.0 / temperature)
    return loss


def backward(ctx, grad_output: torch.Tensor, need_x: bool, need_y: bool):
    """Returns (dx, dy); a side that is not needed comes back as None."""
    refuse_graph_capture()
    x, y, ws = ctx.saved_tensors
    ldx, ldy, n, d, dt, mode, normalize, temperature, grad_scale = ctx.mec
    if mode & 0xFF == _lib.MODE_LIT:
        need_y = False
    if not (need_x or need_y):
        return None, None
    dev = x.device
    di = x.get_device()
    lib = _lib.load()
    go = grad_output
    if go.dtype != torch.float32 or go.device != dev or go.dim() != 0:
        go = go.detach().to(device=dev, dtype=torch.float32).reshape(())
    acc_x = torch.empty((n, d), dtype=torch.float32, device=dev) if need_x else None
    acc_y = torch.empty((n, d), dtype=torch.float32, device=dev) if need_y else None
    if dt in (_lib.DTYPE_F32, _lib.DTYPE_F32_BF16X3, _lib.DTYPE_F32_BF16):
        dx, dy = acc_x, acc_y  # the post-pass runs in place
    else:
        dx = torch.empty((n, d), dtype=x.dtype, device=dev) if need_x else None
        dy = torch.empty((n, d), dtype=y.dtype, device=dev) if need_y else None
    # The gradient scratch comes straight from PyTorch's caching allocator
    # (stream-ordered, like a tensor): the kernels write every byte of it
    # before reading it, so the NaN fill that torch.empty performs under
    # torch.use_deterministic_algorithms(True) (gigabytes at large N) would
    # be wasted work.
    sides = (_lib.SIDE_X if need_x else 0) | (_lib.SIDE_Y if need_y else 0)
    nbytes = lib.mec_grad_scratch_bytes_for(n, d, dt, mode, sides)  # 0 with the kept exponentials

    def ptr(t):
        return None if t is None else t.data_ptr()

    with _on_device(di):
        scratch = torch.cuda.caching_allocator_alloc(nbytes, di, torch.cuda.current_stream(di)) if nbytes > 0 \
            else None
        try:
            _lib.call("mec_backward", x.data_ptr(), ldx, y.data_ptr(), ldy, n, d, dt, mode, int(normalize),
                      temperature, grad_scale, ws.data_ptr(), go.data_ptr(), scratch, nbytes,
                      ptr(acc_x), ptr(acc_y), ptr(dx), ptr(dy), _stream(di))
        finally:
            if scratch is not None:
                torch.cuda.caching_allocator_delete(scratch)
    return dx, dy


class ContrastiveLossFn(torch.autograd.Function):
    """Fused loss used by the nn.Modules (normalisation optionally fused)."""

    @staticmethod
    def forward(ctx, x, y, temperature, mode, normalize, stable):
        return forward(ctx, x, y, temperature, mode, normalize, stable)

    @staticmethod
    def backward(ctx, grad_output):
        dx, dy = backward(ctx, grad_output, ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        return dx, dy, None, None, None, None
