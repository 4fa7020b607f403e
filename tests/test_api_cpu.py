"""Host-side behaviour of the drop-in modules that needs no GPU: class names
and signatures match the reference's, error behaviour on CPU tensors and bad
shapes, no parameters/buffers, and no CPU fallback."""
import inspect

import pytest
import torch

import memoryefficientclip_amd as mec
from memoryefficientclip_amd import clip_loss, lit_loss

REFERENCE_NAMES = {
    clip_loss: ["MemoryEfficientCLIPLossNormed", "MemoryEfficientCLIPLoss", "StableMemoryEfficientCLIPLossNormed",
                "StableMemoryEfficientCLIPLoss"],
    lit_loss: ["MemoryEfficientLiTLossNormed", "MemoryEfficientLiTLoss", "StableMemoryEfficientLiTLossNormed",
               "StableMemoryEfficientLiTLoss"],
}


def test_reference_class_names_exist():
    for mod, names in REFERENCE_NAMES.items():
        for n in names:
            assert hasattr(mod, n) and hasattr(mec, n)


def test_signatures_match_reference():
    # clip_loss.py:260, :265 ; lit_loss.py:251, :256 ; Function.forward clip_loss.py:161
    for cls in [clip_loss.MemoryEfficientCLIPLoss, clip_loss.StableMemoryEfficientCLIPLoss]:
        assert list(inspect.signature(cls.__init__).parameters) == ["self", "temperature", "normalized_inputs"]
        assert list(inspect.signature(cls.forward).parameters) == ["self", "image_features", "text_features"]
    for cls in [lit_loss.MemoryEfficientLiTLoss, lit_loss.StableMemoryEfficientLiTLoss]:
        assert list(inspect.signature(cls.__init__).parameters) == ["self", "temperature", "normalized_inputs"]
        assert list(inspect.signature(cls.forward).parameters) == ["self", "text_features", "image_features"]
    for fn in [clip_loss.MemoryEfficientCLIPLossNormed, lit_loss.MemoryEfficientLiTLossNormed,
               clip_loss.StableMemoryEfficientCLIPLossNormed, lit_loss.StableMemoryEfficientLiTLossNormed]:
        sig = inspect.signature(fn.forward)
        assert list(sig.parameters) == ["ctx", "x_normalized", "y_normalized", "temperature"]
        assert sig.parameters["temperature"].default == 0.07
        assert issubclass(fn, torch.autograd.Function)


def test_defaults_and_empty_state_dict():
    m = clip_loss.MemoryEfficientCLIPLoss()
    assert m.temperature == 0.07 and m.normalized_inputs is False
    assert m.state_dict() == {} and list(m.parameters()) == []


@pytest.mark.parametrize("cls", [clip_loss.MemoryEfficientCLIPLoss, lit_loss.MemoryEfficientLiTLoss,
                                 clip_loss.StableMemoryEfficientCLIPLoss, lit_loss.StableMemoryEfficientLiTLoss])
def test_cpu_tensors_raise_like_reference(cls):
    # reference: assert X.is_cuda and Y.is_cuda (clip_loss.py:166); no CPU fallback here either
    a = torch.randn(8, 16)
    with pytest.raises(AssertionError, match="GPU"):
        cls(0.07)(a, a)
    with pytest.raises(AssertionError, match="GPU"):
        cls(0.07, normalized_inputs=True)(a, a)


def test_normed_function_cpu_raises():
    a = torch.randn(8, 16)
    with pytest.raises(AssertionError):
        clip_loss.MemoryEfficientCLIPLossNormed.apply(a, a, 0.07)
    with pytest.raises(AssertionError):
        lit_loss.MemoryEfficientLiTLossNormed.apply(a, a)


def test_check_inputs_shape_and_dtype_rules():
    from memoryefficientclip_amd._function import check_inputs

    class FakeCuda(torch.Tensor):
        @property
        def is_cuda(self):
            return True

    def fake(shape, dtype=torch.float32):
        return torch.zeros(shape, dtype=dtype).as_subclass(FakeCuda)

    with pytest.raises(AssertionError, match="shape"):
        check_inputs(fake((4, 8)), fake((4, 9)))
    with pytest.raises(ValueError, match="2-D"):
        check_inputs(fake((4,)), fake((4,)))
    with pytest.raises(TypeError, match="unsupported dtype"):
        check_inputs(fake((4, 8), torch.float64), fake((4, 8), torch.float64))
    with pytest.raises(TypeError, match="dtype mismatch"):
        check_inputs(fake((4, 8)), fake((4, 8), torch.bfloat16))
    check_inputs(fake((4, 8), torch.bfloat16), fake((4, 8), torch.bfloat16))
    check_inputs(fake((4, 8), torch.float16), fake((4, 8), torch.float16))


def test_product_path_does_not_import_oracle():
    import ast
    import pathlib
    pkg = pathlib.Path(mec.__file__).parent
    for f in pkg.rglob("*.py"):
        tree = ast.parse(f.read_text())
        for node in ast.walk(tree):
            if isinstance(node, ast.Import):
                assert not any(a.name.split(".")[0] == "oracle" for a in node.names), f
            if isinstance(node, ast.ImportFrom):
                assert (node.module or "").split(".")[0] != "oracle", f


def test_float32_matmul_precision_selects_the_product_mode():
    # "highest" (PyTorch's default): IEEE fp32 products; "high": three bf16
    # terms per product (MEC_DTYPE_F32_BF16X3); "medium": bf16 products
    # (MEC_DTYPE_F32_BF16); 16-bit inputs are unaffected
    from memoryefficientclip_amd import _lib
    from memoryefficientclip_amd._function import compute_dtype

    old = torch.get_float32_matmul_precision()
    try:
        for p, code in (("highest", _lib.DTYPE_F32), ("high", _lib.DTYPE_F32_BF16X3),
                        ("medium", _lib.DTYPE_F32_BF16)):
            torch.set_float32_matmul_precision(p)
            assert compute_dtype(torch.float32) == code
            assert compute_dtype(torch.bfloat16) == _lib.DTYPE_BF16
            assert compute_dtype(torch.float16) == _lib.DTYPE_F16
    finally:
        torch.set_float32_matmul_precision(old)


def test_graph_capture_is_refused(monkeypatch):
    """Forward and backward raise RuntimeError, before touching any tensor,
    while the current stream is capturing a CUDA/HIP graph (capture of the
    loss crashed the host process in capture_end on the GPU box)."""
    from memoryefficientclip_amd import _function
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    monkeypatch.setattr(_function, "check_inputs", lambda x, y: None)
    x = torch.zeros(4, 8)
    with pytest.raises(RuntimeError, match="graph capture"):
        _function.forward(None, x, x, 0.07, 0, True, False)
    with pytest.raises(RuntimeError, match="graph capture"):
        _function.backward(None, torch.ones(()), True, True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    _function.refuse_graph_capture()  # no capture: no error


def test_reference_import_path_works_unchanged():
    """With the drop-in directory on PYTHONPATH, the reference's own imports
    (`from clip_loss import ...`, `from lit_loss import ...`, its README lines
    29 and 50) load this package's classes, with no edit in the caller."""
    import os
    import subprocess
    import sys

    from memoryefficientclip_amd import dropin

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([dropin.PATH, root]))
    code = ("from clip_loss import MemoryEfficientCLIPLoss, MemoryEfficientCLIPLossNormed, "
            "StableMemoryEfficientCLIPLoss, StableMemoryEfficientCLIPLossNormed\n"
            "from lit_loss import MemoryEfficientLiTLoss, MemoryEfficientLiTLossNormed, "
            "StableMemoryEfficientLiTLoss, StableMemoryEfficientLiTLossNormed\n"
            "import memoryefficientclip_amd as m\n"
            "assert MemoryEfficientCLIPLoss is m.MemoryEfficientCLIPLoss\n"
            "assert StableMemoryEfficientLiTLossNormed is m.StableMemoryEfficientLiTLossNormed\n"
            "loss_fn = MemoryEfficientCLIPLoss(temperature=0.07, normalized_inputs=False)\n"
            "print('ok', type(loss_fn).__module__)\n")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "ok memoryefficientclip_amd.clip_loss"
    # python -m memoryefficientclip_amd.dropin prints the directory
    out = subprocess.run([sys.executable, "-m", "memoryefficientclip_amd.dropin"], env=dict(os.environ, PYTHONPATH=root),
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and out.stdout.strip() == dropin.PATH
