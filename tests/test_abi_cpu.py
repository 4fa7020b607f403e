"""The C-ABI library loads on a machine without a GPU, exports every function
declared in include/mec.h, and rejects bad arguments in pure host code (no
GPU work is launched by any call in this file)."""
import ctypes
import os
import re

import pytest

from memoryefficientclip_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mec.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(mec_\w+)\s*\(", src, flags=re.M)))


def test_header_declares_the_abi():
    names = declared_functions()
    assert "mec_forward" in names and "mec_backward" in names and "mec_last_error" in names
    assert set(names) == set(_lib.SIGNATURES), "ctypes table and header disagree"


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert ctypes.cast(getattr(lib, name), ctypes.c_void_p).value


def test_sizes():
    lib = _lib.load()
    # 8 vectors, ceil(n / 1024) fp64 loss partials, 8 vectors of deterministic partial sums
    # 8 vectors, the fp64 loss partials (2 floats per 1024 rows), 48 x n deterministic partials
    assert lib.mec_workspace_floats(1000) == 8000 + 2 + 48000
    assert lib.mec_workspace_floats(1025) == 8 * 1025 + 4 + 48 * 1025
    assert lib.mec_workspace_floats(0) < 0
    # scratch is O(n*d): two block diagonals of the N x N gradient matrix (fp32:
    # in both layouts; bf16 and fp16: transposed only), plus transposed copies of
    # the two inputs; blocks are a multiple of 128 rows (fp32) or 256 rows (the
    # 16-bit types: their tiles are 128 x 256 and 256 x 256)
    for n, d in [(1024, 512), (32768, 1152), (65536, 768), (262144, 1152), (1000, 3), (777, 1152)]:
        for dt, elem, q, copies in [(0, 4, 128, 4), (1, 2, 256, 2), (2, 2, 256, 2)]:
            b = lib.mec_grad_scratch_bytes(n, d, dt)
            bs, nb = _lib.grad_blocking(n, d, dt)
            assert bs % q == 0 and nb * bs >= n > (nb - 1) * bs, (n, d, dt, bs, nb)
            ldt = (n + 127) // 128 * 128
            assert b == (copies * nb * bs * bs + 2 * d * ldt) * elem, (n, d, dt)
            bs_max = 2 * max(1024, (4 if dt == 0 else 16) * d + q)
            assert bs <= bs_max and b <= elem * (4 * (n + bs_max) * bs_max + 2 * d * (n + 128)), (n, d, dt, b)
    assert lib.mec_grad_scratch_bytes(10, 10, 7) < 0


def test_bf16_product_mode_sizes():
    # fp32 data with bf16 split products: the workspace carries split copies of
    # x and y (rows of 3 segments of d rounded up to 8 bf16), the backward uses
    # the bf16 blocking with hi and lo planes of the transposed blocks and inputs
    # (MEC_DTYPE_F32_BF16: one bf16 copy per input, the bf16 scratch layout)
    lib = _lib.load()
    x3, x1 = _lib.DTYPE_F32_BF16X3, _lib.DTYPE_F32_BF16
    for n, d in [(1000, 3), (32768, 1152), (777, 130), (65536, 768)]:
        base = lib.mec_workspace_floats(n)
        for dt in (0, 1, 2):
            assert lib.mec_workspace_floats_for(n, d, dt) == base
        dp = (d + 7) // 8 * 8
        assert lib.mec_workspace_floats_for(n, d, x3) == (base + 3) // 4 * 4 + n * 3 * dp
        assert lib.mec_workspace_floats_for(n, d, x1) == (base + 3) // 4 * 4 + n * dp
        ldt = (n + 127) // 128 * 128
        for dt, planes in ((x3, 4), (x1, 2)):
            assert _lib.grad_blocking(n, d, dt) == _lib.grad_blocking(n, d, 1)
            bs, nb = _lib.grad_blocking(n, d, dt)
            assert lib.mec_grad_scratch_bytes(n, d, dt) == (planes * nb * bs * bs + planes * d * ldt) * 2
    assert lib.mec_workspace_floats_for(10, 0, x3) < 0 and lib.mec_workspace_floats_for(10, 10, 7) < 0
    # the split copies need a 16-byte aligned workspace; rejected before any launch
    for dt in (x3, x1):
        rc = lib.mec_prepass(16, 64, 16, 64, 10, 64, dt, 1, 8, None)
        assert rc == _lib.MEC_ERR_INVALID and "16-byte" in _lib.last_error()


def test_16bit_blocks_fit_the_32bit_operand_range():
    # the direct-to-LDS core reads a transposed gradient-matrix block with 32-bit
    # byte offsets masked at 2^31: (bs - 1) * bs + 256 elements of 2 bytes < 2^31
    for n, d in [(65536, 8192), (65536, 4096), (33000, 4352), (2 ** 22, 1024), (40000, 100000)]:
        for dt in (1, 2):
            bs, nb = _lib.grad_blocking(n, d, dt)
            assert bs <= 32512 and ((bs - 1) * bs + 256) * 2 < 2 ** 31, (n, d, bs)
            assert nb * bs >= n > (nb - 1) * bs
    # fp32 addresses with 64-bit pointers; its ~4d target (131072 rows here)
    # gives way to the memory budget of the gradient-matrix buffers (16 GiB)
    assert _lib.grad_blocking(65536, 32768, 0) == (16384, 4)


def test_blocking_prefers_exact_divisors():
    # the headline and bf16 shapes split into equal blocks (no short last block)
    for n, d in [(32768, 1152), (65536, 768), (262144, 1152), (1024, 512)]:
        for dt in (0, 1, 2):
            bs, nb = _lib.grad_blocking(n, d, dt)
            assert nb * bs == n, (n, d, dt, bs, nb)
    assert _lib.grad_blocking(32768, 1152, 0) == (4096, 8)
    # 16-bit: ~16d rows while 8d would give fewer than 16 blocks, else ~8d
    assert _lib.grad_blocking(65536, 768, 1) == (16384, 4)
    assert _lib.grad_blocking(262144, 1152, 1) == (8192, 32)
    assert _lib.grad_blocking(32768, 1152, _lib.DTYPE_F32_BF16X3) == (16384, 2)
    assert _lib.grad_blocking(1000, 64, 0) == (1024, 1)
    assert _lib.grad_blocking(1000, 64, 1) == (1024, 1)


VALID = dict(x=16, ldx=64, y=16, ldy=64, n=10, d=64, dtype=0, mode=0, normalize=1, temperature=0.07)


@pytest.mark.parametrize("field,value,needle", [
    ("n", 0, "n="), ("d", 0, "d="), ("ldx", 8, "row strides"), ("dtype", 5, "dtype"),
    ("mode", 3, "mode"), ("temperature", -1.0, "temperature"), ("temperature", float("nan"), "temperature"),
    ("x", None, "non-null"),
])
def test_sumexp_rejects_invalid_arguments(field, value, needle):
    a = dict(VALID)
    a[field] = value
    lib = _lib.load()
    rc = lib.mec_sumexp(a["x"], a["ldx"], a["y"], a["ldy"], a["n"], a["d"], a["dtype"], a["mode"], a["normalize"],
                        a["temperature"], 16, None)
    assert rc == _lib.MEC_ERR_INVALID
    assert needle in _lib.last_error()


@pytest.mark.parametrize("mode,ok", [(0, True), (1, True), (0x100, True), (0x101, True), (2, False),
                                     (0x102, False), (0x200, False), (0x300, False), (-1, False)])
def test_mode_and_deterministic_flag(mode, ok):
    # validation only: a null workspace stops every valid call before any launch
    lib = _lib.load()
    a = dict(VALID, mode=mode)
    rc = lib.mec_sumexp(a["x"], a["ldx"], a["y"], a["ldy"], a["n"], a["d"], a["dtype"], mode, a["normalize"],
                        a["temperature"], None, None)
    assert rc == _lib.MEC_ERR_INVALID
    assert ("workspace" if ok else "mode") in _lib.last_error()
    rc = lib.mec_finalize(10, mode, 0.07, None, None, None)
    assert rc == _lib.MEC_ERR_INVALID and (("non-null" if ok else "mode") in _lib.last_error())


def gbuf_bytes(n, d, dt):
    """Bytes of the gradient-matrix buffers: 4 copies (fp32: both layouts,
    double-buffered; bf16x3: hi and lo planes) or 2 copies of nb blocks of bs^2."""
    bs, nb = _lib.grad_blocking(n, d, dt)
    copies = 4 if dt in (0, 3) else 2
    elem = 4 if dt == 0 else 2
    return copies * nb * bs * bs * elem, bs


@pytest.mark.parametrize("dt", [0, 1, 2, 3, 4])
def test_scratch_stays_within_its_budget(dt):
    """The gradient-matrix buffers stay within the bytes of a dense fp32 n x n
    logit matrix and within 16 GiB, unless the 1024-row block floor alone
    exceeds that; the transposed input copies add 2 (bf16x3: 4) n x d planes."""
    lib = _lib.load()
    for n in (1024, 3000, 4096, 8192, 16384, 32768, 65536, 262144, 1 << 21, 1 << 22):
        for d in (64, 512, 768, 1152, 2048, 4096, 8192):
            g, bs = gbuf_bytes(n, d, dt)
            budget = min(n * n * 4, 16 << 30)
            q = 128 if dt == 0 else 256
            floor_rows = max(1024, q)
            elem = 4 if dt == 0 else 2
            copies = 4 if dt in (0, 3) else 2
            nb_floor = -(-n // floor_rows)
            floor_bytes = copies * nb_floor * floor_rows * floor_rows * elem
            assert g <= budget or (bs == floor_rows and g <= floor_bytes), (n, d, dt, bs, g, budget)
            ldt = (n + 127) // 128 * 128
            planes = 4 if dt == 3 else 2
            assert lib.mec_grad_scratch_bytes(n, d, dt) == g + planes * d * ldt * elem


def test_scratch_at_two_million_rows():
    # n = 2^21 pairs at the headline width: 1024-row blocks, about 54 GB of
    # scratch (34 GB gradient-matrix buffers + 19 GB transposed inputs), within
    # the 288 GB of one MI355X beside the inputs and gradients (4 x 9.7 GB)
    lib = _lib.load()
    assert _lib.grad_blocking(1 << 21, 1152, 0) == (1024, 2048)
    assert lib.mec_grad_scratch_bytes(2097152, 1152, 0) <= 60 * 10 ** 9


@pytest.mark.parametrize("dtype", [0, 1, 2, 3, 4])
def test_size_limit(dtype):
    # every dtype supports n <= 2^22: the 16-bit contractions address transposed
    # panels with 32-bit offsets, and the fp32 forward grid of 128 x 128 tiles
    # ((n / 128)^2 workgroups) must stay below 2^31; beyond, every entry point
    # returns MEC_ERR_UNSUPPORTED before any launch
    lib = _lib.load()
    assert lib.mec_workspace_floats((1 << 22) + 1) < 0
    assert lib.mec_grad_scratch_bytes((1 << 22) + 1, 64, dtype) < 0
    assert lib.mec_workspace_floats_for(1 << 22, 64, dtype) > 0
    n_big = (1 << 22) + 1
    for rc in (lib.mec_forward(16, 64, 16, 64, n_big, 64, dtype, 0, 1, 0.07, 16, 16, None),
               lib.mec_prepass(16, 64, 16, 64, n_big, 64, dtype, 1, 16, None),
               lib.mec_finalize(n_big, 0, 0.07, 16, 16, None),
               lib.mec_grad(16, 64, 16, 64, n_big, 64, dtype, 0, 1, 0.07, 16, 16, 1 << 40, 16, 16, None),
               lib.mec_postpass(16, 64, 16, 64, n_big, 64, dtype, 0, 1, 1.0, 16, None, 16, 16, 16, 16, None),
               lib.mec_backward(16, 64, 16, 64, n_big, 64, dtype, 0, 1, 0.07, 1.0, 16, None, 16, 1 << 40, 16,
                                16, 16, 16, None)):
        assert rc == _lib.MEC_ERR_UNSUPPORTED and "2^22" in _lib.last_error()
    with pytest.raises(_lib.MecError, match="2\\^22"):
        _lib.grad_blocking(n_big, 64, dtype)


@pytest.mark.parametrize("dtype", [1, 2, 3, 4])
def test_16bit_size_limit(dtype):
    # the 16-bit contractions address transposed panels with 32-bit offsets
    lib = _lib.load()
    a = dict(VALID, dtype=dtype)
    for n, want in [((1 << 22) + 1, _lib.MEC_ERR_UNSUPPORTED), (1 << 22, None)]:
        rc = lib.mec_sumexp(a["x"], a["ldx"], a["y"], a["ldy"], n, a["d"], dtype, a["mode"], a["normalize"],
                            a["temperature"], None, None)
        if want is None:
            # passes the size check and stops at the null workspace, before any launch
            assert rc == _lib.MEC_ERR_INVALID and "workspace" in _lib.last_error()
        else:
            assert rc == want and "2^22" in _lib.last_error()


def test_grad_rejects_small_scratch_and_missing_outputs():
    lib = _lib.load()
    need = lib.mec_grad_scratch_bytes(10, 64, 0)
    rc = lib.mec_grad(16, 64, 16, 64, 10, 64, 0, 0, 1, 0.07, 16, 16, need - 1, 16, 16, None)
    assert rc == _lib.MEC_ERR_INVALID and "scratch" in _lib.last_error()
    rc = lib.mec_grad(16, 64, 16, 64, 10, 64, 0, 0, 1, 0.07, 16, 16, need, None, None, None)
    assert rc == _lib.MEC_ERR_INVALID and "no gradient" in _lib.last_error()
    rc = lib.mec_grad(16, 64, 16, 64, 10, 64, 0, 0, 1, 0.07, 16, 8, need, 16, 16, None)
    assert rc == _lib.MEC_ERR_INVALID and "aligned" in _lib.last_error()


def test_grad_step_validation():
    lib = _lib.load()
    need = lib.mec_grad_scratch_bytes(10, 64, 0)
    rc = lib.mec_grad_step(16, 64, 16, 64, 10, 64, 0, 0, 1, 0.07, 16, 2, 16, need, 16, 16, None)
    assert rc == _lib.MEC_ERR_INVALID and "step" in _lib.last_error()
    rc = lib.mec_grad_step(16, 64, 16, 64, 10, 64, 0, 0, 1, 0.07, 16, -1, 16, need, 16, 16, None)
    assert rc == _lib.MEC_ERR_INVALID and "step" in _lib.last_error()
    with pytest.raises(_lib.MecError, match="out of range"):
        _lib.grad_blocking(0, 64, 0)
    # the step counter is checked against the blocking of this shape
    bs, nb = _lib.grad_blocking(10, 64, 0)
    rc = lib.mec_grad_step(16, 64, 16, 64, 10, 64, 0, 0, 1, 0.07, 16, nb + 1, 16, need, 16, 16, None)
    assert rc == _lib.MEC_ERR_INVALID and "step" in _lib.last_error()


def test_postpass_and_finalize_validation():
    lib = _lib.load()
    rc = lib.mec_postpass(16, 64, 16, 64, 10, 64, 0, 0, 1, 1.0, 16, None, 16, None, None, None, None)
    assert rc == _lib.MEC_ERR_INVALID and "accumulator" in _lib.last_error()
    rc = lib.mec_postpass(16, 64, 16, 64, 10, 64, 0, 0, 1, float("inf"), 16, None, 16, 16, 16, 16, None)
    assert rc == _lib.MEC_ERR_INVALID and "grad_scale" in _lib.last_error()
    assert lib.mec_finalize(10, 0, 0.07, None, None, None) == _lib.MEC_ERR_INVALID
    assert lib.mec_finalize(0, 0, 0.07, 16, 16, None) == _lib.MEC_ERR_INVALID


def test_error_string_is_thread_local():
    import threading
    lib = _lib.load()
    lib.mec_finalize(10, 9, 0.07, 16, 16, None)
    seen = {}

    def other():
        seen["msg"] = lib.mec_last_error().decode()

    th = threading.Thread(target=other)
    th.start()
    th.join()
    assert seen["msg"] == ""
    assert "mode" in _lib.last_error()


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load(tmp_path / "nope.so")


def test_noalloc_rejects_problems_beyond_its_array():
    # mec_backward_noalloc holds its scratch in a 256 MiB device array: a
    # problem whose scratch does not fit even with 1024-row blocks is refused
    # in host code, before any HIP call (no device here)
    lib = _lib.load()
    n, d = 65536, 768  # config 4 (bf16): the transposed inputs alone are 201 MB
    rc = lib.mec_backward_noalloc(16, d, 16, d, n, d, _lib.DTYPE_BF16, 0, 0, 0.07, 1.0 / 0.07, 16, None, 16, 16,
                                  16, 16, None)
    assert rc == _lib.MEC_ERR_UNSUPPORTED and "mec_backward_noalloc holds" in _lib.last_error()
    n, d = 1 << 20, 1024  # fp32: 8 GB of transposed inputs
    rc = lib.mec_backward_noalloc(16, d, 16, d, n, d, 0, 0, 1, 0.07, 1.0 / 0.07, 16, None, 16, 16, 16, 16, None)
    assert rc == _lib.MEC_ERR_UNSUPPORTED
    # argument errors as mec_backward
    rc = lib.mec_backward_noalloc(16, 64, 16, 64, 10, 64, 0, 0, 1, 0.07, 1.0 / 0.07, 16, None, None, None, None,
                                  None, None)
    assert rc == _lib.MEC_ERR_INVALID and "no gradient" in _lib.last_error()
    rc = lib.mec_backward_noalloc(16, 64, 16, 64, 10, 64, 0, 0, 1, 0.07, float("nan"), 16, None, 16, 16, 16, 16,
                                  None)
    assert rc == _lib.MEC_ERR_INVALID and "grad_scale" in _lib.last_error()
