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


ELEM = {0: 4, 1: 2, 2: 2, 3: 2, 4: 2}   # scratch element bytes per dtype
QUANTUM = {0: 128, 1: 256, 2: 256, 3: 256, 4: 256}


def layout_bytes(n, d, dt, sides, bs, nb):
    """Scratch of the backward for blocks (bs, nb): the gradient-matrix
    diagonal (double-buffered unless one block covers n; bf16x3 hi and lo
    planes) and, for the 16-bit kernels only, one transposed input per side
    (bf16x3: two planes); fp32 reads its raw inputs."""
    elem = ELEM[dt]
    nbuf = 2 if nb > 1 else 1
    planes = 2 if dt == 3 else 1
    ldt = (n + 127) // 128 * 128
    ntp = 0 if dt == 0 else planes
    nsides = bin(sides).count("1")
    return nbuf * planes * nb * bs * bs * elem + nsides * ntp * d * ldt * elem


def budget(n, d, dt):
    """Default bound of the gradient-matrix buffers: 64 n d elements, at
    least 256 MiB, at most 16 GiB."""
    return min(16 << 30, max(64 * n * d * ELEM[dt], 256 << 20))


def test_sizes():
    lib = _lib.load()
    # 8 vectors, the fp64 loss partials (2 floats per 1024 rows), 48 x n deterministic partials
    # 8 vectors, one fp64 loss partial per 256 rows, the deterministic forward's 48 partials per index
    assert lib.mec_workspace_floats(1000) == 8000 + 2 * 4 + 48000
    assert lib.mec_workspace_floats(1025) == 8 * 1025 + 2 * 5 + 48 * 1025
    assert lib.mec_workspace_floats(256) == 56 * 256 + 2
    assert lib.mec_workspace_floats(0) < 0
    for n, d in [(1024, 512), (32768, 1152), (65536, 768), (262144, 1152), (1000, 3), (777, 1152)]:
        for dt in (0, 1, 2, 3, 4):
            bs, nb = _lib.grad_blocking(n, d, dt)
            q = QUANTUM[dt]
            assert bs % q == 0 and nb * bs >= n > (nb - 1) * bs, (n, d, dt, bs, nb)
            assert lib.mec_grad_scratch_bytes(n, d, dt) == layout_bytes(n, d, dt, 3, bs, nb), (n, d, dt)
            for mode, sides in ((0, 1), (0, 2), (0, 3), (1, 1), (1, 3)):
                want = layout_bytes(n, d, dt, 1 if mode == 1 else sides, bs, nb)
                assert lib.mec_grad_scratch_bytes_for(n, d, dt, mode, sides) == want, (n, d, dt, mode, sides)
    assert lib.mec_grad_scratch_bytes(10, 10, 7) < 0
    # bad mode, no side, LiT without its x side
    assert lib.mec_grad_scratch_bytes_for(10, 10, 0, 5, 3) < 0
    assert lib.mec_grad_scratch_bytes_for(10, 10, 0, 0, 0) < 0
    assert lib.mec_grad_scratch_bytes_for(10, 10, 0, 0, 4) < 0
    assert lib.mec_grad_scratch_bytes_for(10, 10, 0, 1, 2) < 0


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
        for dt in (x3, x1):
            # the same bf16 blocking unless the bf16x3 planes meet the budget first
            bs, nb = _lib.grad_blocking(n, d, dt)
            assert bs % 256 == 0 and nb * bs >= n > (nb - 1) * bs
            if dt == x1:
                assert (bs, nb) == _lib.grad_blocking(n, d, 1)
            assert lib.mec_grad_scratch_bytes(n, d, dt) == layout_bytes(n, d, dt, 3, bs, nb)
    assert lib.mec_workspace_floats_for(10, 0, x3) < 0 and lib.mec_workspace_floats_for(10, 10, 7) < 0
    # the split copies need a 16-byte aligned workspace; rejected before any launch
    for dt in (x3, x1):
        rc = lib.mec_prepass(16, 64, 16, 64, 10, 64, dt, 1, 8, None)
        assert rc == _lib.MEC_ERR_INVALID and "16-byte" in _lib.last_error()


def test_blocks_fit_the_32bit_operand_range():
    # the direct-to-LDS core reads a transposed gradient-matrix block with 32-bit
    # byte offsets masked at 2^31: (bs - 1) * bs + 256 elements of 2 bytes
    # (16-bit) or (bs - 1) * bs + 128 floats (fp32, the y side) below 2^31
    for n, d in [(65536, 8192), (65536, 4096), (33000, 4352), (2 ** 22, 1024), (40000, 100000)]:
        for dt in (1, 2):
            bs, nb = _lib.grad_blocking(n, d, dt)
            assert bs <= 32512 and ((bs - 1) * bs + 256) * 2 < 2 ** 31, (n, d, bs)
            assert nb * bs >= n > (nb - 1) * bs
        bs, nb = _lib.grad_blocking(n, d, 0)
        assert bs <= 16384 and ((bs - 1) * bs + 128) * 4 < 2 ** 31, (n, d, bs)
    # fp32's ~4d target (131072 rows here) gives way to that cap
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
    # at least 1024 rows where the budget allows: one block for a small problem
    assert _lib.grad_blocking(1000, 64, 0) == (1024, 1)
    assert _lib.grad_blocking(1000, 64, 1) == (1024, 1)
    assert _lib.grad_blocking(1024, 512, 0) == (1024, 1)


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
                                     (0x102, False), (0x400, False), (0x500, False), (-1, False)])
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


@pytest.mark.parametrize("dt", [0, 1, 2, 3, 4])
def test_scratch_stays_within_its_budget(dt):
    """The gradient-matrix buffers stay within O(n d): 64 n d elements, at
    least 256 MiB, at most 16 GiB; only blocks of a single quantum (128 or
    256 rows, the smallest tile) may exceed that."""
    for n in (1024, 3000, 4096, 8192, 16384, 32768, 65536, 262144, 1 << 21, 1 << 22):
        for d in (1, 16, 64, 512, 768, 1152, 2048, 4096, 8192):
            bs, nb = _lib.grad_blocking(n, d, dt)
            g = layout_bytes(n, d, dt, 0, bs, nb)
            q = QUANTUM[dt]
            assert g <= budget(n, d, dt) or bs == q, (n, d, dt, bs, g)
            # the whole scratch for both sides: buffers plus the transposed inputs
            assert _lib.load().mec_grad_scratch_bytes(n, d, dt) == layout_bytes(n, d, dt, 3, bs, nb)


def test_scratch_at_two_million_rows():
    # n = 2^21 pairs at the headline width: 1024-row blocks within the 16 GiB
    # cap (fp32 keeps no transposed copies), beside the inputs and gradients
    # (4 x 9.7 GB) on one MI355X
    lib = _lib.load()
    assert _lib.grad_blocking(1 << 21, 1152, 0) == (1024, 2048)
    assert lib.mec_grad_scratch_bytes(2097152, 1152, 0) == 16 << 30


def test_scratch_by_mode_and_side():
    # LiT (x side only) and a frozen tower reserve only what their launches use
    lib = _lib.load()
    n, d = 32768, 1152
    clip = lib.mec_grad_scratch_bytes_for(n, d, 0, 0, 3)
    lit = lib.mec_grad_scratch_bytes_for(n, d, 0, 1, 1)
    # config 3 (LiT fp32): one H diagonal, double-buffered (8 blocks of 4096 rows)
    assert lit == 2 * 8 * 4096 * 4096 * 4 <= 1.4e9
    assert clip == lit  # fp32 reads its raw inputs: no side-dependent buffers
    # 16-bit: a transposed input per side computed
    for dt in (1, 2, 3, 4):
        both = lib.mec_grad_scratch_bytes_for(n, d, dt, 0, 3)
        one = lib.mec_grad_scratch_bytes_for(n, d, dt, 0, 1)
        planes = 2 if dt == 3 else 1
        assert both - one == planes * d * n * 2
        assert lib.mec_grad_scratch_bytes_for(n, d, dt, 0, 2) == one
        assert lib.mec_grad_scratch_bytes_for(n, d, dt, 1, 3) == one


def test_config1_extra_memory():
    # benchmark configuration 1 (n = 1024, d = 512, fp32): one block, one H
    # plane; the backward's scratch and the forward's workspace together stay
    # within twice a dense fp32 logit matrix (the returned gradients are the
    # outputs, as in the reference)
    lib = _lib.load()
    n, d = 1024, 512
    dense = n * n * 4
    scratch = lib.mec_grad_scratch_bytes_for(n, d, 0, 0, 3)
    ws = lib.mec_workspace_floats_for(n, d, 0) * 4
    assert scratch == dense
    assert scratch + ws <= 2 * dense


def test_keep_exp_sizes_and_support(monkeypatch):
    # MEC_FLAG_KEEP_EXP (small fp32 problems): the kept matrix and the
    # forward's bookkeeping (tile sums of E, block sums of G' cos, a 64-bit
    # loss accumulator) in the workspace, no gradient scratch
    lib = _lib.load()
    K = _lib.FLAG_KEEP_EXP
    n, d = 1024, 512
    dense = n * n * 4
    base = lib.mec_workspace_floats_for(n, d, 0)
    assert lib.mec_workspace_floats_mode(n, d, 0, 0) == base
    assert lib.mec_workspace_floats_mode(n, d, 0, 0x100) == base

    def up(f):  # 256-byte aligned parts
        return (f + 63) // 64 * 64

    def keep_floats(base, np_):
        kt = np_ // 64
        o = up(up(base) + np_ * np_)  # the kept matrix
        for _ in range(4):  # rowpart, colpart, rowdot, coldot
            o = up(o + kt * np_)
        return o + 2  # the loss accumulator

    expect = keep_floats(base, 1024)
    assert lib.mec_workspace_floats_mode(n, d, 0, K) == expect
    assert lib.mec_workspace_floats_mode(n, d, 0, K | 0x100 | 1) == expect
    # ragged n: np = n rounded up to 64
    assert lib.mec_workspace_floats_mode(1000, d, 0, K) == keep_floats(lib.mec_workspace_floats_for(1000, d, 0), 1024)
    assert lib.mec_workspace_floats_mode(65, 8, 0, K) == keep_floats(lib.mec_workspace_floats_for(65, 8, 0), 128)
    assert lib.mec_grad_scratch_bytes_for(n, d, 0, K, 3) == 0
    assert lib.mec_grad_scratch_bytes_for(n, d, 0, K | 1, 1) == 0
    # configuration 1 with the kept matrix: the workspace is all the extra memory
    assert lib.mec_workspace_floats_mode(n, d, 0, K) * 4 <= 2 * dense
    # limits: fp32 only, n <= 2048
    assert _lib.KEEP_EXP_MAX_N == 2048
    assert lib.mec_workspace_floats_mode(2048, d, 0, K) > 0
    assert lib.mec_workspace_floats_mode(2049, d, 0, K) < 0
    for dt in (1, 2, 3, 4):
        assert lib.mec_workspace_floats_mode(n, d, dt, K) < 0
        assert lib.mec_grad_scratch_bytes_for(n, d, dt, K, 3) < 0
    assert lib.mec_grad_scratch_bytes_for(2049, d, 0, K, 3) < 0
    # which inputs qualify (host-only checks of the pointers and strides)
    A = 1 << 20
    assert lib.mec_keep_exp_supported(A, d, A, d, n, d, 0) == 1
    assert lib.mec_keep_exp_supported(A, d, A, d, 1, 4, 0) == 1
    assert lib.mec_keep_exp_supported(A + 4, d, A, d, n, d, 0) == 0
    assert lib.mec_keep_exp_supported(A, d, A + 8, d, n, d, 0) == 0
    assert lib.mec_keep_exp_supported(A, d + 2, A, d, n, d, 0) == 0
    assert lib.mec_keep_exp_supported(A, 6, A, 6, n, 6, 0) == 0
    assert lib.mec_keep_exp_supported(A, d, A, d, 2049, d, 0) == 0
    assert lib.mec_keep_exp_supported(A, d, A, d, n, d - 1, 0) == 0
    assert lib.mec_keep_exp_supported(None, d, A, d, n, d, 0) == 0
    for dt in (1, 2, 3, 4):
        assert lib.mec_keep_exp_supported(A, d, A, d, n, d, dt) == 0
    monkeypatch.setenv("MEC_KEEP_EXP", "0")
    assert lib.mec_keep_exp_supported(A, d, A, d, n, d, 0) == 0


def test_keep_exp_flag_validation():
    # rejected before any launch: the one-stage functions take no
    # MEC_FLAG_KEEP_EXP, and mec_forward / mec_grad / mec_backward take it only
    # for inputs that qualify and a 16-byte aligned workspace
    lib = _lib.load()
    K = _lib.FLAG_KEEP_EXP
    A = 1 << 20
    rc = lib.mec_sumexp(A, 64, A, 64, 100, 64, 0, K, 1, 0.07, A, None)
    assert rc == _lib.MEC_ERR_INVALID and "MEC_FLAG_KEEP_EXP" in _lib.last_error()
    rc = lib.mec_finalize(100, K, 0.07, A, A, None)
    assert rc == _lib.MEC_ERR_INVALID and "MEC_FLAG_KEEP_EXP" in _lib.last_error()
    rc = lib.mec_grad_step(A, 64, A, 64, 100, 64, 0, K, 1, 0.07, A, 0, A, 1 << 30, A, A, None)
    assert rc == _lib.MEC_ERR_INVALID and "MEC_FLAG_KEEP_EXP" in _lib.last_error()
    for dt in (1, 3):
        rc = lib.mec_forward(A, 64, A, 64, 100, 64, dt, K, 1, 0.07, A, A, None)
        assert rc == _lib.MEC_ERR_INVALID and "needs" in _lib.last_error()
    rc = lib.mec_forward(A, 64, A, 64, 3000, 64, 0, K, 1, 0.07, A, A, None)
    assert rc == _lib.MEC_ERR_INVALID and "n <= 2048" in _lib.last_error()
    rc = lib.mec_forward(A + 4, 64, A, 64, 100, 64, 0, K, 1, 0.07, A, A, None)
    assert rc == _lib.MEC_ERR_INVALID and "aligned rows" in _lib.last_error()
    rc = lib.mec_forward(A, 64, A, 64, 100, 64, 0, K, 1, 0.07, A + 8, A, None)
    assert rc == _lib.MEC_ERR_INVALID and "aligned workspace" in _lib.last_error()
    rc = lib.mec_grad(A, 64, A, 64, 100, 64, 0, K, 1, 0.07, A + 8, None, 0, A, A, None)
    assert rc == _lib.MEC_ERR_INVALID and "aligned workspace" in _lib.last_error()
    rc = lib.mec_backward(A, 62, A, 62, 100, 62, 0, K, 1, 0.07, 1.0, A, None, None, 0, A, A, A, A, None)
    assert rc == _lib.MEC_ERR_INVALID and "MEC_FLAG_KEEP_EXP" in _lib.last_error()
    rc = lib.mec_backward_noalloc(A, 62, A, 62, 100, 62, 0, K, 1, 0.07, 1.0, A, None, A, A, A, A, None)
    assert rc == _lib.MEC_ERR_INVALID and "MEC_FLAG_KEEP_EXP" in _lib.last_error()
    # the plan of a kept-matrix backward
    p = _lib.backward_plan(1000, 512, 0, K, compute_units=256)
    assert (p.block_rows, p.num_blocks, p.scratch_bytes, p.noalloc_scratch_bytes) == (1024, 1, 0, 0)
    assert (p.contract_tile_rows, p.contract_tile_features) == (64, 64)
    with pytest.raises(_lib.MecError, match="MEC_FLAG_KEEP_EXP"):
        _lib.backward_plan(4096, 512, 0, K, compute_units=256)


def test_backward_plan():
    lib = _lib.load()
    p = _lib.backward_plan(32768, 1152, 0, compute_units=256)
    assert (p.block_rows, p.num_blocks, p.scratch_bytes) == (4096, 8, lib.mec_grad_scratch_bytes(32768, 1152, 0))
    assert (p.contract_tile_rows, p.contract_tile_features) == (128, 128)
    p = _lib.backward_plan(1024, 512, 0, compute_units=256)
    assert (p.contract_tile_rows, p.contract_tile_features) == (64, 64)
    # configs 4 and 5 take the 384-wide contraction tiles on 256 CUs
    for n, d in [(65536, 768), (262144, 1152)]:
        p = _lib.backward_plan(n, d, 1, compute_units=256)
        assert (p.contract_tile_rows, p.contract_tile_features, p.narrow_tiles) == (256, 384, 0)
    with pytest.raises(_lib.MecError, match="sides"):
        _lib.backward_plan(1024, 512, 0, sides=0, compute_units=256)
    with pytest.raises(_lib.MecError, match="2\\^22"):
        _lib.backward_plan((1 << 22) + 1, 512, 0, compute_units=256)


def test_fp32_backward_tile_rule(monkeypatch):
    # 64 x 64 backward tiles where a step's 128 x 128 gradient-matrix tiles
    # (ceil(n/128) ceil(bs/128)) are few for their K (tiles x D <= 2^17) or
    # leave the last round of 256 CUs under 90% full; the configurations of
    # the measurements behind the rule, on both sides of it
    monkeypatch.delenv("MEC_F32_SMALL_TILES", raising=False)
    cases = {
        (4096, 128): 64,    # 1024-row blocks: 256 tiles per step, tiles x D = 2^15
        (8192, 256): 64,    # 512 tiles, tiles x D = 2^17
        (12288, 256): 128,  # 768 tiles, 3 full rounds
        (3072, 512): 64,    # 288 tiles: a second round 12% full
        (4096, 512): 128,   # 512 tiles, 2 full rounds
        (5120, 512): 64,    # 800 tiles: 78%
        (6144, 512): 128,   # 768 tiles
        (5120, 1024): 64,   # 1600 tiles: 89%
        (6144, 1024): 128,  # 1152 tiles: 90%
        (2816, 1024): 64,   # below the 512 forward tiles of 128 x 128 (f32_small_n)
        (32768, 1152): 128,  # the headline
    }
    for (n, d), rows in cases.items():
        p = _lib.backward_plan(n, d, 0, compute_units=256)
        assert p.contract_tile_rows == rows, (n, d, p.block_rows, p.contract_tile_rows)
    # the environment override, as the tests use it
    monkeypatch.setenv("MEC_F32_SMALL_TILES", "0")
    assert _lib.backward_plan(4096, 128, 0, compute_units=256).contract_tile_rows == 128
    monkeypatch.setenv("MEC_F32_SMALL_TILES", "1")
    assert _lib.backward_plan(32768, 1152, 0, compute_units=256).contract_tile_rows == 64


def test_wide_contraction_tiles_stay_within_32bit_offsets(monkeypatch):
    # a 384-wide tile reads a 384-row panel of a transposed input ([d][ldt])
    # with 32-bit byte offsets: (383 ldt + bs) x 2 < 2^31, ldt up to ~2.8M;
    # past that the 256-wide tiles (fine up to n = 2^22) are used even where
    # MEC_WIDE_CONTRACT=1 forces the wide ones
    monkeypatch.setenv("MEC_WIDE_CONTRACT", "1")
    for n, ok in [(2_700_000, True), (2_850_000, False), (1 << 22, False)]:
        p = _lib.backward_plan(n, 1152, 1, compute_units=256)
        ldt = (n + 127) // 128 * 128
        assert ((383 * ldt + p.block_rows) * 2 < 2 ** 31) == ok
        assert p.contract_tile_features == (384 if ok else 256), (n, p.contract_tile_features)


def test_noalloc_fit_rule():
    # mec_backward_noalloc's 256 MiB array at d = 1152, CLIP: the largest n it
    # takes per dtype (fp32 holds only H; the 16-bit types also their
    # transposed inputs, 2 d bytes per row and side; bf16x3 two planes)
    d = 1152

    def largest(dt):
        lo, hi = 1, 1 << 22
        while lo < hi:
            mid = (lo + hi + 1) // 2
            if _lib.backward_plan(mid, d, dt, compute_units=256).noalloc_block_rows > 0:
                lo = mid
            else:
                hi = mid - 1
        return lo

    limits = {dt: largest(dt) for dt in (0, 1, 3)}
    mib256 = _lib.NOALLOC_SCRATCH_BYTES
    # fp32: two diagonals of 128-row blocks, 2 x 128 x 4 bytes per row
    assert limits[0] == mib256 // (2 * 128 * 4) == 262144, limits
    # bf16: two diagonals of 256-row blocks (1 KB per row) and the two
    # transposed inputs (2 d x 2 bytes per row, n rounded up to 128)
    assert limits[1] == 47616 and 47616 * (1024 + 4 * d) <= mib256 < 47744 * (1024 + 4 * d), limits
    # bf16x3: hi and lo planes of both
    assert limits[3] == 23808 and 23808 * 2 * (1024 + 4 * d) <= mib256, limits
    # the headline shape fits (fp32, 1024-row blocks), config 5 does not
    p = _lib.backward_plan(32768, 1152, 0, compute_units=256)
    assert p.noalloc_block_rows == 1024 and p.noalloc_scratch_bytes <= _lib.NOALLOC_SCRATCH_BYTES
    assert _lib.backward_plan(262144, 1152, 1, compute_units=256).noalloc_block_rows == -1


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
    # problem whose scratch does not fit even with single-quantum blocks is
    # refused in host code, before any HIP call (no device here)
    lib = _lib.load()
    n, d = 131072, 768  # bf16: the transposed inputs alone are 403 MB
    rc = lib.mec_backward_noalloc(16, d, 16, d, n, d, _lib.DTYPE_BF16, 0, 0, 0.07, 1.0 / 0.07, 16, None, 16, 16,
                                  16, 16, None)
    assert rc == _lib.MEC_ERR_UNSUPPORTED and "mec_backward_noalloc holds" in _lib.last_error()
    n, d = 1 << 20, 1024  # fp32: H at 128-row blocks is 1.07 GB
    rc = lib.mec_backward_noalloc(16, d, 16, d, n, d, 0, 0, 1, 0.07, 1.0 / 0.07, 16, None, 16, 16, 16, 16, None)
    assert rc == _lib.MEC_ERR_UNSUPPORTED
    # argument errors as mec_backward
    rc = lib.mec_backward_noalloc(16, 64, 16, 64, 10, 64, 0, 0, 1, 0.07, 1.0 / 0.07, 16, None, None, None, None,
                                  None, None)
    assert rc == _lib.MEC_ERR_INVALID and "no gradient" in _lib.last_error()
    rc = lib.mec_backward_noalloc(16, 64, 16, 64, 10, 64, 0, 0, 1, 0.07, float("nan"), 16, None, 16, 16, 16, 16,
                                  None)
    assert rc == _lib.MEC_ERR_INVALID and "grad_scale" in _lib.last_error()


def test_graph_capture_is_refused_before_any_launch(monkeypatch):
    # every entry point that launches checks the stream for an active HIP
    # graph capture and returns MEC_ERR_UNSUPPORTED first; the check is
    # stubbed here (no GPU) by MEC_TEST_ASSUME_CAPTURING=1
    monkeypatch.setenv("MEC_TEST_ASSUME_CAPTURING", "1")
    lib = _lib.load()
    n, d = 10, 64
    need = lib.mec_grad_scratch_bytes(n, d, 0)
    calls = {
        "mec_prepass": lambda: lib.mec_prepass(16, d, 16, d, n, d, 0, 1, 16, None),
        "mec_sumexp": lambda: lib.mec_sumexp(16, d, 16, d, n, d, 0, 0, 1, 0.07, 16, None),
        "mec_finalize": lambda: lib.mec_finalize(n, 0, 0.07, 16, 16, None),
        "mec_forward": lambda: lib.mec_forward(16, d, 16, d, n, d, 0, 0, 1, 0.07, 16, 16, None),
        "mec_grad_step": lambda: lib.mec_grad_step(16, d, 16, d, n, d, 0, 0, 1, 0.07, 16, 0, 16, need, 16, 16, None),
        "mec_grad": lambda: lib.mec_grad(16, d, 16, d, n, d, 0, 0, 1, 0.07, 16, 16, need, 16, 16, None),
        "mec_postpass": lambda: lib.mec_postpass(16, d, 16, d, n, d, 0, 0, 1, 1.0, 16, None, 16, 16, 16, 16, None),
        "mec_backward": lambda: lib.mec_backward(16, d, 16, d, n, d, 0, 0, 1, 0.07, 1.0, 16, None, 16, need, 16, 16,
                                                 16, 16, None),
        "mec_backward_noalloc": lambda: lib.mec_backward_noalloc(16, d, 16, d, n, d, 0, 0, 1, 0.07, 1.0, 16, None,
                                                                 16, 16, 16, 16, None),
    }
    for name, call in calls.items():
        assert call() == _lib.MEC_ERR_UNSUPPORTED, name
        assert "graph" in _lib.last_error(), (name, _lib.last_error())
    # argument errors still come first
    assert lib.mec_prepass(16, d, 16, d, 0, d, 0, 1, 16, None) == _lib.MEC_ERR_INVALID
