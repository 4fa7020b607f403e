"""Code generation of the built library (CPU: disassembles this build's own
gfx950 code object with the ROCm LLVM tools, no GPU needed).

The cache policies below are performance properties that the compiler can
drop without any change in results, so no parity test would notice:

* the gradient-matrix kernels (`k_grad_g_chain`, and the 16-bit
  `k_grad_step`) store G'^T non-temporally: every 16-byte store is a
  `buffer_store_dwordx4 ... nt`.  (`__builtin_nontemporal_store` once lost
  its hint in the one-plane case, which cost 3% of a config-4 step.)
* the contractions (`k_grad_contract`) load their gradient-matrix operand
  with direct-to-LDS loads carrying `nt`, and their other operand without.
* the kept-exponential kernels have no cache maintenance at all (the
  finalize's diagonal blocks meet in one atomic word that carries both their
  loss partials and their count): a full fence in every workgroup of the tile
  kernel invalidated the XCD's L2 under the workgroups still running and cost
  14 us of a 31 us launch, and a release/acquire handshake of the loss
  partials cost the finalize about 2 us.
* the kept-exponential forward's similarity stores and the contraction's
  output stores are at device scope (`sc1`, written through the L2), the
  finalize's in-place stores plain: measured, 1.2 us of the forward's 17 us and
  1.3 us of the contraction's 26 us at N = 1024, D = 512, and 0.7 us lost in
  the finalize.
* the kept-exponential finalize issues its loads back to back and waits for
  them once, and the fused backward's loads before the k-loop are not waited
  for before the k-loop's first barrier: written with predicates, the same
  loads compiled to a branch per load with waits in between (a memory round
  trip each), and the block sums' addition was hoisted above the k-loop with
  a wait for them (2-4 us per launch).
"""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "memoryefficientclip_amd", "lib", "libmec.so")
LLVM = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin")
TOOLS = {t: os.path.join(LLVM, t) for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump")}


def _disassembly():
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    missing = [t for t, p in TOOLS.items() if not os.path.exists(p)]
    if missing:
        pytest.skip(f"ROCm LLVM tools missing: {missing}")
    with tempfile.TemporaryDirectory() as tmp:
        fat = os.path.join(tmp, "fatbin.bin")
        co = os.path.join(tmp, "gfx950.o")
        subprocess.run([TOOLS["llvm-objcopy"], f"--dump-section=.hip_fatbin={fat}", LIB, os.devnull], check=True)
        subprocess.run([TOOLS["clang-offload-bundler"], "--unbundle", "--type=o", f"--input={fat}",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"], check=True)
        out = subprocess.run([TOOLS["llvm-objdump"], "-d", "--mcpu=gfx950", co], check=True,
                             capture_output=True, text=True).stdout
    # function symbol -> its instructions
    funcs, cur = {}, None
    for line in out.splitlines():
        m = re.match(r"^[0-9a-f]+ <(\S+)>:$", line)
        if m:
            cur = m.group(1)
            funcs[cur] = []
        elif cur is not None and line.strip():
            funcs[cur].append(line.strip())
    return funcs


@pytest.fixture(scope="module")
def funcs():
    return _disassembly()


def _select(funcs, prefix, exclude=()):
    sel = {k: v for k, v in funcs.items() if k.startswith(prefix) and not any(e in k for e in exclude)}
    assert sel, f"no kernels {prefix}*"
    return sel


def test_gradient_matrix_stores_are_non_temporal(funcs):
    # k_grad_g_chain<T, ...> and the 16-bit k_grad_step<T, ...> (T = bf16 bits `t`, fp16 `DF16_`)
    chain = _select(funcs, "_ZN3mec14k_grad_g_chain")
    step16 = {k: v for k, v in funcs.items()
              if k.startswith("_ZN3mec11k_grad_stepIt") or k.startswith("_ZN3mec11k_grad_stepIDF16_")}
    assert step16
    for name, body in {**chain, **step16}.items():
        stores = [l for l in body if "buffer_store_dwordx4" in l]
        assert stores, name
        assert all(re.search(r"\bnt\b", l) for l in stores), (name, [l for l in stores if " nt" not in l][:3])
        assert not any("global_store_dwordx4" in l for l in body), name


def test_contraction_streams_its_gradient_matrix_operand(funcs):
    for name, body in _select(funcs, "_ZN3mec15k_grad_contract").items():
        loads = [l for l in body if re.match(r"buffer_load_dwordx4 .* lds", l)]
        nt = [l for l in loads if re.search(r"\bnt\b", l)]
        assert nt and len(nt) < len(loads), (name, len(nt), len(loads))


def test_kept_exponential_kernels_need_no_fence(funcs):
    for prefix in ("_ZN3mec14k_keep_forward", "_ZN3mec15k_keep_finalize", "_ZN3mec15k_keep_contract"):
        for name, body in _select(funcs, prefix).items():
            assert not any(re.match(r"buffer_(inv|wbl2)", l) for l in body), name
    for name, body in _select(funcs, "_ZN3mec15k_keep_finalize").items():
        assert sum(bool(re.match(r"global_atomic_add_x2", l)) for l in body) == 1, name


def _max_tiles(name):
    # the kernels' last template argument: tile partials per row (16 or 32)
    m = re.search(r"ELi(\d+)EEEv", name)
    assert m, name
    return int(m.group(1))


def test_kept_exponential_loads_wait_once(funcs):
    fin = _select(funcs, "_ZN3mec15k_keep_finalize")
    assert sorted({_max_tiles(n) for n in fin}) == [16, 32]
    for name, body in fin.items():
        first_wait = next(i for i, l in enumerate(body) if re.match(r"s_waitcnt .*vmcnt", l))
        loads = [l for l in body[:first_wait] if l.startswith("global_load")]
        # the block, the tile sums, 4 workspace values
        assert len(loads) >= _max_tiles(name) + 4, (name, len(loads))
    fused = _select(funcs, "_ZN3mec15k_keep_contractILb1E")
    for name, body in fused.items():
        first_wait = next(i for i, l in enumerate(body) if re.match(r"s_waitcnt .*vmcnt", l))
        assert body[first_wait + 1].startswith("s_barrier"), (name, body[first_wait:first_wait + 2])
        # 16 tile values, the wave's block sums
        assert sum(l.startswith("global_load") for l in body[:first_wait]) >= 16 + _max_tiles(name) // 4, name


def test_kept_exponential_launch_results_store_at_device_scope(funcs):
    def stores(body, form):
        return [l for l in body if l.startswith(form + " ")]
    for name, body in _select(funcs, "_ZN3mec14k_keep_forward").items():
        sc1 = [l for l in stores(body, "global_store_dword") if re.search(r"\bsc1\b", l)]
        assert len(sc1) == 16, (name, len(sc1))  # the wave's 32 x 32 similarities, 16 per lane
    for name, body in _select(funcs, "_ZN3mec15k_keep_contract").items():
        st = stores(body, "global_store_dword")
        assert len(st) == 16 and all(re.search(r"\bsc1\b", l) for l in st), (name, st[:2])
    for name, body in _select(funcs, "_ZN3mec15k_keep_finalize").items():
        st = stores(body, "global_store_dwordx4")
        assert st and not any(re.search(r"\bsc[01]\b", l) for l in st), (name, st[:2])
