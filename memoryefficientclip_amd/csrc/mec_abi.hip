// C-ABI entry points (include/mec.h): argument validation in plain host code,
// then stream-ordered kernel launches.  Nothing here allocates device memory
// or synchronises the host.
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "mec.h"
#include "mec_keep.h"
#include "mec_kernels.h"
#include "mec_rowops.h"

using namespace mec;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

// Compute units of the current device (cached per device; callers on any
// thread may fill the cache, always with the same value).
int compute_units(int* cus) {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(MEC_ERR_HIP, "hipGetDevice failed");
  const bool cached = dev >= 0 && dev < 64;
  if (cached) {
    const int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) {
      *cus = v;
      return MEC_OK;
    }
  }
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 1)
    return fail(MEC_ERR_HIP, "hipDeviceGetAttribute(MultiprocessorCount) failed");
  if (cached) cache[dev].store(v, std::memory_order_relaxed);
  *cus = v;
  return MEC_OK;
}

// Gradient scratch of mec_backward_noalloc: one array per GPU, held until the
// process ends.  Host code never uses the name itself (on the host it is a
// stand-in, not a device address): noalloc_scratch() resolves this device's
// copy with hipGetSymbolAddress once per device.
constexpr int64_t kNoAllocScratch = MEC_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratch];

// Address of the current device's `scratch` (resolved on the first call on
// each device; callers on any thread may fill the cache, always with the
// same value).
int noalloc_scratch(void** out) {
  static std::atomic<void*> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(MEC_ERR_HIP, "hipGetDevice failed");
  const bool cached = dev >= 0 && dev < 64;
  if (cached) {
    void* p = cache[dev].load(std::memory_order_acquire);
    if (p) {
      *out = p;
      return MEC_OK;
    }
  }
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr)
    return fail(MEC_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
  if (cached) cache[dev].store(p, std::memory_order_release);
  *out = p;
  return MEC_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MEC_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return MEC_OK;
}

// Launches into a stream that is being captured into a HIP graph are
// refused (MEC_ERR_UNSUPPORTED, before any launch): capturing a step of the
// loss ended in a host segmentation fault during graph instantiation on the
// MI355X box, with no cause found in these launches.  A legacy default
// stream implicitly joined to another stream's capture counts as capturing.
// MEC_TEST_ASSUME_CAPTURING=1 makes the check report a capture without
// asking HIP (tests of this refusal on machines without a GPU).
int check_not_capturing(void* stream) {
  const char* env = std::getenv("MEC_TEST_ASSUME_CAPTURING");
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  const hipError_t e = (env && env[0] == '1') ? hipSuccess : hipStreamIsCapturing((hipStream_t)stream, &st);
  if ((env && env[0] == '1') || e == hipErrorStreamCaptureImplicit ||
      (e == hipSuccess && st != hipStreamCaptureStatusNone)) {
    if (e != hipSuccess) (void)hipGetLastError();
    return fail(MEC_ERR_UNSUPPORTED,
                "the stream is being captured into a HIP graph; graph capture of these kernels is not supported");
  }
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(MEC_ERR_HIP, "hipStreamIsCapturing: %s", hipGetErrorString(e));
  }
  return MEC_OK;
}

// Largest supported n, every dtype.  The 16-bit contractions address a
// 256-row panel of the transposed inputs ([d][ldt], ldt ~ n) with 32-bit
// buffer offsets, and the forward's grid of 128 x 128 fp32 tiles,
// (n / 128)^2 = 2^30 workgroups at this n, stays below 2^31.
constexpr int64_t kMaxN = int64_t(1) << 22;
constexpr int64_t kMaxD = int64_t(1) << 20;

bool known_dtype(int dtype) {
  return dtype == MEC_DTYPE_F32 || dtype == MEC_DTYPE_BF16 || dtype == MEC_DTYPE_F16 ||
         dtype == MEC_DTYPE_F32_BF16X3 || dtype == MEC_DTYPE_F32_BF16;
}
// fp32 data with bf16 products: bf16 terms per operand value in the
// similarity GEMMs (3: hi, lo; 1: hi), 0 for the other dtypes
int split_terms(int dtype) {
  return dtype == MEC_DTYPE_F32_BF16X3 ? 3 : dtype == MEC_DTYPE_F32_BF16 ? 1 : 0;
}
bool is_split(int dtype) { return split_terms(dtype) > 0; }
bool is_x3(int dtype) { return dtype == MEC_DTYPE_F32_BF16X3; }
// element type of the caller's x, y, dx, dy (the split modes read and write fp32)
int data_dtype(int dtype) { return is_split(dtype) ? MEC_DTYPE_F32 : dtype; }

int check_common(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d,
                 int dtype) {
  if (n < 1) return fail(MEC_ERR_INVALID, "n=%lld must be >= 1", (long long)n);
  if (n > kMaxN) return fail(MEC_ERR_UNSUPPORTED, "n=%lld exceeds the supported maximum 2^22", (long long)n);
  if (d < 1 || d > kMaxD) return fail(MEC_ERR_INVALID, "d=%lld out of range [1, 2^20]", (long long)d);
  if (ldx < d || ldy < d)
    return fail(MEC_ERR_INVALID, "row strides ldx=%lld ldy=%lld must be >= d=%lld", (long long)ldx,
                (long long)ldy, (long long)d);
  if (!known_dtype(dtype)) return fail(MEC_ERR_INVALID, "unknown dtype %d", dtype);
  if (x == nullptr || y == nullptr) return fail(MEC_ERR_INVALID, "x and y must be non-null");
  return MEC_OK;
}

// mode = MEC_MODE_CLIP or MEC_MODE_LIT, optionally OR MEC_FLAG_DETERMINISTIC
// and MEC_FLAG_KEEP_EXP
int check_mode(int mode) {
  const int base = mode & MEC_MODE_MASK, flags = mode & ~MEC_MODE_MASK;
  if ((base != MEC_MODE_CLIP && base != MEC_MODE_LIT) || (flags & ~(MEC_FLAG_DETERMINISTIC | MEC_FLAG_KEEP_EXP)))
    return fail(MEC_ERR_INVALID, "unknown mode %d", mode);
  return MEC_OK;
}

bool keep_flag(int mode) { return (mode & MEC_FLAG_KEEP_EXP) != 0; }
// the functions that run one stage have no kept-matrix variant
int check_no_keep(int mode, const char* fn) {
  if (keep_flag(mode))
    return fail(MEC_ERR_INVALID, "%s: MEC_FLAG_KEEP_EXP applies to mec_forward, mec_grad and mec_backward only", fn);
  return MEC_OK;
}

int check_temperature(float t) {
  if (!(t > 0.f) || !std::isfinite(t)) return fail(MEC_ERR_INVALID, "temperature must be finite and > 0");
  return MEC_OK;
}

bool is_lit(int mode) { return (mode & MEC_MODE_MASK) == MEC_MODE_LIT; }

// workspace: WS_NSLOTS vectors of n floats, the fp64 loss partials, then the
// (DET_Q + DET_P) x n partial sums of the deterministic forward
int64_t loss_partials_floats(int64_t n) { return 2 * ((n + FIN_ROWS - 1) / FIN_ROWS); }
int64_t det_partials_offset(int64_t n) { return (int64_t)WS_NSLOTS * n + loss_partials_floats(n); }
int64_t base_workspace_floats(int64_t n) { return det_partials_offset(n) + (int64_t)(DET_Q + DET_P) * n; }

// Split modes: the bf16 operands of the similarity GEMMs follow, 16-byte
// aligned: A (x rows) and B (y rows), n rows of ld = terms * dp bf16 each,
// dp = d rounded up to 8.  bf16x3: A rows hi | lo | hi, B rows hi | hi | lo
// (k_split3); bf16: A, B rows hi (k_split1).
int64_t split_dp(int64_t d) { return (d + 7) & ~int64_t(7); }
int64_t split_ld(int64_t d, int dtype) { return split_terms(dtype) * split_dp(d); }
int64_t split_offset_floats(int64_t n) { return (base_workspace_floats(n) + 3) & ~int64_t(3); }
int64_t workspace_floats_for(int64_t n, int64_t d, int dtype) {
  if (!is_split(dtype)) return base_workspace_floats(n);
  return split_offset_floats(n) + n * split_ld(d, dtype);  // 2 n ld bf16 = n ld floats
}
const uint16_t* split_a(const float* ws, int64_t n) { return (const uint16_t*)(ws + split_offset_floats(n)); }
const uint16_t* split_b(const float* ws, int64_t n, int64_t d, int dtype) {
  return split_a(ws, n) + n * split_ld(d, dtype);
}

// operands of the similarity GEMMs (forward sums, gradient-matrix tiles)
struct GemmOperands {
  const void* x;
  int64_t ldx;
  const void* y;
  int64_t ldy;
  int64_t d;   // K
  int dtype;   // element type of x, y
};
// split modes: the copies in the workspace, a bf16 problem with K = terms * dp
GemmOperands split_operands(const float* ws, int64_t n, int64_t d, int dtype) {
  const int64_t ld = split_ld(d, dtype);
  return GemmOperands{split_a(ws, n), ld, split_b(ws, n, d, dtype), ld, ld, MEC_DTYPE_BF16};
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The direct-to-LDS core addresses each operand panel with 32-bit byte
// offsets and masks with the offset 2^31, so a panel must span less than 2^31
// bytes: (rows - 1) * ld + kmax elements of esz bytes.  Panels have at most
// 256 rows (16-bit) or 128 rows (fp32).
int64_t dma_max_elems(int dtype) { return ((int64_t(1) << 31) - 1) / (dtype == MEC_DTYPE_F32 ? 4 : 2); }
int64_t dma_rows(int dtype) { return dtype == MEC_DTYPE_F32 ? 128 : 256; }

// 16-byte vector loads are legal when every row start is 16-byte aligned and
// rows hold a whole number of vectors; this also selects the direct-to-LDS
// core for the forward and gradient-matrix tiles, whose panels must fit its
// 32-bit offsets.
bool vec_ok(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t d, int dtype) {
  const int64_t per = dtype == MEC_DTYPE_F32 ? 4 : 8;
  if (!(aligned16(x) && aligned16(y) && d % per == 0 && ldx % per == 0 && ldy % per == 0)) return false;
  const int64_t ld = ldx > ldy ? ldx : ldy;
  return (dma_rows(dtype) - 1) * ld + d <= dma_max_elems(dtype);
}

// Kept exponentials (MEC_FLAG_KEEP_EXP): E and the forward's bookkeeping
// follow the dtype's workspace, each part 256-byte aligned (offsets in floats
// from the workspace start).
static_assert(KEEP_MAX_N == MEC_KEEP_EXP_MAX_N, "one limit");
bool keep_shape_ok(int64_t n, int dtype) { return dtype == MEC_DTYPE_F32 && n <= MEC_KEEP_EXP_MAX_N; }
int64_t align256b(int64_t floats) { return (floats + 63) & ~int64_t(63); }
struct KeepLayout {
  int np, kt;                                     // n rounded up to 64, np / 64
  int64_t s, rowpart, colpart, rowdot, coldot, lacc, total;
};
KeepLayout keep_layout(int64_t n, int64_t d, int dtype) {
  KeepLayout L;
  L.kt = (int)((n + KEEP_T - 1) / KEEP_T);
  L.np = L.kt * KEEP_T;
  const int64_t np = L.np;
  int64_t o = align256b(workspace_floats_for(n, d, dtype));
  L.s = o;
  o = align256b(o + np * np);
  L.rowpart = o;
  o = align256b(o + L.kt * np);
  L.colpart = o;
  o = align256b(o + L.kt * np);
  L.rowdot = o;
  o = align256b(o + L.kt * np);
  L.coldot = o;
  o = align256b(o + L.kt * np);
  L.lacc = o;  // one 64-bit word
  L.total = o + 2;
  return L;
}
int64_t workspace_floats_mode(int64_t n, int64_t d, int dtype, int mode) {
  return keep_flag(mode) ? keep_layout(n, d, dtype).total : workspace_floats_for(n, d, dtype);
}
KeepBufs keep_bufs(const float* workspace, const KeepLayout& L) {
  float* ws = const_cast<float*>(workspace);
  return KeepBufs{ws + L.s,      ws + L.rowpart, ws + L.colpart, ws + L.rowdot,
                  ws + L.coldot, (unsigned long long*)(ws + L.lacc), L.np, L.kt};
}
// MEC_KEEP_EXP=0 reports no support (the glue asks before it sets the flag;
// tests of the other path)
bool keep_supported(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype) {
  if (const char* env = std::getenv("MEC_KEEP_EXP"))
    if (env[0] == '0') return false;
  return n >= 1 && d >= 1 && x && y && ldx >= d && ldy >= d && keep_shape_ok(n, dtype) &&
         vec_ok(x, ldx, y, ldy, d, dtype);
}
int check_keep(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
               const float* workspace) {
  if (!keep_supported(x, ldx, y, ldy, n, d, dtype))
    return fail(MEC_ERR_INVALID,
                "MEC_FLAG_KEEP_EXP needs MEC_DTYPE_F32, n <= %d and 16-byte aligned rows (mec_keep_exp_supported)",
                MEC_KEEP_EXP_MAX_N);
  if (!aligned16(workspace)) return fail(MEC_ERR_INVALID, "MEC_FLAG_KEEP_EXP needs a 16-byte aligned workspace");
  return MEC_OK;
}

// Block decomposition of the N x N gradient matrix for the backward: nb
// blocks of tb quanta of q rows (q = block_quantum: 128 for fp32, 256 for
// the bf16 kernels, so every tile kind divides a block).  Longer blocks mean
// fewer pipeline launches and fewer fp32 accumulator updates through HBM
// (one per launch); the scratch grows as n * bs.  Targets, measured on the
// 128-byte ring:
//   fp32: bs ~ 4d (headline shape: backward 53.2 ms with 2048-row blocks,
//         52.4 ms with 4096);
//   bf16 kernels: bs ~ 8d, or ~16d when n >= 8192 and 8d would give fewer
//         than 16 blocks (n = 65536, d = 768: backward 19.0 -> 18.2 ms with
//         16384-row blocks; n = 262144, d = 1152: 440 ms either way, so the
//         smaller scratch is kept).
// An exact divisor of the quantum count within a factor of two of the
// target is preferred (no short last block, whose contractions would have a
// short K); otherwise the quanta are balanced over the blocks.
//
// The target is at least 1024 rows (fewer launches for a small d).
//
// Memory bound: the gradient-matrix buffers (nbuf x planes x nb x bs^2
// elements, about nbuf x planes x n x bs; nbuf = 2 double-buffered
// diagonals, or 1 when a single block covers n) are kept within `gbudget`
// bytes by shortening the blocks, never below one quantum.  The default
// budget is O(n d): 64 n d scratch elements (32 times the two inputs in the
// scratch element type), at least 256 MiB (so that small problems keep long
// blocks and few launches) and at most 16 GiB; it wins over the 1024-row
// target.
int g_planes(int dtype) { return is_x3(dtype) ? 2 : 1; }
int64_t g_elem(int dtype) { return dtype == MEC_DTYPE_F32 ? 4 : 2; }
// bytes of the gradient-matrix buffers for blocks of tb quanta
int64_t g_bytes(int64_t tiles, int64_t q, int64_t tb, int dtype) {
  const int64_t nb = (tiles + tb - 1) / tb, bs = tb * q;
  return (nb > 1 ? 2 : 1) * g_planes(dtype) * nb * bs * bs * g_elem(dtype);
}
constexpr int64_t kGradBudgetCap = int64_t(16) << 30;
constexpr int64_t kGradBudgetMin = int64_t(256) << 20;
constexpr int64_t kGradBudgetRatio = 64;
constexpr int64_t kTargetMinRows = 1024;
int64_t default_gbudget(int64_t n, int64_t d, int dtype) {
  int64_t b = kGradBudgetRatio * n * d * g_elem(dtype);
  if (b < kGradBudgetMin) b = kGradBudgetMin;
  return b < kGradBudgetCap ? b : kGradBudgetCap;
}
void grad_blocks_budget(int64_t n, int64_t d, int dtype, int64_t gbudget, int* bs, int* nb) {
  const int64_t q = block_quantum(dtype);
  const int64_t tiles = (n + q - 1) / q;
  // The y side of fp32 reads a gradient-matrix block transposed with 32-bit
  // offsets ((bs - 1) * bs + 128 floats within 2^31 bytes: bs <= 16384); the
  // 16-bit contractions read a transposed block as a direct-to-LDS operand
  // ((bs - 1) * bs + 256 elements within 2^31 bytes: bs <= 127 * 256).
  int64_t cap = dtype == MEC_DTYPE_F32 ? 128 : 127;
  if (cap > tiles) cap = tiles;
  // the longest blocks within the budget (at least one quantum): an
  // estimate from the double-buffered size, then a short walk down
  {
    int64_t tb = cap;
    if (g_bytes(tiles, q, tb, dtype) > gbudget) {
      const int64_t per_tb = 2 * (int64_t)g_planes(dtype) * tiles * q * q * g_elem(dtype);
      if (gbudget / per_tb < tb) tb = gbudget / per_tb;
      if (tb < 1) tb = 1;
      while (tb > 1 && g_bytes(tiles, q, tb, dtype) > gbudget) --tb;
    }
    cap = tb;
  }
  int64_t mult = dtype == MEC_DTYPE_F32 ? 4 : 8;
  if (dtype != MEC_DTYPE_F32 && n >= 8192 && n < 16 * 8 * d) mult = 16;
  // at least 1024 rows (below that the pipeline's launches and accumulator
  // updates dominate), where the budget allows
  const int64_t target_rows = mult * d > kTargetMinRows ? mult * d : kTargetMinRows;
  int64_t target = (target_rows + q - 1) / q;
  if (const char* env = std::getenv("MEC_GRAD_BLOCK_TILES")) {
    long v = std::strtol(env, nullptr, 10);
    if (v >= 1 && v <= 4096) target = v;
  }
  if (target > cap) target = cap;
  int64_t tb;
  if (target >= tiles) {
    tb = tiles;
  } else {
    int64_t best = -1;
    for (int64_t c = (target + 1) / 2; c <= 2 * target && c <= tiles && c <= cap; ++c) {
      if (tiles % c) continue;
      const int64_t dc = c > target ? c - target : target - c;
      const int64_t db = best > target ? best - target : target - best;
      if (best < 0 || dc < db || (dc == db && c > best)) best = c;
    }
    if (best > 0) {
      tb = best;
    } else {
      const int64_t nbv = (tiles + target - 1) / target;
      tb = (tiles + nbv - 1) / nbv;
    }
  }
  // balanced blocks may round past the budget: shorten them (not below a quantum)
  while (tb > 1 && g_bytes(tiles, q, tb, dtype) > gbudget) --tb;
  *bs = (int)(tb * q);
  *nb = (int)((tiles + tb - 1) / tb);
}
void grad_blocks(int64_t n, int64_t d, int dtype, int* bs, int* nb) {
  grad_blocks_budget(n, d, dtype, default_gbudget(n, d, dtype), bs, nb);
}

// Sides of the backward: the x side (acc_x, dx) and the y side (CLIP only)
constexpr int kSideX = MEC_SIDE_X, kSideY = MEC_SIDE_Y;

// Scratch layout of the backward (elements: fp32 for MEC_DTYPE_F32, else
// 16-bit), for the sides that are computed:
//   fp32:                  [H0 | H1]
//   bf16, fp16, fp32/bf16: [GT0 | GT1 | XT | YT]
//   bf16x3:                [GT0 | GT1 | GTlo0 | GTlo1 | XT | XTlo | YT | YTlo]
// H0/H1 double-buffer one block diagonal of H = diag(rx) G' diag(ry) (nb
// blocks of bs x bs, row-major); GT0/GT1 the 16-bit types' transposed blocks
// of G' in the blocked layout gdma::gb_offset (bf16x3: hi and lo planes).
// With a single block (nb = 1) only buffer 0 exists.  XT/YT are the
// normalised inputs transposed, [d][ldt] with ldt = n rounded up to 128
// (bf16x3: hi and lo planes), only for the sides computed: YT for the x
// side, XT for the y side.  fp32 reads its raw inputs instead.
struct ScratchLayout {
  int bs, nb;
  int nbuf;            // gradient-matrix diagonals held: 2, or 1 with one block
  int planes;          // planes per diagonal (bf16x3: hi and lo)
  int ntp;             // transposed planes per side (0 for fp32; bf16x3: 2)
  int64_t ldt;         // elements
  int64_t gbuf, tbuf;  // bytes of one diagonal plane / one transposed plane
  int64_t xt, yt;      // byte offsets of XT and YT (-1: not held)
  int64_t total;
};
ScratchLayout scratch_layout_blocks(int64_t n, int64_t d, int dtype, int sides, int bs, int nb) {
  ScratchLayout L;
  L.bs = bs;
  L.nb = nb;
  const int64_t elem = g_elem(dtype);
  L.nbuf = nb > 1 ? 2 : 1;
  L.planes = g_planes(dtype);
  L.ntp = dtype == MEC_DTYPE_F32 ? 0 : (is_x3(dtype) ? 2 : 1);
  L.ldt = (n + 127) / 128 * 128;
  L.gbuf = (int64_t)L.nb * L.bs * L.bs * elem;
  L.tbuf = d * L.ldt * elem;
  int64_t off = (int64_t)L.nbuf * L.planes * L.gbuf;
  L.xt = L.yt = -1;
  if (L.ntp > 0 && (sides & kSideY)) {
    L.xt = off;
    off += L.ntp * L.tbuf;
  }
  if (L.ntp > 0 && (sides & kSideX)) {
    L.yt = off;
    off += L.ntp * L.tbuf;
  }
  L.total = off;
  return L;
}
ScratchLayout scratch_layout(int64_t n, int64_t d, int dtype, int sides) {
  int bs, nb;
  grad_blocks(n, d, dtype, &bs, &nb);
  return scratch_layout_blocks(n, d, dtype, sides, bs, nb);
}
// transposed-input bytes of the scratch for these sides
int64_t trans_bytes(int64_t n, int64_t d, int dtype, int sides) {
  return scratch_layout_blocks(n, d, dtype, sides, 0, 1).total;
}

// The blocking and layout of mec_backward_noalloc: the default blocking when
// its scratch fits the array, else shorter blocks within what the transposed
// inputs leave of it (not below one quantum); ok = false when even that does
// not fit.
ScratchLayout noalloc_layout(int64_t n, int64_t d, int dtype, int sides, bool* ok) {
  const int64_t trans = trans_bytes(n, d, dtype, sides);
  int64_t gbudget = kNoAllocScratch - trans;
  if (gbudget > default_gbudget(n, d, dtype)) gbudget = default_gbudget(n, d, dtype);
  int bs = block_quantum(dtype), nb = 1;
  if (gbudget > 0) grad_blocks_budget(n, d, dtype, gbudget, &bs, &nb);
  const ScratchLayout L = scratch_layout_blocks(n, d, dtype, sides, bs, nb);
  *ok = gbudget > 0 && L.total <= kNoAllocScratch;
  return L;
}

int round8(int v) { return (v + 7) & ~7; }

// 64 x 64 fp32 tiles of the forward (f32_small_fwd) and of the backward's
// steps (f32_small_bwd); MEC_F32_SMALL_TILES=0 or 1 overrides both, for tests
int small_tiles_env() {
  if (const char* env = std::getenv("MEC_F32_SMALL_TILES")) {
    if (env[0] == '0') return 0;
    if (env[0] == '1') return 1;
  }
  return -1;
}
bool f32_small_fwd_tiles(int64_t n, int64_t d, int cus) {
  const int e = small_tiles_env();
  return e >= 0 ? e == 1 : f32_small_fwd(n, d, cus);
}
bool f32_small_bwd_tiles(int64_t n, int64_t d, int64_t bs, int cus) {
  const int e = small_tiles_env();
  return e >= 0 ? e == 1 : f32_small_bwd(n, d, bs, cus);
}

// 16-bit narrow contraction tiles (narrow_contract_shape) for blocks of bs
// rows whose contraction launch has `wide` workgroups of 256 x 256 tiles,
// `narrow` with them, on `cus` compute units.  Used where they measured
// faster: a 512-row panel of the gradient-matrix block (512 x bs x 2 bytes)
// within one XCD's 4 MB L2, i.e. bs <= 4096 (7-13% less contraction time at
// D = 128-640; with larger blocks the narrow tiles fall out of step with the
// wide tiles that share their panel and read it from HBM: 2-11% more), and
// fewer rounds of workgroups over the CUs than the wide tiles alone.
// MEC_NARROW_CONTRACT=0 / 1 turns them off / on wherever the shape allows
// (tests).
bool narrow_contract_use(int bs, int64_t wide, int64_t narrow, int cus) {
  if (const char* env = std::getenv("MEC_NARROW_CONTRACT")) {
    if (env[0] == '0') return false;
    if (env[0] == '1') return true;
  }
  if (bs > 4096 || cus <= 0) return false;
  return (narrow + cus - 1) / cus < (wide + cus - 1) / cus;
}

// 16-bit contraction tiles 384 features wide (ConTileSel::wx / wy; 1.5 times
// the work of a 256 x 256 tile) for a launch of t384 such tiles instead of
// t256 tiles of 256 x 256 (or the narrow ones): where they take fewer
// tile-rounds of work over the compute units, or as many.  At D = 1152
// (config 5) the 256-wide tiles spend a tenth of the launch on a half-empty
// fifth feature column (8.92 -> 7.80 ms per launch); at equal rounds the
// 384-wide tiles' lower share of loads per MFMA wins (N = 65536, D = 768: 2.68
// -> 2.49 ms; D = 1536: 5.28 -> 4.98 ms); with more rounds they lose (D = 512
// and D = 300: 16-23% slower).  A 384-wide tile reads a 384-row panel of a
// transposed input with 32-bit offsets ((383 ldt + bs) x 2 bytes below 2^31,
// ldt up to about 2.8M): beyond that only the 256-wide tiles (whose 256-row
// panels fit up to n = 2^22) are used.  MEC_WIDE_CONTRACT=0 / 1 turns them
// off / on for every D where the panel fits (tests).
bool wide_contract_fits(int64_t ldt, int64_t bs) { return (383 * ldt + bs) * 2 < (int64_t(1) << 31); }
bool wide_contract_use(int64_t t384, int64_t t256, int64_t ldt, int64_t bs, int cus) {
  if (!wide_contract_fits(ldt, bs)) return false;
  if (const char* env = std::getenv("MEC_WIDE_CONTRACT")) {
    if (env[0] == '0') return false;
    if (env[0] == '1') return true;
  }
  if (cus <= 0) return false;
  const int64_t r384 = (t384 + cus - 1) / cus, r256 = (t256 + cus - 1) / cus;
  return 3 * r384 <= 2 * r256;
}

// Tile grid of a backward launch: gradient-matrix tiles of tf, contraction
// tiles of tc; the 16-bit types choose narrow or 384-wide contraction tiles
// for the launch's `sides` (on `cus` compute units).
BlockGrid block_grid(int64_t d, int dtype, int sides, int bs, int nb, int64_t ldt, int cus, TileDims tf, TileDims tc,
                     bool* w384) {
  const int D = (int)d;
  BlockGrid bg{bs, nb, bs / tf.bm, bs / tf.bn, bs / tc.bm, (D + tc.bn - 1) / tc.bn, 0};
  *w384 = false;
  if (separate_contractions(dtype)) {
    const int64_t nsides = ((sides & kSideX) ? 1 : 0) + ((sides & kSideY) ? 1 : 0);
    const int64_t wide = nsides * nb * bg.ctm * bg.ctd;
    int64_t tiles = wide;
    if (narrow_contract_shape(D, bg.ctm)) {
      const int64_t narrow = nsides * nb * (bg.ctm / 2) * (2 * (D / tc.bn) + 1);
      if (narrow_contract_use(bs, wide, narrow, cus)) {
        bg.ctd = D / tc.bn;
        bg.cnw = 1;
        tiles = narrow;
      }
    }
    const int ctd384 = (D + 383) / 384;
    if (wide_contract_use(nsides * nb * bg.ctm * ctd384, tiles, ldt, bs, cus)) {
      *w384 = true;
      bg.ctd = ctd384;
      bg.cnw = 0;
    }
  }
  return bg;
}

// T = element type of dtype: float, bf16 bits (uint16_t) or fp16 (_Float16);
// callers map the split modes to float first (data_dtype)
#define DISPATCH_DTYPE(dtype, T, ...)       \
  do {                                      \
    if ((dtype) == MEC_DTYPE_F32) {         \
      using T = float;                      \
      __VA_ARGS__;                          \
    } else if ((dtype) == MEC_DTYPE_BF16) { \
      using T = uint16_t;                   \
      __VA_ARGS__;                          \
    } else {                                \
      using T = _Float16;                   \
      __VA_ARGS__;                          \
    }                                       \
  } while (0)

#define DISPATCH_BOOL(cond, NAME, ...) \
  do {                                 \
    if (cond) {                        \
      constexpr bool NAME = true;      \
      __VA_ARGS__;                     \
    } else {                           \
      constexpr bool NAME = false;     \
      __VA_ARGS__;                     \
    }                                  \
  } while (0)

}  // namespace

extern "C" {

const char* mec_last_error(void) { return g_err.c_str(); }

const char* mec_version(void) { return "memoryefficientclip_amd 0.1.0 gfx950"; }

int64_t mec_workspace_floats(int64_t n) {
  if (n < 1 || n > kMaxN) return -1;
  return base_workspace_floats(n);
}

int64_t mec_workspace_floats_for(int64_t n, int64_t d, int dtype) {
  if (n < 1 || n > kMaxN || d < 1 || d > kMaxD || !known_dtype(dtype)) return -1;
  return workspace_floats_for(n, d, dtype);
}

int64_t mec_workspace_floats_mode(int64_t n, int64_t d, int dtype, int mode) {
  if (n < 1 || n > kMaxN || d < 1 || d > kMaxD || !known_dtype(dtype)) return -1;
  if (check_mode(mode) != MEC_OK) return -1;
  if (keep_flag(mode) && !keep_shape_ok(n, dtype)) return -1;
  return workspace_floats_mode(n, d, dtype, mode);
}

int mec_keep_exp_supported(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d,
                           int dtype) {
  return keep_supported(x, ldx, y, ldy, n, d, dtype) ? 1 : 0;
}

int64_t mec_grad_scratch_bytes(int64_t n, int64_t d, int dtype) {
  if (n < 1 || n > kMaxN || d < 1 || d > kMaxD) return -1;
  if (!known_dtype(dtype)) return -1;
  return scratch_layout(n, d, dtype, kSideX | kSideY).total;
}

int64_t mec_grad_scratch_bytes_for(int64_t n, int64_t d, int dtype, int mode, int sides) {
  if (n < 1 || n > kMaxN || d < 1 || d > kMaxD || !known_dtype(dtype)) return -1;
  if (check_mode(mode) != MEC_OK) return -1;
  if (is_lit(mode)) sides &= kSideX;
  if (sides < 1 || sides > (kSideX | kSideY)) return -1;
  if (keep_flag(mode)) return keep_shape_ok(n, dtype) ? 0 : -1;  // contracts the kept matrix
  return scratch_layout(n, d, dtype, sides).total;
}

int mec_backward_plan(int64_t n, int64_t d, int dtype, int mode, int sides, int cus, mec_backward_plan_t* plan) {
  g_err.clear();
  if (n < 1 || d < 1 || d > kMaxD) return fail(MEC_ERR_INVALID, "n or d out of range");
  if (n > kMaxN) return fail(MEC_ERR_UNSUPPORTED, "n=%lld exceeds the supported maximum 2^22", (long long)n);
  if (!known_dtype(dtype)) return fail(MEC_ERR_INVALID, "unknown dtype %d", dtype);
  int rc = check_mode(mode);
  if (rc) return rc;
  if (is_lit(mode)) sides &= kSideX;
  if (sides < 1 || sides > (kSideX | kSideY)) return fail(MEC_ERR_INVALID, "sides must name the x or y side");
  if (!plan) return fail(MEC_ERR_INVALID, "plan must be non-null");
  if (keep_flag(mode)) {
    // one block, no scratch, 64 x 64 contraction tiles
    if (!keep_shape_ok(n, dtype))
      return fail(MEC_ERR_INVALID, "MEC_FLAG_KEEP_EXP needs MEC_DTYPE_F32 and n <= %d", MEC_KEEP_EXP_MAX_N);
    const KeepLayout K = keep_layout(n, d, dtype);
    plan->block_rows = plan->noalloc_block_rows = K.np;
    plan->num_blocks = 1;
    plan->scratch_bytes = plan->noalloc_scratch_bytes = 0;
    plan->contract_tile_rows = plan->contract_tile_features = KEEP_T;
    plan->narrow_tiles = 0;
    return MEC_OK;
  }
  if (cus <= 0) {
    rc = compute_units(&cus);
    if (rc) return rc;
  }
  const ScratchLayout L = scratch_layout(n, d, dtype, sides);
  plan->block_rows = L.bs;
  plan->num_blocks = L.nb;
  plan->scratch_bytes = L.total;
  // the tiles of a launch with contractions (16-byte rows assumed)
  const int gdt = is_split(dtype) ? MEC_DTYPE_BF16 : dtype;
  const bool small = gdt == MEC_DTYPE_F32 && f32_small_bwd_tiles(n, d, L.bs, cus);
  bool w384 = false;
  const BlockGrid bg = block_grid(d, gdt, sides, L.bs, L.nb, L.ldt, cus, fwd_tile_dims(gdt, true, small),
                                  con_tile_dims(gdt, small), &w384);
  plan->contract_tile_rows = con_tile_dims(gdt, small).bm;
  plan->contract_tile_features = w384 ? 384 : con_tile_dims(gdt, small).bn;
  plan->narrow_tiles = bg.cnw;
  bool ok = false;
  const ScratchLayout Ln = noalloc_layout(n, d, dtype, sides, &ok);
  plan->noalloc_block_rows = ok ? Ln.bs : -1;
  plan->noalloc_scratch_bytes = ok ? Ln.total : -1;
  return MEC_OK;
}

int mec_prepass(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
                int normalize, float* workspace, void* stream) {
  g_err.clear();
  int rc = check_common(x, ldx, y, ldy, n, d, dtype);
  if (rc) return rc;
  if (!workspace) return fail(MEC_ERR_INVALID, "workspace must be non-null");
  if (is_split(dtype) && !aligned16(workspace))
    return fail(MEC_ERR_INVALID, "workspace must be 16-byte aligned for the bf16-product modes");
  rc = check_not_capturing(stream);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  const int N = (int)n, D = (int)d;
  dim3 grid((unsigned)((n + 3) / 4));
  DISPATCH_DTYPE(data_dtype(dtype), T, DISPATCH_BOOL(normalize, NORM,
      k_prepass<T, NORM><<<grid, 256, 0, s>>>((const T*)x, ldx, (const T*)y, ldy, N, D, workspace)));
  if (is_split(dtype)) {
    // bf16 (split) copies of x and y for the similarity GEMMs (the norms and
    // the diagonal above come from the fp32 inputs)
    const int64_t dp = split_dp(d), ld = split_ld(d, dtype);
    const int64_t nthr = n * (dp / 8);
    if ((nthr + 255) / 256 > 0x7fffffff) return fail(MEC_ERR_UNSUPPORTED, "split grid too large");
    const unsigned sgrid = (unsigned)((nthr + 255) / 256);
    uint16_t* sa = (uint16_t*)split_a(workspace, n);
    uint16_t* sb = (uint16_t*)split_b(workspace, n, d, dtype);
    // (normalize: of x^ and y^, scaled by the norms just computed, so that the
    // GEMM kernels run without the norm scaling)
    const float* rx = workspace + WS_RX * n;
    const float* ry = workspace + WS_RY * n;
    DISPATCH_BOOL(normalize, NORM, {
      if (is_x3(dtype)) {
        k_split3<0, NORM><<<sgrid, 256, 0, s>>>((const float*)x, ldx, N, D, (int)dp, sa, ld, rx);
        k_split3<1, NORM><<<sgrid, 256, 0, s>>>((const float*)y, ldy, N, D, (int)dp, sb, ld, ry);
      } else {
        k_split1<NORM><<<sgrid, 256, 0, s>>>((const float*)x, ldx, N, D, (int)dp, sa, ld, rx);
        k_split1<NORM><<<sgrid, 256, 0, s>>>((const float*)y, ldy, N, D, (int)dp, sb, ld, ry);
      }
    });
  }
  return check_launch("prepass");
}

int mec_sumexp(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
               int mode, int normalize, float temperature, float* workspace, void* stream) {
  g_err.clear();
  int rc = check_common(x, ldx, y, ldy, n, d, dtype);
  if (!rc) rc = check_mode(mode);
  if (!rc) rc = check_no_keep(mode, "mec_sumexp");
  if (!rc) rc = check_temperature(temperature);
  if (rc) return rc;
  if (!workspace) return fail(MEC_ERR_INVALID, "workspace must be non-null");
  if (is_split(dtype) && !aligned16(workspace))
    return fail(MEC_ERR_INVALID, "workspace must be 16-byte aligned for the bf16-product modes");
  rc = check_not_capturing(stream);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  const float c = (float)(1.4426950408889634 / (double)temperature);
  // split modes: the bf16 sums over the copies (K = terms * dp) that mec_prepass
  // wrote, already normalized when normalize is set
  GemmOperands g{x, ldx, y, ldy, d, dtype};
  if (is_split(dtype)) {
    g = split_operands(workspace, n, d, dtype);
    normalize = 0;
  }
  x = g.x, ldx = g.ldx, y = g.y, ldy = g.ldy, d = g.d, dtype = g.dtype;
  const int N = (int)n, D = (int)d;
  const bool vec = vec_ok(x, ldx, y, ldy, d, dtype);
  // Deterministic sums on request, and always for the 16-bit direct-to-LDS
  // tiles without the norm scaling (FwdChain), whose chained block walk is
  // faster than the atomic forward.  They keep the default tile size.
  bool chain = false;
  DISPATCH_DTYPE(dtype, T, DISPATCH_BOOL(normalize, NORM, DISPATCH_BOOL(vec, VEC, {
    chain = FwdChain<T, VEC, NORM>::value;
  })));
  const bool det = (mode & MEC_FLAG_DETERMINISTIC) || chain;
  int cus = 0;
  if (dtype == MEC_DTYPE_F32 && vec && !det) {
    rc = compute_units(&cus);
    if (rc) return rc;
  }
  const bool small = dtype == MEC_DTYPE_F32 && vec && !det && f32_small_fwd_tiles(n, d, cus);
  const TileDims td = fwd_tile_dims(dtype, vec, small);
  const int tiles_m = (int)((n + td.bm - 1) / td.bm), tiles_n = (int)((n + td.bn - 1) / td.bn);
  const int64_t nwg = (int64_t)tiles_m * tiles_n;
  if (nwg > 0x7fffffff) return fail(MEC_ERR_UNSUPPORTED, "forward grid too large");
  const bool lit = is_lit(mode);
  if (det) {
    // one pass over the tile grid in P x Q blocks, then the partials in order
    const int64_t n64 = n;
    float* rowpart = workspace + det_partials_offset(n);
    float* colpart = rowpart + (int64_t)DET_Q * n64;
    const int P = tiles_m < DET_P ? tiles_m : DET_P, Q = tiles_n < DET_Q ? tiles_n : DET_Q;
    const unsigned sum_grid = (unsigned)((n + 255) / 256);
    DISPATCH_DTYPE(dtype, T, DISPATCH_BOOL(lit, LIT, DISPATCH_BOOL(normalize, NORM, DISPATCH_BOOL(vec, VEC, {
      k_sumexp_det<T, LIT, NORM, VEC><<<(unsigned)(P * Q), FwdTile<T, VEC>::NT, 0, s>>>(
          (const T*)x, ldx, (const T*)y, ldy, N, D, D, c, workspace + WS_RX * n64, workspace + WS_RY * n64, rowpart,
          colpart, tiles_m, tiles_n, P, Q);
      k_det_reduce<LIT><<<sum_grid, 256, 0, s>>>(rowpart, Q, colpart, P, N, workspace + WS_ROW_OFF * n64,
                                                 workspace + WS_COL_OFF * n64);
    }))));
    return check_launch("sumexp (deterministic)");
  }
  dim3 grid((unsigned)nwg);
  DISPATCH_DTYPE(dtype, T, DISPATCH_BOOL(lit, LIT, DISPATCH_BOOL(normalize, NORM, DISPATCH_BOOL(vec, VEC, {
    if constexpr (!FwdChain<T, VEC, NORM>::value) {
      if (small) {
        if constexpr (std::is_same<T, float>::value && VEC)
          k_sumexp<T, LIT, NORM, VEC, true><<<grid, GemmTile<T, VEC, true>::NT, 0, s>>>(
              (const T*)x, ldx, (const T*)y, ldy, N, D, D, c, workspace, tiles_m, tiles_n);
      } else {
        k_sumexp<T, LIT, NORM, VEC><<<grid, FwdTile<T, VEC>::NT, 0, s>>>(
            (const T*)x, ldx, (const T*)y, ldy, N, D, D, c, workspace, tiles_m, tiles_n);
      }
    }
  }))));
  return check_launch("sumexp");
}

int mec_finalize(int64_t n, int mode, float temperature, float* workspace, float* loss, void* stream) {
  g_err.clear();
  if (n < 1) return fail(MEC_ERR_INVALID, "n=%lld must be >= 1", (long long)n);
  if (n > kMaxN) return fail(MEC_ERR_UNSUPPORTED, "n=%lld exceeds the supported maximum 2^22", (long long)n);
  int rc = check_mode(mode);
  if (!rc) rc = check_no_keep(mode, "mec_finalize");
  if (!rc) rc = check_temperature(temperature);
  if (rc) return rc;
  if (!workspace || !loss) return fail(MEC_ERR_INVALID, "workspace and loss must be non-null");
  if (reinterpret_cast<uintptr_t>(workspace) & 7u) return fail(MEC_ERR_INVALID, "workspace must be 8-byte aligned");
  rc = check_not_capturing(stream);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  const double inv_t = 1.0 / (double)temperature;
  const int nparts = (int)((n + FIN_ROWS - 1) / FIN_ROWS);
  // partials after the 8 slots (8 n floats: 8-byte aligned when the workspace is)
  double* partial = (double*)(workspace + (int64_t)WS_NSLOTS * n);
  DISPATCH_BOOL(is_lit(mode), LIT, {
    if (n <= FIN_SINGLE_ROWS) {
      k_finalize_rows<LIT, true><<<1, FIN_SINGLE_ROWS, 0, s>>>((int)n, inv_t, workspace, partial, loss);
    } else {
      k_finalize_rows<LIT, false><<<nparts, FIN_ROWS, 0, s>>>((int)n, inv_t, workspace, partial, loss);
      k_finalize_sum<LIT><<<1, 1024, 0, s>>>((int)n, nparts, partial, loss);
    }
  });
  return check_launch("finalize");
}

int mec_forward(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
                int mode, int normalize, float temperature, float* workspace, float* loss, void* stream) {
  g_err.clear();
  int rc = check_common(x, ldx, y, ldy, n, d, dtype);
  if (!rc) rc = check_mode(mode);
  if (!rc) rc = check_temperature(temperature);
  if (rc) return rc;
  if (!workspace || !loss) return fail(MEC_ERR_INVALID, "workspace and loss must be non-null");
  if (keep_flag(mode)) {
    rc = check_keep(x, ldx, y, ldy, n, d, dtype, workspace);
    if (!rc) rc = check_not_capturing(stream);
    if (rc) return rc;
    // the similarity tiles (norms, diagonal, similarities, per-tile sums),
    // then the finalize (sums, loss, similarities -> H, sums of G' cos)
    const KeepLayout L = keep_layout(n, d, dtype);
    const KeepBufs kb = keep_bufs(workspace, L);
    hipStream_t s = (hipStream_t)stream;
    const int N = (int)n, D = (int)d;
    const float c = (float)(1.4426950408889634 / (double)temperature);
    const double inv_t = 1.0 / (double)temperature;
    // fixed-point units of the loss partials: every loss term is at most
    // ln n + 2/T for |cos| <= 1, so the total is at most B = (2n or n)(ln n +
    // 2/T); lscale = 2^floor(log2(2^51 / B)) keeps it within KEEP_LOSS_CAP
    const double bound = (is_lit(mode) ? 1.0 : 2.0) * (double)n * (std::log((double)n) + 2.0 * inv_t) + 1.0;
    const double lscale = std::ldexp(1.0, (int)std::floor(std::log2(std::ldexp(1.0, 51) / bound)));
    const unsigned grid = (unsigned)(kb.kt * kb.kt);
    DISPATCH_BOOL(is_lit(mode), LIT, DISPATCH_BOOL(normalize, NORM, {
      k_keep_forward<LIT, NORM><<<grid, KEEP_NT, 0, s>>>((const float*)x, ldx, (const float*)y, ldy, N, D, c,
                                                         workspace, kb);
      DISPATCH_BOOL(kb.kt <= 16, SMALLT, {
        k_keep_finalize<LIT, NORM, SMALLT ? 16 : KEEP_MAX_KT><<<grid, 256, 0, s>>>(N, c, inv_t, lscale, workspace,
                                                                                 kb, loss);
      });
    }));
    return check_launch("forward (kept exponentials)");
  }
  rc = mec_prepass(x, ldx, y, ldy, n, d, dtype, normalize, workspace, stream);
  if (!rc) rc = mec_sumexp(x, ldx, y, ldy, n, d, dtype, mode, normalize, temperature, workspace, stream);
  if (!rc) rc = mec_finalize(n, mode, temperature, workspace, loss, stream);
  return rc;
}

int mec_grad_blocking(int64_t n, int64_t d, int dtype, int64_t* block_rows, int64_t* num_blocks) {
  g_err.clear();
  if (n < 1 || d < 1 || d > kMaxD) return fail(MEC_ERR_INVALID, "n or d out of range");
  if (n > kMaxN) return fail(MEC_ERR_UNSUPPORTED, "n=%lld exceeds the supported maximum 2^22", (long long)n);
  if (!known_dtype(dtype)) return fail(MEC_ERR_INVALID, "unknown dtype %d", dtype);
  if (!block_rows || !num_blocks) return fail(MEC_ERR_INVALID, "block_rows and num_blocks must be non-null");
  int bs, nb;
  grad_blocks(n, d, dtype, &bs, &nb);
  *block_rows = bs;
  *num_blocks = nb;
  return MEC_OK;
}

// Arguments of one backward pipeline step, checked by the entry points.
struct StepArgs {
  const void* x;
  int64_t ldx;
  const void* y;
  int64_t ldy;
  int64_t n, d;
  int dtype, mode, normalize;
  float temperature;
  const float* workspace;
  float* acc_x;  // null: side skipped (LiT: acc_y always null)
  float* acc_y;
  int sides() const { return (acc_x ? kSideX : 0) | (acc_y ? kSideY : 0); }
};

// fp32 reads its raw input rows as the contractions' feature operand, with
// 32-bit offsets within a 32-row chunk: row strides up to 2^24 elements
constexpr int64_t kMaxLdF32 = int64_t(1) << 24;

// Validation shared by mec_grad_step, mec_grad and mec_backward_noalloc:
// problem, mode, temperature, workspace and at least one accumulator (LiT
// drops acc_y).
static int check_step_args(StepArgs& a) {
  int rc = check_common(a.x, a.ldx, a.y, a.ldy, a.n, a.d, a.dtype);
  if (!rc) rc = check_mode(a.mode);
  if (!rc) rc = check_temperature(a.temperature);
  if (rc) return rc;
  const bool lit = is_lit(a.mode);
  if (lit) a.acc_y = nullptr;
  if (!a.workspace) return fail(MEC_ERR_INVALID, "workspace must be non-null");
  if (!a.acc_x && !a.acc_y)
    return fail(MEC_ERR_INVALID, "no gradient requested (acc_x%s null)", lit ? "" : " and acc_y");
  if (is_split(a.dtype) && !aligned16(a.workspace))
    return fail(MEC_ERR_INVALID, "workspace must be 16-byte aligned for the bf16-product modes");
  if (a.dtype == MEC_DTYPE_F32 && (a.ldx > kMaxLdF32 || a.ldy > kMaxLdF32))
    return fail(MEC_ERR_UNSUPPORTED, "row strides ldx=%lld ldy=%lld: the fp32 backward supports up to 2^24",
                (long long)a.ldx, (long long)a.ldy);
  return MEC_OK;
}

// Pipeline step `step` of a checked problem on the scratch at `scratch`
// (16-byte aligned, laid out as L for the problem's sides: L.total bytes).
static int grad_step_run(const StepArgs& a, int64_t step, const ScratchLayout& L, void* scratch, void* stream) {
  const void *x = a.x, *y = a.y;
  const int64_t ldx = a.ldx, ldy = a.ldy, n = a.n, d = a.d;
  const int dtype = a.dtype, mode = a.mode, normalize = a.normalize;
  const float temperature = a.temperature;
  const float* workspace = a.workspace;
  float *acc_x = a.acc_x, *acc_y = a.acc_y;
  const bool lit = is_lit(mode);
  const int bs = L.bs, nb = L.nb;
  if (step < 0 || step > nb)
    return fail(MEC_ERR_INVALID, "step %lld out of range [0, %d]", (long long)step, nb);
  int cus = 0;  // compute units: the persistent gradient-matrix launch, the contraction tile choice
  int rc = compute_units(&cus);
  if (rc) return rc;
  const int N = (int)n, D = (int)d;
  const float c = (float)(1.4426950408889634 / (double)temperature);
  const bool x3 = is_x3(dtype), split = is_split(dtype);
  // operands of the gradient-matrix tiles (split modes: the copies, K = terms * dp)
  const GemmOperands go = split ? split_operands(workspace, n, d, dtype) : GemmOperands{x, ldx, y, ldy, d, dtype};
  const bool vec = vec_ok(go.x, go.ldx, go.y, go.ldy, go.d, go.dtype);
  if (split && !vec) return fail(MEC_ERR_UNSUPPORTED, "split operands beyond the direct-load range");
  const bool small = dtype == MEC_DTYPE_F32 && vec && f32_small_bwd_tiles(n, d, bs, cus);
  bool w384 = false;  // 16-bit contractions in 256 x 384 tiles
  const BlockGrid bg = block_grid(d, dtype, a.sides(), bs, nb, L.ldt, cus, fwd_tile_dims(dtype, vec, small),
                                  con_tile_dims(dtype, small), &w384);
  const bool sep = separate_contractions(dtype);
  // contraction tiles per block and side
  const int ct_blk = bg.cnw ? (bg.ctm / 2) * (2 * bg.ctd + 1) : bg.ctm * bg.ctd;
  StepPlan sp{};
  sp.diag_g = step < nb ? (int)step : -1;
  sp.diag_c = step > 0 ? (int)step - 1 : -1;
  sp.accumulate = step > 1;
  sp.g_n = sp.diag_g >= 0 ? nb * bg.gtm * bg.gtn : 0;
  sp.cx_n = (sp.diag_c >= 0 && acc_x) ? nb * ct_blk : 0;
  sp.cy_n = (sp.diag_c >= 0 && acc_y) ? nb * ct_blk : 0;
  sp.g_pad = round8(sp.g_n);
  sp.cx_pad = round8(sp.cx_n);
  sp.cy_pad = round8(sp.cy_n);
  // bf16: the contractions of diagonal t-1 run in k_grad_contract, before the
  // G' tiles of diagonal t (different scratch buffers, so either order works)
  StepPlan sp_g = sp, sp_c = sp;
  if (sep) {
    sp_g.cx_n = sp_g.cy_n = sp_g.cx_pad = sp_g.cy_pad = 0;
    sp_c.g_n = sp_c.g_pad = 0;
  }
  const int64_t grid = sep ? (int64_t)sp.g_pad : (int64_t)sp.g_pad + sp.cx_pad + sp.cy_pad;
  const int64_t grid_c = sep ? (int64_t)sp.cx_pad + sp.cy_pad : 0;
  if (grid > 0x7fffffff || grid_c > 0x7fffffff) return fail(MEC_ERR_UNSUPPORTED, "backward grid too large");
  // the layout's buffers: plane p of diagonal buffer s at (p nbuf + s) gbuf
  char* base = (char*)scratch;
  GradBufs gb{};
  for (int sb = 0; sb < 2; ++sb) {
    char* g0 = base + (int64_t)(sb < L.nbuf ? sb : 0) * L.gbuf;
    if (dtype == MEC_DTYPE_F32) {
      gb.g[sb] = g0;
    } else {
      gb.gt[sb] = g0;
      if (x3) gb.gt_lo[sb] = g0 + (int64_t)L.nbuf * L.gbuf;
    }
  }
  if (L.xt >= 0) {
    gb.xt = base + L.xt;
    if (x3) gb.xt_lo = base + L.xt + L.tbuf;
  }
  if (L.yt >= 0) {
    gb.yt = base + L.yt;
    if (x3) gb.yt_lo = base + L.yt + L.tbuf;
  }
  gb.ldt = L.ldt;
  hipStream_t s = (hipStream_t)stream;
  if (step == 0 && dtype != MEC_DTYPE_F32) {
    // transposed normalised operands of the 16-bit contractions: YT for the
    // x side, XT for the y side (fp32 reads its raw inputs instead)
    const int64_t n64 = n;
    // one launch for both sides (blockIdx.z): YT when the x side is wanted,
    // XT when the y side is
    const unsigned nsides = (acc_x ? 1u : 0u) + (acc_y ? 1u : 0u);
    dim3 tgrid((unsigned)(L.ldt / 64), (unsigned)((d + 63) / 64), nsides);
    if (split) {
      using TS = TransSide<float, uint16_t>;
      const TS ty{(const float*)y, ldy, workspace + WS_RY * n64, (uint16_t*)gb.yt, (uint16_t*)gb.yt_lo};
      const TS tx{(const float*)x, ldx, workspace + WS_RX * n64, (uint16_t*)gb.xt, (uint16_t*)gb.xt_lo};
      DISPATCH_BOOL(normalize, NORM, DISPATCH_BOOL(x3, LO,
          k_transpose_split<NORM, LO><<<tgrid, 256, 0, s>>>(acc_x ? ty : tx, tx, N, D, L.ldt)));
    } else {
      DISPATCH_DTYPE(dtype, T, DISPATCH_BOOL(normalize, NORM, {
        if constexpr (Is16<T>::value) {
          using TS = TransSide<T>;
          const TS ty{(const T*)y, ldy, workspace + WS_RY * n64, (T*)gb.yt, nullptr};
          const TS tx{(const T*)x, ldx, workspace + WS_RX * n64, (T*)gb.xt, nullptr};
          k_transpose<T, NORM><<<tgrid, 256, 0, s>>>(acc_x ? ty : tx, tx, N, D, L.ldt);
        }
      }));
    }
    rc = check_launch("transpose");
    if (rc) return rc;
  }
  if (split) {
    // the bf16 kernels on the split operands (bf16x3: with hi/lo planes of
    // the gradient-matrix blocks and of the transposed inputs)
    using T = uint16_t;
    const int DK = (int)go.d;
    DISPATCH_BOOL(x3, X3, {
      if (grid_c > 0) {
        DISPATCH_BOOL(w384, W, k_grad_contract<T, X3, W><<<(unsigned)grid_c, ConTileX<T>::NT, 0, s>>>(
                                   N, D, gb, bg, sp_c, acc_x, acc_y));
        rc = check_launch("grad_contract");
      }
      if (!rc && grid > 0) {
        // (the copies are already normalized: no norm scaling in the tiles; chained tiles)
        DISPATCH_BOOL(lit, LIT,
            k_grad_g_chain<T, LIT, false, X3><<<(unsigned)(grid < cus ? grid : cus), FwdTile<T, true>::NT, 0, s>>>(
                (const T*)go.x, go.ldx, (const T*)go.y, go.ldy, N, DK, DK, c, workspace, gb, bg, sp_g));
      }
    });
    if (rc) return rc;
    return check_launch("grad_step");
  }
  DISPATCH_DTYPE(dtype, T, {
    if (grid_c > 0) {
      if constexpr (Is16<T>::value) {
        DISPATCH_BOOL(w384, W, k_grad_contract<T, false, W><<<(unsigned)grid_c, ConTileX<T>::NT, 0, s>>>(
                                   N, D, gb, bg, sp_c, acc_x, acc_y));
        rc = check_launch("grad_contract");
      }
    }
    if (!rc && grid > 0) {
      if constexpr (Is16<T>::value) {
        if (vec && !normalize) {
          // direct-to-LDS tiles: persistent workgroups, one per CU, chained tiles
          // (the normalising epilogue would spill registers in the tile loop)
          DISPATCH_BOOL(lit, LIT,
              k_grad_g_chain<T, LIT, false><<<(unsigned)(grid < cus ? grid : cus), FwdTile<T, true>::NT, 0, s>>>(
                  (const T*)x, ldx, (const T*)y, ldy, N, D, D, c, workspace, gb, bg, sp_g));
        } else {
          DISPATCH_BOOL(lit, LIT, DISPATCH_BOOL(normalize, NORM, DISPATCH_BOOL(vec, VEC,
              k_grad_step<T, LIT, NORM, VEC><<<(unsigned)grid, FwdTile<T, VEC>::NT, 0, s>>>(
                  (const T*)x, ldx, (const T*)y, ldy, N, D, D, c, workspace, gb, bg, sp_g, acc_x, acc_y))));
        }
      } else if (small) {
        DISPATCH_BOOL(lit, LIT, DISPATCH_BOOL(normalize, NORM,
            k_grad_step<T, LIT, NORM, true, false, true><<<(unsigned)grid, GemmTile<T, true, true>::NT, 0, s>>>(
                (const T*)x, ldx, (const T*)y, ldy, N, D, D, c, workspace, gb, bg, sp, acc_x, acc_y)));
      } else {
        DISPATCH_BOOL(lit, LIT, DISPATCH_BOOL(normalize, NORM, DISPATCH_BOOL(vec, VEC,
            k_grad_step<T, LIT, NORM, VEC><<<(unsigned)grid, FwdTile<T, VEC>::NT, 0, s>>>(
                (const T*)x, ldx, (const T*)y, ldy, N, D, D, c, workspace, gb, bg, sp, acc_x, acc_y))));
      }
    }
  });
  if (rc) return rc;
  return check_launch("grad_step");
}

// The backward's contractions from the kept matrix (MEC_FLAG_KEEP_EXP; a
// checked problem; H since the forward's finalize), one launch: into acc_x /
// acc_y as mec_grad leaves them (post == NULL), or with the post-pass in
// their epilogue into the outputs of *post (mec_backward,
// mec_backward_noalloc).
static int keep_grad_run(const StepArgs& a, const KeepPost* post, void* stream) {
  const KeepLayout L = keep_layout(a.n, a.d, a.dtype);
  const KeepBufs kb = keep_bufs(a.workspace, L);
  const int ctd = (int)((a.d + KEEP_T - 1) / KEEP_T);
  const bool sx = post ? post->dx != nullptr : a.acc_x != nullptr;
  const bool sy = post ? post->dy != nullptr : a.acc_y != nullptr;
  const int nx_pad = sx ? round8(kb.kt * ctd) : 0, ny_pad = sy ? round8(kb.kt * ctd) : 0;
  const unsigned grid = (unsigned)(nx_pad + ny_pad);
  hipStream_t s = (hipStream_t)stream;
  const float* x = (const float*)a.x;
  const float* y = (const float*)a.y;
  if (!post) {
    k_keep_contract<false, false><<<grid, KEEP_NT, 0, s>>>(x, a.ldx, y, a.ldy, (int)a.n, (int)a.d, kb, a.acc_x,
                                                          a.acc_y, KeepPost{}, ctd, nx_pad, ny_pad);
    return check_launch("grad (kept exponentials)");
  }
  DISPATCH_BOOL(a.normalize, NORM, DISPATCH_BOOL(kb.kt <= 16, SMALLT, {
    k_keep_contract<true, NORM, SMALLT ? 16 : KEEP_MAX_KT><<<grid, KEEP_NT, 0, s>>>(
        x, a.ldx, y, a.ldy, (int)a.n, (int)a.d, kb, nullptr, nullptr, *post, ctd, nx_pad, ny_pad);
  }));
  return check_launch("backward (kept exponentials)");
}
// mec_backward and mec_backward_noalloc on the kept matrix (after
// check_step_args): mec_postpass's checks, then the one fused launch (no
// scratch, so the no-allocation array is not touched either)
static int keep_backward(const StepArgs& a, float grad_scale, const float* grad_output, void* dx, void* dy,
                         void* stream) {
  if (!std::isfinite(grad_scale)) return fail(MEC_ERR_INVALID, "grad_scale must be finite");
  if (is_lit(a.mode)) dy = nullptr;
  if ((a.acc_x == nullptr) != (dx == nullptr) || (a.acc_y == nullptr) != (dy == nullptr))
    return fail(MEC_ERR_INVALID, "each side needs both its accumulator and its output (or neither)");
  int rc = check_keep(a.x, a.ldx, a.y, a.ldy, a.n, a.d, a.dtype, a.workspace);
  if (!rc) rc = check_not_capturing(stream);
  if (rc) return rc;
  const float scale = (float)((double)grad_scale / (is_lit(a.mode) ? (double)a.n : 2.0 * (double)a.n));
  const KeepPost post{a.workspace, grad_output, (float*)dx, (float*)dy, scale};
  return keep_grad_run(a, &post, stream);
}

// the caller's scratch against the default layout for the problem's sides
static int check_scratch(const StepArgs& a, void* scratch, int64_t scratch_bytes, ScratchLayout* L) {
  if (!scratch) return fail(MEC_ERR_INVALID, "scratch must be non-null");
  if (!aligned16(scratch)) return fail(MEC_ERR_INVALID, "scratch must be 16-byte aligned");
  *L = scratch_layout(a.n, a.d, a.dtype, a.sides());
  if (scratch_bytes < L->total)
    return fail(MEC_ERR_INVALID, "scratch holds %lld bytes, %lld needed", (long long)scratch_bytes,
                (long long)L->total);
  return MEC_OK;
}

int mec_grad_step(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
                  int mode, int normalize, float temperature, const float* workspace, int64_t step, void* scratch,
                  int64_t scratch_bytes, float* acc_x, float* acc_y, void* stream) {
  g_err.clear();
  StepArgs a{x, ldx, y, ldy, n, d, dtype, mode, normalize, temperature, workspace, acc_x, acc_y};
  int rc = check_step_args(a);
  if (!rc) rc = check_no_keep(mode, "mec_grad_step");
  ScratchLayout L;
  if (!rc) rc = check_scratch(a, scratch, scratch_bytes, &L);
  if (!rc && (step < 0 || step > L.nb))
    rc = fail(MEC_ERR_INVALID, "step %lld out of range [0, %d]", (long long)step, L.nb);
  if (!rc) rc = check_not_capturing(stream);
  if (rc) return rc;
  return grad_step_run(a, step, L, scratch, stream);
}

int mec_grad(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
             int mode, int normalize, float temperature, const float* workspace, void* scratch,
             int64_t scratch_bytes, float* acc_x, float* acc_y, void* stream) {
  g_err.clear();
  StepArgs a{x, ldx, y, ldy, n, d, dtype, mode, normalize, temperature, workspace, acc_x, acc_y};
  int rc = check_step_args(a);
  if (!rc && keep_flag(mode)) {
    // (no scratch: it may be NULL)
    rc = check_keep(x, ldx, y, ldy, n, d, dtype, workspace);
    if (!rc) rc = check_not_capturing(stream);
    if (rc) return rc;
    return keep_grad_run(a, nullptr, stream);
  }
  ScratchLayout L;
  if (!rc) rc = check_scratch(a, scratch, scratch_bytes, &L);
  if (!rc) rc = check_not_capturing(stream);
  if (rc) return rc;
  for (int t = 0; t <= L.nb; ++t) {
    rc = grad_step_run(a, t, L, scratch, stream);
    if (rc) return rc;
  }
  return MEC_OK;
}

int mec_backward_noalloc(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
                         int mode, int normalize, float temperature, float grad_scale, const float* workspace,
                         const float* grad_output, float* acc_x, float* acc_y, void* dx, void* dy, void* stream) {
  g_err.clear();
  StepArgs a{x, ldx, y, ldy, n, d, dtype, mode, normalize, temperature, workspace, acc_x, acc_y};
  int rc = check_step_args(a);
  if (rc) return rc;
  if (keep_flag(mode)) return keep_backward(a, grad_scale, grad_output, dx, dy, stream);
  if (!std::isfinite(grad_scale)) return fail(MEC_ERR_INVALID, "grad_scale must be finite");
  if (is_lit(mode)) dy = nullptr;
  if ((a.acc_x == nullptr) != (dx == nullptr) || (a.acc_y == nullptr) != (dy == nullptr))
    return fail(MEC_ERR_INVALID, "each side needs both its accumulator and its output (or neither)");
  bool ok = false;
  const ScratchLayout L = noalloc_layout(n, d, dtype, a.sides(), &ok);
  if (!ok)
    return fail(MEC_ERR_UNSUPPORTED,
                "the backward of n=%lld d=%lld needs more than the %lld bytes mec_backward_noalloc holds "
                "(use mec_backward with caller scratch)",
                (long long)n, (long long)d, (long long)kNoAllocScratch);
  rc = check_not_capturing(stream);
  if (rc) return rc;
  void* buf = nullptr;
  rc = noalloc_scratch(&buf);
  if (rc) return rc;
  for (int t = 0; t <= L.nb; ++t) {
    rc = grad_step_run(a, t, L, buf, stream);
    if (rc) return rc;
  }
  return mec_postpass(x, ldx, y, ldy, n, d, dtype, mode, normalize, grad_scale, workspace, grad_output, a.acc_x,
                      a.acc_y, dx, dy, stream);
}

int mec_postpass(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
                 int mode, int normalize, float grad_scale, const float* workspace, const float* grad_output,
                 const float* acc_x, const float* acc_y, void* dx, void* dy, void* stream) {
  g_err.clear();
  int rc = check_common(x, ldx, y, ldy, n, d, dtype);
  if (!rc) rc = check_mode(mode);
  if (rc) return rc;
  if (!std::isfinite(grad_scale)) return fail(MEC_ERR_INVALID, "grad_scale must be finite");
  const bool lit = is_lit(mode);
  if (lit) acc_y = nullptr, dy = nullptr;
  if (!workspace) return fail(MEC_ERR_INVALID, "workspace must be non-null");
  if ((acc_x == nullptr) != (dx == nullptr) || (acc_y == nullptr) != (dy == nullptr))
    return fail(MEC_ERR_INVALID, "each side needs both its accumulator and its output (or neither)");
  if (!acc_x && !acc_y) return fail(MEC_ERR_INVALID, "no gradient requested");
  rc = check_not_capturing(stream);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  const int N = (int)n, D = (int)d;
  const int64_t n64 = n;
  const float* rx = workspace + WS_RX * n64;
  const float* ry = workspace + WS_RY * n64;
  const float* kap = workspace + WS_KAPPA * n64;
  const float a = (float)((double)grad_scale / (lit ? (double)n : 2.0 * (double)n));
  // one launch for both sides (blockIdx.y)
  const unsigned nsides = (acc_x ? 1u : 0u) + (acc_y ? 1u : 0u);
  dim3 grid((unsigned)((n + 3) / 4), nsides);
  // fp32 (not the split modes): the accumulators carry the row's inverse norm
  // (the contractions of H = diag(rx) G' diag(ry) with the raw inputs)
  const bool accr = dtype == MEC_DTYPE_F32;
  // fp32 data with every row 16-byte aligned: 16-byte vectors
  const bool pvec = data_dtype(dtype) == MEC_DTYPE_F32 && d % 4 == 0 && ldx % 4 == 0 && ldy % 4 == 0 &&
                    aligned16(x) && aligned16(y) && aligned16(acc_x) && aligned16(acc_y) && aligned16(dx) &&
                    aligned16(dy);
  DISPATCH_DTYPE(data_dtype(dtype), T, DISPATCH_BOOL(normalize, NORM, DISPATCH_BOOL(accr, ACCR, {
    const PostSide<T> px{(const T*)x, ldx, (const T*)y, ldy, rx, ry, acc_x, (T*)dx};
    const PostSide<T> py{(const T*)y, ldy, (const T*)x, ldx, ry, rx, acc_y, (T*)dy};
    if constexpr (std::is_same<T, float>::value) {
      DISPATCH_BOOL(pvec, VEC,
          k_postpass<T, NORM, ACCR, VEC><<<grid, 256, 0, s>>>(acc_x ? px : py, py, N, D, kap, a, grad_output));
    } else if constexpr (!ACCR) {
      k_postpass<T, NORM, ACCR><<<grid, 256, 0, s>>>(acc_x ? px : py, py, N, D, kap, a, grad_output);
    }
  })));
  return check_launch("postpass");
}

int mec_backward(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
                 int mode, int normalize, float temperature, float grad_scale, const float* workspace,
                 const float* grad_output, void* scratch, int64_t scratch_bytes, float* acc_x, float* acc_y,
                 void* dx, void* dy, void* stream) {
  g_err.clear();
  if (keep_flag(mode)) {
    // the kept matrix: one launch, the post-pass in the contractions' epilogue
    StepArgs a{x, ldx, y, ldy, n, d, dtype, mode, normalize, temperature, workspace, acc_x, acc_y};
    const int rc = check_step_args(a);
    return rc ? rc : keep_backward(a, grad_scale, grad_output, dx, dy, stream);
  }
  int rc = mec_grad(x, ldx, y, ldy, n, d, dtype, mode, normalize, temperature, workspace, scratch,
                    scratch_bytes, acc_x, acc_y, stream);
  if (rc) return rc;
  return mec_postpass(x, ldx, y, ldy, n, d, dtype, mode, normalize, grad_scale, workspace, grad_output, acc_x,
                      acc_y, dx, dy, stream);
}

}  // extern "C"
