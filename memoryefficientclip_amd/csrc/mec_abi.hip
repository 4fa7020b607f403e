// C-ABI entry points (include/mec.h): argument validation in plain host code,
// then stream-ordered kernel launches.  Nothing here allocates device memory
// or synchronises the host.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "../../include/mec.h"
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

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MEC_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return MEC_OK;
}

constexpr int64_t kMaxN = int64_t(1) << 30;
constexpr int64_t kMaxD = int64_t(1) << 20;

int check_common(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d,
                 int dtype) {
  if (n < 1 || n > kMaxN) return fail(MEC_ERR_INVALID, "n=%lld out of range [1, 2^30]", (long long)n);
  if (d < 1 || d > kMaxD) return fail(MEC_ERR_INVALID, "d=%lld out of range [1, 2^20]", (long long)d);
  if (ldx < d || ldy < d)
    return fail(MEC_ERR_INVALID, "row strides ldx=%lld ldy=%lld must be >= d=%lld", (long long)ldx,
                (long long)ldy, (long long)d);
  if (dtype != MEC_DTYPE_F32 && dtype != MEC_DTYPE_BF16)
    return fail(MEC_ERR_INVALID, "unknown dtype %d", dtype);
  if (x == nullptr || y == nullptr) return fail(MEC_ERR_INVALID, "x and y must be non-null");
  return MEC_OK;
}

int check_mode(int mode) {
  if (mode != MEC_MODE_CLIP && mode != MEC_MODE_LIT) return fail(MEC_ERR_INVALID, "unknown mode %d", mode);
  return MEC_OK;
}

int check_temperature(float t) {
  if (!(t > 0.f) || !std::isfinite(t)) return fail(MEC_ERR_INVALID, "temperature must be finite and > 0");
  return MEC_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// 16-byte vector loads are legal when every row start is 16-byte aligned and
// rows hold a whole number of vectors.
bool vec_ok(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t d, int dtype) {
  const int64_t per = dtype == MEC_DTYPE_F32 ? 4 : 8;
  return aligned16(x) && aligned16(y) && d % per == 0 && ldx % per == 0 && ldy % per == 0;
}

// Block decomposition of the N x N gradient matrix for the backward: blocks
// of tb 128-row tiles with tb ~ 2d/128 (>= 8), balanced over nb blocks.
void grad_blocks(int64_t n, int64_t d, int* bs, int* nb) {
  const int64_t tiles = (n + 127) / 128;
  int64_t target = (2 * d + 127) / 128;
  if (target < 8) target = 8;
  if (const char* env = std::getenv("MEC_GRAD_BLOCK_TILES")) {
    long v = std::strtol(env, nullptr, 10);
    if (v >= 1 && v <= 4096) target = v;
  }
  if (target > tiles) target = tiles;
  const int64_t nbv = (tiles + target - 1) / target;
  const int64_t tb = (tiles + nbv - 1) / nbv;
  *bs = (int)(tb * 128);
  *nb = (int)nbv;
}

int64_t scratch_bytes_for(int64_t n, int64_t d, int dtype) {
  int bs, nb;
  grad_blocks(n, d, &bs, &nb);
  const int64_t elem = dtype == MEC_DTYPE_F32 ? 4 : 2;
  return (int64_t)nb * bs * bs * elem;
}

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
  return (int64_t)WS_NSLOTS * n;
}

int64_t mec_grad_scratch_bytes(int64_t n, int64_t d, int dtype) {
  if (n < 1 || n > kMaxN || d < 1 || d > kMaxD) return -1;
  if (dtype != MEC_DTYPE_F32 && dtype != MEC_DTYPE_BF16) return -1;
  return scratch_bytes_for(n, d, dtype);
}

int mec_prepass(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
                int normalize, float* workspace, void* stream) {
  g_err.clear();
  int rc = check_common(x, ldx, y, ldy, n, d, dtype);
  if (rc) return rc;
  if (!workspace) return fail(MEC_ERR_INVALID, "workspace must be non-null");
  hipStream_t s = (hipStream_t)stream;
  const int N = (int)n, D = (int)d;
  dim3 grid((unsigned)((n + 3) / 4));
  if (dtype == MEC_DTYPE_F32) {
    DISPATCH_BOOL(normalize, NORM,
                  k_prepass<float, NORM><<<grid, 256, 0, s>>>((const float*)x, ldx, (const float*)y, ldy, N, D,
                                                              workspace));
  } else {
    DISPATCH_BOOL(normalize, NORM,
                  k_prepass<uint16_t, NORM><<<grid, 256, 0, s>>>((const uint16_t*)x, ldx, (const uint16_t*)y,
                                                                 ldy, N, D, workspace));
  }
  return check_launch("prepass");
}

int mec_sumexp(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
               int mode, int normalize, float temperature, float* workspace, void* stream) {
  g_err.clear();
  int rc = check_common(x, ldx, y, ldy, n, d, dtype);
  if (!rc) rc = check_mode(mode);
  if (!rc) rc = check_temperature(temperature);
  if (rc) return rc;
  if (!workspace) return fail(MEC_ERR_INVALID, "workspace must be non-null");
  hipStream_t s = (hipStream_t)stream;
  const int N = (int)n, D = (int)d;
  const float c = (float)(1.4426950408889634 / (double)temperature);
  const int tiles = (int)((n + 127) / 128);
  dim3 grid((unsigned)((int64_t)tiles * tiles));
  const bool vec = vec_ok(x, ldx, y, ldy, d, dtype);
  const bool lit = mode == MEC_MODE_LIT;
  if (dtype == MEC_DTYPE_F32) {
    DISPATCH_BOOL(lit, LIT, DISPATCH_BOOL(normalize, NORM, DISPATCH_BOOL(vec, VEC,
        k_sumexp<float, LIT, NORM, VEC><<<grid, 256, 0, s>>>((const float*)x, ldx, (const float*)y, ldy, N, D,
                                                          c, workspace, tiles))));
  } else {
    DISPATCH_BOOL(lit, LIT, DISPATCH_BOOL(normalize, NORM, DISPATCH_BOOL(vec, VEC,
        k_sumexp<uint16_t, LIT, NORM, VEC><<<grid, 256, 0, s>>>((const uint16_t*)x, ldx, (const uint16_t*)y, ldy,
                                                           N, D, c, workspace, tiles))));
  }
  return check_launch("sumexp");
}

int mec_finalize(int64_t n, int mode, float temperature, float* workspace, float* loss, void* stream) {
  g_err.clear();
  if (n < 1 || n > kMaxN) return fail(MEC_ERR_INVALID, "n=%lld out of range", (long long)n);
  int rc = check_mode(mode);
  if (!rc) rc = check_temperature(temperature);
  if (rc) return rc;
  if (!workspace || !loss) return fail(MEC_ERR_INVALID, "workspace and loss must be non-null");
  hipStream_t s = (hipStream_t)stream;
  const double inv_t = 1.0 / (double)temperature;
  if (mode == MEC_MODE_LIT)
    k_finalize<true><<<1, 1024, 0, s>>>((int)n, inv_t, workspace, loss);
  else
    k_finalize<false><<<1, 1024, 0, s>>>((int)n, inv_t, workspace, loss);
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
  rc = mec_prepass(x, ldx, y, ldy, n, d, dtype, normalize, workspace, stream);
  if (!rc) rc = mec_sumexp(x, ldx, y, ldy, n, d, dtype, mode, normalize, temperature, workspace, stream);
  if (!rc) rc = mec_finalize(n, mode, temperature, workspace, loss, stream);
  return rc;
}

int mec_grad(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
             int mode, int normalize, float temperature, const float* workspace, void* scratch,
             int64_t scratch_bytes, float* acc_x, float* acc_y, void* stream) {
  g_err.clear();
  int rc = check_common(x, ldx, y, ldy, n, d, dtype);
  if (!rc) rc = check_mode(mode);
  if (!rc) rc = check_temperature(temperature);
  if (rc) return rc;
  const bool lit = mode == MEC_MODE_LIT;
  if (lit) acc_y = nullptr;
  if (!workspace || !scratch) return fail(MEC_ERR_INVALID, "workspace and scratch must be non-null");
  if (!acc_x && !acc_y) return fail(MEC_ERR_INVALID, "no gradient requested (acc_x%s null)", lit ? "" : " and acc_y");
  const int64_t need = scratch_bytes_for(n, d, dtype);
  if (scratch_bytes < need)
    return fail(MEC_ERR_INVALID, "scratch holds %lld bytes, %lld needed", (long long)scratch_bytes,
                (long long)need);
  if (!aligned16(scratch)) return fail(MEC_ERR_INVALID, "scratch must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  const int N = (int)n, D = (int)d;
  const float c = (float)(1.4426950408889634 / (double)temperature);
  int bs, nb;
  grad_blocks(n, d, &bs, &nb);
  BlockGrid bg{bs, nb, bs / 128, 0};
  const int tdn = (D + 127) / 128;
  const int tiles_side = nb * bg.tpb * tdn;
  const int tiles_x = acc_x ? tiles_side : 0;
  const unsigned grid_g = (unsigned)(nb * bg.tpb * bg.tpb);
  const unsigned grid_c = (unsigned)(tiles_x + (acc_y ? tiles_side : 0));
  const bool vec = vec_ok(x, ldx, y, ldy, d, dtype);
  for (int shift = 0; shift < nb; ++shift) {
    bg.shift = shift;
    const bool accum = shift > 0;
    if (dtype == MEC_DTYPE_F32) {
      const float* X = (const float*)x;
      const float* Y = (const float*)y;
      float* G = (float*)scratch;
      DISPATCH_BOOL(lit, LIT, DISPATCH_BOOL(normalize, NORM, DISPATCH_BOOL(vec, VEC,
          k_grad_g<float, LIT, NORM, VEC><<<grid_g, 256, 0, s>>>(X, ldx, Y, ldy, N, D, c, workspace, G, bg))));
      rc = check_launch("grad_g");
      if (rc) return rc;
      DISPATCH_BOOL(normalize, NORM, DISPATCH_BOOL(vec, VEC, DISPATCH_BOOL(accum, ACC,
          k_grad_contract<float, NORM, VEC, ACC><<<grid_c, 256, 0, s>>>(X, ldx, Y, ldy, N, D, workspace, G, bg,
                                                                     tiles_x, acc_x, acc_y))));
    } else {
      const uint16_t* X = (const uint16_t*)x;
      const uint16_t* Y = (const uint16_t*)y;
      uint16_t* G = (uint16_t*)scratch;
      DISPATCH_BOOL(lit, LIT, DISPATCH_BOOL(normalize, NORM, DISPATCH_BOOL(vec, VEC,
          k_grad_g<uint16_t, LIT, NORM, VEC><<<grid_g, 256, 0, s>>>(X, ldx, Y, ldy, N, D, c, workspace, G, bg))));
      rc = check_launch("grad_g");
      if (rc) return rc;
      DISPATCH_BOOL(normalize, NORM, DISPATCH_BOOL(vec, VEC, DISPATCH_BOOL(accum, ACC,
          k_grad_contract<uint16_t, NORM, VEC, ACC><<<grid_c, 256, 0, s>>>(X, ldx, Y, ldy, N, D, workspace, G, bg,
                                                                      tiles_x, acc_x, acc_y))));
    }
    rc = check_launch("grad_contract");
    if (rc) return rc;
  }
  return MEC_OK;
}

int mec_postpass(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
                 int mode, int normalize, float grad_scale, const float* workspace, const float* grad_output,
                 const float* acc_x, const float* acc_y, void* dx, void* dy, void* stream) {
  g_err.clear();
  int rc = check_common(x, ldx, y, ldy, n, d, dtype);
  if (!rc) rc = check_mode(mode);
  if (rc) return rc;
  if (!std::isfinite(grad_scale)) return fail(MEC_ERR_INVALID, "grad_scale must be finite");
  const bool lit = mode == MEC_MODE_LIT;
  if (lit) acc_y = nullptr, dy = nullptr;
  if (!workspace) return fail(MEC_ERR_INVALID, "workspace must be non-null");
  if ((acc_x == nullptr) != (dx == nullptr) || (acc_y == nullptr) != (dy == nullptr))
    return fail(MEC_ERR_INVALID, "each side needs both its accumulator and its output (or neither)");
  if (!acc_x && !acc_y) return fail(MEC_ERR_INVALID, "no gradient requested");
  hipStream_t s = (hipStream_t)stream;
  const int N = (int)n, D = (int)d;
  const int64_t n64 = n;
  const float* rx = workspace + WS_RX * n64;
  const float* ry = workspace + WS_RY * n64;
  const float* kap = workspace + WS_KAPPA * n64;
  const float a = (float)((double)grad_scale / (lit ? (double)n : 2.0 * (double)n));
  dim3 grid((unsigned)((n + 3) / 4));
  if (dtype == MEC_DTYPE_F32) {
    DISPATCH_BOOL(normalize, NORM, {
      if (acc_x)
        k_postpass<float, NORM><<<grid, 256, 0, s>>>((const float*)x, ldx, (const float*)y, ldy, N, D, rx, ry,
                                                     kap, a, grad_output, acc_x, (float*)dx);
      if (acc_y)
        k_postpass<float, NORM><<<grid, 256, 0, s>>>((const float*)y, ldy, (const float*)x, ldx, N, D, ry, rx,
                                                     kap, a, grad_output, acc_y, (float*)dy);
    });
  } else {
    DISPATCH_BOOL(normalize, NORM, {
      if (acc_x)
        k_postpass<uint16_t, NORM><<<grid, 256, 0, s>>>((const uint16_t*)x, ldx, (const uint16_t*)y, ldy, N, D,
                                                        rx, ry, kap, a, grad_output, acc_x, (uint16_t*)dx);
      if (acc_y)
        k_postpass<uint16_t, NORM><<<grid, 256, 0, s>>>((const uint16_t*)y, ldy, (const uint16_t*)x, ldx, N,
                                                        D, ry, rx, kap, a, grad_output, acc_y, (uint16_t*)dy);
    });
  }
  return check_launch("postpass");
}

int mec_backward(const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t n, int64_t d, int dtype,
                 int mode, int normalize, float temperature, float grad_scale, const float* workspace,
                 const float* grad_output, void* scratch, int64_t scratch_bytes, float* acc_x, float* acc_y,
                 void* dx, void* dy, void* stream) {
  g_err.clear();
  int rc = mec_grad(x, ldx, y, ldy, n, d, dtype, mode, normalize, temperature, workspace, scratch,
                    scratch_bytes, acc_x, acc_y, stream);
  if (rc) return rc;
  return mec_postpass(x, ldx, y, ldy, n, d, dtype, mode, normalize, grad_scale, workspace, grad_output, acc_x,
                      acc_y, dx, dy, stream);
}

}  // extern "C"
