// fp32 MFMA tile core for gfx950: 128x128 output tile per 256-thread workgroup,
// 4 waves in a 2x2 arrangement, each wave owning a 64x64 sub-tile computed as
// 2x2 blocks of v_mfma_f32_32x32x2_f32.  K is staged through LDS in chunks of
// 16 with double buffering (one barrier per chunk).
//
// Operand staging modes:
//   KMAJOR : element (row, k) at base[row * ld + k]   (k contiguous, e.g. X, Y, G)
//   MNMAJOR: element (k, col) at base[k * ld + col]   (col contiguous, e.g. Y as the
//            right operand of G.Y, or G read transposed)
//
// Within a 16-wide chunk the logical k index fed to MFMA step s (0..7) by lane
// half h = lane/32 is h*8 + s.  Both operands use the same assignment, so the
// contraction is exact; for KMAJOR tiles it makes each lane's 8 values
// contiguous (two ds_read_b128).
#pragma once
#include "mec_common.h"

namespace mec {
namespace g32 {

constexpr int BM = 128;
constexpr int BK = 16;
constexpr int NT = 256;
constexpr int KM_LD = BK + 4;           // 80-byte rows: conflict-free b128 reads
constexpr int MN_LD = BM + 4;           // 528-byte rows
constexpr int KM_TILE = BM * KM_LD;     // 2560 floats
constexpr int MN_TILE = BK * MN_LD;     // 2112 floats
constexpr int TILE = KM_TILE;           // slot size per operand per stage
constexpr int LDS_FLOATS = 2 * 2 * TILE;  // 2 stages x 2 operands = 40 KiB

enum { KMAJOR = 0, MNMAJOR = 1 };

struct Operand {
  const float* base;    // see modes above
  int64_t ld;           // row stride in elements
  int extent;           // KMAJOR: valid rows from base; MNMAJOR: valid columns from base
  int kmax;             // valid k range [0, kmax)
  const float* kscale;  // MNMAJOR: optional scale per k row (nullptr = 1)
};

// Global -> registers for one 16-deep chunk starting at k0.  Each thread moves
// two float4.  VEC requires 16-byte aligned rows and extents (k for KMAJOR,
// columns for MNMAJOR) that are multiples of 4.
template <int MODE, bool VEC>
__device__ __forceinline__ void load_chunk(const Operand& op, int k0, f32x4 (&r)[2]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    if (MODE == KMAJOR) {
      const int row = (t >> 2) + 64 * v;
      const int kk = k0 + (t & 3) * 4;
      const float* p = op.base + (int64_t)row * op.ld + kk;
      if (VEC) {
        if (row < op.extent && kk < op.kmax) r[v] = *(const f32x4*)p;
        else r[v] = f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) r[v][e] = (row < op.extent && kk + e < op.kmax) ? p[e] : 0.f;
      }
    } else {
      const int kr = (t >> 5) + 8 * v;
      const int col = (t & 31) * 4;
      const int kk = k0 + kr;
      const float* p = op.base + (int64_t)kk * op.ld + col;
      const bool krow = kk < op.kmax;
      if (VEC) {
        if (krow && col < op.extent) r[v] = *(const f32x4*)p;
        else r[v] = f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) r[v][e] = (krow && col + e < op.extent) ? p[e] : 0.f;
      }
      if (op.kscale != nullptr && krow) {
        const float sc = op.kscale[kk];
        r[v] *= sc;
      }
    }
  }
}

template <int MODE>
__device__ __forceinline__ void store_chunk(float* lds, const f32x4 (&r)[2]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    if (MODE == KMAJOR) {
      const int row = (t >> 2) + 64 * v;
      *(f32x4*)(lds + row * KM_LD + (t & 3) * 4) = r[v];
    } else {
      const int kr = (t >> 5) + 8 * v;
      *(f32x4*)(lds + kr * MN_LD + (t & 31) * 4) = r[v];
    }
  }
}

// Read this lane's 8 k-values for MFMA block `blk` (32 rows/cols starting at
// `off` within the 128-wide tile).
template <int MODE>
__device__ __forceinline__ void read_operand(const float* lds, int off, int lane, float (&o)[8]) {
  const int q = lane & 31, h = lane >> 5;
  if (MODE == KMAJOR) {
    const float* p = lds + (off + q) * KM_LD + h * 8;
    f32x4 u = *(const f32x4*)p;
    f32x4 w = *(const f32x4*)(p + 4);
    o[0] = u[0]; o[1] = u[1]; o[2] = u[2]; o[3] = u[3];
    o[4] = w[0]; o[5] = w[1]; o[6] = w[2]; o[7] = w[3];
  } else {
#pragma unroll
    for (int s = 0; s < 8; ++s) o[s] = lds[(h * 8 + s) * MN_LD + off + q];
  }
}

template <int AMODE, int BMODE>
__device__ __forceinline__ void compute_chunk(const float* la, const float* lb, int wm, int wn,
                                              int lane, f32x16 (&acc)[2][2]) {
  float a[2][8], b[2][8];
#pragma unroll
  for (int i = 0; i < 2; ++i) read_operand<AMODE>(la, wm * 64 + i * 32, lane, a[i]);
#pragma unroll
  for (int j = 0; j < 2; ++j) read_operand<BMODE>(lb, wn * 64 + j * 32, lane, b[j]);
#pragma unroll
  for (int s = 0; s < 8; ++s)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma_f32_32x32x2(a[i][s], b[j][s], acc[i][j]);
}

// acc[i][j] (this wave's 64x64 sub-tile) = sum_k A(m, k) * B(k, n) over k in [0, K).
// lds must hold LDS_FLOATS floats.  Ends with a barrier, so lds may be reused.
template <int AMODE, int BMODE, bool VEC>
__device__ __forceinline__ void mainloop(const Operand& A, const Operand& B, int K, float* lds,
                                         f32x16 (&acc)[2][2]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  const int nk = (K + BK - 1) / BK;
  if (nk <= 0) return;
  f32x4 ra[2], rb[2];
  load_chunk<AMODE, VEC>(A, 0, ra);
  load_chunk<BMODE, VEC>(B, 0, rb);
  store_chunk<AMODE>(lds, ra);
  store_chunk<BMODE>(lds + TILE, rb);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      load_chunk<AMODE, VEC>(A, (kt + 1) * BK, ra);
      load_chunk<BMODE, VEC>(B, (kt + 1) * BK, rb);
    }
    const float* la = lds + cur * 2 * TILE;
    compute_chunk<AMODE, BMODE>(la, la + TILE, wm, wn, lane, acc);
    if (more) {
      float* ln = lds + (cur ^ 1) * 2 * TILE;
      store_chunk<AMODE>(ln, ra);
      store_chunk<BMODE>(ln + TILE, rb);
    }
    __syncthreads();
  }
}

}  // namespace g32
}  // namespace mec
