// fp32 MFMA tile core for gfx950: 128x128 output tile per 256-thread workgroup,
// 4 waves in a 2x2 arrangement, each wave owning a 64x64 sub-tile computed as
// 2x2 blocks of v_mfma_f32_32x32x2_f32.
//
// Both operands are K-major in global memory: element (row, k) at
// base[row * ld + k] (X, Y, their transposes and the gradient-matrix blocks
// are all stored that way).  K is staged through LDS in chunks of BK as
// [row][k] with a padded row pitch, so every global load is a 16-byte vector
// and every MFMA operand read a conflict-free ds_read_b128.  The next chunk is
// prefetched into registers while the current one is multiplied (STAGES = 2:
// double-buffered LDS, one barrier per chunk; STAGES = 1: one LDS buffer, two
// barriers per chunk, half the LDS).
//
// Within a chunk the logical k fed to MFMA step s (0..BK/2-1) by lane half
// h = lane/32 is h*BK/2 + s for both operands, so the contraction is exact and
// each lane's k-values are contiguous in LDS.
#pragma once
#include "mec_common.h"

#ifndef MEC_F32_BK
#define MEC_F32_BK 16
#endif
#ifndef MEC_F32_STAGES
#define MEC_F32_STAGES 1
#endif

namespace mec {
namespace g32 {

constexpr int BM = 128;
constexpr int BK = MEC_F32_BK;          // k depth of one LDS chunk
constexpr int STAGES = MEC_F32_STAGES;  // LDS buffers
constexpr int NT = 256;
constexpr int LD = BK + 4;              // padded LDS row pitch (floats)
constexpr int TILE = BM * LD;           // floats per operand per stage
constexpr int LDS_FLOATS = STAGES * 2 * TILE;
constexpr int KQ = BK / 4;              // 16-byte k quads per row
constexpr int NV = BM * KQ / NT;        // vectors per thread per operand per chunk
static_assert(BK % 16 == 0 && NV >= 1, "BK must be a multiple of 16");

struct Operand {
  const float* base;  // element (row, k) at base[row * ld + k]
  int64_t ld;         // row stride in elements
  int extent;         // valid rows from base
  int kmax;           // valid k range [0, kmax)
};

// Global -> registers for the chunk starting at k0: KQ consecutive threads
// cover one row.  VEC requires 16-byte aligned rows and, when kmax % 4 != 0,
// finite padding up to the next multiple of 4 behind kmax (it is multiplied
// by zeros of the other operand).
template <bool VEC>
__device__ __forceinline__ void load_chunk(const Operand& op, int k0, f32x4 (&r)[NV]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int row = t / KQ + v * (NT / KQ);
    const int kk = k0 + (t % KQ) * 4;
    const float* p = op.base + (int64_t)row * op.ld + kk;
    if (VEC) {
      if (row < op.extent && kk < op.kmax) r[v] = *(const f32x4*)p;
      else r[v] = f32x4{0.f, 0.f, 0.f, 0.f};
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) r[v][e] = (row < op.extent && kk + e < op.kmax) ? p[e] : 0.f;
    }
  }
}

__device__ __forceinline__ void store_chunk(float* lds, const f32x4 (&r)[NV]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int row = t / KQ + v * (NT / KQ);
    *(f32x4*)(lds + row * LD + (t % KQ) * 4) = r[v];
  }
}

// MFMA steps [s0, s0 + 8) of the chunk in LDS: this lane's k-values of its
// two A rows and two B rows (8 each), then 32 MFMAs.
__device__ __forceinline__ void compute_part(const float* la, const float* lb, int wm, int wn, int lane, int s0,
                                             f32x16 (&acc)[2][2]) {
  const int q = lane & 31, h = lane >> 5;
  f32x4 a[2][2], b[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float* p = la + (wm * 64 + i * 32 + q) * LD + h * (BK / 2) + s0;
    a[i][0] = *(const f32x4*)p;
    a[i][1] = *(const f32x4*)(p + 4);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float* p = lb + (wn * 64 + j * 32 + q) * LD + h * (BK / 2) + s0;
    b[j][0] = *(const f32x4*)p;
    b[j][1] = *(const f32x4*)(p + 4);
  }
#pragma unroll
  for (int s = 0; s < 8; ++s)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = mfma_f32_32x32x2(a[i][s >> 2][s & 3], b[j][s >> 2][s & 3], acc[i][j]);
}

// acc[i][j] (this wave's 64x64 sub-tile) = sum_k A(m, k) * B(n, k) over k in [0, K).
// lds must hold LDS_FLOATS floats.  Ends with a barrier, so lds may be reused.
template <bool VECA, bool VECB>
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
  f32x4 ra[NV], rb[NV];
  load_chunk<VECA>(A, 0, ra);
  load_chunk<VECB>(B, 0, rb);
  store_chunk(lds, ra);
  store_chunk(lds + TILE, rb);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = STAGES == 2 ? (kt & 1) : 0;
    const bool more = kt + 1 < nk;
    if (more) {
      load_chunk<VECA>(A, (kt + 1) * BK, ra);
      load_chunk<VECB>(B, (kt + 1) * BK, rb);
    }
    const float* la = lds + cur * 2 * TILE;
#pragma unroll
    for (int s0 = 0; s0 < BK / 2; s0 += 8) compute_part(la, la + TILE, wm, wn, lane, s0, acc);
    if (STAGES == 2) {
      if (more) {
        float* ln = lds + (cur ^ 1) * 2 * TILE;
        store_chunk(ln, ra);
        store_chunk(ln + TILE, rb);
      }
      __syncthreads();
    } else {
      __syncthreads();
      if (more) {
        store_chunk(lds, ra);
        store_chunk(lds + TILE, rb);
        __syncthreads();
      }
    }
  }
}

}  // namespace g32
}  // namespace mec
