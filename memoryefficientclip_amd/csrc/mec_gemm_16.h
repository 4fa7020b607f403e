// 16-bit (bf16 or fp16) MFMA tile core for gfx950, operands staged through
// registers: 128x128 output tile per 256-thread workgroup, 4 waves in 2x2,
// each wave a 64x64 sub-tile of 2x2 blocks of v_mfma_f32_32x32x16_{bf16,f16}
// (fp32 accumulate; F16 selects the format, the data movement is the same).
//
// Both operands are K-major in global memory (element (row, k) at
// base[row * ld + k]) and in LDS ([row][k], rows padded by 16 bytes): 16-byte
// global loads, conflict-free 16-byte LDS reads.  K is staged in chunks of BK
// (a template parameter: each kernel uses the depth measured best for it)
// with the next chunk prefetched into registers during the MFMAs (STAGES = 2:
// double-buffered LDS, one barrier per chunk; STAGES = 1: two barriers, half
// the LDS).  Within a chunk the logical k fed to MFMA step s (0..BK/16-1) by
// lane half h, element e (0..7) is h*BK/2 + s*8 + e for both operands.
#pragma once
#include "mec_common.h"

#ifndef MEC_16BIT_STAGES
#define MEC_16BIT_STAGES 1
#endif

namespace mec {
namespace g16 {

constexpr int BM = 128;
constexpr int NT = 256;
constexpr int STAGES = MEC_16BIT_STAGES;

// Geometry of a core with K chunks of BK elements.
template <int BK>
struct Cfg {
  static constexpr int LD = BK + 8;              // padded row pitch (elements)
  static constexpr int TILE = BM * LD;           // elements per operand per stage
  static constexpr int LDS_ELEMS = STAGES * 2 * TILE;
  static constexpr int KV = BK / 8;              // 16-byte vectors per row
  static constexpr int NV = BM * KV / NT;        // vectors per thread per operand per chunk
  static constexpr int NS = BK / 16;             // MFMA k-steps per chunk
  static_assert(BK % 32 == 0 && NV >= 1, "BK must be a multiple of 32");
};

struct Operand {
  const uint16_t* base;  // element (row, k) at base[row * ld + k]
  int64_t ld;
  int extent;            // valid rows
  int kmax;              // valid k range [0, kmax)
};

// Vector v of thread t: KV consecutive lanes read one row's BK*2 contiguous
// bytes (the global loads coalesce by consecutive lanes).  VEC requires
// 16-byte aligned rows and, when kmax % 8 != 0, finite padding up to the next
// multiple of 8 behind kmax.
template <int BK, bool VEC>
__device__ __forceinline__ void load_chunk(const Operand& op, int k0, i16x8 (&r)[Cfg<BK>::NV]) {
  using G = Cfg<BK>;
  const int t = threadIdx.x;
#pragma unroll
  for (int v = 0; v < G::NV; ++v) {
    const int row = t / G::KV + v * (NT / G::KV);
    const int kk = k0 + (t % G::KV) * 8;
    const uint16_t* p = op.base + (int64_t)row * op.ld + kk;
    if (VEC) {
      if (row < op.extent && kk < op.kmax) r[v] = *(const i16x8*)p;
      else r[v] = i16x8{0, 0, 0, 0, 0, 0, 0, 0};
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) r[v][e] = (row < op.extent && kk + e < op.kmax) ? (short)p[e] : (short)0;
    }
  }
}

template <int BK>
__device__ __forceinline__ void store_chunk(uint16_t* lds, const i16x8 (&r)[Cfg<BK>::NV]) {
  using G = Cfg<BK>;
  const int t = threadIdx.x;
#pragma unroll
  for (int v = 0; v < G::NV; ++v) {
    const int row = t / G::KV + v * (NT / G::KV);
    *(i16x8*)(lds + row * G::LD + (t % G::KV) * 8) = r[v];
  }
}

// MFMA steps [s0, s0 + 2) of the chunk: this lane's 16 k-values of its two A
// rows and two B rows, then 8 MFMAs.
template <int BK, bool F16>
__device__ __forceinline__ void compute_part(const uint16_t* la, const uint16_t* lb, int wm, int wn, int lane,
                                             int s0, f32x16 (&acc)[2][2]) {
  using G = Cfg<BK>;
  const int q = lane & 31, h = lane >> 5;
  i16x8 a[2][2], b[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint16_t* p = la + (wm * 64 + i * 32 + q) * G::LD + h * (BK / 2) + s0 * 8;
    a[i][0] = *(const i16x8*)p;
    a[i][1] = *(const i16x8*)(p + 8);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint16_t* p = lb + (wn * 64 + j * 32 + q) * G::LD + h * (BK / 2) + s0 * 8;
    b[j][0] = *(const i16x8*)p;
    b[j][1] = *(const i16x8*)(p + 8);
  }
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma16_32x32x16<F16>(a[i][s], b[j][s], acc[i][j]);
}

// acc[i][j] (this wave's 64x64 sub-tile) = sum_k A(m, k) * B(n, k) over k in [0, K).
template <int BK, bool VECA, bool VECB, bool F16>
__device__ __forceinline__ void mainloop(const Operand& A, const Operand& B, int K, uint16_t* lds,
                                         f32x16 (&acc)[2][2]) {
  using G = Cfg<BK>;
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
  i16x8 ra[G::NV], rb[G::NV];
  load_chunk<BK, VECA>(A, 0, ra);
  load_chunk<BK, VECB>(B, 0, rb);
  store_chunk<BK>(lds, ra);
  store_chunk<BK>(lds + G::TILE, rb);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = STAGES == 2 ? (kt & 1) : 0;
    const bool more = kt + 1 < nk;
    if (more) {
      load_chunk<BK, VECA>(A, (kt + 1) * BK, ra);
      load_chunk<BK, VECB>(B, (kt + 1) * BK, rb);
    }
    const uint16_t* la = lds + cur * 2 * G::TILE;
#pragma unroll
    for (int s0 = 0; s0 < G::NS; s0 += 2) compute_part<BK, F16>(la, la + G::TILE, wm, wn, lane, s0, acc);
    if (STAGES == 2) {
      if (more) {
        uint16_t* ln = lds + (cur ^ 1) * 2 * G::TILE;
        store_chunk<BK>(ln, ra);
        store_chunk<BK>(ln + G::TILE, rb);
      }
      __syncthreads();
    } else {
      __syncthreads();
      if (more) {
        store_chunk<BK>(lds, ra);
        store_chunk<BK>(lds + G::TILE, rb);
        __syncthreads();
      }
    }
  }
}

}  // namespace g16
}  // namespace mec
