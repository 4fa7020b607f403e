// bf16 MFMA tile core for gfx950: 128x128 output tile per 256-thread
// workgroup, 4 waves in 2x2, each wave a 64x64 sub-tile of 2x2 blocks of
// v_mfma_f32_32x32x16_bf16 (fp32 accumulate).  K is staged through LDS in
// chunks of 32 with double buffering.
//
// Both operands are K-major in global memory (element (row, k) at
// base[row * ld + k]) and in LDS ([row][k], 80-byte padded rows): 16-byte
// global loads, conflict-free 16-byte LDS reads.  Within a chunk the logical k
// fed to MFMA step s (0..1) by lane half h, element e (0..7) is h*16 + s*8 + e
// for both operands.
#pragma once
#include "mec_common.h"

namespace mec {
namespace g16 {

constexpr int BM = 128;
constexpr int BK = 32;
constexpr int NT = 256;
constexpr int LD = BK + 8;               // 40 bf16 = 80-byte rows
constexpr int TILE = BM * LD;            // 5120 bf16 = 10 KiB per operand per stage
constexpr int LDS_ELEMS = 2 * 2 * TILE;  // 40 KiB

struct Operand {
  const uint16_t* base;  // element (row, k) at base[row * ld + k]
  int64_t ld;
  int extent;            // valid rows
  int kmax;              // valid k range [0, kmax)
};

struct Regs {
  i16x8 v[2];
};

// VEC requires 16-byte aligned rows and, when kmax % 8 != 0, finite padding up
// to the next multiple of 8 behind kmax.
template <bool VEC>
__device__ __forceinline__ void load_chunk(const Operand& op, int k0, Regs& r) {
  const int t = threadIdx.x;
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    const int row = (t >> 2) + 64 * v;
    const int kk = k0 + (t & 3) * 8;
    const uint16_t* p = op.base + (int64_t)row * op.ld + kk;
    if (VEC) {
      if (row < op.extent && kk < op.kmax) r.v[v] = *(const i16x8*)p;
      else r.v[v] = i16x8{0, 0, 0, 0, 0, 0, 0, 0};
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) r.v[v][e] = (row < op.extent && kk + e < op.kmax) ? (short)p[e] : (short)0;
    }
  }
}

__device__ __forceinline__ void store_chunk(uint16_t* lds, const Regs& r) {
  const int t = threadIdx.x;
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    const int row = (t >> 2) + 64 * v;
    *(i16x8*)(lds + row * LD + (t & 3) * 8) = r.v[v];
  }
}

__device__ __forceinline__ void read_operand(const uint16_t* lds, int off, int lane, i16x8 (&o)[2]) {
  const int q = lane & 31, h = lane >> 5;
  const uint16_t* p = lds + (off + q) * LD + h * 16;
  o[0] = *(const i16x8*)p;
  o[1] = *(const i16x8*)(p + 8);
}

__device__ __forceinline__ void compute_chunk(const uint16_t* la, const uint16_t* lb, int wm, int wn, int lane,
                                              f32x16 (&acc)[2][2]) {
  i16x8 a[2][2], b[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i) read_operand(la, wm * 64 + i * 32, lane, a[i]);
#pragma unroll
  for (int j = 0; j < 2; ++j) read_operand(lb, wn * 64 + j * 32, lane, b[j]);
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma_bf16_32x32x16(a[i][s], b[j][s], acc[i][j]);
}

// acc[i][j] (this wave's 64x64 sub-tile) = sum_k A(m, k) * B(n, k) over k in [0, K).
template <bool VECA, bool VECB>
__device__ __forceinline__ void mainloop(const Operand& A, const Operand& B, int K, uint16_t* lds,
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
  Regs ra, rb;
  load_chunk<VECA>(A, 0, ra);
  load_chunk<VECB>(B, 0, rb);
  store_chunk(lds, ra);
  store_chunk(lds + TILE, rb);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      load_chunk<VECA>(A, (kt + 1) * BK, ra);
      load_chunk<VECB>(B, (kt + 1) * BK, rb);
    }
    const uint16_t* la = lds + cur * 2 * TILE;
    compute_chunk(la, la + TILE, wm, wn, lane, acc);
    if (more) {
      uint16_t* ln = lds + (cur ^ 1) * 2 * TILE;
      store_chunk(ln, ra);
      store_chunk(ln + TILE, rb);
    }
    __syncthreads();
  }
}

}  // namespace g16
}  // namespace mec
