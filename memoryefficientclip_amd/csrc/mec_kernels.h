// MFMA tile kernels of the contrastive-loss hot path (fp32 and bf16 inputs;
// the element type selects the MFMA core, the epilogues are shared):
//   k_sumexp        forward: tiled S = X Y^T, E = exp2(S c - c), off-diagonal
//                       row (and column) partial sums, one atomic per row/column
//                       per tile.  Replaces clip_sum_exp_kernel (clip_loss.py:9-64)
//                       and lit_sum_exp_kernel (lit_loss.py:9-62).
//   k_grad_g        backward step 1: recompute S for the block pairs of one
//                       block diagonal and write the gradient-matrix blocks
//                       G'_ij = E_ij (1/R_i + 1/C_j) (LiT: E_ij / R_i), i != j,
//                       to a bounded scratch (clip_loss.py:96-124, lit_loss.py:94-120).
//   k_grad_contract backward step 2: dX_I += G'_IJ Y^_J and dY_J += G'_IJ^T X^_I
//                       as plain MFMA contractions (clip_loss.py:127-156,
//                       lit_loss.py:123-148) without atomics.
#pragma once
#include "mec_gemm_f32.h"
#include "mec_gemm_bf16.h"

namespace mec {

// Element-type traits: which MFMA core runs the tile, and how G is stored.
template <typename T> struct Core;
template <> struct Core<float> {
  using Op = g32::Operand;
  static constexpr int KM = g32::KMAJOR, MN = g32::MNMAJOR;
  static constexpr int LDS_BYTES = g32::LDS_FLOATS * 4;
  template <int AM, int BM_, bool VEC>
  static __device__ __forceinline__ void run(const Op& a, const Op& b, int K, void* lds, f32x16 (&acc)[2][2]) {
    g32::mainloop<AM, BM_, VEC>(a, b, K, (float*)lds, acc);
  }
  static __device__ __forceinline__ float pack(float v) { return v; }
};
template <> struct Core<uint16_t> {
  using Op = g16::Operand;
  static constexpr int KM = g16::KMAJOR, MN = g16::MNMAJOR;
  static constexpr int LDS_BYTES = g16::LDS_ELEMS * 2;
  template <int AM, int BM_, bool VEC>
  static __device__ __forceinline__ void run(const Op& a, const Op& b, int K, void* lds, f32x16 (&acc)[2][2]) {
    g16::mainloop<AM, BM_, VEC>(a, b, K, (uint16_t*)lds, acc);
  }
  static __device__ __forceinline__ uint16_t pack(float v) { return f32_to_bf16(v); }
};

// ---------------------------------------------------------------- forward
template <typename T, bool LIT, bool NORM, bool VEC>
__global__ __launch_bounds__(256, 2) void k_sumexp(const T* __restrict__ X, int64_t ldx,
                                                   const T* __restrict__ Y, int64_t ldy, int N,
                                                   int D, float c, float* __restrict__ ws, int tiles) {
  using C = Core<T>;
  __shared__ __attribute__((aligned(16))) char lds[C::LDS_BYTES];
  __shared__ float s_rx[128], s_ry[128], s_row[128], s_col[128];
  const int64_t n64 = N;
  int tm, tn;
  tile_swizzle(blockIdx.x, gridDim.x, tiles, tiles, 8, tm, tn);
  const int m0 = tm * 128, n0 = tn * 128;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, wm = w >> 1, wn = w & 1;

  typename C::Op A{X + (int64_t)m0 * ldx, ldx, N - m0, D, nullptr};
  typename C::Op B{Y + (int64_t)n0 * ldy, ldy, N - n0, D, nullptr};
  f32x16 acc[2][2];
  C::template run<C::KM, C::KM, VEC>(A, B, D, lds, acc);

  if (t < 128) {
    s_rx[t] = (NORM && m0 + t < N) ? ws[WS_RX * n64 + m0 + t] : 1.f;
    s_row[t] = 0.f;
  } else {
    const int u = t - 128;
    s_ry[u] = (NORM && n0 + u < N) ? ws[WS_RY * n64 + n0 + u] : 1.f;
    s_col[u] = 0.f;
  }
  __syncthreads();

  float rowv[32];
  float colv[2] = {0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 32; ++k) rowv[k] = 0.f;
#pragma unroll
  for (int bm = 0; bm < 2; ++bm) {
#pragma unroll
    for (int bn = 0; bn < 2; ++bn) {
      const int nl = wn * 64 + bn * 32 + (lane & 31);
      const int j = n0 + nl;
      const float ryj = s_ry[nl];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ml = wm * 64 + bm * 32 + acc_row(r, lane);
        const int i = m0 + ml;
        float s = acc[bm][bn][r];
        if (NORM) s *= s_rx[ml] * ryj;
        float e = fast_exp2(fmaf(s, c, -c));
        e = (i < N && j < N && i != j) ? e : 0.f;
        rowv[bm * 16 + r] += e;
        colv[bn] += e;
      }
    }
  }
  const float rs = transpose_reduce32(rowv, lane);
  {
    const int q = lane & 31;
    const int ml = wm * 64 + (q >> 4) * 32 + acc_row(q & 15, lane);
    __hip_atomic_fetch_add(&s_row[ml], rs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  if (!LIT) {
#pragma unroll
    for (int bn = 0; bn < 2; ++bn) {
      colv[bn] += __shfl_xor(colv[bn], 32, 64);
      if (lane < 32)
        __hip_atomic_fetch_add(&s_col[wn * 64 + bn * 32 + lane], colv[bn], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  __syncthreads();
  if (t < 128) {
    if (m0 + t < N)
      __hip_atomic_fetch_add(&ws[WS_ROW_OFF * n64 + m0 + t], s_row[t], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  } else if (!LIT) {
    const int u = t - 128;
    if (n0 + u < N)
      __hip_atomic_fetch_add(&ws[WS_COL_OFF * n64 + n0 + u], s_col[u], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------- backward
// Block decomposition of the N x N gradient matrix: nb blocks of bs rows
// (bs a multiple of 128; the last block may be short).  Diagonal `shift`
// pairs block I with block J = (I + shift) mod nb, so one launch touches every
// block row and every block column exactly once.
struct BlockGrid {
  int bs;      // block size (rows), multiple of 128
  int nb;      // number of blocks
  int tpb;     // 128-tiles per block side = bs / 128
  int shift;   // diagonal index
};

template <typename T, bool LIT, bool NORM, bool VEC>
__global__ __launch_bounds__(256, 2) void k_grad_g(const T* __restrict__ X, int64_t ldx,
                                                   const T* __restrict__ Y, int64_t ldy, int N,
                                                   int D, float c, const float* __restrict__ ws,
                                                   T* __restrict__ G, BlockGrid bg) {
  using C = Core<T>;
  __shared__ __attribute__((aligned(16))) char lds[C::LDS_BYTES];
  __shared__ float s_rx[128], s_ry[128], s_ir[128], s_ic[128];
  const int64_t n64 = N;
  int tmg, tn;
  tile_swizzle(blockIdx.x, gridDim.x, bg.nb * bg.tpb, bg.tpb, 8, tmg, tn);
  const int I = tmg / bg.tpb, tm = tmg - I * bg.tpb;
  const int J = (I + bg.shift) % bg.nb;
  const int i0 = I * bg.bs + tm * 128, j0 = J * bg.bs + tn * 128;
  if (i0 >= N || j0 >= N) return;  // never read by the contraction kernel
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, wm = w >> 1, wn = w & 1;

  typename C::Op A{X + (int64_t)i0 * ldx, ldx, N - i0, D, nullptr};
  typename C::Op B{Y + (int64_t)j0 * ldy, ldy, N - j0, D, nullptr};
  f32x16 acc[2][2];
  C::template run<C::KM, C::KM, VEC>(A, B, D, lds, acc);

  if (t < 128) {
    const bool ok = i0 + t < N;
    s_rx[t] = (NORM && ok) ? ws[WS_RX * n64 + i0 + t] : 1.f;
    s_ir[t] = ok ? ws[WS_INV_ROW * n64 + i0 + t] : 0.f;
  } else {
    const int u = t - 128;
    const bool ok = j0 + u < N;
    s_ry[u] = (NORM && ok) ? ws[WS_RY * n64 + j0 + u] : 1.f;
    s_ic[u] = (!LIT && ok) ? ws[WS_INV_COL * n64 + j0 + u] : 0.f;
  }
  __syncthreads();

  T* Gb = G + (int64_t)I * bg.bs * bg.bs + (int64_t)(tm * 128) * bg.bs + tn * 128;
#pragma unroll
  for (int bm = 0; bm < 2; ++bm) {
#pragma unroll
    for (int bn = 0; bn < 2; ++bn) {
      const int nl = wn * 64 + bn * 32 + (lane & 31);
      const int j = j0 + nl;
      const float ryj = s_ry[nl], icj = s_ic[nl];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ml = wm * 64 + bm * 32 + acc_row(r, lane);
        const int i = i0 + ml;
        float s = acc[bm][bn][r];
        if (NORM) s *= s_rx[ml] * ryj;
        const float e = fast_exp2(fmaf(s, c, -c));
        float gv = LIT ? e * s_ir[ml] : e * (s_ir[ml] + icj);
        gv = (i < N && j < N && i != j) ? gv : 0.f;
        Gb[(int64_t)ml * bg.bs + nl] = C::pack(gv);
      }
    }
  }
}

// One launch per diagonal.  Workgroups [0, tiles_x) produce dX tiles, the rest
// (CLIP only) dY tiles; each output tile is owned by exactly one workgroup, so
// accumulation across diagonals is a plain read-modify-write.
template <typename T, bool NORM, bool VEC, bool ACCUM>
__global__ __launch_bounds__(256, 2) void k_grad_contract(
    const T* __restrict__ X, int64_t ldx, const T* __restrict__ Y, int64_t ldy, int N, int D,
    const float* __restrict__ ws, const T* __restrict__ G, BlockGrid bg, int tiles_x,
    float* __restrict__ acc_x, float* __restrict__ acc_y) {
  using C = Core<T>;
  __shared__ __attribute__((aligned(16))) char lds[C::LDS_BYTES];
  const int64_t n64 = N;
  const int tdn = (D + 127) / 128;
  const bool is_x = (int)blockIdx.x < tiles_x;
  const int bid = is_x ? blockIdx.x : blockIdx.x - tiles_x;
  const int nbid = is_x ? tiles_x : gridDim.x - tiles_x;
  int tmg, td;
  tile_swizzle(bid, nbid, bg.nb * bg.tpb, tdn, 8, tmg, td);
  const int P = tmg / bg.tpb, tm = tmg - P * bg.tpb;  // P: block owning the output rows
  const int r0 = P * bg.bs + tm * 128;
  if (r0 >= N) return;
  const int d0 = td * 128;
  // partner block along the contraction index
  const int Q = is_x ? (P + bg.shift) % bg.nb : (P - bg.shift + bg.nb) % bg.nb;
  const int q0 = Q * bg.bs;
  const int qn = min(bg.bs, N - q0);
  f32x16 acc[2][2];
  if (is_x) {
    // dX[i, d] += sum_j G'[i, j] * ry_j * Y[j, d],  G' block (P, Q) row-major
    typename C::Op A{G + (int64_t)P * bg.bs * bg.bs + (int64_t)(tm * 128) * bg.bs, bg.bs, 128, qn, nullptr};
    typename C::Op B{Y + (int64_t)q0 * ldy + d0, ldy, D - d0, qn, NORM ? ws + WS_RY * n64 + q0 : nullptr};
    C::template run<C::KM, C::MN, VEC>(A, B, qn, lds, acc);
  } else {
    // dY[j, d] += sum_i G'[i, j] * rx_i * X[i, d],  G' block (Q, P) read transposed
    typename C::Op A{G + (int64_t)Q * bg.bs * bg.bs + tm * 128, bg.bs, 128, qn, nullptr};
    typename C::Op B{X + (int64_t)q0 * ldx + d0, ldx, D - d0, qn, NORM ? ws + WS_RX * n64 + q0 : nullptr};
    C::template run<C::MN, C::MN, VEC>(A, B, qn, lds, acc);
  }
  float* out = is_x ? acc_x : acc_y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w >> 1, wn = w & 1;
#pragma unroll
  for (int bm = 0; bm < 2; ++bm) {
#pragma unroll
    for (int bn = 0; bn < 2; ++bn) {
      const int d = d0 + wn * 64 + bn * 32 + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = r0 + wm * 64 + bm * 32 + acc_row(r, lane);
        if (row < N && d < D) {
          float* p = out + (int64_t)row * D + d;
          *p = ACCUM ? *p + acc[bm][bn][r] : acc[bm][bn][r];
        }
      }
    }
  }
}

}  // namespace mec
