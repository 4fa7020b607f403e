// MFMA tile kernels of the contrastive-loss hot path (fp32 and bf16 inputs;
// the element type selects the MFMA core, the epilogues are shared):
//   k_sumexp        forward: tiled S = X Y^T, E = exp2(S c - c), off-diagonal
//                       row (and column) partial sums, one atomic per row/column
//                       per tile.  Replaces clip_sum_exp_kernel (clip_loss.py:9-64)
//                       and lit_sum_exp_kernel (lit_loss.py:9-62).
//   k_grad_step     backward, one launch per pipeline step t = 0..nb over
//                       the block diagonals of the N x N gradient matrix:
//                       recompute S for diagonal t and write the blocks
//                       G'_ij = E_ij (1/R_i + 1/C_j) (LiT: E_ij / R_i), i != j,
//                       to one of two bounded scratch buffers
//                       (clip_loss.py:96-124, lit_loss.py:94-120), while
//                       contracting diagonal t-1 from the other buffer:
//                       dX_I += G'_IJ Y^_J and dY_J += G'_IJ^T X^_I as plain MFMA
//                       contractions without atomics (clip_loss.py:127-156,
//                       lit_loss.py:123-148).
#pragma once
#include "mec_gemm_f32.h"
#include "mec_gemm_bf16.h"

namespace mec {

// Element-type traits: which MFMA core runs the tile, and how G' is stored.
// BKB is the K chunk depth of the bf16 core (the fp32 core has one depth).
#ifndef MEC_BF16_BK_FWD
#define MEC_BF16_BK_FWD 64
#endif
#ifndef MEC_BF16_BK_BWD
#define MEC_BF16_BK_BWD 64
#endif
template <typename T, int BKB> struct Core;
template <int BKB> struct Core<float, BKB> {
  using Op = g32::Operand;
  static constexpr int LDS_BYTES = g32::LDS_FLOATS * 4;
  template <bool VECA, bool VECB>
  static __device__ __forceinline__ void run(const Op& a, const Op& b, int K, void* lds, f32x16 (&acc)[2][2]) {
    g32::mainloop<VECA, VECB>(a, b, K, (float*)lds, acc);
  }
  static __device__ __forceinline__ float pack(float v) { return v; }
  // 4 consecutive values as one vector store
  static __device__ __forceinline__ void store4(float* p, float a, float b, float c, float d) {
    *(f32x4*)p = f32x4{a, b, c, d};
  }
};
template <int BKB> struct Core<uint16_t, BKB> {
  using Op = g16::Operand;
  static constexpr int LDS_BYTES = g16::Cfg<BKB>::LDS_ELEMS * 2;
  template <bool VECA, bool VECB>
  static __device__ __forceinline__ void run(const Op& a, const Op& b, int K, void* lds, f32x16 (&acc)[2][2]) {
    g16::mainloop<BKB, VECA, VECB>(a, b, K, (uint16_t*)lds, acc);
  }
  static __device__ __forceinline__ uint16_t pack(float v) { return f32_to_bf16(v); }
  static __device__ __forceinline__ void store4(uint16_t* p, float a, float b, float c, float d) {
    uint2 u;
    u.x = (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
    u.y = (uint32_t)f32_to_bf16(c) | ((uint32_t)f32_to_bf16(d) << 16);
    *(uint2*)p = u;
  }
};
template <typename T> using CoreFwd = Core<T, MEC_BF16_BK_FWD>;
template <typename T> using CoreBwd = Core<T, MEC_BF16_BK_BWD>;

// ---------------------------------------------------------------- forward
// E = exp2(S c - c) of this wave's 64x64 accumulators (S scaled by rx_i ry_j
// when NORM); rowv[bm * 16 + r] and colv[bn] collect this lane's partial row
// and column sums.  MASK zeroes the diagonal and entries outside [0, N).
template <bool NORM, bool MASK>
__device__ __forceinline__ void sumexp_epilogue(const f32x16 (&acc)[2][2], float c, int m0, int n0, int N,
                                                const float* s_rx, const float* s_ry, float (&rowv)[32],
                                                float (&colv)[2]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w >> 1, wn = w & 1;
#pragma unroll
  for (int k = 0; k < 32; ++k) rowv[k] = 0.f;
#pragma unroll
  for (int bm = 0; bm < 2; ++bm) {
#pragma unroll
    for (int bn = 0; bn < 2; ++bn) {
      const int nl = wn * 64 + bn * 32 + (lane & 31);
      const int j = n0 + nl;
      const float cy = NORM ? c * s_ry[nl] : c;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ml = wm * 64 + bm * 32 + acc_row(r, lane);
        const int i = m0 + ml;
        const float sc = NORM ? acc[bm][bn][r] * s_rx[ml] : acc[bm][bn][r];
        float e = fast_exp2(fmaf(sc, cy, -c));
        if (MASK) e = (i < N && j < N && i != j) ? e : 0.f;
        rowv[bm * 16 + r] += e;
        colv[bn] += e;
      }
    }
  }
}

template <typename T, bool LIT, bool NORM, bool VEC>
__global__ __launch_bounds__(256, 2) void k_sumexp(const T* __restrict__ X, int64_t ldx,
                                                   const T* __restrict__ Y, int64_t ldy, int N,
                                                   int D, float c, float* __restrict__ ws, int tiles) {
  using C = CoreFwd<T>;
  __shared__ __attribute__((aligned(16))) char lds[C::LDS_BYTES];
  __shared__ float s_rx[128], s_ry[128], s_row[128], s_col[128];
  const int64_t n64 = N;
  int tm, tn;
  tile_swizzle(blockIdx.x, gridDim.x, tiles, tiles, 8, tm, tn);
  const int m0 = tm * 128, n0 = tn * 128;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, wm = w >> 1, wn = w & 1;

  typename C::Op A{X + (int64_t)m0 * ldx, ldx, N - m0, D};
  typename C::Op B{Y + (int64_t)n0 * ldy, ldy, N - n0, D};
  f32x16 acc[2][2];
  C::template run<VEC, VEC>(A, B, D, lds, acc);

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
  // interior tiles (no diagonal entry, no row or column beyond N) need no mask
  if (m0 != n0 && m0 + 128 <= N && n0 + 128 <= N)
    sumexp_epilogue<NORM, false>(acc, c, m0, n0, N, s_rx, s_ry, rowv, colv);
  else
    sumexp_epilogue<NORM, true>(acc, c, m0, n0, N, s_rx, s_ry, rowv, colv);
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
// (bs a multiple of 128; the last block may be short).  Diagonal s pairs block
// I with block J = (I + s) mod nb, so one diagonal touches every block row and
// every block column exactly once.
struct BlockGrid {
  int bs;   // block size (rows), multiple of 128
  int nb;   // number of blocks (= number of diagonals)
  int tpb;  // 128-tiles per block side = bs / 128
};

// Scratch of the backward (all in the input dtype T, row-major):
//   G[2]   two buffers of nb blocks of bs x bs: block I of buffer s&1 holds
//          G'(I, (I+s) mod nb) of diagonal s;
//   GT[2]  the same blocks transposed (CLIP only);
//   XT, YT the normalised inputs transposed, [D][ldt] with ldt = N rounded
//          up to 128 and zero columns [N, ldt): element (d, i) = rx_i x_i[d].
// Every contraction operand is then K-major (k contiguous).
struct GradBufs {
  void* g[2];
  void* gt[2];
  const void* xt;
  const void* yt;
  int64_t ldt;
};

// One pipeline step of the backward (launch t = 0 .. nb):
//   workgroups [0, cx_pad)               x side of the contraction of diagonal t-1
//   [cx_pad, cx_pad + cy_pad)            y side (CLIP)
//   [cx_pad + cy_pad, ... + g_pad)       G' tiles of diagonal t
// The long contraction tiles (K = bs) come first so the short G' tiles
// (K = d) fill the tail of the launch.  Each sub-range starts at a multiple
// of 8, so `id % 8` is still the XCD a workgroup runs on.
struct StepPlan {
  int diag_g;        // diagonal whose G' this launch writes (-1: none)
  int diag_c;        // diagonal this launch contracts (-1: none)
  int accumulate;    // contraction adds to the accumulators (else overwrites)
  int g_n, g_pad;    // G' tiles (nb * tpb * tpb or 0), padded to a multiple of 8
  int cx_n, cx_pad;  // x-side contraction tiles (nb * tpb * ceil(D/128) or 0), padded
  int cy_n, cy_pad;  // y-side contraction tiles, padded
};

// G'_ij of this wave's 64x64 accumulators into Gb (and GTb for CLIP).  MASK
// zeroes the diagonal and entries outside [0, N).
template <typename T, bool LIT, bool NORM, bool MASK>
__device__ __forceinline__ void grad_g_store(const f32x16 (&acc)[2][2], float c, int i0, int j0, int N,
                                             T* __restrict__ Gb, T* __restrict__ GTb, int bs, const float* s_rx,
                                             const float* s_ry, const float* s_ir, const float* s_ic) {
  using C = CoreBwd<T>;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w >> 1, wn = w & 1;
#pragma unroll
  for (int bm = 0; bm < 2; ++bm) {
#pragma unroll
    for (int bn = 0; bn < 2; ++bn) {
      const int nl = wn * 64 + bn * 32 + (lane & 31);
      const int j = j0 + nl;
      const float cy = NORM ? c * s_ry[nl] : c;
      const float icj = s_ic[nl];
      float gv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ml = wm * 64 + bm * 32 + acc_row(r, lane);
        const int i = i0 + ml;
        const float sc = NORM ? acc[bm][bn][r] * s_rx[ml] : acc[bm][bn][r];
        const float e = fast_exp2(fmaf(sc, cy, -c));
        float g = LIT ? e * s_ir[ml] : e * (s_ir[ml] + icj);
        if (MASK) g = (i < N && j < N && i != j) ? g : 0.f;
        gv[r] = g;
        Gb[(int64_t)ml * bs + nl] = C::pack(g);
      }
      if (!LIT) {
        // registers 4g..4g+3 hold 4 consecutive rows: one vector store per group
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int ml = wm * 64 + bm * 32 + acc_row(4 * g, lane);
          C::store4(GTb + (int64_t)nl * bs + ml, gv[4 * g], gv[4 * g + 1], gv[4 * g + 2], gv[4 * g + 3]);
        }
      }
    }
  }
}

// Recompute the similarity tile (i0, j0) and store G'_ij = E_ij (1/R_i + 1/C_j)
// (LiT: E_ij / R_i) for i != j, 0 on the diagonal and outside [0, N), into
// the G' block at Gb (row pitch bs) and, for CLIP, transposed at GTb.
// Follows clip_loss.py:96-124 / lit_loss.py:94-120.
template <typename T, bool LIT, bool NORM, bool VEC>
__device__ __forceinline__ void grad_g_tile(const T* __restrict__ X, int64_t ldx, const T* __restrict__ Y,
                                            int64_t ldy, int N, int D, float c, const float* __restrict__ ws,
                                            T* __restrict__ Gb, T* __restrict__ GTb, int bs, int i0, int j0,
                                            char* lds, float* s_rx, float* s_ry, float* s_ir, float* s_ic) {
  using C = CoreBwd<T>;
  const int64_t n64 = N;
  const int t = threadIdx.x;
  typename C::Op A{X + (int64_t)i0 * ldx, ldx, N - i0, D};
  typename C::Op B{Y + (int64_t)j0 * ldy, ldy, N - j0, D};
  f32x16 acc[2][2];
  C::template run<VEC, VEC>(A, B, D, lds, acc);
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
  if (i0 != j0 && i0 + 128 <= N && j0 + 128 <= N)
    grad_g_store<T, LIT, NORM, false>(acc, c, i0, j0, N, Gb, GTb, bs, s_rx, s_ry, s_ir, s_ic);
  else
    grad_g_store<T, LIT, NORM, true>(acc, c, i0, j0, N, Gb, GTb, bs, s_rx, s_ry, s_ir, s_ic);
}

// One 128 x 128 output tile of a contraction: rows r0.. of block P, feature
// columns d0..:
//   x side: acc_x[i, d] (+)= sum_{j in Q} G'(P,Q)[i, j]  * YT[d, j]   (Q = P + s)
//   y side: acc_y[j, d] (+)= sum_{i in Q} G'T(Q,P)[j, i] * XT[d, i]   (Q = P - s)
// Each output tile has one owner per launch: accumulation across launches
// adds each element once per launch, in launch order (the reference instead
// lets every (row-tile, column-tile) program add into dX/dY with contending
// atomics, clip_loss.py:148-156).
template <typename T>
__device__ __forceinline__ void grad_contract_tile(int N, int D, const T* __restrict__ Gblk,
                                                   const T* __restrict__ OT, int64_t ldt, const BlockGrid& bg,
                                                   int P, int Q, int tm, int td, bool accumulate,
                                                   float* __restrict__ out, char* lds) {
  using C = CoreBwd<T>;
  const int r0 = P * bg.bs + tm * 128;
  if (r0 >= N) return;
  const int d0 = td * 128;
  const int q0 = Q * bg.bs;
  const int qn = min(bg.bs, N - q0);
  typename C::Op A{Gblk + (int64_t)(tm * 128) * bg.bs, bg.bs, 128, qn};
  typename C::Op B{OT + (int64_t)d0 * ldt + q0, ldt, D - d0, qn};
  f32x16 acc[2][2];
  C::template run<true, true>(A, B, qn, lds, acc);
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
          // a fire-and-forget add in L2 instead of a load-add-store round trip;
          // the tile has one owner per launch, so the summation order (launch
          // order) and the result are deterministic
          if (accumulate)
            __hip_atomic_fetch_add(p, acc[bm][bn][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          else
            *p = acc[bm][bn][r];
        }
      }
    }
  }
}

template <typename T, bool LIT, bool NORM, bool VEC>
__global__ __launch_bounds__(256, 3) void k_grad_step(const T* __restrict__ X, int64_t ldx,
                                                      const T* __restrict__ Y, int64_t ldy, int N, int D,
                                                      float c, const float* __restrict__ ws, GradBufs gb,
                                                      BlockGrid bg, StepPlan sp, float* __restrict__ acc_x,
                                                      float* __restrict__ acc_y) {
  using C = CoreBwd<T>;
  __shared__ __attribute__((aligned(16))) char lds[C::LDS_BYTES];
  __shared__ float s_rx[128], s_ry[128], s_ir[128], s_ic[128];
  const int tdn = (D + 127) / 128;
  const int64_t blk = (int64_t)bg.bs * bg.bs;  // elements per G' block
  int sub = blockIdx.x;
  if (sub < sp.cx_pad + sp.cy_pad) {
    const bool is_x = sub < sp.cx_pad;
    if (!is_x) sub -= sp.cx_pad;
    const int pid = xcd_remap(sub, is_x ? sp.cx_pad : sp.cy_pad);
    if (pid >= (is_x ? sp.cx_n : sp.cy_n)) return;
    int tmg, td;
    group_tile(pid, bg.nb * bg.tpb, tdn, 8, tmg, td);
    const int P = tmg / bg.tpb, tm = tmg - P * bg.tpb;  // P: block owning the output rows
    const int buf = sp.diag_c & 1;
    if (is_x) {
      const int Q = (P + sp.diag_c) % bg.nb;
      grad_contract_tile<T>(N, D, (const T*)gb.g[buf] + P * blk, (const T*)gb.yt, gb.ldt, bg, P, Q, tm, td,
                            sp.accumulate != 0, acc_x, lds);
    } else {
      const int Q = (P - sp.diag_c + bg.nb) % bg.nb;
      grad_contract_tile<T>(N, D, (const T*)gb.gt[buf] + Q * blk, (const T*)gb.xt, gb.ldt, bg, P, Q, tm, td,
                            sp.accumulate != 0, acc_y, lds);
    }
    return;
  }
  sub -= sp.cx_pad + sp.cy_pad;
  const int pid = xcd_remap(sub, sp.g_pad);
  if (pid >= sp.g_n) return;
  int tmg, tn;
  group_tile(pid, bg.nb * bg.tpb, bg.tpb, 8, tmg, tn);
  const int I = tmg / bg.tpb, tm = tmg - I * bg.tpb;
  const int J = (I + sp.diag_g) % bg.nb;
  const int i0 = I * bg.bs + tm * 128, j0 = J * bg.bs + tn * 128;
  if (i0 >= N || j0 >= N) return;  // never read by the contraction
  const int buf = sp.diag_g & 1;
  T* Gb = (T*)gb.g[buf] + I * blk + (int64_t)(tm * 128) * bg.bs + tn * 128;
  T* GTb = LIT ? nullptr : (T*)gb.gt[buf] + I * blk + (int64_t)(tn * 128) * bg.bs + tm * 128;
  grad_g_tile<T, LIT, NORM, VEC>(X, ldx, Y, ldy, N, D, c, ws, Gb, GTb, bg.bs, i0, j0, lds, s_rx, s_ry, s_ir,
                                 s_ic);
}

}  // namespace mec
