// O(N*D) and O(N) kernels around the MFMA hot loops: the normalisation /
// diagonal pre-pass, the loss finalize, and the gradient post-pass.  These are
// HBM-bound; one 64-lane wave owns one feature row.
#pragma once
#include "mec_common.h"

namespace mec {

template <typename T> struct Elem;
template <> struct Elem<float> {
  static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store(float* p, int64_t i, float v) { p[i] = v; }
};
template <> struct Elem<uint16_t> {  // bf16 bits
  static __device__ __forceinline__ float load(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
  static __device__ __forceinline__ void store(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
};
template <> struct Elem<_Float16> {
  static __device__ __forceinline__ float load(const _Float16* p, int64_t i) { return (float)p[i]; }
  static __device__ __forceinline__ void store(_Float16* p, int64_t i, float v) { p[i] = (_Float16)v; }
};

// Per row i: rx = 1/max(||x_i||, 1e-12) (or 1), ry likewise, diag = x_i . y_i.
// Also clears the off-diagonal sum accumulators used by the sum-exp kernel.
// Follows F.normalize(dim=1) as applied at clip_loss.py:266-268 and the
// einsum('bi,bi->b') diagonal at clip_loss.py:206.
template <typename T, bool NORM>
__global__ __launch_bounds__(256) void k_prepass(const T* __restrict__ X, int64_t ldx,
                                                 const T* __restrict__ Y, int64_t ldy, int N, int D,
                                                 float* __restrict__ ws) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const T* x = X + (int64_t)row * ldx;
  const T* y = Y + (int64_t)row * ldy;
  float sx = 0.f, sy = 0.f, sxy = 0.f;
  for (int d = lane; d < D; d += 64) {
    float a = Elem<T>::load(x, d), b = Elem<T>::load(y, d);
    sx = fmaf(a, a, sx);
    sy = fmaf(b, b, sy);
    sxy = fmaf(a, b, sxy);
  }
  sx = wave_sum(sx);
  sy = wave_sum(sy);
  sxy = wave_sum(sxy);
  if (lane == 0) {
    const int64_t n = N;
    float rx = 1.f, ry = 1.f;
    if (NORM) {
      rx = 1.f / fmaxf(sqrtf(sx), 1e-12f);
      ry = 1.f / fmaxf(sqrtf(sy), 1e-12f);
    }
    ws[WS_RX * n + row] = rx;
    ws[WS_RY * n + row] = ry;
    ws[WS_DIAG * n + row] = sxy;
    ws[WS_ROW_OFF * n + row] = 0.f;
    ws[WS_COL_OFF * n + row] = 0.f;
  }
}

// Loss epilogue (clip_loss.py:206-211, lit_loss.py:199-203) plus the per-row
// quantities the backward needs.  In natural-log units with t_i = (s_ii-1)/T:
//   R_i = row_off_i + e^{t_i},  l^r_i = ln R_i - t_i = softplus(ln row_off_i - t_i)
// which is the same cross-entropy term as -ln(2^Sv_i / R_i) in the reference,
// evaluated without cancellation.  CLIP averages (l^r + l^c)/2, LiT uses l^r.
// kappa_i = -(row_off_i/R_i + col_off_i/C_i) is the exact diagonal entry of
// the gradient matrix in units of a = grad_scale/(2N) (LiT: grad_scale/N).
// Two passes (rows, then the sum of per-workgroup partials), fp64
// accumulation in a fixed order: deterministic.
__device__ __forceinline__ double softplus_log_ratio(double off, double t) {
  if (!(off > 0.0)) return 0.0;
  double u = log(off) - t;
  return u > 0.0 ? u + log1p(exp(-u)) : log1p(exp(u));
}

// The loss term of row i (a CLIP row and column, or a LiT row), and 1/R_i,
// 1/C_i and kappa_i into the workspace.
template <bool LIT>
__device__ __forceinline__ double finalize_row(int i, int64_t n, double inv_t, float* __restrict__ ws) {
  const double s = (double)ws[WS_DIAG * n + i] * (double)ws[WS_RX * n + i] * (double)ws[WS_RY * n + i];
  const double t = (s - 1.0) * inv_t;
  const double e = exp(t);
  const double ro = ws[WS_ROW_OFF * n + i];
  const double R = ro + e;
  double acc = softplus_log_ratio(ro, t);
  ws[WS_INV_ROW * n + i] = (float)(1.0 / R);
  double kap = -(ro / R);
  if (!LIT) {
    const double co = ws[WS_COL_OFF * n + i];
    const double C = co + e;
    acc += softplus_log_ratio(co, t);
    ws[WS_INV_COL * n + i] = (float)(1.0 / C);
    kap -= co / C;
  }
  ws[WS_KAPPA * n + i] = (float)kap;
  return acc;
}

// Pass 1: one thread per row (rows beyond N contribute nothing), FIN_ROWS
// rows per workgroup; each workgroup writes the fp64 sum of its rows' loss
// terms to partial[blockIdx.x].  SINGLE (N <= FIN_SINGLE_ROWS): one
// workgroup of FIN_SINGLE_ROWS threads, one row each, writes the loss itself
// (no second pass).  One row per thread spreads the rows' fp64 work over N /
// 256 CUs: with one 1024-thread workgroup taking up to four rows per thread
// up to N = 4096, the finalize took 11 us at N = 2048 and 21 us at N = 4096
// (each row's loads, fp64 exp / log and stores one after the other on one
// CU), against 8.8 and 9.4 us for both passes now; up to 1024 rows the one
// workgroup stays faster than two launches (6 against 9 us).
constexpr int FIN_SINGLE_ROWS = 1024;
template <bool LIT, bool SINGLE>
__global__ __launch_bounds__(SINGLE ? FIN_SINGLE_ROWS : FIN_ROWS) void k_finalize_rows(
    int N, double inv_t, float* __restrict__ ws, double* __restrict__ partial, float* __restrict__ loss) {
  constexpr int NT = SINGLE ? FIN_SINGLE_ROWS : FIN_ROWS;
  __shared__ double red[NT / 64];
  const int64_t n = N;
  const int i = blockIdx.x * NT + threadIdx.x;
  double acc = i < N ? finalize_row<LIT>(i, n, inv_t, ws) : 0.0;
  acc = wave_sum_f64(acc);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double tot = 0.0;
    for (int k = 0; k < NT / 64; ++k) tot += red[k];
    if (SINGLE)
      *loss = (float)(tot / (LIT ? (double)N : 2.0 * (double)N));
    else
      partial[blockIdx.x] = tot;
  }
}

// Pass 2 (one workgroup): loss = sum of the partials in a fixed order / (N or 2N).
template <bool LIT>
__global__ __launch_bounds__(1024) void k_finalize_sum(int N, int nparts, const double* __restrict__ partial,
                                                       float* __restrict__ loss) {
  __shared__ double red[16];
  double acc = 0.0;
  for (int k = threadIdx.x; k < nparts; k += blockDim.x) acc += partial[k];
  acc = wave_sum_f64(acc);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double tot = 0.0;
    for (int k = 0; k < (int)(blockDim.x >> 6); ++k) tot += red[k];
    *loss = (float)(tot / (LIT ? (double)N : 2.0 * (double)N));
  }
}

// Gradient post-pass for one side.  With acc the off-diagonal contraction
// sum_{j != i} G'_ij * oth^_j (oth^ = normalised other side) and a the
// scale grad_scale/(2N) (LiT: /N):
//   d_own^_i = a * (acc_i + kappa_i * oth^_i)                       (diag term)
//   d_own_i  = r_i (d_own^_i - own^_i <own^_i, d_own^_i>)            (F.normalize bwd)
//            = r_i d_own^_i                                           (if ||own_i|| <= eps)
//   out_i    = grad_output * d_own_i                                 (clip_loss.py:252-254)
// out may alias acc (fp32 outputs): every element is read before it is written
// by the same lane.  One wave per row; rows of D <= 64 * POST_REG are read
// once (held in registers across the reduction), longer rows twice.
constexpr int POST_REG = 32;
// One side of the post-pass (the x side: own = x, oth = y, acc_x -> dx); the
// two sides share one launch: blockIdx.y picks the side.
template <typename T>
struct PostSide {
  const T* own;
  int64_t ld_own;
  const T* oth;
  int64_t ld_oth;
  const float* r_own;
  const float* r_oth;
  const float* acc;
  T* out;
};
// ACCR (fp32 data on the fp32 kernels): the accumulator row carries the
// row's own inverse norm, acc = r_i (sum_j G'_ij y^_j), since the
// contractions multiply H = diag(rx) G' diag(ry) with the raw inputs.  Then
// h = a (kappa_i r_i y^_i + acc) = r_i dx^_i, and the normalisation backward
// r_i (dx^ - x^ <x^, dx^>) is h - x^ <x^, h>: no division by the norm.
// VEC (fp32; every row of own, oth, acc and out 16-byte aligned, D a multiple
// of 4): the register path reads and writes 16-byte vectors, four
// consecutive features per lane.
template <typename T, bool NORM, bool ACCR = false, bool VEC = false>
__global__ __launch_bounds__(256) void k_postpass(PostSide<T> s0, PostSide<T> s1, int N, int D,
                                                  const float* __restrict__ kappa, float a,
                                                  const float* __restrict__ grad_output) {
  static_assert(!VEC || std::is_same<T, float>::value, "16-byte vectors of fp32");
  const PostSide<T>& sd = blockIdx.y ? s1 : s0;
  const T* __restrict__ own = sd.own;
  const int64_t ld_own = sd.ld_own;
  const T* __restrict__ oth = sd.oth;
  const int64_t ld_oth = sd.ld_oth;
  const float* __restrict__ r_own = sd.r_own;
  const float* __restrict__ r_oth = sd.r_oth;
  const float* acc = sd.acc;
  T* out = sd.out;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const T* xo = own + (int64_t)row * ld_own;
  const T* yo = oth + (int64_t)row * ld_oth;
  const float* ac = acc + (int64_t)row * D;
  T* o = out + (int64_t)row * D;
  const float ro = r_own[row];
  const float kq = kappa[row] * r_oth[row] * (ACCR ? ro : 1.f);
  const float go = grad_output ? *grad_output : 1.f;
  if (NORM) {
    float dot = 0.f;
    const bool clamped = ro >= 1e12f;
    if (VEC && D <= 64 * POST_REG) {
      constexpr int NV = POST_REG / 4;
      f32x4 g[NV], xr[NV];
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int d = 4 * lane + 256 * k;
        g[k] = f32x4{0.f, 0.f, 0.f, 0.f};
        xr[k] = g[k];
        if (d < D) {
          const f32x4 yv = *(const f32x4*)(yo + d), av = *(const f32x4*)(ac + d), xv = *(const f32x4*)(xo + d);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            g[k][u] = a * fmaf(kq, yv[u], av[u]);
            xr[k][u] = xv[u] * ro;
            dot = fmaf(xr[k][u], g[k][u], dot);
          }
        }
      }
      dot = wave_sum(dot);
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int d = 4 * lane + 256 * k;
        if (d < D) {
          f32x4 v;
#pragma unroll
          for (int u = 0; u < 4; ++u)
            v[u] = go * (ACCR ? (clamped ? g[k][u] : g[k][u] - xr[k][u] * dot)
                              : (clamped ? ro * g[k][u] : ro * (g[k][u] - xr[k][u] * dot)));
          *(f32x4*)((float*)o + d) = v;
        }
      }
      return;
    }
    if (D <= 64 * POST_REG) {
      // the row stays in registers between the reduction and the stores
      float g[POST_REG], xr[POST_REG];
#pragma unroll
      for (int k = 0; k < POST_REG; ++k) {
        const int d = lane + 64 * k;
        g[k] = 0.f;
        xr[k] = 0.f;
        if (d < D) {
          g[k] = a * fmaf(kq, Elem<T>::load(yo, d), ac[d]);
          xr[k] = Elem<T>::load(xo, d) * ro;
          dot = fmaf(xr[k], g[k], dot);
        }
      }
      dot = wave_sum(dot);
#pragma unroll
      for (int k = 0; k < POST_REG; ++k) {
        const int d = lane + 64 * k;
        if (d < D) {
          const float v = ACCR ? (clamped ? g[k] : g[k] - xr[k] * dot) : (clamped ? ro * g[k] : ro * (g[k] - xr[k] * dot));
          Elem<T>::store(o, d, go * v);
        }
      }
      return;
    }
    for (int d = lane; d < D; d += 64) {
      float g = a * fmaf(kq, Elem<T>::load(yo, d), ac[d]);
      dot = fmaf(Elem<T>::load(xo, d) * ro, g, dot);
    }
    dot = wave_sum(dot);
    for (int d = lane; d < D; d += 64) {
      float g = a * fmaf(kq, Elem<T>::load(yo, d), ac[d]);
      const float xh = Elem<T>::load(xo, d) * ro;
      float v = ACCR ? (clamped ? g : g - xh * dot) : (clamped ? ro * g : ro * (g - xh * dot));
      Elem<T>::store(o, d, go * v);
    }
  } else {
    for (int d = lane; d < D; d += 64) {
      float g = a * fmaf(kq, Elem<T>::load(yo, d), ac[d]);
      Elem<T>::store(o, d, go * g);
    }
  }
}

// One feature matrix to transpose: X (row pitch ldx), its row scales and the
// destination plane(s) (pitch ldt).  The transposes of the two sides share
// one launch: blockIdx.z picks the side.
template <typename T, typename TO = T>
struct TransSide {
  const T* X;
  int64_t ldx;
  const float* scale;
  TO* XT;
  TO* XTl;  // k_transpose_split with LO: the lo plane
};

// Transposed, normalised copy of one feature matrix for the backward's
// contractions: XT[d, i] = scale_i * X[i, d] (scale = 1/max(||x_i||, 1e-12)
// when NORM) for i < N and 0 for N <= i < ldt, rounded to T once.  64 x 64
// tiles through LDS; both the loads and the stores are coalesced.
template <typename T, bool NORM>
__global__ __launch_bounds__(256) void k_transpose(TransSide<T> s0, TransSide<T> s1, int N, int D, int64_t ldt) {
  const TransSide<T>& sd = blockIdx.z ? s1 : s0;
  const T* __restrict__ X = sd.X;
  const int64_t ldx = sd.ldx;
  const float* __restrict__ scale = sd.scale;
  T* __restrict__ XT = sd.XT;
  __shared__ float tile[64][65];
  const int i0 = blockIdx.x * 64, d0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int i = i0 + r, d = d0 + tx;
    float v = 0.f;
    if (i < N && d < D) {
      v = Elem<T>::load(X, (int64_t)i * ldx + d);
      if (NORM) v *= scale[i];
    }
    tile[r][tx] = v;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int d = d0 + r, i = i0 + tx;
    if (d < D && i < ldt) Elem<T>::store(XT, (int64_t)d * ldt + i, tile[tx][r]);
  }
}

// ------------------------------------------------- three-term bf16 split
// fp32 as the sum of two bf16 terms: hi = bf16(v), lo = bf16(v - hi), both
// rounded to nearest even (v - hi is exact in fp32), so v = hi + lo + r with
// |r| <= 2^-16 |v| (bf16 keeps 8 significant bits).  The bf16x3 mode forms
// every product a*b of the hot loops as hi_a*hi_b + lo_a*hi_b + hi_a*lo_b on
// the bf16 MFMA (fp32 accumulate); the dropped lo_a*lo_b and the two
// remainders bound the error of one product by about 3 * 2^-16 |ab|.
__device__ __forceinline__ void split2_bf16(float a, float b, uint32_t& hi, uint32_t& lo) {
  const uint16_t ha = f32_to_bf16(a), hb = f32_to_bf16(b);
  hi = (uint32_t)ha | ((uint32_t)hb << 16);
  lo = pack2_bf16(a - bf16_to_f32(ha), b - bf16_to_f32(hb));
}

// Split copies of the inputs for the similarity GEMMs of the bf16x3 mode.
// Row i of out (pitch ld3 elements) holds three segments of dp = D rounded up
// to 8 elements: ORDER 0 (x side) hi, lo, hi; ORDER 1 (y side) hi, hi, lo.
// The dot product of an x row with a y row over the 3 dp elements is then
// hi.hi + lo.hi + hi.lo, one bf16 GEMM with K = 3 dp.  Columns D .. dp-1 of
// each segment are zero.  NORM: the rows are normalized first (x_i rx_i in
// fp32, rx from the pre-pass), so that the GEMM kernels need no norm scaling.
// One thread per 8 columns; out and ld3 16-byte aligned.
template <int ORDER, bool NORM>
__global__ __launch_bounds__(256) void k_split3(const float* __restrict__ X, int64_t ldx, int N, int D, int dp,
                                                uint16_t* __restrict__ out, int64_t ld3,
                                                const float* __restrict__ rxv) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int vpr = dp / 8;
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (v >= (int64_t)N * vpr) return;
  const int i = (int)(v / vpr), d0 = (int)(v - (int64_t)i * vpr) * 8;
  const float* x = X + (int64_t)i * ldx;
  const float r = NORM ? rxv[i] : 1.f;
  u32x4 hi, lo;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int d = d0 + 2 * e;
    const float a = d < D ? x[d] * r : 0.f, b = d + 1 < D ? x[d + 1] * r : 0.f;
    uint32_t h, l;
    split2_bf16(a, b, h, l);
    hi[e] = h;
    lo[e] = l;
  }
  uint16_t* o = out + (int64_t)i * ld3 + d0;
  *(u32x4*)o = hi;
  *(u32x4*)(o + dp) = ORDER == 0 ? lo : hi;
  *(u32x4*)(o + 2 * dp) = ORDER == 0 ? hi : lo;
}

// bf16 copies of the inputs for the fp32-data / bf16-product mode: row i of
// out (pitch ldo) is bf16(x_i) (NORM: bf16(x_i rx_i)), round to nearest
// even, zero-padded to dp columns.  One thread per 8 columns; out and ldo
// 16-byte aligned.
template <bool NORM>
__global__ __launch_bounds__(256) void k_split1(const float* __restrict__ X, int64_t ldx, int N, int D, int dp,
                                                uint16_t* __restrict__ out, int64_t ldo,
                                                const float* __restrict__ rxv) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int vpr = dp / 8;
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (v >= (int64_t)N * vpr) return;
  const int i = (int)(v / vpr), d0 = (int)(v - (int64_t)i * vpr) * 8;
  const float* x = X + (int64_t)i * ldx;
  const float r = NORM ? rxv[i] : 1.f;
  u32x4 hi;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int d = d0 + 2 * e;
    hi[e] = pack2_bf16(d < D ? x[d] * r : 0.f, d + 1 < D ? x[d + 1] * r : 0.f);
  }
  *(u32x4*)(out + (int64_t)i * ldo + d0) = hi;
}

// k_transpose<float, NORM> into bf16 planes: XT_hi[d][i] = hi(v) and, when
// LO, XT_lo[d][i] = lo(v), with v = scale_i x_i[d] (fp32), zero for
// N <= i < ldt.
template <bool NORM, bool LO>
__global__ __launch_bounds__(256) void k_transpose_split(TransSide<float, uint16_t> s0,
                                                         TransSide<float, uint16_t> s1, int N, int D, int64_t ldt) {
  const TransSide<float, uint16_t>& sd = blockIdx.z ? s1 : s0;
  const float* __restrict__ X = sd.X;
  const int64_t ldx = sd.ldx;
  const float* __restrict__ scale = sd.scale;
  uint16_t* __restrict__ XTh = sd.XT;
  uint16_t* __restrict__ XTl = sd.XTl;
  __shared__ float tile[64][65];
  const int i0 = blockIdx.x * 64, d0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int i = i0 + r, d = d0 + tx;
    float v = 0.f;
    if (i < N && d < D) {
      v = X[(int64_t)i * ldx + d];
      if (NORM) v *= scale[i];
    }
    tile[r][tx] = v;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int d = d0 + r, i = i0 + tx;
    if (d < D && i < ldt) {
      const float v = tile[tx][r];
      const uint16_t h = f32_to_bf16(v);
      XTh[(int64_t)d * ldt + i] = h;
      if (LO) XTl[(int64_t)d * ldt + i] = f32_to_bf16(v - bf16_to_f32(h));
    }
  }
}

}  // namespace mec
