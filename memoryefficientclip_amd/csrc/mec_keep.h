// Small fp32 problems with the similarity matrix kept from the forward to
// the backward (MEC_FLAG_KEEP_EXP, n <= MEC_KEEP_EXP_MAX_N, 16-byte rows).
//
// At n ~ 1000 every launch is short and the similarity GEMM is a large part
// of the step.  The forward keeps the similarities (np x np floats, np = n
// rounded up to 64) and turns them into the scaled gradient matrix H =
// diag(rx) G' diag(ry) once the sums are known; the backward contracts H
// instead of recomputing S tile by tile (clip_loss.py:96-124 recomputes it in
// every backward program).  Launches:
//   forward   k_keep_forward: 64 x 64 similarity tiles (eight waves, a
//             split k); the inverse norms
//             from the tiles' own operand fragments (no pre-pass), the raw
//             diagonal from the diagonal tiles' accumulators, the exponent's
//             row-scaled similarity S_ij rx_i stored, and each tile's row and
//             column sums of E = exp((S-1)/T) written to per-tile slots;
//             k_keep_finalize: per 64 x 64 block, the sums of its rows and
//             columns in tile order, 1/R and 1/C, the block turned into H in
//             place, and the block's row and column sums of G'_ij cos_ij
//             (cos = x^ . y^), which the normalisation backward needs; the
//             diagonal blocks also write the loss terms, kappa and the
//             workspace vectors, and add their loss partials as fixed-point
//             integers into one atomic word, the last of them writing the
//             loss.  Fixed-order or exact sums only: the loss and the
//             gradients are bitwise reproducible.
//   backward  k_keep_contract: 64 x 64 output tiles of H Y and H^T X.
//             mec_backward: with the post-pass in the tiles' epilogue (one
//             launch); mec_grad: the accumulators as mec_grad leaves them for
//             fp32, for the separate post-pass.
#pragma once
#include "mec_kernels.h"
#include "mec_rowops.h"

namespace mec {

constexpr int KEEP_T = 64;                       // tile (and index block) size
constexpr int KEEP_MAX_N = 2048;                 // MEC_KEEP_EXP_MAX_N
constexpr int KEEP_MAX_KT = KEEP_MAX_N / KEEP_T;  // blocks per side
// the finalize's loss word: bits 0-5 count the diagonal blocks, bits 6-61
// hold the fixed-point sum, bit 62 flags a partial past KEEP_LOSS_CAP, bit 63
// a NaN partial
constexpr unsigned long long KEEP_LOSS_OVF = 1ull << 62, KEEP_LOSS_NAN = 1ull << 63;
constexpr double KEEP_LOSS_CAP = 2251799813685248.0;  // 2^51: 32 of them fill bits 6-61
static_assert(KEEP_MAX_KT <= 63 && KEEP_LOSS_CAP * KEEP_MAX_KT * 64 <= (double)KEEP_LOSS_OVF, "loss word fields");

// The kept matrix and the forward's bookkeeping, carved from the workspace by
// the host (256-byte aligned parts).
struct KeepBufs {
  float* S;         // np x np, row-major (pitch np): S_ij rx_i, then H after k_keep_finalize
  float* rowpart;   // [kt][np]: row sums of E over tile (p, q) at rowpart[q * np + i]
  float* colpart;   // [kt][np]: column sums of E over tile (p, q) at colpart[p * np + j] (CLIP)
  float* rowdot;    // [kt][np]: sum over the columns j of block q of G'_ij cos_ij at rowdot[q * np + i]
  float* coldot;    // [kt][np]: sum over the rows i of block p of G'_ij cos_ij at coldot[p * np + j] (CLIP)
  unsigned long long* lacc;  // the finalize's loss accumulator (k_keep_finalize)
  int np, kt;
};

// The 64 x 64 fp32 tiles of the forward and the contractions: 2 x 2
// sub-tiles of 32 x 32, each computed by two waves from alternate halves of
// every chunk's k-steps (KS = 2: eight waves, two per SIMD; one wave per SIMD
// left the MFMA pipe idle while it issued its own operand reads and loads),
// on a ring of SMALL_STAGES stages.  After the k-loop the sums are in k-group
// 0 (threads 0-255, the waves of a 2 x 2 tile); k-group 1 only takes part in
// the barriers.  The y side's contraction reads H transposed; both take the
// raw input rows as a k-major feature operand (16-byte lanes).
constexpr int KEEP_NT = 512;
using KeepTile = TileD<64, 64, false, 2, 2, gdma::K_F32, 2, false, false, 0, SMALL_STAGES, 2>;
using KeepConX = TileD<64, 64, false, 2, 2, gdma::K_F32, 2, false, false, 1, SMALL_STAGES, 2>;
using KeepConY = TileD<64, 64, true, 2, 2, gdma::K_F32, 2, false, false, 1, SMALL_STAGES, 2>;

// Forward tiles: one 64 x 64 tile (p, q) of S per workgroup (kt x kt grid,
// XCD-grouped order).  NORM: rx and ry from the squared norms the tile's own
// fragments accumulate (gdma::NormHook: a wave sees its k-group's half of
// every chunk for its 32 rows and 32 columns, and the two waves of a k-group
// that share those rows (columns) split that half by k parity; the four
// partials are added in a fixed order), written to the workspace by the tiles
// of the first block column (rx) and
// row (ry); rx = ry = 1 otherwise.  Every tile computes the same rx_i and
// ry_j (the same fragments in the same order), so the
// finalize's E_ij = exp2(s_ij c ry_j - c) from the stored s_ij = S_ij rx_i
// and the workspace's ry_j is bitwise the E these sums add.
template <bool LIT, bool NORM>
__global__ __launch_bounds__(KEEP_NT, 2) void k_keep_forward(const float* __restrict__ X, int64_t ldx,
                                                             const float* __restrict__ Y, int64_t ldy, int N, int D,
                                                             float c, float* __restrict__ ws, KeepBufs kb) {
  using TL = KeepTile;
  static_assert(TL::BM == KEEP_T && TL::BN == KEEP_T && TL::NT == KEEP_NT && TL::FM == 1 && TL::FN == 1 &&
                    TL::G::KS == 2,
                "64 x 64 tiles of 2 x 2 x 2 waves");
  __shared__ __attribute__((aligned(1024))) char lds[TL::LDS_BYTES];
  __shared__ float s_rx[KEEP_T], s_ry[KEEP_T], s_row[KEEP_T], s_col[KEEP_T];
  __shared__ float s_pa[2][2][KEEP_T], s_pb[2][2][KEEP_T];  // [k-group][wave column / row][index]
  const int64_t n64 = N;
  const int t = threadIdx.x, lane = t & 63, T = kb.kt;
  const int wm = TL::G::wave_m(), wn = TL::G::wave_n(), g = TL::G::wave_k();
  if (blockIdx.x == 0 && t == 0) *kb.lacc = 0ull;  // (k_keep_finalize runs after this launch)
  int tm, tn;
  tile_swizzle(blockIdx.x, T * T, T, T, 8, tm, tn);
  const int m0 = tm * KEEP_T, n0 = tn * KEEP_T;
  const auto A = tile_op<TL>(X + (int64_t)m0 * ldx, ldx, min(N - m0, KEEP_T), D);
  const auto B = tile_op<TL>(Y + (int64_t)n0 * ldy, ldy, min(N - n0, KEEP_T), D);
  f32x16 acc[1][1];
  float rxv = 1.f, ryv = 1.f;
  if constexpr (NORM) {
    // wave (wm, wn) takes the A squares at the k-values t % 2 == wn and the B
    // squares at t % 2 == wm: the two waves that share a row (column) split
    // its k between them (a compile-time split: one loop per wave position)
    using G = typename TL::G;
    float pa = 0.f, pb = 0.f;
    auto run = [&](auto hook) {
      TL::run_fh(A, B, D, lds, acc, hook);
      pa = hook.sa[0] + __shfl_xor(hook.sa[0], 32, 64);
      pb = hook.sb[0] + __shfl_xor(hook.sb[0], 32, 64);
    };
    if (wm == 0) {
      if (wn == 0)
        run(gdma::NormHook<G, 0, 0>());
      else
        run(gdma::NormHook<G, 1, 0>());
    } else {
      if (wn == 0)
        run(gdma::NormHook<G, 0, 1>());
      else
        run(gdma::NormHook<G, 1, 1>());
    }
    if (lane < 32) {
      s_pa[g][wn][wm * 32 + lane] = pa;
      s_pb[g][wm][wn * 32 + lane] = pb;
    }
    __syncthreads();
    if (t < KEEP_T) {
      // 1/max(||v||, 1e-12), as F.normalize (clip_loss.py:266-268)
      rxv = 1.f / fmaxf(sqrtf((s_pa[0][0][t] + s_pa[0][1][t]) + (s_pa[1][0][t] + s_pa[1][1][t])), 1e-12f);
      ryv = 1.f / fmaxf(sqrtf((s_pb[0][0][t] + s_pb[0][1][t]) + (s_pb[1][0][t] + s_pb[1][1][t])), 1e-12f);
    }
  } else {
    TL::template run<true, true>(A, B, D, lds, acc);
  }
  if (t < KEEP_T) {
    if (tn == 0 && m0 + t < N) ws[WS_RX * n64 + m0 + t] = rxv;
    if (tm == 0 && n0 + t < N) ws[WS_RY * n64 + n0 + t] = ryv;
  }
  // the raw diagonal x_i . y_i (clip_loss.py:206): in a diagonal wave of a
  // diagonal tile, lane l holds entry (c, c), c = l % 32, when l / 32 is bit
  // 2 of c, in accumulator register 4 (c / 8) + c % 4
  if (tm == tn && wm == wn && g == 0) {
    const int cc = lane & 31;
    if ((lane >> 5) == ((cc >> 2) & 1)) {
      const int rr = 4 * (cc >> 3) + (cc & 3);
      float v = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) v = r == rr ? acc[0][0][r] : v;
      const int i = m0 + wm * 32 + cc;
      if (i < N) ws[WS_DIAG * n64 + i] = v;
    }
  }
  float rs, cs;
  sumexp_tile<TL, LIT, NORM, true>(acc, c, m0, n0, N, rxv, ryv, s_rx, s_ry, s_row, s_col, rs, cs,
                                   kb.S + (int64_t)m0 * kb.np + n0, kb.np, g == 0);
  if (t < KEEP_T) {
    kb.rowpart[(int64_t)tn * kb.np + m0 + t] = rs;
    if (!LIT) kb.colpart[(int64_t)tm * kb.np + n0 + t] = cs;
  }
}

// Forward finalize, one 64 x 64 block (p, q) per workgroup: thread r < 64
// takes row i = 64 p + r (R_i = its off-diagonal sum, the tile sums in tile
// order, + e^{t_i}), thread 64 + r column j = 64 q + r (C_j, CLIP), in fp64
// as finalize_row; then, per entry, E_ij = exp2(s_ij c ry_j - c) from the
// stored s_ij = S_ij rx_i (0 on the diagonal and outside [0, N)), G'_ij =
// E_ij (1/R_i + 1/C_j) (LiT: E_ij / R_i), and the block becomes H_ij = rx_i
// ry_j G'_ij in place.  The block's row and column sums of G'_ij cos_ij
// (cos_ij = s_ij ry_j) go to rowdot and coldot: the normalisation backward's
// <x^_i, dx^_i> is a (kappa_i cos_ii + sum_j G'_ij cos_ij), which the fused
// backward takes from these instead of a reduction over the features.  The
// diagonal blocks (p = q: their rows and columns are the same indices) also
// write the loss terms and the workspace vectors of their indices
// (clip_loss.py:206-211, lit_loss.py:199-203).  Their loss partials (fp64
// sums over the block's rows in row order) meet in one 64-bit word, added by
// one atomic each: the partial rounded to a fixed-point integer (lscale, a
// power of two, units per 1), shifted up 6 bits, plus 1 in the low bits
// that count the blocks.  Integer addition is exact and does not depend on
// the order of arrival, so the total is reproducible bit for bit; the word
// carries both the data and the count, so no fence is needed; and the block
// whose addition completes the count writes the loss.  The host sizes lscale
// so that the total stays within KEEP_LOSS_CAP for |cos| <= 1; the 32
// blocks' sums of at most KEEP_LOSS_CAP each fill the 56-bit field below two
// flag bits, which a NaN partial (KEEP_LOSS_NAN: the loss is NaN) or one past
// the cap (KEEP_LOSS_OVF: +inf) set instead of adding.
// MKT >= kt: the tile partials each row's thread loads (16 when kt <= 16,
// which halves the finalize's loads at n <= 1024).
template <bool LIT, bool NORM, int MKT = KEEP_MAX_KT>
__global__ __launch_bounds__(256) void k_keep_finalize(int N, float c, double inv_t, double lscale,
                                                       float* __restrict__ ws, KeepBufs kb, float* __restrict__ loss) {
  static_assert(MKT % 4 == 0 && MKT <= KEEP_MAX_KT, "tile partials per row");
  __shared__ float s_ir[KEEP_T], s_ic[KEEP_T], s_rx[KEEP_T], s_ry[KEEP_T];
  __shared__ double s_term[2 * KEEP_T], s_kap[2 * KEEP_T];
  // G'_ij cos_ij of the block; column j at j ^ 8 in the upper half of the
  // row: with the odd pitch this keeps the 16-column groups of a half-wave's
  // stores (rows r .. r + 7, columns 0, 16, 32, 48 + k) on distinct banks
  __shared__ float s_gc[KEEP_T][KEEP_T + 1];
  auto gcol = [](int j) { return j ^ (((j >> 5) & 1) << 3); };
  const int64_t n64 = N;
  const int t = threadIdx.x, T = kb.kt;
  const int p = blockIdx.x / T, q = blockIdx.x - p * T;
  const bool dg = p == q;
  // thread t's part of the block, row t / 4, 16 consecutive columns: loaded
  // first, so that it lands while the factors are formed
  const int rr = t >> 2, c0 = (t & 3) * 16;
  float* e = kb.S + (int64_t)(p * KEEP_T + rr) * kb.np + q * KEEP_T + c0;
  f32x4 sv[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) sv[v] = *(const f32x4*)(e + 4 * v);
  if (t < 2 * KEEP_T) {
    const int role = t >> 6, r = t & 63;  // role 0: row i of block p; 1: column j of block q
    const int idx = (role ? q : p) * KEEP_T + r;
    // every load unconditional, at a valid address (index clamped to N - 1,
    // tile k to T - 1; what those read is not used), so that they issue
    // back to back and share one memory round trip
    const int ic = min(idx, N - 1);
    const float* part = role ? kb.colpart : kb.rowpart;
    float pv[MKT];
#pragma unroll
    for (int k = 0; k < MKT; ++k) pv[k] = part[(int64_t)min(k, T - 1) * kb.np + ic];
    const float nv = ws[(role ? WS_RY : WS_RX) * n64 + ic];
    const float dgv = ws[WS_DIAG * n64 + ic], rxv = ws[WS_RX * n64 + ic], ryv = ws[WS_RY * n64 + ic];
    double term = 0.0, kap = 0.0;
    float inv = 0.f, nrm = 1.f;
    if (idx < N) {
      nrm = NORM ? nv : 1.f;
      if (!(LIT && role)) {
        float off = 0.f;
#pragma unroll
        for (int k = 0; k < MKT; ++k) off += k < T ? pv[k] : 0.f;
        const double s = (double)dgv * (double)rxv * (double)ryv;
        const double tt = (s - 1.0) * inv_t;
        const double R = (double)off + exp(tt);
        inv = (float)(1.0 / R);
        if (dg) {
          term = softplus_log_ratio(off, tt);
          kap = -((double)off / R);
          ws[(role ? WS_COL_OFF : WS_ROW_OFF) * n64 + idx] = off;
          ws[(role ? WS_INV_COL : WS_INV_ROW) * n64 + idx] = inv;
        }
      }
    }
    (role ? s_ic : s_ir)[r] = inv;
    (role ? s_ry : s_rx)[r] = nrm;
    s_term[t] = term;
    s_kap[t] = kap;
  }
  __syncthreads();
  // the diagonal blocks' loss partial first (its atomic's round trip then
  // overlaps the block's S -> H)
  unsigned long long lword = 0ull;
  bool last = false;
  if (dg && t < KEEP_T) {
    const int i = p * KEEP_T + t;
    const double kap = LIT ? s_kap[t] : s_kap[t] + s_kap[KEEP_T + t];
    const double v = LIT ? s_term[t] : s_term[t] + s_term[KEEP_T + t];
    if (i < N) ws[WS_KAPPA * n64 + i] = (float)kap;
    const double tot = wave_sum_f64(v);  // >= 0: every term is
    if (t == 0) {
      // a NaN partial, or one past the bound (an infinite term, |cos| > 1
      // with normalized_inputs=True), sets a flag bit instead of adding: an
      // OR to the same word, which the last block's addition then returns
      // (one location: this block's OR precedes its own addition, which
      // precedes the last block's)
      const double u = tot * lscale;
      unsigned long long add = 1ull;
      if (u != u)
        __hip_atomic_fetch_or(kb.lacc, KEEP_LOSS_NAN, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else if (!(u <= KEEP_LOSS_CAP))
        __hip_atomic_fetch_or(kb.lacc, KEEP_LOSS_OVF, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        add += (unsigned long long)llrint(u) << 6;
      const unsigned long long old = __hip_atomic_fetch_add(kb.lacc, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = (old & 63ull) == (unsigned long long)(T - 1);
      lword = old + add;
    }
  }
  // S -> H (the forward's E: the same expression on the same values)
  {
    const int i = p * KEEP_T + rr;
    const float ai = s_rx[rr], ir = s_ir[rr];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      f32x4 h;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int jl = c0 + 4 * v + u, j = q * KEEP_T + jl;
        const float ry = s_ry[jl], sc = sv[v][u];
        float ex = fast_exp2(fmaf(sc, NORM ? c * ry : c, -c));
        ex = (i < N && j < N && i != j) ? ex : 0.f;
        const float g = ex * (LIT ? ir : ir + s_ic[jl]);
        s_gc[rr][gcol(jl)] = g * (sc * ry);
        h[u] = g * (ai * ry);
      }
      *(f32x4*)(e + 4 * v) = h;
    }
  }
  __syncthreads();
  // the block's sums of G' cos: thread r < 64 row 64 p + r, thread 64 + r
  // column 64 q + r (CLIP); four interleaved partial sums, then combined, in
  // a fixed order
  if (t < (LIT ? 1 : 2) * KEEP_T) {
    const int role = t >> 6, r = t & 63;
    float v4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < KEEP_T; ++k) v4[k & 3] += role ? s_gc[k][gcol(r)] : s_gc[r][gcol(k)];
    const float v = (v4[0] + v4[1]) + (v4[2] + v4[3]);
    if (role)
      kb.coldot[(int64_t)p * kb.np + q * KEEP_T + r] = v;
    else
      kb.rowdot[(int64_t)q * kb.np + p * KEEP_T + r] = v;
  }
  if (last) {
    const double sum = (double)((lword & (KEEP_LOSS_OVF - 1)) >> 6);
    *loss = (lword & KEEP_LOSS_NAN) ? __builtin_nanf("")
            : (lword & KEEP_LOSS_OVF) ? __builtin_inff()
                                      : (float)(sum / lscale / (LIT ? (double)N : 2.0 * (double)N));
  }
}

// The post-pass operands of the fused backward (mec_backward): the
// workspace vectors, grad_output (device scalar, NULL = 1), the outputs
// (row-major, pitch D; NULL: the side is not computed) and a = grad_scale /
// (2N) (LiT: / N).
struct KeepPost {
  const float* ws;
  const float* grad_output;
  float* dx;
  float* dy;
  float a;
};

// Backward contractions from H (one 64 x 64 output tile per workgroup;
// x-side tiles first, each side's grid padded to a multiple of 8 and
// XCD-grouped): the x side reads H by rows, the y side reads it transposed,
// and both take the raw input rows of the other side as the feature operand
// (16-byte lanes):
//   acc_x[i, d] = sum_j H_ij y_j[d] = rx_i (G' Y^)[i, d]
//   acc_y[j, d] = sum_i H_ij x_i[d] = ry_j (G'^T X^)[j, d]
// i.e. the accumulators as mec_grad leaves them for fp32 (!FUSED: stored to
// acc_x / acc_y for k_postpass).  FUSED: k_postpass's arithmetic on the
// tile, row i of the own side (x: own = x, oth = y; y side the other way
// round), r = own's inverse norm:
//   h   = a (kappa_i r_oth,i r oth_i[d] + acc[i, d])          (= r dx^_i[d])
//   out = grad_output (h - own_i[d] r dot_i)   (NORM and r < 1e12; else h)
// with dot_i = <x^_i, h> = a r (kappa_i cos_ii + sum_j G'_ij cos_ij) from the
// finalize's per-block sums (rowdot, coldot; wave w adds blocks w, w + 4, ...
// in order, then the four in wave order), instead of a reduction over the
// features.  The tile's own and other-side values and the rows' vectors are
// loaded before the k-loop and land during it.  MKT >= kt, as in
// k_keep_finalize.
template <bool FUSED, bool NORM, int MKT = KEEP_MAX_KT>
__global__ __launch_bounds__(KEEP_NT, 2) void k_keep_contract(const float* __restrict__ X, int64_t ldx,
                                                              const float* __restrict__ Y, int64_t ldy, int N, int D,
                                                              KeepBufs kb, float* __restrict__ acc_x,
                                                              float* __restrict__ acc_y, KeepPost pp, int ctd,
                                                              int nx_pad, int ny_pad) {
  using TCX = KeepConX;
  using TCY = KeepConY;
  static_assert(TCX::BM == KEEP_T && TCX::BN == KEEP_T && TCY::BM == KEEP_T && TCY::BN == KEEP_T &&
                    TCX::FM == 1 && TCX::FN == 1 && TCY::FM == 1 && TCY::FN == 1 && TCX::NT == KEEP_NT &&
                    TCY::NT == KEEP_NT && TCX::G::KS == 2 && TCY::G::KS == 2,
                "64 x 64 tiles of 2 x 2 x 2 waves");
  __shared__ __attribute__((aligned(1024))) char lds[CMax<TCX::LDS_BYTES, TCY::LDS_BYTES>::value];
  __shared__ float s_kq[KEEP_T], s_ro[KEEP_T], s_dot[KEEP_T], s_part[4][KEEP_T];
  // waves 0-3 (k-group 0) hold the sums after the k-loop: w is their sub-tile
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const bool g0 = w < 4;
  int sub = blockIdx.x;
  const bool is_x = sub < nx_pad;
  if (!is_x) sub -= nx_pad;
  const int pid = xcd_remap(sub, is_x ? nx_pad : ny_pad);
  if (pid >= kb.kt * ctd) return;
  int tm, td;
  group_tile(pid, kb.kt, ctd, 8, tm, td);
  const int r0 = tm * KEEP_T, d0 = td * KEEP_T;
  const int ncols = min(D - d0, KEEP_T);
  const int wm = (w & 3) / 2, wn = w & 1;
  const int d = d0 + wn * 32 + (lane & 31);
  const int64_t n64 = N;
  // FUSED: this lane's own and other-side values (its accumulator entries),
  // and thread r < 64's row vectors and block sums, issued before the k-loop
  const float* own = is_x ? X : Y;
  const float* oth = is_x ? Y : X;
  const int64_t ldo = is_x ? ldx : ldy, ldt = is_x ? ldy : ldx;
  static_assert(MKT % 4 == 0 && MKT <= KEEP_MAX_KT, "block sums per row");
  constexpr int PW = MKT / 4;  // block sums per wave: blocks w, w + 4, ...
  float ov[16], tv[16];
  float pv[PW];
  float rv_own = 1.f, rv_oth = 1.f, kap = 0.f, dgv = 0.f, go = 1.f;
  if (FUSED && g0) {
    if (pp.grad_output) go = *pp.grad_output;
    // unconditional loads at valid addresses (row, feature and tile indices
    // clamped; what the clamped ones read is not used), issued back to back
    const int dc = min(d, D - 1);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = min(r0 + wm * 32 + acc_row(r, lane), N - 1);
      ov[r] = own[(int64_t)row * ldo + dc];
      tv[r] = oth[(int64_t)row * ldt + dc];
    }
    // row r0 + lane's block sums of G' cos, blocks w, w + 4, ... in wave w
    // (at most 63 loads in flight per wave, the ring's included)
    const int i = min(r0 + lane, N - 1);
    const float* part = is_x ? kb.rowdot : kb.coldot;
#pragma unroll
    for (int k = 0; k < PW; ++k) pv[k] = part[(int64_t)min(4 * k + w, kb.kt - 1) * kb.np + i];
    if (w == 0) {
      rv_own = pp.ws[(is_x ? WS_RX : WS_RY) * n64 + i];
      rv_oth = pp.ws[(is_x ? WS_RY : WS_RX) * n64 + i];
      kap = pp.ws[WS_KAPPA * n64 + i];
      dgv = pp.ws[WS_DIAG * n64 + i];
    }
  }
  f32x16 acc[1][1];
  if (is_x)
    TCX::template run<true, true>(tile_op<TCX>(kb.S + (int64_t)r0 * kb.np, kb.np, KEEP_T, kb.np),
                                  tile_op<TCX>(Y + d0, ldy, ncols, N), kb.np, lds, acc);
  else
    TCY::template run<true, true>(tile_op<TCY>(kb.S + r0, kb.np, KEEP_T, kb.np), tile_op<TCY>(X + d0, ldx, ncols, N),
                                  kb.np, lds, acc);
  if constexpr (!FUSED) {
    float* out = is_x ? acc_x : acc_y;
    if (g0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = r0 + wm * 32 + acc_row(r, lane);
        if (row < N && d < D) store_device(&out[(int64_t)row * D + d], acc[0][0][r]);
      }
    }
  } else {
    // the values loaded before the k-loop are used from here on: the empty
    // asm keeps the arithmetic on them (and so the wait for them) below the
    // k-loop, whose own waits have covered those loads by now
    if (g0) {
#pragma unroll
      for (int k = 0; k < PW; ++k) asm volatile("" : "+v"(pv[k]));
      asm volatile("" : "+v"(rv_own), "+v"(rv_oth), "+v"(kap), "+v"(dgv), "+v"(go));
    }
    const float a = pp.a;
    if (g0) {
      float sum = 0.f;
#pragma unroll
      for (int k = 0; k < PW; ++k) sum += 4 * k + w < kb.kt ? pv[k] : 0.f;
      s_part[w][lane] = sum;
    }
    __syncthreads();
    if (t < KEEP_T) {
      const float sum = (s_part[0][t] + s_part[1][t]) + (s_part[2][t] + s_part[3][t]);
      // cos_ii = x_i . y_i rx_i ry_i
      const float cii = dgv * rv_own * rv_oth;
      s_kq[t] = kap * rv_oth * rv_own;
      s_ro[t] = rv_own;
      s_dot[t] = a * rv_own * fmaf(kap, cii, sum);
    }
    __syncthreads();
    float* out = is_x ? pp.dx : pp.dy;
    // tiles inside [0, N) x [0, D) store without a predicate
    const bool full = r0 + KEEP_T <= N && d0 + KEEP_T <= D;
    if (!g0) return;
    // every value first, then the stores (a store through a generic pointer
    // may alias LDS, so stores between the reads made each read wait), at
    // device scope
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int rl = wm * 32 + acc_row(r, lane);
      const float ro = s_ro[rl], dot = s_dot[rl];
      const float h = a * fmaf(s_kq[rl], tv[r], acc[0][0][r]);
      const float hp = h - (ov[r] * ro) * dot;
      acc[0][0][r] = go * ((NORM && ro < 1e12f) ? hp : h);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = r0 + wm * 32 + acc_row(r, lane);
      if (full || (row < N && d < D)) store_device(&out[(int64_t)row * D + d], acc[0][0][r]);
    }
  }
}

}  // namespace mec
