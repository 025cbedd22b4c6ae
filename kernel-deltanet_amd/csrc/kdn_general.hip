// The chunked gated delta-rule scan at feature widths the D = 512 kernels do not cover (gfx950).
//
// Used for D = 1024 over pre-lifted features: the factored d_k = 128 path of the reference
// (kernels/factored_kernel_deltanet.py:42-183: two 64 -> 512 lifts concatenated and renormalised, then
// the same chunk algebra with 1024 features and d_v = 128).  The rule and readout are those of the
// D = 512 scan: y_t = S_{t-1} phi_q(t), S_t = lambda_t S_{t-1} (I - beta_t phi_k phi_k^T) + beta_t v_t phi_k^T.
//
// Three launches per call, with one fp32 record per (batch, head, 64-token chunk):
//   prep   (parallel)   Grams K K^T and Q K^T from the feature rows in place, A, T = (I + A)^-1 (column-
//                       oriented substitution), Tp = T diag(beta g), P, U~ = T (beta o V); K packed in MFMA
//                       fragment order (rows and transposed)
//   carry  (sequential) S^T at every chunk start; X_K = K S^T, W = U~ - Tp X_K,
//                       S^T <- g_C S^T + K^T (kappa o W); the final state
//   output (parallel)   Y = diag(a) Q S_c^T + P W
// Notation as the D = 512 scan: l_i = sum_{t <= i} log clamp(lambda_t, 1e-5, 1), g = e^l, g_C = g_63,
// a_i = g_{i-1}, kappa_j = g_C / g_j; A_ij = beta_i (g_i/g_j) k_i.k_j, P_ij = (g_{i-1}/g_j) q_i.k_j, j < i.
// Products over the D features use the precision policy P (bf16 operands for bf16 inputs), the 64 x 64
// chunk algebra fp32 MFMA.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <type_traits>
#include "kdn_frag.hpp"
#include "kdn_internal.hpp"
#include "kdn_io.hpp"
#include "kdn_tile.hpp"

namespace kdn {
namespace gen {

constexpr int C = 64;
constexpr int LD = 68;

template <int D, int DV>
struct Rec {
  static constexpr int NV = DV / 16;
  static constexpr size_t KXF = 0;            // K-row fragments [m 4][jb D/32][lane], sized for f32x8
  static constexpr size_t KTF = KXF + C * D;  // K^T-row fragments [ft D/16][jb 2][lane]
  static constexpr size_t S = KTF + C * D;    // S^T at the chunk start as output B fragments [jb D/32][n NV][lane]
  static constexpr size_t TP = S + D * DV;    // [64][64] T diag(beta g)
  static constexpr size_t P = TP + C * C;     // [64][64]
  static constexpr size_t U = P + C * C;      // U~ as tiles [m 4][n NV][lane] f32x4
  static constexpr size_t W = U + C * DV;     // [64][DV]
  static constexpr size_t VEC = W + C * DV;   // l[64], beta[64]
  static constexpr size_t floats = (VEC + 128 + 63) / 64 * 64;
};

// The backward's record (kdn_delta_scan_bwd at D = 1024): the forward's record followed by the
// fields of the gradient (offsets in floats).
template <int D, int DV>
struct BRec {
  static constexpr size_t T = Rec<D, DV>::floats;  // [64][64] (I + A)^-1
  static constexpr size_t G = T + C * C;            // [64][64] K K^T
  static constexpr size_t XK = G + C * C;           // [64][DV] K S^T
  static constexpr size_t SR = XK + C * DV;         // [DV][D] the chunk-start state (S, not S^T), fp32
  static constexpr size_t H1 = SR + D * DV;         // [DV][D] (Q^T (a o dY))^T
  static constexpr size_t RR = H1 + D * DV;         // [64][DV] P^T dY
  static constexpr size_t GR = RR + C * DV;         // [DV][D] (dL/dS^T)^T at the chunk end
  static constexpr size_t X = GR + D * DV;          // [64][DV] K Gamma
  static constexpr size_t DW = X + C * DV;          // [64][DV] dL/dW
  static constexpr size_t ZN = DW + C * DV;         // [64][DV] -Tp^T dW (= dL/dX_K)
  static constexpr size_t AY = ZN + C * DV;         // [64][DV] a o dY
  static constexpr size_t KW = AY + C * DV;         // [64][DV] kappa o W
  static constexpr size_t NN = KW + C * DV;         // [64][64] N
  static constexpr size_t MM = NN + C * C;          // [64][64] M + M^T
  static constexpr size_t floats = (MM + C * C + 63) / 64 * 64;
};

struct Params {
  int64_t B, T, H, nch;
  const void* q; int64_t qs0, qs1, qs2;
  const void* k; int64_t ks0, ks1, ks2;
  const void* v; int64_t vs0, vs1, vs2;
  const float* beta; int64_t bs0, bs1, bs2;
  const float* decay; int64_t ds0, ds1, ds2;
  const float* init; int64_t is0, is1, is2, is3;
  float* fin; int64_t fs0, fs1, fs2, fs3;
  void* y; int64_t ys0, ys1, ys2;
  float* ws;
};

// Record of (b, h, c): the forward's layout, or the backward's longer one.
template <int D, int DV, bool BWD = false>
__device__ __forceinline__ float* record(const Params& p, int64_t b, int64_t h, int64_t c) {
  constexpr int64_t F = BWD ? (int64_t)BRec<D, DV>::floats : (int64_t)Rec<D, DV>::floats;
  return p.ws + ((b * p.H + h) * p.nch + c) * F;
}

// Fragments read straight from the input feature rows of one chunk (row i = token t0 + i, stride rs
// elements; rows at or past `nrows` read as zero).  rows: element (r0 + l%16, k0 + kappa);
// cols: element (c0 + l%16, k0 + kappa) = row k0 + kappa, column c0 + l%16.
template <typename InT>
__device__ __forceinline__ f32x8 frag_rows_in(const InT* base, int64_t rs, int r0, int k0, int lane, int nrows) {
  const int row = r0 + (lane & 15);
  f32x8 r;
  if (row < nrows) {
    const InT* q = base + row * rs + k0 + 4 * (lane >> 4);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      r[s] = ldx(q + s);
      r[4 + s] = ldx(q + 16 + s);
    }
  } else {
#pragma unroll
    for (int s = 0; s < 8; ++s) r[s] = 0.f;
  }
  return r;
}
template <typename InT>
__device__ __forceinline__ f32x8 frag_cols_in(const InT* base, int64_t rs, int c0, int k0, int lane, int nrows) {
  f32x8 r;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const int row = k0 + kappa(lane, s);
    r[s] = row < nrows ? ldx(base + row * rs + c0 + (lane & 15)) : 0.f;
  }
  return r;
}

// ---------------------------------------------------------------------------------------------- prep
template <class PB, typename InT, int D, int DV, bool BWD = false>
__global__ void __launch_bounds__(256) gen_prep_kernel(Params p) {
  using R = Rec<D, DV>;
  constexpr int LDV = DV + 4;
  __shared__ __attribute__((aligned(16))) float bA[C * LD];
  __shared__ __attribute__((aligned(16))) float bT[C * LD];
  __shared__ __attribute__((aligned(16))) float bV[C * LDV];
  __shared__ float s_ell[C], s_beta[C];

  const int64_t c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t t0 = c * C;
  float* rec = record<D, DV, BWD>(p, b, h, c);
  const int r = tid >> 2, part = tid & 3;
  const bool rvalid = t0 + r < p.T;

  if (w == 0) {
    const int64_t t = t0 + lane;
    const bool valid = t < p.T;
    const float be = valid ? p.beta[b * p.bs0 + t * p.bs1 + h * p.bs2] : 0.f;
    const float la = (valid && p.decay) ? p.decay[b * p.ds0 + t * p.ds1 + h * p.ds2] : 1.f;
    float l = logf(fminf(fmaxf(la, 1e-5f), 1.f));
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float u = __shfl_up(l, o);
      if (lane >= o) l += u;
    }
    s_ell[lane] = l;
    s_beta[lane] = be;
    rec[R::VEC + lane] = l;
    rec[R::VEC + 64 + lane] = be;
  }
  // the chunk's feature rows, read in place (rows past T read as zero)
  const int nrows = (int)(p.T - t0 < C ? p.T - t0 : C);
  const InT* Kin = reinterpret_cast<const InT*>(p.k) + b * p.ks0 + t0 * p.ks1 + h * p.ks2;
  const InT* Qin = reinterpret_cast<const InT*>(p.q) + b * p.qs0 + t0 * p.qs1 + h * p.qs2;
  __syncthreads();
  // beta o V in LDS
  {
    const InT* vi = reinterpret_cast<const InT*>(p.v) + b * p.vs0 + (t0 + r) * p.vs1 + h * p.vs2 + part * (DV / 4);
    const float be = s_beta[r];
#pragma unroll
    for (int e = 0; e < DV / 4; ++e) bV[r * LDV + part * (DV / 4) + e] = rvalid ? be * ldx(vi + e) : 0.f;
  }
  // Grams (row tile w) -> A and P
  {
    f32x4 gkk[4], gqk[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) gkk[n] = gqk[n] = zero4();
    for (int jb = 0; jb < D / 32; ++jb) {
      const f32x8 kw = frag_rows_in(Kin, p.ks1, 16 * w, 32 * jb, lane, nrows);
      const f32x8 qw = frag_rows_in(Qin, p.qs1, 16 * w, 32 * jb, lane, nrows);
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const f32x8 kn = frag_rows_in(Kin, p.ks1, 16 * n, 32 * jb, lane, nrows);
        gkk[n] = mm<PB>(gkk[n], kw, kn);
        gqk[n] = mm<PB>(gqk[n], qw, kn);
      }
    }
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ri = 16 * w + 4 * (lane >> 4) + i, cj = 16 * n + (lane & 15);
        const float li = s_ell[ri], lj = s_ell[cj], lim1 = ri > 0 ? s_ell[ri - 1] : 0.f;
        // A transposed for the column-oriented inverse: [j][p][s] = A[4s+p][j]
        bA[(cj * 4 + (ri & 3)) * 16 + (ri >> 2)] = cj < ri ? s_beta[ri] * expf(fminf(li - lj, 0.f)) * gkk[n][i] : 0.f;
        rec[R::P + ri * C + cj] = cj < ri ? expf(fminf(lim1 - lj, 0.f)) * gqk[n][i] : 0.f;
        if constexpr (BWD) rec[BRec<D, DV>::G + ri * C + cj] = gkk[n][i];
      }
  }
  // K packed in fragment order: wave w the row fragments of feature blocks [w D/128, (w+1) D/128) and
  // the transposed fragments of feature tiles [w D/64, (w+1) D/64)
  {
    using frag = typename PB::frag;
    frag* kxf = reinterpret_cast<frag*>(rec + R::KXF);
    frag* ktf = reinterpret_cast<frag*>(rec + R::KTF);
    for (int jj = 0; jj < D / 128; ++jj) {
      const int jb = w * (D / 128) + jj;
#pragma unroll
      for (int m = 0; m < 4; ++m)
        kxf[(m * (D / 32) + jb) * 64 + lane] = PB::from_f32(frag_rows_in(Kin, p.ks1, 16 * m, 32 * jb, lane, nrows));
    }
    for (int tt = 0; tt < D / 64; ++tt) {
      const int ft = w * (D / 64) + tt;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
        ktf[(ft * 2 + jb) * 64 + lane] = PB::from_f32(frag_cols_in(Kin, p.ks1, 16 * ft, 32 * jb, lane, nrows));
    }
  }
  __syncthreads();
  // T = (I + A)^-1 (column-oriented substitution over lane quads)
  unit_lower_inverse(bA, bT, LD, w, lane);
  __syncthreads();
  for (int idx = tid; idx < C * C; idx += 256) {
    const int i = idx >> 6, j = idx & 63;
    rec[R::TP + idx] = bT[i * LD + j] * s_beta[j] * expf(s_ell[j]);
    if constexpr (BWD) rec[BRec<D, DV>::T + idx] = bT[i * LD + j];
  }
  // U~ = T (beta o V), row tile w
  {
    const f32x8 ta0 = frag_rows(bT, LD, 16 * w, 0, lane), ta1 = frag_rows(bT, LD, 16 * w, 32, lane);
#pragma unroll
    for (int n = 0; n < R::NV; ++n) {
      const f32x4 u = mm<PrecF32>(mm<PrecF32>(zero4(), ta0, frag_cols(bV, LDV, 16 * n, 0, lane)), ta1,
                                  frag_cols(bV, LDV, 16 * n, 32, lane));
      reinterpret_cast<f32x4*>(rec + R::U)[(w * R::NV + n) * 64 + lane] = u;
    }
  }
}

// --------------------------------------------------------------------------------------------- carry
// grid: 8 * ceil(B*H / 8) * NV workgroups of 256 threads; workgroup (head-batch hb, value tile n), the
// NV value tiles of a head on one XCD.  Wave w keeps features [w D/4, (w+1) D/4) of its D x 16 slice of
// S^T in registers.  The chunk-start slice is stored as the B fragments of the output's Q S^T product
// (the pairs of 16-feature tiles, kdn_frag.hpp) in the policy's fragment type.  With bf16 fragments the
// next chunk's K-row fragments are loaded one iteration ahead (two register sets).
struct CarryShared {
  f32x4 xp[4][4][64];
  f32x4 x[4][64];
  f32x4 z[4][64];
};

template <class PB, int D>
struct CarryK {
  typename PB::frag kx[4][D / 128];
};

template <class PB, int D, int DV>
__device__ __forceinline__ void carry_load_kx(CarryK<PB, D>& o, const float* rec, int w, int lane) {
  using R = Rec<D, DV>;
  constexpr int JPW = D / 128;
  const typename PB::frag* kxf = reinterpret_cast<const typename PB::frag*>(rec + R::KXF);
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int jj = 0; jj < JPW; ++jj) o.kx[m][jj] = kxf[(m * (D / 32) + w * JPW + jj) * 64 + lane];
}

template <class PB, int D, int DV, bool PIPE, bool BWD>
__device__ __forceinline__ bool carry_step(const Params& p, CarryShared& sh, int64_t b, int64_t h, int64_t c,
                                           CarryK<PB, D>& cur, CarryK<PB, D>& nxt, f32x4 (&Sg)[D / 64], int w,
                                           int lane, int n, unsigned& sink) {
  using R = Rec<D, DV>;
  using frag = typename PB::frag;
  constexpr int NV = R::NV, TPW = D / 64, JPW = D / 128;
  const bool more = c + 1 < p.nch;
  float* rec = record<D, DV, BWD>(p, b, h, c);
  const frag* kxf = reinterpret_cast<const frag*>(rec + R::KXF);
  const f32x8 tp0 = frag_rows(rec + R::TP, C, 16 * w, 0, lane), tp1 = frag_rows(rec + R::TP, C, 16 * w, 32, lane);
  const f32x4 ur = reinterpret_cast<const f32x4*>(rec + R::U)[(w * NV + n) * 64 + lane];
  const f32x4 lr = *reinterpret_cast<const f32x4*>(rec + R::VEC + 16 * w + 4 * (lane >> 4));
  const float l63 = rec[R::VEC + 63];
  unsigned pf = 0;  // L2-prefetch loads, folded into `sink` at the end of the step
  if (more) {
    const float* nrec = record<D, DV, BWD>(p, b, h, c + 1);
    if constexpr (PIPE) carry_load_kx<PB, D, DV>(nxt, nrec, w, lane);
    const unsigned* nr = reinterpret_cast<const unsigned*>(nrec);
    const int idx = n * 256 + (int)threadIdx.x;  // 0 .. 256 NV - 1
    constexpr int KLINES = D * (int)sizeof(frag) / 16;  // 128-byte lines of one packed K (D/8 fragments)
    for (int l = idx; l < KLINES; l += 256 * NV) {
      pf += nr[R::KTF + 32 * l];
      if constexpr (!PIPE) pf += nr[R::KXF + 32 * l];
    }
    if (idx < 128) pf += nr[R::TP + 32 * idx];                       // 128 lines of Tp
    else if (idx < 128 + 2 * DV) pf += nr[R::U + 32 * (idx - 128)];  // 2 DV lines of U~
  }

  // store the chunk-start slice (as output fragments) and form K times it, partial over this wave's features
  // (the backward's recompute keeps the slice in fp32 rows instead: no output kernel reads the fragments)
  if constexpr (BWD) {  // value-major rows: a lane's four features are one 16-byte store
    float* srow = rec + BRec<D, DV>::SR + (int64_t)(16 * n + (lane & 15)) * D + (D / 4) * w + 4 * (lane >> 4);
#pragma unroll
    for (int t = 0; t < TPW; ++t) *reinterpret_cast<f32x4*>(srow + 16 * t) = Sg[t];
  }
  frag* sf = reinterpret_cast<frag*>(rec + R::S);
  f32x4 xp[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) xp[m] = zero4();
#pragma unroll
  for (int jj = 0; jj < JPW; ++jj) {
    const frag sb = PB::from_f32(pair_to8(Sg[2 * jj], Sg[2 * jj + 1]));
    if constexpr (!BWD) sf[((w * JPW + jj) * NV + n) * 64 + lane] = sb;
#pragma unroll
    for (int m = 0; m < 4; ++m)
      xp[m] = PB::mma(xp[m], PIPE ? cur.kx[m][jj] : kxf[(m * (D / 32) + w * JPW + jj) * 64 + lane], sb);
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) sh.xp[w][m][lane] = xp[m];
  const float gC = expf(l63);
#pragma unroll
  for (int t = 0; t < TPW; ++t) Sg[t] = Sg[t] * gC;
  __syncthreads();
  // K^T fragments for the update, issued now (bf16: 128 registers) so that they arrive during the W / Z
  // phase; fp32 fragments are read where the update consumes them
  constexpr bool EARLY = std::is_same<PB, PrecBF16>::value;
  const frag* ktf = reinterpret_cast<const frag*>(rec + R::KTF);
  frag kt[EARLY ? TPW : 1][2];
  if constexpr (EARLY) {
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) kt[t][jb] = ktf[((w * TPW + t) * 2 + jb) * 64 + lane];
  }
  const f32x4 X = sh.xp[0][w][lane] + sh.xp[1][w][lane] + sh.xp[2][w][lane] + sh.xp[3][w][lane];
  sh.x[w][lane] = X;
  if constexpr (BWD) {
#pragma unroll
    for (int i = 0; i < 4; ++i) rec[BRec<D, DV>::XK + (16 * w + 4 * (lane >> 4) + i) * DV + 16 * n + (lane & 15)] = X[i];
  }
  __syncthreads();
  f32x4 tx = mm<PrecF32>(zero4(), tp0, pair_to8(sh.x[0][lane], sh.x[1][lane]));
  tx = mm<PrecF32>(tx, tp1, pair_to8(sh.x[2][lane], sh.x[3][lane]));
  const f32x4 Wt = ur - tx;
  const int vc = 16 * n + (lane & 15);
  f32x4 kap;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    rec[R::W + (16 * w + 4 * (lane >> 4) + i) * DV + vc] = Wt[i];
    kap[i] = expf(l63 - lr[i]);
  }
  sh.z[w][lane] = kap * Wt;
  __syncthreads();
  const frag zb0 = PB::from_f32(pair_to8(sh.z[0][lane], sh.z[1][lane]));
  const frag zb1 = PB::from_f32(pair_to8(sh.z[2][lane], sh.z[3][lane]));
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    if constexpr (EARLY) {
      Sg[t] = PB::mma(PB::mma(Sg[t], kt[t][0], zb0), kt[t][1], zb1);
    } else {
      Sg[t] = PB::mma(PB::mma(Sg[t], ktf[((w * TPW + t) * 2) * 64 + lane], zb0), ktf[((w * TPW + t) * 2 + 1) * 64 + lane],
                      zb1);
    }
  }
  sink += pf;
  return more;
}

template <class PB, int D, int DV, bool BWD = false>
__global__ void __launch_bounds__(256) gen_carry_kernel(Params p) {
  using R = Rec<D, DV>;
  constexpr int NV = R::NV, FPW = D / 4, TPW = FPW / 16;
  constexpr bool PIPE = false;  // two register sets of 32 K fragments do not fit beside the D = 1024 slice
  __shared__ CarryShared sh;
  const int64_t id = blockIdx.x;
  const int64_t xcd = id & 7, jdx = id >> 3;
  const int n = (int)(jdx % NV);
  const int64_t hb = (jdx / NV) * 8 + xcd;
  if (hb >= p.B * p.H) return;
  const int64_t b = hb / p.H, h = hb % p.H;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int vc = 16 * n + (lane & 15);

  f32x4 Sg[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int f = FPW * w + 16 * t + 4 * (lane >> 4) + i;
      Sg[t][i] = p.init ? p.init[b * p.is0 + h * p.is1 + f * p.is2 + vc * p.is3] : 0.f;
    }
  unsigned sink = 0;  // keeps the L2 prefetch loads alive (never stored: nch is positive)
  CarryK<PB, D> ka, kb;
  if constexpr (PIPE) carry_load_kx<PB, D, DV>(ka, record<D, DV, BWD>(p, b, h, 0), w, lane);
  for (int64_t c = 0;; c += 2) {
    if (!carry_step<PB, D, DV, PIPE, BWD>(p, sh, b, h, c, ka, kb, Sg, w, lane, n, sink)) break;
    if (!carry_step<PB, D, DV, PIPE, BWD>(p, sh, b, h, c + 1, kb, ka, Sg, w, lane, n, sink)) break;
  }
  if (p.nch < 0) p.ws[0] = (float)sink;
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int f = FPW * w + 16 * t + 4 * (lane >> 4) + i;
      p.fin[b * p.fs0 + h * p.fs1 + f * p.fs2 + vc * p.fs3] = Sg[t][i];
    }
}

// -------------------------------------------------------------------------------------------- output
// grid (nch, H, B), 256 threads; wave w the 16 tokens of tile w, every value tile.
template <typename T>
__device__ __forceinline__ void store_el(T* p, float v);
template <>
__device__ __forceinline__ void store_el<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_el<__bf16>(__bf16* p, float v) { *p = (__bf16)v; }

template <class PB, typename InT, typename OutT, int D, int DV>
__global__ void __launch_bounds__(256) gen_output_kernel(Params p) {
  using R = Rec<D, DV>;
  constexpr int NV = R::NV;
  const int64_t c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t0 = c * C;
  const float* rec = record<D, DV>(p, b, h, c);
  const int nrows = (int)(p.T - t0 < C ? p.T - t0 : C);
  const InT* Qin = reinterpret_cast<const InT*>(p.q) + b * p.qs0 + t0 * p.qs1 + h * p.qs2;
  f32x4 qs[NV];
#pragma unroll
  for (int n = 0; n < NV; ++n) qs[n] = zero4();
  const typename PB::frag* sf = reinterpret_cast<const typename PB::frag*>(rec + R::S);
  for (int jb = 0; jb < D / 32; ++jb) {
    const typename PB::frag qa = PB::from_f32(frag_rows_in(Qin, p.qs1, 16 * w, 32 * jb, lane, nrows));
#pragma unroll
    for (int n = 0; n < NV; ++n) qs[n] = PB::mma(qs[n], qa, sf[(jb * NV + n) * 64 + lane]);
  }
  const f32x8 p0 = frag_rows(rec + R::P, C, 16 * w, 0, lane), p1 = frag_rows(rec + R::P, C, 16 * w, 32, lane);
  f32x4 a;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ri = 16 * w + 4 * (lane >> 4) + i;
    a[i] = ri > 0 ? expf(rec[R::VEC + ri - 1]) : 1.f;
  }
  OutT* y = reinterpret_cast<OutT*>(p.y);
#pragma unroll
  for (int n = 0; n < NV; ++n) {
    const f32x4 pw = mm<PrecF32>(mm<PrecF32>(zero4(), p0, frag_cols(rec + R::W, DV, 16 * n, 0, lane)), p1,
                                 frag_cols(rec + R::W, DV, 16 * n, 32, lane));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t t = t0 + 16 * w + 4 * (lane >> 4) + i;
      if (t < p.T) store_el<OutT>(y + b * p.ys0 + t * p.ys1 + h * p.ys2 + 16 * n + (lane & 15), a[i] * qs[n][i] + pw[i]);
    }
  }
}

template <class PB, typename InT, typename OutT, int D, int DV>
static int launch(const Params& p, hipStream_t st) {
  const dim3 chunk_grid((unsigned)p.nch, (unsigned)p.H, (unsigned)p.B);
  const unsigned carry_wgs = (unsigned)(((p.B * p.H + 7) / 8) * 8 * (DV / 16));
  hipLaunchKernelGGL((gen_prep_kernel<PB, InT, D, DV>), chunk_grid, dim3(256), 0, st, p);
  hipLaunchKernelGGL((gen_carry_kernel<PB, D, DV>), dim3(carry_wgs), dim3(256), 0, st, p);
  hipLaunchKernelGGL((gen_output_kernel<PB, InT, OutT, D, DV>), chunk_grid, dim3(256), 0, st, p);
  return launch_status();
}

template <int D, int DV>
static int launch_dtypes(const Params& p, int in_dt, int out_dt, hipStream_t st) {
  if (in_dt == KDN_DTYPE_BF16) {
    if (out_dt == KDN_DTYPE_BF16) return launch<PrecBF16, __bf16, __bf16, D, DV>(p, st);
    return launch<PrecBF16, __bf16, float, D, DV>(p, st);
  }
  if (out_dt == KDN_DTYPE_BF16) return launch<PrecF32, float, __bf16, D, DV>(p, st);
  return launch<PrecF32, float, float, D, DV>(p, st);
}

static size_t record_floats(int D, int DV) {
  if (D == 1024 && DV == 64) return Rec<1024, 64>::floats;
  if (D == 1024 && DV == 128) return Rec<1024, 128>::floats;
  return 0;
}

// ============================================================================================ backward
// Backward of the general-D scan (D = 1024 over pre-lifted features, d_v 64 or 128, the delta rule): the
// gradients of a loss with respect to phi_q, phi_k, v, beta, lambda and the initial state, given dL/dy
// and dL/d(final state).  The closed form per chunk is that of the D = 512 backward (kdn_bwd.hip), with
// one record per (batch, head, chunk) for the whole sequence:
//   prep, carry (the forward's kernels)  T, K K^T, Tp, P, U~, W; S^T at every chunk start, X_K = K S^T
//   rh      (parallel)                   R = P^T dY, H = Q^T (a o dY)
//   rchain  (sequential, reversed)       Gamma = dL/dS^T at every chunk end, X = K Gamma,
//                                        dW = R + kappa o X, Z = Tp^T dW, Gamma <- g_C Gamma + H - K^T Z
//   grad    (parallel)                   dv, dbeta, dlambda; the left operands of the feature gradients
//   dphi    (parallel, 256 features per workgroup)
//                                        dphi_q = (a o dY) S + N K
//                                        dphi_k = (kappa o W) Gamma^T - Z S + (M + M^T) K + N^T Q
// with S the chunk-start state as the recurrence's d_v x D matrix (the carries hold S^T, D x d_v),
// N_ij = dP_ij g_{i-1}/g_j and M_ij = dA_ij beta_i g_i/g_j below the diagonal, dP = dY W^T and
// dA = -T^T dT T^T.
// The contractions that involve the features (the carries, H, Q S^T and the feature gradients) take the
// forward's precision policy (bf16 operands with fp32 accumulation for bf16 inputs, as the D = 512
// backward); the 64 x 64 chunk algebra runs on fp32 MFMA.  Every reduction has a fixed order (no
// atomics).

struct BwdP {
  const float* dy; int64_t ys0, ys1, ys2;
  const float* dfin; int64_t fs0, fs1, fs2, fs3;  // dL/dS^T at the end (NULL: zero)
  float* dq; int64_t dqs0, dqs1, dqs2;
  float* dk; int64_t dks0, dks1, dks2;
  float* dv; int64_t dvs0, dvs1, dvs2;
  float* dbeta; int64_t dbs0, dbs1, dbs2;
  float* ddecay; int64_t dds0, dds1, dds2;        // NULL: not wanted
  float* dinit; int64_t gis0, gis1, gis2, gis3;   // dL/dS^T at the start (NULL: not wanted)
};

// ------------------------------------------------------------------------------------------------ rh
// grid (nch, H, B), 256 threads.  Wave w: rows 16w .. of R, feature tiles [w D/64, (w+1) D/64) of H.
template <class PB, typename InT, int D, int DV>
__global__ void __launch_bounds__(256) gbwd_rh_kernel(Params p, BwdP g) {
  using F = Rec<D, DV>;
  using R = BRec<D, DV>;
  constexpr int LDV = DV + 4, NV = DV / 16;
  __shared__ __attribute__((aligned(16))) float bY[C * LDV];   // dY
  __shared__ __attribute__((aligned(16))) float bAY[C * LDV];  // a o dY
  const int64_t c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t t0 = c * C;
  float* rec = record<D, DV, true>(p, b, h, c);
  const int nrows = (int)(p.T - t0 < C ? p.T - t0 : C);
  for (int idx = tid; idx < C * DV; idx += 256) {
    const int r = idx / DV, v = idx % DV;
    const float y = r < nrows ? g.dy[b * g.ys0 + (t0 + r) * g.ys1 + h * g.ys2 + v] : 0.f;
    const float ay = (r > 0 ? expf(rec[F::VEC + r - 1]) : 1.f) * y;
    bY[r * LDV + v] = y;
    bAY[r * LDV + v] = ay;
    rec[R::AY + idx] = ay;
  }
  __syncthreads();
  const f32x8 pa0 = frag_cols(rec + F::P, C, 16 * w, 0, lane), pa1 = frag_cols(rec + F::P, C, 16 * w, 32, lane);
#pragma unroll
  for (int n = 0; n < NV; ++n) {
    const f32x4 rr = mm<PrecF32>(mm<PrecF32>(zero4(), pa0, frag_cols(bY, LDV, 16 * n, 0, lane)), pa1,
                                 frag_cols(bY, LDV, 16 * n, 32, lane));
#pragma unroll
    for (int i = 0; i < 4; ++i) rec[R::RR + (16 * w + 4 * (lane >> 4) + i) * DV + 16 * n + (lane & 15)] = rr[i];
  }
  const InT* Qin = reinterpret_cast<const InT*>(p.q) + b * p.qs0 + t0 * p.qs1 + h * p.qs2;
  for (int tt = 0; tt < D / 64; ++tt) {
    const int ft = w * (D / 64) + tt;
    const typename PB::frag q0 = PB::from_f32(frag_cols_in(Qin, p.qs1, 16 * ft, 0, lane, nrows));
    const typename PB::frag q1 = PB::from_f32(frag_cols_in(Qin, p.qs1, 16 * ft, 32, lane, nrows));
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      const f32x4 hv = PB::mma(PB::mma(zero4(), q0, PB::from_f32(frag_cols(bAY, LDV, 16 * n, 0, lane))), q1,
                               PB::from_f32(frag_cols(bAY, LDV, 16 * n, 32, lane)));
      *reinterpret_cast<f32x4*>(rec + R::H1 + (int64_t)(16 * n + (lane & 15)) * D + 16 * ft + 4 * (lane >> 4)) = hv;
    }
  }
}

// -------------------------------------------------------------------------------------------- rchain
// grid as gen_carry_kernel: workgroup (head-batch hb, value tile n); wave w keeps features
// [w D/4, (w+1) D/4) of its D x 16 slice of Gamma = dL/dS^T in registers, chunks last to first.
template <class PB, int D, int DV>
__global__ void __launch_bounds__(256) gbwd_rchain_kernel(Params p, BwdP g) {
  using F = Rec<D, DV>;
  using R = BRec<D, DV>;
  using frag = typename PB::frag;
  constexpr int NV = DV / 16, FPW = D / 4, TPW = FPW / 16, JPW = D / 128;
  __shared__ CarryShared sh;
  const int64_t id = blockIdx.x;
  const int64_t xcd = id & 7, jdx = id >> 3;
  const int n = (int)(jdx % NV);
  const int64_t hb = (jdx / NV) * 8 + xcd;
  if (hb >= p.B * p.H) return;
  const int64_t b = hb / p.H, h = hb % p.H;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int vc = 16 * n + (lane & 15);

  f32x4 Gg[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int f = FPW * w + 16 * t + 4 * (lane >> 4) + i;
      Gg[t][i] = g.dfin ? g.dfin[b * g.fs0 + h * g.fs1 + f * g.fs2 + vc * g.fs3] : 0.f;
    }
  unsigned sink = 0;  // keeps the L2-prefetch loads alive (never stored: nch is positive)
  for (int64_t c = p.nch - 1; c >= 0; --c) {
    float* rec = record<D, DV, true>(p, b, h, c);
    const frag* kxf = reinterpret_cast<const frag*>(rec + F::KXF);
    const frag* ktf = reinterpret_cast<const frag*>(rec + F::KTF);
    const float l63 = rec[F::VEC + 63];
    if (c > 0) {
      // touch the previous chunk's operands so that its loads hit L2: the packed K (lines shared by the
      // head's NV workgroups), Tp, P^T dY and this workgroup's 16 rows of H (one dword per 128-byte line)
      const unsigned* pr = reinterpret_cast<const unsigned*>(record<D, DV, true>(p, b, h, c - 1));
      const int idx = n * 256 + (int)threadIdx.x;
      constexpr int KLINES = D * (int)sizeof(frag) / 16;
      for (int l = idx; l < KLINES; l += 256 * NV) sink += pr[F::KXF + 32 * l] + pr[F::KTF + 32 * l];
      if (idx < 128) sink += pr[F::TP + 32 * idx];
      else if (idx < 128 + 2 * DV) sink += pr[R::RR + 32 * (idx - 128)];
      for (int l = (int)threadIdx.x; l < 16 * D / 32; l += 256)
        sink += pr[R::H1 + (int64_t)(16 * n + l / (D / 32)) * D + 32 * (l % (D / 32))];
    }
    const f32x4 lr = *reinterpret_cast<const f32x4*>(rec + F::VEC + 16 * w + 4 * (lane >> 4));
    // the step's small operands and this wave's rows of H, issued first so that their latency overlaps
    // the K Gamma products instead of following the last barrier
    float* grow = rec + R::GR + (int64_t)vc * D + FPW * w + 4 * (lane >> 4);
    const float* hrow = rec + R::H1 + (int64_t)vc * D + FPW * w + 4 * (lane >> 4);
    f32x4 hv[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) hv[t] = *reinterpret_cast<const f32x4*>(hrow + 16 * t);
    const f32x8 ta0 = frag_cols(rec + F::TP, C, 16 * w, 0, lane), ta1 = frag_cols(rec + F::TP, C, 16 * w, 32, lane);
    f32x4 rr;
#pragma unroll
    for (int i = 0; i < 4; ++i) rr[i] = rec[R::RR + (16 * w + 4 * (lane >> 4) + i) * DV + vc];
    // Gamma at the chunk end; K Gamma, partial over this wave's features
    f32x4 xp[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) xp[m] = zero4();
#pragma unroll
    for (int jj = 0; jj < JPW; ++jj) {
#pragma unroll
      for (int u = 0; u < 2; ++u) *reinterpret_cast<f32x4*>(grow + 16 * (2 * jj + u)) = Gg[2 * jj + u];
      const frag gb = PB::from_f32(pair_to8(Gg[2 * jj], Gg[2 * jj + 1]));
#pragma unroll
      for (int m = 0; m < 4; ++m) xp[m] = PB::mma(xp[m], kxf[(m * (D / 32) + w * JPW + jj) * 64 + lane], gb);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) sh.xp[w][m][lane] = xp[m];
    __syncthreads();
    // token tile w: X, dW = R + kappa o X
    const f32x4 X = sh.xp[0][w][lane] + sh.xp[1][w][lane] + sh.xp[2][w][lane] + sh.xp[3][w][lane];
    f32x4 dw;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ri = 16 * w + 4 * (lane >> 4) + i;
      dw[i] = rr[i] + expf(l63 - lr[i]) * X[i];
      rec[R::X + ri * DV + vc] = X[i];
      rec[R::DW + ri * DV + vc] = dw[i];
    }
    sh.z[w][lane] = dw;
    __syncthreads();
    // token tile w of Z = Tp^T dW (stored negated: dL/dX_K)
    const f32x4 Z = mm<PrecF32>(mm<PrecF32>(zero4(), ta0, pair_to8(sh.z[0][lane], sh.z[1][lane])), ta1,
                                pair_to8(sh.z[2][lane], sh.z[3][lane]));
    const f32x4 zn = -Z;
#pragma unroll
    for (int i = 0; i < 4; ++i) rec[R::ZN + (16 * w + 4 * (lane >> 4) + i) * DV + vc] = zn[i];
    sh.x[w][lane] = zn;
    __syncthreads();
    // Gamma <- g_C Gamma + H - K^T Z over this wave's features
    const frag zb0 = PB::from_f32(pair_to8(sh.x[0][lane], sh.x[1][lane]));
    const frag zb1 = PB::from_f32(pair_to8(sh.x[2][lane], sh.x[3][lane]));
    const float gC = expf(l63);
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const f32x4 acc = gC * Gg[t] + hv[t];
      Gg[t] = PB::mma(PB::mma(acc, ktf[((w * TPW + t) * 2) * 64 + lane], zb0), ktf[((w * TPW + t) * 2 + 1) * 64 + lane],
                      zb1);
    }
  }
  if (p.nch < 0) p.ws[0] = (float)sink;
  if (g.dinit) {
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int f = FPW * w + 16 * t + 4 * (lane >> 4) + i;
        g.dinit[b * g.gis0 + h * g.gis1 + f * g.gis2 + vc * g.gis3] = Gg[t][i];
      }
  }
}

// ---------------------------------------------------------------------------------------------- grad
// grid (nch, H, B), 256 threads; wave w owns row tile w of the 64 x 64 chunk algebra.  Rows of the
// fixed-order partial-sum tables: dl_i from the kappa term, the column sums of P o dP per row tile (4),
// the row sums of P o dP (at i - 1), beta g (T o dTp) column sums, the a o dY . Q S^T term (at i - 1),
// the column sums of beta o A o dA per row tile (4), its row sums; dbeta_i from the V . T^T dW row sums,
// the Tp column sums and the A o dA row sums.
constexpr int GDL_K = 0, GDL_COLP = 1, GDL_RP = 5, GDL_TS = 6, GDL_DA = 7, GDL_DLC = 8, GDL_A = 12, GNDL = 13;
constexpr int GDB_V = 0, GDB_TS = 1, GDB_A = 2, GNDB = 3;

// Sum over the 64 lanes of a wave in a fixed order (the result in every lane).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <class PB, typename InT, int D, int DV>
__global__ void __launch_bounds__(256) gbwd_grad_kernel(Params p, BwdP g) {
  using F = Rec<D, DV>;
  using R = BRec<D, DV>;
  constexpr int NV = DV / 16;
  __shared__ __attribute__((aligned(16))) float bT[C * LD];   // T
  __shared__ __attribute__((aligned(16))) float bD[C * LD];   // dT
  __shared__ __attribute__((aligned(16))) float bY1[C * LD];  // dT T^T
  __shared__ float s_ell[C], s_beta[C];
  __shared__ float s_dl[GNDL][C], s_db[GNDB][C], s_ts[4][C], s_kt[C], s_63[5];

  const int64_t c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rt = w;
  const int64_t t0 = c * C;
  float* rec = record<D, DV, true>(p, b, h, c);
  const int nrows = (int)(p.T - t0 < C ? p.T - t0 : C);
  const InT* Vin = reinterpret_cast<const InT*>(p.v) + b * p.vs0 + t0 * p.vs1 + h * p.vs2;
  const InT* Qin = reinterpret_cast<const InT*>(p.q) + b * p.qs0 + t0 * p.qs1 + h * p.qs2;
  const float* Yin = g.dy + b * g.ys0 + t0 * g.ys1 + h * g.ys2;

  if (tid < C) {
    s_ell[tid] = rec[F::VEC + tid];
    s_beta[tid] = rec[F::VEC + 64 + tid];
  }
  for (int idx = tid; idx < GNDL * C; idx += 256) (&s_dl[0][0])[idx] = 0.f;
  for (int idx = tid; idx < GNDB * C; idx += 256) (&s_db[0][0])[idx] = 0.f;
  for (int idx = tid; idx < C * C; idx += 256) bT[(idx >> 6) * LD + (idx & 63)] = rec[R::T + idx];
  __syncthreads();
  const float l63 = s_ell[63], gC = expf(l63);

  // ---- phase 1: dTp = -dW X_K^T, dW V^T, dP = dY W^T -> dT, N, the Tp and P o dP sums; T^T dW -> dv, dbeta;
  //      the kappa term and kappa o W
  {
    f32x4 dtp[4], e1[4], dp[4];
#pragma unroll
    for (int n4 = 0; n4 < 4; ++n4) dtp[n4] = e1[n4] = dp[n4] = zero4();
#pragma unroll
    for (int kb = 0; kb < DV / 32; ++kb) {
      const f32x8 da = frag_rows(rec + R::DW, DV, 16 * rt, 32 * kb, lane);
      const f32x8 ya = frag_rows_in(Yin, g.ys1, 16 * rt, 32 * kb, lane, nrows);
#pragma unroll
      for (int n4 = 0; n4 < 4; ++n4) {
        dtp[n4] = mm<PrecF32>(dtp[n4], da, frag_rows(rec + R::XK, DV, 16 * n4, 32 * kb, lane));
        e1[n4] = mm<PrecF32>(e1[n4], da, frag_rows_in(Vin, p.vs1, 16 * n4, 32 * kb, lane, nrows));
        dp[n4] = mm<PrecF32>(dp[n4], ya, frag_rows(rec + F::W, DV, 16 * n4, 32 * kb, lane));
      }
    }
    float rowp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n4 = 0; n4 < 4; ++n4) {
      const int cj = 16 * n4 + (lane & 15);
      const float bj = s_beta[cj], gj = expf(s_ell[cj]);
      float ts = 0.f, colp = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ri = 16 * rt + 4 * (lane >> 4) + i;
        const float dtpv = -dtp[n4][i];
        ts += bT[ri * LD + cj] * dtpv;
        bD[ri * LD + cj] = bj * (e1[n4][i] + gj * dtpv);
        float nv = 0.f;
        if (cj < ri) {
          const float pb = dp[n4][i] * rec[F::P + ri * C + cj];
          rowp[i] += pb;
          colp += pb;
          nv = dp[n4][i] * expf(fminf(s_ell[ri - 1] - s_ell[cj], 0.f));
        }
        rec[R::NN + ri * C + cj] = nv;
      }
      ts = sum_col4(ts);
      colp = sum_col4(colp);
      if (lane < 16) {
        s_ts[rt][cj] = ts;
        s_dl[GDL_COLP + rt][cj] = -colp;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ri = 16 * rt + 4 * (lane >> 4) + i;
      const float rp = sum_row16(rowp[i]);
      if ((lane & 15) == 0 && ri > 0) s_dl[GDL_RP][ri - 1] = rp;
    }
    // T^T dW, rows 16 rt ..: dv and the V . (T^T dW) row sums
    const f32x8 ta0 = frag_cols(bT, LD, 16 * rt, 0, lane), ta1 = frag_cols(bT, LD, 16 * rt, 32, lane);
    float dbv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int nv = 0; nv < NV; ++nv) {
      const f32x4 td = mm<PrecF32>(mm<PrecF32>(zero4(), ta0, frag_cols(rec + R::DW, DV, 16 * nv, 0, lane)), ta1,
                                   frag_cols(rec + R::DW, DV, 16 * nv, 32, lane));
      const int vcol = 16 * nv + (lane & 15);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ri = 16 * rt + 4 * (lane >> 4) + i;
        if (ri < nrows) {
          g.dv[b * g.dvs0 + (t0 + ri) * g.dvs1 + h * g.dvs2 + vcol] = s_beta[ri] * td[i];
          dbv[i] += ldx(Vin + ri * p.vs1 + vcol) * td[i];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ri = 16 * rt + 4 * (lane >> 4) + i;
      const float s = sum_row16(dbv[i]);
      if ((lane & 15) == 0) s_db[GDB_V][ri] = s;
    }
  }
  {
    // the kappa term: dkappa_i = W_i . X_i (row tid / 4, a quarter of the columns per thread, the quad's
    // four partials added in a fixed order); and kappa o W for the feature gradients
    const int r = tid >> 2, q0 = (tid & 3) * (DV / 4);
    const float kap = expf(l63 - s_ell[r]);
    float dk = 0.f;
#pragma unroll 4
    for (int v = q0; v < q0 + DV / 4; v += 4) {
      const f32x4 wv = *reinterpret_cast<const f32x4*>(rec + F::W + r * DV + v);
      const f32x4 xv = *reinterpret_cast<const f32x4*>(rec + R::X + r * DV + v);
      dk += wv[0] * xv[0] + wv[1] * xv[1] + wv[2] * xv[2] + wv[3] * xv[3];
      *reinterpret_cast<f32x4*>(rec + R::KW + r * DV + v) = kap * wv;
    }
    dk += __shfl_xor(dk, 1);
    dk += __shfl_xor(dk, 2);
    if ((tid & 3) == 0) {
      s_dl[GDL_K][r] = -dk * kap;
      s_kt[r] = dk * kap;
    }
  }
  __syncthreads();
  if (w == 0) {
    const float tot = wave_sum(s_kt[lane]);
    if (lane == 0) s_63[0] = tot;
  }

  // ---- phase 2: the Tp sums; Q S^T -> da; <Gamma, S>
  if (tid < C) {
    const float gj = expf(s_ell[tid]), ts = ((s_ts[0][tid] + s_ts[1][tid]) + s_ts[2][tid]) + s_ts[3][tid];
    s_db[GDB_TS][tid] = gj * ts;
    s_dl[GDL_TS][tid] = s_beta[tid] * gj * ts;
  }
  {
    float dap[4] = {0.f, 0.f, 0.f, 0.f};
    f32x4 qs[NV];
#pragma unroll
    for (int nv = 0; nv < NV; ++nv) qs[nv] = zero4();
    for (int jb = 0; jb < D / 32; ++jb) {
      const typename PB::frag qa = PB::from_f32(frag_rows_in(Qin, p.qs1, 16 * rt, 32 * jb, lane, nrows));
#pragma unroll
      for (int nv = 0; nv < NV; ++nv)
        qs[nv] = PB::mma(qs[nv], qa, PB::from_f32(frag_rows(rec + R::SR, D, 16 * nv, 32 * jb, lane)));
    }
#pragma unroll
    for (int nv = 0; nv < NV; ++nv) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ri = 16 * rt + 4 * (lane >> 4) + i;
        if (ri < nrows) dap[i] += Yin[ri * g.ys1 + 16 * nv + (lane & 15)] * qs[nv][i];
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ri = 16 * rt + 4 * (lane >> 4) + i;
      const float da = sum_row16(dap[i]);
      if ((lane & 15) == 0 && ri > 0) s_dl[GDL_DA][ri - 1] = da * expf(s_ell[ri - 1]);
    }
  }
  {
    float gs = 0.f;
    const f32x4* G4 = reinterpret_cast<const f32x4*>(rec + R::GR);
    const f32x4* S4 = reinterpret_cast<const f32x4*>(rec + R::SR);
    for (int e = tid; e < D * DV / 4; e += 256) {
      const f32x4 gg = G4[e], ss = S4[e];
      gs += gg[0] * ss[0] + gg[1] * ss[1] + gg[2] * ss[2] + gg[3] * ss[3];
    }
    gs = wave_sum(gs);
    if (lane == 0) s_63[1 + w] = gs;
  }
  __syncthreads();

  // ---- phase 3: Y1 = dT T^T
  {
    const f32x8 a0 = frag_rows(bD, LD, 16 * rt, 0, lane), a1 = frag_rows(bD, LD, 16 * rt, 32, lane);
#pragma unroll
    for (int n4 = 0; n4 < 4; ++n4) {
      const f32x4 y1 = mm<PrecF32>(mm<PrecF32>(zero4(), a0, frag_rows(bT, LD, 16 * n4, 0, lane)), a1,
                                   frag_rows(bT, LD, 16 * n4, 32, lane));
#pragma unroll
      for (int i = 0; i < 4; ++i) bY1[(16 * rt + 4 * (lane >> 4) + i) * LD + 16 * n4 + (lane & 15)] = y1[i];
    }
  }
  __syncthreads();

  // ---- phase 4: dA = -T^T Y1 (strictly lower); M + M^T; dbeta and dl from A
  {
    const f32x8 ta0 = frag_cols(bT, LD, 16 * rt, 0, lane), ta1 = frag_cols(bT, LD, 16 * rt, 32, lane);
    float dbr[4] = {0.f, 0.f, 0.f, 0.f}, dlr[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n4 = 0; n4 < 4; ++n4) {
      const f32x4 dA = -mm<PrecF32>(mm<PrecF32>(zero4(), ta0, frag_cols(bY1, LD, 16 * n4, 0, lane)), ta1,
                                    frag_cols(bY1, LD, 16 * n4, 32, lane));
      const int cj = 16 * n4 + (lane & 15);
      float dlc = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ri = 16 * rt + 4 * (lane >> 4) + i;
        if (cj < ri) {
          const float ex = expf(fminf(s_ell[ri] - s_ell[cj], 0.f));
          const float e = dA[i] * ex * rec[R::G + ri * C + cj];
          const float ab = s_beta[ri] * e;
          dbr[i] += e;
          dlr[i] += ab;
          dlc += ab;
          const float mv = dA[i] * s_beta[ri] * ex;
          rec[R::MM + ri * C + cj] = mv;
          rec[R::MM + cj * C + ri] = mv;
        } else if (cj == ri) {
          rec[R::MM + ri * C + cj] = 0.f;
        }
      }
      dlc = sum_col4(dlc);
      if (lane < 16) s_dl[GDL_DLC + rt][cj] = -dlc;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ri = 16 * rt + 4 * (lane >> 4) + i;
      const float a = sum_row16(dbr[i]), d = sum_row16(dlr[i]);
      if ((lane & 15) == 0) {
        s_db[GDB_A][ri] = a;
        s_dl[GDL_A][ri] = d;
      }
    }
  }
  __syncthreads();

  // ---- phase 5: dbeta and dlambda (dlog lambda_t = sum_{i >= t} dl_i)
  if (w == 0) {
    float dl = 0.f;
#pragma unroll
    for (int k = 0; k < GNDL; ++k) dl += s_dl[k][lane];
    if (lane == 63) dl += s_63[0] + gC * (((s_63[1] + s_63[2]) + s_63[3]) + s_63[4]);
    float dbeta = 0.f;
#pragma unroll
    for (int k = 0; k < GNDB; ++k) dbeta += s_db[k][lane];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float u = __shfl_down(dl, o);
      if (lane + o < 64) dl += u;
    }
    const int64_t t = t0 + lane;
    if (lane < nrows) {
      g.dbeta[b * g.dbs0 + t * g.dbs1 + h * g.dbs2] = dbeta;
      if (g.ddecay) {
        const float la = p.decay ? p.decay[b * p.ds0 + t * p.ds1 + h * p.ds2] : 1.f;
        g.ddecay[b * g.dds0 + t * g.dds1 + h * g.dds2] = (la >= 1e-5f && la <= 1.f) ? dl / la : 0.f;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------- dphi
// grid (nch * D / 256, H, B), 256 threads; workgroup (chunk, block of 256 features), wave w features
// [64 w, 64 w + 64) of the block for all 64 tokens (each wave loads only its own features' operands).
template <class PB, typename InT, int D, int DV>
__global__ void __launch_bounds__(256) gbwd_dphi_kernel(Params p, BwdP g) {
  using R = BRec<D, DV>;
  constexpr int FB = 256;
  const int64_t c = blockIdx.x / (D / FB), h = blockIdx.y, b = blockIdx.z;
  const int fb = (int)(blockIdx.x % (D / FB));
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t0 = c * C;
  const float* rec = record<D, DV, true>(p, b, h, c);
  const int nrows = (int)(p.T - t0 < C ? p.T - t0 : C);
  const InT* Qin = reinterpret_cast<const InT*>(p.q) + b * p.qs0 + t0 * p.qs1 + h * p.qs2;
  const InT* Kin = reinterpret_cast<const InT*>(p.k) + b * p.ks0 + t0 * p.ks1 + h * p.ks2;
  const int f0 = fb * FB + 64 * w;
  f32x4 aq[4][4], ak[4][4];  // [token tile][feature tile]
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int ft = 0; ft < 4; ++ft) aq[m][ft] = ak[m][ft] = zero4();
  // contractions over the value columns: (a o dY) S, (kappa o W) Gamma^T, -Z S
  for (int kb = 0; kb < DV / 32; ++kb) {
    f32x8 sb[4], gb[4];
#pragma unroll
    for (int ft = 0; ft < 4; ++ft) {
      sb[ft] = frag_cols(rec + R::SR, D, f0 + 16 * ft, 32 * kb, lane);
      gb[ft] = frag_cols(rec + R::GR, D, f0 + 16 * ft, 32 * kb, lane);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const f32x8 ay = frag_rows(rec + R::AY, DV, 16 * m, 32 * kb, lane);
      const f32x8 kw = frag_rows(rec + R::KW, DV, 16 * m, 32 * kb, lane);
      const f32x8 zn = frag_rows(rec + R::ZN, DV, 16 * m, 32 * kb, lane);
#pragma unroll
      for (int ft = 0; ft < 4; ++ft) {
        aq[m][ft] = mm<PB>(aq[m][ft], ay, sb[ft]);
        ak[m][ft] = mm<PB>(mm<PB>(ak[m][ft], kw, gb[ft]), zn, sb[ft]);
      }
    }
  }
  // contractions over the chunk's tokens: N K, (M + M^T) K, N^T Q
  for (int kb = 0; kb < 2; ++kb) {
    f32x8 kf[4], qf[4];
#pragma unroll
    for (int ft = 0; ft < 4; ++ft) {
      kf[ft] = frag_cols_in(Kin, p.ks1, f0 + 16 * ft, 32 * kb, lane, nrows);
      qf[ft] = frag_cols_in(Qin, p.qs1, f0 + 16 * ft, 32 * kb, lane, nrows);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const f32x8 nr = frag_rows(rec + R::NN, C, 16 * m, 32 * kb, lane);
      const f32x8 mr = frag_rows(rec + R::MM, C, 16 * m, 32 * kb, lane);
      const f32x8 nt = frag_cols(rec + R::NN, C, 16 * m, 32 * kb, lane);
#pragma unroll
      for (int ft = 0; ft < 4; ++ft) {
        aq[m][ft] = mm<PB>(aq[m][ft], nr, kf[ft]);
        ak[m][ft] = mm<PB>(mm<PB>(ak[m][ft], mr, kf[ft]), nt, qf[ft]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int ft = 0; ft < 4; ++ft)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ri = 16 * m + 4 * (lane >> 4) + i;
        if (ri < nrows) {
          const int64_t t = t0 + ri;
          const int f = f0 + 16 * ft + (lane & 15);
          g.dq[b * g.dqs0 + t * g.dqs1 + h * g.dqs2 + f] = aq[m][ft][i];
          g.dk[b * g.dks0 + t * g.dks1 + h * g.dks2 + f] = ak[m][ft][i];
        }
      }
}

template <class PB, typename InT, int D, int DV>
static int launch_bwd(const Params& p, const BwdP& g, hipStream_t st) {
  const dim3 chunk_grid((unsigned)p.nch, (unsigned)p.H, (unsigned)p.B);
  const unsigned carry_wgs = (unsigned)(((p.B * p.H + 7) / 8) * 8 * (DV / 16));
  hipLaunchKernelGGL((gen_prep_kernel<PB, InT, D, DV, true>), chunk_grid, dim3(256), 0, st, p);
  hipLaunchKernelGGL((gen_carry_kernel<PB, D, DV, true>), dim3(carry_wgs), dim3(256), 0, st, p);
  hipLaunchKernelGGL((gbwd_rh_kernel<PB, InT, D, DV>), chunk_grid, dim3(256), 0, st, p, g);
  hipLaunchKernelGGL((gbwd_rchain_kernel<PB, D, DV>), dim3(carry_wgs), dim3(256), 0, st, p, g);
  hipLaunchKernelGGL((gbwd_grad_kernel<PB, InT, D, DV>), chunk_grid, dim3(256), 0, st, p, g);
  hipLaunchKernelGGL((gbwd_dphi_kernel<PB, InT, D, DV>), dim3((unsigned)(p.nch * (D / 256)), (unsigned)p.H, (unsigned)p.B),
                     dim3(256), 0, st, p, g);
  return launch_status();
}

// The checkpoint pass of a segmented backward: the recompute and the forward carry of one segment, which
// writes the state at the segment's end to p.fin.
template <class PB, typename InT, int D, int DV>
static int launch_ckpt(const Params& p, hipStream_t st) {
  const dim3 chunk_grid((unsigned)p.nch, (unsigned)p.H, (unsigned)p.B);
  const unsigned carry_wgs = (unsigned)(((p.B * p.H + 7) / 8) * 8 * (DV / 16));
  hipLaunchKernelGGL((gen_prep_kernel<PB, InT, D, DV, true>), chunk_grid, dim3(256), 0, st, p);
  hipLaunchKernelGGL((gen_carry_kernel<PB, D, DV, true>), dim3(carry_wgs), dim3(256), 0, st, p);
  return launch_status();
}

static size_t bwd_record_floats(int D, int DV) {
  if (D == 1024 && DV == 64) return BRec<1024, 64>::floats;
  if (D == 1024 && DV == 128) return BRec<1024, 128>::floats;
  return 0;
}

// Segments of the backward: fwd->segment_chunks when positive, else the largest power of two from 4 to 256
// chunks whose records fit 24 GiB (one 256-chunk segment at B*H = 32, d_v = 128: 26.7 ms per backward
// against 29.7 in two segments of 128, which 12 GiB gave); at most the sequence's chunks.  Workspace: one segment's records, one
// fp32 [B][H][1024][d_v] state per segment boundary (the checkpoints), the carried dL/dS (with more than
// one segment) and the forward carry's final state (scratch).
constexpr size_t BWD_SEGMENT_BUDGET = (size_t)24 << 30;
struct BwdPlan {
  int64_t nch, seg, nsegs;
  size_t rec_bytes, state_bytes, ckpt_off, carry_off, fin_off, total;
};
static BwdPlan bwd_plan(const kdn_scan_args* f) {
  BwdPlan L;
  L.nch = (f->T + C - 1) / C;
  const int64_t heads = f->B * f->H;
  const size_t per_chunk = (size_t)heads * bwd_record_floats((int)f->D, (int)f->d_v) * sizeof(float);
  int64_t seg = 4;
  if (f->segment_chunks > 0) {
    seg = f->segment_chunks;
  } else {
    const size_t fit = BWD_SEGMENT_BUDGET / per_chunk;
    while (seg < 256 && (size_t)(2 * seg) <= fit) seg *= 2;
  }
  if (seg > L.nch) seg = L.nch;
  L.seg = seg;
  L.nsegs = (L.nch + seg - 1) / seg;
  L.rec_bytes = (size_t)seg * per_chunk;
  L.state_bytes = (size_t)heads * (size_t)f->D * (size_t)f->d_v * sizeof(float);
  L.ckpt_off = L.rec_bytes;
  L.carry_off = L.ckpt_off + (size_t)(L.nsegs - 1) * L.state_bytes;
  L.fin_off = L.carry_off + (L.nsegs > 1 ? L.state_bytes : 0);
  L.total = L.fin_off + L.state_bytes;
  return L;
}

}  // namespace gen

bool general_scan_applies(const kdn_scan_args* a) { return a && a->D == 1024; }

int general_scan_validate(const kdn_scan_args* a) {
  if (a->feature_mode != 1 || a->d_k != a->D) return KDN_ERR_UNSUPPORTED;  // pre-lifted features only
  if (a->rule != 0 || a->cu_seqlens || a->state_slots) return KDN_ERR_UNSUPPORTED;
  if (a->d_v != 64 && a->d_v != 128) return KDN_ERR_UNSUPPORTED;
  return KDN_OK;
}

size_t general_scan_workspace_bytes(const kdn_scan_args* a) {
  const int64_t nch = (a->T + gen::C - 1) / gen::C;
  return (size_t)(a->B * a->H * nch) * gen::record_floats(a->D, a->d_v) * sizeof(float);
}

int general_scan(const kdn_scan_args* a, void* stream) {
  if (a->workspace_bytes < general_scan_workspace_bytes(a)) return KDN_ERR_WORKSPACE_TOO_SMALL;
  gen::Params p = {};
  p.B = a->B; p.T = a->T; p.H = a->H; p.nch = (a->T + gen::C - 1) / gen::C;
  if (p.nch > 0x7fffffff) return KDN_ERR_UNSUPPORTED;
  p.q = a->q; p.qs0 = a->q_stride[0]; p.qs1 = a->q_stride[1]; p.qs2 = a->q_stride[2];
  p.k = a->k; p.ks0 = a->k_stride[0]; p.ks1 = a->k_stride[1]; p.ks2 = a->k_stride[2];
  p.v = a->v; p.vs0 = a->v_stride[0]; p.vs1 = a->v_stride[1]; p.vs2 = a->v_stride[2];
  p.beta = a->beta; p.bs0 = a->beta_stride[0]; p.bs1 = a->beta_stride[1]; p.bs2 = a->beta_stride[2];
  p.decay = a->decay; p.ds0 = a->decay_stride[0]; p.ds1 = a->decay_stride[1]; p.ds2 = a->decay_stride[2];
  p.init = a->initial_state;
  p.is0 = a->init_stride[0]; p.is1 = a->init_stride[1]; p.is2 = a->init_stride[2]; p.is3 = a->init_stride[3];
  p.fin = a->final_state;
  p.fs0 = a->final_stride[0]; p.fs1 = a->final_stride[1]; p.fs2 = a->final_stride[2]; p.fs3 = a->final_stride[3];
  p.y = a->y; p.ys0 = a->y_stride[0]; p.ys1 = a->y_stride[1]; p.ys2 = a->y_stride[2];
  p.ws = reinterpret_cast<float*>(a->workspace);
  const hipStream_t st = as_stream(stream);
  if (a->d_v == 64) return gen::launch_dtypes<1024, 64>(p, a->in_dtype, a->out_dtype, st);
  return gen::launch_dtypes<1024, 128>(p, a->in_dtype, a->out_dtype, st);
}

}  // namespace kdn

namespace kdn {

bool general_bwd_applies(const kdn_scan_args* f) { return f && f->D == 1024; }

static int general_bwd_check(const kdn_scan_bwd_args* a) {
  if (!a || !a->fwd) return KDN_ERR_INVALID_ARGUMENT;
  const kdn_scan_args* f = a->fwd;
  if (f->B <= 0 || f->T <= 0 || f->H <= 0 || !valid_dtype(f->in_dtype)) return KDN_ERR_INVALID_ARGUMENT;
  if (f->B > 65535 || f->H > 65535) return KDN_ERR_UNSUPPORTED;  // grid y / z limits of the chunk launches
  const int rc = general_scan_validate(f);
  if (rc != KDN_OK) return rc;
  if (a->dinv_tau) return KDN_ERR_UNSUPPORTED;  // pre-lifted features have no temperature
  if (!f->q || !f->k || !f->v || !f->beta) return KDN_ERR_INVALID_ARGUMENT;
  if (!a->dy || !a->dq || !a->dk || !a->dv || !a->dbeta) return KDN_ERR_INVALID_ARGUMENT;
  if (a->ddecay && !f->decay) return KDN_ERR_INVALID_ARGUMENT;
  for (int i = 0; i < 3; ++i) {
    if (f->q_stride[i] < 0 || f->k_stride[i] < 0 || f->v_stride[i] < 0 || f->beta_stride[i] < 0 ||
        (f->decay && f->decay_stride[i] < 0) || a->dy_stride[i] < 0 || a->dq_stride[i] < 0 || a->dk_stride[i] < 0 ||
        a->dv_stride[i] < 0 || a->dbeta_stride[i] < 0 || (a->ddecay && a->ddecay_stride[i] < 0))
      return KDN_ERR_INVALID_ARGUMENT;
  }
  for (int i = 0; i < 4; ++i) {
    if ((f->initial_state && f->init_stride[i] < 0) || (a->d_final_state && a->dfinal_stride[i] < 0) ||
        (a->d_initial_state && a->dinit_stride[i] < 0))
      return KDN_ERR_INVALID_ARGUMENT;
  }
  const size_t isz = dtype_size(f->in_dtype);
  if (!aligned(f->q, isz) || !aligned(f->k, isz) || !aligned(f->v, isz) || !aligned(f->beta, 4))
    return KDN_ERR_MISALIGNED;
  if (!aligned(a->dy, 4) || !aligned(a->dq, 4) || !aligned(a->dk, 4) || !aligned(a->dv, 4) || !aligned(a->dbeta, 4))
    return KDN_ERR_MISALIGNED;
  return KDN_OK;
}

size_t general_bwd_workspace_bytes(const kdn_scan_bwd_args* a) {
  if (general_bwd_check(a) != KDN_OK) return 0;
  return gen::bwd_plan(a->fwd).total;
}

int64_t general_bwd_segments(const kdn_scan_bwd_args* a, int64_t* segment_chunks) {
  if (general_bwd_check(a) != KDN_OK) return 0;
  const gen::BwdPlan L = gen::bwd_plan(a->fwd);
  if (segment_chunks) *segment_chunks = L.seg;
  return L.nsegs;
}

// Segmented like the D = 512 backward: a checkpoint pass runs the recompute and the forward carry over
// segments 0 .. n-2 and keeps the state at each segment start; then each segment, last first, recomputes
// its chunks from its checkpoint, carries dL/dS back from the next segment (in place in one buffer: every
// workgroup of the reverse carry reads its slice before it writes it) and writes its gradients.  A segment
// is the chunk range [c0, c0 + n) as a sequence of its own (input and gradient pointers advanced by 64 c0
// tokens); the kernels carry the same sums in the same order as over the whole sequence, so the results
// do not depend on the segment length.
template <class PB, typename InT, int D, int DV>
static int general_bwd_run(const gen::Params& p, const gen::BwdP& g, const gen::BwdPlan& L, size_t isz,
                           hipStream_t st) {
  unsigned char* ws = reinterpret_cast<unsigned char*>(p.ws);
  const int64_t ss0 = p.H * D * DV, ss1 = (int64_t)D * DV, ss2 = DV, ss3 = 1;  // checkpoint / carry layout
  auto state_at = [&](size_t off) { return reinterpret_cast<float*>(ws + off); };
  auto segment = [&](int64_t s, gen::Params& ps, gen::BwdP& gs) {
    const int64_t c0 = s * L.seg, n = (L.nch - c0 < L.seg) ? L.nch - c0 : L.seg, t0 = c0 * gen::C;
    ps = p;
    gs = g;
    ps.nch = n;
    ps.T = (p.T - t0 < n * gen::C) ? p.T - t0 : n * gen::C;
    ps.q = static_cast<const unsigned char*>(p.q) + (size_t)(t0 * p.qs1) * isz;
    ps.k = static_cast<const unsigned char*>(p.k) + (size_t)(t0 * p.ks1) * isz;
    ps.v = static_cast<const unsigned char*>(p.v) + (size_t)(t0 * p.vs1) * isz;
    ps.beta = p.beta + t0 * p.bs1;
    if (p.decay) ps.decay = p.decay + t0 * p.ds1;
    gs.dy = g.dy + t0 * g.ys1;
    gs.dq = g.dq + t0 * g.dqs1;
    gs.dk = g.dk + t0 * g.dks1;
    gs.dv = g.dv + t0 * g.dvs1;
    gs.dbeta = g.dbeta + t0 * g.dbs1;
    if (g.ddecay) gs.ddecay = g.ddecay + t0 * g.dds1;
    if (s > 0) {  // the state at the segment start: the checkpoint of segment s - 1's end
      ps.init = state_at(L.ckpt_off + (size_t)(s - 1) * L.state_bytes);
      ps.is0 = ss0; ps.is1 = ss1; ps.is2 = ss2; ps.is3 = ss3;
    }
  };
  for (int64_t s = 0; s + 1 < L.nsegs; ++s) {
    gen::Params ps;
    gen::BwdP gs;
    segment(s, ps, gs);
    ps.fin = state_at(L.ckpt_off + (size_t)s * L.state_bytes);
    ps.fs0 = ss0; ps.fs1 = ss1; ps.fs2 = ss2; ps.fs3 = ss3;
    const int rc = gen::launch_ckpt<PB, InT, D, DV>(ps, st);
    if (rc != KDN_OK) return rc;
  }
  for (int64_t s = L.nsegs - 1; s >= 0; --s) {
    gen::Params ps;
    gen::BwdP gs;
    segment(s, ps, gs);
    ps.fin = state_at(L.fin_off);
    ps.fs0 = ss0; ps.fs1 = ss1; ps.fs2 = ss2; ps.fs3 = ss3;
    if (s + 1 < L.nsegs) {  // dL/dS at the segment end, left by the next segment's reverse carry
      gs.dfin = state_at(L.carry_off);
      gs.fs0 = ss0; gs.fs1 = ss1; gs.fs2 = ss2; gs.fs3 = ss3;
    }
    if (s > 0) {  // dL/dS at the segment start, for the previous segment
      gs.dinit = state_at(L.carry_off);
      gs.gis0 = ss0; gs.gis1 = ss1; gs.gis2 = ss2; gs.gis3 = ss3;
    }
    const int rc = gen::launch_bwd<PB, InT, D, DV>(ps, gs, st);
    if (rc != KDN_OK) return rc;
  }
  return KDN_OK;
}

int general_bwd(const kdn_scan_bwd_args* a, void* stream) {
  const int rc = general_bwd_check(a);
  if (rc != KDN_OK) return rc;
  if (a->workspace_bytes < general_bwd_workspace_bytes(a)) return KDN_ERR_WORKSPACE_TOO_SMALL;
  if (!a->workspace) return KDN_ERR_INVALID_ARGUMENT;
  if (!aligned(a->workspace, 256)) return KDN_ERR_MISALIGNED;
  const kdn_scan_args* f = a->fwd;
  const gen::BwdPlan L = gen::bwd_plan(f);
  gen::Params p = {};
  p.B = f->B; p.T = f->T; p.H = f->H; p.nch = L.nch;
  if (p.nch > 0x7fffffff) return KDN_ERR_UNSUPPORTED;
  p.q = f->q; p.qs0 = f->q_stride[0]; p.qs1 = f->q_stride[1]; p.qs2 = f->q_stride[2];
  p.k = f->k; p.ks0 = f->k_stride[0]; p.ks1 = f->k_stride[1]; p.ks2 = f->k_stride[2];
  p.v = f->v; p.vs0 = f->v_stride[0]; p.vs1 = f->v_stride[1]; p.vs2 = f->v_stride[2];
  p.beta = f->beta; p.bs0 = f->beta_stride[0]; p.bs1 = f->beta_stride[1]; p.bs2 = f->beta_stride[2];
  p.decay = f->decay; p.ds0 = f->decay_stride[0]; p.ds1 = f->decay_stride[1]; p.ds2 = f->decay_stride[2];
  p.init = f->initial_state;
  p.is0 = f->init_stride[0]; p.is1 = f->init_stride[1]; p.is2 = f->init_stride[2]; p.is3 = f->init_stride[3];
  p.ws = reinterpret_cast<float*>(a->workspace);
  const int DV = (int)f->d_v;
  gen::BwdP g = {};
  g.dy = a->dy; g.ys0 = a->dy_stride[0]; g.ys1 = a->dy_stride[1]; g.ys2 = a->dy_stride[2];
  g.dfin = a->d_final_state;
  g.fs0 = a->dfinal_stride[0]; g.fs1 = a->dfinal_stride[1]; g.fs2 = a->dfinal_stride[2]; g.fs3 = a->dfinal_stride[3];
  g.dq = a->dq; g.dqs0 = a->dq_stride[0]; g.dqs1 = a->dq_stride[1]; g.dqs2 = a->dq_stride[2];
  g.dk = a->dk; g.dks0 = a->dk_stride[0]; g.dks1 = a->dk_stride[1]; g.dks2 = a->dk_stride[2];
  g.dv = a->dv; g.dvs0 = a->dv_stride[0]; g.dvs1 = a->dv_stride[1]; g.dvs2 = a->dv_stride[2];
  g.dbeta = a->dbeta; g.dbs0 = a->dbeta_stride[0]; g.dbs1 = a->dbeta_stride[1]; g.dbs2 = a->dbeta_stride[2];
  g.ddecay = a->ddecay; g.dds0 = a->ddecay_stride[0]; g.dds1 = a->ddecay_stride[1]; g.dds2 = a->ddecay_stride[2];
  g.dinit = a->d_initial_state;
  g.gis0 = a->dinit_stride[0]; g.gis1 = a->dinit_stride[1]; g.gis2 = a->dinit_stride[2]; g.gis3 = a->dinit_stride[3];
  const hipStream_t st = as_stream(stream);
  const size_t isz = dtype_size(f->in_dtype);
  if (DV == 64) {
    if (f->in_dtype == KDN_DTYPE_BF16) return general_bwd_run<PrecBF16, __bf16, 1024, 64>(p, g, L, isz, st);
    return general_bwd_run<PrecF32, float, 1024, 64>(p, g, L, isz, st);
  }
  if (f->in_dtype == KDN_DTYPE_BF16) return general_bwd_run<PrecBF16, __bf16, 1024, 128>(p, g, L, isz, st);
  return general_bwd_run<PrecF32, float, 1024, 128>(p, g, L, isz, st);
}

}  // namespace kdn
