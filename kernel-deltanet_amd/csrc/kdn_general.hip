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

template <int D, int DV>
__device__ __forceinline__ float* record(const Params& p, int64_t b, int64_t h, int64_t c) {
  return p.ws + ((b * p.H + h) * p.nch + c) * (int64_t)Rec<D, DV>::floats;
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
template <class PB, typename InT, int D, int DV>
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
  float* rec = record<D, DV>(p, b, h, c);
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

template <class PB, int D, int DV, bool PIPE>
__device__ __forceinline__ bool carry_step(const Params& p, CarryShared& sh, int64_t b, int64_t h, int64_t c,
                                           CarryK<PB, D>& cur, CarryK<PB, D>& nxt, f32x4 (&Sg)[D / 64], int w,
                                           int lane, int n, unsigned& sink) {
  using R = Rec<D, DV>;
  using frag = typename PB::frag;
  constexpr int NV = R::NV, TPW = D / 64, JPW = D / 128;
  const bool more = c + 1 < p.nch;
  float* rec = record<D, DV>(p, b, h, c);
  const frag* kxf = reinterpret_cast<const frag*>(rec + R::KXF);
  const f32x8 tp0 = frag_rows(rec + R::TP, C, 16 * w, 0, lane), tp1 = frag_rows(rec + R::TP, C, 16 * w, 32, lane);
  const f32x4 ur = reinterpret_cast<const f32x4*>(rec + R::U)[(w * NV + n) * 64 + lane];
  const f32x4 lr = *reinterpret_cast<const f32x4*>(rec + R::VEC + 16 * w + 4 * (lane >> 4));
  const float l63 = rec[R::VEC + 63];
  unsigned pf = 0;  // L2-prefetch loads, folded into `sink` at the end of the step
  if (more) {
    const float* nrec = record<D, DV>(p, b, h, c + 1);
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
  frag* sf = reinterpret_cast<frag*>(rec + R::S);
  f32x4 xp[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) xp[m] = zero4();
#pragma unroll
  for (int jj = 0; jj < JPW; ++jj) {
    const frag sb = PB::from_f32(pair_to8(Sg[2 * jj], Sg[2 * jj + 1]));
    sf[((w * JPW + jj) * NV + n) * 64 + lane] = sb;
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

template <class PB, int D, int DV>
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
  if constexpr (PIPE) carry_load_kx<PB, D, DV>(ka, record<D, DV>(p, b, h, 0), w, lane);
  for (int64_t c = 0;; c += 2) {
    if (!carry_step<PB, D, DV, PIPE>(p, sh, b, h, c, ka, kb, Sg, w, lane, n, sink)) break;
    if (!carry_step<PB, D, DV, PIPE>(p, sh, b, h, c + 1, kb, ka, Sg, w, lane, n, sink)) break;
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
