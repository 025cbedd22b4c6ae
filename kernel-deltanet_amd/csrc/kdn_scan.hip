// Chunked gated delta-rule prefill scan of Kernel-DeltaNet on gfx950.
//
// Recurrence (readout before update; tests/test_fused_kernel.py:53-65 of the reference):
//   y_t = S_{t-1} phi_q(t),    S_t = lambda_t S_{t-1} (I - beta_t phi_k(t) phi_k(t)^T) + beta_t v_t phi_k(t)^T
// with S (d_v x D) carried in fp32.  Per 64-token chunk, with g = cumsum(log lambda) inside the chunk
// and K, Q the lifted keys/queries of the chunk (rows), the WY/UT form used here is
//   A[t][j]  = beta_t e^{g_t - g_j} (K K^T)[t][j]                       (j < t)
//   T        = (I + A)^{-1}                                              (unit lower triangular)
//   U~       = T diag(beta) V,       W~ = T diag(beta e^{g}) K
//   E        = U~ - W~ S^T           (the per-token "errors" beta_t (v_t - lambda_t S_{t-1} k_t))
//   Y        = diag(e^{g_{t-1}}) Q S^T + P E,   P[t][j] = e^{g_{t-1} - g_j} (Q K^T)[t][j]   (j < t)
//   S_next   = e^{g_63} S + E^T diag(e^{g_63 - g}) K
// which is algebraically the scan of kernels/fused_kernel_deltanet.py:93-149 (that code factors the
// decay-free homogeneous part through an upper-triangular resolvent; both equal the token recurrence).
//
// Two kernels per segment of chunks:
//   prep (one workgroup per chunk and head, fully parallel): lift q/k on MFMA, Gram matrices, the
//        triangular inverse, and every S-independent factor, written to a workspace in MFMA-fragment
//        order so that the scan reads 16 contiguous bytes per lane.
//   scan (one workgroup per 16 state rows of a head, sequential over chunks): the S-dependent
//        products X = [K; Q] S^T, E, Y and the state update, state resident in accumulators.
// The lifted features are stored unnormalised (cos values); per-row norms are folded into the small
// per-token scale vectors, so the lift never has to hold a whole row before writing it.
#include <type_traits>
#include "kdn_frag.hpp"
#include "kdn_internal.hpp"
#include "kdn_io.hpp"

namespace kdn {

constexpr int CH = 64;  // tokens per chunk (internal; the WY form is exact for any chunk length)

template <class P, int D, int DV>
struct WsLayout {
  static constexpr size_t FB = P::frag_bytes;
  static constexpr int NJ = D / 32;   // 32-deep blocks over features
  static constexpr int NTD = D / 16;  // 16-wide feature tiles
  static constexpr int NV = DV / 16;  // 16-wide value tiles
  static constexpr size_t phiKX = 0;                                // [m 4][j NJ][lane] K row frags
  static constexpr size_t phiQX = phiKX + (size_t)4 * NJ * 64 * FB; // [m 4][j NJ][lane] Q row frags
  static constexpr size_t phiKU = phiQX + (size_t)4 * NJ * 64 * FB; // [t NTD][jb 2][lane] K^T frags
  static constexpr size_t Tp = phiKU + (size_t)NTD * 2 * 64 * FB;   // [m 4][jb 2][lane]  W~ factor
  static constexpr size_t Pm = Tp + (size_t)4 * 2 * 64 * FB;        // [m 4][jb 2][lane]  P
  static constexpr size_t U = Pm + (size_t)4 * 2 * 64 * FB;         // [m 4][n NV][lane] f32x4  U~
  static constexpr size_t VEC = U + (size_t)4 * NV * 64 * 16;       // qscale[64] kscale[64] gammaC
  static constexpr size_t bytes = ((VEC + (64 + 64 + 4) * 4) + 255) / 256 * 256;
};

struct ScanParams {
  int64_t B, T, H;
  const void* q; int64_t qs0, qs1, qs2;
  const void* k; int64_t ks0, ks1, ks2;
  const void* v; int64_t vs0, vs1, vs2;
  const float* beta; int64_t bs0, bs1, bs2;
  const float* decay; int64_t ds0, ds1, ds2;
  const __bf16* omega; const float* phase;
  float inv_tau; int normalize;
  const float* state_in; int64_t is0, is1, is2, is3;
  float* state_out; int64_t os0, os1, os2, os3;
  void* y; int64_t ys0, ys1, ys2;
  unsigned char* ws;
  int64_t chunk0, nseg;  // first global chunk of the segment, chunks in the segment
};

template <class P>
struct PrepOmegaInLds : std::integral_constant<bool, std::is_same<P, PrecBF16>::value> {};

// ------------------------------------------------------------------------------------------------
// prep: grid (nseg, H, B), 256 threads.  Wave w owns token rows [16w, 16w+16) of the chunk.
template <class P, typename InT, int D, int DV>
__global__ void __launch_bounds__(256) prep_kernel(ScanParams p) {
  using L = WsLayout<P, D, DV>;
  using frag = typename P::frag;
  typedef typename std::conditional<std::is_same<P, PrecBF16>::value, __bf16, float>::type FE;  // frag element
  constexpr int NT = D / 16, NJ = D / 32, NV = DV / 16;
  constexpr int NSPLIT = XFrag<InT>::NSPLIT;
  constexpr bool OMEGA_LDS = PrepOmegaInLds<P>::value;
  constexpr size_t OMEGA_BYTES = OMEGA_LDS ? (size_t)NT * 2 * 64 * 16 : 0;
  constexpr size_t PHIK_BYTES = (size_t)4 * NJ * 64 * sizeof(frag);
  // After the Gram the K-fragment area is reused for A (16 KB), T (17 KB) and V.
  static_assert(64 * 64 * 4 + 64 * 68 * 4 + 64 * DV * sizeof(InT) <= PHIK_BYTES, "LDS reuse does not fit");
  __shared__ __attribute__((aligned(16))) unsigned char smem[OMEGA_BYTES + PHIK_BYTES];
  __shared__ __attribute__((aligned(16))) float s_beta[64], s_g[64], s_sq[64], s_sk[64], s_phrev[D];

  bf16x8* s_omega = reinterpret_cast<bf16x8*>(smem);
  frag* s_phik = reinterpret_cast<frag*>(smem + OMEGA_BYTES);
  float* s_A = reinterpret_cast<float*>(smem + OMEGA_BYTES);          // [t][p][k'] = A[t][4k'+p]
  float* s_T = s_A + 64 * 64;                                          // [t][68]
  InT* s_V = reinterpret_cast<InT*>(s_T + 64 * 68);                    // [t][DV]

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t cl = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t t0 = (p.chunk0 + cl) * CH;
  unsigned char* ws = p.ws + ((b * p.H + h) * p.nseg + cl) * L::bytes;

  // ---- stage Omega fragments and phases; beta and the in-chunk log-decay prefix (wave 0)
  if constexpr (OMEGA_LDS) {
    for (int idx = threadIdx.x; idx < NT * 2 * 64; idx += 256) {
      const int l = idx & 63, tk = idx >> 6, t = tk >> 1, kb = tk & 1;
      s_omega[idx] = *reinterpret_cast<const bf16x8*>(p.omega + (int64_t)(16 * t + (l & 15)) * 64 + 32 * kb + 8 * (l >> 4));
    }
  }
  for (int f = threadIdx.x; f < D; f += 256) s_phrev[f] = p.phase[f] * 0.15915494309189535f;
  if (w == 0) {
    const int64_t t = t0 + lane;
    const bool valid = t < p.T;
    const float be = valid ? p.beta[b * p.bs0 + t * p.bs1 + h * p.bs2] : 0.f;
    const float la = (valid && p.decay) ? p.decay[b * p.ds0 + t * p.ds1 + h * p.ds2] : 1.f;
    float g = logf(fminf(fmaxf(la, 1e-5f), 1.f));
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(g, off);
      if (lane >= off) g += o;
    }
    s_beta[lane] = be;
    s_g[lane] = g;
  }
  __syncthreads();

  // ---- lift q and k rows of this wave: Phi^T = Omega X^T, cos, row sums of squares
  const int64_t trow = t0 + 16 * w + (lane & 15);
  const bool rvalid = trow < p.T;
  float xq[2][8], xk[2][8];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    if (rvalid) {
      load8<InT>((const InT*)p.q + b * p.qs0 + trow * p.qs1 + h * p.qs2 + 32 * kb + 8 * (lane >> 4), xq[kb]);
      load8<InT>((const InT*)p.k + b * p.ks0 + trow * p.ks1 + h * p.ks2 + 32 * kb + 8 * (lane >> 4), xk[kb]);
    } else {
#pragma unroll
      for (int s = 0; s < 8; ++s) { xq[kb][s] = 0.f; xk[kb][s] = 0.f; }
    }
  }
  if (p.normalize) {
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int s = 0; s < 8; ++s) { sq += xq[kb][s] * xq[kb][s]; sk += xk[kb][s] * xk[kb][s]; }
    sq = sum_over_lane_groups(sq);
    sk = sum_over_lane_groups(sk);
    const float iq = 1.0f / fmaxf(sqrtf(sq), 1e-6f), ik = 1.0f / fmaxf(sqrtf(sk), 1e-6f);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const float a = xq[kb][s] * iq, c = xk[kb][s] * ik;
        xq[kb][s] = (NSPLIT == 1) ? (float)(__bf16)a : a;
        xk[kb][s] = (NSPLIT == 1) ? (float)(__bf16)c : c;
      }
  }
  bf16x8 xqb[2][NSPLIT], xkb[2][NSPLIT];
  split_frag<NSPLIT>(xq[0], xqb[0]);
  split_frag<NSPLIT>(xq[1], xqb[1]);
  split_frag<NSPLIT>(xk[0], xkb[0]);
  split_frag<NSPLIT>(xk[1], xkb[1]);

  const float ang = p.inv_tau * 0.15915494309189535f;
  frag cq[NJ], ck[NJ];  // X fragments (m = w, j): row 16w + (l&15), feature 32j + kappa(l, s)
  float ssq = 0.f, ssk = 0.f;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    f32x4 aq = zero4(), ak = zero4();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      bf16x8 a;
      if constexpr (OMEGA_LDS) a = s_omega[(t * 2 + kb) * 64 + lane];
      else a = *reinterpret_cast<const bf16x8*>(p.omega + (int64_t)(16 * t + (lane & 15)) * 64 + 32 * kb + 8 * (lane >> 4));
#pragma unroll
      for (int s = 0; s < NSPLIT; ++s) {
        aq = PrecBF16::mma(aq, a, xqb[kb][s]);
        ak = PrecBF16::mma(ak, a, xkb[kb][s]);
      }
    }
    // accumulator lane l: feature 16t + 4(l>>4) + i of row (l & 15)  ->  slot (t & 1) * 4 + i of frag t/2
    const f32x4 ph = *reinterpret_cast<const f32x4*>(&s_phrev[16 * t + 4 * (lane >> 4)]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float rq = aq[i] * ang + ph[i];
      float rk = ak[i] * ang + ph[i];
      rq -= __builtin_rintf(rq);
      rk -= __builtin_rintf(rk);
      const float cqv = __builtin_amdgcn_cosf(rq), ckv = __builtin_amdgcn_cosf(rk);
      ssq += cqv * cqv;
      ssk += ckv * ckv;
      P::set(cq[t >> 1], (t & 1) * 4 + i, cqv);
      P::set(ck[t >> 1], (t & 1) * 4 + i, ckv);
    }
  }
  ssq = sum_over_lane_groups(ssq);
  ssk = sum_over_lane_groups(ssk);
  {
    const float amp = sqrtf(2.0f / (float)D);
    if (lane < 16) {
      s_sq[16 * w + lane] = amp / (amp * sqrtf(ssq) + 1e-8f);
      s_sk[16 * w + lane] = amp / (amp * sqrtf(ssk) + 1e-8f);
    }
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    store_frag<P>(ws + L::phiQX + (size_t)(w * NJ + j) * 64 * L::FB, lane, cq[j]);
    store_frag<P>(ws + L::phiKX + (size_t)(w * NJ + j) * 64 * L::FB, lane, ck[j]);
    s_phik[(w * NJ + j) * 64 + lane] = ck[j];
  }
  __syncthreads();

  // ---- Gram tiles (m, n = w):  Gkk[m][w] = K_m K_w^T,  GqkT[m][w] = K_m Q_w^T  (unnormalised)
  f32x4 gkk[4], gqk[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) { gkk[m] = zero4(); gqk[m] = zero4(); }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const frag a = s_phik[(m * NJ + j) * 64 + lane];
      gkk[m] = P::mma(gkk[m], a, ck[j]);
      gqk[m] = P::mma(gqk[m], a, cq[j]);
    }
  }

  // ---- K^T fragments for the state update: (tile tt, jb) lane l slot s = K[32jb + kappa][16tt + (l&15)]
  {
    const FE* e = reinterpret_cast<const FE*>(s_phik);
    for (int tt = 8 * (NT / 32) * w; tt < 8 * (NT / 32) * (w + 1); ++tt) {
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        frag f;
        const int d = 16 * tt + (lane & 15);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const int c = 32 * jb + kappa(lane, s);
          const int fi = (c >> 4) * NJ + (d >> 5);
          const int sl = (c & 15) + 16 * ((d >> 2) & 3);
          const int ss = 4 * ((d >> 4) & 1) + (d & 3);
          f[s] = e[((size_t)fi * 64 + sl) * 8 + ss];
        }
        store_frag<P>(ws + L::phiKU + (size_t)(tt * 2 + jb) * 64 * L::FB, lane, f);
      }
    }
  }
  __syncthreads();  // K fragments in LDS are dead from here on

  // ---- A (for the inverse), P fragments, V staging, scale vectors
  {
    const int t = 16 * w + (lane & 15);
    const float bt = s_beta[t], gt = s_g[t], gtm1 = t > 0 ? s_g[t - 1] : 0.f;
    const float skt = s_sk[t], sqt = s_sq[t];
    f32x4 pt[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = 16 * m + 4 * (lane >> 4) + i;
        const float gj = s_g[j], skj = s_sk[j];
        const float a = (j < t) ? bt * __expf(fminf(gt - gj, 0.f)) * gkk[m][i] * skt * skj : 0.f;
        s_A[(t * 4 + i) * 16 + 4 * m + (lane >> 4)] = a;  // j = 4(4m + (l>>4)) + i
        pt[m][i] = (j < t) ? __expf(fminf(gtm1 - gj, 0.f)) * gqk[m][i] * sqt * skj : 0.f;
      }
    }
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
      store_frag<P>(ws + L::Pm + (size_t)(w * 2 + jb) * 64 * L::FB, lane, P::from_f32(pair_to8(pt[2 * jb], pt[2 * jb + 1])));
  }
  {
    // V rows of the chunk (zero past T), 16-byte loads
    constexpr int VPR = DV * sizeof(InT) / 16;  // 16-byte pieces per row
    for (int idx = threadIdx.x; idx < 64 * VPR; idx += 256) {
      const int r = idx / VPR, pc = idx % VPR;
      const int64_t t = t0 + r;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (t < p.T) val = *reinterpret_cast<const u32x4*>((const InT*)p.v + b * p.vs0 + t * p.vs1 + h * p.vs2 + pc * (16 / sizeof(InT)));
      *reinterpret_cast<u32x4*>(s_V + r * DV + pc * (16 / sizeof(InT))) = val;
    }
  }
  if (w == 1) {
    float* vec = reinterpret_cast<float*>(ws + L::VEC);
    const float g63 = s_g[63];
    const float gtm1 = lane > 0 ? s_g[lane - 1] : 0.f;
    vec[lane] = __expf(fminf(gtm1, 0.f)) * s_sq[lane];                 // e^{g_{t-1}} * |phi_q| scale
    vec[64 + lane] = __expf(fminf(g63 - s_g[lane], 0.f)) * s_sk[lane]; // e^{g_63 - g_t} * |phi_k| scale
    if (lane == 0) vec[128] = __expf(fminf(g63, 0.f));
  }
  __syncthreads();

  // ---- T = (I + A)^{-1}: column col = 16w + (l>>2) per lane quad; lane p = l&3 keeps rows 4k'+p
  {
    const int col = 16 * w + (lane >> 2), pq = lane & 3;
    float Tr[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) Tr[k] = 0.f;
#pragma unroll
    for (int i = 0; i < 64; ++i) {
      const float* arow = s_A + (i * 4 + pq) * 16;
      float part = 0.f;
#pragma unroll
      for (int k = 0; k < (i + 3) / 4; ++k) part += arow[k] * Tr[k];
      part += xor_shuffle<1>(part);
      part += xor_shuffle<2>(part);
      const float val = (i == col ? 1.f : 0.f) - part;
      if (pq == (i & 3)) Tr[i >> 2] = val;
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) s_T[(4 * k + pq) * 68 + col] = Tr[k];
  }
  __syncthreads();

  // ---- W~ factor T diag(beta e^g |phi_k|) fragments, and U~ = T diag(beta) V   (wave w: rows m = w)
  {
    const int t = 16 * w + (lane & 15);
    f32x8 tb[2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      f32x8 tw;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int j = 32 * jb + kappa(lane, s);
        const float tv = s_T[t * 68 + j];
        tw[s] = tv * s_beta[j] * __expf(s_g[j]) * s_sk[j];
        tb[jb][s] = tv * s_beta[j];
      }
      store_frag<P>(ws + L::Tp + (size_t)(w * 2 + jb) * 64 * L::FB, lane, P::from_f32(tw));
    }
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      f32x4 acc = zero4();
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        f32x8 vv;
#pragma unroll
        for (int s = 0; s < 8; ++s) vv[s] = (float)s_V[(32 * jb + kappa(lane, s)) * DV + 16 * n + (lane & 15)];
        if constexpr (std::is_same<P, PrecBF16>::value) {
          // hi + lo split of T diag(beta): V is exact in bf16, so U~ keeps ~16 bits.
          bf16x8 hi, lo, vb;
#pragma unroll
          for (int s = 0; s < 8; ++s) {
            hi[s] = (__bf16)tb[jb][s];
            lo[s] = (__bf16)(tb[jb][s] - (float)hi[s]);
            vb[s] = (__bf16)vv[s];
          }
          acc = PrecBF16::mma(acc, hi, vb);
          acc = PrecBF16::mma(acc, lo, vb);
        } else {
          acc = P::mma(acc, P::from_f32(tb[jb]), P::from_f32(vv));
        }
      }
      *reinterpret_cast<f32x4*>(ws + L::U + ((size_t)(w * NV + n) * 64 + lane) * 16) = acc;
    }
  }
}

// ------------------------------------------------------------------------------------------------
// scan: one workgroup of 4 waves per (head, 16 value components = 16 state rows).  Wave w owns features
// [128w, 128w + 128) of those rows: S^T tiles (feature tile, row tile) in accumulator layout, lane l holds
// S^T[16tt + 4(l>>4) + i][r0 + (l&15)].  Per chunk:
//   all waves   X partial over their features  X[m] = sum_j frag(m, j) S^T(j), m: 4 K-row tiles, 4 Q-row tiles
//   barrier     wave w reduces tile w over the 8 partials
//   wave w      E tile w  = U~ - Tp X_K,  then (after all E tiles are in LDS)  Y tile w = qscale X_Q + P E
//   all waves   S^T <- gammaC S^T + K^T (kscale o E) on their feature tiles
// The next chunk's operand fragments are loaded while the current chunk is computed (about 192 KB
// in flight per workgroup), since this kernel's only parallelism is B*H*d_v/16 workgroups.
//
// Workgroups are dispatched round-robin over the 8 XCDs (linear id % 8); the value tiles of one head
// get ids with equal residue so that they share one XCD's L2 for the chunk operands they all read.
template <typename T>
__device__ __forceinline__ void store_y(T* p, float v);
template <>
__device__ __forceinline__ void store_y<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_y<__bf16>(__bf16* p, float v) { *p = (__bf16)v; }

constexpr int SCAN_WAVES = 4;

template <class P, int D, int DV>
struct ScanOps {
  using L = WsLayout<P, D, DV>;
  using frag = typename P::frag;
  static constexpr int NJ = D / 32;
  static constexpr int TPW = D / 16 / SCAN_WAVES;  // feature tiles per wave
  static constexpr int JPW = D / 32 / SCAN_WAVES;  // 32-deep feature blocks per wave
  static constexpr int NV = DV / 16;
  struct Small {
    frag tp[2], pm[2];  // Tp and P fragments of row tile w
    f32x4 u;            // U~ tile (w, n)
    f32x4 qs;           // qscale of the rows of tile w
    f32x4 ks[4];        // kscale of the 64 chunk rows in kappa order (jb, half)
    float gC;
  };
  __device__ static void load_x(const unsigned char* ws, int w, int lane, frag (&ax)[8][JPW]) {
#pragma unroll
    for (int jj = 0; jj < JPW; ++jj) {
      const int j = JPW * w + jj;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        ax[m][jj] = load_frag<P>(ws + L::phiKX + (size_t)(m * NJ + j) * 64 * L::FB, lane);
        ax[4 + m][jj] = load_frag<P>(ws + L::phiQX + (size_t)(m * NJ + j) * 64 * L::FB, lane);
      }
    }
  }
  __device__ static frag load_x1(const unsigned char* ws, int w, int lane, int m, int jj) {
    const int j = JPW * w + jj;
    return m < 4 ? load_frag<P>(ws + L::phiKX + (size_t)(m * NJ + j) * 64 * L::FB, lane)
                 : load_frag<P>(ws + L::phiQX + (size_t)((m - 4) * NJ + j) * 64 * L::FB, lane);
  }
  __device__ static frag load_u1(const unsigned char* ws, int w, int lane, int tl, int jb) {
    return load_frag<P>(ws + L::phiKU + (size_t)((TPW * w + tl) * 2 + jb) * 64 * L::FB, lane);
  }
  __device__ static void load_u(const unsigned char* ws, int w, int lane, frag (&au)[TPW][2]) {
#pragma unroll
    for (int tl = 0; tl < TPW; ++tl)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
        au[tl][jb] = load_frag<P>(ws + L::phiKU + (size_t)((TPW * w + tl) * 2 + jb) * 64 * L::FB, lane);
  }
  __device__ static void load_small(const unsigned char* ws, int w, int lane, int n, Small& sm) {
    const float* vec = reinterpret_cast<const float*>(ws + L::VEC);
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      sm.tp[jb] = load_frag<P>(ws + L::Tp + (size_t)(w * 2 + jb) * 64 * L::FB, lane);
      sm.pm[jb] = load_frag<P>(ws + L::Pm + (size_t)(w * 2 + jb) * 64 * L::FB, lane);
    }
    sm.u = *reinterpret_cast<const f32x4*>(ws + L::U + ((size_t)(w * NV + n) * 64 + lane) * 16);
    sm.qs = *reinterpret_cast<const f32x4*>(vec + 16 * w + 4 * (lane >> 4));
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        sm.ks[jb * 2 + hf] = *reinterpret_cast<const f32x4*>(vec + 64 + 32 * jb + 16 * hf + 4 * (lane >> 4));
    sm.gC = vec[128];
  }
};

template <class P, typename OutT, int D, int DV>
__global__ void __launch_bounds__(64 * SCAN_WAVES) scan_kernel(ScanParams p) {
  using O = ScanOps<P, D, DV>;
  using L = typename O::L;
  using frag = typename P::frag;
  constexpr int TPW = O::TPW, JPW = O::JPW, NV = O::NV;
  __shared__ f32x4 s_xp[SCAN_WAVES][8][64];  // per-wave partial X tiles
  __shared__ f32x4 s_x[8][64];               // reduced X (tiles 0-3: K rows, 4-7: Q rows)
  __shared__ f32x4 s_e[4][64];               // E tiles

  // XCD-aware decomposition of the 1-D grid: id = xcd + 8 * (rank * NV + n), head-batch pair
  // hb = rank * 8 + xcd.  Ids that land past B*H exit at once.
  const int64_t id = blockIdx.x;
  const int64_t xcd = id & 7, jdx = id >> 3;
  const int n = (int)(jdx % NV);
  const int64_t hb = (jdx / NV) * 8 + xcd;
  if (hb >= p.B * p.H) return;
  const int64_t b = hb / p.H, h = hb % p.H;

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int r = 16 * n + (lane & 15);

  f32x4 S[TPW];
  if (p.state_in) {
    const float* si = p.state_in + b * p.is0 + h * p.is1 + r * p.is3;
#pragma unroll
    for (int tl = 0; tl < TPW; ++tl)
#pragma unroll
      for (int i = 0; i < 4; ++i) S[tl][i] = si[(int64_t)(16 * (TPW * w + tl) + 4 * (lane >> 4) + i) * p.is2];
  } else {
#pragma unroll
    for (int tl = 0; tl < TPW; ++tl) S[tl] = zero4();
  }

  // bf16 operands: the whole next chunk is prefetched into registers (fits the 512-register budget);
  // fp32 operands are twice as wide, so they are loaded where they are used.
  constexpr bool PF = std::is_same<P, PrecBF16>::value;
  const unsigned char* wsh = p.ws + hb * p.nseg * L::bytes;
  frag ax[8][JPW];
  frag au[TPW][2], au_n[TPW][2];
  typename O::Small sm, sm_n;
  if constexpr (PF) {
    O::load_x(wsh, w, lane, ax);
    O::load_u(wsh, w, lane, au);
    O::load_small(wsh, w, lane, n, sm);
  }

  for (int64_t cl = 0; cl < p.nseg; ++cl) {
    const bool more = cl + 1 < p.nseg;
    const unsigned char* wsc = wsh + cl * L::bytes;
    const unsigned char* wsn = wsh + (cl + 1) * L::bytes;
    if constexpr (!PF) O::load_small(wsc, w, lane, n, sm);
    // ---- X partial over this wave's features
    frag sf[JPW];
#pragma unroll
    for (int jj = 0; jj < JPW; ++jj) sf[jj] = P::from_f32(pair_to8(S[2 * jj], S[2 * jj + 1]));
    f32x4 xp[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      xp[m] = zero4();
#pragma unroll
      for (int jj = 0; jj < JPW; ++jj) {
        if constexpr (PF) xp[m] = P::mma(xp[m], ax[m][jj], sf[jj]);
        else xp[m] = P::mma(xp[m], O::load_x1(wsc, w, lane, m, jj), sf[jj]);
      }
    }
    // ---- prefetch the next chunk's operands (the X fragments were just consumed)
    if constexpr (PF) {
      if (more) {
        O::load_x(wsn, w, lane, ax);
        O::load_u(wsn, w, lane, au_n);
        O::load_small(wsn, w, lane, n, sm_n);
      }
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) s_xp[w][m][lane] = xp[m];
    __syncthreads();
#pragma unroll
    for (int mm = 0; mm < 8 / SCAN_WAVES; ++mm) {
      const int m = SCAN_WAVES * mm + w;
      f32x4 acc = s_xp[0][m][lane];
#pragma unroll
      for (int v = 1; v < SCAN_WAVES; ++v) acc += s_xp[v][m][lane];
      s_x[m][lane] = acc;
    }
    __syncthreads();
    // ---- E tile w:  E = U~ - Tp X_K
    {
      f32x4 ek = zero4();
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
        ek = P::mma(ek, sm.tp[jb], P::from_f32(pair_to8(s_x[2 * jb][lane], s_x[2 * jb + 1][lane])));
      s_e[w][lane] = sm.u - ek;
    }
    __syncthreads();
    // ---- Y tile w:  Y = qscale X_Q + P E
    {
      f32x4 y = zero4();
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
        y = P::mma(y, sm.pm[jb], P::from_f32(pair_to8(s_e[2 * jb][lane], s_e[2 * jb + 1][lane])));
      const f32x4 xq = s_x[4 + w][lane];
      const int64_t tb = (p.chunk0 + cl) * CH + 16 * w + 4 * (lane >> 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t t = tb + i;
        if (t < p.T) store_y<OutT>((OutT*)p.y + b * p.ys0 + t * p.ys1 + h * p.ys2 + r, y[i] + sm.qs[i] * xq[i]);
      }
    }
    // ---- state update on this wave's feature tiles:  S^T = gammaC S^T + K^T (kscale o E)
    frag eb[2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
      eb[jb] = P::from_f32(pair_to8(s_e[2 * jb][lane] * sm.ks[2 * jb], s_e[2 * jb + 1][lane] * sm.ks[2 * jb + 1]));
#pragma unroll
    for (int tl = 0; tl < TPW; ++tl) {
      f32x4 acc = S[tl] * sm.gC;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        if constexpr (PF) acc = P::mma(acc, au[tl][jb], eb[jb]);
        else acc = P::mma(acc, O::load_u1(wsc, w, lane, tl, jb), eb[jb]);
      }
      S[tl] = acc;
    }
    if constexpr (PF) {
      if (more) {
#pragma unroll
        for (int tl = 0; tl < TPW; ++tl) { au[tl][0] = au_n[tl][0]; au[tl][1] = au_n[tl][1]; }
        sm = sm_n;
      }
    }
  }

#pragma unroll
  for (int tl = 0; tl < TPW; ++tl) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t d = 16 * (TPW * w + tl) + 4 * (lane >> 4) + i;
      p.state_out[b * p.os0 + h * p.os1 + d * p.os2 + r * p.os3] = S[tl][i];
    }
  }
}

static inline unsigned scan_grid(int64_t B, int64_t H, int nv) { return (unsigned)(8 * ((B * H + 7) / 8) * nv); }

// ------------------------------------------------------------------------------------------------
enum Phase { PHASE_PREP = 1, PHASE_STATE = 2, PHASE_BOTH = 3 };

static ScanParams fill_params(const kdn_scan_args* a) {
  ScanParams p;
  p.B = a->B; p.T = a->T; p.H = a->H;
  p.q = a->q; p.qs0 = a->q_stride[0]; p.qs1 = a->q_stride[1]; p.qs2 = a->q_stride[2];
  p.k = a->k; p.ks0 = a->k_stride[0]; p.ks1 = a->k_stride[1]; p.ks2 = a->k_stride[2];
  p.v = a->v; p.vs0 = a->v_stride[0]; p.vs1 = a->v_stride[1]; p.vs2 = a->v_stride[2];
  p.beta = a->beta; p.bs0 = a->beta_stride[0]; p.bs1 = a->beta_stride[1]; p.bs2 = a->beta_stride[2];
  p.decay = a->decay; p.ds0 = a->decay_stride[0]; p.ds1 = a->decay_stride[1]; p.ds2 = a->decay_stride[2];
  p.omega = (const __bf16*)a->omega_bf16; p.phase = a->phase;
  p.inv_tau = a->inv_tau; p.normalize = a->normalize_input ? 1 : 0;
  p.state_out = a->final_state;
  p.os0 = a->final_stride[0]; p.os1 = a->final_stride[1]; p.os2 = a->final_stride[2]; p.os3 = a->final_stride[3];
  p.y = a->y; p.ys0 = a->y_stride[0]; p.ys1 = a->y_stride[1]; p.ys2 = a->y_stride[2];
  p.ws = (unsigned char*)a->workspace;
  return p;
}

// Runs chunks [c_begin, c_end) in segments of `seg` chunks: per segment the prep and/or state kernel.
// The state kernel of the segment starting at chunk 0 reads initial_state (zeros if NULL); later
// segments continue from final_state.
template <class P, typename InT, typename OutT, int D, int DV>
static int run_scan(const kdn_scan_args* a, int64_t c_begin, int64_t c_end, int64_t seg, int phases, hipStream_t st) {
  ScanParams p = fill_params(a);
  for (int64_t c0 = c_begin; c0 < c_end; c0 += seg) {
    p.chunk0 = c0;
    p.nseg = (c_end - c0 < seg) ? (c_end - c0) : seg;
    if (c0 == 0) {
      p.state_in = a->initial_state;
      p.is0 = a->init_stride[0]; p.is1 = a->init_stride[1]; p.is2 = a->init_stride[2]; p.is3 = a->init_stride[3];
    } else {
      p.state_in = a->final_state;
      p.is0 = p.os0; p.is1 = p.os1; p.is2 = p.os2; p.is3 = p.os3;
    }
    if (phases & PHASE_PREP) {
      hipLaunchKernelGGL((prep_kernel<P, InT, D, DV>), dim3((unsigned)p.nseg, (unsigned)p.H, (unsigned)p.B), dim3(256), 0, st, p);
      if (hipGetLastError() != hipSuccess) return KDN_ERR_DEVICE;
    }
    if (phases & PHASE_STATE) {
      hipLaunchKernelGGL((scan_kernel<P, OutT, D, DV>), dim3(scan_grid(p.B, p.H, DV / 16)), dim3(64 * SCAN_WAVES), 0, st, p);
      if (hipGetLastError() != hipSuccess) return KDN_ERR_DEVICE;
    }
  }
  return KDN_OK;
}

template <class P, typename InT, typename OutT, int D>
static int dispatch_dv(const kdn_scan_args* a, int64_t c_begin, int64_t c_end, int64_t seg, int phases, hipStream_t st) {
  switch (a->d_v) {
    case 16: return run_scan<P, InT, OutT, D, 16>(a, c_begin, c_end, seg, phases, st);
    case 32: return run_scan<P, InT, OutT, D, 32>(a, c_begin, c_end, seg, phases, st);
    case 64: return run_scan<P, InT, OutT, D, 64>(a, c_begin, c_end, seg, phases, st);
    case 128: return run_scan<P, InT, OutT, D, 128>(a, c_begin, c_end, seg, phases, st);
    default: return KDN_ERR_UNSUPPORTED;
  }
}

static int dispatch(const kdn_scan_args* a, int64_t c_begin, int64_t c_end, int64_t seg, int phases, hipStream_t st) {
  if (a->in_dtype == KDN_DTYPE_BF16) {
    if (a->out_dtype == KDN_DTYPE_BF16) return dispatch_dv<PrecBF16, __bf16, __bf16, 512>(a, c_begin, c_end, seg, phases, st);
    return dispatch_dv<PrecBF16, __bf16, float, 512>(a, c_begin, c_end, seg, phases, st);
  }
  if (a->out_dtype == KDN_DTYPE_BF16) return dispatch_dv<PrecF32, float, __bf16, 512>(a, c_begin, c_end, seg, phases, st);
  return dispatch_dv<PrecF32, float, float, 512>(a, c_begin, c_end, seg, phases, st);
}

static size_t chunk_bytes(const kdn_scan_args* a) {
  const bool f32 = a->in_dtype == KDN_DTYPE_F32;
  switch (a->d_v) {
#define KDN_CB(DVV) \
  case DVV: return f32 ? WsLayout<PrecF32, 512, DVV>::bytes : WsLayout<PrecBF16, 512, DVV>::bytes;
    KDN_CB(16) KDN_CB(32) KDN_CB(64) KDN_CB(128)
#undef KDN_CB
    default: return 0;
  }
}

// Default segment: enough chunks that the workspace stays near 1 GiB.
static int64_t choose_segment(const kdn_scan_args* a) {
  const int64_t nchunks = (a->T + CH - 1) / CH;
  if (a->segment_chunks > 0) return a->segment_chunks < nchunks ? a->segment_chunks : nchunks;
  const size_t per_step = chunk_bytes(a) * (size_t)a->B * (size_t)a->H;
  int64_t seg = (int64_t)(((size_t)1 << 30) / (per_step ? per_step : 1));
  if (seg < 1) seg = 1;
  return seg < nchunks ? seg : nchunks;
}

static int validate(const kdn_scan_args* a) {
  if (!a) return KDN_ERR_INVALID_ARGUMENT;
  if (a->B <= 0 || a->T <= 0 || a->H <= 0) return KDN_ERR_INVALID_ARGUMENT;
  if (a->B > 65535 || a->H > 65535) return KDN_ERR_UNSUPPORTED;
  if (!valid_dtype(a->in_dtype) || !valid_dtype(a->out_dtype)) return KDN_ERR_INVALID_ARGUMENT;
  if (a->d_k != 64 || a->D != 512) return KDN_ERR_UNSUPPORTED;
  if (a->d_v != 16 && a->d_v != 32 && a->d_v != 64 && a->d_v != 128) return KDN_ERR_UNSUPPORTED;
  if (a->segment_chunks < 0) return KDN_ERR_INVALID_ARGUMENT;
  if (!(a->inv_tau == a->inv_tau)) return KDN_ERR_INVALID_ARGUMENT;
  return KDN_OK;
}

}  // namespace kdn

using namespace kdn;

extern "C" size_t kdn_scan_workspace_bytes(const kdn_scan_args* a) {
  if (validate(a) != KDN_OK) return 0;
  const int64_t seg = choose_segment(a);
  return chunk_bytes(a) * (size_t)a->B * (size_t)a->H * (size_t)seg;
}

// Pointer, stride and alignment checks shared by the launching entry points.
static int validate_launch(const kdn_scan_args* a) {
  int rc = validate(a);
  if (rc != KDN_OK) return rc;
  if (!a->q || !a->k || !a->v || !a->beta || !a->omega_bf16 || !a->phase || !a->final_state || !a->y || !a->workspace)
    return KDN_ERR_INVALID_ARGUMENT;
  // 16-byte row loads of q, k, v; 16-byte fragment traffic in the workspace.
  const size_t isz = dtype_size(a->in_dtype);
  if (!aligned(a->q, 16) || !aligned(a->k, 16) || !aligned(a->v, 16) || !aligned(a->omega_bf16, 16) ||
      !aligned(a->phase, 16) || !aligned(a->workspace, 256))
    return KDN_ERR_MISALIGNED;
  for (int i = 0; i < 3; ++i) {
    if (((a->q_stride[i] * (int64_t)isz) % 16) != 0 || ((a->k_stride[i] * (int64_t)isz) % 16) != 0 ||
        ((a->v_stride[i] * (int64_t)isz) % 16) != 0)
      return KDN_ERR_MISALIGNED;
  }
  return KDN_OK;
}

extern "C" int kdn_delta_scan_fwd(const kdn_scan_args* a, void* stream) {
  int rc = validate_launch(a);
  if (rc != KDN_OK) return rc;
  const int64_t seg = choose_segment(a);
  const size_t need = chunk_bytes(a) * (size_t)a->B * (size_t)a->H * (size_t)seg;
  if (a->workspace_bytes < need) return KDN_ERR_WORKSPACE_TOO_SMALL;
  const int64_t nchunks = (a->T + CH - 1) / CH;
  return dispatch(a, 0, nchunks, seg, PHASE_BOTH, as_stream(stream));
}

static int run_phase(const kdn_scan_args* a, int64_t chunk0, int64_t nchunks, int phase, void* stream) {
  int rc = validate_launch(a);
  if (rc != KDN_OK) return rc;
  const int64_t total = (a->T + CH - 1) / CH;
  if (chunk0 < 0 || nchunks < 1 || chunk0 + nchunks > total) return KDN_ERR_INVALID_ARGUMENT;
  const size_t need = chunk_bytes(a) * (size_t)a->B * (size_t)a->H * (size_t)nchunks;
  if (a->workspace_bytes < need) return KDN_ERR_WORKSPACE_TOO_SMALL;
  return dispatch(a, chunk0, chunk0 + nchunks, nchunks, phase, as_stream(stream));
}

extern "C" int kdn_scan_prep(const kdn_scan_args* a, int64_t chunk0, int64_t nchunks, void* stream) {
  return run_phase(a, chunk0, nchunks, PHASE_PREP, stream);
}

extern "C" int kdn_scan_state(const kdn_scan_args* a, int64_t chunk0, int64_t nchunks, void* stream) {
  return run_phase(a, chunk0, nchunks, PHASE_STATE, stream);
}
