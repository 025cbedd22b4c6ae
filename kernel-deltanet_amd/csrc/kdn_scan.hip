// Chunked gated delta-rule prefill scan of Kernel-DeltaNet on gfx950.
//
// Recurrence (readout before update; tests/test_fused_kernel.py:53-65 of the reference):
//   y_t = S_{t-1} phi_q(t),    S_t = lambda_t S_{t-1} (I - beta_t phi_k(t) phi_k(t)^T) + beta_t v_t phi_k(t)^T
// with S (d_v x D) carried in fp32.  Per 64-token chunk, with g = cumsum(log lambda) inside the chunk
// and K, Q the lifted keys/queries of the chunk (rows), the WY/UT form used here is
//   A[t][j]  = beta_t e^{g_t - g_j} (K K^T)[t][j]                       (j < t)
//   T        = (I + A)^{-1}                                              (unit lower triangular)
//   U~       = T diag(beta) V,       W~ = T diag(beta e^{g}) K
//   E        = U~ - W~ S^T           (the per-token errors beta_t (v_t - lambda_t S_{t-1} k_t))
//   Y        = diag(e^{g_{t-1}}) Q S^T + P E,   P[t][j] = e^{g_{t-1} - g_j} (Q K^T)[t][j]   (j < t)
//   S_next   = e^{g_63} S + E^T diag(e^{g_63 - g}) K
// which is algebraically the scan of kernels/fused_kernel_deltanet.py:93-149 (that code factors the
// decay-free homogeneous part through an upper-triangular resolvent; both equal the token recurrence).
//
// Three kernels per segment of chunks, so that the only sequential kernel streams as few bytes per
// chunk as possible (64 KB of K per chunk and head):
//   prep   (one workgroup per chunk and head): lift q and k on MFMA, Gram matrices, the triangular
//          inverse and every S-independent factor; writes K, Tp = T diag(beta e^g |phi_k|), P, U~ and
//          per-token scale vectors to the workspace in MFMA-fragment order.
//   state  (one workgroup per head and 16 value components, sequential over chunks): X_K = K S^T,
//          E = U~ - Tp X_K and the state update; checkpoints each chunk's starting S^T and E.
//   output (one workgroup per chunk and head): re-lifts q, Y = diag(qscale) Q S^T + P E.
// The lifted features are stored unnormalised (cos values); per-row norms are folded into the small
// per-token scale vectors, so a lift never has to hold a whole row before using it.
#include <type_traits>
#include "kdn_frag.hpp"
#include "kdn_internal.hpp"
#include "kdn_io.hpp"

namespace kdn {

constexpr int CH = 64;  // tokens per chunk (internal; the WY form is exact for any chunk length)

// Per (chunk, head) workspace record.  A segment of nseg chunks uses nseg + 1 records per head: the
// last one is scratch for the state kernel's writes past the final chunk.
template <class P, int D, int DV>
struct WsLayout {
  static constexpr size_t FB = P::frag_bytes;
  static constexpr int NJ = D / 32;   // 32-deep blocks over features
  static constexpr int NV = DV / 16;  // 16-wide value tiles
  static constexpr size_t phiK = 0;                                 // [m 4][j NJ][lane] K row frags (cos)
  static constexpr size_t Tp = phiK + (size_t)4 * NJ * 64 * FB;     // [m 4][jb 2][lane]  T diag(beta e^g s_k)
  static constexpr size_t Pm = Tp + (size_t)4 * 2 * 64 * FB;        // [m 4][jb 2][lane]  P
  static constexpr size_t U = Pm + (size_t)4 * 2 * 64 * FB;         // [m 4][n NV][lane] f32x4  U~
  static constexpr size_t VEC = U + (size_t)4 * NV * 64 * 16;       // qscale[64] kscale[64] gammaC
  static constexpr size_t Sfr = VEC + 1024;                         // [j NJ][n NV][lane] chunk-start S^T frags
  static constexpr size_t Eck = Sfr + (size_t)NJ * NV * 64 * FB;    // [m 4][n NV][lane] f32x4  E
  static constexpr size_t phiQ = Eck + (size_t)4 * NV * 64 * 16;    // [m 4][j NJ][lane] Q row frags (cos)
  static constexpr size_t bytes = (phiQ + (size_t)4 * NJ * 64 * FB + 255) / 256 * 256;
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
  int prep_run;          // chunks per prep workgroup (bf16)
  // feature map: per-head Omega (hi [+ lo]) / phases / 1/tau, renormalisation, pre-lifted inputs
  const __bf16* omega_lo; int64_t oms, phs;
  const float* inv_tau_head;
  int no_renorm, prelifted;
  int linear;  // update rule without the erasure term: T = I, Tp = 0
  // ragged batches: sequence b is token rows seq_lo[b] .. seq_hi[b] (stride 1 of each token tensor; for
  // cu_seqlens, seq_hi = cu_seqlens + 1); its state is slot slots[b] (stride 0 of the state tensors)
  const int64_t* seq_lo;
  const int64_t* seq_hi;
  const int* slots;
};

// Sequence b of the batch: element offsets of its first token in each token-indexed tensor, and its
// length.  A uniform batch addresses b * stride0 and has T tokens per sequence; a ragged batch
// addresses rows seq_lo[b] .. seq_hi[b] of one packed token dimension.
struct Seq {
  int64_t q, k, v, be, de, y, len;
};
__device__ __forceinline__ Seq seq_of(const ScanParams& p, int64_t b) {
  Seq s;
  if (p.seq_lo) {
    const int64_t r0 = p.seq_lo[b];
    s.q = r0 * p.qs1; s.k = r0 * p.ks1; s.v = r0 * p.vs1;
    s.be = r0 * p.bs1; s.de = r0 * p.ds1; s.y = r0 * p.ys1;
    s.len = p.seq_hi[b] - r0;
  } else {
    s.q = b * p.qs0; s.k = b * p.ks0; s.v = b * p.vs0;
    s.be = b * p.bs0; s.de = b * p.ds0; s.y = b * p.ys0;
    s.len = p.T;
  }
  return s;
}
// Chunks of the current segment that hold tokens of the sequence (0 once it has ended).
__device__ __forceinline__ int64_t seg_chunks(const ScanParams& p, const Seq& s) {
  const int64_t n = (s.len + CH - 1) / CH - p.chunk0;
  return n <= 0 ? 0 : (n < p.nseg ? n : p.nseg);
}

// Feature modes of the prep kernel: Omega exact in bf16 (the structured projection), Omega as hi + lo
// bf16 parts (general projections), or q / k already lifted (d_k = D).
enum FeatureMode { FM_EXACT = 0, FM_HILO = 1, FM_PRELIFTED = 2 };

template <class P>
struct IsBF16 : std::integral_constant<bool, std::is_same<P, PrecBF16>::value> {};

// ------------------------------------------------------------------------------------------------
// Raw 16-byte pieces of one lane's part of an input row (8 elements per 32-deep block kb): 1 piece per
// block for bf16, 2 for fp32.
template <typename InT>
struct RawRow {
  static constexpr int R = (int)(8 * sizeof(InT) / 16);
  u32x4 piece[2 * R];
  __device__ __forceinline__ void load(const InT* row, bool valid, int lane) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        u32x4 z = {0u, 0u, 0u, 0u};
        piece[kb * R + r] = valid ? reinterpret_cast<const u32x4*>(row + 32 * kb + 8 * (lane >> 4))[r] : z;
      }
  }
  __device__ __forceinline__ void to_f32(int kb, float* o) const {
    if constexpr (R == 1) {
      const bf16x8 v = __builtin_bit_cast(bf16x8, piece[kb]);
#pragma unroll
      for (int s = 0; s < 8; ++s) o[s] = (float)v[s];
    } else {
      const f32x4 a = __builtin_bit_cast(f32x4, piece[kb * 2]), c = __builtin_bit_cast(f32x4, piece[kb * 2 + 1]);
      o[0] = a[0]; o[1] = a[1]; o[2] = a[2]; o[3] = a[3];
      o[4] = c[0]; o[5] = c[1]; o[6] = c[2]; o[7] = c[3];
    }
  }
};

// Lift of one 16-row tile per wave, for NX inputs at once (each Omega fragment feeds NX MFMAs).
// Projection in the transposed orientation Phi^T = Omega X^T: accumulator tile t holds, in lane l,
// feature 16t + 4(l>>4) + i of row (l & 15), which is slot (t & 1) * 4 + i of X fragment t / 2.
// The angle in revolutions is reduced with v_fract before v_cos (which takes revolutions), so any
// finite angle stays inside the instruction's domain.
// Output: unnormalised cos values as X fragments, and each row's sum of squares (all lanes).
template <class P, typename InT, int D, bool OMEGA_LDS, int NX, bool LO = false>
__device__ __forceinline__ void lift_tile(const RawRow<InT> (&raw)[NX], int normalize,
                                          const bf16x8* s_omega, const __bf16* omega, const float* s_phrev,
                                          float ang, int lane, typename P::frag (&out)[NX][D / 32],
                                          float (&ss)[NX], const __bf16* omega_lo = nullptr) {
  constexpr int NT = D / 16;
  constexpr int NSPLIT = XFrag<InT>::NSPLIT;
  float xv[NX][2][8];
#pragma unroll
  for (int x = 0; x < NX; ++x)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) raw[x].to_f32(kb, xv[x][kb]);
  if (normalize) {
#pragma unroll
    for (int x = 0; x < NX; ++x) {
      float sq = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int s = 0; s < 8; ++s) sq += xv[x][kb][s] * xv[x][kb][s];
      sq = sum_over_lane_groups(sq);
      const float inv = 1.0f / fmaxf(sqrtf(sq), 1e-6f);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const float a = xv[x][kb][s] * inv;
          xv[x][kb][s] = (NSPLIT == 1) ? (float)(__bf16)a : a;  // F.normalize output keeps x's dtype
        }
    }
  }
  bf16x8 xb[NX][2][NSPLIT];
#pragma unroll
  for (int x = 0; x < NX; ++x) {
    split_frag<NSPLIT>(xv[x][0], xb[x][0]);
    split_frag<NSPLIT>(xv[x][1], xb[x][1]);
    ss[x] = 0.f;
  }
  // Feature tile t: acc[x] = x . Omega[16t .. 16t+16)^T.  Software-pipelined: the MFMAs of tile t+1 are
  // issued in the scheduling region of the cosines of tile t.
  auto project = [&](int t, f32x4 (&acc)[NX]) {
#pragma unroll
    for (int x = 0; x < NX; ++x) acc[x] = zero4();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      bf16x8 a;
      if constexpr (OMEGA_LDS) a = s_omega[(t * 2 + kb) * 64 + lane];
      else a = *reinterpret_cast<const bf16x8*>(omega + (int64_t)(16 * t + (lane & 15)) * 64 + 32 * kb + 8 * (lane >> 4));
#pragma unroll
      for (int s = 0; s < NSPLIT; ++s)
#pragma unroll
        for (int x = 0; x < NX; ++x) acc[x] = PrecBF16::mma(acc[x], a, xb[x][kb][s]);
      if constexpr (LO) {
        const bf16x8 alo = *reinterpret_cast<const bf16x8*>(omega_lo + (int64_t)(16 * t + (lane & 15)) * 64 + 32 * kb + 8 * (lane >> 4));
#pragma unroll
        for (int s = 0; s < NSPLIT; ++s)
#pragma unroll
          for (int x = 0; x < NX; ++x) acc[x] = PrecBF16::mma(acc[x], alo, xb[x][kb][s]);
      }
    }
  };
  f32x4 acc[NX];
  project(0, acc);
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    // one feature tile per scheduling region: hoisting the Omega reads of every tile to the top
    // would hold them all in registers at once
    __builtin_amdgcn_sched_barrier(0);
    f32x4 next[NX];
    if (t + 1 < NT) project(t + 1, next);
    const f32x4 ph = *reinterpret_cast<const f32x4*>(&s_phrev[16 * t + 4 * (lane >> 4)]);
#pragma unroll
    for (int x = 0; x < NX; ++x)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float c = __builtin_amdgcn_cosf(__builtin_amdgcn_fractf(acc[x][i] * ang + ph[i]));
        ss[x] += c * c;
        P::set(out[x][t >> 1], (t & 1) * 4 + i, c);
      }
    if (t + 1 < NT) {
#pragma unroll
      for (int x = 0; x < NX; ++x) acc[x] = next[x];
    }
  }
#pragma unroll
  for (int x = 0; x < NX; ++x) ss[x] = sum_over_lane_groups(ss[x]);
}

// Omega as A fragments in LDS (lane l of fragment (t, kb): Omega[16t + (l&15)][32kb + 8(l>>4) .. +8])
// and phase / (2 pi).
template <int D, bool OMEGA_LDS>
__device__ __forceinline__ void stage_omega(const __bf16* omega, const float* phase, bf16x8* s_omega, float* s_phrev) {
  if constexpr (OMEGA_LDS) {
    for (int idx = threadIdx.x; idx < (D / 16) * 2 * 64; idx += blockDim.x) {
      const int l = idx & 63, tk = idx >> 6, t = tk >> 1, kb = tk & 1;
      s_omega[idx] = *reinterpret_cast<const bf16x8*>(omega + (int64_t)(16 * t + (l & 15)) * 64 + 32 * kb + 8 * (l >> 4));
    }
  }
  for (int f = threadIdx.x; f < D; f += blockDim.x) s_phrev[f] = phase[f] * 0.15915494309189535f;
}

// ------------------------------------------------------------------------------------------------
// prep: grid (ceil(nseg / run), H, B), 256 threads.  A workgroup prepares `run` consecutive chunks
// of one head: Omega and the phases are staged in LDS once, and the raw q / k / v / beta / decay of the
// next chunk are loaded into registers while the current chunk is processed.  Wave w owns token rows
// [16w, 16w+16) of a chunk.
// Chunks per prep workgroup: chosen at launch for bf16 with the exact or given features
// (ScanParams::prep_run); 1 for fp32, whose fragments (twice as wide) leave no registers for the
// prefetch, and for the hi + lo projection, whose second operand stream does the same.
template <class P, int FM>
struct PrepRun : std::integral_constant<int, (IsBF16<P>::value && FM != FM_HILO) ? 0 : 1> {};

// Raw inputs of one chunk for one thread of the prep workgroup: the q / k row pieces of the lane's row
// and beta / decay of token `lane` (prefetched one chunk ahead), and the V pieces of the thread
// (loaded at the start of the chunk; they are first needed after the Gram).
template <typename InT, int DV>
struct PrepInputs {
  static constexpr int VPR = DV * (int)sizeof(InT) / 16;        // 16-byte pieces per V row
  static constexpr int VPT = (64 * VPR + 255) / 256;             // pieces per thread
  RawRow<InT> qk[2];
  float be, la;
  __device__ __forceinline__ void load_qk(const ScanParams& p, const Seq& sq, int64_t h, int64_t t0, int w, int lane) {
    const int64_t trow = t0 + 16 * w + (lane & 15);
    const bool rvalid = trow < sq.len;
    qk[0].load((const InT*)p.q + sq.q + trow * p.qs1 + h * p.qs2, rvalid, lane);
    qk[1].load((const InT*)p.k + sq.k + trow * p.ks1 + h * p.ks2, rvalid, lane);
    const int64_t t = t0 + lane;
    const bool valid = t < sq.len;
    be = valid ? p.beta[sq.be + t * p.bs1 + h * p.bs2] : 0.f;
    la = (valid && p.decay) ? p.decay[sq.de + t * p.ds1 + h * p.ds2] : 1.f;
  }
  __device__ __forceinline__ static void load_v(const ScanParams& p, const Seq& sq, int64_t h, int64_t t0, u32x4 (&v)[VPT]) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int idx = (int)threadIdx.x + 256 * i;
      const int r = idx / VPR, pc = idx % VPR;
      const int64_t t = t0 + r;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (idx < 64 * VPR && t < sq.len)
        val = *reinterpret_cast<const u32x4*>((const InT*)p.v + sq.v + t * p.vs1 + h * p.vs2 + pc * (16 / (int)sizeof(InT)));
      v[i] = val;
    }
  }
};

// Lifted features given as input (FM_PRELIFTED): X fragment j of the lane's row, features 32j + kappa(l, s)
// (two runs of four: 32j + 4(l>>4) .. +3 and 32j + 16 + 4(l>>4) .. +3).
template <class P, typename InT, int D>
__device__ __forceinline__ void load_lifted(const InT* row, bool valid, int lane, typename P::frag (&out)[D / 32]) {
#pragma unroll
  for (int j = 0; j < D / 32; ++j) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const InT* src = row + 32 * j + 16 * half + 4 * (lane >> 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) P::set(out[j], 4 * half + i, valid ? (float)src[i] : 0.f);
    }
  }
}

template <class P, typename InT, int D, int DV, int FM>
__global__ void __launch_bounds__(256) prep_kernel(ScanParams p) {
  using L = WsLayout<P, D, DV>;
  using frag = typename P::frag;
  using In = PrepInputs<InT, DV>;
  constexpr int NT = D / 16, NJ = D / 32, NV = DV / 16;
  constexpr bool OMEGA_LDS = IsBF16<P>::value && FM != FM_PRELIFTED;
  constexpr size_t OMEGA_BYTES = OMEGA_LDS ? (size_t)NT * 2 * 64 * 16 : 0;
  constexpr size_t PHIK_BYTES = (size_t)4 * NJ * 64 * sizeof(frag);
  // After the Gram the K-fragment area is reused for A (16 KB), T (17 KB) and V.
  static_assert(64 * 64 * 4 + 64 * 68 * 4 + 64 * DV * sizeof(InT) <= PHIK_BYTES, "LDS reuse does not fit");
  __shared__ __attribute__((aligned(16))) unsigned char smem[OMEGA_BYTES + PHIK_BYTES];
  __shared__ __attribute__((aligned(16))) float s_beta[64], s_g[64], s_sq[64], s_sk[64], s_phrev[D];

  bf16x8* s_omega = reinterpret_cast<bf16x8*>(smem);
  frag* s_phik = reinterpret_cast<frag*>(smem + OMEGA_BYTES);
  float* s_A = reinterpret_cast<float*>(smem + OMEGA_BYTES);          // [j][p][s] = A[4s+p][j]
  float* s_T = s_A + 64 * 64;                                          // [t][68]
  InT* s_V = reinterpret_cast<InT*>(s_T + 64 * 68);                    // [t][DV]

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t h = blockIdx.y, b = blockIdx.z;
  constexpr int RUN = PrepRun<P, FM>::value;  // 0: runtime run length with prefetch
  const int run = RUN ? RUN : p.prep_run;
  const int64_t cl0 = (int64_t)blockIdx.x * run;
  const Seq sq = seq_of(p, b);
  const int64_t nloc = seg_chunks(p, sq);
  if (cl0 >= nloc) return;  // past the end of this sequence (ragged batches): nothing to prepare
  const int64_t cl_end = (cl0 + run < nloc) ? cl0 + run : nloc;

  const __bf16* omega_h = p.omega + h * p.oms;
  const __bf16* omega_lo_h = (FM == FM_HILO) ? p.omega_lo + h * p.oms : nullptr;
  const float ang = (p.inv_tau_head ? p.inv_tau_head[h] : p.inv_tau) * 0.15915494309189535f;
  In in;
  if constexpr (FM != FM_PRELIFTED) {
    stage_omega<D, OMEGA_LDS>(omega_h, p.phase + h * p.phs, s_omega, s_phrev);
    in.load_qk(p, sq, h, (p.chunk0 + cl0) * CH, w, lane);
  } else {
    // no lift: only beta / decay come through the prefetch
    const int64_t t = (p.chunk0 + cl0) * CH + lane;
    const bool valid = t < sq.len;
    in.be = valid ? p.beta[sq.be + t * p.bs1 + h * p.bs2] : 0.f;
    in.la = (valid && p.decay) ? p.decay[sq.de + t * p.ds1 + h * p.ds2] : 1.f;
  }

  auto process = [&](int64_t cl) {
    const int64_t t0 = (p.chunk0 + cl) * CH;
    unsigned char* ws = p.ws + ((b * p.H + h) * (p.nseg + 1) + cl) * L::bytes;
    u32x4 vraw[In::VPT];
    if constexpr (RUN != 1) In::load_v(p, sq, h, t0, vraw);  // early: first needed after the Gram
    __syncthreads();  // Omega staged (first chunk); the previous chunk's LDS reads are done

    // ---- beta and the in-chunk log-decay prefix (wave 0)
    if (w == 0) {
      float g = logf(fminf(fmaxf(in.la, 1e-5f), 1.f));
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float o = __shfl_up(g, off);
        if (lane >= off) g += o;
      }
      s_beta[lane] = in.be;
      s_g[lane] = g;
    }

    // ---- lift q and k rows of this wave (or load the given features)
    frag cqk[2][NJ];  // [0] = q, [1] = k; X fragments (m = w, j): row 16w + (l&15), feature 32j + kappa(l, s)
    float ss[2] = {0.f, 0.f};
    if constexpr (FM == FM_PRELIFTED) {
      const int64_t trow = t0 + 16 * w + (lane & 15);
      load_lifted<P, InT, D>((const InT*)p.q + sq.q + trow * p.qs1 + h * p.qs2, trow < sq.len, lane, cqk[0]);
      load_lifted<P, InT, D>((const InT*)p.k + sq.k + trow * p.ks1 + h * p.ks2, trow < sq.len, lane, cqk[1]);
      const int64_t tn = (p.chunk0 + ((cl + 1 < cl_end) ? cl + 1 : cl)) * CH + lane;
      in.be = (tn < sq.len) ? p.beta[sq.be + tn * p.bs1 + h * p.bs2] : 0.f;
      in.la = (tn < sq.len && p.decay) ? p.decay[sq.de + tn * p.ds1 + h * p.ds2] : 1.f;
    } else {
      lift_tile<P, InT, D, OMEGA_LDS, 2, FM == FM_HILO>(in.qk, p.normalize, s_omega, omega_h, s_phrev, ang, lane,
                                                         cqk, ss, omega_lo_h);
      // the next chunk's rows travel while this one is processed (clamped: the last chunk reloads itself)
      if constexpr (RUN != 1) in.load_qk(p, sq, h, (p.chunk0 + ((cl + 1 < cl_end) ? cl + 1 : cl)) * CH, w, lane);
    }
    {
      // per-row scale of the stored (unnormalised) features: 1 for given features, sqrt(2/D) without
      // renormalisation, sqrt(2/D) / (||sqrt(2/D) c|| + 1e-8) with it
      const float amp = sqrtf(2.0f / (float)D);
      if (lane < 16) {
        float sq_, sk_;
        if constexpr (FM == FM_PRELIFTED) {
          sq_ = 1.f; sk_ = 1.f;
        } else if (p.no_renorm) {
          sq_ = amp; sk_ = amp;
        } else {
          sq_ = amp / (amp * sqrtf(ss[0]) + 1e-8f);
          sk_ = amp / (amp * sqrtf(ss[1]) + 1e-8f);
        }
        s_sq[16 * w + lane] = sq_;
        s_sk[16 * w + lane] = sk_;
      }
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      // The records are read back by the state and output kernels a segment or more later, long after
      // they could still sit in L2: streaming stores keep them from evicting the state kernel's lines.
      store_frag_nt<P>(ws + L::phiK + (size_t)(w * NJ + j) * 64 * L::FB, lane, cqk[1][j]);
      store_frag_nt<P>(ws + L::phiQ + (size_t)(w * NJ + j) * 64 * L::FB, lane, cqk[0][j]);
      s_phik[(w * NJ + j) * 64 + lane] = cqk[1][j];
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
        gkk[m] = P::mma(gkk[m], a, cqk[1][j]);
        gqk[m] = P::mma(gqk[m], a, cqk[0][j]);
      }
    }
    __syncthreads();  // K fragments in LDS are dead from here on

    // ---- A (for the inverse), P fragments, V staging, scale vectors
    {
      const int t = 16 * w + (lane & 15);
      // the linear rule has no erasure coupling: A = 0, so T = I below
      const float bt = p.linear ? 0.f : s_beta[t], gt = s_g[t], gtm1 = t > 0 ? s_g[t - 1] : 0.f;
      const float skt = s_sk[t], sqt = s_sq[t];
      f32x4 pt[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = 16 * m + 4 * (lane >> 4) + i;
          const float gj = s_g[j], skj = s_sk[j];
          const float a = (j < t) ? bt * __expf(fminf(gt - gj, 0.f)) * gkk[m][i] * skt * skj : 0.f;
          s_A[(j * 4 + (t & 3)) * 16 + (t >> 2)] = a;
          pt[m][i] = (j < t) ? __expf(fminf(gtm1 - gj, 0.f)) * gqk[m][i] * sqt * skj : 0.f;
        }
      }
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
        store_frag_nt<P>(ws + L::Pm + (size_t)(w * 2 + jb) * 64 * L::FB, lane, P::from_f32(pair_to8(pt[2 * jb], pt[2 * jb + 1])));
    }
    if constexpr (RUN == 1) In::load_v(p, sq, h, t0, vraw);
#pragma unroll
    for (int i = 0; i < In::VPT; ++i) {
      const int idx = (int)threadIdx.x + 256 * i;
      if (idx < 64 * In::VPR) *reinterpret_cast<u32x4*>(s_V + (idx / In::VPR) * DV + (idx % In::VPR) * (16 / (int)sizeof(InT))) = vraw[i];
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

    // ---- T = (I + A)^{-1}: column col = 16w + (l>>2) per lane quad; lane p = l&3 keeps rows 4s+p.
    // Column-oriented forward substitution: once row i of the column is final (lane i & 3, slot i >> 2)
    // it is broadcast over the quad and every later row takes its term A[r][i] T[i][col] at once, so
    // the sequential chain per row is one broadcast and one FMA.  acc[s] = -(partial T[4s+p][col]);
    // the entries of A on and above the diagonal are zero, so updating every slot from i >> 2 on leaves
    // rows r <= i unchanged.
    {
      const int col = 16 * w + (lane >> 2), pq = lane & 3;
      float acc[16];
#pragma unroll
      for (int s2 = 0; s2 < 16; ++s2) acc[s2] = (4 * s2 + pq == col) ? -1.f : 0.f;
      // Column i of A for the lane's rows, in 16-byte pieces from piece i >> 4 on (the earlier rows of
      // the column are zero), loaded AHEAD steps before it is used so that no step waits for LDS.
      constexpr int AHEAD = 3;
      f32x4 acol[AHEAD][4];
      auto load_col = [&](int i, f32x4 (&dst)[4]) {
        const f32x4* src = reinterpret_cast<const f32x4*>(s_A + (i * 4 + pq) * 16);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (q >= (i >> 4)) dst[q] = src[q];
      };
#pragma unroll
      for (int i = 0; i < AHEAD; ++i) load_col(i, acol[i]);
#pragma unroll
      for (int i = 0; i < 63; ++i) {
        float bc;  // -T[i][col]
        switch (i & 3) {
          case 0: bc = quad_bcast<0>(acc[i >> 2]); break;
          case 1: bc = quad_bcast<1>(acc[i >> 2]); break;
          case 2: bc = quad_bcast<2>(acc[i >> 2]); break;
          default: bc = quad_bcast<3>(acc[i >> 2]); break;
        }
        const f32x4 (&a)[4] = acol[i % AHEAD];
#pragma unroll
        for (int s2 = i >> 2; s2 < 16; ++s2) acc[s2] = fmaf(-a[s2 >> 2][s2 & 3], bc, acc[s2]);
        if (i + AHEAD < 63) load_col(i + AHEAD, acol[i % AHEAD]);
      }
#pragma unroll
      for (int s2 = 0; s2 < 16; ++s2) s_T[(4 * s2 + pq) * 68 + col] = -acc[s2];
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
          tw[s] = p.linear ? 0.f : tv * s_beta[j] * __expf(s_g[j]) * s_sk[j];  // linear: E = U~
          tb[jb][s] = tv * s_beta[j];
        }
        store_frag_nt<P>(ws + L::Tp + (size_t)(w * 2 + jb) * 64 * L::FB, lane, P::from_f32(tw));
      }
#pragma unroll
      for (int n = 0; n < NV; ++n) {
        f32x4 acc = zero4();
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
          f32x8 vv;
#pragma unroll
          for (int s = 0; s < 8; ++s) vv[s] = (float)s_V[(32 * jb + kappa(lane, s)) * DV + 16 * n + (lane & 15)];
          if constexpr (IsBF16<P>::value) {
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
        __builtin_nontemporal_store(acc, reinterpret_cast<f32x4*>(ws + L::U + ((size_t)(w * NV + n) * 64 + lane) * 16));
      }
    }
  };
  if constexpr (RUN == 1) {
    process(cl0);
  } else {
    for (int64_t cl = cl0; cl < cl_end; ++cl) process(cl);
  }
}

// ------------------------------------------------------------------------------------------------
// state: one workgroup of 4 waves per (head, 16 value components = 16 state rows), sequential over the
// chunks of the segment.  Wave w owns features [128w, 128w + 128) of those rows: S^T tiles (feature
// tile, row tile) in accumulator layout, lane l holds S^T[16tt + 4(l>>4) + i][r0 + (l&15)].  Per chunk:
//   checkpoint the chunk-start S^T (B fragments in the operand precision) for the output kernel
//   X_K partial over the wave's features -> LDS -> barrier -> wave w reduces token tile w -> LDS -> barrier
//   E tile w = U~ - Tp X_K (checkpointed) -> LDS -> barrier
//   S^T <- gammaC S^T + K^T (kscale o E) on the wave's feature tiles, with the K^T operand read back
//   transposed (ds_read_b64_tr_b16) from a wave-private LDS copy of the wave's K fragments.
// Three workgroup barriers per chunk.  bf16: the K fragments and small operands of chunk c+1 are loaded
// at the start of chunk c (a two-slot register ring) while an L2 prefetch runs L2_AHEAD chunks ahead;
// the refill is unconditional (its chunk index is clamped to the segment) so that the compiler's
// memory-counter waits stay static and only wait for the slot that is about to be used.
//
// Workgroups are dispatched round-robin over the 8 XCDs (linear id % 8); the value tiles of one head
// get ids with equal residue so that they share one XCD's L2 for the K fragments they all read.
template <class P, int D, int DV>
struct StateOps {
  using L = WsLayout<P, D, DV>;
  using frag = typename P::frag;
  static constexpr int NJ = D / 32;
  static constexpr int TPW = D / 64;   // feature tiles per wave
  static constexpr int JPW = D / 128;  // 32-deep feature blocks per wave
  static constexpr int NV = DV / 16;
  static constexpr int L2_AHEAD = 3;  // chunks ahead of the current one that the L2 prefetch touches (3 measured best of 1, 3, 6)
  // dword loads per wave that cover the operand area [0, Sfr) of one chunk record at one per line
  static constexpr int L2_LOADS = (int)((L::Sfr / 128 + 4 * NV * 64 - 1) / (4 * NV * 64));
  struct Small {
    frag tp[2];  // Tp fragments of row tile w
    f32x4 u;     // U~ tile (w, n)
    f32x4 ks;    // kscale of the rows of token tile w, accumulator order
    float gC;
  };
  // The operands of one chunk in four parts (token tile m of K plus one small operand each), so that
  // the refill of a slot can be spread over the four barrier-separated phases of a step instead of
  // queueing ~20 KB of loads per wave at once behind the texture unit.
  template <int PART>
  __device__ static void load_part(const unsigned char* ws, int w, int lane, int n, frag (&ak)[4][JPW], Small& sm) {
#pragma unroll
    for (int jj = 0; jj < JPW; ++jj) ak[PART][jj] = load_frag<P>(ws + L::phiK + (size_t)(PART * NJ + JPW * w + jj) * 64 * L::FB, lane);
    if constexpr (PART == 0) {
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) sm.tp[jb] = load_frag<P>(ws + L::Tp + (size_t)(w * 2 + jb) * 64 * L::FB, lane);
    } else if constexpr (PART == 1) {
      sm.u = *reinterpret_cast<const f32x4*>(ws + L::U + ((size_t)(w * NV + n) * 64 + lane) * 16);
    } else if constexpr (PART == 2) {
      sm.ks = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(ws + L::VEC) + 64 + 16 * w + 4 * (lane >> 4));
    } else {
      sm.gC = reinterpret_cast<const float*>(ws + L::VEC)[128];
    }
  }
  __device__ static void load_all(const unsigned char* ws, int w, int lane, int n, frag (&ak)[4][JPW], Small& sm) {
    load_part<0>(ws, w, lane, n, ak, sm);
    load_part<1>(ws, w, lane, n, ak, sm);
    load_part<2>(ws, w, lane, n, ak, sm);
    load_part<3>(ws, w, lane, n, ak, sm);
  }
};

struct StateShared {
  f32x4 xp[4][4][64];  // per-wave partial X_K tiles [wave][token tile][lane]
  f32x4 x[4][64];      // reduced X_K [token tile][lane]
  f32x4 e[4][64];      // E tiles [token tile][lane]
};

// Wave-private LDS copy of the wave's 16 K fragments (token tile m, local 32-feature block jj), from
// which the K^T operand of the state update is read back transposed.
//   bf16: two planes of 8 KB; plane h holds bytes [8h, 8h+8) of every lane's 16-byte fragment slot
//         (features 16h .. 16h+15 of the 32-block) at (fragment * 64 + lane) * 8, so that each
//         transposed read below covers 512 contiguous bytes (no bank conflicts).
//   fp32: fragments in lane order, 32 bytes per lane.
template <class P>
__device__ __forceinline__ void stage_k(typename P::frag* kl, int lane, const typename P::frag (&ak)[4][4]);

template <>
__device__ __forceinline__ void stage_k<PrecBF16>(PrecBF16::frag* kl, int lane, const PrecBF16::frag (&ak)[4][4]) {
  typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
  unsigned char* base = reinterpret_cast<unsigned char*>(kl);
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int fi = m * 4 + jj;
      *reinterpret_cast<bf16x4*>(base + (size_t)(fi * 64 + lane) * 8) = __builtin_shufflevector(ak[m][jj], ak[m][jj], 0, 1, 2, 3);
      *reinterpret_cast<bf16x4*>(base + 8192 + (size_t)(fi * 64 + lane) * 8) =
          __builtin_shufflevector(ak[m][jj], ak[m][jj], 4, 5, 6, 7);
    }
}

template <>
__device__ __forceinline__ void stage_k<PrecF32>(PrecF32::frag* kl, int lane, const PrecF32::frag (&ak)[4][4]) {
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) kl[(m * 4 + jj) * 64 + lane] = ak[m][jj];
}

// K^T operand (wave-local feature tile tl, chunk block jb) from the staged copy:
// lane l slot s = K[32jb + kappa(l,s)][16tl + (l&15)].
template <class P>
__device__ __forceinline__ typename P::frag kt_frag(const typename P::frag* kl, int lane, int tl, int jb);

template <>
__device__ __forceinline__ PrecBF16::frag kt_frag<PrecBF16>(const PrecBF16::frag* kl, int lane, int tl, int jb) {
  // ds_read_b64_tr_b16: in each 16-lane group, output lane i slot v = element (i & 3) of the 8-byte run
  // addressed by lane 4v + (i >> 2).  Source lane (group g, j = l & 15) addresses the 4 features
  // 16tl + 4(j & 3) .. +3 of chunk row c = 32jb + 16 half + 4g + (j >> 2); in X-fragment order that run
  // is half (tl & 1) of fragment (c >> 4, tl >> 1), lane (c & 15) + 16 (j & 3), i.e. plane (tl & 1).
  // The two 4-element halves are combined as whole vectors: building the fragment element by element
  // through scalar bf16 bit casts was miscompiled (every slot took element 0).
  typedef __attribute__((ext_vector_type(4))) short s16x4;
  typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
  const int g = lane >> 4, j = lane & 15;
  const unsigned char* plane = reinterpret_cast<const unsigned char*>(kl) + 8192 * (tl & 1);
  bf16x4 part[2];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int c = 32 * jb + 16 * half + 4 * g + (j >> 2);
    const unsigned char* a = plane + (size_t)(((c >> 4) * 4 + (tl >> 1)) * 64 + (c & 15) + 16 * (j & 3)) * 8;
    part[half] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(a)));
  }
  return __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7);
}

template <>
__device__ __forceinline__ PrecF32::frag kt_frag<PrecF32>(const PrecF32::frag* kl, int lane, int tl, int jb) {
  const float* e = reinterpret_cast<const float*>(kl);
  PrecF32::frag f;
  const int d = 16 * tl + (lane & 15);  // wave-local feature
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const int c = 32 * jb + kappa(lane, s);
    const int fi = (c >> 4) * 4 + (d >> 5);
    f[s] = e[((size_t)fi * 64 + (c & 15) + 16 * ((d >> 2) & 3)) * 8 + 4 * ((d >> 4) & 1) + (d & 3)];
  }
  return f;
}

// The sequential loop is rotated so that one scheduling region (between the third barrier of chunk c
// and the first barrier of chunk c+1) holds the state update of chunk c, the refill loads, the
// checkpoint stores and the X_K product of chunk c+1.  Per CU each chunk moves ~100 KB through the
// texture unit (64 KB of K, the checkpoint and the small operands) at ~64 B/clk, so these memory
// instructions are interleaved one-for-one with the MFMAs of the region (sched_group_barrier) instead
// of being issued in a burst that would block the in-order wave for ~1500 cycles.

// Phase 1 of chunk cl (region ending at barrier A): checkpoint S^T, X_K partial from the K fragments
// in `ak`, stage `ak` for the transposed read, publish the partial.
template <class P, int D, int DV>
__device__ __forceinline__ void state_phase1(StateShared& sh, typename P::frag* kl, unsigned char* cur, int w, int lane,
                                             int n, const f32x4 (&S)[D / 64], const typename P::frag (&ak)[4][D / 128]) {
  using O = StateOps<P, D, DV>;
  using L = typename O::L;
  using frag = typename P::frag;
  constexpr int JPW = O::JPW, NV = O::NV;
  frag sf[JPW];
#pragma unroll
  for (int jj = 0; jj < JPW; ++jj) {
    sf[jj] = P::from_f32(pair_to8(S[2 * jj], S[2 * jj + 1]));
    store_frag<P>(cur + L::Sfr + (size_t)((JPW * w + jj) * NV + n) * 64 * L::FB, lane, sf[jj]);
  }
  f32x4 xp[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    xp[m] = zero4();
#pragma unroll
    for (int jj = 0; jj < JPW; ++jj) xp[m] = P::mma(xp[m], ak[m][jj], sf[jj]);
  }
  stage_k<P>(kl, lane, ak);
#pragma unroll
  for (int m = 0; m < 4; ++m) sh.xp[w][m][lane] = xp[m];
}

// Phase 2 of chunk cl (after barrier A, through barrier C): reduce X_K tile w, E tile w = U~ - Tp X_K
// (checkpointed; shared scaled by kscale).
template <class P, int D, int DV>
__device__ __forceinline__ void state_phase2(StateShared& sh, unsigned char* cur, int w, int lane, int n,
                                             const typename StateOps<P, D, DV>::Small& sm) {
  using O = StateOps<P, D, DV>;
  using L = typename O::L;
  constexpr int NV = O::NV;
  sh.x[w][lane] = sh.xp[0][w][lane] + sh.xp[1][w][lane] + sh.xp[2][w][lane] + sh.xp[3][w][lane];
  __syncthreads();
  f32x4 ek = zero4();
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) ek = P::mma(ek, sm.tp[jb], P::from_f32(pair_to8(sh.x[2 * jb][lane], sh.x[2 * jb + 1][lane])));
  const f32x4 e = sm.u - ek;
  sh.e[w][lane] = e * sm.ks;
  *reinterpret_cast<f32x4*>(cur + L::Eck + ((size_t)(w * NV + n) * 64 + lane) * 16) = e;
  __syncthreads();
}

// Phase 3 of chunk cl: S^T = gammaC S^T + K^T (kscale o E) on the wave's feature tiles.
template <class P, int D, int DV, bool DECAY>
__device__ __forceinline__ void state_phase3(StateShared& sh, const typename P::frag* kl, int lane, f32x4 (&S)[D / 64],
                                             float gC) {
  using frag = typename P::frag;
  constexpr int TPW = D / 64;
  frag eb[2];
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) eb[jb] = P::from_f32(pair_to8(sh.e[2 * jb][lane], sh.e[2 * jb + 1][lane]));
#pragma unroll
  for (int tl = 0; tl < TPW; ++tl) {
    f32x4 acc = S[tl];
    if constexpr (DECAY) acc = acc * gC;  // without decay gammaC is exactly 1
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) acc = P::mma(acc, kt_frag<P>(kl, lane, tl, jb), eb[jb]);
    S[tl] = acc;
  }
}

// L2 prefetch of the operands of chunk cp: the 4 NV waves of a head touch one dword per 128-byte line
// of its K / Tp / P / U~ / scale area.  The dword loaded one iteration earlier is folded into l2acc so
// that the load is kept; it has long completed by then.
template <class P, int D, int DV>
__device__ __forceinline__ void l2_prefetch(const unsigned char* base, int w, int lane, int n, unsigned& slot, unsigned& acc) {
  using O = StateOps<P, D, DV>;
  using L = typename O::L;
  acc += slot;
  unsigned v = 0;
#pragma unroll
  for (int i = 0; i < O::L2_LOADS; ++i) {
    const size_t off = ((size_t)((i * 4 * O::NV + n * 4 + w) * 64 + lane)) * 128;
    if (off < L::Sfr) v += *reinterpret_cast<const unsigned*>(base + off);
  }
  slot = v;
}

// One iteration of the rotated loop for chunk cl, whose operands are in (ak_c, sm_c) and whose K is
// staged in LDS; (ak_n, sm_n) hold chunk cl+1.  Phase 2 and 3 of chunk cl, then -- if cl+1 exists --
// the refill of (ak_c, sm_c) with chunk min(cl+2, last) and phase 1 of chunk cl+1, then barrier A.
template <class P, int D, int DV, bool DECAY>
__device__ __forceinline__ bool state_iter(const ScanParams& p, StateShared& sh, typename P::frag* kl, unsigned char* wsh,
                                           int64_t cl, int w, int lane, int n, f32x4 (&S)[D / 64],
                                           typename P::frag (&ak_c)[4][D / 128], typename StateOps<P, D, DV>::Small& sm_c,
                                           typename P::frag (&ak_n)[4][D / 128], typename StateOps<P, D, DV>::Small& sm_n,
                                           unsigned& l2slot, unsigned& l2acc, int64_t nloc) {
  using O = StateOps<P, D, DV>;
  using L = typename O::L;
  unsigned char* cur = wsh + cl * L::bytes;
  state_phase2<P, D, DV>(sh, cur, w, lane, n, sm_c);
  const float gC = sm_c.gC;
  state_phase3<P, D, DV, DECAY>(sh, kl, lane, S, gC);
  // Unconditional (no branch splits the region): after the last chunk, phase 1 runs on the clamped
  // operands of the last chunk and writes its checkpoint into the record after the last chunk (the
  // spare record nseg of the head, or an unused record of a ragged sequence that ends earlier).
  const int64_t cr = (cl + 2 < nloc) ? cl + 2 : nloc - 1;
  O::load_all(wsh + cr * L::bytes, w, lane, n, ak_c, sm_c);
  const int64_t cp = (cl + 1 + O::L2_AHEAD < nloc) ? cl + 1 + O::L2_AHEAD : nloc - 1;
  l2_prefetch<P, D, DV>(wsh + cp * L::bytes, w, lane, n, l2slot, l2acc);
  state_phase1<P, D, DV>(sh, kl, cur + L::bytes, w, lane, n, S, ak_n);
  // 32 MFMAs (16 update, 16 X_K) and ~26 memory instructions: alternate them.
#pragma unroll
  for (int i = 0; i < 26; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);  // one vector-memory instruction
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);
  __syncthreads();
  return cl + 1 < nloc;
}

template <class P, int D, int DV, bool DECAY>
__global__ void __launch_bounds__(256) state_kernel(ScanParams p) {
  using O = StateOps<P, D, DV>;
  using L = typename O::L;
  using frag = typename P::frag;
  constexpr int TPW = O::TPW, JPW = O::JPW, NV = O::NV;
  __shared__ StateShared sh;
  __shared__ frag s_kl[4][4 * JPW * 64];  // wave-private K fragments

  // XCD-aware decomposition of the 1-D grid: id = xcd + 8 * (rank * NV + n), head-batch pair
  // hb = rank * 8 + xcd.  Ids that land past B*H exit at once.
  const int64_t id = blockIdx.x;
  const int64_t xcd = id & 7, jdx = id >> 3;
  const int n = (int)(jdx % NV);
  const int64_t hb = (jdx / NV) * 8 + xcd;
  if (hb >= p.B * p.H) return;
  const int64_t b = hb / p.H, h = hb % p.H;
  const Seq sq = seq_of(p, b);
  const int64_t nloc = seg_chunks(p, sq);
  // A sequence that ended in an earlier segment has its final state already; one without tokens gets
  // its initial state copied through (below, no chunk is run).
  if (nloc == 0 && !(sq.len <= 0 && p.chunk0 == 0)) return;
  const int64_t sl = p.slots ? (int64_t)p.slots[b] : b;

  const int lane = threadIdx.x & 63;
  // The wave index is uniform across the wave; reading it into a scalar register lets every
  // fragment address be a scalar base plus the per-lane offset.
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = 16 * n + (lane & 15);
  frag* kl = s_kl[w];

  f32x4 S[TPW];
  if (p.state_in) {
    const float* si = p.state_in + sl * p.is0 + h * p.is1 + r * p.is3;
#pragma unroll
    for (int tl = 0; tl < TPW; ++tl)
#pragma unroll
      for (int i = 0; i < 4; ++i) S[tl][i] = si[(int64_t)(16 * (TPW * w + tl) + 4 * (lane >> 4) + i) * p.is2];
  } else {
#pragma unroll
    for (int tl = 0; tl < TPW; ++tl) S[tl] = zero4();
  }

  unsigned char* wsh = p.ws + hb * (p.nseg + 1) * L::bytes;
  frag k0[4][JPW], k1[4][JPW];
  typename O::Small s0, s1;
  unsigned l2acc = 0, l2s0 = 0, l2s1 = 0;  // sink of the L2-prefetch loads (never stored; see below)
  if (nloc > 0) {  // an empty sequence (uniform across the workgroup) runs no chunk
    // Prologue: chunk 0 in slot 0, chunk min(1, last) in slot 1, phase 1 of chunk 0.
    O::load_all(wsh, w, lane, n, k0, s0);
    O::load_all(wsh + (nloc > 1 ? L::bytes : 0), w, lane, n, k1, s1);
    state_phase1<P, D, DV>(sh, kl, wsh, w, lane, n, S, k0);
    __syncthreads();
    for (int64_t cl = 0;; cl += 2) {
      if (!state_iter<P, D, DV, DECAY>(p, sh, kl, wsh, cl, w, lane, n, S, k0, s0, k1, s1, l2s0, l2acc, nloc)) break;
      if (!state_iter<P, D, DV, DECAY>(p, sh, kl, wsh, cl + 1, w, lane, n, S, k1, s1, k0, s0, l2s1, l2acc, nloc)) break;
    }
    l2acc += l2s0 + l2s1;
  }

  float* so = p.state_out + sl * p.os0 + h * p.os1 + r * p.os3;
#pragma unroll
  for (int tl = 0; tl < TPW; ++tl)
#pragma unroll
    for (int i = 0; i < 4; ++i) so[(int64_t)(16 * (TPW * w + tl) + 4 * (lane >> 4) + i) * p.os2] = S[tl][i];
  // Keeps the prefetch loads alive: nseg is at least 1, so this branch never runs.
  if (p.nseg < 0) so[0] = (float)l2acc;
}

// ------------------------------------------------------------------------------------------------
// output: grid (nseg, H, B), 256 threads.  Y = diag(qscale) Q S_c^T + P E for one (chunk, head).
// Wave w keeps the lifted query fragments of token tile w (written by prep) in registers; the
// chunk-start S^T fragments are staged in LDS, NG value tiles per pass, and read by all four waves.
// Each wave assembles its 16 x d_v block of Y in a wave-private LDS tile and writes whole rows with
// 16-byte stores.
template <class P, typename OutT, int D, int DV>
__global__ void __launch_bounds__(256) output_kernel(ScanParams p) {
  using L = WsLayout<P, D, DV>;
  using frag = typename P::frag;
  constexpr int NJ = D / 32, NV = DV / 16;
  constexpr int NG0 = IsBF16<P>::value ? 2 : 1;  // value tiles per LDS pass (32 KB of S fragments)
  constexpr int NG = NV < NG0 ? NV : NG0;
  constexpr int YS = DV + 4;                     // padded row of the Y tile
  __shared__ frag s_s[NJ * NG * 64];
  __shared__ __attribute__((aligned(16))) float s_y[4][16 * YS];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t cl = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const Seq sq = seq_of(p, b);
  if (cl >= seg_chunks(p, sq)) return;  // past the end of this sequence (ragged batches)
  const int64_t t0 = (p.chunk0 + cl) * CH;
  const unsigned char* ws = p.ws + ((b * p.H + h) * (p.nseg + 1) + cl) * L::bytes;
  const float* vec = reinterpret_cast<const float*>(ws + L::VEC);

  frag aq[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) aq[j] = load_frag<P>(ws + L::phiQ + (size_t)(w * NJ + j) * 64 * L::FB, lane);
  frag pf[2];
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) pf[jb] = load_frag<P>(ws + L::Pm + (size_t)(w * 2 + jb) * 64 * L::FB, lane);
  const f32x4 qs = *reinterpret_cast<const f32x4*>(vec + 16 * w + 4 * (lane >> 4));
  float* yt = s_y[w];

  for (int n0 = 0; n0 < NV; n0 += NG) {
    if (n0 > 0) __syncthreads();  // the previous pass's fragments have been read
    for (int idx = threadIdx.x; idx < NJ * NG * 64; idx += 256) {
      const int l = idx & 63, g = (idx >> 6) % NG, j = idx / (64 * NG);
      s_s[idx] = load_frag<P>(ws + L::Sfr + (size_t)(j * NV + n0 + g) * 64 * L::FB, l);
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int n = n0 + g;
      f32x4 xq = zero4();
#pragma unroll
      for (int j = 0; j < NJ; ++j) xq = P::mma(xq, aq[j], s_s[(j * NG + g) * 64 + lane]);
      frag eb[2];
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        const f32x4 e0 = *reinterpret_cast<const f32x4*>(ws + L::Eck + ((size_t)((2 * jb) * NV + n) * 64 + lane) * 16);
        const f32x4 e1 = *reinterpret_cast<const f32x4*>(ws + L::Eck + ((size_t)((2 * jb + 1) * NV + n) * 64 + lane) * 16);
        eb[jb] = P::from_f32(pair_to8(e0, e1));
      }
      f32x4 y = zero4();
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) y = P::mma(y, pf[jb], eb[jb]);
#pragma unroll
      for (int i = 0; i < 4; ++i) yt[(4 * (lane >> 4) + i) * YS + 16 * n + (lane & 15)] = y[i] + qs[i] * xq[i];
    }
  }
  // Rows of the wave's tile: (16 rows) x (DV / 8 pieces of 8 elements); the tile was written by this
  // wave only, and a wave's LDS accesses are performed in order.
  constexpr int PIECES = 16 * (DV / 8);
#pragma unroll
  for (int base = 0; base < PIECES; base += 64) {
    const int idx = base + lane;
    if (idx < PIECES) {
      const int row = idx / (DV / 8), pc = idx % (DV / 8);
      const int64_t t = t0 + 16 * w + row;
      if (t < sq.len) {
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(yt + row * YS + 8 * pc);
        const f32x4 v1 = *reinterpret_cast<const f32x4*>(yt + row * YS + 8 * pc + 4);
        const float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        store_row8<OutT>((OutT*)p.y + sq.y + t * p.ys1 + h * p.ys2 + 8 * pc, v);
      }
    }
  }
}

static inline unsigned state_grid(int64_t B, int64_t H, int nv) { return (unsigned)(8 * ((B * H + 7) / 8) * nv); }

// ------------------------------------------------------------------------------------------------
enum Phase { PHASE_PREP = 1, PHASE_STATE = 2, PHASE_OUTPUT = 4, PHASE_ALL = 7 };

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
  p.omega_lo = (const __bf16*)a->omega_lo;
  p.oms = a->omega_head_stride;
  p.phs = a->phase_head_stride;
  p.inv_tau_head = a->inv_tau_head;
  p.no_renorm = a->no_renorm ? 1 : 0;
  p.prelifted = a->feature_mode == 1 ? 1 : 0;
  p.linear = a->rule == 1 ? 1 : 0;
  p.seq_lo = a->cu_seqlens;
  p.seq_hi = a->cu_seqlens ? a->cu_seqlens + 1 : nullptr;
  p.slots = a->state_slots;
  return p;
}

// Chunks per prep workgroup: each workgroup of the prep kernel holds a CU alone (its LDS), so the
// kernel runs in ceil(workgroups / CUs) rounds, each costing the staging of Omega (about 0.3 of a
// chunk, measured) plus `run` chunks.  Pick the run length (1..8) with the least total for the CUs
// left free (all of them, or those the concurrent state kernel does not occupy).
static int choose_prep_run(int64_t nseg, int64_t heads, int cus) {
  if (cus <= 0) return 4;
  int best = 1;
  int64_t best_cost = INT64_MAX;
  for (int run = 1; run <= 8; ++run) {
    const int64_t wgs = (nseg + run - 1) / run * heads;
    const int64_t cost = (wgs + cus - 1) / cus * (10 * run + 3);
    if (cost < best_cost) { best_cost = cost; best = run; }
  }
  return best;
}

// How the launches of one call are scheduled.
struct RunSpec {
  int64_t c_begin, c_end, seg;
  int phases;
  hipStream_t st;
  hipStream_t aux;   // non-null: pipelined over `nbuf` buffers of `buf_bytes`
  int nbuf;
  size_t buf_bytes;
  hipStream_t aux_out = nullptr;  // non-null and not aux: output kernels on their own stream
  // ragged sequences given as separate start / end arrays (device), overriding cu_seqlens
  const int64_t* seq_lo = nullptr;
  const int64_t* seq_hi = nullptr;
};

// Parameters of one segment: chunks [c0, c0 + nseg) with its records at `ws`.  The state kernel of the
// segment starting at chunk 0 reads initial_state (zeros if NULL); later segments continue from
// final_state.
static ScanParams segment_params(const kdn_scan_args* a, const RunSpec& r, int64_t c0, int64_t nseg, void* ws,
                                 int prep_cus) {
  ScanParams p = fill_params(a);
  if (r.seq_lo) {
    p.seq_lo = r.seq_lo;
    p.seq_hi = r.seq_hi;
  }
  p.chunk0 = c0;
  p.nseg = nseg;
  p.ws = (unsigned char*)ws;
  p.prep_run = choose_prep_run(nseg, a->B * a->H, prep_cus);
  if (c0 == 0) {
    p.state_in = a->initial_state;
    p.is0 = a->init_stride[0]; p.is1 = a->init_stride[1]; p.is2 = a->init_stride[2]; p.is3 = a->init_stride[3];
  } else {
    p.state_in = a->final_state;
    p.is0 = p.os0; p.is1 = p.os1; p.is2 = p.os2; p.is3 = p.os3;
  }
  return p;
}

// The state kernel keeps its CU to itself: 40 KB of unused dynamic LDS raise its request to 128 KB, so
// that neither a prep workgroup (~131 KB) nor an output workgroup (~49 KB) fits beside it in the CU's
// 160 KB and takes issue slots from the sequential chain.
constexpr int STATE_EXCLUSIVE_LDS = 40 * 1024;

template <class P, typename InT, typename OutT, int D, int DV>
static int launch_phase(const ScanParams& p, int phase, hipStream_t st) {
  const dim3 chunk_grid((unsigned)p.nseg, (unsigned)p.H, (unsigned)p.B);
  if (phase == PHASE_PREP) {
    const int fm = p.prelifted ? FM_PRELIFTED : (p.omega_lo ? FM_HILO : FM_EXACT);
    const int run_t = fm == FM_PRELIFTED ? PrepRun<P, FM_PRELIFTED>::value
                    : fm == FM_HILO ? PrepRun<P, FM_HILO>::value : PrepRun<P, FM_EXACT>::value;
    const int run = run_t ? run_t : p.prep_run;
    const dim3 prep_grid((unsigned)((p.nseg + run - 1) / run), (unsigned)p.H, (unsigned)p.B);
    if (fm == FM_PRELIFTED) hipLaunchKernelGGL((prep_kernel<P, InT, D, DV, FM_PRELIFTED>), prep_grid, dim3(256), 0, st, p);
    else if (fm == FM_HILO) hipLaunchKernelGGL((prep_kernel<P, InT, D, DV, FM_HILO>), prep_grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((prep_kernel<P, InT, D, DV, FM_EXACT>), prep_grid, dim3(256), 0, st, p);
  } else if (phase == PHASE_STATE) {
    // The state workgroups are the sequential critical path: reserve enough LDS that no prep or output
    // workgroup can share their CU (a CU has 160 KB; the bf16 state kernel uses 88 KB statically).
    const size_t excl = IsBF16<P>::value ? (size_t)STATE_EXCLUSIVE_LDS : 0;
    if (p.decay) hipLaunchKernelGGL((state_kernel<P, D, DV, true>), dim3(state_grid(p.B, p.H, DV / 16)), dim3(256), excl, st, p);
    else hipLaunchKernelGGL((state_kernel<P, D, DV, false>), dim3(state_grid(p.B, p.H, DV / 16)), dim3(256), excl, st, p);
  } else {
    hipLaunchKernelGGL((output_kernel<P, OutT, D, DV>), chunk_grid, dim3(256), 0, st, p);
  }
  return hipGetLastError() == hipSuccess ? KDN_OK : KDN_ERR_DEVICE;
}

// Runs chunks [c_begin, c_end) in segments of `seg` chunks, all in one workspace buffer: per segment the
// selected kernels, in the order prep, state, output.
template <class P, typename InT, typename OutT, int D, int DV>
static int run_scan(const kdn_scan_args* a, const RunSpec& r) {
  const int cus = device_cus();
  for (int64_t c0 = r.c_begin; c0 < r.c_end; c0 += r.seg) {
    const ScanParams p = segment_params(a, r, c0, (r.c_end - c0 < r.seg) ? (r.c_end - c0) : r.seg, a->workspace, cus);
    for (int ph : {PHASE_PREP, PHASE_STATE, PHASE_OUTPUT}) {
      if (!(r.phases & ph)) continue;
      const int rc = launch_phase<P, InT, OutT, D, DV>(p, ph, r.st);
      if (rc != KDN_OK) return rc;
    }
  }
  return KDN_OK;
}

// Events of the pipelined scan, released when the call returns (destroying an event whose record is
// still pending is allowed; its resources are freed once it completes).
struct EventSet {
  hipEvent_t ev[16];
  int n = 0;
  int create(int count) {
    for (; n < count; ++n)
      if (hipEventCreateWithFlags(&ev[n], hipEventDisableTiming) != hipSuccess) return KDN_ERR_DEVICE;
    return KDN_OK;
  }
  ~EventSet() {
    for (int i = 0; i < n; ++i) (void)hipEventDestroy(ev[i]);
  }
};

// Segments rotate through `nbuf` workspace buffers.  The state chain runs on `st` (the caller's stream);
// prep runs on `aux` and output on `aux_out` (the same stream as prep when only one auxiliary stream is
// given, in the order prep(s+1), output(s)), so that while state(s) occupies its B*H*d_v/16 workgroups the
// other CUs prepare the next segment and finish the previous one.
//   state(s)  waits for prep(s)          (event P[s % nbuf])
//   output(s) waits for state(s)         (event S[s % nbuf])
//   prep(s)   reuses the buffer of segment s - nbuf: on a separate output stream it waits for that
//             segment's output (event O[s % nbuf]); on one auxiliary stream the order ensures it
// the auxiliary streams first wait for the work already queued on st, and st finally waits for the last
// output.
template <class P, typename InT, typename OutT, int D, int DV>
static int run_pipelined(const kdn_scan_args* a, const RunSpec& r) {
  const int64_t seg = r.seg;
  const int nbuf = r.nbuf;
  const size_t buf_bytes = r.buf_bytes;
  const hipStream_t st = r.st, aux = r.aux;
  const hipStream_t aux_out = r.aux_out ? r.aux_out : r.aux;
  const bool split = aux_out != aux;
  const int64_t nchunks = (a->T + CH - 1) / CH;
  const int64_t nsegs = (nchunks + seg - 1) / seg;
  EventSet evs;
  int rc = evs.create(3 * nbuf + 2);
  if (rc != KDN_OK) return rc;
  hipEvent_t* evP = evs.ev;
  hipEvent_t* evS = evs.ev + nbuf;
  hipEvent_t* evO = evs.ev + 2 * nbuf;
  hipEvent_t evIn = evs.ev[3 * nbuf], evOut = evs.ev[3 * nbuf + 1];
  // prep shares the device with the state kernel's workgroups (one per CU)
  const int prep_cus = device_cus() - (int)state_grid(a->B, a->H, DV / 16);
  auto seg_p = [&](int64_t s) {
    const int64_t c0 = s * seg;
    return segment_params(a, r, c0, (nchunks - c0 < seg) ? (nchunks - c0) : seg,
                          (unsigned char*)a->workspace + (size_t)(s % nbuf) * buf_bytes, prep_cus);
  };
#define KDN_TRY(x) do { if ((x) != hipSuccess) return KDN_ERR_DEVICE; } while (0)
#define KDN_TRYK(x) do { const int _rc = (x); if (_rc != KDN_OK) return _rc; } while (0)
  KDN_TRY(hipEventRecord(evIn, st));
  KDN_TRY(hipStreamWaitEvent(aux, evIn, 0));
  if (split) KDN_TRY(hipStreamWaitEvent(aux_out, evIn, 0));
  KDN_TRYK((launch_phase<P, InT, OutT, D, DV>(seg_p(0), PHASE_PREP, aux)));
  KDN_TRY(hipEventRecord(evP[0], aux));
  for (int64_t s = 0; s < nsegs; ++s) {
    const ScanParams ps = seg_p(s);
    KDN_TRY(hipStreamWaitEvent(st, evP[s % nbuf], 0));
    KDN_TRYK((launch_phase<P, InT, OutT, D, DV>(ps, PHASE_STATE, st)));
    KDN_TRY(hipEventRecord(evS[s % nbuf], st));
    if (s + 1 < nsegs) {
      if (split && s + 1 >= nbuf) KDN_TRY(hipStreamWaitEvent(aux, evO[(s + 1) % nbuf], 0));
      KDN_TRYK((launch_phase<P, InT, OutT, D, DV>(seg_p(s + 1), PHASE_PREP, aux)));
      KDN_TRY(hipEventRecord(evP[(s + 1) % nbuf], aux));
    }
    KDN_TRY(hipStreamWaitEvent(aux_out, evS[s % nbuf], 0));
    KDN_TRYK((launch_phase<P, InT, OutT, D, DV>(ps, PHASE_OUTPUT, aux_out)));
    if (split) KDN_TRY(hipEventRecord(evO[s % nbuf], aux_out));
  }
  KDN_TRY(hipEventRecord(evOut, aux_out));
  KDN_TRY(hipStreamWaitEvent(st, evOut, 0));
#undef KDN_TRY
#undef KDN_TRYK
  return KDN_OK;
}

template <class P, typename InT, typename OutT, int D, int DV>
static int run(const kdn_scan_args* a, const RunSpec& r) {
  if (r.aux) return run_pipelined<P, InT, OutT, D, DV>(a, r);
  return run_scan<P, InT, OutT, D, DV>(a, r);
}

template <class P, typename InT, typename OutT, int D>
static int dispatch_dv(const kdn_scan_args* a, const RunSpec& r) {
  switch (a->d_v) {
    case 16: return run<P, InT, OutT, D, 16>(a, r);
    case 32: return run<P, InT, OutT, D, 32>(a, r);
    case 64: return run<P, InT, OutT, D, 64>(a, r);
    case 128: return run<P, InT, OutT, D, 128>(a, r);
    default: return KDN_ERR_UNSUPPORTED;
  }
}

static int dispatch(const kdn_scan_args* a, const RunSpec& r) {
  if (a->in_dtype == KDN_DTYPE_BF16) {
    if (a->out_dtype == KDN_DTYPE_BF16) return dispatch_dv<PrecBF16, __bf16, __bf16, 512>(a, r);
    return dispatch_dv<PrecBF16, __bf16, float, 512>(a, r);
  }
  if (a->out_dtype == KDN_DTYPE_BF16) return dispatch_dv<PrecF32, float, __bf16, 512>(a, r);
  return dispatch_dv<PrecF32, float, float, 512>(a, r);
}

static int dispatch(const kdn_scan_args* a, int64_t c_begin, int64_t c_end, int64_t seg, int phases, hipStream_t st) {
  const RunSpec r = {c_begin, c_end, seg, phases, st, nullptr, 0, 0};
  return dispatch(a, r);
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

// Default segment: the workspace of one segment stays near 64 MiB (so that the state and output
// kernels mostly re-read what prep just wrote from the 256 MB last-level cache), at least 8 chunks.
static int64_t choose_segment(const kdn_scan_args* a) {
  const int64_t nchunks = (a->T + CH - 1) / CH;
  if (a->segment_chunks > 0) return a->segment_chunks < nchunks ? a->segment_chunks : nchunks;
  const size_t per_step = chunk_bytes(a) * (size_t)a->B * (size_t)a->H;
  int64_t seg = (int64_t)(((size_t)64 << 20) / (per_step ? per_step : 1));
  if (seg < 8) seg = 8;
  return seg < nchunks ? seg : nchunks;
}

static int validate(const kdn_scan_args* a) {
  if (!a) return KDN_ERR_INVALID_ARGUMENT;
  if (a->B <= 0 || a->T <= 0 || a->H <= 0) return KDN_ERR_INVALID_ARGUMENT;
  if (a->B > 65535 || a->H > 65535) return KDN_ERR_UNSUPPORTED;
  if (!valid_dtype(a->in_dtype) || !valid_dtype(a->out_dtype)) return KDN_ERR_INVALID_ARGUMENT;
  if (a->feature_mode != 0 && a->feature_mode != 1) return KDN_ERR_INVALID_ARGUMENT;
  if (a->rule != 0 && a->rule != 1) return KDN_ERR_INVALID_ARGUMENT;
  if (general_scan_applies(a)) {
    const int rc = general_scan_validate(a);  // D = 1024: pre-lifted features, kdn_general.hip
    if (rc != KDN_OK) return rc;
  } else if (a->D != 512) {
    return KDN_ERR_UNSUPPORTED;
  }
  if (a->feature_mode == 0 ? a->d_k != 64 : a->d_k != a->D) return KDN_ERR_UNSUPPORTED;
  if (a->omega_head_stride < 0 || a->phase_head_stride < 0) return KDN_ERR_INVALID_ARGUMENT;
  if (a->d_v != 16 && a->d_v != 32 && a->d_v != 64 && a->d_v != 128) return KDN_ERR_UNSUPPORTED;
  if (a->segment_chunks < 0) return KDN_ERR_INVALID_ARGUMENT;
  if (!(a->inv_tau == a->inv_tau)) return KDN_ERR_INVALID_ARGUMENT;
  return KDN_OK;
}

// Pointer, stride and alignment checks shared by the launching entry points.
static int validate_launch(const kdn_scan_args* a) {
  int rc = validate(a);
  if (rc != KDN_OK) return rc;
  if (!a->q || !a->k || !a->v || !a->beta || !a->final_state || !a->y || !a->workspace) return KDN_ERR_INVALID_ARGUMENT;
  if (a->feature_mode == 0 && (!a->omega_bf16 || !a->phase)) return KDN_ERR_INVALID_ARGUMENT;
  if (a->feature_mode == 0 && ((a->omega_lo && !aligned(a->omega_lo, 16)) || (a->omega_head_stride % 8) != 0 ||
                               (a->phase_head_stride % 4) != 0))
    return KDN_ERR_MISALIGNED;
  // 16-byte row loads of q, k, v; 16-byte fragment traffic in the workspace.
  const size_t isz = dtype_size(a->in_dtype);
  if (!aligned(a->q, 16) || !aligned(a->k, 16) || !aligned(a->v, 16) || !aligned(a->workspace, 256))
    return KDN_ERR_MISALIGNED;
  if (a->feature_mode == 0 && (!aligned(a->omega_bf16, 16) || !aligned(a->phase, 16))) return KDN_ERR_MISALIGNED;
  const size_t osz = dtype_size(a->out_dtype);
  if (!aligned(a->y, 16)) return KDN_ERR_MISALIGNED;
  for (int i = 0; i < 3; ++i) {
    if (((a->q_stride[i] * (int64_t)isz) % 16) != 0 || ((a->k_stride[i] * (int64_t)isz) % 16) != 0 ||
        ((a->v_stride[i] * (int64_t)isz) % 16) != 0 || ((a->y_stride[i] * (int64_t)osz) % 16) != 0)
      return KDN_ERR_MISALIGNED;
  }
  return KDN_OK;
}

static int run_phase(const kdn_scan_args* a, int64_t chunk0, int64_t nchunks, int phase, void* stream) {
  int rc = validate_launch(a);
  if (rc != KDN_OK) return rc;
  if (general_scan_applies(a)) return KDN_ERR_UNSUPPORTED;  // the general-D scan has no phase entry points
  const int64_t total = (a->T + CH - 1) / CH;
  if (chunk0 < 0 || nchunks < 1 || chunk0 + nchunks > total) return KDN_ERR_INVALID_ARGUMENT;
  const size_t need = chunk_bytes(a) * (size_t)a->B * (size_t)a->H * (size_t)(nchunks + 1);
  if (a->workspace_bytes < need) return KDN_ERR_WORKSPACE_TOO_SMALL;
  return dispatch(a, chunk0, chunk0 + nchunks, nchunks, phase, as_stream(stream));
}

}  // namespace kdn

using namespace kdn;

extern "C" size_t kdn_scan_workspace_bytes(const kdn_scan_args* a) {
  if (validate(a) != KDN_OK) return 0;
  if (general_scan_applies(a)) return general_scan_workspace_bytes(a);
  const int64_t seg = choose_segment(a);
  return chunk_bytes(a) * (size_t)a->B * (size_t)a->H * (size_t)(seg + 1);
}

extern "C" int kdn_delta_scan_fwd(const kdn_scan_args* a, void* stream) {
  int rc = validate_launch(a);
  if (rc != KDN_OK) return rc;
  if (general_scan_applies(a)) return general_scan(a, stream);
  const int64_t seg = choose_segment(a);
  const size_t need = chunk_bytes(a) * (size_t)a->B * (size_t)a->H * (size_t)(seg + 1);
  if (a->workspace_bytes < need) return KDN_ERR_WORKSPACE_TOO_SMALL;
  const int64_t nchunks = (a->T + CH - 1) / CH;
  return dispatch(a, 0, nchunks, seg, PHASE_ALL, as_stream(stream));
}

// Default segment of the pipelined scan: 64 chunks (4096 tokens), fewer for short sequences.
static int64_t pipeline_segment(const kdn_scan_args* a) {
  const int64_t nchunks = (a->T + CH - 1) / CH;
  const int64_t seg = a->segment_chunks > 0 ? a->segment_chunks : 64;
  return seg < nchunks ? seg : nchunks;
}

extern "C" size_t kdn_scan_workspace_bytes_pipelined(const kdn_scan_args* a) {
  return scan_workspace_bytes_pipelined(a);
}

namespace kdn {
// The pipelined scan (serial when aux_stream is NULL or the workspace holds one segment buffer), with
// ragged sequences optionally given as device start / end arrays.
int scan_pipelined(const kdn_scan_args* a, const int64_t* seq_lo, const int64_t* seq_hi, void* stream,
                   void* aux_stream, void* out_stream) {
  int rc = validate_launch(a);
  if (rc != KDN_OK) return rc;
  if (general_scan_applies(a)) return seq_lo ? KDN_ERR_UNSUPPORTED : general_scan(a, stream);
  const int64_t seg = pipeline_segment(a);
  const size_t buf = chunk_bytes(a) * (size_t)a->B * (size_t)a->H * (size_t)(seg + 1);
  if (a->workspace_bytes < buf) return KDN_ERR_WORKSPACE_TOO_SMALL;
  const int64_t nchunks = (a->T + CH - 1) / CH;
  const int64_t nsegs = (nchunks + seg - 1) / seg;
  size_t fit = a->workspace_bytes / buf;
  const int nbuf = (int)(fit < 3 ? fit : 3);
  RunSpec r = {0, nchunks, seg, PHASE_ALL, as_stream(stream), as_stream(aux_stream), nbuf, buf};
  r.seq_lo = seq_lo;
  r.seq_hi = seq_hi;
  if (out_stream && out_stream != stream && out_stream != aux_stream) r.aux_out = as_stream(out_stream);
  if (!aux_stream || aux_stream == stream || nbuf < 2 || nsegs < 2) {
    r.aux = nullptr;
    r.aux_out = nullptr;
  }
  return dispatch(a, r);
}

size_t scan_workspace_bytes_pipelined(const kdn_scan_args* a) {
  if (validate(a) != KDN_OK) return 0;
  if (general_scan_applies(a)) return general_scan_workspace_bytes(a);
  const int64_t seg = pipeline_segment(a);
  const int64_t nsegs = ((a->T + CH - 1) / CH + seg - 1) / seg;
  const int64_t nbuf = nsegs < 3 ? nsegs : 3;
  return chunk_bytes(a) * (size_t)a->B * (size_t)a->H * (size_t)(seg + 1) * (size_t)nbuf;
}
}  // namespace kdn

extern "C" int kdn_delta_scan_fwd_pipelined(const kdn_scan_args* a, void* stream, void* aux_stream) {
  return scan_pipelined(a, nullptr, nullptr, stream, aux_stream, nullptr);
}

extern "C" int kdn_delta_scan_fwd_streams(const kdn_scan_args* a, void* stream, void* prep_stream, void* output_stream) {
  return scan_pipelined(a, nullptr, nullptr, stream, prep_stream, output_stream);
}

extern "C" int kdn_scan_prep(const kdn_scan_args* a, int64_t chunk0, int64_t nchunks, void* stream) {
  return run_phase(a, chunk0, nchunks, PHASE_PREP, stream);
}

extern "C" int kdn_scan_state(const kdn_scan_args* a, int64_t chunk0, int64_t nchunks, void* stream) {
  return run_phase(a, chunk0, nchunks, PHASE_STATE, stream);
}

extern "C" int kdn_scan_output(const kdn_scan_args* a, int64_t chunk0, int64_t nchunks, void* stream) {
  return run_phase(a, chunk0, nchunks, PHASE_OUTPUT, stream);
}
