// Prep kernel of the D = 512 prefill scan (the S-independent per-chunk factors; the algebra and the
// record it writes are described in kdn_scan.hip and kdn_scan_common.hpp).
#include <type_traits>
#include "kdn_frag.hpp"
#include "kdn_internal.hpp"
#include "kdn_io.hpp"
#include "kdn_lift_tile.hpp"
#include "kdn_tile.hpp"
#include "kdn_scan_common.hpp"

namespace kdn {

// ------------------------------------------------------------------------------------------------
// prep: grid (ceil(nseg / run), H, B), 256 threads.  A workgroup prepares `run` consecutive chunks of one
// head.  Wave w owns token rows [16w, 16w+16) of a chunk.  The waves exchange data through LDS only, so
// the barriers order LDS only (lds_barrier): the global loads issued early (q, k, V rows) travel across
// them instead of being drained at every barrier.
// bf16 lifts (exact or hi + lo projection): one chunk per workgroup, two workgroups per CU (67 KB of LDS,
// at most 256 registers per wave), each hiding the other's latencies.  The exact projection's Omega is
// staged in LDS in the area the K fragments take later; the hi + lo parts are read from L2.  The exact
// projection with queries runs the eight-wave form below (prep8_kernel) instead: four waves per SIMD.
// Given features (bf16): runs of `run` chunks chosen at launch (ScanParams::prep_run), the next chunk's
// beta / decay prefetched.  fp32: one chunk, one workgroup per CU (its fragments are twice as wide).
template <class P, int FM>
struct PrepRun : std::integral_constant<int, (IsBF16<P>::value && FM == FM_PRELIFTED) ? 0 : 1> {};
template <class P, int FM>
struct PrepWaves : std::integral_constant<int, (IsBF16<P>::value && FM != FM_PRELIFTED) ? 2 : 1> {};

// Raw inputs of one chunk for one thread of the prep workgroup: the q / k row pieces of the lane's row
// and beta / decay of token `lane` (prefetched one chunk ahead), and the V pieces of the thread
// (loaded at the start of the chunk; they are first needed after the Gram).
template <typename InT, int DV>
struct PrepInputs {
  static constexpr int VPR = DV * (int)sizeof(InT) / 16;        // 16-byte pieces per V row
  static constexpr int VPT = (64 * VPR + 255) / 256;             // pieces per thread
  RawRow<InT> qk[2];
  float be, la;
  template <bool NOQ = false>
  __device__ __forceinline__ void load_qk(const ScanParams& p, const Seq& sq, int64_t h, int64_t t0, int w, int lane) {
    const int64_t trow = t0 + 16 * w + (lane & 15);
    const bool rvalid = trow < sq.len;
    if constexpr (!NOQ) qk[0].load((const InT*)p.q + sq.q + trow * p.qs1 + h * p.qs2, rvalid, lane);
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

// NOQ (exact projection only, ScanParams::prep_no_q): no output kernel reads this segment's records (the
// backward's checkpoint pass runs prep and state only), so the queries are not lifted and neither P nor
// the query scales are formed.
template <class P, typename InT, int D, int DV, int FM, bool NOQ = false>
__global__ void __launch_bounds__(256, (PrepWaves<P, FM>::value)) prep_kernel(ScanParams p) {
  static_assert(!NOQ || FM == FM_EXACT, "the key-only prep is the exact projection's");
  using L = WsLayout<P, D, DV>;
  using frag = typename P::frag;
  using In = PrepInputs<InT, DV>;
  constexpr int NT = D / 16, NJ = D / 32, NV = DV / 16;
  // The exact projection's Omega (64 KB of bf16 A fragments) is staged in the LDS area that holds the K
  // fragments for the Gram later: the lift reads it from LDS (from L2 it waited on every feature tile's
  // fragments), and the kernel still fits two workgroups per CU.  The hi + lo projection reads its two
  // parts from L2.
  constexpr bool OMEGA_LDS = FM == FM_EXACT;
  constexpr size_t PHIK_BYTES = (size_t)4 * NJ * 64 * sizeof(frag);
  static_assert(!OMEGA_LDS || (size_t)NT * 2 * 64 * 16 <= PHIK_BYTES, "Omega does not fit the K-fragment area");
  // After the Gram the K-fragment area is reused for A (16 KB), T (16 KB) and V.  V rows are padded by
  // four elements: the fragment reads below take rows 4 apart in the four lane groups, which then fall
  // on disjoint banks (unpadded they hit the same banks, a four-way conflict on every read).
  constexpr int DVP = DV + 4;
  static_assert(64 * 64 * 4 + 64 * 64 * 4 + 64 * DVP * sizeof(InT) <= PHIK_BYTES, "LDS reuse does not fit");
  __shared__ __attribute__((aligned(16))) unsigned char smem[PHIK_BYTES];
  __shared__ __attribute__((aligned(16))) float s_beta[64], s_g[64], s_sq[64], s_sk[64], s_phrev[D];

  bf16x8* s_omega = reinterpret_cast<bf16x8*>(smem);                 // during the lift (OMEGA_LDS)
  frag* s_phik = reinterpret_cast<frag*>(smem);                       // from the lift to the Gram
  float* s_A = reinterpret_cast<float*>(smem);                        // [j][p][s'] = A[4s+p][j] (s swizzled, a_swizzle)
  float* s_T = s_A + 64 * 64;                                          // [t][64] (columns swizzled, t_swizzle)
  InT* s_V = reinterpret_cast<InT*>(s_T + 64 * 64);                    // [t][DVP]

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int RUN = PrepRun<P, FM>::value;  // 0: runtime run length with prefetch
  const int run = RUN ? RUN : p.prep_run;
  // chunks [cl0, cl_end) of sequence b (chunk indices of the segment, chunk0 + cl in the sequence) with
  // their records from rec0; a packed window gives each workgroup the one chunk of its slot
  const int64_t h = blockIdx.y;
  int64_t b, cl0, nloc;
  unsigned char* rec0;
  if (p.fl_off) {
    const FlatChunk fc = flat_chunk(p, blockIdx.x);
    if (!fc.ok) return;  // a spare slot, or past the last
    b = fc.b;
    cl0 = fc.c;
    nloc = fc.c + 1;
    rec0 = p.ws + (h * (p.nseg + 1) + blockIdx.x) * L::bytes;
  } else {
    b = blockIdx.z;
    cl0 = (int64_t)blockIdx.x * run;
    nloc = seg_chunks(p, seq_of(p, b));
    if (cl0 >= nloc) return;  // past the end of this sequence (ragged batches): nothing to prepare
    rec0 = p.ws + ((b * p.H + h) * (p.nseg + 1) + cl0) * L::bytes;
  }
  const Seq sq = seq_of(p, b);
  const int64_t cl_end = (cl0 + run < nloc) ? cl0 + run : nloc;

  const __bf16* omega_h = p.omega + h * p.oms;
  const __bf16* omega_lo_h = (FM == FM_HILO) ? p.omega_lo + h * p.oms : nullptr;
  const float ang = (p.inv_tau_head ? p.inv_tau_head[h] : p.inv_tau) * 0.15915494309189535f;
  In in;
  // Record stores: streaming for the state / output kernels, which read a record a segment or more later
  // (so that it does not evict the lines the concurrent kernels are about to read); cacheable for the
  // fused chain, so that its records stay in the last-level cache until the chain reads them.
  const bool cached = p.k_plain != 0;
  auto put = [&](void* base, const frag& f) {
    if (cached) store_frag<P>(base, lane, f);
    else store_frag_nt<P>(base, lane, f);
  };
  if constexpr (FM != FM_PRELIFTED) {
    stage_omega<D, OMEGA_LDS>(omega_h, p.phase + h * p.phs, s_omega, s_phrev);
    in.template load_qk<NOQ>(p, sq, h, (p.chunk0 + cl0) * CH, w, lane);
  } else {
    // no lift: only beta / decay come through the prefetch
    const int64_t t = (p.chunk0 + cl0) * CH + lane;
    const bool valid = t < sq.len;
    in.be = valid ? p.beta[sq.be + t * p.bs1 + h * p.bs2] : 0.f;
    in.la = (valid && p.decay) ? p.decay[sq.de + t * p.ds1 + h * p.ds2] : 1.f;
  }

  auto process = [&](int64_t cl) {
    const int64_t t0 = (p.chunk0 + cl) * CH;
    unsigned char* ws = rec0 + (cl - cl0) * L::bytes;
    u32x4 vraw[In::VPT];
    In::load_v(p, sq, h, t0, vraw);  // early: first needed after the Gram, its latency hides behind the lift
    lds_barrier();  // Omega staged (first chunk); the previous chunk's LDS reads are done

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
    // X fragments (m = w, j): row 16w + (l&15), feature 32j + kappa(l, s); [QI] = q, [KI] = k
    constexpr int NX = NOQ ? 1 : 2, QI = 0, KI = NX - 1;
    frag cqk[NX][NJ];
    float ss[NX];
    if constexpr (FM == FM_PRELIFTED) {
      const int64_t trow = t0 + 16 * w + (lane & 15);
      load_lifted<P, InT, D>((const InT*)p.q + sq.q + trow * p.qs1 + h * p.qs2, trow < sq.len, lane, cqk[0]);
      load_lifted<P, InT, D>((const InT*)p.k + sq.k + trow * p.ks1 + h * p.ks2, trow < sq.len, lane, cqk[1]);
      const int64_t tn = (p.chunk0 + ((cl + 1 < cl_end) ? cl + 1 : cl)) * CH + lane;
      in.be = (tn < sq.len) ? p.beta[sq.be + tn * p.bs1 + h * p.bs2] : 0.f;
      in.la = (tn < sq.len && p.decay) ? p.decay[sq.de + tn * p.ds1 + h * p.ds2] : 1.f;
    } else {
      if constexpr (NOQ) {
        const RawRow<InT> kraw[1] = {in.qk[1]};
        lift_tile<P, InT, D, OMEGA_LDS, 1>(kraw, p.normalize, s_omega, omega_h, s_phrev, ang, lane, cqk, ss);
      } else {
        lift_tile<P, InT, D, OMEGA_LDS, 2, FM == FM_HILO>(in.qk, p.normalize, s_omega, omega_h, s_phrev, ang, lane,
                                                           cqk, ss, omega_lo_h);
      }
      // the next chunk's rows travel while this one is processed (clamped: the last chunk reloads itself)
      if constexpr (RUN != 1) in.template load_qk<NOQ>(p, sq, h, (p.chunk0 + ((cl + 1 < cl_end) ? cl + 1 : cl)) * CH, w, lane);
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
          sq_ = NOQ ? 0.f : amp / (amp * sqrtf(ss[QI]) + 1e-8f);
          sk_ = amp / (amp * sqrtf(ss[KI]) + 1e-8f);
        }
        if constexpr (!NOQ) s_sq[16 * w + lane] = sq_;
        s_sk[16 * w + lane] = sk_;
      }
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      // The records are read back by the state and output kernels a segment or more later, long after
      // they could still sit in L2: streaming stores keep them from evicting the state kernel's lines.
      if constexpr (IsBF16<P>::value && D == 512) {
        if (p.k_plain) put(ws + L::phiK + (size_t)(w * NJ + j) * 64 * L::FB, cqk[KI][j]);
        else store_k_image(ws + L::phiK, w, j, lane, cqk[KI][j]);
      } else {
        store_frag_nt<P>(ws + L::phiK + (size_t)(w * NJ + j) * 64 * L::FB, lane, cqk[KI][j]);
      }
      if constexpr (!NOQ) {
        if (!p.q_relift) put(ws + L::phiQ + (size_t)(w * NJ + j) * 64 * L::FB, cqk[QI][j]);
      }
    }
    if constexpr (OMEGA_LDS) lds_barrier();  // every wave's lift has read Omega from the area
#pragma unroll
    for (int j = 0; j < NJ; ++j) s_phik[(w * NJ + j) * 64 + lane] = cqk[KI][j];
    lds_barrier();

    // ---- Gram tiles (m, n = w):  Gkk[m][w] = K_m K_w^T,  GqkT[m][w] = K_m Q_w^T  (unnormalised)
    f32x4 gkk[4], gqk[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) { gkk[m] = zero4(); gqk[m] = zero4(); }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const frag a = s_phik[(m * NJ + j) * 64 + lane];
        gkk[m] = P::mma(gkk[m], a, cqk[KI][j]);
        if constexpr (!NOQ) gqk[m] = P::mma(gqk[m], a, cqk[QI][j]);
      }
    }
    lds_barrier();  // K fragments in LDS are dead from here on

    // ---- A (for the inverse), P fragments, V staging, scale vectors
    {
      const int t = 16 * w + (lane & 15);
      // the linear rule has no erasure coupling: A = 0, so T = I below
      const float bt = p.linear ? 0.f : s_beta[t], gt = s_g[t], gtm1 = t > 0 ? s_g[t - 1] : 0.f;
      const float skt = s_sk[t], sqt = NOQ ? 0.f : s_sq[t];
      f32x4 pt[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = 16 * m + 4 * (lane >> 4) + i;
          const float gj = s_g[j], skj = s_sk[j];
          const float a = (j < t) ? bt * __expf(fminf(gt - gj, 0.f)) * gkk[m][i] * skt * skj : 0.f;
          s_A[(j * 4 + (t & 3)) * 16 + a_swizzle(j, t >> 2, t & 3)] = a;
          if constexpr (!NOQ) pt[m][i] = (j < t) ? __expf(fminf(gtm1 - gj, 0.f)) * gqk[m][i] * sqt * skj : 0.f;
        }
      }
      if constexpr (!NOQ) {
#pragma unroll
        for (int jb = 0; jb < 2; ++jb)
          put(ws + L::Pm + (size_t)(w * 2 + jb) * 64 * L::FB, P::from_f32(pair_to8(pt[2 * jb], pt[2 * jb + 1])));
      }
    }
#pragma unroll
    for (int i = 0; i < In::VPT; ++i) {
      const int idx = (int)threadIdx.x + 256 * i;
      if (idx < 64 * In::VPR) {
        // padded rows are 8-byte aligned: two 8-byte stores per 16-byte piece
        u32x2* d = reinterpret_cast<u32x2*>(s_V + (idx / In::VPR) * DVP + (idx % In::VPR) * (16 / (int)sizeof(InT)));
        d[0] = __builtin_shufflevector(vraw[i], vraw[i], 0, 1);
        d[1] = __builtin_shufflevector(vraw[i], vraw[i], 2, 3);
      }
    }
    if (w == 1) {
      float* vec = reinterpret_cast<float*>(ws + L::VEC);
      const float g63 = s_g[63];
      const float gtm1 = lane > 0 ? s_g[lane - 1] : 0.f;
      if constexpr (!NOQ) vec[lane] = __expf(fminf(gtm1, 0.f)) * s_sq[lane];  // e^{g_{t-1}} * |phi_q| scale
      vec[64 + lane] = __expf(fminf(g63 - s_g[lane], 0.f)) * s_sk[lane]; // e^{g_63 - g_t} * |phi_k| scale
      if (lane == 0) vec[128] = __expf(fminf(g63, 0.f));
    }
    lds_barrier();

    // ---- T = (I + A)^{-1} (16 x 16 blocks: substitution on the diagonal, MFMA products below it)
    unit_lower_inverse_blocked(s_A, s_T, w, lane);
    lds_barrier();

    // ---- W~ factor T diag(beta e^g |phi_k|) fragments, and U~ = T diag(beta) V   (wave w: rows m = w)
    {
      const int t = 16 * w + (lane & 15);
      f32x8 tb[2];
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        f32x8 tw;
        // slots 4h .. 4h + 3 are the four consecutive columns j = 32jb + 16h + 4(lane >> 4) + 0..3
        // (kappa), read as one 16-byte vector from each array (T's rows swizzled by t_swizzle: the 16
        // rows of a lane group fall on distinct banks)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int j0 = 32 * jb + 16 * hh + 4 * (lane >> 4);
          const f32x4 tv = *reinterpret_cast<const f32x4*>(s_T + t * 64 + t_swizzle(t, j0));
          const f32x4 be = *reinterpret_cast<const f32x4*>(s_beta + j0);
          const f32x4 gj = *reinterpret_cast<const f32x4*>(s_g + j0);
          const f32x4 sk = *reinterpret_cast<const f32x4*>(s_sk + j0);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            tw[4 * hh + i] = p.linear ? 0.f : tv[i] * be[i] * __expf(gj[i]) * sk[i];  // linear: E = U~
            tb[jb][4 * hh + i] = tv[i] * be[i];
          }
        }
        put(ws + L::Tp + (size_t)(w * 2 + jb) * 64 * L::FB, P::from_f32(tw));
      }
#pragma unroll
      for (int n = 0; n < NV; ++n) {
        f32x4 acc = zero4();
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
          f32x8 vv;
#pragma unroll
          for (int s = 0; s < 8; ++s) vv[s] = (float)s_V[(32 * jb + kappa(lane, s)) * DVP + 16 * n + (lane & 15)];
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
        f32x4* ud = reinterpret_cast<f32x4*>(ws + L::U + ((size_t)(w * NV + n) * 64 + lane) * 16);
        if (cached) *ud = acc;
        else __builtin_nontemporal_store(acc, ud);
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
// prep8: the bf16 exact-projection prep (no ScanParams::prep_no_q) with eight waves per workgroup, 512
// threads, one chunk per workgroup and two workgroups per CU at <= 128 registers: four waves per SIMD to
// hide each phase's latencies instead of two.  Wave w = 4 hf + m owns token tile m (rows 16m .. 16m + 15)
// and feature half hf (features 256 hf .. + 255, 32-feature blocks 8 hf .. 8 hf + 7): it lifts its rows
// of q and k on that half only (64 fragment registers instead of 128), stores those record fragments and
// forms the half's partial Gram tiles.  The halves meet in LDS: the rows' sums of squares, then the
// partial Grams (hf = 0 hands over its K Q^T part, hf = 1 its K K^T part), after which the hf = 0 waves
// form A and the hf = 1 waves P; waves 0-3 invert the diagonal blocks and 0-2 walk the block columns;
// the Tp tiles are hf = 0's and the U~ tiles are split between the halves.  It writes the record
// prep_kernel<PrecBF16, __bf16, 512, DV, FM_EXACT> writes: the same K and Q features bit for bit; the
// scales and Grams summed in two halves (rounding order only).
template <int DV>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) prep8_kernel(ScanParams p) {
  using P = PrecBF16;
  using InT = __bf16;
  constexpr int D = 512;
  using L = WsLayout<P, D, DV>;
  using frag = typename P::frag;
  constexpr int NJ = D / 32, NJH = NJ / 2, NV = DV / 16;
  constexpr int NVH = NV > 1 ? NV / 2 : 1;              // U~ tiles per half
  constexpr int VPR = DV * (int)sizeof(InT) / 16;       // 16-byte pieces per V row
  constexpr int VPT = (64 * VPR + 511) / 512;           // pieces per thread
  constexpr size_t PHIK_BYTES = (size_t)4 * NJ * 64 * sizeof(frag);
  static_assert((size_t)(D / 16) * 2 * 64 * 16 <= PHIK_BYTES, "Omega does not fit the K-fragment area");
  // After the Gram the K-fragment area holds A [0, 16 KB), T [16 KB, 32 KB) and, from 32 KB, first the
  // partial Grams (32 KB) and then V (rows padded by four elements, as in prep_kernel).
  constexpr int DVP = DV + 4;
  static_assert(64 * 64 * 4 + 64 * 64 * 4 + 64 * DVP * sizeof(InT) <= PHIK_BYTES, "LDS reuse does not fit");
  static_assert(PHIK_BYTES / 2 + (size_t)2 * 4 * 4 * 64 * 16 <= PHIK_BYTES, "Gram partials do not fit");
  __shared__ __attribute__((aligned(16))) unsigned char smem[PHIK_BYTES];
  __shared__ __attribute__((aligned(16))) float s_beta[64], s_g[64], s_sq[64], s_sk[64], s_phrev[D], s_ss[2][2][64];

  bf16x8* s_omega = reinterpret_cast<bf16x8*>(smem);                 // during the lift
  frag* s_phik = reinterpret_cast<frag*>(smem);                       // from the lift to the Gram
  float* s_A = reinterpret_cast<float*>(smem);                        // [j][p][s'] (a_swizzle)
  float* s_T = s_A + 64 * 64;                                          // [t][64] (t_swizzle)
  f32x4* s_part = reinterpret_cast<f32x4*>(smem + PHIK_BYTES / 2);    // [hf][m][mm][lane] Gram partials
  InT* s_V = reinterpret_cast<InT*>(s_T + 64 * 64);                    // [t][DVP], after the partials

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int m = w & 3, hf = w >> 2;
  const int64_t h = blockIdx.y;
  int64_t b, cl;
  unsigned char* ws;
  if (p.fl_off) {
    const FlatChunk fc = flat_chunk(p, blockIdx.x);
    if (!fc.ok) return;  // a spare slot, or past the last
    b = fc.b;
    cl = fc.c;
    ws = p.ws + (h * (p.nseg + 1) + blockIdx.x) * L::bytes;
  } else {
    b = blockIdx.z;
    cl = blockIdx.x;
    if (cl >= seg_chunks(p, seq_of(p, b))) return;  // past the end of this sequence
    ws = p.ws + ((b * p.H + h) * (p.nseg + 1) + cl) * L::bytes;
  }
  const Seq sq = seq_of(p, b);
  const int64_t t0 = (p.chunk0 + cl) * CH;
  const __bf16* omega_h = p.omega + h * p.oms;
  const float ang = (p.inv_tau_head ? p.inv_tau_head[h] : p.inv_tau) * 0.15915494309189535f;
  const bool cached = p.k_plain != 0;
  auto put = [&](void* base, const frag& f) {
    if (cached) store_frag<P>(base, lane, f);
    else store_frag_nt<P>(base, lane, f);
  };

  stage_omega<D, true, 512>(omega_h, p.phase + h * p.phs, s_omega, s_phrev);
  RawRow<InT> qk[2];
  {
    const int64_t trow = t0 + 16 * m + (lane & 15);
    const bool rvalid = trow < sq.len;
    qk[0].load((const InT*)p.q + sq.q + trow * p.qs1 + h * p.qs2, rvalid, lane);
    qk[1].load((const InT*)p.k + sq.k + trow * p.ks1 + h * p.ks2, rvalid, lane);
  }
  float be = 0.f, la = 1.f;
  if (w == 0) {
    const int64_t t = t0 + lane;
    const bool valid = t < sq.len;
    be = valid ? p.beta[sq.be + t * p.bs1 + h * p.bs2] : 0.f;
    la = (valid && p.decay) ? p.decay[sq.de + t * p.ds1 + h * p.ds2] : 1.f;
  }
  lds_barrier();  // Omega staged

  // ---- beta and the in-chunk log-decay prefix (wave 0)
  if (w == 0) {
    float g = logf(fminf(fmaxf(la, 1e-5f), 1.f));
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(g, off);
      if (lane >= off) g += o;
    }
    s_beta[lane] = be;
    s_g[lane] = g;
  }

  // ---- lift q and k of tile m on feature half hf: fragment jl holds features 32 (8 hf + jl) .. + 31
  frag cqk[2][NJH];
  float ss[2];
  lift_tile<P, InT, D, true, 2, false, NJ>(qk, p.normalize, s_omega, omega_h, s_phrev, ang, lane, cqk, ss, nullptr,
                                           NJ * hf);
  if (lane < 16) {
    s_ss[hf][0][16 * m + lane] = ss[0];
    s_ss[hf][1][16 * m + lane] = ss[1];
  }
  // V pieces: first needed after the inverse; their latency hides behind the Gram
  u32x4 vraw[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = (int)threadIdx.x + 512 * i;
    const int r = idx / VPR, pc = idx % VPR;
    const int64_t t = t0 + r;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (idx < 64 * VPR && t < sq.len)
      val = *reinterpret_cast<const u32x4*>((const InT*)p.v + sq.v + t * p.vs1 + h * p.vs2 + pc * (16 / (int)sizeof(InT)));
    vraw[i] = val;
  }
  lds_barrier();  // every wave's lift has read Omega; both halves' sums of squares are in

  // ---- per-row scales of the stored (unnormalised) features (hf = 0 waves, rows of tile m)
  if (hf == 0 && lane < 16) {
    const int r = 16 * m + lane;
    const float amp = sqrtf(2.0f / (float)D);
    float sq_ = amp, sk_ = amp;
    if (!p.no_renorm) {
      sq_ = amp / (amp * sqrtf(s_ss[0][0][r] + s_ss[1][0][r]) + 1e-8f);
      sk_ = amp / (amp * sqrtf(s_ss[0][1][r] + s_ss[1][1][r]) + 1e-8f);
    }
    s_sq[r] = sq_;
    s_sk[r] = sk_;
  }
#pragma unroll
  for (int jl = 0; jl < NJH; ++jl) {
    const int jg = NJH * hf + jl;
    if (p.k_plain) put(ws + L::phiK + (size_t)(m * NJ + jg) * 64 * L::FB, cqk[1][jl]);
    else store_k_image(ws + L::phiK, m, jg, lane, cqk[1][jl]);
    if (!p.q_relift) put(ws + L::phiQ + (size_t)(m * NJ + jg) * 64 * L::FB, cqk[0][jl]);
    s_phik[(m * NJ + jg) * 64 + lane] = cqk[1][jl];
  }
  lds_barrier();

  // ---- partial Gram tiles over feature half hf: Gkk[mm][m] = K_mm K_m^T, GqkT[mm][m] = K_mm Q_m^T
  f32x4 gkk[4], gqk[4];
#pragma unroll
  for (int mm = 0; mm < 4; ++mm) { gkk[mm] = zero4(); gqk[mm] = zero4(); }
#pragma unroll
  for (int jl = 0; jl < NJH; ++jl) {
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
      const frag a = s_phik[(mm * NJ + NJH * hf + jl) * 64 + lane];
      gkk[mm] = P::mma(gkk[mm], a, cqk[1][jl]);
      gqk[mm] = P::mma(gqk[mm], a, cqk[0][jl]);
    }
  }
  lds_barrier();  // K fragments in LDS are dead from here on
#pragma unroll
  for (int mm = 0; mm < 4; ++mm) {
    if (hf == 0) s_part[(m * 4 + mm) * 64 + lane] = gqk[mm];
    else s_part[((4 + m) * 4 + mm) * 64 + lane] = gkk[mm];
  }
  lds_barrier();

  // ---- A (hf = 0) and P (hf = 1) of rows 16m .. 16m + 15, scale vectors (wave 5)
  {
    const int t = 16 * m + (lane & 15);
    const float gt = s_g[t], gtm1 = t > 0 ? s_g[t - 1] : 0.f;
    if (hf == 0) {
      // the linear rule has no erasure coupling: A = 0, so T = I below
      const float bt = p.linear ? 0.f : s_beta[t], skt = s_sk[t];
#pragma unroll
      for (int mm = 0; mm < 4; ++mm) {
        const f32x4 gk = gkk[mm] + s_part[((4 + m) * 4 + mm) * 64 + lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = 16 * mm + 4 * (lane >> 4) + i;
          const float a = (j < t) ? bt * __expf(fminf(gt - s_g[j], 0.f)) * gk[i] * skt * s_sk[j] : 0.f;
          s_A[(j * 4 + (t & 3)) * 16 + a_swizzle(j, t >> 2, t & 3)] = a;
        }
      }
    } else {
      const float sqt = s_sq[t];
      f32x4 pt[4];
#pragma unroll
      for (int mm = 0; mm < 4; ++mm) {
        const f32x4 gq = s_part[(m * 4 + mm) * 64 + lane] + gqk[mm];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = 16 * mm + 4 * (lane >> 4) + i;
          pt[mm][i] = (j < t) ? __expf(fminf(gtm1 - s_g[j], 0.f)) * gq[i] * sqt * s_sk[j] : 0.f;
        }
      }
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
        put(ws + L::Pm + (size_t)(m * 2 + jb) * 64 * L::FB, P::from_f32(pair_to8(pt[2 * jb], pt[2 * jb + 1])));
    }
  }
  if (w == 5) {
    float* vec = reinterpret_cast<float*>(ws + L::VEC);
    const float g63 = s_g[63];
    const float gtm1 = lane > 0 ? s_g[lane - 1] : 0.f;
    vec[lane] = __expf(fminf(gtm1, 0.f)) * s_sq[lane];                  // e^{g_{t-1}} * |phi_q| scale
    vec[64 + lane] = __expf(fminf(g63 - s_g[lane], 0.f)) * s_sk[lane];  // e^{g_63 - g_t} * |phi_k| scale
    if (lane == 0) vec[128] = __expf(fminf(g63, 0.f));
  }
  lds_barrier();  // A complete; the partials are read

  // ---- V staged over the partials; T = (I + A)^{-1}: diagonal blocks (waves 0-3), block columns (0-2)
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = (int)threadIdx.x + 512 * i;
    if (idx < 64 * VPR) {
      u32x2* d = reinterpret_cast<u32x2*>(s_V + (idx / VPR) * DVP + (idx % VPR) * (16 / (int)sizeof(InT)));
      d[0] = __builtin_shufflevector(vraw[i], vraw[i], 0, 1);
      d[1] = __builtin_shufflevector(vraw[i], vraw[i], 2, 3);
    }
  }
  if (w < 4) inverse_diag_block(s_A, s_T, w, lane);
  lds_barrier();
  inverse_block_columns(s_A, s_T, w, lane);
  lds_barrier();

  // ---- W~ factor T diag(beta e^g |phi_k|) (hf = 0) and U~ = T diag(beta) V (tiles n of half hf)
  {
    const int t = 16 * m + (lane & 15);
    f32x8 tb[2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      f32x8 tw;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int j0 = 32 * jb + 16 * hh + 4 * (lane >> 4);
        const f32x4 tv = *reinterpret_cast<const f32x4*>(s_T + t * 64 + t_swizzle(t, j0));
        const f32x4 bej = *reinterpret_cast<const f32x4*>(s_beta + j0);
        const f32x4 gj = *reinterpret_cast<const f32x4*>(s_g + j0);
        const f32x4 sk = *reinterpret_cast<const f32x4*>(s_sk + j0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          tw[4 * hh + i] = p.linear ? 0.f : tv[i] * bej[i] * __expf(gj[i]) * sk[i];  // linear: E = U~
          tb[jb][4 * hh + i] = tv[i] * bej[i];
        }
      }
      if (hf == 0) put(ws + L::Tp + (size_t)(m * 2 + jb) * 64 * L::FB, P::from_f32(tw));
    }
#pragma unroll
    for (int nn = 0; nn < NVH; ++nn) {
      const int n = NVH * hf + nn;
      if (n >= NV) break;
      f32x4 acc = zero4();
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        // hi + lo split of T diag(beta): V is exact in bf16, so U~ keeps ~16 bits
        bf16x8 hi, lo, vb;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          hi[s] = (__bf16)tb[jb][s];
          lo[s] = (__bf16)(tb[jb][s] - (float)hi[s]);
          vb[s] = s_V[(32 * jb + kappa(lane, s)) * DVP + 16 * n + (lane & 15)];
        }
        acc = PrecBF16::mma(acc, hi, vb);
        acc = PrecBF16::mma(acc, lo, vb);
      }
      f32x4* ud = reinterpret_cast<f32x4*>(ws + L::U + ((size_t)(m * NV + n) * 64 + lane) * 16);
      if (cached) *ud = acc;
      else __builtin_nontemporal_store(acc, ud);
    }
  }
}

template <class P, typename InT, int D, int DV>
int launch_prep(const ScanParams& p, hipStream_t st) {
  const int fm = p.prelifted ? FM_PRELIFTED : (p.omega_lo ? FM_HILO : FM_EXACT);
  const int run_t = fm == FM_PRELIFTED ? PrepRun<P, FM_PRELIFTED>::value
                  : fm == FM_HILO ? PrepRun<P, FM_HILO>::value : PrepRun<P, FM_EXACT>::value;
  const int run = run_t ? run_t : p.prep_run;
  const dim3 prep_grid = p.fl_off ? dim3((unsigned)p.nseg, (unsigned)p.H, 1u)
                                  : dim3((unsigned)((p.nseg + run - 1) / run), (unsigned)p.H, (unsigned)p.B);
  if (fm == FM_PRELIFTED) hipLaunchKernelGGL((prep_kernel<P, InT, D, DV, FM_PRELIFTED>), prep_grid, dim3(256), 0, st, p);
  else if (fm == FM_HILO) hipLaunchKernelGGL((prep_kernel<P, InT, D, DV, FM_HILO>), prep_grid, dim3(256), 0, st, p);
  else if (p.prep_no_q) hipLaunchKernelGGL((prep_kernel<P, InT, D, DV, FM_EXACT, true>), prep_grid, dim3(256), 0, st, p);
  else if constexpr (IsBF16<P>::value && D == 512) hipLaunchKernelGGL((prep8_kernel<DV>), prep_grid, dim3(512), 0, st, p);
  else hipLaunchKernelGGL((prep_kernel<P, InT, D, DV, FM_EXACT>), prep_grid, dim3(256), 0, st, p);
  return hipGetLastError() == hipSuccess ? KDN_OK : KDN_ERR_DEVICE;
}

#define KDN_PREP_INST(P, InT, DV) template int launch_prep<P, InT, 512, DV>(const ScanParams&, hipStream_t);
KDN_PREP_INST(PrecBF16, __bf16, 16)
KDN_PREP_INST(PrecBF16, __bf16, 32)
KDN_PREP_INST(PrecBF16, __bf16, 64)
KDN_PREP_INST(PrecBF16, __bf16, 128)
KDN_PREP_INST(PrecF32, float, 16)
KDN_PREP_INST(PrecF32, float, 32)
KDN_PREP_INST(PrecF32, float, 64)
KDN_PREP_INST(PrecF32, float, 128)
#undef KDN_PREP_INST

}  // namespace kdn
