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
// Three kernels per segment of chunks (the split schedule), so that the only sequential kernel streams as
// few bytes per chunk as possible (64 KB of K per chunk and head):
//   prep   (one workgroup per chunk and head; kdn_prep.hip): lift q and k on MFMA, Gram matrices, the
//          triangular inverse and every S-independent factor; writes K, Tp = T diag(beta e^g |phi_k|),
//          P, U~ and per-token scale vectors to the workspace in MFMA-fragment order.
//   state  (one workgroup per head and 16 value components, sequential over chunks): X_K = K S^T,
//          E = U~ - Tp X_K and the state update; checkpoints each chunk's starting S^T and E.
//   output (one workgroup per chunk and head): Y = diag(qscale) Q S^T + P E.
// The fused schedule (kdn_chain.hip) runs prep and one sequential kernel that forms Y as well.
// The lifted features are stored unnormalised (cos values); per-row norms are folded into the small
// per-token scale vectors, so a lift never has to hold a whole row before using it.
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <vector>
#include "kdn_frag.hpp"
#include "kdn_internal.hpp"
#include "kdn_io.hpp"
#include "kdn_scan_common.hpp"
#include "kdn_lift_tile.hpp"

namespace kdn {

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
//         (features 16h .. 16h+15 of the 32-block) at (fragment * 64 + kimg_swizzle(lane)) * 8, the
//         layout of the record's K image (bank-conflict-free for the plain and the transposed read).
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
      *reinterpret_cast<bf16x4*>(base + (size_t)(fi * 64 + kimg_swizzle(lane)) * 8) =
          __builtin_shufflevector(ak[m][jj], ak[m][jj], 0, 1, 2, 3);
      *reinterpret_cast<bf16x4*>(base + 8192 + (size_t)(fi * 64 + kimg_swizzle(lane)) * 8) =
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
  // is half (tl & 1) of fragment (c >> 4, tl >> 1), lane (c & 15) + 16 (j & 3), i.e. plane (tl & 1), at
  // that lane's swizzled slot.
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
    const unsigned char* a = plane + (size_t)(((c >> 4) * 4 + (tl >> 1)) * 64 + kimg_swizzle((c & 15) + 16 * (j & 3))) * 8;
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
  store_e_tile<P>(cur + L::Eck, (size_t)(w * NV + n), lane, e);
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
  int64_t b, h, nloc, cfirst;
  size_t woff;
  if (!state_item<L::bytes>(p, hb, b, h, nloc, woff, cfirst)) return;
  const int64_t sl = p.slots ? (int64_t)p.slots[b] : b;
  if (sl < 0) return;  // a skipped sequence of a ragged step (its state is not touched)

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

  unsigned char* wsh = p.ws + woff;
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
// state (bf16, D = 512): the carry of state_kernel with each chunk's lifted keys streamed by a fifth
// wave.  Waves 0-3 carry the state as state_kernel does (wave w owns features [128w, 128w + 128) of the
// workgroup's 16 state rows; the same products in the same order, so the results are identical).  Wave 4
// copies each chunk's K image (64 KB, written by prep in the LDS layout, store_k_image) into a two-slot
// LDS ring with global_load_lds_dwordx4 one chunk ahead, and touches the records L2_AHEAD chunks ahead
// so that the copies hit L2.  The carry waves issue no load of K (a burst of 24 such loads per wave and
// chunk stalled their in-order issue): their vector-memory traffic is the small per-chunk operands (a
// register ring two chunks ahead) and the checkpoint stores.  Four barriers per chunk:
//   phase 1: checkpoint S^T, X_K partial from the ring        | A
//   reduce X_K token tile w                                   | B
//   E tile w = U~ - Tp X_K (checkpointed), refill small ops   | C
//   S^T <- gammaC S^T + K^T (kscale o E), K^T from the ring   | D
// Slot c % 2 is read from phase 1 to the update of chunk c; the copy of chunk c+1 into the other slot is
// issued after barrier D of chunk c-1, and the loader waits for it before barrier D of chunk c.
__device__ __forceinline__ PrecBF16::frag kimg_frag(const unsigned char* kw, int lane, int m, int jj) {
  typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
  const unsigned char* a = kw + (size_t)((m * 4 + jj) * 64 + kimg_swizzle(lane)) * 8;
  const bf16x4 lo = *reinterpret_cast<const bf16x4*>(a);
  const bf16x4 hi = *reinterpret_cast<const bf16x4*>(a + KIMG_PLANE);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// s_waitcnt for at most n outstanding vector-memory operations (other counters left alone).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <int DV>
struct DmaState {
  using O = StateOps<PrecBF16, 512, DV>;
  using L = typename O::L;
  static constexpr int NV = DV / 16;
  static constexpr int KIMG = 4 * KIMG_SLICE;  // bytes of a chunk's K image
  // dword loads of the L2 prefetch per loader wave: one per 128-byte line of the operand area [0, Sfr),
  // shared by the NV workgroups of a head
  static constexpr int L2_LOADS = (int)((L::Sfr / 128 + 64 * NV - 1) / (64 * NV));
  __device__ static void load_small(const unsigned char* ws, int w, int lane, int n, typename O::Small& sm) {
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) sm.tp[jb] = load_frag<PrecBF16>(ws + L::Tp + (size_t)(w * 2 + jb) * 64 * L::FB, lane);
    sm.u = *reinterpret_cast<const f32x4*>(ws + L::U + ((size_t)(w * NV + n) * 64 + lane) * 16);
    sm.ks = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(ws + L::VEC) + 64 + 16 * w + 4 * (lane >> 4));
    sm.gC = reinterpret_cast<const float*>(ws + L::VEC)[128];
  }
  // The loader wave's copy of one chunk's K image into a ring slot: 64 instructions of 1 KB.
  __device__ static void copy_k(const unsigned char* src, unsigned char* slot, int lane) {
#pragma unroll
    for (int i = 0; i < KIMG / 1024; ++i)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src + (size_t)i * 1024 + lane * 16),
                                       (__attribute__((address_space(3))) void*)(slot + i * 1024), 16, 0, 0);
  }
};

// One chunk of a carry wave (four barriers); kw is the wave's slice of the ring slot holding the chunk,
// sm its small operands, refilled here with those of chunk min(cl + 2, last).
template <int DV, bool DECAY>
__device__ __forceinline__ void dma_step(StateShared& sh, const unsigned char* kw, unsigned char* wsh, int64_t cl,
                                         int w, int lane, int n, f32x4 (&S)[8], typename StateOps<PrecBF16, 512, DV>::Small& sm,
                                         int64_t nloc) {
  using P = PrecBF16;
  using Dm = DmaState<DV>;
  using L = typename Dm::L;
  using frag = P::frag;
  constexpr int NV = Dm::NV;
  unsigned char* cur = wsh + cl * L::bytes;
  // phase 1: checkpoint of the chunk-start S^T, X_K partial over the wave's 128 features
  frag sf[4];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    sf[jj] = P::from_f32(pair_to8(S[2 * jj], S[2 * jj + 1]));
    store_frag<P>(cur + L::Sfr + (size_t)((4 * w + jj) * NV + n) * 64 * L::FB, lane, sf[jj]);
  }
  f32x4 xp[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    xp[m] = zero4();
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) xp[m] = P::mma(xp[m], kimg_frag(kw, lane, m, jj), sf[jj]);
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) sh.xp[w][m][lane] = xp[m];
  __syncthreads();  // A
  sh.x[w][lane] = sh.xp[0][w][lane] + sh.xp[1][w][lane] + sh.xp[2][w][lane] + sh.xp[3][w][lane];
  __syncthreads();  // B
  f32x4 ek = zero4();
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) ek = P::mma(ek, sm.tp[jb], P::from_f32(pair_to8(sh.x[2 * jb][lane], sh.x[2 * jb + 1][lane])));
  const f32x4 e = sm.u - ek;
  sh.e[w][lane] = e * sm.ks;
  store_e_tile<P>(cur + L::Eck, (size_t)(w * NV + n), lane, e);
  const float gC = sm.gC;
  Dm::load_small(wsh + ((cl + 2 < nloc) ? cl + 2 : nloc - 1) * L::bytes, w, lane, n, sm);
  __syncthreads();  // C
  frag eb[2];
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) eb[jb] = P::from_f32(pair_to8(sh.e[2 * jb][lane], sh.e[2 * jb + 1][lane]));
  const frag* kl = reinterpret_cast<const frag*>(kw);
#pragma unroll
  for (int tl = 0; tl < 8; ++tl) {
    f32x4 acc = S[tl];
    if constexpr (DECAY) acc = acc * gC;  // without decay gammaC is exactly 1
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) acc = P::mma(acc, kt_frag<P>(kl, lane, tl, jb), eb[jb]);
    S[tl] = acc;
  }
  __syncthreads();  // D
}

template <int DV, bool DECAY>
__global__ void __launch_bounds__(320) state_kernel_dma(ScanParams p) {
  using P = PrecBF16;
  using Dm = DmaState<DV>;
  using O = typename Dm::O;
  using L = typename Dm::L;
  constexpr int NV = Dm::NV;
  __shared__ StateShared sh;
  __shared__ __attribute__((aligned(16))) unsigned char s_ring0[Dm::KIMG];
  __shared__ __attribute__((aligned(16))) unsigned char s_ring1[Dm::KIMG];
  __shared__ __attribute__((aligned(16))) unsigned s_sink[64];  // target of the loader's L2-prefetch copies

  // the XCD-aware grid decomposition and early exits of state_kernel (uniform per workgroup)
  const int64_t id = blockIdx.x;
  const int64_t xcd = id & 7, jdx = id >> 3;
  const int n = (int)(jdx % NV);
  const int64_t hb = (jdx / NV) * 8 + xcd;
  if (hb >= p.B * p.H) return;
  int64_t b, h, nloc, cfirst;
  size_t woff;
  if (!state_item<L::bytes>(p, hb, b, h, nloc, woff, cfirst)) return;
  const int64_t sl = p.slots ? (int64_t)p.slots[b] : b;
  if (sl < 0) return;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  unsigned char* wsh = p.ws + woff;

  if (w == 4) {
    // loader: barrier P after chunk 0 has landed, then per chunk A, B, C, (copy of the next chunk
    // complete) D -- the carry waves' barriers, one for one
    if (nloc == 0) return;
    Dm::copy_k(wsh, s_ring0, lane);
    // The loader's barriers are bare s_barrier: __syncthreads() adds a workgroup release fence, for which
    // the compiler drains every outstanding copy into LDS; the loader orders its copies itself instead
    // (vmcnt waits before P and D), and it touches no LDS that another wave writes.
    wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();  // P
    for (int64_t cl = 0; cl < nloc; ++cl) {
      if (cl + 1 < nloc) Dm::copy_k(wsh + (cl + 1) * L::bytes, ((cl + 1) & 1) ? s_ring1 : s_ring0, lane);
      // L2 prefetch: one dword per 128-byte line of the operand area of chunk cl + 1 + L2_AHEAD, each lane
      // its own line, copied into a scratch LDS word (no register result, so nothing waits for it)
      const int64_t cp = (cl + 1 + O::L2_AHEAD < nloc) ? cl + 1 + O::L2_AHEAD : nloc - 1;
      const unsigned char* pb = wsh + cp * L::bytes;
#pragma unroll
      for (int i = 0; i < Dm::L2_LOADS; ++i) {
        const size_t off = ((size_t)((i * NV + n) * 64 + lane)) * 128;
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(pb + (off < L::Sfr ? off : 0)),
                                         (__attribute__((address_space(3))) void*)s_sink, 4, 0, 0);
      }
      __builtin_amdgcn_s_barrier();  // A
      __builtin_amdgcn_s_barrier();  // B
      __builtin_amdgcn_s_barrier();  // C
      wait_vmcnt<Dm::L2_LOADS>();    // the copy has landed (only the prefetches issued after it may be pending)
      __builtin_amdgcn_s_barrier();  // D
    }
    return;
  }

  const int r = 16 * n + (lane & 15);
  f32x4 S[8];
  if (p.state_in) {
    const float* si = p.state_in + sl * p.is0 + h * p.is1 + r * p.is3;
#pragma unroll
    for (int tl = 0; tl < 8; ++tl)
#pragma unroll
      for (int i = 0; i < 4; ++i) S[tl][i] = si[(int64_t)(16 * (8 * w + tl) + 4 * (lane >> 4) + i) * p.is2];
  } else {
#pragma unroll
    for (int tl = 0; tl < 8; ++tl) S[tl] = zero4();
  }
  if (nloc > 0) {
    typename O::Small sm0, sm1;
    Dm::load_small(wsh, w, lane, n, sm0);
    Dm::load_small(wsh + (nloc > 1 ? L::bytes : 0), w, lane, n, sm1);
    __syncthreads();  // P: slot 0 holds chunk 0
    for (int64_t cl = 0; cl < nloc; cl += 2) {
      dma_step<DV, DECAY>(sh, s_ring0 + w * KIMG_SLICE, wsh, cl, w, lane, n, S, sm0, nloc);
      if (cl + 1 >= nloc) break;
      dma_step<DV, DECAY>(sh, s_ring1 + w * KIMG_SLICE, wsh, cl + 1, w, lane, n, S, sm1, nloc);
    }
  }
  float* so = p.state_out + sl * p.os0 + h * p.os1 + r * p.os3;
#pragma unroll
  for (int tl = 0; tl < 8; ++tl)
#pragma unroll
    for (int i = 0; i < 4; ++i) so[(int64_t)(16 * (8 * w + tl) + 4 * (lane >> 4) + i) * p.os2] = S[tl][i];
}

// ------------------------------------------------------------------------------------------------
// output: 256 threads per workgroup, workgroup i taking (chunk, head, sequence) items i, i + grid, ...
// (one item each with a grid of nseg * H * B).  Y = diag(qscale) Q S_c^T + P E for one (chunk, head).
// Wave w keeps the lifted query fragments of token tile w (read back from the record) in registers.
// The chunk-start S^T fragments are staged in LDS, NG value tiles per pass, and read by all four waves.  Each wave assembles its 16 x d_v block of Y in a wave-private LDS tile and writes
// whole rows with 16-byte stores.  Every operand is read once: streaming loads.
template <class P, int D, int DV>
struct OutputLds {
  static constexpr int NJ = D / 32, NV = DV / 16;
  static constexpr int NG0 = IsBF16<P>::value ? 2 : 1;  // value tiles per LDS pass (32 KB of S fragments)
  static constexpr int NG = NV < NG0 ? NV : NG0;
  static constexpr int YS = DV + 4;                     // padded row of the Y tile
  static constexpr size_t bytes = (size_t)NJ * NG * 64 * P::frag_bytes + (size_t)4 * 16 * YS * 4;
};

//
// RELIFT (the resident form beside the state chain, bf16, one shared exact Omega): instead of reading the
// record's Q fragments (64 KB per item, written by prep), the workgroup stages Omega and the phases in LDS
// once and lifts its q rows again per item, with the code and inputs that prep's lift uses, so the
// fragments are the same bits; 120 KB less HBM traffic per (head, chunk) beside the chain.
template <class P, typename OutT, int D, int DV, bool RELIFT = false>
__global__ void __launch_bounds__(256) output_kernel(ScanParams p) {
  using L = WsLayout<P, D, DV>;
  using frag = typename P::frag;
  using O = OutputLds<P, D, DV>;
  constexpr int NJ = O::NJ, NV = O::NV, NG = O::NG, YS = O::YS;
  static_assert(!RELIFT || (IsBF16<P>::value && D == 512), "the q re-lift is the bf16 D = 512 path's");
  __shared__ frag s_s[NJ * NG * 64];
  __shared__ __attribute__((aligned(16))) float s_y[4][16 * YS];
  __shared__ bf16x8 s_om[RELIFT ? (D / 16) * 2 * 64 : 1];
  __shared__ __attribute__((aligned(16))) float s_phr[RELIFT ? D : 1];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if constexpr (RELIFT) {
    stage_omega<D, true>(p.omega, p.phase, s_om, s_phr);
    __syncthreads();
  }
  const int64_t items = p.nseg * p.H * (p.fl_off ? 1 : p.B);
  for (int64_t it = blockIdx.x; it < items; it += gridDim.x) {
  if (it != (int64_t)blockIdx.x) __syncthreads();  // the previous item's LDS tiles have been read
  const int64_t x = it % p.nseg, h = (it / p.nseg) % p.H;
  // chunk cl (chunk0 + cl in the sequence) of sequence b, its record at ws
  int64_t b, cl;
  const unsigned char* ws;
  if (p.fl_off) {
    const FlatChunk fc = flat_chunk(p, x);
    if (!fc.ok) continue;  // a spare slot, or past the last
    b = fc.b;
    cl = fc.c;
    ws = p.ws + (h * (p.nseg + 1) + x) * L::bytes;
  } else {
    b = it / (p.nseg * p.H);
    cl = x;
    if (cl >= seg_chunks(p, seq_of(p, b))) continue;  // past the end of this sequence (ragged batches)
    ws = p.ws + ((b * p.H + h) * (p.nseg + 1) + cl) * L::bytes;
  }
  const Seq sq = seq_of(p, b);
  const int64_t t0 = (p.chunk0 + cl) * CH;
  const float* vec = reinterpret_cast<const float*>(ws + L::VEC);

  frag aq[NJ];
  if constexpr (RELIFT) {
    // the lifted queries of token tile w, as prep lifts them (unnormalised cos values; the per-row
    // scale comes from the record)
    const int64_t trow = t0 + 16 * w + (lane & 15);
    RawRow<__bf16> raw[1];
    raw[0].load((const __bf16*)p.q + sq.q + trow * p.qs1 + h * p.qs2, trow < sq.len, lane);
    const float ang = (p.inv_tau_head ? p.inv_tau_head[h] : p.inv_tau) * 0.15915494309189535f;
    frag cq[1][NJ];
    float ssq[1];
    lift_tile<P, __bf16, D, true, 1>(raw, p.normalize, s_om, p.omega, s_phr, ang, lane, cq, ssq);
#pragma unroll
    for (int j = 0; j < NJ; ++j) aq[j] = cq[0][j];
  } else {
#pragma unroll
    for (int j = 0; j < NJ; ++j) aq[j] = load_frag_nt<P>(ws + L::phiQ + (size_t)(w * NJ + j) * 64 * L::FB, lane);
  }
  frag pf[2];
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) pf[jb] = load_frag_nt<P>(ws + L::Pm + (size_t)(w * 2 + jb) * 64 * L::FB, lane);
  const f32x4 qs = *reinterpret_cast<const f32x4*>(vec + 16 * w + 4 * (lane >> 4));
  float* yt = s_y[w];

  for (int n0 = 0; n0 < NV; n0 += NG) {
    if (n0 > 0) __syncthreads();  // the previous pass's fragments have been read
    for (int idx = threadIdx.x; idx < NJ * NG * 64; idx += 256) {
      const int l = idx & 63, g = (idx >> 6) % NG, j = idx / (64 * NG);
      s_s[idx] = load_frag_nt<P>(ws + L::Sfr + (size_t)(j * NV + n0 + g) * 64 * L::FB, l);
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
      for (int jb = 0; jb < 2; ++jb)
        eb[jb] = load_e_frag<P>(ws + L::Eck, (size_t)((2 * jb) * NV + n), (size_t)((2 * jb + 1) * NV + n), lane);
      f32x4 y = zero4();
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) y = P::mma(y, pf[jb], eb[jb]);
#pragma unroll
      for (int i = 0; i < 4; ++i) yt[(4 * (lane >> 4) + i) * YS + 16 * n + (lane & 15)] = y[i] + qs[i] * xq[i];
    }
  }
  // Rows of the wave's tile: (16 rows) x (DV / 8 pieces of 8 elements); the tile was written by this
  // wave only.
  wave_lds_sync();
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
}

static inline unsigned state_grid(int64_t B, int64_t H, int nv) { return (unsigned)(8 * ((B * H + 7) / 8) * nv); }

// ------------------------------------------------------------------------------------------------
// PHASE_PREP_FUSED is prep writing the fused chain's record layout (K as plain fragments, Q stored).
enum Phase { PHASE_PREP = 1, PHASE_STATE = 2, PHASE_OUTPUT = 4, PHASE_ALL = 7, PHASE_CHAIN = 8, PHASE_PREP_FUSED = 16 };

// Two schedules for a whole-scan call with bf16 inputs:
//  - split: prep / state / output (the state kernel streams only K, 64 KB per chunk, through its LDS ring;
//    the output kernel reads the state checkpoints);
//  - fused: prep + the fused chain (kdn_chain.hip: state update and readout in one sequential kernel, no
//    output kernel and no checkpoints; each chain workgroup streams K and Q, 128 KB per chunk).
// With few heads the chain is a latency-bound sequence of steps, and the split schedule's shorter step
// wins (config 3, 16 heads: 2.7 against 5.3 ms); once the split schedule's state workgroups (4 per head at
// d_v = 64) fill the GPU the layer is throughput-bound and the fused one wins (B = 32, H = 16, T = 16384:
// 13.0 against 16.1 ms).  KDN_SCAN_SCHEDULE=split / fused overrides the choice (tuning and tests).
// fp32 inputs and the phase entry points always run the split kernels.
template <class P, int D>
struct Fused : std::integral_constant<bool, IsBF16<P>::value && D == 512> {};

static bool use_fused(const kdn_scan_args* a) {
  const char* e = getenv("KDN_SCAN_SCHEDULE");  // read per call, so that a process can switch it
  if (e && !strcmp(e, "fused")) return true;
  if (e && !strcmp(e, "split")) return false;
  const int cus = device_cus();
  return cus > 0 && (int64_t)state_grid(a->B, a->H, a->d_v / 16) >= cus;
}

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
  p.fl_off = nullptr;
  p.fl_first = nullptr;
  p.fl_total = nullptr;
  p.fl_lo = 0;
  p.fl_nseq = 0;
  p.prep_no_q = 0;
  p.k_plain = 0;
  p.q_relift = 0;
  p.prep_run = 0;
  p.out_wgs = 0;
  return p;
}

// Chunks per prep workgroup for given (pre-lifted) features, whose prep workgroup holds a CU alone, so
// that the kernel runs in ceil(workgroups / CUs) rounds, each costing a fixed start-up (about 0.3 of a
// chunk) plus `run` chunks.  Pick the run length (1..8) with the least total for the CUs left free (all
// of them, or those the concurrent state kernel does not occupy).  The lifting prep kernels take one
// chunk per workgroup.
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
  // packed windows instead of segments (the sequences' layout planned on the device)
  const FlatPlan* flat = nullptr;
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
  p.out_wgs = 0;
  if (c0 == 0) {
    p.state_in = a->initial_state;
    p.is0 = a->init_stride[0]; p.is1 = a->init_stride[1]; p.is2 = a->init_stride[2]; p.is3 = a->init_stride[3];
  } else {
    p.state_in = a->final_state;
    p.is0 = p.os0; p.is1 = p.os1; p.is2 = p.os2; p.is3 = p.os3;
  }
  return p;
}

// Parameters of packed window s (slots [s * win, (s + 1) * win)) with its records at `ws`: the states
// are read and written in place (initial_state is final_state).
static ScanParams flat_params(const kdn_scan_args* a, const RunSpec& r, int64_t s, void* ws) {
  ScanParams p = fill_params(a);
  p.seq_lo = r.seq_lo;
  p.seq_hi = r.seq_hi;
  p.chunk0 = 0;
  p.nseg = r.flat->win;
  p.ws = (unsigned char*)ws;
  p.prep_run = 1;
  p.out_wgs = 0;
  p.state_in = a->final_state;
  p.is0 = p.os0; p.is1 = p.os1; p.is2 = p.os2; p.is3 = p.os3;
  p.fl_off = r.flat->off;
  p.fl_first = r.flat->first;
  p.fl_total = r.flat->total;
  p.fl_lo = s * r.flat->win;
  p.fl_nseq = r.flat->nseq;
  return p;
}

// The state kernel keeps its CU to itself: 40 KB of unused dynamic LDS raise its request to 128 KB, so
// that neither a prep workgroup (~131 KB) nor an output workgroup (~49 KB) fits beside it in the CU's
// 160 KB and takes issue slots from the sequential chain.
constexpr int STATE_EXCLUSIVE_LDS = 40 * 1024;

template <class P, typename InT, typename OutT, int D, int DV>
static int launch_phase(const ScanParams& p, int phase, hipStream_t st) {
  if (phase == PHASE_PREP) {
    return launch_prep<P, InT, D, DV>(p, st);
  } else if (phase == PHASE_CHAIN) {
    if constexpr (Fused<P, D>::value) return launch_chain<OutT, DV>(p, st);
    return KDN_ERR_UNSUPPORTED;
  } else if (phase == PHASE_STATE) {
    // The state workgroups are the sequential critical path: reserve enough LDS that no prep or output
    // workgroup can share their CU (a CU has 160 KB; the bf16 state kernel uses 88 KB statically).
    // (bf16: the streaming kernel's 152 KB of LDS keep its CU exclusive by themselves.)
    if constexpr (IsBF16<P>::value && D == 512) {
      if (p.decay) hipLaunchKernelGGL((state_kernel_dma<DV, true>), dim3(state_grid(p.B, p.H, DV / 16)), dim3(320), 0, st, p);
      else hipLaunchKernelGGL((state_kernel_dma<DV, false>), dim3(state_grid(p.B, p.H, DV / 16)), dim3(320), 0, st, p);
    } else {
      const size_t excl = IsBF16<P>::value ? (size_t)STATE_EXCLUSIVE_LDS : 0;
      if (p.decay) hipLaunchKernelGGL((state_kernel<P, D, DV, true>), dim3(state_grid(p.B, p.H, DV / 16)), dim3(256), excl, st, p);
      else hipLaunchKernelGGL((state_kernel<P, D, DV, false>), dim3(state_grid(p.B, p.H, DV / 16)), dim3(256), excl, st, p);
    }
  } else {
    // Beside the state kernel (p.out_wgs > 0): at most one workgroup per CU it leaves free, each CU held
    // alone (LDS padded past half a CU), all resident from the start.  The state kernel of the next
    // segment becomes ready together with this one, and needs whole CUs: a grid of one workgroup per
    // (chunk, head) took every free CU and held up a quarter of its workgroups by ~55 us per segment
    // (config 3: 2.59 against 2.41 ms per layer, measured with clock stamps).
    const int64_t items = (int64_t)p.nseg * p.H * (p.fl_off ? 1 : p.B);
    if constexpr (IsBF16<P>::value && D == 512) {
      if (p.q_relift) {
        // prep stored no Q for this segment: the re-lifting form, whatever the item count (Omega and the
        // phases in LDS make the workgroup more than half a CU: no pad needed)
        const int64_t grid = p.out_wgs < items ? p.out_wgs : items;
        hipLaunchKernelGGL((output_kernel<P, OutT, D, DV, true>), dim3((unsigned)grid), dim3(256), 0, st, p);
        return hipGetLastError() == hipSuccess ? KDN_OK : KDN_ERR_DEVICE;
      }
    }
    if (p.out_wgs > 0 && p.out_wgs < items) {
      constexpr size_t excl = CU_LDS_BYTES / 2 + 1024;
      const size_t pad = OutputLds<P, D, DV>::bytes < excl ? excl - OutputLds<P, D, DV>::bytes : 0;
      hipLaunchKernelGGL((output_kernel<P, OutT, D, DV>), dim3((unsigned)p.out_wgs), dim3(256), pad, st, p);
    } else {
      hipLaunchKernelGGL((output_kernel<P, OutT, D, DV>), dim3((unsigned)items), dim3(256), 0, st, p);
    }
  }
  return hipGetLastError() == hipSuccess ? KDN_OK : KDN_ERR_DEVICE;
}

// Runs chunks [c_begin, c_end) in segments of `seg` chunks, all in one workspace buffer: per segment the
// selected kernels, in the order prep, state, output (split) or prep, chain (fused).  A whole-scan call
// (PHASE_ALL) takes the schedule use_fused() picks.
template <class P, typename InT, typename OutT, int D, int DV>
static int run_scan(const kdn_scan_args* a, const RunSpec& r) {
  const int cus = device_cus();
  if (r.flat) {  // packed windows, one after another
    const bool fused = Fused<P, D>::value && r.phases == PHASE_ALL && use_fused(a);
    for (int64_t s = 0; s < r.flat->nwin; ++s) {
      ScanParams p = flat_params(a, r, s, a->workspace);
      p.k_plain = fused ? 1 : 0;
      for (int ph : {PHASE_PREP, PHASE_STATE, PHASE_CHAIN, PHASE_OUTPUT}) {
        if ((ph == PHASE_CHAIN) != fused && ph != PHASE_PREP) continue;
        const int rc = launch_phase<P, InT, OutT, D, DV>(p, ph, r.st);
        if (rc != KDN_OK) return rc;
      }
    }
    return KDN_OK;
  }
  int phases = r.phases;
  if (phases == PHASE_ALL && Fused<P, D>::value && use_fused(a)) phases = PHASE_PREP_FUSED | PHASE_CHAIN;
  for (int64_t c0 = r.c_begin; c0 < r.c_end; c0 += r.seg) {
    ScanParams p = segment_params(a, r, c0, (r.c_end - c0 < r.seg) ? (r.c_end - c0) : r.seg, a->workspace, cus);
    if (phases & (PHASE_PREP_FUSED | PHASE_CHAIN)) p.k_plain = 1;
    for (int ph : {PHASE_PREP, PHASE_PREP_FUSED, PHASE_STATE, PHASE_CHAIN, PHASE_OUTPUT}) {
      if (!(phases & ph)) continue;
      const int rc = launch_phase<P, InT, OutT, D, DV>(p, ph == PHASE_PREP_FUSED ? PHASE_PREP : ph, r.st);
      if (rc != KDN_OK) return rc;
    }
  }
  return KDN_OK;
}

// Segment starts of the pipelined split schedule (nsegs + 1 entries).  With at least three segments'
// worth of chunks the first two segments take seg / 4 and seg / 2 chunks and the last two seg / 2 and
// seg / 4: the first prep and the last output run alone, and short segments there shorten the layer's
// head and tail; each prep still fits beside the state launch before it (prep takes about half a state
// launch's time per chunk).  The chunks and the state carried between segments are the same for any
// boundaries, so the results do not depend on them.
static std::vector<int64_t> split_bounds(int64_t nchunks, int64_t seg) {
  std::vector<int64_t> b{0};
  auto add = [&](int64_t n) { if (n > 0) b.push_back(b.back() + n); };
  if (seg >= 4 && nchunks >= 3 * seg) {
    const int64_t q = seg / 4, hh = seg / 2;
    add(q);
    add(hh);
    const int64_t rest = nchunks - 2 * (q + hh);
    for (int64_t i = 0; i < rest / seg; ++i) add(seg);
    add(rest % seg);
    add(hh);
    add(q);
  } else {
    for (int64_t c = 0; c < nchunks; c += seg) add(nchunks - c < seg ? nchunks - c : seg);
  }
  return b;
}

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
  const std::vector<int64_t> bounds = r.flat ? std::vector<int64_t>{} : split_bounds(nchunks, seg);
  const int64_t nsegs = r.flat ? r.flat->nwin : (int64_t)bounds.size() - 1;
  EventSet evs;
  int rc = evs.create(3 * nbuf + 2);
  if (rc != KDN_OK) return rc;
  hipEvent_t* evP = evs.ev;
  hipEvent_t* evS = evs.ev + nbuf;
  hipEvent_t* evO = evs.ev + 2 * nbuf;
  hipEvent_t evIn = evs.ev[3 * nbuf], evOut = evs.ev[3 * nbuf + 1];
  // prep and output share the device with the state kernel's workgroups (one per CU)
  const int prep_cus = device_cus() - (int)state_grid(a->B, a->H, DV / 16);
  auto seg_p = [&](int64_t s) {
    void* buf = (unsigned char*)a->workspace + (size_t)(s % nbuf) * buf_bytes;
    ScanParams p = r.flat ? flat_params(a, r, s, buf)
                          : segment_params(a, r, bounds[s], bounds[s + 1] - bounds[s], buf, prep_cus);
    p.out_wgs = prep_cus > 0 ? prep_cus : 0;
    // the resident output workgroups lift q again (one shared exact bf16 Omega and phases): prep stores
    // no Q fragments
    p.q_relift = (IsBF16<P>::value && D == 512 && p.out_wgs > 0 && !p.prelifted && !p.omega_lo && p.oms == 0 &&
                  p.phs == 0) ? 1 : 0;
    return p;
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

// The fused schedule: the chain of segment s runs on `st` while prep of segment s + 1 runs on `aux`;
// segments rotate through `nbuf` >= 2 workspace buffers.
//   chain(s) waits for prep(s)                 (event P[s % nbuf])
//   prep(s)  waits for chain(s - nbuf), the last reader of its buffer (event C[s % nbuf])
// aux first waits for the work already queued on st; the last chain, on st, ends the call.
template <class P, typename InT, typename OutT, int D, int DV>
static int run_pipelined_fused(const kdn_scan_args* a, const RunSpec& r) {
  const int64_t seg = r.seg;
  const int nbuf = r.nbuf;
  const hipStream_t st = r.st, aux = r.aux;
  const int64_t nchunks = (a->T + CH - 1) / CH;
  const int64_t nsegs = r.flat ? r.flat->nwin : (nchunks + seg - 1) / seg;
  EventSet evs;
  int rc = evs.create(2 * nbuf + 1);
  if (rc != KDN_OK) return rc;
  hipEvent_t* evP = evs.ev;
  hipEvent_t* evC = evs.ev + nbuf;
  hipEvent_t evIn = evs.ev[2 * nbuf];
  const int prep_cus = device_cus() - (int)(a->B * a->H * (DV / (DV >= 32 ? 32 : 16)));
  auto seg_p = [&](int64_t s) {
    const int64_t c0 = s * seg;
    void* buf = (unsigned char*)a->workspace + (size_t)(s % nbuf) * r.buf_bytes;
    ScanParams p = r.flat ? flat_params(a, r, s, buf)
                          : segment_params(a, r, c0, (nchunks - c0 < seg) ? (nchunks - c0) : seg, buf, prep_cus);
    p.k_plain = 1;
    return p;
  };
#define KDN_TRY(x) do { if ((x) != hipSuccess) return KDN_ERR_DEVICE; } while (0)
#define KDN_TRYK(x) do { const int _rc = (x); if (_rc != KDN_OK) return _rc; } while (0)
  KDN_TRY(hipEventRecord(evIn, st));
  KDN_TRY(hipStreamWaitEvent(aux, evIn, 0));
  KDN_TRYK((launch_phase<P, InT, OutT, D, DV>(seg_p(0), PHASE_PREP, aux)));
  KDN_TRY(hipEventRecord(evP[0], aux));
  for (int64_t s = 0; s < nsegs; ++s) {
    KDN_TRY(hipStreamWaitEvent(st, evP[s % nbuf], 0));
    KDN_TRYK((launch_phase<P, InT, OutT, D, DV>(seg_p(s), PHASE_CHAIN, st)));
    KDN_TRY(hipEventRecord(evC[s % nbuf], st));
    if (s + 1 < nsegs) {
      if (s + 1 >= nbuf) KDN_TRY(hipStreamWaitEvent(aux, evC[(s + 1) % nbuf], 0));
      KDN_TRYK((launch_phase<P, InT, OutT, D, DV>(seg_p(s + 1), PHASE_PREP, aux)));
      KDN_TRY(hipEventRecord(evP[(s + 1) % nbuf], aux));
    }
  }
#undef KDN_TRY
#undef KDN_TRYK
  return KDN_OK;
}

template <class P, typename InT, typename OutT, int D, int DV>
static int run(const kdn_scan_args* a, const RunSpec& r) {
  if (r.aux && Fused<P, D>::value && r.phases == PHASE_ALL && use_fused(a))
    return run_pipelined_fused<P, InT, OutT, D, DV>(a, r);
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
  if (a->D != 512) return KDN_ERR_UNSUPPORTED;  // narrower lifts arrive here replicated to 512 (kdn_frep.hip)
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
  } else if (a->D != 512 && !frep_applies(a)) {  // D = 128, 256: lifted, then replicated to 512
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
  // neither the general-D scan nor the replicated narrower lifts have phase entry points
  if (general_scan_applies(a) || frep_applies(a)) return KDN_ERR_UNSUPPORTED;
  // the fused schedule's phases exist for bf16 inputs at D = 512
  if ((phase & (PHASE_PREP_FUSED | PHASE_CHAIN)) && a->in_dtype != KDN_DTYPE_BF16) return KDN_ERR_UNSUPPORTED;
  const int64_t total = (a->T + CH - 1) / CH;
  if (chunk0 < 0 || nchunks < 1 || chunk0 + nchunks > total) return KDN_ERR_INVALID_ARGUMENT;
  const size_t need = chunk_bytes(a) * (size_t)a->B * (size_t)a->H * (size_t)(nchunks + 1);
  if (a->workspace_bytes < need) return KDN_ERR_WORKSPACE_TOO_SMALL;
  return dispatch(a, chunk0, chunk0 + nchunks, nchunks, phase, as_stream(stream));
}

size_t scan_checkpoint_buffer_bytes(const kdn_scan_args* a, int64_t seg) {
  return chunk_bytes(a) * (size_t)a->B * (size_t)a->H * (size_t)(seg + 1);
}

// The states at the starts of segments 1 .. n (of `seg` chunks) by the prep and state kernels alone; see
// kdn_internal.hpp.
template <class P, typename InT>
static int checkpoints_t(const kdn_scan_args* a, int64_t seg, int64_t n, float* ckpt, unsigned char* ws,
                         size_t buf_bytes, int nbuf, hipStream_t st, hipStream_t aux) {
  const int64_t nchunks = (a->T + CH - 1) / CH;
  const int64_t heads = a->B * a->H;
  const size_t state_floats = (size_t)heads * 512 * 64;
  const bool side = aux && aux != st && nbuf >= 2 && n >= 2;
  const RunSpec r = {0, nchunks, seg, PHASE_PREP | PHASE_STATE, st, nullptr, 0, 0};
  const int prep_cus = side ? device_cus() - (int)state_grid(a->B, a->H, 4) : device_cus();
  auto seg_p = [&](int64_t s) {
    const int64_t c0 = s * seg;
    ScanParams p = segment_params(a, r, c0, (nchunks - c0 < seg) ? (nchunks - c0) : seg,
                                  ws + (size_t)(side ? s % nbuf : 0) * buf_bytes, prep_cus);
    p.prep_no_q = 1;  // no output kernel reads the lifted queries
    p.y = nullptr;
    if (s > 0) {
      p.state_in = ckpt + (size_t)(s - 1) * state_floats;
      p.is0 = a->H * 512 * 64; p.is1 = 512 * 64; p.is2 = 64; p.is3 = 1;
    }
    p.state_out = ckpt + (size_t)s * state_floats;
    p.os0 = a->H * 512 * 64; p.os1 = 512 * 64; p.os2 = 64; p.os3 = 1;
    return p;
  };
  if (!side) {
    for (int64_t s = 0; s < n; ++s) {
      const ScanParams p = seg_p(s);
      int rc = launch_phase<P, InT, float, 512, 64>(p, PHASE_PREP, st);
      if (rc == KDN_OK) rc = launch_phase<P, InT, float, 512, 64>(p, PHASE_STATE, st);
      if (rc != KDN_OK) return rc;
    }
    return KDN_OK;
  }
  // prep(s + 1) on aux beside state(s) on st, over two buffers:
  //   state(s) waits for prep(s) (event P[s % 2]); prep(s) waits for state(s - 2), the last reader of
  //   its buffer (event S[s % 2]); st finally waits for nothing more (the last state kernel is on it)
  EventSet evs;
  int rc = evs.create(5);
  if (rc != KDN_OK) return rc;
  hipEvent_t* evP = evs.ev;
  hipEvent_t* evS = evs.ev + 2;
  hipEvent_t evIn = evs.ev[4];
#define KDN_TRY(x) do { if ((x) != hipSuccess) return KDN_ERR_DEVICE; } while (0)
#define KDN_TRYK(x) do { const int _rc = (x); if (_rc != KDN_OK) return _rc; } while (0)
  KDN_TRY(hipEventRecord(evIn, st));
  KDN_TRY(hipStreamWaitEvent(aux, evIn, 0));
  KDN_TRYK((launch_phase<P, InT, float, 512, 64>(seg_p(0), PHASE_PREP, aux)));
  KDN_TRY(hipEventRecord(evP[0], aux));
  for (int64_t s = 0; s < n; ++s) {
    KDN_TRY(hipStreamWaitEvent(st, evP[s % 2], 0));
    KDN_TRYK((launch_phase<P, InT, float, 512, 64>(seg_p(s), PHASE_STATE, st)));
    KDN_TRY(hipEventRecord(evS[s % 2], st));
    if (s + 1 < n) {
      if (s >= 1) KDN_TRY(hipStreamWaitEvent(aux, evS[(s + 1) % 2], 0));
      KDN_TRYK((launch_phase<P, InT, float, 512, 64>(seg_p(s + 1), PHASE_PREP, aux)));
      KDN_TRY(hipEventRecord(evP[(s + 1) % 2], aux));
    }
  }
#undef KDN_TRY
#undef KDN_TRYK
  return KDN_OK;
}

int scan_checkpoints(const kdn_scan_args* a, int64_t seg, int64_t n, float* ckpt, void* ws, size_t buf_bytes,
                     int nbuf, hipStream_t st, hipStream_t aux) {
  if (n <= 0) return KDN_OK;
  if (a->D != 512 || a->d_v != 64 || a->feature_mode != 0 || a->cu_seqlens || a->state_slots)
    return KDN_ERR_UNSUPPORTED;
  unsigned char* w = static_cast<unsigned char*>(ws);
  if (a->in_dtype == KDN_DTYPE_BF16) return checkpoints_t<PrecBF16, __bf16>(a, seg, n, ckpt, w, buf_bytes, nbuf, st, aux);
  return checkpoints_t<PrecF32, float>(a, seg, n, ckpt, w, buf_bytes, nbuf, st, aux);
}

}  // namespace kdn

using namespace kdn;

// D = 128 / 256 (feature replication, kdn_frep.hip): the 512-wide request's workspace, then the replicated
// tables and two 512-wide states (initial, final).
static size_t frep_workspace(const kdn_scan_args* a, bool pipelined) {
  if (a->cu_seqlens || a->state_slots) return 0;  // uniform batches only
  const kdn_scan_args w = frep_wide(a, nullptr, nullptr);
  const size_t base = pipelined ? scan_workspace_bytes_pipelined(&w) : kdn_scan_workspace_bytes(&w);
  return base ? frep_layout(a, base, 2).total : 0;
}

// The D-wide scan as the 512-wide one: replicate the tables and the initial state into the workspace, run,
// fold the 512-wide final state into final_state.  All on `stream` (the pipelined form joins its auxiliary
// streams back into it).
static int frep_scan(const kdn_scan_args* a, bool pipelined, void* stream, void* aux, void* out) {
  int rc = validate_launch(a);
  if (rc != KDN_OK) return rc;
  const size_t need = frep_workspace(a, pipelined);
  if (!need) return KDN_ERR_UNSUPPORTED;
  if (a->workspace_bytes < need) return KDN_ERR_WORKSPACE_TOO_SMALL;
  const kdn_scan_args w0 = frep_wide(a, nullptr, nullptr);
  const size_t base = pipelined ? scan_workspace_bytes_pipelined(&w0) : kdn_scan_workspace_bytes(&w0);
  const FrepLayout L = frep_layout(a, base, 2);
  kdn_scan_args w = frep_wide(a, &L, a->workspace);
  unsigned char* ws = static_cast<unsigned char*>(a->workspace);
  float* s_in = reinterpret_cast<float*>(ws + L.state[0]);
  float* s_out = reinterpret_cast<float*>(ws + L.state[1]);
  int64_t cs[4];
  frep_contiguous_strides(a, cs);
  w.initial_state = a->initial_state ? s_in : nullptr;
  w.final_state = s_out;
  for (int i = 0; i < 4; ++i) w.init_stride[i] = w.final_stride[i] = cs[i];
  const hipStream_t st = as_stream(stream);
  rc = frep_tables(a, &L, a->workspace, st);
  if (rc == KDN_OK && a->initial_state) rc = frep_state_lift(a, a->initial_state, a->init_stride, s_in, st);
  if (rc != KDN_OK) return rc;
  rc = pipelined ? scan_pipelined(&w, nullptr, nullptr, stream, aux, out) : kdn_delta_scan_fwd(&w, stream);
  if (rc != KDN_OK) return rc;
  return frep_state_fold(a, s_out, a->final_state, a->final_stride, st);
}

extern "C" size_t kdn_scan_workspace_bytes(const kdn_scan_args* a) {
  if (validate(a) != KDN_OK) return 0;
  if (general_scan_applies(a)) return general_scan_workspace_bytes(a);
  if (frep_applies(a)) return frep_workspace(a, false);
  const int64_t seg = choose_segment(a);
  return chunk_bytes(a) * (size_t)a->B * (size_t)a->H * (size_t)(seg + 1);
}

extern "C" int kdn_delta_scan_fwd(const kdn_scan_args* a, void* stream) {
  int rc = validate_launch(a);
  if (rc != KDN_OK) return rc;
  if (general_scan_applies(a)) return general_scan(a, stream);
  if (frep_applies(a)) return frep_scan(a, false, stream, nullptr, nullptr);
  const int64_t seg = choose_segment(a);
  const size_t need = chunk_bytes(a) * (size_t)a->B * (size_t)a->H * (size_t)(seg + 1);
  if (a->workspace_bytes < need) return KDN_ERR_WORKSPACE_TOO_SMALL;
  const int64_t nchunks = (a->T + CH - 1) / CH;
  return dispatch(a, 0, nchunks, seg, PHASE_ALL, as_stream(stream));
}

// Default segment of the pipelined scan: 64 or 128 chunks, fewer for short sequences
// (128 while the split schedule's state workgroups leave CUs idle, where the chain is a latency-bound
// sequence and longer segments mean fewer launch gaps on it: config 3 2.565 against 2.598 ms for 64.)
static int64_t pipeline_segment(const kdn_scan_args* a) {
  const int64_t nchunks = (a->T + CH - 1) / CH;
  int64_t seg = a->segment_chunks;
  if (seg <= 0) {
    const int cus = device_cus();
    seg = (cus > 0 && (int64_t)state_grid(a->B, a->H, a->d_v / 16) < cus) ? 128 : 64;
  }
  return seg < nchunks ? seg : nchunks;
}

extern "C" int64_t kdn_scan_segment_chunks(const kdn_scan_args* a, int pipelined) {
  if (validate(a) != KDN_OK || general_scan_applies(a)) return 0;
  if (frep_applies(a)) {
    const kdn_scan_args w = frep_wide(a, nullptr, nullptr);
    return pipelined ? pipeline_segment(&w) : choose_segment(&w);
  }
  return pipelined ? pipeline_segment(a) : choose_segment(a);
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
  if (frep_applies(a)) return seq_lo ? KDN_ERR_UNSUPPORTED : frep_scan(a, true, stream, aux_stream, out_stream);
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

size_t scan_flat_buffer_bytes(const kdn_scan_args* a, int64_t win) {
  return chunk_bytes(a) * (size_t)a->H * (size_t)(win + 1);
}

int scan_flat(const kdn_scan_args* a, const int64_t* seq_lo, const int64_t* seq_hi, const FlatPlan& fp, void* stream,
              void* aux_stream) {
  int rc = validate_launch(a);
  if (rc != KDN_OK) return rc;
  if (general_scan_applies(a) || frep_applies(a) || a->D != 512) return KDN_ERR_UNSUPPORTED;
  if (a->initial_state != a->final_state || !a->state_slots || !seq_lo || !seq_hi || fp.win < 1 || fp.nwin < 0)
    return KDN_ERR_INVALID_ARGUMENT;
  const size_t buf = scan_flat_buffer_bytes(a, fp.win);
  if (a->workspace_bytes < buf) return KDN_ERR_WORKSPACE_TOO_SMALL;
  if (fp.nwin == 0) return KDN_OK;
  const size_t fit = a->workspace_bytes / buf;
  const int nbuf = (int)(fit < 3 ? fit : 3);
  RunSpec r = {0, 0, fp.win, PHASE_ALL, as_stream(stream), as_stream(aux_stream), nbuf, buf};
  r.seq_lo = seq_lo;
  r.seq_hi = seq_hi;
  r.flat = &fp;
  if (!aux_stream || aux_stream == stream || nbuf < 2 || fp.nwin < 2) r.aux = nullptr;
  return dispatch(a, r);
}

size_t scan_workspace_bytes_pipelined(const kdn_scan_args* a) {
  if (validate(a) != KDN_OK) return 0;
  if (general_scan_applies(a)) return general_scan_workspace_bytes(a);
  if (frep_applies(a)) return frep_workspace(a, true);
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

extern "C" int kdn_scan_prep_fused(const kdn_scan_args* a, int64_t chunk0, int64_t nchunks, void* stream) {
  return run_phase(a, chunk0, nchunks, PHASE_PREP_FUSED, stream);
}

extern "C" int kdn_scan_chain(const kdn_scan_args* a, int64_t chunk0, int64_t nchunks, void* stream) {
  return run_phase(a, chunk0, nchunks, PHASE_CHAIN, stream);
}

extern "C" int kdn_scan_schedule(const kdn_scan_args* a) {
  const int rc = validate(a);
  if (rc != KDN_OK) return rc;
  if (general_scan_applies(a)) return KDN_SCHEDULE_GENERAL;
  return (a->in_dtype == KDN_DTYPE_BF16 && use_fused(a)) ? KDN_SCHEDULE_FUSED : KDN_SCHEDULE_SPLIT;  // same at D < 512
}

// ------------------------------------------------------------------------------------------------
// Allocation-free scan: the workspace of one segment lives in the fixed scratch array of kdn_noalloc.hip
// instead of a caller buffer.  The array keeps its contents between calls and nothing reads a record
// before the segment's prep has written it, so no clearing is needed; calls that overlap on one GPU share
// the array and race.
extern "C" int kdn_delta_scan_fwd_noalloc(const kdn_scan_args* a, void* stream) {
  int rc = validate(a);
  if (rc != KDN_OK) return rc;
  if (general_scan_applies(a)) return KDN_ERR_UNSUPPORTED;  // its workspace spans the whole sequence
  if (frep_applies(a)) return KDN_ERR_UNSUPPORTED;          // nor for the replicated narrower lifts
  // Segments of as many chunks as the scratch holds: one record per (head, chunk) plus a spare per head.
  const size_t per_chunk = chunk_bytes(a) * (size_t)a->B * (size_t)a->H;
  const int64_t fit = (int64_t)(KDN_NOALLOC_SCRATCH_BYTES / per_chunk) - 1;
  if (fit < 1) return KDN_ERR_WORKSPACE_TOO_SMALL;  // more heads than one segment of scratch can hold
  const int64_t nchunks = (a->T + CH - 1) / CH;
  int64_t seg = fit < nchunks ? fit : nchunks;
  if (a->segment_chunks > 0 && a->segment_chunks < seg) seg = a->segment_chunks;
  void* ws = nullptr;
  rc = noalloc_scratch_address(&ws);
  if (rc != KDN_OK) return rc;
  kdn_scan_args b = *a;
  b.workspace = ws;
  b.workspace_bytes = KDN_NOALLOC_SCRATCH_BYTES;
  b.segment_chunks = seg;
  rc = validate_launch(&b);
  if (rc != KDN_OK) return rc;
  return dispatch(&b, 0, nchunks, seg, PHASE_ALL, as_stream(stream));
}
