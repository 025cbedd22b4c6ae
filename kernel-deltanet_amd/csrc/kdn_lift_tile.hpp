// Lift of 16-row tiles of q / k on MFMA plus v_cos, for the prep kernel of the D = 512 scan (kdn_prep.hip).
#pragma once
#include <type_traits>
#include "kdn_frag.hpp"
#include "kdn_io.hpp"

namespace kdn {

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
// Output: unnormalised cos values as X fragments, and each row's sum of squares (all lanes).  NTL tiles
// from tile0 (default: all D / 16): fragment j of `out` holds features 32 (tile0 / 2 + j) .. + 31, and ss
// the sum over those features.
template <class P, typename InT, int D, bool OMEGA_LDS, int NX, bool LO = false, int NTL = D / 16>
__device__ __forceinline__ void lift_tile(const RawRow<InT> (&raw)[NX], int normalize,
                                          const bf16x8* s_omega, const __bf16* omega, const float* s_phrev,
                                          float ang, int lane, typename P::frag (&out)[NX][NTL / 2],
                                          float (&ss)[NX], const __bf16* omega_lo = nullptr, int tile0 = 0) {
  constexpr int NT = NTL;
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
  // issued in the scheduling region of the cosines of tile t, with Omega's fragments for them read one
  // tile earlier still (so that the read's latency is covered by a tile's cosines, not waited on by the
  // MFMAs that follow it).
  auto fetch = [&](int t, bf16x8 (&a)[2]) {
    const int tg = tile0 + t;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      if constexpr (OMEGA_LDS) a[kb] = s_omega[(tg * 2 + kb) * 64 + lane];
      else a[kb] = *reinterpret_cast<const bf16x8*>(omega + (int64_t)(16 * tg + (lane & 15)) * 64 + 32 * kb + 8 * (lane >> 4));
    }
  };
  // tiles of Omega in flight ahead of the one projected (one; the exact projection reading Omega from L2
  // three tiles ahead instead of staging it in LDS measured slower: config-3 prep 139 -> 150 us)
  constexpr int PF = 1;
  bf16x8 om_ring[PF][2];
  auto project = [&](int t, f32x4 (&acc)[NX]) {
    bf16x8 om_t[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) om_t[kb] = om_ring[t % PF][kb];
    if (t + PF < NT) fetch(t + PF, om_ring[t % PF]);
#pragma unroll
    for (int x = 0; x < NX; ++x) acc[x] = zero4();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const bf16x8 a = om_t[kb];
#pragma unroll
      for (int s = 0; s < NSPLIT; ++s)
#pragma unroll
        for (int x = 0; x < NX; ++x) acc[x] = PrecBF16::mma(acc[x], a, xb[x][kb][s]);
      if constexpr (LO) {
        const bf16x8 alo = *reinterpret_cast<const bf16x8*>(omega_lo + (int64_t)(16 * (tile0 + t) + (lane & 15)) * 64 + 32 * kb + 8 * (lane >> 4));
#pragma unroll
        for (int s = 0; s < NSPLIT; ++s)
#pragma unroll
          for (int x = 0; x < NX; ++x) acc[x] = PrecBF16::mma(acc[x], alo, xb[x][kb][s]);
      }
    }
  };
  f32x4 acc[NX];
#pragma unroll
  for (int t = 0; t < PF; ++t) fetch(t, om_ring[t]);
  project(0, acc);
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    // two feature tiles per scheduling region (16 independent cosine chains to interleave; measured
    // ~3 % faster than one tile and than four): hoisting the Omega reads of every tile to the top would
    // hold them all in registers at once
    if (t % 2 == 0) __builtin_amdgcn_sched_barrier(0);
    f32x4 next[NX];
    if (t + 1 < NT) project(t + 1, next);
    const f32x4 ph = *reinterpret_cast<const f32x4*>(&s_phrev[16 * (tile0 + t) + 4 * (lane >> 4)]);
#pragma unroll
    for (int x = 0; x < NX; ++x)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float c = __builtin_amdgcn_cosf(__builtin_amdgcn_fractf(acc[x][i] * ang + ph[i]));
        ss[x] += c * c;
        P::set(out[x][t >> 1], (t & 1) * 4 + i, c);
      }
    if constexpr (std::is_same<P, PrecBF16>::value) {
      // Pin each completed fragment in its packed bf16 form here: otherwise the conversions are sunk
      // to the fragments' first use after the lift, keeping all 256 fp32 cosines of the lane live.
      if (t & 1) {
#pragma unroll
        for (int x = 0; x < NX; ++x) asm volatile("" : "+v"(out[x][t >> 1]));
      }
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
// and phase / (2 pi), by a workgroup of NTHREADS threads.  The fragment loop has a fixed trip count, so
// that every load is issued before the first LDS store waits for one (a loop bounded by blockDim is not
// unrolled and pays one L2 round trip per iteration).
template <int D, bool OMEGA_LDS, int NTHREADS = 256>
__device__ __forceinline__ void stage_omega(const __bf16* omega, const float* phase, bf16x8* s_omega, float* s_phrev) {
  if constexpr (OMEGA_LDS) {
    constexpr int NF = (D / 16) * 2 * 64;
    static_assert(NF % NTHREADS == 0, "fragment slots per thread");
    bf16x8 v[NF / NTHREADS];
#pragma unroll
    for (int i = 0; i < NF / NTHREADS; ++i) {
      const int idx = (int)threadIdx.x + NTHREADS * i;
      const int l = idx & 63, tk = idx >> 6, t = tk >> 1, kb = tk & 1;
      v[i] = *reinterpret_cast<const bf16x8*>(omega + (int64_t)(16 * t + (l & 15)) * 64 + 32 * kb + 8 * (l >> 4));
    }
#pragma unroll
    for (int i = 0; i < NF / NTHREADS; ++i) s_omega[(int)threadIdx.x + NTHREADS * i] = v[i];
  }
  static_assert(D % NTHREADS == 0, "phases per thread");
  float ph[D / NTHREADS];
#pragma unroll
  for (int i = 0; i < D / NTHREADS; ++i) ph[i] = phase[(int)threadIdx.x + NTHREADS * i];
#pragma unroll
  for (int i = 0; i < D / NTHREADS; ++i) s_phrev[(int)threadIdx.x + NTHREADS * i] = ph[i] * 0.15915494309189535f;
}

}  // namespace kdn
