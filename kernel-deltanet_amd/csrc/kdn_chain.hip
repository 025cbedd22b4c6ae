// Fused chain of the D = 512 prefill scan for bf16 inputs: the sequential state update and the readout
// Y in one kernel, so that no per-chunk state checkpoint leaves the chain and no output kernel runs.
//
// Per 64-token chunk, with the prep kernel's record (kdn_prep.hip: K and Q as unnormalised cos values
// in MFMA fragment order, Tp, P, U~ and the per-token scales; kdn_scan.hip states the algebra):
//   X_K = K S^T,  X_Q = Q S^T                              (S^T at the chunk start, bf16 operands)
//   E   = U~ - Tp X_K
//   Y   = diag(qscale) X_Q + P E                            (written to y)
//   S^T <- gammaC S^T + K^T (kscale o E)
// which are the products the state and output kernels of kdn_scan.hip form, in the same precision and
// (for X_K, E and the state) the same order, so the carried state is bit-identical to theirs.
//
// One workgroup of 4 waves per (sequence, head, 16 NVW value columns), sequential over the chunks of the
// segment.  Wave w owns features [128w, 128w + 128) of the workgroup's state columns: S^T tiles (feature
// tile tl = 0..7, value tile n) in accumulator layout, lane l holding S^T[128w + 16tl + 4(l>>4) + i]
// [col0 + 16n + (l&15)].  Per chunk, three workgroup barriers:
//   P1  X_K partial over the wave's features (K fragments from registers)  -> LDS;
//       the K^T fragments of the wave's features (identity products, below)           | A
//   P2  X_Q partial (Q fragments from registers) -> LDS; X_K token tile w reduced -> LDS  | B
//   P3  E tile w = U~ - Tp X_K -> LDS; X_Q token tile w reduced                         | C
//   P4  Y tile w = diag(qscale) X_Q + P E, stored as whole rows through a wave-private LDS
//       tile; S^T <- gammaC S^T + K^T (kscale o E); bf16 S^T operands for the next chunk.
// No barrier is needed between P4 and the next P1: every LDS area written in P1 / P2 / P3 was last read
// before the barrier that precedes the phase writing it again.
//
// Operand streaming.  Each wave loads its 16 K and 16 Q fragments of a chunk (16 KB each, one 1 KB
// contiguous run per fragment) straight from L2 into registers, the next chunk's K right after the
// current K's last use in P1 and the next Q right after X_Q in P2, so they travel during the rest of the
// step; the small per-chunk operands are reloaded after their last use in P4.  The waves touch one dword
// per 128-byte line of the record L2_AHEAD chunks ahead, so that those loads hit L2.  The barriers wait
// for LDS operations only (s_waitcnt lgkmcnt(0); s_barrier), so the loads in flight are not drained at
// every barrier the way a full workgroup release fence would drain them.
//
// K^T without a second copy of K.  The update contracts over tokens and needs K with 8 consecutive
// tokens per lane (a "K^T fragment"), while X_K contracts over features and needs 8 consecutive
// features per lane (the stored K fragment).  An MFMA with the stored K fragment (m, jj) as A and an
// identity slab I_h as B (lane l, slot s = 1 where depth kappa(l, s) = (l & 15) + 16h) returns the
// 16 x 16 block K[16m .. +16][32jj + 16h .. +16] in accumulator layout: lane l holds tokens
// 16m + 4(l>>4) .. +3 of feature 32jj + 16h + (l & 15).  The accumulators of token tiles 2jb and 2jb+1
// are, slot for slot, the K^T fragment (feature tile 2jj + h, token block jb) (the kappa order of
// kdn_frag.hpp).  Exact: one product per output element, and K is bf16.
#include <type_traits>
#include "kdn_frag.hpp"
#include "kdn_internal.hpp"
#include "kdn_io.hpp"
#include "kdn_scan_common.hpp"

namespace kdn {

namespace {

__device__ __forceinline__ bf16x8 identity_slab(int lane, int hsel) {
  bf16x8 r;
#pragma unroll
  for (int s = 0; s < 8; ++s) r[s] = (kappa(lane, s) == (lane & 15) + 16 * hsel) ? (__bf16)1.0f : (__bf16)0.0f;
  return r;
}

}  // namespace

template <int DV, int NVW>
struct ChainCfg {
  static_assert(DV % (16 * NVW) == 0, "value tiles per workgroup must divide d_v");
  using L = WsLayout<PrecBF16, 512, DV>;
  static constexpr int NV = DV / 16;    // value tiles per head
  static constexpr int NWG = NV / NVW;  // workgroups per head
  static constexpr int L2_AHEAD = 3;    // chunks ahead of the current one that the L2 touch covers
  // 128-byte lines of the record the chain reads: [0, Sfr) (K, Tp, P, U~, scales) and the Q fragments
  static constexpr int LINES_K = (int)(L::Sfr / 128);
  static constexpr int LINES = LINES_K + (int)((size_t)4 * 16 * 64 * 16 / 128);
  // dword touches per thread and chunk (the lines are shared out over the NWG workgroups of a head)
  // (0: no touches; the records are then read from the last-level cache that prep's stores fill)
  static constexpr int TOUCH = 0;
};

template <int DV, int NVW, typename OutT, bool DECAY>
__global__ void __launch_bounds__(256) chain_kernel(ScanParams p) {
  using P = PrecBF16;
  using C = ChainCfg<DV, NVW>;
  using L = typename C::L;
  using frag = bf16x8;
  constexpr int NV = C::NV, NWG = C::NWG;
  constexpr int YS = 16 * NVW + 4;  // padded fp32 row of the Y staging tile
  __shared__ f32x4 s_pk[4][4][NVW][64];  // X_K partials [wave][token tile][value tile][lane]
  __shared__ f32x4 s_pq[4][4][NVW][64];  // X_Q partials
  __shared__ f32x4 s_x[4][NVW][64];      // X_K [token tile][value tile][lane]
  __shared__ f32x4 s_e[4][NVW][64];      // E
  __shared__ __attribute__((aligned(16))) float s_y[4][16 * YS];

  // XCD-aware decomposition of the 1-D grid (as the state kernel's): id = xcd + 8 (rank NWG + vh), with
  // head-batch pair hb = 8 rank + xcd, so the NWG workgroups of a head share one XCD's L2.
  const int64_t id = blockIdx.x;
  const int64_t xcd = id & 7, jdx = id >> 3;
  const int vh = (int)(jdx % NWG);
  const int64_t hb = (jdx / NWG) * 8 + xcd;
  if (hb >= p.B * p.H) return;
  int64_t b, h, nloc, cfirst;
  size_t woff;
  if (!state_item<L::bytes>(p, hb, b, h, nloc, woff, cfirst)) return;
  const Seq sq = seq_of(p, b);
  const int64_t sl = p.slots ? (int64_t)p.slots[b] : b;
  if (sl < 0) return;  // a skipped sequence of a ragged step

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col0 = 16 * NVW * vh;
  const unsigned char* wsh = p.ws + woff;

  f32x4 S[8][NVW];
  if (p.state_in) {
    const float* si = p.state_in + sl * p.is0 + h * p.is1;
#pragma unroll
    for (int tl = 0; tl < 8; ++tl)
#pragma unroll
      for (int n = 0; n < NVW; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          S[tl][n][i] = si[(int64_t)(16 * (8 * w + tl) + 4 * (lane >> 4) + i) * p.is2 +
                           (int64_t)(col0 + 16 * n + (lane & 15)) * p.is3];
  } else {
#pragma unroll
    for (int tl = 0; tl < 8; ++tl)
#pragma unroll
      for (int n = 0; n < NVW; ++n) S[tl][n] = zero4();
  }

  if (nloc > 0) {
    const frag I0 = identity_slab(lane, 0), I1 = identity_slab(lane, 1);
    // K / Q fragment (token tile m, local 32-feature block jj) of the wave: fragment (m, 4w + jj) of the
    // record's [m][j][lane] area
    auto load_rows = [&](frag (&dst)[4][4], const unsigned char* area) {
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) dst[m][jj] = load_frag<P>(area + (size_t)(m * 16 + 4 * w + jj) * 64 * 16, lane);
    };
    struct Small {
      frag tp[2];      // Tp row block w
      frag pf[2];      // P row block w
      f32x4 u[NVW];    // U~ tiles (w, value tiles of the workgroup)
      f32x4 qs;        // qscale of the rows of token tile w (accumulator order)
      f32x4 ks[4];     // kscale in kappa order: [2 jb + half] = rows 32jb + 16 half + 4(l>>4) .. +3
      float gC;
    } sm;
    // the operands of E (used in P3) and those of Y and the update (used in P4), each reloaded for the
    // next chunk right after its last use
    auto load_small_e = [&](const unsigned char* rec) {
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) sm.tp[jb] = load_frag<P>(rec + L::Tp + (size_t)(w * 2 + jb) * 64 * 16, lane);
#pragma unroll
      for (int n = 0; n < NVW; ++n)
        sm.u[n] = *reinterpret_cast<const f32x4*>(rec + L::U + ((size_t)(w * NV + NVW * vh + n) * 64 + lane) * 16);
    };
    auto load_small_y = [&](const unsigned char* rec) {
      const float* vec = reinterpret_cast<const float*>(rec + L::VEC);
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) sm.pf[jb] = load_frag<P>(rec + L::Pm + (size_t)(w * 2 + jb) * 64 * 16, lane);
      sm.qs = *reinterpret_cast<const f32x4*>(vec + 16 * w + 4 * (lane >> 4));
#pragma unroll
      for (int q = 0; q < 4; ++q) sm.ks[q] = *reinterpret_cast<const f32x4*>(vec + 64 + 16 * q + 4 * (lane >> 4));
      sm.gC = vec[128];
    };
    frag kf[4][4], qf[4][4], sf[4][NVW];
    auto make_sf = [&]() {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int n = 0; n < NVW; ++n) sf[jj][n] = P::from_f32(pair_to8(S[2 * jj][n], S[2 * jj + 1][n]));
    };
    load_rows(kf, wsh + L::phiK);
    load_rows(qf, wsh + L::phiQ);
    load_small_e(wsh);
    load_small_y(wsh);
    make_sf();
    // Drain the prologue's loads, so that the loop's first waits are set by the loop's own load order
    // (merged with a different pending order at the loop header they would wait for every load).
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) (lgkmcnt(0) too; expcnt left alone)
    // L2 touches (C::TOUCH > 0): one dword per 128-byte line of the record L2_AHEAD chunks ahead
    // (clamped), loaded into registers that are only added up one chunk later
    unsigned touch_acc = 0, touch_val[C::TOUCH > 0 ? C::TOUCH : 1];
#pragma unroll
    for (int k = 0; k < C::TOUCH; ++k) touch_val[k] = 0;
    size_t touch_off[C::TOUCH > 0 ? C::TOUCH : 1];
#pragma unroll
    for (int k = 0; k < C::TOUCH; ++k) {
      int li = vh + NWG * ((int)threadIdx.x + 256 * k);
      li = li < C::LINES ? li : C::LINES - 1;  // surplus lanes repeat the last line
      touch_off[k] = li < C::LINES_K ? (size_t)li * 128 : L::phiQ + (size_t)(li - C::LINES_K) * 128;
    }
    float* yt = s_y[w];
    const int64_t t0_seq = cfirst * CH;

    for (int64_t c = 0; c < nloc; ++c) {
      // the next chunk's record (the last chunk reloads its own, so that the loads stay unconditional)
      const unsigned char* nxt = wsh + ((c + 1 < nloc) ? c + 1 : c) * L::bytes;
      {
        const unsigned char* pb = wsh + ((c + C::L2_AHEAD < nloc) ? c + C::L2_AHEAD : nloc - 1) * L::bytes;
#pragma unroll
        for (int k = 0; k < C::TOUCH; ++k) {
          touch_acc += touch_val[k];
          touch_val[k] = *reinterpret_cast<const unsigned*>(pb + touch_off[k]);
        }
      }

      // ---- P1: X_K partial over the wave's features; K^T fragments by identity products
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int n = 0; n < NVW; ++n) {
          f32x4 a = zero4();
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) a = P::mma(a, kf[m][jj], sf[jj][n]);
          s_pk[w][m][n][lane] = a;
        }
      frag ktf[8][2];
#pragma unroll
      for (int tl = 0; tl < 8; ++tl)
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
          const frag& id_h = (tl & 1) ? I1 : I0;
          const f32x4 lo = P::mma(zero4(), kf[2 * jb][tl >> 1], id_h);
          const f32x4 hi = P::mma(zero4(), kf[2 * jb + 1][tl >> 1], id_h);
          ktf[tl][jb] = P::from_f32(pair_to8(lo, hi));
        }
      load_rows(kf, nxt + L::phiK);
      lds_barrier();  // A

      // ---- P2: X_Q partial; X_K token tile w
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int n = 0; n < NVW; ++n) {
          f32x4 a = zero4();
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) a = P::mma(a, qf[m][jj], sf[jj][n]);
          s_pq[w][m][n][lane] = a;
        }
      load_rows(qf, nxt + L::phiQ);
#pragma unroll
      for (int n = 0; n < NVW; ++n)
        s_x[w][n][lane] = s_pk[0][w][n][lane] + s_pk[1][w][n][lane] + s_pk[2][w][n][lane] + s_pk[3][w][n][lane];
      lds_barrier();  // B

      // ---- P3: E tile w = U~ - Tp X_K; X_Q token tile w
#pragma unroll
      for (int n = 0; n < NVW; ++n) {
        f32x4 ek = zero4();
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) ek = P::mma(ek, sm.tp[jb], P::from_f32(pair_to8(s_x[2 * jb][n][lane], s_x[2 * jb + 1][n][lane])));
        s_e[w][n][lane] = sm.u[n] - ek;
      }
      load_small_e(nxt);
      f32x4 xq[NVW];
#pragma unroll
      for (int n = 0; n < NVW; ++n)
        xq[n] = s_pq[0][w][n][lane] + s_pq[1][w][n][lane] + s_pq[2][w][n][lane] + s_pq[3][w][n][lane];
      lds_barrier();  // C

      // ---- P4: Y tile w; the state update
      frag eb[2][NVW], es[2][NVW];
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        const f32x8 k8 = pair_to8(sm.ks[2 * jb], sm.ks[2 * jb + 1]);
#pragma unroll
        for (int n = 0; n < NVW; ++n) {
          f32x8 e8 = pair_to8(s_e[2 * jb][n][lane], s_e[2 * jb + 1][n][lane]);
          eb[jb][n] = P::from_f32(e8);
#pragma unroll
          for (int s = 0; s < 8; ++s) e8[s] *= k8[s];
          es[jb][n] = P::from_f32(e8);
        }
      }
#pragma unroll
      for (int n = 0; n < NVW; ++n) {
        f32x4 y = zero4();
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) y = P::mma(y, sm.pf[jb], eb[jb][n]);
#pragma unroll
        for (int i = 0; i < 4; ++i) yt[(4 * (lane >> 4) + i) * YS + 16 * n + (lane & 15)] = y[i] + sm.qs[i] * xq[n][i];
      }
      const float gC = sm.gC;
      load_small_y(nxt);
#pragma unroll
      for (int tl = 0; tl < 8; ++tl)
#pragma unroll
        for (int n = 0; n < NVW; ++n) {
          f32x4 acc = S[tl][n];
          if constexpr (DECAY) acc = acc * gC;  // without decay gammaC is exactly 1
#pragma unroll
          for (int jb = 0; jb < 2; ++jb) acc = P::mma(acc, ktf[tl][jb], es[jb][n]);
          S[tl][n] = acc;
        }
      // rows of the wave's Y tile: 16 rows x 2 NVW pieces of 8 values (the tile was written by this wave)
      wave_lds_sync();
      {
        constexpr int PPR = 2 * NVW;
        const int64_t t0 = t0_seq + c * CH + 16 * w;
#pragma unroll
        for (int base = 0; base < 16 * PPR; base += 64) {
          const int idx = base + lane;
          if (idx < 16 * PPR) {
            const int row = idx / PPR, pc = idx % PPR;
            const int64_t t = t0 + row;
            if (t < sq.len) {
              const f32x4 v0 = *reinterpret_cast<const f32x4*>(yt + row * YS + 8 * pc);
              const f32x4 v1 = *reinterpret_cast<const f32x4*>(yt + row * YS + 8 * pc + 4);
              const float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
              store_row8<OutT>((OutT*)p.y + sq.y + t * p.ys1 + h * p.ys2 + col0 + 8 * pc, v);
            }
          }
        }
      }
      make_sf();
    }
    // Keeps the L2 touches alive: nseg is at least 1, so this branch never runs.
    if (p.nseg < 0) {
#pragma unroll
      for (int k = 0; k < C::TOUCH; ++k) touch_acc += touch_val[k];
      reinterpret_cast<unsigned*>(p.state_out)[0] = touch_acc;
    }
  }

  float* so = p.state_out + sl * p.os0 + h * p.os1;
#pragma unroll
  for (int tl = 0; tl < 8; ++tl)
#pragma unroll
    for (int n = 0; n < NVW; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        so[(int64_t)(16 * (8 * w + tl) + 4 * (lane >> 4) + i) * p.os2 + (int64_t)(col0 + 16 * n + (lane & 15)) * p.os3] =
            S[tl][n][i];
}

template <typename OutT, int DV>
int launch_chain(const ScanParams& p, hipStream_t st) {
  constexpr int NVW = DV >= 32 ? 2 : 1;
  const unsigned grid = chain_grid(p.B, p.H, DV);
  if (p.decay) hipLaunchKernelGGL((chain_kernel<DV, NVW, OutT, true>), dim3(grid), dim3(256), 0, st, p);
  else hipLaunchKernelGGL((chain_kernel<DV, NVW, OutT, false>), dim3(grid), dim3(256), 0, st, p);
  return hipGetLastError() == hipSuccess ? KDN_OK : KDN_ERR_DEVICE;
}

#define KDN_CHAIN_INST(OutT, DV) template int launch_chain<OutT, DV>(const ScanParams&, hipStream_t);
KDN_CHAIN_INST(__bf16, 16)
KDN_CHAIN_INST(__bf16, 32)
KDN_CHAIN_INST(__bf16, 64)
KDN_CHAIN_INST(__bf16, 128)
KDN_CHAIN_INST(float, 16)
KDN_CHAIN_INST(float, 32)
KDN_CHAIN_INST(float, 64)
KDN_CHAIN_INST(float, 128)
#undef KDN_CHAIN_INST

}  // namespace kdn
