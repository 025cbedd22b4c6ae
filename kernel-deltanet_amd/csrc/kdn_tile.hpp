// Row-major fp32 tiles <-> MFMA fragments, and small wave reductions (gfx950), shared by the kernels
// that keep their per-chunk matrices as plain fp32 rows (the backward pass and the general-D scan).
#pragma once
#include <hip/hip_runtime.h>
#include "kdn_frag.hpp"

namespace kdn {

template <typename T>
__device__ __forceinline__ float ldx(const T* p) { return (float)*p; }

// Fragment loads (kappa order, see kdn_frag.hpp).  rows: element (r0 + l%16, k0 + kappa) = base[row * ld + depth]
// (two 16-byte loads); cols: element (c0 + l%16, k0 + kappa) = base[depth * ld + c0 + l%16] (eight loads).
__device__ __forceinline__ f32x8 frag_rows(const float* base, int ld, int r0, int k0, int lane) {
  const float* p = base + (size_t)(r0 + (lane & 15)) * ld + k0 + 4 * (lane >> 4);
  const f32x4 lo = *reinterpret_cast<const f32x4*>(p);
  const f32x4 hi = *reinterpret_cast<const f32x4*>(p + 16);
  return pair_to8(lo, hi);
}
__device__ __forceinline__ f32x8 frag_cols(const float* base, int ld, int c0, int k0, int lane) {
  f32x8 r;
#pragma unroll
  for (int s = 0; s < 8; ++s) r[s] = base[(size_t)(k0 + kappa(lane, s)) * ld + c0 + (lane & 15)];
  return r;
}
__device__ __forceinline__ f32x8 frag_rows_bf16(const __bf16* base, int ld, int r0, int k0, int lane) {
  typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
  const __bf16* p = base + (size_t)(r0 + (lane & 15)) * ld + k0 + 4 * (lane >> 4);
  const bf16x4 lo = *reinterpret_cast<const bf16x4*>(p);
  const bf16x4 hi = *reinterpret_cast<const bf16x4*>(p + 16);
  f32x8 r;
#pragma unroll
  for (int s = 0; s < 4; ++s) { r[s] = (float)lo[s]; r[4 + s] = (float)hi[s]; }
  return r;
}
__device__ __forceinline__ f32x8 frag_cols_bf16(const __bf16* base, int ld, int c0, int k0, int lane) {
  f32x8 r;
#pragma unroll
  for (int s = 0; s < 8; ++s) r[s] = (float)base[(size_t)(k0 + kappa(lane, s)) * ld + c0 + (lane & 15)];
  return r;
}

// Fragments in plain depth order (slot s of lane l at depth k0 + 8(l>>4) + s, one 16- or 32-byte run
// per lane): a product is exact in any depth order as long as both operands use the same one.
__device__ __forceinline__ f32x8 frag_rows_plain(const float* base, int ld, int r0, int k0, int lane) {
  const float* p = base + (size_t)(r0 + (lane & 15)) * ld + k0 + 8 * (lane >> 4);
  return pair_to8(*reinterpret_cast<const f32x4*>(p), *reinterpret_cast<const f32x4*>(p + 4));
}
__device__ __forceinline__ f32x8 frag_rows_plain_bf16(const __bf16* base, int ld, int r0, int k0, int lane) {
  const bf16x8 v = *reinterpret_cast<const bf16x8*>(base + (size_t)(r0 + (lane & 15)) * ld + k0 + 8 * (lane >> 4));
  f32x8 r;
#pragma unroll
  for (int s = 0; s < 8; ++s) r[s] = (float)v[s];
  return r;
}

// sin of an angle in radians via v_sin_f32 (revolutions), reduced to [-0.5, 0.5] revolutions as
// cos_rad (kdn_frag.hpp) does.
__device__ __forceinline__ float sin_rad(float angle) {
  float r = angle * 0.15915494309189535f;  // 1 / (2 pi)
  r = r - __builtin_rintf(r);
  return __builtin_amdgcn_sinf(r);
}

template <class P>
__device__ __forceinline__ f32x4 mm(f32x4 acc, const f32x8& a, const f32x8& b) {
  return P::mma(acc, P::from_f32(a), P::from_f32(b));
}

// T = (I + A)^{-1} of a strictly lower triangular 64 x 64 A, by column-oriented forward substitution:
// wave w (0..3) computes columns 16w .. 16w+15, one per lane quad (col = 16w + (lane >> 2)); lane
// pq = lane & 3 keeps rows 4s + pq.  Once row i of the column is final (lane i & 3, slot i >> 2) it is
// broadcast over the quad and every later row takes its term at once: one broadcast and one FMA per row
// on the sequential chain.  acc[s] = -(partial T[4s+pq][col]); A is zero on and above its diagonal, so
// updating every slot from i >> 2 on leaves rows r <= i unchanged.  The columns of A are loaded three
// rows ahead.
//   At: A transposed in LDS, At[(j * 4 + p) * 16 + s] = A[4s + p][j] (16-byte aligned)
//   T:  output rows, T[r * ldt + c] (LDS)
__device__ __forceinline__ void unit_lower_inverse(const float* At, float* T, int ldt, int w, int lane) {
  const int col = 16 * w + (lane >> 2), pq = lane & 3;
  float acc[16];
#pragma unroll
  for (int s2 = 0; s2 < 16; ++s2) acc[s2] = (4 * s2 + pq == col) ? -1.f : 0.f;
  constexpr int AHEAD = 3;
  f32x4 acol[AHEAD][4];
  auto load_col = [&](int i, f32x4 (&dst)[4]) {
    const f32x4* src = reinterpret_cast<const f32x4*>(At + (i * 4 + pq) * 16);
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
  for (int s2 = 0; s2 < 16; ++s2) T[(4 * s2 + pq) * ldt + col] = -acc[s2];
}

// Swizzled layouts of A and T for unit_lower_inverse_blocked: At[(j * 4 + p) * 16 + a_swizzle(j, s, p)] =
// A[4s + p][j] and T[r * 64 + t_swizzle(r, c)] = T[r][c].
// 4-byte LDS accesses are served per half-wave over 32 banks (16-byte reads per 16 lanes over 64; measured
// with SQ_LDS_BANK_CONFLICT on a probe of both).  a_swizzle keeps each group of four s (one 16-byte read)
// contiguous and spreads a half-wave's 4-byte accesses of A over 32 banks: the writer storing one element
// per lane (p = lane & 3, s & 3 = (lane >> 2) & 3, column group g = lane >> 4) and the column walk reading
// A[16i + m][16k + 4g + kb] (p = m & 3, s & 3 = m >> 2).  Row j * 4 + p puts p & 1 on bank bit 4; XORing
// the group index with (j >> 2) & 3 and with 2 (p >> 1) separates the two lane groups of a half-wave and
// p from p ^ 2.
__device__ __forceinline__ int a_swizzle(int j, int s, int p) {
  return 4 * ((s >> 2) ^ ((j >> 2) & 3) ^ (2 * (p >> 1))) + (s & 3);
}
// t_swizzle XORs the 16-byte group index of column c in row r (ldt = 64) with h(r) = 4 (a ^ p) + a,
// a = (r >> 2) & 3, p = r & 3, so that each of these falls on distinct banks: 4-byte accesses of rows
// 4a + 0..3 (a fixed) or of rows 4·0..3 + p (p fixed) at 16 consecutive columns of one 16-column block per
// instruction (h >> 2 differs over p for fixed a and over a for fixed p), and 16-byte reads of four
// consecutive columns of 16 consecutive rows (h is a bijection on a 16-row block).
__device__ __forceinline__ int t_swizzle(int r, int c) {
  const int a = (r >> 2) & 3, p = r & 3;
  return c ^ (16 * (a ^ p)) ^ (4 * a);
}

// Block column J of T below the diagonal (step 2 of unit_lower_inverse_blocked): T_iJ for i = J+1 .. 3.
template <int J>
__device__ __forceinline__ void inverse_block_column(const float* At, float* T, int lane) {
  auto at_idx = [](int r, int c) { return (c * 4 + (r & 3)) * 16 + a_swizzle(c, r >> 2, r & 3); };
  auto t_idx = [](int r, int c) { return r * 64 + t_swizzle(r, c); };
  const int g = lane >> 4, m = lane & 15;
  // operands read first: L_ik as A operands (depth 4g + kb) and T_ii rows, for every i > J and k in [J, i)
  float la[4][4][4];  // la[i][k][kb] = A[16i + m][16k + 4g + kb]
#pragma unroll
  for (int i = J + 1; i < 4; ++i)
#pragma unroll
    for (int k = J; k < i; ++k)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) la[i][k][kb] = At[at_idx(16 * i + m, 16 * k + 4 * g + kb)];
  f32x4 tii[4];  // T_ii[m][4g .. 4g + 3]
#pragma unroll
  for (int i = J + 1; i < 4; ++i) tii[i] = *reinterpret_cast<const f32x4*>(T + t_idx(16 * i + m, 16 * i + 4 * g));
  f32x4 tcol[4];  // T_kJ in accumulator layout: tcol[k][e] = T[16k + 4g + e][16J + m]
#pragma unroll
  for (int e = 0; e < 4; ++e) tcol[J][e] = T[t_idx(16 * J + 4 * g + e, 16 * J + m)];
#pragma unroll
  for (int i = J + 1; i < 4; ++i) {
    f32x4 S = zero4();
#pragma unroll
    for (int k = J; k < i; ++k)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) S = __builtin_amdgcn_mfma_f32_16x16x4f32(la[i][k][kb], tcol[k][kb], S, 0, 0, 0);
    f32x4 tn = zero4();
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) tn = __builtin_amdgcn_mfma_f32_16x16x4f32(tii[i][kb], S[kb], tn, 0, 0, 0);
    tcol[i] = -tn;
#pragma unroll
    for (int e = 0; e < 4; ++e) T[t_idx(16 * i + 4 * g + e, 16 * J + m)] = tcol[i][e];
  }
}

// The same inverse in 16 x 16 blocks, for the swizzled layouts above (At by a_swizzle, T by t_swizzle with
// ldt = 64).  L = I + A with blocks L_ik; T_ii = L_ii^{-1} and T_ij = -T_ii sum_{k=j}^{i-1} L_ik T_kj (i > j).
//   1. wave b inverts diagonal block b by the column substitution above restricted to 16 rows (15 steps of
//      one quad broadcast and at most four FMAs), writes T_bb and the zero blocks to its right;
//   2. after a barrier, wave j (0..2) walks down block column j: S = sum_k L_ik T_kj, T_ij = -T_ii S, as
//      fp32 16x16x4 MFMAs.  Lane group g supplies depth 4g + kb to MFMA kb for both operands, so a product
//      in accumulator layout (lane l: rows 4(l >> 4) + e of column l & 15) is the B operand of the next
//      one as it stands (element kb), and L_ik and T_ii enter as A operands read from LDS.
// The sequential chain is 15 substitution steps plus three dependent block products (wave 0), against
// 63 substitution steps column by column.  Ends with the stores of T issued: the caller's barrier orders
// them for its readers.
// Step 1 for diagonal block b (one wave).
__device__ __forceinline__ void inverse_diag_block(const float* At, float* T, int b, int lane) {
  auto t_idx = [](int r, int c) { return r * 64 + t_swizzle(r, c); };
  {
    // diagonal block b: lane quad c = lane >> 2 holds column c, lane pq = lane & 3 rows 4s + pq
    const int c = lane >> 2, pq = lane & 3;
    float acc[4];  // -(partial T_bb[4s + pq][c])
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[s] = (4 * s + pq == c) ? -1.f : 0.f;
    // column i of L_bb's strict lower part, rows 16b + 4s + pq (s = 0..3): one 16-byte group of At
    auto col = [&](int i) {
      const int C = 16 * b + i;
      return *reinterpret_cast<const f32x4*>(At + (C * 4 + pq) * 16 + 4 * (b ^ ((C >> 2) & 3) ^ (2 * (pq >> 1))));
    };
    // every column's read issued before the chain starts (nothing else is live here)
    f32x4 acol[15];
#pragma unroll
    for (int i = 0; i < 15; ++i) acol[i] = col(i);
#pragma unroll
    for (int i = 0; i < 15; ++i) {
      const f32x4 a = acol[i];
      float bc;  // -T[i][c], held by lane pq = i & 3, slot i >> 2 of the quad
      switch (i & 3) {
        case 0: bc = quad_bcast<0>(acc[i >> 2]); break;
        case 1: bc = quad_bcast<1>(acc[i >> 2]); break;
        case 2: bc = quad_bcast<2>(acc[i >> 2]); break;
        default: bc = quad_bcast<3>(acc[i >> 2]); break;
      }
#pragma unroll
      for (int s = i >> 2; s < 4; ++s) acc[s] = fmaf(-a[s], bc, acc[s]);
    }
    // store k writes row 4s + pq with s = k ^ 2 (pq >> 1): a half-wave (columns c = 0..7) then spans bank
    // bit 3 through s as well as bit 4 through pq, 32 distinct banks (s = k for every lane: 16)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int s = k ^ (2 * (pq >> 1));
      const int r = 16 * b + 4 * s + pq;
      T[t_idx(r, 16 * b + c)] = (pq & 2) ? -acc[k ^ 2] : -acc[k];
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
        if (blk > b) T[t_idx(r, 16 * blk + c)] = 0.f;
    }
  }
}

// Step 2 for block column j = w (waves 0..2; others return), one code path per wave so that every LDS
// read of the walk can be issued ahead of the products.
__device__ __forceinline__ void inverse_block_columns(const float* At, float* T, int w, int lane) {
  switch (w) {
    case 0: inverse_block_column<0>(At, T, lane); break;
    case 1: inverse_block_column<1>(At, T, lane); break;
    case 2: inverse_block_column<2>(At, T, lane); break;
    default: break;
  }
}

__device__ __forceinline__ void unit_lower_inverse_blocked(const float* At, float* T, int w, int lane) {
  inverse_diag_block(At, T, w, lane);
  lds_barrier();
  inverse_block_columns(At, T, w, lane);
}

// Sum over the 16 lanes sharing (lane >> 4) (one tile row) / over the 4 lane groups (one tile column).
__device__ __forceinline__ float sum_row16(float v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 8);
  return v;
}
__device__ __forceinline__ float sum_col4(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

}  // namespace kdn
