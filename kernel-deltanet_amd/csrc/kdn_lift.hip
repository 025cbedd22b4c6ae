// Feature-lift kernels of the Kernel-DeltaNet prefill path (gfx950).
//
//  * kdn_build_omega : Omega[D][64] from the packed Rademacher table with wave64 butterflies
//                      (DPP / ds_swizzle / ds_bpermute cross-lane exchanges), exact integer/8 values.
//                      Follows the construction of kernels/fwht.py:94-111.
//  * kdn_fwht        : plain natural-order FWHT of rows of length n <= 64 (kernels/fwht.py:25-45).
//  * kdn_fwht_lift   : phi_hat = normalise(sqrt(2/D) cos(x Omega^T / tau + b)) (kernels/fwht.py:122-131)
//                      with the projection on MFMA.  Omega is exact in bf16, so with bf16 inputs the
//                      products are exact; fp32 inputs are split into three bf16 parts (exact products).
//                      A dense 64 x D MFMA projection costs ~4 MFMA issues per row versus ~430 VALU
//                      issues for the 8-block x 3-stage butterfly, so the lift's hot path uses MFMA and
//                      the butterfly builds Omega once.
#include <type_traits>
#include "kdn_frag.hpp"
#include "kdn_internal.hpp"
#include "kdn_io.hpp"
#include "kdn_tile.hpp"

namespace kdn {

// ------------------------------------------------------------------------------------------------
// Wave64 natural-order Walsh-Hadamard transform: lane i holds element i.
// Butterfly at stride h: lanes with bit h clear get u + v, lanes with bit h set get u - v, where u is
// the element with the bit clear (the ordering of kernels/fwht.py:35-44).
template <int H>
__device__ __forceinline__ float fwht_stage(float v, int lane) {
  float p = xor_shuffle<H>(v);
  return (lane & H) ? (p - v) : (v + p);
}

template <int N>
__device__ __forceinline__ float fwht_wave(float v, int lane) {
  if constexpr (N > 1) v = fwht_stage<1>(v, lane);
  if constexpr (N > 2) v = fwht_stage<2>(v, lane);
  if constexpr (N > 4) v = fwht_stage<4>(v, lane);
  if constexpr (N > 8) v = fwht_stage<8>(v, lane);
  if constexpr (N > 16) v = fwht_stage<16>(v, lane);
  if constexpr (N > 32) v = fwht_stage<32>(v, lane);
  return v;
}

__device__ __forceinline__ float sign_of(int64_t bits, int i) { return ((bits >> i) & 1) ? -1.f : 1.f; }

// One wave per (block m, column j): column j of W_m = H d3 o (H d2 o (H (d1 o e_j))) / 8.
template <typename OutT>
__global__ void __launch_bounds__(256) build_omega_kernel(const int64_t* __restrict__ bits, int M, OutT* __restrict__ omega) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m = blockIdx.x;
  const int64_t b1 = bits[m * 3 + 0], b2 = bits[m * 3 + 1], b3 = bits[m * 3 + 2];
  for (int j = wave; j < 64; j += 4) {
    float v = (lane == j) ? sign_of(b1, j) : 0.f;
    v = fwht_wave<64>(v, lane);
    v *= sign_of(b2, lane);
    v = fwht_wave<64>(v, lane);
    v *= sign_of(b3, lane);
    v = fwht_wave<64>(v, lane);
    omega[(int64_t)(m * 64 + lane) * 64 + j] = (OutT)(v * 0.125f);
  }
}

// Plain FWHT of rows of length N (one wave per row, lanes >= N idle), fp32 arithmetic.
template <typename T, int N>
__global__ void __launch_bounds__(256) fwht_rows_kernel(const T* __restrict__ x, int64_t rows, int64_t xs,
                                                        T* __restrict__ out, int64_t os) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  float v = (lane < N) ? (float)x[row * xs + lane] : 0.f;
  // Butterflies at strides >= N never mix valid lanes with each other because N is a power of two
  // and only strides < N are applied.
  v = fwht_wave<N>(v, lane);
  if (lane < N) out[row * os + lane] = (T)v;
}

// ------------------------------------------------------------------------------------------------
// Waves (16-row tiles) per lift workgroup.  The bf16 -> bf16 D = 512 lift takes 180 registers: eight
// waves (two per SIMD) share one LDS copy of Omega with nothing spilled, measured 8 % faster at config 2
// than twelve waves squeezed into 168 registers (three spilled to scratch); the other variants keep four.
template <typename InT, typename OutT, int D>
struct LiftWaves {
  static constexpr int value =
      (std::is_same<InT, __bf16>::value && std::is_same<OutT, __bf16>::value && D == 512) ? 8 : 4;
};

// Lift: one wave per 16-row tile, LiftWaves tiles per workgroup, persistent over tiles.
// Projection in the transposed orientation  Phi^T[f][r] = sum_k Omega[f][k] x[r][k]:
//   A = Omega fragments (f rows, k depth)   read from LDS (staged once per workgroup)
//   B = x fragments      (k depth, r column) read from global, 16/32 bytes per lane
// Accumulator tile (f-tile t): lane l holds Phi^T[16t + 4(l>>4) + i][row (l & 15)].
//
// FROM_BITS: Omega is not read from memory; each workgroup builds it in LDS from the packed Rademacher
// table bits[D/64][3] (the reference's native boundary, kernels/fwht_cuda.cpp:29-32): wave w takes
// columns j of block m in turn, column j of H d1 is (-1)^popcount(lane & j) d1_j in lane `lane`, then the
// d2 / d3 sign flips and two wave64 butterflies (fwht_wave) give Omega[64m + lane][j] * 8 exactly, and
// each lane writes its element into the A fragment that the staged copy would hold.
// Output staging tile (16 rows of 128 bytes per wave): chunk c (16 bytes) of row r sits at chunk
// position c ^ ((r >> 1) & 7).  With bf16 output each lane stores 8 bytes (one half of a chunk) of its row,
// and the halves of a chunk are swapped in rows with h(r) = (r ^ (r >> 1)) & 1 = 1.  8-byte stores are
// served 16 lanes per cycle from a 128-byte bank window: the 16 rows of a store take 16 distinct 8-byte
// slots (h separates rows 2k and 2k + 1, whose chunk positions agree).  The read-back takes each chunk as
// its two halves in row order; 8-byte reads are served 32 lanes (4 rows) per cycle from 256 bytes, where
// h separates rows 4k and 4k + 2 (and 4k + 1, 4k + 3).  Both measured on probes of the access widths.
__device__ __forceinline__ int stage_h(int r) { return (r ^ (r >> 1)) & 1; }
template <typename OutT>
__device__ __forceinline__ int stage_off(int r, int byte) {
  const int half = sizeof(OutT) == 2 ? ((byte & 15) ^ (8 * stage_h(r))) : (byte & 15);
  return r * 128 + 16 * ((byte >> 4) ^ ((r >> 1) & 7)) + half;
}
template <typename OutT>
__device__ __forceinline__ u32x4 stage_read(const unsigned char* stg, int r, int pos) {
  const unsigned char* c = stg + r * 128 + 16 * pos;
  if constexpr (sizeof(OutT) == 2) {
    const int lo = 8 * stage_h(r);
    const u32x2 a = *reinterpret_cast<const u32x2*>(c + lo), b = *reinterpret_cast<const u32x2*>(c + (8 ^ lo));
    return __builtin_shufflevector(a, b, 0, 1, 2, 3);
  } else {
    return *reinterpret_cast<const u32x4*>(c);
  }
}

template <typename InT, typename OutT, int D, bool FROM_BITS>
__global__ void __launch_bounds__((64 * LiftWaves<InT, OutT, D>::value)) lift_kernel(const InT* __restrict__ x, int64_t rows, int64_t xs, int normalize,
                                                   const __bf16* __restrict__ omega, const int64_t* __restrict__ bits,
                                                   const float* __restrict__ phase,
                                                   float inv_tau, OutT* __restrict__ out, int64_t os) {
  constexpr int NT = D / 16;                 // feature tiles
  constexpr int NW = LiftWaves<InT, OutT, D>::value;
  constexpr int NSPLIT = XFrag<InT>::NSPLIT;
  __shared__ bf16x8 s_omega[NT * 2 * 64];    // [t][kb][lane] A fragments, D*64*2 bytes
  // phase / (2 pi) per tile and lane: entry (t, l) holds the phases of the features 16t + 4(l >> 4) + 0..3
  // that lane l's accumulator rows take, so that each tile's read is one 16-byte load per lane at its own
  // address (reads of one shared 2 KB table, sixteen lanes to an address, were counted as bank conflicts:
  // 128 cycles per 16-row tile)
  __shared__ f32x4 s_phr[NT * 64];
  // Per-wave staging of 16 rows x 128 bytes of output (stage_off, stage_read): the accumulator stores
  // (16 rows x 8 or 16 bytes per instruction) and the row read-back (two whole rows per 16 lanes) fall on
  // distinct banks.  (Rows padded by 16 bytes instead: the read-back's two rows overlapped on one bank.)
  constexpr int TG = 128 / (16 * (int)sizeof(OutT));  // feature tiles per staged group: 128 bytes of a row
  constexpr int SRS = 16 * TG * (int)sizeof(OutT);   // row stride in bytes (128)
  constexpr int SCPR = 16 * TG * (int)sizeof(OutT) / 16;  // 16-byte chunks per staged row (8)
  static_assert(SCPR == 8, "the staging swizzle assumes 8 chunks per row");
  __shared__ __attribute__((aligned(16))) unsigned char s_stage[NW][16 * SRS];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  // Stage Omega as A fragments: lane l of fragment (t, kb) holds Omega[16t + (l&15)][32kb + 8(l>>4) .. +8].
  if constexpr (FROM_BITS) {
    __bf16* so = reinterpret_cast<__bf16*>(s_omega);
    for (int cj = wave; cj < D; cj += NW) {
      const int m = cj >> 6, j = cj & 63;
      const int64_t b1 = bits[3 * m + 0], b2 = bits[3 * m + 1], b3 = bits[3 * m + 2];
      float v = (__builtin_popcount(lane & j) & 1) ? -sign_of(b1, j) : sign_of(b1, j);
      v *= sign_of(b2, lane);
      v = fwht_wave<64>(v, lane);
      v *= sign_of(b3, lane);
      v = fwht_wave<64>(v, lane);
      const int f = 64 * m + lane;  // feature row of this lane's element
      so[(((f >> 4) * 2 + (j >> 5)) * 64 + (f & 15) + 16 * ((j & 31) >> 3)) * 8 + (j & 7)] = (__bf16)(v * 0.125f);
    }
  } else {
    for (int idx = threadIdx.x; idx < NT * 2 * 64; idx += 64 * NW) {
      const int l = idx & 63, tk = idx >> 6, t = tk >> 1, kb = tk & 1;
      s_omega[idx] = *reinterpret_cast<const bf16x8*>(omega + (int64_t)(16 * t + (l & 15)) * 64 + 32 * kb + 8 * (l >> 4));
    }
  }
  for (int idx = threadIdx.x; idx < NT * 64; idx += 64 * NW) {
    const int f0 = 16 * (idx >> 6) + 4 * ((idx & 63) >> 4);
    f32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = phase[f0 + i] * 0.15915494309189535f;
    s_phr[idx] = v;
  }
  __syncthreads();

  const float ang_scale = inv_tau * 0.15915494309189535f;  // radians -> revolutions folded in
  const float amp = sqrtf(2.0f / (float)D);
  const int64_t ntiles = (rows + 15) / 16;

  // The x fragments of the wave's next tile are loaded while the current one is processed.  The row
  // index is clamped to the last row, so every load is unconditional and in bounds; rows past the end
  // are zeroed after the load and never stored.
  constexpr int PIECES = 2 * (int)sizeof(InT) / 2;  // 16-byte pieces per lane: 8 elements per depth block
  const int64_t stride = (int64_t)gridDim.x * NW;
  auto load_tile = [&](int64_t t, u32x4 (&raw)[PIECES]) {
    int64_t row = t * 16 + (lane & 15);
    row = row < rows ? row : rows - 1;
    const unsigned char* src = reinterpret_cast<const unsigned char*>(x + row * xs) + 8 * (lane >> 4) * sizeof(InT);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int pc = 0; pc < PIECES / 2; ++pc)
        raw[kb * (PIECES / 2) + pc] = *reinterpret_cast<const u32x4*>(src + 32 * kb * sizeof(InT) + 16 * pc);
  };
  u32x4 nraw[PIECES];
  int64_t tile = (int64_t)blockIdx.x * NW + wave;
  if (tile < ntiles) load_tile(tile, nraw);
  for (; tile < ntiles; tile += stride) {
    const int64_t row = tile * 16 + (lane & 15);
    const bool valid = row < rows;
    u32x4 raw[PIECES];
#pragma unroll
    for (int i = 0; i < PIECES; ++i) raw[i] = nraw[i];
    load_tile(tile + stride < ntiles ? tile + stride : tile, nraw);
    // x fragments for depth blocks kb = 0, 1: slots k = 32kb + 8(l>>4) + s.
    float xv[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      load8<InT>(reinterpret_cast<const InT*>(&raw[kb * (PIECES / 2)]), xv[kb]);
#pragma unroll
      for (int s = 0; s < 8; ++s) xv[kb][s] = valid ? xv[kb][s] : 0.f;
    }
    if (normalize) {
      float ss = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int s = 0; s < 8; ++s) ss += xv[kb][s] * xv[kb][s];
      ss = sum_over_lane_groups(ss);
      const float inv = 1.0f / fmaxf(sqrtf(ss), 1e-6f);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          float y = xv[kb][s] * inv;
          xv[kb][s] = (NSPLIT == 1) ? (float)(__bf16)y : y;  // F.normalize output keeps x's dtype
        }
    }
    bf16x8 xb[2][NSPLIT];
    split_frag<NSPLIT>(xv[0], xb[0]);
    split_frag<NSPLIT>(xv[1], xb[1]);

    // Feature tile t: acc = x . Omega[16t .. 16t+16)^T.  Software-pipelined: the MFMAs of tile t+1 are
    // issued in the same scheduling region as the cosines of tile t, with their Omega fragments read one
    // tile earlier still (the LDS read's latency covered by a tile's cosines).
    bf16x8 om_next[2];
    auto fetch = [&](int t) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) om_next[kb] = s_omega[(t * 2 + kb) * 64 + lane];
    };
    auto project = [&](int t) {
      const bf16x8 om_t[2] = {om_next[0], om_next[1]};
      if (t + 1 < NT) fetch(t + 1);
      f32x4 acc = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int p = 0; p < NSPLIT; ++p) acc = PrecBF16::mma(acc, om_t[kb], xb[kb][p]);
      }
      return acc;
    };
    float c[NT][4];
    float ss = 0.f;
    fetch(0);
    f32x4 acc = project(0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      // one feature tile per scheduling region: hoisting the Omega reads of every tile to the top
      // would need 256 registers for them alone
      __builtin_amdgcn_sched_barrier(0);
      const f32x4 next = (t + 1 < NT) ? project(t + 1) : zero4();
      const f32x4 ph = s_phr[t * 64 + lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float cv = __builtin_amdgcn_cosf(__builtin_amdgcn_fractf(acc[i] * ang_scale + ph[i]));
        c[t][i] = cv;
        ss += cv * cv;
      }
      acc = next;
    }
    ss = sum_over_lane_groups(ss);
    // phi = amp * c ; out = phi / (||phi|| + 1e-8)
    const float scale = amp / (amp * sqrtf(ss) + 1e-8f);
    // Store 128 bytes of each of the 16 rows at a time (64 bf16 or 32 fp32 features) through the wave's
    // staging tile, so that every lane writes 16 contiguous bytes and each store instruction covers
    // whole 128-byte lines of rows.
    unsigned char* stg = s_stage[wave];
#pragma unroll
    for (int g = 0; g < NT / TG; ++g) {
#pragma unroll
      for (int tp = 0; tp < TG; ++tp) {
        const int t = TG * g + tp;
        float v[4] = {c[t][0] * scale, c[t][1] * scale, c[t][2] * scale, c[t][3] * scale};
        const int r = lane & 15, byte = (int)sizeof(OutT) * (16 * tp + 4 * (lane >> 4));
        store4<OutT>(reinterpret_cast<OutT*>(stg + stage_off<OutT>(r, byte)), v);
      }
      // The read-back below takes rows other lanes wrote, and the next group's stores overwrite rows
      // other lanes read.
      wave_lds_sync();
#pragma unroll
      for (int j = 0; j < 16 * SCPR / 64; ++j) {
        const int q = 64 * j + lane, r = q / SCPR, pos = q % SCPR, ch = pos ^ ((r >> 1) & 7);
        const u32x4 val = stage_read<OutT>(stg, r, pos);
        const int64_t grow = tile * 16 + r;
        // streaming stores: the features are far larger than the caches, and their readers come later
        // (13 back-to-back config-2 lifts: 0.46 against 0.50 ms per launch once the clocks have settled)
        if (grow < rows) __builtin_nontemporal_store(val, reinterpret_cast<u32x4*>(reinterpret_cast<unsigned char*>(out + grow * os + 16 * TG * g) + 16 * ch));
      }
      wave_lds_sync();
    }
  }
}

// ------------------------------------------------------------------------------------------------
// The same lift with the projection by in-register butterflies instead of the MFMA product (the design
// of the reference's CUDA P3 kernel, kernels/in_register_fwht.cu:10-93 / .cuh, with the semantics of
// kernels/fwht.py:122-131): one wave per row, lane i holding x_i; for each 64-feature block m the sign
// flips d1, d2, d3 and three wave64 Walsh-Hadamard transforms give 8 (Omega x)[64m + lane] with no
// Omega table (Omega_m = H D3 H D2 H D1 / 8).  Kept as the measured alternative to lift_kernel: each
// wave64 transform is six stages of a lane exchange (DPP, ds_swizzle or ds_bpermute), a select and an
// add, and a 512-feature row takes 24 transforms, where the MFMA form needs 4 MFMA issues per row.
template <int H>
__device__ __forceinline__ float wave_sum_step(float v) { return v + xor_shuffle<H>(v); }
__device__ __forceinline__ float wave_sum64(float v) {
  v = wave_sum_step<1>(v);
  v = wave_sum_step<2>(v);
  v = wave_sum_step<4>(v);
  v = wave_sum_step<8>(v);
  v = wave_sum_step<16>(v);
  return wave_sum_step<32>(v);
}

template <typename InT, typename OutT, int D>
__global__ void __launch_bounds__(256) lift_butterfly_kernel(const InT* __restrict__ x, int64_t rows, int64_t xs,
                                                            int normalize, const int64_t* __restrict__ bits,
                                                            const float* __restrict__ phase, float inv_tau,
                                                            OutT* __restrict__ out, int64_t os) {
  constexpr int M = D / 64;
  const int lane = threadIdx.x & 63;
  // this lane's signs (d1, d2, d3 of each block) and phases (in revolutions)
  float s1[M], s2[M], s3[M], ph[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    s1[m] = sign_of(bits[3 * m + 0], lane);
    s2[m] = sign_of(bits[3 * m + 1], lane);
    s3[m] = sign_of(bits[3 * m + 2], lane);
    ph[m] = phase[64 * m + lane] * 0.15915494309189535f;
  }
  const float ang_scale = inv_tau * 0.15915494309189535f;
  const float amp = sqrtf(2.0f / (float)D);
  const int64_t stride = (int64_t)gridDim.x * 4;
  int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  float xn = row < rows ? (float)x[row * xs + lane] : 0.f;
  for (; row < rows; row += stride) {
    float xv = xn;
    if (row + stride < rows) xn = (float)x[(row + stride) * xs + lane];
    if (normalize) {
      const float inv = 1.0f / fmaxf(sqrtf(wave_sum64(xv * xv)), 1e-6f);
      xv *= inv;
      if constexpr (std::is_same<InT, __bf16>::value) xv = (float)(__bf16)xv;  // F.normalize keeps x's dtype
    }
    float c[M];
    float ss = 0.f;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float v = fwht_wave<64>(xv * s1[m], lane);
      v = fwht_wave<64>(v * s2[m], lane);
      v = fwht_wave<64>(v * s3[m], lane);
      c[m] = __builtin_amdgcn_cosf(__builtin_amdgcn_fractf(v * 0.125f * ang_scale + ph[m]));
      ss += c[m] * c[m];
    }
    const float scale = amp / (amp * sqrtf(wave_sum64(ss)) + 1e-8f);
#pragma unroll
    for (int m = 0; m < M; ++m) out[row * os + 64 * m + lane] = (OutT)(c[m] * scale);
  }
}

template <typename InT, typename OutT, int D>
static void launch_lift_butterfly(const void* x, int64_t rows, int64_t xs, int normalize, const int64_t* bits,
                                  const float* phase, float inv_tau, void* out, int64_t os, hipStream_t st) {
  int64_t wgs = (rows + 3) / 4;
  const int cus = device_cus() > 0 ? device_cus() : 256;
  if (wgs > (int64_t)cus * 8) wgs = (int64_t)cus * 8;  // persistent: eight 4-wave workgroups per CU
  hipLaunchKernelGGL((lift_butterfly_kernel<InT, OutT, D>), dim3((unsigned)wgs), dim3(256), 0, st, (const InT*)x, rows,
                     xs, normalize, bits, phase, inv_tau, (OutT*)out, os);
}

template <typename InT, typename OutT, int D>
static void launch_lift(const void* x, int64_t rows, int64_t xs, int normalize, const void* omega, const int64_t* bits,
                        const float* phase, float inv_tau, void* out, int64_t os, hipStream_t st) {
  const int64_t ntiles = (rows + 15) / 16;
  constexpr int NW = LiftWaves<InT, OutT, D>::value;
  int64_t wgs = (ntiles + NW - 1) / NW;
  // one round of resident workgroups (as many per CU as the LDS allows); the kernel loops over tiles
  constexpr size_t lds = (size_t)D * 64 * 2 + (size_t)D * 4 + NW * 16 * (128 + 16);
  const int per_cu = (int)(CU_LDS_BYTES / lds) > 0 ? (int)(CU_LDS_BYTES / lds) : 1;
  const int cus = device_cus() > 0 ? device_cus() : 256;
  const int64_t cap = (int64_t)cus * per_cu;
  if (wgs > cap) wgs = cap;
  if (bits)
    hipLaunchKernelGGL((lift_kernel<InT, OutT, D, true>), dim3((unsigned)wgs), dim3(64 * NW), 0, st, (const InT*)x, rows, xs,
                       normalize, nullptr, bits, phase, inv_tau, (OutT*)out, os);
  else
    hipLaunchKernelGGL((lift_kernel<InT, OutT, D, false>), dim3((unsigned)wgs), dim3(64 * NW), 0, st, (const InT*)x, rows, xs,
                       normalize, (const __bf16*)omega, nullptr, phase, inv_tau, (OutT*)out, os);
}

template <typename InT, typename OutT>
static int dispatch_lift_D(int D, const void* x, int64_t rows, int64_t xs, int normalize, const void* omega,
                           const int64_t* bits, const float* phase, float inv_tau, void* out, int64_t os, hipStream_t st,
                           bool butterfly) {
  if (butterfly) {
    switch (D) {
      case 128: launch_lift_butterfly<InT, OutT, 128>(x, rows, xs, normalize, bits, phase, inv_tau, out, os, st); break;
      case 256: launch_lift_butterfly<InT, OutT, 256>(x, rows, xs, normalize, bits, phase, inv_tau, out, os, st); break;
      case 512: launch_lift_butterfly<InT, OutT, 512>(x, rows, xs, normalize, bits, phase, inv_tau, out, os, st); break;
      default: return KDN_ERR_UNSUPPORTED;
    }
    return launch_status();
  }
  switch (D) {
    case 128: launch_lift<InT, OutT, 128>(x, rows, xs, normalize, omega, bits, phase, inv_tau, out, os, st); break;
    case 256: launch_lift<InT, OutT, 256>(x, rows, xs, normalize, omega, bits, phase, inv_tau, out, os, st); break;
    case 512: launch_lift<InT, OutT, 512>(x, rows, xs, normalize, omega, bits, phase, inv_tau, out, os, st); break;
    default: return KDN_ERR_UNSUPPORTED;
  }
  return launch_status();
}

// The lift with Omega given as the bf16 table (omega) or as the packed sign table (bits); exactly one is
// non-null (butterfly: bits, projected by lift_butterfly_kernel).  Argument checks of kdn_fwht_lift /
// kdn_fwht_lift_bits / kdn_fwht_lift_bits_butterfly.
static int fwht_lift_impl(const void* x, int64_t rows, int64_t x_row_stride, int x_dtype, int normalize_input,
                          const void* omega_bf16, const int64_t* bits, const float* phase, int d_k, int D,
                          float inv_tau, void* out, int64_t out_row_stride, int out_dtype, void* stream,
                          bool butterfly = false) {
  if (!x || !(omega_bf16 || bits) || !phase || !out || rows < 0) return KDN_ERR_INVALID_ARGUMENT;
  if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype)) return KDN_ERR_INVALID_ARGUMENT;
  if (d_k != 64) return KDN_ERR_UNSUPPORTED;
  if (D != 128 && D != 256 && D != 512) return KDN_ERR_UNSUPPORTED;
  if (x_row_stride < d_k || out_row_stride < D) return KDN_ERR_INVALID_ARGUMENT;
  if (!(inv_tau == inv_tau)) return KDN_ERR_INVALID_ARGUMENT;
  // 16-byte vector accesses: row starts of x and out, omega rows, phase; 8-byte words of the sign table.
  if (!aligned(x, 16) || !aligned(out, 16) || !aligned(phase, 16)) return KDN_ERR_MISALIGNED;
  if ((omega_bf16 && !aligned(omega_bf16, 16)) || (bits && !aligned(bits, 8))) return KDN_ERR_MISALIGNED;
  if ((x_row_stride * (int64_t)dtype_size(x_dtype)) % 16 != 0) return KDN_ERR_MISALIGNED;
  if ((out_row_stride * (int64_t)dtype_size(out_dtype)) % 16 != 0) return KDN_ERR_MISALIGNED;
  if (rows == 0) return KDN_OK;
  hipStream_t st = as_stream(stream);
  const int nz = normalize_input ? 1 : 0;
  if (x_dtype == KDN_DTYPE_BF16) {
    if (out_dtype == KDN_DTYPE_BF16)
      return dispatch_lift_D<__bf16, __bf16>(D, x, rows, x_row_stride, nz, omega_bf16, bits, phase, inv_tau, out, out_row_stride, st, butterfly);
    return dispatch_lift_D<__bf16, float>(D, x, rows, x_row_stride, nz, omega_bf16, bits, phase, inv_tau, out, out_row_stride, st, butterfly);
  }
  if (out_dtype == KDN_DTYPE_BF16)
    return dispatch_lift_D<float, __bf16>(D, x, rows, x_row_stride, nz, omega_bf16, bits, phase, inv_tau, out, out_row_stride, st, butterfly);
  return dispatch_lift_D<float, float>(D, x, rows, x_row_stride, nz, omega_bf16, bits, phase, inv_tau, out, out_row_stride, st, butterfly);
}

}  // namespace kdn

using namespace kdn;

extern "C" int kdn_build_omega(const int64_t* sign_bits, int d_k, int D, void* omega, int omega_dtype, void* stream) {
  if (!sign_bits || !omega) return KDN_ERR_INVALID_ARGUMENT;
  if (!valid_dtype(omega_dtype)) return KDN_ERR_INVALID_ARGUMENT;
  if (d_k != 64) return KDN_ERR_UNSUPPORTED;
  if (D <= 0 || D % 64 != 0 || D > 1024) return KDN_ERR_UNSUPPORTED;
  const int M = D / 64;
  hipStream_t st = as_stream(stream);
  if (omega_dtype == KDN_DTYPE_BF16)
    hipLaunchKernelGGL((build_omega_kernel<__bf16>), dim3(M), dim3(256), 0, st, sign_bits, M, (__bf16*)omega);
  else
    hipLaunchKernelGGL((build_omega_kernel<float>), dim3(M), dim3(256), 0, st, sign_bits, M, (float*)omega);
  return launch_status();
}

extern "C" int kdn_fwht(const void* x, int64_t rows, int64_t x_row_stride, int n, int dtype, void* out,
                        int64_t out_row_stride, void* stream) {
  if (!x || !out || rows < 0) return KDN_ERR_INVALID_ARGUMENT;
  if (!valid_dtype(dtype)) return KDN_ERR_INVALID_ARGUMENT;
  if (n < 1 || n > 64 || (n & (n - 1)) != 0) return KDN_ERR_UNSUPPORTED;
  if (x_row_stride < n || out_row_stride < n) return KDN_ERR_INVALID_ARGUMENT;
  if (rows == 0) return KDN_OK;
  hipStream_t st = as_stream(stream);
  const int64_t wgs = (rows + 3) / 4;
  if (wgs > 0x7fffffff) return KDN_ERR_UNSUPPORTED;
#define KDN_FWHT_CASE(T, N)                                                                                   \
  case N:                                                                                                     \
    hipLaunchKernelGGL((fwht_rows_kernel<T, N>), dim3((unsigned)wgs), dim3(256), 0, st, (const T*)x, rows, \
                       x_row_stride, (T*)out, out_row_stride);                                                \
    break;
  if (dtype == KDN_DTYPE_F32) {
    switch (n) { KDN_FWHT_CASE(float, 1) KDN_FWHT_CASE(float, 2) KDN_FWHT_CASE(float, 4) KDN_FWHT_CASE(float, 8)
                 KDN_FWHT_CASE(float, 16) KDN_FWHT_CASE(float, 32) KDN_FWHT_CASE(float, 64) }
  } else {
    switch (n) { KDN_FWHT_CASE(__bf16, 1) KDN_FWHT_CASE(__bf16, 2) KDN_FWHT_CASE(__bf16, 4) KDN_FWHT_CASE(__bf16, 8)
                 KDN_FWHT_CASE(__bf16, 16) KDN_FWHT_CASE(__bf16, 32) KDN_FWHT_CASE(__bf16, 64) }
  }
#undef KDN_FWHT_CASE
  return launch_status();
}

extern "C" int kdn_fwht_lift(const void* x, int64_t rows, int64_t x_row_stride, int x_dtype, int normalize_input,
                             const void* omega_bf16, const float* phase, int d_k, int D, float inv_tau, void* out,
                             int64_t out_row_stride, int out_dtype, void* stream) {
  if (!omega_bf16) return KDN_ERR_INVALID_ARGUMENT;
  return fwht_lift_impl(x, rows, x_row_stride, x_dtype, normalize_input, omega_bf16, nullptr, phase, d_k, D, inv_tau,
                        out, out_row_stride, out_dtype, stream);
}

extern "C" int kdn_fwht_lift_bits(const void* x, int64_t rows, int64_t x_row_stride, int x_dtype, int d_k,
                                  const int64_t* rademacher_bits, int D_lifted, float tau_star_inv, const float* phase,
                                  int normalize_input, void* out, int64_t out_row_stride, int out_dtype, void* stream) {
  if (!rademacher_bits) return KDN_ERR_INVALID_ARGUMENT;
  return fwht_lift_impl(x, rows, x_row_stride, x_dtype, normalize_input, nullptr, rademacher_bits, phase, d_k,
                        D_lifted, tau_star_inv, out, out_row_stride, out_dtype, stream);
}

extern "C" int kdn_fwht_lift_bits_butterfly(const void* x, int64_t rows, int64_t x_row_stride, int x_dtype, int d_k,
                                            const int64_t* rademacher_bits, int D_lifted, float tau_star_inv,
                                            const float* phase, int normalize_input, void* out, int64_t out_row_stride,
                                            int out_dtype, void* stream) {
  if (!rademacher_bits) return KDN_ERR_INVALID_ARGUMENT;
  return fwht_lift_impl(x, rows, x_row_stride, x_dtype, normalize_input, nullptr, rademacher_bits, phase, d_k,
                        D_lifted, tau_star_inv, out, out_row_stride, out_dtype, stream, true);
}

namespace kdn {
// Row renormalisation in place of rows of 1024 elements: x[r] <- x[r] / (||x[r]||_2 + eps).  One wave per
// row; lane l holds the 16 contiguous elements 16l .. 16l+15 (16- or 32-byte vector accesses).
template <typename T>
__global__ void __launch_bounds__(256) renorm_rows_kernel(T* x, int64_t rows, int64_t stride, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  T* p = x + row * stride + 16 * lane;
  float v[16];
  load8<T>(p, v);
  load8<T>(p + 8, v + 8);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) ss += v[e] * v[e];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
  const float inv = 1.f / (sqrtf(ss) + eps);
#pragma unroll
  for (int e = 0; e < 16; ++e) v[e] *= inv;
  store_row8<T>(p, v);
  store_row8<T>(p + 8, v + 8);
}
}  // namespace kdn

namespace kdn {
// The factored lift d_k = 128 -> D = 1024 in one pass (bf16 inputs): a workgroup of 8 waves, wave w lifting
// half h = w >> 2 of row tile base + (w & 3) with that half's Omega (both staged in LDS) exactly as
// lift_kernel lifts one half: phi_h = amp cos / (amp |cos| + 1e-8), rounded to the output type.  The
// halves' sums of squares of those rounded values meet in LDS, and each wave scales its half by
// 1 / (sqrt(n_0^2 + n_1^2) + 1e-7) before its only store: the concatenation renormalised onto S^1023
// (kernels/factored_kernel_deltanet.py:60-74) without a second pass over the output.
template <typename OutT>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (std::is_same<OutT, __bf16>::value) return (float)(__bf16)v;
  else return v;
}

template <typename OutT>
__global__ void __launch_bounds__(512) lift_factored_kernel(const __bf16* __restrict__ x, int64_t rows, int64_t xs,
                                                            const __bf16* __restrict__ om1, const float* __restrict__ ph1,
                                                            const __bf16* __restrict__ om2, const float* __restrict__ ph2,
                                                            float inv_tau, OutT* __restrict__ out, int64_t os) {
  constexpr int D = 512, NT = D / 16;
  // output staging as in lift_kernel (stage_off / stage_read)
  constexpr int TG = 128 / (16 * (int)sizeof(OutT));
  constexpr int SRS = 16 * TG * (int)sizeof(OutT);
  constexpr int SCPR = 16 * TG * (int)sizeof(OutT) / 16;
  static_assert(SCPR == 8, "the staging swizzle assumes 8 chunks per row");
  __shared__ bf16x8 s_omega[2][NT * 2 * 64];
  __shared__ __attribute__((aligned(16))) float s_phase_rev[2][D];
  __shared__ __attribute__((aligned(16))) unsigned char s_stage[8][16 * SRS];
  __shared__ float s_n2[2][2][4][16];  // [iteration parity][half][row tile][row]

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int h = wave >> 2, slot = wave & 3;
  for (int idx = threadIdx.x; idx < 2 * NT * 2 * 64; idx += 512) {
    const int hh = idx / (NT * 2 * 64), i = idx % (NT * 2 * 64);
    const int l = i & 63, t = i >> 7, kb = (i >> 6) & 1;
    const __bf16* om = hh ? om2 : om1;
    s_omega[hh][i] = *reinterpret_cast<const bf16x8*>(om + (int64_t)(16 * t + (l & 15)) * 64 + 32 * kb + 8 * (l >> 4));
  }
  for (int f = threadIdx.x; f < 2 * D; f += 512) s_phase_rev[f / D][f % D] = (f < D ? ph1[f] : ph2[f - D]) * 0.15915494309189535f;
  __syncthreads();

  const float ang_scale = inv_tau * 0.15915494309189535f;
  const float amp = sqrtf(2.0f / (float)D);
  const int64_t ntiles = (rows + 15) / 16;
  const int64_t stride = (int64_t)gridDim.x * 4;
  const __bf16* xh = x + 64 * h;
  // rows clamped to the last one: every load is in bounds (rows > 0); rows past the end are never stored
  auto load_tile = [&](int64_t t, u32x4 (&raw)[2]) {
    int64_t row = t * 16 + (lane & 15);
    row = row < rows ? row : rows - 1;
    const __bf16* src = xh + row * xs + 8 * (lane >> 4);
    raw[0] = *reinterpret_cast<const u32x4*>(src);
    raw[1] = *reinterpret_cast<const u32x4*>(src + 32);
  };
  u32x4 nraw[2];
  load_tile((int64_t)blockIdx.x * 4 + slot, nraw);
  int par = 0;
  for (int64_t base = (int64_t)blockIdx.x * 4; base < ntiles; base += stride, par ^= 1) {
    const int64_t tile = base + slot;
    const u32x4 raw[2] = {nraw[0], nraw[1]};
    load_tile(tile + stride, nraw);
    const bool valid = tile * 16 + (lane & 15) < rows;
    float xv[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      load8<__bf16>(reinterpret_cast<const __bf16*>(&raw[kb]), xv[kb]);
#pragma unroll
      for (int s = 0; s < 8; ++s) xv[kb][s] = valid ? xv[kb][s] : 0.f;
    }
    bf16x8 xb[2][1];
    split_frag<1>(xv[0], xb[0]);
    split_frag<1>(xv[1], xb[1]);
    auto project = [&](int t) {
      f32x4 acc = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) acc = PrecBF16::mma(acc, s_omega[h][(t * 2 + kb) * 64 + lane], xb[kb][0]);
      return acc;
    };
    float c[NT][4];
    float ss = 0.f;
    f32x4 acc = project(0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      __builtin_amdgcn_sched_barrier(0);
      const f32x4 next = (t + 1 < NT) ? project(t + 1) : zero4();
      const f32x4 ph = *reinterpret_cast<const f32x4*>(&s_phase_rev[h][16 * t + 4 * (lane >> 4)]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float cv = __builtin_amdgcn_cosf(__builtin_amdgcn_fractf(acc[i] * ang_scale + ph[i]));
        c[t][i] = cv;
        ss += cv * cv;
      }
      acc = next;
    }
    ss = sum_over_lane_groups(ss);
    const float scale = amp / (amp * sqrtf(ss) + 1e-8f);
    // this half's values as the single lift stores them, and their sum of squares per row
    float n2 = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c[t][i] = round_to<OutT>(c[t][i] * scale);
        n2 += c[t][i] * c[t][i];
      }
    n2 = sum_over_lane_groups(n2);
    if (lane < 16) s_n2[par][h][slot][lane] = n2;
    // One barrier per tile: a wave writes the other parity's slots next, and cannot pass the next
    // barrier before every wave has read these.
    __syncthreads();
    const float inv = 1.f / (sqrtf(s_n2[par][0][slot][lane & 15] + s_n2[par][1][slot][lane & 15]) + 1e-7f);
    unsigned char* stg = s_stage[wave];
#pragma unroll
    for (int g = 0; g < NT / TG; ++g) {
#pragma unroll
      for (int tp = 0; tp < TG; ++tp) {
        const int t = TG * g + tp;
        float v[4] = {c[t][0] * inv, c[t][1] * inv, c[t][2] * inv, c[t][3] * inv};
        const int r = lane & 15, byte = (int)sizeof(OutT) * (16 * tp + 4 * (lane >> 4));
        store4<OutT>(reinterpret_cast<OutT*>(stg + stage_off<OutT>(r, byte)), v);
      }
      wave_lds_sync();
#pragma unroll
      for (int j = 0; j < 16 * SCPR / 64; ++j) {
        const int q = 64 * j + lane, r = q / SCPR, pos = q % SCPR, ch = pos ^ ((r >> 1) & 7);
        const u32x4 val = stage_read<OutT>(stg, r, pos);
        const int64_t grow = tile * 16 + r;
        if (grow < rows)
          *reinterpret_cast<u32x4*>(reinterpret_cast<unsigned char*>(out + grow * os + D * h + 16 * TG * g) + 16 * ch) = val;
      }
      wave_lds_sync();
    }
  }
}
}  // namespace kdn

extern "C" int kdn_fwht_lift_factored(const void* x, int64_t rows, int64_t x_row_stride, int x_dtype,
                                      const void* omega1_bf16, const float* phase1, const void* omega2_bf16,
                                      const float* phase2, float inv_tau, void* out, int64_t out_row_stride,
                                      int out_dtype, void* stream) {
  if (!x || !omega1_bf16 || !phase1 || !omega2_bf16 || !phase2 || !out || rows < 0) return KDN_ERR_INVALID_ARGUMENT;
  if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype)) return KDN_ERR_INVALID_ARGUMENT;
  if (x_row_stride < 128 || out_row_stride < 1024) return KDN_ERR_INVALID_ARGUMENT;
  const size_t isz = dtype_size(x_dtype), osz = dtype_size(out_dtype);
  if (x_dtype == KDN_DTYPE_BF16 && rows > 0) {
    // bf16 inputs: both halves and the renormalisation in one pass, one 8-wave workgroup per CU (151 KB
    // of LDS), persistent over 4-tile groups (x and out rows 16-byte aligned, as below)
    if (!aligned(x, 16) || !aligned(out, 16) || !aligned(omega1_bf16, 16) || !aligned(omega2_bf16, 16) ||
        !aligned(phase1, 16) || !aligned(phase2, 16) ||
        (x_row_stride * (int64_t)isz) % 16 != 0 || (out_row_stride * (int64_t)osz) % 16 != 0)
      return KDN_ERR_MISALIGNED;
    int64_t wgs = ((rows + 15) / 16 + 3) / 4;
    const int cus = device_cus() > 0 ? device_cus() : 256;
    if (wgs > cus) wgs = cus;
    if (out_dtype == KDN_DTYPE_BF16)
      hipLaunchKernelGGL(lift_factored_kernel<__bf16>, dim3((unsigned)wgs), dim3(512), 0, as_stream(stream),
                         static_cast<const __bf16*>(x), rows, x_row_stride, static_cast<const __bf16*>(omega1_bf16),
                         phase1, static_cast<const __bf16*>(omega2_bf16), phase2, inv_tau, static_cast<__bf16*>(out),
                         out_row_stride);
    else
      hipLaunchKernelGGL(lift_factored_kernel<float>, dim3((unsigned)wgs), dim3(512), 0, as_stream(stream),
                         static_cast<const __bf16*>(x), rows, x_row_stride, static_cast<const __bf16*>(omega1_bf16),
                         phase1, static_cast<const __bf16*>(omega2_bf16), phase2, inv_tau, static_cast<float*>(out),
                         out_row_stride);
    return launch_status();
  }
  // each half: the structured lift of 64 features into 512 (rows of x and out stay 16-byte aligned)
  int rc = kdn_fwht_lift(x, rows, x_row_stride, x_dtype, 0, omega1_bf16, phase1, 64, 512, inv_tau, out,
                         out_row_stride, out_dtype, stream);
  if (rc != KDN_OK) return rc;
  rc = kdn_fwht_lift(static_cast<const unsigned char*>(x) + 64 * isz, rows, x_row_stride, x_dtype, 0, omega2_bf16,
                     phase2, 64, 512, inv_tau, static_cast<unsigned char*>(out) + 512 * osz, out_row_stride, out_dtype,
                     stream);
  if (rc != KDN_OK || rows == 0) return rc;
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (out_dtype == KDN_DTYPE_BF16)
    hipLaunchKernelGGL(renorm_rows_kernel<__bf16>, grid, dim3(256), 0, as_stream(stream), static_cast<__bf16*>(out),
                       rows, out_row_stride, 1e-7f);
  else
    hipLaunchKernelGGL(renorm_rows_kernel<float>, grid, dim3(256), 0, as_stream(stream), static_cast<float*>(out), rows,
                       out_row_stride, 1e-7f);
  return launch_status();
}

namespace kdn {
constexpr int FLB_TILES = 2;
// Backward of the factored lift: dx = (d out / d x)^T dout, one wave per 16 x FLB_TILES rows.  Each wave forms the
// transposed angles theta^T = Omega_h x_h^T (features x rows) on MFMA, feature tile by feature tile, so
// that a lane holds four consecutive features of one row (16-byte loads of the phases and of dout), and
// needs two passes over them:
//   1. per half h and row: n_h^2 = sum cs^2 and t_h = sum cs g (cs = sqrt(2/512) cos theta, g = dout);
//      the renormalisations' backward needs only these four sums per row:
//        E = |c| + 1e-7 with |c|^2 = sum_h n_h^2 / e_h^2, e_h = n_h + 1e-8, c = cs / e_h;
//        dc = g / E - c (c . g) / (E^2 |c|);  s_h = cs . dc = t_h / E - (c . g) / (E^2 |c|) n_h^2 / e_h;
//        dphi~ = dc / e_h - cs s_h / (e_h^2 n_h)
//   2. dL/dtheta = -sqrt(2/512) sin(theta) dphi~, and dx_h^T += Omega_h^T dtheta^T: the accumulator
//      tiles of two feature tiles are the B operand of that product as they stand (kappa order).
// A wave takes FLB_TILES row tiles, so that each Omega fragment it loads feeds that many products.
// Per-row sums run over the four lane groups in a fixed order.  Products take the precision policy P
// (bf16 operands for bf16 inputs: x and Omega are exact in bf16, so the angles equal the forward's).
template <class P, typename InT>
__global__ void __launch_bounds__(256) lift_factored_bwd_kernel(const InT* x, int64_t rows, int64_t xs,
                                                                const __bf16* om1, const float* ph1,
                                                                const __bf16* om2, const float* ph2, float inv_tau,
                                                                const float* dout, int64_t ds, float* dx,
                                                                int64_t dxs) {
  using frag = typename P::frag;
  constexpr int RT = FLB_TILES;  // 16-row tiles per wave: each Omega fragment feeds RT products
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t r0 = ((int64_t)blockIdx.x * 4 + w) * 16 * RT;
  if (r0 >= rows) return;  // wave-uniform; the kernel has no barriers
  const int fq = 4 * (lane >> 4);  // this lane's first feature inside a 16-feature tile
  int64_t row[RT];
  bool valid[RT];
  frag xb[RT][2][2];  // x^T as B fragments: row tile, half h, 32-deep block kb
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    row[rt] = r0 + 16 * rt + (lane & 15);
    valid[rt] = row[rt] < rows;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        f32x8 v;
#pragma unroll
        for (int s = 0; s < 8; ++s)
          v[s] = valid[rt] ? (float)x[row[rt] * xs + 64 * h + 32 * kb + kappa(lane, s)] : 0.f;
        xb[rt][h][kb] = P::from_f32(v);
      }
  }
  const float amp = sqrtf(2.f / 512.f);
  // pass 1
  float n2[RT][2], tg[RT][2];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) n2[rt][0] = n2[rt][1] = tg[rt][0] = tg[rt][1] = 0.f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const __bf16* om = h ? om2 : om1;
    const float* ph = h ? ph2 : ph1;
    for (int ft = 0; ft < 32; ++ft) {
      const int f0 = 16 * ft;
      const frag oa0 = P::from_f32(frag_rows_bf16(om, 64, f0, 0, lane));
      const frag oa1 = P::from_f32(frag_rows_bf16(om, 64, f0, 32, lane));
      const f32x4 b4 = *reinterpret_cast<const f32x4*>(ph + f0 + fq);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const f32x4 acc = P::mma(P::mma(zero4(), oa0, xb[rt][h][0]), oa1, xb[rt][h][1]);
        const f32x4 g4 =
            valid[rt] ? *reinterpret_cast<const f32x4*>(dout + row[rt] * ds + 512 * h + f0 + fq) : zero4();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float cs = amp * cos_rad(acc[i] * inv_tau + b4[i]);
          n2[rt][h] += cs * cs;
          tg[rt][h] += cs * g4[i];
        }
      }
    }
  }
  // per row: 1/e_h, 1/E, and the coefficients of dphi~ = g / (E e_h) - cs (corr / e_h^2 + k_h)
  float ie[RT][2], ca[RT][2], cb[RT][2];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float nn[2], e[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      n2[rt][h] = sum_over_lane_groups(n2[rt][h]);
      tg[rt][h] = sum_over_lane_groups(tg[rt][h]);
      nn[h] = sqrtf(n2[rt][h]);
      e[h] = nn[h] + 1e-8f;
      ie[rt][h] = 1.f / e[h];
    }
    const float cn = sqrtf(n2[rt][0] * ie[rt][0] * ie[rt][0] + n2[rt][1] * ie[rt][1] * ie[rt][1]);
    const float iE = 1.f / (cn + 1e-7f);
    const float sc = tg[rt][0] * ie[rt][0] + tg[rt][1] * ie[rt][1];
    const float corr = cn > 0.f ? sc * iE * iE / cn : 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float sh = tg[rt][h] * iE - corr * n2[rt][h] * ie[rt][h];
      const float kh = nn[h] > 0.f ? sh * ie[rt][h] * ie[rt][h] / nn[h] : 0.f;
      ca[rt][h] = iE * ie[rt][h];                   // times g
      cb[rt][h] = corr * ie[rt][h] * ie[rt][h] + kh;  // times cs
    }
  }
  // pass 2
  f32x4 dxt[RT][2][4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const __bf16* om = h ? om2 : om1;
    const float* ph = h ? ph2 : ph1;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) dxt[rt][h][jt] = zero4();
    for (int fb = 0; fb < 16; ++fb) {
      f32x4 dth[RT][2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int f0 = 32 * fb + 16 * u;
        const frag oa0 = P::from_f32(frag_rows_bf16(om, 64, f0, 0, lane));
        const frag oa1 = P::from_f32(frag_rows_bf16(om, 64, f0, 32, lane));
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(ph + f0 + fq);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const f32x4 acc = P::mma(P::mma(zero4(), oa0, xb[rt][h][0]), oa1, xb[rt][h][1]);
          const f32x4 g4 =
              valid[rt] ? *reinterpret_cast<const f32x4*>(dout + row[rt] * ds + 512 * h + f0 + fq) : zero4();
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float th = acc[i] * inv_tau + b4[i];
            const float cs = amp * cos_rad(th), sn = amp * sin_rad(th);
            dth[rt][u][i] = -sn * (g4[i] * ca[rt][h] - cs * cb[rt][h]);
          }
        }
      }
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const frag ot = P::from_f32(frag_cols_bf16(om, 64, 16 * jt, 32 * fb, lane));
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) dxt[rt][h][jt] = P::mma(dxt[rt][h][jt], ot, P::from_f32(pair_to8(dth[rt][0], dth[rt][1])));
      }
    }
  }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    if (valid[rt]) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
          *reinterpret_cast<f32x4*>(dx + row[rt] * dxs + 64 * h + 16 * jt + fq) = inv_tau * dxt[rt][h][jt];
    }
  }
}
}  // namespace kdn

extern "C" int kdn_fwht_lift_factored_bwd(const void* x, int64_t rows, int64_t x_row_stride, int x_dtype,
                                          const void* omega1_bf16, const float* phase1, const void* omega2_bf16,
                                          const float* phase2, float inv_tau, const float* dout,
                                          int64_t dout_row_stride, float* dx, int64_t dx_row_stride, void* stream) {
  if (!x || !omega1_bf16 || !phase1 || !omega2_bf16 || !phase2 || !dout || !dx || rows < 0)
    return KDN_ERR_INVALID_ARGUMENT;
  if (!valid_dtype(x_dtype)) return KDN_ERR_INVALID_ARGUMENT;
  if (x_row_stride < 128 || dout_row_stride < 1024 || dx_row_stride < 128) return KDN_ERR_INVALID_ARGUMENT;
  if (!(inv_tau == inv_tau)) return KDN_ERR_INVALID_ARGUMENT;
  // phases, dout and dx rows are read and written 16 bytes at a time, Omega rows 8 bytes at a time
  if (!aligned(omega1_bf16, 8) || !aligned(omega2_bf16, 8) || !aligned(x, dtype_size(x_dtype))) return KDN_ERR_MISALIGNED;
  if (!aligned(phase1, 16) || !aligned(phase2, 16) || !aligned(dout, 16) || !aligned(dx, 16) || dout_row_stride % 4 ||
      dx_row_stride % 4)
    return KDN_ERR_MISALIGNED;
  if (rows == 0) return KDN_OK;
  const int64_t wgs = (rows + 64 * FLB_TILES - 1) / (64 * FLB_TILES);
  if (wgs > 0x7fffffff) return KDN_ERR_UNSUPPORTED;
  const hipStream_t st = as_stream(stream);
  const __bf16* o1 = static_cast<const __bf16*>(omega1_bf16);
  const __bf16* o2 = static_cast<const __bf16*>(omega2_bf16);
  if (x_dtype == KDN_DTYPE_BF16)
    hipLaunchKernelGGL((lift_factored_bwd_kernel<PrecBF16, __bf16>), dim3((unsigned)wgs), dim3(256), 0, st,
                       static_cast<const __bf16*>(x), rows, x_row_stride, o1, phase1, o2, phase2, inv_tau, dout,
                       dout_row_stride, dx, dx_row_stride);
  else
    hipLaunchKernelGGL((lift_factored_bwd_kernel<PrecF32, float>), dim3((unsigned)wgs), dim3(256), 0, st,
                       static_cast<const float*>(x), rows, x_row_stride, o1, phase1, o2, phase2, inv_tau, dout,
                       dout_row_stride, dx, dx_row_stride);
  return launch_status();
}
