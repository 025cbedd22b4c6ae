// MFMA fragment conventions shared by every kernel of the Kernel-DeltaNet prefill path (gfx950 only).
//
// All matrix products use the 16x16 output-tile MFMAs of CDNA4 (wave64):
//   v_mfma_f32_16x16x32_bf16 : A[16][32] * B[32][16] -> D[16][16]
//   v_mfma_f32_16x16x4_f32   : A[16][4]  * B[4][16]  -> D[16][16]
// Hardware lane layout (verified on gfx950 by an in-bounds probe):
//   bf16: lane l holds A[l%16][8*(l/16)+s] and B[8*(l/16)+s][l%16], s = 0..7
//   f32 : lane l holds A[l%16][l/16]       and B[l/16][l%16]
//   D   : lane l holds D[4*(l/16)+i][l%16], i = 0..3            (both)
//
// A "fragment" is a 16-row x 32-deep operand slab held by one wave: lane l, slot s (0..7) holds
// row (l & 15) at logical depth kappa(l, s) = 16*(s>>2) + 4*(l>>4) + (s&3).  For bf16 the eight
// slots feed one MFMA; for f32 slot s feeds the s-th of eight 16x16x4 MFMAs.  Because A and B are
// indexed by the same (l, s) -> depth map, the permuted depth order is invisible in the product.
//
// The point of kappa: two vertically adjacent 16x16 accumulator tiles of C (rows 0-15 and 16-31 of a
// 32-row block) hold, in lane l, exactly rows kappa(l, 0..7) of column (l & 15).  So the accumulator
// of one product is, register for register, a B fragment of the next product contracting over C's
// row index (or an A fragment of C^T).  The scan chains its products this way with no shuffles.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kdn {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) float f32x8;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;

__device__ __forceinline__ int kappa(int lane, int s) { return 16 * (s >> 2) + 4 * (lane >> 4) + (s & 3); }

__device__ __forceinline__ f32x4 zero4() { f32x4 z = {0.f, 0.f, 0.f, 0.f}; return z; }

// bf16 precision policy: operands rounded to bf16, fp32 accumulation.
struct PrecBF16 {
  typedef bf16x8 frag;
  static constexpr int frag_bytes = 16;
  __device__ __forceinline__ static f32x4 mma(f32x4 acc, const frag& a, const frag& b) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  __device__ __forceinline__ static frag from_f32(const f32x8& v) {
    frag r;
#pragma unroll
    for (int s = 0; s < 8; ++s) r[s] = (__bf16)v[s];
    return r;
  }
  __device__ __forceinline__ static float get(const frag& f, int s) { return (float)f[s]; }
  __device__ __forceinline__ static void set(frag& f, int s, float v) { f[s] = (__bf16)v; }
};

// fp32 precision policy: exact fp32 products (eight 16x16x4 MFMAs per 32-deep fragment).
struct PrecF32 {
  typedef f32x8 frag;
  static constexpr int frag_bytes = 32;
  __device__ __forceinline__ static f32x4 mma(f32x4 acc, const frag& a, const frag& b) {
#pragma unroll
    for (int s = 0; s < 8; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], acc, 0, 0, 0);
    return acc;
  }
  __device__ __forceinline__ static frag from_f32(const f32x8& v) { return v; }
  __device__ __forceinline__ static float get(const frag& f, int s) { return f[s]; }
  __device__ __forceinline__ static void set(frag& f, int s, float v) { f[s] = v; }
};

// Two accumulator tiles (rows 0-15, 16-31 of a 32-block) -> the eight kappa-ordered values.
__device__ __forceinline__ f32x8 pair_to8(const f32x4& lo, const f32x4& hi) {
  f32x8 r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

// Fragment load/store: lane l's slots are contiguous (frag_bytes), a wave's fragment is contiguous.
template <class P>
__device__ __forceinline__ typename P::frag load_frag(const void* base, int lane) {
  return reinterpret_cast<const typename P::frag*>(base)[lane];
}
template <class P>
__device__ __forceinline__ void store_frag(void* base, int lane, const typename P::frag& f) {
  reinterpret_cast<typename P::frag*>(base)[lane] = f;
}
// Streaming store (nt): for data no kernel reads back while it could still be in L2, so that it does
// not evict lines other kernels running at the same time are about to read.
template <class P>
__device__ __forceinline__ void store_frag_nt(void* base, int lane, const typename P::frag& f) {
  __builtin_nontemporal_store(f, reinterpret_cast<typename P::frag*>(base) + lane);
}

// Streaming load (nt): for data read once by the last kernel that uses it, so that it does not evict
// lines other kernels running at the same time are about to read.
template <class P>
__device__ __forceinline__ typename P::frag load_frag_nt(const void* base, int lane) {
  return __builtin_nontemporal_load(reinterpret_cast<const typename P::frag*>(base) + lane);
}

// Read-only streaming loads that bypass nothing: plain global loads (the workspace is re-read once).
__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

// Orders one wave's LDS accesses at this point for exchanges between its lanes (a lane reading what
// another lane of the same wave stored): the hardware performs a wave's LDS operations in order, so no
// instruction is emitted at wavefront scope, but the compiler may no longer move loads or stores across
// it (it could otherwise reorder accesses that look disjoint from one lane's point of view).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Workgroup barrier that orders LDS only: this wave's LDS operations are complete, then s_barrier.  Unlike
// __syncthreads() it does not drain the wave's outstanding global loads and stores (whose release fence the
// compiler implements as s_waitcnt vmcnt(0)), so loads issued early keep travelling across it.  For
// kernels whose waves exchange data through LDS only.  The memory clobber keeps the compiler from moving
// memory operations across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 64-lane butterfly partner exchange: value held by lane (lane ^ H).
template <int H>
__device__ __forceinline__ float xor_shuffle(float v) {
  if constexpr (H == 1) {
    // DPP quad_perm [1,0,3,2]
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
  } else if constexpr (H == 2) {
    // DPP quad_perm [2,3,0,1]
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
  } else if constexpr (H == 4 || H == 8 || H == 16) {
    // ds_swizzle bit-mask mode within 32 lanes: and_mask=0x1F, or_mask=0, xor_mask=H
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), (H << 10) | 0x1F));
  } else {
    static_assert(H == 32, "xor_shuffle: H must be a power of two below 64");
    // ds_bpermute across the two 32-lane halves
    int lane = __lane_id();
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, v)));
  }
}

// Sum over the lanes that share (lane & 15): lanes l, l^16, l^32, l^48.
// The value of lane 4 (l >> 2) + P of each lane's quad (DPP quad_perm [P, P, P, P]).
template <int P>
__device__ __forceinline__ float quad_bcast(float v) {
  static_assert(P >= 0 && P < 4, "quad_bcast: P must be a lane of the quad");
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), P * 0x55, 0xF, 0xF, true));
}

__device__ __forceinline__ float sum_over_lane_groups(float v) {
  v += xor_shuffle<16>(v);
  v += xor_shuffle<32>(v);
  return v;
}

// cos of an angle in radians via v_cos_f32 (which takes revolutions), with explicit reduction of the
// revolution count to [-0.5, 0.5] so that any finite angle stays inside the instruction's domain.
__device__ __forceinline__ float cos_rad(float angle) {
  float r = angle * 0.15915494309189535f;  // 1 / (2 pi)
  r = r - __builtin_rintf(r);
  return __builtin_amdgcn_cosf(r);
}

}  // namespace kdn
