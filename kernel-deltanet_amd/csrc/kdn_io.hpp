// Element loads/stores and the bf16 splitting used by the MFMA feature lift (gfx950).
#pragma once
#include "kdn_frag.hpp"

namespace kdn {

template <typename InT>
struct XFrag;
template <>
struct XFrag<__bf16> {
  static constexpr int NSPLIT = 1;
};
template <>
struct XFrag<float> {
  static constexpr int NSPLIT = 3;
};

template <typename T>
__device__ __forceinline__ void load8(const T* p, float* out8);
template <>
__device__ __forceinline__ void load8<__bf16>(const __bf16* p, float* o) {
  bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int s = 0; s < 8; ++s) o[s] = (float)v[s];
}
template <>
__device__ __forceinline__ void load8<float>(const float* p, float* o) {
  f32x4 a = *reinterpret_cast<const f32x4*>(p);
  f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
  o[0] = a[0]; o[1] = a[1]; o[2] = a[2]; o[3] = a[3];
  o[4] = b[0]; o[5] = b[1]; o[6] = b[2]; o[7] = b[3];
}

// Eight consecutive elements from fp32 values (one 16-byte store for bf16, two for fp32).
template <typename T>
__device__ __forceinline__ void store_row8(T* p, const float* v);
template <>
__device__ __forceinline__ void store_row8<__bf16>(__bf16* p, const float* v) {
  bf16x8 r;
#pragma unroll
  for (int s = 0; s < 8; ++s) r[s] = (__bf16)v[s];
  *reinterpret_cast<bf16x8*>(p) = r;
}
template <>
__device__ __forceinline__ void store_row8<float>(float* p, const float* v) {
  f32x4 a = {v[0], v[1], v[2], v[3]}, c = {v[4], v[5], v[6], v[7]};
  reinterpret_cast<f32x4*>(p)[0] = a;
  reinterpret_cast<f32x4*>(p)[1] = c;
}

template <typename T>
__device__ __forceinline__ void store4(T* p, const float* v);
template <>
__device__ __forceinline__ void store4<__bf16>(__bf16* p, const float* v) {
  typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
  bf16x4 r;
  r[0] = (__bf16)v[0]; r[1] = (__bf16)v[1]; r[2] = (__bf16)v[2]; r[3] = (__bf16)v[3];
  *reinterpret_cast<bf16x4*>(p) = r;
}
template <>
__device__ __forceinline__ void store4<float>(float* p, const float* v) {
  f32x4 r = {v[0], v[1], v[2], v[3]};
  *reinterpret_cast<f32x4*>(p) = r;
}

// Splits x (fp32 per slot) into NSPLIT bf16 fragments whose sum reproduces x exactly for bf16
// inputs (NSPLIT = 1) and to within 2^-24 relative for fp32 inputs (NSPLIT = 3).
template <int NSPLIT>
__device__ __forceinline__ void split_frag(const float* x8, bf16x8* parts) {
  float r[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) r[s] = x8[s];
#pragma unroll
  for (int p = 0; p < NSPLIT; ++p) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      __bf16 h = (__bf16)r[s];
      parts[p][s] = h;
      r[s] -= (float)h;
    }
  }
}

}  // namespace kdn
