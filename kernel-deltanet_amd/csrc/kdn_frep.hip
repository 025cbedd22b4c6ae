// Lifts of D = 128 and 256 features (d_k = 64) on the D = 512 kernels, by feature replication.
//
// With Omega' = [Omega; ...; Omega] and phase' = [phase; ...; phase] (r = 512 / D copies), the D = 512
// lift gives phi' = sqrt(2/512) cos(x Omega'^T / tau + phase') = J phi, J = [I; ...; I] / sqrt(r), where
// phi = sqrt(2/D) cos(x Omega^T / tau + phase) is the D-wide lift; ||phi'|| = ||phi||, so the renormalised
// features are J phi-hat likewise.  J^T J = I, so every product the scan forms (K K^T, Q K^T, S phi)
// is that of the D-wide scan, and for a 512-wide state S' the projection P(S') = S' J (the sum of its r
// feature blocks over sqrt(r)) follows the D-wide recurrence exactly:
//   P(lambda S' (I - beta k' k'^T) + beta v k'^T) = lambda P(S') (I - beta k k^T) + beta v k^T,
//   S' q' = P(S') q,
// for any S'_0 with P(S'_0) = S_0; the 512-wide scan starts from L(S_0) = S_0 J^T (each block S_0 / sqrt(r))
// and the final state is P(S'_T).  The backward takes dL/dS'_T = L(dL/dS_T) and returns
// dL/dS_0 = P(dL/dS'_0); the gradients of q, k, v, beta, lambda and 1/tau sum over the r copies of each
// feature inside the 512-wide backward, which is the chain rule through phi' = J phi.
// The cost is that of the 512-wide scan.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include "kdn_internal.hpp"

namespace kdn {

constexpr int WD = 512;  // the width the kernels run at

bool frep_applies(const kdn_scan_args* a) { return a && a->feature_mode == 0 && (a->D == 128 || a->D == 256); }

static size_t up256(size_t x) { return (x + 255) / 256 * 256; }

static int64_t omega_heads(const kdn_scan_args* a) { return a->omega_head_stride ? a->H : 1; }
static int64_t phase_heads(const kdn_scan_args* a) { return a->phase_head_stride ? a->H : 1; }

size_t frep_state_bytes(const kdn_scan_args* a) { return (size_t)a->B * a->H * WD * a->d_v * sizeof(float); }

FrepLayout frep_layout(const kdn_scan_args* a, size_t base, int nstates) {
  FrepLayout L = {};
  size_t o = up256(base);
  L.base = base;
  L.omega = o; o += up256((size_t)omega_heads(a) * WD * 64 * 2);
  if (a->omega_lo) { L.omega_lo = o; o += up256((size_t)omega_heads(a) * WD * 64 * 2); }
  L.phase = o; o += up256((size_t)phase_heads(a) * WD * 4);
  for (int i = 0; i < nstates && i < 3; ++i) { L.state[i] = o; o += up256(frep_state_bytes(a)); }
  L.total = o;
  return L;
}

kdn_scan_args frep_wide(const kdn_scan_args* a, const FrepLayout* L, void* ws) {
  kdn_scan_args w = *a;
  w.D = WD;
  if (a->omega_head_stride) w.omega_head_stride = (int64_t)WD * 64;
  if (a->phase_head_stride) w.phase_head_stride = WD;
  if (L && ws) {
    unsigned char* b = static_cast<unsigned char*>(ws);
    w.omega_bf16 = b + L->omega;
    w.omega_lo = a->omega_lo ? b + L->omega_lo : nullptr;
    w.phase = reinterpret_cast<const float*>(b + L->phase);
    w.workspace = ws;
    w.workspace_bytes = L->base;
  }
  return w;
}

void frep_contiguous_strides(const kdn_scan_args* a, int64_t s[4]) {
  s[0] = a->H * WD * a->d_v; s[1] = (int64_t)WD * a->d_v; s[2] = a->d_v; s[3] = 1;
}

// dst row f' (wu 32-bit words) of head y = src row f' % D of head y (src heads `src_hw` words apart)
__global__ void __launch_bounds__(256) frep_rows_kernel(const uint32_t* src, int64_t src_hw, int D, int wu,
                                                       uint32_t* dst) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  const int64_t n = (int64_t)WD * wu;
  if (i >= n) return;
  const int64_t y = blockIdx.y;
  const int64_t f = i / wu, e = i % wu;
  dst[y * n + i] = src[y * src_hw + (f % D) * wu + e];
}

// L: dst[b][h][f'][c] = s(b, h, f' % D, c) * scale
__global__ void __launch_bounds__(256) frep_lift_kernel(const float* s, int64_t s0, int64_t s1, int64_t s2, int64_t s3,
                                                       int64_t H, int D, int dv, float scale, float* dst, int64_t n) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t c = i % dv, f = (i / dv) % WD, bh = i / ((int64_t)dv * WD);
    dst[i] = s[(bh / H) * s0 + (bh % H) * s1 + (f % D) * s2 + c * s3] * scale;
  }
}

// P: s(b, h, f, c) = sum_i src[b][h][f + D i][c] * scale
__global__ void __launch_bounds__(256) frep_fold_kernel(const float* src, int64_t H, int D, int dv, float scale, float* s,
                                                       int64_t s0, int64_t s1, int64_t s2, int64_t s3, int64_t n) {
  const int r = WD / D;
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t c = i % dv, f = (i / dv) % D, bh = i / ((int64_t)dv * D);
    float acc = 0.f;
    for (int k = 0; k < r; ++k) acc += src[(bh * WD + f + (int64_t)D * k) * dv + c];
    s[(bh / H) * s0 + (bh % H) * s1 + f * s2 + c * s3] = acc * scale;
  }
}

static unsigned blocks_for(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return (unsigned)(b < 4096 ? b : 4096);
}

static float inv_sqrt_r(const kdn_scan_args* a) { return 1.0f / sqrtf((float)(WD / a->D)); }

int frep_tables(const kdn_scan_args* a, const FrepLayout* L, void* ws, hipStream_t st) {
  unsigned char* b = static_cast<unsigned char*>(ws);
  const unsigned gx = (unsigned)((WD * 32 + 255) / 256);
  hipLaunchKernelGGL(frep_rows_kernel, dim3(gx, (unsigned)omega_heads(a)), dim3(256), 0, st,
                     static_cast<const uint32_t*>(a->omega_bf16), a->omega_head_stride / 2, a->D, 32,
                     reinterpret_cast<uint32_t*>(b + L->omega));
  if (a->omega_lo)
    hipLaunchKernelGGL(frep_rows_kernel, dim3(gx, (unsigned)omega_heads(a)), dim3(256), 0, st,
                       static_cast<const uint32_t*>(a->omega_lo), a->omega_head_stride / 2, a->D, 32,
                       reinterpret_cast<uint32_t*>(b + L->omega_lo));
  hipLaunchKernelGGL(frep_rows_kernel, dim3((WD + 255) / 256, (unsigned)phase_heads(a)), dim3(256), 0, st,
                     reinterpret_cast<const uint32_t*>(a->phase), a->phase_head_stride, a->D, 1,
                     reinterpret_cast<uint32_t*>(b + L->phase));
  return hipGetLastError() == hipSuccess ? KDN_OK : KDN_ERR_DEVICE;
}

int frep_state_lift(const kdn_scan_args* a, const float* s, const int64_t* s4, float* dst, hipStream_t st) {
  const int64_t n = a->B * a->H * WD * a->d_v;
  hipLaunchKernelGGL(frep_lift_kernel, dim3(blocks_for(n)), dim3(256), 0, st, s, s4[0], s4[1], s4[2], s4[3], a->H,
                     a->D, a->d_v, inv_sqrt_r(a), dst, n);
  return hipGetLastError() == hipSuccess ? KDN_OK : KDN_ERR_DEVICE;
}

int frep_state_fold(const kdn_scan_args* a, const float* src, float* s, const int64_t* s4, hipStream_t st) {
  const int64_t n = a->B * a->H * (int64_t)a->D * a->d_v;
  hipLaunchKernelGGL(frep_fold_kernel, dim3(blocks_for(n)), dim3(256), 0, st, src, a->H, a->D, a->d_v, inv_sqrt_r(a), s,
                     s4[0], s4[1], s4[2], s4[3], n);
  return hipGetLastError() == hipSuccess ? KDN_OK : KDN_ERR_DEVICE;
}

}  // namespace kdn
