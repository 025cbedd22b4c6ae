// Serving step for gfx950: one ragged batch of sequences that continue from states resident in a slab.
//
//  * kdn_ragged_step : sequences of one token (decode) run decode_kernel, a single pass over each state
//                      (lift of q and k, y = S phi(q), rank-1 update); longer ones (prefill) run the
//                      chunked scan over their token ranges with the state slots read and written in
//                      place.  The split into the two lists happens on the device (ragged_split_kernel),
//                      so the caller's device copies of cu_seqlens and slots are used as they are.
//
// The reference serving op (serving/vllm_kernel_deltanet_op.cpp:11-34) declares this step but leaves
// its body empty; the recurrence is the one of kernels/kernel_deltanet_fused.py:288-300 (readout before
// update) with the structured lift of kernels/fwht.py:122-131.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "kdn_frag.hpp"
#include "kdn_internal.hpp"
#include "kdn_io.hpp"

namespace kdn {

constexpr int SRV_D = 512;   // lifted features
constexpr int SRV_DK = 64;   // input features

// ---- split ----------------------------------------------------------------------------------------
// One workgroup: thread t counts the decode / prefill sequences of its contiguous range, an inclusive
// Hillis-Steele scan over the 1024 counts gives each range its output offsets, and the ranges are then
// written in sequence order.  The lists are first filled with skip entries (slot -1, no tokens), so
// that a launch sized from host counts that differ from the device offsets reads no unwritten entry.
// A sequence whose slot lies outside [0, num_slots) (a negative slot is the padding convention) keeps
// its place in its list with slot -1 and no tokens: the decode and scan kernels skip it, its state is
// not touched and its y rows are not written.
__global__ void __launch_bounds__(1024) ragged_split_kernel(const int64_t* __restrict__ cu, const int32_t* __restrict__ slots,
                                                            int64_t n, int64_t num_slots, int64_t* __restrict__ dec_row,
                                                            int32_t* __restrict__ dec_slot, int64_t* __restrict__ pre_lo,
                                                            int64_t* __restrict__ pre_hi, int32_t* __restrict__ pre_slot) {
  __shared__ int64_t s_d[1024], s_p[1024];
  const int t = threadIdx.x;
  for (int64_t i = t; i < n; i += 1024) {
    dec_row[i] = 0;
    dec_slot[i] = -1;
    pre_lo[i] = 0;
    pre_hi[i] = 0;
    pre_slot[i] = -1;
  }
  __syncthreads();
  const int64_t per = (n + 1023) / 1024;
  const int64_t i0 = t * per, i1 = (i0 + per < n) ? i0 + per : n;
  int64_t nd = 0, np = 0;
  for (int64_t i = i0; i < i1; ++i) {
    const int64_t len = cu[i + 1] - cu[i];
    nd += len == 1;
    np += len >= 2;
  }
  s_d[t] = nd;
  s_p[t] = np;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int64_t ad = t >= off ? s_d[t - off] : 0, ap = t >= off ? s_p[t - off] : 0;
    __syncthreads();
    s_d[t] += ad;
    s_p[t] += ap;
    __syncthreads();
  }
  int64_t od = s_d[t] - nd, op = s_p[t] - np;
  for (int64_t i = i0; i < i1; ++i) {
    const int64_t lo = cu[i], hi = cu[i + 1];
    const int32_t sl = slots[i];
    const bool ok = sl >= 0 && (int64_t)sl < num_slots;
    if (hi - lo == 1) {
      dec_row[od] = lo;
      dec_slot[od] = ok ? sl : -1;
      ++od;
    } else if (hi - lo >= 2) {
      pre_lo[op] = ok ? lo : 0;
      pre_hi[op] = ok ? hi : 0;
      pre_slot[op] = ok ? sl : -1;
      ++op;
    }
  }
}

// ---- decode -----------------------------------------------------------------------------------------
struct DecodeParams {
  const int64_t* rows;   // token row of decode sequence i
  const int32_t* slots;  // its state slot
  const void* q; int64_t qs0, qs1;
  const void* k; int64_t ks0, ks1;
  const void* v; int64_t vs0, vs1;
  const float* beta; int64_t bs0, bs1;
  const float* decay; int64_t ds0, ds1;
  const __bf16* omega; const float* phase;
  float inv_tau; int normalize; int linear;
  float* states; int64_t ss0, ss1, ss2, ss3;
  void* y; int64_t ys0, ys1;
};

// Threads per (sequence, head): at least 256 and 8 per value column, so that each thread holds at most
// 64 state elements.
template <int DV>
struct DecodeThreads : std::integral_constant<int, (8 * DV > 256) ? 8 * DV : 256> {};

__device__ __forceinline__ float wave_sum(float v) {
  v += xor_shuffle<1>(v);
  v += xor_shuffle<2>(v);
  v += xor_shuffle<4>(v);
  v += xor_shuffle<8>(v);
  v += xor_shuffle<16>(v);
  v += xor_shuffle<32>(v);
  return v;
}

// grid (decode sequences, H, d_v / DV).  One workgroup per (sequence, head, slice of DV value columns;
// the columns are independent, so d_v = 128 runs as two slices that each lift q and k):
//   1. q and k rows (optionally F.normalize'd, rounded to the input dtype as the scan does) into LDS;
//   2. the lift, thread t computing features t, t + NT, ...: fp32 dot products with the bf16 Omega rows,
//      c = cos(2 pi frac(x.Omega_f inv_tau / 2 pi + phase_f / 2 pi)), and the renormalisation of
//      sqrt(2/D) c from the block's sum of squares;
//   3. thread (g, j) holds state elements S[f][j] for its feature group g (FPT features, loaded before
//      step 1 so that their latency overlaps the lift): partial
//      S^T phi(k) and S^T phi(q) per group, summed in LDS in group order; y = S^T phi(q) (before the
//      update); S[f][j] <- lambda S[f][j] + beta phi_k[f] (v_j - lambda u_j)  (delta rule), or
//      lambda S[f][j] + beta phi_k[f] v_j (linear rule); written back in place.
// One read and one write of the state: the kernel is bound by HBM.
template <typename InT, typename OutT, int DV>
__global__ void __launch_bounds__(DecodeThreads<DV>::value) decode_kernel(DecodeParams p) {
  constexpr int NT = DecodeThreads<DV>::value;
  constexpr int G = NT / DV;        // feature groups of the state pass
  constexpr int FPT = SRV_D / G;    // features per thread in the state pass
  constexpr int LPT = SRV_D / NT;  // lifted features per thread and input
  __shared__ float s_x[2][SRV_DK];
  __shared__ float s_c[2][SRV_D];
  __shared__ float s_ss[NT / 64][2];
  __shared__ float s_part[G][2][DV];

  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int64_t i = blockIdx.x, h = blockIdx.y, c0 = (int64_t)blockIdx.z * DV;
  const int64_t sl = p.slots[i];
  if (sl < 0) return;  // padding, an out-of-range slot or an entry the split did not fill (uniform)
  const int64_t row = p.rows[i];

  // The state elements of thread (g, j) and its scalar inputs are loaded first: they do not depend on
  // the lift, so their memory latency overlaps it.
  const int j = t % DV, g = t / DV;
  float* sp = p.states + sl * p.ss0 + h * p.ss1 + (int64_t)(g * FPT) * p.ss2 + (c0 + j) * p.ss3;
  float S[FPT];
#pragma unroll
  for (int l = 0; l < FPT; ++l) S[l] = sp[l * p.ss2];
  const float be = p.beta[row * p.bs0 + h * p.bs1];
  const float la = p.decay ? fminf(fmaxf(p.decay[row * p.ds0 + h * p.ds1], 1e-5f), 1.f) : 1.f;
  const float vin = (float)((const InT*)p.v)[row * p.vs0 + h * p.vs1 + c0 + j];

  // 1. inputs (waves 0 and 1: q and k)
  if (t < 2 * SRV_DK) {
    const int m = t >> 6;
    const InT* src = m == 0 ? (const InT*)p.q + row * p.qs0 + h * p.qs1 : (const InT*)p.k + row * p.ks0 + h * p.ks1;
    float x = (float)src[lane];
    if (p.normalize) {
      const float inv = 1.0f / fmaxf(sqrtf(wave_sum(x * x)), 1e-6f);
      x = (float)(InT)(x * inv);  // F.normalize keeps the input dtype
    }
    s_x[m][lane] = x;
  }
  __syncthreads();

  // 2. lift
  const float ang = p.inv_tau * 0.15915494309189535f;
  float ss[2] = {0.f, 0.f};
#pragma unroll
  for (int l = 0; l < LPT; ++l) {
    const int f = t + NT * l;
    const bf16x8* orow = reinterpret_cast<const bf16x8*>(p.omega + (int64_t)f * SRV_DK);
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int c8 = 0; c8 < SRV_DK / 8; ++c8) {
      const bf16x8 o = orow[c8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float w = (float)o[e];
        acc[0] += s_x[0][8 * c8 + e] * w;
        acc[1] += s_x[1][8 * c8 + e] * w;
      }
    }
    const float ph = p.phase[f] * 0.15915494309189535f;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const float c = __builtin_amdgcn_cosf(__builtin_amdgcn_fractf(acc[m] * ang + ph));
      s_c[m][f] = c;
      ss[m] += c * c;
    }
  }
  ss[0] = wave_sum(ss[0]);
  ss[1] = wave_sum(ss[1]);
  if (lane == 0) {
    s_ss[wv][0] = ss[0];
    s_ss[wv][1] = ss[1];
  }
  __syncthreads();
  float tot[2] = {0.f, 0.f};
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    tot[0] += s_ss[w][0];
    tot[1] += s_ss[w][1];
  }
  const float amp = sqrtf(2.0f / (float)SRV_D);
  const float scq = amp / (amp * sqrtf(tot[0]) + 1e-8f);  // phi = scq * c
  const float sck = amp / (amp * sqrtf(tot[1]) + 1e-8f);

  // 3. state pass
  float pu = 0.f, py = 0.f;
#pragma unroll
  for (int l = 0; l < FPT; ++l) {
    pu += S[l] * s_c[1][g * FPT + l];
    py += S[l] * s_c[0][g * FPT + l];
  }
  s_part[g][0][j] = pu;
  s_part[g][1][j] = py;
  __syncthreads();
  float u = 0.f, yv = 0.f;
#pragma unroll
  for (int gg = 0; gg < G; ++gg) {
    u += s_part[gg][0][j];
    yv += s_part[gg][1][j];
  }
  u *= sck;
  yv *= scq;
  if (g == 0) ((OutT*)p.y)[row * p.ys0 + h * p.ys1 + c0 + j] = (OutT)yv;
  const float coef = be * sck * (p.linear ? vin : vin - la * u);  // times c_k[f]
#pragma unroll
  for (int l = 0; l < FPT; ++l) sp[l * p.ss2] = la * S[l] + coef * s_c[1][g * FPT + l];
}

template <typename InT, typename OutT>
static int launch_decode(const DecodeParams& dp, int64_t n, int64_t H, int dv, hipStream_t st) {
  const dim3 grid((unsigned)n, (unsigned)H, (unsigned)(dv > 64 ? dv / 64 : 1));
  switch (dv) {
    case 16: hipLaunchKernelGGL((decode_kernel<InT, OutT, 16>), grid, dim3(DecodeThreads<16>::value), 0, st, dp); break;
    case 32: hipLaunchKernelGGL((decode_kernel<InT, OutT, 32>), grid, dim3(DecodeThreads<32>::value), 0, st, dp); break;
    case 64:
    case 128: hipLaunchKernelGGL((decode_kernel<InT, OutT, 64>), grid, dim3(DecodeThreads<64>::value), 0, st, dp); break;
    default: return KDN_ERR_UNSUPPORTED;
  }
  return launch_status();
}

// ---- host -------------------------------------------------------------------------------------------
static size_t round256(size_t x) { return (x + 255) & ~(size_t)255; }

// Counts and the longest prefill sequence, from the host copy of cu_seqlens; -1 if it is not ordered.
struct RaggedPlan {
  int64_t n_dec = 0, n_pre = 0, t_max = 0;
  size_t small_bytes = 0;
};

static int ragged_plan(const kdn_ragged_args* a, RaggedPlan& pl) {
  if (!a || a->num_seqs < 0 || a->H <= 0 || a->H > 65535) return KDN_ERR_INVALID_ARGUMENT;
  if (!valid_dtype(a->in_dtype) || !valid_dtype(a->out_dtype) || (a->rule != 0 && a->rule != 1))
    return KDN_ERR_INVALID_ARGUMENT;
  if (a->d_k != SRV_DK || a->D != SRV_D) return KDN_ERR_UNSUPPORTED;
  if (a->d_v != 16 && a->d_v != 32 && a->d_v != 64 && a->d_v != 128) return KDN_ERR_UNSUPPORTED;
  if (!(a->inv_tau == a->inv_tau)) return KDN_ERR_INVALID_ARGUMENT;
  if (a->num_seqs > 0 && (!a->cu_seqlens_host || a->num_slots <= 0)) return KDN_ERR_INVALID_ARGUMENT;
  for (int64_t i = 0; i < a->num_seqs; ++i) {
    const int64_t lo = a->cu_seqlens_host[i], hi = a->cu_seqlens_host[i + 1];
    if (lo < 0 || hi < lo) return KDN_ERR_INVALID_ARGUMENT;
    if (hi - lo == 1) ++pl.n_dec;
    if (hi - lo >= 2) {
      ++pl.n_pre;
      if (hi - lo > pl.t_max) pl.t_max = hi - lo;
    }
  }
  if (pl.n_pre > 65535) return KDN_ERR_UNSUPPORTED;
  const size_t n = (size_t)(a->num_seqs > 0 ? a->num_seqs : 1);
  pl.small_bytes = 3 * round256(n * 8) + 2 * round256(n * 8) + round256(n * 4);
  return KDN_OK;
}

// The scan arguments of the prefill part: n_pre sequences (start / end arrays passed separately).
static kdn_scan_args prefill_args(const kdn_ragged_args* a, const RaggedPlan& pl) {
  kdn_scan_args s = {};
  s.B = pl.n_pre; s.T = pl.t_max; s.H = a->H;
  s.d_k = a->d_k; s.D = a->D; s.d_v = a->d_v;
  s.in_dtype = a->in_dtype; s.out_dtype = a->out_dtype;
  s.normalize_input = a->normalize_input; s.inv_tau = a->inv_tau; s.rule = a->rule;
  s.q = a->q; s.q_stride[0] = 0; s.q_stride[1] = a->q_stride[0]; s.q_stride[2] = a->q_stride[1];
  s.k = a->k; s.k_stride[0] = 0; s.k_stride[1] = a->k_stride[0]; s.k_stride[2] = a->k_stride[1];
  s.v = a->v; s.v_stride[0] = 0; s.v_stride[1] = a->v_stride[0]; s.v_stride[2] = a->v_stride[1];
  s.beta = a->beta; s.beta_stride[0] = 0; s.beta_stride[1] = a->beta_stride[0]; s.beta_stride[2] = a->beta_stride[1];
  s.decay = a->decay; s.decay_stride[0] = 0; s.decay_stride[1] = a->decay_stride[0]; s.decay_stride[2] = a->decay_stride[1];
  s.omega_bf16 = a->omega_bf16; s.phase = a->phase;
  s.initial_state = a->states; s.final_state = a->states;
  for (int d = 0; d < 4; ++d) s.init_stride[d] = s.final_stride[d] = a->state_stride[d];
  s.y = a->y; s.y_stride[0] = 0; s.y_stride[1] = a->y_stride[0]; s.y_stride[2] = a->y_stride[1];
  return s;
}

}  // namespace kdn

using namespace kdn;

extern "C" size_t kdn_ragged_workspace_bytes(const kdn_ragged_args* a) {
  RaggedPlan pl;
  if (ragged_plan(a, pl) != KDN_OK) return 0;
  size_t scan = 0;
  if (pl.n_pre > 0) {
    const kdn_scan_args s = prefill_args(a, pl);
    scan = scan_workspace_bytes_pipelined(&s);
    if (scan == 0) return 0;
  }
  return pl.small_bytes + scan;
}

extern "C" int kdn_ragged_step(const kdn_ragged_args* a, void* stream, void* aux_stream) {
  RaggedPlan pl;
  int rc = ragged_plan(a, pl);
  if (rc != KDN_OK) return rc;
  if (a->num_seqs == 0 || pl.n_dec + pl.n_pre == 0) return KDN_OK;
  if (!a->cu_seqlens || !a->slots || !a->q || !a->k || !a->v || !a->beta || !a->omega_bf16 || !a->phase ||
      !a->states || !a->y || !a->workspace)
    return KDN_ERR_INVALID_ARGUMENT;
  if (!aligned(a->workspace, 256) || !aligned(a->omega_bf16, 16)) return KDN_ERR_MISALIGNED;
  const size_t need = kdn_ragged_workspace_bytes(a);
  if (need == 0) return KDN_ERR_INVALID_ARGUMENT;
  if (a->workspace_bytes < need) return KDN_ERR_WORKSPACE_TOO_SMALL;
  const hipStream_t st = as_stream(stream);
  const size_t n = (size_t)a->num_seqs;
  unsigned char* w = (unsigned char*)a->workspace;
  int64_t* dec_row = (int64_t*)w;            w += round256(n * 8);
  int64_t* pre_lo = (int64_t*)w;             w += round256(n * 8);
  int64_t* pre_hi = (int64_t*)w;             w += round256(n * 8);
  int32_t* dec_slot = (int32_t*)w;           w += round256(n * 8);
  int32_t* pre_slot = (int32_t*)w;           w += round256(n * 8);
  w += round256(n * 4);
  hipLaunchKernelGGL(ragged_split_kernel, dim3(1), dim3(1024), 0, st, a->cu_seqlens, a->slots, a->num_seqs,
                     a->num_slots, dec_row, dec_slot, pre_lo, pre_hi, pre_slot);
  rc = launch_status();
  if (rc != KDN_OK) return rc;
  if (pl.n_dec > 0) {
    DecodeParams dp;
    dp.rows = dec_row; dp.slots = dec_slot;
    dp.q = a->q; dp.qs0 = a->q_stride[0]; dp.qs1 = a->q_stride[1];
    dp.k = a->k; dp.ks0 = a->k_stride[0]; dp.ks1 = a->k_stride[1];
    dp.v = a->v; dp.vs0 = a->v_stride[0]; dp.vs1 = a->v_stride[1];
    dp.beta = a->beta; dp.bs0 = a->beta_stride[0]; dp.bs1 = a->beta_stride[1];
    dp.decay = a->decay; dp.ds0 = a->decay_stride[0]; dp.ds1 = a->decay_stride[1];
    dp.omega = (const __bf16*)a->omega_bf16; dp.phase = a->phase;
    dp.inv_tau = a->inv_tau; dp.normalize = a->normalize_input ? 1 : 0; dp.linear = a->rule == 1 ? 1 : 0;
    dp.states = a->states;
    dp.ss0 = a->state_stride[0]; dp.ss1 = a->state_stride[1]; dp.ss2 = a->state_stride[2]; dp.ss3 = a->state_stride[3];
    dp.y = a->y; dp.ys0 = a->y_stride[0]; dp.ys1 = a->y_stride[1];
    if (a->in_dtype == KDN_DTYPE_BF16)
      rc = a->out_dtype == KDN_DTYPE_BF16 ? launch_decode<__bf16, __bf16>(dp, pl.n_dec, a->H, a->d_v, st)
                                          : launch_decode<__bf16, float>(dp, pl.n_dec, a->H, a->d_v, st);
    else
      rc = a->out_dtype == KDN_DTYPE_BF16 ? launch_decode<float, __bf16>(dp, pl.n_dec, a->H, a->d_v, st)
                                          : launch_decode<float, float>(dp, pl.n_dec, a->H, a->d_v, st);
    if (rc != KDN_OK) return rc;
  }
  if (pl.n_pre > 0) {
    kdn_scan_args s = prefill_args(a, pl);
    s.state_slots = pre_slot;
    s.workspace = w;
    s.workspace_bytes = a->workspace_bytes - (size_t)(w - (unsigned char*)a->workspace);
    rc = scan_pipelined(&s, pre_lo, pre_hi, stream, aux_stream, nullptr);
    if (rc != KDN_OK) return rc;
  }
  return KDN_OK;
}
