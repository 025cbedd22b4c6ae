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

// ---- runs of a slot map (kdn_slot_step) -------------------------------------------------------------
// Two passes over blocks of `span` tokens (a multiple of RUN_TILE; at most RUN_BLOCKS_MAX blocks): a run
// starts at token 0 and wherever a token's slot differs from the previous token's.
//   slot_count_kernel: block b counts the run starts among its tokens (coalesced loads) -> cnt[b];
//   slot_runs_kernel:  block b takes its first run index from the counts of the blocks before it, then
//     writes its runs in token order, RUN_TILE tokens per pass (thread t owns 8 consecutive tokens, an
//     exclusive scan over the workgroup orders them): cu[r] = first token of run r, slot[r] = its slot.
// Entries from the number of runs to `cap` get cu = n (no tokens) and slot -1.  More runs than `cap` (a
// map whose distinct runs do not have distinct slots) mark every run skipped and set *status to 1.
constexpr int RUN_THREADS = 256, RUN_PER_THREAD = 8, RUN_TILE = RUN_THREADS * RUN_PER_THREAD;
constexpr int64_t RUN_BLOCKS_MAX = 1024;

struct RunGrid {
  int64_t span, blocks;
};
static RunGrid run_grid(int64_t n) {
  const int64_t tiles = (n + RUN_TILE - 1) / RUN_TILE;
  const int64_t per = (tiles + RUN_BLOCKS_MAX - 1) / RUN_BLOCKS_MAX;
  RunGrid g;
  g.span = (per > 0 ? per : 1) * RUN_TILE;
  g.blocks = n > 0 ? (n + g.span - 1) / g.span : 1;
  return g;
}

__device__ __forceinline__ int64_t slot_at(const void* sm, int slot_bytes, int64_t i) {
  return slot_bytes == 8 ? reinterpret_cast<const int64_t*>(sm)[i] : (int64_t)reinterpret_cast<const int32_t*>(sm)[i];
}

// Sum over the workgroup (256 threads); every thread gets the result.
__device__ __forceinline__ int64_t run_block_sum(int64_t v, int64_t* s_w) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int t = threadIdx.x;
  __syncthreads();
  if ((t & 63) == 0) s_w[t >> 6] = v;
  __syncthreads();
  return s_w[0] + s_w[1] + s_w[2] + s_w[3];
}

__global__ void __launch_bounds__(RUN_THREADS) slot_count_kernel(const void* __restrict__ sm, int slot_bytes, int64_t n,
                                                                 int64_t span, int64_t* __restrict__ cnt) {
  __shared__ int64_t s_w[4];
  const int64_t lo = (int64_t)blockIdx.x * span, hi = lo + span < n ? lo + span : n;
  int64_t c = 0;
  for (int64_t i = lo + threadIdx.x; i < hi; i += RUN_THREADS)
    c += (i == 0 || slot_at(sm, slot_bytes, i) != slot_at(sm, slot_bytes, i - 1));
  c = run_block_sum(c, s_w);
  if (threadIdx.x == 0) cnt[blockIdx.x] = c;
}

__global__ void __launch_bounds__(RUN_THREADS) slot_runs_kernel(const void* __restrict__ sm, int slot_bytes, int64_t n,
                                                                int64_t span, int64_t nblocks,
                                                                const int64_t* __restrict__ cnt, int64_t cap,
                                                                int64_t* __restrict__ cu, int32_t* __restrict__ slot,
                                                                int32_t* __restrict__ status) {
  __shared__ int64_t s_w[4];
  __shared__ int s_scan[4];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  int64_t pre = 0, tot = 0;
  for (int64_t g = t; g < nblocks; g += RUN_THREADS) {
    const int64_t v = cnt[g];
    tot += v;
    pre += g < (int64_t)blockIdx.x ? v : 0;
  }
  pre = run_block_sum(pre, s_w);
  tot = run_block_sum(tot, s_w);
  const bool over = tot > cap;
  const int64_t lo = (int64_t)blockIdx.x * span, hi = lo + span < n ? lo + span : n;
  int64_t r0 = pre;
  for (int64_t base = lo; base < hi; base += RUN_TILE) {
    const int64_t i0 = base + (int64_t)RUN_PER_THREAD * t;
    int64_t v[RUN_PER_THREAD + 1];
#pragma unroll
    for (int k = 0; k <= RUN_PER_THREAD; ++k) {
      const int64_t i = i0 - 1 + k;
      v[k] = (i >= 0 && i < hi) ? slot_at(sm, slot_bytes, i) : 0;
    }
    int c = 0;
#pragma unroll
    for (int k = 1; k <= RUN_PER_THREAD; ++k) {
      const int64_t i = i0 - 1 + k;
      c += (i < hi && (i == 0 || v[k] != v[k - 1])) ? 1 : 0;
    }
    // exclusive scan of c over the workgroup
    int inc = c;
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(inc, o);
      if (lane >= o) inc += u;
    }
    __syncthreads();
    if (lane == 63) s_scan[wv] = inc;
    __syncthreads();
    int wbase = 0;
    for (int q = 0; q < wv; ++q) wbase += s_scan[q];
    const int tile_total = s_scan[0] + s_scan[1] + s_scan[2] + s_scan[3];
    int64_t r = r0 + wbase + inc - c;
#pragma unroll
    for (int k = 1; k <= RUN_PER_THREAD; ++k) {
      const int64_t i = i0 - 1 + k;
      if (i < hi && (i == 0 || v[k] != v[k - 1])) {
        if (r < cap) {
          cu[r] = i;
          const int64_t sv = v[k];
          slot[r] = (over || sv < 0 || sv > 0x7fffffff) ? -1 : (int32_t)sv;
        }
        ++r;
      }
    }
    r0 += tile_total;
  }
  const int64_t used = over ? cap : tot;
  for (int64_t k = used + (int64_t)blockIdx.x * RUN_THREADS + t; k < cap; k += nblocks * RUN_THREADS) {
    cu[k] = n;
    slot[k] = -1;
  }
  if (blockIdx.x == 0 && t == 0) {
    cu[cap] = n;
    if (status) *status = over ? 1 : 0;
  }
}

// The packed slot layout of the prefill list (ragged_split_kernel's pre_lo / pre_hi, `cap` entries):
// entry i takes ceil(len / 64) chunk slots and one spare when it has tokens, none otherwise; off[i] is the
// exclusive prefix of those counts (off[cap] = *total) and first[w] the entry holding slot w * win (for
// windows past the total, the last entry).  One workgroup: thread t sums a contiguous range of entries and
// an inclusive scan over the 1024 sums gives each range its offset.
__global__ void __launch_bounds__(1024) flat_plan_kernel(const int64_t* __restrict__ lo, const int64_t* __restrict__ hi,
                                                         int64_t cap, int64_t win, int64_t nwin, int64_t* __restrict__ off,
                                                         int64_t* __restrict__ first, int64_t* __restrict__ total) {
  __shared__ int64_t s_c[1024];
  const int t = threadIdx.x;
  const int64_t per = (cap + 1023) / 1024;
  const int64_t i0 = t * per < cap ? t * per : cap, i1 = (i0 + per < cap) ? i0 + per : cap;
  auto slots_of = [&](int64_t i) -> int64_t {
    const int64_t len = hi[i] - lo[i];
    return len >= 2 ? (len + 63) / 64 + 1 : 0;
  };
  int64_t cnt = 0;
  for (int64_t i = i0; i < i1; ++i) cnt += slots_of(i);
  s_c[t] = cnt;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const int64_t a = t >= o ? s_c[t - o] : 0;
    __syncthreads();
    s_c[t] += a;
    __syncthreads();
  }
  int64_t acc = s_c[t] - cnt;
  for (int64_t i = i0; i < i1; ++i) {
    off[i] = acc;
    acc += slots_of(i);
  }
  if (t == 1023) {
    off[cap] = s_c[1023];
    *total = s_c[1023];
  }
  __syncthreads();  // off[] complete (the block's global writes are visible to its own threads after the barrier)
  for (int64_t w = t; w < nwin; w += 1024) {
    const int64_t g = w * win;
    int64_t a = 0, b = cap;  // the last i in [0, cap) with off[i] <= g
    while (b - a > 1) {
      const int64_t m = (a + b) >> 1;
      if (off[m] <= g) a = m;
      else b = m;
    }
    first[w] = a;
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
  // With an auxiliary stream and both kinds of sequences, the decode runs on it after the prefill's prep
  // launches (which fill the GPU), beside the prefill's last chain launches (which do not): the two share
  // no state slot and no row of y.  Events order it after the split and `stream` after it.
  const hipStream_t aux = aux_stream ? as_stream(aux_stream) : nullptr;
  const bool dec_aux = pl.n_dec > 0 && pl.n_pre > 0 && aux && aux != st;
  EventSet evs;
  if (dec_aux) {
    rc = evs.create(2);
    if (rc != KDN_OK) return rc;
    if (hipEventRecord(evs.ev[0], st) != hipSuccess || hipStreamWaitEvent(aux, evs.ev[0], 0) != hipSuccess)
      return KDN_ERR_DEVICE;
  }
  auto run_decode = [&](hipStream_t ds) -> int {
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
      return a->out_dtype == KDN_DTYPE_BF16 ? launch_decode<__bf16, __bf16>(dp, pl.n_dec, a->H, a->d_v, ds)
                                            : launch_decode<__bf16, float>(dp, pl.n_dec, a->H, a->d_v, ds);
    return a->out_dtype == KDN_DTYPE_BF16 ? launch_decode<float, __bf16>(dp, pl.n_dec, a->H, a->d_v, ds)
                                          : launch_decode<float, float>(dp, pl.n_dec, a->H, a->d_v, ds);
  };
  if (pl.n_dec > 0 && !dec_aux) {
    rc = run_decode(st);
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
  if (dec_aux) {
    rc = run_decode(aux);
    if (rc != KDN_OK) return rc;
    if (hipEventRecord(evs.ev[1], aux) != hipSuccess || hipStreamWaitEvent(st, evs.ev[1], 0) != hipSuccess)
      return KDN_ERR_DEVICE;
  }
  return KDN_OK;
}

// ---- the step from a slot map ----------------------------------------------------------------------
namespace kdn {

// Packed chunk slots per prefill window: at most SLOT_WIN_MAX (the sequences of one window carry their
// states side by side, so a window must hold many of them: 128 slots, about two config-5 prefills per
// window, took 5.8 ms for the config-5 step against 3.7 with host offsets), fewer when all fit.
constexpr int64_t SLOT_WIN_MAX = 1024;

// Sizes of kdn_slot_step's workspace, all bounds from num_tokens and num_slots: `cap` runs at most (one
// per slot, and the padding runs between them), n_pre prefills (two tokens or more each), G packed slots
// (each prefill's chunks and its spare), `nwin` windows of SLOT_WIN slots.
struct SlotPlan {
  int64_t cap, n_pre, win, nwin, seq_bound;
  size_t small_bytes, buf_bytes, total;
};

static kdn_scan_args slot_scan_args(const kdn_slot_step_args* a, int64_t seq_bound) {
  kdn_scan_args s = {};
  s.B = seq_bound; s.T = a->num_tokens; s.H = a->H;
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

static int slot_plan(const kdn_slot_step_args* a, SlotPlan& pl) {
  if (!a || a->num_tokens < 0 || a->H <= 0 || a->H > 65535) return KDN_ERR_INVALID_ARGUMENT;
  if (!valid_dtype(a->in_dtype) || !valid_dtype(a->out_dtype) || (a->rule != 0 && a->rule != 1))
    return KDN_ERR_INVALID_ARGUMENT;
  if (a->slot_bytes != 4 && a->slot_bytes != 8) return KDN_ERR_INVALID_ARGUMENT;
  if (a->d_k != SRV_DK || a->D != SRV_D) return KDN_ERR_UNSUPPORTED;
  if (a->d_v != 16 && a->d_v != 32 && a->d_v != 64 && a->d_v != 128) return KDN_ERR_UNSUPPORTED;
  if (!(a->inv_tau == a->inv_tau) || a->num_slots <= 0) return KDN_ERR_INVALID_ARGUMENT;
  const int64_t n = a->num_tokens;
  pl.cap = 2 * a->num_slots + 1 < n ? 2 * a->num_slots + 1 : n;
  if (pl.cap < 1) pl.cap = 1;
  pl.n_pre = pl.cap < n / 2 ? pl.cap : n / 2;
  const int64_t g = (n + 63) / 64 + 2 * pl.n_pre;
  pl.win = (g + 63) / 64 * 64 < SLOT_WIN_MAX ? (g + 63) / 64 * 64 : SLOT_WIN_MAX;
  pl.nwin = pl.n_pre > 0 ? (g + pl.win - 1) / pl.win : 0;
  pl.seq_bound = pl.win / 2 + 1 < pl.cap ? pl.win / 2 + 1 : pl.cap;
  const size_t c = (size_t)pl.cap;
  pl.small_bytes = round256((size_t)run_grid(n).blocks * 8)                      // run counts per block
                 + round256((c + 1) * 8) + round256(c * 4)                       // runs
                 + 3 * round256(c * 8) + 2 * round256(c * 4)                      // decode / prefill lists
                 + round256((c + 1) * 8) + round256(8) + round256((size_t)(pl.nwin > 0 ? pl.nwin : 1) * 8);  // layout
  pl.buf_bytes = 0;
  if (pl.nwin > 0) {
    const kdn_scan_args s = slot_scan_args(a, pl.seq_bound);
    pl.buf_bytes = round256(scan_flat_buffer_bytes(&s, pl.win));
  }
  const size_t nbuf = pl.nwin >= 3 ? 3 : (size_t)pl.nwin;
  pl.total = pl.small_bytes + nbuf * pl.buf_bytes;
  return KDN_OK;
}

}  // namespace kdn

extern "C" size_t kdn_slot_step_workspace_bytes(const kdn_slot_step_args* a) {
  SlotPlan pl;
  if (slot_plan(a, pl) != KDN_OK) return 0;
  return pl.total;
}

extern "C" int kdn_slot_step(const kdn_slot_step_args* a, void* stream, void* aux_stream) {
  SlotPlan pl;
  int rc = slot_plan(a, pl);
  if (rc != KDN_OK) return rc;
  if (a->num_tokens == 0) return KDN_OK;
  if (!a->slot_mapping || !a->q || !a->k || !a->v || !a->beta || !a->omega_bf16 || !a->phase || !a->states || !a->y ||
      !a->workspace)
    return KDN_ERR_INVALID_ARGUMENT;
  if (!aligned(a->workspace, 256) || !aligned(a->omega_bf16, 16) || !aligned(a->slot_mapping, (size_t)a->slot_bytes))
    return KDN_ERR_MISALIGNED;
  if (a->workspace_bytes < pl.total) return KDN_ERR_WORKSPACE_TOO_SMALL;
  const hipStream_t st = as_stream(stream);
  const size_t c = (size_t)pl.cap;
  const RunGrid rg = run_grid(a->num_tokens);
  unsigned char* w = (unsigned char*)a->workspace;
  int64_t* rcnt = (int64_t*)w;      w += round256((size_t)rg.blocks * 8);
  int64_t* cu = (int64_t*)w;        w += round256((c + 1) * 8);
  int32_t* rslot = (int32_t*)w;     w += round256(c * 4);
  int64_t* dec_row = (int64_t*)w;   w += round256(c * 8);
  int64_t* pre_lo = (int64_t*)w;    w += round256(c * 8);
  int64_t* pre_hi = (int64_t*)w;    w += round256(c * 8);
  int32_t* dec_slot = (int32_t*)w;  w += round256(c * 4);
  int32_t* pre_slot = (int32_t*)w;  w += round256(c * 4);
  int64_t* fl_off = (int64_t*)w;    w += round256((c + 1) * 8);
  int64_t* fl_total = (int64_t*)w;  w += round256(8);
  int64_t* fl_first = (int64_t*)w;  w += round256((size_t)(pl.nwin > 0 ? pl.nwin : 1) * 8);
  hipLaunchKernelGGL(slot_count_kernel, dim3((unsigned)rg.blocks), dim3(RUN_THREADS), 0, st, a->slot_mapping,
                     a->slot_bytes, a->num_tokens, rg.span, rcnt);
  hipLaunchKernelGGL(slot_runs_kernel, dim3((unsigned)rg.blocks), dim3(RUN_THREADS), 0, st, a->slot_mapping,
                     a->slot_bytes, a->num_tokens, rg.span, rg.blocks, (const int64_t*)rcnt, pl.cap, cu, rslot, a->status);
  hipLaunchKernelGGL(ragged_split_kernel, dim3(1), dim3(1024), 0, st, (const int64_t*)cu, (const int32_t*)rslot,
                     pl.cap, a->num_slots, dec_row, dec_slot, pre_lo, pre_hi, pre_slot);
  rc = launch_status();
  if (rc != KDN_OK) return rc;
  // with an auxiliary stream the decode runs on it after the prefill's prep launches, as in
  // kdn_ragged_step
  const hipStream_t aux = aux_stream ? as_stream(aux_stream) : nullptr;
  const bool dec_aux = pl.nwin > 0 && aux && aux != st;
  EventSet evs;
  if (dec_aux) {
    rc = evs.create(2);
    if (rc != KDN_OK) return rc;
    if (hipEventRecord(evs.ev[0], st) != hipSuccess || hipStreamWaitEvent(aux, evs.ev[0], 0) != hipSuccess)
      return KDN_ERR_DEVICE;
  }
  // decode: one entry per possible run; entries the split did not fill have slot -1 and exit at once
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
  auto run_decode = [&](hipStream_t ds) -> int {
    if (a->in_dtype == KDN_DTYPE_BF16)
      return a->out_dtype == KDN_DTYPE_BF16 ? launch_decode<__bf16, __bf16>(dp, pl.cap, a->H, a->d_v, ds)
                                            : launch_decode<__bf16, float>(dp, pl.cap, a->H, a->d_v, ds);
    return a->out_dtype == KDN_DTYPE_BF16 ? launch_decode<float, __bf16>(dp, pl.cap, a->H, a->d_v, ds)
                                          : launch_decode<float, float>(dp, pl.cap, a->H, a->d_v, ds);
  };
  if (!dec_aux) {
    rc = run_decode(st);
    if (rc != KDN_OK) return rc;
  }
  if (pl.nwin == 0) return KDN_OK;
  // prefill: the packed layout, then the split scan over its windows
  hipLaunchKernelGGL(flat_plan_kernel, dim3(1), dim3(1024), 0, st, (const int64_t*)pre_lo, (const int64_t*)pre_hi,
                     pl.cap, pl.win, pl.nwin, fl_off, fl_first, fl_total);
  rc = launch_status();
  if (rc != KDN_OK) return rc;
  kdn_scan_args s = slot_scan_args(a, pl.seq_bound);
  s.state_slots = pre_slot;
  s.workspace = w;
  s.workspace_bytes = a->workspace_bytes - (size_t)(w - (unsigned char*)a->workspace);
  FlatPlan fp;
  fp.off = fl_off; fp.first = fl_first; fp.total = fl_total;
  fp.nseq = pl.cap; fp.win = pl.win; fp.nwin = pl.nwin;
  rc = scan_flat(&s, pre_lo, pre_hi, fp, stream, aux_stream);
  if (rc != KDN_OK) return rc;
  if (dec_aux) {
    rc = run_decode(aux);
    if (rc != KDN_OK) return rc;
    if (hipEventRecord(evs.ev[1], aux) != hipSuccess || hipStreamWaitEvent(st, evs.ev[1], 0) != hipSuccess)
      return KDN_ERR_DEVICE;
  }
  return KDN_OK;
}
