// Definitions shared by the prep kernel (kdn_prep.hip) and the state / output kernels and the launch
// code (kdn_scan.hip) of the D = 512 prefill scan: the per-chunk workspace record, the kernel parameter
// block and ragged-sequence addressing.
#pragma once
#include <type_traits>
#include "kdn_frag.hpp"
#include "kdn_internal.hpp"

namespace kdn {

constexpr int CH = 64;  // tokens per chunk (internal; the WY form is exact for any chunk length)

// Per (chunk, head) workspace record.  A segment of nseg chunks uses nseg + 1 records per head: the
// last one is scratch for the state kernel's writes past the final chunk.
template <class P, int D, int DV>
struct WsLayout {
  static constexpr size_t FB = P::frag_bytes;
  static constexpr int NJ = D / 32;   // 32-deep blocks over features
  static constexpr int NV = DV / 16;  // 16-wide value tiles
  static constexpr size_t phiK = 0;                                 // [m 4][j NJ][lane] K row frags (cos)
  static constexpr size_t Tp = phiK + (size_t)4 * NJ * 64 * FB;     // [m 4][jb 2][lane]  T diag(beta e^g s_k)
  static constexpr size_t Pm = Tp + (size_t)4 * 2 * 64 * FB;        // [m 4][jb 2][lane]  P
  static constexpr size_t U = Pm + (size_t)4 * 2 * 64 * FB;         // [m 4][n NV][lane] f32x4  U~
  static constexpr size_t VEC = U + (size_t)4 * NV * 64 * 16;       // qscale[64] kscale[64] gammaC
  static constexpr size_t Sfr = VEC + 1024;                         // [j NJ][n NV][lane] chunk-start S^T frags
  static constexpr size_t EB = FB / 2;                              // bytes of a lane's E tile (bf16x4 / f32x4)
  static constexpr size_t Eck = Sfr + (size_t)NJ * NV * 64 * FB;    // [m 4][n NV][lane] E tiles
  static constexpr size_t phiQ = Eck + (size_t)4 * NV * 64 * EB;    // [m 4][j NJ][lane] Q row frags (cos)
  static constexpr size_t bytes = (phiQ + (size_t)4 * NJ * 64 * FB + 255) / 256 * 256;
};

// bf16, D = 512: the K area of a record holds the chunk's lifted keys as the exact LDS image that the
// state kernel streams into its ring with global_load_lds (1 KB per instruction, copied verbatim): four
// slices of 16 KB, slice s for the state wave that owns features [128s, 128s + 128); inside a slice,
// plane h (8 KB) holds bytes [8h, 8h + 8) of each lane's 16-byte fragment slot at
// (fi * 64 + kimg_swizzle(lane)) * 8, fi = 4 m + jj for token tile m and the slice's 32-feature block jj.
// The state kernel reads a fragment back with one ds_read2st64_b64 and K^T from the same planes with
// ds_read_b64_tr_b16.  The swizzle (bits 2-3 of the 8-byte slot index XORed with bits 4-5) makes both
// conflict-free: a 16-lane group of the plain read covers slots 16k .. 16k + 15 and one of the
// transposed read slots {4g + q + 16r}; after the swizzle each group's 16 slots differ modulo 16, i.e.
// fall on distinct bank pairs.  Without it the transposed read conflicts two ways (measured with
// SQ_LDS_BANK_CONFLICT on a probe of both layouts: half its busy LDS cycles, none after the swizzle).
__device__ __forceinline__ constexpr int kimg_swizzle(int s) { return s ^ (((s >> 4) & 3) << 2); }
constexpr int KIMG_SLICE = 16384;
constexpr int KIMG_PLANE = 8192;
__device__ __forceinline__ void store_k_image(unsigned char* kimg, int m, int j, int lane, const bf16x8& f) {
  typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
  unsigned char* base = kimg + (size_t)(j >> 2) * KIMG_SLICE + (size_t)((m * 4 + (j & 3)) * 64 + kimg_swizzle(lane)) * 8;
  __builtin_nontemporal_store(__builtin_shufflevector(f, f, 0, 1, 2, 3), reinterpret_cast<bf16x4*>(base));
  __builtin_nontemporal_store(__builtin_shufflevector(f, f, 4, 5, 6, 7), reinterpret_cast<bf16x4*>(base + KIMG_PLANE));
}

// E tiles in the record, lane l holding rows 4(l>>4) .. +3 of column (l & 15) of tile `tile`: bf16 for
// bf16 inputs (the output kernel's product P E takes bf16 operands, so storing the rounded values
// changes no result and halves the bytes), fp32 otherwise.
template <class P>
__device__ __forceinline__ void store_e_tile(unsigned char* eck, size_t tile, int lane, const f32x4& e) {
  if constexpr (P::frag_bytes == 16) {
    typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
    const bf16x4 b = {(__bf16)e[0], (__bf16)e[1], (__bf16)e[2], (__bf16)e[3]};
    *reinterpret_cast<bf16x4*>(eck + (tile * 64 + lane) * 8) = b;
  } else {
    *reinterpret_cast<f32x4*>(eck + (tile * 64 + lane) * 16) = e;
  }
}
// The B fragment (32 token rows in kappa order, 16 columns) made of E tiles t0 (rows 0-15) and t1 (rows
// 16-31), read with streaming loads (the output kernel is the last reader).
template <class P>
__device__ __forceinline__ typename P::frag load_e_frag(const unsigned char* eck, size_t t0, size_t t1, int lane) {
  if constexpr (P::frag_bytes == 16) {
    typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
    const bf16x4 lo = __builtin_nontemporal_load(reinterpret_cast<const bf16x4*>(eck + (t0 * 64 + lane) * 8));
    const bf16x4 hi = __builtin_nontemporal_load(reinterpret_cast<const bf16x4*>(eck + (t1 * 64 + lane) * 8));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  } else {
    const f32x4 e0 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(eck + (t0 * 64 + lane) * 16));
    const f32x4 e1 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(eck + (t1 * 64 + lane) * 16));
    return P::from_f32(pair_to8(e0, e1));
  }
}

struct ScanParams {
  int64_t B, T, H;
  const void* q; int64_t qs0, qs1, qs2;
  const void* k; int64_t ks0, ks1, ks2;
  const void* v; int64_t vs0, vs1, vs2;
  const float* beta; int64_t bs0, bs1, bs2;
  const float* decay; int64_t ds0, ds1, ds2;
  const __bf16* omega; const float* phase;
  float inv_tau; int normalize;
  const float* state_in; int64_t is0, is1, is2, is3;
  float* state_out; int64_t os0, os1, os2, os3;
  void* y; int64_t ys0, ys1, ys2;
  unsigned char* ws;
  int64_t chunk0, nseg;  // first global chunk of the segment, chunks in the segment
  int prep_run;          // chunks per prep workgroup (bf16)
  int64_t out_wgs;       // output workgroups beside the state kernel (0: one per chunk and head)
  // feature map: per-head Omega (hi [+ lo]) / phases / 1/tau, renormalisation, pre-lifted inputs
  const __bf16* omega_lo; int64_t oms, phs;
  const float* inv_tau_head;
  int no_renorm, prelifted;
  int linear;  // update rule without the erasure term: T = I, Tp = 0
  // no output kernel reads the segment (the backward's checkpoint pass): prep lifts only the keys
  int prep_no_q;
  // the fused chain reads the segment (kdn_chain.hip): prep stores K as plain fragments (each lane's 16
  // bytes contiguous) instead of the state kernel's LDS image
  int k_plain;
  // the resident output kernel lifts q again (bf16, one shared exact Omega): prep stores no Q fragments
  int q_relift;
  // ragged batches: sequence b is token rows seq_lo[b] .. seq_hi[b] (stride 1 of each token tensor; for
  // cu_seqlens, seq_hi = cu_seqlens + 1); its state is slot slots[b] (stride 0 of the state tensors)
  const int64_t* seq_lo;
  const int64_t* seq_hi;
  const int* slots;
  // Packed windows (ragged batches sized on the device, the serving step from a slot map): sequence b's
  // chunks and one spare slot take the consecutive slots fl_off[b] .. fl_off[b+1]-1 of a packed slot
  // space (the spare last; a sequence without tokens takes none), *fl_total slots in all.  A call covers
  // the window of slots [fl_lo, fl_lo + nseg): its records are [head][slot - fl_lo], nseg + 1 per head
  // (the last is the spare of a sequence that the window's end cuts), chunk0 is 0 and B bounds the
  // sequences that meet one window.  fl_first[w] is the sequence holding slot w * nseg; fl_nseq the
  // entries of fl_off less one.  fl_off NULL: the layouts above.
  const int64_t* fl_off;
  const int64_t* fl_first;
  const int64_t* fl_total;
  int64_t fl_lo, fl_nseq;
};

// Slot x of the current packed window: its sequence, its chunk index in that sequence, and whether it
// holds one (a spare slot or a slot past the last holds none).
struct FlatChunk {
  int64_t b, c;
  bool ok;
};
__device__ __forceinline__ FlatChunk flat_chunk(const ScanParams& p, int64_t x) {
  FlatChunk r = {0, 0, false};
  const int64_t g = p.fl_lo + x;
  if (g >= *p.fl_total) return r;
  // the last sequence whose first slot is at or before g (fl_off is nondecreasing from 0)
  int64_t lo = p.fl_first[p.fl_lo / p.nseg], hi = p.fl_nseq;
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (p.fl_off[mid] <= g) lo = mid;
    else hi = mid;
  }
  r.b = lo;
  r.c = g - p.fl_off[lo];
  r.ok = r.c < p.fl_off[lo + 1] - p.fl_off[lo] - 1;
  return r;
}

// The real chunks of sequence fl_first[window] + i inside the current packed window: first slot (window-
// relative) and count (0: none).
__device__ __forceinline__ int64_t flat_run(const ScanParams& p, int64_t b, int64_t* first) {
  if (b >= p.fl_nseq) return 0;
  const int64_t a0 = p.fl_off[b], a1 = p.fl_off[b + 1] - 1;  // real chunks [a0, a1)
  const int64_t lo = a0 > p.fl_lo ? a0 : p.fl_lo;
  int64_t hi = a1 < p.fl_lo + p.nseg ? a1 : p.fl_lo + p.nseg;
  const int64_t tot = *p.fl_total;
  if (hi > tot) hi = tot;
  *first = lo - p.fl_lo;
  return hi > lo ? hi - lo : 0;
}

// Sequence b of the batch: element offsets of its first token in each token-indexed tensor, and its
// length.  A uniform batch addresses b * stride0 and has T tokens per sequence; a ragged batch
// addresses rows seq_lo[b] .. seq_hi[b] of one packed token dimension.
struct Seq {
  int64_t q, k, v, be, de, y, len;
};
__device__ __forceinline__ Seq seq_of(const ScanParams& p, int64_t b) {
  Seq s;
  if (p.seq_lo) {
    const int64_t r0 = p.seq_lo[b];
    s.q = r0 * p.qs1; s.k = r0 * p.ks1; s.v = r0 * p.vs1;
    s.be = r0 * p.bs1; s.de = r0 * p.ds1; s.y = r0 * p.ys1;
    s.len = p.seq_hi[b] - r0;
  } else {
    s.q = b * p.qs0; s.k = b * p.ks0; s.v = b * p.vs0;
    s.be = b * p.bs0; s.de = b * p.ds0; s.y = b * p.ys0;
    s.len = p.T;
  }
  return s;
}
// Chunks of the current segment that hold tokens of the sequence (0 once it has ended).
__device__ __forceinline__ int64_t seg_chunks(const ScanParams& p, const Seq& s) {
  const int64_t n = (s.len + CH - 1) / CH - p.chunk0;
  return n <= 0 ? 0 : (n < p.nseg ? n : p.nseg);
}

// The work of state workgroup row hb (b_local * H + h): sequence b and head h, the chunks it carries
// (nloc) and the byte offset of its first record in the segment's buffer; false: nothing to do (a
// sequence that ended in an earlier segment has its final state already; one without tokens gets its
// initial state copied through, with no chunk run).
// cfirst: the chunk index in the sequence of its first chunk here.
template <size_t BYTES>
__device__ __forceinline__ bool state_item(const ScanParams& p, int64_t hb, int64_t& b, int64_t& h, int64_t& nloc,
                                           size_t& off, int64_t& cfirst) {
  h = hb % p.H;
  if (p.fl_off) {
    b = p.fl_first[p.fl_lo / p.nseg] + hb / p.H;
    int64_t first = 0;
    nloc = flat_run(p, b, &first);
    off = (size_t)(h * (p.nseg + 1) + first) * BYTES;
    cfirst = nloc > 0 ? p.fl_lo + first - p.fl_off[b] : 0;
    return nloc > 0;
  }
  b = hb / p.H;
  const Seq sq = seq_of(p, b);
  nloc = seg_chunks(p, sq);
  off = (size_t)hb * (p.nseg + 1) * BYTES;
  cfirst = p.chunk0;
  return !(nloc == 0 && !(sq.len <= 0 && p.chunk0 == 0));
}

// Feature modes of the prep kernel: Omega exact in bf16 (the structured projection), Omega as hi + lo
// bf16 parts (general projections), or q / k already lifted (d_k = D).
enum FeatureMode { FM_EXACT = 0, FM_HILO = 1, FM_PRELIFTED = 2 };

template <class P>
struct IsBF16 : std::integral_constant<bool, std::is_same<P, PrecBF16>::value> {};

// Launches the prep kernel of one segment (kdn_prep.hip; compiled on its own so that its MFMA results
// can be kept in VGPRs: it post-processes nearly all of them on the VALU).
template <class P, typename InT, int D, int DV>
int launch_prep(const ScanParams& p, hipStream_t st);

// The fused chain (kdn_chain.hip, bf16 inputs, D = 512): the state update and the readout of one segment
// in one sequential kernel.  16 * min(2, d_v / 16) value columns per workgroup, the workgroups of a head
// on one XCD (ids xcd + 8 (rank * per_head + part)).
inline unsigned chain_grid(int64_t B, int64_t H, int dv) {
  const int nwg = dv / (dv >= 32 ? 32 : 16);
  return (unsigned)(8 * ((B * H + 7) / 8) * nwg);
}
template <typename OutT, int DV>
int launch_chain(const ScanParams& p, hipStream_t st);

}  // namespace kdn
