// Internal helpers shared by the C-ABI entry points (status codes, dtype tags, launch checks).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include "../../include/kdn.h"

namespace kdn {

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? KDN_OK : KDN_ERR_DEVICE;
}

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline bool valid_dtype(int dt) { return dt == KDN_DTYPE_F32 || dt == KDN_DTYPE_BF16; }

inline size_t dtype_size(int dt) { return dt == KDN_DTYPE_F32 ? 4 : 2; }

// Compute units of the current device (0 if it cannot be queried).
inline int device_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return n;
}

constexpr size_t CU_LDS_BYTES = 160 * 1024;  // LDS per CU on gfx950

// The pipelined scan of kdn_delta_scan_fwd_pipelined / _streams (out_stream NULL: output kernels on
// aux_stream), with ragged sequences optionally given as device start / end arrays (sequence b = token
// rows seq_lo[b] .. seq_hi[b]-1) instead of cu_seqlens.
int scan_pipelined(const kdn_scan_args* a, const int64_t* seq_lo, const int64_t* seq_hi, void* stream,
                   void* aux_stream, void* out_stream);
size_t scan_workspace_bytes_pipelined(const kdn_scan_args* a);

// Packed windows of a ragged prefill whose layout is planned on the device (the serving step from a slot
// map, kdn_serve.hip): `off` (nseq + 1 slot offsets), `first` (per window) and `total` as ScanParams
// describes them; windows of `win` slots, `nwin` of them (a bound: windows past *total do nothing).
struct FlatPlan {
  const int64_t* off;
  const int64_t* first;
  const int64_t* total;
  int64_t nseq, win, nwin;
};
// The split schedule over packed windows: a->B bounds the sequences that meet one window and a->T the
// longest; sequence b is token rows seq_lo[b] .. seq_hi[b]-1 with state slot a->state_slots[b], read and
// written in place (a->initial_state is a->final_state).  The workspace holds one to three window buffers
// of scan_flat_buffer_bytes each (pipelined over aux_stream when two or more fit).
int scan_flat(const kdn_scan_args* a, const int64_t* seq_lo, const int64_t* seq_hi, const FlatPlan& fp, void* stream,
              void* aux_stream);
size_t scan_flat_buffer_bytes(const kdn_scan_args* a, int64_t win);

// Segment checkpoints of the D = 512, d_v = 64 scan (the backward's first pass): the states at the starts
// of segments 1 .. n of `seg` chunks each, written as fp32 [B][H][512][64] arrays one after another from
// `ckpt` (segment s's at ckpt + (s - 1) * B*H*512*64), by the scan's prep and state kernels alone (no
// output kernel); segment 0 starts from a->initial_state (zeros if NULL).  Each equals, bit for bit, the
// state that kdn_delta_scan_fwd with segment_chunks = seg carries across that boundary.  `ws` holds `nbuf`
// buffers of `buf_bytes` >= scan_checkpoint_buffer_bytes(a, seg); with aux (not st) and two buffers, prep
// of segment s + 1 runs on aux beside the state kernel of segment s.  The last launch is on st.
size_t scan_checkpoint_buffer_bytes(const kdn_scan_args* a, int64_t seg);
int scan_checkpoints(const kdn_scan_args* a, int64_t seg, int64_t n, float* ckpt, void* ws, size_t buf_bytes,
                     int nbuf, hipStream_t st, hipStream_t aux);

// The general-D scan (kdn_general.hip): D = 1024 over pre-lifted features, d_v 64 or 128, the delta rule,
// uniform batches.  general_scan_applies selects it; the other functions assume it applies and that the
// common argument checks have passed.
bool general_scan_applies(const kdn_scan_args* a);
int general_scan_validate(const kdn_scan_args* a);
size_t general_scan_workspace_bytes(const kdn_scan_args* a);
int general_scan(const kdn_scan_args* a, void* stream);
// Its backward (kdn_delta_scan_bwd for D = 1024 over pre-lifted features: dq, dk are dL/dphi_q, dL/dphi_k):
// one workspace record per (batch, head, chunk) for the whole sequence, one launch sequence on one stream.
bool general_bwd_applies(const kdn_scan_args* f);
size_t general_bwd_workspace_bytes(const kdn_scan_bwd_args* a);
int64_t general_bwd_segments(const kdn_scan_bwd_args* a, int64_t* segment_chunks);
int general_bwd(const kdn_scan_bwd_args* a, void* stream);
// Device address of the current device's copy of kdn_delta_scan_fwd_noalloc's scratch array (kdn_noalloc.hip).
int noalloc_scratch_address(void** out);

// D = 128 and 256 lifts on the D = 512 kernels by feature replication (kdn_frep.hip).  Workspace of such a
// request: [0, base) the 512-wide request's own workspace, then the replicated Omega (and low parts) and
// phases, then up to three 512-wide fp32 states [B][H][512][d_v] (offsets from the workspace start).
bool frep_applies(const kdn_scan_args* a);
struct FrepLayout {
  size_t base, omega, omega_lo, phase, state[3], total;
};
FrepLayout frep_layout(const kdn_scan_args* a, size_t base, int nstates);
size_t frep_state_bytes(const kdn_scan_args* a);
// *a at D = 512: per-head strides of the replicated tables; with L and ws, tables and workspace in ws
// (workspace_bytes = L->base); the state pointers are left as in *a
kdn_scan_args frep_wide(const kdn_scan_args* a, const FrepLayout* L, void* ws);
void frep_contiguous_strides(const kdn_scan_args* a, int64_t s[4]);
int frep_tables(const kdn_scan_args* a, const FrepLayout* L, void* ws, hipStream_t st);
// L(S) = S J^T into a contiguous 512-wide state, and P(S') = S' J from one (s4: the D-wide state's strides)
int frep_state_lift(const kdn_scan_args* a, const float* s, const int64_t* s4, float* dst, hipStream_t st);
int frep_state_fold(const kdn_scan_args* a, const float* src, float* s, const int64_t* s4, hipStream_t st);

// Events of a multi-stream launch sequence, released when the call returns (destroying an event whose
// record is still pending is allowed; its resources are freed once it completes).  They only order
// kernels of one device against each other (hipStreamWaitEvent; the host never waits on them), so they
// carry no system-scope fence: the kernels' own end-of-kernel release makes their writes visible to the
// device's later kernels, and the caller's synchronisation makes the results visible to the host.
// Without the fence every record wrote back the caches at each segment boundary: config 3's layer
// 2.09 -> 2.05 ms.
struct EventSet {
  hipEvent_t ev[16];
  int n = 0;
  int create(int count) {
    if (count > 16) return KDN_ERR_INVALID_ARGUMENT;
    for (; n < count; ++n)
      if (hipEventCreateWithFlags(&ev[n], hipEventDisableTiming | hipEventDisableSystemFence) != hipSuccess)
        return KDN_ERR_DEVICE;
    return KDN_OK;
  }
  ~EventSet() {
    for (int i = 0; i < n; ++i) (void)hipEventDestroy(ev[i]);
  }
};

}  // namespace kdn
