/* kdn.h -- C ABI of the MI355X (gfx950) Kernel-DeltaNet prefill path.
 *
 * The path: spherical-normalise + structured-FWHT feature lift (d_k = 64 -> D = 512), then the exact
 * chunked gated delta-rule scan  y_t = S_{t-1} phi(q_t),
 *                                S_t = lambda_t S_{t-1} (I - beta_t phi(k_t) phi(k_t)^T) + beta_t v_t phi(k_t)^T.
 *
 * Conventions (every entry point):
 *   - All tensor pointers are device pointers; the caller allocates every buffer (inputs, outputs,
 *     workspace).  The library allocates no device memory at run time.  The one exception is
 *     kdn_delta_scan_fwd_noalloc's fixed scratch array (KDN_NOALLOC_SCRATCH_BYTES per GPU), a device
 *     global of its own code object that is reserved on a GPU from the first call of that entry point
 *     there until the process ends.
 *   - Work is enqueued on `stream` (a hipStream_t passed as void*; NULL = the null stream) and is
 *     stream-ordered; entry points return without synchronising.
 *   - Return 0 (KDN_OK) or a negative kdn_status.  No exception or abort crosses the ABI.  Argument
 *     errors are detected on the host before anything is enqueued.
 *   - Reentrant and safe to call from several host threads.  The only process-wide state is the
 *     per-device address of the noalloc scratch array (looked up once per device, under a lock) and
 *     the state pool handles (single-threaded each).
 *   - Strides are in elements; the innermost (feature) dimension of every tensor must be contiguous.
 *
 * Reference interfaces replaced (paths relative to jatin-yadav-acad/kernel-deltanet):
 *   kdn_build_omega     <- FastWalshHadamardProjection.__init__ Omega build, kernels/fwht.py:94-111
 *   kdn_fwht            <- fast_walsh_hadamard_transform, kernels/fwht.py:25-45
 *   kdn_fwht_lift_bits  <- pybind fwht_forward(input, rademacher_bits, D_lifted, tau_star_inv),
 *                          kernels/fwht_cuda.cpp:29-32, with the semantics of the torch branch of
 *                          FastWalshHadamardProjection.forward, kernels/fwht.py:122-131
 *   kdn_fwht_lift       <- the same forward with Omega passed as its bf16 table (kernels/fwht.py:122-131)
 *   kdn_delta_scan_fwd  <- fused_chunked_deltanet_forward, kernels/fused_kernel_deltanet.py:31-155
 *   kdn_scan_prep       <- the S-independent part of its chunk loop, kernels/fused_kernel_deltanet.py:95-122
 *   kdn_scan_state      <- the state carry, kernels/fused_kernel_deltanet.py:128-129,144-149
 *   kdn_scan_output     <- the chunk readout, kernels/fused_kernel_deltanet.py:118-141
 *   kdn_scan_prep_fused, kdn_scan_chain <- the same chunk loop as prep + one sequential kernel that carries
 *                          the state and reads out y (kernels/fused_kernel_deltanet.py:95-149)
 *   kdn_slot_step       <- vllm_hybrid_recurrent_forward(query, ..., recurrent_states, slot_mapping, output),
 *                          serving/vllm_kernel_deltanet_op.cpp:11-34 (declared there with an empty body)
 *
 * ABI 2.0 (breaking): kdn_scan_bwd_args and kdn_ragged_args gained trailing fields that the library reads
 * on every call (dinv_tau, num_slots) and kdn_scan_bwd_phase gained its `segment` argument in 1.6-1.8;
 * callers built against a header older than 1.8 must be recompiled.  2.0 adds kdn_scan_schedule,
 * kdn_scan_prep_fused and kdn_scan_chain.  2.1 accepts D = 128 and 256 (scan and backward) and d_v 16,
 * 32 and 128 in the D = 512 backward.  2.2 adds kdn_slot_step (the serving step from a slot map).
 */
#ifndef KDN_H
#define KDN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum kdn_status {
  KDN_OK = 0,
  KDN_ERR_INVALID_ARGUMENT = -1,  /* null pointer, non-positive size, bad stride, bad dtype tag */
  KDN_ERR_UNSUPPORTED = -2,       /* valid request outside what the kernels implement (d_k, D, d_v) */
  KDN_ERR_WORKSPACE_TOO_SMALL = -3,
  KDN_ERR_MISALIGNED = -4,        /* a pointer or row stride breaks the 16-byte vector-access rule */
  KDN_ERR_DEVICE = -5,            /* a HIP launch reported an error */
  KDN_ERR_CAPACITY = -6           /* the state pool has no free slot */
} kdn_status;

typedef enum kdn_dtype {
  KDN_DTYPE_F32 = 0,
  KDN_DTYPE_BF16 = 1
} kdn_dtype;

/* Human-readable text for a kdn_status value (static storage, never NULL). */
const char* kdn_strerror(int status);

/* ABI version: (major << 16) | minor. */
int kdn_abi_version(void);

/* Build the explicit structured projection Omega[D][d_k] = concat_m (H D3_m H D2_m H D1_m) / sqrt(d_k)
 * from the packed Rademacher table sign_bits[M][3] (M = D / d_k; column s = stage d1,d2,d3; bit i set
 * <=> entry i is -1), with H the natural-order (Sylvester) Hadamard matrix.  Computed with wave64
 * butterflies; every entry is an integer / 8 for d_k = 64 and is stored exactly in either dtype.
 * Replaces kernels/fwht.py:94-111 (and the bit table of :74-83 is its input).
 * d_k must be 64; D a multiple of 64 up to 1024. */
int kdn_build_omega(const int64_t* sign_bits, int d_k, int D, void* omega, int omega_dtype, void* stream);

/* Unnormalised natural-order Walsh-Hadamard transform of each row (length n, a power of two <= 64).
 * out may alias x.  Replaces fast_walsh_hadamard_transform, kernels/fwht.py:25-45. */
int kdn_fwht(const void* x, int64_t rows, int64_t x_row_stride, int n, int dtype,
             void* out, int64_t out_row_stride, void* stream);

/* Feature lift of `rows` vectors x[r][0:d_k] -> out[r][0:D]:
 *   xh  = normalize_input ? x / max(||x||_2, 1e-6) (rounded to x's dtype) : x
 *   phi = sqrt(2/D) cos(xh Omega^T * inv_tau + phase),   out = phi / (||phi||_2 + 1e-8)
 * omega is the bf16 [D][d_k] table from kdn_build_omega (exact in bf16); phase is fp32 [D].
 * Products are exact (bf16 operands; fp32 inputs are split into three bf16 parts), sums in fp32.
 * The torch branch of FastWalshHadamardProjection.forward, kernels/fwht.py:122-131, with Omega given as
 * its bf16 table (the scan and callers that keep Omega resident); kdn_fwht_lift_bits below is the same
 * lift at the reference's native boundary, kernels/fwht_cuda.cpp:29-32.
 * d_k must be 64; D in {128, 256, 512}.  x, out, omega and phase 16-byte aligned; row strides in bytes
 * multiples of 16. */
int kdn_fwht_lift(const void* x, int64_t rows, int64_t x_row_stride, int x_dtype, int normalize_input,
                  const void* omega_bf16, const float* phase, int d_k, int D, float inv_tau,
                  void* out, int64_t out_row_stride, int out_dtype, void* stream);

/* The same lift at the reference's native boundary (ABI 1.5): pybind fwht_forward(input, rademacher_bits,
 * D_lifted, tau_star_inv) of kernels/fwht_cuda.cpp:11-32 takes the packed sign table, not Omega.  Here
 * rademacher_bits is that table, device int64 [D_lifted / 64][3] (column s = stage d1, d2, d3; bit i set
 * <=> entry i is -1; the module buffer of kernels/fwht.py:74-83); every workgroup builds Omega from it in
 * LDS with wave64 butterflies (the sign flips fused into the transform), then lifts as kdn_fwht_lift.
 * The torch-branch semantics this lift implements (kernels/fwht.py:122-131) also need the module's phases
 * b, passed as `phase` (device fp32 [D_lifted]); the reference's CUDA function has no phase argument.
 * normalize_input as kdn_fwht_lift (0 in the reference's call).  d_k must be 64; D_lifted in
 * {128, 256, 512}; x, out and phase 16-byte aligned, rademacher_bits 8-byte aligned; row strides in bytes
 * multiples of 16. */
int kdn_fwht_lift_bits(const void* x, int64_t rows, int64_t x_row_stride, int x_dtype, int d_k,
                       const int64_t* rademacher_bits, int D_lifted, float tau_star_inv, const float* phase,
                       int normalize_input, void* out, int64_t out_row_stride, int out_dtype, void* stream);

/* kdn_fwht_lift_bits with the projection by in-register wave64 butterflies (ABI 1.6): the design of the
 * reference's CUDA lift, kernels/in_register_fwht.cu:10-93 (one wave per row, the sign flips and three
 * Walsh-Hadamard transforms per 64-feature block, no Omega table), with the semantics of
 * kernels/fwht.py:122-131.  Same arguments, checks and results up to fp32 summation order; kept as the
 * measured alternative to the MFMA projection of kdn_fwht_lift_bits, which is faster on gfx950. */
int kdn_fwht_lift_bits_butterfly(const void* x, int64_t rows, int64_t x_row_stride, int x_dtype, int d_k,
                                 const int64_t* rademacher_bits, int D_lifted, float tau_star_inv,
                                 const float* phase, int normalize_input, void* out, int64_t out_row_stride,
                                 int out_dtype, void* stream);

/* Factored lift for d_k = 128 -> D = 1024 (ABI 1.4): out[r][0:512] = lift(x[r][0:64]; omega1, phase1),
 * out[r][512:1024] = lift(x[r][64:128]; omega2, phase2) (each as kdn_fwht_lift without input
 * normalisation, the two projections of seeds s and s + 1000), then out[r] <- out[r] / (||out[r]|| + 1e-7).
 * Replaces FactoredFastWalshHadamardProjection.forward, kernels/factored_kernel_deltanet.py:42-74.
 * Alignment as kdn_fwht_lift; x_row_stride >= 128, out_row_stride >= 1024. */
int kdn_fwht_lift_factored(const void* x, int64_t rows, int64_t x_row_stride, int x_dtype,
                           const void* omega1_bf16, const float* phase1, const void* omega2_bf16,
                           const float* phase2, float inv_tau, void* out, int64_t out_row_stride, int out_dtype,
                           void* stream);

/* Backward of kdn_fwht_lift_factored (ABI 1.8): dx[r] = (d out[r] / d x[r])^T dout[r] for the same x, Omega
 * and phase arguments, with dout fp32 rows of 1024 (dout_row_stride) and dx fp32 rows of 128
 * (dx_row_stride).  The lift is recomputed in fp32 from x (the forward's bf16 rounding of its output is
 * not differentiated).  Replaces autograd through FactoredFastWalshHadamardProjection.forward,
 * kernels/factored_kernel_deltanet.py:60-74.  Omega 8-byte aligned; phases, dout and dx 16-byte aligned
 * with row strides that are multiples of 4; x element-aligned. */
int kdn_fwht_lift_factored_bwd(const void* x, int64_t rows, int64_t x_row_stride, int x_dtype,
                               const void* omega1_bf16, const float* phase1, const void* omega2_bf16,
                               const float* phase2, float inv_tau, const float* dout, int64_t dout_row_stride,
                               float* dx, int64_t dx_row_stride, void* stream);

/* Arguments of the chunked delta-rule prefill scan.  Tensors are addressed as
 *   q[b][t][h][0:d_k], k[b][t][h][0:d_k], v[b][t][h][0:d_v], beta[b][t][h], decay[b][t][h],
 *   y[b][t][h][0:d_v], state[b][h][0:D][0:d_v]   (state element (d, j) = S[j][d] of the recurrence)
 * through the given element strides, so (B*H, T, d), (B, T, H, d) and (B, H, T, d) layouts all work
 * without copies (fold heads into batch with H = 1).  The reference state layout (B, d_v, D) is
 * state stride {d_v*D, 0, 1, D}. */
typedef struct kdn_scan_args {
  int64_t B, T, H;
  int d_k, D, d_v;             /* d_k = 64, D = 512, d_v 16, 32, 64 or 128; or (ABI 2.1) D = 128 or 256, run
                                * on the D = 512 kernels with Omega and the phases replicated 512 / D times
                                * (exact: the replicated features have the D-wide inner products; the state
                                * is folded back to D columns), uniform batches, full-scan entry points only;
                                * or (ABI 1.4) pre-lifted features with d_k = D = 1024, d_v 64 or 128, the
                                * delta rule, uniform batches (the factored d_k = 128 path; full-scan entry
                                * points only) */
  int in_dtype;                /* dtype of q, k, v */
  int out_dtype;               /* dtype of y */
  int normalize_input;         /* L2-normalise q, k rows (F.normalize, eps 1e-6) before the lift */
  float inv_tau;               /* 1 / tau*, tau* = d_k^(1/4) in the reference */
  const void* q;   int64_t q_stride[3];
  const void* k;   int64_t k_stride[3];
  const void* v;   int64_t v_stride[3];
  const float* beta;  int64_t beta_stride[3];
  const float* decay; int64_t decay_stride[3];   /* NULL means lambda = 1 */
  const void* omega_bf16;      /* [D][d_k] from kdn_build_omega */
  const float* phase;          /* [D] */
  const float* initial_state; int64_t init_stride[4];   /* NULL means S_0 = 0 */
  float* final_state;         int64_t final_stride[4];  /* required; may alias initial_state */
  void* y;         int64_t y_stride[3];
  void* workspace; size_t workspace_bytes;
  int64_t segment_chunks;      /* 64-token chunks per segment; 0 lets the library choose */
  /* Feature map (ABI 1.1).  All-zero values select the structured-FWHT lift above (kernels/fwht.py):
   *   phi = cos(xh Omega_h^T inv_tau_h + phase_h) * sqrt(2/D), divided by (||.|| + 1e-8) unless
   *   no_renorm is set.  General projections (kernels/kernel_deltanet_fused.py:238-251 and
   *   core/rkhs_features.py:107-131 of the reference) pass Omega as hi + lo bf16 parts. */
  const void* omega_lo;        /* bf16 [D][d_k] low part of Omega (Omega = hi + lo); NULL when hi is exact */
  int64_t omega_head_stride;   /* elements between heads' Omega (hi and lo); 0 = one Omega for all heads */
  int64_t phase_head_stride;   /* elements between heads' phases; 0 = shared */
  const float* inv_tau_head;   /* [H] per-head 1/tau; NULL = inv_tau for every head */
  int no_renorm;               /* 1: phi = sqrt(2/D) cos(.), no division by its norm */
  int feature_mode;            /* 0: lift q, k (d_k -> D); 1: q and k are already lifted features (d_k = D) */
  /* Update rule.  0: the gated delta rule above.  1: gated linear attention without the erasure term,
   *   S_t = lambda_t S_{t-1} + beta_t v_t phi(k_t)^T, readout y_t = S_{t-1} phi(q_t) as before
   *   (the recurrence of core/chunked_scan.py:145-186, with beta = eta and lambda per head). */
  int rule;
  /* Ragged batches (ABI 1.2).  With cu_seqlens (device int64 [B+1]) sequence b is the token rows
   * cu_seqlens[b] .. cu_seqlens[b+1]-1 of a packed token dimension: q, k, v, beta, decay and y are
   * addressed with stride[1] only (stride[0] is ignored) and T must be at least the longest sequence.
   * A sequence without tokens gets final = initial state.  With state_slots (device int32 [B])
   * sequence b reads and writes state slot state_slots[b] (stride[0] of the state tensors); slots must
   * be distinct.  NULL keeps the uniform layout above. */
  const int64_t* cu_seqlens;
  const int32_t* state_slots;
} kdn_scan_args;

/* Workspace bytes kdn_delta_scan_fwd needs for these arguments (0 if the arguments are invalid).
 * Only the shape, dtype and segment_chunks fields are read, and at D = 128 or 256 also omega_lo (NULL or
 * not), omega_head_stride and phase_head_stride (zero or not), which size the replicated tables. */
size_t kdn_scan_workspace_bytes(const kdn_scan_args* a);

/* The exact chunked gated delta rule with readout before update (see top of file), carried in fp32,
 * continuing from initial_state and writing the state after the last token to final_state.  Tokens
 * past T inside the last chunk are treated as beta = 0, lambda = 1 (exact no-ops), as the reference
 * pads them (kernels/fused_kernel_deltanet.py:55-62).  log(lambda) is clamped to [log 1e-5, 0]
 * (kernels/fused_kernel_deltanet.py:74).  Replaces kernels/fused_kernel_deltanet.py:31-155. */
int kdn_delta_scan_fwd(const kdn_scan_args* a, void* stream);

/* The three phases kdn_delta_scan_fwd runs per segment, for callers that schedule them themselves
 * (per-phase timing, overlapping phases of different segments on several streams).  Each acts on
 * chunks [chunk0, chunk0 + nchunks) (64 tokens each) using workspace slots 0 .. nchunks-1, so
 * a->workspace_bytes must be at least kdn_scan_workspace_bytes() of the same arguments with
 * segment_chunks = nchunks (segment_chunks itself is ignored).  On a given slot they must run in the
 * order prep, state, output (stream order or events).
 *   kdn_scan_prep   : lift of q and k, Gram matrices, triangular inverse and every state-independent
 *                     factor of each chunk, written to the slot.  Replaces
 *                     kernels/fused_kernel_deltanet.py:95-122.
 *   kdn_scan_state  : the sequential carry: reads the prepared chunks in order, checkpoints each
 *                     chunk's starting state and its error terms E into the slot, reads initial_state
 *                     when chunk0 == 0 (zeros if NULL) and final_state otherwise, writes final_state.
 *                     Replaces kernels/fused_kernel_deltanet.py:128-129,144-149.
 *   kdn_scan_output : y of each chunk from its slot.  Replaces kernels/fused_kernel_deltanet.py:118-141.
 * These are the split schedule's phases; kdn_scan_schedule says which schedule the whole-scan entry
 * points run, and kdn_scan_prep_fused / kdn_scan_chain below are the fused schedule's. */
/* kdn_delta_scan_fwd scheduled over two streams.  The sequence is cut into segments of
 * a->segment_chunks chunks (0 = 64).  The segments rotate through as many workspace buffers of
 * kdn_scan_workspace_bytes() (for that segment size) as a->workspace_bytes holds, up to three.
 *   - The sequential state kernel of segment s runs on `stream`.
 *   - The prep of segment s+1 and the output of segment s-1 run on `aux_stream`, concurrently, on
 *     the CUs the state kernel leaves free.
 * aux_stream first waits for the work already queued on `stream`; `stream` finally waits for
 * aux_stream.  To the caller this is one stream-ordered operation on `stream`, with the same results
 * as kdn_delta_scan_fwd, bit for bit.  With fewer than two buffers, a single segment, or a NULL
 * aux_stream (or aux_stream == stream) it runs serially on `stream`.  Both streams should have default
 * priority.  Replaces kernels/fused_kernel_deltanet.py:31-155, like kdn_delta_scan_fwd. */
int kdn_delta_scan_fwd_pipelined(const kdn_scan_args* a, void* stream, void* aux_stream);

/* Workspace bytes for three segment buffers of kdn_delta_scan_fwd_pipelined (fewer when the sequence
 * has fewer segments); 0 if the arguments are invalid. */
size_t kdn_scan_workspace_bytes_pipelined(const kdn_scan_args* a);

/* kdn_delta_scan_fwd_pipelined with the prep kernels on prep_stream and the output kernels on their own
 * output_stream (three streams), so that neither waits behind the other; same workspace and results.
 * output_stream NULL (or equal to another stream) falls back to kdn_delta_scan_fwd_pipelined. */
int kdn_delta_scan_fwd_streams(const kdn_scan_args* a, void* stream, void* prep_stream, void* output_stream);

/* kdn_delta_scan_fwd without a caller workspace (ABI 1.5).  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The workspace of one segment of chunks lives in a fixed device array
 * of KDN_NOALLOC_SCRATCH_BYTES that the library holds on each GPU it runs on until the process ends; the
 * call allocates nothing.  a->workspace and a->workspace_bytes are ignored; segments are as long as the
 * array allows (at most a->segment_chunks when that is positive), so the results equal
 * kdn_delta_scan_fwd's bit for bit.  A request whose heads need more than the array for one chunk
 * (B * H * 2 records, 238,592 bytes each at D = 512, d_v = 64, bf16: up to B * H = 562) returns
 * KDN_ERR_WORKSPACE_TOO_SMALL; the pre-lifted D = 1024 path returns KDN_ERR_UNSUPPORTED.  All calls on one
 * GPU share its array: calls that overlap in time on one GPU (two streams, two host threads) race and must
 * be serialised by the caller. */
#define KDN_NOALLOC_SCRATCH_BYTES ((size_t)256 << 20)
int kdn_delta_scan_fwd_noalloc(const kdn_scan_args* a, void* stream);

int kdn_scan_prep(const kdn_scan_args* a, int64_t chunk0, int64_t nchunks, void* stream);
int kdn_scan_state(const kdn_scan_args* a, int64_t chunk0, int64_t nchunks, void* stream);
int kdn_scan_output(const kdn_scan_args* a, int64_t chunk0, int64_t nchunks, void* stream);

/* The schedule that kdn_delta_scan_fwd, _pipelined, _streams and _noalloc run for these arguments on the
 * current device (ABI 2.0), or a negative kdn_status for invalid arguments:
 *   KDN_SCHEDULE_SPLIT   per segment the prep, state and output kernels above: the state kernel carries only
 *                        the state and checkpoints it per chunk, the output kernel reads y out;
 *   KDN_SCHEDULE_FUSED   per segment the prep kernel and the fused chain, which carries the state and writes y
 *                        itself (no checkpoints, no output kernel).  bf16 inputs at D = 512, chosen when the
 *                        split schedule's state workgroups (B * H * d_v / 16, heads rounded up to 8) fill the
 *                        GPU: a few heads are a latency-bound sequence whose shortest step is the split
 *                        state kernel's, many heads are throughput-bound and the fused chain does less work;
 *   KDN_SCHEDULE_GENERAL the pre-lifted D = 1024 scan.
 * The environment variable KDN_SCAN_SCHEDULE=split or =fused, read at every call, overrides the choice
 * between the first two.  Both give the same final state bit for bit; y differs by the order of one fp32
 * sum (Q S^T over four feature quarters). */
#define KDN_SCHEDULE_SPLIT 0
#define KDN_SCHEDULE_FUSED 1
#define KDN_SCHEDULE_GENERAL 2
int kdn_scan_schedule(const kdn_scan_args* a);

/* The fused schedule's two phases (ABI 2.0), used like kdn_scan_prep / kdn_scan_state: on chunks
 * [chunk0, chunk0 + nchunks) with workspace slots 0 .. nchunks-1, in the order prep, chain.
 *   kdn_scan_prep_fused : kdn_scan_prep writing the chain's slot layout (the lifted keys as plain MFMA
 *                         fragments and the lifted queries stored).
 *   kdn_scan_chain      : the sequential carry as kdn_scan_state (initial_state when chunk0 == 0, zeros if
 *                         NULL, final_state otherwise; writes final_state) that also writes y of each chunk.
 * bf16 inputs at D = 512 only (KDN_ERR_UNSUPPORTED otherwise).  Replace kernels/fused_kernel_deltanet.py:95-149. */
int kdn_scan_prep_fused(const kdn_scan_args* a, int64_t chunk0, int64_t nchunks, void* stream);
/* The segment length (chunks) that kdn_delta_scan_fwd (pipelined = 0) or the pipelined entry points
 * (pipelined != 0) use for these arguments on the current device: a->segment_chunks when positive, else the
 * default, at most the sequence's chunks.  0 for invalid arguments or the D = 1024 scan (ABI 2.0). */
int64_t kdn_scan_segment_chunks(const kdn_scan_args* a, int pipelined);
int kdn_scan_chain(const kdn_scan_args* a, int64_t chunk0, int64_t nchunks, void* stream);

/* ---- Backward of the scan (ABI 1.3; segmented and deterministic since ABI 1.6) ----------------------
 * Gradients of a loss L through kdn_delta_scan_fwd, given dL/dy and optionally dL/d(final state).
 * Replaces the autograd recompute of FusedKernelDeltaNetFunction.backward,
 * kernels/fused_kernel_deltanet.py:168-179.  `fwd` holds the forward's arguments (shapes, q, k, v, beta,
 * decay, omega_bf16, phase, inv_tau, normalize_input, initial_state, segment_chunks; its y, final_state
 * and workspace are ignored).  Supported: d_k = 64, D = 512, d_v = 64, the delta rule (rule 0) or the
 * linear rule (rule 1), the lifted features of feature mode 0 with every feature-map field (one shared or
 * per-head Omega, with or without low parts, shared or per-head phases and 1/tau, with or without
 * renormalisation; ABI 1.7, before which only one shared structured Omega), uniform batches (no
 * cu_seqlens / state_slots); and (ABI 1.8) D = 1024 over pre-lifted features (feature mode 1, d_k = D,
 * d_v 64 or 128, the delta rule: the scan of the factored d_k = 128 path, whose reference trains through
 * autograd of kernels/factored_kernel_deltanet.py:77-183), where dq and dk are dL/dphi_q and dL/dphi_k.
 * Other requests return KDN_ERR_UNSUPPORTED.  dy and
 * d_final_state are fp32; every gradient is written in fp32 with the layout of its input: dq, dk
 * (B, T, H, d_k), dv (B, T, H, d_v), dbeta, ddecay (B, T, H), d_initial_state (B, H, D, d_v).
 * d_final_state NULL means dL/dS_T = 0; ddecay (allowed only with decay) and d_initial_state may be
 * NULL.  The gradient of lambda is zero where the forward's clamp to [1e-5, 1] is active.
 *
 * The backward runs in segments of fwd->segment_chunks 64-token chunks (0: the largest power of two
 * from 4 to 256 whose per-chunk records fit 4.5 GiB), last segment first: a checkpoint pass of the
 * forward scan's prep and state kernels stores the state at each segment start, then each segment
 * recomputes its chunks, carries the state forward from its checkpoint and dL/dS backward from the
 * next segment, and writes its gradients.  The workspace (256-byte aligned) holds up to three segments'
 * records (1,099,776 bytes per (batch, head, chunk)), one fp32 [B][H][512][64] state per segment
 * boundary plus one more, up to two buffers of the forward scan's records and a 64 KB table of Omega^T
 * fragments (one per head with per-head Omega, twice that with low parts; with dinv_tau, 4 bytes per
 * (batch, head, chunk) more): it grows
 * with the segment, not with T, apart from the 128 KB per head per segment boundary.  Every reduction
 * runs in a fixed order: the results are identical bit for bit from run to run and between
 * kdn_delta_scan_bwd and kdn_delta_scan_bwd_streams.
 *
 * At D = 1024 (ABI 1.8) the backward runs on one stream (the auxiliary stream is not used, and
 * kdn_scan_bwd_phase returns KDN_ERR_UNSUPPORTED), in segments of fwd->segment_chunks chunks (0: the
 * largest power of two from 4 to 256 whose records fit 24 GiB; ABI 2.3): a checkpoint pass of the
 * recompute and the forward carry stores the state at each segment start, then each segment, last first,
 * recomputes its chunks, carries the state forward from its checkpoint and dL/dS backward from the next
 * segment (a reverse carry from its last chunk to its first), and two parallel launches write its
 * gradients.  Its workspace is one record per (batch, head, chunk) of a segment (3,015,168 bytes at
 * d_v = 128, 1,819,136 at d_v = 64), one fp32 [B][H][1024][d_v] state per segment boundary, one more for
 * the carried dL/dS with more than one segment and one for the forward carry's final state.  The results
 * do not depend on the segment length (bit for bit), and its reductions run in a fixed order. */
typedef struct kdn_scan_bwd_args {
  const kdn_scan_args* fwd;
  const float* dy;            int64_t dy_stride[3];
  const float* d_final_state; int64_t dfinal_stride[4];
  float* dq;                  int64_t dq_stride[3];
  float* dk;                  int64_t dk_stride[3];
  float* dv;                  int64_t dv_stride[3];
  float* dbeta;               int64_t dbeta_stride[3];
  float* ddecay;              int64_t ddecay_stride[3];
  float* d_initial_state;     int64_t dinit_stride[4];
  void* workspace;            size_t workspace_bytes;
  /* ABI 1.7: dL/d(1/tau) per head, float32 [H] (NULL: not computed).  With per-head 1/tau
   * (fwd->inv_tau_head) it is that head's gradient; with the shared fwd->inv_tau the H values sum to its
   * gradient.  Reduced in a fixed order over batches and chunks (deterministic). */
  float* dinv_tau;
} kdn_scan_bwd_args;

/* Workspace bytes kdn_delta_scan_bwd needs (0 if the arguments are invalid or unsupported). */
size_t kdn_scan_bwd_workspace_bytes(const kdn_scan_bwd_args* a);

/* Segments of the backward (ABI 1.6): returns their number (0 if the arguments are invalid or
 * unsupported) and, when segment_chunks is not NULL, their length in 64-token chunks. */
int64_t kdn_scan_bwd_segments(const kdn_scan_bwd_args* a, int64_t* segment_chunks);

/* Enqueues the backward on `stream`: the checkpoint pass, then per segment (last first) the per-chunk
 * recompute of the lift and the chunk matrices, the forward state carry (state at every chunk start),
 * the reverse carry of dL/dS, and the per-chunk gradients with the lift's backward. */
int kdn_delta_scan_bwd(const kdn_scan_bwd_args* a, void* stream);

/* kdn_delta_scan_bwd over two streams: both carries of each segment (one launch) and its gradient
 * algebra run back to back on `stream` while aux_stream runs the recompute and dx launches of the
 * segments around them (and the checkpoint pass's prep kernels beside its state kernels).  Same workspace, same
 * results bit for bit.  aux_stream NULL (or equal to `stream`) is kdn_delta_scan_bwd.  Both streams
 * should have default priority.  Replaces kernels/fused_kernel_deltanet.py:168-179, like
 * kdn_delta_scan_bwd. */
int kdn_delta_scan_bwd_streams(const kdn_scan_bwd_args* a, void* stream, void* aux_stream);

/* One launch group of kdn_delta_scan_bwd (ABI 1.6 signature), for callers that time or schedule them:
 * phase 0 is the start of a call (the Omega^T table and the checkpoint pass; `segment` ignored); phases
 * 1 (per-chunk recompute), 2 (forward carry), 3 (reverse carry) and 4 (gradients) are those of segment
 * `segment` (0 .. kdn_scan_bwd_segments - 1).  On one workspace they must run in the order of
 * kdn_delta_scan_bwd: 0, then for segments from the last to the first 1, 2, 3, 4 (stream order or
 * events).  Same arguments and checks. */
int kdn_scan_bwd_phase(const kdn_scan_bwd_args* a, int phase, int64_t segment, void* stream);

/* ---- Serving: ragged mixed prefill + decode step over resident states -------------------------
 * One step of a batch of sequences that continue from states resident in a slab (the reference's
 * serving op vllm_hybrid_recurrent_forward, serving/vllm_kernel_deltanet_op.cpp:11-34, whose body is a
 * stub; its packing follows serving/vllm_ragged_batching.py:56-66).  Sequence i is the token rows
 * cu_seqlens[i] .. cu_seqlens[i+1]-1 of q / k / v / beta / decay / y ([token][head][...]) and continues
 * from state slot slots[i] of `states` ([slot][head][0:D][0:d_v] fp32, updated in place).  Sequences of
 * one token run the decode kernel (lift of q and k, readout y = S phi(q), rank-1 update of S; one pass
 * over the state); longer ones run the ragged chunked scan; sequences without tokens are left alone.
 * The recurrence, feature map (the structured lift: omega_bf16, phase, inv_tau, normalize_input) and
 * tolerances are those of kdn_delta_scan_fwd; rule 1 selects the linear rule as there. */
typedef struct kdn_ragged_args {
  int64_t num_seqs, H;
  int d_k, D, d_v;             /* d_k = 64, D = 512, d_v in {16, 32, 64, 128} */
  int in_dtype, out_dtype, normalize_input, rule;
  float inv_tau;
  const int64_t* cu_seqlens;       /* device [num_seqs + 1] */
  const int64_t* cu_seqlens_host;  /* the same offsets in host memory (scheduling: counts, longest); they
                                    * must equal the device copy (entries the two disagree on are
                                    * skipped, never read unwritten) */
  const int32_t* slots;            /* device [num_seqs]: distinct state slots (see num_slots) */
  const void* q;   int64_t q_stride[2];   /* [token][head] element strides; innermost contiguous */
  const void* k;   int64_t k_stride[2];
  const void* v;   int64_t v_stride[2];
  const float* beta;  int64_t beta_stride[2];
  const float* decay; int64_t decay_stride[2];   /* NULL means lambda = 1 */
  const void* omega_bf16; const float* phase;
  float* states;   int64_t state_stride[4];       /* [slot][head][feature][value] */
  void* y;         int64_t y_stride[2];
  void* workspace; size_t workspace_bytes;
  int64_t num_slots;   /* (ABI 1.5) slots in `states`; required.  A sequence whose slot lies outside
                        * [0, num_slots) -- a negative slot is the padding convention -- is skipped on the
                        * device: its state is not touched and its y rows are not written. */
} kdn_ragged_args;

/* Workspace bytes kdn_ragged_step needs (0 if the arguments are invalid); reads the shape fields and
 * cu_seqlens_host. */
size_t kdn_ragged_workspace_bytes(const kdn_ragged_args* a);

/* Runs the step on `stream`.  With aux_stream (not NULL, not `stream`) the prefill part uses the
 * pipelined scan and the decode part runs on aux_stream after the prefill's prep launches; aux_stream
 * first waits for the work queued on `stream`, and `stream` finally waits for aux_stream. */
int kdn_ragged_step(const kdn_ragged_args* a, void* stream, void* aux_stream);

/* The same step described by a token -> slot map alone, with nothing read back to the host (ABI 2.2):
 * the reference op's own arguments, vllm_hybrid_recurrent_forward(query, key, value, beta, decay,
 * recurrent_states, slot_mapping, output), serving/vllm_kernel_deltanet_op.cpp:11-34.  A sequence is a
 * run of consecutive tokens with one slot; a negative slot, or one at or above num_slots, marks padding
 * (skipped: no state touched, no y row written).  The runs, the decode / prefill split and the prefill's
 * packed layout are all formed on the device and every launch is sized from num_tokens and num_slots, so
 * distinct runs must have distinct slots (not checked); a map with more than 2 * num_slots + 1 runs is
 * invalid, and then nothing runs and *status (device int32, if not NULL) is set to 1 (else 0).  The
 * prefill runs the split scan over windows of 128 packed chunk slots (each sequence's chunks plus one spare
 * slot), pipelined over aux_stream when it is not NULL. */
typedef struct kdn_slot_step_args {
  int64_t num_tokens, H;
  int d_k, D, d_v;             /* d_k = 64, D = 512, d_v in {16, 32, 64, 128} */
  int in_dtype, out_dtype, normalize_input, rule;
  float inv_tau;
  const void* slot_mapping;    /* device [num_tokens] */
  int slot_bytes;              /* 4 (int32) or 8 (int64) bytes per slot_mapping entry */
  const void* q;   int64_t q_stride[2];   /* [token][head] element strides; innermost contiguous */
  const void* k;   int64_t k_stride[2];
  const void* v;   int64_t v_stride[2];
  const float* beta;  int64_t beta_stride[2];
  const float* decay; int64_t decay_stride[2];   /* NULL means lambda = 1 */
  const void* omega_bf16; const float* phase;
  float* states;   int64_t state_stride[4];       /* [slot][head][feature][value] */
  int64_t num_slots;
  void* y;         int64_t y_stride[2];
  void* workspace; size_t workspace_bytes;
  int32_t* status;
} kdn_slot_step_args;

/* Workspace bytes kdn_slot_step needs (0 if the arguments are invalid); reads the shape fields only. */
size_t kdn_slot_step_workspace_bytes(const kdn_slot_step_args* a);
/* Streams as kdn_ragged_step. */
int kdn_slot_step(const kdn_slot_step_args* a, void* stream, void* aux_stream);

/* ---- Slab state pool --------------------------------------------------------------------------
 * Slot bookkeeping over a caller-allocated slab of `max_slots` equal fp32 state slots of slot_bytes
 * each (for example [slot][layer][head][D][d_v]); the reference's HybridMemoryPool recurrent slab,
 * serving/hybrid_memory_pool.{h,cpp} (the softmax anchor pages of that class are not part of this path).
 * Host-side and single-threaded per pool; functions that take a slab pointer also enqueue device work
 * on `stream` (zeroing a new slot, copying a forked one), and skip it when slab is NULL. */
typedef struct kdn_pool kdn_pool;
int kdn_pool_create(int64_t max_slots, int64_t slot_bytes, kdn_pool** out);
void kdn_pool_destroy(kdn_pool* pool);
/* A free slot (>= 0), zeroed on the device when slab is not NULL; KDN_ERR_CAPACITY when none is free. */
int kdn_pool_allocate(kdn_pool* pool, void* slab, void* stream);
/* A new slot holding a copy of active slot `parent` (hybrid_memory_pool.cpp:86-116); negative on error. */
int kdn_pool_fork(kdn_pool* pool, int parent, void* slab, void* stream);
/* Returns an active slot to the pool (hybrid_memory_pool.cpp:118-135); negative if it is not active. */
int kdn_pool_release(kdn_pool* pool, int slot);
int64_t kdn_pool_active(const kdn_pool* pool);
int64_t kdn_pool_allocated_bytes(const kdn_pool* pool);
int64_t kdn_pool_free_bytes(const kdn_pool* pool);

#ifdef __cplusplus
}
#endif

#endif /* KDN_H */
