/*
 * gdn_hip.h -- C ABI of libgdn_hip.so, the MI355X (gfx950) Gated DeltaNet
 * decode and prefill operators.
 *
 * Conventions (all entry points):
 *   - plain device pointers to contiguous row-major tensors; bf16 tensors are
 *     passed as uint16_t (raw bf16 bits), fp32 as float;
 *   - the caller owns every buffer; nothing here allocates device memory;
 *   - work is enqueued on `stream` (a hipStream_t, NULL = default stream),
 *     asynchronously, with no host synchronisation;
 *   - return 0 on success, a negative GDN_ERR_* code for an argument error
 *     (nothing launched), or -(hipError_t) if a launch failed;
 *   - an array with no elements may be NULL: decode with B = 0 reads and
 *     writes nothing; prefill with T = 0 needs only cu_seqlens and, when
 *     N > 0, A_log, dt_bias and final_state (the initial states are copied);
 *   - no C++ exception crosses the ABI.
 *
 * Layouts (D = 128 = K = V; qk-head of v-head h is h / (HV/HQ)):
 *   decode : q, k [B, HQ, D] bf16; v [B, HV, D] bf16; a, b [B, HV] bf16;
 *            A_log, dt_bias [HV] fp32; state [B, HV, V, K] fp32 (k-last);
 *            out [B, HV, D] bf16.
 *   prefill: q, k [T, HQ, D] bf16; v [T, HV, D] bf16; a, b [T, HV] bf16;
 *            cu_seqlens [N+1] (int64, or int32 when cu_is_int32 != 0);
 *            state / final_state [N, HV, V, K] fp32; out [T, HV, D] bf16.
 */
#ifndef GDN_HIP_H_
#define GDN_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN_ABI_VERSION 1

#define GDN_OK 0
#define GDN_ERR_NULL (-1001)      /* a required pointer is NULL */
#define GDN_ERR_SHAPE (-1002)     /* an unsupported size or head configuration */
#define GDN_ERR_WORKSPACE (-1003) /* workspace missing or too small */

/* Option bits of the *_ex entry points and gdn_decode_multi_fwd.
 * GDN_QK_L2NORM: every q and k row (128 elements) is used L2-normalised,
 *   x (sum x^2 + 1e-6)^(-1/2), computed in fp32 inside the kernel.  The
 *   reference expects normalised inputs from its caller and has no such
 *   option. */
#define GDN_QK_L2NORM 1
/* GDN_NO_SEAMS (prefill entry points): the split path (with few chains)
 *   and the fused kernel under a plan (gdn_prefill_plan_fwd) may cut the
 *   longest sequences in two in time -- the tail runs from a zero state
 *   beside a transition chain (v = 0 from the identity) and a seam pass adds
 *   the head's state to the tail's outputs and final state -- so that CUs
 *   left idle shorten the longest chain (no reference counterpart; the
 *   reference runs every chain serially).  Results then agree with the
 *   serial chain to the rounding of the state path.  This bit runs every
 *   chain whole.  Decode entry points reject it. */
#define GDN_NO_SEAMS 2
/* GDN_PLAN_FUSED (gdn_prefill_plan only): plan the fused kernel (with its
 *   seams) whatever the lengths favour. */
#define GDN_PLAN_FUSED 4
#define GDN_FLAGS_ALL 3
#define GDN_DECODE_FLAGS_ALL 1

/* ABI version of the loaded library (GDN_ABI_VERSION). */
int gdn_abi_version(void);

/* Human-readable text for a return code of this library. */
const char* gdn_error_string(int code);

/*
 * One decode step for B sequences.
 * Replaces the reference decode entry `run(q, k, v, state, A_log, a, dt_bias,
 * b, scale)` (gdn_decode_qk4_v8_d128_k_last/solution/triton/kernel.py:100-146)
 * and its kernel (same file :26-79).
 *   state      : [B, HV, V, K] fp32, or NULL for a zero state (kernel.py:86-94).
 *   new_state  : [B, HV, V, K] fp32 output; may equal `state` (in-place update).
 *   scale      : applied to q; the caller resolves None/0 to 1/sqrt(D)
 *                (kernel.py:112-115).
 * HV must be a multiple of HQ.
 */
int gdn_decode_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                   const float* state, float* new_state,
                   const float* A_log, const uint16_t* a, const float* dt_bias,
                   const uint16_t* b, uint16_t* out,
                   int B, int HQ, int HV, float scale, void* stream);

/*
 * gdn_decode_fwd with option bits (GDN_QK_L2NORM); flags = 0 is
 * gdn_decode_fwd.  Unknown bits: GDN_ERR_SHAPE.
 */
int gdn_decode_ex_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                      const float* state, float* new_state,
                      const float* A_log, const uint16_t* a, const float* dt_bias,
                      const uint16_t* b, uint16_t* out,
                      int B, int HQ, int HV, float scale, int flags, void* stream);

/*
 * One decode step against a state pool, updated in place:
 * state_pool[slot_ids[n]] is read and overwritten for every n < B.
 * No reference counterpart: the reference decode takes one dense state per
 * sequence (kernel.py:100-146).  This serves callers that keep recurrent
 * states in a slot pool (serving engines).  slot_ids must be distinct; a
 * slot outside [0, pool_size) leaves the pool untouched and yields a zero
 * output row.
 */
int gdn_decode_pool_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                        float* state_pool, int pool_size, const int32_t* slot_ids,
                        const float* A_log, const uint16_t* a, const float* dt_bias,
                        const uint16_t* b, uint16_t* out,
                        int B, int HQ, int HV, float scale, void* stream);

/*
 * T consecutive decode steps per sequence (multi-token / speculative decode):
 * for t = 0..T-1 in order, the step of gdn_decode_fwd with token t's inputs,
 * the state kept on chip in between (read once, written once).
 * No reference counterpart: the reference decode asserts one token per call
 * (gdn_decode_qk4_v8_d128_k_last/solution/triton/kernel.py:117-119); this
 * serves callers that verify several draft tokens per sequence.
 *   q, k : [B, T, HQ, D] bf16;  v : [B, T, HV, D] bf16;  a, b : [B, T, HV] bf16;
 *   out  : [B, T, HV, D] bf16;  state / new_state : [B, HV, V, K] fp32 as in
 *   gdn_decode_fwd (state NULL = zeros; new_state may equal state).
 * T must be >= 1; flags as for gdn_decode_ex_fwd.  The result equals T
 * successive gdn_decode_ex_fwd calls with the same flags bit for bit.
 */
int gdn_decode_multi_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                         const float* state, float* new_state,
                         const float* A_log, const uint16_t* a, const float* dt_bias,
                         const uint16_t* b, uint16_t* out,
                         int B, int T, int HQ, int HV, float scale, int flags, void* stream);

/*
 * Workspace bytes gdn_prefill_fwd uses for this problem on the current
 * device: the split path's workspace when it would run (few chains, see
 * gdn_prefill_fwd), else 0.
 */
size_t gdn_prefill_workspace_bytes(int N, int T, int HQ, int HV);

/*
 * Chunked (64-token) varlen prefill.
 * Replaces the reference prefill entry `run(q, k, v, state, A_log, a,
 * dt_bias, b, cu_seqlens, scale)`
 * (gdn_prefill_qk4_v8_d128_k_last/solution/triton/kernel.py:1762-1802) and
 * the five kernels it launches (kernel.py:1570-1633, 1728-1759).
 *   state       : [N, HV, V, K] fp32 initial states, or NULL for zeros.
 *   final_state : [N, HV, V, K] fp32 output.
 *   cu_seqlens  : device array, N+1 entries, cu_seqlens[0] == 0,
 *                 cu_seqlens[N] == T, non-decreasing (empty sequences allowed).
 *   scale       : any float; the caller resolves None/0 to 1/sqrt(D)
 *                 (kernel.py:1777-1778).  A negative scale negates the output.
 *   workspace   : device buffer of gdn_prefill_workspace_bytes(...) bytes, or
 *                 NULL.  With few (sequence, v-head) chains the split path
 *                 runs when the workspace is given (gdn_prefill_split_fwd with
 *                 the automatic slice count); without it, and with many
 *                 chains, one fused workgroup per chain.
 * Input range: the state path multiplies fp16 operands (k, the state, X and
 * Vn); values must stay below 65504 in magnitude (normalised q / k, v and
 * states of ordinary magnitude are far inside), else results overflow.
 * Sequences whose cu_seqlens ranges overlap or run backwards are read in
 * bounds, but their results are unspecified.
 */
int gdn_prefill_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                    const float* state, const float* A_log, const uint16_t* a,
                    const float* dt_bias, const uint16_t* b,
                    const void* cu_seqlens, int cu_is_int32, int N, int T,
                    int HQ, int HV, float scale,
                    uint16_t* out, float* final_state,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * gdn_prefill_fwd with option bits (GDN_QK_L2NORM); flags = 0 is
 * gdn_prefill_fwd.  Unknown bits: GDN_ERR_SHAPE.
 */
int gdn_prefill_ex_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                       const float* state, const float* A_log, const uint16_t* a,
                       const float* dt_bias, const uint16_t* b,
                       const void* cu_seqlens, int cu_is_int32, int N, int T,
                       int HQ, int HV, float scale,
                       uint16_t* out, float* final_state,
                       void* workspace, size_t workspace_bytes, int flags, void* stream);

/*
 * State slices per chain the automatic path selection of gdn_prefill_fwd uses
 * for N sequences of HV v-heads on the current device: 8 or 4 (split path),
 * or 0 (the fused chain kernel).
 */
int gdn_prefill_auto_slices(int N, int HV);

/*
 * The path choice from the sequence lengths, for callers that hold
 * cu_seqlens on the host (reads a HOST copy, N+1 entries): 8 or 4 state
 * slices per chain (gdn_prefill_split_fwd) or 0 (the fused chain kernel:
 * gdn_prefill_ex_fwd without a workspace), whichever a cost model of the
 * launches (cycles per chunk of each kernel measured on MI355X, the split
 * path's preparation per (chunk, v-head), the slice workgroups scheduled
 * longest sequence first on `cus` CUs, one per CU; seams on neither path,
 * the qk-heads being unknown here) finishes first.  Only batches of at most
 * one chain per CU are considered for the split path.
 * `cus` <= 0: the current device's CU count.  -1 on a NULL pointer or
 * negative N / T or HV <= 0.  gdn_prefill_auto_slices decides from N and HV
 * alone and may pick the split path where the fused kernel is faster (four
 * 5348-token sequences at 32 v-heads: split 390 us, fused 267 us).  No
 * reference counterpart (the reference has one path).
 */
int gdn_prefill_choose_slices(const void* cu_seqlens_host, int cu_is_int32, int N, int T, int HV,
                              int cus);

/*
 * Launch plan of a prefill call, made on the host from a HOST copy of
 * cu_seqlens (N+1 entries; the reference's run() reads cu_seqlens back for
 * its cu_seqlens[-1] == T check, PRE:1665, so its caller holds one): the
 * path of gdn_prefill_choose_slices's model with each path's seams (the
 * split path's as its launch chooses them, XCD by XCD), and for the fused
 * kernel the seams that its cost model finds to finish first -- with at
 * most one chain per CU, the
 * longest sequences cut at a common chunk M, their tails run (from a zero
 * state and as the transition chain) by workgroups that take the CUs shorter
 * chains free, then a seam pass (8 sequences of 2394-5348 tokens at 32
 * v-heads: the 84-chunk chain becomes about 72 chunk periods).  `plan`
 * receives GDN_PREFILL_PLAN_BYTES bytes (host memory, opaque, reusable for
 * calls with the same cu_seqlens on the same device); *workspace_bytes (if
 * not NULL) the device workspace gdn_prefill_plan_fwd needs (0: none).
 * `cus` <= 0: the current device's CU count.  flags: GDN_NO_SEAMS plans no
 * seams, GDN_PLAN_FUSED the fused kernel.  No reference counterpart.
 */
#define GDN_PREFILL_PLAN_BYTES 512
int gdn_prefill_plan(const void* cu_seqlens_host, int cu_is_int32, int N, int T, int HQ, int HV,
                     int cus, int flags, void* plan, size_t* workspace_bytes);

/* Of a plan: the path (*slices: 4 / 8 split, 0 fused); *seams: the fused
 * kernel's seams, or on the split path the seam slots its launch reserves
 * (the seams themselves chosen on the device; any slot adds the seam pass);
 * the fused seams' cut chunk (*split_chunk, 0 without seams) and the
 * modelled fused finish in chunk periods (*periods, the seam pass excluded);
 * any pointer may be NULL.  GDN_ERR_SHAPE if `plan` is not one. */
int gdn_prefill_plan_info(const void* plan, int* slices, int* seams, int* split_chunk, int* periods);

/*
 * gdn_prefill_ex_fwd on the path and seams of `plan` (from gdn_prefill_plan
 * with the same N, T, HQ, HV and the same cu_seqlens contents, else
 * GDN_ERR_SHAPE or results that are not specified).  The workspace
 * (device) holds the plan's workspace bytes: on the fused path the seam
 * region (the seam plan, three fp32 [128][128] states per seam and v-head,
 * the transition outputs of the tails), which nothing has to clear.  flags:
 * GDN_QK_L2NORM, GDN_NO_SEAMS (the plan's fused seams are then not run).
 */
int gdn_prefill_plan_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                         const float* state, const float* A_log, const uint16_t* a,
                         const float* dt_bias, const uint16_t* b, const void* cu_seqlens,
                         int cu_is_int32, int N, int T, int HQ, int HV, float scale,
                         uint16_t* out, float* final_state, const void* plan, void* workspace,
                         size_t workspace_bytes, int flags, void* stream);

/*
 * Workspace bytes of gdn_prefill_split_fwd: 14 080 bytes per (chunk, v-head)
 * and 18 432 per (chunk, qk-head) for an upper bound of T / 64 + N chunks,
 * plus the sequences' launch order (N ints, rounded up to 256 bytes).
 */
size_t gdn_prefill_split_workspace_bytes(int N, int T, int HQ, int HV);

/*
 * gdn_prefill_ex_fwd on the split path, for batches with fewer chains than
 * the GPU has CUs: a launch over all (chunk, v-head) pairs forms each
 * chunk's state-independent operands (gates, the diagonal blocks of
 * (I + A)^-1, -A_ba, P, fp16 K) in the workspace, then every chain runs as
 * `slices` workgroups (4 or 8), each owning 128 / slices rows of the state.
 * This is how the reference spreads its recurrence over the GPU: the
 * per-chunk kernels over all chunks, the recurrence over V-slices
 * (gdn_prefill_qk4_v8_d128_k_last/solution/triton/kernel.py:544, 1005, 1369).
 * Without GDN_QK_L2NORM the state-path operations are gdn_prefill_ex_fwd's
 * in the same order: final states equal bit for bit but for rare last-place
 * differences (one or two sequences in thousands); outputs agree to within
 * 1e-4.
 *   workspace : at least gdn_prefill_split_workspace_bytes(...) bytes, else
 *               GDN_ERR_WORKSPACE.  Other slice counts: GDN_ERR_SHAPE.
 */
int gdn_prefill_split_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                          const float* state, const float* A_log, const uint16_t* a,
                          const float* dt_bias, const uint16_t* b,
                          const void* cu_seqlens, int cu_is_int32, int N, int T,
                          int HQ, int HV, float scale,
                          uint16_t* out, float* final_state, int slices,
                          void* workspace, size_t workspace_bytes, int flags, void* stream);

/*
 * gdn_prefill_split_fwd without a caller workspace and without any device
 * allocation: no reference counterpart.  It serves callers that cannot
 * allocate (code under HIP graph capture, tight serving loops).  The
 * workspace is a static device array of gdn_prefill_split_noalloc_max_bytes()
 * (32 MiB) that each GPU the library runs on holds until the process ends;
 * problems whose gdn_prefill_split_workspace_bytes exceed it return
 * GDN_ERR_WORKSPACE before any launch (for example T = 4096, N = 1 at
 * qk4 / v8 needs 12.1 MB).  All calls on one GPU share the array: calls that
 * overlap on one GPU (other streams, other threads) race.  Results equal
 * gdn_prefill_split_fwd's bit for bit.
 */
size_t gdn_prefill_split_noalloc_max_bytes(void);
int gdn_prefill_split_noalloc_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                  const float* state, const float* A_log, const uint16_t* a,
                                  const float* dt_bias, const uint16_t* b,
                                  const void* cu_seqlens, int cu_is_int32, int N, int T,
                                  int HQ, int HV, float scale,
                                  uint16_t* out, float* final_state, int slices, int flags,
                                  void* stream);

/*
 * Number of 64-token chunks of a varlen batch, sum over n of
 * ceil(len_n / 64) with len_n from cu_seqlens clamped into [0, T] as the
 * kernels clamp it: the first dimension of the h output below.  Reads a HOST
 * copy of cu_seqlens (N+1 entries).  Returns -1 on a NULL pointer or
 * negative N / T.  Counterpart of the chunk count `NT = len(chunk_indices)`
 * and of `prepare_chunk_offsets` (gdn_prefill_qk4_v8_d128_k_last/solution/
 * triton/kernel.py:1358-1361, 172-209).
 */
long long gdn_prefill_chunk_count(const void* cu_seqlens_host, int cu_is_int32, int N, int T);

/*
 * gdn_prefill_ex_fwd that also writes the state entering every chunk:
 * h[chunk_offset(n) + i][hv][v][k], bf16 (round to nearest even), with
 * chunk_offset(n) the chunks of sequences 0 .. n-1 and i the chunk within
 * sequence n; h[chunk_offset(n)] is the initial state (zeros without one).
 * Replaces `chunk_gated_delta_rule_fwd_h`'s h output, `h = k.new_empty(B, NT,
 * H, V, K)` stored before each chunk's update
 * (gdn_prefill_qk4_v8_d128_k_last/solution/triton/kernel.py:1341-1398,
 * 1153-1160), the per-chunk states a training backward reads.
 *   h        : device [h_chunks, HV, 128, 128] bf16.
 *   h_chunks : capacity of h in chunks; gdn_prefill_chunk_count(...) gives
 *              the number written.  Slots at or past h_chunks are skipped.
 *   workspace: as for gdn_prefill_ex_fwd: with few chains and the workspace
 *              of gdn_prefill_workspace_bytes the split path runs (the
 *              reference writes h from its V-split recurrence grid at any
 *              batch size, kernel.py:1369), else one fused workgroup per
 *              chain.
 * out / final_state are those of gdn_prefill_ex_fwd on the same path, bit
 * for bit; h is the bf16 image of the state the path forms either way.
 */
int gdn_prefill_h_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                      const float* state, const float* A_log, const uint16_t* a,
                      const float* dt_bias, const uint16_t* b,
                      const void* cu_seqlens, int cu_is_int32, int N, int T,
                      int HQ, int HV, float scale,
                      uint16_t* out, float* final_state, uint16_t* h, int h_chunks,
                      void* workspace, size_t workspace_bytes, int flags, void* stream);

/*
 * gdn_prefill_h_fwd forced onto the split path with `slices` (4 or 8) state
 * slices per chain, as gdn_prefill_split_fwd (the counterpart of
 * chunk_gated_delta_rule_fwd_h's V-split grid, kernel.py:1365-1393, with h
 * stored per chunk as at kernel.py:1153-1160).  The workspace is that of
 * gdn_prefill_split_workspace_bytes; GDN_ERR_WORKSPACE when NULL or short,
 * GDN_ERR_SHAPE for another slice count.
 */
int gdn_prefill_split_h_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            const float* state, const float* A_log, const uint16_t* a,
                            const float* dt_bias, const uint16_t* b,
                            const void* cu_seqlens, int cu_is_int32, int N, int T,
                            int HQ, int HV, float scale,
                            uint16_t* out, float* final_state, uint16_t* h, int h_chunks,
                            int slices, void* workspace, size_t workspace_bytes, int flags,
                            void* stream);

/*
 * Backward of the prefill (no counterpart in the reference, which is
 * forward-only: gdn_prefill_qk4_v8_d128_k_last/solution/triton/kernel.py:1;
 * it consumes the per-chunk states h that chunk_gated_delta_rule_fwd_h
 * produces, kernel.py:1153-1160, here gdn_prefill_h_fwd).
 *
 * Device workspace bytes of gdn_prefill_bwd: per (64-token chunk slot,
 * v-head) 96 KiB (the chunk's state-gradient transition and the gradient of
 * the state leaving it).  0 for invalid sizes.
 */
size_t gdn_prefill_bwd_workspace_bytes(int N, int T, int HQ, int HV);

/*
 * Gradients of a loss L(out, final_state) of gdn_prefill_fwd with respect to
 * its inputs, given dL/d out and dL/d final_state.
 *   q, k, v, A_log, a, dt_bias, b, cu_seqlens, cu_is_int32, N, T, HQ, HV,
 *   scale      : the forward's inputs (scale as the forward used it).
 *   h          : [h_chunks, HV, 128, 128] bf16, the states entering every
 *                chunk as gdn_prefill_h_fwd wrote them for the same inputs;
 *                h_chunks must be at least gdn_prefill_chunk_count(...).
 *   d_out      : [T, HV, 128] bf16.
 *   d_final_state : [N, HV, 128, 128] fp32, or NULL for zeros.
 * Outputs (fp32, written whole):
 *   dq, dk     : [T, HQ, 128] (summed over the v-heads sharing a qk-head).
 *   dv         : [T, HV, 128].
 *   dg, dbeta  : [T, HV]: gradients of the per-token log-decay
 *                g = -exp(A_log) softplus(a + dt_bias) and of beta = sigmoid(b);
 *                gdn_gate_bwd maps them to a, b, A_log, dt_bias.
 *   d_initial_state : [N, HV, 128, 128], or NULL when not wanted.
 * Products take bf16 operands with fp32 accumulation.  Three launches
 * (plus one when HV > HQ) on `stream`: per-chunk state-gradient transitions
 * (all chunks at once), the chain over each sequence's chunks in reverse,
 * and the per-chunk gradients.  Not q/k L2-normalising (GDN_QK_L2NORM has no
 * backward here).  GDN_ERR_WORKSPACE when the workspace is NULL or short.
 */
int gdn_prefill_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                    const float* A_log, const uint16_t* a, const float* dt_bias,
                    const uint16_t* b, const void* cu_seqlens, int cu_is_int32, int N, int T,
                    int HQ, int HV, float scale, const uint16_t* h, int h_chunks,
                    const uint16_t* d_out, const float* d_final_state, float* dq, float* dk,
                    float* dv, float* dg, float* dbeta, float* d_initial_state,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * Gradients of the prefill gating (kernel.py:1706-1722) per token and v-head:
 *   da = dg (-exp(A_log) sigmoid(a + dt_bias)),   db = dbeta beta (1 - beta),
 *   dA_log = sum_t dg g,   ddt_bias = sum_t da    (fixed summation order).
 * a, b: [T, HV] bf16; dg, dbeta, da, db: [T, HV] fp32; A_log, dt_bias,
 * dA_log, ddt_bias: [HV] fp32.  No counterpart in the reference.
 */
int gdn_gate_bwd(const float* A_log, const uint16_t* a, const float* dt_bias, const uint16_t* b,
                 const float* dg, const float* dbeta, int T, int HV, float* da, float* db,
                 float* dA_log, float* ddt_bias, void* stream);

/* Activations of the q/k/v convolution. */
#define GDN_ACT_NONE 0
#define GDN_ACT_SILU 1

/*
 * Short causal convolution ahead of GDN (no reference counterpart: the
 * reference operators take q, k, v after it).  In a Qwen3-Next-style layer
 * the q, k, v projections, concatenated channel-wise ("mixed_qkv"), pass
 * through a depthwise causal conv1d of kernel size W and SiLU before GDN:
 *   y[t, c] = act(bias[c] + sum_w weight[c, w] h[t - (W - 1) + w, c]),
 * h being each sequence's inputs preceded by its conv state (or zeros).
 *   x          : [T, C] bf16 (token-major, C a multiple of 8).
 *   weight     : [C, W] fp32, W in 2..4;  bias : [C] fp32 or NULL.
 *   cu_seqlens : as for gdn_prefill_fwd (int64, or int32 when cu_is_int32),
 *                N >= 1 when T > 0 (else GDN_ERR_SHAPE).  Tokens outside
 *                every sequence (a padded batch with cu_seqlens[N] < T, or
 *                ranges that run backwards) get zero outputs; reads stay in
 *                bounds.
 *   conv_state_in  : [N, C, state_len] bf16 (the inputs that preceded each
 *                    sequence, oldest first) or NULL for zeros.
 *   conv_state_out : [N, C, state_len] bf16 or NULL: the last state_len inputs
 *                    of every sequence (its state entries where the sequence is
 *                    shorter).  Must not alias conv_state_in.
 *   state_len  : W - 1 .. 8.
 *   out_q, out_k, out_v : the output split by channel into three row-major
 *                    tensors of widths cq, ck and C - cq - ck (multiples of
 *                    8): GDN's q [T, HQ, 128], k [T, HQ, 128], v [T, HV, 128]
 *                    with cq = ck = 128 HQ.  With out_k = out_v = NULL the
 *                    whole [T, C] output goes to out_q.
 *   activation : GDN_ACT_SILU or GDN_ACT_NONE.
 */
int gdn_qkv_conv1d_fwd(const uint16_t* x, const float* weight, const float* bias,
                       const void* cu_seqlens, int cu_is_int32, int N, int T, int C, int W,
                       const uint16_t* conv_state_in, uint16_t* conv_state_out, int state_len,
                       uint16_t* out_q, uint16_t* out_k, uint16_t* out_v, int cq, int ck,
                       int activation, void* stream);

/*
 * One decode token per sequence through the same convolution, the conv state
 * updated in place (shifted by one, the token appended).
 *   x          : [B, C] bf16.
 *   conv_state : [pool, C, state_len] bf16, state_len W - 1 or W (else
 *                GDN_ERR_SHAPE); row slot_ids[b] (or b when
 *                slot_ids is NULL, then pool_size >= B) serves sequence b.
 *                Distinct slots; a slot outside [0, pool_size) leaves the
 *                state untouched and yields a zero output row.
 *   outputs, weight, bias, activation as for gdn_qkv_conv1d_fwd (B tokens).
 * Equal bit for bit to gdn_qkv_conv1d_fwd over length-1 sequences.
 */
int gdn_qkv_conv1d_update(const uint16_t* x, const float* weight, const float* bias,
                          uint16_t* conv_state, int state_len, const int32_t* slot_ids,
                          int pool_size, int B, int C, int W, uint16_t* out_q, uint16_t* out_k,
                          uint16_t* out_v, int cq, int ck, int activation, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN_HIP_H_ */
