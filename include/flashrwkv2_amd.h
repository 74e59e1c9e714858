/*
 * flashrwkv2_amd — C ABI of the MI355X (gfx950) WKV7 operator library.
 *
 * Every entry point takes device pointers, integer sizes, a token dtype tag
 * and a HIP stream (passed as `void*`, a `hipStream_t`), enqueues its kernels
 * on that stream and returns an `fr2_status_t`.  Nothing here allocates device
 * memory; the caller owns every buffer.  No entry point synchronises the
 * stream.  The library holds no global mutable state, so concurrent calls on
 * different streams are safe.
 *
 * Layouts (all row-major, contiguous):
 *   token tensors   r, decay_logits, k, v, a, b, output : [total_tokens, H, D]
 *   decay_bias      [H, D] (nullable), same dtype as the tokens
 *   state pool      [slots, H, D, D]  (S[slot, h, key, value])
 *   metadata        query_start_loc [N+1] int32, state_indices [N] int32
 *   status          int32[3] = {error bits, active tokens, active sequences}
 *
 * Recurrence (per token, per head; fp32 arithmetic):
 *   w[k]  = exp(-exp(-1/2) * sigmoid(decay_logits[k] + decay_bias[h,k]))
 *   sa[v] = sum_k a[k] S[k,v]                       (pre-update state)
 *   S[k,v] = w[k] S[k,v] + b[k] sa[v] + k[k] v[v]
 *   y[v]  = scale * sum_k r[k] S[k,v]               (post-update state)
 *
 * Reference interfaces replaced are cited per entry point as
 * path:line inside rwkv-rs/FlashRWKV2 v0.1.0a7.
 */
#ifndef FLASHRWKV2_AMD_H_
#define FLASHRWKV2_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  FR2_OK = 0,
  FR2_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad size or count */
  FR2_ERR_UNSUPPORTED = 2,      /* head size / dtype / chunk size not built */
  FR2_ERR_LAUNCH = 3,           /* hipGetLastError() after a launch */
} fr2_status_t;

typedef enum {
  FR2_DTYPE_FLOAT16 = 0,
  FR2_DTYPE_BFLOAT16 = 1,
} fr2_dtype_t;

/* Device-detected metadata error bits written to status[0]
 * (replaces the MetadataError enum, csrc/validation/recurrent_metadata.cu:15-22). */
enum {
  FR2_META_INVALID_ENDPOINT = 1 << 0,
  FR2_META_INVALID_SEQUENCE_RANGE = 1 << 1,
  FR2_META_INVALID_STATE_SLOT = 1 << 2,
  FR2_META_DUPLICATE_STATE_SLOT = 1 << 3,
  FR2_META_INVALID_ACTIVE_COUNT = 1 << 4,
  FR2_META_SEQUENCE_TOO_LONG = 1 << 5,
};

/* Library ABI version (major*10000 + minor*100 + patch). */
int fr2_abi_version(void);

/* Static text for an fr2_status_t value. */
const char* fr2_status_string(int status);

/*
 * Text of the last failure in this thread: the HIP error of a failing
 * launch, or the reason an entry rejected its arguments where it gives one
 * ("" if none).  Reading it clears it.
 */
const char* fr2_last_error(void);

/*
 * Count of chunked-kernel blocks that failed closed since the last reset on
 * the current device: a wave hand-off wait inside the block gave up, so the
 * block wrote NaN outputs and left its state untouched.  Waits for `stream`.
 * No counterpart in the reference (its kernels have no bounded waits); the
 * fail-closed result mirrors the metadata path
 * (csrc/validation/recurrent_metadata.cu:24-132).
 */
int fr2_handoff_fault_count(int32_t* count, int32_t reset, void* stream);

/*
 * Test hook: polls a hand-off wait makes before giving up, for later launches
 * (negative: the default 2^20).  No counterpart in the reference.
 */
int fr2_debug_set_handoff_spin_limit(int32_t polls);

/*
 * Test hook: while on (non-zero), the chunked kernel's key waves never
 * publish their operators, so each block's state waves stall at their first
 * operator wait and, after the spin limit, the block fails closed.  Forces a
 * real stall from the host while every kernel still runs to its end.  No
 * counterpart in the reference.
 */
int fr2_debug_set_handoff_stall(int32_t on);

/*
 * Test hook: selects the variant of the workgroup-per-unit chunked kernel
 * that the plain fp32-state contract runs, for later launches in the
 * process: 0 = two key waves per chunk (each a key half, partial token-token
 * blocks summed through LDS), 1 = one key wave per whole chunk over a ring
 * of four chunk operator blocks (the default).  The ring variant serves the
 * plain fp32-state contract and the sequence split's real passes; chunk
 * lists, segment ends, boundary snapshots, sa / read-out outputs and the
 * bf16-state entry always run the key-half variant.  No counterpart in the
 * reference.
 */
int fr2_debug_set_chunk_ring(int32_t on);

/*
 * Device-side validation of packed metadata, one 256-thread workgroup.
 * Writes status[3]; copies query_start_loc/state_indices into the snapshot
 * buffers when they are non-null (static tickets) and validates the copies.
 * num_active_tokens / num_active_sequences (device int32[1], nullable) make it
 * the live graph form: only the active prefix is checked.
 * seen_slots is a caller workspace of state_pool_size int32 (initialised by
 * the kernel itself, no memset node).
 * Replaces prepare_recurrent_metadata_cuda / prepare_recurrent_graph_metadata_cuda
 * (csrc/validation/recurrent_metadata.cu:24-132, :196-225).
 */
int fr2_wkv7_prepare_metadata(const int32_t* query_start_loc,
                              const int32_t* state_indices,
                              int32_t num_sequences, int32_t total_tokens,
                              int32_t state_pool_size, int32_t max_seqlen,
                              const int32_t* num_active_tokens,
                              const int32_t* num_active_sequences,
                              int32_t* status, int32_t* seen_slots,
                              int32_t* query_start_loc_snapshot,
                              int32_t* state_indices_snapshot, void* stream);

/*
 * Packed varlen recurrence with an fp32 state pool updated in place at
 * state_indices.  `status` is the validated ticket status (required): a
 * non-zero status[0] makes every output element NaN and leaves the pool
 * untouched; sequences at or beyond status[2] are skipped.  max_seqlen <= 0
 * means "unknown" (general kernel).  head_size in {64, 128, 256}.
 * The kernel family (decode / token-serial / chunked MFMA) is chosen
 * internally from (head_size, num_sequences, max_seqlen).
 * Replaces tmix_wkv7_recurrent_fp32_from_decay_logits_cuda
 * (csrc/sm120/tmix/wkv7/infer_recurrent_fp32io16_forward_varlen.cu:457-517).
 */
int fr2_wkv7_recurrent_fp32_forward(
    const int32_t* query_start_loc, const int32_t* state_indices,
    const int32_t* status, int32_t num_sequences, int32_t num_heads,
    int32_t head_size, int64_t total_tokens, int32_t max_seqlen, int32_t dtype,
    float* state, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a,
    const void* b, void* output, float scale, void* stream);

/*
 * Same contract, but the kernel family is forced: 0 = token-serial,
 * 1 = decode (state streaming), 2 = chunked MFMA, one workgroup per
 * (sequence, head), 4 = chunked MFMA, one wavefront per (sequence, head)
 * (2 and 4: head_size 64 only).
 * Used by tests and benchmarks to pin each kernel against the oracle.
 * Has no reference counterpart (the reference's dispatch is internal,
 * README.md:81-85); it exposes the same kernels as the entry above.
 */
int fr2_wkv7_recurrent_fp32_forward_kernel(
    int32_t kernel, const int32_t* query_start_loc,
    const int32_t* state_indices, const int32_t* status,
    int32_t num_sequences, int32_t num_heads, int32_t head_size,
    int64_t total_tokens, int32_t max_seqlen, int32_t dtype, float* state,
    const void* r, const void* decay_logits, const void* decay_bias,
    const void* k, const void* v, const void* a, const void* b, void* output,
    float scale, void* stream);

/*
 * The kernel family fr2_wkv7_recurrent_fp32_forward picks for a launch of
 * this shape, written to *kernel: 0 = token-serial, 1 = decode, 2 = chunked
 * MFMA with one workgroup per (sequence, head), 4 = chunked MFMA with one
 * wavefront per (sequence, head), 5 = the same in longest-first order of the
 * sequences.  Pure host computation (no device access, no state), so
 * benchmarks and tests name the kernel that ran without restating the
 * policy.  No reference counterpart: it reports the choice that replaces
 * use_small_auto (csrc/sm120/tmix/wkv7/infer_recurrent_fp32io16_forward_varlen.cu:378-391).
 */
int fr2_wkv7_recurrent_fp32_dispatch(int32_t num_sequences, int32_t num_heads,
                                     int32_t head_size, int64_t total_tokens,
                                     int32_t max_seqlen, int32_t* kernel);

/*
 * Sequence-split plan for the chunked prefill (head_size 64).  With few
 * (sequence, head) units one block per unit leaves most of the GPU idle; the
 * plan cuts every sequence into up to *pieces pieces: piece 0 of *lead_len
 * tokens, the others of *piece_len tokens (multiples of 32; a sequence's last
 * piece is shorter), and reports the device workspace
 * fr2_wkv7_recurrent_fp32_forward_split needs.  The plan is the pipelined
 * split (see below): 256/units + 1 pieces, piece 0 about 1.2x the others.
 * *pieces is 1 when splitting does not pay (more than 128 units, or pieces
 * shorter than 384 tokens).  No reference counterpart: the reference runs
 * one CUDA block per (sequence, head) in launch_recurrent_fp32
 * (csrc/sm120/tmix/wkv7/infer_recurrent_fp32io16_forward_varlen.cu:393-453).
 */
int fr2_wkv7_recurrent_fp32_split_plan(int32_t num_sequences, int32_t num_heads,
                                       int32_t head_size, int32_t max_seqlen,
                                       int32_t* pieces, int32_t* piece_len,
                                       int32_t* lead_len, int64_t* workspace_bytes);

/*
 * fr2_wkv7_recurrent_fp32_forward with the sequence split of a plan (same
 * results within fp32 rounding).  A summary pass computes a piece's
 * zero-start final state F and its transition Phi (identity start, V = 0), a
 * combine kernel chains S(j+1) = Phi_j S(j) + F_j, and the chunked kernel
 * runs each piece from its start state; the last piece of each sequence
 * writes the slot.
 *   lead_len == 0 (classic): pieces of piece_len tokens; summaries of pieces
 *     0..P-2, the chain starts from the slot state, then every piece runs.
 *   lead_len > 0 (pipelined): piece 0 has lead_len tokens and runs from the
 *     slot state on aux_stream, concurrently with the summaries of pieces
 *     1..P-2 on stream (events order the two streams; under graph capture
 *     aux_stream joins the capture); the chain starts from piece 0's end
 *     state, then pieces 1..P-1 run.  aux_stream NULL runs piece 0 on stream
 *     too (same results, no overlap).
 * workspace: device memory of at least the plan's workspace_bytes, owned by
 * the caller, not read after the call's kernels finish.  Replaces, for long
 * sequences, the single-block-per-(sequence, head) launch of
 * tmix_wkv7_recurrent_fp32_from_decay_logits (…fp32io16_forward_varlen.cpp:330-387).
 */
int fr2_wkv7_recurrent_fp32_forward_split(
    const int32_t* query_start_loc, const int32_t* state_indices,
    const int32_t* status, int32_t num_sequences, int32_t num_heads,
    int32_t head_size, int64_t total_tokens, int32_t max_seqlen, int32_t dtype,
    float* state, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a,
    const void* b, void* output, float scale, int32_t pieces, int32_t piece_len,
    int32_t lead_len, void* workspace, int64_t workspace_bytes, void* stream,
    void* aux_stream);

/*
 * The packed fp32-state recurrence with wkv_prepare's kk / a-gate stage
 * fused into the chunked kernel's load stage (fp16 or bf16 tokens,
 * head_size 64).  Inputs: r, decay_logits, v as for
 * fr2_wkv7_recurrent_fp32_forward; k the projected key (before the gate);
 * a12 the low-rank a-gate logits [total_tokens, H, 64]; k_k, a0, k_a the
 * per-channel parameters [H * 64].  Per (token, head) the kernel forms
 *   u = k k_k, kk = u / max(|u|, 1e-12), g = sigmoid(a0 + a12),
 *   key = k (1 + (g - 1) k_a), a = -kk, b = kk g
 * in fp32, runs the recurrence on (key, a, b) and writes key to new_k (the
 * readout's input); a and b are never stored.  Runs on the chunked kernel
 * fr2_wkv7_recurrent_fp32_forward would pick for this launch (one workgroup
 * or one wavefront per (sequence, head)).  Where that entry would run the
 * decode kernel (max_seqlen <= 4, or <= 6 with 16 384 or more units; or
 * max_seqlen <= 0, unknown), bf16 tokens run on the wavefront chunked kernel
 * and fp16 tokens return FR2_ERR_UNSUPPORTED, as does head_size != 64: the
 * caller then runs fr2_tmix_kk_a_gate_forward (fp16) and
 * fr2_wkv7_recurrent_fp32_forward.  Replaces
 * the pair tmix_kk_a_gate_forward_varlen_cuda
 * (csrc/sm120/tmix/wkv_prepare/internal/kk_a_gate/infer_fp16_forward_varlen.cu)
 * + tmix_wkv7_recurrent_fp32_from_decay_logits_cuda
 * (…/infer_recurrent_fp32io16_forward_varlen.cu:457-517), which the reference
 * runs as two kernels with k, a, b round-tripping through HBM.
 */
int fr2_wkv7_recurrent_fp32_forward_kk_gate(
    const int32_t* query_start_loc, const int32_t* state_indices, const int32_t* status,
    int32_t num_sequences, int32_t num_heads, int32_t head_size, int64_t total_tokens,
    int32_t max_seqlen, int32_t dtype, float* state, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a12, const void* k_k,
    const void* a0, const void* k_a, void* new_k, void* output, float scale, void* stream);

/*
 * fr2_wkv7_recurrent_fp32_forward_kk_gate with the readout's elementwise
 * stage fused into the output write-back: per (token, head),
 *   readout = (GroupNorm(y) * ln_weight + ln_bias + (sum_c r k' r_k) v) * g
 * with GroupNorm over the head's channels of y as rounded to the token dtype
 * (eps 64e-5), k' the gated key as stored, r_k / ln_weight / ln_bias of
 * shape [H*D] and g [total_tokens, H, D] in the token dtype.  `readout`
 * receives it; `output` (y) is written only when not null.  Replaces the
 * triple tmix_kk_a_gate_forward_varlen_cuda
 * (csrc/sm120/tmix/wkv_prepare/internal/kk_a_gate/infer_fp16_forward_varlen.cu),
 * tmix_wkv7_recurrent_fp32_from_decay_logits_cuda
 * (…/infer_recurrent_fp32io16_forward_varlen.cu:457-517) and
 * tmix_lnx_rkvres_xg_forward_varlen_cuda
 * (csrc/sm120/tmix/readout/infer_fp16_forward_varlen.cu), which the reference
 * runs as three kernels with k, a, b and y round-tripping through HBM.
 * Same FR2_ERR_UNSUPPORTED cases as the kk-gate entry.
 */
int fr2_wkv7_recurrent_fp32_forward_kk_gate_readout(
    const int32_t* query_start_loc, const int32_t* state_indices, const int32_t* status,
    int32_t num_sequences, int32_t num_heads, int32_t head_size, int64_t total_tokens,
    int32_t max_seqlen, int32_t dtype, float* state, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a12, const void* k_k,
    const void* a0, const void* k_a, const void* g, const void* r_k, const void* ln_weight,
    const void* ln_bias, void* new_k, void* readout, void* output, float scale, void* stream);

/*
 * fr2_wkv7_recurrent_fp32_forward_split without a workspace argument: the
 * library's own device scratch array (FR2_NOALLOC_SCRATCH_BYTES per GPU, held
 * until the process ends) replaces it, and the call allocates nothing (no
 * hipMalloc/hipFree, no allocating library routine) and runs every pass on
 * `stream`.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  A plan whose workspace exceeds the
 * scratch (num_sequences * (3 pieces - 2) * num_heads * 16 KiB bytes) is
 * rejected with FR2_ERR_INVALID_ARGUMENT and an fr2_last_error() text.
 * Every call on one GPU shares that GPU's scratch: calls that overlap on one
 * GPU (two streams, two threads) race.
 */
#define FR2_NOALLOC_SCRATCH_BYTES (16ll << 20)
int fr2_wkv7_recurrent_fp32_forward_split_noalloc(
    const int32_t* query_start_loc, const int32_t* state_indices, const int32_t* status,
    int32_t num_sequences, int32_t num_heads, int32_t head_size, int64_t total_tokens,
    int32_t max_seqlen, int32_t dtype, float* state, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a, const void* b,
    void* output, float scale, int32_t pieces, int32_t piece_len, int32_t lead_len,
    void* stream);

/*
 * Packed varlen recurrence with an FP16 state pool [slots,H,D,D] updated in
 * place (the "Albatross" FP16-state contract, fp16 token tensors only):
 *   delta  = fp16(w - 1 + dither(phase)),
 *   dither = int32(0x9E3779B9 * phase mod 2^32) * 2^-41,
 *   phase  = elapsed_state[slot] + h*D + key + token offset in the sequence,
 *   S      = fp16(S + S*delta + b*sa + k*v^T) after every token (fp32 math),
 *   y      = fp16(scale * S^T r) from the rounded state.
 * Afterwards elapsed_state[slot] += sequence length for every active
 * sequence (enqueued on the same stream).  A non-zero status[0] makes every
 * output element NaN and leaves the pool and the elapsed counts untouched.
 * head_size in {64, 128, 256}.
 * Replaces tmix_wkv7_recurrent_fp16_from_decay_logits_cuda and
 * recurrent_fp16_advance_i32_varlen_cuda
 * (csrc/sm120/tmix/wkv7/infer_recurrent_fp16_forward_varlen.cpp:121-187,
 *  infer_recurrent_fp16_forward_varlen.cu:60-75, :243-336).
 */
int fr2_wkv7_recurrent_fp16_forward(
    const int32_t* query_start_loc, const int32_t* state_indices,
    const int32_t* status, int32_t* elapsed_state, int32_t num_sequences,
    int32_t num_heads, int32_t head_size, int64_t total_tokens,
    int32_t max_seqlen, void* state_f16, const void* r,
    const void* decay_logits, const void* decay_bias, const void* k,
    const void* v, const void* a, const void* b, void* output, float scale,
    void* stream);

/*
 * The two halves of fr2_wkv7_recurrent_fp16_forward, as the reference splits
 * them: the state update and outputs (reads elapsed_state for the dither
 * phase, does not advance it) replaces tmix_wkv7_recurrent_fp16_from_decay_logits_cuda,
 * and the elapsed advance (elapsed_state[slot] += sequence length for every
 * active sequence) replaces recurrent_fp16_advance_i32_varlen_cuda
 * (csrc/sm120/tmix/wkv7/infer_recurrent_fp16_forward_varlen.cpp:121-187).
 * Calling the first, then the second, on one stream equals the combined entry.
 */
int fr2_wkv7_recurrent_fp16_update(
    const int32_t* query_start_loc, const int32_t* state_indices,
    const int32_t* status, const int32_t* elapsed_state, int32_t num_sequences,
    int32_t num_heads, int32_t head_size, int64_t total_tokens,
    int32_t max_seqlen, void* state_f16, const void* r,
    const void* decay_logits, const void* decay_bias, const void* k,
    const void* v, const void* a, const void* b, void* output, float scale,
    void* stream);
/*
 * fr2_wkv7_recurrent_fp16_update with the kernel forced: 0 = the token-serial
 * workgroup kernel (a barrier per token; every head size), 1 = the decode
 * kernel (head_size 64), 6 = the barrier-free token-serial kernel (head_size
 * 64; bit-identical to 0 at 256 or fewer (sequence, head) units).  Used by
 * tests and benchmarks to pin each kernel; no reference counterpart (the
 * reference's family selection is internal).
 */
int fr2_wkv7_recurrent_fp16_update_kernel(
    int32_t kernel, const int32_t* query_start_loc, const int32_t* state_indices,
    const int32_t* status, const int32_t* elapsed_state, int32_t num_sequences,
    int32_t num_heads, int32_t head_size, int64_t total_tokens,
    int32_t max_seqlen, void* state_f16, const void* r,
    const void* decay_logits, const void* decay_bias, const void* k,
    const void* v, const void* a, const void* b, void* output, float scale,
    void* stream);
int fr2_wkv7_recurrent_fp16_advance_elapsed(const int32_t* query_start_loc,
                                            const int32_t* state_indices,
                                            const int32_t* status, int32_t* elapsed_state,
                                            int32_t num_sequences, void* stream);

/*
 * [B,T,H,D] bf16 training forward with zero initial state.  Writes y (bf16),
 * state_dot_a [B,T,H,D] fp32 (the pre-update sa of every token) and
 * boundary [B,H,T/16,D,D] fp32, the post-chunk state after every 16 tokens.
 * Requires T % 16 == 0.
 * Replaces forward / cuda_forward_v3
 * (csrc/sm120/tmix/wkv7/pretrain_recurrent_bf16_forward.cpp:20-27,
 *  pretrain_recurrent_bf16_forward.cu:32-101).
 */
int fr2_wkv7_pretrain_forward(int32_t batch, int32_t tokens, int32_t num_heads,
                              int32_t head_size, const void* r, const void* w,
                              const void* k, const void* v, const void* a,
                              const void* b, void* output, float* boundary,
                              float* state_dot_a, void* stream);

/*
 * Training backward of fr2_wkv7_pretrain_forward: gradients (bf16,
 * [B,T,H,D]) of sum(y * grad_output) with respect to r, the decay logits w,
 * k, v, a and b.  boundary and state_dot_a are the forward's outputs.
 * workspace holds fr2_wkv7_pretrain_backward_workspace_floats(...) floats
 * (the per-token gradient of sa, and at D = 64 the value pass's snapshots of
 * dL/dS every few chunks); it needs no initialisation.  Kernels on `stream`.
 * Requires T % 16 == 0.
 * Replaces backward / cuda_backward_v3 / cuda_backward_split /
 * cuda_backward_tiled256
 * (csrc/sm120/tmix/wkv7/pretrain_recurrent_bf16_forward.cpp:29-46,
 *  pretrain_recurrent_bf16_forward.cu:163-486).
 */
/*
 * fp32 elements of fr2_wkv7_pretrain_backward's workspace, or -1 for sizes
 * that entry rejects.  No reference counterpart: the reference allocates its
 * N = 256 workspace inside the binding
 * (csrc/sm120/tmix/wkv7/pretrain_recurrent_bf16_forward.cpp:40-44).
 */
int64_t fr2_wkv7_pretrain_backward_workspace_floats(int32_t batch, int32_t tokens,
                                                    int32_t num_heads, int32_t head_size);

int fr2_wkv7_pretrain_backward(int32_t batch, int32_t tokens, int32_t num_heads,
                               int32_t head_size, const void* r, const void* w,
                               const void* k, const void* v, const void* a,
                               const void* b, const void* grad_output,
                               const float* boundary, const float* state_dot_a,
                               float* workspace, void* grad_r, void* grad_w,
                               void* grad_k, void* grad_v, void* grad_a, void* grad_b,
                               void* stream);

/*
 * Packed varlen recurrence with a bf16 state pool [slots,H,64,64] updated in
 * place (fp32 carry inside the call, rounded to bf16 on store).
 * Replaces infer_tmix_wkv7_chunk_bf16_forward_varlen_cuda
 * (csrc/sm120/tmix/wkv7/infer_chunk_bf16_forward_varlen.cu:276-340,
 *  binding infer_chunk_bf16_forward_varlen.cpp:77-192).
 */
int fr2_wkv7_chunk_bf16_forward(
    const int32_t* query_start_loc, const int32_t* state_indices,
    const int32_t* status, int32_t num_sequences, int32_t num_heads,
    int64_t total_tokens, int32_t chunk_size, int32_t max_seqlen,
    uint16_t* state_bf16, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a,
    const void* b, void* output, float scale, void* stream);

/*
 * fr2_wkv7_chunk_bf16_forward with the sequence split of
 * fr2_wkv7_recurrent_fp32_split_plan (head_size 64): the same passes, classic
 * or pipelined, as fr2_wkv7_recurrent_fp32_forward_split; the bf16 slot state
 * is widened once (by the combine kernel, or by piece 0 in the pipelined
 * split) and rounded once by each sequence's last piece.  Replaces,
 * for few long sequences, the one-block-per-(sequence, head) launch of
 * infer_tmix_wkv7_chunk_bf16_forward_varlen_cuda
 * (…/infer_chunk_bf16_forward_varlen.cu:276-340).
 */
int fr2_wkv7_chunk_bf16_forward_split(
    const int32_t* query_start_loc, const int32_t* state_indices,
    const int32_t* status, int32_t num_sequences, int32_t num_heads,
    int64_t total_tokens, int32_t chunk_size, int32_t max_seqlen,
    uint16_t* state_bf16, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a,
    const void* b, void* output, float scale, int32_t pieces, int32_t piece_len,
    int32_t lead_len, void* workspace, int64_t workspace_bytes, void* stream,
    void* aux_stream);

/*
 * RL/Infctx fp32-state chunked forward over chunk metadata
 * (sequence_chunk_offsets [N+1], chunk_token_starts/ends [C]).  `state` is the
 * working pool [N,H,D,D] (slot i = sequence i), updated in place to the final
 * states.  strategy 0 = materialized, 1 = recompute; chunk_size in {16,32,64}.
 * Replaces rl_infctx_tmix_wkv7_chunk_fp32io16_forward's kernels
 * (csrc/sm120/tmix/wkv7/rl_infctx_chunk_fp32io16_forward.cpp:158-230,
 *  rl_infctx_chunk_fp32io16_forward.cu:42-135, :318-539).
 */
int fr2_wkv7_rl_infctx_forward(
    const int32_t* sequence_chunk_offsets, const int32_t* chunk_token_starts,
    const int32_t* chunk_token_ends, int32_t num_sequences, int32_t num_chunks,
    int32_t num_heads, int32_t head_size, int64_t total_tokens,
    int32_t max_seqlen, int32_t chunk_size, int32_t strategy, int32_t dtype,
    float* state, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a,
    const void* b, void* output, float scale, void* stream);

/*
 * Replays chunks [chunk_token_starts[c], chunk_token_ends[c]) from the
 * start-of-chunk states boundary[c] ([C,H,D,D] fp32, read only) and writes
 * output and state_dot_a ([total_tokens,H,D] fp32) for those tokens.
 * Replaces rl_infctx_tmix_wkv7_chunk_fp32io16_backward_replay_cuda
 * (csrc/sm120/tmix/wkv7/rl_infctx_chunk_fp32io16_backward.cu:45-126,
 *  binding rl_infctx_chunk_fp32io16_backward.cpp:100-125).
 */
int fr2_wkv7_rl_infctx_replay(const int32_t* chunk_token_starts,
                              const int32_t* chunk_token_ends,
                              int32_t num_chunks, int32_t num_heads,
                              int32_t head_size, int64_t total_tokens,
                              int32_t dtype, const float* boundary,
                              const void* r, const void* decay_logits,
                              const void* decay_bias, const void* k,
                              const void* v, const void* a, const void* b,
                              void* output, float* state_dot_a, float scale,
                              void* stream);

/* ------------------------------------------------------------------------
 * StateTune: the recurrence from a trainable fp32 initial state over a chunk
 * list, and its training backward.
 *
 * Sequence s runs chunks sequence_chunk_offsets[s] .. [s+1]-1 in order;
 * chunk c covers token rows [chunk_token_starts[c], chunk_token_ends[c]) of
 * the packed [total_tokens, H, D] tensors (fp16 or bf16, one dtype for all).
 * Chunks must not overlap; rows outside every chunk are not written.
 * ---------------------------------------------------------------------- */

/*
 * Forward: state [B,H,D,D] fp32 holds the initial state on entry and the
 * final state on return.  Writes output = scale * S_t^T r_t (token dtype),
 * state_dot_a [T,H,D] fp32 (pre-update sa) and boundary [C,H,D,D] fp32, the
 * state at the start of every chunk.
 * Replaces statetune_tmix_wkv7_recurrent_fp32io16_forward
 * (csrc/sm120/tmix/wkv7/statetune_recurrent_fp32io16_forward.cpp:26-44,
 *  statetune_recurrent_fp32io16_forward.cu:32-131).
 */
int fr2_wkv7_statetune_forward(const int32_t* sequence_chunk_offsets,
                               const int32_t* chunk_token_starts,
                               const int32_t* chunk_token_ends, int32_t num_sequences,
                               int32_t num_chunks, int64_t total_tokens, int32_t num_heads,
                               int32_t head_size, int32_t dtype, float* state, const void* r,
                               const void* decay_logits, const void* k, const void* v,
                               const void* a, const void* b, void* output, float* boundary,
                               float* state_dot_a, float scale, void* stream);

/*
 * fp32 elements of fr2_wkv7_statetune_backward's workspace, or -1 for sizes
 * it rejects.  No reference counterpart: the reference's backward rebuilds
 * states by dividing by the decay over whole chunks and needs no workspace.
 */
int64_t fr2_wkv7_statetune_backward_workspace_floats(int64_t total_tokens, int32_t num_heads,
                                                     int32_t head_size);

/*
 * Backward: gradients of sum(output * grad_output) + sum(S_final *
 * grad_final_state) with respect to r, decay_logits, k, v, a, b (token dtype,
 * [T,H,D]) and the initial state (grad_initial_state, fp32 [B,H,D,D]).
 * grad_output / grad_final_state may be NULL (zero cotangent); every
 * gradient pointer may be NULL (not written).  state_dot_a and boundary are
 * the forward's outputs; the workspace needs no initialisation.  The
 * reference's final_state argument is not taken: chunk-end states are
 * rebuilt from the boundaries.
 * Replaces statetune_tmix_wkv7_recurrent_fp32io16_backward
 * (csrc/sm120/tmix/wkv7/statetune_recurrent_fp32io16_backward.cpp:34-67,
 *  statetune_recurrent_fp32io16_backward.cu:49-255, 317-502).
 */
int fr2_wkv7_statetune_backward(
    const int32_t* sequence_chunk_offsets, const int32_t* chunk_token_starts,
    const int32_t* chunk_token_ends, int32_t num_sequences, int32_t num_chunks,
    int64_t total_tokens, int32_t num_heads, int32_t head_size, int32_t dtype, const void* r,
    const void* decay_logits, const void* k, const void* v, const void* a, const void* b,
    const float* state_dot_a, const void* grad_output, const float* grad_final_state,
    const float* boundary, float* workspace, void* grad_r, void* grad_decay_logits,
    void* grad_k, void* grad_v, void* grad_a, void* grad_b, float* grad_initial_state,
    float scale, void* stream);

/*
 * StateTune on the chunked MFMA kernels, for the common layout: D = 64, bf16
 * tokens, `batch` sequences of `tokens` rows each, packed back to back
 * ([batch*tokens, H, 64]), each run as tokens / chunk_len chunks of
 * chunk_len rows (chunk_len % 16 == 0).  That is the chunk list
 * sequence_chunk_offsets[s] = s * nck, chunk_token_starts[c] = c * chunk_len,
 * chunk_token_ends[c] = (c + 1) * chunk_len of fr2_wkv7_statetune_forward,
 * with the same outputs, plus `snapshots` [batch, H, tokens/16, 64, 64] fp32:
 * the state after every 16 tokens, which the backward reads.
 * Same reference interface as fr2_wkv7_statetune_forward.
 */
int fr2_wkv7_statetune_uniform_forward(int32_t batch, int32_t tokens, int32_t num_heads,
                                       int32_t chunk_len, float* state, const void* r,
                                       const void* decay_logits, const void* k, const void* v,
                                       const void* a, const void* b, void* output,
                                       float* boundary, float* state_dot_a, float* snapshots,
                                       float scale, void* stream);

/*
 * fp32 elements of fr2_wkv7_statetune_uniform_backward's workspace, or -1.
 * No reference counterpart (see fr2_wkv7_statetune_backward_workspace_floats).
 */
int64_t fr2_wkv7_statetune_uniform_backward_workspace_floats(int32_t batch, int32_t tokens,
                                                             int32_t num_heads);

/*
 * Backward of fr2_wkv7_statetune_uniform_forward (same gradients as
 * fr2_wkv7_statetune_backward; grad_output and every gradient are required,
 * grad_final_state may be NULL).  snapshots are the forward's.
 * Same reference interface as fr2_wkv7_statetune_backward.
 */
int fr2_wkv7_statetune_uniform_backward(
    int32_t batch, int32_t tokens, int32_t num_heads, int32_t chunk_len, const void* r,
    const void* decay_logits, const void* k, const void* v, const void* a, const void* b,
    const float* state_dot_a, const void* grad_output, const float* grad_final_state,
    const float* boundary, const float* snapshots, float* workspace, void* grad_r,
    void* grad_decay_logits, void* grad_k, void* grad_v, void* grad_a, void* grad_b,
    float* grad_initial_state, float scale, void* stream);

/*
 * StateTune over any chunk list (ragged, empty or gapped chunks) at
 * head_size 64 with bf16 tokens, on the chunked MFMA kernels: each
 * sequence's chunks are laid out back to back in a [batch, padded_tokens]
 * token grid (padded_tokens a multiple of 16), every chunk starting on a
 * 16-token boundary, with identity tokens in between (zero r, k, v, a, b and
 * a decay logit of -80, whose retention is 1 in fp32: the state and the
 * adjoint pass them unchanged).  row_source [batch * padded_tokens] maps a
 * grid row to its packed token row, or -1 for an identity row;
 * chunk_seq / chunk_pstart [num_chunks] give each chunk's sequence and its
 * start in the grid.  The caller (the host, from the chunk metadata) builds
 * the three tables.  Outputs as fr2_wkv7_statetune_forward, plus snapshots
 * [batch, H, padded_tokens/16, 64, 64] fp32 for the backward; workspace of
 * fr2_wkv7_statetune_padded_workspace_bytes(..., 0) bytes (16-byte
 * aligned).  Token rows that belong to no chunk are not written.
 * Same reference interface as fr2_wkv7_statetune_forward
 * (csrc/sm120/tmix/wkv7/statetune_recurrent_fp32io16_forward.cpp:26-56).
 */
int64_t fr2_wkv7_statetune_padded_workspace_bytes(int32_t batch, int32_t padded_tokens,
                                                  int32_t num_heads, int32_t backward);
int fr2_wkv7_statetune_padded_forward(
    int32_t batch, int32_t padded_tokens, int32_t num_heads, int32_t num_chunks,
    const int32_t* row_source, const int32_t* chunk_seq, const int32_t* chunk_pstart,
    float* state, const void* r, const void* decay_logits, const void* k, const void* v,
    const void* a, const void* b, void* output, float* boundary, float* state_dot_a,
    float* snapshots, void* workspace, float scale, void* stream);

/*
 * Backward of fr2_wkv7_statetune_padded_forward on the same grid
 * (seq_first_chunk [batch]: each sequence's first chunk, -1 if it has none);
 * grad_output and every gradient are required; workspace of
 * fr2_wkv7_statetune_padded_workspace_bytes(..., 1) bytes.  Gradient rows of
 * tokens that belong to no chunk are not written.
 * Same reference interface as fr2_wkv7_statetune_backward
 * (csrc/sm120/tmix/wkv7/statetune_recurrent_fp32io16_backward.cpp:34-82).
 */
int fr2_wkv7_statetune_padded_backward(
    int32_t batch, int32_t padded_tokens, int32_t num_heads, const int32_t* row_source,
    const int32_t* seq_first_chunk, const void* r, const void* decay_logits, const void* k,
    const void* v, const void* a, const void* b, const float* state_dot_a,
    const void* grad_output, const float* grad_final_state, const float* boundary,
    const float* snapshots, void* workspace, void* grad_r, void* grad_decay_logits,
    void* grad_k, void* grad_v, void* grad_a, void* grad_b, float* grad_initial_state,
    float scale, void* stream);

/* ------------------------------------------------------------------------
 * Producer and consumer stages of the WKV7 path (fp16 tensors, fp32 math).
 * ---------------------------------------------------------------------- */

/*
 * Key / a-gate stage: per (token, head) of [tokens, H*D] fp16 rows,
 *   u = k * k_k, kk = u / max(|u|, 1e-12), a = sigmoid(a0 + a12),
 *   new_k = k * (1 + (a - 1) * k_a), neg_kk = -kk, kka = kk * a,
 * with k_k, a0, k_a of shape [H*D].  Replaces tmix_kk_a_gate_forward_varlen_cuda
 * (csrc/sm120/tmix/wkv_prepare/internal/kk_a_gate/infer_fp16_forward_varlen.cu,
 *  called from csrc/sm120/tmix/wkv_prepare/infer_fp16_forward_varlen.cpp:520-528).
 */
int fr2_tmix_kk_a_gate_forward(int64_t tokens, int32_t num_heads, int32_t head_size,
                               const void* k, const void* k_k, const void* a0,
                               const void* a12, const void* k_a, void* new_k,
                               void* neg_kk, void* kka, void* stream);

/*
 * Low-rank branch activations: tanh_out = tanh(tanh_in) over n_tanh values
 * and sigmoid_out = sigmoid(sigmoid_in) over n_sigmoid values (fp16, one
 * launch).  Replaces lowrank_tanh_f16_cuda / lowrank_sigmoid_f16_cuda
 * (csrc/sm120/tmix/wkv_prepare/internal/lowrank/infer_fp16_forward_varlen.cu:423-448).
 */
int fr2_tmix_lowrank_activate(int64_t n_tanh, const void* tanh_in, void* tanh_out,
                              int64_t n_sigmoid, const void* sigmoid_in, void* sigmoid_out,
                              void* stream);

/*
 * Value residual of later layers over [tokens, C] fp16 (C % 8 == 0):
 *   output = value + (v_first - value) * sigmoid(v0 + v12),  v0 of shape [C].
 * Replaces wkv_prepare_vres_forward_varlen_cuda
 * (csrc/sm120/tmix/wkv_prepare/internal/lowrank/infer_vres_fp16_forward_varlen.cu).
 */
int fr2_tmix_vres_forward(int64_t tokens, int32_t channels, const void* value,
                          const void* v_first, const void* v0, const void* v12,
                          void* output, void* stream);

/*
 * Readout before the output projection: per (token, head) of [tokens, H*D]
 * fp16 rows, group norm of the WKV output (eps 64e-5) with ln_weight /
 * ln_bias, plus sum(r * k * r_k) * v, times the gate; fp16 result.
 * Replaces tmix_lnx_rkvres_xg_forward_varlen_cuda
 * (csrc/sm120/tmix/readout/infer_fp16_forward_varlen.cu, called from
 *  csrc/sm120/tmix/readout/infer_fp16_forward_varlen.cpp:44-86).
 */
int fr2_tmix_readout_prelinear_forward(int64_t tokens, int32_t num_heads, int32_t head_size,
                                       const void* wkv_output, const void* r, const void* k,
                                       const void* v, const void* r_k, const void* ln_weight,
                                       const void* ln_bias, const void* gate, void* output,
                                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHRWKV2_AMD_H_ */
