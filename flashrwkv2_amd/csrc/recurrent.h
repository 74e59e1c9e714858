// Segment descriptor shared by every WKV7 kernel, and the launchers.
#pragma once

#include "common.h"
#include "../../include/flashrwkv2_amd.h"

namespace fr2 {

// A launch runs grid (H, num_segments); segment i covers tokens [t0, t1) of
// the packed [total_tokens, H, D] tensors and reads/writes state slot
// `slots[i]` (identity when null).  Segment bounds come from, in order of
// precedence:
//   uniform_len > 0  : [i*L, (i+1)*L)                       ([B,T,H,D] layout)
//   chunk_offsets    : [bounds[co[i]], ends[co[i+1]-1])     (RL/Infctx chunks)
//   ends             : [bounds[i], ends[i])                 (chunk replay)
//   otherwise        : [bounds[i], bounds[i+1])             (cu_seqlens)
struct SegArgs {
  const int32_t* bounds = nullptr;
  const int32_t* ends = nullptr;
  const int32_t* chunk_offsets = nullptr;
  const int32_t* slots = nullptr;
  const int32_t* status = nullptr;  // validated ticket status, or null
  int uniform_len = 0;
  int num_heads = 0;
  int64_t out_elems = 0;            // for the fail-closed NaN fill
  const void* state_in = nullptr;   // null: zero initial state
  void* state_out = nullptr;        // null: final state not written
  bool state_bf16 = false;          // chunked kernel: state_in/out hold bf16
  const void* r = nullptr;
  const void* logits = nullptr;
  const void* bias = nullptr;       // [H, D] or null
  const void* k = nullptr;
  const void* v = nullptr;
  const void* a = nullptr;
  const void* b = nullptr;
  void* y = nullptr;
  float* sa_out = nullptr;          // per-token pre-update sa, or null
  float* boundary = nullptr;        // post-chunk state snapshots, or null
  int boundary_len = 16;
  int boundary_per_seg = 0;
  float scale = 1.0f;
  // FP16-state (Albatross) mode: per-slot elapsed token counts (the dither
  // phase base); null for every other mode
  const int32_t* elapsed = nullptr;
  // Reverse mode of the chunked kernel (the training backward's value pass):
  // position p of a segment [t0, t1) reads token row t1-1-p, plus one row for
  // tensor j when bit j of shift_mask is set (tensors r, logits, k, v, a, b
  // = bits 0..5); a shifted row past t1-1 reads as zero operands with unit
  // retention.  y rows go to t1-1-p, sa rows to t0 + (n-p) mod n (n = t1-t0)
  // and the snapshot after chunk c to index boundary_per_seg-1-c.
  bool reverse = false;
  int shift_mask = 0;
  // reverse mode: factor on the k operand (the value pass's r_t), i.e. the
  // forward's output scale
  float kv_scale = 1.0f;
  // with boundary set: keep only the snapshots whose index is a multiple of
  // boundary_every, at index / boundary_every
  int boundary_every = 1;
  // Sequence split of the chunked kernel (few long sequences).  Sequence n
  // is cut into pieces of split_len tokens (the last one shorter); piece j
  // covers [q0 + j*split_len, min(q0 + (j+1)*split_len, q1)).
  //   real pass (split_pieces > 0, grid y = N * split_pieces): piece j of
  //     sequence n is segment n*split_pieces + j; it starts from the slot
  //     state (j = 0) or from split_state[(n*split_pieces + j), H, D, D],
  //     and only the sequence's last piece writes the slot;
  //   summary pass (chunk64_kernel with kSum): see launch_split_summary.
  int split_pieces = 0;
  int split_len = 0;
  float* split_state = nullptr;
  float* split_summary = nullptr;
  // Pipelined ("lead") split: piece 0 has split_lead tokens (0: split_len)
  // and pieces j >= 1 cover [q0 + lead + (j-1)*split_len, ...).  A launch's
  // grid covers pieces split_first .. split_first + split_count - 1 of every
  // sequence (split_count 0: every piece, or every piece but the last in the
  // summary pass).  split_lead_pass: piece 0 starts from the slot state and,
  // unless it is the sequence's last piece, hands its end state to
  // split_state[n * split_pieces + 1].
  int split_lead = 0;
  int split_first = 0;
  int split_count = 0;
  bool split_lead_pass = false;
  // Bounded waits of the chunked kernel's wave hand-off: polls before a wait
  // gives up, and the device word that counts blocks that gave up (the block
  // then fails closed: NaN outputs, state untouched)
  int spin_limit = 1 << 20;
  int* handoff_fault = nullptr;
  // test hook: the key waves never publish their operators, so the state
  // waves' waits give up (forces a real stall from the host)
  bool handoff_stall = false;
  // Fused kk / a-gate producer stage (chunked kernel only): `k` holds the
  // projected key, `a` the low-rank a-gate logits a12, `b` is unused; per
  // channel k_k, a0, k_a ([H, D]); the gated key is written to new_k.
  const void* kk_scale = nullptr;
  const void* a_bias = nullptr;
  const void* k_a = nullptr;
  void* new_k = nullptr;
  // Fused readout prelinear stage (chunked kernel with the kk / a gate):
  // per (token, head) out = (GroupNorm(y) * ln_w + ln_b + (sum r k' r_k) v) * g
  // over the head's channels, written to ro_out ([T, H, D], token dtype);
  // ro_g is the gate [T, H, D], r_k / ln_w / ln_b are [H, D].  y itself is
  // written only when `y` is set.
  const void* ro_g = nullptr;
  const void* ro_rk = nullptr;
  const void* ro_lnw = nullptr;
  const void* ro_lnb = nullptr;
  void* ro_out = nullptr;
};

// Token range [t0, t1) and state slot of segment `seg` (see SegArgs).
__device__ __forceinline__ bool resolve_segment(const SegArgs& p, int seg,
                                                int& t0, int& t1, int& slot) {
  if (p.uniform_len > 0) {
    t0 = seg * p.uniform_len;
    t1 = t0 + p.uniform_len;
  } else if (p.chunk_offsets != nullptr) {
    const int c0 = p.chunk_offsets[seg];
    const int c1 = p.chunk_offsets[seg + 1];
    t0 = p.bounds[c0];
    t1 = p.ends[c1 - 1];
  } else if (p.ends != nullptr) {
    t0 = p.bounds[seg];
    t1 = p.ends[seg];
  } else {
    t0 = p.bounds[seg];
    t1 = p.bounds[seg + 1];
  }
  slot = p.slots ? p.slots[seg] : seg;
  return true;
}

// Token range [start, start + len) of piece j of a split sequence of n
// tokens, and the index of the sequence's last piece.
__host__ __device__ inline void split_piece(const SegArgs& p, int n, int j, int& start,
                                            int& len, int& last) {
  const int lead = p.split_lead > 0 ? p.split_lead : p.split_len;
  last = n <= lead ? 0 : 1 + (n - lead - 1) / p.split_len;
  start = j == 0 ? 0 : lead + (j - 1) * p.split_len;
  len = j == 0 ? lead : p.split_len;
}

int launch_serial(int D, int dtype, bool bf16_state, const SegArgs& p, int nseg,
                  hipStream_t s);
int launch_decode(int D, int dtype, const SegArgs& p, int nseg, hipStream_t s);
// FP16 state pool with the Albatross delta update (fp16 tokens), followed by
// the elapsed-count advance of every active sequence's slot.
// family: -1 the policy; kFp16Serial (serial_kernel), kFp16Decode (D = 64),
// kFp16SerialWave (D = 64, barrier-free)
constexpr int kFp16Serial = 0, kFp16Decode = 1, kFp16SerialWave = 6;
int launch_fp16_state(int D, const SegArgs& p, int nseg, int max_seqlen, int32_t* elapsed,
                      hipStream_t s, bool advance, int family = -1);
// elapsed[slot] += length for every active sequence (after the update)
int launch_advance_elapsed(const SegArgs& p, int nseg, int32_t* elapsed, hipStream_t s);
// Chunked MFMA prefill (D = 64, fp32 state).  Returns FR2_ERR_UNSUPPORTED
// for contracts it does not cover (sa output / boundaries / bf16 state).
// The chunked kernel with the kk / a-gate stage fused into its load stage
// (p.kk_scale, p.a_bias, p.k_a, p.new_k set).
int launch_chunked_kk(int dtype, const SegArgs& p, int nseg, hipStream_t s);
int launch_chunked(int dtype, const SegArgs& p, int nseg, int max_seqlen,
                   hipStream_t s);
// The chunked prefill with one wavefront per (sequence, head) unit (plain
// contract: no sa / boundary outputs, fp32 state), for launches with many
// units.
int launch_chunked_wave(int dtype, const SegArgs& p, int nseg, int max_seqlen, hipStream_t s);
// Whether that kernel runs its units in longest-first order of their
// sequences (packed plain batches: few sequences, one long one).
bool wave_longest_first(int nseg, int max_seqlen, int64_t total_tokens);
// Sequence-split chunked prefill (D = 64, fp32 state, plain contract):
// `pieces` pieces per sequence, of `piece_len` tokens except piece 0, which
// has lead_len tokens when lead_len > 0 (the pipelined split: piece 0 runs on
// `aux` concurrently with the summary pass; aux null runs it on s).
// workspace holds split_workspace_floats(nseg, H, pieces) floats.
int64_t split_workspace_floats(int nseg, int H, int pieces);
// Device address of the current device's hand-off fault counter (null if the
// symbol lookup failed) and the spin limit every chunked launch uses.
int* handoff_fault_word();
int handoff_spin_limit();
void set_handoff_spin_limit(int polls);   // negative: the default
bool handoff_stall();
void set_handoff_stall(bool on);
bool chunk_ring_enabled();
void set_chunk_ring(int on);
int launch_chunked_split(int dtype, SegArgs p, int nseg, int pieces, int piece_len,
                         int lead_len, float* workspace, hipStream_t s, hipStream_t aux);

// Training backward of the [B,T,H,D] zero-state path: bf16 token tensors and
// gradients, the forward's fp32 boundary [B,H,T/16,D,D] and state_dot_a
// [B,T,H,D], and an fp32 [B,T,H,D] workspace that carries dsa from the value
// pass to the key pass.
struct PretrainBwdArgs {
  int batch = 0, tokens = 0, heads = 0;
  const void *r = nullptr, *w = nullptr, *k = nullptr, *v = nullptr, *a = nullptr,
             *b = nullptr, *dy = nullptr;
  const float* boundary = nullptr;
  const float* state_dot_a = nullptr;
  float* workspace = nullptr;
  void *dr = nullptr, *dw = nullptr, *dk = nullptr, *dv = nullptr, *da = nullptr,
       *db = nullptr;
  // StateTune at D = 64 (uniform layout): y = scale * S^T r, the start state
  // of each sequence (state0 + b * state0_stride, [H,D,D]), dL/dS_final
  // [B,H,D,D], the output dL/dS_initial [B,H,D,D] and an fp32 [B,H,D,D]
  // buffer for dL/dS at each sequence's first token; null / 1 for pretrain
  float scale = 1.0f;
  const float* state0 = nullptr;
  int64_t state0_stride = 0;
  const float* dfinal = nullptr;
  float* dstate0 = nullptr;
  float* pfirst = nullptr;
};
int launch_pretrain_backward(int D, const PretrainBwdArgs& p, hipStream_t s);
// fp32 elements of the backward's workspace: dsa [B,T,H,D], and at D = 64
// the value pass's P snapshots [B,H,spans,D,D] (one per span of chunks)
int64_t pretrain_backward_workspace_floats(int B, int T, int H, int D);
// chunks per workgroup span of the key pass (and per P snapshot of the
// value pass) for a [B, T, H] backward
int key_chunk_span(int batch, int tokens, int heads);
int launch_key_chunk(const PretrainBwdArgs& a, const float* pbnd, int nspan, int cps,
                     hipStream_t s);

// StateTune: the recurrence from a trainable initial state over a chunk
// list, and its backward (token I/O fp16 or bf16, fp32 state).
struct StateTuneArgs {
  const int32_t* offsets = nullptr;  // [B+1] chunk range of each sequence
  const int32_t* starts = nullptr;   // [C] first token row of each chunk
  const int32_t* ends = nullptr;     // [C] one past its last token row
  int num_seq = 0, num_chunks = 0, heads = 0;
  int64_t tokens = 0;
  const void *r = nullptr, *w = nullptr, *k = nullptr, *v = nullptr, *a = nullptr,
             *b = nullptr;
  float scale = 1.0f;
  // forward
  float* state = nullptr;      // [B,H,D,D] initial state in, final state out
  void* y = nullptr;           // [T,H,D]
  float* sa = nullptr;         // state_dot_a [T,H,D] (written forward, read backward)
  float* boundary = nullptr;   // [C,H,D,D] state at the start of each chunk
  // backward
  const void* dy = nullptr;        // [T,H,D] or null (zero)
  const float* dfinal = nullptr;   // [B,H,D,D] or null (zero)
  float* snap = nullptr;           // [ceil(T/TT),H,D,D] replay snapshots
  float* dsa = nullptr;            // [T,H,D]
  void *dr = nullptr, *dw = nullptr, *dk = nullptr, *dv = nullptr, *da = nullptr,
       *db = nullptr;              // [T,H,D] each, nullable
  float* dstate0 = nullptr;        // [B,H,D,D], nullable
};
int launch_statetune_forward(int D, int dtype, const StateTuneArgs& p, hipStream_t s);
// workspace: dsa [T,H,D] then the replay snapshots [ceil(T/TT),H,D,D]
int launch_statetune_backward(int D, int dtype, StateTuneArgs p, float* workspace,
                              hipStream_t s);
int64_t statetune_backward_workspace_floats(int64_t T, int H, int D);
// D = 64, bf16, B sequences of T tokens each as T / chunk_len chunks
// (chunk_len % 16 == 0): the chunked MFMA kernels.  snap holds the
// post-16-token states [B,H,T/16,64,64]; the backward's workspace is
// pretrain_backward_workspace_floats(B, T, H, 64) + B*H*64*64 floats.
int launch_statetune_uniform_forward(int B, int T, int H, int chunk_len, const StateTuneArgs& a,
                                     float* snap, hipStream_t s);
int launch_statetune_uniform_backward(int B, int T, int H, int chunk_len, const StateTuneArgs& a,
                                      const float* snap, float* workspace, hipStream_t s);
// Any chunk list at D = 64, bf16, on the chunked MFMA kernels: the chunks of
// sequence b laid out from padded row b * Tp on, each starting on a 16-token
// boundary, identity tokens in between (row_source [B*Tp]: packed row or -1;
// chunk_seq / chunk_pstart [C]: each chunk's sequence and padded start).
// snap [B,H,Tp/16,64,64]; ws of statetune_padded_workspace_bytes bytes.
int64_t statetune_padded_workspace_bytes(int B, int Tp, int H, bool backward);
int launch_statetune_padded_forward(int B, int Tp, int H, int C, const int32_t* row_source,
                                    const int32_t* chunk_seq, const int32_t* chunk_pstart,
                                    const StateTuneArgs& a, float* snap, void* ws, hipStream_t s);
// seq_first_chunk [B]: the index of each sequence's first chunk, -1 if none
int launch_statetune_padded_backward(int B, int Tp, int H, const int32_t* row_source,
                                     const int32_t* seq_first_chunk, const StateTuneArgs& a,
                                     const float* snap, void* ws, hipStream_t s);

// Elementwise producer / consumer stages of the layer (fp16 I/O).
int launch_kk_a_gate(int64_t tokens, int H, int D, const void* k, const void* k_k, const void* a0,
                     const void* a12, const void* k_a, void* new_k, void* neg_kk, void* kka,
                     hipStream_t s);
int launch_lowrank_act(int64_t n_t, const void* xt, void* yt, int64_t n_s, const void* xs, void* ys,
                       hipStream_t s);
int launch_vres(int64_t tokens, int C, const void* value, const void* v_first, const void* v0,
                const void* v12, void* out, hipStream_t s);
int launch_readout_prelinear(int64_t tokens, int H, int D, const void* x, const void* r,
                             const void* k, const void* v, const void* r_k, const void* ln_w,
                             const void* ln_b, const void* g, void* out, hipStream_t s);

}  // namespace fr2
