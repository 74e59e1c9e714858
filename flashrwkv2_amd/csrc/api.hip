// extern "C" entry points of the WKV7 operator (declared in
// include/flashrwkv2_amd.h).  Each validates pointers and sizes, fills a
// segment descriptor and enqueues the chosen kernel family on `stream`.
#include "recurrent.h"
#include "../../include/flashrwkv2_amd.h"

#include <algorithm>
#include <atomic>
#include <initializer_list>

namespace {

using fr2::SegArgs;

// Kernel-family policy at D = 64 (replaces use_small_auto,
// csrc/sm120/tmix/wkv7/infer_recurrent_fp32io16_forward_varlen.cu:378-391),
// by the longest sequence L, the (sequence, head) unit count U and the mean
// length of the launch.  Measured with each family forced on equal-length
// batches, H = 32 (ms per call):
//   L <= 4: the decode kernel (one wave per unit, tokens in order) streams
//     the state once and is the fastest at every U; at U >= 16384 also up
//     to L = 6 (U = 65536, L = 6: decode 0.472, chunked-wave 0.490);
//   U <= 256 (at most one block per CU): the chunked kernel with one
//     512-thread workgroup per unit from L = 5 on (L = 1024: 0.098 against
//     0.399 with one wave per unit);
//   larger U: the chunked kernel with one wave per unit (chunkw.hip), whose
//     units hide each other's latency, up to L = 24 (U <= 512) and at every
//     L beyond that (U = 1024, L = 1024: 0.351 against 0.395; U = 65536,
//     L = 64: 1.41 against 2.85), except for skewed batches whose longest
//     sequence exceeds twice the mean: a long sequence is one wave's serial
//     chain there, and the workgroup-per-unit kernel finishes it sooner.
// The token-serial kernel wins only within launch latency (U = 512, L = 5-8:
// 0.0104 against 0.0114 ms); it remains the kernel of D != 64.
constexpr int kDecodeMaxSeqlen = 4;
constexpr int kChunkMinSeqlen = 5;   // the smallest chunked threshold (U <= 256)

bool decode_first(int64_t units, int max_seqlen) {
  return max_seqlen <= kDecodeMaxSeqlen || (units >= 16384 && max_seqlen <= 6);
}
// one wave per unit (true) or one workgroup per unit, for a chunked launch
bool wave_per_unit(int64_t units, int max_seqlen, int64_t total_tokens, int64_t nseg) {
  if (units <= 256) return false;
  if (units <= 512) return max_seqlen <= 24;
  return max_seqlen <= 512 || static_cast<int64_t>(max_seqlen) * nseg <= 2 * total_tokens;
}
// the public policy's choice is the workgroup-per-unit chunked kernel (the
// kernel the fused kk-gate / readout stages live in)
bool workgroup_chunked(int64_t units, int max_seqlen, int64_t total_tokens, int64_t nseg) {
  return max_seqlen > 0 && !decode_first(units, max_seqlen) &&
         !wave_per_unit(units, max_seqlen, total_tokens, nseg);
}

enum Family { kAuto = -1, kSerial = 0, kDecode = 1, kChunked = 2, kChunkedWave = 4 };

// The family the public fp32-state policy picks for a plain launch (no sa /
// boundary outputs, fp32 state); the one source of the choice that
// run_family applies and fr2_wkv7_recurrent_fp32_dispatch reports.
int plain_family(int D, int64_t units, int max_seqlen, int64_t total_tokens, int64_t nseg) {
  if (D != 64 || max_seqlen <= 0) return kSerial;
  if (decode_first(units, max_seqlen)) return kDecode;
  return wave_per_unit(units, max_seqlen, total_tokens, nseg) ? kChunkedWave : kChunked;
}

// Token tensors are read and written as 16-byte vectors: every token
// pointer must be present and 16-byte aligned (a contiguous view with an odd
// storage offset is rejected instead of faulting on a misaligned access).
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool tokens_ok(const void* r, const void* l, const void* k, const void* v,
               const void* a, const void* b, const void* y) {
  if (!(r && l && k && v && a && b && y)) return false;
  if (aligned16(r) && aligned16(l) && aligned16(k) && aligned16(v) && aligned16(a) &&
      aligned16(b) && aligned16(y))
    return true;
  fr2::set_last_error("token tensors must be 16-byte aligned (a view with an odd storage "
                      "offset needs an aligned copy)");
  return false;
}
// Per-channel parameters ([H, D] vectors: decay bias, kk / a-gate and
// readout parameters) are read as 16-byte vectors too; null means absent.
bool params_aligned(std::initializer_list<const void*> ptrs) {
  for (const void* q : ptrs) {
    if (q != nullptr && !aligned16(q)) {
      fr2::set_last_error("per-channel parameter tensors must be 16-byte aligned (a view "
                          "with an odd storage offset needs an aligned copy)");
      return false;
    }
  }
  return true;
}

int run_family(int family, int D, int dtype, bool bf16_state, const SegArgs& p,
               int nseg, int max_seqlen, hipStream_t s) {
  if (family == kAuto) {
    const bool plain = p.sa_out == nullptr && p.boundary == nullptr && !bf16_state;
    const int64_t units = static_cast<int64_t>(nseg) * p.num_heads;
    family = kSerial;
    if (plain) {
      const int64_t total = p.out_elems / (static_cast<int64_t>(p.num_heads) * D);
      const int f = plain_family(D, units, max_seqlen, total, nseg);
      if (f == kDecode) {
        family = kDecode;
      } else if (f != kSerial) {
        const int rc = f == kChunkedWave
                           ? fr2::launch_chunked_wave(dtype, p, nseg, max_seqlen, s)
                           : fr2::launch_chunked(dtype, p, nseg, max_seqlen, s);
        if (rc != FR2_ERR_UNSUPPORTED) return rc;
      }
    }
  }
  switch (family) {
    case kSerial: return fr2::launch_serial(D, dtype, bf16_state, p, nseg, s);
    case kDecode:
      if (bf16_state) return FR2_ERR_UNSUPPORTED;
      return fr2::launch_decode(D, dtype, p, nseg, s);
    case kChunked:
      if (bf16_state || D != 64) return FR2_ERR_UNSUPPORTED;
      return fr2::launch_chunked(dtype, p, nseg, max_seqlen, s);
    case kChunkedWave:
      if (bf16_state || D != 64) return FR2_ERR_UNSUPPORTED;
      return fr2::launch_chunked_wave(dtype, p, nseg, max_seqlen, s);
    default: return FR2_ERR_INVALID_ARGUMENT;
  }
}

int recurrent_fp32(int family, const int32_t* qsl, const int32_t* slots,
                   const int32_t* status, int32_t n, int32_t H, int32_t D,
                   int64_t total_tokens, int32_t max_seqlen, int32_t dtype,
                   float* state, const void* r, const void* l, const void* bias,
                   const void* k, const void* v, const void* a, const void* b,
                   void* out, float scale, void* stream) {
  if (!qsl || !slots || !status || !state || !tokens_ok(r, l, k, v, a, b, out))
    return FR2_ERR_INVALID_ARGUMENT;
  if (n <= 0 || n > 65535 || H <= 0 || total_tokens <= 0)
    return FR2_ERR_INVALID_ARGUMENT;
  if (D != 64 && D != 128 && D != 256) return FR2_ERR_UNSUPPORTED;
  SegArgs p;
  p.bounds = qsl;
  p.slots = slots;
  p.status = status;
  p.num_heads = H;
  p.out_elems = total_tokens * H * D;
  p.state_in = state;
  p.state_out = state;
  p.r = r; p.logits = l; p.bias = bias; p.k = k; p.v = v; p.a = a; p.b = b;
  p.y = out;
  p.scale = scale;
  return run_family(family, D, dtype, false, p, n, max_seqlen,
                    static_cast<hipStream_t>(stream));
}

}  // namespace

extern "C" int fr2_wkv7_recurrent_fp32_forward(
    const int32_t* query_start_loc, const int32_t* state_indices,
    const int32_t* status, int32_t num_sequences, int32_t num_heads,
    int32_t head_size, int64_t total_tokens, int32_t max_seqlen, int32_t dtype,
    float* state, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a,
    const void* b, void* output, float scale, void* stream) {
  if (!params_aligned({decay_bias})) return FR2_ERR_INVALID_ARGUMENT;
  return recurrent_fp32(kAuto, query_start_loc, state_indices, status,
                        num_sequences, num_heads, head_size, total_tokens,
                        max_seqlen, dtype, state, r, decay_logits, decay_bias, k,
                        v, a, b, output, scale, stream);
}

extern "C" int fr2_wkv7_recurrent_fp32_dispatch(int32_t num_sequences, int32_t num_heads,
                                                int32_t head_size, int64_t total_tokens,
                                                int32_t max_seqlen, int32_t* kernel) {
  if (kernel == nullptr || num_sequences <= 0 || num_sequences > 65535 || num_heads <= 0 ||
      total_tokens <= 0)
    return FR2_ERR_INVALID_ARGUMENT;
  if (head_size != 64 && head_size != 128 && head_size != 256) return FR2_ERR_UNSUPPORTED;
  const int64_t units = static_cast<int64_t>(num_sequences) * num_heads;
  int f = plain_family(head_size, units, max_seqlen, total_tokens, num_sequences);
  if (f == kChunkedWave && fr2::wave_longest_first(num_sequences, max_seqlen, total_tokens))
    f = 5;
  *kernel = f;
  return FR2_OK;
}

extern "C" int fr2_wkv7_recurrent_fp32_forward_kernel(
    int32_t kernel, const int32_t* query_start_loc,
    const int32_t* state_indices, const int32_t* status,
    int32_t num_sequences, int32_t num_heads, int32_t head_size,
    int64_t total_tokens, int32_t max_seqlen, int32_t dtype, float* state,
    const void* r, const void* decay_logits, const void* decay_bias,
    const void* k, const void* v, const void* a, const void* b, void* output,
    float scale, void* stream) {
  if (!params_aligned({decay_bias})) return FR2_ERR_INVALID_ARGUMENT;
  if (kernel != kSerial && kernel != kDecode && kernel != kChunked && kernel != kChunkedWave)
    return FR2_ERR_INVALID_ARGUMENT;
  return recurrent_fp32(kernel, query_start_loc, state_indices, status,
                        num_sequences, num_heads, head_size, total_tokens,
                        max_seqlen, dtype, state, r, decay_logits, decay_bias, k,
                        v, a, b, output, scale, stream);
}

// Sequence split of the chunked prefill.  With few (sequence, head) units
// the chunked kernel leaves most CUs idle (one block per unit, one block per
// CU), so long sequences are cut into pieces.  The plan is the pipelined
// ("lead") split: piece 0 runs from the slot state concurrently with a
// summary pass over pieces 1..P-2 (one block per unit and piece), then a
// combine kernel chains the start states and pieces 1..P-1 run.  With
// Q = 256/units and P = Q + 1 pieces, both phases hold one block per CU.  A
// summary block and a real block next to it run at about the same rate per
// token (config 4: 85 and 86 ns per token), so piece 0 gets 1.05x the
// tokens of the others (config 4, lead lengths 13 120-15 104 tokens: 2.14-
// 2.16 ms at 13 440-13 760, 2.25 ms at 15 104).  Q is also capped so that
// pieces keep at least 384 tokens: shorter pieces lose to the fixed cost of
// the extra passes (1024 tokens on 32 units: 3 pieces 0.095 ms, unsplit
// 0.083 ms; 2048 tokens: 5 pieces 0.120 ms, unsplit 0.164 ms).  Split only
// when Q >= 2 (at most 128 units).
constexpr int kSplitMaxUnits = 128;
constexpr int kSplitMinPiece = 384;
constexpr int kSplitAlign = 32;
constexpr float kSplitLeadRatio = 1.05f;

extern "C" int fr2_wkv7_recurrent_fp32_split_plan(int32_t num_sequences, int32_t num_heads,
                                                  int32_t head_size, int32_t max_seqlen,
                                                  int32_t* pieces, int32_t* piece_len,
                                                  int32_t* lead_len, int64_t* workspace_bytes) {
  if (!pieces || !piece_len || !lead_len || !workspace_bytes || num_sequences <= 0 ||
      num_heads <= 0)
    return FR2_ERR_INVALID_ARGUMENT;
  *pieces = 1;
  *piece_len = max_seqlen;
  *lead_len = 0;
  *workspace_bytes = 0;
  const int64_t units = static_cast<int64_t>(num_sequences) * num_heads;
  if (head_size != 64 || max_seqlen < kChunkMinSeqlen || units > kSplitMaxUnits)
    return FR2_OK;
  // pieces after the lead piece: one block per CU in each phase, and pieces
  // of at least kSplitMinPiece tokens
  const int Q = static_cast<int>(std::min<int64_t>(
      256 / units,
      static_cast<int64_t>(static_cast<float>(max_seqlen) / kSplitMinPiece - kSplitLeadRatio)));
  if (Q < 2) return FR2_OK;
  int len = static_cast<int>(max_seqlen / (Q + kSplitLeadRatio));
  len = (len + kSplitAlign - 1) / kSplitAlign * kSplitAlign;
  if (len < kSplitMinPiece) return FR2_OK;
  int lead = max_seqlen - Q * len;
  lead = (lead + kSplitAlign - 1) / kSplitAlign * kSplitAlign;
  if (lead < len) lead = len;
  // pieces the longest sequence actually has with these lengths
  const int P = max_seqlen <= lead ? 1 : 2 + (max_seqlen - lead - 1) / len;
  if (P < 3 || static_cast<int64_t>(num_sequences) * P * 2 > 65535) return FR2_OK;
  *pieces = P;
  *piece_len = len;
  *lead_len = lead;
  *workspace_bytes = fr2::split_workspace_floats(num_sequences, num_heads, P) * 4;
  return FR2_OK;
}

extern "C" int fr2_wkv7_recurrent_fp32_forward_split(
    const int32_t* query_start_loc, const int32_t* state_indices, const int32_t* status,
    int32_t num_sequences, int32_t num_heads, int32_t head_size, int64_t total_tokens,
    int32_t max_seqlen, int32_t dtype, float* state, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a, const void* b,
    void* output, float scale, int32_t pieces, int32_t piece_len, int32_t lead_len,
    void* workspace, int64_t workspace_bytes, void* stream, void* aux_stream) {
  if (!params_aligned({decay_bias})) return FR2_ERR_INVALID_ARGUMENT;
  (void)max_seqlen;
  if (!query_start_loc || !state_indices || !status || !state || !workspace ||
      !tokens_ok(r, decay_logits, k, v, a, b, output))
    return FR2_ERR_INVALID_ARGUMENT;
  if (num_sequences <= 0 || num_sequences > 65535 || num_heads <= 0 || total_tokens <= 0)
    return FR2_ERR_INVALID_ARGUMENT;
  if (head_size != 64) return FR2_ERR_UNSUPPORTED;
  if (pieces < 2 || workspace_bytes < fr2::split_workspace_floats(num_sequences, num_heads,
                                                                   pieces) * 4)
    return FR2_ERR_INVALID_ARGUMENT;
  SegArgs p;
  p.bounds = query_start_loc;
  p.slots = state_indices;
  p.status = status;
  p.num_heads = num_heads;
  p.out_elems = total_tokens * num_heads * head_size;
  p.state_in = state;
  p.state_out = state;
  p.r = r; p.logits = decay_logits; p.bias = decay_bias; p.k = k; p.v = v; p.a = a; p.b = b;
  p.y = output;
  p.scale = scale;
  return fr2::launch_chunked_split(dtype, p, num_sequences, pieces, piece_len, lead_len,
                                   static_cast<float*>(workspace),
                                   static_cast<hipStream_t>(stream),
                                   static_cast<hipStream_t>(aux_stream));
}

// ---------------------------------------------------------------------------
// No-allocation form of fr2_wkv7_recurrent_fp32_forward_split.  Its
// workspace is `scratch`, a file-scope device array of kNoAllocScratchFloats
// floats that every GPU the library runs on holds until the process ends.
// The array's name is a host-side stand-in for the device symbol: host code
// uses only the device address hipGetSymbolAddress returns, looked up once
// per device with that device current and kept in g_scratch_ptr.
// No clearing is needed: every float of the workspace a call reads was
// written earlier in the same call (summaries, then chained start states).
// Calls that overlap on one GPU share the array and race.
// ---------------------------------------------------------------------------
constexpr int64_t kNoAllocScratchFloats = int64_t{4} << 20;   // 16 MiB
static_assert(kNoAllocScratchFloats * 4 == FR2_NOALLOC_SCRATCH_BYTES,
              "header and library must agree on the scratch size");
__device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {
std::atomic<float*> g_scratch_ptr[64];

float* scratch_address() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  float* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    if (hipGetSymbolAddress(reinterpret_cast<void**>(&ptr), HIP_SYMBOL(scratch)) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    g_scratch_ptr[dev].store(ptr, std::memory_order_release);
  }
  return ptr;
}
}  // namespace

extern "C" int fr2_wkv7_recurrent_fp32_forward_split_noalloc(
    const int32_t* query_start_loc, const int32_t* state_indices, const int32_t* status,
    int32_t num_sequences, int32_t num_heads, int32_t head_size, int64_t total_tokens,
    int32_t max_seqlen, int32_t dtype, float* state, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a, const void* b,
    void* output, float scale, int32_t pieces, int32_t piece_len, int32_t lead_len,
    void* stream) {
  if (!params_aligned({decay_bias})) return FR2_ERR_INVALID_ARGUMENT;
  // the bounds the split itself enforces, checked before the workspace size
  // is formed from them (so that the product cannot overflow)
  if (num_sequences <= 0 || num_sequences > 65535 || num_heads <= 0 || pieces < 2 ||
      pieces > 65535 || static_cast<int64_t>(num_sequences) * pieces > 65535)
    return FR2_ERR_INVALID_ARGUMENT;
  const int64_t need = fr2::split_workspace_floats(num_sequences, num_heads, pieces);
  if (need > kNoAllocScratchFloats) {
    fr2::set_last_error(
        "fr2_wkv7_recurrent_fp32_forward_split_noalloc: the split's workspace exceeds the "
        "16 MiB no-allocation scratch (num_sequences * (3 pieces - 2) * num_heads * 16 KiB)");
    return FR2_ERR_INVALID_ARGUMENT;
  }
  float* ws = scratch_address();
  if (ws == nullptr) {
    fr2::set_last_error("fr2_wkv7_recurrent_fp32_forward_split_noalloc: scratch lookup failed");
    return FR2_ERR_LAUNCH;
  }
  // one stream: the pipelined split's second stream would need events
  return fr2_wkv7_recurrent_fp32_forward_split(
      query_start_loc, state_indices, status, num_sequences, num_heads, head_size, total_tokens,
      max_seqlen, dtype, state, r, decay_logits, decay_bias, k, v, a, b, output, scale, pieces,
      piece_len, lead_len, ws, need * 4, stream, nullptr);
}

namespace {
int recurrent_fp16(int family, bool advance, const int32_t* query_start_loc,
                   const int32_t* state_indices,
                   const int32_t* status, int32_t* elapsed_state, int32_t num_sequences,
                   int32_t num_heads, int32_t head_size, int64_t total_tokens,
                   int32_t max_seqlen, void* state_f16, const void* r, const void* decay_logits,
                   const void* decay_bias, const void* k, const void* v, const void* a,
                   const void* b, void* output, float scale, void* stream) {
  if (!query_start_loc || !state_indices || !status || !elapsed_state || !state_f16 ||
      !tokens_ok(r, decay_logits, k, v, a, b, output))
    return FR2_ERR_INVALID_ARGUMENT;
  if (num_sequences <= 0 || num_sequences > 65535 || num_heads <= 0 || total_tokens <= 0)
    return FR2_ERR_INVALID_ARGUMENT;
  if (head_size != 64 && head_size != 128 && head_size != 256) return FR2_ERR_UNSUPPORTED;
  SegArgs p;
  p.bounds = query_start_loc;
  p.slots = state_indices;
  p.status = status;
  p.num_heads = num_heads;
  p.out_elems = total_tokens * num_heads * head_size;
  p.state_in = state_f16;
  p.state_out = state_f16;
  p.r = r; p.logits = decay_logits; p.bias = decay_bias; p.k = k; p.v = v; p.a = a; p.b = b;
  p.y = output;
  p.scale = scale;
  return fr2::launch_fp16_state(head_size, p, num_sequences, max_seqlen, elapsed_state,
                                static_cast<hipStream_t>(stream), advance, family);
}
}  // namespace

extern "C" int fr2_wkv7_recurrent_fp16_forward(
    const int32_t* query_start_loc, const int32_t* state_indices,
    const int32_t* status, int32_t* elapsed_state, int32_t num_sequences,
    int32_t num_heads, int32_t head_size, int64_t total_tokens, int32_t max_seqlen,
    void* state_f16, const void* r, const void* decay_logits, const void* decay_bias,
    const void* k, const void* v, const void* a, const void* b, void* output, float scale,
    void* stream) {
  if (!params_aligned({decay_bias})) return FR2_ERR_INVALID_ARGUMENT;
  return recurrent_fp16(-1, true, query_start_loc, state_indices, status, elapsed_state,
                        num_sequences, num_heads, head_size, total_tokens, max_seqlen, state_f16,
                        r, decay_logits, decay_bias, k, v, a, b, output, scale, stream);
}

extern "C" int fr2_wkv7_recurrent_fp16_update(
    const int32_t* query_start_loc, const int32_t* state_indices,
    const int32_t* status, const int32_t* elapsed_state, int32_t num_sequences,
    int32_t num_heads, int32_t head_size, int64_t total_tokens, int32_t max_seqlen,
    void* state_f16, const void* r, const void* decay_logits, const void* decay_bias,
    const void* k, const void* v, const void* a, const void* b, void* output, float scale,
    void* stream) {
  if (!params_aligned({decay_bias})) return FR2_ERR_INVALID_ARGUMENT;
  return recurrent_fp16(-1, false, query_start_loc, state_indices, status,
                        const_cast<int32_t*>(elapsed_state), num_sequences, num_heads, head_size,
                        total_tokens, max_seqlen, state_f16, r, decay_logits, decay_bias, k, v, a,
                        b, output, scale, stream);
}

extern "C" int fr2_wkv7_recurrent_fp16_update_kernel(
    int32_t kernel, const int32_t* query_start_loc, const int32_t* state_indices,
    const int32_t* status, const int32_t* elapsed_state, int32_t num_sequences,
    int32_t num_heads, int32_t head_size, int64_t total_tokens, int32_t max_seqlen,
    void* state_f16, const void* r, const void* decay_logits, const void* decay_bias,
    const void* k, const void* v, const void* a, const void* b, void* output, float scale,
    void* stream) {
  if (!params_aligned({decay_bias})) return FR2_ERR_INVALID_ARGUMENT;
  if (kernel != fr2::kFp16Serial && kernel != fr2::kFp16Decode &&
      kernel != fr2::kFp16SerialWave)
    return FR2_ERR_INVALID_ARGUMENT;
  return recurrent_fp16(kernel, false, query_start_loc, state_indices, status,
                        const_cast<int32_t*>(elapsed_state), num_sequences, num_heads, head_size,
                        total_tokens, max_seqlen, state_f16, r, decay_logits, decay_bias, k, v, a,
                        b, output, scale, stream);
}

extern "C" int fr2_wkv7_recurrent_fp16_advance_elapsed(const int32_t* query_start_loc,
                                                       const int32_t* state_indices,
                                                       const int32_t* status,
                                                       int32_t* elapsed_state,
                                                       int32_t num_sequences, void* stream) {
  if (!query_start_loc || !state_indices || !status || !elapsed_state || num_sequences <= 0 ||
      num_sequences > 65535)
    return FR2_ERR_INVALID_ARGUMENT;
  SegArgs p;
  p.bounds = query_start_loc;
  p.slots = state_indices;
  p.status = status;
  return fr2::launch_advance_elapsed(p, num_sequences, elapsed_state,
                                     static_cast<hipStream_t>(stream));
}

extern "C" int fr2_wkv7_pretrain_forward(int32_t batch, int32_t tokens,
                                         int32_t num_heads, int32_t head_size,
                                         const void* r, const void* w,
                                         const void* k, const void* v,
                                         const void* a, const void* b,
                                         void* output, float* boundary,
                                         float* state_dot_a, void* stream) {
  if (!tokens_ok(r, w, k, v, a, b, output) || !boundary || !state_dot_a)
    return FR2_ERR_INVALID_ARGUMENT;
  if (batch <= 0 || batch > 65535 || tokens <= 0 || tokens % 16 != 0 || num_heads <= 0)
    return FR2_ERR_INVALID_ARGUMENT;
  if (head_size != 64 && head_size != 128 && head_size != 256) return FR2_ERR_UNSUPPORTED;
  SegArgs p;
  p.uniform_len = tokens;
  p.num_heads = num_heads;
  p.out_elems = static_cast<int64_t>(batch) * tokens * num_heads * head_size;
  p.r = r; p.logits = w; p.k = k; p.v = v; p.a = a; p.b = b;
  p.y = output;
  p.sa_out = state_dot_a;
  p.boundary = boundary;
  p.boundary_len = 16;
  p.boundary_per_seg = tokens / 16;
  // D = 64 runs the chunked MFMA kernel, which emits sa and the post-chunk
  // states of its 16-token chunks directly; other head sizes run token-serial
  if (head_size == 64) {
    const int rc = fr2::launch_chunked(FR2_DTYPE_BFLOAT16, p, batch, tokens,
                                       static_cast<hipStream_t>(stream));
    if (rc != FR2_ERR_UNSUPPORTED) return rc;
  }
  return fr2::launch_serial(head_size, FR2_DTYPE_BFLOAT16, false, p, batch,
                            static_cast<hipStream_t>(stream));
}

extern "C" int64_t fr2_wkv7_pretrain_backward_workspace_floats(int32_t batch, int32_t tokens,
                                                               int32_t num_heads,
                                                               int32_t head_size) {
  if (batch <= 0 || tokens <= 0 || tokens % 16 != 0 || num_heads <= 0) return -1;
  if (head_size != 64 && head_size != 128 && head_size != 256) return -1;
  return fr2::pretrain_backward_workspace_floats(batch, tokens, num_heads, head_size);
}

extern "C" int fr2_wkv7_pretrain_backward(
    int32_t batch, int32_t tokens, int32_t num_heads, int32_t head_size, const void* r,
    const void* w, const void* k, const void* v, const void* a, const void* b,
    const void* grad_output, const float* boundary, const float* state_dot_a,
    float* workspace, void* grad_r, void* grad_w, void* grad_k, void* grad_v,
    void* grad_a, void* grad_b, void* stream) {
  if (!tokens_ok(r, w, k, v, a, b, grad_output) || !boundary || !state_dot_a ||
      !workspace || !grad_r || !grad_w || !grad_k || !grad_v || !grad_a || !grad_b)
    return FR2_ERR_INVALID_ARGUMENT;
  if (batch <= 0 || tokens <= 0 || tokens % 16 != 0 || num_heads <= 0 ||
      static_cast<int64_t>(batch) * num_heads > (int64_t{1} << 30) / 4)
    return FR2_ERR_INVALID_ARGUMENT;
  if (head_size != 64 && head_size != 128 && head_size != 256) return FR2_ERR_UNSUPPORTED;
  fr2::PretrainBwdArgs p;
  p.batch = batch; p.tokens = tokens; p.heads = num_heads;
  p.r = r; p.w = w; p.k = k; p.v = v; p.a = a; p.b = b; p.dy = grad_output;
  p.boundary = boundary; p.state_dot_a = state_dot_a; p.workspace = workspace;
  p.dr = grad_r; p.dw = grad_w; p.dk = grad_k; p.dv = grad_v; p.da = grad_a; p.db = grad_b;
  return fr2::launch_pretrain_backward(head_size, p, static_cast<hipStream_t>(stream));
}

extern "C" int fr2_wkv7_chunk_bf16_forward(
    const int32_t* query_start_loc, const int32_t* state_indices,
    const int32_t* status, int32_t num_sequences, int32_t num_heads,
    int64_t total_tokens, int32_t chunk_size, int32_t max_seqlen,
    uint16_t* state_bf16, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a,
    const void* b, void* output, float scale, void* stream) {
  if (!params_aligned({decay_bias})) return FR2_ERR_INVALID_ARGUMENT;
  if (!query_start_loc || !state_indices || !status || !state_bf16 ||
      !tokens_ok(r, decay_logits, k, v, a, b, output))
    return FR2_ERR_INVALID_ARGUMENT;
  if (num_sequences <= 0 || num_sequences > 65535 || num_heads <= 0 ||
      total_tokens <= 0 || chunk_size <= 0)
    return FR2_ERR_INVALID_ARGUMENT;
  SegArgs p;
  p.bounds = query_start_loc;
  p.slots = state_indices;
  p.status = status;
  p.num_heads = num_heads;
  p.out_elems = total_tokens * num_heads * 64;
  p.state_in = state_bf16;
  p.state_out = state_bf16;
  p.r = r; p.logits = decay_logits; p.bias = decay_bias; p.k = k; p.v = v;
  p.a = a; p.b = b;
  p.y = output;
  p.scale = scale;
  // The contract keeps the state in fp32 inside the call and rounds it to
  // bf16 once at the end (infer_chunk_bf16_forward_varlen.cu:195-270), so the
  // request runs on a chunked MFMA kernel with a bf16 state load / store
  // (chunk_size only shapes the reference's workspace, not the arithmetic):
  // the wavefront-per-unit kernel where the fp32-state policy picks it, and
  // also for sequences of at most 4 tokens (which have no decode form here;
  // it beats the token-serial kernel there at every unit count measured),
  // otherwise the workgroup-per-unit kernel.
  const int64_t units = static_cast<int64_t>(num_sequences) * num_heads;
  p.state_bf16 = true;
  const int rc =
      (max_seqlen < kChunkMinSeqlen || wave_per_unit(units, max_seqlen, total_tokens, num_sequences))
          ? fr2::launch_chunked_wave(FR2_DTYPE_BFLOAT16, p, num_sequences, max_seqlen,
                                     static_cast<hipStream_t>(stream))
          : fr2::launch_chunked(FR2_DTYPE_BFLOAT16, p, num_sequences, max_seqlen,
                                static_cast<hipStream_t>(stream));
  if (rc != FR2_ERR_UNSUPPORTED) return rc;
  p.state_bf16 = false;
  return fr2::launch_serial(64, FR2_DTYPE_BFLOAT16, true, p, num_sequences,
                            static_cast<hipStream_t>(stream));
}

extern "C" int fr2_wkv7_chunk_bf16_forward_split(
    const int32_t* query_start_loc, const int32_t* state_indices,
    const int32_t* status, int32_t num_sequences, int32_t num_heads,
    int64_t total_tokens, int32_t chunk_size, int32_t max_seqlen,
    uint16_t* state_bf16, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a,
    const void* b, void* output, float scale, int32_t pieces, int32_t piece_len,
    int32_t lead_len, void* workspace, int64_t workspace_bytes, void* stream,
    void* aux_stream) {
  if (!params_aligned({decay_bias})) return FR2_ERR_INVALID_ARGUMENT;
  (void)max_seqlen;
  if (!query_start_loc || !state_indices || !status || !state_bf16 || !workspace ||
      !tokens_ok(r, decay_logits, k, v, a, b, output))
    return FR2_ERR_INVALID_ARGUMENT;
  if (num_sequences <= 0 || num_sequences > 65535 || num_heads <= 0 ||
      total_tokens <= 0 || chunk_size <= 0)
    return FR2_ERR_INVALID_ARGUMENT;
  if (pieces < 2 || workspace_bytes < fr2::split_workspace_floats(num_sequences, num_heads,
                                                                   pieces) * 4)
    return FR2_ERR_INVALID_ARGUMENT;
  SegArgs p;
  p.bounds = query_start_loc;
  p.slots = state_indices;
  p.status = status;
  p.num_heads = num_heads;
  p.out_elems = total_tokens * num_heads * 64;
  p.state_in = state_bf16;
  p.state_out = state_bf16;
  p.state_bf16 = true;
  p.r = r; p.logits = decay_logits; p.bias = decay_bias; p.k = k; p.v = v;
  p.a = a; p.b = b;
  p.y = output;
  p.scale = scale;
  return fr2::launch_chunked_split(FR2_DTYPE_BFLOAT16, p, num_sequences, pieces, piece_len,
                                   lead_len, static_cast<float*>(workspace),
                                   static_cast<hipStream_t>(stream),
                                   static_cast<hipStream_t>(aux_stream));
}

extern "C" int fr2_wkv7_rl_infctx_forward(
    const int32_t* sequence_chunk_offsets, const int32_t* chunk_token_starts,
    const int32_t* chunk_token_ends, int32_t num_sequences, int32_t num_chunks,
    int32_t num_heads, int32_t head_size, int64_t total_tokens,
    int32_t max_seqlen, int32_t chunk_size, int32_t strategy, int32_t dtype,
    float* state, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a,
    const void* b, void* output, float scale, void* stream) {
  if (!params_aligned({decay_bias})) return FR2_ERR_INVALID_ARGUMENT;
  if (!sequence_chunk_offsets || !chunk_token_starts || !chunk_token_ends ||
      !state || !tokens_ok(r, decay_logits, k, v, a, b, output))
    return FR2_ERR_INVALID_ARGUMENT;
  if (num_sequences <= 0 || num_sequences > 65535 || num_chunks <= 0 ||
      num_heads <= 0 || total_tokens <= 0)
    return FR2_ERR_INVALID_ARGUMENT;
  if (chunk_size != 16 && chunk_size != 32 && chunk_size != 64) return FR2_ERR_UNSUPPORTED;
  if (strategy != 0 && strategy != 1) return FR2_ERR_INVALID_ARGUMENT;
  if (head_size != 64 && head_size != 128 && head_size != 256) return FR2_ERR_UNSUPPORTED;
  SegArgs p;
  p.bounds = chunk_token_starts;
  p.ends = chunk_token_ends;
  p.chunk_offsets = sequence_chunk_offsets;
  p.num_heads = num_heads;
  p.out_elems = total_tokens * num_heads * head_size;
  p.state_in = state;
  p.state_out = state;
  p.r = r; p.logits = decay_logits; p.bias = decay_bias; p.k = k; p.v = v;
  p.a = a; p.b = b;
  p.y = output;
  p.scale = scale;
  return run_family(kAuto, head_size, dtype, false, p, num_sequences, max_seqlen,
                    static_cast<hipStream_t>(stream));
}

extern "C" int fr2_wkv7_rl_infctx_replay(
    const int32_t* chunk_token_starts, const int32_t* chunk_token_ends,
    int32_t num_chunks, int32_t num_heads, int32_t head_size,
    int64_t total_tokens, int32_t dtype, const float* boundary, const void* r,
    const void* decay_logits, const void* decay_bias, const void* k,
    const void* v, const void* a, const void* b, void* output,
    float* state_dot_a, float scale, void* stream) {
  if (!params_aligned({decay_bias})) return FR2_ERR_INVALID_ARGUMENT;
  if (!chunk_token_starts || !chunk_token_ends || !boundary || !state_dot_a ||
      !tokens_ok(r, decay_logits, k, v, a, b, output))
    return FR2_ERR_INVALID_ARGUMENT;
  if (num_chunks <= 0 || num_chunks > 65535 || num_heads <= 0 || total_tokens <= 0)
    return FR2_ERR_INVALID_ARGUMENT;
  if (head_size != 64 && head_size != 128 && head_size != 256) return FR2_ERR_UNSUPPORTED;
  SegArgs p;
  p.bounds = chunk_token_starts;
  p.ends = chunk_token_ends;
  p.num_heads = num_heads;
  p.out_elems = total_tokens * num_heads * head_size;
  p.state_in = boundary;
  p.r = r; p.logits = decay_logits; p.bias = decay_bias; p.k = k; p.v = v;
  p.a = a; p.b = b;
  p.y = output;
  p.sa_out = state_dot_a;
  p.scale = scale;
  // chunks of at most 64 tokens from their boundary states: at D = 64 the
  // chunked kernel with one wavefront per (chunk, head) unit, which also
  // writes sa, beats the token-serial and decode kernels at every unit count
  // and length of run_family's grid (256 units, L = 16: 0.011 vs 0.013 ms
  // serial; 65 536 units, L = 16: 0.62 vs 0.90 ms decode)
  if (head_size == 64)
    return fr2::launch_chunked_wave(dtype, p, num_chunks, 0, static_cast<hipStream_t>(stream));
  return fr2::launch_serial(head_size, dtype, false, p, num_chunks,
                            static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// StateTune (trainable initial state over a chunk list)
// ---------------------------------------------------------------------------
namespace {

bool statetune_sizes_ok(int32_t num_sequences, int32_t num_chunks, int64_t total_tokens,
                        int32_t num_heads) {
  return num_sequences > 0 && num_chunks > 0 && num_heads > 0 && total_tokens > 0 &&
         total_tokens < (int64_t{1} << 31);
}

}  // namespace

extern "C" int fr2_wkv7_statetune_forward(
    const int32_t* sequence_chunk_offsets, const int32_t* chunk_token_starts,
    const int32_t* chunk_token_ends, int32_t num_sequences, int32_t num_chunks,
    int64_t total_tokens, int32_t num_heads, int32_t head_size, int32_t dtype, float* state,
    const void* r, const void* decay_logits, const void* k, const void* v, const void* a,
    const void* b, void* output, float* boundary, float* state_dot_a, float scale,
    void* stream) {
  if (!sequence_chunk_offsets || !chunk_token_starts || !chunk_token_ends || !state ||
      !tokens_ok(r, decay_logits, k, v, a, b, output) || !boundary || !state_dot_a)
    return FR2_ERR_INVALID_ARGUMENT;
  if (!statetune_sizes_ok(num_sequences, num_chunks, total_tokens, num_heads))
    return FR2_ERR_INVALID_ARGUMENT;
  if (head_size != 64 && head_size != 128 && head_size != 256) return FR2_ERR_UNSUPPORTED;
  if (dtype != FR2_DTYPE_FLOAT16 && dtype != FR2_DTYPE_BFLOAT16) return FR2_ERR_UNSUPPORTED;
  fr2::StateTuneArgs p;
  p.offsets = sequence_chunk_offsets;
  p.starts = chunk_token_starts;
  p.ends = chunk_token_ends;
  p.num_seq = num_sequences;
  p.num_chunks = num_chunks;
  p.heads = num_heads;
  p.tokens = total_tokens;
  p.r = r; p.w = decay_logits; p.k = k; p.v = v; p.a = a; p.b = b;
  p.scale = scale;
  p.state = state;
  p.y = output;
  p.sa = state_dot_a;
  p.boundary = boundary;
  return fr2::launch_statetune_forward(head_size, dtype, p, static_cast<hipStream_t>(stream));
}

extern "C" int64_t fr2_wkv7_statetune_backward_workspace_floats(int64_t total_tokens,
                                                                int32_t num_heads,
                                                                int32_t head_size) {
  if (total_tokens <= 0 || total_tokens >= (int64_t{1} << 31) || num_heads <= 0) return -1;
  if (head_size != 64 && head_size != 128 && head_size != 256) return -1;
  return fr2::statetune_backward_workspace_floats(total_tokens, num_heads, head_size);
}

extern "C" int fr2_wkv7_statetune_backward(
    const int32_t* sequence_chunk_offsets, const int32_t* chunk_token_starts,
    const int32_t* chunk_token_ends, int32_t num_sequences, int32_t num_chunks,
    int64_t total_tokens, int32_t num_heads, int32_t head_size, int32_t dtype, const void* r,
    const void* decay_logits, const void* k, const void* v, const void* a, const void* b,
    const float* state_dot_a, const void* grad_output, const float* grad_final_state,
    const float* boundary, float* workspace, void* grad_r, void* grad_decay_logits,
    void* grad_k, void* grad_v, void* grad_a, void* grad_b, float* grad_initial_state,
    float scale, void* stream) {
  if (!sequence_chunk_offsets || !chunk_token_starts || !chunk_token_ends ||
      !tokens_ok(r, decay_logits, k, v, a, b, r) || !state_dot_a || !boundary || !workspace ||
      (grad_output != nullptr && !aligned16(grad_output)))
    return FR2_ERR_INVALID_ARGUMENT;
  if (!statetune_sizes_ok(num_sequences, num_chunks, total_tokens, num_heads))
    return FR2_ERR_INVALID_ARGUMENT;
  if (head_size != 64 && head_size != 128 && head_size != 256) return FR2_ERR_UNSUPPORTED;
  if (dtype != FR2_DTYPE_FLOAT16 && dtype != FR2_DTYPE_BFLOAT16) return FR2_ERR_UNSUPPORTED;
  fr2::StateTuneArgs p;
  p.offsets = sequence_chunk_offsets;
  p.starts = chunk_token_starts;
  p.ends = chunk_token_ends;
  p.num_seq = num_sequences;
  p.num_chunks = num_chunks;
  p.heads = num_heads;
  p.tokens = total_tokens;
  p.r = r; p.w = decay_logits; p.k = k; p.v = v; p.a = a; p.b = b;
  p.scale = scale;
  p.sa = const_cast<float*>(state_dot_a);
  p.boundary = const_cast<float*>(boundary);
  p.dy = grad_output;
  p.dfinal = grad_final_state;
  p.dr = grad_r; p.dw = grad_decay_logits; p.dk = grad_k; p.dv = grad_v;
  p.da = grad_a; p.db = grad_b;
  p.dstate0 = grad_initial_state;
  return fr2::launch_statetune_backward(head_size, dtype, p, workspace,
                                        static_cast<hipStream_t>(stream));
}

namespace {

bool statetune_uniform_ok(int32_t batch, int32_t tokens, int32_t num_heads, int32_t chunk_len) {
  return batch > 0 && num_heads > 0 && tokens > 0 && chunk_len > 0 && chunk_len % 16 == 0 &&
         tokens % chunk_len == 0 &&
         static_cast<int64_t>(batch) * num_heads <= (int64_t{1} << 30) / 4 &&
         static_cast<int64_t>(batch) * tokens < (int64_t{1} << 31);
}

}  // namespace

extern "C" int fr2_wkv7_statetune_uniform_forward(
    int32_t batch, int32_t tokens, int32_t num_heads, int32_t chunk_len, float* state,
    const void* r, const void* decay_logits, const void* k, const void* v, const void* a,
    const void* b, void* output, float* boundary, float* state_dot_a, float* snapshots,
    float scale, void* stream) {
  if (!state || !tokens_ok(r, decay_logits, k, v, a, b, output) || !boundary || !state_dot_a ||
      !snapshots)
    return FR2_ERR_INVALID_ARGUMENT;
  if (!statetune_uniform_ok(batch, tokens, num_heads, chunk_len)) return FR2_ERR_INVALID_ARGUMENT;
  fr2::StateTuneArgs p;
  p.heads = num_heads;
  p.r = r; p.w = decay_logits; p.k = k; p.v = v; p.a = a; p.b = b;
  p.scale = scale;
  p.state = state;
  p.y = output;
  p.sa = state_dot_a;
  p.boundary = boundary;
  return fr2::launch_statetune_uniform_forward(batch, tokens, num_heads, chunk_len, p, snapshots,
                                               static_cast<hipStream_t>(stream));
}

extern "C" int64_t fr2_wkv7_statetune_uniform_backward_workspace_floats(int32_t batch,
                                                                        int32_t tokens,
                                                                        int32_t num_heads) {
  if (batch <= 0 || tokens <= 0 || tokens % 16 != 0 || num_heads <= 0) return -1;
  return fr2::pretrain_backward_workspace_floats(batch, tokens, num_heads, 64) +
         static_cast<int64_t>(batch) * num_heads * 64 * 64;
}

extern "C" int fr2_wkv7_statetune_uniform_backward(
    int32_t batch, int32_t tokens, int32_t num_heads, int32_t chunk_len, const void* r,
    const void* decay_logits, const void* k, const void* v, const void* a, const void* b,
    const float* state_dot_a, const void* grad_output, const float* grad_final_state,
    const float* boundary, const float* snapshots, float* workspace, void* grad_r,
    void* grad_decay_logits, void* grad_k, void* grad_v, void* grad_a, void* grad_b,
    float* grad_initial_state, float scale, void* stream) {
  if (!tokens_ok(r, decay_logits, k, v, a, b, grad_output) || !state_dot_a || !boundary ||
      !snapshots || !workspace || !grad_r || !grad_decay_logits || !grad_k || !grad_v ||
      !grad_a || !grad_b || !grad_initial_state)
    return FR2_ERR_INVALID_ARGUMENT;
  if (!statetune_uniform_ok(batch, tokens, num_heads, chunk_len)) return FR2_ERR_INVALID_ARGUMENT;
  fr2::StateTuneArgs p;
  p.heads = num_heads;
  p.r = r; p.w = decay_logits; p.k = k; p.v = v; p.a = a; p.b = b;
  p.scale = scale;
  p.sa = const_cast<float*>(state_dot_a);
  p.boundary = const_cast<float*>(boundary);
  p.dy = grad_output;
  p.dfinal = grad_final_state;
  p.dr = grad_r; p.dw = grad_decay_logits; p.dk = grad_k; p.dv = grad_v;
  p.da = grad_a; p.db = grad_b;
  p.dstate0 = grad_initial_state;
  return fr2::launch_statetune_uniform_backward(batch, tokens, num_heads, chunk_len, p, snapshots,
                                                workspace, static_cast<hipStream_t>(stream));
}

extern "C" int64_t fr2_wkv7_statetune_padded_workspace_bytes(int32_t batch,
                                                             int32_t padded_tokens,
                                                             int32_t num_heads,
                                                             int32_t backward) {
  if (batch <= 0 || batch > 65535 || padded_tokens <= 0 || padded_tokens % 16 != 0 ||
      num_heads <= 0)
    return -1;
  return fr2::statetune_padded_workspace_bytes(batch, padded_tokens, num_heads, backward != 0);
}

extern "C" int fr2_wkv7_statetune_padded_forward(
    int32_t batch, int32_t padded_tokens, int32_t num_heads, int32_t num_chunks,
    const int32_t* row_source, const int32_t* chunk_seq, const int32_t* chunk_pstart,
    float* state, const void* r, const void* decay_logits, const void* k, const void* v,
    const void* a, const void* b, void* output, float* boundary, float* state_dot_a,
    float* snapshots, void* workspace, float scale, void* stream) {
  if (!state || !tokens_ok(r, decay_logits, k, v, a, b, output) || !boundary || !state_dot_a ||
      !snapshots || !workspace || !row_source || !chunk_seq || !chunk_pstart ||
      !aligned16(workspace))
    return FR2_ERR_INVALID_ARGUMENT;
  if (batch <= 0 || batch > 65535 || padded_tokens <= 0 || padded_tokens % 16 != 0 ||
      num_heads <= 0 || num_chunks <= 0)
    return FR2_ERR_INVALID_ARGUMENT;
  fr2::StateTuneArgs p;
  p.heads = num_heads;
  p.r = r; p.w = decay_logits; p.k = k; p.v = v; p.a = a; p.b = b;
  p.scale = scale;
  p.state = state;
  p.y = output;
  p.sa = state_dot_a;
  p.boundary = boundary;
  return fr2::launch_statetune_padded_forward(batch, padded_tokens, num_heads, num_chunks,
                                              row_source, chunk_seq, chunk_pstart, p, snapshots,
                                              workspace, static_cast<hipStream_t>(stream));
}

extern "C" int fr2_wkv7_statetune_padded_backward(
    int32_t batch, int32_t padded_tokens, int32_t num_heads, const int32_t* row_source,
    const int32_t* seq_first_chunk, const void* r, const void* decay_logits, const void* k,
    const void* v, const void* a, const void* b, const float* state_dot_a,
    const void* grad_output, const float* grad_final_state, const float* boundary,
    const float* snapshots, void* workspace, void* grad_r, void* grad_decay_logits,
    void* grad_k, void* grad_v, void* grad_a, void* grad_b, float* grad_initial_state,
    float scale, void* stream) {
  if (!tokens_ok(r, decay_logits, k, v, a, b, grad_output) || !state_dot_a || !boundary ||
      !snapshots || !workspace || !aligned16(workspace) || !row_source || !seq_first_chunk ||
      !grad_initial_state || !params_aligned({grad_r, grad_decay_logits, grad_k, grad_v, grad_a,
                                              grad_b, state_dot_a}) ||
      !grad_r || !grad_decay_logits || !grad_k || !grad_v || !grad_a || !grad_b)
    return FR2_ERR_INVALID_ARGUMENT;
  if (batch <= 0 || batch > 65535 || padded_tokens <= 0 || padded_tokens % 16 != 0 ||
      num_heads <= 0)
    return FR2_ERR_INVALID_ARGUMENT;
  fr2::StateTuneArgs p;
  p.heads = num_heads;
  p.r = r; p.w = decay_logits; p.k = k; p.v = v; p.a = a; p.b = b;
  p.scale = scale;
  p.sa = const_cast<float*>(state_dot_a);
  p.boundary = const_cast<float*>(boundary);
  p.dy = grad_output;
  p.dfinal = grad_final_state;
  p.dr = grad_r; p.dw = grad_decay_logits; p.dk = grad_k; p.dv = grad_v;
  p.da = grad_a; p.db = grad_b;
  p.dstate0 = grad_initial_state;
  return fr2::launch_statetune_padded_backward(batch, padded_tokens, num_heads, row_source,
                                               seq_first_chunk, p, snapshots, workspace,
                                               static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// producer / consumer stages of the layer (fp16)
// ---------------------------------------------------------------------------
// The packed fp32-state recurrence with the kk / a-gate producer stage of
// wkv_prepare fused into the chunked kernel's load stage: the recurrence's
// k, a, b come from the projected key, the low-rank a-gate logits a12 and the
// per-channel k_k, a0, k_a (never stored), and the gated key the readout
// needs is written to new_k.  On the chunked kernel the plain entry's
// policy picks (one workgroup or one wavefront per unit); where that policy
// picks the decode kernel (the longest sequence at most 4 tokens, 6 with
// many units) or at head sizes other than 64, FR2_ERR_UNSUPPORTED (the caller
// then runs fr2_tmix_kk_a_gate_forward and the plain entry).
extern "C" int fr2_wkv7_recurrent_fp32_forward_kk_gate(
    const int32_t* query_start_loc, const int32_t* state_indices, const int32_t* status,
    int32_t num_sequences, int32_t num_heads, int32_t head_size, int64_t total_tokens,
    int32_t max_seqlen, int32_t dtype, float* state, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a12, const void* k_k,
    const void* a0, const void* k_a, void* new_k, void* output, float scale, void* stream) {
  if (!params_aligned({decay_bias, k_k, a0, k_a})) return FR2_ERR_INVALID_ARGUMENT;
  if (!query_start_loc || !state_indices || !status || !state || !k_k || !a0 || !k_a ||
      !tokens_ok(r, decay_logits, k, v, a12, new_k, output))
    return FR2_ERR_INVALID_ARGUMENT;
  if (num_sequences <= 0 || num_sequences > 65535 || num_heads <= 0 || total_tokens <= 0)
    return FR2_ERR_INVALID_ARGUMENT;
  const int64_t units = static_cast<int64_t>(num_sequences) * num_heads;
  // where the plain policy picks the decode kernel (or the longest sequence
  // is unknown), fp16 batches take the two-kernel form (the separate gate
  // kernel is fp16); bf16 batches run on the wavefront chunked kernel, which
  // handles sequences of any length
  const bool short_batch = max_seqlen <= 0 || decode_first(units, max_seqlen);
  if (head_size != 64 || (short_batch && dtype != FR2_DTYPE_BFLOAT16))
    return FR2_ERR_UNSUPPORTED;
  SegArgs p;
  p.bounds = query_start_loc;
  p.slots = state_indices;
  p.status = status;
  p.num_heads = num_heads;
  p.out_elems = total_tokens * num_heads * head_size;
  p.state_in = state;
  p.state_out = state;
  p.r = r; p.logits = decay_logits; p.bias = decay_bias; p.k = k; p.v = v; p.a = a12;
  p.b = k;   // unused by the fused stage (slot 5 reads the key's other half)
  p.kk_scale = k_k; p.a_bias = a0; p.k_a = k_a; p.new_k = new_k;
  p.y = output;
  p.scale = scale;
  // the chunked kernel the plain entry's policy picks, with the stage fused
  return !short_batch && workgroup_chunked(units, max_seqlen, total_tokens, num_sequences)
             ? fr2::launch_chunked_kk(dtype, p, num_sequences, static_cast<hipStream_t>(stream))
             : fr2::launch_chunked_wave(dtype, p, num_sequences, max_seqlen,
                                        static_cast<hipStream_t>(stream));
}

extern "C" int fr2_wkv7_recurrent_fp32_forward_kk_gate_readout(
    const int32_t* query_start_loc, const int32_t* state_indices, const int32_t* status,
    int32_t num_sequences, int32_t num_heads, int32_t head_size, int64_t total_tokens,
    int32_t max_seqlen, int32_t dtype, float* state, const void* r, const void* decay_logits,
    const void* decay_bias, const void* k, const void* v, const void* a12, const void* k_k,
    const void* a0, const void* k_a, const void* g, const void* r_k, const void* ln_weight,
    const void* ln_bias, void* new_k, void* readout, void* output, float scale,
    void* stream) {
  if (!params_aligned({decay_bias, k_k, a0, k_a, r_k, ln_weight, ln_bias}))
    return FR2_ERR_INVALID_ARGUMENT;
  if (!query_start_loc || !state_indices || !status || !state || !k_k || !a0 || !k_a ||
      !r_k || !ln_weight || !ln_bias || !tokens_ok(r, decay_logits, k, v, a12, new_k, readout) ||
      !aligned16(g) || !g || (output != nullptr && !aligned16(output)))
    return FR2_ERR_INVALID_ARGUMENT;
  if (num_sequences <= 0 || num_sequences > 65535 || num_heads <= 0 || total_tokens <= 0)
    return FR2_ERR_INVALID_ARGUMENT;
  const int64_t units = static_cast<int64_t>(num_sequences) * num_heads;
  // where the plain policy picks the decode kernel (or the longest sequence
  // is unknown), fp16 batches take the two-kernel form (the separate gate
  // kernel is fp16); bf16 batches run on the wavefront chunked kernel, which
  // handles sequences of any length
  const bool short_batch = max_seqlen <= 0 || decode_first(units, max_seqlen);
  if (head_size != 64 || (short_batch && dtype != FR2_DTYPE_BFLOAT16))
    return FR2_ERR_UNSUPPORTED;
  SegArgs p;
  p.bounds = query_start_loc;
  p.slots = state_indices;
  p.status = status;
  p.num_heads = num_heads;
  p.out_elems = total_tokens * num_heads * head_size;
  p.state_in = state;
  p.state_out = state;
  p.r = r; p.logits = decay_logits; p.bias = decay_bias; p.k = k; p.v = v; p.a = a12;
  p.b = k;   // unused by the fused stage (slot 5 reads the key's other half)
  p.kk_scale = k_k; p.a_bias = a0; p.k_a = k_a; p.new_k = new_k;
  p.ro_g = g; p.ro_rk = r_k; p.ro_lnw = ln_weight; p.ro_lnb = ln_bias; p.ro_out = readout;
  p.y = output;
  p.scale = scale;
  // the chunked kernel the plain entry's policy picks, with the stage fused
  return !short_batch && workgroup_chunked(units, max_seqlen, total_tokens, num_sequences)
             ? fr2::launch_chunked_kk(dtype, p, num_sequences, static_cast<hipStream_t>(stream))
             : fr2::launch_chunked_wave(dtype, p, num_sequences, max_seqlen,
                                        static_cast<hipStream_t>(stream));
}

extern "C" int fr2_tmix_kk_a_gate_forward(int64_t tokens, int32_t num_heads, int32_t head_size,
                                          const void* k, const void* k_k, const void* a0,
                                          const void* a12, const void* k_a, void* new_k,
                                          void* neg_kk, void* kka, void* stream) {
  if (!params_aligned({k_k, a0, k_a, k, a12, new_k, neg_kk, kka}))
    return FR2_ERR_INVALID_ARGUMENT;
  if (!k || !k_k || !a0 || !a12 || !k_a || !new_k || !neg_kk || !kka)
    return FR2_ERR_INVALID_ARGUMENT;
  if (tokens <= 0 || num_heads <= 0) return FR2_ERR_INVALID_ARGUMENT;
  if (head_size != 64 && head_size != 128 && head_size != 256) return FR2_ERR_UNSUPPORTED;
  return fr2::launch_kk_a_gate(tokens, num_heads, head_size, k, k_k, a0, a12, k_a, new_k, neg_kk,
                               kka, static_cast<hipStream_t>(stream));
}

extern "C" int fr2_tmix_lowrank_activate(int64_t n_tanh, const void* tanh_in, void* tanh_out,
                                         int64_t n_sigmoid, const void* sigmoid_in,
                                         void* sigmoid_out, void* stream) {
  if (!params_aligned({tanh_in, tanh_out, sigmoid_in, sigmoid_out}))
    return FR2_ERR_INVALID_ARGUMENT;
  if (n_tanh < 0 || n_sigmoid < 0) return FR2_ERR_INVALID_ARGUMENT;
  if ((n_tanh > 0 && (!tanh_in || !tanh_out)) || (n_sigmoid > 0 && (!sigmoid_in || !sigmoid_out)))
    return FR2_ERR_INVALID_ARGUMENT;
  return fr2::launch_lowrank_act(n_tanh, tanh_in, tanh_out, n_sigmoid, sigmoid_in, sigmoid_out,
                                 static_cast<hipStream_t>(stream));
}

extern "C" int fr2_tmix_vres_forward(int64_t tokens, int32_t channels, const void* value,
                                     const void* v_first, const void* v0, const void* v12,
                                     void* output, void* stream) {
  if (!params_aligned({value, v_first, v0, v12, output})) return FR2_ERR_INVALID_ARGUMENT;
  if (!value || !v_first || !v0 || !v12 || !output) return FR2_ERR_INVALID_ARGUMENT;
  if (tokens <= 0 || channels <= 0 || channels % 8 != 0) return FR2_ERR_INVALID_ARGUMENT;
  return fr2::launch_vres(tokens, channels, value, v_first, v0, v12, output,
                          static_cast<hipStream_t>(stream));
}

extern "C" int fr2_tmix_readout_prelinear_forward(int64_t tokens, int32_t num_heads,
                                                  int32_t head_size, const void* wkv_output,
                                                  const void* r, const void* k, const void* v,
                                                  const void* r_k, const void* ln_weight,
                                                  const void* ln_bias, const void* gate,
                                                  void* output, void* stream) {
  if (!params_aligned({r_k, ln_weight, ln_bias, wkv_output, r, k, v, gate, output}))
    return FR2_ERR_INVALID_ARGUMENT;
  if (!wkv_output || !r || !k || !v || !r_k || !ln_weight || !ln_bias || !gate || !output)
    return FR2_ERR_INVALID_ARGUMENT;
  if (tokens <= 0 || num_heads <= 0) return FR2_ERR_INVALID_ARGUMENT;
  if (head_size != 64 && head_size != 128 && head_size != 256) return FR2_ERR_UNSUPPORTED;
  return fr2::launch_readout_prelinear(tokens, num_heads, head_size, wkv_output, r, k, v, r_k,
                                       ln_weight, ln_bias, gate, output,
                                       static_cast<hipStream_t>(stream));
}

// Blocks of the chunked kernels that failed closed because a wave hand-off
// wait gave up (their outputs are NaN and their state untouched).  Waits for
// `stream`, reads the current device's counter and, with reset != 0, clears
// it.  No counterpart in the reference, whose kernels have no bounded waits.
extern "C" int fr2_handoff_fault_count(int32_t* count, int32_t reset, void* stream) {
  if (!count) return FR2_ERR_INVALID_ARGUMENT;
  int* word = fr2::handoff_fault_word();
  if (word == nullptr) return FR2_ERR_LAUNCH;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int32_t host = 0;
  if (hipMemcpyAsync(&host, word, sizeof(host), hipMemcpyDeviceToHost, s) != hipSuccess ||
      (reset != 0 && hipMemsetAsync(word, 0, sizeof(int32_t), s) != hipSuccess) ||
      hipStreamSynchronize(s) != hipSuccess) {
    (void)hipGetLastError();
    return FR2_ERR_LAUNCH;
  }
  *count = host;
  return FR2_OK;
}

// Polls a chunked-kernel hand-off wait makes before it gives up, for every
// later launch in the process (negative: the default, 2^20).  A test hook:
// with 0 the first wait that finds its counter short gives up, which lets a
// test check the fail-closed path while every kernel still exits normally.
extern "C" int fr2_debug_set_handoff_spin_limit(int32_t polls) {
  fr2::set_handoff_spin_limit(polls);
  return FR2_OK;
}

// Variant switch of the workgroup-per-unit chunked kernel for the plain
// contract (0: two key waves per chunk, 1: one key wave per chunk, a ring
// of four chunks): for measuring the two against each other.
extern "C" int fr2_debug_set_chunk_ring(int32_t on) {
  fr2::set_chunk_ring(on);
  return FR2_OK;
}

// Test hook: while on, the chunked kernel's key waves never publish their
// operators to the state waves, so every block stalls at its first
// operator wait and, after the spin limit, fails closed; every kernel still
// runs to its end.
extern "C" int fr2_debug_set_handoff_stall(int32_t on) {
  fr2::set_handoff_stall(on != 0);
  return FR2_OK;
}
