// Device-side validation of packed varlen metadata (one workgroup).
//
// Behaviour follows validate_recurrent_metadata_kernel
// (csrc/validation/recurrent_metadata.cu:24-132): status[0] collects error
// bits, status[1..2] hold the active token / sequence counts (zeroed on
// error), and a static ticket validates a private snapshot of the metadata so
// that later writes to the caller's tensors cannot change what the kernels
// read.  The graph form reads the active counts from device scalars and only
// checks the active prefix, so padded tails may hold anything.
#include "common.h"
#include "../../include/flashrwkv2_amd.h"

namespace fr2 {

constexpr int kMetaThreads = 256;

__global__ __launch_bounds__(kMetaThreads) void validate_metadata_kernel(
    const int32_t* __restrict__ qsl, const int32_t* __restrict__ slots,
    int num_sequences, int total_tokens, int pool_size, int max_seqlen,
    const int32_t* __restrict__ live_tokens,
    const int32_t* __restrict__ live_sequences, int32_t* __restrict__ status,
    int32_t* __restrict__ seen, int32_t* __restrict__ qsl_copy,
    int32_t* __restrict__ slots_copy) {
  __shared__ int err_bits;
  __shared__ int n_tok;
  __shared__ int n_seq;
  const int tid = threadIdx.x;

  if (tid == 0) {
    int t = live_tokens ? live_tokens[0] : total_tokens;
    int s = live_sequences ? live_sequences[0] : num_sequences;
    int e = 0;
    const bool bad = t < 0 || t > total_tokens || s < 0 || s > num_sequences ||
                     ((t == 0) != (s == 0));
    if (bad) {
      e = FR2_META_INVALID_ACTIVE_COUNT;
      t = 0;
      s = 0;
    }
    err_bits = e;
    n_tok = t;
    n_seq = s;
  }

  for (int i = tid; i < pool_size; i += kMetaThreads) seen[i] = -1;
  if (qsl_copy != nullptr) {
    for (int i = tid; i <= num_sequences; i += kMetaThreads) {
      qsl_copy[i] = qsl[i];
      if (i < num_sequences) slots_copy[i] = slots[i];
    }
  }
  __syncthreads();

  const int32_t* q = qsl_copy ? qsl_copy : qsl;
  const int32_t* sl = slots_copy ? slots_copy : slots;
  const int active_tokens = n_tok;
  const int active_seqs = n_seq;

  if (tid == 0 && err_bits == 0) {
    if (q[0] != 0 || q[active_seqs] != active_tokens) {
      atomicOr(&err_bits, FR2_META_INVALID_ENDPOINT);
    }
  }

  int mine = 0;
  for (int i = tid; i < active_seqs; i += kMetaThreads) {
    const int lo = q[i];
    const int hi = q[i + 1];
    if (lo < 0 || hi <= lo || hi > active_tokens) {
      mine |= FR2_META_INVALID_SEQUENCE_RANGE;
    } else if (hi - lo > max_seqlen) {
      mine |= FR2_META_SEQUENCE_TOO_LONG;
    }
    const int slot = sl[i];
    if (slot < 0 || slot >= pool_size) {
      mine |= FR2_META_INVALID_STATE_SLOT;
    } else if (atomicCAS(&seen[slot], -1, i) != -1) {
      mine |= FR2_META_DUPLICATE_STATE_SLOT;
    }
  }
  if (mine) atomicOr(&err_bits, mine);
  __syncthreads();

  if (tid == 0) {
    const int e = err_bits;
    status[0] = e;
    status[1] = e ? 0 : active_tokens;
    status[2] = e ? 0 : active_seqs;
  }
}

}  // namespace fr2

extern "C" int fr2_wkv7_prepare_metadata(
    const int32_t* query_start_loc, const int32_t* state_indices,
    int32_t num_sequences, int32_t total_tokens, int32_t state_pool_size,
    int32_t max_seqlen, const int32_t* num_active_tokens,
    const int32_t* num_active_sequences, int32_t* status, int32_t* seen_slots,
    int32_t* query_start_loc_snapshot, int32_t* state_indices_snapshot,
    void* stream) {
  if (!query_start_loc || !state_indices || !status || !seen_slots)
    return FR2_ERR_INVALID_ARGUMENT;
  if (num_sequences <= 0 || state_pool_size <= 0 || total_tokens < 0)
    return FR2_ERR_INVALID_ARGUMENT;
  if ((query_start_loc_snapshot == nullptr) != (state_indices_snapshot == nullptr))
    return FR2_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(fr2::validate_metadata_kernel, dim3(1),
                     dim3(fr2::kMetaThreads), 0,
                     static_cast<hipStream_t>(stream), query_start_loc,
                     state_indices, num_sequences, total_tokens,
                     state_pool_size, max_seqlen, num_active_tokens,
                     num_active_sequences, status, seen_slots,
                     query_start_loc_snapshot, state_indices_snapshot);
  return fr2::record_launch();
}
