// Chunked MFMA prefill (placeholder until the kernel lands).
#include "recurrent.h"

namespace fr2 {
int launch_chunked(int dtype, const SegArgs& p, int nseg, int max_seqlen,
                   hipStream_t s) {
  (void)dtype; (void)p; (void)nseg; (void)max_seqlen; (void)s;
  return FR2_ERR_UNSUPPORTED;
}
}  // namespace fr2
