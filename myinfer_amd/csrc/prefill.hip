// Causal chunked-prefill attention over the quantized cache (MFMA). Placeholder until the
// kernel lands: reports "not supported" so callers fail loudly.

#include "common.h"
#include "launch.h"

namespace kvq {

size_t prefill_workspace_bytes(int, int, int, int, int, int, int, int) { return 256; }

hipError_t launch_prefill(const kvq_rows*, const kvq_qtensor*, const kvq_qtensor*, const int32_t*, const kvq_rows*,
                          int, int, int, int, int, int, int, int, float, int, int, void*, hipStream_t) {
  return hipErrorNotSupported;
}

}  // namespace kvq
