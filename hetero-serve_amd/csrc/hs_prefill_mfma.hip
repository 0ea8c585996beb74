// Matrix-core causal prefill over the paged cache (gfx950 MFMA).
#include "hs_kernels.h"

namespace hs {

int launch_prefill_mfma(const float*, const int32_t*, int, int, const void*, const void*, int, int,
                        const int32_t*, const int32_t*, float*, int, int, int, int, int, int,
                        float, hipStream_t) {
  return fail(HS_EUNSUPPORTED, "MFMA prefill is not built in this library yet");
}

}  // namespace hs
