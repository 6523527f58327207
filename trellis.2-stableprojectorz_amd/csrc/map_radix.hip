// Radix-sort neighbor-map path (placeholder until the LSD radix sort lands).
#include "tsc_internal.h"

namespace tsc {
int map_build_radix(tsc_ctx*, const int32_t*, int64_t, int32_t, int32_t, int32_t, int32_t,
                    const int32_t*, void*, int32_t*, int32_t*, uint32_t*) {
  return fail(TSC_ERR_UNSUPPORTED, "map_build: radix path not built yet");
}
}  // namespace tsc
