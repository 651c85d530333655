// Causal prefill attention (MFMA) -- placeholder until the tiled kernel lands.
#include "common.h"
#include "internal.h"

namespace qxh {

hipError_t launch_prefill_attention(const ShapeDims& s, const KvLayer& kv, uint32_t start_position, uint32_t tokens,
                                    const void* query, int query_dtype, void* out, int out_dtype, hipStream_t st,
                                    int* dispatches) {
    (void)s; (void)kv; (void)start_position; (void)tokens; (void)query; (void)query_dtype; (void)out;
    (void)out_dtype; (void)st;
    *dispatches = 0;
    return hipErrorNotSupported;
}

}  // namespace qxh
