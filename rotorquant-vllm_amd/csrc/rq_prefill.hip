// INT8-MFMA causal prefill over the packed cache (placeholder until the kernel lands).
#include "rq_common.h"

extern "C" int rq_int8_prefill(const void *, int32_t, int64_t, int32_t, int64_t, int64_t, const int32_t *, int64_t,
                               int64_t, const uint8_t *, int64_t, int32_t, int64_t, int64_t, int32_t, int32_t,
                               const int32_t *, int64_t, int64_t, const int32_t *, const float *, int32_t,
                               const float *, int32_t, const float *, int32_t, float, void *, int64_t, int64_t,
                               void *) {
    rq::set_error("rq_int8_prefill: not implemented yet");
    return RQ_EINVAL;
}
