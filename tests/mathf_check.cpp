// Host build of tmq_mathf.h for the CPU tests: compares the engine's expf
// and logf with the host libm's over a strided sample of all 2^32 float bit
// patterns, and exports the RoPE table the engine uploads at load.
#include <cmath>
#include <cstdint>
#include <cstring>

#include "tmq_mathf.h"

extern "C" uint64_t tmqm_expf_mismatches(uint64_t stride, uint64_t offset, uint32_t* first_bad) {
    uint64_t bad = 0;
    for (uint64_t u = offset; u < (1ull << 32); u += stride) {
        float x;
        const uint32_t b = (uint32_t)u;
        memcpy(&x, &b, 4);
        const float a = tmq_math::tmq_expf(x), e = expf(x);
        uint32_t ab, eb;
        memcpy(&ab, &a, 4);
        memcpy(&eb, &e, 4);
        const bool both_nan = std::isnan(a) && std::isnan(e);
        if (ab != eb && !both_nan) {
            if (!bad && first_bad) *first_bad = b;
            bad++;
        }
    }
    return bad;
}

extern "C" float tmqm_expf(float x) { return tmq_math::tmq_expf(x); }

extern "C" uint64_t tmqm_logf_mismatches(uint64_t stride, uint64_t offset, uint32_t* first_bad) {
    uint64_t bad = 0;
    for (uint64_t u = offset; u < (1ull << 32); u += stride) {
        float x;
        const uint32_t b = (uint32_t)u;
        memcpy(&x, &b, 4);
        const float a = tmq_math::tmq_logf(x), e = logf(x);
        uint32_t ab, eb;
        memcpy(&ab, &a, 4);
        memcpy(&eb, &e, 4);
        const bool both_nan = std::isnan(a) && std::isnan(e);
        if (ab != eb && !both_nan) {
            if (!bad && first_bad) *first_bad = b;
            bad++;
        }
    }
    return bad;
}

extern "C" float tmqm_logf(float x) { return tmq_math::tmq_logf(x); }

extern "C" void tmqm_rope_table(float base, int head_dim, int max_pos, float* out) {
    tmq_math::rope_table(base, head_dim, max_pos, out);
}
