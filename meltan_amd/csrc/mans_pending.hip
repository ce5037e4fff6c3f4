// Entry points whose kernels are not in this build yet.  Each reports
// MANS_PIPELINE_UNAVAILABLE (tier-degradeable, Errors.swift:21-31), so a
// caller falls back to the next tier instead of failing.
#include "mans_hip.h"
#include "mans_runtime.hpp"

using namespace mans;

static int unavailable(const char* what) {
    return fail(MANS_PIPELINE_UNAVAILABLE, std::string(what) + " is not available in this build");
}

extern "C" {
int mans_ivfpq_build(mans_ctx*, const mans_corpus*, const float*, int64_t, const float*, int64_t,
                     uint32_t, mans_ivfpq** out) {
    if (out) *out = nullptr;
    return unavailable("IVF-PQ");
}
int mans_ivfpq_search(mans_ctx*, const mans_ivfpq*, const float*, int64_t, int64_t, int64_t, int64_t,
                      float*, uint32_t*) { return unavailable("IVF-PQ"); }
int mans_ivfpq_search_device(mans_ctx*, const mans_ivfpq*, const float*, int64_t, int64_t, int64_t,
                             int64_t, float*, uint32_t*, void*) { return unavailable("IVF-PQ"); }
int mans_ivfpq_download_codes(const mans_ivfpq*, uint8_t*, int32_t*) { return unavailable("IVF-PQ"); }
void mans_ivfpq_release(mans_ivfpq*) {}
}
