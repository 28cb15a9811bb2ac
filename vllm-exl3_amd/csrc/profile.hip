// Per-phase timing ring (see profile.h).
#include "profile.h"

#include <vector>

#include "exl3_common.h"

namespace exl3 {
namespace {

struct Ring {
    bool on = false;
    int max_calls = 0;
    int calls = 0;        // calls begun
    int max_bound = 0;    // highest boundary index recorded + 1
    std::vector<hipEvent_t> ev;  // [max_calls][kProfilePhases + 1]
};

Ring& ring() {
    static Ring r;
    return r;
}

}  // namespace

void profile_begin_call() {
    Ring& r = ring();
    if (r.on) ++r.calls;
}

void profile_mark(int b, hipStream_t st) {
    Ring& r = ring();
    if (!r.on || r.calls < 1 || r.calls > r.max_calls || b < 0 || b > kProfilePhases) return;
    (void)hipEventRecord(r.ev[(size_t)(r.calls - 1) * (kProfilePhases + 1) + b], st);
    if (b + 1 > r.max_bound) r.max_bound = b + 1;
}

}  // namespace exl3

using namespace exl3;

EXL3_API int exl3_profile_begin(int max_calls) {
    EXL3_CHECK(max_calls >= 1 && max_calls <= 100000, "max_calls must be in [1, 100000]");
    Ring& r = ring();
    const size_t need = (size_t)max_calls * (kProfilePhases + 1);
    while (r.ev.size() < need) {
        hipEvent_t e;
        EXL3_HIP(hipEventCreate(&e));
        r.ev.push_back(e);
    }
    r.on = true;
    r.max_calls = max_calls;
    r.calls = 0;
    r.max_bound = 0;
    return kOk;
}

// phase_ms[p] = sum over recorded calls of elapsed(boundary p -> p + 1);
// *n_calls = calls recorded, *n_phases = phases seen.  Waits for the events.
EXL3_API int exl3_profile_end(double* phase_ms, int max_phases, int* n_calls, int* n_phases) {
    Ring& r = ring();
    EXL3_CHECK(r.on, "profiling was not started");
    r.on = false;
    const int calls = r.calls < r.max_calls ? r.calls : r.max_calls;
    const int phases = r.max_bound > 0 ? r.max_bound - 1 : 0;
    for (int p = 0; p < max_phases; ++p) phase_ms[p] = 0.0;
    for (int c = 0; c < calls; ++c) {
        for (int p = 0; p < phases && p < max_phases; ++p) {
            hipEvent_t a = r.ev[(size_t)c * (kProfilePhases + 1) + p];
            hipEvent_t b = r.ev[(size_t)c * (kProfilePhases + 1) + p + 1];
            EXL3_HIP(hipEventSynchronize(b));
            float ms = 0.f;
            EXL3_HIP(hipEventElapsedTime(&ms, a, b));
            phase_ms[p] += ms;
        }
    }
    *n_calls = calls;
    *n_phases = phases;
    return kOk;
}
