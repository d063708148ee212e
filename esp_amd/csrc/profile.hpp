// Per-kernel-family launch timing with HIP events recorded on the launch
// stream. Disabled families cost one map lookup per launch.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

namespace esp {

bool prof_enabled(const char *family);
void prof_record(const char *family, hipEvent_t start, hipEvent_t end);
hipEvent_t prof_event();  // from the pool

// Capturing code must not record events: profiling is eager-only.
extern thread_local bool g_capturing;

struct Prof {
    const char *fam;
    hipStream_t s;
    hipEvent_t a = nullptr, b = nullptr;
    Prof(const char *family, hipStream_t stream) : fam(family), s(stream) {
        if (!g_capturing && prof_enabled(fam)) {
            a = prof_event();
            b = prof_event();
            (void)hipEventRecord(a, s);
        }
    }
    ~Prof() {
        if (a) {
            (void)hipEventRecord(b, s);
            prof_record(fam, a, b);
        }
    }
};

// Count one occurrence of a host-side event under `family` (read back as
// its launch count, total time 0), whether or not timing is enabled.
void prof_count(const char *family);
int prof_enable(const char *family, int on);
int prof_read(const char *family, unsigned long long *launches, double *total_ms);

}  // namespace esp
