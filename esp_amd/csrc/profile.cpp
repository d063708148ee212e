#include "profile.hpp"

#include <map>
#include <mutex>
#include <utility>
#include <vector>

namespace esp {

thread_local bool g_capturing = false;

namespace {
struct Fam {
    bool on = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
    unsigned long long launches = 0;
    double ms = 0;
};
std::mutex mu;
std::map<std::string, Fam> fams;
std::vector<hipEvent_t> pool;
bool any_on = false;

void drain(Fam &f) {
    for (auto &e : f.pending) {
        float ms = 0;
        if (hipEventSynchronize(e.second) == hipSuccess && hipEventElapsedTime(&ms, e.first, e.second) == hipSuccess) {
            f.ms += ms;
            ++f.launches;
        }
        pool.push_back(e.first);
        pool.push_back(e.second);
    }
    f.pending.clear();
}
}  // namespace

bool prof_enabled(const char *family) {
    if (!any_on) return false;
    std::lock_guard<std::mutex> g(mu);
    auto it = fams.find(family);
    return it != fams.end() && it->second.on;
}

hipEvent_t prof_event() {
    std::lock_guard<std::mutex> g(mu);
    if (!pool.empty()) {
        hipEvent_t e = pool.back();
        pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    (void)hipEventCreate(&e);
    return e;
}

void prof_record(const char *family, hipEvent_t start, hipEvent_t end) {
    std::lock_guard<std::mutex> g(mu);
    Fam &f = fams[family];
    f.pending.emplace_back(start, end);
    if (f.pending.size() > 4096) drain(f);
}

void prof_count(const char *family) {
    std::lock_guard<std::mutex> g(mu);
    ++fams[family].launches;
}

int prof_enable(const char *family, int on) {
    std::lock_guard<std::mutex> g(mu);
    Fam &f = fams[family];
    drain(f);
    f.on = on != 0;
    f.launches = 0;
    f.ms = 0;
    any_on = false;
    for (auto &kv : fams) any_on |= kv.second.on;
    return 0;
}

int prof_read(const char *family, unsigned long long *launches, double *total_ms) {
    std::lock_guard<std::mutex> g(mu);
    Fam &f = fams[family];
    drain(f);
    if (launches) *launches = f.launches;
    if (total_ms) *total_ms = f.ms;
    return 0;
}

}  // namespace esp
