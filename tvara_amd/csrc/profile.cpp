// Per-kernel timing of the library's own launches: start/stop events that the
// runtime stamps with each kernel's execution (hipExtLaunchKernel).
#include <hip/hip_runtime.h>

#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "common.hpp"

namespace tvara_amd {
namespace {
struct Pending {
    std::string name;
    hipEvent_t begin, end;
};
std::mutex mutex;
bool enabled = false;
std::vector<Pending> pending;
std::map<std::string, std::pair<double, size_t>> totals;

void drain() {
    for (auto& p : pending) {
        float ms = 0.f;
        TVARA_HIP(hipEventSynchronize(p.end));
        TVARA_HIP(hipEventElapsedTime(&ms, p.begin, p.end));
        auto& t = totals[p.name];
        t.first += ms;
        t.second += 1;
        (void)hipEventDestroy(p.begin);
        (void)hipEventDestroy(p.end);
    }
    pending.clear();
}
}  // namespace

bool profile_events(hipEvent_t* start, hipEvent_t* stop) {
    std::lock_guard<std::mutex> lock(mutex);
    if (!enabled) return false;
    TVARA_HIP(hipEventCreate(start));
    if (hipEventCreate(stop) != hipSuccess) {
        (void)hipEventDestroy(*start);
        throw std::runtime_error("hipEventCreate failed");
    }
    return true;
}

void profile_record(const char* name, hipEvent_t start, hipEvent_t stop) {
    std::lock_guard<std::mutex> lock(mutex);
    pending.push_back({name, start, stop});
}

void profile_enable(bool on) {
    std::lock_guard<std::mutex> lock(mutex);
    enabled = on;
}

void profile_read(const char* prefix, double* ms, size_t* launches) {
    std::lock_guard<std::mutex> lock(mutex);
    drain();
    double total = 0;
    size_t count = 0;
    for (auto& [name, t] : totals) {
        if (prefix && *prefix && name != prefix) continue;  // NULL or "" selects every kernel
        total += t.first;
        count += t.second;
    }
    *ms = total;
    *launches = count;
}

void profile_reset() {
    std::lock_guard<std::mutex> lock(mutex);
    drain();
    totals.clear();
}

}  // namespace tvara_amd
