// Device-to-pageable-host copies at pinned-memory speed: the data moves in
// chunks through two pinned staging buffers (DMA of chunk i+1 in flight while
// chunk i is copied out) and a small pool of host threads copies each chunk
// into the caller's buffer.  A single hipMemcpy into pageable memory stages
// through the driver's own buffers on one thread.
#pragma once

#include <hip/hip_runtime.h>

#include <condition_variable>
#include <cstddef>
#include <mutex>
#include <thread>
#include <vector>

namespace tvara_amd {

class HostCopier {
public:
    HostCopier();
    ~HostCopier();
    HostCopier(const HostCopier&) = delete;
    HostCopier& operator=(const HostCopier&) = delete;
    // synchronous: returns when `bytes` from device `src` (after the work
    // already queued on `s`) are in host `dst`
    void from_device(void* dst, const void* src, size_t bytes, hipStream_t s);
    // host-to-host copy split over the pool's threads, parts of at least
    // 2^min_part_log2 bytes (one thread copies 512 KiB in about 5 us, under
    // the cost of waking the pool)
    void parallel_copy(char* dst, const char* src, size_t bytes, int min_part_log2 = 21);

    // a process-wide copier; calls on it are serialised by its own lock
    static HostCopier& shared();
    std::mutex& lock() { return use_; }

private:
    void worker(int index);

    static constexpr size_t kChunk = size_t(4) << 20;
    void* pinned_[2] = {nullptr, nullptr};
    hipEvent_t done_[2] = {nullptr, nullptr};
    std::vector<std::thread> threads_;
    std::mutex mu_, use_;
    std::condition_variable work_cv_, done_cv_;
    // the current job: part k of parts goes to worker k - 1 (part 0 stays on
    // the calling thread)
    char* job_dst_ = nullptr;
    const char* job_src_ = nullptr;
    size_t job_bytes_ = 0;
    int parts_ = 0, pending_ = 0;
    unsigned long generation_ = 0;
    bool stop_ = false;
};

}  // namespace tvara_amd
