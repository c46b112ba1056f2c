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
    // `height` rows of `width` bytes (row pitches dpitch and spitch), the rows
    // split over the pool's threads
    void parallel_copy_rows(char* dst, const char* src, size_t height, size_t width, size_t dpitch, size_t spitch);
    // synchronous: columns [bounds[i], bounds[i+1]) of the n x width f32
    // matrix src, each band once ready[i] has completed, into the same columns
    // of host dst.  The bands cross the bus on stream cs into two pinned
    // buffers, band i + 1 in flight while band i is copied out.
    void bands_from_device(float* dst, const float* src, size_t n, size_t width, const size_t* bounds,
                           const hipEvent_t* ready, int bands, hipStream_t cs);

    // a process-wide copier; calls on it are serialised by its own lock
    static HostCopier& shared();
    std::mutex& lock() { return use_; }

private:
    void worker(int index);

    static constexpr size_t kChunk = size_t(4) << 20;
    void* pinned_[2] = {nullptr, nullptr};
    hipEvent_t done_[2] = {nullptr, nullptr};
    void* band_pinned_[2] = {nullptr, nullptr};  // bands_from_device's staging, grown as needed
    size_t band_bytes_ = 0;
    hipEvent_t band_done_[2] = {nullptr, nullptr};
    std::vector<std::thread> threads_;
    std::mutex mu_, use_;
    std::condition_variable work_cv_, done_cv_;
    // the current job: part k of parts goes to worker k - 1 (part 0 stays on
    // the calling thread)
    char* job_dst_ = nullptr;
    const char* job_src_ = nullptr;
    size_t job_bytes_ = 0;
    // a job of rows (job_rows_ > 0): job_bytes_ per row at these pitches
    size_t job_rows_ = 0, job_dpitch_ = 0, job_spitch_ = 0;
    int parts_ = 0, pending_ = 0;
    unsigned long generation_ = 0;
    bool stop_ = false;
};

}  // namespace tvara_amd
