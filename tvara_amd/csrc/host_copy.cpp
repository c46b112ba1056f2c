// Chunked, multi-threaded device-to-host copies (see host_copy.hpp).
#include "host_copy.hpp"

#include <algorithm>
#include <cstring>

#include "common.hpp"

namespace tvara_amd {

HostCopier::HostCopier() {
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const int workers = static_cast<int>(std::min(7u, hw > 1 ? hw / 2 : 0u));
    for (int i = 0; i < workers; ++i) threads_.emplace_back([this, i] { worker(i); });
}

HostCopier::~HostCopier() {
    {
        std::lock_guard<std::mutex> lock(mu_);
        stop_ = true;
    }
    work_cv_.notify_all();
    for (std::thread& t : threads_) t.join();
    for (int i = 0; i < 2; ++i) {
        if (done_[i]) (void)hipEventDestroy(done_[i]);
        if (pinned_[i]) (void)hipHostFree(pinned_[i]);
        if (band_done_[i]) (void)hipEventDestroy(band_done_[i]);
        if (band_pinned_[i]) (void)hipHostFree(band_pinned_[i]);
    }
}

void HostCopier::worker(int index) {
    unsigned long seen = 0;
    for (;;) {
        char* dst;
        const char* src;
        size_t bytes, rows, dpitch, spitch;
        int parts;
        {
            std::unique_lock<std::mutex> lock(mu_);
            work_cv_.wait(lock, [&] { return stop_ || generation_ != seen; });
            if (stop_) return;
            seen = generation_;
            dst = job_dst_;
            src = job_src_;
            bytes = job_bytes_;
            rows = job_rows_;
            dpitch = job_dpitch_;
            spitch = job_spitch_;
            parts = parts_;
        }
        const int part = index + 1;
        if (part < parts && rows) {
            const size_t per = (rows + parts - 1) / parts;
            const size_t b = std::min(rows, per * part), e = std::min(rows, b + per);
            for (size_t r = b; r < e; ++r) std::memcpy(dst + r * dpitch, src + r * spitch, bytes);
        } else if (part < parts) {
            const size_t per = (bytes + parts - 1) / parts;
            const size_t b = std::min(bytes, per * part), e = std::min(bytes, b + per);
            if (e > b) std::memcpy(dst + b, src + b, e - b);
        }
        {
            std::lock_guard<std::mutex> lock(mu_);
            if (--pending_ == 0) done_cv_.notify_one();
        }
    }
}

// never destroyed: its threads wait on a condition variable until the
// process ends, and nothing runs at static destruction
HostCopier& HostCopier::shared() {
    static HostCopier* copier = new HostCopier;
    return *copier;
}

void HostCopier::parallel_copy(char* dst, const char* src, size_t bytes, int min_part_log2) {
    const int parts =
        static_cast<int>(std::min<size_t>(threads_.size() + 1, std::max<size_t>(1, bytes >> min_part_log2)));
    if (parts <= 1) {
        std::memcpy(dst, src, bytes);
        return;
    }
    {
        std::lock_guard<std::mutex> lock(mu_);
        job_dst_ = dst;
        job_src_ = src;
        job_bytes_ = bytes;
        job_rows_ = 0;
        parts_ = parts;
        pending_ = static_cast<int>(threads_.size());
        ++generation_;
    }
    work_cv_.notify_all();
    const size_t per = (bytes + parts - 1) / parts;
    std::memcpy(dst, src, std::min(bytes, per));
    std::unique_lock<std::mutex> lock(mu_);
    done_cv_.wait(lock, [&] { return pending_ == 0; });
}

void HostCopier::parallel_copy_rows(char* dst, const char* src, size_t height, size_t width, size_t dpitch,
                                    size_t spitch) {
    const int parts = static_cast<int>(
        std::min<size_t>({threads_.size() + 1, height, std::max<size_t>(1, (height * width) >> 19)}));
    if (parts <= 1) {
        for (size_t r = 0; r < height; ++r) std::memcpy(dst + r * dpitch, src + r * spitch, width);
        return;
    }
    {
        std::lock_guard<std::mutex> lock(mu_);
        job_dst_ = dst;
        job_src_ = src;
        job_bytes_ = width;
        job_rows_ = height;
        job_dpitch_ = dpitch;
        job_spitch_ = spitch;
        parts_ = parts;
        pending_ = static_cast<int>(threads_.size());
        ++generation_;
    }
    work_cv_.notify_all();
    const size_t per = (height + parts - 1) / parts;
    for (size_t r = 0; r < std::min(height, per); ++r) std::memcpy(dst + r * dpitch, src + r * spitch, width);
    std::unique_lock<std::mutex> lock(mu_);
    done_cv_.wait(lock, [&] { return pending_ == 0; });
}

void HostCopier::bands_from_device(float* dst, const float* src, size_t n, size_t width, const size_t* bounds,
                                   const hipEvent_t* ready, int bands, hipStream_t cs) {
    size_t widest = 0;
    for (int i = 0; i < bands; ++i) widest = std::max(widest, bounds[i + 1] - bounds[i]);
    const size_t need = n * widest * sizeof(float);
    if (band_bytes_ < need) {
        for (int i = 0; i < 2; ++i) {
            if (band_pinned_[i]) TVARA_HIP(hipHostFree(band_pinned_[i]));
            band_pinned_[i] = nullptr;
        }
        band_bytes_ = 0;
        for (int i = 0; i < 2; ++i) TVARA_HIP(hipHostMalloc(&band_pinned_[i], need, hipHostMallocDefault));
        band_bytes_ = need;
    }
    for (int i = 0; i < 2; ++i)
        if (!band_done_[i]) TVARA_HIP(hipEventCreateWithFlags(&band_done_[i], hipEventDisableTiming));
    auto issue = [&](int i) {
        const size_t b0 = bounds[i], w = bounds[i + 1] - b0;
        TVARA_HIP(hipStreamWaitEvent(cs, ready[i], 0));
        TVARA_HIP(hipMemcpy2DAsync(band_pinned_[i % 2], w * sizeof(float), src + b0, width * sizeof(float),
                                   w * sizeof(float), n, hipMemcpyDeviceToHost, cs));
        TVARA_HIP(hipEventRecord(band_done_[i % 2], cs));
    };
    issue(0);
    if (bands > 1) issue(1);
    for (int i = 0; i < bands; ++i) {
        TVARA_HIP(hipEventSynchronize(band_done_[i % 2]));
        const size_t b0 = bounds[i], w = bounds[i + 1] - b0;
        parallel_copy_rows(reinterpret_cast<char*>(dst + b0), static_cast<const char*>(band_pinned_[i % 2]), n,
                           w * sizeof(float), width * sizeof(float), w * sizeof(float));
        if (i + 2 < bands) issue(i + 2);
    }
}

void HostCopier::from_device(void* dst, const void* src, size_t bytes, hipStream_t s) {
    if (bytes < (size_t(1) << 20)) {  // small: one plain copy after the queued work
        TVARA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
        TVARA_HIP(hipStreamSynchronize(s));
        return;
    }
    for (int i = 0; i < 2; ++i) {
        if (!pinned_[i]) TVARA_HIP(hipHostMalloc(&pinned_[i], kChunk, hipHostMallocDefault));
        if (!done_[i]) TVARA_HIP(hipEventCreateWithFlags(&done_[i], hipEventDisableTiming));
    }
    auto* out = static_cast<char*>(dst);
    const auto* in = static_cast<const char*>(src);
    const size_t n = (bytes + kChunk - 1) / kChunk;
    auto issue = [&](size_t i) {
        const size_t off = i * kChunk, len = std::min(kChunk, bytes - off);
        TVARA_HIP(hipMemcpyAsync(pinned_[i % 2], in + off, len, hipMemcpyDeviceToHost, s));
        TVARA_HIP(hipEventRecord(done_[i % 2], s));
    };
    issue(0);
    if (n > 1) issue(1);
    for (size_t i = 0; i < n; ++i) {
        TVARA_HIP(hipEventSynchronize(done_[i % 2]));
        const size_t off = i * kChunk, len = std::min(kChunk, bytes - off);
        parallel_copy(out + off, static_cast<const char*>(pinned_[i % 2]), len, 17);
        if (i + 2 < n) issue(i + 2);
    }
}

}  // namespace tvara_amd
