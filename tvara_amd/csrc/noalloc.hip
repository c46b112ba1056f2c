// tvara_attn_decode for callers that cannot allocate device memory (serving
// loops, harnesses that forbid hipMalloc; not graph capture: the call copies
// its plan from host memory and synchronises the cache's stream): the same
// plan and kernels, with the plan's device half (block ids, rows,
// work items, split counters, error flag, split partials) in a file-scope
// device array instead of library-owned buffers.
//
// The array is one per GPU, 32 MiB, held until the process ends.  Host code
// never passes the array's name to a kernel or copy (in host code it is a
// stand-in, not a device address): each device's address comes from
// hipGetSymbolAddress, looked up once per device with that device current,
// and only that address is used.  Calls on one GPU share the array; they are
// serialised by a lock per device and each waits for its own work before
// returning, so two calls never have work in flight on it at once.  Every
// call uploads its plan together with zeros for the counters and the flag,
// so nothing left by an earlier call is read.
#include <hip/hip_runtime.h>

#include <array>
#include <mutex>
#include <vector>

#include "abi.hpp"
#include "kv_cache.hpp"

namespace tvara_amd {
namespace {

constexpr size_t kScratchBytes = size_t(32) << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) char scratch[kScratchBytes];

struct DeviceSlot {
    std::mutex lock;
    char* base = nullptr;  // this device's copy of `scratch`
};
std::array<DeviceSlot, kMaxDevices> slots;

// the current device's slot, with its scratch address looked up on first use
DeviceSlot& current_slot() {
    int dev = 0;
    TVARA_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) throw std::runtime_error("device index outside the no-allocation table");
    return slots[static_cast<size_t>(dev)];
}

char* scratch_address(DeviceSlot& slot) {
    if (!slot.base) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            throw std::runtime_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        slot.base = static_cast<char*>(p);
    }
    return slot.base;
}

}  // namespace
}  // namespace tvara_amd

using tvara_amd::abi::guard;

extern "C" {

size_t tvara_attn_decode_noalloc_limit(void) { return tvara_amd::kScratchBytes; }

int tvara_attn_decode_noalloc(tvara_kv_cache* cache, const uint64_t* sequences, size_t count, size_t layer,
                              size_t heads, size_t context, const float* q, const float* tail_keys,
                              const float* tail_values, const size_t* visible, float* out) {
    return guard([&] {
        tvara_amd::DeviceCache& c = tvara_amd::device_cache(cache);
        tvara_amd::check_attention_config(c, heads, context);
        if (!count) return;
        if (!sequences || !q || !out || (tail_keys == nullptr) != (tail_values == nullptr))
            throw std::invalid_argument("invalid fused attention shape");
        if (layer >= c.geometry().layers) throw std::invalid_argument("invalid fused attention shape");
        auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
        if (!aligned(q) || !aligned(out) || (tail_keys && (!aligned(tail_keys) || !aligned(tail_values))))
            throw std::invalid_argument("device buffers must be 16-byte aligned");
        const bool tail = tail_keys != nullptr;
        std::vector<uint64_t> seq_of_row;
        std::vector<size_t> cached;
        std::vector<uint8_t> tails;
        tvara_amd::attention_rows(c, sequences, count, context, tail, visible, seq_of_row, cached, tails);
        tvara_amd::AttnPlan plan;
        plan.compute(&c, seq_of_row, cached, tails, static_cast<int>(heads), 0);
        size_t copied = 0;
        const size_t need = plan.region_bytes(&copied);
        if (need > tvara_amd::kScratchBytes)
            throw std::invalid_argument("attention batch needs " + std::to_string(need) +
                                        " bytes of plan and split partials, above the " +
                                        std::to_string(tvara_amd::kScratchBytes) + "-byte no-allocation scratch");
        tvara_amd::DeviceSlot& slot = tvara_amd::current_slot();
        std::lock_guard<std::mutex> hold(slot.lock);
        char* base = tvara_amd::scratch_address(slot);
        // host image of the packed plan; the call waits for its copy below
        std::vector<char> image(copied);
        hipStream_t s = c.stream();
        plan.place_in(base, tvara_amd::kScratchBytes, s, image.data());
        plan.launch(static_cast<int>(layer), q, tail_keys, tail_values, out, s);
        int flag = 0;
        plan.check_into(&flag);  // waits for the stream: the copy in and the launch are done
    });
}

}  // extern "C"
