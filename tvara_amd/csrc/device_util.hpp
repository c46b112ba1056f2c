// Device-only helpers shared by the HIP kernels (included by .hip files).
#pragma once

#include <cstdint>

namespace tvara_amd {

// Signed byte B of w to float in one instruction (SDWA byte select with sign
// extension); the compiler's own lowering takes a shift, a bit-field extract
// and a conversion.
template <int B>
__device__ __forceinline__ float sbyte_to_float(uint32_t w) {
    float r;
    if constexpr (B == 0)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(w));
    else if constexpr (B == 1)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(w));
    else if constexpr (B == 2)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(w));
    else
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(w));
    return r;
}

}  // namespace tvara_amd
