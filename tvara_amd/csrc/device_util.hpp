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

// Cross-row reductions with gfx950's permlane swaps.  permlane32_swap(x, y)
// returns (x.lo | y.lo, x.hi | y.hi) by 32-lane half and permlane16_swap
// returns (x.r0, y.r0, x.r2, y.r2 | x.r1, y.r1, x.r3, y.r3) by 16-lane row, so
// with y = x the two results hold a lane's value and its partner's.  (The
// results are copied to scalars before the bit cast: __builtin_bit_cast of a
// vector element reads element 0 with this compiler.)
template <class Op>
__device__ __forceinline__ float cross_row_reduce(float v, Op op) {
    const unsigned a = __builtin_bit_cast(unsigned, v);
    const auto h = __builtin_amdgcn_permlane32_swap(a, a, false, false);
    const unsigned h0 = h[0], h1 = h[1];
    v = op(__builtin_bit_cast(float, h0), __builtin_bit_cast(float, h1));
    const unsigned b = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    const unsigned r0 = r[0], r1 = r[1];
    return op(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
}

// sum / max over lanes l%16 + 16r (the four 16-lane rows); every lane gets
// the same bits
__device__ __forceinline__ float cross_row_sum(float v) {
    return cross_row_reduce(v, [](float x, float y) { return x + y; });
}

__device__ __forceinline__ float cross_row_max(float v) {
    return cross_row_reduce(v, [](float x, float y) { return fmaxf(x, y); });
}

}  // namespace tvara_amd
