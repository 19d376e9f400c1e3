// dpp.h — wave-wide sums and maxima on gfx950 without an LDS round trip (device code only).
//
// Partners 1 and 2 lanes apart are combined by DPP quad permutes, 4 and 8 apart by the row
// half-mirror and mirror (after the previous steps every quad / half-row holds one value), and the
// four 16-lane rows by the row-swap permutes (v_permlane16_swap, v_permlane32_swap). Each step
// combines two values, so partner lanes get the same result and every lane ends with the same
// value in a fixed order: reruns are bit-identical.
#pragma once

namespace tsn {

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141;  // lane i of 8 <- lane 7 - i
constexpr int DPP_MIRROR = 0x140;       // lane i of 16 <- lane 15 - i

// sum over each group of 16 lanes (a row)
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_mov<DPP_XOR1>(v);
    v += dpp_mov<DPP_XOR2>(v);
    v += dpp_mov<DPP_HALF_MIRROR>(v);
    return v + dpp_mov<DPP_MIRROR>(v);
}

__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_mov<DPP_XOR1>(v));
    v = fmaxf(v, dpp_mov<DPP_XOR2>(v));
    v = fmaxf(v, dpp_mov<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_mov<DPP_MIRROR>(v));
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

} // namespace tsn
