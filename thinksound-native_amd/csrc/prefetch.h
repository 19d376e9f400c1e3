// prefetch.h — workgroups that touch weight lines for a following GEMM (device code only).
//
// A prefetch workgroup of WAVES waves loads one dword of each 128-byte line of lines
// [pw*L, pw*L + L) of the two PfRange ranges laid end to end (L = WAVES*64*PF_PER_LANE), issues
// every load before waiting, and keeps the values alive until its end; it does nothing else, so the
// workgroups it shares a launch with never wait for it. The lines then sit in the last-level cache
// when the GEMM reads them.
#pragma once
#include "kernels.h"

namespace tsn {

template <int WAVES>
__device__ __forceinline__ void prefetch_wg(const PfRange (&pf)[2], int pw, int wave, int lane) {
    const long long lpr0 = pf[0].row_bytes >> 7, lpr1 = pf[1].row_bytes >> 7;
    const long long L0 = pf[0].rows * lpr0, L = L0 + pf[1].rows * lpr1;
    const long long g0 = (long long)pw * (WAVES * 64 * PF_PER_LANE) + wave * (64 * PF_PER_LANE) + lane;
    float v[PF_PER_LANE];
#pragma unroll
    for (int j = 0; j < PF_PER_LANE; ++j) {
        const long long g = g0 + 64 * j;
        v[j] = 0.0f;
        if (g < L) {
            const int ri = g < L0 ? 0 : 1;
            const long long gl = ri ? g - L0 : g, lpr = ri ? lpr1 : lpr0;
            const long long row = gl / lpr;
            v[j] = *(const float *)((const char *)pf[ri].p + row * pf[ri].ld + (gl - row * lpr) * 128);
        }
    }
#pragma unroll
    for (int j = 0; j < PF_PER_LANE; ++j) asm volatile("" ::"v"(v[j]));
}

} // namespace tsn
