// prefetch.h — workgroups that touch weight lines for a following GEMM (device code only).
//
// A prefetch workgroup of WAVES waves loads one dword of each 128-byte line of lines
// [pw*L, pw*L + L) of the PfRange ranges laid end to end (L = WAVES*64*PF_PER_LANE), issues
// every load before waiting, and keeps the values alive until its end; it does nothing else, so the
// workgroups it shares a launch with never wait for it. The lines then sit in the last-level cache
// when the GEMM reads them.
#pragma once
#include "kernels.h"

namespace tsn {

template <int WAVES>
__device__ __forceinline__ void prefetch_wg(const PfRange (&pf)[PF_RANGES], int pw, int wave, int lane) {
    long long start[PF_RANGES + 1];
    start[0] = 0;
#pragma unroll
    for (int r = 0; r < PF_RANGES; ++r) start[r + 1] = start[r] + (long long)pf[r].rows * (pf[r].row_bytes >> 7);
    const long long g0 = (long long)pw * (WAVES * 64 * PF_PER_LANE) + wave * (64 * PF_PER_LANE) + lane;
    float v[PF_PER_LANE];
#pragma unroll
    for (int j = 0; j < PF_PER_LANE; ++j) {
        const long long g = g0 + 64 * j;
        v[j] = 0.0f;
        if (g < start[PF_RANGES]) {
            // the range holding line g, by selects (no indexing into the argument block)
            const char *p = (const char *)pf[0].p;
            long long ld = pf[0].ld, lpr = pf[0].row_bytes >> 7, base = 0;
#pragma unroll
            for (int r = 1; r < PF_RANGES; ++r)
                if (g >= start[r]) {
                    p = (const char *)pf[r].p;
                    ld = pf[r].ld;
                    lpr = pf[r].row_bytes >> 7;
                    base = start[r];
                }
            const long long gl = g - base, row = gl / lpr;
            v[j] = *(const float *)(p + row * ld + (gl - row * lpr) * 128);
        }
    }
#pragma unroll
    for (int j = 0; j < PF_PER_LANE; ++j) asm volatile("" ::"v"(v[j]));
}

} // namespace tsn
