// snake.h — sin(x)^2 of the snake activation (y = x + sin(x*e^alpha)^2 * e^-beta), f32.
//
// Cody-Waite reduction r = x - k*pi, k = rint(x/pi), with pi split into three f32 parts whose
// products are folded in by fmas (exact for |k| well beyond the snake's arguments), then the odd
// Taylor series of sin(r) through r^13 on [-pi/2, pi/2] (truncation below 7e-10). sin^2 drops the
// (-1)^k sign of the reduction. Constants: the f32 parts of pi and 1/n! as f32.
#pragma once
#include <hip/hip_runtime.h>

namespace tsn {

__device__ __forceinline__ float snake_sin2(float x) {
    const float k = rintf(x * 0x1.45f306p-2f);   // x / pi
    float r = fmaf(-k, 0x1.921fb6p+1f, x);        // pi = A + B + C
    r = fmaf(-k, -0x1.777a5cp-24f, r);
    r = fmaf(-k, -0x1.ee59dap-49f, r);
    const float r2 = r * r;
    float p = 0x1.612462p-33f;              // 1/13!
    p = fmaf(p, r2, -0x1.ae6456p-26f);      // -1/11!
    p = fmaf(p, r2, 0x1.71de3ap-19f);       // 1/9!
    p = fmaf(p, r2, -0x1.a01a02p-13f);      // -1/7!
    p = fmaf(p, r2, 0x1.111112p-7f);        // 1/5!
    p = fmaf(p, r2, -0x1.555556p-3f);       // -1/3!
    const float s = fmaf(r * r2, p, r);
    return s * s;
}

} // namespace tsn
