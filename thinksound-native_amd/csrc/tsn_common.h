// tsn_common.h — shared types and helpers for the gfx950 DiT velocity path.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace tsn {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

// GEMM / kernel row m -> physical row: (m / L) * seg + off + (m % L).
// Lets one launch address a stream's rows inside the joint [B, S, H] layout (L rows per
// sample, seg = S rows between samples, off = first row of the stream in a sample).
struct RowMap {
    int L, seg, off;
};
__host__ __device__ inline RowMap rowmap_dense(int M) { return RowMap{M > 0 ? M : 1, M > 0 ? M : 1, 0}; }
__host__ __device__ inline long long rowmap_phys(const RowMap &r, int m) {
    const int b = m / r.L;
    return (long long)b * r.seg + r.off + (m - b * r.L);
}

// status codes of the C ABI (include/tsn.h)
enum {
    TSN_OK = 0,
    TSN_ERR_ARG = 1,
    TSN_ERR_HIP = 2,
    TSN_ERR_UNSUPPORTED = 3,
    TSN_ERR_OOM = 4,
    TSN_ERR_STATE = 5,
};
enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

// per-thread last error message
void set_error(const std::string &msg);
const char *last_error();

#define TSN_HIP_CHECK(expr)                                                             \
    do {                                                                                \
        hipError_t e_ = (expr);                                                         \
        if (e_ != hipSuccess) {                                                         \
            ::tsn::set_error(std::string(#expr) + ": " + hipGetErrorString(e_));        \
            return TSN_ERR_HIP;                                                         \
        }                                                                               \
    } while (0)

#define TSN_REQUIRE(cond, msg)                                                          \
    do {                                                                                \
        if (!(cond)) {                                                                  \
            ::tsn::set_error(std::string("argument check failed: ") + (msg));           \
            return TSN_ERR_ARG;                                                         \
        }                                                                               \
    } while (0)

#define TSN_TRY(expr)                                                                   \
    do {                                                                                \
        int s_ = (expr);                                                                \
        if (s_ != TSN_OK) return s_;                                                    \
    } while (0)

// Event pair armed for the next kernel launch of the calling thread (per-kernel profiling). Every
// kernel goes through TSN_LAUNCH: when a pair is armed it is attached to the dispatch itself with
// hipExtLaunchKernelGGL, so the events bracket exactly that kernel's execution, and disarmed.
struct LaunchEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};
LaunchEvents &next_launch_events();

#define TSN_LAUNCH(kernel, grid, block, shm, st, ...)                                           \
    do {                                                                                        \
        ::tsn::LaunchEvents &ev_ = ::tsn::next_launch_events();                                 \
        if (ev_.start) {                                                                        \
            hipExtLaunchKernelGGL(kernel, grid, block, shm, st, ev_.start, ev_.stop, 0, __VA_ARGS__); \
            ev_.start = ev_.stop = nullptr;                                                     \
        } else {                                                                                \
            hipLaunchKernelGGL(kernel, grid, block, shm, st, __VA_ARGS__);                      \
        }                                                                                       \
    } while (0)

// bf16 bits -> f32 (exact)
__host__ __device__ inline float bf16_to_f32(uint16_t b) {
    union { uint32_t u; float f; } c;
    c.u = (uint32_t)b << 16;
    return c.f;
}

// f32 -> f16 bits as the reference's weight upload converts (src/net.mm:144-164): round to nearest
// even in the normal range, f32 zero/denormal inputs -> signed zero, results below the f16 normal
// range truncated to a subnormal (or zero), overflow -> infinity, NaN -> quiet NaN
__device__ inline half_t f32_to_f16_upload(float f) {
    const unsigned x = __float_as_uint(f);
    const unsigned short sign = (unsigned short)((x >> 16) & 0x8000u);
    const unsigned e8 = (x >> 23) & 0xFFu, man = x & 0x7FFFFFu;
    unsigned short h;
    if (e8 == 0xFFu) {
        h = sign | 0x7C00u | (man ? 0x200u : 0u);
    } else if (e8 == 0u) {
        h = sign;
    } else {
        const int e = (int)e8 - 112;   // f16 biased exponent
        if (e >= 31) {
            h = sign | 0x7C00u;
        } else if (e <= 0) {
            h = e < -10 ? sign : (unsigned short)(sign | ((man | 0x800000u) >> (14 - e)));
        } else {
            h = (unsigned short)(sign | ((unsigned)e << 10) | (man >> 13));
            const unsigned rest = man & 0x1FFFu;
            if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h = (unsigned short)(h + 1u);
        }
    }
    return __builtin_bit_cast(half_t, h);
}

} // namespace tsn
