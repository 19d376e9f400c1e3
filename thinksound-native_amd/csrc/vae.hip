// vae.hip — the element-wise and output kernels of the VAE decoder (src/vae.cpp:17-86): the
// three-part f16 split of f32 rows (optionally after the snake activation), and the final
// snake + narrow conv to the audio channels.
#include <hip/hip_runtime.h>

#include "kernels.h"

namespace tsn {

namespace {

// One thread per 8 channels of a row: v = x (or snake(x) with ea = exp(alpha), eb = exp(-beta)),
// hi = f16(v), lo = f16(v - hi); the row of out holds three C-wide parts: [hi | lo | hi] when
// lo_part == 1 (an activation operand), [hi | hi | lo] when lo_part == 2 (a weight operand).
__global__ void split3_kernel(const float *__restrict__ x, long long rows, int C, const float *__restrict__ ab,
                              int lo_part, half_t *__restrict__ out) {
    const int cg = C >> 3;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * cg) return;
    const long long r = i / cg;
    const int c = (int)(i - r * cg) * 8;
    const float *xp = x + r * C + c;
    const float4 x0 = *(const float4 *)xp, x1 = *(const float4 *)(xp + 4);
    float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    if (ab) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float sn = sinf(v[e] * ab[c + e]);
            v[e] = v[e] + sn * sn * ab[C + c + e];
        }
    }
    half8 hi, lo;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        hi[e] = (half_t)v[e];
        lo[e] = (half_t)(v[e] - (float)hi[e]);
    }
    half_t *o = out + r * 3 * C + c;
    *(half8 *)o = hi;
    *(half8 *)(o + C) = lo_part == 1 ? lo : hi;
    *(half8 *)(o + 2 * C) = lo_part == 1 ? hi : lo;
}

constexpr int CO_TB = 64;   // output rows per workgroup
constexpr int CO_CH = 64;   // channels per LDS chunk
constexpr int CO_KMAX = 15; // largest kernel width

// y[t][c] = sum_{i,k} snake(x)[t - pad + k][i] * W[c][i][k], zero rows outside [0, T); OC in {1, 2, 4}.
// 256 threads: output (row r, channel c) is summed by 4/OC adjacent lanes, each over its share of
// every channel chunk, then combined in lane order.
__global__ void __launch_bounds__(256) conv_out_kernel(const float *__restrict__ x, const float *__restrict__ ab,
                                                       const float *__restrict__ W, float *__restrict__ y, int T, int C,
                                                       int OC, int KK, int pad) {
    __shared__ float xs[(CO_TB + CO_KMAX - 1) * (CO_CH + 1)];
    __shared__ float ws[4 * CO_CH * CO_KMAX];
    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * CO_TB;
    const int tpo = 4 / OC;
    const int o = tid / tpo, h = tid - o * tpo;
    const int r = o / OC, c = o - r * OC;
    const int share = CO_CH / tpo;
    const int rows = CO_TB + KK - 1;
    float acc = 0.0f;
    for (int c0 = 0; c0 < C; c0 += CO_CH) {
        for (int e = tid; e < rows * CO_CH; e += 256) {
            const int rr = e / CO_CH, i = e - rr * CO_CH;
            const int t = t0 - pad + rr;
            float v = 0.0f;
            if (t >= 0 && t < T) {
                const float u = x[(long long)t * C + c0 + i];
                const float sn = sinf(u * ab[c0 + i]);
                v = u + sn * sn * ab[C + c0 + i];
            }
            xs[rr * (CO_CH + 1) + i] = v;
        }
        for (int e = tid; e < OC * CO_CH * KK; e += 256) {
            const int cc = e / (CO_CH * KK), rem = e - cc * CO_CH * KK;
            const int i = rem / KK, k = rem - i * KK;
            ws[e] = W[((long long)cc * C + c0 + i) * KK + k];
        }
        __syncthreads();
        const float *wc = ws + c * CO_CH * KK;
        for (int i = h * share; i < (h + 1) * share; ++i)
            for (int k = 0; k < KK; ++k) acc = fmaf(xs[(r + k) * (CO_CH + 1) + i], wc[i * KK + k], acc);
        __syncthreads();
    }
    // combine the tpo partial sums of one output (adjacent lanes) in lane order
    if (tpo == 4) {
        const float a1 = __shfl_down(acc, 1, 4), a2 = __shfl_down(acc, 2, 4), a3 = __shfl_down(acc, 3, 4);
        acc = ((acc + a1) + a2) + a3;
    } else if (tpo == 2) {
        acc = acc + __shfl_down(acc, 1, 2);
    }
    if (h == 0 && t0 + r < T) y[(long long)(t0 + r) * OC + c] = acc;
}

} // namespace

int launch_split3(const float *x, long long rows, int C, const float *ab, int lo_part, half_t *out, hipStream_t st) {
    TSN_REQUIRE(x && out && rows > 0 && C > 0 && C % 8 == 0 && (lo_part == 1 || lo_part == 2),
                "split3: arguments (C a multiple of 8, lo part 1 or 2)");
    TSN_REQUIRE((((uintptr_t)x) & 15) == 0 && (((uintptr_t)out) & 15) == 0, "split3: 16-byte aligned rows");
    const long long n = rows * (C / 8);
    TSN_LAUNCH(split3_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, rows, C, ab, lo_part, out);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_conv_out(const float *x, const float *ab, const float *W, float *y, int T, int C, int OC, int KK, int pad,
                    hipStream_t st) {
    TSN_REQUIRE(x && ab && W && y && T > 0, "conv_out: arguments");
    TSN_REQUIRE(OC == 1 || OC == 2 || OC == 4, "conv_out: 1, 2 or 4 output channels");
    TSN_REQUIRE(C > 0 && C % CO_CH == 0, "conv_out: input channels must be a multiple of 64");
    TSN_REQUIRE(KK >= 1 && KK <= CO_KMAX && pad >= 0 && pad < KK, "conv_out: kernel width 1..15, pad < width");
    TSN_LAUNCH(conv_out_kernel, dim3((unsigned)((T + CO_TB - 1) / CO_TB)), dim3(256), 0, st, x, ab, W, y, T, C, OC,
               KK, pad);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

} // namespace tsn
