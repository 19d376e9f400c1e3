// vae.hip — the element-wise and output kernels of the VAE decoder (src/vae.cpp:17-86): the
// three-part f16 split of f32 rows (optionally after the snake activation), and the final
// snake + narrow conv to the audio channels.
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "dpp.h"
#include "snake.h"

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
            v[e] = v[e] + snake_sin2(v[e] * ab[c + e]) * ab[C + c + e];
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

constexpr int CO_TB = 64;    // output rows per workgroup (16 per wave)
constexpr int CO_CH = 128;   // channels per LDS chunk (2 per lane)
constexpr int CO_K = 7;      // kernel width
constexpr int CO_ROWS = CO_TB + CO_K - 1;
constexpr int CO_PER = (CO_ROWS * CO_CH + 255) / 256;   // staged elements per thread and chunk

// y[t][c] = sum_{i,k} snake(x)[t - pad + k][i] * W[c][i][k], zero rows outside [0, T), k < 7, OC in {1, 2, 4}.
// The workgroup stages snake(x) rows of a 128-channel chunk in LDS; lane l of wave w holds channels
// 2l, 2l+1 and accumulates all 16 x OC outputs of the wave's rows from them (each staged row read
// once, feeding up to 7 outputs). The lanes' partial sums are then added by an xor butterfly, the
// same order for every output.
template <int OC>
__global__ void __launch_bounds__(256) conv_out_kernel(const float *__restrict__ x, const float *__restrict__ ab,
                                                       const float *__restrict__ W, float *__restrict__ y, int T, int C,
                                                       int pad) {
    __shared__ float xs[CO_ROWS * CO_CH];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.x * CO_TB;
    float acc[16][OC];
#pragma unroll
    for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int c = 0; c < OC; ++c) acc[r][c] = 0.0f;
    for (int c0 = 0; c0 < C; c0 += CO_CH) {
        const int cw = min(CO_CH, C - c0);   // channels of this chunk; the rest stay zero
        float v[CO_PER];
#pragma unroll
        for (int j = 0; j < CO_PER; ++j) {
            const int e = tid + 256 * j;
            const int rr = e / CO_CH, i = e - rr * CO_CH;
            const int t = t0 - pad + rr;
            v[j] = (rr < CO_ROWS && i < cw && t >= 0 && t < T) ? x[(long long)t * C + c0 + i] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < CO_PER; ++j) {
            const int e = tid + 256 * j;
            const int rr = e / CO_CH, i = e - rr * CO_CH;
            if (rr < CO_ROWS) {
                float u = 0.0f;   // snake(0) = 0: padding rows and channels past the chunk stay zero
                if (i < cw) {
                    u = v[j] + snake_sin2(v[j] * ab[c0 + i]) * ab[C + c0 + i];
                }
                xs[e] = u;
            }
        }
        // this lane's weights: w[c][j][k] for channels c0 + 2*lane + j
        float w[OC][2][CO_K];
#pragma unroll
        for (int c = 0; c < OC; ++c)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int i = 2 * lane + j;
#pragma unroll
                for (int k = 0; k < CO_K; ++k) w[c][j][k] = i < cw ? W[((long long)c * C + c0 + i) * CO_K + k] : 0.0f;
            }
        __syncthreads();
#pragma unroll
        for (int jr = 0; jr < 16 + CO_K - 1; ++jr) {   // staged row 16*wave + jr feeds outputs r = jr - k
            const float2 xv = *(const float2 *)&xs[(16 * wave + jr) * CO_CH + 2 * lane];
#pragma unroll
            for (int k = 0; k < CO_K; ++k) {
                const int r = jr - k;
                if (r < 0 || r >= 16) continue;
#pragma unroll
                for (int c = 0; c < OC; ++c) acc[r][c] = fmaf(xv.y, w[c][1][k], fmaf(xv.x, w[c][0][k], acc[r][c]));
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int c = 0; c < OC; ++c) {
            acc[r][c] = wave_sum(acc[r][c]);
        }
    // lane r*OC + c writes output (row r, channel c) of the wave's 16 rows
    float mine = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int c = 0; c < OC; ++c)
            if (lane == r * OC + c) mine = acc[r][c];
    const int t = t0 + 16 * wave + lane / OC;
    if (lane < 16 * OC && t < T) y[(long long)t * OC + (lane % OC)] = mine;
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
    TSN_REQUIRE(C > 0 && C % 8 == 0, "conv_out: input channels must be a multiple of 8");
    TSN_REQUIRE(KK == CO_K && pad >= 0 && pad < KK, "conv_out: kernel width 7, pad < width");
    const dim3 grid((unsigned)((T + CO_TB - 1) / CO_TB)), block(256);
    if (OC == 1) TSN_LAUNCH(conv_out_kernel<1>, grid, block, 0, st, x, ab, W, y, T, C, pad);
    else if (OC == 2) TSN_LAUNCH(conv_out_kernel<2>, grid, block, 0, st, x, ab, W, y, T, C, pad);
    else TSN_LAUNCH(conv_out_kernel<4>, grid, block, 0, st, x, ab, W, y, T, C, pad);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

} // namespace tsn
