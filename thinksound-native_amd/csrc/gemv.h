// gemv.h — the per-wave body of the HBM-bound GEMV (device code only). The standalone
// gemv_kernel and the GEMV workgroups of a GEMM grid (GemmBatch::gv) run the same code, so a row's
// value does not depend on where it was computed.
#pragma once
#include "kernels.h"

namespace tsn {

__device__ __forceinline__ float gemv_silu(float v) { return v / (1.0f + __expf(-v)); }

/* ---------------- GEMV (shaders/gemm_attn.metal:47-74, batched over nb rows of X) ---------------- */
template <typename WT>
__device__ inline void load_w8(const WT *p, float (&w)[8]);
template <>
__device__ inline void load_w8<uint16_t>(const uint16_t *p, float (&w)[8]) {
    const u16x8 u = *(const u16x8 *)p;
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = bf16_to_f32(u[e]);
}
template <>
__device__ inline void load_w8<half_t>(const half_t *p, float (&w)[8]) {
    const half8 u = *(const half8 *)p;
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = (float)u[e];
}
template <>
__device__ inline void load_w8<float>(const float *p, float (&w)[8]) {
    const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

constexpr int GEMV_ROWS = 4;   // rows of W per wave

// Rows n0 .. n0 + GEMV_ROWS - 1 of Y = W X (+ bias, + addv, SiLU, Y2 = silu(Y)) for the NB input
// rows, by one wave (lane = its lane index); rows past a.N are computed on row N-1 and not written.
template <typename WT, int NB>
__device__ __forceinline__ void gemv_rows(const GemvArgs &a, int n0, int lane) {
    const WT *W = (const WT *)a.W;
    float acc[GEMV_ROWS][NB];
#pragma unroll
    for (int rr = 0; rr < GEMV_ROWS; ++rr)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[rr][b] = 0.0f;
    for (int k = lane * 8; k < a.K; k += 512) {
        float w[GEMV_ROWS][8];
#pragma unroll
        for (int rr = 0; rr < GEMV_ROWS; ++rr) {
            const int n = min(n0 + rr, a.N - 1);
            load_w8<WT>(W + (long long)n * a.ldw + k, w[rr]);
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float *xp = a.X + (long long)b * a.ldx + k;
            const float4 x0 = *(const float4 *)xp, x1 = *(const float4 *)(xp + 4);
            const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int rr = 0; rr < GEMV_ROWS; ++rr)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[rr][b] += w[rr][e] * xs[e];
        }
    }
    // Reduce-scatter of the V = GEMV_ROWS*NB partial sums over the wave: at the xor step of lane
    // bit 32, 16, ... each lane keeps half of its values (the upper half when its bit is set) and
    // adds the partner's copy of that half, so V values cost V - 1 shuffles; a butterfly over the
    // remaining low lane bits finishes the sum. Lane l then holds value index
    // sum_j bit_j(l) * V / 2^(j+1) over the scatter bits (fixed order: deterministic).
    constexpr int V = GEMV_ROWS * NB;
    float vals[V];
#pragma unroll
    for (int rr = 0; rr < GEMV_ROWS; ++rr)
#pragma unroll
        for (int b = 0; b < NB; ++b) vals[rr * NB + b] = acc[rr][b];
    int idx = 0;
#pragma unroll
    for (int h = V / 2, bit = 32; h >= 1; h >>= 1, bit >>= 1) {
        const bool upper = (lane & bit) != 0;
#pragma unroll
        for (int i = 0; i < h; ++i) {
            const float lo = vals[i], hi = vals[i + h];
            vals[i] = (upper ? hi : lo) + __shfl_xor(upper ? lo : hi, bit);
        }
        idx += upper ? h : 0;
    }
#pragma unroll
    for (int bit = 32 / V; bit >= 1; bit >>= 1) vals[0] += __shfl_xor(vals[0], bit);
    const int rr = idx / NB, b = idx - rr * NB, n = n0 + rr;
    if ((lane & (64 / V - 1)) == 0 && n < a.N) {
        float v = vals[0];
        if (a.bias) v += a.bias[n];
        if (a.addv) v += a.addv[(long long)b * a.ld_add + n];
        if (a.silu) v = gemv_silu(v);
        a.Y[(long long)b * a.ldy + n] = v;
        if (a.Y2) a.Y2[(long long)b * a.ldy2 + n] = gemv_silu(v);
    }
}

} // namespace tsn
