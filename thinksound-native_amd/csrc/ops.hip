// ops.hip — HBM-bound kernels of the DiT path on gfx950: LayerNorm+adaLN modulate, the
// small-M GEMV (adaLN modulation, timestep MLP), an f32 SIMT linear for the K=64 input and
// N=64 output projections, the sampler update, format conversions, and the reference-surface
// elementwise ops.
//
// Reductions are wave-level butterflies (DPP and row-swap permutes, dpp.h; the GEMV's
// reduce-scatter by __shfl_xor), so every lane ends with the same value and the order is fixed:
// reruns are bit-identical. No float atomics anywhere.
#include "kernels.h"
#include "dpp.h"
#include "prefetch.h"
#include "gemv.h"

#include <string.h>

#include <algorithm>

namespace tsn {

namespace {


/* ---------------- LayerNorm + adaLN modulate (shaders/ops_conv.metal:127-144) ---------------- */
// one wave per row; lane holds columns 4*lane + 256*c, c < NV (H = 256*NV)
template <int YMODE, int NV>
__global__ __launch_bounds__(256) void ln_mod_kernel(const LnArgs a) {
    // wave-uniform: the segment's fields come through scalar loads
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if ((int)blockIdx.x < a.pf_nwg) {
        prefetch_wg<4>(a.pf, blockIdx.x, wave, lane);
        return;
    }
    int v = ((int)blockIdx.x - a.pf_nwg) * 4 + wave;
    int si = 0;
    while (si < a.nseg && v >= a.seg[si].rows) v -= a.seg[si++].rows;
    if (si >= a.nseg) return;
    const LnSeg &S = a.seg[si];
    const float *x = S.X + rowmap_phys(S.xmap, v) * (long long)S.ldx;
    float4 xv[NV], sh[NV], scl[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c) xv[c] = *(const float4 *)(x + c * 256 + lane * 4);
    // the modulation rows are loaded with the row, not after its statistics: one global latency
    const int b = v / S.mod_L;
    const float *mb = S.mod + (long long)b * S.mod_ld;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        sh[c] = *(const float4 *)(mb + S.shift_off + c * 256 + lane * 4);
        scl[c] = *(const float4 *)(mb + S.scale_off + c * 256 + lane * 4);
    }

    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < NV; ++c) sum += (xv[c].x + xv[c].y) + (xv[c].z + xv[c].w);
    const float inv_h = 1.0f / (float)(NV * 256);
    const float mean = wave_sum(sum) * inv_h;
    float var = 0.0f;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        const float d0 = xv[c].x - mean, d1 = xv[c].y - mean, d2 = xv[c].z - mean, d3 = xv[c].w - mean;
        var += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
    }
    var = wave_sum(var) * inv_h;
    const float inv = 1.0f / sqrtf(var + a.eps);
    const long long yrow = rowmap_phys(S.ymap, v) * (long long)S.ldy;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        const int col = c * 256 + lane * 4;
        const float y0 = (xv[c].x - mean) * inv * (1.0f + scl[c].x) + sh[c].x;
        const float y1 = (xv[c].y - mean) * inv * (1.0f + scl[c].y) + sh[c].y;
        const float y2 = (xv[c].z - mean) * inv * (1.0f + scl[c].z) + sh[c].z;
        const float y3 = (xv[c].w - mean) * inv * (1.0f + scl[c].w) + sh[c].w;
        if constexpr (YMODE == LN_F16) {
            *(half4 *)((half_t *)S.Y + yrow + col) = half4{(half_t)y0, (half_t)y1, (half_t)y2, (half_t)y3};
        } else if constexpr (YMODE == LN_F16_HILO) {
            const half4 hi = half4{(half_t)y0, (half_t)y1, (half_t)y2, (half_t)y3};
            const half4 lo = half4{(half_t)(y0 - (float)hi[0]), (half_t)(y1 - (float)hi[1]),
                                   (half_t)(y2 - (float)hi[2]), (half_t)(y3 - (float)hi[3])};
            *(half4 *)((half_t *)S.Y + yrow + col) = hi;
            *(half4 *)((half_t *)S.Y + yrow + NV * 256 + col) = lo;
        } else {
            *(float4 *)((float *)S.Y + yrow + col) = make_float4(y0, y1, y2, y3);
        }
    }
}


/* ---------------- split-K reduce + gated residual + LayerNorm/adaLN (one workgroup per row) ---------------- */
// H/4 threads per row, 4 consecutive columns (one float4) per thread; the split partials of a row
// are summed in fixed split order, the LN statistics are two-pass (mean, then centred squares)
// with fixed-order wave and cross-wave sums.
__device__ __forceinline__ float block_sum(float v, float *red, int nw) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
    for (int w = 0; w < nw; ++w) t += red[w];
    return t;
}

template <int YMODE>
__global__ __launch_bounds__(512) void reduce_ln_kernel(const RedLnArgs a) {
    __shared__ float red[2][8];
    if ((int)blockIdx.x < a.pf_nwg) {
        prefetch_wg<4>(a.pf, blockIdx.x, threadIdx.x >> 6, threadIdx.x & 63);
        return;
    }
    int v = (int)blockIdx.x - a.pf_nwg, si = 0;
    while (si < a.nseg && v >= a.seg[si].M) v -= a.seg[si++].M;
    if (si >= a.nseg) return;   // uniform over the workgroup
    const RedLnSeg &S = a.seg[si];
    const int H = a.H, col = threadIdx.x * 4;
    float *x = S.X + rowmap_phys(S.xmap, v) * (long long)S.ldx + col;
    float4 xv = *(const float4 *)x;
    const int nwv = blockDim.x >> 6;
    if (S.splits > 1) {
        const float *w = S.ws + (long long)v * H + col;
        const long long step = (long long)S.M * H;
        float4 acc = *(const float4 *)w;
#pragma unroll 4
        for (int k = 1; k < S.splits; ++k) {
            const float4 u = *(const float4 *)(w + k * step);
            acc.x += u.x; acc.y += u.y; acc.z += u.z; acc.w += u.w;
        }
        if (S.bias) {
            const float4 b = *(const float4 *)(S.bias + col);
            acc.x += b.x; acc.y += b.y; acc.z += b.z; acc.w += b.w;
        }
        const float4 g = *(const float4 *)(S.gate + (long long)(v / S.gate_L) * S.gate_ld + col);
        xv.x = xv.x + acc.x * g.x; xv.y = xv.y + acc.y * g.y; xv.z = xv.z + acc.z * g.z; xv.w = xv.w + acc.w * g.w;
        *(float4 *)x = xv;
    }
    if (!S.ln) return;   // uniform over the workgroup
    const int b = v / S.mod_L;
    if (v - b * S.mod_L >= S.ln_len) return;
    const float inv_h = 1.0f / (float)H;
    const float mean = block_sum((xv.x + xv.y) + (xv.z + xv.w), red[0], nwv) * inv_h;
    const float d0 = xv.x - mean, d1 = xv.y - mean, d2 = xv.z - mean, d3 = xv.w - mean;
    const float var = block_sum((d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3), red[1], nwv) * inv_h;
    const float inv = 1.0f / sqrtf(var + a.eps);
    const float *mb = S.mod + (long long)b * S.mod_ld;
    const float4 sh = *(const float4 *)(mb + S.shift_off + col);
    const float4 scl = *(const float4 *)(mb + S.scale_off + col);
    const float y0 = d0 * inv * (1.0f + scl.x) + sh.x;
    const float y1 = d1 * inv * (1.0f + scl.y) + sh.y;
    const float y2 = d2 * inv * (1.0f + scl.z) + sh.z;
    const float y3 = d3 * inv * (1.0f + scl.w) + sh.w;
    half_t *y = (half_t *)S.Y + rowmap_phys(S.ymap, v) * (long long)S.ldy + col;
    const half4 hi = half4{(half_t)y0, (half_t)y1, (half_t)y2, (half_t)y3};
    *(half4 *)y = hi;
    if (YMODE == LN_F16_HILO || S.hilo)   // uniform over the workgroup
        *(half4 *)(y + H) = half4{(half_t)(y0 - (float)hi[0]), (half_t)(y1 - (float)hi[1]),
                                  (half_t)(y2 - (float)hi[2]), (half_t)(y3 - (float)hi[3])};
}

/* ---------------- calibration probes (achievable MFMA and HBM rates) ---------------- */
// 16 independent v_mfma_f32_16x16x32_f16 chains per wave, iters rounds; the result is written so
// the chains stay live
__global__ __launch_bounds__(512) void mfma_peak_kernel(float *out, int iters) {
    floatx4 acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    half8 x, y;
#pragma unroll
    for (int e = 0; e < 8; ++e) { x[e] = (half_t)((threadIdx.x & 7) * 1e-3f); y[e] = (half_t)(e * 1e-3f); }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x, y, acc[i], 0, 0, 0);
    }
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) sum += (acc[i][0] + acc[i][1]) + (acc[i][2] + acc[i][3]);
    out[blockIdx.x * blockDim.x + threadIdx.x] = sum;
}
// one float4 per thread over n/256 workgroups: the fastest plain copy shape measured here
__global__ __launch_bounds__(256) void copy_peak_kernel(const float4 *src, float4 *dst, size_t n) {
    const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

/* ---------------- GEMV (shaders/gemm_attn.metal:47-74, batched over nb rows of X; gemv.h) ---------------- */
template <typename WT, int NB>
__global__ __launch_bounds__(256) void gemv_kernel(const GemvArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n0 = (blockIdx.x * 4 + wave) * GEMV_ROWS;
    if (n0 >= a.N) return;
    gemv_rows<WT, NB>(a, n0, lane);
}

// Sixteen input rows with bf16 W on MFMA. X is split exactly into three bf16 terms (h = bf16(x),
// m = bf16(x - h), l = x - h - m, which bf16 holds exactly: x - h keeps at most 16 significant bits
// and x - h - m at most 8), so each product W*h, W*m, W*l is exact in f32 and the MFMA sums them in
// f32: an f32-accurate GEMV whose work sits on the matrix cores instead of the VALU (the f32 body
// above spends 8 FMAs and 32 bytes of X reads per weight byte at 16 rows and runs well below the
// HBM rate). Workgroup: 8 waves; the three X planes in LDS (row pitch KS*32 + 8 halves: the 16
// rows of an operand read sit 16 bytes apart mod 128); wave w takes groups of 16 W rows and, per
// group, issues all KS 16-byte row-slice loads before its 3*KS MFMAs (v_mfma_f32_16x16x32_bf16:
// A = 16 W rows x 32 K, B = 32 K x 16 X rows). Output lane l holds rows n0 + 4(l >> 4) + r of
// X row l & 15.
typedef __bf16 gv_bf16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
    const unsigned u = __float_as_uint(x);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
template <int KS>
__global__ __launch_bounds__(512, 1) void gemv_mfma16_kernel(const GemvArgs a) {
    constexpr int K = KS * 32, KP = K + 8, NW = 8;
    constexpr int XIT = 16 * K / 4 / (NW * 64);   // float4 of X per thread
    __shared__ __attribute__((aligned(16))) uint16_t xs[3][16 * KP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // all of this thread's X loads first, then the splits (one load latency, not XIT)
    float4 xv[XIT];
#pragma unroll
    for (int j = 0; j < XIT; ++j) {
        const int i = tid + j * NW * 64, b = i / (K / 4), k = (i - b * (K / 4)) * 4;
        xv[j] = *(const float4 *)(a.X + (long long)b * a.ldx + k);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < XIT; ++j) {
        const int i = tid + j * NW * 64, b = i / (K / 4), k = (i - b * (K / 4)) * 4;
        const float v[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
        ushort4 t[3];
        uint16_t *tp[3] = {(uint16_t *)&t[0], (uint16_t *)&t[1], (uint16_t *)&t[2]};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint16_t h = f32_to_bf16_rne(v[e]);
            const float r1 = v[e] - bf16_to_f32(h);
            const uint16_t m = f32_to_bf16_rne(r1);
            tp[0][e] = h;
            tp[1][e] = m;
            tp[2][e] = f32_to_bf16_rne(r1 - bf16_to_f32(m));
        }
#pragma unroll
        for (int p = 0; p < 3; ++p) *(ushort4 *)(&xs[p][b * KP + k]) = t[p];
    }
    __syncthreads();
    const uint16_t *W = (const uint16_t *)a.W;
    const int kq = (lane >> 4) * 8;
    const int xo = (lane & 15) * KP + kq;
    const int ngroups = (a.N + 15) / 16;
    for (int g = blockIdx.x * NW + wave; g < ngroups; g += gridDim.x * NW) {
        // keeps the X fragment reads inside the loop: hoisted out of it, they hold 3 * KS * 4
        // registers and push the KS row-slice loads into one dependent chain
        asm volatile("" ::: "memory");
        const int n0 = g * 16;
        const int nr = min(n0 + (lane & 15), a.N - 1);
        const uint16_t *wr = W + (long long)nr * a.ldw + kq;
        u16x8 wf[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) wf[s] = *(const u16x8 *)(wr + 32 * s);
        __builtin_amdgcn_sched_barrier(0);   // every slice load issued before the first use
        floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const gv_bf16x8 w = __builtin_bit_cast(gv_bf16x8, wf[s]);
#pragma unroll
            for (int p = 0; p < 3; ++p)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    w, __builtin_bit_cast(gv_bf16x8, *(const u16x8 *)(&xs[p][xo + 32 * s])), acc, 0, 0, 0);
        }
        const int b = lane & 15;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int n = n0 + 4 * (lane >> 4) + r;
            if (n >= a.N) continue;
            float v = acc[r];
            if (a.bias) v += a.bias[n];
            if (a.addv) v += a.addv[(long long)b * a.ld_add + n];
            if (a.silu) v = gemv_silu(v);
            a.Y[(long long)b * a.ldy + n] = v;
            if (a.Y2) a.Y2[(long long)b * a.ldy2 + n] = gemv_silu(v);
        }
    }
}

/* ---------------- f32 SIMT linear: 64x64 tile, 4x4 outputs per thread ---------------- */
template <typename WT>
__device__ inline float load_w1(const WT *p);
template <> __device__ inline float load_w1<uint16_t>(const uint16_t *p) { return bf16_to_f32(*p); }
template <> __device__ inline float load_w1<half_t>(const half_t *p) { return (float)*p; }
template <> __device__ inline float load_w1<float>(const float *p) { return *p; }

template <typename WT>
__global__ __launch_bounds__(256) void linear_f32_kernel(const LinArgs a) {
    __shared__ float sX[16][65];
    __shared__ float sW[16][65];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const WT *W = (const WT *)a.W;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < a.K; k0 += 16) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int idx = tid + 256 * e;       // 1024 = 64 rows x 16 k
            const int rr = idx >> 4, kk = idx & 15;
            const int m = m0 + rr, n = n0 + rr, k = k0 + kk;
            sX[kk][rr] = (m < a.M && k < a.K) ? a.X[rowmap_phys(a.xmap, m) * (long long)a.ldx + k] : 0.0f;
            sW[kk][rr] = (n < a.N && k < a.K) ? load_w1<WT>(W + (long long)n * a.ldw + k) : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            float xr[4], wr[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) xr[i] = sX[kk][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) wr[j] = sW[kk][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] += xr[i] * wr[j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + ty + 16 * i;
        if (m >= a.M) continue;
        float *y = a.Y + rowmap_phys(a.ymap, m) * (long long)a.ldy;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + tx + 16 * j;
            if (n < a.N) y[n] = acc[i][j] + (a.bias ? a.bias[n] : 0.0f);
        }
    }
}

/* ---------------- small kernels ---------------- */
// src/dit_fwd.cpp:111-119: fr_k = (10000/max_period) * 10000^(-2k/D), cos half then sin half
__device__ __forceinline__ void temb_elem(const float *t, float *out, int nb, int D, float max_period, int idx) {
    const int half = D / 2;
    if (idx >= nb * half) return;
    const int b = idx / half, k = idx - b * half;
    const float fr = (10000.0f / max_period) * powf(10000.0f, -2.0f * (float)k / (float)D);
    const float arg = t[b] * fr;
    out[(long long)b * D + k] = cosf(arg);
    out[(long long)b * D + half + k] = sinf(arg);
}
__global__ void temb_kernel(const float *t, float *out, int nb, int D, float max_period) {
    temb_elem(t, out, nb, D, max_period, blockIdx.x * blockDim.x + threadIdx.x);
}

__device__ __forceinline__ void copy_row(const float *src, int lds, RowMap smap, float *dst, int ldd, RowMap dmap, int H, int m) {
    const float *s = src + rowmap_phys(smap, m) * (long long)lds;
    float *d = dst + rowmap_phys(dmap, m) * (long long)ldd;
    for (int c = threadIdx.x; c < H; c += blockDim.x) d[c] = s[c];
}
__global__ void copy_rows_kernel(const float *src, int lds, RowMap smap, float *dst, int ldd, RowMap dmap, int M, int H) {
    const int m = blockIdx.x;
    if (m >= M) return;
    copy_row(src, lds, smap, dst, ldd, dmap, H, m);
}

// shaders/ops_conv.metal:193-201 applied to CFG pairs; both arms of prompt p receive the new x
__global__ void cfg_euler_pairs_kernel(const float *V, float *x2, int P, int n, float cfg, float dt) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)P * n) return;
    const int p = (int)(idx / n), i = (int)(idx - (long long)p * n);
    const float fc = V[(long long)(2 * p) * n + i], fu = V[(long long)(2 * p + 1) * n + i];
    const float v = fu + (fc - fu) * cfg;
    const float xn = x2[(long long)(2 * p) * n + i] + dt * v;
    x2[(long long)(2 * p) * n + i] = xn;
    x2[(long long)(2 * p + 1) * n + i] = xn;
}

__device__ __forceinline__ void split_hilo_elem(const float *x, int ldx, RowMap xmap, half_t *out, int M, int K, long long i) {
    if (i >= (long long)M * K) return;
    const int m = (int)(i / K), k = (int)(i - (long long)m * K);
    const float v = x[rowmap_phys(xmap, m) * (long long)ldx + k];
    const half_t hi = (half_t)v;
    out[(long long)m * 2 * K + k] = hi;
    out[(long long)m * 2 * K + K + k] = (half_t)(v - (float)hi);
}
__global__ void split_hilo_kernel(const float *x, int ldx, RowMap xmap, half_t *out, int M, int K) {
    split_hilo_elem(x, ldx, xmap, out, M, K, (long long)blockIdx.x * blockDim.x + threadIdx.x);
}

// The start of an evaluation in one launch: the timestep sinusoid (optional), the hi|lo split of
// the input latent and the copy of the text rows into the residual stream run on disjoint ranges
// of workgroups (the same element code as temb_kernel, split_hilo_kernel and copy_rows_kernel).
__global__ void eval_prep_kernel(const EvalPrepArgs a) {
    const int nt = a.t ? (int)((a.tnb * (a.tD / 2) + 255) / 256) : 0;
    const int ns = (int)(((long long)a.sM * a.sK + 255) / 256);
    const int blk = blockIdx.x;
    if (blk < nt) {
        temb_elem(a.t, a.temb, a.tnb, a.tD, a.tmax, blk * 256 + threadIdx.x);
    } else if (blk < nt + ns) {
        split_hilo_elem(a.z, a.ldz, a.zmap, a.z2, a.sM, a.sK, (long long)(blk - nt) * 256 + threadIdx.x);
    } else if (blk - nt - ns < a.cM) {
        copy_row(a.csrc, a.clds, a.csmap, a.cdst, a.cldd, a.cdmap, a.cH, blk - nt - ns);
    }
}
__global__ void dup_cols_kernel(const uint16_t *src, half_t *dst, int N, int K) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)N * K) return;
    const int n = (int)(i / K), k = (int)(i - (long long)n * K);
    const half_t w = (half_t)bf16_to_f32(src[i]);
    dst[(long long)n * 2 * K + k] = w;
    dst[(long long)n * 2 * K + K + k] = w;
}
__global__ void bf16_to_f16_kernel(const uint16_t *s, half_t *d, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) d[i] = (half_t)bf16_to_f32(s[i]);
}
__global__ void bf16_to_f32_kernel(const uint16_t *s, float *d, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) d[i] = bf16_to_f32(s[i]);
}
__global__ void f16_to_f32_kernel(const half_t *s, float *d, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) d[i] = (float)s[i];
}
// [OC][IC][K] -> [OC][K][IC]
__global__ void conv_reorder_kernel(const void *src, int src_bf16, half_t *dst, int OC, int IC, int K) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)OC * IC * K;
    if (i >= total) return;
    const int ic = (int)(i % IC);
    const long long r = i / IC;
    const int k = (int)(r % K);
    const int oc = (int)(r / K);
    const long long si = ((long long)oc * IC + ic) * K + k;
    dst[i] = src_bf16 ? (half_t)bf16_to_f32(((const uint16_t *)src)[si]) : ((const half_t *)src)[si];
}

// Upload-time weight layout: src [OC][IC][KT] (bf16, or f32 when src_f32) -> dst row
// r(oc) = (oc % ra)*rb + (oc / ra)*rc + rd, tap-major [KT][IC] within the row, each tap's IC channels
// written twice ([w | w]) when dup; f16 (reference upload rounding) or f32 when out_f32.
// f16 bits -> f32 with subnormals flushed to signed zero (the reference's host conversion of F16
// tensors and Q8_0 block scales, src/gguf.cpp)
__device__ inline float f16_bits_ftz(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1F, m = h & 0x3FF;
    const uint32_t f = e == 0 ? sign : e == 31 ? (sign | 0x7F800000u | (m << 13)) : (sign | ((e + 112) << 23) | (m << 13));
    return __uint_as_float(f);
}

// element si of a source tensor stored as src_type (WP_SRC_*): BF16 exact, f32, F16 with
// subnormals flushed, Q8_0 (blocks of 32: f16 scale, then 32 int8) as scale * q
__device__ inline float wp_load(const void *src, int src_type, long long si) {
    switch (src_type) {
    case WP_SRC_F32: return ((const float *)src)[si];
    case WP_SRC_F16: return f16_bits_ftz(((const uint16_t *)src)[si]);
    case WP_SRC_Q8_0: {
        const unsigned char *blk = (const unsigned char *)src + (si >> 5) * 34;
        const float scale = f16_bits_ftz((uint16_t)(blk[0] | (blk[1] << 8)));
        return scale * (float)(signed char)blk[2 + (si & 31)];
    }
    default: return bf16_to_f32(((const uint16_t *)src)[si]);
    }
}

__global__ void weight_prep_kernel(const void *src, int src_type, void *dst, int out_f32, int OC, int IC, int KT,
                                   int dup, int ra, int rb, int rc, int rd) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)OC * IC * KT) return;
    const int ic = (int)(i % IC);
    const long long q = i / IC;
    const int k = (int)(q % KT);
    const int oc = (int)(q / KT);
    const long long si = ((long long)oc * IC + ic) * KT + k;
    const float w = wp_load(src, src_type, si);
    const long long row = (long long)(oc % ra) * rb + (long long)(oc / ra) * rc + rd;
    const int w_ic = IC * (dup ? 2 : 1);
    const long long d = row * KT * w_ic + (long long)k * w_ic + ic;
    if (out_f32) {
        ((float *)dst)[d] = w;
        if (dup) ((float *)dst)[d + IC] = w;
    } else {
        const half_t h = f32_to_f16_upload(w);
        ((half_t *)dst)[d] = h;
        if (dup) ((half_t *)dst)[d + IC] = h;
    }
}

// y = silu(x[m][c] + v[m / L][c]) as an f16 hi|lo pair: y[m][c] = hi = f16(y), y[m][H + c] =
// f16(y - hi). Rows of extended_c = sync_gather + global_c with SiLU applied, the operand of the
// per-row modulation GEMM against [W | W] (src/dit_fwd.cpp:133-136).
__global__ void bcast_add_silu_kernel(const float *x, const float *v, half_t *y, int L, int M, int H) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)M * H) return;
    const int m = (int)(i / H), c = (int)(i - (long long)m * H);
    const float a = x[i] + v[(long long)(m / L) * H + c];
    const float s = a / (1.0f + __expf(-a));
    const half_t hi = (half_t)s;
    y[(long long)m * 2 * H + c] = hi;
    y[(long long)m * 2 * H + H + c] = (half_t)(s - (float)hi);
}

// out [M][2K] f16 hi|lo of x[m][k] + pe[m % P][k] (pe may be null): the sync features plus their
// 8-periodic positional embedding (src/dit.cpp:93-99), as the operand of the following conv
__global__ void add_period_hilo_kernel(const float *x, const float *pe, int P, half_t *out, int M, int K) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)M * K) return;
    const int m = (int)(i / K), k = (int)(i - (long long)m * K);
    const float v = x[i] + (pe ? pe[(long long)(m % P) * K + k] : 0.0f);
    const half_t hi = (half_t)v;
    out[(long long)m * 2 * K + k] = hi;
    out[(long long)m * 2 * K + K + k] = (half_t)(v - (float)hi);
}

// dst[i] = src[idx[i]], rows of H floats
__global__ void gather_rows_kernel(const float *src, const int32_t *idx, float *dst, int rows, int H) {
    const int r = blockIdx.x;
    if (r >= rows) return;
    const float *s = src + (long long)idx[r] * H;
    float *d = dst + (long long)r * H;
    for (int c = threadIdx.x; c < H; c += blockDim.x) d[c] = s[c];
}

// out[c] = (sum over rows r in order of x[r][c]) / rows: one thread per column, fixed order
__global__ void mean_rows_kernel(const float *x, int rows, int H, float *out) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= H) return;
    float acc = 0.0f;
    for (int r = 0; r < rows; ++r) acc += x[(long long)r * H + c];
    out[c] = acc / (float)rows;
}

// reference-surface elementwise kernels (shaders/ops_conv.metal:9-57,146-169,193-201)
__global__ void silu_kernel(float *x, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = x[i] / (1.0f + expf(-x[i]));
}
__global__ void copy_kernel(const float *x, float *y, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = x[i];
}
__global__ void swiglu_kernel(const float *a, const float *b, float *y, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) { const float va = a[i]; y[i] = (va / (1.0f + expf(-va))) * b[i]; }
}
__global__ void add_kernel(const float *a, const float *b, float *y, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = a[i] + b[i];
}
__global__ void add_bcast_col_kernel(const float *x, const float *v, float *y, int H, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = x[i] + v[i % H];
}
__global__ void cfg_euler_kernel(const float *fc, const float *fu, float *x, size_t n, float cfg, float dt) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) { const float v = fu[i] + (fc[i] - fu[i]) * cfg; x[i] += dt * v; }
}
__global__ void gate_add_kernel(const float *x, const float *f, const float *mod, float *y, int H, int per_row,
                                int chunks, int gate_idx, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const size_t s = i / H, c = i % H;
    const float *m = mod + (per_row ? s * (size_t)chunks * H : 0);
    y[i] = x[i] + f[i] * m[(size_t)gate_idx * H + c];
}
// one wave per (row, head)
__global__ void rms_head_kernel(float *x, const float *w, int rows, int nh, int ld, int hd, int col_off,
                                int row_off, float eps) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int id = blockIdx.x * 4 + wave;
    if (id >= rows * nh) return;
    const int r = id / nh, h = id - r * nh;
    float *p = x + (long long)(row_off + r) * ld + col_off + (long long)h * hd;
    float ss = 0.0f;
    for (int i = lane; i < hd; i += 64) ss += p[i] * p[i];
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)hd + eps);
    for (int i = lane; i < hd; i += 64) p[i] = p[i] * inv * w[i];
}
__global__ void rope_pairs_kernel(float *x, const int32_t *pos, int rows, int nh, int ld, int hd, int col_off,
                                  int row_off, float fscale, float base) {
    const long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int npair = hd / 2;
    if (id >= (long long)rows * nh * npair) return;
    const int r = (int)(id / (nh * npair));
    const int rem = (int)(id - (long long)r * nh * npair);
    const int h = rem / npair, j = rem - h * npair;
    const float inv = powf(base, -2.0f * (float)j / (float)hd);
    const float ang = (float)(pos ? pos[r] : r) * fscale * inv;
    const float cs = cosf(ang), sn = sinf(ang);
    float *p = x + (long long)(row_off + r) * ld + col_off + (long long)h * hd;
    const float x0 = p[2 * j], x1 = p[2 * j + 1];
    p[2 * j] = x0 * cs - x1 * sn;
    p[2 * j + 1] = x0 * sn + x1 * cs;
}

inline unsigned blocks_for(size_t n, unsigned t = 256) { return (unsigned)((n + t - 1) / t); }

/* ---------------- final layer: adaLN + projection to the latent channels (src/dit_fwd.cpp:287-303) ---------------- */
// 16 audio rows per workgroup. Wave w normalises rows 4w .. 4w + 3 exactly as ln_mod_kernel does
// (f32 statistics, one wave per row) and parks y as an f16 hi|lo pair in an LDS tile (row pitch
// 2H + 8 halves: the 16 rows of an MFMA operand read fall 16 bytes apart mod 128, no bank
// conflicts). Then wave w computes output columns 16w .. 16w + 15 for the 16 rows with
// v_mfma_f32_16x16x32_f16, the hi half and the lo half of each 32-wide K slice against the same f16
// weight columns (an f32-accurate operand), and adds the bias. One launch instead of an LN launch, a
// split-K GEMM and its reduce.
//
// Latency, not work, sets its time (32 workgroups at 8 s): the loads of the first eight weight
// slices are issued at entry, before the normalisation they do not depend on, and each later slice
// eight steps ahead of its use; a wave's rows are normalised in batches whose loads are all issued
// before the first row's reductions.
template <int NV>
__global__ __launch_bounds__(256) void final_out_kernel(const FinalArgs a) {
    constexpr int H = 256 * NV, P = 2 * H + 8;
    constexpr int RB = NV <= 4 ? 4 : 2;   // rows per load batch (RB * 3 * NV float4 registers)
    constexpr int WD = 8;                 // weight slices in flight
    __shared__ __attribute__((aligned(16))) half_t tileA[16 * P];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row0 = blockIdx.x * 16;
    const int n0 = wave * 16;
    const bool has_n = n0 < a.N;   // wave-uniform
    const int n = n0 + (lane & 15), kg = (lane >> 4) * 8;
    const half_t *wrow = a.W + (long long)(has_n ? n : 0) * a.ldw + kg;
    half8 wb[WD];
    if (has_n) {
#pragma unroll
        for (int i = 0; i < WD; ++i) wb[i] = *(const half8 *)(wrow + 32 * i);
    }
#pragma unroll 1
    for (int j0 = 0; j0 < 4; j0 += RB) {
        float4 xv[RB][NV], sh[RB][NV], scl[RB][NV];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int v = row0 + wave * 4 + j0 + r;
            if (v >= a.rows) break;   // wave-uniform
            const float *x = a.X + rowmap_phys(a.xmap, v) * (long long)a.ldx;
            const float *mb = a.mod + (long long)(v / a.mod_L) * a.mod_ld;
#pragma unroll
            for (int c = 0; c < NV; ++c) {
                xv[r][c] = *(const float4 *)(x + c * 256 + lane * 4);
                sh[r][c] = *(const float4 *)(mb + a.shift_off + c * 256 + lane * 4);
                scl[r][c] = *(const float4 *)(mb + a.scale_off + c * 256 + lane * 4);
            }
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int lr = wave * 4 + j0 + r, v = row0 + lr;
            if (v >= a.rows) break;   // rows past the end are never stored
            float sum = 0.0f;
#pragma unroll
            for (int c = 0; c < NV; ++c) sum += (xv[r][c].x + xv[r][c].y) + (xv[r][c].z + xv[r][c].w);
            const float inv_h = 1.0f / (float)H;
            const float mean = wave_sum(sum) * inv_h;
            float var = 0.0f;
#pragma unroll
            for (int c = 0; c < NV; ++c) {
                const float d0 = xv[r][c].x - mean, d1 = xv[r][c].y - mean, d2 = xv[r][c].z - mean, d3 = xv[r][c].w - mean;
                var += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
            }
            var = wave_sum(var) * inv_h;
            const float inv = 1.0f / sqrtf(var + a.eps);
#pragma unroll
            for (int c = 0; c < NV; ++c) {
                const int col = c * 256 + lane * 4;
                const float y0 = (xv[r][c].x - mean) * inv * (1.0f + scl[r][c].x) + sh[r][c].x;
                const float y1 = (xv[r][c].y - mean) * inv * (1.0f + scl[r][c].y) + sh[r][c].y;
                const float y2 = (xv[r][c].z - mean) * inv * (1.0f + scl[r][c].z) + sh[r][c].z;
                const float y3 = (xv[r][c].w - mean) * inv * (1.0f + scl[r][c].w) + sh[r][c].w;
                const half4 hi = half4{(half_t)y0, (half_t)y1, (half_t)y2, (half_t)y3};
                *(half4 *)(tileA + lr * P + col) = hi;
                *(half4 *)(tileA + lr * P + H + col) = half4{(half_t)(y0 - (float)hi[0]), (half_t)(y1 - (float)hi[1]),
                                                             (half_t)(y2 - (float)hi[2]), (half_t)(y3 - (float)hi[3])};
            }
        }
    }
    __syncthreads();
    if (!has_n) return;
    const half_t *arow = tileA + (lane & 15) * P + kg;
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int k0 = 0; k0 < H; k0 += 32 * WD) {
#pragma unroll
        for (int i = 0; i < WD; ++i) {
            const half8 bf = wb[i];
            const int k = k0 + 32 * i;
            if (k0 + 32 * WD < H) wb[i] = *(const half8 *)(wrow + k + 32 * WD);   // uniform
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const half8 *)(arow + k), bf, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const half8 *)(arow + H + k), bf, acc, 0, 0, 0);
        }
    }
    const float bn = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int v = row0 + 4 * (lane >> 4) + r;
        if (v < a.rows) a.Y[(long long)v * a.ldy + n] = acc[r] + bn;
    }
}

} // namespace

int launch_final_out(const FinalArgs &a, hipStream_t st) {
    TSN_REQUIRE(a.X && a.mod && a.W && a.Y && a.rows > 0 && a.mod_L > 0 && a.xmap.L > 0, "final: arguments");
    TSN_REQUIRE(a.H % 256 == 0 && a.H >= 256 && a.H <= 2048, "final: H must be a multiple of 256 in [256, 2048]");
    TSN_REQUIRE(a.N > 0 && a.N <= 64 && a.N % 16 == 0, "final: N must be a multiple of 16 up to 64");
    TSN_REQUIRE(a.ldx % 4 == 0 && a.mod_ld % 4 == 0 && a.shift_off % 4 == 0 && a.scale_off % 4 == 0 && a.ldw % 8 == 0 &&
                    a.ldw >= a.H && (((uintptr_t)a.W) & 15) == 0 && (((uintptr_t)a.X | (uintptr_t)a.mod) & 15) == 0,
                "final: strides, offsets and alignment");
    const dim3 grid((unsigned)((a.rows + 15) / 16)), block(256);
    switch (a.H / 256) {
        case 1: TSN_LAUNCH(final_out_kernel<1>, grid, block, 0, st, a); break;
        case 2: TSN_LAUNCH(final_out_kernel<2>, grid, block, 0, st, a); break;
        case 3: TSN_LAUNCH(final_out_kernel<3>, grid, block, 0, st, a); break;
        case 4: TSN_LAUNCH(final_out_kernel<4>, grid, block, 0, st, a); break;
        case 5: TSN_LAUNCH(final_out_kernel<5>, grid, block, 0, st, a); break;
        case 6: TSN_LAUNCH(final_out_kernel<6>, grid, block, 0, st, a); break;
        case 7: TSN_LAUNCH(final_out_kernel<7>, grid, block, 0, st, a); break;
        default: TSN_LAUNCH(final_out_kernel<8>, grid, block, 0, st, a); break;
    }
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

bool pf_ranges_ok(const PfRange (&pf)[PF_RANGES]) {
    for (int i = 0; i < PF_RANGES; ++i)
        if (pf[i].rows < 0 || (pf[i].rows > 0 && (!pf[i].p || pf[i].row_bytes <= 0 || pf[i].row_bytes % 128 ||
                                                   pf[i].ld % 128 || pf[i].ld < pf[i].row_bytes)))
            return false;
    return true;
}

int pf_workgroups(const PfRange (&pf)[PF_RANGES], int waves) {
    long long lines = 0;
    for (int i = 0; i < PF_RANGES; ++i) lines += (long long)pf[i].rows * (pf[i].row_bytes >> 7);
    const long long per = (long long)waves * 64 * PF_PER_LANE;
    return (int)((lines + per - 1) / per);
}

int launch_ln_mod(const LnArgs &a, int ymode, hipStream_t st) {
    TSN_REQUIRE(ymode == LN_F32 || ymode == LN_F16 || ymode == LN_F16_HILO, "ln: output mode");
    TSN_REQUIRE(a.nseg >= 1 && a.nseg <= 3, "ln: 1 to 3 segments");
    TSN_REQUIRE(a.H % 256 == 0 && a.H >= 256 && a.H <= 2048, "ln: H must be a multiple of 256 in [256, 2048]");
    int total = 0;
    for (int i = 0; i < a.nseg; ++i) {
        const LnSeg &s = a.seg[i];
        TSN_REQUIRE(s.X && s.Y && s.mod && s.rows > 0 && s.mod_L > 0 && s.xmap.L > 0 && s.ymap.L > 0, "ln: segment");
        TSN_REQUIRE(s.ldx % 4 == 0 && s.ldy % 4 == 0 && s.mod_ld % 4 == 0 && s.shift_off % 4 == 0 && s.scale_off % 4 == 0,
                    "ln: strides and offsets must be multiples of 4");
        TSN_REQUIRE(ymode != LN_F16_HILO || s.ldy >= 2 * a.H, "ln: hi|lo output needs ldy >= 2H");
        total += s.rows;
    }
    TSN_REQUIRE(pf_ranges_ok(a.pf), "ln: prefetch ranges");
    LnArgs b = a;
    b.pf_nwg = pf_workgroups(a.pf, 4);
    dim3 grid(b.pf_nwg + (total + 3) / 4), block(256);
    const int nv = a.H / 256;
#define TSN_LN_CASE(NVV)                                                                           \
    case NVV:                                                                                      \
        if (ymode == LN_F16) TSN_LAUNCH((ln_mod_kernel<LN_F16, NVV>), grid, block, 0, st, b); \
        else if (ymode == LN_F16_HILO)                                                             \
            TSN_LAUNCH((ln_mod_kernel<LN_F16_HILO, NVV>), grid, block, 0, st, b);          \
        else TSN_LAUNCH((ln_mod_kernel<LN_F32, NVV>), grid, block, 0, st, b);              \
        break;
    switch (nv) {
        TSN_LN_CASE(1) TSN_LN_CASE(2) TSN_LN_CASE(3) TSN_LN_CASE(4)
        TSN_LN_CASE(5) TSN_LN_CASE(6) TSN_LN_CASE(7) TSN_LN_CASE(8)
        default: set_error("ln: unsupported H"); return TSN_ERR_UNSUPPORTED;
    }
#undef TSN_LN_CASE
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_reduce_ln(const RedLnArgs &a, hipStream_t st) {
    TSN_REQUIRE(a.nseg >= 1 && a.nseg <= 3, "reduce_ln: 1 to 3 segments");
    TSN_REQUIRE(a.H % 256 == 0 && a.H >= 256 && a.H <= 2048, "reduce_ln: H must be a multiple of 256 in [256, 2048]");
    TSN_REQUIRE(a.ymode == LN_F16 || a.ymode == LN_F16_HILO, "reduce_ln: output mode");
    int total = 0;
    for (int i = 0; i < a.nseg; ++i) {
        const RedLnSeg &s = a.seg[i];
        TSN_REQUIRE(s.X && s.M > 0 && s.xmap.L > 0 && s.ldx % 4 == 0, "reduce_ln: residual rows");
        TSN_REQUIRE(s.splits <= 1 || (s.ws && s.gate && s.gate_L > 0 && s.gate_ld % 4 == 0), "reduce_ln: partials");
        TSN_REQUIRE(!s.ln || (s.mod && s.Y && s.mod_L > 0 && s.ymap.L > 0 && s.mod_ld % 4 == 0 &&
                              s.shift_off % 4 == 0 && s.scale_off % 4 == 0 && s.ldy % 4 == 0),
                    "reduce_ln: layer-norm output");
        TSN_REQUIRE(!s.ln || (a.ymode != LN_F16_HILO && !s.hilo) || s.ldy >= 2 * a.H,
                    "reduce_ln: hi|lo output needs ldy >= 2H");
        total += s.M;
    }
    TSN_REQUIRE(pf_ranges_ok(a.pf) && (pf_workgroups(a.pf, 4) == 0 || a.H == 1024),
                "reduce_ln: prefetch ranges (prefetch workgroups need 4 waves: H = 1024)");
    RedLnArgs b = a;
    b.pf_nwg = pf_workgroups(a.pf, 4);
    dim3 grid(b.pf_nwg + total), block(a.H / 4);
    if (a.ymode == LN_F16_HILO) TSN_LAUNCH((reduce_ln_kernel<LN_F16_HILO>), grid, block, 0, st, b);
    else TSN_LAUNCH((reduce_ln_kernel<LN_F16>), grid, block, 0, st, b);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_mfma_peak(float *out, int nwg, int iters, hipStream_t st) {
    TSN_REQUIRE(out && nwg > 0 && iters > 0, "mfma probe: arguments");
    TSN_LAUNCH(mfma_peak_kernel, dim3(nwg), dim3(512), 0, st, out, iters);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_copy_peak(const float *src, float *dst, size_t n4, hipStream_t st) {
    TSN_REQUIRE(src && dst && n4 > 0, "copy probe: arguments");
    TSN_REQUIRE((n4 + 255) / 256 <= 0x7FFFFFFFull, "copy probe: too many elements");
    TSN_LAUNCH(copy_peak_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, (const float4 *)src, (float4 *)dst, n4);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_gemv(const GemvArgs &a, hipStream_t st) {
    TSN_REQUIRE(a.W && a.X && a.Y && a.N > 0 && a.K > 0, "gemv: arguments");
    TSN_REQUIRE(a.nb >= 1 && a.nb <= 16, "gemv: 1..16 input rows");
    TSN_REQUIRE(a.K % 8 == 0 && a.ldw % 8 == 0 && a.ldx % 4 == 0, "gemv: K, ldw multiple of 8; ldx multiple of 4");
    const int rows_per_block = 4 * GEMV_ROWS;
    dim3 grid((a.N + rows_per_block - 1) / rows_per_block), block(256);
#define TSN_GEMV_NB(WT, NBV)                                                                       \
    case NBV: TSN_LAUNCH((gemv_kernel<WT, NBV>), grid, block, 0, st, a); break;
#define TSN_GEMV_W(WT)                                                                             \
    switch (nb) {                                                                                  \
        TSN_GEMV_NB(WT, 1) TSN_GEMV_NB(WT, 2) TSN_GEMV_NB(WT, 4) TSN_GEMV_NB(WT, 8)                \
        TSN_GEMV_NB(WT, 16)                                                                        \
        default: break;                                                                            \
    }
    // round nb up to a compiled batch count; extra rows are computed but never written
    int nb = a.nb <= 1 ? 1 : a.nb <= 2 ? 2 : a.nb <= 4 ? 4 : a.nb <= 8 ? 8 : 16;
    if (nb != a.nb) {
        // the kernel reads X rows up to nb-1: only valid when the caller's X has them
        set_error("gemv: nb must be 1, 2, 4, 8 or 16");
        return TSN_ERR_UNSUPPORTED;
    }
    const int ks = a.K / 32;
    // Sixteen rows of X on MFMA: a workgroup per CU at most, each wave over groups of 16 W rows
    // (batch-16 adaLN modulation, 131072 x 1024: about 90 against 200 us per launch; batch-16
    // evaluation 7.158 -> 7.048 ms, same box). Routing the 1024 x 1024 t-MLP layer (64 row groups)
    // to the f32 body instead measured no better (7.060 ms).
    if (a.wdt == DT_BF16 && nb == 16 && a.K % 32 == 0 && (ks == 8 || ks == 16 || ks == 32) &&
        (((uintptr_t)a.W | (uintptr_t)a.X) & 15) == 0) {
        const int groups = (a.N + 15) / 16;
        const dim3 g2((unsigned)std::min(256, (groups + 7) / 8)), b2(512);
        if (ks == 8) TSN_LAUNCH(gemv_mfma16_kernel<8>, g2, b2, 0, st, a);
        else if (ks == 16) TSN_LAUNCH(gemv_mfma16_kernel<16>, g2, b2, 0, st, a);
        else TSN_LAUNCH(gemv_mfma16_kernel<32>, g2, b2, 0, st, a);
    } else if (a.wdt == DT_BF16) { TSN_GEMV_W(uint16_t) }
    else if (a.wdt == DT_F16) { TSN_GEMV_W(half_t) }
    else if (a.wdt == DT_F32) { TSN_GEMV_W(float) }
    else { set_error("gemv: weight dtype"); return TSN_ERR_ARG; }
#undef TSN_GEMV_W
#undef TSN_GEMV_NB
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_linear_f32(const LinArgs &a, hipStream_t st) {
    TSN_REQUIRE(a.X && a.W && a.Y && a.M > 0 && a.N > 0 && a.K > 0, "linear_f32: arguments");
    TSN_REQUIRE(a.xmap.L > 0 && a.ymap.L > 0, "linear_f32: row maps");
    dim3 grid((a.N + 63) / 64, (a.M + 63) / 64), block(256);
    if (a.wdt == DT_BF16) TSN_LAUNCH(linear_f32_kernel<uint16_t>, grid, block, 0, st, a);
    else if (a.wdt == DT_F16) TSN_LAUNCH(linear_f32_kernel<half_t>, grid, block, 0, st, a);
    else if (a.wdt == DT_F32) TSN_LAUNCH(linear_f32_kernel<float>, grid, block, 0, st, a);
    else { set_error("linear_f32: weight dtype"); return TSN_ERR_ARG; }
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_temb_sinusoid(const float *t, float *out, int nb, int D, float max_period, hipStream_t st) {
    TSN_REQUIRE(t && out && nb > 0 && D > 0 && D % 2 == 0, "temb: arguments");
    TSN_LAUNCH(temb_kernel, dim3(blocks_for((size_t)nb * D / 2)), dim3(256), 0, st, t, out, nb, D, max_period);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_copy_rows(const float *src, int lds, RowMap smap, float *dst, int ldd, RowMap dmap, int M, int H, hipStream_t st) {
    TSN_REQUIRE(src && dst && M > 0 && H > 0 && smap.L > 0 && dmap.L > 0, "copy_rows: arguments");
    TSN_LAUNCH(copy_rows_kernel, dim3(M), dim3(256), 0, st, src, lds, smap, dst, ldd, dmap, M, H);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_cfg_euler_pairs(const float *V, float *x2, int P, int n, float cfg, float dt, hipStream_t st) {
    TSN_REQUIRE(V && x2 && P > 0 && n > 0, "cfg_euler_pairs: arguments");
    TSN_LAUNCH(cfg_euler_pairs_kernel, dim3(blocks_for((size_t)P * n)), dim3(256), 0, st, V, x2, P, n, cfg, dt);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_eval_prep(const EvalPrepArgs &a, hipStream_t st) {
    TSN_REQUIRE(!a.t || (a.temb && a.tnb > 0 && a.tD > 0 && a.tD % 2 == 0), "eval_prep: timestep part");
    TSN_REQUIRE(a.z && a.z2 && a.sM > 0 && a.sK > 0 && a.zmap.L > 0, "eval_prep: split part");
    TSN_REQUIRE(a.cM == 0 || (a.csrc && a.cdst && a.cH > 0 && a.csmap.L > 0 && a.cdmap.L > 0), "eval_prep: copy part");
    const long long nt = a.t ? (a.tnb * (long long)(a.tD / 2) + 255) / 256 : 0;
    const long long ns = ((long long)a.sM * a.sK + 255) / 256;
    TSN_LAUNCH(eval_prep_kernel, dim3((unsigned)(nt + ns + a.cM)), dim3(256), 0, st, a);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_split_hilo(const float *x, int ldx, RowMap xmap, half_t *out, int M, int K, hipStream_t st) {
    TSN_REQUIRE(x && out && M > 0 && K > 0 && xmap.L > 0, "split_hilo: arguments");
    TSN_LAUNCH(split_hilo_kernel, dim3(blocks_for((size_t)M * K)), dim3(256), 0, st, x, ldx, xmap, out, M, K);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_dup_cols_bf16_to_f16(const uint16_t *src, half_t *dst, int N, int K, hipStream_t st) {
    TSN_REQUIRE(src && dst && N > 0 && K > 0, "dup_cols: arguments");
    TSN_LAUNCH(dup_cols_kernel, dim3(blocks_for((size_t)N * K)), dim3(256), 0, st, src, dst, N, K);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_bf16_to_f16(const uint16_t *src, half_t *dst, size_t n, hipStream_t st) {
    if (n == 0) return TSN_OK;
    TSN_LAUNCH(bf16_to_f16_kernel, dim3(blocks_for(n)), dim3(256), 0, st, src, dst, n);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_bf16_to_f32(const uint16_t *src, float *dst, size_t n, hipStream_t st) {
    if (n == 0) return TSN_OK;
    TSN_LAUNCH(bf16_to_f32_kernel, dim3(blocks_for(n)), dim3(256), 0, st, src, dst, n);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_f16_to_f32(const half_t *src, float *dst, size_t n, hipStream_t st) {
    if (n == 0) return TSN_OK;
    TSN_LAUNCH(f16_to_f32_kernel, dim3(blocks_for(n)), dim3(256), 0, st, src, dst, n);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_conv_weight_reorder(const void *src, int src_bf16, half_t *dst, int OC, int IC, int K, hipStream_t st) {
    TSN_REQUIRE(src && dst && OC > 0 && IC > 0 && K > 0, "conv_reorder: arguments");
    const size_t n = (size_t)OC * IC * K;
    TSN_LAUNCH(conv_reorder_kernel, dim3(blocks_for(n)), dim3(256), 0, st, src, src_bf16, dst, OC, IC, K);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_weight_prep(const void *src, int src_type, void *dst, int out_f32, int OC, int IC, int KT, int dup, int ra,
                       int rb, int rc, int rd, long long dst_rows, hipStream_t st) {
    TSN_REQUIRE(src && dst && OC > 0 && IC > 0 && KT > 0 && ra > 0 && dst_rows > 0, "weight_prep: arguments");
    TSN_REQUIRE(src_type >= WP_SRC_BF16 && src_type <= WP_SRC_Q8_0, "weight_prep: source type");
    TSN_REQUIRE(src_type != WP_SRC_Q8_0 || ((long long)OC * IC * KT) % 32 == 0, "weight_prep: Q8_0 needs whole blocks of 32");
    TSN_REQUIRE(((uintptr_t)src) % (src_type == WP_SRC_F32 ? 4 : src_type == WP_SRC_Q8_0 ? 1 : 2) == 0,
                "weight_prep: misaligned source");
    for (int oc = 0; oc < OC; ++oc) {   // every destination row inside the destination
        const long long row = (long long)(oc % ra) * rb + (long long)(oc / ra) * rc + rd;
        TSN_REQUIRE(row >= 0 && row < dst_rows, "weight_prep: row map leaves the destination");
    }
    const size_t n = (size_t)OC * IC * KT;
    TSN_LAUNCH(weight_prep_kernel, dim3(blocks_for(n)), dim3(256), 0, st, src, src_type, dst, out_f32, OC, IC, KT, dup,
               ra, rb, rc, rd);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_bcast_add_silu_f16(const float *x, const float *v, half_t *y, int L, int M, int H, hipStream_t st) {
    TSN_REQUIRE(x && v && y && L > 0 && M > 0 && H > 0, "bcast_add_silu: arguments");
    TSN_LAUNCH(bcast_add_silu_kernel, dim3(blocks_for((size_t)M * H)), dim3(256), 0, st, x, v, y, L, M, H);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_add_period_hilo(const float *x, const float *pe, int P, half_t *out, int M, int K, hipStream_t st) {
    TSN_REQUIRE(x && out && M > 0 && K > 0 && (!pe || P > 0), "add_period_hilo: arguments");
    TSN_LAUNCH(add_period_hilo_kernel, dim3(blocks_for((size_t)M * K)), dim3(256), 0, st, x, pe, P, out, M, K);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_gather_rows(const float *src, const int32_t *idx, float *dst, int rows, int H, hipStream_t st) {
    TSN_REQUIRE(src && idx && dst && rows > 0 && H > 0, "gather_rows: arguments");
    TSN_LAUNCH(gather_rows_kernel, dim3(rows), dim3(256), 0, st, src, idx, dst, rows, H);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_mean_rows(const float *x, int rows, int H, float *out, hipStream_t st) {
    TSN_REQUIRE(x && out && rows > 0 && H > 0, "mean_rows: arguments");
    TSN_LAUNCH(mean_rows_kernel, dim3((H + 255) / 256), dim3(256), 0, st, x, rows, H, out);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_silu(float *x, size_t n, hipStream_t st) {
    TSN_REQUIRE(x || n == 0, "silu: null");
    if (n == 0) return TSN_OK;
    TSN_LAUNCH(silu_kernel, dim3(blocks_for(n)), dim3(256), 0, st, x, n);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_copy(const float *x, float *y, size_t n, hipStream_t st) {
    TSN_REQUIRE((x && y) || n == 0, "copy: null");
    if (n == 0) return TSN_OK;
    TSN_LAUNCH(copy_kernel, dim3(blocks_for(n)), dim3(256), 0, st, x, y, n);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_swiglu(const float *a, const float *b, float *y, size_t n, hipStream_t st) {
    TSN_REQUIRE((a && b && y) || n == 0, "swiglu: null");
    if (n == 0) return TSN_OK;
    TSN_LAUNCH(swiglu_kernel, dim3(blocks_for(n)), dim3(256), 0, st, a, b, y, n);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_add(const float *a, const float *b, float *y, size_t n, hipStream_t st) {
    TSN_REQUIRE((a && b && y) || n == 0, "add: null");
    if (n == 0) return TSN_OK;
    TSN_LAUNCH(add_kernel, dim3(blocks_for(n)), dim3(256), 0, st, a, b, y, n);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_add_bcast_col(const float *x, const float *v, float *y, int S, int H, hipStream_t st) {
    TSN_REQUIRE(x && v && y && S > 0 && H > 0, "add_bcast_col: arguments");
    const size_t n = (size_t)S * H;
    TSN_LAUNCH(add_bcast_col_kernel, dim3(blocks_for(n)), dim3(256), 0, st, x, v, y, H, n);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_cfg_euler(const float *fc, const float *fu, float *x, size_t n, float cfg, float dt, hipStream_t st) {
    TSN_REQUIRE((fc && fu && x) || n == 0, "cfg_euler: null");
    if (n == 0) return TSN_OK;
    TSN_LAUNCH(cfg_euler_kernel, dim3(blocks_for(n)), dim3(256), 0, st, fc, fu, x, n, cfg, dt);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_gate_add(const float *x, const float *f, const float *mod, float *y, int rows, int H, int per_row,
                    int chunks, int gate_idx, hipStream_t st) {
    TSN_REQUIRE(x && f && mod && y && rows > 0 && H > 0 && gate_idx >= 0 && gate_idx < chunks, "gate_add: arguments");
    const size_t n = (size_t)rows * H;
    TSN_LAUNCH(gate_add_kernel, dim3(blocks_for(n)), dim3(256), 0, st, x, f, mod, y, H, per_row, chunks, gate_idx, n);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_rms_head(float *x, const float *w, int rows, int nh, int ld, int hd, int col_off, int row_off,
                    float eps, hipStream_t st) {
    TSN_REQUIRE(x && w && rows > 0 && nh > 0 && hd > 0, "rms_head: arguments");
    const int n = rows * nh;
    TSN_LAUNCH(rms_head_kernel, dim3((n + 3) / 4), dim3(256), 0, st, x, w, rows, nh, ld, hd, col_off, row_off, eps);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}
int launch_rope_pairs(float *x, const int32_t *pos, int rows, int nh, int ld, int hd, int col_off, int row_off,
                      float fscale, float base, hipStream_t st) {
    TSN_REQUIRE(x && rows > 0 && nh > 0 && hd > 0 && hd % 2 == 0, "rope_pairs: arguments");
    const size_t n = (size_t)rows * nh * (hd / 2);
    TSN_LAUNCH(rope_pairs_kernel, dim3(blocks_for(n)), dim3(256), 0, st, x, pos, rows, nh, ld, hd, col_off,
                       row_off, fscale, base);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

} // namespace tsn
