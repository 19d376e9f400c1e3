// enc.hip — kernels of the text encoders (src/clip.cpp, src/t5.cpp): f32 GEMM on the f32 MFMA,
// LayerNorm with weight and bias, RMSNorm with weight, attention over one short context with the
// CLIP causal/EOT mask or the T5 bucketed relative bias and padding mask, GEGLU, and the token
// (+ position) embedding gather. Everything stays f32: T5's activations leave the f16 range.
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "dpp.h"

namespace tsn {

namespace {

typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int FB_MT = 5;                 // 16-row MFMA blocks per tile: 80 rows hold a 77-token prompt
constexpr int FB_M = 16 * FB_MT, FB_N = 64, FB_K = 64, FB_LD = FB_K + 1;

// The epilogue of one output element: v = sum + bias, then Y = act(v) or Y += v.
__device__ __forceinline__ void enc_epi(const EncGemmArgs &g, int m, int n, float v) {
    if (g.bias) v += g.bias[n];
    float *y = g.Y + (long long)m * g.ldy + n;
    if (g.resid) {
        *y = *y + v;
    } else {
        if (g.act == 1) v = v / (1.0f + expf(-1.702f * v));   // quick GELU (shaders/ops_conv.metal:25-29)
        *y = v;
    }
}

// 4 waves; wave w owns columns 16w..16w+15 of an 80x64 tile (five 16x16 blocks of
// v_mfma_f32_16x16x4_f32 per 4-wide K slice). With 80 rows a whole prompt is one row tile, so each
// weight is read from HBM once. A and W reach LDS in 64-wide K stages; the next stage is loaded into
// registers while the current one is multiplied. blockIdx.z = split: K tiles [z*kps, (z+1)*kps);
// with more than one split the raw sums go to ws[z][M][N] and enc_gemm_reduce_kernel adds them in
// split order.
__global__ __launch_bounds__(256) void gemm_f32_kernel(const EncGemmArgs g) {
    __shared__ float As[2][FB_M * FB_LD];
    __shared__ float Ws[2][FB_N * FB_LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * FB_N, m0 = blockIdx.y * FB_M, z = blockIdx.z;
    const int M = g.M, N = g.N, K = g.K;
    const int nkt = (K + FB_K - 1) / FB_K;
    const int kt0 = z * g.kps, kt1 = min(nkt, kt0 + g.kps);
    // loader: 16 lanes per 64-wide row (4 floats each); A rows lr + 16i (i < 5), W rows lr + 16i (i < 4).
    // Two register sets: K tile kt + 2 is fetched while kt is multiplied and kt + 1 waits in the
    // other set, so a tile has two K steps of MFMA work to arrive from HBM.
    const int lr = tid >> 4, lc = (tid & 15) * 4;
    float4 ra0[FB_MT], rw0[4], ra1[FB_MT], rw1[4];
    auto fetch = [&](int kt, float4 (&ra)[FB_MT], float4 (&rw)[4]) {
        const int k = kt * FB_K + lc;
        const bool kin = k < K;
        const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < FB_MT; ++i) {
            const int m = m0 + lr + 16 * i;
            ra[i] = (kin && m < M) ? *(const float4 *)(g.A + (long long)m * g.lda + k) : z4;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = n0 + lr + 16 * i;
            rw[i] = (kin && n < N) ? *(const float4 *)(g.W + (long long)n * g.ldw + k) : z4;
        }
    };
    auto stash = [&](int b, const float4 (&ra)[FB_MT], const float4 (&rw)[4]) {
#pragma unroll
        for (int i = 0; i < FB_MT; ++i) {
            float *a = &As[b][(lr + 16 * i) * FB_LD + lc];
            a[0] = ra[i].x; a[1] = ra[i].y; a[2] = ra[i].z; a[3] = ra[i].w;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float *w = &Ws[b][(lr + 16 * i) * FB_LD + lc];
            w[0] = rw[i].x; w[1] = rw[i].y; w[2] = rw[i].z; w[3] = rw[i].w;
        }
    };
    floatx4_t acc[FB_MT];
#pragma unroll
    for (int i = 0; i < FB_MT; ++i) acc[i] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    const int r16 = lane & 15, kq = lane >> 4;   // operand lane: row / column r16, k offset kq
    auto compute = [&](int b) {
        const float *as = As[b], *ws = Ws[b];
#pragma unroll
        for (int kk = 0; kk < FB_K; kk += 4) {
            const float bv = ws[(wave * 16 + r16) * FB_LD + kk + kq];
#pragma unroll
            for (int i = 0; i < FB_MT; ++i)
                acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(as[(16 * i + r16) * FB_LD + kk + kq], bv, acc[i], 0, 0, 0);
        }
    };
    // K tile kt0 + r lives in LDS buffer r & 1 and, before that, in register set r & 1
    if (kt0 < kt1) {
        fetch(kt0, ra0, rw0);
        stash(0, ra0, rw0);
        if (kt0 + 1 < kt1) fetch(kt0 + 1, ra1, rw1);
        __syncthreads();
        for (int kt = kt0; kt < kt1; kt += 2) {
            // even step: tile kt in buffer 0; set 0 is free, set 1 holds kt + 1
            if (kt + 2 < kt1) fetch(kt + 2, ra0, rw0);
            compute(0);
            if (kt + 1 >= kt1) break;
            stash(1, ra1, rw1);
            __syncthreads();
            // odd step: tile kt + 1 in buffer 1; set 1 is free, set 0 holds kt + 2
            if (kt + 3 < kt1) fetch(kt + 3, ra1, rw1);
            compute(1);
            if (kt + 2 >= kt1) break;
            stash(0, ra0, rw0);
            __syncthreads();
        }
    }
    // lane holds rows 16i + 4*(lane/16) + r, column lane%16 of the wave's 16 columns
    const int n = n0 + wave * 16 + r16;
    if (n >= N) return;
#pragma unroll
    for (int i = 0; i < FB_MT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + 16 * i + 4 * kq + r;
            if (m >= M) continue;
            if (g.splits > 1) g.ws[((long long)z * M + m) * N + n] = acc[i][r];
            else enc_epi(g, m, n, acc[i][r]);
        }
}

// split-K finish: sum the partials in split order, then the epilogue
__global__ void enc_gemm_reduce_kernel(const EncGemmArgs g) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)g.M * g.N) return;
    const int m = (int)(i / g.N), n = (int)(i - (long long)m * g.N);
    float v = 0.0f;
    for (int z = 0; z < g.splits; ++z) v += g.ws[(long long)z * g.M * g.N + i];
    enc_epi(g, m, n, v);
}

// one 256-thread workgroup per row: LayerNorm (w, b; mean then variance of the centred row) or
// RMSNorm (w); sums reduced per wave, then across the 4 waves in wave order through LDS
template <bool LN>
__global__ __launch_bounds__(256) void enc_norm_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                       const float *__restrict__ w, const float *__restrict__ b,
                                                       int rows, int H, float eps) {
    __shared__ float part[4];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *xr = x + (long long)row * H;
    auto block_sum = [&](float v) {
        v = wave_sum(v);
        __syncthreads();   // part[] free from the previous reduction
        if (lane == 0) part[wave] = v;
        __syncthreads();
        return ((part[0] + part[1]) + part[2]) + part[3];
    };
    // the row in registers: columns 4*tid + 1024*j .. + 3 (H % 4 == 0, H <= 2048)
    float4 v[2];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int c = 4 * tid + 1024 * j;
        v[j] = c < H ? *(const float4 *)(xr + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        s += LN ? (v[j].x + v[j].y) + (v[j].z + v[j].w)
                : (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
    }
    s = block_sum(s);
    float mean = 0.0f, inv;
    if (LN) {
        mean = s / (float)H;
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; ++j)
            if (4 * tid + 1024 * j < H) {
                const float d0 = v[j].x - mean, d1 = v[j].y - mean, d2 = v[j].z - mean, d3 = v[j].w - mean;
                q += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
            }
        q = block_sum(q);
        inv = 1.0f / sqrtf(q / (float)H + eps);
    } else {
        inv = 1.0f / sqrtf(s / (float)H + eps);
    }
    float *yr = y + (long long)row * H;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int c = 4 * tid + 1024 * j;
        if (c >= H) continue;
        const float4 wv = *(const float4 *)(w + c);
        float4 o;
        if (LN) {
            const float4 bv = *(const float4 *)(b + c);
            o = make_float4((v[j].x - mean) * inv * wv.x + bv.x, (v[j].y - mean) * inv * wv.y + bv.y,
                            (v[j].z - mean) * inv * wv.z + bv.z, (v[j].w - mean) * inv * wv.w + bv.w);
        } else {
            o = make_float4(v[j].x * inv * wv.x, v[j].y * inv * wv.y, v[j].z * inv * wv.z, v[j].w * inv * wv.w);
        }
        *(float4 *)(yr + c) = o;
    }
}

constexpr int EA_Q = 16;      // queries per workgroup
constexpr int EA_SMAX = 128;  // longest context
constexpr int EA_HD = 64;
constexpr int EA_KP = EA_HD + 4;   // K row pitch (floats): 16-byte rows, 16 consecutive keys in distinct banks
constexpr int EA_PP = EA_SMAX + 1;

// one workgroup per (16 queries, head): scores, mask / bias, softmax and P·V in f32. Thread t
// serves query t / 16: its scores are keys t % 16 + 16j (query row in registers, K rows read as
// float4), its outputs columns 4 (t % 16) .. + 3 (V rows read as float4).
__global__ __launch_bounds__(256) void enc_attn_kernel(const EncAttnArgs a) {
    __shared__ __attribute__((aligned(16))) float Ks[EA_SMAX * EA_KP];
    __shared__ __attribute__((aligned(16))) float Vs[EA_SMAX * EA_HD];
    __shared__ __attribute__((aligned(16))) float Qs[EA_Q * EA_HD];
    __shared__ float P[EA_Q * EA_PP];
    const int tid = threadIdx.x, h = blockIdx.y, q0 = blockIdx.x * EA_Q, S = a.S;
    for (int e = tid; e < S * (EA_HD / 4); e += 256) {
        const int k = e >> 4, d = (e & 15) * 4;
        const float *row = a.qkv + (long long)k * a.ld + h * EA_HD + d;
        *(float4 *)&Ks[k * EA_KP + d] = *(const float4 *)(row + a.k_off);
        *(float4 *)&Vs[k * EA_HD + d] = *(const float4 *)(row + a.v_off);
    }
    {
        const int q = tid >> 4, d = (tid & 15) * 4;
        *(float4 *)&Qs[q * EA_HD + d] = q0 + q < S
            ? *(const float4 *)(a.qkv + (long long)(q0 + q) * a.ld + a.q_off + h * EA_HD + d)
            : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    const int q = tid >> 4, t16 = tid & 15, qg = q0 + q;
    {
        float4 qv[EA_HD / 4];
#pragma unroll
        for (int i = 0; i < EA_HD / 4; ++i) qv[i] = *(const float4 *)&Qs[q * EA_HD + 4 * i];
        for (int k = t16; k < S; k += 16) {
            const float *kr = &Ks[k * EA_KP];
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < EA_HD / 4; ++i) {
                const float4 kv = *(const float4 *)(kr + 4 * i);
                s += qv[i].x * kv.x;
                s += qv[i].y * kv.y;
                s += qv[i].z * kv.z;
                s += qv[i].w * kv.w;
            }
            s *= a.scale;
            if (a.mode == 1) {   // T5: padded keys masked, else the head's bias for the bucket of (q, k)
                if (a.pad && a.pad[k] == 0) s = -INFINITY;
                else if (qg < S) s += a.rel[a.bucket[qg * S + k] * a.nh + h];
            } else if (a.mode == 2) {   // CLIP: causal, and nothing past the end-of-text token
                if (!(k <= qg && k <= a.eot)) s = -INFINITY;
            }
            P[q * EA_PP + k] = s;
        }
    }
    __syncthreads();
    {   // softmax: wave w takes rows w, w+4, w+8, w+12
        const int lane = tid & 63, wave = tid >> 6;
        for (int r = wave; r < EA_Q; r += 4) {
            float *pr = P + r * EA_PP;
            float mx = -INFINITY;
            for (int k = lane; k < S; k += 64) mx = fmaxf(mx, pr[k]);
            mx = wave_max(mx);
            float sum = 0.0f;
            for (int k = lane; k < S; k += 64) {
                const float e = expf(pr[k] - mx);
                pr[k] = e;
                sum += e;
            }
            sum = wave_sum(sum);
            const float inv = 1.0f / sum;
            for (int k = lane; k < S; k += 64) pr[k] *= inv;
        }
    }
    __syncthreads();
    if (qg >= S) return;
    const int d = t16 * 4;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = 0; k < S; ++k) {
        const float pk = P[q * EA_PP + k];
        const float4 v = *(const float4 *)&Vs[k * EA_HD + d];
        o.x += pk * v.x;
        o.y += pk * v.y;
        o.z += pk * v.z;
        o.w += pk * v.w;
    }
    *(float4 *)(a.out + (long long)qg * a.ldo + h * EA_HD + d) = o;
}

// y[r][c] = gelu_tanh(u[r][c]) * u[r][F + c] (tanh form, argument clamped to +-10: shaders/ops_conv.metal:15-24)
__global__ void geglu_rows_kernel(const float *__restrict__ u, float *__restrict__ y, int rows, int F) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)rows * F) return;
    const long long r = i / F;
    const int c = (int)(i - r * F);
    const float v = u[r * 2 * F + c], g = u[r * 2 * F + F + c];
    const float t = 0.7978845608f * (v + 0.044715f * v * v * v);
    y[i] = 0.5f * v * (1.0f + tanhf(fminf(fmaxf(t, -10.0f), 10.0f))) * g;
}

// x[s][c] = tok[ids[s]][c] (+ pos[s][c])
__global__ void embed_rows_kernel(const int32_t *__restrict__ ids, const float *__restrict__ tok,
                                  const float *__restrict__ pos, float *__restrict__ x, int S, int H) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)S * H) return;
    const int s = (int)(i / H), c = (int)(i - (long long)s * H);
    float v = tok[(long long)ids[s] * H + c];
    if (pos) v += pos[i];
    x[i] = v;
}

} // namespace

int launch_gemm_f32(const EncGemmArgs &gin, hipStream_t st) {
    EncGemmArgs g = gin;
    TSN_REQUIRE(g.A && g.W && g.Y && g.M > 0 && g.N > 0 && g.K > 0, "gemm_f32: null operand or empty shape");
    TSN_REQUIRE(g.K % 4 == 0 && g.lda % 4 == 0 && g.ldw % 4 == 0 && g.lda >= g.K && g.ldw >= g.K && g.ldy >= g.N,
                "gemm_f32: K and row strides multiples of 4, strides covering the rows");
    TSN_REQUIRE((((uintptr_t)g.A) & 15) == 0 && (((uintptr_t)g.W) & 15) == 0, "gemm_f32: 16-byte aligned A and W");
    TSN_REQUIRE(g.act == 0 || g.act == 1, "gemm_f32: activation 0 (none) or 1 (quick GELU)");
    // The f32 MFMA bounds these GEMMs, so the K split balances K tiles per CU: estimated time in K
    // tiles = rounds of 256 workgroups x K tiles per split, plus the partial sums written and read
    // (about 8 MB per K-tile time) and a reduce launch. Splits are powers of two with at least 2 K
    // tiles each, and the workspace must hold the partials.
    const int tiles = ((g.N + FB_N - 1) / FB_N) * ((g.M + FB_M - 1) / FB_M);
    const int nkt = (g.K + FB_K - 1) / FB_K;
    int splits = 1;
    double best = (double)((tiles + 255) / 256) * nkt;
    for (int s = 2; g.ws && nkt / s >= 2 && (size_t)s * g.M * g.N * sizeof(float) <= g.ws_bytes; s *= 2) {
        const double cost = (double)((tiles * s + 255) / 256) * ((nkt + s - 1) / s) + 1.0 +
                            2.0 * s * g.M * (double)g.N * sizeof(float) / 8e6;
        if (cost < best) {
            best = cost;
            splits = s;
        }
    }
    g.kps = (nkt + splits - 1) / splits;
    g.splits = (nkt + g.kps - 1) / g.kps;
    TSN_LAUNCH(gemm_f32_kernel, dim3((g.N + FB_N - 1) / FB_N, (g.M + FB_M - 1) / FB_M, g.splits), dim3(256), 0, st, g);
    TSN_HIP_CHECK(hipGetLastError());
    if (g.splits > 1) {
        const long long n = (long long)g.M * g.N;
        TSN_LAUNCH(enc_gemm_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g);
        TSN_HIP_CHECK(hipGetLastError());
    }
    return TSN_OK;
}

int launch_enc_norm(const float *x, float *y, const float *w, const float *b, int rows, int H, float eps, bool ln,
                    hipStream_t st) {
    TSN_REQUIRE(x && y && w && rows > 0 && H > 0 && (!ln || b), "enc_norm: arguments");
    TSN_REQUIRE(H % 4 == 0 && H <= 2048 && ((((uintptr_t)x) | ((uintptr_t)y) | ((uintptr_t)w) | ((uintptr_t)b)) & 15) == 0,
                "enc_norm: rows of at most 2048 floats, a multiple of 4, 16-byte aligned");
    if (ln) TSN_LAUNCH(enc_norm_kernel<true>, dim3(rows), dim3(256), 0, st, x, y, w, b, rows, H, eps);
    else TSN_LAUNCH(enc_norm_kernel<false>, dim3(rows), dim3(256), 0, st, x, y, w, b, rows, H, eps);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_enc_attention(const EncAttnArgs &a, hipStream_t st) {
    TSN_REQUIRE(a.qkv && a.out && a.S > 0 && a.S <= EA_SMAX && a.nh > 0 && a.hd == EA_HD,
                "enc_attention: context 1..128, head width 64");
    TSN_REQUIRE(a.mode == 0 || a.mode == 2 || (a.mode == 1 && a.rel && a.bucket), "enc_attention: mode and tables");
    TSN_REQUIRE((((uintptr_t)a.qkv | (uintptr_t)a.out) & 15) == 0 && a.ld % 4 == 0 && a.ldo % 4 == 0 &&
                    a.q_off % 4 == 0 && a.k_off % 4 == 0 && a.v_off % 4 == 0,
                "enc_attention: 16-byte aligned rows (qkv, out, strides and offsets multiples of 4 floats)");
    TSN_LAUNCH(enc_attn_kernel, dim3((a.S + EA_Q - 1) / EA_Q, a.nh), dim3(256), 0, st, a);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_geglu_rows(const float *u, float *y, int rows, int F, hipStream_t st) {
    TSN_REQUIRE(u && y && rows > 0 && F > 0, "geglu: arguments");
    const long long n = (long long)rows * F;
    TSN_LAUNCH(geglu_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, u, y, rows, F);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_embed_rows(const int32_t *ids, const float *tok, const float *pos, float *x, int S, int H, hipStream_t st) {
    TSN_REQUIRE(ids && tok && x && S > 0 && H > 0, "embed: arguments");
    const long long n = (long long)S * H;
    TSN_LAUNCH(embed_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, ids, tok, pos, x, S, H);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

} // namespace tsn
