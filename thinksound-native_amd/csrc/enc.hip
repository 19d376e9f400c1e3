// enc.hip — kernels of the text encoders (src/clip.cpp, src/t5.cpp): f32 GEMM on the f32 MFMA,
// LayerNorm with weight and bias, RMSNorm with weight, attention over one short context with the
// CLIP causal/EOT mask or the T5 bucketed relative bias and padding mask, GEGLU, and the token
// (+ position) embedding gather. Everything stays f32: T5's activations leave the f16 range.
#include <hip/hip_runtime.h>

#include "kernels.h"

namespace tsn {

namespace {

typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int FB_M = 32, FB_N = 64, FB_K = 32, FB_LD = FB_K + 1;

// Y = act(A·Wᵀ + bias) or Y += A·Wᵀ + bias. 4 waves; wave w owns columns 16w..16w+15 of a 32x64
// tile (two 16x16 blocks of v_mfma_f32_16x16x4_f32 per 4-wide K slice). A and W tiles are staged
// through LDS, the next K tile is held in registers while the current one is multiplied.
__global__ __launch_bounds__(256) void gemm_f32_kernel(const EncGemmArgs g) {
    __shared__ float As[2][FB_M * FB_LD];
    __shared__ float Ws[2][FB_N * FB_LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * FB_N, m0 = blockIdx.y * FB_M;
    const int M = g.M, N = g.N, K = g.K;
    // loader: A row tid/8 (32 rows), W rows tid/8 and 32 + tid/8; 4 floats at column (tid%8)*4
    const int lr = tid >> 3, lc = (tid & 7) * 4;
    const bool a_ok = m0 + lr < M, w0_ok = n0 + lr < N, w1_ok = n0 + 32 + lr < N;
    const float *ap = g.A + (long long)(a_ok ? m0 + lr : 0) * g.lda + lc;
    const float *wp0 = g.W + (long long)(w0_ok ? n0 + lr : 0) * g.ldw + lc;
    const float *wp1 = g.W + (long long)(w1_ok ? n0 + 32 + lr : 0) * g.ldw + lc;
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 ra, rw0, rw1;
    auto fetch = [&](int k0) {
        ra = a_ok ? *(const float4 *)(ap + k0) : z4;
        rw0 = w0_ok ? *(const float4 *)(wp0 + k0) : z4;
        rw1 = w1_ok ? *(const float4 *)(wp1 + k0) : z4;
    };
    auto stash = [&](int b) {
        float *a = &As[b][lr * FB_LD + lc];
        a[0] = ra.x; a[1] = ra.y; a[2] = ra.z; a[3] = ra.w;
        float *w = &Ws[b][lr * FB_LD + lc];
        w[0] = rw0.x; w[1] = rw0.y; w[2] = rw0.z; w[3] = rw0.w;
        float *w1 = &Ws[b][(32 + lr) * FB_LD + lc];
        w1[0] = rw1.x; w1[1] = rw1.y; w1[2] = rw1.z; w1[3] = rw1.w;
    };
    floatx4_t acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    const int r16 = lane & 15, kq = lane >> 4;   // operand lane: row / column r16, k offset kq
    const int nk = K / FB_K;
    fetch(0);
    stash(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int b = kt & 1;
        if (kt + 1 < nk) fetch((kt + 1) * FB_K);
        const float *as = As[b], *ws = Ws[b];
#pragma unroll
        for (int kk = 0; kk < FB_K; kk += 4) {
            const float bv = ws[(wave * 16 + r16) * FB_LD + kk + kq];
            const float a0 = as[r16 * FB_LD + kk + kq];
            const float a1 = as[(16 + r16) * FB_LD + kk + kq];
            acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, bv, acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, bv, acc[1], 0, 0, 0);
        }
        if (kt + 1 < nk) {
            stash(b ^ 1);
            __syncthreads();
        }
    }
    // lane holds rows 16i + 4*(lane/16) + r, column lane%16 of the wave's 16 columns
    const int n = n0 + wave * 16 + r16;
    if (n >= N) return;
    const float bn = g.bias ? g.bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + 16 * i + 4 * kq + r;
            if (m >= M) continue;
            float v = acc[i][r] + bn;
            float *y = g.Y + (long long)m * g.ldy + n;
            if (g.resid) {
                *y = *y + v;
            } else {
                if (g.act == 1) v = v / (1.0f + expf(-1.702f * v));   // quick GELU (shaders/ops_conv.metal:25-29)
                *y = v;
            }
        }
}

// one wave per row: LayerNorm (w, b; mean then variance of the centred row) or RMSNorm (w)
template <bool LN>
__global__ __launch_bounds__(256) void enc_norm_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                       const float *__restrict__ w, const float *__restrict__ b,
                                                       int rows, int H, float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + (long long)row * H;
    float s = 0.0f;
    for (int c = lane; c < H; c += 64) s += LN ? xr[c] : xr[c] * xr[c];
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    float mean = 0.0f, inv;
    if (LN) {
        mean = s / (float)H;
        float v = 0.0f;
        for (int c = lane; c < H; c += 64) {
            const float d = xr[c] - mean;
            v += d * d;
        }
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
        inv = 1.0f / sqrtf(v / (float)H + eps);
    } else {
        inv = 1.0f / sqrtf(s / (float)H + eps);
    }
    float *yr = y + (long long)row * H;
    for (int c = lane; c < H; c += 64) yr[c] = LN ? (xr[c] - mean) * inv * w[c] + b[c] : xr[c] * inv * w[c];
}

constexpr int EA_Q = 16;      // queries per workgroup
constexpr int EA_SMAX = 128;  // longest context
constexpr int EA_HD = 64;

// one workgroup per (16 queries, head): scores, mask / bias, softmax and P·V in f32
__global__ __launch_bounds__(256) void enc_attn_kernel(const EncAttnArgs a) {
    __shared__ float Ks[EA_SMAX * (EA_HD + 1)];
    __shared__ float Vs[EA_SMAX * EA_HD];
    __shared__ float Qs[EA_Q * EA_HD];
    __shared__ float P[EA_Q * (EA_SMAX + 1)];
    const int tid = threadIdx.x, h = blockIdx.y, q0 = blockIdx.x * EA_Q, S = a.S;
    for (int e = tid; e < S * EA_HD; e += 256) {
        const int k = e >> 6, d = e & 63;
        const float *row = a.qkv + (long long)k * a.ld + h * EA_HD + d;
        Ks[k * (EA_HD + 1) + d] = row[a.k_off];
        Vs[k * EA_HD + d] = row[a.v_off];
    }
    for (int e = tid; e < EA_Q * EA_HD; e += 256) {
        const int q = e >> 6, d = e & 63;
        Qs[e] = q0 + q < S ? a.qkv[(long long)(q0 + q) * a.ld + a.q_off + h * EA_HD + d] : 0.0f;
    }
    __syncthreads();
    for (int e = tid; e < EA_Q * S; e += 256) {
        const int q = e / S, k = e - q * S, qg = q0 + q;
        float s = 0.0f;
        for (int d = 0; d < EA_HD; ++d) s += Qs[q * EA_HD + d] * Ks[k * (EA_HD + 1) + d];
        s *= a.scale;
        if (a.mode == 1) {   // T5: padded keys masked, else the head's bias for the bucket of (q, k)
            if (a.pad && a.pad[k] == 0) s = -INFINITY;
            else if (qg < S) s += a.rel[a.bucket[qg * S + k] * a.nh + h];
        } else if (a.mode == 2) {   // CLIP: causal, and nothing past the end-of-text token
            if (!(k <= qg && k <= a.eot)) s = -INFINITY;
        }
        P[q * (EA_SMAX + 1) + k] = s;
    }
    __syncthreads();
    {   // softmax: wave w takes rows w, w+4, w+8, w+12
        const int lane = tid & 63, wave = tid >> 6;
        for (int q = wave; q < EA_Q; q += 4) {
            float *pr = P + q * (EA_SMAX + 1);
            float mx = -INFINITY;
            for (int k = lane; k < S; k += 64) mx = fmaxf(mx, pr[k]);
            for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
            float sum = 0.0f;
            for (int k = lane; k < S; k += 64) {
                const float e = expf(pr[k] - mx);
                pr[k] = e;
                sum += e;
            }
            for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
            const float inv = 1.0f / sum;
            for (int k = lane; k < S; k += 64) pr[k] *= inv;
        }
    }
    __syncthreads();
    for (int e = tid; e < EA_Q * EA_HD; e += 256) {
        const int q = e >> 6, d = e & 63;
        if (q0 + q >= S) continue;
        float o = 0.0f;
        for (int k = 0; k < S; ++k) o += P[q * (EA_SMAX + 1) + k] * Vs[k * EA_HD + d];
        a.out[(long long)(q0 + q) * a.ldo + h * EA_HD + d] = o;
    }
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

int launch_gemm_f32(const EncGemmArgs &g, hipStream_t st) {
    TSN_REQUIRE(g.A && g.W && g.Y && g.M > 0 && g.N > 0 && g.K > 0, "gemm_f32: null operand or empty shape");
    TSN_REQUIRE(g.K % FB_K == 0 && g.lda % 4 == 0 && g.ldw % 4 == 0 && g.lda >= g.K && g.ldw >= g.K && g.ldy >= g.N,
                "gemm_f32: K a multiple of 32, row strides multiples of 4 covering the rows");
    TSN_REQUIRE((((uintptr_t)g.A) & 15) == 0 && (((uintptr_t)g.W) & 15) == 0, "gemm_f32: 16-byte aligned A and W");
    TSN_REQUIRE(g.act == 0 || g.act == 1, "gemm_f32: activation 0 (none) or 1 (quick GELU)");
    TSN_LAUNCH(gemm_f32_kernel, dim3((g.N + FB_N - 1) / FB_N, (g.M + FB_M - 1) / FB_M), dim3(256), 0, st, g);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_enc_norm(const float *x, float *y, const float *w, const float *b, int rows, int H, float eps, bool ln,
                    hipStream_t st) {
    TSN_REQUIRE(x && y && w && rows > 0 && H > 0 && (!ln || b), "enc_norm: arguments");
    if (ln) TSN_LAUNCH(enc_norm_kernel<true>, dim3((rows + 3) / 4), dim3(256), 0, st, x, y, w, b, rows, H, eps);
    else TSN_LAUNCH(enc_norm_kernel<false>, dim3((rows + 3) / 4), dim3(256), 0, st, x, y, w, b, rows, H, eps);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_enc_attention(const EncAttnArgs &a, hipStream_t st) {
    TSN_REQUIRE(a.qkv && a.out && a.S > 0 && a.S <= EA_SMAX && a.nh > 0 && a.hd == EA_HD,
                "enc_attention: context 1..128, head width 64");
    TSN_REQUIRE(a.mode == 0 || a.mode == 2 || (a.mode == 1 && a.rel && a.bucket), "enc_attention: mode and tables");
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
