// netops.hip — kernels behind the net.h launcher surface (src/net.h:18-51) that the model graphs
// do not use: conv weight preparation into zero-padded f16 rows, the gathered operand of strided,
// dilated and transposed convs, a direct f32 conv for narrow outputs, and the remaining
// reference launchers (ln_plain, geglu, gelu_quick, qkv_split3).
//
// Operand formats for f32-accurate products on f16 MFMA (x f32 in every case):
//   f16 weights: x as an f16 hi|lo pair, hi = f16(x), lo = f16(x - hi), against [W | W];
//   f32 weights: x as three parts [hi | lo | hi] against [W_hi | W_hi | W_lo]
//   (hi·W_hi + lo·W_hi + hi·W_lo; the dropped lo·W_lo term is below 2^-22 relative).
#include "kernels.h"
#include "dpp.h"

namespace tsn {

namespace {

// source row of conv tap k for output row t (shaders/ops_conv.metal:226-236,266-283, im2col): strided and
// dilated conv ti = t*stride - pad + k*dil; transposed conv over the zero-stuffed input
// ui = t - pad + k, a tap only where ui >= 0 is a multiple of stride (ti = ui / stride). -1: zero.
__device__ inline int conv_src_row(int t, int k, const ConvGeom &g) {
    int ti;
    if (g.convt) {
        const int ui = t - g.pad + k;
        if (ui < 0 || ui % g.stride != 0) return -1;
        ti = ui / g.stride;
    } else {
        ti = t * g.stride - g.pad + k * g.dil;
    }
    return ti >= 0 && ti < g.T ? ti : -1;
}

// Wp [OC][Kp] f16 from W [OC][IC][K]: tap-major columns, zero from the data's end to Kp.
// parts 1 (f16 or bf16 source): column k*IC + ic = w, bf16 converted with the reference upload's
// rounding; parts 3 (f32 source): tap k holds [hi | hi | lo] of its IC channels at k*3IC.
__global__ void conv_prep_kernel(const void *src, int sdt, half_t *dst, int OC, int IC, int K, int parts, int Kp) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)OC * Kp) return;
    const int oc = (int)(i / Kp), j = (int)(i - (long long)oc * Kp);
    half_t out = (half_t)0.0f;
    if (j < K * IC * parts) {
        const int w_ic = IC * parts;
        const int k = j / w_ic, q = j - k * w_ic, part = q / IC, ic = q - part * IC;
        const long long si = ((long long)oc * IC + ic) * K + k;
        if (sdt == DT_F16) {
            out = ((const half_t *)src)[si];
        } else if (sdt == DT_BF16) {
            out = f32_to_f16_upload(bf16_to_f32(((const uint16_t *)src)[si]));
        } else {
            const float w = ((const float *)src)[si];
            const half_t hi = (half_t)w;
            out = part < 2 ? hi : (half_t)(w - (float)hi);
        }
    }
    dst[i] = out;
}

// Gathered conv operand rows t0 .. t0 + rows - 1 (the im2col of src/net.mm:36-48, in the layout of
// the prepared weight). parts 1: row [2*Kp] = [hi (Kp) | lo (Kp)], column k*IC + ic of each half;
// parts 3: row [Kp], tap k = [hi | lo | hi] of its IC channels at k*3IC. Zero past the data.
__global__ void conv_gather_kernel(const float *x, ConvGeom g, int t0, int rows, int parts, int Kp, half_t *out) {
    const int width = parts == 1 ? 2 * Kp : Kp;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)rows * width) return;
    const int r = (int)(i / width), c = (int)(i - (long long)r * width);
    const int j = parts == 1 ? (c < Kp ? c : c - Kp) : c;
    half_t out_v = (half_t)0.0f;
    if (j < g.K * g.IC * parts) {
        const int w_ic = g.IC * parts;
        const int k = j / w_ic, q = j - k * w_ic, part = q / g.IC, ic = q - part * g.IC;
        const int ti = conv_src_row(t0 + r, k, g);
        const float v = ti >= 0 ? x[(long long)ti * g.ldx + ic] : 0.0f;
        const half_t hi = (half_t)v;
        const bool lo = parts == 1 ? c >= Kp : part == 1;
        out_v = lo ? (half_t)(v - (float)hi) : hi;
    }
    out[i] = out_v;
}

// Direct conv for outputs too narrow for a GEMM tile: one thread per (t, oc), taps then channels in
// order, f32 FMA. w = Wp[oc][k*IC*parts + ic] (+ the lo part Wp[... + 2IC + ic] for parts 3).
__global__ void conv_direct_kernel(const float *x, ConvGeom g, const half_t *Wp, int parts, int Kp, const float *bias,
                                   float *y) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)g.OL * g.OC) return;
    const int t = (int)(i / g.OC), oc = (int)(i - (long long)t * g.OC);
    const half_t *wr = Wp + (long long)oc * Kp;
    float acc = bias ? bias[oc] : 0.0f;
    for (int k = 0; k < g.K; ++k) {
        const int ti = conv_src_row(t, k, g);
        if (ti < 0) continue;
        const float *xr = x + (long long)ti * g.ldx;
        const half_t *wk = wr + (long long)k * g.IC * parts;
        for (int ic = 0; ic < g.IC; ++ic) {
            const float w = parts == 1 ? (float)wk[ic] : (float)wk[ic] + (float)wk[2 * g.IC + ic];
            acc = fmaf(xr[ic], w, acc);
        }
    }
    y[(long long)t * g.OC + oc] = acc;
}

// LayerNorm without affine (shaders/ops_conv.metal:77-89): one wave per row, two passes over the row
// (mean, then the biased variance of the centred row), fixed butterfly order
__global__ __launch_bounds__(256) void ln_plain_kernel(const float *x, float *y, int S, int H, float eps) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + wave;
    if (row >= S) return;
    const float *r = x + (long long)row * H;
    float s = 0.0f;
    for (int c = lane; c < H; c += 64) s += r[c];
    s = wave_sum(s);
    const float mean = s / (float)H;
    float q = 0.0f;
    for (int c = lane; c < H; c += 64) {
        const float d = r[c] - mean;
        q += d * d;
    }
    q = wave_sum(q);
    const float inv = 1.0f / sqrtf(q / (float)H + eps);
    float *o = y + (long long)row * H;
    for (int c = lane; c < H; c += 64) o[c] = (r[c] - mean) * inv;
}

// y = gelu_tanh(a) * b with the tanh argument clamped to [-10, 10] (shaders/ops_conv.metal:15-24)
__global__ void geglu_kernel(const float *a, const float *b, float *y, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = a[i];
    const float arg = 0.7978845608f * (v + 0.044715f * v * v * v);
    y[i] = 0.5f * v * (1.0f + tanhf(fminf(fmaxf(arg, -10.0f), 10.0f))) * b[i];
}

// x = x * sigmoid(1.702 x) in place (shaders/ops_conv.metal:25-29)
__global__ void gelu_quick_kernel(float *x, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    x[i] = v / (1.0f + expf(-1.702f * v));
}

// element-interleaved qkv rows (column 3c + j) -> block q|k|v rows at row_off (shaders/ops_conv.metal:60-74)
__global__ void qkv_split3_kernel(const float *src, float *dst, int rows, int H, int row_off) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)rows * H) return;
    const int r = (int)(i / H), c = (int)(i - (long long)r * H);
    const float *s = src + (long long)r * 3 * H + 3 * c;
    float *d = dst + (long long)(row_off + r) * 3 * H + c;
    d[0] = s[0];
    d[H] = s[1];
    d[2 * H] = s[2];
}

inline unsigned blocks_for(long long n, unsigned t = 256) { return (unsigned)((n + t - 1) / t); }

} // namespace

int conv_prep_cols(int sdt, int IC, int K) {
    const long long c = (long long)K * IC * (sdt == DT_F32 ? 3 : 1);
    return (int)((c + 63) / 64 * 64);
}

int launch_conv_prepare(const void *W, int sdt, half_t *Wp, int OC, int IC, int K, hipStream_t st) {
    TSN_REQUIRE(W && Wp && OC > 0 && IC > 0 && K > 0, "conv_prepare: arguments");
    TSN_REQUIRE(sdt == DT_F16 || sdt == DT_BF16 || sdt == DT_F32, "conv_prepare: weight dtype f16, bf16 or f32");
    TSN_REQUIRE((long long)K * IC * 3 < (1LL << 30), "conv_prepare: K*IC too large");
    const int Kp = conv_prep_cols(sdt, IC, K);
    TSN_LAUNCH(conv_prep_kernel, dim3(blocks_for((long long)OC * Kp)), dim3(256), 0, st, W, sdt, Wp, OC, IC, K,
               sdt == DT_F32 ? 3 : 1, Kp);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_conv_gather(const float *x, const ConvGeom &g, int t0, int rows, int parts, int Kp, half_t *out,
                       hipStream_t st) {
    TSN_REQUIRE(x && out && rows > 0 && t0 >= 0 && t0 + rows <= g.OL && (parts == 1 || parts == 3) &&
                    Kp >= g.K * g.IC * parts,
                "conv_gather: arguments");
    const long long n = (long long)rows * (parts == 1 ? 2 * Kp : Kp);
    TSN_LAUNCH(conv_gather_kernel, dim3(blocks_for(n)), dim3(256), 0, st, x, g, t0, rows, parts, Kp, out);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_conv_direct(const float *x, const ConvGeom &g, const half_t *Wp, int parts, int Kp, const float *bias,
                       float *y, hipStream_t st) {
    TSN_REQUIRE(x && Wp && y && g.OL > 0 && g.OC > 0 && (parts == 1 || parts == 3), "conv_direct: arguments");
    TSN_LAUNCH(conv_direct_kernel, dim3(blocks_for((long long)g.OL * g.OC)), dim3(256), 0, st, x, g, Wp, parts, Kp,
               bias, y);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_ln_plain(const float *x, float *y, int S, int H, float eps, hipStream_t st) {
    TSN_REQUIRE(x && y && S > 0 && H > 0, "ln_plain: arguments");
    TSN_LAUNCH(ln_plain_kernel, dim3((S + 3) / 4), dim3(256), 0, st, x, y, S, H, eps);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_geglu(const float *a, const float *b, float *y, size_t n, hipStream_t st) {
    TSN_REQUIRE((a && b && y) || n == 0, "geglu: null");
    if (n == 0) return TSN_OK;
    TSN_LAUNCH(geglu_kernel, dim3(blocks_for((long long)n)), dim3(256), 0, st, a, b, y, n);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_gelu_quick(float *x, size_t n, hipStream_t st) {
    TSN_REQUIRE(x || n == 0, "gelu_quick: null");
    if (n == 0) return TSN_OK;
    TSN_LAUNCH(gelu_quick_kernel, dim3(blocks_for((long long)n)), dim3(256), 0, st, x, n);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_qkv_split3(const float *src, float *dst, int rows, int H, int row_off, hipStream_t st) {
    TSN_REQUIRE(src && dst && rows > 0 && H > 0 && row_off >= 0, "qkv_split3: arguments");
    TSN_LAUNCH(qkv_split3_kernel, dim3(blocks_for((long long)rows * H)), dim3(256), 0, st, src, dst, rows, H,
               row_off);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

} // namespace tsn
