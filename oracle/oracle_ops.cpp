// oracle_ops.cpp — single-op CPU f32 restatements (test infrastructure only; see oracle.h).
//
// Determinism: every output element is reduced in one fixed sequential order (k = 0..K-1,
// fused multiply-add, then the bias), whatever the blocking and the OpenMP thread count.
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <vector>

typedef float v8f __attribute__((vector_size(32)));

static inline v8f v8_load(const float *p) { v8f v; memcpy(&v, p, sizeof v); return v; }
static inline void v8_store(float *p, v8f v) { memcpy(p, &v, sizeof v); }
static inline v8f v8_bcast(float x) { return (v8f){x, x, x, x, x, x, x, x}; }

extern "C" int orc_num_threads(void) { return omp_get_max_threads(); }

// Y = X·Wᵀ (+b). shaders/gemm_mpp.metal:18-48 computes the same contract with f32 accumulation
// (bias added after the product, :39-46); src/net.mm:14-23 supplies the ld defaults.
// Blocking: tasks of 64 output rows x 64 output columns; W is packed k-major per 256-wide k
// chunk so the inner loop vectorises over output columns. Each element's accumulator walks k in
// increasing order, so the blocking does not change any result.
extern "C" void orc_gemm(const float *W, const float *X, float *Y, const float *bias,
                         int M, int N, int K, int ldx, int ldw, int ldy) {
    if (M <= 0 || N <= 0) return;
    const int NB = 64, MB = 64, KC = 256;
    const int tn_count = (N + NB - 1) / NB, tm_count = (M + MB - 1) / MB;
#pragma omp parallel
    {
        std::vector<float> wp((size_t)KC * NB);
        std::vector<float> acc((size_t)MB * NB);
#pragma omp for collapse(2) schedule(dynamic)
        for (int tn = 0; tn < tn_count; ++tn) {
            for (int tm = 0; tm < tm_count; ++tm) {
                const int n0 = tn * NB, nb = std::min(NB, N - n0);
                const int m0 = tm * MB, mb = std::min(MB, M - m0);
                std::fill(acc.begin(), acc.end(), 0.0f);
                for (int k0 = 0; k0 < K; k0 += KC) {
                    const int kc = std::min(KC, K - k0);
                    for (int k = 0; k < kc; ++k)
                        for (int j = 0; j < NB; ++j)
                            wp[(size_t)k * NB + j] = j < nb ? W[(size_t)(n0 + j) * ldw + k0 + k] : 0.0f;
                    int m = 0;
                    for (; m + 2 <= mb; m += 2) {
                        const float *x0 = X + (size_t)(m0 + m) * ldx + k0;
                        const float *x1 = x0 + ldx;
                        for (int jg = 0; jg < NB; jg += 32) {
                            float *a0 = &acc[(size_t)m * NB + jg], *a1 = a0 + NB;
                            v8f c00 = v8_load(a0), c01 = v8_load(a0 + 8), c02 = v8_load(a0 + 16), c03 = v8_load(a0 + 24);
                            v8f c10 = v8_load(a1), c11 = v8_load(a1 + 8), c12 = v8_load(a1 + 16), c13 = v8_load(a1 + 24);
                            for (int k = 0; k < kc; ++k) {
                                const float *w = &wp[(size_t)k * NB + jg];
                                const v8f w0 = v8_load(w), w1 = v8_load(w + 8), w2 = v8_load(w + 16), w3 = v8_load(w + 24);
                                const v8f b0 = v8_bcast(x0[k]), b1 = v8_bcast(x1[k]);
                                c00 += b0 * w0; c01 += b0 * w1; c02 += b0 * w2; c03 += b0 * w3;
                                c10 += b1 * w0; c11 += b1 * w1; c12 += b1 * w2; c13 += b1 * w3;
                            }
                            v8_store(a0, c00); v8_store(a0 + 8, c01); v8_store(a0 + 16, c02); v8_store(a0 + 24, c03);
                            v8_store(a1, c10); v8_store(a1 + 8, c11); v8_store(a1 + 16, c12); v8_store(a1 + 24, c13);
                        }
                    }
                    for (; m < mb; ++m) {
                        const float *x0 = X + (size_t)(m0 + m) * ldx + k0;
                        for (int jg = 0; jg < NB; jg += 32) {
                            float *a0 = &acc[(size_t)m * NB + jg];
                            v8f c00 = v8_load(a0), c01 = v8_load(a0 + 8), c02 = v8_load(a0 + 16), c03 = v8_load(a0 + 24);
                            for (int k = 0; k < kc; ++k) {
                                const float *w = &wp[(size_t)k * NB + jg];
                                const v8f w0 = v8_load(w), w1 = v8_load(w + 8), w2 = v8_load(w + 16), w3 = v8_load(w + 24);
                                const v8f b0 = v8_bcast(x0[k]);
                                c00 += b0 * w0; c01 += b0 * w1; c02 += b0 * w2; c03 += b0 * w3;
                            }
                            v8_store(a0, c00); v8_store(a0 + 8, c01); v8_store(a0 + 16, c02); v8_store(a0 + 24, c03);
                        }
                    }
                }
                for (int m = 0; m < mb; ++m)
                    for (int j = 0; j < nb; ++j)
                        Y[(size_t)(m0 + m) * ldy + n0 + j] =
                            acc[(size_t)m * NB + j] + (bias ? bias[n0 + j] : 0.0f);
            }
        }
    }
}

// M = 1 GEMV: shaders/gemm_attn.metal:47-56 (bias first, then k = 0..K-1).
extern "C" void orc_gemv(const float *W, const float *x, float *y, const float *bias, int N, int K, int ldw) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) {
        const float *w = W + (size_t)n * ldw;
        float acc = bias ? bias[n] : 0.0f;
        for (int k = 0; k < K; ++k) acc += w[k] * x[k];
        y[n] = acc;
    }
}

// im2col (shaders/ops_conv.metal:262-283) then GEMM with W [OC][IC][K] read as W[OC, IC*K]
// (shaders/ops_conv.metal:262-264; src/net.mm:38-48). Forward conv only (no convT).
extern "C" void orc_conv1d(const float *W, const float *bias, const float *x, float *y,
                           int T, int OL, int IC, int OC, int K, int stride, int pad, int dil) {
    const size_t KC = (size_t)IC * K;
    std::vector<float> col((size_t)OL * KC);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < OL; ++t)
        for (int ic = 0; ic < IC; ++ic)
            for (int k = 0; k < K; ++k) {
                const int ti = t * stride - pad + k * dil;
                col[(size_t)t * KC + (size_t)ic * K + k] =
                    (ti >= 0 && ti < T) ? x[(size_t)ti * IC + ic] : 0.0f;
            }
    orc_gemm(W, col.data(), y, bias, OL, OC, (int)KC, (int)KC, (int)KC, OC);
}

// direct conv: shaders/ops_conv.metal:221-246 (loop ic outer, k inner, skip out-of-range taps)
extern "C" void orc_conv1d_direct(const float *W, const float *bias, const float *x, float *y,
                                  int T, int OL, int IC, int OC, int K, int stride, int pad, int dil) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < OL; ++t)
        for (int oc = 0; oc < OC; ++oc) {
            float acc = bias ? bias[oc] : 0.0f;
            for (int ic = 0; ic < IC; ++ic)
                for (int k = 0; k < K; ++k) {
                    const int ti = t * stride - pad + k * dil;
                    if (ti < 0 || ti >= T) continue;
                    acc += x[(size_t)ti * IC + ic] * W[((size_t)oc * IC + ic) * K + k];
                }
            y[(size_t)t * OC + oc] = acc;
        }
}

// shaders/ops_conv.metal:127-144: two-pass mean/variance (biased), inv = 1/sqrt(var+eps),
// y = (x-mean)*inv*(1+m[H+i]) + m[i] with m = mod + (per_row ? row*chunks*H : 0) + base.
extern "C" void orc_adaln_ln(const float *x, const float *mod, float *y, int rows, int H,
                             int per_row, int chunks, int base, float eps) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float *xr = x + (size_t)r * H;
        const float *m = mod + (per_row ? (size_t)r * chunks * H : 0) + base;
        float *o = y + (size_t)r * H;
        float mean = 0.0f, var = 0.0f;
        for (int i = 0; i < H; ++i) mean += xr[i];
        mean /= (float)H;
        for (int i = 0; i < H; ++i) { const float d = xr[i] - mean; var += d * d; }
        var /= (float)H;
        const float inv = 1.0f / sqrtf(var + eps);
        for (int i = 0; i < H; ++i) o[i] = (xr[i] - mean) * inv * (1.0f + m[H + i]) + m[i];
    }
}

// shaders/ops_conv.metal:146-154
extern "C" void orc_gate_add(const float *x, const float *f, const float *mod, float *y, int rows, int H,
                             int per_row, int chunks, int gate_idx) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float *m = mod + (per_row ? (size_t)r * chunks * H : 0) + (size_t)gate_idx * H;
        for (int c = 0; c < H; ++c) {
            const size_t i = (size_t)r * H + c;
            y[i] = x[i] + f[i] * m[c];
        }
    }
}

// shaders/ops_conv.metal:115-125
extern "C" void orc_rms_head(float *x, const float *w, int rows, int nh, int ld, int hd,
                             int col_off, int row_off, float eps) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < rows; ++r)
        for (int h = 0; h < nh; ++h) {
            float *p = x + (size_t)(row_off + r) * ld + col_off + (size_t)h * hd;
            float ss = 0.0f;
            for (int i = 0; i < hd; ++i) ss += p[i] * p[i];
            const float inv = 1.0f / sqrtf(ss / (float)hd + eps);
            for (int i = 0; i < hd; ++i) p[i] = p[i] * inv * w[i];
        }
}

// shaders/ops_conv.metal:156-169
extern "C" void orc_rope_pairs(float *x, const int32_t *pos, int rows, int nh, int ld, int hd,
                               int col_off, int row_off, float fscale, float base) {
    const int npair = hd / 2;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r)
        for (int h = 0; h < nh; ++h)
            for (int j = 0; j < npair; ++j) {
                const float inv = powf(base, -2.0f * (float)j / (float)hd);
                const float ang = (float)(pos ? pos[r] : r) * fscale * inv;
                const float cs = cosf(ang), sn = sinf(ang);
                float *p = x + (size_t)(row_off + r) * ld + col_off + (size_t)h * hd;
                const float x0 = p[2 * j], x1 = p[2 * j + 1];
                p[2 * j] = x0 * cs - x1 * sn;
                p[2 * j + 1] = x0 * sn + x1 * cs;
            }
}

// shaders/gemm_attn.metal:96-202 without bias/mask modes (the DiT passes bias_mode 0,
// src/dit_fwd.cpp:90): scores = scale*q·k, softmax_rows (:145-157), O = P·V (:159-202).
extern "C" void orc_attention(const float *qkv, float *out, int S, int nh, int hd, int ld, int ldo,
                              int q_off, int k_off, int v_off, int o_off, float scale) {
#pragma omp parallel
    {
        std::vector<float> row(S);
#pragma omp for collapse(2) schedule(static)
        for (int h = 0; h < nh; ++h)
            for (int q = 0; q < S; ++q) {
                const float *qp = qkv + (size_t)q * ld + q_off + (size_t)h * hd;
                float mx = -INFINITY;
                for (int k = 0; k < S; ++k) {
                    const float *kp = qkv + (size_t)k * ld + k_off + (size_t)h * hd;
                    float s = 0.0f;
                    for (int d = 0; d < hd; ++d) s += qp[d] * kp[d];
                    s *= scale;
                    row[k] = s;
                    mx = std::max(mx, s);
                }
                float sum = 0.0f;
                for (int k = 0; k < S; ++k) { row[k] = expf(row[k] - mx); sum += row[k]; }
                const float inv = 1.0f / sum;
                for (int k = 0; k < S; ++k) row[k] *= inv;
                float *op = out + (size_t)q * ldo + o_off + (size_t)h * hd;
                for (int d = 0; d < hd; ++d) {
                    float acc = 0.0f;
                    for (int k = 0; k < S; ++k) acc += row[k] * qkv[(size_t)k * ld + v_off + (size_t)h * hd + d];
                    op[d] = acc;
                }
            }
    }
}

// shaders/ops_conv.metal:9-13
extern "C" void orc_silu(float *x, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) x[i] = x[i] / (1.0f + expf(-x[i]));
}
// shaders/ops_conv.metal:36-42
extern "C" void orc_swiglu(const float *a, const float *b, float *y, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) y[i] = (a[i] / (1.0f + expf(-a[i]))) * b[i];
}
// shaders/ops_conv.metal:43-48
extern "C" void orc_add(const float *a, const float *b, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = a[i] + b[i];
}
// shaders/ops_conv.metal:50-57
extern "C" void orc_add_bcast_col(const float *x, const float *v, float *y, int S, int H) {
    for (size_t i = 0; i < (size_t)S * H; ++i) y[i] = x[i] + v[i % H];
}
// shaders/ops_conv.metal:193-201: v = fu + (fc - fu)*cfg; x += dt*v
extern "C" void orc_cfg_euler(const float *fc, const float *fu, float *x, size_t n, float cfg, float dt) {
    for (size_t i = 0; i < n; ++i) {
        const float v = fu[i] + (fc[i] - fu[i]) * cfg;
        x[i] += dt * v;
    }
}
// shaders/ops_conv.metal:15-24: y = 0.5 v (1 + tanh(clamp(0.7978845608 (v + 0.044715 v^3), -10, 10))) b
extern "C" void orc_geglu(const float *a, const float *b, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float v = a[i];
        const float arg = 0.7978845608f * (v + 0.044715f * v * v * v);
        y[i] = 0.5f * v * (1.0f + tanhf(fminf(fmaxf(arg, -10.0f), 10.0f))) * b[i];
    }
}
// shaders/ops_conv.metal:25-29: x = x / (1 + exp(-1.702 x))
extern "C" void orc_gelu_quick(float *x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = x[i] / (1.0f + expf(-1.702f * x[i]));
}
// shaders/ops_conv.metal:77-89: per row, mean then the biased variance of the centred row, no affine
extern "C" void orc_ln_plain(const float *x, float *y, int S, int H, float eps) {
    for (int r = 0; r < S; ++r) {
        const float *xr = x + (size_t)r * H;
        float mean = 0.0f, var = 0.0f;
        for (int i = 0; i < H; ++i) mean += xr[i];
        mean /= (float)H;
        for (int i = 0; i < H; ++i) { const float d = xr[i] - mean; var += d * d; }
        var /= (float)H;
        const float inv = 1.0f / sqrtf(var + eps);
        for (int i = 0; i < H; ++i) y[(size_t)r * H + i] = (xr[i] - mean) * inv;
    }
}
// shaders/ops_conv.metal:171-193 (Runtime::mean_cols, src/net.mm:103-106): y[c] = sum_s x[s][c] / S
extern "C" void orc_mean_cols(const float *x, float *y, int S, int H) {
    for (int c = 0; c < H; ++c) {
        float acc = 0.0f;
        for (int s = 0; s < S; ++s) acc += x[(size_t)s * H + c];
        y[c] = acc / (float)S;
    }
}
// shaders/ops_conv.metal:60-74: src row r column 3c + j -> dst row row_off + r column j*H + c
extern "C" void orc_qkv_split3(const float *src, float *dst, int rows, int H, int row_off) {
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < H; ++c)
            for (int j = 0; j < 3; ++j)
                dst[(size_t)(row_off + r) * 3 * H + (size_t)j * H + c] = src[(size_t)r * 3 * H + 3 * c + j];
}
// src/dit_fwd.cpp:111-119
extern "C" void orc_timestep_embedding(float t, int D, float max_period, float *out) {
    const int half = D / 2;
    const float fscale = 10000.0f / max_period;
    for (int k = 0; k < half; ++k) {
        const float fr = fscale * powf(10000.0f, -2.0f * (float)k / (float)D);
        out[k] = cosf(t * fr);
        out[half + k] = sinf(t * fr);
    }
}
