// oracle_enc.cpp — CPU f32 restatement of the reference's text encoders (test infrastructure only):
// ClipModel::encode (src/clip.cpp:34-122) and T5Model::encode (src/t5.cpp:57-131), with the
// reference's op kernels: ln_wb and rms_w (shaders/ops_conv.metal:90-113), gelu_quick and geglu
// (:15-29), and attn_qk / softmax_rows / attn_pav with its bias modes (shaders/gemm_attn.metal:84-202).
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <string>
#include <vector>

#include "oracle.h"

namespace {

struct Tensor { std::string name; int64_t numel; };

std::vector<Tensor> clip_manifest(const orc_clip_spec &s) {
    std::vector<Tensor> v;
    const int64_t H = s.H;
    auto add = [&](const std::string &n, int64_t k) { v.push_back({n, k}); };
    add("tok_emb", (int64_t)s.vocab * H);
    add("pos_emb", (int64_t)s.ctx * H);
    for (int l = 0; l < s.NL; ++l) {
        const std::string b = "blk." + std::to_string(l);
        for (const char *t : {".ln1", ".q", ".k", ".v", ".out", ".ln2", ".fc1", ".fc2"}) {
            const std::string p = b + t;
            const bool norm = t[1] == 'l';
            const int64_t rows = std::string(t) == ".fc1" ? 4 * H : H;
            const int64_t cols = norm ? 1 : std::string(t) == ".fc2" ? 4 * H : H;
            add(p + ".w", rows * cols);
            add(p + ".b", rows);
        }
    }
    add("out_ln.w", H);
    add("out_ln.b", H);
    add("text_proj", H * H);
    return v;
}

std::vector<Tensor> t5_manifest(const orc_t5_spec &s) {
    std::vector<Tensor> v;
    const int64_t d = s.d, F = s.d_ff;
    auto add = [&](const std::string &n, int64_t k) { v.push_back({n, k}); };
    add("tok_emb", (int64_t)s.vocab * d);
    for (int l = 0; l < s.NL; ++l) {
        const std::string b = "blk." + std::to_string(l);
        add(b + ".attn_norm", d);
        for (const char *t : {".q", ".k", ".v", ".o"}) add(b + t, d * d);
        add(b + ".ffn_norm", d);
        add(b + ".wi_0", F * d);
        add(b + ".wi_1", F * d);
        add(b + ".wo", d * F);
    }
    add("rel_bias", (int64_t)s.n_bucket * s.NH);
    add("out_norm", d);
    return v;
}

struct Weights {
    std::map<std::string, const float *> at;
    Weights(const std::vector<Tensor> &m, const float *w) {
        int64_t o = 0;
        for (const auto &t : m) { at[t.name] = w + o; o += t.numel; }
    }
    const float *get(const std::string &n) const {
        const auto it = at.find(n);
        if (it == at.end()) { fprintf(stderr, "oracle: missing tensor %s\n", n.c_str()); abort(); }
        return it->second;
    }
};

// Y[n][N] at column offset yoff of rows ldy = X[n][K] · W[N][K]ᵀ (+ b)
void linear(const float *W, const float *b, const float *X, float *Y, int n, int N, int K, int ldy) {
    orc_gemm(W, X, Y, b, n, N, K, K, K, ldy);
}

} // namespace

extern "C" {

int orc_clip_manifest_count(const orc_clip_spec *s) { return (int)clip_manifest(*s).size(); }
int64_t orc_clip_manifest_numel(const orc_clip_spec *s, int i) { return clip_manifest(*s)[i].numel; }
void orc_clip_manifest_name(const orc_clip_spec *s, int i, char *buf, int cap) {
    snprintf(buf, cap, "%s", clip_manifest(*s)[i].name.c_str());
}
int orc_t5_manifest_count(const orc_t5_spec *s) { return (int)t5_manifest(*s).size(); }
int64_t orc_t5_manifest_numel(const orc_t5_spec *s, int i) { return t5_manifest(*s)[i].numel; }
void orc_t5_manifest_name(const orc_t5_spec *s, int i, char *buf, int cap) {
    snprintf(buf, cap, "%s", t5_manifest(*s)[i].name.c_str());
}

// shaders/ops_conv.metal:90-103: mean, variance of the centred row, (x - mean)/sqrt(var + eps)*w + b
void orc_ln_wb(const float *x, float *y, const float *w, const float *b, int rows, int H, float eps) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float *xr = x + (size_t)r * H;
        float mean = 0.0f;
        for (int i = 0; i < H; ++i) mean += xr[i];
        mean /= (float)H;
        float var = 0.0f;
        for (int i = 0; i < H; ++i) { const float d = xr[i] - mean; var += d * d; }
        var /= (float)H;
        const float inv = 1.0f / sqrtf(var + eps);
        for (int i = 0; i < H; ++i) y[(size_t)r * H + i] = (xr[i] - mean) * inv * w[i] + b[i];
    }
}

// shaders/ops_conv.metal:104-113: x / sqrt(mean(x^2) + eps) * w
void orc_rms_w(const float *x, float *y, const float *w, int rows, int H, float eps) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float *xr = x + (size_t)r * H;
        float ss = 0.0f;
        for (int i = 0; i < H; ++i) ss += xr[i] * xr[i];
        const float inv = 1.0f / sqrtf(ss / (float)H + eps);
        for (int i = 0; i < H; ++i) y[(size_t)r * H + i] = xr[i] * inv * w[i];
    }
}

// src/t5.cpp:6-19
int orc_t5_bucket(int rel, int num_buckets, int max_dist) {
    int ret = 0;
    num_buckets /= 2;
    if (rel > 0) ret += num_buckets;
    const int n = abs(rel);
    const int max_exact = num_buckets / 2;
    if (n < max_exact) return ret + n;
    const int v = max_exact + (int)(log((double)n / max_exact) / log((double)max_dist / max_exact) *
                                    (num_buckets - max_exact));
    return ret + (v < num_buckets - 1 ? v : num_buckets - 1);
}

// shaders/gemm_attn.metal:84-202: scores over heads of hd columns, mode 1 (T5: pad keys -inf, else
// + rel[bucket[q*S+k]*nh + h]) or 2 (CLIP: -inf unless k <= q and k <= eot), max-subtracted softmax,
// P·V into out[q*ldo + h*hd + d]
void orc_enc_attention(const float *qkv, float *out, int S, int nh, int hd, int ld, int q_off, int k_off, int v_off,
                       int ldo, float scale, int mode, const int32_t *bucket, const float *rel, const int32_t *pad,
                       int eot) {
#pragma omp parallel for schedule(static)
    for (int h = 0; h < nh; ++h) {
        std::vector<float> p((size_t)S);
        for (int q = 0; q < S; ++q) {
            float mx = -INFINITY;
            for (int k = 0; k < S; ++k) {
                float s = 0.0f;
                for (int d = 0; d < hd; ++d)
                    s += qkv[(size_t)q * ld + q_off + h * hd + d] * qkv[(size_t)k * ld + k_off + h * hd + d];
                s *= scale;
                if (mode == 1) {
                    if (pad && pad[k] == 0) s = -INFINITY;
                    else s += rel[(size_t)bucket[(size_t)q * S + k] * nh + h];
                } else if (mode == 2) {
                    if (!(k <= q && k <= eot)) s = -INFINITY;
                }
                p[k] = s;
                mx = fmaxf(mx, s);
            }
            float sum = 0.0f;
            for (int k = 0; k < S; ++k) { p[k] = expf(p[k] - mx); sum += p[k]; }
            const float inv = 1.0f / sum;
            for (int k = 0; k < S; ++k) p[k] *= inv;
            for (int d = 0; d < hd; ++d) {
                float o = 0.0f;
                for (int k = 0; k < S; ++k) o += p[k] * qkv[(size_t)k * ld + v_off + h * hd + d];
                out[(size_t)q * ldo + h * hd + d] = o;
            }
        }
    }
}

// ClipModel::encode (src/clip.cpp:34-92)
void orc_clip_encode(const orc_clip_spec *sp, const float *weights, const int32_t *ids, float *per_token,
                     float *global) {
    const orc_clip_spec &s = *sp;
    const Weights W(clip_manifest(s), weights);
    const int n = s.ctx, H = s.H;
    std::vector<float> x((size_t)n * H), r((size_t)n * H), qkv((size_t)n * 3 * H), att((size_t)n * H),
        ff((size_t)n * 4 * H), t((size_t)n * H);
    const float *tok = W.get("tok_emb"), *pos = W.get("pos_emb");
    for (int i = 0; i < n; ++i)
        for (int c = 0; c < H; ++c) x[(size_t)i * H + c] = tok[(size_t)ids[i] * H + c] + pos[(size_t)i * H + c];
    int eos = 0;
    for (int i = 1; i < n; ++i) if (ids[i] > ids[eos]) eos = i;
    for (int l = 0; l < s.NL; ++l) {
        const std::string b = "blk." + std::to_string(l);
        orc_ln_wb(x.data(), r.data(), W.get(b + ".ln1.w"), W.get(b + ".ln1.b"), n, H, s.eps);
        linear(W.get(b + ".q.w"), W.get(b + ".q.b"), r.data(), qkv.data(), n, H, H, 3 * H);
        linear(W.get(b + ".k.w"), W.get(b + ".k.b"), r.data(), qkv.data() + H, n, H, H, 3 * H);
        linear(W.get(b + ".v.w"), W.get(b + ".v.b"), r.data(), qkv.data() + 2 * H, n, H, H, 3 * H);
        orc_enc_attention(qkv.data(), att.data(), n, s.NH, H / s.NH, 3 * H, 0, H, 2 * H, H,
                          1.0f / sqrtf((float)(H / s.NH)), 2, nullptr, nullptr, nullptr, eos);
        linear(W.get(b + ".out.w"), W.get(b + ".out.b"), att.data(), t.data(), n, H, H, H);
        orc_add(x.data(), t.data(), x.data(), x.size());
        orc_ln_wb(x.data(), r.data(), W.get(b + ".ln2.w"), W.get(b + ".ln2.b"), n, H, s.eps);
        linear(W.get(b + ".fc1.w"), W.get(b + ".fc1.b"), r.data(), ff.data(), n, 4 * H, H, 4 * H);
        for (auto &v : ff) v = v / (1.0f + expf(-1.702f * v));
        linear(W.get(b + ".fc2.w"), W.get(b + ".fc2.b"), ff.data(), t.data(), n, H, 4 * H, H);
        orc_add(x.data(), t.data(), x.data(), x.size());
    }
    orc_ln_wb(x.data(), per_token, W.get("out_ln.w"), W.get("out_ln.b"), n, H, s.eps);
    orc_gemv(W.get("text_proj"), per_token + (size_t)eos * H, global, nullptr, H, H, H);
}

// T5Model::encode (src/t5.cpp:88-131)
void orc_t5_encode(const orc_t5_spec *sp, const float *weights, const int32_t *ids, float *out) {
    const orc_t5_spec &s = *sp;
    const Weights W(t5_manifest(s), weights);
    const int n = s.ctx, d = s.d, F = s.d_ff;
    std::vector<int32_t> bucket((size_t)n * n), pad((size_t)n);
    for (int q = 0; q < n; ++q)
        for (int k = 0; k < n; ++k) bucket[(size_t)q * n + k] = orc_t5_bucket(k - q, s.n_bucket, s.max_dist);
    for (int i = 0; i < n; ++i) pad[i] = ids[i] != 0;
    std::vector<float> x((size_t)n * d), r((size_t)n * d), qkv((size_t)n * 3 * d), att((size_t)n * d),
        f1((size_t)n * F), f2((size_t)n * F), t((size_t)n * d);
    const float *tok = W.get("tok_emb");
    for (int i = 0; i < n; ++i) memcpy(&x[(size_t)i * d], tok + (size_t)ids[i] * d, (size_t)d * sizeof(float));
    for (int l = 0; l < s.NL; ++l) {
        const std::string b = "blk." + std::to_string(l);
        orc_rms_w(x.data(), r.data(), W.get(b + ".attn_norm"), n, d, s.eps);
        linear(W.get(b + ".q"), nullptr, r.data(), qkv.data(), n, d, d, 3 * d);
        linear(W.get(b + ".k"), nullptr, r.data(), qkv.data() + d, n, d, d, 3 * d);
        linear(W.get(b + ".v"), nullptr, r.data(), qkv.data() + 2 * d, n, d, d, 3 * d);
        orc_enc_attention(qkv.data(), att.data(), n, s.NH, d / s.NH, 3 * d, 0, d, 2 * d, d, 1.0f, 1, bucket.data(),
                          W.get("rel_bias"), pad.data(), 0);
        linear(W.get(b + ".o"), nullptr, att.data(), t.data(), n, d, d, d);
        orc_add(x.data(), t.data(), x.data(), x.size());
        orc_rms_w(x.data(), r.data(), W.get(b + ".ffn_norm"), n, d, s.eps);
        linear(W.get(b + ".wi_0"), nullptr, r.data(), f1.data(), n, F, d, F);
        linear(W.get(b + ".wi_1"), nullptr, r.data(), f2.data(), n, F, d, F);
        for (size_t i = 0; i < f1.size(); ++i) {   // shaders/ops_conv.metal:15-24
            const float v = f1[i];
            const float arg = 0.7978845608f * (v + 0.044715f * v * v * v);
            f1[i] = 0.5f * v * (1.0f + tanhf(fminf(fmaxf(arg, -10.0f), 10.0f))) * f2[i];
        }
        linear(W.get(b + ".wo"), nullptr, f1.data(), t.data(), n, d, F, d);
        orc_add(x.data(), t.data(), x.data(), x.size());
    }
    orc_rms_w(x.data(), out, W.get("out_norm"), n, d, s.eps);
}

} // extern "C"
