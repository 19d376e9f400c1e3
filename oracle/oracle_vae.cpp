// oracle_vae.cpp — CPU f32 restatement of the reference's VAE decoder (test infrastructure only):
// VaeModel::decode (src/vae.cpp:17-86) with the reference's conv routing (src/net.mm:25-49) and
// kernels (shaders/ops_conv.metal:204-213 snake, 262-283 im2col incl. the transposed-conv gather).
//
//   latent [T, 64] -> conv k7 pad 3 (+b) -> 5 x { snake -> transposed conv (stride s, kernel K,
//   pad K-1-s/2, +b) -> 3 x residual unit (dilation 1, 3, 9) } -> snake -> conv k7 pad 3 (no bias)
//   -> audio [T * prod(s), 2]
//   residual unit: x += conv_k1(snake(conv_k7_dil(snake(x))))  (k7 pad 3*dil, both with bias)
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "oracle.h"

namespace {

struct Tensor { std::string name; int64_t numel; };

const int DILS[3] = {1, 3, 9};

// Weight manifest of the decoder in flat-buffer order (the reference's GGUF tensor names).
// Conv weights [OC][IC][K] (the transposed convs already in the gather form the reference's
// im2col reads), snake alpha/beta [C].
std::vector<Tensor> vae_manifest(const orc_vae_spec &s) {
    std::vector<Tensor> v;
    auto add = [&](const std::string &n, int64_t numel) { v.push_back({n, numel}); };
    auto snake = [&](const std::string &p, int64_t C) {
        add(p + ".alpha", C);
        add(p + ".beta", C);
    };
    add("decoder.layers.0.weight", (int64_t)s.width[0] * s.latent * 7);
    add("decoder.layers.0.bias", s.width[0]);
    for (int n = 0; n < 5; ++n) {
        const std::string bp = "decoder.layers." + std::to_string(n + 1);
        const int64_t ci = s.width[n], co = s.width[n + 1];
        snake(bp + ".layers.0", ci);
        add(bp + ".layers.1.weight", co * ci * s.kt[n]);
        add(bp + ".layers.1.bias", co);
        for (int r = 0; r < 3; ++r) {
            const std::string rp = bp + ".layers." + std::to_string(r + 2);
            snake(rp + ".layers.0", co);
            add(rp + ".layers.1.weight", co * co * 7);
            add(rp + ".layers.1.bias", co);
            snake(rp + ".layers.2", co);
            add(rp + ".layers.3.weight", co * co);
            add(rp + ".layers.3.bias", co);
        }
    }
    snake("decoder.layers.6", s.width[5]);
    add("decoder.layers.7.weight", (int64_t)s.out_ch * s.width[5] * 7);
    return v;
}

struct VaeWeights {
    std::vector<Tensor> m;
    std::vector<int64_t> off;
    const float *base;
    VaeWeights(const orc_vae_spec &s, const float *w) : m(vae_manifest(s)), base(w) {
        int64_t o = 0;
        for (const auto &t : m) { off.push_back(o); o += t.numel; }
    }
    const float *get(const std::string &name) const {
        for (size_t i = 0; i < m.size(); ++i)
            if (m[i].name == name) return base + off[i];
        fprintf(stderr, "oracle: missing tensor %s\n", name.c_str());
        abort();
    }
};

} // namespace

extern "C" int orc_vae_manifest_count(const orc_vae_spec *s) { return (int)vae_manifest(*s).size(); }
extern "C" int64_t orc_vae_manifest_numel(const orc_vae_spec *s, int idx) { return vae_manifest(*s)[idx].numel; }
extern "C" void orc_vae_manifest_name(const orc_vae_spec *s, int idx, char *buf, int cap) {
    snprintf(buf, cap, "%s", vae_manifest(*s)[idx].name.c_str());
}

// shaders/ops_conv.metal:204-213: y = x + sin(x * exp(alpha[c]))^2 * exp(-beta[c])
extern "C" void orc_snake(const float *x, float *y, const float *alpha, const float *beta, int S, int C) {
    std::vector<float> ea(C), eb(C);
    for (int c = 0; c < C; ++c) {
        ea[c] = expf(alpha[c]);
        eb[c] = expf(-beta[c]);
    }
#pragma omp parallel for schedule(static)
    for (int t = 0; t < S; ++t)
        for (int c = 0; c < C; ++c) {
            const float v = x[(size_t)t * C + c];
            const float sn = sinf(v * ea[c]);
            y[(size_t)t * C + c] = v + sn * sn * eb[c];
        }
}

// Transposed conv the reference's way (src/net.mm:36-48, shaders/ops_conv.metal:262-283): im2col
// over the zero-stuffed input, then a GEMM with W [OC][IC*K]. Output row t, tap k reads input
// row (t - pad + k) / stride when t - pad + k >= 0 and divisible by stride, else zero.
extern "C" void orc_conv1d_t(const float *W, const float *bias, const float *x, float *y, int T, int OL, int IC,
                             int OC, int K, int stride, int pad) {
    const size_t KC = (size_t)IC * K;
    std::vector<float> col((size_t)OL * KC);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < OL; ++t)
        for (int ic = 0; ic < IC; ++ic)
            for (int k = 0; k < K; ++k) {
                const int ui = t - pad + k;
                float v = 0.0f;
                if (ui >= 0 && ui % stride == 0 && ui / stride < T) v = x[(size_t)(ui / stride) * IC + ic];
                col[(size_t)t * KC + (size_t)ic * K + k] = v;
            }
    orc_gemm(W, col.data(), y, bias, OL, OC, (int)KC, (int)KC, (int)KC, OC);
}

extern "C" int64_t orc_vae_audio_len(const orc_vae_spec *s) {
    int64_t T = s->T;
    for (int n = 0; n < 5; ++n) T *= s->stride[n];
    return T;
}

// VaeModel::decode (src/vae.cpp:17-86); latent [T, latent] -> audio [T_audio, out_ch]
extern "C" void orc_vae_decode(const orc_vae_spec *sp, const float *weights, const float *latent, float *audio) {
    const orc_vae_spec &s = *sp;
    const VaeWeights W(s, weights);
    int T = s.T, C = s.width[0];
    std::vector<float> x((size_t)T * C);
    // conv1: [T, latent] -> [T, width0], k7 pad 3 (src/vae.cpp:57-58)
    orc_conv1d(W.get("decoder.layers.0.weight"), W.get("decoder.layers.0.bias"), latent, x.data(), T, T, s.latent, C,
               7, 1, 3, 1);
    for (int n = 0; n < 5; ++n) {
        const std::string bp = "decoder.layers." + std::to_string(n + 1);
        const int st = s.stride[n], K = s.kt[n], co = s.width[n + 1];
        // snake -> transposed conv, pad K - 1 - st/2 (src/vae.cpp:62-67)
        std::vector<float> h((size_t)T * C);
        orc_snake(x.data(), h.data(), W.get(bp + ".layers.0.alpha"), W.get(bp + ".layers.0.beta"), T, C);
        const int OL = T * st;
        std::vector<float> xn((size_t)OL * co);
        orc_conv1d_t(W.get(bp + ".layers.1.weight"), W.get(bp + ".layers.1.bias"), h.data(), xn.data(), T, OL, C, co,
                     K, st, K - 1 - st / 2);
        x.swap(xn);
        T = OL;
        C = co;
        // three residual units (src/vae.cpp:69-77)
        std::vector<float> a((size_t)T * C), g((size_t)T * C);
        for (int r = 0; r < 3; ++r) {
            const std::string rp = bp + ".layers." + std::to_string(r + 2);
            const int d = DILS[r];
            orc_snake(x.data(), a.data(), W.get(rp + ".layers.0.alpha"), W.get(rp + ".layers.0.beta"), T, C);
            orc_conv1d(W.get(rp + ".layers.1.weight"), W.get(rp + ".layers.1.bias"), a.data(), g.data(), T, T, C, C, 7,
                       1, 3 * d, d);
            orc_snake(g.data(), a.data(), W.get(rp + ".layers.2.alpha"), W.get(rp + ".layers.2.beta"), T, C);
            orc_gemm(W.get(rp + ".layers.3.weight"), a.data(), g.data(), W.get(rp + ".layers.3.bias"), T, C, C, C, C,
                     C);
            orc_add(x.data(), g.data(), x.data(), (size_t)T * C);
        }
    }
    // final snake + conv k7 pad 3, no bias (src/vae.cpp:79-80); fewer than 32 output channels take the
    // reference's direct conv (src/net.mm:32-36)
    std::vector<float> h((size_t)T * C);
    orc_snake(x.data(), h.data(), W.get("decoder.layers.6.alpha"), W.get("decoder.layers.6.beta"), T, C);
    orc_conv1d_direct(W.get("decoder.layers.7.weight"), nullptr, h.data(), audio, T, T, C, s.out_ch, 7, 1, 3, 1);
}
