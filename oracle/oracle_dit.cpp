// oracle_dit.cpp — CPU f32 restatement of the DiT block graph (test infrastructure only).
//
// Graph: the two-stream MMDiT of the measured workloads. It follows the reference forward
// (src/dit_fwd.cpp:104-304) with these graph choices, each a flag-free restatement of the
// workload definition:
//   * joint blocks carry two streams, audio (RoPE, conv-k3 FFN) and text (linear FFN, no RoPE),
//     joined for one softmax over La+Lt rows (src/dit_fwd.cpp:180-257 with the clip stream
//     dropped);
//   * fused blocks run one weight set over the concatenated La+Lt rows with linear out-proj and
//     MLP; RoPE on audio rows only (src/dit_fwd.cpp:267-279 over the joined rows);
//   * adaLN modulation is per sample: silu(g)·Wᵀ + b (src/dit_fwd.cpp:193-207);
//   * the FFN activation is SiLU (src/dit_fwd.cpp:67-76 with the SwiGLU gate removed);
//   * input projection Linear latent->H + b; final layer adaLN (2 chunks) + Linear H->latent + b
//     (src/dit_fwd.cpp:142-149,287-303 with linear projections);
//   * timestep sinusoid of width temb_dim, MLP temb_dim->H->H, g = t_emb + pooled
//     (src/dit_fwd.cpp:111-131).
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

namespace {

struct Tensor { std::string name; int64_t numel; };

// Weight manifest, in the order the flat weight buffer holds the tensors. Shapes are noted in
// comments; 2-D weights are [out, in] row-major, conv weights [OC][IC][K] (src/dit_fwd.cpp
// weight names; src/net.mm:129-134 for the [N,K] convention).
std::vector<Tensor> manifest(const orc_spec &s) {
    std::vector<Tensor> v;
    const int64_t H = s.H, F = s.F, HD = s.HD;
    auto add = [&](const std::string &n, int64_t numel) { v.push_back({n, numel}); };
    add("t_embed.mlp.0.weight", H * s.temb_dim);
    add("t_embed.mlp.0.bias", H);
    add("t_embed.mlp.2.weight", H * H);
    add("t_embed.mlp.2.bias", H);
    add("audio_input_proj.weight", H * s.latent);
    add("audio_input_proj.bias", H);
    for (int i = 0; i < s.n_joint; ++i) {
        for (int st = 0; st < 2; ++st) {
            const std::string p = "joint_blocks." + std::to_string(i) + (st == 0 ? ".latent_block" : ".text_block");
            add(p + ".adaLN_modulation.1.weight", 6 * H * H);
            add(p + ".adaLN_modulation.1.bias", 6 * H);
            add(p + ".attn.qkv.weight", 3 * H * H);
            add(p + ".attn.qkv.bias", 3 * H);
            add(p + ".attn.q_norm.weight", HD);
            add(p + ".attn.k_norm.weight", HD);
            add(p + ".linear1.weight", H * H);
            add(p + ".linear1.bias", H);
            const int64_t taps = (st == 0 && s.audio_ffn_conv) ? 3 : 1;
            add(p + ".ffn.w1.weight", F * H * taps);
            add(p + ".ffn.w2.weight", H * F * taps);
        }
    }
    for (int i = 0; i < s.n_fused; ++i) {
        const std::string p = "fused_blocks." + std::to_string(i);
        add(p + ".adaLN_modulation.1.weight", 6 * H * H);
        add(p + ".adaLN_modulation.1.bias", 6 * H);
        add(p + ".attn.qkv.weight", 3 * H * H);
        add(p + ".attn.qkv.bias", 3 * H);
        add(p + ".attn.q_norm.weight", HD);
        add(p + ".attn.k_norm.weight", HD);
        add(p + ".linear1.weight", H * H);
        add(p + ".linear1.bias", H);
        add(p + ".ffn.w1.weight", F * H);
        add(p + ".ffn.w2.weight", H * F);
    }
    add("final_layer.adaLN_modulation.1.weight", 2 * H * H);
    add("final_layer.adaLN_modulation.1.bias", 2 * H);
    add("final_layer.linear.weight", (int64_t)s.latent * H);
    add("final_layer.linear.bias", s.latent);
    return v;
}

struct Weights {
    std::vector<Tensor> m;
    std::vector<int64_t> off;
    const float *base;
    Weights(const orc_spec &s, const float *w) : m(manifest(s)), base(w) {
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

// Stream rows of sample b inside X [B, S, H]: copy out / copy back.
void rows_out(const float *X, float *dst, int b, int S, int off, int L, int H) {
    memcpy(dst, X + ((size_t)b * S + off) * H, (size_t)L * H * sizeof(float));
}
void rows_in(float *X, const float *src, int b, int S, int off, int L, int H) {
    memcpy(X + ((size_t)b * S + off) * H, src, (size_t)L * H * sizeof(float));
}

// pre_attn for one stream of one sample (src/dit_fwd.cpp:24-49): adaLN(base 0) -> QKV + b ->
// per-head RMS on q and k -> RoPE on q and k (audio rows) -> rows [row_off, row_off+L) of J.
void pre_attn(const orc_spec &s, const Weights &W, const std::string &p, const float *x, int L,
              const float *mod, bool rope, float *J, int row_off) {
    const int H = s.H;
    std::vector<float> xn((size_t)L * H);
    orc_adaln_ln(x, mod, xn.data(), L, H, 0, 6, 0, s.ln_eps);
    float *dst = J + (size_t)row_off * 3 * H;
    orc_gemm(W.get(p + ".attn.qkv.weight"), xn.data(), dst, W.get(p + ".attn.qkv.bias"),
             L, 3 * H, H, H, H, 3 * H);
    orc_rms_head(J, W.get(p + ".attn.q_norm.weight"), L, s.NH, 3 * H, s.HD, 0, row_off, s.rms_eps);
    orc_rms_head(J, W.get(p + ".attn.k_norm.weight"), L, s.NH, 3 * H, s.HD, H, row_off, s.rms_eps);
    if (rope) {
        orc_rope_pairs(J, nullptr, L, s.NH, 3 * H, s.HD, 0, row_off, 1.0f, s.rope_theta);
        orc_rope_pairs(J, nullptr, L, s.NH, 3 * H, s.HD, H, row_off, 1.0f, s.rope_theta);
    }
}

// post_attn for one stream of one sample (src/dit_fwd.cpp:51-81): out-proj + b -> gate_add(2)
// -> adaLN(base 3H) -> FFN (conv k3 or linear, SiLU between, no bias) -> gate_add(5).
void post_attn(const orc_spec &s, const Weights &W, const std::string &p, float *x, int L,
               const float *attn_rows, const float *mod, bool conv_ffn) {
    const int H = s.H, F = s.F;
    std::vector<float> o((size_t)L * H), xn((size_t)L * H), h((size_t)L * F);
    orc_gemm(W.get(p + ".linear1.weight"), attn_rows, o.data(), W.get(p + ".linear1.bias"), L, H, H, H, H, H);
    orc_gate_add(x, o.data(), mod, x, L, H, 0, 6, 2);
    orc_adaln_ln(x, mod, xn.data(), L, H, 0, 6, 3 * H, s.ln_eps);
    if (conv_ffn) {
        orc_conv1d(W.get(p + ".ffn.w1.weight"), nullptr, xn.data(), h.data(), L, L, H, F, 3, 1, 1, 1);
        orc_silu(h.data(), h.size());
        orc_conv1d(W.get(p + ".ffn.w2.weight"), nullptr, h.data(), o.data(), L, L, F, H, 3, 1, 1, 1);
    } else {
        orc_gemm(W.get(p + ".ffn.w1.weight"), xn.data(), h.data(), nullptr, L, F, H, H, H, F);
        orc_silu(h.data(), h.size());
        orc_gemm(W.get(p + ".ffn.w2.weight"), h.data(), o.data(), nullptr, L, H, F, F, F, H);
    }
    orc_gate_add(x, o.data(), mod, x, L, H, 0, 6, 5);
}

void modulation(const orc_spec &s, const Weights &W, const std::string &p, const float *gs_b,
                float *mod, int chunks) {
    orc_gemv(W.get(p + ".adaLN_modulation.1.weight"), gs_b, mod, W.get(p + ".adaLN_modulation.1.bias"),
             chunks * s.H, s.H, s.H);
}

} // namespace

extern "C" int orc_manifest_count(const orc_spec *s) { return (int)manifest(*s).size(); }
extern "C" int64_t orc_manifest_numel(const orc_spec *s, int idx) { return manifest(*s)[idx].numel; }
extern "C" int64_t orc_manifest_total(const orc_spec *s) {
    int64_t t = 0;
    for (const auto &e : manifest(*s)) t += e.numel;
    return t;
}
extern "C" void orc_manifest_name(const orc_spec *s, int idx, char *buf, int cap) {
    const std::string n = manifest(*s)[idx].name;
    snprintf(buf, cap, "%s", n.c_str());
}

// Joint block: src/dit_fwd.cpp:180-257 (latent + text streams; clip stream absent).
extern "C" void orc_joint_block(const orc_spec *sp, const float *weights, int block, float *X, const float *gs) {
    const orc_spec &s = *sp;
    const Weights W(s, weights);
    const int H = s.H, S = s.La + s.Lt;
    const std::string pa = "joint_blocks." + std::to_string(block) + ".latent_block";
    const std::string pt = "joint_blocks." + std::to_string(block) + ".text_block";
    std::vector<float> J((size_t)S * 3 * H), A((size_t)S * H);
    std::vector<float> ma((size_t)6 * H), mt((size_t)6 * H);
    std::vector<float> xa((size_t)s.La * H), xt((size_t)s.Lt * H);
    for (int b = 0; b < s.B; ++b) {
        modulation(s, W, pa, gs + (size_t)b * H, ma.data(), 6);
        modulation(s, W, pt, gs + (size_t)b * H, mt.data(), 6);
        rows_out(X, xa.data(), b, S, 0, s.La, H);
        rows_out(X, xt.data(), b, S, s.La, s.Lt, H);
        pre_attn(s, W, pa, xa.data(), s.La, ma.data(), true, J.data(), 0);
        pre_attn(s, W, pt, xt.data(), s.Lt, mt.data(), false, J.data(), s.La);
        orc_attention(J.data(), A.data(), S, s.NH, s.HD, 3 * H, H, 0, H, 2 * H, 0, 1.0f / sqrtf((float)s.HD));
        post_attn(s, W, pa, xa.data(), s.La, A.data(), ma.data(), s.audio_ffn_conv != 0);
        post_attn(s, W, pt, xt.data(), s.Lt, A.data() + (size_t)s.La * H, mt.data(), false);
        rows_in(X, xa.data(), b, S, 0, s.La, H);
        rows_in(X, xt.data(), b, S, s.La, s.Lt, H);
    }
}

// Fused block: src/dit_fwd.cpp:267-279 over the joined La+Lt rows.
extern "C" void orc_fused_block(const orc_spec *sp, const float *weights, int block, float *X, const float *gs) {
    const orc_spec &s = *sp;
    const Weights W(s, weights);
    const int H = s.H, S = s.La + s.Lt;
    const std::string p = "fused_blocks." + std::to_string(block);
    std::vector<float> J((size_t)S * 3 * H), A((size_t)S * H), m((size_t)6 * H), xn((size_t)S * H);
    for (int b = 0; b < s.B; ++b) {
        float *x = X + (size_t)b * S * H;
        modulation(s, W, p, gs + (size_t)b * H, m.data(), 6);
        orc_adaln_ln(x, m.data(), xn.data(), S, H, 0, 6, 0, s.ln_eps);
        orc_gemm(W.get(p + ".attn.qkv.weight"), xn.data(), J.data(), W.get(p + ".attn.qkv.bias"),
                 S, 3 * H, H, H, H, 3 * H);
        orc_rms_head(J.data(), W.get(p + ".attn.q_norm.weight"), S, s.NH, 3 * H, s.HD, 0, 0, s.rms_eps);
        orc_rms_head(J.data(), W.get(p + ".attn.k_norm.weight"), S, s.NH, 3 * H, s.HD, H, 0, s.rms_eps);
        orc_rope_pairs(J.data(), nullptr, s.La, s.NH, 3 * H, s.HD, 0, 0, 1.0f, s.rope_theta);
        orc_rope_pairs(J.data(), nullptr, s.La, s.NH, 3 * H, s.HD, H, 0, 1.0f, s.rope_theta);
        orc_attention(J.data(), A.data(), S, s.NH, s.HD, 3 * H, H, 0, H, 2 * H, 0, 1.0f / sqrtf((float)s.HD));
        post_attn(s, W, p, x, S, A.data(), m.data(), false);
    }
}

// src/dit_fwd.cpp:104-304 restated for the two-stream graph.
extern "C" void orc_dit_forward(const orc_spec *sp, const float *weights, const float *z, const float *t,
                                const float *text, const float *pooled, float *v, float *taps, float *gs_out) {
    const orc_spec &s = *sp;
    const Weights W(s, weights);
    const int H = s.H, S = s.La + s.Lt, B = s.B;
    std::vector<float> gs((size_t)B * H), temb(s.temb_dim), h1(H), te(H);
    // timestep embedding + MLP (src/dit_fwd.cpp:111-128), g = pooled + t_emb (:131), silu (:140)
    for (int b = 0; b < B; ++b) {
        orc_timestep_embedding(t[b], s.temb_dim, s.t_max_period, temb.data());
        orc_gemv(W.get("t_embed.mlp.0.weight"), temb.data(), h1.data(), W.get("t_embed.mlp.0.bias"), H, s.temb_dim, s.temb_dim);
        orc_silu(h1.data(), H);
        orc_gemv(W.get("t_embed.mlp.2.weight"), h1.data(), te.data(), W.get("t_embed.mlp.2.bias"), H, H, H);
        orc_add(pooled + (size_t)b * H, te.data(), gs.data() + (size_t)b * H, H);
        orc_silu(gs.data() + (size_t)b * H, H);
    }
    if (gs_out) memcpy(gs_out, gs.data(), gs.size() * sizeof(float));
    // input projection (src/dit_fwd.cpp:142-149) and the text stream start (:166-167)
    std::vector<float> X((size_t)B * S * H);
    for (int b = 0; b < B; ++b) {
        orc_gemm(W.get("audio_input_proj.weight"), z + (size_t)b * s.La * s.latent, X.data() + (size_t)b * S * H,
                 W.get("audio_input_proj.bias"), s.La, H, s.latent, s.latent, s.latent, H);
        memcpy(X.data() + ((size_t)b * S + s.La) * H, text + (size_t)b * s.Lt * H, (size_t)s.Lt * H * sizeof(float));
    }
    int tap = 0;
    for (int i = 0; i < s.n_joint; ++i) {
        orc_joint_block(sp, weights, i, X.data(), gs.data());
        if (taps) memcpy(taps + (size_t)(tap++) * B * S * H, X.data(), X.size() * sizeof(float));
    }
    for (int i = 0; i < s.n_fused; ++i) {
        orc_fused_block(sp, weights, i, X.data(), gs.data());
        if (taps) memcpy(taps + (size_t)(tap++) * B * S * H, X.data(), X.size() * sizeof(float));
    }
    // final layer (src/dit_fwd.cpp:287-303): adaLN with 2 chunks on audio rows, then Linear
    std::vector<float> mf((size_t)2 * H), xn((size_t)s.La * H);
    for (int b = 0; b < B; ++b) {
        orc_gemv(W.get("final_layer.adaLN_modulation.1.weight"), gs.data() + (size_t)b * H, mf.data(),
                 W.get("final_layer.adaLN_modulation.1.bias"), 2 * H, H, H);
        orc_adaln_ln(X.data() + (size_t)b * S * H, mf.data(), xn.data(), s.La, H, 0, 2, 0, s.ln_eps);
        orc_gemm(W.get("final_layer.linear.weight"), xn.data(), v + (size_t)b * s.La * s.latent,
                 W.get("final_layer.linear.bias"), s.La, s.latent, H, H, H, s.latent);
    }
}

// src/pipeline.cpp:141-155: per step two arms (folded into the batch), then cfg_euler.
extern "C" void orc_dit_sample(const orc_spec *sp, const float *weights, float *x, const float *text,
                               const float *pooled, int steps, float cfg) {
    const orc_spec &s = *sp;
    const int P = s.B / 2;
    const size_t per = (size_t)s.La * s.latent;
    std::vector<float> z((size_t)s.B * per), v((size_t)s.B * per), t(s.B);
    for (int st = 0; st < steps; ++st) {
        const float t_curr = 1.0f - (float)st / (float)steps;
        const float t_prev = 1.0f - (float)(st + 1) / (float)steps;
        const float dt = t_prev - t_curr;
        for (int b = 0; b < s.B; ++b) {
            t[b] = t_curr;
            memcpy(z.data() + (size_t)b * per, x + (size_t)(b / 2) * per, per * sizeof(float));
        }
        orc_dit_forward(sp, weights, z.data(), t.data(), text, pooled, v.data(), nullptr, nullptr);
        for (int p = 0; p < P; ++p)
            orc_cfg_euler(v.data() + (size_t)(2 * p) * per, v.data() + (size_t)(2 * p + 1) * per,
                          x + (size_t)p * per, per, cfg, dt);
    }
}
