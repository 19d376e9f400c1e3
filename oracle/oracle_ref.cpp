// oracle_ref.cpp — CPU f32 restatement of the reference's own DiT graph (test infrastructure only).
//
// The three-stream graph of src/dit_fwd.cpp:104-304, batched over B samples (CFG arms), each
// sample run exactly as one reference forward:
//   * t -> H-wide sinusoid -> GEMV + SiLU -> GEMV = t_emb; global_c = gcmlp + t_emb;
//     extended_c[T, H] = sync_gather + global_c (per row); the latent, fused and final adaLN read
//     silu(extended_c) row by row (a GEMM, M = T), the clip and text adaLN read silu(global_c)
//     (src/dit_fwd.cpp:111-140,186-207,271-274,288-291);
//   * input projection: conv k3 (latent -> H) + b, SiLU, SwiGLU conv-MLP w1/w3 (conv k3) -> w2
//     (conv k3), no bias, no residual (src/dit_fwd.cpp:142-149);
//   * joint blocks: streams latent (T rows, RoPE pos 0..T-1), clip (C rows, RoPE scaled by T/C),
//     text (TS rows, no RoPE), one softmax over T + C + TS rows; out-proj conv k3 + b for latent and
//     clip, linear + b for text; SwiGLU FFN (conv k3 for latent and clip, linear for text, no
//     bias); the last joint block is pre-only: clip and text take 2 modulation chunks and are not
//     updated after attention (src/dit_fwd.cpp:24-81,180-257);
//   * fused blocks: the latent rows alone, same as a latent stream (src/dit_fwd.cpp:267-279);
//   * final layer: per-row adaLN (2 chunks), conv k7 pad 3 + b -> latent (src/dit_fwd.cpp:287-303).
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

namespace {

struct Tensor { std::string name; int64_t numel; };

// Weight manifest of the reference graph, in flat-buffer order. Conv weights are [OC][IC][K],
// linear weights [N][K]; adaLN weights [chunks*H][H]; qkv weight [3H][H] and bias [3H] with rows
// element-interleaved (row 3c + j: channel c of q, k, v).
std::vector<Tensor> ref_manifest(const orc_ref_spec &s) {
    std::vector<Tensor> v;
    const int64_t H = s.H, F = s.F, HD = s.HD, L = s.latent;
    auto add = [&](const std::string &n, int64_t numel) { v.push_back({n, numel}); };
    add("t_embed.mlp.0.weight", H * H);
    add("t_embed.mlp.0.bias", H);
    add("t_embed.mlp.2.weight", H * H);
    add("t_embed.mlp.2.bias", H);
    add("audio_input_proj.0.weight", H * L * 3);
    add("audio_input_proj.0.bias", H);
    add("audio_input_proj.2.w1.weight", F * H * 3);
    add("audio_input_proj.2.w3.weight", F * H * 3);
    add("audio_input_proj.2.w2.weight", H * F * 3);
    auto stream = [&](const std::string &p, int chunks, bool post, int64_t taps) {
        add(p + ".adaLN_modulation.1.weight", chunks * H * H);
        add(p + ".adaLN_modulation.1.bias", chunks * H);
        add(p + ".attn.qkv.weight", 3 * H * H);
        add(p + ".attn.qkv.bias", 3 * H);
        add(p + ".attn.q_norm.weight", HD);
        add(p + ".attn.k_norm.weight", HD);
        if (!post) return;
        add(p + ".linear1.weight", H * H * taps);
        add(p + ".linear1.bias", H);
        add(p + ".ffn.w1.weight", F * H * taps);
        add(p + ".ffn.w3.weight", F * H * taps);
        add(p + ".ffn.w2.weight", H * F * taps);
    };
    for (int i = 0; i < s.n_joint; ++i) {
        const bool pre_only = i == s.n_joint - 1;
        const std::string p = "joint_blocks." + std::to_string(i);
        stream(p + ".latent_block", 6, true, 3);
        stream(p + ".clip_block", pre_only ? 2 : 6, !pre_only, 3);
        stream(p + ".text_block", pre_only ? 2 : 6, !pre_only, 1);
    }
    for (int i = 0; i < s.n_fused; ++i) stream("fused_blocks." + std::to_string(i), 6, true, 3);
    add("final_layer.adaLN_modulation.1.weight", 2 * H * H);
    add("final_layer.adaLN_modulation.1.bias", 2 * H);
    add("final_layer.conv.weight", L * H * 7);
    add("final_layer.conv.bias", L);
    return v;
}

struct RefWeights {
    std::vector<Tensor> m;
    std::vector<int64_t> off;
    const float *base;
    RefWeights(const orc_ref_spec &s, const float *w) : m(ref_manifest(s)), base(w) {
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

void conv3(const float *W, const float *b, const float *x, float *y, int T, int IC, int OC) {
    orc_conv1d(W, b, x, y, T, T, IC, OC, 3, 1, 1, 1);
}

// SwiGLU FFN (src/dit.cpp:14-27 convmlp / mlp): y = w2(silu(w1 x) * w3 x), conv k3 or linear
void swiglu_ffn(const RefWeights &W, const std::string &p, const float *x, float *y, int L, int H, int F,
                bool conv) {
    std::vector<float> h1((size_t)L * F), h3((size_t)L * F);
    if (conv) {
        conv3(W.get(p + ".w1.weight"), nullptr, x, h1.data(), L, H, F);
        conv3(W.get(p + ".w3.weight"), nullptr, x, h3.data(), L, H, F);
    } else {
        orc_gemm(W.get(p + ".w1.weight"), x, h1.data(), nullptr, L, F, H, H, H, F);
        orc_gemm(W.get(p + ".w3.weight"), x, h3.data(), nullptr, L, F, H, H, H, F);
    }
    orc_swiglu(h1.data(), h3.data(), h1.data(), h1.size());
    if (conv) conv3(W.get(p + ".w2.weight"), nullptr, h1.data(), y, L, F, H);
    else orc_gemm(W.get(p + ".w2.weight"), h1.data(), y, nullptr, L, H, F, F, F, H);
}

// adaLN (base 0) -> QKV + b -> de-interleave -> RMS q, k -> RoPE (fscale; none when fscale == 0)
// into rows [row_off, row_off + L) of J [S, 3H]. mod: per row (stride chunks*H) or one row.
// The checkpoint's qkv weight and bias are element-interleaved: output column 3c + j is channel c
// of q (j = 0), k (1) or v (2); it lands at column j*H + c of J (qkv_split3,
// shaders/ops_conv.metal:60-74, called at src/dit_fwd.cpp:33-36).
void ref_pre_attn(const orc_ref_spec &s, const RefWeights &W, const std::string &p, const float *x, int L,
                  const float *mod, int per_row, int chunks, float fscale, float *J, int row_off) {
    const int H = s.H;
    std::vector<float> xn((size_t)L * H), qi((size_t)L * 3 * H);
    orc_adaln_ln(x, mod, xn.data(), L, H, per_row, chunks, 0, s.ln_eps);
    orc_gemm(W.get(p + ".attn.qkv.weight"), xn.data(), qi.data(), W.get(p + ".attn.qkv.bias"), L, 3 * H, H, H, H,
             3 * H);
    for (int r = 0; r < L; ++r)
        for (int c = 0; c < H; ++c)
            for (int j = 0; j < 3; ++j)
                J[(size_t)(row_off + r) * 3 * H + (size_t)j * H + c] = qi[(size_t)r * 3 * H + 3 * c + j];
    orc_rms_head(J, W.get(p + ".attn.q_norm.weight"), L, s.NH, 3 * H, s.HD, 0, row_off, s.rms_eps);
    orc_rms_head(J, W.get(p + ".attn.k_norm.weight"), L, s.NH, 3 * H, s.HD, H, row_off, s.rms_eps);
    if (fscale != 0.0f) {
        orc_rope_pairs(J, nullptr, L, s.NH, 3 * H, s.HD, 0, row_off, fscale, s.rope_theta);
        orc_rope_pairs(J, nullptr, L, s.NH, 3 * H, s.HD, H, row_off, fscale, s.rope_theta);
    }
}

// out-proj (conv k3 or linear) + b -> gate 2 -> adaLN (base 3H) -> SwiGLU FFN -> gate 5
void ref_post_attn(const orc_ref_spec &s, const RefWeights &W, const std::string &p, float *x, int L,
                   const float *att, const float *mod, int per_row, bool conv) {
    const int H = s.H;
    std::vector<float> o((size_t)L * H), xn((size_t)L * H);
    if (conv) conv3(W.get(p + ".linear1.weight"), W.get(p + ".linear1.bias"), att, o.data(), L, H, H);
    else orc_gemm(W.get(p + ".linear1.weight"), att, o.data(), W.get(p + ".linear1.bias"), L, H, H, H, H, H);
    orc_gate_add(x, o.data(), mod, x, L, H, per_row, 6, 2);
    orc_adaln_ln(x, mod, xn.data(), L, H, per_row, 6, 3 * H, s.ln_eps);
    swiglu_ffn(W, p + ".ffn", xn.data(), o.data(), L, H, s.F, conv);
    orc_gate_add(x, o.data(), mod, x, L, H, per_row, 6, 5);
}

} // namespace

extern "C" int orc_ref_manifest_count(const orc_ref_spec *s) { return (int)ref_manifest(*s).size(); }
extern "C" int64_t orc_ref_manifest_numel(const orc_ref_spec *s, int idx) { return ref_manifest(*s)[idx].numel; }
extern "C" void orc_ref_manifest_name(const orc_ref_spec *s, int idx, char *buf, int cap) {
    snprintf(buf, cap, "%s", ref_manifest(*s)[idx].name.c_str());
}

extern "C" void orc_ref_dit_forward(const orc_ref_spec *sp, const float *weights, const float *x,
                                    const float *t, const float *clip_pp, const float *text_pp,
                                    const float *gcmlp, const float *sync_gather, float *v, float *taps) {
    const orc_ref_spec &s = *sp;
    const RefWeights W(s, weights);
    const int H = s.H, T = s.T, C = s.C, TS = s.TS, S = T + C + TS, F = s.F, L = s.latent;
    const int nblk = s.n_joint + s.n_fused;
    std::vector<float> temb(H), h(H), te(H), gc(H), gs(H), extc((size_t)T * H);
    std::vector<float> X((size_t)S * H), J((size_t)S * 3 * H), A((size_t)S * H);
    std::vector<float> mod_lat((size_t)T * 6 * H), mod_c(6 * H), mod_t(6 * H), mod_fin((size_t)T * 2 * H);
    std::vector<float> xa((size_t)T * H), xb((size_t)T * F), xc((size_t)T * F), xn((size_t)T * H);
    for (int b = 0; b < s.B; ++b) {
        // conditioning
        orc_timestep_embedding(t[b], H, s.t_max_period, temb.data());
        orc_gemv(W.get("t_embed.mlp.0.weight"), temb.data(), h.data(), W.get("t_embed.mlp.0.bias"), H, H, H);
        orc_silu(h.data(), H);
        orc_gemv(W.get("t_embed.mlp.2.weight"), h.data(), te.data(), W.get("t_embed.mlp.2.bias"), H, H, H);
        orc_add(gcmlp + (size_t)b * H, te.data(), gc.data(), H);
        orc_add_bcast_col(sync_gather + (size_t)b * T * H, gc.data(), extc.data(), T, H);
        orc_silu(extc.data(), extc.size());
        memcpy(gs.data(), gc.data(), H * sizeof(float));
        orc_silu(gs.data(), H);
        // input projection -> latent rows of X; clip and text rows from the prepared streams
        float *lat = X.data(), *clip = X.data() + (size_t)T * H, *text = X.data() + (size_t)(T + C) * H;
        conv3(W.get("audio_input_proj.0.weight"), W.get("audio_input_proj.0.bias"), x + (size_t)b * T * L,
              xa.data(), T, L, H);
        orc_silu(xa.data(), xa.size());
        swiglu_ffn(W, "audio_input_proj.2", xa.data(), lat, T, H, F, true);
        memcpy(clip, clip_pp + (size_t)b * C * H, (size_t)C * H * sizeof(float));
        memcpy(text, text_pp + (size_t)b * TS * H, (size_t)TS * H * sizeof(float));
        int tap = 0;
        auto save_tap = [&]() {
            if (taps) memcpy(taps + (((size_t)tap * s.B + b) * S) * H, X.data(), (size_t)S * H * sizeof(float));
            ++tap;
        };
        for (int i = 0; i < s.n_joint; ++i) {
            const bool pre_only = i == s.n_joint - 1;
            const int cc = pre_only ? 2 : 6;
            const std::string p = "joint_blocks." + std::to_string(i);
            orc_gemm(W.get(p + ".latent_block.adaLN_modulation.1.weight"), extc.data(), mod_lat.data(),
                     W.get(p + ".latent_block.adaLN_modulation.1.bias"), T, 6 * H, H, H, H, 6 * H);
            orc_gemv(W.get(p + ".clip_block.adaLN_modulation.1.weight"), gs.data(), mod_c.data(),
                     W.get(p + ".clip_block.adaLN_modulation.1.bias"), cc * H, H, H);
            orc_gemv(W.get(p + ".text_block.adaLN_modulation.1.weight"), gs.data(), mod_t.data(),
                     W.get(p + ".text_block.adaLN_modulation.1.bias"), cc * H, H, H);
            ref_pre_attn(s, W, p + ".latent_block", lat, T, mod_lat.data(), 1, 6, 1.0f, J.data(), 0);
            ref_pre_attn(s, W, p + ".clip_block", clip, C, mod_c.data(), 0, cc, (float)T / (float)C, J.data(), T);
            ref_pre_attn(s, W, p + ".text_block", text, TS, mod_t.data(), 0, cc, 0.0f, J.data(), T + C);
            orc_attention(J.data(), A.data(), S, s.NH, s.HD, 3 * H, H, 0, H, 2 * H, 0, 1.0f / sqrtf((float)s.HD));
            ref_post_attn(s, W, p + ".latent_block", lat, T, A.data(), mod_lat.data(), 1, true);
            if (!pre_only) {
                ref_post_attn(s, W, p + ".clip_block", clip, C, A.data() + (size_t)T * H, mod_c.data(), 0, true);
                ref_post_attn(s, W, p + ".text_block", text, TS, A.data() + (size_t)(T + C) * H, mod_t.data(), 0,
                              false);
            }
            save_tap();
        }
        for (int i = 0; i < s.n_fused; ++i) {
            const std::string p = "fused_blocks." + std::to_string(i);
            orc_gemm(W.get(p + ".adaLN_modulation.1.weight"), extc.data(), mod_lat.data(),
                     W.get(p + ".adaLN_modulation.1.bias"), T, 6 * H, H, H, H, 6 * H);
            ref_pre_attn(s, W, p, lat, T, mod_lat.data(), 1, 6, 1.0f, J.data(), 0);
            orc_attention(J.data(), A.data(), T, s.NH, s.HD, 3 * H, H, 0, H, 2 * H, 0, 1.0f / sqrtf((float)s.HD));
            ref_post_attn(s, W, p, lat, T, A.data(), mod_lat.data(), 1, true);
            save_tap();
        }
        (void)nblk;
        orc_gemm(W.get("final_layer.adaLN_modulation.1.weight"), extc.data(), mod_fin.data(),
                 W.get("final_layer.adaLN_modulation.1.bias"), T, 2 * H, H, H, H, 2 * H);
        orc_adaln_ln(lat, mod_fin.data(), xn.data(), T, H, 1, 2, 0, s.ln_eps);
        orc_conv1d(W.get("final_layer.conv.weight"), W.get("final_layer.conv.bias"), xn.data(),
                   v + (size_t)b * T * L, T, T, H, L, 7, 1, 3, 1);
    }
}

extern "C" void orc_ref_dit_sample(const orc_ref_spec *sp, const float *weights, float *x, const float *clip_pp,
                                   const float *text_pp, const float *gcmlp, const float *sync_gather, int steps,
                                   float cfg) {
    const orc_ref_spec &s = *sp;
    const int P = s.B / 2;
    const size_t n = (size_t)s.T * s.latent;
    std::vector<float> x2((size_t)s.B * n), vv((size_t)s.B * n), t(s.B);
    for (int b = 0; b < s.B; ++b) memcpy(x2.data() + b * n, x + (b / 2) * n, n * sizeof(float));
    for (int st = 0; st < steps; ++st) {
        const float t_curr = 1.0f - (float)st / (float)steps, t_prev = 1.0f - (float)(st + 1) / (float)steps;
        for (int b = 0; b < s.B; ++b) t[b] = t_curr;
        orc_ref_dit_forward(sp, weights, x2.data(), t.data(), clip_pp, text_pp, gcmlp, sync_gather, vv.data(), nullptr);
        for (int p = 0; p < P; ++p) {
            orc_cfg_euler(vv.data() + 2 * p * n, vv.data() + (2 * p + 1) * n, x2.data() + 2 * p * n, n, cfg,
                          t_prev - t_curr);
            memcpy(x2.data() + (2 * p + 1) * n, x2.data() + 2 * p * n, n * sizeof(float));
        }
    }
    for (int p = 0; p < P; ++p) memcpy(x + p * n, x2.data() + 2 * p * n, n * sizeof(float));
}
