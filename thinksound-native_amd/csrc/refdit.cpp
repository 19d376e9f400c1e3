// refdit.cpp — RefDitModel on HIP: the reference checkpoint's three-stream DiT graph.
//
// Per evaluation (B samples folded into GEMM rows; src/dit_fwd.cpp:104-304 for the reference
// sequence):
//   sinusoid (H wide) -> GEMV + SiLU -> GEMV + gcmlp = global_c, silu(global_c) -> GEMV for every
//   clip/text modulation; silu(sync_gather + global_c) -> one GEMM for every per-row modulation
//   input: conv k3 on hi|lo x + b, SiLU -> SwiGLU conv k3 (w1|w3, one GEMM) -> conv k3 w2 -> X
//   per joint block: LN (3 streams) | QKV (3 problems; RMS + RoPE epilogue) | attention over S |
//                    out-proj (conv k3 / conv k3 / linear; gated residual) + LN2 | SwiGLU FFN1 |
//                    FFN2 (gated residual) + next block's LN
//   per fused block: the same over the latent rows, attention over T
//   final: per-row adaLN (f16 hi|lo) fused into the last reduce, conv k7 pad 3 -> v
#include "refdit.h"

#include "gguf.h"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <map>

namespace tsn {

std::vector<ManifestEntry> refdit_manifest(const RefDitSpec &s) {
    std::vector<ManifestEntry> v;
    const int64_t H = s.H, F = s.F, HD = s.HD, L = s.latent;
    int64_t off = 0;
    auto add = [&](const std::string &n, int64_t numel) {
        v.push_back({n, numel, off});
        off += numel;
    };
    add("t_embed.mlp.0.weight", H * H);
    add("t_embed.mlp.0.bias", H);
    add("t_embed.mlp.2.weight", H * H);
    add("t_embed.mlp.2.bias", H);
    add("audio_input_proj.0.weight", H * L * 3);
    add("audio_input_proj.0.bias", H);
    add("audio_input_proj.2.w1.weight", F * H * 3);
    add("audio_input_proj.2.w3.weight", F * H * 3);
    add("audio_input_proj.2.w2.weight", H * F * 3);
    // one stream of a block: adaLN (chunks x H rows), attention, and unless pre-only the out-proj
    // and SwiGLU FFN (taps 3: conv weights [OC][IC][3])
    auto stream = [&](const std::string &p, int64_t chunks, bool post, int64_t taps) {
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

int refdit_spec_check(const RefDitSpec &s) {
    TSN_REQUIRE(s.B == 1 || s.B == 2 || s.B == 4 || s.B == 8 || s.B == 16, "refdit spec: B must be 1, 2, 4, 8 or 16");
    TSN_REQUIRE(s.T > 0 && s.C >= 0 && s.TS >= 0, "refdit spec: T > 0, C >= 0, TS >= 0");
    TSN_REQUIRE(s.n_joint == 0 || (s.C > 0 && s.TS > 0), "refdit spec: joint blocks need clip and text rows");
    TSN_REQUIRE(s.HD == 64, "refdit spec: head dim must be 64");
    TSN_REQUIRE(s.H == s.NH * s.HD && s.H % 256 == 0 && s.H <= 2048, "refdit spec: H = NH*64, multiple of 256, <= 2048");
    TSN_REQUIRE(s.F % 64 == 0 && s.F > 0, "refdit spec: F must be a multiple of 64");
    TSN_REQUIRE(s.latent > 0 && s.latent % 64 == 0, "refdit spec: latent must be a multiple of 64");
    TSN_REQUIRE(s.n_joint >= 0 && s.n_fused >= 0, "refdit spec: block counts");
    return TSN_OK;
}

RefDitSpec refdit_spec_for_duration(int dur_s, int B) {
    RefDitSpec s{};
    s.B = B;
    s.T = (int)llround(44100.0 / 2048.0 * dur_s);
    s.C = 8 * dur_s;
    s.TS = 154;
    s.H = 1024; s.NH = 16; s.HD = 64; s.F = 2816; s.latent = 64;
    s.n_joint = 7; s.n_fused = 14;
    s.rope_theta = 10000.0f; s.t_max_period = 1.0f; s.ln_eps = 1e-5f; s.rms_eps = 1e-6f;
    return s;
}

namespace {
// RoPE table [pos][32][(cos, sin)]: ang = pos * fscale * base^(-2j/64), the expression and
// evaluation order of shaders/ops_conv.metal:162-163
std::vector<float> rope_table(int n, float fscale, float base) {
    std::vector<float> tab((size_t)n * 64);
    for (int p = 0; p < n; ++p)
        for (int j = 0; j < 32; ++j) {
            const float inv = powf(base, -2.0f * (float)j / 64.0f);
            const float ang = (float)p * fscale * inv;
            tab[((size_t)p * 32 + j) * 2] = cosf(ang);
            tab[((size_t)p * 32 + j) * 2 + 1] = sinf(ang);
        }
    return tab;
}
// A operand as f16 hi|lo pairs against W with half the channels per tap (f32-accurate operand)
void half_w(GemmProblem &p) {
    p.w_half = 1;
    p.ldw = p.taps * p.Kc / 2;
}
} // namespace

int RefDitModel::create(Runtime *r, const RefDitSpec &sp) {
    TSN_REQUIRE(r, "refdit: null runtime");
    TSN_TRY(refdit_spec_check(sp));
    rt = r;
    s = sp;
    S = s.T + s.C + s.TS;
    Sp = (S + 63) / 64 * 64;
    SpF = (s.T + 63) / 64 * 64;
    const size_t B = s.B, H = s.H, T = s.T;
    NMODL = (s.n_joint + s.n_fused) * 6 * s.H + 2 * s.H;
    NMODG = 0;
    for (int i = 0; i < s.n_joint; ++i) NMODG += (i == s.n_joint - 1 ? 4 : 12) * s.H;
    if (NMODG == 0) NMODG = s.H;   // keeps the buffers non-empty without joint blocks
    auto af = [&](float **p, size_t n) { return alloc(n * sizeof(float), (void **)p); };
    auto ah = [&](half_t **p, size_t n) { return alloc(n * sizeof(half_t), (void **)p); };
    TSN_TRY(af(&X_, B * S * H));
    TSN_TRY(af(&MODL_, B * T * NMODL));
    TSN_TRY(af(&MODG_, B * NMODG));
    TSN_TRY(af(&temb_, B * H));
    TSN_TRY(af(&h1_, B * H));
    TSN_TRY(af(&gc_, B * H));
    TSN_TRY(af(&gs_, B * H));
    TSN_TRY(af(&t_dev, B));
    TSN_TRY(ah(&XN_, B * S * 2 * H));   // [hi | lo] rows; lo written for latent FFN inputs only
    TSN_TRY(ah(&XE_, B * T * 2 * H));
    TSN_TRY(ah(&Z2_, B * T * 2 * (size_t)s.latent));
    TSN_TRY(ah(&XF2_, B * T * 2 * H));
    TSN_TRY(ah(&Q_, B * S * H));
    TSN_TRY(ah(&K_, B * S * H));
    TSN_TRY(ah(&Vt_, B * s.NH * 64 * (size_t)Sp));    // zero-filled: keys >= S stay zero
    TSN_TRY(ah(&VtF_, B * s.NH * 64 * (size_t)SpF));  // keys >= T stay zero
    TSN_TRY(ah(&AO_, B * S * 2 * H));
    TSN_TRY(ah(&HF_, B * S * 2 * (size_t)s.F));
    TSN_TRY(af(&Vv_, B * T * s.latent));
    TSN_TRY(af(&x2_, B * T * s.latent));
    // split-K partials: up to 8 splits of the largest residual output (B*S x H f32)
    ws_bytes_ = std::max((size_t)8 * B * S * H * sizeof(float), (size_t)40 << 20);   // split-K / stream-K
    TSN_TRY(alloc(ws_bytes_, (void **)&ws_));
    TSN_TRY(alloc_skcnt());
    // latent positions 0..T-1 (fscale 1); clip positions 0..C-1 scaled by T/C (src/dit_fwd.cpp:167-178)
    const std::vector<float> tl = rope_table(s.T, 1.0f, s.rope_theta);
    TSN_TRY(af(&rope_l_, tl.size()));
    TSN_TRY(rt->dev.upload(rope_l_, tl.data(), tl.size() * 4));
    if (s.C > 0) {
        const std::vector<float> tc = rope_table(s.C, (float)s.T / (float)s.C, s.rope_theta);
        TSN_TRY(af(&rope_c_, tc.size()));
        TSN_TRY(rt->dev.upload(rope_c_, tc.data(), tc.size() * 4));
    }
    return TSN_OK;
}

int RefDitModel::upload_weights(const uint16_t *host, size_t numel) { return upload(host, false, numel); }

int RefDitModel::upload_weights_f32(const float *host, size_t numel) { return upload(host, true, numel); }

// The flat buffer (bf16 or f32, manifest order) goes to the device once; every tensor is laid out
// and converted from there, then the staging buffer is freed.
int RefDitModel::upload(const void *host, bool src_f32, size_t numel) {
    TSN_REQUIRE(rt && host, "refdit: not created / null weights");
    TSN_REQUIRE(!ready_, "refdit: weights already uploaded");
    const auto man = refdit_manifest(s);
    const size_t total = (size_t)(man.back().offset + man.back().numel);
    TSN_REQUIRE(numel == total, "refdit: weight count does not match the manifest (" + std::to_string(total) + ")");
    const size_t esz = src_f32 ? 4 : 2;
    TSN_TRY(alloc(total * esz, &wraw_));
    TSN_TRY(rt->dev.upload(wraw_, host, total * esz));
    std::map<std::string, GgufDeviceTensor> raw;
    for (const auto &e : man)
        raw[e.name] = GgufDeviceTensor{(const char *)wraw_ + e.offset * esz, src_f32 ? WP_SRC_F32 : WP_SRC_BF16};
    return prepare(raw);
}

// Every tensor laid out and converted on the device from its raw source (address and encoding per
// name), then the source buffer (wraw_) is freed.
int RefDitModel::prepare(const std::map<std::string, GgufDeviceTensor> &raw) {
    const auto man = refdit_manifest(s);
    std::map<std::string, const ManifestEntry *> idx;
    for (const auto &e : man) idx[e.name] = &e;
    const hipStream_t st = rt->dev.stream();
    const int H = s.H, F = s.F, L = s.latent;
    // prep(name, OC, IC, KT, dup, row map ra/rb/rc/rd, dst, dst_rows, f32 out)
    auto prep = [&](const std::string &n, int OC, int IC, int KT, int dup, int ra, int rb, int rc, int rd, void *dst,
                    long long dst_rows, int out_f32) -> int {
        TSN_REQUIRE(idx.at(n)->numel == (int64_t)OC * IC * KT, "refdit: tensor size mismatch: " + n);
        const GgufDeviceTensor &r = raw.at(n);
        return launch_weight_prep(r.p, r.type, dst, out_f32, OC, IC, KT, dup, ra, rb, rc, rd, dst_rows, st);
    };
    auto new_f16 = [&](size_t n, half_t **p) { return alloc(n * 2, (void **)p); };
    auto new_f32 = [&](size_t n, float **p) { return alloc(n * 4, (void **)p); };
    // plain copies: f16 [OC][IC] (or tap-major conv [OC][KT][IC]), f32 vectors
    auto f16w = [&](const std::string &n, int OC, int IC, int KT, const half_t **out) -> int {
        half_t *p;
        TSN_TRY(new_f16((size_t)OC * IC * KT, &p));
        TSN_TRY(prep(n, OC, IC, KT, 0, 1, 0, 1, 0, p, OC, 0));
        *out = p;
        return TSN_OK;
    };
    auto f32v = [&](const std::string &n, int N, const float **out) -> int {
        float *p;
        TSN_TRY(new_f32(N, &p));
        TSN_TRY(prep(n, N, 1, 1, 0, 1, 0, 1, 0, p, N, 1));
        *out = p;
        return TSN_OK;
    };
    // SwiGLU pair: w1 and w3 [F][IC][KT] -> [2F][KT][IC], 64-row blocks w1 j, w3 j
    auto swiglu_w = [&](const std::string &p, int IC, int KT, const half_t **out) -> int {
        half_t *w;
        TSN_TRY(new_f16((size_t)2 * F * IC * KT, &w));
        TSN_TRY(prep(p + ".w1.weight", F, IC, KT, 0, 64, 1, 128, 0, w, 2LL * F, 0));
        TSN_TRY(prep(p + ".w3.weight", F, IC, KT, 0, 64, 1, 128, 64, w, 2LL * F, 0));
        *out = w;
        return TSN_OK;
    };
    half_t *wmodl, *wmodg;
    float *bmodl, *bmodg;
    TSN_TRY(new_f16((size_t)NMODL * H, &wmodl));
    TSN_TRY(new_f32(NMODL, &bmodl));
    TSN_TRY(new_f16((size_t)NMODG * H, &wmodg));
    TSN_TRY(new_f32(NMODG, &bmodg));
    int rowl = 0, rowg = 0;
    // per-row modulation weights gathered as f16 rows of one GEMM (read by both halves of the hi|lo
    // operand); per-sample ones as f16 rows of one GEMV
    auto mod_rows = [&](const std::string &p, int chunks, bool per_row, int *off) -> int {
        const std::string wn = p + ".adaLN_modulation.1.weight", bn = p + ".adaLN_modulation.1.bias";
        TSN_REQUIRE(idx.at(wn)->numel == (int64_t)chunks * H * H, "refdit: adaLN size: " + p);
        if (per_row) {
            *off = rowl;
            TSN_TRY(prep(wn, chunks * H, H, 1, 0, 1, 0, 1, rowl, wmodl, NMODL, 0));
            TSN_TRY(prep(bn, chunks * H, 1, 1, 0, 1, 0, 1, rowl, bmodl, NMODL, 1));
            rowl += chunks * H;
        } else {
            *off = rowg;
            TSN_TRY(prep(wn, chunks * H, H, 1, 0, 1, 0, 1, rowg, wmodg, NMODG, 0));
            TSN_TRY(prep(bn, chunks * H, 1, 1, 0, 1, 0, 1, rowg, bmodg, NMODG, 1));
            rowg += chunks * H;
        }
        return TSN_OK;
    };
    auto stream = [&](const std::string &p, int chunks, bool post, int taps, bool per_row, StreamW &w) -> int {
        TSN_TRY(mod_rows(p, chunks, per_row, &w.mod_off));
        half_t *q;
        float *bq;
        // qkv rows 3c + j (channel c of q, k, v) -> row j*H + c
        TSN_TRY(new_f16((size_t)3 * H * H, &q));
        TSN_TRY(prep(p + ".attn.qkv.weight", 3 * H, H, 1, 0, 3, H, 1, 0, q, 3LL * H, 0));
        TSN_TRY(new_f32((size_t)3 * H, &bq));
        TSN_TRY(prep(p + ".attn.qkv.bias", 3 * H, 1, 1, 0, 3, H, 1, 0, bq, 3LL * H, 1));
        w.Wqkv = q;
        w.bqkv = bq;
        TSN_TRY(f32v(p + ".attn.q_norm.weight", s.HD, &w.qn));
        TSN_TRY(f32v(p + ".attn.k_norm.weight", s.HD, &w.kn));
        w.taps = taps;
        w.post = post ? 1 : 0;
        w.hl = per_row ? 1 : 0;   // latent rows: out-proj and FFN over hi|lo operands
        if (!post) return TSN_OK;
        TSN_TRY(f16w(p + ".linear1.weight", H, H, taps, &w.Wo));
        TSN_TRY(f32v(p + ".linear1.bias", H, &w.bo));
        TSN_TRY(swiglu_w(p + ".ffn", H, taps, &w.W13));
        TSN_TRY(f16w(p + ".ffn.w2.weight", H, F, taps, &w.W2));
        return TSN_OK;
    };
    jl_.assign(s.n_joint, StreamW{});
    jc_.assign(s.n_joint, StreamW{});
    jt_.assign(s.n_joint, StreamW{});
    fu_.assign(s.n_fused, StreamW{});
    for (int i = 0; i < s.n_joint; ++i) {
        const bool pre_only = i == s.n_joint - 1;
        const std::string p = "joint_blocks." + std::to_string(i);
        TSN_TRY(stream(p + ".latent_block", 6, true, 3, true, jl_[i]));
        TSN_TRY(stream(p + ".clip_block", pre_only ? 2 : 6, !pre_only, 3, false, jc_[i]));
        TSN_TRY(stream(p + ".text_block", pre_only ? 2 : 6, !pre_only, 1, false, jt_[i]));
    }
    for (int i = 0; i < s.n_fused; ++i) TSN_TRY(stream("fused_blocks." + std::to_string(i), 6, true, 3, true, fu_[i]));
    TSN_TRY(mod_rows("final_layer", 2, true, &fin_off_));
    WmodL_ = wmodl;
    bmodL_ = bmodl;
    WmodG_ = wmodg;
    bmodG_ = bmodg;
    TSN_TRY(f16w("t_embed.mlp.0.weight", H, H, 1, &Wt0_));
    TSN_TRY(f16w("t_embed.mlp.2.weight", H, H, 1, &Wt2_));
    TSN_TRY(f32v("t_embed.mlp.0.bias", H, &bt0_));
    TSN_TRY(f32v("t_embed.mlp.2.bias", H, &bt2_));
    // input conv [H][L][3] and final conv [L][H][7], tap-major
    TSN_TRY(f16w("audio_input_proj.0.weight", H, L, 3, &Win_));
    TSN_TRY(f16w("final_layer.conv.weight", L, H, 7, &Wfin_));
    TSN_TRY(f32v("audio_input_proj.0.bias", H, &bin_));
    TSN_TRY(f32v("final_layer.conv.bias", L, &bfin_));
    TSN_TRY(swiglu_w("audio_input_proj.2", H, 3, &W13in_));
    TSN_TRY(f16w("audio_input_proj.2.w2.weight", H, F, 3, &W2in_));
    TSN_TRY(rt->dev.sync());
    TSN_TRY(release(wraw_));
    wraw_ = nullptr;
    ready_ = true;
    return TSN_OK;
}

// WeightSet::load + DitModel::load (src/net.mm:126-173, src/dit.cpp:29-47): every tensor the graph
// needs is looked up by name and its payload goes to HBM as stored in the file (BF16, F16, F32 or
// Q8_0 bytes, no host conversion and no host copy beyond the mapping and two pinned transfer
// buffers); the device then converts and lays out each tensor: GEMM and GEMV weights f16 with the
// reference's rounding, vectors f32.
int RefDitModel::load_gguf(const char *path) {
    TSN_REQUIRE(rt, "refdit: not created");
    TSN_REQUIRE(!ready_, "refdit: weights already uploaded");
    GgufReader g;
    TSN_TRY(g.open(path));
    std::map<std::string, GgufDeviceTensor> raw;
    size_t moved = 0;
    TSN_TRY(gguf_stage_manifest(g, refdit_manifest(s), rt->dev,
                                [&](size_t n, void **p) {
                                    TSN_TRY(alloc(n, p));
                                    wraw_ = *p;
                                    return (int)TSN_OK;
                                },
                                raw, &moved));
    load_bytes_ = moved;
    return prepare(raw);
}

int refdit_spec_from_gguf(const char *path, int B, int T, int C, int TS, RefDitSpec *out) {
    TSN_REQUIRE(out, "refdit gguf: null spec");
    GgufReader g;
    TSN_TRY(g.open(path));
    RefDitSpec s{};
    s.B = B; s.T = T; s.C = C; s.TS = TS;
    s.H = (int)g.get_i64("dit.hidden_dim", 1024);
    s.NH = (int)g.get_i64("dit.num_heads", 16);
    TSN_REQUIRE(s.NH > 0 && s.H % s.NH == 0, "refdit gguf: hidden_dim must be a multiple of num_heads");
    s.HD = s.H / s.NH;
    const int depth = (int)g.get_i64("dit.depth", 21);
    s.n_fused = (int)g.get_i64("dit.fused_depth", 14);
    s.n_joint = depth - s.n_fused;
    s.latent = (int)g.get_i64("dit.latent_dim", 64);
    s.rope_theta = (float)g.get_f64("dit.rope_theta", 10000.0);
    s.t_max_period = (float)g.get_f64("dit.t_embed_max_period", 1.0);
    // SwiGLU width from the first latent FFN conv weight, ne = [3, H, F]
    const GgufTensorInfo *w1 = g.find("joint_blocks.0.latent_block.ffn.w1.weight");
    s.F = w1 && w1->n_dims >= 3 ? (int)w1->ne[2] : 2816;
    s.ln_eps = 1e-5f;
    s.rms_eps = 1e-6f;
    TSN_TRY(refdit_spec_check(s));
    *out = s;
    return TSN_OK;
}

RowMap RefDitModel::stream_map(int kind) const {
    return kind == ST_LAT ? RowMap{s.T, S, 0} : kind == ST_CLIP ? RowMap{s.C, S, s.T} : RowMap{s.TS, S, s.T + s.C};
}

// LN1 segment of one stream: latent rows read their own modulation row, clip and text rows their
// sample's (src/dit_fwd.cpp:28-30 with per_row 1 / 0)
void RefDitModel::ln1_seg(LnSeg &g, int kind, const StreamW &w) {
    const RowMap m = stream_map(kind);
    const int rows = s.B * m.L;
    if (kind == ST_LAT) ln_seg(g, X_, s.H, m, XN_, MODL_, NMODL, 1, w.mod_off, rows);
    else ln_seg(g, X_, s.H, m, XN_, modg_, NMODG, m.L, w.mod_off, rows);
    g.ldy = 2 * s.H;
}

// Fill the LN part of r's segments (one per stream of the residual GEMM) for the adaLN that runs
// next: LN1 of the next joint block (every stream) or fused block (latent), or the final layer's
// (latent rows as f16 hi|lo into XF2). LN1 output is f16 hi|lo in every stream (the QKV operand).
// ln2: the LN2 of block next.idx instead of its LN1 (chunks 3, 4), f16 hi|lo for latent rows (the
// FFN operand), hi only for clip and text rows.
void RefDitModel::next_ln(RedLnArgs &r, Next next, const int *kinds, int nseg, bool ln2) {
    memset(&r, 0, sizeof r);
    r.ymode = next.kind == NEXT_FINAL ? LN_F16_HILO : LN_F16;
    for (int i = 0; i < nseg; ++i) {
        RedLnSeg &g = r.seg[i];
        const int k = kinds[i];
        const RowMap m = stream_map(k);
        g.Y = XN_; g.ldy = 2 * s.H; g.ymap = m;
        g.hilo = !ln2 || k == ST_LAT;   // LN1 (QKV operand) in every stream, LN2 (FFN operand) for latent rows
        if (k == ST_LAT) { g.mod = MODL_; g.mod_ld = NMODL; g.mod_L = 1; g.ln_len = 1; }
        else { g.mod = modg_; g.mod_ld = NMODG; g.mod_L = m.L; g.ln_len = m.L; }
        switch (next.kind) {
        case NEXT_JOINT: g.ln = 1; g.shift_off = (k == ST_LAT ? jl_ : k == ST_CLIP ? jc_ : jt_)[next.idx].mod_off; break;
        case NEXT_FUSED: g.ln = k == ST_LAT; g.shift_off = fu_[next.idx].mod_off; break;
        case NEXT_FINAL:
            g.ln = k == ST_LAT;
            g.shift_off = fin_off_;
            g.Y = XF2_; g.ldy = 2 * s.H; g.ymap = RowMap{s.T, s.T, 0};
            break;
        default: g.ln = 0; break;
        }
        if (ln2) g.shift_off += 3 * s.H;
        g.scale_off = g.shift_off + s.H;
    }
}

// Joint block: src/dit_fwd.cpp:180-257 (pre_attn :24-49, attention :83-102, post_attn :51-81)
int RefDitModel::block_joint(int i, bool ln1, Next next) {
    const hipStream_t st = rt->dev.stream();
    const StreamW *w[3] = {&jl_[i], &jc_[i], &jt_[i]};
    const int B = s.B, H = s.H;
    const int kinds[3] = {ST_LAT, ST_CLIP, ST_TEXT};
    if (ln1) {   // otherwise the previous block's last reduce kernel produced it
        LnArgs ln;
        memset(&ln, 0, sizeof ln);
        ln.nseg = 3; ln.H = H; ln.eps = s.ln_eps;
        for (int k = 0; k < 3; ++k) ln1_seg(ln.seg[k], kinds[k], *w[k]);
        TSN_TRY(run(K_LNHL, 0, ln_bytes(ln, true), [&] { return launch_ln_mod(ln, LN_F16_HILO, st); }));
    }
    // q|k|v with per-head RMS; RoPE on latent (positions 0..T-1) and clip (scaled by T/C) rows
    GemmBatch qb;
    qb.nprob = 3;
    const int soff[3] = {0, s.T, s.T + s.C};
    const int rlen[3] = {s.T, s.C, 0};
    const float *rope[3] = {rope_l_, rope_c_, rope_l_};
    for (int k = 0; k < 3; ++k) {
        const RowMap m = stream_map(kinds[k]);
        qkv_problem(qb.p[k], XN_, m, B * m.L, w[k]->Wqkv, w[k]->bqkv, w[k]->qn, w[k]->kn, H, s.NH, Q_, K_, Vt_, S, Sp,
                    m.L, soff[k], rlen[k], rope[k], s.rms_eps);
        qb.p[k].lda = qb.p[k].Kc = qb.p[k].K = 2 * H;   // XN rows as hi|lo
        half_w(qb.p[k]);
    }
    qb.ws = ws_;
    qb.ws_bytes = ws_bytes_;
    TSN_TRY(gemm_run(qb, EPI_QKV));

    AttnArgs at;
    memset(&at, 0, sizeof at);
    at.Q = Q_; at.K = K_; at.Vt = Vt_; at.S = S; at.Sp = Sp; at.nh = s.NH; at.BH = B * s.NH;
    at.O = AO_; at.o_f32 = 0; at.ldo = 2 * H; at.o_lo = H; at.omap = rowmap_dense(B * S);
    TSN_TRY(run(K_ATTN, 4.0 * B * s.NH * (double)S * S * 64, 8.0 * B * (double)S * H,
                [&] { return launch_attention(at, st); }));

    // the pre-only block updates the latent stream alone
    const int np = w[1]->post ? 3 : 1;
    GemmBatch ob;
    ob.nprob = np;
    ob.ws = ws_;
    ob.ws_bytes = ws_bytes_;
    ob.split_waves = 1;
    for (int k = 0; k < np; ++k) {
        const RowMap m = stream_map(kinds[k]);
        const bool lat = kinds[k] == ST_LAT;
        resid_problem(ob.p[k], AO_, 2 * H, m, w[k]->taps, w[k]->hl ? 2 * H : H, B * m.L, H, w[k]->Wo, w[k]->bo, X_, H,
                      (lat ? MODL_ : modg_) + w[k]->mod_off + 2 * H, lat ? NMODL : NMODG);
        if (lat) ob.p[k].gate_L = 1;   // gate per latent row
        if (w[k]->hl) half_w(ob.p[k]);
    }
    RedLnArgs r;
    next_ln(r, Next{NEXT_JOINT, i}, kinds, np, true);   // LN2 of this block
    TSN_TRY(resid_ln(ob, r, H, s.ln_eps));

    GemmBatch f1;
    f1.nprob = np;
    for (int k = 0; k < np; ++k) {
        const RowMap m = stream_map(kinds[k]);
        store_problem(f1.p[k], XN_, 2 * H, m, w[k]->taps, w[k]->hl ? 2 * H : H, B * m.L, 2 * s.F, w[k]->W13, HF_,
                      2 * s.F, 0);
        f1.p[k].y_lo = w[k]->hl ? s.F : 0;
        if (w[k]->hl) half_w(f1.p[k]);
    }
    f1.ws = ws_;
    f1.ws_bytes = ws_bytes_;
    TSN_TRY(gemm_run(f1, EPI_SWIGLU));

    GemmBatch f2;
    f2.nprob = np;
    f2.ws = ws_;
    f2.ws_bytes = ws_bytes_;
    f2.split_waves = 1;   // long K over few tiles: a classic split keeps each W tile's readers together
    for (int k = 0; k < np; ++k) {
        const RowMap m = stream_map(kinds[k]);
        const bool lat = kinds[k] == ST_LAT;
        resid_problem(f2.p[k], HF_, 2 * s.F, m, w[k]->taps, w[k]->hl ? 2 * s.F : s.F, B * m.L, H, w[k]->W2, nullptr,
                      X_, H, (lat ? MODL_ : modg_) + w[k]->mod_off + 5 * H, lat ? NMODL : NMODG);
        if (lat) f2.p[k].gate_L = 1;
        if (w[k]->hl) half_w(f2.p[k]);
    }
    next_ln(r, next, kinds, np);
    return resid_ln(f2, r, H, s.ln_eps);
}

// Fused block: src/dit_fwd.cpp:267-279 over the latent rows, attention over T
int RefDitModel::block_fused(int i, bool ln1, Next next) {
    const hipStream_t st = rt->dev.stream();
    const StreamW &w = fu_[i];
    const int B = s.B, H = s.H, T = s.T, M = B * T;
    const RowMap Lm = stream_map(ST_LAT);
    const int kinds[1] = {ST_LAT};
    if (ln1) {
        LnArgs ln;
        memset(&ln, 0, sizeof ln);
        ln.nseg = 1; ln.H = H; ln.eps = s.ln_eps;
        ln1_seg(ln.seg[0], ST_LAT, w);
        TSN_TRY(run(K_LNHL, 0, ln_bytes(ln, true), [&] { return launch_ln_mod(ln, LN_F16_HILO, st); }));
    }
    GemmBatch qb;
    qb.nprob = 1;
    qkv_problem(qb.p[0], XN_, Lm, M, w.Wqkv, w.bqkv, w.qn, w.kn, H, s.NH, Q_, K_, VtF_, T, SpF, T, 0, T, rope_l_,
                s.rms_eps);
    qb.p[0].lda = qb.p[0].Kc = qb.p[0].K = 2 * H;   // XN rows as hi|lo
    half_w(qb.p[0]);
    qb.ws = ws_;
    qb.ws_bytes = ws_bytes_;
    TSN_TRY(gemm_run(qb, EPI_QKV));

    AttnArgs at;
    memset(&at, 0, sizeof at);
    at.Q = Q_; at.K = K_; at.Vt = VtF_; at.S = T; at.Sp = SpF; at.nh = s.NH; at.BH = B * s.NH;
    at.O = AO_; at.o_f32 = 0; at.ldo = 2 * H; at.o_lo = H; at.omap = Lm;
    TSN_TRY(run(K_ATTN, 4.0 * B * s.NH * (double)T * T * 64, 8.0 * B * (double)T * H,
                [&] { return launch_attention(at, st); }));

    GemmBatch ob;
    ob.nprob = 1;
    ob.ws = ws_;
    ob.ws_bytes = ws_bytes_;
    ob.split_waves = 1;
    resid_problem(ob.p[0], AO_, 2 * H, Lm, w.taps, 2 * H, M, H, w.Wo, w.bo, X_, H, MODL_ + w.mod_off + 2 * H, NMODL);
    ob.p[0].gate_L = 1;
    half_w(ob.p[0]);
    RedLnArgs r;
    next_ln(r, Next{NEXT_FUSED, i}, kinds, 1, true);   // LN2 of this block
    TSN_TRY(resid_ln(ob, r, H, s.ln_eps));

    GemmBatch f1;
    f1.nprob = 1;
    store_problem(f1.p[0], XN_, 2 * H, Lm, w.taps, 2 * H, M, 2 * s.F, w.W13, HF_, 2 * s.F, 0);
    f1.p[0].y_lo = s.F;
    half_w(f1.p[0]);
    f1.ws = ws_;
    f1.ws_bytes = ws_bytes_;
    TSN_TRY(gemm_run(f1, EPI_SWIGLU));

    GemmBatch f2;
    f2.nprob = 1;
    f2.ws = ws_;
    f2.ws_bytes = ws_bytes_;
    f2.split_waves = 1;   // long K over few tiles: a classic split keeps each W tile's readers together
    resid_problem(f2.p[0], HF_, 2 * s.F, Lm, w.taps, 2 * s.F, M, H, w.W2, nullptr, X_, H, MODL_ + w.mod_off + 5 * H,
                  NMODL);
    f2.p[0].gate_L = 1;
    half_w(f2.p[0]);
    next_ln(r, next, kinds, 1);
    return resid_ln(f2, r, H, s.ln_eps);
}

// H-wide sinusoid -> GEMV + SiLU -> GEMV + b + gcmlp = global_c, gs = silu(global_c)
// (src/dit_fwd.cpp:111-140), then every clip/text modulation in one HBM-bound GEMV
// (src/dit_fwd.cpp:195-207). Rows in GEMV batches of up to 16; gcmlp row r is gcmlp[r % 16]
// (callers pass B rows for B <= 16, or the 16-row repetition).
int RefDitModel::enqueue_conditioning(const float *t, int rows, const float *gcmlp, float *temb, float *h1, float *gc,
                                      float *gs, float *modg) {
    const hipStream_t st = rt->dev.stream();
    const int H = s.H;
    TSN_TRY(run("temb_kernel", 0, 0, [&] { return launch_temb_sinusoid(t, temb, rows, H, s.t_max_period, st); }));
    for (int r0 = 0; r0 < rows; r0 += 16) {
        const int rem = rows - r0;
        const int nb = rem >= 16 ? 16 : rem > 8 ? 16 : rem > 4 ? 8 : rem > 2 ? 4 : rem;   // rows past `rows` are padding
        GemvArgs g1;
        memset(&g1, 0, sizeof g1);
        g1.W = Wt0_; g1.ldw = H; g1.wdt = DT_F16; g1.X = temb + (size_t)r0 * H; g1.ldx = H;
        g1.Y = h1 + (size_t)r0 * H; g1.ldy = H; g1.bias = bt0_; g1.N = H; g1.K = H; g1.nb = nb; g1.silu = 1;
        TSN_TRY(run(K_GEMV, 2.0 * nb * H * H, 2.0 * H * H, [&] { return launch_gemv(g1, st); }));
        GemvArgs g2;
        memset(&g2, 0, sizeof g2);
        g2.W = Wt2_; g2.ldw = H; g2.wdt = DT_F16; g2.X = h1 + (size_t)r0 * H; g2.ldx = H;
        g2.Y = gc + (size_t)r0 * H; g2.ldy = H; g2.bias = bt2_; g2.addv = gcmlp; g2.ld_add = H;
        g2.Y2 = gs + (size_t)r0 * H; g2.ldy2 = H; g2.N = H; g2.K = H; g2.nb = nb;
        TSN_TRY(run(K_GEMV, 2.0 * nb * H * H, 2.0 * H * H, [&] { return launch_gemv(g2, st); }));
        if (s.n_joint == 0) continue;
        GemvArgs m;
        memset(&m, 0, sizeof m);
        m.W = WmodG_; m.ldw = H; m.wdt = DT_F16;
        m.X = gs + (size_t)r0 * H; m.ldx = H;
        m.Y = modg + (size_t)r0 * NMODG; m.ldy = NMODG;
        m.bias = bmodG_; m.N = NMODG; m.K = H; m.nb = nb;
        TSN_TRY(run(K_GEMV, 2.0 * nb * (double)NMODG * H, 2.0 * (double)NMODG * H + 4.0 * nb * NMODG,
                    [&] { return launch_gemv(m, st); }));
    }
    return TSN_OK;
}

int RefDitModel::enqueue_forward(const float *x, const float *t, const float *clip_pp, const float *text_pp,
                                 const float *gcmlp, const float *sync_gather, float *v, float *taps) {
    return enqueue_eval(x, t, clip_pp, text_pp, gcmlp, sync_gather, v, taps, nullptr, nullptr);
}

// One evaluation. gc_pre / modg_pre: this evaluation's global_c rows and clip/text modulation,
// computed beforehand (the sampler); null: computed here from t and gcmlp.
int RefDitModel::enqueue_eval(const float *x, const float *t, const float *clip_pp, const float *text_pp,
                              const float *gcmlp, const float *sync_gather, float *v, float *taps, const float *gc_pre,
                              const float *modg_pre) {
    TSN_REQUIRE(ready_, "refdit: weights not uploaded");
    TSN_REQUIRE(x && (t || gc_pre) && (gcmlp || gc_pre) && sync_gather && v, "refdit forward: null input");
    TSN_REQUIRE((clip_pp || s.C == 0) && (text_pp || s.TS == 0), "refdit forward: null clip/text input");
    TSN_TRY(rt->dev.make_current());
    const hipStream_t st = rt->dev.stream();
    const int B = s.B, H = s.H, T = s.T, L = s.latent;
    const float *gc = gc_pre;
    if (gc_pre) {
        modg_ = modg_pre;
    } else {
        TSN_TRY(enqueue_conditioning(t, B, gcmlp, temb_, h1_, gc_, gs_, MODG_));
        gc = gc_;
        modg_ = MODG_;
    }
    // extended_c = sync_gather + global_c per row, SiLU, as f16 hi|lo; then every per-row modulation
    // (latent and fused blocks, final layer) in one GEMM with M = B*T against [W | W], f32-accurate
    // in the operand (src/dit_fwd.cpp:133-136,186-189,271-274,288-291)
    TSN_TRY(run("bcast_add_silu_kernel", 0, 12.0 * B * T * (double)H,
                [&] { return launch_bcast_add_silu_f16(sync_gather, gc, XE_, T, B * T, H, st); }));
    {
        GemmBatch mb;
        mb.nprob = 1;
        GemmProblem &p = mb.p[0];
        gemm_problem_init(p);
        p.A = XE_; p.lda = 2 * H; p.amap = rowmap_dense(B * T); p.taps = 1; p.Kc = 2 * H; p.a_T = B * T;
        p.W = WmodL_; p.bias = bmodL_; p.M = B * T; p.N = NMODL; p.K = 2 * H;
        p.Y = MODL_; p.ldy = NMODL; p.ymap = rowmap_dense(B * T); p.y_f16 = 0;
        half_w(p);
        mb.ws = ws_;
        mb.ws_bytes = ws_bytes_;
        TSN_TRY(gemm_run(mb, EPI_STORE));
    }
    // input projection (src/dit_fwd.cpp:142-149): conv k3 over x as f16 hi|lo against [W|W]
    // (f32-accurate) + b, SiLU -> SwiGLU conv k3 (w1|w3 in one GEMM) -> conv k3 w2 into the
    // latent rows of X, every operand f16 hi|lo
    const RowMap D{T, T, 0};   // dense rows, sample boundaries every T rows (conv zero padding)
    TSN_TRY(run(K_SPLIT, 0, 8.0 * B * T * L, [&] { return launch_split_hilo(x, L, rowmap_dense(B * T), Z2_, B * T, L, st); }));
    {
        GemmBatch ib;
        ib.nprob = 1;
        store_problem(ib.p[0], Z2_, 2 * L, D, 3, 2 * L, B * T, H, Win_, XN_, 2 * H, 1);
        ib.p[0].bias = bin_;
        ib.p[0].y_lo = H;
        half_w(ib.p[0]);
        ib.ws = ws_;
        ib.ws_bytes = ws_bytes_;
        TSN_TRY(gemm_run(ib, EPI_STORE));
        GemmBatch sb;
        sb.nprob = 1;
        store_problem(sb.p[0], XN_, 2 * H, D, 3, 2 * H, B * T, 2 * s.F, W13in_, HF_, 2 * s.F, 0);
        sb.p[0].y_lo = s.F;
        half_w(sb.p[0]);
        sb.ws = ws_;
        sb.ws_bytes = ws_bytes_;
        TSN_TRY(gemm_run(sb, EPI_SWIGLU));
        GemmBatch ob;
        ob.nprob = 1;
        ob.ws = ws_;
        ob.ws_bytes = ws_bytes_;
        store_problem(ob.p[0], HF_, 2 * s.F, D, 3, 2 * s.F, B * T, H, W2in_, nullptr, 0, 0);
        ob.p[0].Y = X_; ob.p[0].ldy = H; ob.p[0].ymap = stream_map(ST_LAT); ob.p[0].y_f16 = 0;
        half_w(ob.p[0]);
        TSN_TRY(gemm_run(ob, EPI_STORE));
    }
    // clip and text streams start from the prepared features every evaluation (src/dit_fwd.cpp:162-163)
    if (s.C > 0)
        TSN_TRY(run("copy_rows_kernel", 0, 8.0 * B * s.C * (double)H, [&] {
            return launch_copy_rows(clip_pp, H, rowmap_dense(B * s.C), X_, H, stream_map(ST_CLIP), B * s.C, H, st);
        }));
    if (s.TS > 0)
        TSN_TRY(run("copy_rows_kernel", 0, 8.0 * B * s.TS * (double)H, [&] {
            return launch_copy_rows(text_pp, H, rowmap_dense(B * s.TS), X_, H, stream_map(ST_TEXT), B * s.TS, H, st);
        }));
    const size_t tap_n = (size_t)B * S * H;
    int tap = 0;
    const int nblk = s.n_joint + s.n_fused;
    for (int k = 0; k < nblk; ++k) {
        const Next next = k + 1 == nblk ? Next{NEXT_FINAL, 0}
                          : k + 1 < s.n_joint ? Next{NEXT_JOINT, k + 1}
                                              : Next{NEXT_FUSED, k + 1 - s.n_joint};
        if (k < s.n_joint) TSN_TRY(block_joint(k, k == 0, next));
        else TSN_TRY(block_fused(k - s.n_joint, k == 0, next));
        if (taps) TSN_TRY(rt->dev.copy_d2d(taps + tap_n * tap++, X_, tap_n * 4));
    }
    // final layer (src/dit_fwd.cpp:287-303): per-row adaLN (2 chunks) as f16 hi|lo, conv k7 pad 3
    // + b against [W|W] (f32-accurate), split over K
    if (nblk == 0) {
        LnArgs ln;
        memset(&ln, 0, sizeof ln);
        ln.nseg = 1; ln.H = H; ln.eps = s.ln_eps;
        LnSeg &g = ln.seg[0];
        g.X = X_; g.ldx = H; g.xmap = stream_map(ST_LAT);
        g.Y = XF2_; g.ldy = 2 * H; g.ymap = D;
        g.mod = MODL_; g.mod_ld = NMODL; g.mod_L = 1; g.shift_off = fin_off_; g.scale_off = fin_off_ + H;
        g.rows = B * T;
        TSN_TRY(run(K_LNHL, 0, B * T * (double)H * 8.0, [&] { return launch_ln_mod(ln, LN_F16_HILO, st); }));
    }
    GemmBatch fb;
    fb.nprob = 1;
    fb.ws = ws_;
    fb.ws_bytes = ws_bytes_;
    store_problem(fb.p[0], XF2_, 2 * H, D, 7, 2 * H, B * T, L, Wfin_, nullptr, 0, 0);
    fb.p[0].bias = bfin_;
    fb.p[0].Y = v; fb.p[0].ldy = L; fb.p[0].ymap = D; fb.p[0].y_f16 = 0;
    half_w(fb.p[0]);
    return gemm_run(fb, EPI_STORE);
}

// src/pipeline.cpp:141-155: t_s = 1 - s/steps, dt = t_{s+1} - t_s, two arms then cfg_euler
int RefDitModel::enqueue_sample(float *x, const float *clip_pp, const float *text_pp, const float *gcmlp,
                                const float *sync_gather, int steps, float cfg) {
    TSN_REQUIRE(ready_, "refdit: weights not uploaded");
    TSN_REQUIRE(x && gcmlp && sync_gather && (clip_pp || s.C == 0) && (text_pp || s.TS == 0) && steps > 0,
                "refdit sample: arguments");
    TSN_REQUIRE(s.B % 2 == 0, "refdit sample: B must be even (cond/uncond pairs)");
    TSN_REQUIRE(tsched_ && tsched_steps_ == steps && cond_, "refdit sample: schedule not prepared for this step count");
    const int P = s.B / 2;
    const size_t n = (size_t)s.T * s.latent;
    const hipStream_t st = rt->dev.stream();
    for (int b = 0; b < s.B; ++b) TSN_TRY(rt->dev.copy_d2d(x2_ + b * n, x + (b / 2) * n, n * 4));
    // global_c and the clip/text modulation depend on t only: every step's in one pass over the
    // weights per 16 rows, before the step loop (row st*B + b = step st, sample b)
    TSN_TRY(launch_copy_rows(gcmlp, s.H, RowMap{s.B, 0, 0}, gcmlp_rep_, s.H, rowmap_dense(16), 16, s.H, st));
    TSN_TRY(enqueue_conditioning(tsched_, steps * s.B, gcmlp_rep_, temb_all_, h1_all_, gc_all_, gs_all_, modg_all_));
    for (int k = 0; k < steps; ++k) {
        const float t_curr = 1.0f - (float)k / (float)steps;
        const float t_prev = 1.0f - (float)(k + 1) / (float)steps;
        TSN_TRY(enqueue_eval(x2_, nullptr, clip_pp, text_pp, nullptr, sync_gather, Vv_, nullptr,
                             gc_all_ + (size_t)k * s.B * s.H, modg_all_ + (size_t)k * s.B * NMODG));
        TSN_TRY(launch_cfg_euler_pairs(Vv_, x2_, P, (int)n, cfg, t_prev - t_curr, st));
    }
    for (int p = 0; p < P; ++p) TSN_TRY(rt->dev.copy_d2d(x + p * n, x2_ + 2 * p * n, n * 4));
    return TSN_OK;
}

int RefDitModel::prepare_sample(int steps) {
    TSN_REQUIRE(steps > 0, "refdit sample: steps must be positive");
    TSN_REQUIRE(s.B <= 16 && 16 % s.B == 0, "refdit sample: B must divide 16");
    TSN_TRY(rt->dev.make_current());
    if (tsched_ && tsched_steps_ == steps && cond_) return TSN_OK;
    if (tsched_) TSN_TRY(release(tsched_));
    tsched_ = nullptr;
    std::vector<float> h((size_t)steps * s.B);
    for (int k = 0; k < steps; ++k)
        for (int b = 0; b < s.B; ++b) h[(size_t)k * s.B + b] = 1.0f - (float)k / (float)steps;
    TSN_TRY(alloc(h.size() * 4, (void **)&tsched_));
    TSN_TRY(rt->dev.upload(tsched_, h.data(), h.size() * 4));
    tsched_steps_ = steps;
    if (cond_) TSN_TRY(release(cond_));
    cond_ = nullptr;
    const size_t R = ((size_t)steps * s.B + 15) / 16 * 16, H = s.H;
    const size_t n_h = R * H, n_mod = R * (size_t)NMODG, n_rep = 16 * H;
    TSN_TRY(alloc((4 * n_h + n_mod + n_rep) * sizeof(float), (void **)&cond_));   // zero-filled
    temb_all_ = cond_;
    h1_all_ = temb_all_ + n_h;
    gc_all_ = h1_all_ + n_h;
    gs_all_ = gc_all_ + n_h;
    modg_all_ = gs_all_ + n_h;
    gcmlp_rep_ = modg_all_ + n_mod;
    return TSN_OK;
}

int RefDitModel::capture_forward(const float *x, const float *t, const float *clip_pp, const float *text_pp,
                                 const float *gcmlp, const float *sync_gather, float *v) {
    TSN_REQUIRE(ready_, "refdit: weights not uploaded");
    return capture([&] { return enqueue_forward(x, t, clip_pp, text_pp, gcmlp, sync_gather, v, nullptr); });
}

int RefDitModel::capture_sample(float *x, const float *clip_pp, const float *text_pp, const float *gcmlp,
                                const float *sync_gather, int steps, float cfg) {
    TSN_REQUIRE(ready_, "refdit: weights not uploaded");
    TSN_TRY(prepare_sample(steps));
    return capture([&] { return enqueue_sample(x, clip_pp, text_pp, gcmlp, sync_gather, steps, cfg); });
}

int RefDitModel::profile_forward(const float *x, const float *t, const float *clip_pp, const float *text_pp,
                                 const float *gcmlp, const float *sync_gather, float *v, std::vector<KernelStat> &stats) {
    return profile([&] { return enqueue_forward(x, t, clip_pp, text_pp, gcmlp, sync_gather, v, nullptr); }, stats);
}

} // namespace tsn
