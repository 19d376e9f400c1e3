// dit.cpp — DitModel on HIP: weight upload, one velocity evaluation, the CFG Euler sampler.
//
// Per evaluation (B samples folded into GEMM rows; src/dit_fwd.cpp:104-304 for the reference
// sequence):
//   1 sinusoid -> 2 GEMVs (t-MLP; + pooled -> g, silu(g)) -> 1 GEMV for every adaLN modulation
//   input projection (f32) + text rows copy
//   per joint block: LN(both streams) | QKV (2 problems; RMS+RoPE epilogue) | flash attention |
//                    out-proj (2 problems; gated residual) | LN | FFN1 (conv k3 + linear; SiLU) |
//                    FFN2 (conv k3 + linear; gated residual)                        = 7 launches
//   per fused block: the same 7 launches with one problem each
//   final LN (f32 out) + output projection (f32)
#include "dit.h"

#include <math.h>
#include <string.h>

#include <map>

namespace tsn {

std::vector<ManifestEntry> dit_manifest(const DitSpec &s) {
    std::vector<ManifestEntry> v;
    const int64_t H = s.H, F = s.F, HD = s.HD;
    int64_t off = 0;
    auto add = [&](const std::string &n, int64_t numel) {
        v.push_back({n, numel, off});
        off += numel;
    };
    add("t_embed.mlp.0.weight", H * s.temb_dim);
    add("t_embed.mlp.0.bias", H);
    add("t_embed.mlp.2.weight", H * H);
    add("t_embed.mlp.2.bias", H);
    add("audio_input_proj.weight", H * s.latent);
    add("audio_input_proj.bias", H);
    auto block = [&](const std::string &p, int64_t taps) {
        add(p + ".adaLN_modulation.1.weight", 6 * H * H);
        add(p + ".adaLN_modulation.1.bias", 6 * H);
        add(p + ".attn.qkv.weight", 3 * H * H);
        add(p + ".attn.qkv.bias", 3 * H);
        add(p + ".attn.q_norm.weight", HD);
        add(p + ".attn.k_norm.weight", HD);
        add(p + ".linear1.weight", H * H);
        add(p + ".linear1.bias", H);
        add(p + ".ffn.w1.weight", F * H * taps);
        add(p + ".ffn.w2.weight", H * F * taps);
    };
    for (int i = 0; i < s.n_joint; ++i) {
        block("joint_blocks." + std::to_string(i) + ".latent_block", s.audio_ffn_conv ? 3 : 1);
        block("joint_blocks." + std::to_string(i) + ".text_block", 1);
    }
    for (int i = 0; i < s.n_fused; ++i) block("fused_blocks." + std::to_string(i), 1);
    add("final_layer.adaLN_modulation.1.weight", 2 * H * H);
    add("final_layer.adaLN_modulation.1.bias", 2 * H);
    add("final_layer.linear.weight", (int64_t)s.latent * H);
    add("final_layer.linear.bias", s.latent);
    return v;
}

int dit_spec_check(const DitSpec &s) {
    TSN_REQUIRE(s.B == 1 || s.B == 2 || s.B == 4 || s.B == 8 || s.B == 16, "spec: B must be 1, 2, 4, 8 or 16");
    TSN_REQUIRE(s.La > 0 && s.Lt >= 0, "spec: La > 0, Lt >= 0");
    TSN_REQUIRE(s.HD == 64, "spec: head dim must be 64");
    TSN_REQUIRE(s.H == s.NH * s.HD && s.H % 256 == 0 && s.H <= 2048, "spec: H = NH*64, multiple of 256, <= 2048");
    TSN_REQUIRE(s.F % 128 == 0 && s.F > 0, "spec: F must be a multiple of 128");
    TSN_REQUIRE(s.latent > 0 && s.latent % 8 == 0, "spec: latent must be a multiple of 8");
    TSN_REQUIRE(s.temb_dim > 0 && s.temb_dim % 8 == 0, "spec: temb_dim must be a multiple of 8");
    TSN_REQUIRE(s.n_joint >= 0 && s.n_fused >= 0, "spec: block counts");
    TSN_REQUIRE(s.Lt > 0 || s.n_joint == 0, "spec: joint blocks need text rows");
    return TSN_OK;
}

int DitModel::create(Runtime *r, const DitSpec &sp) {
    TSN_REQUIRE(r, "dit: null runtime");
    TSN_TRY(dit_spec_check(sp));
    rt = r;
    s = sp;
    S = s.La + s.Lt;
    Sp = (S + 63) / 64 * 64;
    NMOD = (2 * s.n_joint + s.n_fused) * 6 * s.H + 2 * s.H;
    const size_t B = s.B, H = s.H;
    auto af = [&](float **p, size_t n) { return alloc(n * sizeof(float), (void **)p); };
    auto ah = [&](half_t **p, size_t n) { return alloc(n * sizeof(half_t), (void **)p); };
    TSN_TRY(af(&X_, B * S * H));
    TSN_TRY(af(&MOD_, B * NMOD));
    TSN_TRY(af(&g_, B * H));
    TSN_TRY(af(&gs_, B * H));
    TSN_TRY(af(&temb_, B * s.temb_dim));
    TSN_TRY(af(&h1_, B * H));
    TSN_TRY(ah(&XF2_, B * s.La * 2 * H));
    TSN_TRY(ah(&Z2_, B * s.La * 2 * (size_t)s.latent));
    TSN_TRY(af(&Vv_, B * s.La * s.latent));
    TSN_TRY(af(&x2_, B * s.La * s.latent));
    TSN_TRY(af(&t_dev, B));
    TSN_TRY(ah(&XN_, B * S * H));
    TSN_TRY(ah(&Q_, B * S * H));
    TSN_TRY(ah(&K_, B * S * H));
    TSN_TRY(ah(&Vt_, B * s.NH * 64 * (size_t)Sp));   // zero-filled: keys >= S stay zero
    TSN_TRY(ah(&AO_, B * S * H));
    TSN_TRY(ah(&HF_, B * S * (size_t)s.F));
    // split-K partials: up to 8 splits of the largest residual GEMM output (B*S x H f32)
    ws_bytes_ = (size_t)8 * B * S * H * sizeof(float);
    TSN_TRY(alloc(ws_bytes_, (void **)&ws_));
    TSN_TRY(alloc_skcnt());
    // RoPE table: same expression as shaders/ops_conv.metal:162-164 with fscale 1 (audio rows)
    std::vector<float> tab((size_t)s.La * 32 * 2);
    for (int p = 0; p < s.La; ++p)
        for (int j = 0; j < 32; ++j) {
            const float inv = powf(s.rope_theta, -2.0f * (float)j / (float)s.HD);
            const float ang = (float)p * 1.0f * inv;
            tab[((size_t)p * 32 + j) * 2] = cosf(ang);
            tab[((size_t)p * 32 + j) * 2 + 1] = sinf(ang);
        }
    TSN_TRY(af(&rope_, tab.size()));
    TSN_TRY(rt->dev.upload(rope_, tab.data(), tab.size() * sizeof(float)));
    return TSN_OK;
}

int DitModel::upload_weights(const uint16_t *host, size_t numel) {
    TSN_REQUIRE(rt && host, "dit: not created / null weights");
    const auto man = dit_manifest(s);
    const size_t total = (size_t)(man.back().offset + man.back().numel);
    TSN_REQUIRE(numel == total, "dit: weight count does not match the manifest (" + std::to_string(total) + ")");
    TSN_TRY(alloc(total * 2, &wraw_));
    TSN_TRY(rt->dev.upload(wraw_, host, total * 2));
    std::map<std::string, const ManifestEntry *> idx;
    for (const auto &e : man) idx[e.name] = &e;
    const hipStream_t st = rt->dev.stream();
    auto raw = [&](const std::string &n) -> const uint16_t * {
        return (const uint16_t *)wraw_ + idx.at(n)->offset;
    };
    auto numel_of = [&](const std::string &n) { return (size_t)idx.at(n)->numel; };
    auto f16 = [&](const std::string &n, const half_t **out) -> int {
        half_t *p;
        TSN_TRY(alloc(numel_of(n) * 2, (void **)&p));
        TSN_TRY(launch_bf16_to_f16(raw(n), p, numel_of(n), st));
        *out = p;
        return TSN_OK;
    };
    auto f32 = [&](const std::string &n, const float **out) -> int {
        float *p;
        TSN_TRY(alloc(numel_of(n) * 4, (void **)&p));
        TSN_TRY(launch_bf16_to_f32(raw(n), p, numel_of(n), st));
        *out = p;
        return TSN_OK;
    };
    auto convw = [&](const std::string &n, int OC, int IC, const half_t **out) -> int {
        half_t *p;
        TSN_TRY(alloc(numel_of(n) * 2, (void **)&p));
        TSN_TRY(launch_conv_weight_reorder(raw(n), 1, p, OC, IC, 3, st));
        *out = p;
        return TSN_OK;
    };
    const size_t H = s.H;
    uint16_t *wmod;
    TSN_TRY(alloc((size_t)NMOD * H * 2, (void **)&wmod));
    float *bmod;
    TSN_TRY(alloc((size_t)NMOD * 4, (void **)&bmod));
    int mod_row = 0;
    auto stream = [&](const std::string &p, bool conv, StreamW &w) -> int {
        w.mod_off = mod_row;
        TSN_TRY(rt->dev.copy_d2d(wmod + (size_t)mod_row * H, raw(p + ".adaLN_modulation.1.weight"), 6 * H * H * 2));
        TSN_TRY(launch_bf16_to_f32(raw(p + ".adaLN_modulation.1.bias"), bmod + mod_row, 6 * H, st));
        mod_row += 6 * (int)H;
        TSN_TRY(f16(p + ".attn.qkv.weight", &w.Wqkv));
        TSN_TRY(f32(p + ".attn.qkv.bias", &w.bqkv));
        TSN_TRY(f32(p + ".attn.q_norm.weight", &w.qn));
        TSN_TRY(f32(p + ".attn.k_norm.weight", &w.kn));
        TSN_TRY(f16(p + ".linear1.weight", &w.Wo));
        TSN_TRY(f32(p + ".linear1.bias", &w.bo));
        w.conv = conv ? 1 : 0;
        if (conv) {
            TSN_TRY(convw(p + ".ffn.w1.weight", s.F, s.H, &w.W1));
            TSN_TRY(convw(p + ".ffn.w2.weight", s.H, s.F, &w.W2));
        } else {
            TSN_TRY(f16(p + ".ffn.w1.weight", &w.W1));
            TSN_TRY(f16(p + ".ffn.w2.weight", &w.W2));
        }
        return TSN_OK;
    };
    ja_.assign(s.n_joint, StreamW{});
    jt_.assign(s.n_joint, StreamW{});
    fu_.assign(s.n_fused, StreamW{});
    for (int i = 0; i < s.n_joint; ++i) {
        TSN_TRY(stream("joint_blocks." + std::to_string(i) + ".latent_block", s.audio_ffn_conv != 0, ja_[i]));
        TSN_TRY(stream("joint_blocks." + std::to_string(i) + ".text_block", false, jt_[i]));
    }
    for (int i = 0; i < s.n_fused; ++i) TSN_TRY(stream("fused_blocks." + std::to_string(i), false, fu_[i]));
    fin_mod_off_ = mod_row;
    TSN_TRY(rt->dev.copy_d2d(wmod + (size_t)mod_row * H, raw("final_layer.adaLN_modulation.1.weight"), 2 * H * H * 2));
    TSN_TRY(launch_bf16_to_f32(raw("final_layer.adaLN_modulation.1.bias"), bmod + mod_row, 2 * H, st));
    Wmod_ = wmod;
    bmod_ = bmod;
    // GEMV / f32-linear weights are read as bf16 straight from the uploaded buffer
    Wt0_ = raw("t_embed.mlp.0.weight");
    Wt2_ = raw("t_embed.mlp.2.weight");
    {
        half_t *w;
        TSN_TRY(alloc((size_t)H * 2 * s.latent * 2, (void **)&w));
        TSN_TRY(launch_dup_cols_bf16_to_f16(raw("audio_input_proj.weight"), w, (int)H, s.latent, st));
        Win2_ = w;
        TSN_TRY(alloc((size_t)s.latent * 2 * H * 2, (void **)&w));
        TSN_TRY(launch_dup_cols_bf16_to_f16(raw("final_layer.linear.weight"), w, s.latent, (int)H, st));
        Wfin2_ = w;
    }
    TSN_TRY(f32("t_embed.mlp.0.bias", &bt0_));
    TSN_TRY(f32("t_embed.mlp.2.bias", &bt2_));
    TSN_TRY(f32("audio_input_proj.bias", &bin_));
    TSN_TRY(f32("final_layer.linear.bias", &bfin_));
    TSN_TRY(rt->dev.sync());
    ready_ = true;
    return TSN_OK;
}

GemvArgs DitModel::mod_args(const float *gs, int row0, int rows) const {
    GemvArgs a;
    memset(&a, 0, sizeof a);
    a.W = Wmod_ + (size_t)row0 * s.H; a.ldw = s.H; a.wdt = DT_BF16;
    a.X = gs; a.ldx = s.H;
    a.Y = MOD_ + row0; a.ldy = NMOD;
    a.bias = bmod_ + row0;
    a.N = rows; a.K = s.H; a.nb = s.B;
    return a;
}

int DitModel::modulation(const float *gs, int row0, int rows) {
    return launch_gemv(mod_args(gs, row0, rows), rt->dev.stream());
}

bool DitModel::mod_grid_ok() const {
    if (s.B != 2 || s.H != 1024 || s.n_joint + s.n_fused == 0) return false;
    const int tn = 3 * s.H / 128, spare = 32, ncu = 256;   // 128x128 QKV tiles
    const int tj = ((s.B * s.La + 127) / 128 + (s.B * s.Lt + 127) / 128) * tn;
    const int tf = (s.B * S + 127) / 128 * tn;
    return (s.n_joint == 0 || tj <= ncu - spare) && (s.n_fused == 0 || tf <= ncu - spare);
}

// block 0's rows: both streams of joint block 0 (audio then text, adjacent), or fused block 0's
int DitModel::first_mod_rows() const {
    return s.n_joint > 0 ? jt_[0].mod_off + 6 * s.H : fu_[0].mod_off + 6 * s.H;
}

void DitModel::next_mod_gemv(GemmBatch &qb, Next next) const {
    if (!mod_in_grid_) return;
    int row0 = 0, rows = 0;
    switch (next.kind) {
        case NEXT_JOINT: row0 = ja_[next.idx].mod_off; rows = jt_[next.idx].mod_off + 6 * s.H - row0; break;
        case NEXT_FUSED: row0 = fu_[next.idx].mod_off; rows = 6 * s.H; break;
        case NEXT_FINAL: row0 = fin_mod_off_; rows = 2 * s.H; break;
        default: return;
    }
    qb.gv = mod_args(gs_, row0, rows);
}

int DitModel::gs_from_g(const float *g) {
    const hipStream_t st = rt->dev.stream();
    TSN_TRY(launch_copy(g, gs_, (size_t)s.B * s.H, st));
    return launch_silu(gs_, (size_t)s.B * s.H, st);
}

// Fill the LN part of r's segments (one per row map of the residual GEMM) for the adaLN that
// runs next: LN1 of a joint or fused block (f16 into XN), or the final layer's (f16 hi|lo of the
// audio rows into XF2).
void DitModel::next_ln(RedLnArgs &r, Next next, const RowMap *maps, int nseg) {
    memset(&r, 0, sizeof r);
    r.ymode = next.kind == NEXT_FINAL ? LN_F16_HILO : LN_F16;
    for (int i = 0; i < nseg; ++i) {
        RedLnSeg &g = r.seg[i];
        const RowMap &m = maps[i];
        const bool text = m.off >= s.La;   // rows of the text stream inside the joint layout
        g.mod = mod_; g.mod_ld = NMOD; g.mod_L = m.L; g.ln_len = m.L;
        g.Y = XN_; g.ldy = s.H; g.ymap = m;
        switch (next.kind) {
        case NEXT_JOINT: g.ln = 1; g.shift_off = (text ? jt_ : ja_)[next.idx].mod_off; break;
        case NEXT_FUSED: g.ln = 1; g.shift_off = fu_[next.idx].mod_off; break;
        case NEXT_FINAL:
            g.ln = text || final_fused() ? 0 : 1;   // the fused final kernel normalises its own rows
            g.shift_off = fin_mod_off_;
            g.ln_len = m.L < s.La ? m.L : s.La;
            g.Y = XF2_; g.ldy = 2 * s.H; g.ymap = RowMap{m.L, s.La, 0};   // audio row t of sample b -> b*La + t
            break;
        default: g.ln = 0; break;
        }
        g.scale_off = g.shift_off + s.H;
    }
}

// Weight prefetch from the LN kernels (PfRange): only when the LN kernel is long enough to hide
// the extra workgroups' line fetches, i.e. at 4096 rows and more (batch 16 at 8 s: 7.56 -> 7.38 ms
// per evaluation; at 794 rows (8 s, batch 2) and 2202 rows (30 s) the LN kernels lengthened by more
// than the GEMMs gained).
bool DitModel::ln_prefetch() const { return (long long)s.B * S >= 4096; }
// FFN1's and the next QKV's weights from the spare CUs of the out-projection and FFN2 grids: above
// 1024 rows, where those grids run two workgroups per CU with free slots (30 s: 3.978 -> 3.909 ms).
// At 794 rows (8 s) the out-projection's small tiles share their CUs with the prefetch and FFN2's
// single round leaves 16 CUs for it: 8 s 1.871 -> 1.886 ms, so not there.
bool DitModel::grid_prefetch() const { return (long long)s.B * S > 1024 && !ln_prefetch(); }

// The next block's QKV weights: touched by the reduce + LN kernel that runs before that GEMM, or
// by the FFN2 GEMM's spare CUs (ln_prefetch, grid_prefetch).
void DitModel::next_qkv_prefetch(RedLnArgs &r, GemmBatch &f2, Next next) const {
    if (!ln_prefetch() && !grid_prefetch()) return;
    PfRange (&pf)[PF_RANGES] = ln_prefetch() ? r.pf : f2.pf;
    if (next.kind == NEXT_JOINT) {
        pf[0] = PfRange{ja_[next.idx].Wqkv, 3 * s.H, 2 * s.H, 2LL * s.H};
        pf[1] = PfRange{jt_[next.idx].Wqkv, 3 * s.H, 2 * s.H, 2LL * s.H};
    } else if (next.kind == NEXT_FUSED) {
        pf[0] = PfRange{fu_[next.idx].Wqkv, 3 * s.H, 2 * s.H, 2LL * s.H};
    }
}

// Joint block: src/dit_fwd.cpp:180-257 (pre_attn :24-49, attention :83-102, post_attn :51-81)
int DitModel::block_joint(int i, bool ln1, Next next) {
    const hipStream_t st = rt->dev.stream();
    const StreamW &a = ja_[i], &t = jt_[i];
    const int B = s.B, H = s.H, La = s.La, Lt = s.Lt;
    const RowMap Sa{La, S, 0}, St{Lt, S, La};
    const RowMap maps[2] = {Sa, St};
    if (ln1) {   // otherwise the previous block's last reduce kernel produced it
        LnArgs ln;
        memset(&ln, 0, sizeof ln);
        ln.nseg = 2; ln.H = H; ln.eps = s.ln_eps;
        ln_seg(ln.seg[0], X_, H, Sa, XN_, mod_, NMOD, La, a.mod_off, B * La);
        ln_seg(ln.seg[1], X_, H, St, XN_, mod_, NMOD, Lt, t.mod_off, B * Lt);
        TSN_TRY(run(K_LN16, 0, ln_bytes(ln, true), [&] { return launch_ln_mod(ln, LN_F16, st); }));
    }

    GemmBatch qb;
    qb.nprob = 2;
    qkv_problem(qb.p[0], XN_, Sa, B * La, a.Wqkv, a.bqkv, a.qn, a.kn, H, s.NH, Q_, K_, Vt_, S, Sp, La, 0, La, rope_, s.rms_eps);
    qkv_problem(qb.p[1], XN_, St, B * Lt, t.Wqkv, t.bqkv, t.qn, t.kn, H, s.NH, Q_, K_, Vt_, S, Sp, Lt, La, 0, rope_, s.rms_eps);
    qb.pf[0] = PfRange{a.Wo, H, H * 2, (long long)H * 2};   // the out-projection's weights
    qb.pf[1] = PfRange{t.Wo, H, H * 2, (long long)H * 2};
    if (!ln_prefetch() && !grid_prefetch()) {   // and FFN1's (first tap of the conv), read three launches later
        qb.pf[2] = PfRange{a.W1, s.F, H * 2, (long long)(a.conv ? 3 : 1) * H * 2};
        qb.pf[3] = PfRange{t.W1, s.F, H * 2, (long long)H * 2};
    }
    next_mod_gemv(qb, next);
    TSN_TRY(gemm_run(qb, EPI_QKV));

    AttnArgs at;
    memset(&at, 0, sizeof at);
    at.Q = Q_; at.K = K_; at.Vt = Vt_; at.S = S; at.Sp = Sp; at.nh = s.NH; at.BH = B * s.NH;
    at.O = AO_; at.o_f32 = 0; at.ldo = H; at.omap = rowmap_dense(B * S);
    TSN_TRY(run(K_ATTN, 4.0 * B * s.NH * (double)S * S * 64, 8.0 * B * (double)S * H,
                [&] { return launch_attention(at, st); }));

    GemmBatch ob;
    ob.nprob = 2;
    ob.small = 1;   // 64x64 tiles over the full K while 128x128 tiles would fill under one round
    ob.ws = ws_;
    ob.ws_bytes = ws_bytes_;
    resid_problem(ob.p[0], AO_, H, Sa, 1, H, B * La, H, a.Wo, a.bo, X_, H, mod_ + a.mod_off + 2 * H, NMOD);
    resid_problem(ob.p[1], AO_, H, St, 1, H, B * Lt, H, t.Wo, t.bo, X_, H, mod_ + t.mod_off + 2 * H, NMOD);
    const int ta = a.conv ? 3 : 1;
    RedLnArgs r;
    next_ln(r, Next{NEXT_JOINT, i}, maps, 2);   // LN2 of this block: modulation chunks 3, 4
    r.seg[0].shift_off += 3 * H; r.seg[0].scale_off += 3 * H;
    r.seg[1].shift_off += 3 * H; r.seg[1].scale_off += 3 * H;
    if (ln_prefetch() || grid_prefetch()) {   // FFN1's weights, read next (the audio conv's first
        // tap: the first third of its K), from the LN kernel or from the out-projection's spare CUs
        PfRange (&pf)[PF_RANGES] = ln_prefetch() ? r.pf : ob.pf;
        pf[0] = PfRange{a.W1, s.F, H * 2, (long long)ta * H * 2};
        pf[1] = PfRange{t.W1, s.F, H * 2, (long long)H * 2};
    }
    TSN_TRY(resid_ln(ob, r, s.H, s.ln_eps));

    // Two launches instead of one batch when the batch is larger than one round of 128x128 tiles:
    // the audio conv (K = 3 x H) then no longer shares the two-stage kernel's CUs with the text
    // linear (K = H), and when it fills a round of 256x256 tiles with K >= 2048 (batch 16) it takes
    // the wide kernel. Same box: 30 s 3.869 -> 3.738 ms, batch 16 7.071 -> 6.796 ms; the 8 s batch
    // (224 tiles) stays one launch
    const bool wide_audio = (B * La + 255) / 256 * ((s.F + 255) / 256) >= 256 && ta * H >= 2048;
    const int t128 = ((B * La + 127) / 128 + (B * Lt + 127) / 128) * ((s.F + 127) / 128);
    if (wide_audio || t128 > 256) {
        GemmBatch fa;
        fa.nprob = 1;
        store_problem(fa.p[0], XN_, H, Sa, ta, H, B * La, s.F, a.W1, HF_, s.F, 1);
        TSN_TRY(gemm_run(fa, EPI_STORE));
        GemmBatch ft;
        ft.nprob = 1;
        store_problem(ft.p[0], XN_, H, St, 1, H, B * Lt, s.F, t.W1, HF_, s.F, 1);
        ft.pf[0] = PfRange{a.W2, H, ta * s.F * 2, (long long)ta * s.F * 2};   // FFN2's weights, read next
        ft.pf[1] = PfRange{t.W2, H, s.F * 2, (long long)s.F * 2};
        TSN_TRY(gemm_run(ft, EPI_STORE));
    } else {
        GemmBatch f1;
        f1.nprob = 2;
        store_problem(f1.p[0], XN_, H, Sa, ta, H, B * La, s.F, a.W1, HF_, s.F, 1);
        store_problem(f1.p[1], XN_, H, St, 1, H, B * Lt, s.F, t.W1, HF_, s.F, 1);
        f1.pf[0] = PfRange{a.W2, H, ta * s.F * 2, (long long)ta * s.F * 2};   // FFN2's weights, read next
        f1.pf[1] = PfRange{t.W2, H, s.F * 2, (long long)s.F * 2};
        TSN_TRY(gemm_run(f1, EPI_STORE));
    }

    GemmBatch f2;
    f2.nprob = 2;
    f2.ws = ws_;
    f2.ws_bytes = ws_bytes_;
    resid_problem(f2.p[0], HF_, s.F, Sa, ta, s.F, B * La, H, a.W2, nullptr, X_, H, mod_ + a.mod_off + 5 * H, NMOD);
    resid_problem(f2.p[1], HF_, s.F, St, 1, s.F, B * Lt, H, t.W2, nullptr, X_, H, mod_ + t.mod_off + 5 * H, NMOD);
    next_ln(r, next, maps, 2);
    next_qkv_prefetch(r, f2, next);
    return resid_ln(f2, r, s.H, s.ln_eps);
}

// Fused block: src/dit_fwd.cpp:267-279 over the joined rows
int DitModel::block_fused(int i, bool ln1, Next next) {
    const hipStream_t st = rt->dev.stream();
    const StreamW &w = fu_[i];
    const int B = s.B, H = s.H, M = B * S;
    const RowMap D{S, S, 0};
    if (ln1) {   // otherwise the previous block's last reduce kernel produced it
        LnArgs ln;
        memset(&ln, 0, sizeof ln);
        ln.nseg = 1; ln.H = H; ln.eps = s.ln_eps;
        ln_seg(ln.seg[0], X_, H, D, XN_, mod_, NMOD, S, w.mod_off, M);
        TSN_TRY(run(K_LN16, 0, ln_bytes(ln, true), [&] { return launch_ln_mod(ln, LN_F16, st); }));
    }

    GemmBatch qb;
    qb.nprob = 1;
    qkv_problem(qb.p[0], XN_, D, M, w.Wqkv, w.bqkv, w.qn, w.kn, H, s.NH, Q_, K_, Vt_, S, Sp, S, 0, s.La, rope_, s.rms_eps);
    qb.pf[0] = PfRange{w.Wo, H, H * 2, (long long)H * 2};   // the out-projection's weights
    if (!ln_prefetch() && !grid_prefetch())   // and FFN1's, read three launches later
        qb.pf[1] = PfRange{w.W1, s.F, H * 2, (long long)H * 2};
    next_mod_gemv(qb, next);
    TSN_TRY(gemm_run(qb, EPI_QKV));

    AttnArgs at;
    memset(&at, 0, sizeof at);
    at.Q = Q_; at.K = K_; at.Vt = Vt_; at.S = S; at.Sp = Sp; at.nh = s.NH; at.BH = B * s.NH;
    at.O = AO_; at.o_f32 = 0; at.ldo = H; at.omap = rowmap_dense(M);
    TSN_TRY(run(K_ATTN, 4.0 * B * s.NH * (double)S * S * 64, 8.0 * B * (double)S * H,
                [&] { return launch_attention(at, st); }));

    GemmBatch ob;
    ob.nprob = 1;
    ob.small = 1;   // 64x64 tiles over the full K while 128x128 tiles would fill under one round
    ob.ws = ws_;
    ob.ws_bytes = ws_bytes_;
    resid_problem(ob.p[0], AO_, H, D, 1, H, M, H, w.Wo, w.bo, X_, H, mod_ + w.mod_off + 2 * H, NMOD);
    RedLnArgs r;
    next_ln(r, Next{NEXT_FUSED, i}, &D, 1);   // LN2 of this block: modulation chunks 3, 4
    r.seg[0].shift_off += 3 * H; r.seg[0].scale_off += 3 * H;
    // FFN1's weights, read next, from the LN kernel or from the out-projection's spare CUs
    if (ln_prefetch() || grid_prefetch())
        (ln_prefetch() ? r.pf : ob.pf)[0] = PfRange{w.W1, s.F, H * 2, (long long)H * 2};
    TSN_TRY(resid_ln(ob, r, s.H, s.ln_eps));

    GemmBatch f1;
    f1.nprob = 1;
    store_problem(f1.p[0], XN_, H, D, 1, H, M, s.F, w.W1, HF_, s.F, 1);
    f1.pf[0] = PfRange{w.W2, H, s.F * 2, (long long)s.F * 2};   // FFN2's weights, read next
    TSN_TRY(gemm_run(f1, EPI_STORE));

    GemmBatch f2;
    f2.nprob = 1;
    // 64x64 tiles over the full K while 128x128 tiles would fill under one round (8 s: 794 rows,
    // 56 tiles; 30 s: 144 tiles): no split-K partials, and the LN that follows is the plain ln_mod
    // kernel instead of the reduce + LN over the partials (8 s evaluation 1.839 -> 1.820 ms, same box)
    f2.small = 1;
    f2.ws = ws_;
    f2.ws_bytes = ws_bytes_;
    resid_problem(f2.p[0], HF_, s.F, D, 1, s.F, M, H, w.W2, nullptr, X_, H, mod_ + w.mod_off + 5 * H, NMOD);
    next_ln(r, next, &D, 1);
    next_qkv_prefetch(r, f2, next);
    return resid_ln(f2, r, s.H, s.ln_eps);
}

// timestep embedding + MLP, g = t_emb + pooled, gs = silu(g) (src/dit_fwd.cpp:111-140), then every
// adaLN modulation in one HBM-bound GEMV (src/dit_fwd.cpp:186-207,271-274,288-291). Rows are
// processed in GEMV batches of up to 16 (the weights are read once per batch); pooled row r is
// pooled[r % 16] (callers pass B rows for B <= 16 batches, or the 16-row repetition).
int DitModel::enqueue_conditioning(const float *t, int rows, const float *pooled, float *temb, float *h1, float *g,
                                   float *gs, float *mod, int mod_rows, bool temb_done) {
    const hipStream_t st = rt->dev.stream();
    const int H = s.H;
    if (!temb_done)   // an evaluation computes it in its eval_prep launch
        TSN_TRY(run("temb_kernel", 0, 0, [&] { return launch_temb_sinusoid(t, temb, rows, s.temb_dim, s.t_max_period, st); }));
    for (int r0 = 0; r0 < rows; r0 += 16) {
        const int rem = rows - r0;
        const int nb = rem >= 16 ? 16 : rem > 8 ? 16 : rem > 4 ? 8 : rem > 2 ? 4 : rem;   // rows past `rows` are padding
        GemvArgs g1;
        memset(&g1, 0, sizeof g1);
        g1.W = Wt0_; g1.ldw = s.temb_dim; g1.wdt = DT_BF16; g1.X = temb + (size_t)r0 * s.temb_dim; g1.ldx = s.temb_dim;
        g1.Y = h1 + (size_t)r0 * H; g1.ldy = H; g1.bias = bt0_; g1.N = H; g1.K = s.temb_dim; g1.nb = nb; g1.silu = 1;
        TSN_TRY(run(K_GEMV, 2.0 * nb * H * s.temb_dim, 2.0 * H * s.temb_dim, [&] { return launch_gemv(g1, st); }));
        GemvArgs g2;
        memset(&g2, 0, sizeof g2);
        g2.W = Wt2_; g2.ldw = H; g2.wdt = DT_BF16; g2.X = h1 + (size_t)r0 * H; g2.ldx = H;
        g2.Y = g + (size_t)r0 * H; g2.ldy = H; g2.bias = bt2_; g2.addv = pooled; g2.ld_add = H;
        g2.Y2 = gs + (size_t)r0 * H; g2.ldy2 = H; g2.N = H; g2.K = H; g2.nb = nb;
        TSN_TRY(run(K_GEMV, 2.0 * nb * H * H, 2.0 * H * H, [&] { return launch_gemv(g2, st); }));
        GemvArgs m;
        memset(&m, 0, sizeof m);
        m.W = Wmod_; m.ldw = H; m.wdt = DT_BF16;
        m.X = gs + (size_t)r0 * H; m.ldx = H;
        m.Y = mod + (size_t)r0 * NMOD; m.ldy = NMOD;
        m.bias = bmod_; m.N = mod_rows; m.K = H; m.nb = nb;
        if (mod_rows > 0)
            TSN_TRY(run(K_GEMV, 2.0 * nb * (double)mod_rows * H, 2.0 * (double)mod_rows * H + 4.0 * nb * mod_rows,
                        [&] { return launch_gemv(m, st); }));
    }
    return TSN_OK;
}

int DitModel::enqueue_forward(const float *z, const float *t, const float *text, const float *pooled, float *v,
                              float *taps) {
    return enqueue_eval(z, t, text, pooled, v, taps, nullptr);
}

// One evaluation. mod_pre: this evaluation's modulation rows, computed beforehand (the sampler);
// null: computed here from t and pooled.
int DitModel::enqueue_eval(const float *z, const float *t, const float *text, const float *pooled, float *v,
                           float *taps, const float *mod_pre) {
    TSN_REQUIRE(ready_, "dit: weights not uploaded");
    TSN_REQUIRE(z && (t || mod_pre) && (pooled || mod_pre) && v && (text || s.Lt == 0), "dit forward: null input");
    TSN_TRY(rt->dev.make_current());
    const hipStream_t st = rt->dev.stream();
    const int B = s.B, H = s.H;
    mod_in_grid_ = !mod_pre && mod_grid_ok();
    // one launch for the timestep sinusoid, the hi|lo split of z (the input projection's operand)
    // and the copy of the text rows into the residual stream (src/dit_fwd.cpp:111-119,142-149,160)
    {
        EvalPrepArgs ep;
        memset(&ep, 0, sizeof ep);
        if (!mod_pre) {
            ep.t = t; ep.temb = temb_; ep.tnb = B; ep.tD = s.temb_dim; ep.tmax = s.t_max_period;
        }
        ep.z = z; ep.ldz = s.latent; ep.zmap = rowmap_dense(B * s.La); ep.z2 = Z2_; ep.sM = B * s.La; ep.sK = s.latent;
        if (s.Lt > 0) {
            ep.csrc = text; ep.clds = H; ep.csmap = rowmap_dense(B * s.Lt); ep.cdst = X_; ep.cldd = H;
            ep.cdmap = RowMap{s.Lt, S, s.La}; ep.cM = B * s.Lt; ep.cH = H;
        }
        TSN_TRY(run("eval_prep_kernel", 0, 8.0 * B * s.La * s.latent + 8.0 * B * s.Lt * (double)H,
                    [&] { return launch_eval_prep(ep, st); }));
    }
    if (mod_pre) {
        mod_ = mod_pre;
    } else {
        TSN_TRY(enqueue_conditioning(t, B, pooled, temb_, h1_, g_, gs_, MOD_, mod_in_grid_ ? 0 : NMOD, true));
        mod_ = MOD_;
    }
    // input projection (src/dit_fwd.cpp:142-149): z split into f16 hi|lo halves (above), one MFMA
    // GEMM against [W|W] (f32-accurate), bias added, written into the audio rows of X
    {
        GemmBatch ib;
        ib.nprob = 1;
        GemmProblem &p = ib.p[0];
        gemm_problem_init(p);
        p.A = Z2_; p.lda = 2 * s.latent; p.amap = rowmap_dense(B * s.La); p.taps = 1; p.Kc = 2 * s.latent;
        p.a_T = B * s.La; p.W = Win2_; p.ldw = 2 * s.latent; p.bias = bin_;
        p.M = B * s.La; p.N = H; p.K = 2 * s.latent;
        p.Y = X_; p.ldy = H; p.ymap = RowMap{s.La, S, 0}; p.y_f16 = 0;
        if (mod_in_grid_) ib.gv = mod_args(gs_, 0, first_mod_rows());   // block 0's modulation rows
        TSN_TRY(gemm_run(ib, EPI_STORE));
    }
    const size_t tap_n = (size_t)B * S * H;
    int tap = 0;
    // each block's last reduce kernel also applies the next adaLN (the next block's LN1, or the
    // final layer's)
    const int nblk = s.n_joint + s.n_fused;
    for (int k = 0; k < nblk; ++k) {
        const Next next = k + 1 == nblk ? Next{NEXT_FINAL, 0}
                          : k + 1 < s.n_joint ? Next{NEXT_JOINT, k + 1}
                                              : Next{NEXT_FUSED, k + 1 - s.n_joint};
        if (k < s.n_joint) TSN_TRY(block_joint(k, k == 0, next));
        else TSN_TRY(block_fused(k - s.n_joint, k == 0, next));
        if (taps) TSN_TRY(rt->dev.copy_d2d(taps + tap_n * tap++, X_, tap_n * 4));
    }
    // final layer (src/dit_fwd.cpp:287-303): adaLN (2 chunks) of the audio rows and the projection
    // to the latent channels in one kernel
    if (final_fused()) {
        FinalArgs f;
        memset(&f, 0, sizeof f);
        f.X = X_; f.ldx = H; f.xmap = RowMap{s.La, S, 0};
        f.mod = mod_; f.mod_ld = NMOD; f.mod_L = s.La; f.shift_off = fin_mod_off_; f.scale_off = fin_mod_off_ + H;
        f.W = Wfin2_; f.ldw = 2 * H; f.bias = bfin_;
        f.Y = v; f.ldy = s.latent;
        f.rows = B * s.La; f.H = H; f.N = s.latent; f.eps = s.ln_eps;
        return run("final_out_kernel", 2.0 * B * s.La * (double)s.latent * H,
                   B * s.La * (double)H * 4.0 + (double)s.latent * H * 2.0 + B * s.La * (double)s.latent * 4.0,
                   [&] { return launch_final_out(f, st); });
    }
    // otherwise: adaLN on audio rows as f16 hi|lo, projection to latent by one MFMA GEMM against
    // [W|W] (f32-accurate), split over K
    if (nblk == 0) {
        LnArgs ln;
        memset(&ln, 0, sizeof ln);
        ln.nseg = 1; ln.H = H; ln.eps = s.ln_eps;
        LnSeg &g = ln.seg[0];
        g.X = X_; g.ldx = H; g.xmap = RowMap{s.La, S, 0};
        g.Y = XF2_; g.ldy = 2 * H; g.ymap = rowmap_dense(B * s.La);
        g.mod = mod_; g.mod_ld = NMOD; g.mod_L = s.La; g.shift_off = fin_mod_off_; g.scale_off = fin_mod_off_ + H;
        g.rows = B * s.La;
        TSN_TRY(run(K_LNHL, 0, B * s.La * (double)H * 8.0, [&] { return launch_ln_mod(ln, LN_F16_HILO, st); }));
    }
    GemmBatch fb;
    fb.nprob = 1;
    fb.ws = ws_;
    fb.ws_bytes = ws_bytes_;
    GemmProblem &p = fb.p[0];
    gemm_problem_init(p);
    p.A = XF2_; p.lda = 2 * H; p.amap = rowmap_dense(B * s.La); p.taps = 1; p.Kc = 2 * H; p.a_T = B * s.La;
    p.W = Wfin2_; p.ldw = 2 * H; p.bias = bfin_;
    p.M = B * s.La; p.N = s.latent; p.K = 2 * H;
    p.Y = v; p.ldy = s.latent; p.ymap = rowmap_dense(B * s.La); p.y_f16 = 0;
    return gemm_run(fb, EPI_STORE);
}

int DitModel::enqueue_joint_block(int block, float *X, const float *g) {
    TSN_REQUIRE(ready_, "dit: weights not uploaded");
    TSN_REQUIRE(block >= 0 && block < s.n_joint && X && g, "dit joint block: arguments");
    TSN_TRY(rt->dev.make_current());
    const size_t n = (size_t)s.B * S * s.H;
    TSN_TRY(gs_from_g(g));
    TSN_TRY(modulation(gs_, ja_[block].mod_off, 12 * s.H));
    mod_ = MOD_;
    TSN_TRY(rt->dev.copy_d2d(X_, X, n * 4));
    TSN_TRY(block_joint(block, true, Next{NEXT_NONE, 0}));
    return rt->dev.copy_d2d(X, X_, n * 4);
}

int DitModel::enqueue_fused_block(int block, float *X, const float *g) {
    TSN_REQUIRE(ready_, "dit: weights not uploaded");
    TSN_REQUIRE(block >= 0 && block < s.n_fused && X && g, "dit fused block: arguments");
    TSN_TRY(rt->dev.make_current());
    const size_t n = (size_t)s.B * S * s.H;
    TSN_TRY(gs_from_g(g));
    TSN_TRY(modulation(gs_, fu_[block].mod_off, 6 * s.H));
    mod_ = MOD_;
    TSN_TRY(rt->dev.copy_d2d(X_, X, n * 4));
    TSN_TRY(block_fused(block, true, Next{NEXT_NONE, 0}));
    return rt->dev.copy_d2d(X, X_, n * 4);
}

// src/pipeline.cpp:141-155: t_s = 1 - s/steps, dt = t_{s+1} - t_s, two arms then cfg_euler
int DitModel::enqueue_sample(float *x, const float *text, const float *pooled, int steps, float cfg) {
    TSN_REQUIRE(ready_, "dit: weights not uploaded");
    TSN_REQUIRE(x && pooled && (text || s.Lt == 0) && steps > 0, "dit sample: arguments");
    TSN_REQUIRE(s.B % 2 == 0, "dit sample: B must be even (cond/uncond pairs)");
    TSN_REQUIRE(tsched_ && tsched_steps_ == steps, "dit sample: schedule not prepared for this step count");
    const int P = s.B / 2;
    const size_t n = (size_t)s.La * s.latent;
    for (int b = 0; b < s.B; ++b) TSN_TRY(rt->dev.copy_d2d(x2_ + b * n, x + (b / 2) * n, n * 4));
    // the conditioning depends on t only: every step's modulation in one pass over the weights
    // per 16 rows, before the step loop (row st*B + b = step st, sample b)
    TSN_TRY(launch_copy_rows(pooled, s.H, RowMap{s.B, 0, 0}, pooled_rep_, s.H, rowmap_dense(16), 16, s.H,
                             rt->dev.stream()));
    TSN_TRY(enqueue_conditioning(tsched_, steps * s.B, pooled_rep_, temb_all_, h1_all_, g_all_, gs_all_, mod_all_, NMOD));
    for (int st = 0; st < steps; ++st) {
        const float t_curr = 1.0f - (float)st / (float)steps;
        const float t_prev = 1.0f - (float)(st + 1) / (float)steps;
        TSN_TRY(enqueue_eval(x2_, nullptr, text, nullptr, Vv_, nullptr, mod_all_ + (size_t)st * s.B * NMOD));
        TSN_TRY(launch_cfg_euler_pairs(Vv_, x2_, P, (int)n, cfg, t_prev - t_curr, rt->dev.stream()));
    }
    for (int p = 0; p < P; ++p) TSN_TRY(rt->dev.copy_d2d(x + p * n, x2_ + 2 * p * n, n * 4));
    return TSN_OK;
}

int DitModel::capture_forward(const float *z, const float *t, const float *text, const float *pooled, float *v) {
    TSN_REQUIRE(ready_, "dit: weights not uploaded");
    return capture([&] { return enqueue_forward(z, t, text, pooled, v, nullptr); });
}

int DitModel::capture_sample(float *x, const float *text, const float *pooled, int steps, float cfg) {
    TSN_REQUIRE(ready_, "dit: weights not uploaded");
    TSN_TRY(rt->dev.make_current());
    TSN_TRY(prepare_sample(steps));
    return capture([&] { return enqueue_sample(x, text, pooled, steps, cfg); });
}

int DitModel::profile_forward(const float *z, const float *t, const float *text, const float *pooled, float *v,
                              std::vector<KernelStat> &stats) {
    return profile([&] { return enqueue_forward(z, t, text, pooled, v, nullptr); }, stats);
}

int DitModel::prepare_sample(int steps) {
    TSN_REQUIRE(steps > 0, "dit sample: steps must be positive");
    TSN_REQUIRE(s.B <= 16 && 16 % s.B == 0, "dit sample: B must divide 16");
    TSN_TRY(rt->dev.make_current());
    if (tsched_ && tsched_steps_ == steps && cond_) return TSN_OK;
    if (tsched_) TSN_TRY(release(tsched_));
    tsched_ = nullptr;
    // t of step st for sample b at row st*B + b (src/pipeline.cpp:146: t = 1 - st/steps)
    std::vector<float> h((size_t)steps * s.B);
    for (int st = 0; st < steps; ++st)
        for (int b = 0; b < s.B; ++b) h[(size_t)st * s.B + b] = 1.0f - (float)st / (float)steps;
    TSN_TRY(alloc(h.size() * 4, (void **)&tsched_));
    TSN_TRY(rt->dev.upload(tsched_, h.data(), h.size() * 4));
    tsched_steps_ = steps;
    if (cond_) TSN_TRY(release(cond_));
    cond_ = nullptr;
    const size_t R = ((size_t)steps * s.B + 15) / 16 * 16, H = s.H;
    const size_t n_temb = R * s.temb_dim, n_h = R * H, n_mod = R * (size_t)NMOD, n_rep = 16 * H;
    TSN_TRY(alloc((n_temb + 3 * n_h + n_h + n_mod + n_rep) * sizeof(float), (void **)&cond_));   // zero-filled
    temb_all_ = cond_;
    h1_all_ = temb_all_ + n_temb;
    g_all_ = h1_all_ + n_h;
    gs_all_ = g_all_ + n_h;
    mod_all_ = gs_all_ + n_h + n_h;
    pooled_rep_ = mod_all_ + n_mod;
    return TSN_OK;
}

} // namespace tsn
