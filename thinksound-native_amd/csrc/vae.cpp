// vae.cpp — VaeModel: the reference's VAE decoder on HIP (src/vae.cpp:17-86).
#include "vae.h"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <map>

#include "gguf.h"

namespace tsn {

namespace {

const int DILS[3] = {1, 3, 9};   // residual-unit dilations (src/vae.cpp:21)
const int KRES = 7;              // residual-unit and input/output conv width

// transposed-conv pad of the reference (src/vae.cpp:66)
int convt_pad(int K, int s) { return K - 1 - s / 2; }
// phase r: first weight tap k0 = (pad - r) mod s, first input row offset c = -floor((pad - r) / s)
int phase_k0(int pad, int r, int s) { return (((pad - r) % s) + s) % s; }
int phase_c(int pad, int r, int s) {
    const int d = pad - r;
    return d >= 0 ? -(d / s) : (-d + s - 1) / s;
}

} // namespace

std::vector<ManifestEntry> vae_manifest(const VaeSpec &s) {
    std::vector<ManifestEntry> v;
    int64_t off = 0;
    auto add = [&](const std::string &n, int64_t numel) {
        v.push_back({n, numel, off});
        off += numel;
    };
    auto snake = [&](const std::string &p, int64_t C) {
        add(p + ".alpha", C);
        add(p + ".beta", C);
    };
    add("decoder.layers.0.weight", (int64_t)s.width[0] * s.latent * KRES);
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
            add(rp + ".layers.1.weight", co * co * KRES);
            add(rp + ".layers.1.bias", co);
            snake(rp + ".layers.2", co);
            add(rp + ".layers.3.weight", co * co);
            add(rp + ".layers.3.bias", co);
        }
    }
    snake("decoder.layers.6", s.width[5]);
    add("decoder.layers.7.weight", (int64_t)s.out_ch * s.width[5] * KRES);
    return v;
}

long long vae_audio_len(const VaeSpec &s) {
    long long T = s.T;
    for (int n = 0; n < 5; ++n) T *= s.stride[n];
    return T;
}

int vae_spec_check(const VaeSpec &s) {
    TSN_REQUIRE(s.T > 0, "vae spec: T must be positive");
    TSN_REQUIRE(s.latent > 0 && s.latent % 64 == 0, "vae spec: latent width must be a multiple of 64");
    for (int i = 0; i < 6; ++i)
        TSN_REQUIRE(s.width[i] > 0 && s.width[i] % 64 == 0 && s.width[i] <= 8192,
                    "vae spec: widths must be multiples of 64, at most 8192");
    long long T = s.T;
    for (int n = 0; n < 5; ++n) {
        const int st = s.stride[n], K = s.kt[n];
        // K a multiple of s, at least 2s: every phase then reads K/s input rows starting at q - 1 or q
        TSN_REQUIRE(st >= 1 && st <= 64 && K >= 2 * st && K % st == 0,
                    "vae spec: transposed-conv kernel must be a multiple of its stride, at least twice it");
        T *= st;
        TSN_REQUIRE(T < (1LL << 30), "vae spec: audio too long");
        // every GEMM operand row [hi | lo | hi] is addressed with 32-bit byte offsets (up to twice the
        // rows of a stage, conv halo included)
        TSN_REQUIRE(2 * T * 3 * s.width[n + 1] * 2 < (1LL << 31),
                    "vae spec: audio too long for one decode (split the latent into shorter segments)");
    }
    TSN_REQUIRE(s.out_ch == 1 || s.out_ch == 2 || s.out_ch == 4, "vae spec: 1, 2 or 4 audio channels");
    return TSN_OK;
}

VaeSpec vae_spec_for_duration(int dur_s) {
    VaeSpec s{};
    s.T = (int)llround(44100.0 / 2048.0 * dur_s);
    s.latent = 64;
    const int w[6] = {2048, 1024, 512, 256, 128, 128};
    const int st[5] = {8, 8, 4, 4, 2};
    for (int i = 0; i < 6; ++i) s.width[i] = w[i];
    for (int i = 0; i < 5; ++i) {
        s.stride[i] = st[i];
        s.kt[i] = 2 * st[i];
    }
    s.out_ch = 2;
    return s;
}

int vae_spec_from_gguf(const char *path, int T, VaeSpec *out) {
    TSN_REQUIRE(out, "vae gguf: null spec");
    GgufReader g;
    TSN_TRY(g.open(path));
    VaeSpec s = vae_spec_for_duration(1);
    s.T = T;
    // conv weights are [OC][IC][K]: ne = (K, IC, OC)
    auto shape = [&](const std::string &n, const GgufTensorInfo **t) -> int {
        *t = g.find(n);
        TSN_REQUIRE(*t && (*t)->n_dims == 3, "vae gguf: missing 3-d tensor " + n);
        return TSN_OK;
    };
    const GgufTensorInfo *t;
    TSN_TRY(shape("decoder.layers.0.weight", &t));
    s.latent = (int)t->ne[1];
    s.width[0] = (int)t->ne[2];
    for (int n = 0; n < 5; ++n) {
        TSN_TRY(shape("decoder.layers." + std::to_string(n + 1) + ".layers.1.weight", &t));
        s.kt[n] = (int)t->ne[0];
        s.width[n + 1] = (int)t->ne[2];
    }
    TSN_TRY(shape("decoder.layers.7.weight", &t));
    s.out_ch = (int)t->ne[2];
    TSN_TRY(vae_spec_check(s));
    *out = s;
    return TSN_OK;
}

int VaeModel::create(Runtime *r, const VaeSpec &sp) {
    TSN_REQUIRE(r, "vae: null runtime");
    TSN_TRY(vae_spec_check(sp));
    rt = r;
    s = sp;
    // largest [rows][C] activation over the stages (the residual stream of every stage and the
    // input conv's output)
    size_t tc = (size_t)s.T * std::max(s.width[0], s.latent);
    long long T = s.T;
    int wmax = s.width[0];
    for (int n = 0; n < 5; ++n) {
        T *= s.stride[n];
        tc = std::max(tc, (size_t)T * s.width[n + 1]);
        wmax = std::max(wmax, s.width[n + 1]);
    }
    TSN_TRY(alloc(tc * sizeof(float), (void **)&X_));
    TSN_TRY(alloc(tc * 3 * sizeof(half_t), (void **)&A1_));
    TSN_TRY(alloc(tc * 3 * sizeof(half_t), (void **)&A2_));
    std::vector<float> ones((size_t)wmax, 1.0f);
    TSN_TRY(alloc(ones.size() * sizeof(float), (void **)&ones_));
    TSN_TRY(rt->dev.upload(ones_, ones.data(), ones.size() * sizeof(float)));
    ws_bytes_ = (size_t)64 << 20;
    TSN_TRY(alloc(ws_bytes_, (void **)&ws_));
    TSN_TRY(alloc_skcnt());
    return TSN_OK;
}

int VaeModel::load_gguf(const char *path) {
    GgufReader g;
    TSN_TRY(g.open(path));
    std::vector<float> host;
    TSN_TRY(gguf_read_manifest(g, vae_manifest(s), host));
    return upload(host.data(), host.size());
}

int VaeModel::upload_weights(const float *host, size_t numel) { return upload(host, numel); }

// Host side: conv weights reordered to [rows][taps][IC] f32 (transposed convs split into phase
// groups), snake parameters turned into [exp(alpha) | exp(-beta)] tables (double precision, then
// rounded), biases repeated per phase. One f32 upload of each set; the device splits the conv
// weights into f16 [rows][taps][W_hi | W_hi | W_lo].
int VaeModel::upload(const float *host, size_t numel) {
    TSN_REQUIRE(rt && host, "vae: not created / null weights");
    TSN_REQUIRE(!ready_, "vae: weights already uploaded");
    const auto man = vae_manifest(s);
    const size_t total = (size_t)(man.back().offset + man.back().numel);
    TSN_REQUIRE(numel == total, "vae: weight count does not match the manifest (" + std::to_string(total) + ")");
    std::map<std::string, const ManifestEntry *> idx;
    for (const auto &e : man) idx[e.name] = &e;
    auto src = [&](const std::string &n) { return host + idx.at(n)->offset; };

    std::vector<float> wconv, wf32;   // to split into f16 parts / used as f32
    struct Pending { size_t off; long long rows; int IC; const half_t **dst; };
    std::vector<Pending> convs;
    std::vector<std::pair<size_t, const float **>> f32s;
    auto align4 = [](std::vector<float> &v) { v.resize((v.size() + 3) & ~(size_t)3, 0.0f); };
    // [OC][IC][K] rows -> [rows][taps][IC]: row (oc, tap j) takes weight tap kmap(oc_row, j)
    auto conv_w = [&](const std::string &n, int OC, int IC, int K, const half_t **dst) {
        const float *w = src(n);
        const size_t off = wconv.size();
        wconv.resize(off + (size_t)OC * K * IC);
        float *d = wconv.data() + off;
        for (int oc = 0; oc < OC; ++oc)
            for (int k = 0; k < K; ++k)
                for (int ic = 0; ic < IC; ++ic) d[((size_t)oc * K + k) * IC + ic] = w[((size_t)oc * IC + ic) * K + k];
        convs.push_back({off, (long long)OC * K, IC, dst});
    };
    auto vec = [&](const float *v, int n, const float **dst) {
        align4(wf32);
        f32s.push_back({wf32.size(), dst});
        wf32.insert(wf32.end(), v, v + n);
    };
    auto snake_tab = [&](const std::string &p, int C, const float **dst) {
        const float *a = src(p + ".alpha"), *b = src(p + ".beta");
        std::vector<float> t(2 * (size_t)C);
        for (int c = 0; c < C; ++c) {
            t[c] = (float)exp((double)a[c]);
            t[C + c] = (float)exp(-(double)b[c]);
        }
        vec(t.data(), 2 * C, dst);
    };

    conv_w("decoder.layers.0.weight", s.width[0], s.latent, KRES, &W0_);
    vec(src("decoder.layers.0.bias"), s.width[0], &b0_);
    for (int n = 0; n < 5; ++n) {
        Stage &g = st_[n];
        const std::string bp = "decoder.layers." + std::to_string(n + 1);
        const int ci = s.width[n], co = s.width[n + 1], stv = s.stride[n], K = s.kt[n], pad = convt_pad(K, stv);
        snake_tab(bp + ".layers.0", ci, &g.ab_in);
        // phase groups: consecutive phases with the same input row offset
        g.taps = K / stv;
        g.ngroups = 0;
        for (int r = 0; r < stv; ++r) {
            const int c = phase_c(pad, r, stv);
            if (g.ngroups > 0 && -g.pad[g.ngroups - 1] == c) {
                ++g.nph[g.ngroups - 1];
                continue;
            }
            TSN_REQUIRE(g.ngroups < 2, "vae: more than two phase groups");
            g.r0[g.ngroups] = r;
            g.nph[g.ngroups] = 1;
            g.pad[g.ngroups] = -c;
            ++g.ngroups;
        }
        const float *w = src(bp + ".layers.1.weight"), *b = src(bp + ".layers.1.bias");
        const float *a0 = src(bp + ".layers.2.layers.0.alpha"), *b0 = src(bp + ".layers.2.layers.0.beta");
        for (int q = 0; q < g.ngroups; ++q) {
            const size_t off = wconv.size();
            const int rows = g.nph[q] * co;
            wconv.resize(off + (size_t)rows * g.taps * ci);
            float *d = wconv.data() + off;
            for (int p = 0; p < g.nph[q]; ++p) {
                const int r = g.r0[q] + p, k0 = phase_k0(pad, r, stv);
                for (int oc = 0; oc < co; ++oc)
                    for (int j = 0; j < g.taps; ++j)
                        for (int ic = 0; ic < ci; ++ic)
                            d[(((size_t)p * co + oc) * g.taps + j) * ci + ic] =
                                w[((size_t)oc * ci + ic) * K + k0 + j * stv];
            }
            convs.push_back({off, (long long)rows * g.taps, ci, &g.Wt[q]});
            std::vector<float> brep((size_t)rows);
            for (int p = 0; p < g.nph[q]; ++p) memcpy(brep.data() + (size_t)p * co, b, (size_t)co * sizeof(float));
            vec(brep.data(), rows, &g.bt[q]);
            // the first residual unit's snake, applied in this conv's epilogue: table per output column
            std::vector<float> tab(2 * (size_t)rows);
            for (int p = 0; p < g.nph[q]; ++p)
                for (int c = 0; c < co; ++c) {
                    tab[(size_t)p * co + c] = (float)exp((double)a0[c]);
                    tab[(size_t)rows + (size_t)p * co + c] = (float)exp(-(double)b0[c]);
                }
            vec(tab.data(), 2 * rows, &g.abt[q]);
        }
        for (int r = 0; r < 3; ++r) {
            Unit &u = g.u[r];
            const std::string rp = bp + ".layers." + std::to_string(r + 2);
            snake_tab(rp + ".layers.0", co, &u.ab1);
            conv_w(rp + ".layers.1.weight", co, co, KRES, &u.W7);
            vec(src(rp + ".layers.1.bias"), co, &u.b7);
            snake_tab(rp + ".layers.2", co, &u.ab2);
            conv_w(rp + ".layers.3.weight", co, co, 1, &u.W1);
            vec(src(rp + ".layers.3.bias"), co, &u.b1);
        }
    }
    snake_tab("decoder.layers.6", s.width[5], &ab_out_);
    vec(src("decoder.layers.7.weight"), s.out_ch * s.width[5] * KRES, &Wout_);

    // f32 parameters: used in place
    float *pf;
    TSN_TRY(alloc(wf32.size() * sizeof(float), (void **)&pf));
    TSN_TRY(rt->dev.upload(pf, wf32.data(), wf32.size() * sizeof(float)));
    for (auto &e : f32s) *e.second = pf + e.first;
    // conv weights: f32 staging, split into the f16 three-part rows
    size_t parts = 0;
    for (const auto &c : convs) parts += (size_t)c.rows * 3 * c.IC;
    half_t *ph;
    float *stage;
    TSN_TRY(alloc(parts * sizeof(half_t), (void **)&ph));
    TSN_TRY(alloc(wconv.size() * sizeof(float), (void **)&stage));
    TSN_TRY(rt->dev.upload(stage, wconv.data(), wconv.size() * sizeof(float)));
    size_t o = 0;
    for (const auto &c : convs) {
        TSN_TRY(launch_split3(stage + c.off, c.rows, c.IC, nullptr, 2, ph + o, rt->dev.stream()));
        *c.dst = ph + o;
        o += (size_t)c.rows * 3 * c.IC;
    }
    TSN_TRY(rt->dev.sync());
    TSN_TRY(release(stage));
    ready_ = true;
    return TSN_OK;
}

int VaeModel::enqueue_decode(const float *latent, float *audio) {
    TSN_REQUIRE(ready_, "vae: weights not uploaded");
    TSN_REQUIRE(latent && audio, "vae: null latent or audio");
    TSN_REQUIRE((((uintptr_t)latent) & 15) == 0, "vae: latent must be 16-byte aligned");
    const hipStream_t stq = rt->dev.stream();
    const double third = 1.0 / 3.0;   // profiled flops: the f32 GEMM's 2*M*N*K, not the three f16 products
    // three-part operands ping-pong between A1 and A2: each GEMM reads `in` and writes `out`
    half_t *in = A1_, *out = A2_;
    auto flip = [&]() { std::swap(in, out); };
    // conv GEMM over the three-part operand A (lda = 3 IC); taps of width 3 IC
    auto conv = [&](GemmProblem &p, const half_t *A, int M, int IC, int taps, int pad, int dil, const half_t *W,
                    const float *bias, int N) {
        gemm_problem_init(p);
        p.A = A; p.lda = 3 * IC; p.amap = rowmap_dense(M);
        p.taps = taps; p.Kc = 3 * IC; p.pad = pad; p.a_T = M; p.dil = dil;
        p.W = W; p.ldw = taps * 3 * IC; p.bias = bias;
        p.M = M; p.N = N; p.K = taps * 3 * IC;
    };
    auto batch = [&](GemmBatch &b, int n) {
        b.nprob = n;
        b.ws = ws_;
        b.ws_bytes = ws_bytes_;
        b.split_waves = 1;   // long-K stages: classic split-K, which keeps W and A tiles shared in L2
    };

    int T = s.T, C = s.width[0];
    // input conv k7 pad 3 + b, then the first stage's snake: latent -> snake(x0) three-part
    TSN_TRY(run("split3_kernel", 0, (double)T * s.latent * 10.0,
                [&] { return launch_split3(latent, T, s.latent, nullptr, 1, in, stq); }));
    {
        GemmBatch b;
        batch(b, 1);
        GemmProblem &p = b.p[0];
        conv(p, in, T, s.latent, KRES, 3, 1, W0_, b0_, C);
        p.Y = out; p.ldy = 3 * C; p.ymap = rowmap_dense(T);
        p.y_f16 = 1; p.y_lo = C; p.y_hi2 = 2 * C; p.snake = st_[0].ab_in;
        TSN_TRY(gemm_run(b, EPI_SNAKE, third));
        flip();
    }
    for (int n = 0; n < 5; ++n) {
        const Stage &g = st_[n];
        const int stv = s.stride[n], co = s.width[n + 1];
        // transposed conv as phase-group convs: x rows interleave straight into X, and the first
        // residual unit's snake(x) into the three-part rows of `out`
        {
            GemmBatch b;
            batch(b, g.ngroups);
            for (int q = 0; q < g.ngroups; ++q) {
                GemmProblem &p = b.p[q];
                conv(p, in, T, C, g.taps, g.pad[q], 1, g.Wt[q], g.bt[q], g.nph[q] * co);
                p.R = X_ + (size_t)g.r0[q] * co; p.ldr = stv * co; p.rmap = rowmap_dense(T); p.r_add = 0;
                p.Y = out + (size_t)g.r0[q] * 3 * co; p.ldy = stv * 3 * co; p.ymap = rowmap_dense(T);
                p.y_lo = co; p.snake = g.abt[q];
            }
            TSN_TRY(gemm_run(b, EPI_RSNAKE, third));
            flip();
        }
        T *= stv;
        C = co;
        for (int r = 0; r < 3; ++r) {
            const Unit &u = g.u[r];
            const int d = DILS[r];
            {   // conv k7, dilation d, + bias -> snake -> three-part f16
                GemmBatch b;
                batch(b, 1);
                GemmProblem &p = b.p[0];
                conv(p, in, T, C, KRES, 3 * d, d, u.W7, u.b7, C);
                p.Y = out; p.ldy = 3 * C; p.ymap = rowmap_dense(T);
                p.y_f16 = 1; p.y_lo = C; p.y_hi2 = 2 * C; p.snake = u.ab2;
                TSN_TRY(gemm_run(b, EPI_SNAKE, third));
                flip();
            }
            {   // conv k1 + bias added to x; the next snake (next unit, or next stage's input) from the new x
                const float *next = r < 2 ? g.u[r + 1].ab1 : n < 4 ? st_[n + 1].ab_in : nullptr;
                GemmBatch b;
                batch(b, 1);
                GemmProblem &p = b.p[0];
                conv(p, in, T, C, 1, 0, 1, u.W1, u.b1, C);
                p.R = X_; p.ldr = C; p.rmap = rowmap_dense(T);
                if (next) {
                    p.r_add = 1;
                    p.Y = out; p.ldy = 3 * C; p.ymap = rowmap_dense(T);
                    p.y_lo = C; p.snake = next;
                    TSN_TRY(gemm_run(b, EPI_RSNAKE, third));
                    flip();
                } else {   // the final snake belongs to the output conv
                    p.gate = ones_; p.gate_ld = 0; p.gate_L = T;
                    TSN_TRY(gemm_run(b, EPI_RESID, third));
                }
            }
        }
    }
    // final snake + conv k7 pad 3 (no bias) -> audio [T][out_ch]
    const double fl = 2.0 * T * (double)s.out_ch * C * KRES;
    return run("conv_out_kernel", fl, (double)T * C * 4.0 + (double)T * s.out_ch * 4.0,
               [&] { return launch_conv_out(X_, ab_out_, Wout_, audio, T, C, s.out_ch, KRES, 3, stq); });
}

} // namespace tsn
