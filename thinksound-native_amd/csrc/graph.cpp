// graph.cpp — GraphRunner plumbing and the GEMM-problem / LN-segment builders.
#include "graph.h"

#include <string.h>

namespace tsn {

GraphRunner::~GraphRunner() {
    if (gexec_) hipGraphExecDestroy(gexec_);
    if (graph_) hipGraphDestroy(graph_);
    if (rt)
        for (void *p : owned_) rt->dev.free(p);
}

int GraphRunner::alloc(size_t bytes, void **p) {
    TSN_TRY(rt->dev.alloc(bytes, p));
    owned_.push_back(*p);
    return TSN_OK;
}

int GraphRunner::release(void *p) {
    for (auto it = owned_.begin(); it != owned_.end(); ++it)
        if (*it == p) {
            // a captured graph may hold this buffer's address: it is no longer replayable
            drop_graph();
            owned_.erase(it);
            return rt->dev.free(p);
        }
    TSN_REQUIRE(false, "release: not an allocation of this model");
}

void GraphRunner::drop_graph() {
    if (gexec_) { hipGraphExecDestroy(gexec_); gexec_ = nullptr; }
    if (graph_) { hipGraphDestroy(graph_); graph_ = nullptr; }
}

int GraphRunner::capture(const std::function<int()> &enqueue) {
    TSN_TRY(rt->dev.make_current());
    drop_graph();
    const hipStream_t st = rt->dev.stream();
    TSN_HIP_CHECK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    const int rc = enqueue();
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(st, &g);
    if (rc != TSN_OK) { if (g) hipGraphDestroy(g); return rc; }
    TSN_HIP_CHECK(e);
    graph_ = g;
    TSN_HIP_CHECK(hipGraphInstantiate(&gexec_, graph_, nullptr, nullptr, 0));
    return TSN_OK;
}

int GraphRunner::replay() {
    if (!gexec_) {
        set_error("no captured graph (none was captured, or a buffer it used has been reallocated since)");
        return TSN_ERR_STATE;
    }
    TSN_TRY(rt->dev.make_current());
    TSN_HIP_CHECK(hipGraphLaunch(gexec_, rt->dev.stream()));
    return TSN_OK;
}

int GraphRunner::profile(const std::function<int()> &enqueue, std::vector<KernelStat> &stats) {
    std::vector<ProfRec> recs;
    prof_ = &recs;
    const int rc = enqueue();
    prof_ = nullptr;
    int rc2 = rt->dev.sync();
    stats.clear();
    for (auto &r : recs) {
        float ms = 0.0f;
        if (rc == TSN_OK && rc2 == TSN_OK && hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) rc2 = TSN_ERR_HIP;
        hipEventDestroy(r.a);
        hipEventDestroy(r.b);
        KernelStat *k = nullptr;
        for (auto &e : stats)
            if (e.name == r.name) k = &e;
        if (!k) {
            stats.push_back(KernelStat{});
            k = &stats.back();
            k->name = r.name;
        }
        k->launches += 1;
        k->ms += ms;
        k->flops += r.flops;
        k->bytes += r.bytes;
    }
    if (rc != TSN_OK) return rc;
    if (rc2 != TSN_OK) set_error("profile: event timing failed");
    return rc2;
}

int GraphRunner::alloc_skcnt() {
    void *p = nullptr;
    TSN_TRY(alloc(SK_COUNTERS * sizeof(unsigned), &p));
    skcnt_ = (unsigned *)p;
    return TSN_OK;
}

int GraphRunner::gemm_run(GemmBatch &b, int epi, double flop_scale) {
    const hipStream_t st = rt->dev.stream();
    if (!b.sk_cnt && skcnt_) {
        b.sk_cnt = skcnt_;
        b.sk_cnt_n = SK_COUNTERS;
    }
    TSN_TRY(gemm_plan(b, epi, false));
    TSN_TRY(run(b.kname, gemm_flops(b) * flop_scale, gemm_bytes(b, epi),
                [&] { return gemm_launch_planned(b, epi, false, st); }));
    if (!gemm_needs_reduce(b)) return TSN_OK;
    double red = 0;
    for (int i = 0; i < b.nprob; ++i)
        if (b.p[i].splits > 1) red += (4.0 * b.p[i].splits + (epi == EPI_RESID ? 8.0 : 4.0)) * b.p[i].M * (double)b.p[i].N;
    if (b.sk) red = 2.0 * b.sk_g * 128 * 128 * 4.0;   // every partial slot read once (upper bound)
    return run(gemm_reduce_name(b, epi), 0, red, [&] { return launch_gemm_reduce(b, epi, st); });
}

// Residual GEMM batch followed by one reduce kernel that finishes the split-K sum into X
// (x += gate * (sum + bias), fixed split order) and applies the adaLN that follows (r.seg[i].ln).
// Segment i covers the rows of problem i. Without split and without a following LN the reduce
// kernel is skipped (the GEMM epilogue already updated X).
int GraphRunner::resid_ln(GemmBatch &b, RedLnArgs &r, int H, float eps) {
    const hipStream_t st = rt->dev.stream();
    if (!b.sk_cnt && skcnt_) {
        b.sk_cnt = skcnt_;
        b.sk_cnt_n = SK_COUNTERS;
    }
    TSN_TRY(gemm_plan(b, EPI_RESID, false));
    TSN_TRY(run(b.kname, gemm_flops(b), gemm_bytes(b, EPI_RESID), [&] { return gemm_launch_planned(b, EPI_RESID, false, st); }));
    if (b.sk)   // stream-K: the fixup applies the residual epilogue to the cut tiles
        TSN_TRY(run(gemm_reduce_name(b, EPI_RESID), 0, 2.0 * b.sk_g * 128 * 128 * 4.0,
                    [&] { return launch_gemm_reduce(b, EPI_RESID, st); }));
    r.nseg = b.nprob;
    r.H = H;
    r.eps = eps;
    bool work = false;
    double bytes = 0;
    for (int i = 0; i < b.nprob; ++i) {
        const GemmProblem &p = b.p[i];
        RedLnSeg &g = r.seg[i];
        g.ws = p.ws; g.splits = p.splits; g.M = p.M;
        g.bias = p.bias; g.gate = p.gate; g.gate_ld = p.gate_ld; g.gate_L = p.gate_L;
        g.X = p.R; g.ldx = p.ldr; g.xmap = p.rmap;
        work = work || g.ln || g.splits > 1;
        bytes += (double)p.M * p.N * (4.0 + (p.splits > 1 ? 4.0 * p.splits + 4.0 : 0.0));
        if (g.ln) bytes += (double)g.ln_len * (p.M / g.mod_L) * p.N * (r.ymode == LN_F16_HILO || g.hilo ? 4.0 : 2.0);
    }
    if (!work) return TSN_OK;
    // nothing to sum (no split) and a plain f16 LN of every row of each segment: the one-wave-per-row
    // LN kernel does the same job with less synchronization
    bool plain_ln = r.ymode == LN_F16;
    for (int i = 0; i < r.nseg; ++i) {
        const RedLnSeg &g = r.seg[i];
        plain_ln = plain_ln && g.splits <= 1 && g.ln && g.ln_len == g.mod_L && !g.hilo;
    }
    if (plain_ln) {
        LnArgs ln;
        memset(&ln, 0, sizeof ln);
        ln.nseg = r.nseg; ln.H = H; ln.eps = eps;
        for (int k = 0; k < PF_RANGES; ++k) ln.pf[k] = r.pf[k];
        for (int i = 0; i < r.nseg; ++i) {
            const RedLnSeg &g = r.seg[i];
            LnSeg &l = ln.seg[i];
            l.X = g.X; l.ldx = g.ldx; l.xmap = g.xmap;
            l.Y = g.Y; l.ldy = g.ldy; l.ymap = g.ymap;
            l.mod = g.mod; l.mod_ld = g.mod_ld; l.mod_L = g.mod_L; l.shift_off = g.shift_off; l.scale_off = g.scale_off;
            l.rows = g.M;
        }
        return run(K_LN16, 0, bytes, [&] { return launch_ln_mod(ln, LN_F16, st); });
    }
    return run(r.ymode == LN_F16_HILO ? K_RLNHL : K_RLN16, 0, bytes, [&] { return launch_reduce_ln(r, st); });
}

// The batch's GEMV rows (GemmBatch::gv: run by extra workgroups of the grid, or as a kernel of its
// own just before it) count toward the launch that runs them: 2*nb*N*K flops; W once at its
// storage type, the nb rows of X, and Y (plus silu(Y) when Y2 is set) as f32.
static double gemv_flops(const GemvArgs &g) { return g.N > 0 ? 2.0 * g.nb * (double)g.N * g.K : 0.0; }
static double gemv_bytes(const GemvArgs &g) {
    if (g.N <= 0) return 0.0;
    const double wb = g.wdt == DT_F32 ? 4.0 : 2.0;
    return wb * g.N * (double)g.K + 4.0 * g.nb * (double)g.K + 4.0 * g.nb * (double)g.N * (g.Y2 ? 2 : 1);
}

double gemm_flops(const GemmBatch &b) {
    double f = gemv_flops(b.gv);
    for (int i = 0; i < b.nprob; ++i) f += 2.0 * b.p[i].M * (double)b.p[i].N * b.p[i].K / (b.p[i].w_half ? 2 : 1);
    return f;
}

// A once (conv taps re-read the same rows), W once, output at its storage type (residual: read +
// write f32; SwiGLU: half the columns), plus the batch's GEMV rows. Flops of a hi|lo operand
// against half-width W count the model's K (half the K the MFMAs run).
double gemm_bytes(const GemmBatch &b, int epi) {
    double x = gemv_bytes(b.gv);
    for (int i = 0; i < b.nprob; ++i) {
        const GemmProblem &p = b.p[i];
        double out = epi == EPI_RESID ? 8.0 : epi == EPI_SWIGLU ? 1.0 : epi == EPI_SNAKE ? 6.0
                   : epi == EPI_RSNAKE ? (p.r_add ? 14.0 : 10.0) : (p.y_f16 || epi == EPI_QKV ? 2.0 : 4.0);
        if (p.y_lo && (epi == EPI_STORE || epi == EPI_SWIGLU)) out *= 2.0;
        x += 2.0 * p.M * (double)p.Kc + 2.0 * p.N * (double)p.K / (p.w_half ? 2 : 1) + out * p.M * (double)p.N;
    }
    return x;
}

double ln_bytes(const LnArgs &a, bool f16) {
    double r = 0;
    for (int i = 0; i < a.nseg; ++i) r += a.seg[i].rows;
    return r * a.H * (4.0 + (f16 ? 2.0 : 4.0));
}

void qkv_problem(GemmProblem &p, const half_t *A, RowMap amap, int M, const half_t *W, const float *bias,
                 const float *qn, const float *kn, int H, int nh, half_t *Q, half_t *K, half_t *Vt, int S, int Sp,
                 int q_L, int q_soff, int rope_len, const float *rope, float eps) {
    gemm_problem_init(p);
    p.A = A; p.lda = H; p.amap = amap; p.taps = 1; p.Kc = H; p.pad = 0; p.a_T = amap.L;
    p.W = W; p.ldw = H; p.bias = bias; p.M = M; p.N = 3 * H; p.K = H;
    p.Q = Q; p.Kd = K; p.Vt = Vt; p.S_att = S; p.Sp = Sp; p.nh = nh; p.Hq = H;
    p.q_L = q_L; p.q_soff = q_soff; p.rope_len = rope_len; p.rope = rope;
    // softmax scale 1/sqrt(64) and log2(e), folded into q before its f16 rounding: attention's
    // products are then scores in log2 units
    p.qn = qn; p.kn = kn; p.rms_eps = eps; p.q_scale = 0.125f * 1.4426950408889634f;
}

void resid_problem(GemmProblem &p, const half_t *A, int lda, RowMap amap, int taps, int Kc, int M, int N,
                   const half_t *W, const float *bias, float *R, int ldr, const float *gate, int gate_ld) {
    gemm_problem_init(p);
    p.A = A; p.lda = lda; p.amap = amap; p.taps = taps; p.Kc = Kc; p.pad = taps / 2; p.a_T = amap.L;
    p.W = W; p.ldw = taps * Kc; p.bias = bias; p.M = M; p.N = N; p.K = taps * Kc;
    p.R = R; p.ldr = ldr; p.rmap = amap; p.gate = gate; p.gate_ld = gate_ld; p.gate_L = amap.L;
}

void store_problem(GemmProblem &p, const half_t *A, int lda, RowMap amap, int taps, int Kc, int M, int N,
                   const half_t *W, half_t *Y, int ldy, int silu) {
    gemm_problem_init(p);
    p.A = A; p.lda = lda; p.amap = amap; p.taps = taps; p.Kc = Kc; p.pad = taps / 2; p.a_T = amap.L;
    p.W = W; p.ldw = taps * Kc; p.bias = nullptr; p.M = M; p.N = N; p.K = taps * Kc;
    p.Y = Y; p.ldy = ldy; p.ymap = amap; p.y_f16 = 1; p.silu = silu;
}

void ln_seg(LnSeg &g, const float *X, int H, RowMap map, half_t *Y, const float *mod, int nmod, int L,
            int shift_off, int rows) {
    g.X = X; g.ldx = H; g.xmap = map;
    g.Y = Y; g.ldy = H; g.ymap = map;
    g.mod = mod; g.mod_ld = nmod; g.mod_L = L; g.shift_off = shift_off; g.scale_off = shift_off + H;
    g.rows = rows;
}

} // namespace tsn
