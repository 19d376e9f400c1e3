// runtime.cpp — Device (HIP) and the net.h-shaped launcher runtime.
#include "runtime.h"

#include <math.h>
#include <string.h>

#include <algorithm>

namespace tsn {

namespace {
thread_local std::string g_last_error;
}
void set_error(const std::string &msg) { g_last_error = msg; }
LaunchEvents &next_launch_events() {
    static thread_local LaunchEvents ev;
    return ev;
}
const char *last_error() { return g_last_error.c_str(); }

/* ---------------------------------------------------------------- Device */

Device::~Device() {
    if (dev_ < 0) return;
    hipSetDevice(dev_);
    if (stream_) hipStreamSynchronize(stream_);
    for (void *p : owned_) hipFree(p);
    if (ev0_) hipEventDestroy(ev0_);
    if (ev1_) hipEventDestroy(ev1_);
    if (stream_) hipStreamDestroy(stream_);
}

int Device::init(int device) {
    int n = 0;
    TSN_HIP_CHECK(hipGetDeviceCount(&n));
    TSN_REQUIRE(device >= 0 && device < n, "device index out of range");
    dev_ = device;
    TSN_HIP_CHECK(hipSetDevice(dev_));
    // default priority, non-blocking with respect to the null stream
    TSN_HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
    TSN_HIP_CHECK(hipEventCreate(&ev0_));
    TSN_HIP_CHECK(hipEventCreate(&ev1_));
    return TSN_OK;
}

int Device::make_current() const {
    TSN_REQUIRE(dev_ >= 0, "device not initialised");
    TSN_HIP_CHECK(hipSetDevice(dev_));
    return TSN_OK;
}

int Device::alloc(size_t bytes, void **p) {
    TSN_REQUIRE(p, "alloc: null out pointer");
    TSN_TRY(make_current());
    if (bytes == 0) bytes = 256;
    void *q = nullptr;
    hipError_t e = hipMalloc(&q, bytes);
    if (e != hipSuccess) {
        set_error(std::string("hipMalloc(") + std::to_string(bytes) + "): " + hipGetErrorString(e));
        return TSN_ERR_OOM;
    }
    // zero fill, outside any captured graph (allocation is never captured)
    e = hipMemsetAsync(q, 0, bytes, stream_);
    if (e == hipSuccess) e = hipStreamSynchronize(stream_);
    if (e != hipSuccess) {
        hipFree(q);
        set_error(std::string("alloc zero-fill: ") + hipGetErrorString(e));
        return TSN_ERR_HIP;
    }
    owned_.push_back(q);
    *p = q;
    return TSN_OK;
}

int Device::free(void *p) {
    if (!p) return TSN_OK;
    auto it = std::find(owned_.begin(), owned_.end(), p);
    TSN_REQUIRE(it != owned_.end(), "free: pointer not owned by this runtime");
    TSN_TRY(make_current());
    TSN_HIP_CHECK(hipStreamSynchronize(stream_));
    TSN_HIP_CHECK(hipFree(p));
    owned_.erase(it);
    return TSN_OK;
}

int Device::upload(void *dst, const void *src, size_t bytes) {
    TSN_REQUIRE(dst && src, "upload: null pointer");
    TSN_TRY(make_current());
    TSN_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream_));
    TSN_HIP_CHECK(hipStreamSynchronize(stream_));
    return TSN_OK;
}

int Device::download(void *dst, const void *src, size_t bytes) {
    TSN_REQUIRE(dst && src, "download: null pointer");
    TSN_TRY(make_current());
    TSN_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream_));
    TSN_HIP_CHECK(hipStreamSynchronize(stream_));
    return TSN_OK;
}

int Device::copy_d2d(void *dst, const void *src, size_t bytes) {
    TSN_REQUIRE(dst && src, "copy: null pointer");
    TSN_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream_));
    return TSN_OK;
}

int Device::begin() {
    TSN_TRY(make_current());
    TSN_HIP_CHECK(hipEventRecord(ev0_, stream_));
    begun_ = true;
    return TSN_OK;
}

int Device::commit() {
    TSN_TRY(make_current());
    if (begun_) TSN_HIP_CHECK(hipEventRecord(ev1_, stream_));
    TSN_HIP_CHECK(hipStreamSynchronize(stream_));
    if (begun_) {
        float ms = 0.0f;
        TSN_HIP_CHECK(hipEventElapsedTime(&ms, ev0_, ev1_));
        last_ms_ = ms;
        begun_ = false;
    }
    return TSN_OK;
}

int Device::sync() {
    TSN_TRY(make_current());
    TSN_HIP_CHECK(hipStreamSynchronize(stream_));
    return TSN_OK;
}

/* ---------------------------------------------------------------- Runtime */

int Runtime::scratch(size_t bytes, void **p) {
    if (bytes > scratch_bytes_) {
        if (scratch_) TSN_TRY(dev.free(scratch_));
        scratch_ = nullptr;
        scratch_bytes_ = 0;
        TSN_TRY(dev.alloc(bytes, &scratch_));
        scratch_bytes_ = bytes;
    }
    *p = scratch_;
    return TSN_OK;
}

int Runtime::gemm(int wdt, const void *W, const void *X, int xdt, void *Y, int ydt, const float *bias,
                  const GemmParams &p) {
    TSN_REQUIRE(W && X && Y, "gemm: null operand");
    TSN_REQUIRE(p.M > 0 && p.N > 0 && p.K > 0, "gemm: empty shape");
    const int ldx = p.ldx ? (int)p.ldx : (int)p.K, ldw = p.ldw ? (int)p.ldw : (int)p.K;
    const int ldy = p.ldy ? (int)p.ldy : (int)p.N;
    TSN_TRY(dev.make_current());
    if (wdt == DT_F16) {
        TSN_REQUIRE(xdt == DT_F32 || xdt == DT_F16, "gemm: X must be f32 or f16");
        TSN_REQUIRE(ydt == DT_F32 || ydt == DT_F16, "gemm: Y must be f32 or f16");
        GemmBatch b;
        gemm_problem_init(b.p[0]);
        GemmProblem &q = b.p[0];
        q.A = X; q.lda = ldx; q.amap = rowmap_dense((int)p.M);
        q.taps = 1; q.Kc = (int)p.K; q.pad = 0; q.a_T = (int)p.M;
        q.W = (const half_t *)W; q.ldw = ldw; q.bias = bias;
        q.M = (int)p.M; q.N = (int)p.N; q.K = (int)p.K;
        q.Y = Y; q.ldy = ldy; q.ymap = rowmap_dense((int)p.M); q.y_f16 = ydt == DT_F16;
        b.nprob = 1;
        return launch_gemm(b, EPI_STORE, xdt == DT_F32, dev.stream());
    }
    TSN_REQUIRE(wdt == DT_F32 || wdt == DT_BF16, "gemm: weight dtype");
    TSN_REQUIRE(xdt == DT_F32 && ydt == DT_F32, "gemm: f32/bf16 weights take f32 X and Y");
    LinArgs a;
    a.X = (const float *)X; a.ldx = ldx; a.xmap = rowmap_dense((int)p.M);
    a.W = W; a.ldw = ldw; a.wdt = wdt; a.bias = bias;
    a.Y = (float *)Y; a.ldy = ldy; a.ymap = rowmap_dense((int)p.M);
    a.M = (int)p.M; a.N = (int)p.N; a.K = (int)p.K;
    return launch_linear_f32(a, dev.stream());
}

int Runtime::gemv(const void *W, const float *X, float *Y, const float *bias, uint32_t N, uint32_t K,
                  uint32_t ldw, int wdt) {
    TSN_TRY(dev.make_current());
    GemvArgs a;
    memset(&a, 0, sizeof a);
    a.W = W; a.ldw = ldw ? (int)ldw : (int)K; a.wdt = wdt;
    a.X = X; a.ldx = (int)K; a.Y = Y; a.ldy = (int)N; a.bias = bias;
    a.N = (int)N; a.K = (int)K; a.nb = 1;
    return launch_gemv(a, dev.stream());
}

int Runtime::conv_prepare(const void *W, int w_bf16, void *Wp, uint32_t OC, uint32_t IC, uint32_t K) {
    TSN_TRY(dev.make_current());
    return launch_conv_weight_reorder(W, w_bf16, (half_t *)Wp, (int)OC, (int)IC, (int)K, dev.stream());
}

int Runtime::conv(const void *Wp, const float *bias, const float *x, float *y, uint32_t T, uint32_t OL,
                  uint32_t IC, uint32_t OC, uint32_t K, uint32_t stride, uint32_t pad, uint32_t dil) {
    TSN_REQUIRE(Wp && x && y, "conv: null operand");
    if (stride != 1 || dil != 1) {
        set_error("conv: only stride 1, dilation 1 (the DiT convs) are implemented");
        return TSN_ERR_UNSUPPORTED;
    }
    TSN_REQUIRE((int)OL == (int)T + 2 * (int)pad - (int)K + 1, "conv: OL must equal T + 2*pad - K + 1");
    TSN_REQUIRE(K == 1 || IC % 64 == 0, "conv: IC must be a multiple of 64 for K > 1");
    TSN_TRY(dev.make_current());
    GemmBatch b;
    gemm_problem_init(b.p[0]);
    GemmProblem &q = b.p[0];
    q.A = x; q.lda = (int)IC; q.amap = rowmap_dense((int)OL);
    q.taps = (int)K; q.Kc = (int)IC; q.pad = (int)pad; q.a_T = (int)T;
    q.W = (const half_t *)Wp; q.ldw = (int)(IC * K); q.bias = bias;
    q.M = (int)OL; q.N = (int)OC; q.K = (int)(IC * K);
    q.Y = y; q.ldy = (int)OC; q.ymap = rowmap_dense((int)OL); q.y_f16 = 0;
    b.nprob = 1;
    return launch_gemm(b, EPI_STORE, true, dev.stream());
}

int Runtime::silu(float *x, size_t n) { TSN_TRY(dev.make_current()); return launch_silu(x, n, dev.stream()); }
int Runtime::copy(const float *x, float *y, size_t n) { TSN_TRY(dev.make_current()); return launch_copy(x, y, n, dev.stream()); }
int Runtime::swiglu(const float *a, const float *b, float *y, size_t n) {
    TSN_TRY(dev.make_current());
    return launch_swiglu(a, b, y, n, dev.stream());
}
int Runtime::add_(const float *a, const float *b, float *y, size_t n) {
    TSN_TRY(dev.make_current());
    return launch_add(a, b, y, n, dev.stream());
}
int Runtime::add_bcast_col(const float *x, const float *v, float *y, uint32_t S, uint32_t H) {
    TSN_TRY(dev.make_current());
    return launch_add_bcast_col(x, v, y, (int)S, (int)H, dev.stream());
}
int Runtime::cfg_euler(const float *fc, const float *fu, float *x, size_t n, float cfg, float dt) {
    TSN_TRY(dev.make_current());
    return launch_cfg_euler(fc, fu, x, n, cfg, dt, dev.stream());
}

int Runtime::adaln_ln(const float *x, const float *mod, void *y, int ydt, uint32_t rows, uint32_t H,
                      uint32_t per_row, uint32_t chunks, uint32_t base, float eps) {
    TSN_REQUIRE(ydt == DT_F32 || ydt == DT_F16, "adaln_ln: y dtype");
    TSN_REQUIRE(base + 2 * H <= chunks * H, "adaln_ln: base + 2H exceeds the modulation row");
    TSN_TRY(dev.make_current());
    LnArgs a;
    memset(&a, 0, sizeof a);
    LnSeg &s = a.seg[0];
    s.X = x; s.ldx = (int)H; s.xmap = rowmap_dense((int)rows);
    s.Y = y; s.ldy = (int)H; s.ymap = rowmap_dense((int)rows);
    s.mod = mod; s.mod_ld = (int)(chunks * H); s.mod_L = per_row ? 1 : (int)rows;
    s.shift_off = (int)base; s.scale_off = (int)(base + H);
    s.rows = (int)rows;
    a.nseg = 1; a.H = (int)H; a.eps = eps;
    return launch_ln_mod(a, ydt == DT_F16 ? LN_F16 : LN_F32, dev.stream());
}

int Runtime::gate_add(const float *x, const float *f, const float *mod, float *y, uint32_t rows, uint32_t H,
                      uint32_t per_row, uint32_t chunks, uint32_t gate_idx) {
    TSN_TRY(dev.make_current());
    return launch_gate_add(x, f, mod, y, (int)rows, (int)H, (int)per_row, (int)chunks, (int)gate_idx, dev.stream());
}

int Runtime::rms_head(float *x, const float *w, uint32_t rows, uint32_t nh, uint32_t ld, uint32_t hd,
                      uint32_t col_off, uint32_t row_off, float eps) {
    TSN_TRY(dev.make_current());
    return launch_rms_head(x, w, (int)rows, (int)nh, (int)ld, (int)hd, (int)col_off, (int)row_off, eps, dev.stream());
}

int Runtime::rope_pairs(float *x, const int32_t *pos, uint32_t rows, uint32_t nh, uint32_t ld, uint32_t hd,
                        uint32_t col_off, uint32_t row_off, float fscale, float base) {
    TSN_TRY(dev.make_current());
    return launch_rope_pairs(x, pos, (int)rows, (int)nh, (int)ld, (int)hd, (int)col_off, (int)row_off, fscale, base,
                             dev.stream());
}

int Runtime::attention(const float *qkv, float *out, uint32_t S, uint32_t nh, uint32_t hd, uint32_t ld,
                       uint32_t ldo, uint32_t q_off, uint32_t k_off, uint32_t v_off, uint32_t o_off, float scale) {
    TSN_REQUIRE(qkv && out && S > 0 && nh > 0, "attention: arguments");
    if (hd != 64) {
        set_error("attention: head dim must be 64");
        return TSN_ERR_UNSUPPORTED;
    }
    TSN_REQUIRE(ldo % 4 == 0 && o_off % 4 == 0, "attention: ldo and o_off must be multiples of 4");
    TSN_TRY(dev.make_current());
    const int Sp = (int)((S + 63) / 64 * 64);
    const size_t qk = (size_t)nh * S * 64, vt = (size_t)nh * 64 * Sp;
    void *buf = nullptr;
    TSN_TRY(scratch((2 * qk + vt) * sizeof(half_t) + 256, &buf));
    half_t *Q = (half_t *)buf, *K = Q + qk, *Vt = K + qk;
    // keep Vt 16-byte aligned
    Vt = (half_t *)(((uintptr_t)Vt + 15) & ~(uintptr_t)15);
    TSN_TRY(launch_attn_pack(qkv, (int)S, (int)nh, (int)ld, (int)q_off, (int)k_off, (int)v_off, Q, K, Vt, Sp, dev.stream()));
    AttnArgs a;
    memset(&a, 0, sizeof a);
    a.Q = Q; a.K = K; a.Vt = Vt; a.S = (int)S; a.Sp = Sp; a.nh = (int)nh; a.BH = (int)nh;
    a.O = out + o_off; a.o_f32 = 1; a.ldo = (int)ldo; a.omap = rowmap_dense((int)S);
    a.scale_log2 = scale * 1.4426950408889634f;
    return launch_attention(a, dev.stream());
}

int Runtime::probe_peaks(double *mfma_tflops, double *hbm_gbs) {
    TSN_REQUIRE(mfma_tflops && hbm_gbs, "probe: null output");
    TSN_TRY(dev.make_current());
    const hipStream_t st = dev.stream();
    int ncu = 0;
    TSN_HIP_CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev.device()));
    TSN_REQUIRE(ncu > 0, "probe: no compute units");
    const size_t copy_bytes = (size_t)1 << 30;
    float *buf = nullptr, *src = nullptr, *dst = nullptr;
    TSN_TRY(dev.alloc((size_t)ncu * 512 * sizeof(float), (void **)&buf));
    int rc = dev.alloc(copy_bytes, (void **)&src);
    if (rc == TSN_OK) rc = dev.alloc(copy_bytes, (void **)&dst);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (rc == TSN_OK && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)) {
        set_error("probe: event creation failed");
        rc = TSN_ERR_HIP;
    }
    const int iters = 40000;   // about 20 ms: the sustained rate, after clocks settle under MFMA load
    float ms_mfma = 0.0f, ms_copy = 0.0f;
    if (rc == TSN_OK) rc = launch_mfma_peak(buf, ncu, 100, st);   // warm-up
    if (rc == TSN_OK && hipEventRecord(e0, st) != hipSuccess) rc = TSN_ERR_HIP;
    if (rc == TSN_OK) rc = launch_mfma_peak(buf, ncu, iters, st);
    if (rc == TSN_OK && hipEventRecord(e1, st) != hipSuccess) rc = TSN_ERR_HIP;
    if (rc == TSN_OK && (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms_mfma, e0, e1) != hipSuccess))
        rc = TSN_ERR_HIP;
    if (rc == TSN_OK) rc = launch_copy_peak(src, dst, copy_bytes / 16, st);   // warm-up
    if (rc == TSN_OK && hipEventRecord(e0, st) != hipSuccess) rc = TSN_ERR_HIP;
    for (int r = 0; r < 5 && rc == TSN_OK; ++r) rc = launch_copy_peak(src, dst, copy_bytes / 16, st);
    if (rc == TSN_OK && hipEventRecord(e1, st) != hipSuccess) rc = TSN_ERR_HIP;
    if (rc == TSN_OK && (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms_copy, e0, e1) != hipSuccess))
        rc = TSN_ERR_HIP;
    if (rc == TSN_ERR_HIP && last_error()[0] == 0) set_error("probe: HIP event failure");
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (dst) dev.free(dst);
    if (src) dev.free(src);
    dev.free(buf);
    if (rc != TSN_OK) return rc;
    *mfma_tflops = (double)ncu * 8 * iters * 16 * 16384.0 / (ms_mfma * 1e-3) / 1e12;
    *hbm_gbs = 5.0 * 2.0 * copy_bytes / (ms_copy * 1e-3) / 1e9;
    return TSN_OK;
}

} // namespace tsn
