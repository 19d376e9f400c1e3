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
    // device address of the allocation-free GEMM's static scratch on this GPU
    return noalloc_init(dev_);
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
    owned_sz_.push_back(bytes);
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
    owned_sz_.erase(owned_sz_.begin() + (it - owned_.begin()));
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

int Runtime::init(int device) {
    TSN_TRY(dev.init(device));
    return dev.alloc(SPLIT_WS_BYTES, (void **)&split_ws_);
}

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

namespace {
bool aligned16(const void *p) { return (((uintptr_t)p) & 15) == 0; }

// one plain-store GEMM: 64x64 tiles when asked for and the kernel takes it, else the classic K
// split chosen by estimated time (split_waves) when ws holds the partials, then the split-order
// reduce that applies bias, SiLU and the output type
int store_gemm(GemmBatch &b, float *ws, size_t ws_bytes, hipStream_t st) {
    b.ws = ws;
    b.ws_bytes = ws ? ws_bytes : 0;
    b.split_waves = 1;
    b.split_overhead = 10.0f;   // the reduce is an eager launch of its own (256x3072x1024 split in two
                                // measured 12.1 -> 15.7 us under the graph-replay charge of 2)
    TSN_TRY(launch_gemm(b, EPI_STORE, false, st));
    return gemm_needs_reduce(b) ? launch_gemm_reduce(b, EPI_STORE, st) : TSN_OK;
}
}

bool gemm_hilo_ok(const void *W, uint32_t ldw, const void *Y, int ydt, uint32_t ldy, const float *bias,
                  uint32_t M, uint32_t N, uint32_t K) {
    // what the pipelined kernel takes for a hi|lo operand (gemm_plan): K a multiple of 64, 8-aligned
    // strides, 16-byte aligned W, bias and Y, operand offsets below 2^31 bytes
    return M > 0 && N > 0 && K > 0 && K % 64 == 0 && ldw % 8 == 0 && ldw >= K && N % 8 == 0 && aligned16(W) &&
           aligned16(bias) && aligned16(Y) && ldy >= N && ldy % (ydt == DT_F16 ? 8 : 4) == 0 &&
           (unsigned long long)N * ldw * 2 < (1ULL << 31) && 4ULL * M * K * 2 < (1ULL << 31);
}

size_t gemm_hilo_bytes(uint32_t M, uint32_t K) { return (size_t)M * 2 * K * sizeof(half_t); }

int gemm_hilo(const half_t *W, uint32_t ldw, const float *X, uint32_t ldx, void *Y, int ydt, uint32_t ldy,
              const float *bias, uint32_t M, uint32_t N, uint32_t K, half_t *hl, float *ws, size_t ws_bytes,
              hipStream_t st) {
    TSN_REQUIRE(W && X && Y && hl && aligned16(hl), "gemm: null operand or unaligned operand buffer");
    TSN_REQUIRE(ydt == DT_F32 || ydt == DT_F16, "gemm: Y must be f32 or f16");
    TSN_REQUIRE(gemm_hilo_ok(W, ldw, Y, ydt, ldy, bias, M, N, K), "gemm: shape outside the hi|lo MFMA path");
    TSN_TRY(launch_split_hilo(X, (int)ldx, rowmap_dense((int)M), hl, (int)M, (int)K, st));
    GemmBatch b;
    gemm_problem_init(b.p[0]);
    GemmProblem &q = b.p[0];
    q.A = hl; q.lda = (int)(2 * K); q.amap = rowmap_dense((int)M);
    q.taps = 1; q.Kc = (int)(2 * K); q.pad = 0; q.a_T = (int)M;
    q.W = W; q.ldw = (int)ldw; q.w_half = 1; q.bias = bias;
    q.M = (int)M; q.N = (int)N; q.K = (int)(2 * K);
    q.Y = Y; q.ldy = (int)ldy; q.ymap = rowmap_dense((int)M); q.y_f16 = ydt == DT_F16;
    b.nprob = 1;
    return store_gemm(b, ws, ws_bytes, st);
}

int Runtime::gemm(int wdt, const void *W, const void *X, int xdt, void *Y, int ydt, const float *bias,
                  const GemmParams &p) {
    TSN_REQUIRE(W && X && Y, "gemm: null operand");
    TSN_REQUIRE(p.M > 0 && p.N > 0 && p.K > 0, "gemm: empty shape");
    const uint32_t ldx = p.ldx ? p.ldx : p.K, ldw = p.ldw ? p.ldw : p.K, ldy = p.ldy ? p.ldy : p.N;
    TSN_REQUIRE(ldx >= p.K && ldw >= p.K && ldy >= p.N, "gemm: leading dimension below the row width");
    TSN_TRY(dev.make_current());
    const hipStream_t st = dev.stream();
    if (wdt == DT_F16 && xdt == DT_F32) {
        // the reference's f32-activation contract (shaders/gemm_mpp.metal:19-25: X stays f32)
        if (gemm_hilo_ok(W, ldw, Y, ydt, ldy, bias, p.M, p.N, p.K)) {
            void *hl = nullptr;
            TSN_TRY(scratch(gemm_hilo_bytes(p.M, p.K), &hl));
            return gemm_hilo((const half_t *)W, ldw, (const float *)X, ldx, Y, ydt, ldy, bias, p.M, p.N, p.K,
                             (half_t *)hl, split_ws(), split_ws_bytes(), st);
        }
        if (ydt != DT_F32) {
            set_error("gemm: f32 X with f16 Y needs K % 64 == 0, N % 8 == 0 and 16-byte aligned W, bias and Y");
            return TSN_ERR_UNSUPPORTED;
        }
        // shapes outside the MFMA tiling: exact f32 products on the SIMT path
    } else if (wdt == DT_F16) {
        TSN_REQUIRE(xdt == DT_F16, "gemm: X must be f32 or f16");
        TSN_REQUIRE(ydt == DT_F32 || ydt == DT_F16, "gemm: Y must be f32 or f16");
        GemmBatch b;
        gemm_problem_init(b.p[0]);
        GemmProblem &q = b.p[0];
        q.A = X; q.lda = (int)ldx; q.amap = rowmap_dense((int)p.M);
        q.taps = 1; q.Kc = (int)p.K; q.pad = 0; q.a_T = (int)p.M;
        q.W = (const half_t *)W; q.ldw = (int)ldw; q.bias = bias;
        q.M = (int)p.M; q.N = (int)p.N; q.K = (int)p.K;
        q.Y = Y; q.ldy = (int)ldy; q.ymap = rowmap_dense((int)p.M); q.y_f16 = ydt == DT_F16;
        b.nprob = 1;
        b.small = 1;   // 64x64 tiles over the full K when the 128x128 grid is under one round
        return store_gemm(b, split_ws(), split_ws_bytes(), st);
    } else if (wdt == DT_BF16 && xdt == DT_BF16) {
        // bf16 operands on MFMA (bf16 products, f32 accumulation and Y)
        TSN_REQUIRE(ydt == DT_F32, "gemm: bf16 X and W give f32 Y");
        GemmBatch b;
        gemm_problem_init(b.p[0]);
        GemmProblem &q = b.p[0];
        q.A = X; q.lda = (int)ldx; q.amap = rowmap_dense((int)p.M);
        q.taps = 1; q.Kc = (int)p.K; q.pad = 0; q.a_T = (int)p.M;
        q.W = (const half_t *)W; q.ldw = (int)ldw; q.bias = bias;
        q.M = (int)p.M; q.N = (int)p.N; q.K = (int)p.K;
        q.Y = Y; q.ldy = (int)ldy; q.ymap = rowmap_dense((int)p.M); q.y_f16 = 0;
        b.nprob = 1;
        b.bf16 = 1;
        const int rc = gemm_plan(b, EPI_STORE, false);
        if (rc != TSN_OK) return rc == TSN_ERR_ARG ? TSN_ERR_UNSUPPORTED : rc;
        return gemm_launch_planned(b, EPI_STORE, false, st);
    } else {
        TSN_REQUIRE(wdt == DT_F32 || wdt == DT_BF16, "gemm: weight dtype");
        TSN_REQUIRE(xdt == DT_F32 && ydt == DT_F32, "gemm: f32/bf16 weights take f32 X and Y (or bf16 X with bf16 W)");
    }
    LinArgs a;
    a.X = (const float *)X; a.ldx = (int)ldx; a.xmap = rowmap_dense((int)p.M);
    a.W = W; a.ldw = (int)ldw; a.wdt = wdt; a.bias = bias;
    a.Y = (float *)Y; a.ldy = (int)ldy; a.ymap = rowmap_dense((int)p.M);
    a.M = (int)p.M; a.N = (int)p.N; a.K = (int)p.K;
    return launch_linear_f32(a, st);
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

int Runtime::conv_prepare(const void *W, int wdt, void *Wp, uint32_t OC, uint32_t IC, uint32_t K) {
    TSN_TRY(dev.make_current());
    return launch_conv_prepare(W, wdt, (half_t *)Wp, (int)OC, (int)IC, (int)K, dev.stream());
}

// Three routes, all f32-accurate (f16 weights: x as hi|lo against [W | W]; f32 weights: three-part
// products against [W_hi | W_hi | W_lo]):
//   * stride 1, dilation 1, IC % 64 == 0: implicit GEMM over the split input, taps in K (no im2col);
//   * other strides, dilations, transposed convs and channel counts: the gathered operand (the
//     reference's im2col, src/net.mm:36-48) in chunks of at most 64 MB, one GEMM per chunk;
//   * outputs too narrow for a GEMM tile (OC % 8 != 0) or unaligned: a direct f32 conv.
int Runtime::conv(int wdt, const void *Wp, const float *bias, const float *x, float *y, uint32_t T, uint32_t OL,
                  uint32_t IC, uint32_t OC, uint32_t K, uint32_t stride, uint32_t pad, uint32_t dil, uint32_t convt) {
    TSN_REQUIRE(Wp && x && y, "conv: null operand");
    TSN_REQUIRE(wdt == DT_F16 || wdt == DT_BF16 || wdt == DT_F32, "conv: weight dtype f16, bf16 or f32");
    TSN_REQUIRE(T > 0 && OL > 0 && IC > 0 && OC > 0 && K > 0 && stride > 0 && dil > 0,
                "conv: empty shape, or zero stride or dilation");
    TSN_REQUIRE((unsigned long long)OL * OC < (1ULL << 31) && (unsigned long long)T * IC < (1ULL << 31) &&
                    (unsigned long long)K * IC * 3 < (1ULL << 30) && pad < (1u << 30),
                "conv: sizes beyond 32-bit indexing");
    TSN_TRY(dev.make_current());
    const hipStream_t st = dev.stream();
    const int parts = wdt == DT_F32 ? 3 : 1;
    const int Kp = conv_prep_cols(wdt, (int)IC, (int)K);
    const ConvGeom g{(int)T, (int)OL, (int)IC, (int)OC, (int)K, (int)stride, (int)pad, (int)dil, convt ? 1 : 0,
                     (int)IC};
    if (OC % 8 != 0 || !aligned16(y) || !aligned16(bias) || !aligned16(Wp) ||
        (unsigned long long)OC * Kp * 2 >= (1ULL << 31))
        return launch_conv_direct(x, g, (const half_t *)Wp, parts, Kp, bias, y, st);
    GemmBatch b;
    gemm_problem_init(b.p[0]);
    GemmProblem &q = b.p[0];
    q.W = (const half_t *)Wp; q.ldw = Kp; q.bias = bias; q.w_half = parts == 1;
    q.N = (int)OC; q.ldy = (int)OC; q.y_f16 = 0;
    b.nprob = 1;
    const int ich = (int)IC * (parts == 1 ? 2 : 3);   // split input row: [hi | lo] or [hi | lo | hi]
    if (stride == 1 && dil == 1 && !convt && IC % 64 == 0 && aligned16(x) &&
        2ULL * (OL + T) * ich * 2 < (1ULL << 31)) {
        void *buf = nullptr;
        TSN_TRY(scratch((size_t)T * ich * sizeof(half_t), &buf));
        if (parts == 1) TSN_TRY(launch_split_hilo(x, (int)IC, rowmap_dense((int)T), (half_t *)buf, (int)T, (int)IC, st));
        else TSN_TRY(launch_split3(x, (long long)T, (int)IC, nullptr, 1, (half_t *)buf, st));
        q.A = buf; q.lda = ich; q.amap = rowmap_dense((int)OL);
        q.taps = (int)K; q.Kc = ich; q.pad = (int)pad; q.a_T = (int)T;
        q.M = (int)OL; q.K = (int)K * ich;
        q.Y = y; q.ymap = rowmap_dense((int)OL);
        return launch_gemm(b, EPI_STORE, false, st);
    }
    const int width = parts == 1 ? 2 * Kp : Kp;
    const size_t row_bytes = (size_t)width * sizeof(half_t);
    const uint32_t rows = (uint32_t)std::max<size_t>(1, std::min<size_t>(OL, ((size_t)64 << 20) / row_bytes));
    void *buf = nullptr;
    TSN_TRY(scratch((size_t)rows * row_bytes, &buf));
    for (uint32_t t0 = 0; t0 < OL; t0 += rows) {
        const uint32_t n = std::min(rows, OL - t0);
        TSN_TRY(launch_conv_gather(x, g, (int)t0, (int)n, parts, Kp, (half_t *)buf, st));
        q.A = buf; q.lda = width; q.amap = rowmap_dense((int)n);
        q.taps = 1; q.Kc = width; q.pad = 0; q.a_T = (int)n;
        q.M = (int)n; q.K = width;
        q.Y = y + (size_t)t0 * OC; q.ymap = rowmap_dense((int)n);
        TSN_TRY(launch_gemm(b, EPI_STORE, false, st));
    }
    return TSN_OK;
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

int Runtime::geglu(const float *a, const float *b, float *y, size_t n) {
    TSN_TRY(dev.make_current());
    return launch_geglu(a, b, y, n, dev.stream());
}
int Runtime::gelu_quick(float *x, size_t n) {
    TSN_TRY(dev.make_current());
    return launch_gelu_quick(x, n, dev.stream());
}
int Runtime::ln_plain(const float *x, float *y, uint32_t S, uint32_t H, float eps) {
    TSN_TRY(dev.make_current());
    return launch_ln_plain(x, y, (int)S, (int)H, eps, dev.stream());
}
int Runtime::ln_wb(const float *x, float *y, const float *w, const float *b, uint32_t S, uint32_t H, float eps) {
    TSN_REQUIRE(b, "ln_wb: null bias");
    TSN_TRY(dev.make_current());
    return launch_enc_norm(x, y, w, b, (int)S, (int)H, eps, true, dev.stream());
}
int Runtime::rms_w(const float *x, float *y, const float *w, uint32_t S, uint32_t H, float eps) {
    TSN_TRY(dev.make_current());
    return launch_enc_norm(x, y, w, nullptr, (int)S, (int)H, eps, false, dev.stream());
}
int Runtime::mean_cols(const float *x, float *y, uint32_t S, uint32_t H) {
    TSN_TRY(dev.make_current());
    return launch_mean_rows(x, (int)S, (int)H, y, dev.stream());
}
int Runtime::qkv_split3(const float *src, float *dst, uint32_t rows, uint32_t H, uint32_t row_off) {
    TSN_REQUIRE(src != dst, "qkv_split3: source and destination must differ");
    TSN_TRY(dev.make_current());
    return launch_qkv_split3(src, dst, (int)rows, (int)H, (int)row_off, dev.stream());
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
    // q * scale * log2(e) before the f16 rounding: the kernels' products are scores in log2 units
    TSN_TRY(launch_attn_pack(qkv, scale * 1.4426950408889634f, (int)S, (int)nh, (int)ld, (int)q_off, (int)k_off,
                             (int)v_off, Q, K, Vt, Sp, dev.stream()));
    AttnArgs a;
    memset(&a, 0, sizeof a);
    a.Q = Q; a.K = K; a.Vt = Vt; a.S = (int)S; a.Sp = Sp; a.nh = (int)nh; a.BH = (int)nh;
    a.O = out + o_off; a.o_f32 = 1; a.ldo = (int)ldo; a.omap = rowmap_dense((int)S);
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
