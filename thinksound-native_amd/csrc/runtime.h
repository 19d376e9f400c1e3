// runtime.h — HIP device harness and launcher runtime.
//
// Device replaces the reference's Metal harness tn::gpu::Device (src/gpu.h:20-48). The reference
// relies on unified memory (Buf.p is host and device at once, src/gpu.h:13-18); here memory is
// device memory, moved only by explicit upload()/download() on the runtime's one stream.
// begin()/commit() keep the reference's batching contract: launches are asynchronous and commit()
// waits, recording the GPU time between the two in last_gpu_ms() (src/gpu.mm:164-177).
//
// Runtime mirrors tn::Runtime (src/net.h:18-51): the same launcher names and argument meaning,
// plus the named kernels dit_fwd.cpp dispatches directly (adaln_ln, gate_add, rms_head,
// rope_pairs, attention; src/dit_fwd.cpp:16-102) as methods. Every call returns a TSN_* status.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "kernels.h"

namespace tsn {

struct GemmParams {  // src/net.h:13-16; a zero ld means the packed default
    uint32_t M, N, K;
    uint32_t ldx, ldw, ldy;
};

// Y = X·Wᵀ (+bias) with f32 X and f16 W as an f32-accurate MFMA product: X is split into an f16
// hi|lo pair in hl (M x 2K halves) and multiplied against [W | W]. gemm_hilo_ok tells whether the
// pipelined kernel takes the shape; hl needs gemm_hilo_bytes(M, K) bytes, 16-byte aligned. ws (f32,
// ws_bytes; null for none) holds the partial sums of a classic K split, taken when the 128x128 grid
// would leave most CUs idle over a long K; the partials are summed in split order, so the result
// depends only on the operands and ws_bytes (no stream-K, no atomics).
bool gemm_hilo_ok(const void *W, uint32_t ldw, const void *Y, int ydt, uint32_t ldy, const float *bias,
                  uint32_t M, uint32_t N, uint32_t K);
size_t gemm_hilo_bytes(uint32_t M, uint32_t K);
int gemm_hilo(const half_t *W, uint32_t ldw, const float *X, uint32_t ldx, void *Y, int ydt, uint32_t ldy,
              const float *bias, uint32_t M, uint32_t N, uint32_t K, half_t *hl, float *ws, size_t ws_bytes,
              hipStream_t st);

// The allocation-free GEMM (noalloc.hip): a fixed device array per GPU replaces the runtime scratch.
// noalloc_init takes that array's device address on `device` (which must be current); Device::init
// calls it once per runtime.
int noalloc_init(int device);
size_t noalloc_scratch_bytes();
class Runtime;
struct GemmParams;
int gemm_noalloc(Runtime &rt, int wdt, const void *W, const void *X, int xdt, void *Y, int ydt, const float *bias,
                 const GemmParams &p);

class Device {
public:
    ~Device();
    int init(int device);
    int alloc(size_t bytes, void **p);   // zero-filled device memory owned by the Device
    int free(void *p);
    int upload(void *dst, const void *src, size_t bytes);
    int download(void *dst, const void *src, size_t bytes);
    int copy_d2d(void *dst, const void *src, size_t bytes);
    int begin();
    int commit();
    int sync();
    double last_gpu_ms() const { return last_ms_; }
    hipStream_t stream() const { return stream_; }
    int device() const { return dev_; }
    int make_current() const;
    // live allocations owned by this Device (count and bytes as requested)
    size_t owned_count() const { return owned_.size(); }
    size_t owned_bytes() const {
        size_t b = 0;
        for (size_t s : owned_sz_) b += s;
        return b;
    }

private:
    int dev_ = -1;
    hipStream_t stream_ = nullptr;
    hipEvent_t ev0_ = nullptr, ev1_ = nullptr;
    bool begun_ = false;
    double last_ms_ = 0.0;
    std::vector<void *> owned_;
    std::vector<size_t> owned_sz_;   // bytes of owned_[i]
};

class Runtime {
public:
    Device dev;
    // the Device, then the split-K workspace (allocated here, once, so no GEMM call allocates it)
    int init(int device);

    // Y[M,N] = X[M,K]·W[N,K]ᵀ (+bias)                              (src/net.h:24-26)
    // wdt F16, X f32: f32-accurate MFMA product (X as an f16 hi|lo pair against [W | W]), Y f32 or f16;
    //   shapes the pipelined kernel does not take run the f32 SIMT path (Y f32 only).
    // wdt F16, X f16: plain f16 MFMA product. wdt BF16, X bf16: bf16 MFMA product (f32 Y; MFMA
    // tiling only). wdt F32 / BF16 with X f32: f32 SIMT path (X, Y f32).
    int gemm(int wdt, const void *W, const void *X, int xdt, void *Y, int ydt, const float *bias,
             const GemmParams &p);
    // y[n] = bias[n] + W[n,:]·x                                      (src/net.h:27-28)
    int gemv(const void *W, const float *X, float *Y, const float *bias, uint32_t N, uint32_t K,
             uint32_t ldw, int wdt);
    // Upload-time conv weight transform: W [OC][IC][K] (f16, bf16 or f32) -> Wp [OC][conv_prep_cols]
    // f16, tap-major (three parts per tap for f32 weights), zero padded.
    int conv_prepare(const void *W, int wdt, void *Wp, uint32_t OC, uint32_t IC, uint32_t K);
    // conv1d on a prepared weight (wdt = the dtype it was prepared from); x [T,IC] f32, y [OL,OC]
    // f32 (+bias); strided, dilated or transposed (convt) as the reference's im2col defines them.
    // f32-accurate for every weight dtype.                           (src/net.h:29-34)
    int conv(int wdt, const void *Wp, const float *bias, const float *x, float *y, uint32_t T, uint32_t OL,
             uint32_t IC, uint32_t OC, uint32_t K, uint32_t stride, uint32_t pad, uint32_t dil, uint32_t convt);
    // elementwise (src/net.h:37-49)
    int silu(float *x, size_t n);
    int copy(const float *x, float *y, size_t n);
    int swiglu(const float *a, const float *b, float *y, size_t n);
    int add_(const float *a, const float *b, float *y, size_t n);
    int add_bcast_col(const float *x, const float *v, float *y, uint32_t S, uint32_t H);
    int cfg_euler(const float *fc, const float *fu, float *x, size_t n, float cfg, float dt);
    int geglu(const float *a, const float *b, float *y, size_t n);
    int gelu_quick(float *x, size_t n);
    int ln_plain(const float *x, float *y, uint32_t S, uint32_t H, float eps);
    int ln_wb(const float *x, float *y, const float *w, const float *b, uint32_t S, uint32_t H, float eps);
    int rms_w(const float *x, float *y, const float *w, uint32_t S, uint32_t H, float eps);
    int mean_cols(const float *x, float *y, uint32_t S, uint32_t H);
    // named kernels of src/dit_fwd.cpp:16-22,83-102
    int adaln_ln(const float *x, const float *mod, void *y, int ydt, uint32_t rows, uint32_t H,
                 uint32_t per_row, uint32_t chunks, uint32_t base, float eps);
    int gate_add(const float *x, const float *f, const float *mod, float *y, uint32_t rows, uint32_t H,
                 uint32_t per_row, uint32_t chunks, uint32_t gate_idx);
    int qkv_split3(const float *src, float *dst, uint32_t rows, uint32_t H, uint32_t row_off);
    int rms_head(float *x, const float *w, uint32_t rows, uint32_t nh, uint32_t ld, uint32_t hd,
                 uint32_t col_off, uint32_t row_off, float eps);
    int rope_pairs(float *x, const int32_t *pos, uint32_t rows, uint32_t nh, uint32_t ld, uint32_t hd,
                   uint32_t col_off, uint32_t row_off, float fscale, float base);
    int attention(const float *qkv, float *out, uint32_t S, uint32_t nh, uint32_t hd, uint32_t ld,
                  uint32_t ldo, uint32_t q_off, uint32_t k_off, uint32_t v_off, uint32_t o_off, float scale);

    // calibration: achievable dense f16 MFMA TFLOP/s (one workgroup of 8 waves per CU) and
    // device-to-device copy GB/s (read + write of a 1 GiB buffer), timed with events on the stream
    int probe_peaks(double *mfma_tflops, double *hbm_gbs);

    // the f32 workspace of the f16 GEMM routes' K split: fixed size, allocated by init
    float *split_ws() const { return split_ws_; }
    size_t split_ws_bytes() const { return split_ws_ ? SPLIT_WS_BYTES : 0; }

private:
    // 8 Mi floats of partial sums: M*N*splits <= 8 Mi (794 x 1024 x 4 splits takes 3.3 Mi)
    static constexpr size_t SPLIT_WS_BYTES = (size_t)32 << 20;
    float *split_ws_ = nullptr;
    // grow-on-demand scratch (the role of the reference's im2col buffer, src/net.h:34)
    int scratch(size_t bytes, void **p);
    void *scratch_ = nullptr;
    size_t scratch_bytes_ = 0;
};

} // namespace tsn
