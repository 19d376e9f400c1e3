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

private:
    int dev_ = -1;
    hipStream_t stream_ = nullptr;
    hipEvent_t ev0_ = nullptr, ev1_ = nullptr;
    bool begun_ = false;
    double last_ms_ = 0.0;
    std::vector<void *> owned_;
};

class Runtime {
public:
    Device dev;
    int init(int device) { return dev.init(device); }

    // Y[M,N] = X[M,K]·W[N,K]ᵀ (+bias). wdt F16: MFMA path, X f32 or f16, Y f32 or f16.
    // wdt F32 / BF16: f32 SIMT path (X, Y f32).                    (src/net.h:24-26)
    int gemm(int wdt, const void *W, const void *X, int xdt, void *Y, int ydt, const float *bias,
             const GemmParams &p);
    // y[n] = bias[n] + W[n,:]·x                                      (src/net.h:27-28)
    int gemv(const void *W, const float *X, float *Y, const float *bias, uint32_t N, uint32_t K,
             uint32_t ldw, int wdt);
    // Upload-time weight transform for conv: [OC][IC][K] f16 -> [OC][K][IC] f16.
    int conv_prepare(const void *W, int w_bf16, void *Wp, uint32_t OC, uint32_t IC, uint32_t K);
    // conv1d on a prepared weight; x [T,IC] f32, y [OL,OC] f32 (+bias). stride = dil = 1,
    // OL = T + 2*pad - K + 1, IC % 64 == 0 unless K == 1.            (src/net.h:29-34)
    int conv(const void *Wp, const float *bias, const float *x, float *y, uint32_t T, uint32_t OL,
             uint32_t IC, uint32_t OC, uint32_t K, uint32_t stride, uint32_t pad, uint32_t dil);
    // elementwise (src/net.h:37-49)
    int silu(float *x, size_t n);
    int copy(const float *x, float *y, size_t n);
    int swiglu(const float *a, const float *b, float *y, size_t n);
    int add_(const float *a, const float *b, float *y, size_t n);
    int add_bcast_col(const float *x, const float *v, float *y, uint32_t S, uint32_t H);
    int cfg_euler(const float *fc, const float *fu, float *x, size_t n, float cfg, float dt);
    // named kernels of src/dit_fwd.cpp:16-22,83-102
    int adaln_ln(const float *x, const float *mod, void *y, int ydt, uint32_t rows, uint32_t H,
                 uint32_t per_row, uint32_t chunks, uint32_t base, float eps);
    int gate_add(const float *x, const float *f, const float *mod, float *y, uint32_t rows, uint32_t H,
                 uint32_t per_row, uint32_t chunks, uint32_t gate_idx);
    int rms_head(float *x, const float *w, uint32_t rows, uint32_t nh, uint32_t ld, uint32_t hd,
                 uint32_t col_off, uint32_t row_off, float eps);
    int rope_pairs(float *x, const int32_t *pos, uint32_t rows, uint32_t nh, uint32_t ld, uint32_t hd,
                   uint32_t col_off, uint32_t row_off, float fscale, float base);
    int attention(const float *qkv, float *out, uint32_t S, uint32_t nh, uint32_t hd, uint32_t ld,
                  uint32_t ldo, uint32_t q_off, uint32_t k_off, uint32_t v_off, uint32_t o_off, float scale);

    // calibration: achievable dense f16 MFMA TFLOP/s (one workgroup of 8 waves per CU) and
    // device-to-device copy GB/s (read + write of a 1 GiB buffer), timed with events on the stream
    int probe_peaks(double *mfma_tflops, double *hbm_gbs);

private:
    // grow-on-demand scratch (the role of the reference's im2col buffer, src/net.h:34)
    int scratch(size_t bytes, void **p);
    void *scratch_ = nullptr;
    size_t scratch_bytes_ = 0;
};

} // namespace tsn
