// vae.h — the reference's VAE decoder on one GPU: VaeModel::decode (src/vae.cpp:17-86).
//
//   latent [T][64] -> conv k7 pad 3 (+b) -> 5 stages { snake -> transposed conv (stride s, kernel
//   2s, +b) -> 3 residual units (dilation 1, 3, 9): x += conv_k1(snake(conv_k7_dil(snake(x)))) }
//   -> snake -> conv k7 pad 3 (no bias) -> audio [T*prod(s)][2]
//
// The reference keeps this network in f32 (src/vae.cpp:12). Every GEMM here runs f32-accurate
// on f16 MFMA with three products per term: the activation row is stored [hi | lo | hi] and the
// weight row [W_hi | W_hi | W_lo], so one f16 GEMM over K = 3*IC sums hi*W_hi + lo*W_hi + hi*W_lo
// (the dropped lo*W_lo term is below 2^-22 relative). The residual stream x stays f32.
//
// Every snake runs in the epilogue of the GEMM that produces its input (the residual units' closing
// k1 conv writes x and snake(x) for the next unit or stage), so x is read once per GEMM.
//
// Transposed convs are decomposed by output phase: output row s*q + r reads input rows q + c_r + j
// (j < K/s) with weight taps k0(r) + j*s, k0(r) = (pad - r) mod s, c_r = -floor((pad - r)/s). Phases
// with the same c_r form one conv GEMM whose N stacks the phases (N = phases*OC); written with row
// stride s*OC, its output is the interleaved [T*s][OC] rows directly, with no zero-stuffed input.
#pragma once
#include <vector>

#include "graph.h"

namespace tsn {

struct VaeSpec {   // field meaning documented in include/tsn.h (tsn_vae_spec)
    int T, latent;
    int width[6];
    int stride[5];
    int kt[5];
    int out_ch;
};

std::vector<ManifestEntry> vae_manifest(const VaeSpec &s);
int vae_spec_check(const VaeSpec &s);
long long vae_audio_len(const VaeSpec &s);
// geometry of a dur-second generation (T = llround(44100/2048*dur), src/models.h:16-21) with the
// reference decoder's widths and strides
VaeSpec vae_spec_for_duration(int dur_s);
// widths and transposed-conv kernel sizes from a checkpoint's tensor shapes; T from the caller
int vae_spec_from_gguf(const char *path, int T, VaeSpec *out);

class VaeModel : public GraphRunner {
public:
    int create(Runtime *rt, const VaeSpec &s);
    int upload_weights(const float *host_f32, size_t numel);   // flat f32, manifest order
    int load_gguf(const char *path);
    // latent [T][latent] -> audio [T_audio][out_ch], device pointers (f32)
    int enqueue_decode(const float *latent, float *audio);

    VaeSpec s{};

private:
    struct Unit {   // one residual unit
        const float *ab1 = nullptr, *ab2 = nullptr;   // snake tables [exp(alpha) | exp(-beta)]
        const half_t *W7 = nullptr, *W1 = nullptr;    // [C][7][3C], [C][3C]
        const float *b7 = nullptr, *b1 = nullptr;
    };
    struct Stage {
        const float *ab_in = nullptr;   // snake before the transposed conv, [2][C_in]
        int ngroups = 0, taps = 0;
        int r0[2] = {0, 0}, nph[2] = {0, 0}, pad[2] = {0, 0};   // phase group: first phase, phases, row pad
        const half_t *Wt[2] = {nullptr, nullptr};               // [nph*C_out][taps][3 C_in]
        const float *bt[2] = {nullptr, nullptr};                // bias repeated per phase
        const float *abt[2] = {nullptr, nullptr};               // first unit's snake table, per phase
        Unit u[3];
    };
    Stage st_[5];
    const half_t *W0_ = nullptr;
    const float *b0_ = nullptr, *ab_out_ = nullptr, *Wout_ = nullptr;
    float *X_ = nullptr, *ones_ = nullptr, *ws_ = nullptr;
    half_t *A1_ = nullptr, *A2_ = nullptr;
    size_t ws_bytes_ = 0;
    bool ready_ = false;
    int upload(const float *host, size_t numel);
};

} // namespace tsn
