// refdit.h — the reference checkpoint's own DiT graph on one GPU (src/dit_fwd.cpp:104-304).
//
// Mirrors tn::DitModel::forward (src/models.h:83-84) with its three token streams and the CFG
// arms folded into the batch (sample 2p = conditional, 2p+1 = unconditional arm of prompt p):
//   latent  T rows per sample   RoPE positions 0..T-1, per-row adaLN from extended_c
//   clip    C rows per sample   RoPE positions scaled by T/C, adaLN from silu(global_c)
//   text    TS rows per sample  no RoPE, adaLN from silu(global_c)
// Joint blocks attend over all S = T + C + TS rows of a sample; the last joint block is pre-only
// (clip and text rows are not updated after its attention); fused blocks run the latent rows
// alone; the final layer is a per-row adaLN and a k=7 conv to the latent channels.
//
// HBM layout (B samples, S rows per sample: latent, then clip, then text):
//   X    f32 [B][S][H]       residual streams, updated in place by GEMM epilogues
//   XN   f16 [B][S][2H]      adaLN output (GEMM A operand), hi at [0, H), lo at [H, 2H): LN1 of
//                            every stream (QKV operand), LN2 of the latent rows (FFN operand); rows
//                            [0, B*T) double as the input projection's hidden (hi|lo)
//   XE   f16 [B*T][2H]       silu(extended_c) as hi|lo, A operand of the per-row modulation GEMM
//   MODL f32 [B*T][NMODL]    per-row modulation: every latent and fused block (6 chunks), final (2)
//   MODG f32 [B][NMODG]      per-sample modulation of the clip and text streams (6, or 2 when pre-only)
//   Q,K  f16 [B][NH][S][64], Vt f16 [B][NH][64][Sp] (joint); VtF [B][NH][64][SpF] (fused, S = T)
//   AO   f16 [B][S][2H]      attention output as hi|lo
//   HF   f16 [B][S][2F]      SwiGLU hidden, hi|lo for latent rows
// Every QKV GEMM and the latent stream's out-proj and FFN GEMMs read hi|lo operands, each half
// against the same weight columns (f32-accurate operands); the clip and text out-proj and FFN read
// the hi halves only.
#pragma once
#include <map>
#include <string>
#include <vector>

#include "gguf.h"
#include "graph.h"

namespace tsn {

struct RefDitSpec {   // field meaning documented in include/tsn.h (tsn_refdit_spec)
    int B, T, C, TS;
    int H, NH, HD, F;
    int latent;
    int n_joint, n_fused;
    float rope_theta, t_max_period, ln_eps, rms_eps;
};

std::vector<ManifestEntry> refdit_manifest(const RefDitSpec &s);
int refdit_spec_check(const RefDitSpec &s);
// geometry of a generation of dur seconds (src/models.h:14-22, src/pipeline.cpp:81-83)
RefDitSpec refdit_spec_for_duration(int dur_s, int B);
// hyperparameters from a checkpoint's dit.* metadata and the SwiGLU width from its first latent
// FFN weight (src/dit.cpp:29-47); geometry B, T, C, TS from the caller
int refdit_spec_from_gguf(const char *path, int B, int T, int C, int TS, RefDitSpec *out);

class RefDitModel : public GraphRunner {
public:
    int create(Runtime *rt, const RefDitSpec &s);
    // WeightSet::load (src/net.mm:126-173) for a flat BF16 buffer in manifest order, with the
    // upload-time transforms: qkv rows de-interleaved to q|k|v blocks, conv weights tap-major
    // [OC][K][IC], w1/w3 interleaved in 64-row blocks for the SwiGLU epilogue, input and final conv
    // weights duplicated as [w | w] for f32-accurate hi|lo operands, all GEMM weights f16.
    int upload_weights(const uint16_t *host_bf16, size_t numel);
    // the same from an f32 buffer (dequantized checkpoint tensors)
    int upload_weights_f32(const float *host_f32, size_t numel);
    // every tensor of the manifest from a GGUF checkpoint (any of F32, F16, BF16, Q8_0): raw
    // payloads to HBM, converted there
    int load_gguf(const char *path);
    // bytes the last load_gguf moved to the device (the needed tensors' payloads)
    size_t load_bytes() const { return load_bytes_; }

    // one velocity evaluation, device pointers: x [B][T][latent], t [B], clip_pp [B][C][H],
    // text_pp [B][TS][H], gcmlp [B][H], sync_gather [B][T][H] -> v [B][T][latent].
    // taps (optional): X after every block, [n_joint + n_fused][B][S][H].
    int enqueue_forward(const float *x, const float *t, const float *clip_pp, const float *text_pp,
                        const float *gcmlp, const float *sync_gather, float *v, float *taps);
    // sampler (src/pipeline.cpp:141-155): x [B/2][T][latent] in/out; conditioning tensors [B][...]
    // per arm. prepare_sample(steps) before enqueue_sample (outside capture).
    int prepare_sample(int steps);
    int enqueue_sample(float *x, const float *clip_pp, const float *text_pp, const float *gcmlp,
                       const float *sync_gather, int steps, float cfg);

    int capture_forward(const float *x, const float *t, const float *clip_pp, const float *text_pp,
                        const float *gcmlp, const float *sync_gather, float *v);
    int capture_sample(float *x, const float *clip_pp, const float *text_pp, const float *gcmlp,
                       const float *sync_gather, int steps, float cfg);
    int profile_forward(const float *x, const float *t, const float *clip_pp, const float *text_pp,
                        const float *gcmlp, const float *sync_gather, float *v, std::vector<KernelStat> &stats);

    RefDitSpec s{};
    int S = 0, Sp = 0, SpF = 0, NMODL = 0, NMODG = 0;
    float *t_dev = nullptr;   // [B] scratch for host-supplied t

private:
    struct StreamW {
        const half_t *Wqkv = nullptr, *Wo = nullptr, *W13 = nullptr, *W2 = nullptr;
        const float *bqkv = nullptr, *bo = nullptr, *qn = nullptr, *kn = nullptr;
        int taps = 1;      // 3: conv k3 out-proj and FFN, 1: linear
        int post = 1;      // 0: pre-only stream (no out-proj, no FFN)
        int mod_off = 0;   // first modulation column (MODL for latent/fused, MODG for clip/text)
        int hl = 0;        // out-proj / FFN GEMMs over hi|lo operands (latent rows), half-width W
    };
    enum { NEXT_NONE = 0, NEXT_JOINT = 1, NEXT_FUSED = 2, NEXT_FINAL = 3 };
    enum { ST_LAT = 0, ST_CLIP = 1, ST_TEXT = 2 };
    struct Next {
        int kind, idx;
    };
    int upload(const void *host, bool src_f32, size_t numel);
    int enqueue_conditioning(const float *t, int rows, const float *gcmlp, float *temb, float *h1, float *gc,
                             float *gs, float *modg);
    int enqueue_eval(const float *x, const float *t, const float *clip_pp, const float *text_pp, const float *gcmlp,
                     const float *sync_gather, float *v, float *taps, const float *gc_pre, const float *modg_pre);
    int block_joint(int i, bool ln1, Next next);
    int block_fused(int i, bool ln1, Next next);
    RowMap stream_map(int kind) const;
    void ln1_seg(LnSeg &g, int kind, const StreamW &w);
    void next_ln(RedLnArgs &r, Next next, const int *kinds, int nseg, bool ln2 = false);

    std::vector<StreamW> jl_, jc_, jt_, fu_;
    const half_t *WmodL_ = nullptr;                       // [NMODL][H] f16
    const half_t *WmodG_ = nullptr, *Wt0_ = nullptr, *Wt2_ = nullptr;   // f16 GEMV weights
    const float *bmodL_ = nullptr, *bmodG_ = nullptr, *bt0_ = nullptr, *bt2_ = nullptr;
    const half_t *Win_ = nullptr, *W13in_ = nullptr, *W2in_ = nullptr, *Wfin_ = nullptr;
    const float *bin_ = nullptr, *bfin_ = nullptr;
    int fin_off_ = 0;
    float *rope_l_ = nullptr, *rope_c_ = nullptr;
    float *X_ = nullptr, *MODL_ = nullptr, *MODG_ = nullptr;
    float *temb_ = nullptr, *h1_ = nullptr, *gc_ = nullptr, *gs_ = nullptr;
    half_t *XN_ = nullptr, *XE_ = nullptr, *Z2_ = nullptr, *XF2_ = nullptr;
    half_t *Q_ = nullptr, *K_ = nullptr, *Vt_ = nullptr, *VtF_ = nullptr, *AO_ = nullptr, *HF_ = nullptr;
    const float *modg_ = nullptr;   // per-sample modulation rows the current evaluation reads
    float *ws_ = nullptr;
    size_t ws_bytes_ = 0;
    void *wraw_ = nullptr;
    size_t load_bytes_ = 0;
    int prepare(const std::map<std::string, GgufDeviceTensor> &raw);
    // sampler state
    float *Vv_ = nullptr, *x2_ = nullptr, *tsched_ = nullptr;
    int tsched_steps_ = 0;
    float *cond_ = nullptr, *temb_all_ = nullptr, *h1_all_ = nullptr, *gc_all_ = nullptr, *gs_all_ = nullptr;
    float *modg_all_ = nullptr, *gcmlp_rep_ = nullptr;
    bool ready_ = false;
};

} // namespace tsn
