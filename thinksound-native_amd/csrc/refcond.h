// refcond.h — the reference's conditioning prep on one GPU: DitModel::prep_conditioning and
// DitModel::prep_text_arm (src/dit.cpp:55-191), once per generation / per CFG arm.
//
//   sync:  sync_f [sync_S][768] + sync_pos_emb[s % 8] -> conv k7 pad 3 + b -> SiLU -> SwiGLU conv-MLP
//          (k3) -> sync_gather [T][H]: row i = row floor((i + 0.5)*sync_S/T)
//   clip:  clip_f [C][1024] -> linear + b -> SiLU -> SwiGLU conv-MLP = clip_pp [C][H];
//          clip_fc = clip_cond_proj(mean of the clip_pp rows) [H]
//   text arm: text_cat [TS][2048] -> linear + b -> SiLU -> SwiGLU MLP = text_pp [TS][H];
//          gcmlp = SwiGLU MLP(text_cond_proj(gtext) + b + clip_fc) [H]
//
// Every GEMM reads f32-accurate f16 hi|lo operands (this runs once per generation, so the doubled K
// costs nothing that matters); the one-row steps are f32 GEMVs over f16 weights.
#pragma once
#include <vector>

#include "graph.h"

namespace tsn {

struct RefCondSpec {   // field meaning documented in include/tsn.h (tsn_refcond_spec)
    int H, F, T, C, sync_S, TS;
    int sync_dim, clip_dim, text_dim, gtext_dim;
};

std::vector<ManifestEntry> refcond_manifest(const RefCondSpec &s);
int refcond_spec_check(const RefCondSpec &s);
// geometry of a dur-second generation (src/pipeline.cpp:81-83), the reference's widths
RefCondSpec refcond_spec_for_duration(int dur_s);
// widths from a checkpoint's tensors (H from dit.hidden_dim, F and the feature widths from the
// input projections' shapes); geometry from the caller
int refcond_spec_from_gguf(const char *path, int T, int C, int sync_S, int TS, RefCondSpec *out);

class RefCondModel : public GraphRunner {
public:
    int create(Runtime *rt, const RefCondSpec &s);
    int upload_weights(const uint16_t *host_bf16, size_t numel);   // flat BF16, manifest order
    int upload_weights_f32(const float *host_f32, size_t numel);
    int load_gguf(const char *path);

    // device pointers: clip_f [C][clip_dim], sync_f [sync_S][sync_dim] -> clip_pp [C][H],
    // sync_gather [T][H], clip_fc [H]
    int enqueue_prep_conditioning(const float *clip_f, const float *sync_f, float *clip_pp, float *sync_gather,
                                  float *clip_fc);
    // text_cat [TS][text_dim], gtext [gtext_dim], clip_fc [H] -> text_pp [TS][H], gcmlp [H]
    int enqueue_prep_text_arm(const float *text_cat, const float *gtext, const float *clip_fc, float *text_pp,
                              float *gcmlp);

    RefCondSpec s{};

private:
    int upload(const void *host, bool src_f32, size_t numel);
    // hi|lo rows [rows][2H] at XA -> SwiGLU (w1|w3, taps) -> hi|lo HF -> w2 (taps) -> y f32 [rows][H]
    int swiglu_mlp(int rows, int taps, const half_t *W13, const half_t *W2, float *y);
    // hi|lo input [rows][2K] at IN -> (conv taps, pad taps/2) + b -> SiLU -> hi|lo XA [rows][2H]
    int proj_silu(int rows, int K, int taps, const half_t *W, const float *b);

    const float *pe_ = nullptr;
    const half_t *Ws0_ = nullptr, *W13s_ = nullptr, *W2s_ = nullptr;
    const half_t *Wc0_ = nullptr, *W13c_ = nullptr, *W2c_ = nullptr, *Wcfc_ = nullptr;
    const half_t *Wt0_ = nullptr, *W13t_ = nullptr, *W2t_ = nullptr, *Wtfc_ = nullptr;
    const half_t *Wg1_ = nullptr, *Wg3_ = nullptr, *Wg2_ = nullptr;
    const float *bs0_ = nullptr, *bc0_ = nullptr, *bcfc_ = nullptr, *bt0_ = nullptr, *btfc_ = nullptr;
    half_t *IN_ = nullptr, *XA_ = nullptr, *HF_ = nullptr;
    float *SMID_ = nullptr, *cmean_ = nullptr, *fc_ = nullptr, *ga_ = nullptr, *gb_ = nullptr;
    int32_t *idx_ = nullptr;   // sync row gathered for each latent row
    float *ws_ = nullptr;
    size_t ws_bytes_ = 0;
    void *wraw_ = nullptr;
    bool ready_ = false;
};

} // namespace tsn
