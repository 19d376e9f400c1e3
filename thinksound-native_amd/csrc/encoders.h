// encoders.h — the reference's text encoders on one GPU, f32 throughout (the reference loads both
// checkpoints as f32, src/clip.cpp:7, src/t5.cpp:22):
//
//   CLIP (src/clip.cpp:34-122): x = tok_emb[ids] + pos_emb; NL x { x += out(attn(LN1(x))) with the
//   causal / end-of-text mask; x += fc2(quick_gelu(fc1(LN2(x)))) }; per_token = out_ln(x);
//   global = text_proj · per_token[eos], eos = the first position of the largest id.
//   T5 v1.1 (src/t5.cpp:39-131): x = tok_emb[ids]; NL x { x += o(attn(rms(x))) with the bucketed
//   relative bias (shared by all layers, scale 1) and pad-key mask; x += wo(gelu_tanh(wi_0 h) *
//   wi_1 h), h = rms(x) }; out = rms(x) · out_norm.
//
// q, k, v weights run as one GEMM (rows concatenated at upload), as do wi_0 and wi_1.
#pragma once
#include <vector>

#include "graph.h"

namespace tsn {

constexpr size_t ENC_WS_BYTES = (size_t)32 << 20;   // split-K partials of the f32 GEMMs

struct ClipSpec {   // field meaning documented in include/tsn.h (tsn_clip_spec)
    int H, NL, NH, ctx, vocab;
    float eps;
};
struct T5Spec {   // include/tsn.h (tsn_t5_spec)
    int d, d_ff, NL, NH, ctx, vocab, n_bucket, max_dist;
    float eps;
};

std::vector<ManifestEntry> clip_manifest(const ClipSpec &s);
std::vector<ManifestEntry> t5_manifest(const T5Spec &s);
int clip_spec_check(const ClipSpec &s);
int t5_spec_check(const T5Spec &s);
ClipSpec clip_spec_default();   // MetaCLIP text tower of the reference: 1024, 24 layers, 16 heads, 77
T5Spec t5_spec_default();       // T5 v1.1 XL encoder: 2048, 5120, 24 layers, 32 heads, 77, 32 buckets, 128
int clip_spec_from_gguf(const char *path, ClipSpec *out);   // clip.* metadata
int t5_spec_from_gguf(const char *path, T5Spec *out);       // t5.* metadata
// bidirectional bucket of relative position rel = k - q (src/t5.cpp:6-19)
int t5_bucket(int rel, int n_bucket, int max_dist);

class ClipModel : public GraphRunner {
public:
    int create(Runtime *rt, const ClipSpec &s);
    int upload_weights(const float *host, size_t numel);   // flat f32, manifest order
    int load_gguf(const char *path);
    // ids [ctx] (host) -> per_token [ctx][H], global [H] (device)
    int encode(const int32_t *ids_host, float *per_token, float *global);

    ClipSpec s{};

private:
    struct Layer {
        const float *ln1w, *ln1b, *Wqkv, *bqkv, *Wo, *bo, *ln2w, *ln2b, *W1, *b1, *W2, *b2;
    };
    std::vector<Layer> L_;
    const float *tok_ = nullptr, *pos_ = nullptr, *lnw_ = nullptr, *lnb_ = nullptr, *proj_ = nullptr;
    float *X_ = nullptr, *R_ = nullptr, *QKV_ = nullptr, *ATT_ = nullptr, *FF_ = nullptr, *ws_ = nullptr;
    int32_t *ids_ = nullptr;
    bool ready_ = false;
    int upload(const float *host, size_t numel);
};

class T5Model : public GraphRunner {
public:
    int create(Runtime *rt, const T5Spec &s);
    int upload_weights(const float *host, size_t numel);   // flat f32, manifest order
    int load_gguf(const char *path);
    // ids [ctx] (host) -> out [ctx][d] (device)
    int encode(const int32_t *ids_host, float *out);

    T5Spec s{};

private:
    struct Layer {
        const float *an, *Wqkv, *Wo, *fn, *Wi, *Wout;
    };
    std::vector<Layer> L_;
    const float *tok_ = nullptr, *rel_ = nullptr, *on_ = nullptr;
    float *X_ = nullptr, *R_ = nullptr, *QKV_ = nullptr, *ATT_ = nullptr, *U_ = nullptr, *G_ = nullptr, *ws_ = nullptr;
    int32_t *ids_ = nullptr, *pad_ = nullptr, *bucket_ = nullptr;
    bool ready_ = false;
    int upload(const float *host, size_t numel);
};

} // namespace tsn
