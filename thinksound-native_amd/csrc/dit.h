// dit.h — the 21-block MMDiT velocity evaluation and the CFG Euler sampler on one GPU.
//
// Mirrors tn::DitModel (src/models.h:55-85): load weights once, then forward() per velocity
// evaluation (src/dit_fwd.cpp:104-304) and the sampler loop of src/pipeline.cpp:141-155.
// CFG arms are folded into the batch (sample 2p = conditional, 2p+1 = unconditional arm of
// prompt p), so one forward evaluates both arms.
//
// HBM layout (B samples, S = La + Lt rows per sample, audio rows first):
//   X   f32 [B][S][H]      residual stream, updated in place by GEMM epilogues
//   XN  f16 [B][S][H]      LayerNorm + adaLN output (GEMM A operand)
//   Q,K f16 [B][NH][S][64] attention layout written by the QKV epilogue (RMS + RoPE applied)
//   Vt  f16 [B][NH][64][Sp] V transposed, Sp = S rounded up to 64, keys >= S kept zero
//   AO  f16 [B][S][H]      attention output
//   HF  f16 [B][S][F]      FFN hidden (SiLU applied)
//   MOD f32 [B][NMOD]      every adaLN modulation of the eval, from one batched GEMV
#pragma once
#include <vector>

#include "graph.h"

namespace tsn {

struct DitSpec {   // field meaning documented in include/tsn.h (tsn_dit_spec)
    int B, La, Lt;
    int H, NH, HD, F;
    int latent, temb_dim;
    int n_joint, n_fused;
    int audio_ffn_conv;
    float rope_theta, t_max_period, ln_eps, rms_eps;
};

std::vector<ManifestEntry> dit_manifest(const DitSpec &s);
int dit_spec_check(const DitSpec &s);

class DitModel : public GraphRunner {
public:
    int create(Runtime *rt, const DitSpec &s);
    // WeightSet::load equivalent (src/net.mm:126-173): the flat BF16 buffer in manifest order is
    // uploaded once; GEMM weights become f16 (exact for |w| >= 2^-14), conv weights are reordered
    // to [OC][K][IC], biases and norm weights become f32, the adaLN weights are gathered into
    // one [NMOD][H] bf16 matrix.
    int upload_weights(const uint16_t *host_bf16, size_t numel);

    // one velocity evaluation, all device pointers: z [B][La][latent], t [B], text [B][Lt][H],
    // pooled [B][H] -> v [B][La][latent]. taps (optional): X after every block, [nblk][B][S][H].
    int enqueue_forward(const float *z, const float *t, const float *text, const float *pooled, float *v,
                        float *taps);
    // one joint block on X [B][S][H] in place with g [B][H] (silu applied inside)
    int enqueue_joint_block(int block, float *X, const float *g);
    int enqueue_fused_block(int block, float *X, const float *g);

    // sampler: x [P][La][latent] in/out, text [B][Lt][H], pooled [B][H] with B = 2P.
    // prepare_sample(steps) uploads the t schedule; call it before enqueue_sample (outside capture).
    int prepare_sample(int steps);
    int enqueue_sample(float *x, const float *text, const float *pooled, int steps, float cfg);

    // hipGraph of one forward on fixed pointers; replay() re-runs it
    int capture_forward(const float *z, const float *t, const float *text, const float *pooled, float *v);
    int capture_sample(float *x, const float *text, const float *pooled, int steps, float cfg);

    // one eager evaluation with a HIP event pair around every launch; stats per kernel symbol
    int profile_forward(const float *z, const float *t, const float *text, const float *pooled, float *v,
                        std::vector<KernelStat> &stats);

    DitSpec s{};
    int S = 0, Sp = 0, NMOD = 0;
    float *t_dev = nullptr;   // [B] scratch for host-supplied t

private:
    struct StreamW {
        const half_t *Wqkv = nullptr, *Wo = nullptr, *W1 = nullptr, *W2 = nullptr;
        const float *bqkv = nullptr, *bo = nullptr, *qn = nullptr, *kn = nullptr;
        int conv = 0;
        int mod_off = 0;
    };
    // The adaLN that follows a block's last residual GEMM, fused into that GEMM's reduce kernel:
    // the next joint block's, the next fused block's, the final layer's, or none.
    enum { NEXT_NONE = 0, NEXT_JOINT = 1, NEXT_FUSED = 2, NEXT_FINAL = 3 };
    struct Next {
        int kind, idx;
    };
    // timestep embedding -> t-MLP (+ pooled) -> silu -> every adaLN modulation, for `rows` rows
    // (t [rows], pooled rows [rows][H] at ld H or repeated with period per, outputs [rows][.]),
    // in GEMV batches of up to 16 rows; modulation rows [0, mod_rows) only
    int enqueue_conditioning(const float *t, int rows, const float *pooled, float *temb, float *h1, float *g,
                             float *gs, float *mod, int mod_rows, bool temb_done = false);
    int enqueue_eval(const float *z, const float *t, const float *text, const float *pooled, float *v, float *taps,
                     const float *mod_pre);
    bool ln_prefetch() const;
    bool grid_prefetch() const;
    void next_qkv_prefetch(RedLnArgs &r, GemmBatch &f2, Next next) const;
    int block_joint(int i, bool ln1, Next next);
    int block_fused(int i, bool ln1, Next next);
    void next_ln(RedLnArgs &r, Next next, const RowMap *maps, int nseg);
    int modulation(const float *gs, int row0, int rows);
    GemvArgs mod_args(const float *gs, int row0, int rows) const;
    // an evaluation's modulation rows are computed by free CUs of GEMM grids: block 0's by the
    // input projection's, later blocks' (and the final layer's) by the QKV grid of the block
    // before the one that reads them (B = 2, every QKV grid a single round)
    bool mod_grid_ok() const;
    int first_mod_rows() const;
    void next_mod_gemv(GemmBatch &qb, Next next) const;
    bool mod_in_grid_ = false;
    int gs_from_g(const float *g);

    std::vector<StreamW> ja_, jt_, fu_;
    const uint16_t *Wmod_ = nullptr, *Wt0_ = nullptr, *Wt2_ = nullptr;
    const half_t *Win2_ = nullptr, *Wfin2_ = nullptr;   // [W|W] f16 for the hi|lo projections
    const float *bmod_ = nullptr, *bt0_ = nullptr, *bt2_ = nullptr, *bin_ = nullptr, *bfin_ = nullptr;
    int fin_mod_off_ = 0;
    // the final adaLN + projection as one kernel (launch_final_out) where the shapes allow it
    bool final_fused() const { return s.H % 256 == 0 && s.H <= 2048 && s.latent % 16 == 0 && s.latent <= 64; }
    float *rope_ = nullptr;
    float *X_ = nullptr, *MOD_ = nullptr, *g_ = nullptr, *gs_ = nullptr, *temb_ = nullptr, *h1_ = nullptr;
    half_t *XF2_ = nullptr, *Z2_ = nullptr;               // hi|lo operands of the projections
    float *Vv_ = nullptr, *x2_ = nullptr, *tsched_ = nullptr;
    int tsched_steps_ = 0;
    // sampler: conditioning of every step computed before the step loop (rows = steps*B, padded
    // to 16): temb, h1, g, gs, modulation, and pooled repeated over 16 rows
    float *cond_ = nullptr, *temb_all_ = nullptr, *h1_all_ = nullptr, *g_all_ = nullptr, *gs_all_ = nullptr;
    float *mod_all_ = nullptr, *pooled_rep_ = nullptr;
    const float *mod_ = nullptr;      // modulation rows the blocks of the current evaluation read
    half_t *XN_ = nullptr, *Q_ = nullptr, *K_ = nullptr, *Vt_ = nullptr, *AO_ = nullptr, *HF_ = nullptr;
    void *wraw_ = nullptr, *wf16_ = nullptr;
    float *ws_ = nullptr;            // split-K partials of the residual GEMMs
    size_t ws_bytes_ = 0;
    bool ready_ = false;
};

} // namespace tsn
