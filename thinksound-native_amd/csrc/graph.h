// graph.h — launch plumbing shared by the DiT graphs: owned allocations, per-launch profiling,
// GEMM plan + launch (+ split-K reduce), the fused residual reduce + adaLN, hipGraph capture and
// replay, and the builders of the GEMM problems and LN segments the blocks are made of.
#pragma once
#include <functional>
#include <string>
#include <vector>

#include "runtime.h"

namespace tsn {

// per-kernel statistics of one profiled evaluation (event pairs around every launch)
struct KernelStat {
    std::string name;   // kernel symbol
    int launches = 0;
    double ms = 0.0;     // summed event time
    double flops = 0.0;  // algorithmic: 2*M*N*K per GEMM (conv K = taps*IC), 4*B*NH*S^2*64 attention
    double bytes = 0.0;  // algorithmic HBM bytes (each operand once at its storage type)
};

struct ManifestEntry {
    std::string name;
    int64_t numel;
    int64_t offset;
};

// kernel symbols used as profile names
constexpr const char *K_ATTN = "flash_attn_kernel";
constexpr const char *K_GEMV = "gemv_kernel";
constexpr const char *K_LN16 = "ln_mod_kernel<1, 4>";
constexpr const char *K_LNHL = "ln_mod_kernel<2, 4>";
constexpr const char *K_SPLIT = "split_hilo_kernel";
constexpr const char *K_RLN16 = "reduce_ln_kernel<1>";
constexpr const char *K_RLNHL = "reduce_ln_kernel<2>";

class GraphRunner {
public:
    Runtime *rt = nullptr;
    virtual ~GraphRunner();
    // capture what enqueue() launches on the runtime's stream as a hipGraph (replacing any
    // previous one); replay() launches it again
    int capture(const std::function<int()> &enqueue);
    int replay();
    // run enqueue() eagerly with an event pair around every launch; stats per kernel symbol
    int profile(const std::function<int()> &enqueue, std::vector<KernelStat> &stats);

protected:
    struct ProfRec {
        const char *name;
        double flops, bytes;
        hipEvent_t a, b;
    };
    std::vector<ProfRec> *prof_ = nullptr;
    std::vector<void *> owned_;
    hipGraph_t graph_ = nullptr;
    hipGraphExec_t gexec_ = nullptr;

    int alloc(size_t bytes, void **p);   // zero-filled, freed with the runner
    // zero-initialised per-tile arrival counters for the stream-K kernel's own fixup
    // (GemmBatch::sk_cnt); gemm_run and resid_ln hand them to every batch once allocated
    static constexpr int SK_COUNTERS = 16384;
    int alloc_skcnt();
    unsigned *skcnt_ = nullptr;
    // frees one allocation made by alloc(); drops the captured graph, which may address it
    int release(void *p);
    void drop_graph();
    // launch() under the profiler when profiling (one record per launched kernel)
    template <typename F>
    int run(const char *name, double flops, double bytes, F &&launch) {
        if (!prof_) return launch();
        ProfRec r{name, flops, bytes, nullptr, nullptr};
        TSN_HIP_CHECK(hipEventCreate(&r.a));
        TSN_HIP_CHECK(hipEventCreate(&r.b));
        LaunchEvents &ev = next_launch_events();
        ev.start = r.a;
        ev.stop = r.b;
        const int rc = launch();
        const bool consumed = ev.start == nullptr;
        ev.start = ev.stop = nullptr;
        if (!consumed) {   // nothing was launched: no timing for this record
            hipEventDestroy(r.a);
            hipEventDestroy(r.b);
            return rc;
        }
        prof_->push_back(r);
        return rc;
    }
    // plan, launch (timed under the kernel's own symbol) and, when K was split, reduce; the
    // profiled algorithmic flops are gemm_flops(b) * flop_scale
    int gemm_run(GemmBatch &b, int epi, double flop_scale = 1.0);
    // residual GEMM batch + one reduce kernel that finishes the split-K sum into X and applies
    // the adaLN set up in r (segment i covers problem i's rows)
    int resid_ln(GemmBatch &b, RedLnArgs &r, int H, float eps);
};

double gemm_flops(const GemmBatch &b);
double gemm_bytes(const GemmBatch &b, int epi);
double ln_bytes(const LnArgs &a, bool f16);

// QKV problem: bias, per-head RMS (qn, kn), RoPE from `rope` for the first rope_len rows of each
// sample, q scaled by 1/8, heads stored to Q/K [b][h][S][64] and Vt [b][h][64][Sp]; rows of the
// stream at positions q_soff.. of each sample
void qkv_problem(GemmProblem &p, const half_t *A, RowMap amap, int M, const half_t *W, const float *bias,
                 const float *qn, const float *kn, int H, int nh, half_t *Q, half_t *K, half_t *Vt, int S, int Sp,
                 int q_L, int q_soff, int rope_len, const float *rope, float eps);
// gated residual: R += gate * (A·Wᵀ + bias); conv when taps > 1 (pad taps/2), gate per L rows
void resid_problem(GemmProblem &p, const half_t *A, int lda, RowMap amap, int taps, int Kc, int M, int N,
                   const half_t *W, const float *bias, float *R, int ldr, const float *gate, int gate_ld);
// f16 store of act(A·Wᵀ) (SiLU when silu), conv when taps > 1
void store_problem(GemmProblem &p, const half_t *A, int lda, RowMap amap, int taps, int Kc, int M, int N,
                   const half_t *W, half_t *Y, int ldy, int silu);
// LN segment: rows of X through map, modulation rows every L rows of mod (stride nmod)
void ln_seg(LnSeg &g, const float *X, int H, RowMap map, half_t *Y, const float *mod, int nmod, int L,
            int shift_off, int rows);

} // namespace tsn
