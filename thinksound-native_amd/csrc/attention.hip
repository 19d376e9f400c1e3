// attention.hip — joint audio+text flash attention for gfx950 (hd = 64, non-causal).
//
// Replaces the reference's three-pass attention (src/dit_fwd.cpp:83-102 dispatching
// shaders/gemm_attn.metal:96-202: attn_qk materialises [nh,S,S] f32 scores, softmax_rows runs one
// thread per row, attn_pav reads the scores back). Here one workgroup owns 64 queries of one
// (sample, head) and the softmax is online, so no score buffer exists.
//
// 8 waves: wave w serves queries 16*(w&3)..+15; waves 0-3 take the even 64-key blocks and waves
// 4-7 the odd ones, each half keeping its own running max / sum / output; at the end each half
// merges and stores 32 of the 64 output columns through LDS. K and Vᵀ blocks reach LDS by
// direct-to-LDS buffer loads (no register staging). At S <= 512 all of them (128 KB) are loaded
// at once, every K block before the Vᵀ blocks are needed,
// and each half's key loop is software-pipelined (the next block's scores are multiplied before
// this block's PV product); longer contexts use a two-stage ring. The running max is shared by the
// four lanes holding a query's keys (row-swap permutes); the running sum is an MFMA product of the
// probabilities with ones.
//
// MFMA formulation (v_mfma_f32_16x16x32_f16; A row = lane&15, B col = lane&15, K group = lane>>4,
// D[4*(lane>>4)+r][lane&15]):
//   Sᵀ = K·Qᵀ  : A = K rows from LDS (row order permuted, see compute), B = the wave's Q rows
//                (registers). Lane l then holds the scores of query l&15 for keys 32c + 8g + 0..7
//                of each 32-key chunk c (g = l>>4).
//   Oᵀ += Vᵀ·Pᵀ: B = the lane's own probabilities (those 8 keys are the 8 K-values of group g),
//                A = Vᵀ rows read from LDS, one 16-byte chunk per lane. Lane l holds
//                Oᵀ[d = 16dt + 4g + r][query l&15], so the per-query rescale and 1/l are lane-local.
// Probabilities are rounded to f16 before both the PV product and the row sum, so numerator and
// denominator see the same values.
//
// LDS rows are 128 B (64 halves = 8 chunks of 16 B); chunk c of row r sits at slot c ^ sw(r).
#include "kernels.h"

namespace tsn {

namespace {

constexpr int AKB = 64;       // keys per block
constexpr int ASTAGE = 16384; // halves per stage

typedef __attribute__((address_space(3))) char lds_char;
typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ inline half8 zero_h8() { return half8{0, 0, 0, 0, 0, 0, 0, 0}; }

__device__ __forceinline__ i32x4 make_rsrc(const void *p) {
    const unsigned long long a = (unsigned long long)p;
    return i32x4{(int)(unsigned)a, (int)((a >> 32) & 0xFFFF), 0x7FFFFFFF, 0x00020000};
}
// 16 bytes per lane, global -> LDS slot (lane) of the 1 KB block at lds (see gemm.hip: issued from
// inline asm and ordered by explicit vmcnt waits; s_nop 0 covers the M0 -> LDS-DMA hazard)
__device__ __forceinline__ void dma16(i32x4 rs, unsigned voff, lds_char *lds) {
    const unsigned l = __builtin_amdgcn_readfirstlane((unsigned)(unsigned long)lds);
    // the resource is wave-uniform; make that explicit so it is kept in SGPRs
    rs = i32x4{__builtin_amdgcn_readfirstlane(rs[0]), __builtin_amdgcn_readfirstlane(rs[1]),
               __builtin_amdgcn_readfirstlane(rs[2]), __builtin_amdgcn_readfirstlane(rs[3])};
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(voff), "s"(rs), "s"(l)
                 : "memory");
}
// s_waitcnt vmcnt(n) (n in {0, 4, 8, 12}), expcnt/lgkmcnt left at their maxima
__device__ __forceinline__ void wait_vmcnt(int n) {
    if (n >= 12) __builtin_amdgcn_s_waitcnt(12 | (7 << 4) | (0xF << 8));
    else if (n >= 8) __builtin_amdgcn_s_waitcnt(8 | (7 << 4) | (0xF << 8));
    else if (n >= 4) __builtin_amdgcn_s_waitcnt(4 | (7 << 4) | (0xF << 8));
    else __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (0xF << 8));
}
// s_waitcnt lgkmcnt(0), then s_barrier: this wave's LDS reads have completed before any wave
// passes, so a stage refilled by direct-to-LDS DMA after the barrier is never still being read
// (s_barrier alone does not wait for them, and the compiler issues the next MFMAs' operand reads
// ahead of it)
__device__ __forceinline__ void block_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);   // vmcnt 63, expcnt 7: no wait; lgkmcnt 0
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Max over the four 16-lane rows holding one query's keys (lanes l, l^16, l^32, l^48),
// with the gfx950 row-swap permutes (VALU, no LDS round trip). permlane16_swap(x, x) yields the
// even-row and the odd-row copy of each row pair, permlane32_swap(x, x) the lower- and the
// upper-half copy; combining them gives every lane of a group the same value.
// With NaNs ruled out at compile time (this file's flags) fmaxf is one v_max_f32, and nested
// fmaxf of three operands one v_max3_f32 (no quieting of the operands).
__device__ __forceinline__ float max2f(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ float max3f(float a, float b, float c) { return fmaxf(fmaxf(a, b), c); }
__device__ __forceinline__ float rows_max(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = max2f(__uint_as_float(p[0]), __uint_as_float(p[1]));
    const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return max2f(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
// maximum of the lane's scores in the first nj (2 or 4) 16-key MFMA blocks: 4 or 8 instructions
__device__ __forceinline__ float lane_max(const floatx4 (&sc)[4], int nj) {
    float m = max3f(sc[0][0], sc[0][1], sc[0][2]);
    m = max3f(m, sc[0][3], sc[1][0]);
    m = max3f(m, sc[1][1], sc[1][2]);
    if (nj <= 2) return max2f(m, sc[1][3]);
    m = max3f(m, sc[1][3], sc[2][0]);
    m = max3f(m, sc[2][1], sc[2][2]);
    m = max3f(m, sc[2][3], sc[3][0]);
    m = max3f(m, sc[3][1], sc[3][2]);
    return max2f(m, sc[3][3]);
}

// LDS slot of 16-byte chunk c of row r: c ^ sw(r). Rows 8 apart get different slots too, so the
// 16 rows one operand read touches (K rows 8 apart, see below) fall in distinct banks.
__device__ __forceinline__ int sw(int r) { return (r & 7) ^ ((r >> 3) & 7); }

// Online softmax of one 16-query group, with the reference subtracted inside the score product.
// Q holds q * scale * log2(e), so q.k is the score s in log2 units, and the QK product of a key
// block starts from the accumulator nb = -base: it yields s - base with no per-score VALU. base
// is the running reference m (0 before the first block, where m holds the sentinel -1e30, whose
// exp2 differences are 0). The reference moves only when a block's row maximum exceeds it by
// more than 8, so the probabilities exp2(s - m) stay below 2^8 (well inside f16) and most blocks
// skip the rescale of O and the row sum and the shift of the scores: the common path is the row
// maximum, one compare, and per score one exp2 and half a packed f16 conversion. The wave branches
// on whether any of its lanes moves; a lane that does not keeps alpha = 1 and shift = 0. The
// result is the softmax of the same scores: numerator and denominator share every factor.
// (A branchless form, one exp2 and 20 multiplies every block, measured 0.35% slower per 8 s
// evaluation in the pipelined resident path.)
struct SoftRef {
    float m = -1e30f, base = 0.0f;
    floatx4 nb = floatx4{0.f, 0.f, 0.f, 0.f};   // -base, the QK products' initial accumulator
};
// sc = s - base for the first nj 16-key blocks (-inf for masked keys); on return pf holds the f16
// probabilities (zero beyond nj blocks) as the PV product's two B operands
__device__ __forceinline__ void block_probs(floatx4 (&sc)[4], int nj, SoftRef &R, floatx4 (&o)[4], floatx4 &lsum,
                                            half8 (&pf)[2]) {
    const float mb = R.base + rows_max(lane_max(sc, nj));   // the block's row maximum
    const bool up = mb > R.m + 8.0f;
    if (__builtin_amdgcn_ballot_w64(up) != 0) {
        const float m_new = up ? mb : R.m;
        const float alpha = __builtin_amdgcn_exp2f(R.m - m_new), shift = m_new - R.base;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
        lsum *= alpha;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (j < nj) sc[j] -= shift;
        R.m = m_new;
        R.base = m_new;
        R.nb = floatx4{-m_new, -m_new, -m_new, -m_new};
    }
    half_t ph[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) ph[j][r] = j < nj ? (half_t)__builtin_amdgcn_exp2f(sc[j][r]) : (half_t)0.0f;
#pragma unroll
    for (int c = 0; c < 2; ++c)
        pf[c] = half8{ph[2 * c][0], ph[2 * c][1], ph[2 * c][2], ph[2 * c][3],
                      ph[2 * c + 1][0], ph[2 * c + 1][1], ph[2 * c + 1][2], ph[2 * c + 1][3]};
}
__device__ inline int attn_xcd_remap(int bid, int nwg) {
    const int xcd = bid & 7, idx = bid >> 3;
    const int base = nwg >> 3, rem = nwg & 7;
    return (xcd < rem ? xcd * (base + 1) : rem * (base + 1) + (xcd - rem) * base) + idx;
}

// NSTG stages of two key blocks each: 4 (128 KB, one workgroup per CU; up to 512 keys, all loaded
// at once) or 2 (a 64 KB ring, two workgroups per CU, one pair of key blocks in flight while the
// other is multiplied; for longer contexts, where the second workgroup covers the load latency)
template <int NSTG>
__global__ __launch_bounds__(512, NSTG == 2 ? 2 : 1) void flash_attn_kernel(const AttnArgs a) {
    // NSTG stages of two key blocks, then the 64-row query tile (resident path)
    __shared__ __attribute__((aligned(1024))) half_t smem[NSTG * ASTAGE + 4096];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar DMA choices
    const int half = wave >> 2, wq = wave & 3;
    // workgroup -> (head, 64-query tile), the query tiles of one head consecutive; consecutive
    // workgroups run on one XCD (dispatch is round-robin over the 8 XCDs), so a head's K and Vt
    // come from HBM once into that XCD's L2
    const int nqt = (a.S + 63) >> 6;
    const int wg = attn_xcd_remap(blockIdx.x, gridDim.x);
    const int bh = wg / nqt, qt = wg - bh * nqt;
    const int S = a.S, Sp = a.Sp;
    const half_t *Qp = a.Q + (long long)bh * S * 64;
    const i32x4 rk = make_rsrc(a.K + (long long)bh * S * 64);
    const i32x4 rv = make_rsrc(a.Vt + (long long)bh * 64 * Sp);

    const int q = qt * 64 + wq * 16 + (lane & 15);
    const int g = lane >> 4;
    half8 qf[2];

    const int nkb = (S + AKB - 1) / AKB;
    const int npair = (nkb + 1) / 2;
    // DMA of pair p: 32 blocks of 1 KB (K of block 2p, K of 2p+1, Vt of 2p, Vt of 2p+1, 8 each);
    // wave w issues blocks 4w..4w+3. Block sub holds rows 8sub..8sub+7; lane l writes slot l & 7
    // of row lr = l >> 3, i.e. source chunk lc = (l & 7) ^ sw(8sub + lr).
    const int lr = lane >> 3;
    auto issue = [&](int p, int stage) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = wave * 4 + i, part = d >> 3, sub = d & 7;
            const int lc = (lane & 7) ^ lr ^ sub;
            const int blk = 2 * p + (part & 1);
            unsigned vo = 0x80000000u;
            if (part < 2) {
                const int key = blk * AKB + sub * 8 + lr;
                if (key < S) vo = (unsigned)((key * 64 + lc * 8) * 2);
            } else if (blk < nkb) {
                vo = (unsigned)(((sub * 8 + lr) * Sp + blk * AKB + lc * 8) * 2);
            }
            dma16(part < 2 ? rk : rv, vo, (lds_char *)(smem + stage * ASTAGE + part * 4096 + sub * 512));
        }
    };

    // running reference (log2 units) of this half's queries; Oᵀ and the running row sum live in
    // MFMA accumulators: the sum is Pᵀ multiplied by a tile of ones, i.e. exactly the f32 sum of
    // the f16 probabilities the numerator uses, already reduced over all keys of the block.
    SoftRef R;
    floatx4 o[4], lsum = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    const half8 ones = half8{1, 1, 1, 1, 1, 1, 1, 1};

    // key block blk of this half, resident in stage st
    auto compute = [&](int st, int blk) {
        const half_t *sK = smem + st * ASTAGE + half * 4096;
        const half_t *sV = smem + st * ASTAGE + 8192 + half * 4096;
        // Sᵀ row i of MFMA block j is key 32(j>>1) + 8(i>>2) + 4(j&1) + (i&3), so lane group g
        // ends up with keys 32c + 8g + 0..7 of each 32-key chunk c (j = 2c, 2c+1): exactly the K
        // order of one contiguous 16-byte Vᵀ read in the PV product.
        floatx4 sc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            sc[j] = R.nb;
            const int i = lane & 15;
            const int r = 32 * (j >> 1) + 8 * (i >> 2) + 4 * (j & 1) + (i & 3);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const half8 kf = *(const half8 *)(sK + r * 64 + (((ks * 4 + g) ^ sw(r)) * 8));
                sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[ks], sc[j], 0, 0, 0);
            }
        }
        if (blk * AKB + AKB > S) {   // the last, partial key block only (wave-uniform)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (blk * AKB + 32 * (j >> 1) + 8 * g + 4 * (j & 1) + r >= S) sc[j][r] = -INFINITY;
        }
        half8 pf[2];
        block_probs(sc, 4, R, o, lsum, pf);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                // Vt row d = 16dt + (lane&15), keys 32c + 8g + 0..7 (chunk 4c + g)
                const int d = dt * 16 + (lane & 15);
                const half8 vf = *(const half8 *)(sV + d * 64 + (((c * 4 + g) ^ sw(d)) * 8));
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[c], o[dt], 0, 0, 0);
            }
            lsum = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf[c], lsum, 0, 0, 0);
        }
    };

    if constexpr (NSTG == 4) {
        // Every key block fits (S <= 512; the launcher takes this kernel only then). Wave w loads
        // rows 8w..8w+7 of the query tile, then the K rows of key block w, then its Vt columns (16
        // bytes per lane; K of block b at b*8 KB, Vt of block b at 64 KB + b*8 KB); blocks past the
        // last read as zero, so every wave issues 17 loads. Waiting for all but the last 8 (vmcnt 8)
        // covers the queries and the K blocks: each half multiplies its first key block and forms
        // its probabilities while the Vt blocks still land.
        half_t *sQ = smem + NSTG * ASTAGE;
        {
            const int qrow = qt * 64 + wave * 8 + lr;
            const int lc = (lane & 7) ^ lr ^ wave;
            dma16(make_rsrc(Qp), qrow < S ? (unsigned)((qrow * 64 + lc * 8) * 2) : 0x80000000u,
                  (lds_char *)(sQ + wave * 512));
        }
        // (the ring holds 2*NSTG key blocks: waves past that load only their query rows)
        const int kb = wave;
        const bool kv = kb < 2 * NSTG;
        if (kv) {
#pragma unroll
            for (int sub = 0; sub < 8; ++sub) {
                const int lc = (lane & 7) ^ lr ^ sub, key = kb * AKB + sub * 8 + lr;
                dma16(rk, key < S ? (unsigned)((key * 64 + lc * 8) * 2) : 0x80000000u,
                      (lds_char *)(smem + kb * 4096 + sub * 512));
            }
#pragma unroll
            for (int sub = 0; sub < 8; ++sub) {
                const int lc = (lane & 7) ^ lr ^ sub;
                dma16(rv, kb < nkb ? (unsigned)(((sub * 8 + lr) * Sp + kb * AKB + lc * 8) * 2) : 0x80000000u,
                      (lds_char *)(smem + 32768 + kb * 4096 + sub * 512));
            }
        }
        wait_vmcnt(kv ? 8 : 0);
        block_barrier();
        {
            const int r = wq * 16 + (lane & 15);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) qf[ks] = *(const half8 *)(sQ + r * 64 + (((ks * 4 + g) ^ sw(r)) * 8));
        }
        // The lane's fragment offsets (halves) for this half's blocks half, half + 2, ...: K block b
        // at b*4096, Vt block b at 32768 + b*4096, so the half's i-th block adds i*8192 (16 KB), an
        // immediate of the LDS reads once the loop below is unrolled (unsigned, so it folds).
        unsigned k_off[4][2], v_off[2][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = lane & 15;
            const int r = 32 * (j >> 1) + 8 * (i >> 2) + 4 * (j & 1) + (i & 3);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) k_off[j][ks] = half * 4096 + r * 64 + (((ks * 4 + g) ^ sw(r)) * 8);
        }
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const int d = dt * 16 + (lane & 15);
                v_off[c][dt] = 32768 + half * 4096 + d * 64 + (((c * 4 + g) ^ sw(d)) * 8);
            }
        // scores of this half's key block i (block half + 2i) for the first NJ 16-key MFMA blocks
        // (NJ = 4: all 64 keys, 2: the first 32), layout as in compute()
        auto qk = [&](int i, int nj, floatx4 (&sc)[4]) {
            const half_t *sK = smem + i * 8192;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sc[j] = R.nb;
                if (j < nj) {
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        const half8 kf = *(const half8 *)(sK + k_off[j][ks]);
                        sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[ks], sc[j], 0, 0, 0);
                    }
                }
            }
        };
        // probabilities of keys < lim (the block's valid keys) as the PV product's B operands; the
        // block's QK product started from R.nb, which no other block has moved since (each block's
        // probabilities are formed before the next block's QK product is issued)
        auto softmax = [&](floatx4 (&sc)[4], int nj, int lim, half8 (&pf)[2]) {
            if (lim < AKB) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (32 * (j >> 1) + 8 * g + 4 * (j & 1) + r >= lim) sc[j][r] = -INFINITY;
            }
            block_probs(sc, nj, R, o, lsum, pf);
        };
        auto pv = [&](int i, int nc, const half8 (&pf)[2]) {
            const half_t *sV = smem + i * 8192;
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                if (c < nc) {
#pragma unroll
                    for (int dt = 0; dt < 4; ++dt) {
                        const half8 vf = *(const half8 *)(sV + v_off[c][dt]);
                        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[c], o[dt], 0, 0, 0);
                    }
                    lsum = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf[c], lsum, 0, 0, 0);
                }
            }
        };
        // full key blocks half, half + 2, ... < nfull; the partial last block (if any) goes to the
        // half of its parity and runs after them, on 32 keys when it has no more
        const int nfull = S / AKB, lim_t = S - nfull * AKB;
        const int nf = (nfull - half + 1) >> 1;
        const bool own_tail = lim_t > 0 && (nfull & 1) == half;
        half8 pf[2];
        if (nf > 0) {
            floatx4 sc[4];
            qk(0, 4, sc);
            softmax(sc, 4, AKB, pf);
        }
        wait_vmcnt(0);
        block_barrier();   // every Vt block visible
        if (nf > 0) {
            // the next block's score products are issued before this block's PV products; its
            // probabilities (after the rescale that follows this block's PV) come last (at most
            // four blocks per half: unrolled, so every block offset is a constant)
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                if (i + 1 < nf) {
                    floatx4 sn[4];
                    qk(i + 1, 4, sn);
                    pv(i, 2, pf);
                    softmax(sn, 4, AKB, pf);
                }
            }
            pv(nf - 1, 2, pf);
        }
        if (own_tail) {   // block nfull = half + 2*nf
            floatx4 sc[4];
            if (lim_t <= 32) {
                qk(nf, 2, sc);
                softmax(sc, 2, lim_t, pf);
                pv(nf, 1, pf);
            } else {
                qk(nf, 4, sc);
                softmax(sc, 4, lim_t, pf);
                pv(nf, 2, pf);
            }
        }
    } else {
        // two stages: pair p + 1 lands while pair p is multiplied
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            qf[ks] = q < S ? *(const half8 *)(Qp + (long long)q * 64 + ks * 32 + g * 8) : zero_h8();
        issue(0, 0);
        wait_vmcnt(0);
        block_barrier();
        issue(1, 1);
        for (int p = 0; p < npair; ++p) {
            const int st = p & 1;
            if (2 * p + half < nkb) compute(st, 2 * p + half);
            if (p + 1 < npair) {
                wait_vmcnt(0);      // pair p + 1, the only one in flight, has landed
                block_barrier();    // and every wave is done with stage st
                if (p + 2 < npair) issue(p + 2, st);
            }
        }
    }
    float l_i = lsum[0];   // every row of the ones product holds the same sum

    // merge the two halves: half h combines and stores output columns 32h..32h+31 (dt = 2h, 2h+1).
    // Each half parks its (m, l) and the two column groups the other half stores in LDS; the
    // combination is the same per element whichever half forms it (o_0*f_0 + o_1*f_1, 1/l).
    block_barrier();
    const float m_i = R.m;   // -1e30 for a half that had no key block: its terms get weight 0
    float *red = (float *)smem;
    float *mine = red + ((half * 4 + wq) * 64 + lane) * 10;
    const float *other = red + (((half ^ 1) * 4 + wq) * 64 + lane) * 10;
    mine[0] = m_i;
    mine[1] = l_i;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) mine[2 + j * 4 + r] = half ? o[j][r] : o[2 + j][r];   // selects: o stays in registers
    block_barrier();
    const float m_o = other[0], l_o = other[1];
    const float m = fmaxf(m_i, m_o);
    const float f_s = exp2f(m_i - m), f_o = exp2f(m_o - m);
    // half 0's terms first in both halves: l = l_0*f_0 + l_1*f_1
    const float l = half == 0 ? l_i * f_s + l_o * f_o : l_o * f_o + l_i * f_s;
    float om[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float own = (half ? o[2 + j][r] : o[j][r]) * f_s, oth = other[2 + j * 4 + r] * f_o;
            om[j][r] = half == 0 ? own + oth : oth + own;
        }

    if (q < S) {
        const float inv = 1.0f / l;
        const int b = bh / a.nh, h = bh - b * a.nh;
        const long long orow = rowmap_phys(a.omap, b * S + q) * (long long)a.ldo + h * 64;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int dt = 2 * half + j;
            const float (&od)[4] = om[j];
            const int d0 = dt * 16 + g * 4;
            if (a.o_f32) {
                float *op = (float *)a.O + orow + d0;
                *(float4 *)op = make_float4(od[0] * inv, od[1] * inv, od[2] * inv, od[3] * inv);
            } else {
                half_t *op = (half_t *)a.O + orow + d0;
                const float y0 = od[0] * inv, y1 = od[1] * inv, y2 = od[2] * inv, y3 = od[3] * inv;
                const half4 hi = half4{(half_t)y0, (half_t)y1, (half_t)y2, (half_t)y3};
                *(half4 *)op = hi;
                if (a.o_lo)   // f16 remainder at column offset o_lo: hi + lo carries the f32 value
                    *(half4 *)(op + a.o_lo) = half4{(half_t)(y0 - (float)hi[0]), (half_t)(y1 - (float)hi[1]),
                                                    (half_t)(y2 - (float)hi[2]), (half_t)(y3 - (float)hi[3])};
            }
        }
    }
}

// Four-wave variant for grids beyond one round of the eight-wave kernel (long contexts, large
// batches): 64 queries per workgroup, wave w serves queries 16w..16w+15 over every key block (no
// key split, no merge), and a three-stage ring of single key blocks (K 8 KB + Vt 8 KB per stage),
// 48 KB of LDS and at most 128 VGPRs, so three workgroups share a CU. At 30 s (S = 1101, 576
// workgroups) the whole grid is resident at once instead of running in two rounds. The MFMA
// formulation, the online softmax and the probability rounding are the eight-wave kernel's.
__global__ __launch_bounds__(256, 3) void flash_attn4_kernel(const AttnArgs a) {
    constexpr int STG = 8192;   // halves per stage: K block (64 keys x 64) then Vt block (64 d x 64 keys)
    constexpr int NST = 3;      // ring stages: two key blocks in flight while one is multiplied
    __shared__ __attribute__((aligned(1024))) half_t smem[NST * STG];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nqt = (a.S + 63) >> 6;
    const int wg = attn_xcd_remap(blockIdx.x, gridDim.x);
    const int bh = wg / nqt, qt = wg - bh * nqt;
    const int S = a.S, Sp = a.Sp;
    const half_t *Qp = a.Q + (long long)bh * S * 64;
    // K rows past S read as zero through the buffer range (num_records = the head's S rows)
    const unsigned long long ka = (unsigned long long)(a.K + (long long)bh * S * 64);
    const i32x4 rk = i32x4{(int)(unsigned)ka, (int)((ka >> 32) & 0xFFFF), S * 128, 0x00020000};
    const i32x4 rv = make_rsrc(a.Vt + (long long)bh * 64 * Sp);

    const int q = qt * 64 + wave * 16 + (lane & 15);
    const int g = lane >> 4;
    half8 qf[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
        qf[ks] = q < S ? *(const half8 *)(Qp + (long long)q * 64 + ks * 32 + g * 8) : zero_h8();

    const int nkb = (S + AKB - 1) / AKB;
    // DMA of key block b: 16 chunks of 1 KB (K rows 8sub.., then Vt rows 8sub..); wave w issues
    // chunks 4w..4w+3. Lane l writes slot l & 7 of row lr = l >> 3 (source chunk lc = (l & 7) ^ sw(row)).
    // The lane's byte offsets inside a block are fixed; a block adds 8 KB (K) or 128 B (Vt).
    const int lr = lane >> 3;
    unsigned voff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = wave * 4 + i, part = d >> 3, sub = d & 7;
        const int lc = (lane & 7) ^ lr ^ sub;
        voff[i] = part == 0 ? (unsigned)(((sub * 8 + lr) * 64 + lc * 8) * 2)
                            : (unsigned)(((sub * 8 + lr) * Sp + lc * 8) * 2);
    }
    auto issue = [&](int b, int st) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = wave * 4 + i, part = d >> 3, sub = d & 7;
            const unsigned vo = voff[i] + (part == 0 ? (unsigned)b * 8192u : (unsigned)b * 128u);
            dma16(part == 0 ? rk : rv, vo, (lds_char *)(smem + st * STG + part * 4096 + sub * 512));
        }
    };

    SoftRef R;
    floatx4 o[4], lsum = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    const half8 ones = half8{1, 1, 1, 1, 1, 1, 1, 1};

    // the lane's fragment offsets (halves) inside a stage, the same for every key block: K rows of
    // MFMA block j, K half ks; Vt rows of d tile dt, key chunk c
    unsigned k_off[4][2], v_off[2][4];   // unsigned: the stage offset folds into the reads
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = lane & 15;
        const int r = 32 * (j >> 1) + 8 * (i >> 2) + 4 * (j & 1) + (i & 3);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) k_off[j][ks] = r * 64 + (((ks * 4 + g) ^ sw(r)) * 8);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const int d = dt * 16 + (lane & 15);
            v_off[c][dt] = 4096 + d * 64 + (((c * 4 + g) ^ sw(d)) * 8);
        }

    auto compute = [&](int st, int blk) {
        const half_t *sK = smem + st * STG;
        floatx4 sc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            sc[j] = R.nb;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const half8 kf = *(const half8 *)(sK + k_off[j][ks]);
                sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[ks], sc[j], 0, 0, 0);
            }
        }
        if (blk * AKB + AKB > S) {   // the last, partial key block only (wave-uniform)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (blk * AKB + 32 * (j >> 1) + 8 * g + 4 * (j & 1) + r >= S) sc[j][r] = -INFINITY;
        }
        half8 pf[2];
        block_probs(sc, 4, R, o, lsum, pf);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const half8 vf = *(const half8 *)(sK + v_off[c][dt]);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[c], o[dt], 0, 0, 0);
            }
            lsum = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf[c], lsum, 0, 0, 0);
        }
    };

    // ring: block b in stage b % 3; blocks b + 1 and b + 2 land while b is multiplied
    issue(0, 0);
    if (nkb > 1) issue(1, 1);
    wait_vmcnt(nkb > 1 ? 4 : 0);
    block_barrier();
    if (nkb > 2) issue(2, 2);
    // unrolled over the three stages, so each stage's LDS offset is a constant of the fragment reads
    // and DMA targets (no per-block address arithmetic)
    for (int b0 = 0; b0 < nkb; b0 += NST) {
#pragma unroll
        for (int u = 0; u < NST; ++u) {
            const int b = b0 + u;
            if (b < nkb) {
                compute(u, b);
                if (b + 1 < nkb) {
                    wait_vmcnt(b + 2 < nkb ? 4 : 0);   // block b + 1 has landed (b + 2 may still be in flight)
                    block_barrier();                    // and every wave is done with stage u = b % 3
                    if (b + NST < nkb) issue(b + NST, u);
                }
            }
        }
    }
    if (q < S) {
        const float inv = 1.0f / lsum[0];   // every row of the ones product holds the same sum
        const int b = bh / a.nh, h = bh - b * a.nh;
        const long long orow = rowmap_phys(a.omap, b * S + q) * (long long)a.ldo + h * 64;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const int d0 = dt * 16 + g * 4;
            if (a.o_f32) {
                float *op = (float *)a.O + orow + d0;
                *(float4 *)op = make_float4(o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv);
            } else {
                half_t *op = (half_t *)a.O + orow + d0;
                const float y0 = o[dt][0] * inv, y1 = o[dt][1] * inv, y2 = o[dt][2] * inv, y3 = o[dt][3] * inv;
                const half4 hi = half4{(half_t)y0, (half_t)y1, (half_t)y2, (half_t)y3};
                *(half4 *)op = hi;
                if (a.o_lo)
                    *(half4 *)(op + a.o_lo) = half4{(half_t)(y0 - (float)hi[0]), (half_t)(y1 - (float)hi[1]),
                                                    (half_t)(y2 - (float)hi[2]), (half_t)(y3 - (float)hi[3])};
            }
        }
    }
}

// Four-wave kernel with two query groups per wave: 128 queries per workgroup, wave w serves
// queries 32w .. 32w + 31 as two groups of 16 over every key block. Each K and Vt fragment read from
// LDS feeds both groups' MFMAs (half the LDS operand reads per flop of flash_attn4_kernel), and each
// wave carries two independent softmax chains. Ring, MFMA formulation, online softmax and
// probability rounding as flash_attn4_kernel; for grids whose 64-query version exceeds a round.
__global__ __launch_bounds__(256, 3) void flash_attn4q2_kernel(const AttnArgs a) {
    constexpr int STG = 8192;
    constexpr int NST = 3;
    __shared__ __attribute__((aligned(1024))) half_t smem[NST * STG];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nqt = (a.S + 127) >> 7;
    const int wg = attn_xcd_remap(blockIdx.x, gridDim.x);
    const int bh = wg / nqt, qt = wg - bh * nqt;
    const int S = a.S, Sp = a.Sp;
    const half_t *Qp = a.Q + (long long)bh * S * 64;
    const unsigned long long ka = (unsigned long long)(a.K + (long long)bh * S * 64);
    const i32x4 rk = i32x4{(int)(unsigned)ka, (int)((ka >> 32) & 0xFFFF), S * 128, 0x00020000};
    const i32x4 rv = make_rsrc(a.Vt + (long long)bh * 64 * Sp);

    const int g = lane >> 4;
    int q[2];
    half8 qf[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        q[u] = qt * 128 + wave * 32 + u * 16 + (lane & 15);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            qf[u][ks] = q[u] < S ? *(const half8 *)(Qp + (long long)q[u] * 64 + ks * 32 + g * 8) : zero_h8();
    }
    // whole wave past the last query: its MFMAs are skipped (it still takes its DMA share and barriers)
    const bool live = qt * 128 + wave * 32 < S;

    const int nkb = (S + AKB - 1) / AKB;
    const int lr = lane >> 3;
    unsigned voff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = wave * 4 + i, part = d >> 3, sub = d & 7;
        const int lc = (lane & 7) ^ lr ^ sub;
        voff[i] = part == 0 ? (unsigned)(((sub * 8 + lr) * 64 + lc * 8) * 2)
                            : (unsigned)(((sub * 8 + lr) * Sp + lc * 8) * 2);
    }
    auto issue = [&](int b, int st) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = wave * 4 + i, part = d >> 3, sub = d & 7;
            const unsigned vo = voff[i] + (part == 0 ? (unsigned)b * 8192u : (unsigned)b * 128u);
            dma16(part == 0 ? rk : rv, vo, (lds_char *)(smem + st * STG + part * 4096 + sub * 512));
        }
    };

    SoftRef R[2];
    floatx4 o[2][4], lsum[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        lsum[u] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[u][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    const half8 ones = half8{1, 1, 1, 1, 1, 1, 1, 1};

    unsigned k_off[4][2], v_off[2][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = lane & 15;
        const int r = 32 * (j >> 1) + 8 * (i >> 2) + 4 * (j & 1) + (i & 3);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) k_off[j][ks] = r * 64 + (((ks * 4 + g) ^ sw(r)) * 8);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const int d = dt * 16 + (lane & 15);
            v_off[c][dt] = 4096 + d * 64 + (((c * 4 + g) ^ sw(d)) * 8);
        }

    auto compute = [&](int st, int blk) {
        const half_t *sK = smem + st * STG;
        floatx4 sc[2][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            sc[0][j] = R[0].nb;
            sc[1][j] = R[1].nb;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const half8 kf = *(const half8 *)(sK + k_off[j][ks]);
                sc[0][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[0][ks], sc[0][j], 0, 0, 0);
                sc[1][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[1][ks], sc[1][j], 0, 0, 0);
            }
        }
        if (blk * AKB + AKB > S) {   // the last, partial key block only (wave-uniform)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (blk * AKB + 32 * (j >> 1) + 8 * g + 4 * (j & 1) + r >= S) sc[u][j][r] = -INFINITY;
        }
        half8 pf[2][2];
#pragma unroll
        for (int u = 0; u < 2; ++u) block_probs(sc[u], 4, R[u], o[u], lsum[u], pf[u]);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const half8 vf = *(const half8 *)(sK + v_off[c][dt]);
                o[0][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[0][c], o[0][dt], 0, 0, 0);
                o[1][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[1][c], o[1][dt], 0, 0, 0);
            }
            lsum[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf[0][c], lsum[0], 0, 0, 0);
            lsum[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf[1][c], lsum[1], 0, 0, 0);
        }
    };

    issue(0, 0);
    if (nkb > 1) issue(1, 1);
    wait_vmcnt(nkb > 1 ? 4 : 0);
    block_barrier();
    if (nkb > 2) issue(2, 2);
    for (int b0 = 0; b0 < nkb; b0 += NST) {
#pragma unroll
        for (int u = 0; u < NST; ++u) {
            const int b = b0 + u;
            if (b < nkb) {
                if (live) compute(u, b);
                if (b + 1 < nkb) {
                    wait_vmcnt(b + 2 < nkb ? 4 : 0);
                    block_barrier();
                    if (b + NST < nkb) issue(b + NST, u);
                }
            }
        }
    }
    const int bb = bh / a.nh, h = bh - bb * a.nh;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        if (q[u] >= S) continue;
        const float inv = 1.0f / lsum[u][0];
        const long long orow = rowmap_phys(a.omap, bb * S + q[u]) * (long long)a.ldo + h * 64;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const int d0 = dt * 16 + g * 4;
            if (a.o_f32) {
                float *op = (float *)a.O + orow + d0;
                *(float4 *)op = make_float4(o[u][dt][0] * inv, o[u][dt][1] * inv, o[u][dt][2] * inv, o[u][dt][3] * inv);
            } else {
                half_t *op = (half_t *)a.O + orow + d0;
                const float y0 = o[u][dt][0] * inv, y1 = o[u][dt][1] * inv, y2 = o[u][dt][2] * inv, y3 = o[u][dt][3] * inv;
                const half4 hi = half4{(half_t)y0, (half_t)y1, (half_t)y2, (half_t)y3};
                *(half4 *)op = hi;
                if (a.o_lo)
                    *(half4 *)(op + a.o_lo) = half4{(half_t)(y0 - (float)hi[0]), (half_t)(y1 - (float)hi[1]),
                                                    (half_t)(y2 - (float)hi[2]), (half_t)(y3 - (float)hi[3])};
            }
        }
    }
}

// f32 [S, ld] q/k/v slices -> Q/K [nh][S][64], Vt [nh][64][Sp] (f16), one thread per element
__global__ void attn_pack_kernel(const float *qkv, float q_scale, int S, int nh, int ld, int q_off, int k_off,
                                 int v_off, half_t *Q, half_t *K, half_t *Vt, int Sp) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)nh * Sp * 64;
    if (idx >= total) return;
    const int d = (int)(idx & 63);
    const long long rest = idx >> 6;
    const int s = (int)(rest % Sp);
    const int h = (int)(rest / Sp);
    if (s < S) {
        const float *row = qkv + (long long)s * ld + h * 64 + d;
        Q[((long long)h * S + s) * 64 + d] = (half_t)(row[q_off] * q_scale);
        K[((long long)h * S + s) * 64 + d] = (half_t)row[k_off];
        Vt[((long long)h * 64 + d) * Sp + s] = (half_t)row[v_off];
    } else {
        Vt[((long long)h * 64 + d) * Sp + s] = (half_t)0.0f;
    }
}

} // namespace

int launch_attention(const AttnArgs &a, hipStream_t st) {
    TSN_REQUIRE(a.Q && a.K && a.Vt && a.O, "attention: null pointer");
    TSN_REQUIRE(a.S > 0 && a.Sp >= a.S && a.Sp % 64 == 0, "attention: Sp must be a multiple of 64 and >= S");
    TSN_REQUIRE(a.BH > 0 && a.nh > 0 && a.BH % a.nh == 0, "attention: BH must be a multiple of nh");
    TSN_REQUIRE(a.omap.L > 0, "attention: output row map");
    TSN_REQUIRE(a.ldo % 4 == 0, "attention: ldo must be a multiple of 4");
    TSN_REQUIRE(a.o_lo == 0 || (!a.o_f32 && a.o_lo % 4 == 0 && a.o_lo >= a.nh * 64 && a.ldo >= a.o_lo + a.nh * 64),
                "attention: hi|lo output needs f16 O, o_lo >= nh*64 (multiple of 4) and ldo >= o_lo + nh*64");
    TSN_REQUIRE((((uintptr_t)a.Q) & 15) == 0 && (((uintptr_t)a.K) & 15) == 0 && (((uintptr_t)a.Vt) & 15) == 0,
                "attention: 16-byte aligned Q/K/Vt");
    TSN_REQUIRE((long long)a.S * 64 * 2 < (1LL << 31) && (long long)a.Sp * 64 * 2 < (1LL << 31),
                "attention: per-head K/Vt extent must stay below 2 GB (buffer addressing)");
    TSN_REQUIRE((long long)((a.S + 63) / 64) * a.BH < (1LL << 31), "attention: too many query tiles");
    TSN_REQUIRE((long long)a.S * 128 < (1LL << 31), "attention: K extent per head below 2 GB");
    dim3 grid((unsigned)((a.S + 63) / 64 * a.BH)), block(512);
    // up to 512 keys and at most one workgroup per CU: all key blocks in LDS at once; grids beyond
    // one round (256 workgroups): the four-wave kernel, up to four workgroups per CU
    // grids of at least two workgroups per CU in 128-query workgroups: the two-group kernel (batch
    // 16 at 8 s: 1024 workgroups, 7.25 -> 7.20-7.23 ms per evaluation); with fewer (30 s: 288) it
    // leaves too few waves per CU and the 64-query kernel is faster (3.99 -> 4.05 ms measured)
    const long long g2 = (long long)(a.S + 127) / 128 * a.BH;
    if (a.S <= 4 * 2 * AKB && grid.x <= 256) TSN_LAUNCH(flash_attn_kernel<4>, grid, block, 0, st, a);
    else if (g2 >= 512) TSN_LAUNCH(flash_attn4q2_kernel, dim3((unsigned)g2), dim3(256), 0, st, a);
    else if (grid.x > 256) TSN_LAUNCH(flash_attn4_kernel, grid, dim3(256), 0, st, a);
    else TSN_LAUNCH(flash_attn_kernel<2>, grid, block, 0, st, a);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_attn_pack(const float *qkv, float q_scale, int S, int nh, int ld, int q_off, int k_off, int v_off,
                     half_t *Q, half_t *K, half_t *Vt, int Sp, hipStream_t st) {
    TSN_REQUIRE(qkv && Q && K && Vt && S > 0 && nh > 0 && Sp >= S, "attn_pack: arguments");
    const long long total = (long long)nh * Sp * 64;
    const int blocks = (int)((total + 255) / 256);
    TSN_LAUNCH(attn_pack_kernel, dim3(blocks), dim3(256), 0, st, qkv, q_scale, S, nh, ld, q_off, k_off, v_off, Q, K,
               Vt, Sp);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

} // namespace tsn
