// gemm.hip — MFMA GEMM / implicit-GEMM conv1d for gfx950 with fused epilogues.
//
// Replaces the reference's GEMM route (src/net.mm:14-23 -> shaders/gemm_mpp.metal:18-48) and its
// conv route (src/net.mm:25-49: im2col + GEMM). The conv is an implicit GEMM: the weight is
// stored [OC][K][IC] so each 64-wide K tile is one tap of IC channels, and the A loader reads
// row t - pad + tap of the same sample (zero outside the sample) — no im2col buffer.
//
// Kernels in this file (all 128x128 C tiles over 64-wide K tiles unless noted; MFMA
// v_mfma_f32_16x16x32_f16, or _bf16 for bf16 operands, with f32 accumulation):
//  * gemm_pipe_kernel / _hl / _bf16 (the production path): 512 threads = 8 waves, two per SIMD,
//    each wave a 32x64 block. Operands move global -> LDS by direct-to-LDS DMA
//    (buffer_load_dwordx4 ... lds) into a ring of NS = 4 stages (128 KB), rows XOR-swizzled in
//    16-byte chunks so MFMA operand reads are conflict-free; one barrier per K tile; the C tile is
//    staged through LDS and the epilogue runs on 16-byte chunks. One workgroup per CU.
//  * gemm_pipe2_kernel / _hl / _bf16: the same loop with two stages (68 KB), two workgroups per CU,
//    for data-parallel grids of more than one round (one workgroup's epilogue and waits overlap the
//    other's K loop).
//  * gemm_wide_kernel: 256x256 tiles, 8 waves of 128x64, two 64 KB stages, one workgroup per CU,
//    for long-K grids of at least a round of such tiles.
//  * gemm_small_kernel / gemm_small2_kernel / gemm_small3_kernel: 64x64 tiles over the full K,
//    4 waves of 32x32 (small2: two groups of 4 waves over alternate K tiles), with 16 KB stages:
//    five (two workgroups per CU), three per group (one per CU) or three (three per CU, for grids
//    past 512 tiles); residual epilogue in place or plain store, for GEMMs whose 128x128 grid
//    cannot fill one round of the chip.
//  * gemm_sk_kernel + gemm_fixup_kernel: stream-K over (tile, K tile) units, with the cut tiles
//    finished in-kernel by their last contributor or by the fixup launch.
//  * splitk_reduce_kernel: classic split-K sum in split order, then the epilogue.
//  * gemm_f16_kernel: register-staged 256-thread kernel (4 waves of 64x64, two padded LDS stages)
//    for shapes the pipelined kernels do not take (f32 A, K not a multiple of 64, unaligned rows).
//
// Work order: grid = all tiles of all problems (<= 3, e.g. audio + text stream of a joint block).
// Workgroup IDs are remapped so each XCD (8 per MI355X, dispatched round-robin by workgroup ID)
// receives one contiguous range of tiles (xcd_remap), and tiles are grouped by up to 8 m tiles with
// n slow inside a group (tile_mn), so the workgroups of one XCD share A rows and W columns in that
// XCD's L2. Deterministic: every sum runs in a fixed order, no float atomics.
#include "kernels.h"
#include "dpp.h"
#include "prefetch.h"
#include "gemv.h"
#include "snake.h"

#include <string.h>

#include <algorithm>

namespace tsn {

namespace {

constexpr int BM = 128, BN = 128, BK = 64, LDSW = BK + 8;
// stream-K: workgroups of one grid (one per CU of an MI355X), the fewest K tiles one takes, and
// the per-workgroup cost of pipeline fill, partial store and the fixup launch in K-tile units
// (the fixup kernel alone takes 8-10 us, about 20 K tiles)
constexpr int NCU = 256, SK_MIN_UNITS = 8, SK_OVERHEAD = 20;
// with the fixup inside the stream-K kernel (GemmBatch::sk_cnt): partial store written through,
// arrival, and the last contributor's sum of the slots. Measured about as long as the fixup launch
// it replaces (3.345 -> 3.324 ms per reference-graph evaluation with the same plans; a charge of 8
// K tiles picked stream-K for more GEMMs and measured 3.369 -> 3.411 ms)
constexpr int SK_OVERHEAD_IN = 20;
// the wide kernel (gemm_wide_kernel) is taken for grids of at least a round of 256x256 tiles whose
// every problem has K >= WIDE_MIN_K (measured faster there, slower at K = 1024)
constexpr int WIDE_MIN_TILES = 256, WIDE_MIN_K = 2048;
// 64x64 grids of more tiles than this take the three-stage small kernel (three workgroups per CU)
constexpr int SMALL3_MIN_TILES = 2 * NCU;

__device__ inline int xcd_remap(int bid, int nwg) {
    const int xcd = bid & 7, idx = bid >> 3;
    const int base = nwg >> 3, rem = nwg & 7;
    return (xcd < rem ? xcd * (base + 1) : rem * (base + 1) + (xcd - rem) * base) + idx;
}

__device__ inline half8 zero_h8() { return half8{0, 0, 0, 0, 0, 0, 0, 0}; }

// x·sigmoid(x) with the hardware reciprocal (1 ulp): exp(-v) = inf gives rcp = 0, so silu -> -0
__device__ inline float silu_f(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// Fused epilogue shared by both kernels. acc[i][j][r] holds C[row][col] of the wave's 64x64
// block: row = wm*64 + i*16 + (lane>>4)*4 + r, col = wn*64 + j*16 + (lane&15).
template <int EPI>
__device__ __forceinline__ void gemm_epilogue(const GemmProblem &P, floatx4 (&acc)[4][4], int m0, int n0, int wm,
                                              int wn, int lane) {
    const int M = P.M, N = P.N;
    const int col_l = wn * 64 + (lane & 15);
    const int row_l = wm * 64 + (lane >> 4) * 4;
    if constexpr (EPI == EPI_STORE) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + row_l + i * 16 + r;
                if (m >= M) continue;
                const long long yrow = rowmap_phys(P.ymap, m) * (long long)P.ldy;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int n = n0 + col_l + j * 16;
                    if (n >= N) continue;
                    float v = acc[i][j][r] + (P.bias ? P.bias[n] : 0.0f);
                    if (P.silu) v = silu_f(v);
                    if (P.y_f16) ((half_t *)P.Y)[yrow + n] = (half_t)v;
                    else ((float *)P.Y)[yrow + n] = v;
                }
            }
    } else if constexpr (EPI == EPI_RESID) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + row_l + i * 16 + r;
                if (m >= M) continue;
                float *xr = P.R + rowmap_phys(P.rmap, m) * (long long)P.ldr;
                const float *g = P.gate + (long long)(m / P.gate_L) * P.gate_ld;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int n = n0 + col_l + j * 16;
                    if (n >= N) continue;
                    const float v = acc[i][j][r] + (P.bias ? P.bias[n] : 0.0f);
                    xr[n] = xr[n] + v * g[n];
                }
            }
    } else {  // EPI_QKV: the wave's 64 columns are exactly one head of q, k or v
        const int c0 = n0 + wn * 64;
        const int region = c0 / P.Hq;
        const int h = (c0 - region * P.Hq) >> 6;
        const int dl = lane & 15;
        float v[4][4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float bj = P.bias ? P.bias[c0 + j * 16 + dl] : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) v[i][j][r] = acc[i][j][r] + bj;
        }
        if (region < 2) {
            const float *nw = region == 0 ? P.qn : P.kn;
            float w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = nw[j * 16 + dl];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float ss = 0.0f;
#pragma unroll
                    for (int j = 0; j < 4; ++j) ss += v[i][j][r] * v[i][j][r];
                    ss = row16_sum(ss);
                    const float inv = 1.0f / sqrtf(ss / 64.0f + P.rms_eps);
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[i][j][r] = v[i][j][r] * inv * w[j];
                }
            const bool odd = lane & 1;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = m0 + row_l + i * 16 + r;
                    const int t = (m < M ? m : 0) % P.q_L;
                    const bool rot = (m < M) && t < P.rope_len;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float partner = dpp_mov<DPP_XOR1>(v[i][j][r]);
                        if (rot) {
                            const int pj = (j * 16 + dl) >> 1;
                            const float cs = P.rope[(t * 32 + pj) * 2], sn = P.rope[(t * 32 + pj) * 2 + 1];
                            v[i][j][r] = odd ? partner * sn + v[i][j][r] * cs : v[i][j][r] * cs - partner * sn;
                        }
                    }
                }
            half_t *dst = region == 0 ? P.Q : P.Kd;
            const float sc = region == 0 ? P.q_scale : 1.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = m0 + row_l + i * 16 + r;
                    if (m >= M) continue;
                    const int b = m / P.q_L, s = P.q_soff + (m - b * P.q_L);
                    half_t *o = dst + (((long long)b * P.nh + h) * P.S_att + s) * 64;
#pragma unroll
                    for (int j = 0; j < 4; ++j) o[j * 16 + dl] = (half_t)(v[i][j][r] * sc);
                }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = m0 + row_l + i * 16 + r;
                    if (m >= M) continue;
                    const int b = m / P.q_L, s = P.q_soff + (m - b * P.q_L);
                    half_t *o = P.Vt + ((long long)b * P.nh + h) * 64 * (long long)P.Sp + s;
#pragma unroll
                    for (int j = 0; j < 4; ++j) o[(long long)(j * 16 + dl) * P.Sp] = (half_t)v[i][j][r];
                }
        }
    }
}


// tile index -> (m tile, n tile). Tiles come in groups of up to 8 m tiles; inside a group n is the
// slow index and m the fast one. Consecutive workgroups land on one XCD (xcd_remap), so the tiles an
// XCD runs together share the group's A rows and a few W columns in its L2. With 8 or fewer m tiles
// this is the plain m-fastest order.
__device__ __forceinline__ void tile_mn(int t, int tiles_m, int tiles_n, int &tm, int &tn) {
    constexpr int GM = 8;
    const int grp = t / (GM * tiles_n);
    const int m_first = grp * GM;
    const int gm = min(GM, tiles_m - m_first);
    const int r = t - grp * GM * tiles_n;
    tn = r / gm;
    tm = m_first + (r - tn * gm);
}

template <bool A_F32, int EPI>
__global__ __launch_bounds__(256, 2) void gemm_f16_kernel(const GemmBatch bt) {
    __shared__ __attribute__((aligned(16))) half_t sA[2][BM * LDSW];
    __shared__ __attribute__((aligned(16))) half_t sB[2][BN * LDSW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile = xcd_remap(blockIdx.x, gridDim.x);
    const int pi = (bt.nprob > 2 && tile >= bt.p[2].tile_start) ? 2 : (bt.nprob > 1 && tile >= bt.p[1].tile_start) ? 1 : 0;
    const GemmProblem &P = bt.p[pi];

    const int local = tile - P.tile_start;
    int tm, tn;
    tile_mn(local, P.tiles_m, P.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int M = P.M, N = P.N, K = P.K;

    // loader assignment: rows lrow + 32*r (r < 4), 16-byte chunk lch of the 64-wide K slab
    const int lrow = tid >> 3, lch = tid & 7;
    long long a_base[4];
    int a_t[4];
    bool a_ok[4];
    const half_t *b_ptr[4];
    bool b_ok[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = m0 + lrow + 32 * r;
        a_ok[r] = m < M;
        const int mm = a_ok[r] ? m : 0;
        const int b = mm / P.amap.L;
        a_t[r] = mm - b * P.amap.L;
        a_base[r] = (long long)b * P.amap.seg + P.amap.off;
        const int n = n0 + lrow + 32 * r;
        b_ok[r] = n < N;
        b_ptr[r] = P.W + (long long)(b_ok[r] ? n : 0) * P.ldw + lch * 8;
    }

    half8 ra[4], rb[4];
    auto load_tile = [&](int k0) {
        const int tap = k0 / P.Kc;
        const int c = k0 - tap * P.Kc + lch * 8;
        const bool kin = (k0 + lch * 8) < K;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int ts = a_t[r] - P.pad + tap;
            const bool ok = a_ok[r] && kin && ts >= 0 && ts < P.a_T;
            const long long off = (a_base[r] + ts) * (long long)P.lda + c;
            if constexpr (A_F32) {
                const float *ap = (const float *)P.A + off;
                float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
                if (ok) { x0 = *(const float4 *)ap; x1 = *(const float4 *)(ap + 4); }
                ra[r] = half8{(half_t)x0.x, (half_t)x0.y, (half_t)x0.z, (half_t)x0.w,
                              (half_t)x1.x, (half_t)x1.y, (half_t)x1.z, (half_t)x1.w};
            } else {
                ra[r] = ok ? *(const half8 *)((const half_t *)P.A + off) : zero_h8();
            }
            rb[r] = (b_ok[r] && kin) ? *(const half8 *)(b_ptr[r] + k0) : zero_h8();
        }
    };
    auto store_tile = [&](int s) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            *(half8 *)&sA[s][(lrow + 32 * r) * LDSW + lch * 8] = ra[r];
            *(half8 *)&sB[s][(lrow + 32 * r) * LDSW + lch * 8] = rb[r];
        }
    };

    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int wm = wave >> 1, wn = wave & 1;
    const int nk = (K + BK - 1) / BK;
    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int s = kt & 1;
        if (kt + 1 < nk) load_tile((kt + 1) * BK);
        const half_t *as = &sA[s][(wm * 64 + (lane & 15)) * LDSW + (lane >> 4) * 8];
        const half_t *bs = &sB[s][(wn * 64 + (lane & 15)) * LDSW + (lane >> 4) * 8];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            half8 af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) af[i] = *(const half8 *)(as + i * 16 * LDSW + ks * 32);
#pragma unroll
            for (int j = 0; j < 4; ++j) bf[j] = *(const half8 *)(bs + j * 16 * LDSW + ks * 32);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store_tile(s ^ 1);
        __syncthreads();
    }

    gemm_epilogue<EPI>(P, acc, m0, n0, wm, wn, lane);
}


// ---------------------------------------------------------------------------------------------
// Pipelined kernel (f16 A, K % 64 == 0). 512 threads = 8 waves, two per SIMD; wave w owns the
// 32x64 block (rows 32*(w>>1), columns 64*(w&1)) of the 128x128 tile over the full K. Two waves
// per SIMD let one wave's LDS reads hide behind the other's MFMAs.
//
// Operands go global -> LDS with buffer_load_dwordx4 ... lds (no register staging, see dma16) into
// NS = 4 stages of one 128x64 A tile + one 128x64 W tile each (128 KB): three K tiles are in flight
// while the fourth is multiplied, with one barrier per K tile. The C tile is staged through LDS for
// the epilogue (f32, pitch TP).
//
// LDS layout of a stage: row r (128 B = 8 chunks of 8 halves) keeps chunk c at slot c ^ (r & 7).
// A direct-to-LDS load writes lane l's 16 bytes to slot l of a 1 KB block (8 rows), so lane l of
// block b loads row 8b + (l >> 3), chunk (l & 7) ^ (l >> 3). MFMA operand reads (lane: row
// l & 15, chunk ks*4 + (l >> 4)) then touch 8 distinct 16-byte slots per 8 lanes: no bank
// conflicts. Rows outside the problem (M tail, conv halo, N tail) get an out-of-range buffer
// offset and the hardware writes zeros.
// ---------------------------------------------------------------------------------------------
typedef __attribute__((address_space(3))) char lds_char;
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int CPOL_SC1 = 16;   // cache-policy bit sc1 of a buffer access: device-coherent (written through / read past L1)

// raw buffer descriptor: base, stride 0, num_records 2^31-1, 32-bit data format; an offset at or
// above 0x80000000 is out of range and reads as zero
__device__ __forceinline__ i32x4 make_rsrc(const void *p) {
    const unsigned long long a = (unsigned long long)p;
    return i32x4{(int)(unsigned)a, (int)((a >> 32) & 0xFFFF), 0x7FFFFFFF, 0x00020000};
}

// the same descriptor as the buffer type of the compiler's buffer builtins
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_brsrc(const void *p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, 0x7FFFFFFF, 0x00020000);
}

// 16 bytes per lane, global -> LDS slot (lane) of the 1 KB block at lds. Issued from inline asm so
// the compiler's own LDS-DMA bookkeeping (which turns conservative at loop merges and would wait for
// every load in flight) stays out of the pipeline; the kernel orders it with explicit vmcnt waits
// and barriers. s_nop 0 covers the M0-write -> LDS-DMA hazard.
__device__ __forceinline__ void dma16(i32x4 rs, unsigned voff, lds_char *lds) {
    const unsigned l = __builtin_amdgcn_readfirstlane((unsigned)(unsigned long)lds);
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(voff), "s"(rs), "s"(l)
                 : "memory");
}

// The same with a wave-uniform byte offset in soffset: the per-row part of the address (voff) stays
// in a register across K tiles and only the scalar K offset moves, so a K tile's refill costs no
// vector instructions. Rows outside the operand carry voff = 0x80000000, out of range with or
// without the scalar offset.
// lds is the LDS byte address of the 1 KB block. Both scalars are wave-uniform; readfirstlane
// costs nothing where the compiler already holds them in scalar registers.
__device__ __forceinline__ void dma16s(i32x4 rs, unsigned voff, unsigned soff, unsigned lds) {
    asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :
                 : "v"(voff), "s"(rs), "s"(__builtin_amdgcn_readfirstlane(soff)),
                   "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}
// LDS byte address of element e of an LDS array (wave-uniform when e is)
__device__ __forceinline__ unsigned lds_addr(const half_t *base) {
    return (unsigned)(unsigned long)(const lds_char *)base;
}

// s_waitcnt vmcnt(n) (n in {0, 4, 8, 12}) with expcnt/lgkmcnt left at their maxima
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

constexpr int STAGE = BM * BK;   // halves per operand tile of one stage
constexpr int NS = 4;            // LDS stages (4 x 32 KB = 128 KB): NS-1 K tiles in flight.
                                 // Measured per 8 s evaluation: 5 stages 2.026 ms, 4 stages 1.965,
                                 // 3 stages 1.987 (same box); a fifth stage only adds L2 traffic in
                                 // flight, the loop is bound by the L2 -> LDS rate and the LDS port
constexpr int TP = 132;          // pitch (floats) of the f32 C tile staged in LDS for the epilogue:
                                 // 4 rows apart = 528 floats = 16 banks apart, so MFMA-layout writes
                                 // from the 4 lane groups of a wave never collide

// Epilogue on the LDS-staged C tile (128 x 128, row-major f32, pitch PITCH). Thread tid handles 8-column chunks
// c = tid + 512*p (row c >> 4, columns (c & 15)*8 .. +7) — 16-byte reads from LDS and 16-byte
// global stores. Requires N % 8 == 0 and 16-byte aligned output rows (checked by the launcher).
__device__ __forceinline__ void load8(const float *t, float (&v)[8]) {
    const floatx4 a = *(const floatx4 *)t, b = *(const floatx4 *)(t + 4);
    v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3]; v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
}
__device__ __forceinline__ void ldsum8(const float *t, int off, float (&v)[8]) { load8(t + off, v); }
__device__ __forceinline__ float ldsum1(const float *t, int off) { return t[off]; }
__device__ __forceinline__ void add8(float (&v)[8], const float *p) {
    const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
    v[0] += a.x; v[1] += a.y; v[2] += a.z; v[3] += a.w; v[4] += b.x; v[5] += b.y; v[6] += b.z; v[7] += b.w;
}

// snake activation (shaders/ops_conv.metal:204-213) with exp(alpha) and exp(-beta) precomputed per column
__device__ __forceinline__ void snake8(float (&v)[8], const float (&a)[8], const float (&b)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        v[e] = v[e] + snake_sin2(v[e] * a[e]) * b[e];
    }
}

template <int EPI, int PITCH = TP>
__device__ __forceinline__ void tile_epilogue(const GemmProblem &P, const float *tile, int m0, int n0, int ks, int tid) {
    const int M = P.M, N = P.N;
    if (P.splits > 1) {
        // raw f32 partial of this split: ws[(ks*M + m)*N + n]
        float *w = P.ws + (long long)ks * M * N;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int c = tid + 512 * p, row = c >> 4, col = (c & 15) * 8;
            const int m = m0 + row, n = n0 + col;
            if (m < M && n < N) {
                float *o = w + (long long)m * N + n;
                float v[8];
                ldsum8(tile, row * PITCH + col, v);
                *(float4 *)o = make_float4(v[0], v[1], v[2], v[3]);
                *(float4 *)(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
            }
        }
        return;
    }
    if constexpr (EPI == EPI_STORE) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int c = tid + 512 * p, row = c >> 4, col = (c & 15) * 8;
            const int m = m0 + row, n = n0 + col;
            if (m >= M || n >= N) continue;
            float v[8];
            ldsum8(tile, row * PITCH + col, v);
            if (P.bias) add8(v, P.bias + n);
            if (P.silu)
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = silu_f(v[e]);
            const long long o = rowmap_phys(P.ymap, m) * (long long)P.ldy + n;
            if (P.y_f16) {
                half8 hi;
#pragma unroll
                for (int e = 0; e < 8; ++e) hi[e] = (half_t)v[e];
                *(half8 *)((half_t *)P.Y + o) = hi;
                if (P.y_lo) {
                    half8 lo;
#pragma unroll
                    for (int e = 0; e < 8; ++e) lo[e] = (half_t)(v[e] - (float)hi[e]);
                    *(half8 *)((half_t *)P.Y + o + P.y_lo) = lo;
                }
            } else {
                float *y = (float *)P.Y + o;
                *(float4 *)y = make_float4(v[0], v[1], v[2], v[3]);
                *(float4 *)(y + 4) = make_float4(v[4], v[5], v[6], v[7]);
            }
        }
    } else if constexpr (EPI == EPI_SWIGLU) {
        // tile columns 0..63: w1 rows 64j.., columns 64..127: the matching w3 rows (j = n0 / 128)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int c = tid + 512 * p, row = c >> 3, col = (c & 7) * 8;
            const int m = m0 + row;
            if (m >= M) continue;
            float a[8], b[8];
            ldsum8(tile, row * PITCH + col, a);
            ldsum8(tile, row * PITCH + 64 + col, b);
            float y[8];
            half8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                y[e] = silu_f(a[e]) * b[e];
                o[e] = (half_t)y[e];
            }
            half_t *dst = (half_t *)P.Y + rowmap_phys(P.ymap, m) * (long long)P.ldy + n0 / 2 + col;
            *(half8 *)dst = o;
            if (P.y_lo) {
                half8 lo;
#pragma unroll
                for (int e = 0; e < 8; ++e) lo[e] = (half_t)(y[e] - (float)o[e]);
                *(half8 *)(dst + P.y_lo) = lo;
            }
        }
    } else if constexpr (EPI == EPI_SNAKE) {
        // the thread's 8 columns are the same in every pass: bias and snake table loaded once, before
        // any store (inside the loop each load would wait for the previous pass's store, which may
        // alias it)
        const int col = (tid & 15) * 8, n = n0 + col;
        float bv[8], ea[8], eb[8];
        if (n < N) {
            if (P.bias) load8(P.bias + n, bv);
            load8(P.snake + n, ea);
            load8(P.snake + N + n, eb);
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int row = (tid >> 4) + 32 * p;
            const int m = m0 + row;
            if (m >= M || n >= N) continue;
            float v[8];
            ldsum8(tile, row * PITCH + col, v);
            if (P.bias)
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] += bv[e];
            snake8(v, ea, eb);
            half8 hi, lo;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                hi[e] = (half_t)v[e];
                lo[e] = (half_t)(v[e] - (float)hi[e]);
            }
            half_t *y = (half_t *)P.Y + rowmap_phys(P.ymap, m) * (long long)P.ldy + n;
            *(half8 *)y = hi;
            *(half8 *)(y + P.y_lo) = lo;
            *(half8 *)(y + P.y_hi2) = hi;
        }
    } else if constexpr (EPI == EPI_RSNAKE) {
        // bias and snake table as in EPI_SNAKE; the stream rows of all four passes are read before
        // the first store
        const int col = (tid & 15) * 8, n = n0 + col;
        float bv[8], ea[8], eb[8], xr[4][8];
        if (n < N) {
            if (P.bias) load8(P.bias + n, bv);
            load8(P.snake + n, ea);
            load8(P.snake + N + n, eb);
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int m = m0 + (tid >> 4) + 32 * p;
            if (P.r_add && m < M && n < N) load8(P.R + rowmap_phys(P.rmap, m) * (long long)P.ldr + n, xr[p]);
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int row = (tid >> 4) + 32 * p;
            const int m = m0 + row;
            if (m >= M || n >= N) continue;
            float v[8];
            ldsum8(tile, row * PITCH + col, v);
            if (P.bias)
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] += bv[e];
            if (P.r_add)
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] += xr[p][e];
            float *x = P.R + rowmap_phys(P.rmap, m) * (long long)P.ldr + n;
            *(float4 *)x = make_float4(v[0], v[1], v[2], v[3]);
            *(float4 *)(x + 4) = make_float4(v[4], v[5], v[6], v[7]);
            snake8(v, ea, eb);
            half8 hi, lo;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                hi[e] = (half_t)v[e];
                lo[e] = (half_t)(v[e] - (float)hi[e]);
            }
            const int C = P.y_lo;
            half_t *y = (half_t *)P.Y + rowmap_phys(P.ymap, m) * (long long)P.ldy + n + 2 * C * (n / C);
            *(half8 *)y = hi;
            *(half8 *)(y + C) = lo;
            *(half8 *)(y + 2 * C) = hi;
        }
    } else if constexpr (EPI == EPI_RESID) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int c = tid + 512 * p, row = c >> 4, col = (c & 15) * 8;
            const int m = m0 + row, n = n0 + col;
            if (m >= M || n >= N) continue;
            float v[8];
            ldsum8(tile, row * PITCH + col, v);
            if (P.bias) add8(v, P.bias + n);
            const float *g = P.gate + (long long)(m / P.gate_L) * P.gate_ld + n;
            float *x = P.R + rowmap_phys(P.rmap, m) * (long long)P.ldr + n;
            const float4 g0 = *(const float4 *)g, g1 = *(const float4 *)(g + 4);
            float4 x0 = *(float4 *)x, x1 = *(float4 *)(x + 4);
            x0.x = x0.x + v[0] * g0.x; x0.y = x0.y + v[1] * g0.y; x0.z = x0.z + v[2] * g0.z; x0.w = x0.w + v[3] * g0.w;
            x1.x = x1.x + v[4] * g1.x; x1.y = x1.y + v[5] * g1.y; x1.z = x1.z + v[6] * g1.z; x1.w = x1.w + v[7] * g1.w;
            *(float4 *)x = x0;
            *(float4 *)(x + 4) = x1;
        }
    } else {  // EPI_QKV: the 128 columns of the tile lie in one of q, k, v (Hq % 128 == 0)
        const int region = n0 / P.Hq;
        if (region < 2) {
            const float *nw = region == 0 ? P.qn : P.kn;
            half_t *dst = region == 0 ? P.Q : P.Kd;
            const float sc = region == 0 ? P.q_scale : 1.0f;
            // this thread's 8 columns are the same in every pass: bias and norm weight loaded once
            const int col = (tid & 15) * 8, n = n0 + col;
            const int h = (n - region * P.Hq) >> 6, d0 = n & 63;
            float bw[8], nwv[8];
            if (P.bias) load8(P.bias + n, bw);
            else
#pragma unroll
                for (int e = 0; e < 8; ++e) bw[e] = 0.0f;
            load8(nw + d0, nwv);
            // the RoPE rows of all four passes, loaded before any store: a store to Q/K may alias
            // the table, so a load left inside the loop would wait for the previous pass's store
            float cs4[4][8];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int m = m0 + (tid >> 4) + 32 * p;
                const int t = m < M ? m % P.q_L : P.rope_len;
                if (t < P.rope_len) load8(P.rope + (t * 32 + (d0 >> 1)) * 2, cs4[p]);
            }
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int row = (tid >> 4) + 32 * p, m = m0 + row;
                float v[8];
                ldsum8(tile, row * PITCH + col, v);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] += bw[e];
                // per-head RMS over the 64 columns held by 8 neighbouring lanes (same row, same head)
                float ss = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
                // partners 1, 2 (quad permutes) and 4 (row half-mirror) lanes apart
                ss += dpp_mov<DPP_XOR1>(ss);
                ss += dpp_mov<DPP_XOR2>(ss);
                ss += dpp_mov<DPP_HALF_MIRROR>(ss);
                const float inv = 1.0f / sqrtf(ss / 64.0f + P.rms_eps);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = v[e] * inv * nwv[e];
                if (m >= M) continue;
                const int b = m / P.q_L, t = m - b * P.q_L, s = P.q_soff + t;
                if (t < P.rope_len) {
                    const float *cv = cs4[p];
#pragma unroll
                    for (int e = 0; e < 8; e += 2) {
                        const float x0 = v[e], x1 = v[e + 1];
                        v[e] = x0 * cv[e] - x1 * cv[e + 1];
                        v[e + 1] = x0 * cv[e + 1] + x1 * cv[e];
                    }
                }
                half_t *o = dst + (((long long)b * P.nh + h) * P.S_att + s) * 64 + d0;
                *(half8 *)o = half8{(half_t)(v[0] * sc), (half_t)(v[1] * sc), (half_t)(v[2] * sc), (half_t)(v[3] * sc),
                                    (half_t)(v[4] * sc), (half_t)(v[5] * sc), (half_t)(v[6] * sc), (half_t)(v[7] * sc)};
            }
        } else {
            // V, stored transposed along s: Vt[b][h][d][s]. The tile's rows are cut into chunks of 8
            // positions aligned in s (per sample), so interior chunks are one 16-byte store; chunks at
            // a sample or tile edge store only their valid elements. Lanes run along columns, so the
            // LDS reads of a chunk (8 rows, one column) are conflict-free.
            const int col = tid & 127, n = n0 + col;
            const int h = (n - 2 * P.Hq) >> 6, d = n & 63;
            const float bn = P.bias ? P.bias[n] : 0.0f;
            const int m1 = min(m0 + BM, M);
            const int b0 = m0 / P.q_L, b1 = (m1 - 1) / P.q_L;
            int total = 0;
            for (int b = b0; b <= b1; ++b) {
                const int ta = max(m0 - b * P.q_L, 0), tb = min(m1 - b * P.q_L, P.q_L);
                total += (P.q_soff + tb + 7) / 8 - (P.q_soff + ta) / 8;
            }
            for (int g = tid >> 7; g < total; g += 4) {
                int b = b0, j = g, ta = 0, tb = 0;
                for (;; ++b) {   // the sample this chunk belongs to (every g < total has one)
                    ta = max(m0 - b * P.q_L, 0);
                    tb = min(m1 - b * P.q_L, P.q_L);
                    const int nb = (P.q_soff + tb + 7) / 8 - (P.q_soff + ta) / 8;
                    if (j < nb) break;
                    j -= nb;
                }
                const int s8 = ((P.q_soff + ta) / 8 + j) * 8;    // first s of the chunk
                const int r8 = b * P.q_L + (s8 - P.q_soff) - m0;  // tile row of s8 (may lie outside)
                half_t *o = P.Vt + (((long long)b * P.nh + h) * 64 + d) * P.Sp + s8;
                if (s8 >= P.q_soff + ta && s8 + 8 <= P.q_soff + tb) {
                    half8 hv;
#pragma unroll
                    for (int e = 0; e < 8; ++e) hv[e] = (half_t)(ldsum1(tile, (r8 + e) * PITCH + col) + bn);
                    *(half8 *)o = hv;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int ss = s8 + e;
                        if (ss >= P.q_soff + ta && ss < P.q_soff + tb) o[e] = (half_t)(ldsum1(tile, (r8 + e) * PITCH + col) + bn);
                    }
                }
            }
        }
    }
}

// In-kernel stream-K fixup of one cut tile: its arrival counter (zero before the first arrival,
// reset by the last), and its contributors, workgroups w0 .. w0 + nc - 1 of G over U units, whose
// partial slots in ws follow the slot rule of gemm_sk_kernel (slot 0 when the tile is the
// workgroup's first segment, i.e. the workgroup starts at or after the tile's first unit a)
struct SkFix {
    unsigned *cnt;
    const float *ws;
    long long U, G, a, w0;
    int nc;
    __device__ const float *slot(int j) const {
        const long long ww = w0 + j;
        return ws + (ww * 2 + (ww * U / G >= a ? 0 : 1)) * (long long)(BM * BN);
    }
};

// One C tile (rows m0.., columns n0..) over the K tiles [kbeg, kbeg + nk): the pipelined K loop,
// then either the epilogue (part == null; ks = split index for a classic split-K partial) or a raw
// f32 [BM][BN] store of the accumulators to part (a stream-K segment, finished by the fixup kernel).
// HL: problems may read half-width W (hi|lo A operand); SEG: more tiles follow in this workgroup
// (stream-K), so the LDS C tile is released with a barrier at the end.
// NSX: LDS stages (4: 128 KB, one workgroup per CU; 2: 68 KB, two workgroups per CU, for grids
// of several rounds where the second workgroup covers the first's barrier and load waits).
template <int EPI, bool HL, bool SEG, int NSX = NS, bool BF = false>
__device__ __forceinline__ void pipe_tile(const GemmProblem &P, int m0, int n0, int kbeg, int nk, float *part, int ks,
                                          int tid, const SkFix *fx = nullptr) {
    // stage s: A tile at smem + s*STAGE, W tile at smem + (NSX + s)*STAGE; reused for the C tile
    constexpr int SMEM = 2 * NSX * STAGE > BM * TP * 2 ? 2 * NSX * STAGE : BM * TP * 2;
    __shared__ __attribute__((aligned(1024))) half_t smem[SMEM];

    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = P.M, N = P.N, lda = P.lda, Kc = P.Kc, pad = P.pad, aT = P.a_T;
    // w_half: W holds hc = Kc/2 channels per tap and the A row of a tap is [hi (hc) | lo (hc)]; the
    // tap's K tiles run interleaved (hi chunk c, lo chunk c, hi chunk c+1, ...) so the second read
    // of a W tile follows the first at once (L2 hit)
    const int hl = HL && P.w_half ? 1 : 0, hc = Kc / 2;
    const RowMap am = P.amap;
    const int ldw = P.ldw;

    const i32x4 rsa = make_rsrc(P.A);
    const i32x4 rsb = make_rsrc(P.W);

    // loader rows of this lane: wave*16 + i*8 + (lane >> 3), chunk (lane & 7) ^ (lane >> 3).
    // A row offsets are kept for tap 0 (byte offset of source row t - pad); tap j adds j*lda.
    const int lr = lane >> 3, lc = (lane & 7) ^ lr;
    int a_base[2], a_ts0[2], b_off[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = wave * 16 + i * 8 + lr;
        const int m = m0 + r;
        const int mm = m < M ? m : 0;
        const int b = mm / am.L;
        const int t = mm - b * am.L;
        a_ts0[i] = m < M ? t - pad : -(1 << 29);   // source position at tap 0; invalid rows never pass
        a_base[i] = ((b * am.seg + am.off + t - pad) * lda + lc * 8) * 2;
        const int n = n0 + r;
        b_off[i] = n < N ? (n * ldw + lc * 8) * 2 : -1;
    }
    const int lda2 = lda * 2;
    // K tiles are issued in order kbeg, kbeg + 1, ...: the source-row offset of the tap (tap*dil),
    // the channel offset and the W column of the next one are carried from call to call (no
    // division in the loop). The taps run in order (each tap's hi and lo chunks interleaved for
    // hi|lo problems), except in the snake-conv kernels: there K tile kt is channel chunk
    // kt / taps of tap kt % taps, so the 7 taps of a chunk re-read the same A rows (shifted by
    // dil) in consecutive K tiles while they are still in L2 (4% of a VAE decode; the DiT's k3
    // convs measured 0.4% slower that way).
    constexpr bool chunk_major = EPI == EPI_SNAKE || EPI == EPI_RSNAKE;
    const int dil = EPI == EPI_SNAKE ? P.dil : 1;   // dilated taps only in the snake-conv kernels
    const int taps = P.taps;
    int nt_tap, nt_trow, nt_kin, nt_kw;
    if (!chunk_major || hl) {
        nt_tap = kbeg * BK / Kc;
        nt_trow = nt_tap * dil;
        nt_kin = kbeg * BK - nt_tap * Kc;
        nt_kw = hl ? nt_tap * hc + ((nt_kin >> 7) << 6) : kbeg * BK;
    } else {
        const int c0 = kbeg / taps;
        nt_tap = kbeg - c0 * taps;
        nt_trow = nt_tap * dil;
        nt_kin = c0 * BK;
        nt_kw = nt_tap * Kc + nt_kin;
    }
    // A row offsets of the tap whose source-row shift is va_trow (byte offset of the source row, or
    // out of range where it falls outside its sample), rebuilt after an issue whose successor
    // shifts the rows (every K tile of the snake convs, once per tap otherwise): the rebuild's
    // branch then follows the DMAs instead of splitting them from the MFMAs around the barrier.
    // W row offsets are fixed.
    unsigned va[2], vb[2];
    int va_trow = nt_trow;
    auto set_va = [&]() {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int ts = a_ts0[i] + va_trow;
            va[i] = (ts >= 0 && ts < aT) ? (unsigned)(a_base[i] + va_trow * lda2) : 0x80000000u;
        }
    };
    set_va();
#pragma unroll
    for (int i = 0; i < 2; ++i) vb[i] = b_off[i] >= 0 ? (unsigned)b_off[i] : 0x80000000u;
    const unsigned ldsw = lds_addr(smem) + wave * 2048;   // this wave's 2 KB of each operand tile
    auto issue = [&](int kt, int stage) {
        (void)kt;   // = the previous call's kt + 1
        const int kin = nt_kin, kw = nt_kw;
        // hi|lo: K tile j of the tap is chunk j >> 1 of the hi (j even) or lo (j odd) half
        const int odd = (kin >> 6) & 1;
        const int acol = hl ? odd * hc + ((kin >> 7) << 6) : kin;
        if (!chunk_major || hl) {
            nt_kw += (hl && !odd) ? 0 : BK;
            nt_kin += BK;
            if (nt_kin == Kc) {
                nt_kin = 0;
                nt_trow += dil;
            }
        } else if (++nt_tap == taps) {
            nt_tap = 0;
            nt_trow = 0;
            nt_kin += BK;
            nt_kw = nt_kin;
        } else {
            nt_trow += dil;
            nt_kw += Kc;
        }
        const unsigned sa = ldsw + stage * STAGE * 2, sb = ldsw + (NSX + stage) * STAGE * 2;
#pragma unroll
        for (int i = 0; i < 2; ++i) dma16s(rsa, va[i], (unsigned)acol * 2, sa + i * 1024);
#pragma unroll
        for (int i = 0; i < 2; ++i) dma16s(rsb, vb[i], (unsigned)kw * 2, sb + i * 1024);
        if (nt_trow != va_trow) {
            va_trow = nt_trow;
            set_va();
        }
    };

    // wave w owns rows 32*(w>>1)..+31 and columns 64*(w&1)..+63 of the tile over the full K:
    // 2 x 4 MFMA blocks of 16x16, two 32-wide K halves per 64-wide stage
    floatx4 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int wm = wave >> 1, wn = wave & 1;
    // operand read offsets (halves) inside a stage, per K half kh: slot (4kh + lane>>4) ^ (row & 7)
    int a_rd[2][2], b_rd[2][4];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
        const int slot = (kh * 4 + (lane >> 4)) ^ (lane & 7);
#pragma unroll
        for (int i = 0; i < 2; ++i) a_rd[kh][i] = (wm * 32 + i * 16 + (lane & 15)) * BK + slot * 8;
#pragma unroll
        for (int j = 0; j < 4; ++j) b_rd[kh][j] = (wn * 64 + j * 16 + (lane & 15)) * BK + slot * 8;
    }
    auto compute = [&](int stage) {
        const half_t *sa = smem + stage * STAGE, *sb = smem + (NSX + stage) * STAGE;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
            half8 af[2], bf[4];
#pragma unroll
            for (int i = 0; i < 2; ++i) af[i] = *(const half8 *)(sa + a_rd[kh][i]);
#pragma unroll
            for (int j = 0; j < 4; ++j) bf[j] = *(const half8 *)(sb + b_rd[kh][j]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if constexpr (BF)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[i]),
                                                                            __builtin_bit_cast(bf16x8, bf[j]), acc[i][j], 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
                }
        }
    };

    // Loop invariant at the top of an iteration: tile kt has landed in stage kt%NS for every wave,
    // tiles kt+1..kt+NS-1 are in flight. Each step multiplies one stage, waits for its own DMAs of
    // the next tile (4 per wave per tile), meets the other waves at the barrier (the stage just used
    // is now free) and refills that stage NS tiles ahead.
    issue(0, 0);
#pragma unroll
    for (int j = 1; j < NSX - 1; ++j)
        if (nk > j) issue(j, j);
    wait_vmcnt(4 * min(nk - 1, NSX - 2));
    block_barrier();
    if (nk > NSX - 1) issue(NSX - 1, NSX - 1);
#define TSN_GEMM_STEP(NEXT, S)                                                                  \
    {                                                                                           \
        compute(S);                                                                             \
        wait_vmcnt(4 * (NSX - 2));                                                              \
        block_barrier();                                                                        \
        issue(NEXT, S);                                                                         \
    }
    int kt = 0;
    for (; kt + 2 * NSX <= nk; kt += NSX) {
#pragma unroll
        for (int s2 = 0; s2 < NSX; ++s2) TSN_GEMM_STEP(kt + NSX + s2, s2)
    }
#undef TSN_GEMM_STEP
    // tail: the last < 2*NSX tiles; tile kt is visible, kt+1..min(kt+NSX-1, nk-1) in flight
    for (; kt < nk; ++kt) {
        const int st = kt % NSX;
        compute(st);
        if (kt + 1 < nk) {
            wait_vmcnt(4 * min(nk - 2 - kt, NSX - 2));
            block_barrier();
            if (kt + NSX < nk) issue(kt + NSX, st);
        }
    }
    // Every DMA has landed (the last tile was waited for). The waves store their accumulators as a
    // row-major f32 C tile in LDS, then all 8 waves run the epilogue on 8-column chunks (16-byte
    // accesses).
    block_barrier();
    float *tile = (float *)smem;
    {
        const int rb = wm * 32 + (lane >> 4) * 4, cb = wn * 64 + (lane & 15);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) tile[(rb + i * 16 + r) * TP + cb + j * 16] = acc[i][j][r];
        block_barrier();
    }
    if (SEG && part && fx) {
        // raw partial tile written through to memory (sc1), so the tile's last contributor reads
        // it from any XCD; then the arrival. The last of the tile's contributors sums every
        // contributor's slot in K order into the LDS C tile and runs the epilogue.
        //
        // Why no release/acquire fence is needed: on gfx942/gfx950 the SC1 bit of a buffer access
        // sets its scope to agent. An agent-scope store is written through the XCD's L2 to memory,
        // and its vmcnt decrement comes with that write's acknowledgement; an agent-scope load is
        // served from memory, never from a stale line of another XCD's L2. The AMDGPU memory
        // model's agent-scope fences exist for PLAIN accesses: release = buffer_wbl2 sc1 (write
        // back dirty L2 lines of plain stores), acquire = buffer_inv sc1 (drop L2 lines before
        // plain loads). No plain access takes part in this hand-off: every slot store and every
        // slot load is SC1. Order: each thread's slot stores complete (s_waitcnt vmcnt(0)) before
        // the barrier; the arrival atomic (agent scope, performed at the coherence point) is
        // issued after it; the slot loads are issued only after the counter's value came back
        // and passed a second barrier (control dependence). So every contributor's partial is in
        // memory before the last arrival is counted, and the last contributor reads it from
        // there. A fence pair here would add an L2 write-back and an L2 invalidate (measured at
        // about 7 us for buffer_inv sc1) per cut tile.
        const __amdgpu_buffer_rsrc_t rp = make_brsrc(part);
#pragma unroll 1
        for (int p = 0; p < 8; ++p) {
            const int c = tid + 512 * p, row = c >> 5, col = (c & 31) * 4;
            const floatx4 v = *(const floatx4 *)(tile + row * TP + col);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rp, (row * BN + col) * 4, 0, CPOL_SC1);
        }
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (0xF << 8));   // this thread's partial stores are done
        int *s_last = (int *)(tile + BM * TP);   // LDS word past the C tile
        block_barrier();
        if (tid == 0) {
            const unsigned old = __hip_atomic_fetch_add(fx->cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *s_last = old + 1 == (unsigned)fx->nc;
        }
        block_barrier();
        if (*s_last) {
            float v[8][4];
#pragma unroll
            for (int p = 0; p < 8; ++p) v[p][0] = v[p][1] = v[p][2] = v[p][3] = 0.0f;
            for (int j = 0; j < fx->nc; ++j) {
                const __amdgpu_buffer_rsrc_t rs = make_brsrc(fx->slot(j));
                u32x4 x[8];
#pragma unroll
                for (int p = 0; p < 8; ++p) x[p] = __builtin_amdgcn_raw_buffer_load_b128(rs, (tid + 512 * p) * 16, 0, CPOL_SC1);
#pragma unroll
                for (int p = 0; p < 8; ++p) {
                    v[p][0] += __uint_as_float(x[p][0]); v[p][1] += __uint_as_float(x[p][1]);
                    v[p][2] += __uint_as_float(x[p][2]); v[p][3] += __uint_as_float(x[p][3]);
                }
            }
#pragma unroll
            for (int p = 0; p < 8; ++p) {
                const int c = tid + 512 * p, row = c >> 5, col = (c & 31) * 4;
                *(floatx4 *)(tile + row * TP + col) = floatx4{v[p][0], v[p][1], v[p][2], v[p][3]};
            }
            block_barrier();
            tile_epilogue<EPI>(P, tile, m0, n0, 0, tid);
            if (tid == 0) __hip_atomic_store(fx->cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else if (SEG && part) {
        // raw partial tile, row-major [BM][BN], 16-byte stores (not unrolled: keeps registers free)
#pragma unroll 1
        for (int p = 0; p < 8; ++p) {
            const int c = tid + 512 * p, row = c >> 5, col = (c & 31) * 4;
            *(float4 *)(part + row * BN + col) = *(const float4 *)(tile + row * TP + col);
        }
    } else {
        tile_epilogue<EPI>(P, tile, m0, n0, ks, tid);
    }
    if (SEG) block_barrier();   // the LDS C tile is free again for the next tile
}

// gemm_pipe_kernel, data-parallel: workgroup -> (problem, split, n tile, m tile), m fastest so
// neighbouring workgroups share W columns.
// gemm_sk_kernel, stream-K (bt.sk == 1): the batch's work is a list of units (tile, K tile), problem-major,
// tile-major, K innermost; workgroup w of G takes units [w*U/G, (w+1)*U/G) and computes each tile it
// touches over its part of K. A tile covered whole gets the epilogue here; a tile cut by a
// workgroup boundary leaves f32 partials in bt.ws slot (w, 0) for the first tile of w or (w, 1) for
// its last. With bt.sk_cnt the last contributor to arrive (per-tile counter) sums the slots in K
// order and finishes the tile in this kernel; otherwise gemm_fixup_kernel does, in the same order
// (deterministic for a given G either way: the sum does not depend on who arrives last).
template <int EPI, bool HL, int NSX = NS, bool BF = false>
__device__ __forceinline__ void pipe_dp(const GemmBatch &bt) {
    const int tid = threadIdx.x;
    if ((int)blockIdx.x >= bt.total_tiles) {   // GEMV, then prefetch workgroups after the tiles
        const int e = blockIdx.x - bt.total_tiles, wave = tid >> 6, lane = tid & 63;
        if (e < bt.gv_nwg) {   // 4-row groups of the GEMV, strided over its workgroups' waves
            for (int n0 = (e * 8 + wave) * GEMV_ROWS; n0 < bt.gv.N; n0 += bt.gv_nwg * 8 * GEMV_ROWS)
                gemv_rows<uint16_t, 2>(bt.gv, n0, lane);
            for (int c = e; c < bt.pf_nwg; c += bt.gv_nwg) prefetch_wg<8>(bt.pf, c, wave, lane);   // then the prefetch
            return;
        }
        prefetch_wg<8>(bt.pf, e, wave, lane);   // gv_nwg == 0 here
        return;
    }
    const int wg = xcd_remap(blockIdx.x, bt.total_tiles);
    const int pi = (bt.nprob > 2 && wg >= bt.p[2].tile_start) ? 2 : (bt.nprob > 1 && wg >= bt.p[1].tile_start) ? 1 : 0;
    const GemmProblem &P = bt.p[pi];
    const int local = wg - P.tile_start;
    const int per_split = P.tiles_m * P.tiles_n;
    const int ks = local / per_split;
    const int rem = local - ks * per_split;
    int tm, tn;
    tile_mn(rem, P.tiles_m, P.tiles_n, tm, tn);
    const int nk = P.K / BK / P.splits;
    pipe_tile<EPI, HL, false, NSX, BF>(P, tm * BM, tn * BN, ks * nk, nk, nullptr, ks, tid);
}
template <int EPI>
__global__ __launch_bounds__(512, 1) void gemm_pipe_kernel(const GemmBatch bt) {
    pipe_dp<EPI, false>(bt);
}
// the same for batches with a half-width-W problem
template <int EPI>
__global__ __launch_bounds__(512, 1) void gemm_pipe_hl_kernel(const GemmBatch bt) {
    pipe_dp<EPI, true>(bt);
}
// bf16 A and W: the same tiles and schedules with bf16 MFMA products
template <int EPI>
__global__ __launch_bounds__(512, 1) void gemm_pipe_bf16_kernel(const GemmBatch bt) {
    pipe_dp<EPI, false, NS, true>(bt);
}
template <int EPI>
__global__ __launch_bounds__(512, 2) void gemm_pipe2_bf16_kernel(const GemmBatch bt) {
    pipe_dp<EPI, false, 2, true>(bt);
}
// two LDS stages, two workgroups per CU (grids of several rounds)
template <int EPI>
__global__ __launch_bounds__(512, 2) void gemm_pipe2_kernel(const GemmBatch bt) {
    pipe_dp<EPI, false, 2>(bt);
}
template <int EPI>
__global__ __launch_bounds__(512, 2) void gemm_pipe2_hl_kernel(const GemmBatch bt) {
    pipe_dp<EPI, true, 2>(bt);
}

// ---------------------------------------------------------------------------------------------
// Wide kernel for data-parallel grids of several rounds: 256x256 C tiles, 512 threads = 8 waves
// (two per SIMD); wave w owns the 128x64 block (rows 128*(w>>2), columns 64*(w&3)) over the full
// K: 8 x 4 MFMA blocks of 16x16, 128 f32 accumulators per lane.
//
// Why this shape: a 256x256 tile reads half the operand bytes per flop of a 128x128 tile, so half
// the L2 -> LDS traffic and half the bytes in flight for the same MFMA rate. K tiles are 64 wide:
// each stage holds 256 A rows and 256 W rows of 128 bytes (64 KB), in a ring of WNS = 2 stages (one
// K tile in flight while the other is multiplied, one barrier per K tile). Every row of a stage is
// one whole 128-byte L2 line and one request. A five-stage ring of 32-wide K tiles (64-byte rows,
// four tiles in flight) measured slower on every shape although it kept twice the bytes in
// flight: it needs twice the requests per byte (L2 requests per 8192^3 product 136 M against
// hipBLASLt's 69 M), and a laboratory copy of that loop ran its DMA-only path at half the rate of
// whole 1 KB blocks. Same box, two repetitions: 4096 x 4096 x 3072 102.3 -> 99.4 us, 4096^3 128.8
// -> 124.6 us, 8192^3 952.8 -> 900.4 us, 6352 x 4096 x 2048 124.7 -> 118.4 us.
//
// Stage layout as in pipe_tile: row r (128 B = 8 chunks of 8 halves) keeps chunk c at slot
// c ^ (r & 7). A direct-to-LDS load writes lane l's 16 bytes to slot l of a 1 KB block (8 rows),
// so lane l loads row 8b + (l >> 3), chunk (l & 7) ^ (l >> 3). MFMA operand reads (lane: row l &
// 15, chunk 4kh + (l >> 4)) touch 8 distinct 16-byte slots mod 128 bytes per 8 lanes: no bank
// conflicts. LDS operand reads per K tile: 8 waves x 24 KB against 8 x 64 MFMAs.
//
// The MFMAs take the W fragment as their first operand, so each 16x16 accumulator block is C's
// block transposed: a lane holds four adjacent columns of one row. The C tile is staged through
// LDS in two passes of 128 rows (f32, pitch WTP, one 16-byte write per block row) and each pass
// runs the 128x128 epilogue on both column halves, so every epilogue of the pipelined kernels
// applies (QKV and SwiGLU need a 128-column half inside one of q/k/v or one w1|w3 block pair, as
// there). Writing plain stores straight from the accumulators instead (8 bytes of f16 per row and
// block, no LDS, no barrier) measured slower: 4096 x 4096 x 3072 98.5 -> 104 us, the batch-16
// evaluation 6.77 -> 6.82 ms, same box; the staged 16-byte stores of whole rows write L2 lines
// whole. The per-element order of the f32 sums is that of the 128x128 kernels (K tiles in order,
// 32-wide MFMA K steps in order).
//
// Where it pays: long K (K >= 2048 and a round of tiles; against the two-stage 128x128 kernel on
// the box of the first measurements, 4096^3 170.4 -> 144.8 us with the five-stage ring). At K =
// 1024 it loses: 6352 x 3072 x 1024 51.2 -> 65.7 us (300 tiles quantise to two rounds of 256
// CUs), 6352 x 4096 x 1024 73.2 -> 71.2 us, and the batch-16 evaluation 6.75 -> 7.45 ms with it.
// ---------------------------------------------------------------------------------------------
constexpr int WB = 256, WK = 64, WNS = 2;
constexpr int WSTAGE = WB * WK;   // halves per operand tile of one stage (32 KB)
constexpr int WTP = 260;          // pitch (floats) of the staged f32 half C tile (128 x 256): 4 rows
                                  // = 16 banks apart, as TP

template <int EPI>
__device__ __forceinline__ void wide_tile(const GemmProblem &P, int m0, int n0, int tid) {
    constexpr int WKX = WK, WNX = WNS, WSX = WSTAGE, LPW = 4;   // LPW: DMAs per operand per wave per K tile
    // stage s: A tile at smem + s*WSTAGE, W tile at smem + (WNS + s)*WSTAGE; reused for the C tile
    constexpr int SMEM = 2 * WNX * WSX > 128 * WTP * 2 ? 2 * WNX * WSX : 128 * WTP * 2;
    __shared__ __attribute__((aligned(1024))) half_t smem[SMEM];

    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = P.M, N = P.N, lda = P.lda, Kc = P.Kc, pad = P.pad, aT = P.a_T;
    const RowMap am = P.amap;
    const int ldw = P.ldw;
    const i32x4 rsa = make_rsrc(P.A);
    const i32x4 rsb = make_rsrc(P.W);

    // loader rows of this lane: 32*wave + 8*i + (lane >> 3), chunk (lane & 7) ^ (lane >> 3)
    const int lr = lane >> 3, lc = (lane & 7) ^ lr;
    int a_base[LPW], a_ts0[LPW], b_off[LPW];
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
        const int r = wave * 32 + i * (32 / LPW) + lr;
        const int m = m0 + r;
        const int mm = m < M ? m : 0;
        const int b = mm / am.L;
        const int t = mm - b * am.L;
        a_ts0[i] = m < M ? t - pad : -(1 << 29);
        a_base[i] = ((b * am.seg + am.off + t - pad) * lda + lc * 8) * 2;
        const int n = n0 + r;
        b_off[i] = n < N ? (n * ldw + lc * 8) * 2 : -1;
    }
    const int lda2 = lda * 2;
    // K tiles in order; the tap's source-row offset, the channel offset and the W column carried
    int nt_trow = 0, nt_kin = 0, nt_kw = 0;
    // per-row A offsets of the current tap and fixed W row offsets, as in pipe_tile
    unsigned va[LPW], vb[LPW];
    int va_trow = 0;
    auto set_va = [&]() {
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int ts = a_ts0[i] + va_trow;
            va[i] = (ts >= 0 && ts < aT) ? (unsigned)(a_base[i] + va_trow * lda2) : 0x80000000u;
        }
    };
    set_va();
#pragma unroll
    for (int i = 0; i < LPW; ++i) vb[i] = b_off[i] >= 0 ? (unsigned)b_off[i] : 0x80000000u;
    const unsigned ldsw = lds_addr(smem) + wave * LPW * 1024;
    auto issue = [&](int stage) {
        const int kin = nt_kin, kw = nt_kw;
        nt_kw += WKX;
        nt_kin += WKX;
        if (nt_kin == Kc) {
            nt_kin = 0;
            ++nt_trow;
        }
        const unsigned sa = ldsw + stage * WSX * 2, sb = ldsw + (WNX + stage) * WSX * 2;
#pragma unroll
        for (int i = 0; i < LPW; ++i) dma16s(rsa, va[i], (unsigned)kin * 2, sa + i * 1024);
#pragma unroll
        for (int i = 0; i < LPW; ++i) dma16s(rsb, vb[i], (unsigned)kw * 2, sb + i * 1024);
        if (nt_trow != va_trow) {   // the next K tile starts a tap
            va_trow = nt_trow;
            set_va();
        }
    };

    floatx4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int wm = wave >> 2, wn = wave & 3;
    // operand read offsets (halves) inside a stage, per 32-wide K half kh: row (lane & 15) of each
    // 16-row block, chunk 4kh + (lane >> 4) at slot (4kh + (lane >> 4)) ^ (row & 7)
    constexpr int NKH = WKX / 32;
    int a_rd[NKH], b_rd[NKH];
#pragma unroll
    for (int kh = 0; kh < NKH; ++kh) {
        const int slot = (kh * 4 + (lane >> 4)) ^ (lane & 7);
        const int rd = (lane & 15) * WKX + slot * 8;
        a_rd[kh] = wm * 128 * WKX + rd;
        b_rd[kh] = wn * 64 * WKX + rd;
    }
    auto compute = [&](int stage) {
#pragma unroll
        for (int kh = 0; kh < NKH; ++kh) {
            const half_t *sa = smem + stage * WSX + a_rd[kh], *sb = smem + (WNX + stage) * WSX + b_rd[kh];
            half8 af[8], bf[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) bf[j] = *(const half8 *)(sb + j * 16 * WKX);
#pragma unroll
            for (int i = 0; i < 8; ++i) af[i] = *(const half8 *)(sa + i * 16 * WKX);
            // W rows as the MFMA's first operand: the block comes out transposed, so lane l holds
            // C[row l & 15][columns 4 (l >> 4) .. + 3] of each 16x16 block (four adjacent columns of
            // one row, stored as one vector); the products and their K order are unchanged
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[j], af[i], acc[i][j], 0, 0, 0);
        }
    };

    // ring as in pipe_tile: at the top of a step tile kt has landed in stage kt % WNS for every
    // wave and tiles kt+1 .. kt+WNS-1 are in flight (four DMAs per wave per tile)
    const int nk = P.K / WKX;
    issue(0);
#pragma unroll
    for (int j = 1; j < WNX - 1; ++j)
        if (nk > j) issue(j);
    wait_vmcnt(2 * LPW * min(nk - 1, WNX - 2));
    block_barrier();
    if (nk > WNX - 1) issue(WNX - 1);
    int kt = 0;
    for (; kt + 2 * WNX <= nk; kt += WNX) {
#pragma unroll
        for (int s2 = 0; s2 < WNX; ++s2) {
            compute(s2);
            wait_vmcnt(2 * LPW * (WNX - 2));
            block_barrier();
            issue(s2);
        }
    }
    for (; kt < nk; ++kt) {
        const int st = kt % WNX;
        compute(st);
        if (kt + 1 < nk) {
            wait_vmcnt(2 * LPW * min(nk - 2 - kt, WNX - 2));
            block_barrier();
            if (kt + WNX < nk) issue(st);
        }
    }
    // two passes of 128 rows: the waves of that row half store their accumulators as a row-major
    // f32 [128][256] tile in LDS (four adjacent columns per 16-byte write), then all 8 waves run
    // the epilogue on each 128-column half
    block_barrier();
    float *tile = (float *)smem;
#pragma unroll 1
    for (int p = 0; p < 2; ++p) {
        if (wm == p) {
            const int rb = lane & 15, cb = wn * 64 + (lane >> 4) * 4;
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    *(float4 *)(tile + (rb + i * 16) * WTP + cb + j * 16) =
                        make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
        }
        block_barrier();
        if (m0 + p * 128 < M) {
            tile_epilogue<EPI, WTP>(P, tile, m0 + p * 128, n0, 0, tid);
            if (n0 + 128 < N) tile_epilogue<EPI, WTP>(P, tile + 128, m0 + p * 128, n0 + 128, 0, tid);
        }
        block_barrier();
    }
}

// workgroup -> (problem, 256x256 tile) with the XCD remap and the grouped tile order of the
// 128x128 kernels
template <int EPI>
__global__ __launch_bounds__(512, 1) void gemm_wide_kernel(const GemmBatch bt) {
    const int wg = xcd_remap(blockIdx.x, bt.total_tiles);
    const int pi = (bt.nprob > 2 && wg >= bt.p[2].tile_start) ? 2 : (bt.nprob > 1 && wg >= bt.p[1].tile_start) ? 1 : 0;
    const GemmProblem &P = bt.p[pi];
    int tm, tn;
    tile_mn(wg - P.tile_start, P.tiles_m, P.tiles_n, tm, tn);
    wide_tile<EPI>(P, tm * WB, tn * WB, threadIdx.x);
}

// gemm_small_kernel: plain GEMMs (one tap), 64x64 C tiles over the full K, 4 waves of 32x32
// (2 x 2 MFMA blocks of 16x16), the same swizzled direct-to-LDS ring as pipe_tile (5 stages of
// 16 KB, two workgroups per CU) and the residual epilogue in place. For GEMMs whose 128x128 grid
// would need a K split to fill the chip (M ~ 800, N = 1024, K = 1024): 64x64 tiles give four times
// the workgroups with no f32 partials to write and sum.
constexpr int SB = 64;              // tile rows and columns
constexpr int SSTAGE = SB * BK;     // halves per operand tile of one stage (8 KB)
constexpr int SNS = 5;              // LDS stages of the small-tile ring (5 x 16 KB)
constexpr int STP = 68;             // pitch (floats) of the staged f32 C tile: 4 rows = 16 banks apart

// G = 2 (gemm_small2_kernel): two groups of four waves share the tile; group g multiplies the K
// tiles of parity g through its own ring of SNS2 stages, and the two f32 partial tiles are summed
// (group 0's first) before the epilogue. For grids of at most one workgroup per CU, where the
// four-wave kernel leaves one wave per SIMD to cover every LDS and barrier latency alone. Same
// box, 8 s evaluation (its out-projections and fused FFN2s, 208 tiles): 1.7816 -> 1.7554 ms with
// four stages per group; three stages 1.7426 against 1.7597 (four) and 1.7674 (five); two
// stages 1.883.
constexpr int SNS2 = 3;   // stages per group of the two-group kernel (2 x 3 x 16 KB = 96 KB)
// gemm_small3_kernel: the four-wave kernel with three stages (48 KB), three workgroups per CU, for
// grids past one round of two workgroups per CU (the 30 s fused FFN2 and out-projections: 560 tiles)
constexpr int SNS3 = 3;
template <int EPI, int G, int NSX>
__device__ __forceinline__ void small_tile(const GemmBatch &bt) {
    static_assert(EPI == EPI_RESID || EPI == EPI_STORE, "gemm_small_kernel: residual or plain store epilogue");
    constexpr int SMEM = 2 * NSX * SSTAGE * G > 2 * SB * STP * G ? 2 * NSX * SSTAGE * G : 2 * SB * STP * G;
    __shared__ __attribute__((aligned(1024))) half_t smem[SMEM];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = G == 2 ? wave >> 2 : 0, w4 = wave & 3;   // group, wave inside the group
    if ((int)blockIdx.x >= bt.total_tiles) {   // prefetch workgroups after the tiles (GemmBatch::pf)
        prefetch_wg<4 * G>(bt.pf, blockIdx.x - bt.total_tiles, wave, lane);
        return;
    }
    const int wg = xcd_remap(blockIdx.x, bt.total_tiles);
    const int pi = (bt.nprob > 2 && wg >= bt.p[2].tile_start) ? 2 : (bt.nprob > 1 && wg >= bt.p[1].tile_start) ? 1 : 0;
    const GemmProblem &P = bt.p[pi];
    int tm, tn;
    tile_mn(wg - P.tile_start, P.tiles_m, P.tiles_n, tm, tn);
    const int m0 = tm * SB, n0 = tn * SB;
    const int M = P.M, N = P.N, lda = P.lda, pad = P.pad, aT = P.a_T, ldw = P.ldw;
    const RowMap am = P.amap;
    const i32x4 rsa = make_rsrc(P.A);
    const i32x4 rsb = make_rsrc(P.W);

    // The epilogue's operands (bias, gate rows and the stream rows this thread updates: columns
    // (tid & 7)*8 .. +7 of rows (tid >> 3) and + 32 (G = 1; one pass of rows tid >> 3 for G = 2))
    // do not depend on the product: they are read here and arrive during the K loop. Read after it,
    // each pass would wait for a global load, the second behind the first pass's store (the
    // pointers may alias).
    constexpr int NPASS = 2 / G;
    const int ecol = (tid & 7) * 8, en = n0 + ecol;
    float eb[8], eg[NPASS][8], ex[NPASS][8];
#pragma unroll
    for (int e = 0; e < 8; ++e) eb[e] = 0.0f;
    if (P.bias && en < N) load8(P.bias + en, eb);
    if constexpr (EPI == EPI_RESID) {
#pragma unroll
        for (int p = 0; p < NPASS; ++p) {
            const int m = m0 + (tid >> 3) + 32 * p;
            if (m < M && en < N) {
                load8(P.gate + (long long)(m / P.gate_L) * P.gate_ld + en, eg[p]);
                load8(P.R + rowmap_phys(P.rmap, m) * (long long)P.ldr + en, ex[p]);
            }
        }
    }

    // loader rows of this lane: w4*16 + i*8 + (lane >> 3), 16-byte chunk (lane & 7) ^ (lane >> 3)
    const int lr = lane >> 3, lc = (lane & 7) ^ lr;
    int a_base[2], a_ts0[2], b_off[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = w4 * 16 + i * 8 + lr;
        const int m = m0 + r;
        const int mm = m < M ? m : 0;
        const int b = mm / am.L;
        const int t = mm - b * am.L;
        a_ts0[i] = m < M ? t - pad : -(1 << 29);
        a_base[i] = ((b * am.seg + am.off + t - pad) * lda + lc * 8) * 2;
        const int n = n0 + r;
        b_off[i] = n < N ? (n * ldw + lc * 8) * 2 : -1;
    }
    int nt_k = grp * BK;   // K column of the group's next K tile (one tap: A and W share it)
    // row offsets fixed over K (out of range outside the operand); the K column goes in soffset
    unsigned va[2], vb[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        va[i] = (a_ts0[i] >= 0 && a_ts0[i] < aT) ? (unsigned)a_base[i] : 0x80000000u;
        vb[i] = b_off[i] >= 0 ? (unsigned)b_off[i] : 0x80000000u;
    }
    // the group's ring: A stages then W stages, NSX of each
    const unsigned ldsw = lds_addr(smem) + grp * (2 * NSX * SSTAGE * 2) + w4 * 2048;
    auto issue = [&](int stage) {
        const int k = nt_k;
        nt_k += G * BK;
        const unsigned sa = ldsw + stage * SSTAGE * 2, sb = ldsw + (NSX + stage) * SSTAGE * 2;
#pragma unroll
        for (int i = 0; i < 2; ++i) dma16s(rsa, va[i], (unsigned)k * 2, sa + i * 1024);
#pragma unroll
        for (int i = 0; i < 2; ++i) dma16s(rsb, vb[i], (unsigned)k * 2, sb + i * 1024);
    };

    floatx4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int wm = w4 >> 1, wn = w4 & 1;
    int a_rd[2][2], b_rd[2][2];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
        const int slot = (kh * 4 + (lane >> 4)) ^ (lane & 7);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            a_rd[kh][i] = (wm * 32 + i * 16 + (lane & 15)) * BK + slot * 8;
            b_rd[kh][i] = (wn * 32 + i * 16 + (lane & 15)) * BK + slot * 8;
        }
    }
    const half_t *gring = smem + grp * 2 * NSX * SSTAGE;   // this group's ring
    auto compute = [&](int stage) {
        const half_t *sa = gring + stage * SSTAGE, *sb = gring + (NSX + stage) * SSTAGE;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
            half8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                af[i] = *(const half8 *)(sa + a_rd[kh][i]);
                bf[i] = *(const half8 *)(sb + b_rd[kh][i]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };

    // the K loop of pipe_tile over the group's K tiles (every G-th; the launcher makes K a
    // multiple of G*BK, so both groups take the same count): the group's tile kt landed in stage
    // kt%NSX, tiles kt+1..kt+NSX-1 in flight; the barriers are shared by both groups
    const int nk = P.K / BK / G;
    issue(0);
#pragma unroll
    for (int j = 1; j < NSX - 1; ++j)
        if (nk > j) issue(j);
    wait_vmcnt(4 * min(nk - 1, NSX - 2));
    block_barrier();
    if (nk > NSX - 1) issue(NSX - 1);
#define TSN_SMALL_STEP(S)                                                                       \
    {                                                                                           \
        compute(S);                                                                             \
        wait_vmcnt(4 * (NSX - 2));                                                              \
        block_barrier();                                                                        \
        issue(S);                                                                               \
    }
    int kt = 0;
    for (; kt + 2 * NSX <= nk; kt += NSX) {
#pragma unroll
        for (int s2 = 0; s2 < NSX; ++s2) TSN_SMALL_STEP(s2)
    }
#undef TSN_SMALL_STEP
    for (; kt < nk; ++kt) {
        const int st = kt % NSX;
        compute(st);
        if (kt + 1 < nk) {
            wait_vmcnt(4 * min(nk - 2 - kt, NSX - 2));
            block_barrier();
            if (kt + NSX < nk) issue(st);
        }
    }
    // C tile (one per group) through LDS, then 16-byte residual updates: x += gate * (acc + bias),
    // or 16-byte stores of acc + bias (SiLU on request) as f32 or f16; acc = group 0's partial +
    // group 1's
    block_barrier();
    float *tile = (float *)smem + grp * SB * STP;
    {
        const int rb = wm * 32 + (lane >> 4) * 4, cb = wn * 32 + (lane & 15);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) tile[(rb + i * 16 + r) * STP + cb + j * 16] = acc[i][j][r];
    }
    block_barrier();
    tile = (float *)smem;
#pragma unroll
    for (int p = 0; p < NPASS; ++p) {
        const int row = (tid >> 3) + 32 * p, col = ecol;
        const int m = m0 + row, n = en;
        if (m >= M || n >= N) continue;
        float v[8];
        load8(tile + row * STP + col, v);
        if constexpr (G == 2) {
            float v1[8];
            load8(tile + SB * STP + row * STP + col, v1);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] += v1[e];
        }
        if (P.bias)
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] += eb[e];
        if constexpr (EPI == EPI_STORE) {
            if (P.silu)
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = silu_f(v[e]);
            const long long o = rowmap_phys(P.ymap, m) * (long long)P.ldy + n;
            if (P.y_f16) {
                half8 h;
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = (half_t)v[e];
                *(half8 *)((half_t *)P.Y + o) = h;
            } else {
                float *y = (float *)P.Y + o;
                *(float4 *)y = make_float4(v[0], v[1], v[2], v[3]);
                *(float4 *)(y + 4) = make_float4(v[4], v[5], v[6], v[7]);
            }
        } else {
            float *x = P.R + rowmap_phys(P.rmap, m) * (long long)P.ldr + n;
#pragma unroll
            for (int e = 0; e < 8; ++e) ex[p][e] = ex[p][e] + v[e] * eg[p][e];
            *(float4 *)x = make_float4(ex[p][0], ex[p][1], ex[p][2], ex[p][3]);
            *(float4 *)(x + 4) = make_float4(ex[p][4], ex[p][5], ex[p][6], ex[p][7]);
        }
    }
}
template <int EPI>
__global__ __launch_bounds__(256, 2) void gemm_small_kernel(const GemmBatch bt) {
    small_tile<EPI, 1, SNS>(bt);
}
template <int EPI>
__global__ __launch_bounds__(256, 3) void gemm_small3_kernel(const GemmBatch bt) {
    small_tile<EPI, 1, SNS3>(bt);
}
template <int EPI>
__global__ __launch_bounds__(512, 1) void gemm_small2_kernel(const GemmBatch bt) {
    small_tile<EPI, 2, SNS2>(bt);
}

// the workgroup w of G holding unit u: w*U/G <= u < (w + 1)*U/G
__device__ __forceinline__ long long sk_owner(long long u, long long U, long long G) {
    long long w = u * G / U;
    while (w + 1 < G && (w + 1) * U / G <= u) ++w;
    while (w > 0 && w * U / G > u) --w;
    return w;
}

template <int EPI>
__global__ __launch_bounds__(512, 1) void gemm_sk_kernel(const GemmBatch bt) {
    const int tid = threadIdx.x;
    const int wg = xcd_remap(blockIdx.x, gridDim.x);
    const long long U = bt.sk_units, G = gridDim.x;
    long long u = wg * U / G;
    const long long ue = (wg + 1) * U / G;
    for (int seg = 0; u < ue; ++seg) {
        const int pi = (bt.nprob > 2 && u >= bt.p[2].unit_start) ? 2 : (bt.nprob > 1 && u >= bt.p[1].unit_start) ? 1 : 0;
        const GemmProblem &P = bt.p[pi];
        const int nkp = P.K / BK;
        const long long lu = u - P.unit_start;
        const int tile = (int)(lu / nkp);
        const int kbeg = (int)(lu - (long long)tile * nkp);
        const int nk = (int)min((long long)(nkp - kbeg), ue - u);
        int tm, tn;
        tile_mn(tile, P.tiles_m, P.tiles_n, tm, tn);
        float *part = (kbeg == 0 && nk == nkp) ? nullptr : bt.ws + ((long long)wg * 2 + (seg == 0 ? 0 : 1)) * (BM * BN);
        if (part && bt.sk_cnt) {
            // cut tile finished here by its last contributor: contributors are the workgroups
            // holding units a .. a + nkp - 1 of the tile
            SkFix fx;
            const long long a = P.unit_start + (long long)tile * nkp, b = a + nkp;
            fx.cnt = bt.sk_cnt + P.tile_start + tile;
            fx.ws = bt.ws;
            fx.U = U;
            fx.G = G;
            fx.a = a;
            fx.w0 = sk_owner(a, U, G);
            fx.nc = (int)(sk_owner(b - 1, U, G) - fx.w0 + 1);
            pipe_tile<EPI, true, true>(P, tm * BM, tn * BN, kbeg, nk, part, 0, tid, &fx);
        } else {
            pipe_tile<EPI, true, true>(P, tm * BM, tn * BN, kbeg, nk, part, 0, tid);
        }
        u += nk;
    }
}

// Stream-K fixup: one workgroup per tile of the batch; tiles cut by a workgroup boundary sum their
// partial slots in workgroup (= K) order into the LDS C tile and run the epilogue, the rest return.
template <int EPI>
__global__ __launch_bounds__(512) void gemm_fixup_kernel(const GemmBatch bt) {
    __shared__ __attribute__((aligned(16))) float tile[BM * TP];
    const int tid = threadIdx.x, t = blockIdx.x;
    const int pi = (bt.nprob > 2 && t >= bt.p[2].tile_start) ? 2 : (bt.nprob > 1 && t >= bt.p[1].tile_start) ? 1 : 0;
    const GemmProblem &P = bt.p[pi];
    const int local = t - P.tile_start;
    const int nkp = P.K / BK;
    const long long U = bt.sk_units, G = bt.sk_g;
    const long long a = P.unit_start + (long long)local * nkp, b = a + nkp;
    long long w = a * G / U;   // workgroup holding unit a: B(w) <= a < B(w + 1), B(w) = w*U/G
    while (w + 1 < G && (w + 1) * U / G <= a) ++w;
    while (w > 0 && w * U / G > a) --w;
    if ((w + 1) * U / G >= b) return;   // the tile lies inside one workgroup: finished there
    float v[8][4];
#pragma unroll
    for (int p = 0; p < 8; ++p) v[p][0] = v[p][1] = v[p][2] = v[p][3] = 0.0f;
    for (long long ww = w; ww < G && ww * U / G < b; ++ww) {
        const int slot = ww * U / G >= a ? 0 : 1;   // this tile is the first of ww, or (ww == w) its last
        const float *src = bt.ws + (ww * 2 + slot) * (BM * BN);
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const int c = tid + 512 * p;
            const float4 x = *(const float4 *)(src + c * 4);
            v[p][0] += x.x; v[p][1] += x.y; v[p][2] += x.z; v[p][3] += x.w;
        }
    }
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int c = tid + 512 * p, row = c >> 5, col = (c & 31) * 4;
        *(float4 *)(tile + row * TP + col) = make_float4(v[p][0], v[p][1], v[p][2], v[p][3]);
    }
    __syncthreads();
    int tm, tn;
    tile_mn(local, P.tiles_m, P.tiles_n, tm, tn);
    tile_epilogue<EPI>(P, tile, tm * BM, tn * BN, 0, tid);
}

// split-K reduction + epilogue, one thread per 4 columns; partials summed in split order
// (deterministic). EPI_RESID: R[rmap(m)][n] += gate[m/gate_L][n] * (sum + bias[n]);
// EPI_STORE: Y[ymap(m)][n] = act(sum + bias[n]) as f16 or f32.
template <int EPI>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const GemmBatch bt) {
    long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    // problems with a split come one after the other, M*N/4 threads each
    int pi = -1;
    for (int q = 0; q < bt.nprob; ++q) {
        if (bt.p[q].splits <= 1) continue;
        const long long nq = (long long)bt.p[q].M * bt.p[q].N / 4;
        if (idx < nq) { pi = q; break; }
        idx -= nq;
    }
    if (pi < 0) return;
    const GemmProblem &P = bt.p[pi];
    const int n4 = P.N / 4;
    const int m = (int)(idx / n4), n = (int)(idx - (long long)m * n4) * 4;
    float4 v = *(const float4 *)(P.ws + (long long)m * P.N + n);
    for (int k = 1; k < P.splits; ++k) {
        const float4 u = *(const float4 *)(P.ws + ((long long)k * P.M + m) * P.N + n);
        v.x += u.x; v.y += u.y; v.z += u.z; v.w += u.w;
    }
    if (P.bias) {
        const float4 b = *(const float4 *)(P.bias + n);
        v.x += b.x; v.y += b.y; v.z += b.z; v.w += b.w;
    }
    if constexpr (EPI == EPI_SNAKE) {
        float e[4] = {v.x, v.y, v.z, v.w};
        half4 hi, lo;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            e[j] = e[j] + snake_sin2(e[j] * P.snake[n + j]) * P.snake[P.N + n + j];
            hi[j] = (half_t)e[j];
            lo[j] = (half_t)(e[j] - (float)hi[j]);
        }
        half_t *y = (half_t *)P.Y + rowmap_phys(P.ymap, m) * (long long)P.ldy + n;
        *(half4 *)y = hi;
        *(half4 *)(y + P.y_lo) = lo;
        *(half4 *)(y + P.y_hi2) = hi;
    } else if constexpr (EPI == EPI_RSNAKE) {
        float4 *xr = (float4 *)(P.R + rowmap_phys(P.rmap, m) * (long long)P.ldr + n);
        if (P.r_add) {
            const float4 x = *xr;
            v.x += x.x; v.y += x.y; v.z += x.z; v.w += x.w;
        }
        *xr = v;
        float e[4] = {v.x, v.y, v.z, v.w};
        half4 hi, lo;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            e[j] = e[j] + snake_sin2(e[j] * P.snake[n + j]) * P.snake[P.N + n + j];
            hi[j] = (half_t)e[j];
            lo[j] = (half_t)(e[j] - (float)hi[j]);
        }
        const int C = P.y_lo;
        half_t *y = (half_t *)P.Y + rowmap_phys(P.ymap, m) * (long long)P.ldy + n + 2 * C * (n / C);
        *(half4 *)y = hi;
        *(half4 *)(y + C) = lo;
        *(half4 *)(y + 2 * C) = hi;
    } else if constexpr (EPI == EPI_RESID) {
        const float4 g = *(const float4 *)(P.gate + (long long)(m / P.gate_L) * P.gate_ld + n);
        float4 *xr = (float4 *)(P.R + rowmap_phys(P.rmap, m) * (long long)P.ldr + n);
        float4 x = *xr;
        x.x = x.x + v.x * g.x; x.y = x.y + v.y * g.y; x.z = x.z + v.z * g.z; x.w = x.w + v.w * g.w;
        *xr = x;
    } else {
        if (P.silu) { v.x = silu_f(v.x); v.y = silu_f(v.y); v.z = silu_f(v.z); v.w = silu_f(v.w); }
        const long long o = rowmap_phys(P.ymap, m) * (long long)P.ldy + n;
        if (P.y_f16) *(half4 *)((half_t *)P.Y + o) = half4{(half_t)v.x, (half_t)v.y, (half_t)v.z, (half_t)v.w};
        else *(float4 *)((float *)P.Y + o) = v;
    }
}

} // namespace

int launch_gemm(GemmBatch &b, int epi, bool a_f32, hipStream_t st) {
    TSN_TRY(gemm_plan(b, epi, a_f32));
    return gemm_launch_planned(b, epi, a_f32, st);
}

int launch_gemm_reduce(const GemmBatch &b, int epi, hipStream_t st) {
    if (b.sk && b.sk_cnt) return TSN_OK;   // finished inside the stream-K kernel
    if (b.sk) {
        const dim3 grid(b.total_tiles), block(512);
        if (epi == EPI_STORE) TSN_LAUNCH((gemm_fixup_kernel<EPI_STORE>), grid, block, 0, st, b);
        else if (epi == EPI_RESID) TSN_LAUNCH((gemm_fixup_kernel<EPI_RESID>), grid, block, 0, st, b);
        else if (epi == EPI_QKV) TSN_LAUNCH((gemm_fixup_kernel<EPI_QKV>), grid, block, 0, st, b);
        else if (epi == EPI_SNAKE) TSN_LAUNCH((gemm_fixup_kernel<EPI_SNAKE>), grid, block, 0, st, b);
        else if (epi == EPI_RSNAKE) TSN_LAUNCH((gemm_fixup_kernel<EPI_RSNAKE>), grid, block, 0, st, b);
        else TSN_LAUNCH((gemm_fixup_kernel<EPI_SWIGLU>), grid, block, 0, st, b);
        TSN_HIP_CHECK(hipGetLastError());
        return TSN_OK;
    }
    long long red = 0;
    for (int i = 0; i < b.nprob; ++i)
        if (b.p[i].splits > 1) red += (long long)b.p[i].M * b.p[i].N / 4;
    if (red == 0) return TSN_OK;
    const dim3 grid((unsigned)((red + 255) / 256)), block(256);
    if (epi == EPI_RESID) TSN_LAUNCH(splitk_reduce_kernel<EPI_RESID>, grid, block, 0, st, b);
    else if (epi == EPI_STORE) TSN_LAUNCH(splitk_reduce_kernel<EPI_STORE>, grid, block, 0, st, b);
    else if (epi == EPI_RSNAKE) TSN_LAUNCH(splitk_reduce_kernel<EPI_RSNAKE>, grid, block, 0, st, b);
    else if (epi == EPI_SNAKE) TSN_LAUNCH(splitk_reduce_kernel<EPI_SNAKE>, grid, block, 0, st, b);
    else { set_error("gemm reduce: epilogue without split-K support"); return TSN_ERR_ARG; }
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

bool gemm_needs_reduce(const GemmBatch &b) {
    if (b.sk) return b.sk_cnt == nullptr;
    for (int i = 0; i < b.nprob; ++i)
        if (b.p[i].splits > 1) return true;
    return false;
}

const char *gemm_reduce_name(const GemmBatch &b, int epi) {
    if (b.sk)
        return epi == EPI_STORE ? "gemm_fixup_kernel<0>" : epi == EPI_RESID ? "gemm_fixup_kernel<1>"
               : epi == EPI_QKV ? "gemm_fixup_kernel<2>" : epi == EPI_SNAKE ? "gemm_fixup_kernel<4>"
               : epi == EPI_RSNAKE ? "gemm_fixup_kernel<5>" : "gemm_fixup_kernel<3>";
    return epi == EPI_RESID ? "splitk_reduce_kernel<1>" : epi == EPI_RSNAKE ? "splitk_reduce_kernel<5>"
           : epi == EPI_SNAKE ? "splitk_reduce_kernel<4>" : "splitk_reduce_kernel<0>";
}

void gemm_problem_init(GemmProblem &p) {
    memset(&p, 0, sizeof p);
    p.taps = 1;
    p.dil = 1;
    p.gate_L = 1;
    p.q_L = 1;
    p.q_scale = 1.0f;
    p.splits = 1;
}

int gemm_plan(GemmBatch &b, int epi, bool a_f32) {
    TSN_REQUIRE(b.nprob >= 1 && b.nprob <= 3, "gemm: 1 to 3 problems");
    b.pf_nwg = 0;
    b.gv_nwg = 0;
    if (b.bf16) {   // one data-parallel schedule: no workspace, so no split and no stream-K
        TSN_REQUIRE(epi == EPI_STORE && !a_f32 && !b.small, "gemm bf16: plain store epilogue, bf16 A");
        b.ws = nullptr;
        b.ws_bytes = 0;
        for (int i = 0; i < b.nprob; ++i)
            TSN_REQUIRE(!b.p[i].y_f16 && !b.p[i].w_half && !b.p[i].y_lo && b.p[i].taps == 1,
                        "gemm bf16: one tap, f32 Y, no hi|lo operands");
    }
    int tiles = 0;
    for (int i = 0; i < b.nprob; ++i) {
        GemmProblem &p = b.p[i];
        TSN_REQUIRE(p.A && p.W && p.M > 0 && p.N > 0 && p.K > 0, "gemm: null operand or empty shape");
        TSN_REQUIRE(p.K % 8 == 0 && p.lda % 8 == 0 && p.ldw % 8 == 0, "gemm: K, lda, ldw must be multiples of 8");
        TSN_REQUIRE(p.taps >= 1 && p.Kc * p.taps == p.K, "gemm: K must equal taps*Kc");
        TSN_REQUIRE(p.taps == 1 || p.Kc % BK == 0, "gemm: conv channels must be a multiple of 64");
        TSN_REQUIRE(p.amap.L > 0 && p.a_T > 0, "gemm: row map");
        if (p.dil < 1) p.dil = 1;
        TSN_REQUIRE(p.dil == 1 || epi == EPI_SNAKE, "gemm: dilated taps only with the snake epilogue");
        TSN_REQUIRE((((uintptr_t)p.A) & 15) == 0 && (((uintptr_t)p.W) & 15) == 0, "gemm: A and W must be 16-byte aligned");
        if (epi == EPI_STORE) TSN_REQUIRE(p.Y && p.ymap.L > 0, "gemm: output");
        if (p.w_half)
            TSN_REQUIRE(p.Kc % (2 * BK) == 0 && p.ldw >= p.taps * (p.Kc / 2),
                        "gemm: half-width W needs Kc a multiple of 128 and ldw >= taps*Kc/2");
        if (p.y_lo && epi != EPI_SNAKE && epi != EPI_RSNAKE) {
            const int wout = epi == EPI_SWIGLU ? p.N / 2 : p.N;
            TSN_REQUIRE((epi == EPI_STORE || epi == EPI_SWIGLU) && p.y_f16 && p.y_lo % 8 == 0 && p.y_lo >= wout &&
                            p.ldy >= p.y_lo + wout,
                        "gemm: hi|lo output needs f16 Y, lo offset a multiple of 8 past the hi columns, ldy >= y_lo + width");
        }
        if (epi == EPI_SNAKE)
            TSN_REQUIRE(p.Y && p.ymap.L > 0 && p.snake && (((uintptr_t)p.snake) & 15) == 0 && p.N % 8 == 0 &&
                            p.y_lo % 8 == 0 && p.y_hi2 % 8 == 0 && p.y_lo >= p.N && p.y_hi2 >= p.y_lo + p.N &&
                            p.ldy >= p.y_hi2 + p.N && p.ldy % 8 == 0 && !p.w_half,
                        "gemm snake: table, three 8-aligned N-wide parts (hi, lo at y_lo, hi at y_hi2) inside ldy");
        else if (epi == EPI_RSNAKE)
            TSN_REQUIRE(p.R && p.rmap.L > 0 && p.Y && p.ymap.L > 0 && p.snake && (((uintptr_t)p.snake) & 15) == 0 &&
                            p.y_lo > 0 && p.y_lo % 8 == 0 && p.N % p.y_lo == 0 && p.ldr % 4 == 0 && p.ldy % 8 == 0 &&
                            !p.w_half,
                        "gemm residual snake: stream R, table, phases of y_lo (a multiple of 8) columns");
        else
            TSN_REQUIRE(!p.snake && !p.y_hi2, "gemm: snake table and second hi part only with the snake epilogues");
        if (epi == EPI_SWIGLU)
            TSN_REQUIRE(p.Y && p.ymap.L > 0 && p.y_f16 && p.N % BN == 0 && p.ldy % 8 == 0 &&
                            (((uintptr_t)p.Y) & 15) == 0,
                        "gemm swiglu: f16 output, N (= 2F) a multiple of 128, 16-byte aligned rows");
        if (epi == EPI_RESID) TSN_REQUIRE(p.R && p.gate && p.rmap.L > 0 && p.gate_L > 0, "gemm: residual output");
        if (epi == EPI_QKV) {
            TSN_REQUIRE(p.Q && p.Kd && p.Vt && p.qn && p.kn, "gemm qkv: outputs and norm weights");
            TSN_REQUIRE(p.N == 3 * p.Hq && p.Hq % BN == 0 && p.Hq == p.nh * 64, "gemm qkv: N = 3*nh*64, nh*64 % 128 == 0");
            TSN_REQUIRE(p.q_L > 0 && p.q_soff + p.q_L <= p.S_att && p.S_att <= p.Sp, "gemm qkv: attention rows");
            TSN_REQUIRE(p.rope_len == 0 || p.rope, "gemm qkv: rope table");
            TSN_REQUIRE(p.M % p.q_L == 0, "gemm qkv: M must be whole samples");
        }
        p.tiles_m = (p.M + BM - 1) / BM;
        p.tiles_n = (p.N + BN - 1) / BN;
        p.tile_start = tiles;
        tiles += p.tiles_m * p.tiles_n;
    }
    b.total_tiles = tiles;
    // the pipelined kernel needs f16 A, whole 64-wide K tiles that never straddle a conv tap,
    // 16-byte aligned rows, and every operand byte offset below 2^31 (buffer addressing)
    bool pipe = !a_f32;
    for (int i = 0; i < b.nprob && pipe; ++i) {
        const GemmProblem &p = b.p[i];
        const long long last_row = rowmap_phys(p.amap, p.M - 1) + p.a_T;
        pipe = p.K % BK == 0 && p.Kc % BK == 0 && p.lda % 8 == 0 && p.ldw % 8 == 0 && p.N % 8 == 0 &&
               (last_row + 1) * (long long)p.lda * 2 < (1LL << 31) && (long long)p.N * p.ldw * 2 < (1LL << 31) &&
               (((uintptr_t)p.bias) & 15) == 0;
        // the C-tile epilogue writes 8 columns with 16-byte accesses
        if (epi == EPI_STORE) pipe = pipe && (((uintptr_t)p.Y) & 15) == 0 && p.ldy % (p.y_f16 ? 8 : 4) == 0;
        if (epi == EPI_SNAKE) pipe = pipe && (((uintptr_t)p.Y) & 15) == 0;
        if (epi == EPI_RSNAKE) pipe = pipe && ((((uintptr_t)p.Y) | ((uintptr_t)p.R)) & 15) == 0;
        if (epi == EPI_RESID)
            pipe = pipe && (((uintptr_t)p.R) & 15) == 0 && (((uintptr_t)p.gate) & 15) == 0 && p.ldr % 4 == 0 &&
                   p.gate_ld % 4 == 0;
        // q/k rows and s-aligned chunks of Vt rows as 16-byte stores; norm weights and rope rows as
        // 16-byte loads
        if (epi == EPI_QKV)
            pipe = pipe && ((((uintptr_t)p.Q) | ((uintptr_t)p.Kd) | ((uintptr_t)p.Vt) | ((uintptr_t)p.qn) |
                             ((uintptr_t)p.kn) | ((uintptr_t)p.rope)) & 15) == 0 && p.Sp % 8 == 0;
    }
    // Split-K (pipelined kernel, residual epilogue, workspace given): one common K chunk of kc
    // tiles for every problem, the largest kc (>= 4) that divides every problem's K tiles and gives
    // at least 224 workgroups; otherwise the smallest such kc. Partials need splits*M*N floats.
    bool any_lo = false;
    for (int i = 0; i < b.nprob; ++i) {
        b.p[i].splits = 1;
        b.p[i].ws = nullptr;
        any_lo = any_lo || b.p[i].y_lo;
    }
    bool any_half = false;
    for (int i = 0; i < b.nprob; ++i) any_half = any_half || b.p[i].w_half;
    TSN_REQUIRE(pipe || !any_lo, "gemm: hi|lo output needs the pipelined kernel (f16 A, 16-byte aligned rows)");
    TSN_REQUIRE(pipe || (epi != EPI_SNAKE && epi != EPI_RSNAKE),
                "gemm snake: needs the pipelined kernel (f16 A, 16-byte aligned rows)");
    TSN_REQUIRE(pipe || !any_half, "gemm: half-width W needs the pipelined kernel (f16 A, 16-byte aligned rows)");
    // small tiles when asked for, for plain GEMMs (one tap), when the 128x128 grid would fill under
    // one round of the chip: they replace a K split and its reduce. Same box, two repetitions: the
    // 30 s evaluation's residual GEMMs (144 tiles of 128x128) 3.825 -> 3.752 ms with them; at
    // batch 16 (400 tiles) they measured 7.13 -> 7.64 ms, so the limit stays at one round
    bool one_tap = true;
    for (int i = 0; i < b.nprob; ++i) one_tap = one_tap && b.p[i].taps == 1;
    b.small = b.small && one_tap && tiles < NCU ? 1 : 0;
    // a plain store asks softly: operands outside what the small kernel takes keep the other plans,
    // and so do grids of more than one round of 64x64 tiles (two workgroups per CU). Standalone f16
    // GEMMs, same box: 794x1024x4096 31.8 -> 15.2 us, 1600x1024x1024 (400 tiles) 12.6 -> 9.8 us;
    // past one round 2202x1024x1024 (560 tiles) 13.1 -> 14.5 us, 794x4096x1024 (832) 14.0 -> 17.5 us
    if (b.small && epi == EPI_STORE) {
        long long st = 0;
        for (int i = 0; i < b.nprob; ++i)
            st += (long long)((b.p[i].M + SB - 1) / SB) * ((b.p[i].N + SB - 1) / SB);
        if (!(pipe && !any_half && !any_lo && !b.bf16) || st > 2 * NCU) b.small = 0;
    }
    if (b.small) {
        TSN_REQUIRE((epi == EPI_RESID || epi == EPI_STORE) && pipe && !any_half && !any_lo && !b.bf16,
                    "gemm small tiles: residual or plain store epilogue, f16 A and 16-byte aligned operands, no "
                    "half-width W, no hi|lo output");
        tiles = 0;
        for (int i = 0; i < b.nprob; ++i) {
            GemmProblem &p = b.p[i];
            p.tiles_m = (p.M + SB - 1) / SB;
            p.tiles_n = (p.N + SB - 1) / SB;
            p.tile_start = tiles;
            tiles += p.tiles_m * p.tiles_n;
        }
        b.total_tiles = tiles;
        b.sk = 0;
        b.pipe = 1;
        b.hl = 0;
        TSN_REQUIRE(pf_ranges_ok(b.pf), "gemm: prefetch ranges");
        // two groups of four waves per tile (gemm_small2_kernel) when the grid, prefetch
        // workgroups included, holds at most one workgroup per CU and every K splits into an even
        // number of K tiles
        bool even = true;
        for (int i = 0; i < b.nprob; ++i) even = even && b.p[i].K % (2 * BK) == 0;
        const bool st = epi == EPI_STORE;
        if (even && tiles + pf_workgroups(b.pf, 8) <= NCU) {
            b.small = 2;
            b.kname = st ? "gemm_small2_kernel<0>" : "gemm_small2_kernel<1>";
            b.pf_nwg = pf_workgroups(b.pf, 8);
        } else if (tiles > SMALL3_MIN_TILES) {
            b.small = 3;
            b.kname = st ? "gemm_small3_kernel<0>" : "gemm_small3_kernel<1>";
            b.pf_nwg = pf_workgroups(b.pf, 4);
        } else {
            b.kname = st ? "gemm_small_kernel<0>" : "gemm_small_kernel<1>";
            b.pf_nwg = pf_workgroups(b.pf, 4);
        }
        return TSN_OK;
    }
    const bool snake_epi = epi == EPI_SNAKE || epi == EPI_RSNAKE;
    if (pipe && (epi == EPI_RESID || epi == EPI_STORE || snake_epi) && b.ws && (!any_lo || snake_epi)) {
        int nkmin = 1 << 30;
        for (int i = 0; i < b.nprob; ++i) nkmin = std::min(nkmin, b.p[i].K / BK);
        int best = 0;
        if (b.split_waves) {
            // estimated time in K tiles: waves x tiles per split, plus the partial sums written and read
            // (about 2.15 MB per K-tile time) when split
            double best_cost = 1e30;
            for (int kc = nkmin; kc >= 2; --kc) {
                bool divides = true;
                long long wg = 0;
                double part = 0;
                for (int i = 0; i < b.nprob; ++i) {
                    const int nkp = b.p[i].K / BK;
                    divides = divides && nkp % kc == 0;
                    wg += (long long)b.p[i].tiles_m * b.p[i].tiles_n * (nkp / kc);
                    part += 8.0 * (nkp / kc) * b.p[i].M * (double)b.p[i].N;
                }
                if (!divides) continue;
                const bool split = kc < nkmin || wg > b.total_tiles;
                const double cost = (double)((wg + NCU - 1) / NCU) * kc + (split ? b.split_overhead + part / 2.15e6 : 0.0);
                if (cost < best_cost) {
                    best_cost = cost;
                    best = kc;
                }
            }
        } else {
            for (int kc = nkmin; kc >= 4; --kc) {
                bool divides = true;
                long long wg = 0;
                for (int i = 0; i < b.nprob; ++i) {
                    const int nkp = b.p[i].K / BK;
                    divides = divides && nkp % kc == 0;
                    wg += (long long)b.p[i].tiles_m * b.p[i].tiles_n * (nkp / kc);
                }
                if (!divides) continue;
                best = kc;
                if (wg >= 224) break;
            }
        }
        if (best > 0 && best < nkmin + 1) {
            size_t need = 0;
            for (int i = 0; i < b.nprob; ++i)
                need += (size_t)(b.p[i].K / BK / best) * b.p[i].M * b.p[i].N * sizeof(float);
            bool any = false;
            for (int i = 0; i < b.nprob; ++i) any = any || (b.p[i].K / BK / best) > 1;
            if (any && need <= b.ws_bytes) {
                size_t off = 0;
                tiles = 0;
                for (int i = 0; i < b.nprob; ++i) {
                    GemmProblem &p = b.p[i];
                    p.splits = p.K / BK / best;
                    if (p.splits > 1) {
                        TSN_REQUIRE(p.N % 4 == 0 && ((epi == EPI_STORE || epi == EPI_SNAKE)
                                                         ? p.ldy % 4 == 0
                                                         : p.ldr % 4 == 0 && p.gate_ld % 4 == 0),
                                    "gemm split-K: N and output strides must be multiples of 4");
                        p.ws = b.ws + off / sizeof(float);
                        off += (size_t)p.splits * p.M * p.N * sizeof(float);
                    }
                    p.tile_start = tiles;
                    tiles += p.tiles_m * p.tiles_n * p.splits;
                }
                b.total_tiles = tiles;
            }
        }
    }
    // Stream-K when the grid chosen above leaves CUs idle. Estimated critical path in K tiles:
    // that grid = waves * longest K range per workgroup (+2 for a split-K reduce); stream-K = units
    // per workgroup + pipeline fill, partial store and fixup.
    b.sk = 0;
    if (pipe && b.ws && !b.split_waves) {
        long long units = 0, cur = 0;
        int nkmax = 0, split = 0;
        for (int i = 0; i < b.nprob; ++i) {
            b.p[i].unit_start = units;
            units += (long long)b.p[i].tiles_m * b.p[i].tiles_n * (b.p[i].K / BK);
            nkmax = std::max(nkmax, b.p[i].K / BK / b.p[i].splits);
            split = split || b.p[i].splits > 1;
        }
        cur = (long long)((b.total_tiles + NCU - 1) / NCU) * nkmax + (split ? 2 : 0);
        const long long g = std::min<long long>(NCU, std::max<long long>(1, units / SK_MIN_UNITS));
        const bool fix_in = b.sk_cnt && b.sk_cnt_n >= b.total_tiles;
        const long long skt = (units + g - 1) / g + (fix_in ? SK_OVERHEAD_IN : SK_OVERHEAD);
        const size_t need = (size_t)g * 2 * BM * BN * sizeof(float);
        if (g > 1 && skt * 10 < cur * 8 && need <= b.ws_bytes) {
            b.sk = 1;
            b.sk_g = (int)g;
            b.sk_units = units;
            int tiles = 0;
            for (int i = 0; i < b.nprob; ++i) {   // back to one tile per (m, n): no classic split
                GemmProblem &p = b.p[i];
                p.splits = 1;
                p.ws = nullptr;
                p.tile_start = tiles;
                tiles += p.tiles_m * p.tiles_n;
            }
            b.total_tiles = tiles;
            if (!fix_in) b.sk_cnt = nullptr;   // the fixup kernel finishes the cut tiles
        }
    }
    if (!b.sk) b.sk_cnt = nullptr;
    TSN_REQUIRE(pipe || epi != EPI_SWIGLU, "gemm swiglu: needs K and row strides the pipelined kernel takes");
    b.pipe = pipe ? 1 : 0;
    b.hl = any_half ? 1 : 0;
    TSN_REQUIRE((epi != EPI_SNAKE && epi != EPI_RSNAKE) || !b.hl, "gemm snake: no half-width W");
    b.kname = b.sk ? (epi == EPI_STORE ? "gemm_sk_kernel<0>" : epi == EPI_RESID ? "gemm_sk_kernel<1>"
                      : epi == EPI_QKV ? "gemm_sk_kernel<2>" : epi == EPI_SNAKE ? "gemm_sk_kernel<4>"
                      : epi == EPI_RSNAKE ? "gemm_sk_kernel<5>" : "gemm_sk_kernel<3>")
            : pipe && b.hl ? (epi == EPI_STORE ? "gemm_pipe_hl_kernel<0>" : epi == EPI_RESID ? "gemm_pipe_hl_kernel<1>"
                              : epi == EPI_QKV ? "gemm_pipe_hl_kernel<2>" : "gemm_pipe_hl_kernel<3>")
            : pipe ? (epi == EPI_STORE ? "gemm_pipe_kernel<0>" : epi == EPI_RESID ? "gemm_pipe_kernel<1>"
                      : epi == EPI_QKV ? "gemm_pipe_kernel<2>" : epi == EPI_SNAKE ? "gemm_pipe_kernel<4>"
                      : epi == EPI_RSNAKE ? "gemm_pipe_kernel<5>" : "gemm_pipe_kernel<3>")
                   : a_f32 ? "gemm_f16_kernel<true, 0>"
                   : (epi == EPI_STORE ? "gemm_f16_kernel<false, 0>" : epi == EPI_RESID ? "gemm_f16_kernel<false, 1>"
                                                                        : "gemm_f16_kernel<false, 2>");
    // two LDS stages and two workgroups per CU once the data-parallel grid exceeds one round
    b.ns2 = pipe && !b.sk && b.total_tiles > NCU ? 1 : 0;
    // 256x256 tiles instead, when that grid still fills the chip and K is long (no split, no
    // half-width W, one of the epilogues the wide kernel stages)
    b.wide = 0;
    if (b.ns2 && !b.hl && !b.bf16 && (epi == EPI_STORE || epi == EPI_RESID || epi == EPI_QKV || epi == EPI_SWIGLU)) {
        bool nosplit = true;
        long long wt = 0;
        for (int i = 0; i < b.nprob; ++i) {
            nosplit = nosplit && b.p[i].splits == 1 && b.p[i].K >= WIDE_MIN_K;
            wt += (long long)((b.p[i].M + WB - 1) / WB) * ((b.p[i].N + WB - 1) / WB);
        }
        if (nosplit && wt >= WIDE_MIN_TILES) {
            int t = 0;
            for (int i = 0; i < b.nprob; ++i) {
                GemmProblem &p = b.p[i];
                p.tiles_m = (p.M + WB - 1) / WB;
                p.tiles_n = (p.N + WB - 1) / WB;
                p.tile_start = t;
                t += p.tiles_m * p.tiles_n;
            }
            b.total_tiles = t;
            b.wide = 1;
            b.ns2 = 0;
        }
    }
    // weight prefetch workgroups after the tiles: data-parallel pipelined kernels only
    TSN_REQUIRE(pf_ranges_ok(b.pf), "gemm: prefetch ranges");
    b.pf_nwg = pipe && !b.sk && !b.wide ? pf_workgroups(b.pf, 8) : 0;
    // GEMV rows on the CUs a single-round grid leaves free (one pipelined workgroup per CU); they
    // replace the prefetch workgroups
    b.gv_nwg = 0;
    if (b.gv.N > 0) {
        const GemvArgs &g = b.gv;
        TSN_REQUIRE(g.W && g.X && g.Y && g.wdt == DT_BF16 && g.nb == 2 && g.K == 1024 && g.ldw % 8 == 0 &&
                        g.ldx % 4 == 0 && !g.addv && !g.Y2 && !g.silu,
                    "gemm: grid GEMV needs BF16 W, two X rows, K = 1024, no addv / Y2 / SiLU");
        if (pipe && !b.sk && !b.ns2 && !b.small && NCU - b.total_tiles >= 32)
            b.gv_nwg = NCU - b.total_tiles;   // the prefetch chunks then follow each one's GEMV rows

    }
    if (b.bf16) {
        TSN_REQUIRE(pipe, "gemm bf16: needs K % 64 == 0, N % 8 == 0 and 16-byte aligned rows, W, bias and Y");
        b.kname = b.ns2 ? "gemm_pipe2_bf16_kernel<0>" : "gemm_pipe_bf16_kernel<0>";
    }
    if (b.wide)
        b.kname = epi == EPI_STORE ? "gemm_wide_kernel<0>" : epi == EPI_RESID ? "gemm_wide_kernel<1>"
                  : epi == EPI_QKV ? "gemm_wide_kernel<2>" : "gemm_wide_kernel<3>";
    else if (b.ns2 && b.hl)
        b.kname = epi == EPI_STORE ? "gemm_pipe2_hl_kernel<0>" : epi == EPI_RESID ? "gemm_pipe2_hl_kernel<1>"
                  : epi == EPI_QKV ? "gemm_pipe2_hl_kernel<2>" : "gemm_pipe2_hl_kernel<3>";
    else if (b.ns2)
        b.kname = epi == EPI_STORE ? "gemm_pipe2_kernel<0>" : epi == EPI_RESID ? "gemm_pipe2_kernel<1>"
                  : epi == EPI_QKV ? "gemm_pipe2_kernel<2>" : epi == EPI_SNAKE ? "gemm_pipe2_kernel<4>"
                  : epi == EPI_RSNAKE ? "gemm_pipe2_kernel<5>" : "gemm_pipe2_kernel<3>";
    if (a_f32) TSN_REQUIRE(epi == EPI_STORE, "gemm: f32 A operand only with a plain store epilogue");
    TSN_REQUIRE(epi == EPI_STORE || epi == EPI_RESID || epi == EPI_QKV || epi == EPI_SWIGLU || epi == EPI_SNAKE ||
                    epi == EPI_RSNAKE,
                "gemm: unknown epilogue");
    return TSN_OK;
}

int gemm_launch_planned(const GemmBatch &b, int epi, bool a_f32, hipStream_t st) {
    if (b.gv.N > 0 && b.gv_nwg == 0) TSN_TRY(launch_gemv(b.gv, st));   // no free CUs in this grid
    if (b.small) {
        const dim3 grid(b.total_tiles + b.pf_nwg);
        if (epi == EPI_RESID) {
            if (b.small == 2) TSN_LAUNCH((gemm_small2_kernel<EPI_RESID>), grid, dim3(512), 0, st, b);
            else if (b.small == 3) TSN_LAUNCH((gemm_small3_kernel<EPI_RESID>), grid, dim3(256), 0, st, b);
            else TSN_LAUNCH((gemm_small_kernel<EPI_RESID>), grid, dim3(256), 0, st, b);
        } else if (epi == EPI_STORE) {
            if (b.small == 2) TSN_LAUNCH((gemm_small2_kernel<EPI_STORE>), grid, dim3(512), 0, st, b);
            else if (b.small == 3) TSN_LAUNCH((gemm_small3_kernel<EPI_STORE>), grid, dim3(256), 0, st, b);
            else TSN_LAUNCH((gemm_small_kernel<EPI_STORE>), grid, dim3(256), 0, st, b);
        } else {
            set_error("gemm small tiles: residual or plain store epilogue only");
            return TSN_ERR_ARG;
        }
        TSN_HIP_CHECK(hipGetLastError());
        return TSN_OK;
    }
    dim3 grid(b.sk ? b.sk_g : b.total_tiles + (b.gv_nwg ? b.gv_nwg : b.pf_nwg)), block(b.pipe ? 512 : 256);
    if (b.bf16) {
        TSN_REQUIRE(b.pipe && epi == EPI_STORE, "gemm bf16: pipelined store kernel only");
        if (b.ns2) TSN_LAUNCH((gemm_pipe2_bf16_kernel<EPI_STORE>), grid, block, 0, st, b);
        else TSN_LAUNCH((gemm_pipe_bf16_kernel<EPI_STORE>), grid, block, 0, st, b);
        TSN_HIP_CHECK(hipGetLastError());
        return TSN_OK;
    }
    if (b.wide) {
        if (epi == EPI_STORE) TSN_LAUNCH((gemm_wide_kernel<EPI_STORE>), grid, block, 0, st, b);
        else if (epi == EPI_RESID) TSN_LAUNCH((gemm_wide_kernel<EPI_RESID>), grid, block, 0, st, b);
        else if (epi == EPI_QKV) TSN_LAUNCH((gemm_wide_kernel<EPI_QKV>), grid, block, 0, st, b);
        else if (epi == EPI_SWIGLU) TSN_LAUNCH((gemm_wide_kernel<EPI_SWIGLU>), grid, block, 0, st, b);
        else { set_error("gemm: no wide kernel for this epilogue"); return TSN_ERR_ARG; }
        TSN_HIP_CHECK(hipGetLastError());
        return TSN_OK;
    }
    if (b.pipe) {
        if (b.sk) {
            if (epi == EPI_STORE) TSN_LAUNCH((gemm_sk_kernel<EPI_STORE>), grid, block, 0, st, b);
            else if (epi == EPI_RESID) TSN_LAUNCH((gemm_sk_kernel<EPI_RESID>), grid, block, 0, st, b);
            else if (epi == EPI_QKV) TSN_LAUNCH((gemm_sk_kernel<EPI_QKV>), grid, block, 0, st, b);
            else if (epi == EPI_SWIGLU) TSN_LAUNCH((gemm_sk_kernel<EPI_SWIGLU>), grid, block, 0, st, b);
            else if (epi == EPI_SNAKE) TSN_LAUNCH((gemm_sk_kernel<EPI_SNAKE>), grid, block, 0, st, b);
            else if (epi == EPI_RSNAKE) TSN_LAUNCH((gemm_sk_kernel<EPI_RSNAKE>), grid, block, 0, st, b);
            else { set_error("gemm: unknown epilogue"); return TSN_ERR_ARG; }
        } else if (b.hl && b.ns2) {
            if (epi == EPI_STORE) TSN_LAUNCH((gemm_pipe2_hl_kernel<EPI_STORE>), grid, block, 0, st, b);
            else if (epi == EPI_RESID) TSN_LAUNCH((gemm_pipe2_hl_kernel<EPI_RESID>), grid, block, 0, st, b);
            else if (epi == EPI_QKV) TSN_LAUNCH((gemm_pipe2_hl_kernel<EPI_QKV>), grid, block, 0, st, b);
            else if (epi == EPI_SWIGLU) TSN_LAUNCH((gemm_pipe2_hl_kernel<EPI_SWIGLU>), grid, block, 0, st, b);
            else { set_error("gemm: unknown epilogue"); return TSN_ERR_ARG; }
        } else if (b.hl) {
            if (epi == EPI_STORE) TSN_LAUNCH((gemm_pipe_hl_kernel<EPI_STORE>), grid, block, 0, st, b);
            else if (epi == EPI_RESID) TSN_LAUNCH((gemm_pipe_hl_kernel<EPI_RESID>), grid, block, 0, st, b);
            else if (epi == EPI_QKV) TSN_LAUNCH((gemm_pipe_hl_kernel<EPI_QKV>), grid, block, 0, st, b);
            else if (epi == EPI_SWIGLU) TSN_LAUNCH((gemm_pipe_hl_kernel<EPI_SWIGLU>), grid, block, 0, st, b);
            else { set_error("gemm: unknown epilogue"); return TSN_ERR_ARG; }
        } else if (b.ns2) {
            if (epi == EPI_STORE) TSN_LAUNCH((gemm_pipe2_kernel<EPI_STORE>), grid, block, 0, st, b);
            else if (epi == EPI_RESID) TSN_LAUNCH((gemm_pipe2_kernel<EPI_RESID>), grid, block, 0, st, b);
            else if (epi == EPI_SWIGLU) TSN_LAUNCH((gemm_pipe2_kernel<EPI_SWIGLU>), grid, block, 0, st, b);
            else if (epi == EPI_SNAKE) TSN_LAUNCH((gemm_pipe2_kernel<EPI_SNAKE>), grid, block, 0, st, b);
            else if (epi == EPI_RSNAKE) TSN_LAUNCH((gemm_pipe2_kernel<EPI_RSNAKE>), grid, block, 0, st, b);
            else if (epi == EPI_QKV) TSN_LAUNCH((gemm_pipe2_kernel<EPI_QKV>), grid, block, 0, st, b);
            else { set_error("gemm: no two-stage kernel for this epilogue"); return TSN_ERR_ARG; }
        } else if (epi == EPI_STORE) TSN_LAUNCH((gemm_pipe_kernel<EPI_STORE>), grid, block, 0, st, b);
        else if (epi == EPI_RESID) TSN_LAUNCH((gemm_pipe_kernel<EPI_RESID>), grid, block, 0, st, b);
        else if (epi == EPI_QKV) TSN_LAUNCH((gemm_pipe_kernel<EPI_QKV>), grid, block, 0, st, b);
        else if (epi == EPI_SWIGLU) TSN_LAUNCH((gemm_pipe_kernel<EPI_SWIGLU>), grid, block, 0, st, b);
        else if (epi == EPI_SNAKE) TSN_LAUNCH((gemm_pipe_kernel<EPI_SNAKE>), grid, block, 0, st, b);
        else if (epi == EPI_RSNAKE) TSN_LAUNCH((gemm_pipe_kernel<EPI_RSNAKE>), grid, block, 0, st, b);
        else { set_error("gemm: unknown epilogue"); return TSN_ERR_ARG; }
    } else if (a_f32) {
        TSN_LAUNCH((gemm_f16_kernel<true, EPI_STORE>), grid, block, 0, st, b);
    } else if (epi == EPI_STORE) {
        TSN_LAUNCH((gemm_f16_kernel<false, EPI_STORE>), grid, block, 0, st, b);
    } else if (epi == EPI_RESID) {
        TSN_LAUNCH((gemm_f16_kernel<false, EPI_RESID>), grid, block, 0, st, b);
    } else if (epi == EPI_QKV) {
        TSN_LAUNCH((gemm_f16_kernel<false, EPI_QKV>), grid, block, 0, st, b);
    } else {
        set_error("gemm: unknown epilogue");
        return TSN_ERR_ARG;
    }
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

} // namespace tsn
