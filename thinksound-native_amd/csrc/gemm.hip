// gemm.hip — MFMA GEMM / implicit-GEMM conv1d for gfx950 with fused epilogues.
//
// Replaces the reference's GEMM route (src/net.mm:14-23 -> shaders/gemm_mpp.metal:18-48) and its
// conv route (src/net.mm:25-49: im2col + GEMM). The conv is an implicit GEMM: the weight is
// stored [OC][K][IC] so each 64-wide K tile is one tap of IC channels, and the A loader reads
// row t - pad + tap of the same sample (zero outside the sample) — no im2col buffer.
//
// Tile: 128x128x64, 256 threads = 4 waves in 2x2, each wave 64x64 = 4x4 MFMA 16x16x32 f16
// blocks (64 f32 accumulators per lane). LDS: A and B tiles, two stages, rows padded to 72
// halves (144 B) so the 16 rows one MFMA operand read touches fall in distinct banks.
// One barrier per K tile: the next tile is loaded into registers before the MFMAs of the
// current tile and written to the other LDS stage after them.
//
// Work order: grid = all tiles of all problems (<= 2, e.g. audio + text stream of a joint
// block). Workgroup IDs are remapped so each XCD (8 per MI355X, dispatched round-robin by
// workgroup ID) receives one contiguous range of tiles, and tiles are numbered n-major, so the
// workgroups of one XCD share W column blocks in that XCD's L2.
#include "kernels.h"

#include <string.h>

namespace tsn {

namespace {

constexpr int BM = 128, BN = 128, BK = 64, LDSW = BK + 8;

__device__ inline int xcd_remap(int bid, int nwg) {
    const int xcd = bid & 7, idx = bid >> 3;
    const int base = nwg >> 3, rem = nwg & 7;
    return (xcd < rem ? xcd * (base + 1) : rem * (base + 1) + (xcd - rem) * base) + idx;
}

__device__ inline half8 zero_h8() { return half8{0, 0, 0, 0, 0, 0, 0, 0}; }

__device__ inline float silu_f(float v) { return v / (1.0f + __expf(-v)); }

template <bool A_F32, int EPI>
__global__ __launch_bounds__(256, 2) void gemm_f16_kernel(const GemmBatch bt) {
    __shared__ __attribute__((aligned(16))) half_t sA[2][BM * LDSW];
    __shared__ __attribute__((aligned(16))) half_t sB[2][BN * LDSW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile = xcd_remap(blockIdx.x, gridDim.x);
    const int pi = (bt.nprob > 1 && tile >= bt.p[1].tile_start) ? 1 : 0;
    const GemmProblem &P = bt.p[pi];

    const int local = tile - P.tile_start;
    const int tn = local / P.tiles_m, tm = local - tn * P.tiles_m;
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

    // ---------------- epilogue ----------------
    // acc[i][j][r] holds C[row][col]: row = wm*64 + i*16 + (lane>>4)*4 + r, col = wn*64 + j*16 + (lane&15)
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
                    ss += __shfl_xor(ss, 1);
                    ss += __shfl_xor(ss, 2);
                    ss += __shfl_xor(ss, 4);
                    ss += __shfl_xor(ss, 8);
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
                        const float partner = __shfl_xor(v[i][j][r], 1);
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

} // namespace

void gemm_problem_init(GemmProblem &p) {
    memset(&p, 0, sizeof p);
    p.taps = 1;
    p.gate_L = 1;
    p.q_L = 1;
    p.q_scale = 1.0f;
}

int launch_gemm(GemmBatch &b, int epi, bool a_f32, hipStream_t st) {
    TSN_REQUIRE(b.nprob >= 1 && b.nprob <= 2, "gemm: 1 or 2 problems");
    int tiles = 0;
    for (int i = 0; i < b.nprob; ++i) {
        GemmProblem &p = b.p[i];
        TSN_REQUIRE(p.A && p.W && p.M > 0 && p.N > 0 && p.K > 0, "gemm: null operand or empty shape");
        TSN_REQUIRE(p.K % 8 == 0 && p.lda % 8 == 0 && p.ldw % 8 == 0, "gemm: K, lda, ldw must be multiples of 8");
        TSN_REQUIRE(p.taps >= 1 && p.Kc * p.taps == p.K, "gemm: K must equal taps*Kc");
        TSN_REQUIRE(p.taps == 1 || p.Kc % BK == 0, "gemm: conv channels must be a multiple of 64");
        TSN_REQUIRE(p.amap.L > 0 && p.a_T > 0, "gemm: row map");
        TSN_REQUIRE((((uintptr_t)p.A) & 15) == 0 && (((uintptr_t)p.W) & 15) == 0, "gemm: A and W must be 16-byte aligned");
        if (epi == EPI_STORE) TSN_REQUIRE(p.Y && p.ymap.L > 0, "gemm: output");
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
    dim3 grid(tiles), block(256);
    if (a_f32) {
        TSN_REQUIRE(epi == EPI_STORE, "gemm: f32 A operand only with a plain store epilogue");
        hipLaunchKernelGGL((gemm_f16_kernel<true, EPI_STORE>), grid, block, 0, st, b);
    } else if (epi == EPI_STORE) {
        hipLaunchKernelGGL((gemm_f16_kernel<false, EPI_STORE>), grid, block, 0, st, b);
    } else if (epi == EPI_RESID) {
        hipLaunchKernelGGL((gemm_f16_kernel<false, EPI_RESID>), grid, block, 0, st, b);
    } else if (epi == EPI_QKV) {
        hipLaunchKernelGGL((gemm_f16_kernel<false, EPI_QKV>), grid, block, 0, st, b);
    } else {
        set_error("gemm: unknown epilogue");
        return TSN_ERR_ARG;
    }
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

} // namespace tsn
