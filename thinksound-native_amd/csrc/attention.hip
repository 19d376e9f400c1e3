// attention.hip — joint audio+text flash attention for gfx950 (hd = 64, non-causal).
//
// Replaces the reference's three-pass attention (src/dit_fwd.cpp:83-102 dispatching
// shaders/gemm_attn.metal:96-202: attn_qk materialises [nh,S,S] f32 scores, softmax_rows runs one
// thread per row, attn_pav reads the scores back). Here one workgroup owns 64 queries of one
// (sample, head); 4 waves own 16 queries each; K and Vᵀ tiles of 64 keys are staged in LDS
// (two stages, register prefetch) and the softmax is online, so no score buffer exists.
//
// MFMA formulation (v_mfma_f32_16x16x32_f16; A row = lane&15, B col = lane&15, K group = lane>>4,
// D[4*(lane>>4)+r][lane&15]):
//   Sᵀ = K·Qᵀ  : A = K rows from LDS, B = the wave's Q rows (registers). Lane l then holds the
//                scores of query l&15 for keys 16j + 4(l>>4) + r.
//   Oᵀ += Vᵀ·Pᵀ: B = the lane's own probabilities (keys 32c + 4g + r and 32c + 16 + 4g + r form
//                the 8 K-values of group g = l>>4 — the same key order is used for Vᵀ), A = Vᵀ
//                rows read from LDS. Lane l holds Oᵀ[d = 16dt + 4g + r][query l&15], so the
//                per-query rescale and the final 1/l are lane-local.
// Probabilities are rounded to f16 before both the PV product and the row sum, so numerator and
// denominator see the same values.
#include "kernels.h"

namespace tsn {

namespace {

constexpr int KB = 64, LDSW = 72;

__device__ inline half8 zero_h8() { return half8{0, 0, 0, 0, 0, 0, 0, 0}; }

__global__ __launch_bounds__(256) void flash_attn_kernel(const AttnArgs a) {
    __shared__ __attribute__((aligned(16))) half_t sK[2][KB * LDSW];
    __shared__ __attribute__((aligned(16))) half_t sV[2][KB * LDSW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int bh = blockIdx.y;
    const int S = a.S, Sp = a.Sp;
    const half_t *Qp = a.Q + (long long)bh * S * 64;
    const half_t *Kp = a.K + (long long)bh * S * 64;
    const half_t *Vp = a.Vt + (long long)bh * 64 * Sp;

    const int q = blockIdx.x * 64 + wave * 16 + (lane & 15);
    const int g = lane >> 4;
    half8 qf[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
        qf[ks] = q < S ? *(const half8 *)(Qp + (long long)q * 64 + ks * 32 + g * 8) : zero_h8();

    const int lrow = tid >> 3, lch = tid & 7;
    half8 rk[2], rv[2];
    auto load = [&](int kb) {
        const int key0 = kb * KB;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int key = key0 + lrow + 32 * r;
            rk[r] = key < S ? *(const half8 *)(Kp + (long long)key * 64 + lch * 8) : zero_h8();
            rv[r] = *(const half8 *)(Vp + (long long)(lrow + 32 * r) * Sp + key0 + lch * 8);
        }
    };
    auto store = [&](int s) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            *(half8 *)&sK[s][(lrow + 32 * r) * LDSW + lch * 8] = rk[r];
            *(half8 *)&sV[s][(lrow + 32 * r) * LDSW + lch * 8] = rv[r];
        }
    };

    float m_i = -INFINITY, l_i = 0.0f;
    floatx4 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int nkb = (S + KB - 1) / KB;
    load(0);
    store(0);
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
        const int s = kb & 1;
        if (kb + 1 < nkb) load(kb + 1);
        floatx4 sc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            sc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const half8 kf = *(const half8 *)&sK[s][(j * 16 + (lane & 15)) * LDSW + ks * 32 + g * 8];
                sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[ks], sc[j], 0, 0, 0);
            }
        }
        float x[4][4];
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = kb * KB + j * 16 + g * 4 + r;
                x[j][r] = key < S ? sc[j][r] * a.scale_log2 : -INFINITY;
                mx = fmaxf(mx, x[j][r]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_i, mx);
        const float alpha = exp2f(m_i - m_new);
        half_t ph[4][4];
        float psum = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                ph[j][r] = (half_t)exp2f(x[j][r] - m_new);
                psum += (float)ph[j][r];
            }
        psum += __shfl_xor(psum, 16);
        psum += __shfl_xor(psum, 32);
        l_i = l_i * alpha + psum;
        m_i = m_new;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const half8 pf = half8{ph[2 * c][0], ph[2 * c][1], ph[2 * c][2], ph[2 * c][3],
                                   ph[2 * c + 1][0], ph[2 * c + 1][1], ph[2 * c + 1][2], ph[2 * c + 1][3]};
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const half_t *vr = &sV[s][(dt * 16 + (lane & 15)) * LDSW + c * 32 + g * 4];
                const half4 lo = *(const half4 *)vr, hi = *(const half4 *)(vr + 16);
                const half8 vf = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf, o[dt], 0, 0, 0);
            }
        }
        if (kb + 1 < nkb) store(s ^ 1);
        __syncthreads();
    }

    if (q < S) {
        const float inv = 1.0f / l_i;
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
                *(half4 *)op = half4{(half_t)(o[dt][0] * inv), (half_t)(o[dt][1] * inv),
                                     (half_t)(o[dt][2] * inv), (half_t)(o[dt][3] * inv)};
            }
        }
    }
}

// f32 [S, ld] q/k/v slices -> Q/K [nh][S][64], Vt [nh][64][Sp] (f16), one thread per element
__global__ void attn_pack_kernel(const float *qkv, int S, int nh, int ld, int q_off, int k_off, int v_off,
                                 half_t *Q, half_t *K, half_t *Vt, int Sp) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)nh * Sp * 64;
    if (idx >= total) return;
    const int d = (int)(idx & 63);
    const long long rest = idx >> 6;
    const int s = (int)(rest % Sp);
    const int h = (int)(rest / Sp);
    if (s < S) {
        const float *row = qkv + (long long)s * ld + h * 64 + d;
        Q[((long long)h * S + s) * 64 + d] = (half_t)row[q_off];
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
    TSN_REQUIRE((((uintptr_t)a.Q) & 15) == 0 && (((uintptr_t)a.K) & 15) == 0 && (((uintptr_t)a.Vt) & 15) == 0,
                "attention: 16-byte aligned Q/K/Vt");
    dim3 grid((a.S + 63) / 64, a.BH), block(256);
    hipLaunchKernelGGL(flash_attn_kernel, grid, block, 0, st, a);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

int launch_attn_pack(const float *qkv, int S, int nh, int ld, int q_off, int k_off, int v_off,
                     half_t *Q, half_t *K, half_t *Vt, int Sp, hipStream_t st) {
    TSN_REQUIRE(qkv && Q && K && Vt && S > 0 && nh > 0 && Sp >= S, "attn_pack: arguments");
    const long long total = (long long)nh * Sp * 64;
    const int blocks = (int)((total + 255) / 256);
    hipLaunchKernelGGL(attn_pack_kernel, dim3(blocks), dim3(256), 0, st, qkv, S, nh, ld, q_off, k_off, v_off, Q, K, Vt, Sp);
    TSN_HIP_CHECK(hipGetLastError());
    return TSN_OK;
}

} // namespace tsn
