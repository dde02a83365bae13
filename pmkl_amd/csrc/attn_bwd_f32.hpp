// fp32 backward of the attention output (gfx950, VALU): the reference's
// algorithm (fused_self_attention.cpp:66-135) in the same two passes and with
// the same workspace as the 16-bit kernels (attn_bwd_kernels.hpp), on the
// vector ALUs.  The float path serves the reference's own float
// configuration (small, launch-bound shapes), so it is written for clarity:
// one wave per owned row, four waves per workgroup.
//
//   attn_bwd_f32_dq_kernel    wave = query row i.  Lane = key j within a chunk
//                             of 64 for s_ij = <q_i, k_j> and dP_ij =
//                             <dout_i, v_j> (q_i and dout_i spread over the
//                             lanes by head_dim element and broadcast with
//                             readlane), then lane = head_dim element for
//                             dq_i += dS_ij k_j, dS_ij taken lane by lane.
//                             Writes lse2_i and D_i to the workspace.
//   attn_bwd_f32_dkdv_kernel  wave = key row j, lane = query i in a chunk of
//                             64 for s_ij, dP_ij, P_ij = exp2(s_ij c - lse2_i)
//                             and dS_ij = P_ij (dP_ij - D_i); then lane =
//                             head_dim element for dv_j += P_ij dout_i and
//                             dk_j += dS_ij q_i.
#pragma once

#include "attn_bwd_kernels.hpp"

namespace pmkl_amd {

constexpr int kBwdF32Waves = 4;   // owned rows per workgroup (one per wave)

__device__ __forceinline__ float bwd_f32_wave_sum(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

// Value of lane `src` (uniform) of x.
__device__ __forceinline__ float bwd_f32_lane(float x, int src) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), src));
}

// <a, row>: a[d] is held by lane d % 64 in register a[d / 64]; row is this
// lane's own 16-byte aligned row of D floats.
template <int D>
__device__ __forceinline__ float bwd_f32_dot(const float (&a)[(D + 63) / 64], const float *row) {
    float acc = 0.f;
#pragma unroll
    for (int d = 0; d < D; d += 4) {
        const f32x4_t r = *(const f32x4_t *)(row + d);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = __builtin_fmaf(bwd_f32_lane(a[(d + e) / 64], (d + e) % 64), r[e], acc);
    }
    return acc;
}

template <int D, bool CAUSAL>
__global__ __launch_bounds__(kBwdF32Waves * 64) void attn_bwd_f32_dq_kernel(BwdParams p) {
    constexpr int NE = (D + 63) / 64;   // head_dim elements per lane
    const int lane = threadIdx.x & 63;
    const int S = p.S;
    const int64_t row = (int64_t)blockIdx.x * kBwdF32Waves + (threadIdx.x >> 6);   // bh * S + qi
    if (row >= (int64_t)p.BH * S) return;   // the whole wave
    const int64_t bh = row / S;
    const int qi = (int)(row - bh * S);
    const float *kg = bwd_head<const float>(p, p.k, BK, (int)bh);
    const float *vg = bwd_head<const float>(p, p.v, BV, (int)bh);
    const int kss = p.ss[BK], vss = p.ss[BV];
    const float *qr_i = bwd_head<const float>(p, p.q, BQ, (int)bh) + (int64_t)qi * p.ss[BQ];
    const float *dr_i = bwd_head<const float>(p, p.dout, BDOUT, (int)bh) + (int64_t)qi * p.ss[BDOUT];

    float qv[NE], dov[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) {
        const int d = lane + 64 * e;
        qv[e] = d < D ? qr_i[d] : 0.f;
        dov[e] = d < D ? dr_i[d] : 0.f;
    }
    const float m_i = bwd_load_ml<float>(p.m, row, true);
    const float l_i = bwd_load_ml<float>(p.l, row, true);
    const float lse2 = m_i * 1.4426950408889634f + __log2f(l_i);
    const float c = p.scale_log2;
    const int last = CAUSAL ? qi : S - 1;   // last visible key

    // P and dP of this lane's key j0 + lane (0 past the last visible key)
    auto prob = [&](int j0, float &pv, float &dp) __attribute__((always_inline)) {
        const int j = j0 + lane;
        const int jc = j <= last ? j : last;
        const float s = bwd_f32_dot<D>(qv, kg + (int64_t)jc * kss);
        dp = bwd_f32_dot<D>(dov, vg + (int64_t)jc * vss);
        pv = j <= last ? fast_exp2(__builtin_fmaf(s, c, -lse2)) : 0.f;
    };

    float drow;
    if (p.o != nullptr) {
        const float *or_i = bwd_head<const float>(p, p.o, BO, (int)bh) + (int64_t)qi * p.ss[BO];
        float part = 0.f;
#pragma unroll
        for (int e = 0; e < NE; ++e) {
            const int d = lane + 64 * e;
            if (d < D) part = __builtin_fmaf(or_i[d], dov[e], part);
        }
        drow = bwd_f32_wave_sum(part);
    } else {
        float part = 0.f;
        for (int j0 = 0; j0 <= last; j0 += 64) {
            float pv, dp;
            prob(j0, pv, dp);
            part = __builtin_fmaf(pv, dp, part);
        }
        drow = bwd_f32_wave_sum(part);
    }
    if (lane == 0) {
        p.lse2[row] = lse2;
        p.drow[row] = drow;
    }

    float acc[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) acc[e] = 0.f;
    for (int j0 = 0; j0 <= last; j0 += 64) {
        float pv, dp;
        prob(j0, pv, dp);
        const float ds = pv * (dp - drow);
        const int n = min(64, last - j0 + 1);
        for (int jj = 0; jj < n; ++jj) {
            const float dsj = bwd_f32_lane(ds, jj);
            const float *kr = kg + (int64_t)(j0 + jj) * kss;
#pragma unroll
            for (int e = 0; e < NE; ++e) {
                const int d = lane + 64 * e;
                if (d < D) acc[e] = __builtin_fmaf(dsj, kr[d], acc[e]);
            }
        }
    }
    float *dq_i = bwd_head<float>(p, p.dq, BDQ, (int)bh) + (int64_t)qi * p.ss[BDQ];
#pragma unroll
    for (int e = 0; e < NE; ++e) {
        const int d = lane + 64 * e;
        if (d < D) dq_i[d] = acc[e] * p.scale;
    }
}

template <int D, bool CAUSAL>
__global__ __launch_bounds__(kBwdF32Waves * 64) void attn_bwd_f32_dkdv_kernel(BwdParams p) {
    constexpr int NE = (D + 63) / 64;
    const int lane = threadIdx.x & 63;
    const int S = p.S;
    const int64_t row = (int64_t)blockIdx.x * kBwdF32Waves + (threadIdx.x >> 6);   // bh * S + kj
    if (row >= (int64_t)p.BH * S) return;
    const int64_t bh = row / S;
    const int kj = (int)(row - bh * S);
    const float *qg = bwd_head<const float>(p, p.q, BQ, (int)bh);
    const float *dog = bwd_head<const float>(p, p.dout, BDOUT, (int)bh);
    const int qss = p.ss[BQ], doss = p.ss[BDOUT];
    const float *lse2g = p.lse2 + bh * S;
    const float *drowg = p.drow + bh * S;
    const float *kr_j = bwd_head<const float>(p, p.k, BK, (int)bh) + (int64_t)kj * p.ss[BK];
    const float *vr_j = bwd_head<const float>(p, p.v, BV, (int)bh) + (int64_t)kj * p.ss[BV];

    float kv[NE], vv[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) {
        const int d = lane + 64 * e;
        kv[e] = d < D ? kr_j[d] : 0.f;
        vv[e] = d < D ? vr_j[d] : 0.f;
    }
    const float c = p.scale_log2;
    const int first = CAUSAL ? kj : 0;   // first query that sees key kj

    float acc_k[NE], acc_v[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) acc_k[e] = acc_v[e] = 0.f;
    for (int i0 = first; i0 < S; i0 += 64) {
        const int i = i0 + lane;
        const int ic = i < S ? i : S - 1;
        const float s = bwd_f32_dot<D>(kv, qg + (int64_t)ic * qss);
        const float dp = bwd_f32_dot<D>(vv, dog + (int64_t)ic * doss);
        const float pv = i < S ? fast_exp2(__builtin_fmaf(s, c, -lse2g[ic])) : 0.f;
        const float ds = pv * (dp - drowg[ic]);
        const int n = min(64, S - i0);
        for (int ii = 0; ii < n; ++ii) {
            const float pi = bwd_f32_lane(pv, ii);
            const float dsi = bwd_f32_lane(ds, ii);
            const float *qr = qg + (int64_t)(i0 + ii) * qss;
            const float *dr = dog + (int64_t)(i0 + ii) * doss;
#pragma unroll
            for (int e = 0; e < NE; ++e) {
                const int d = lane + 64 * e;
                if (d < D) {
                    acc_v[e] = __builtin_fmaf(pi, dr[d], acc_v[e]);
                    acc_k[e] = __builtin_fmaf(dsi, qr[d], acc_k[e]);
                }
            }
        }
    }
    float *dk_j = bwd_head<float>(p, p.dk, BDK, (int)bh) + (int64_t)kj * p.ss[BDK];
    float *dv_j = bwd_head<float>(p, p.dv, BDV, (int)bh) + (int64_t)kj * p.ss[BDV];
#pragma unroll
    for (int e = 0; e < NE; ++e) {
        const int d = lane + 64 * e;
        if (d < D) {
            dk_j[d] = acc_k[e] * p.scale;
            dv_j[d] = acc_v[e];
        }
    }
}

}  // namespace pmkl_amd
