// Software-pipelined gfx950 kernel of the fused causal self-attention
// forward (bf16 / fp16, head_dim 32 / 64 / 128).
//
// Mathematics and operand layouts are those of attn_fwd_mfma16_kernel
// (S^T = K Q^T on v_mfma_f32_32x32x16, in-lane softmax, P kept in registers as
// the B operand of O^T = V^T P^T, V^T through ds_read_b64_tr_b16).  What this
// kernel adds is the schedule:
//
//  * Each wave overlaps its own matrix and vector work.  Step j is
//      phase 1:  MFMA  S_{j+1} = K_{j+1} Q^T
//                VALU  O *= alpha_j,  l = alpha_j * l + sum(P_j)
//      phase 2:  MFMA  O^T += V_j^T P_j^T
//                VALU  row max of S_{j+1}, alpha_{j+1}, P_{j+1} = exp2(...)
//                      packed to 16 bits
//    and both phases are interleaved by hand (one MFMA, its LDS operand
//    read, a slice of VALU), fenced with sched_barrier so the compiler keeps
//    the order.  Measured on MI355X, VALU issued between a wave's own MFMAs
//    hides about 70% of its time, against about 40% when it comes from the
//    other wave of the SIMD.
//  * K/V tiles reach LDS by LDS-DMA (buffer_load_dwordx4 ... lds): no staging
//    VGPRs and no ds_write.  K and V each have a ring of three 64-key stages;
//    DMAs run two steps ahead (K one tile ahead of V), so a step only waits
//    for loads issued a full step earlier, then one barrier publishes them.
//  * LDS rows are padded instead of XOR-swizzled, so every operand read is a
//    lane base plus an immediate offset:
//      K rows D*2 + 16 bytes, stored in the order the MFMA A rows read them;
//      V rows D*2 + 64 bytes (D >= 64), natural key order for the transpose
//      read.  Both keep the 64 lanes of a read on distinct banks.
//  * Causal workgroups are issued XCD by XCD in pairs of heads, longest query
//    tile first within the pair: each XCD's L2 holds the K/V of about two
//    heads at a time, and the longest tiles still start first.
#pragma once

#include <type_traits>

#include "attn_fwd_kernels.hpp"

namespace pmkl_amd {

template <int D, int NW>
struct PipeLayout {
    static constexpr int BN = 64;                              // keys per tile
    static constexpr int K_STRIDE = D * 2 + 16;                // bytes per K row
    static constexpr int V_STRIDE = D * 2 + (D >= 64 ? 64 : 0);
    static constexpr int K_TILE = BN * K_STRIDE;               // multiple of 1 KiB
    static constexpr int V_TILE = BN * V_STRIDE;
    static constexpr int NSTAGE = 3;
    static constexpr int K_SLOTS = K_TILE / 1024;              // 1 KiB DMA slots per tile
    static constexpr int V_SLOTS = V_TILE / 1024;
    static constexpr int PER_WAVE = (K_SLOTS + V_SLOTS + NW - 1) / NW;   // DMAs per wave per step
    static constexpr int K_RING = 0;
    static constexpr int V_RING = NSTAGE * K_TILE;
    static constexpr int DUMMY = V_RING + NSTAGE * V_TILE;     // sink of the unused slots
    static constexpr int BYTES = DUMMY + 1024;
    static_assert(K_TILE % 1024 == 0 && V_TILE % 1024 == 0, "tiles must be whole DMA slots");
};

// LDS row of key kk (0..63) in the K tile: the A-row that reads it.
// key_of_arow(i) maps A-row i = t + 4h + 8g to key t + 4g + 16h; this is
// its inverse, per 32-key block.
__device__ __forceinline__ int arow_of_key(int kk) {
    return (kk & 32) | (kk & 3) | (((kk >> 4) & 1) << 2) | (((kk >> 2) & 3) << 3);
}
__device__ __forceinline__ int key_of_lds_row(int r) { return (r & 32) | key_of_arow(r & 31); }

template <int V>
using int_c = std::integral_constant<int, V>;

// One LDS-DMA of 16 bytes per lane: bytes [off, off+16) of the buffer r land
// at LDS address m0 + 16 * lane.  Issued from inline asm so that the compiler
// does not wait for it before unrelated LDS reads; the kernel waits on vmcnt
// itself before the barrier that publishes the data.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, int off, unsigned m0) {
    asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds" ::"v"(off), "s"(m0), "s"(r)
                 : "memory");
}

template <typename T, int D, bool CAUSAL, int NW>
__global__ __launch_bounds__(NW * 64, 1) void attn_fwd_pipe_kernel(AttnParams p) {
    using E = Elt16<T>;
    using frag = typename E::frag;
    using LY = PipeLayout<D, NW>;
    constexpr int BM = 32 * NW;
    constexpr int BN = LY::BN;
    constexpr int NDB = D / 32;
    constexpr int NDK = D / 16;

    __shared__ __attribute__((aligned(1024))) unsigned char smem[LY::BYTES];
    const unsigned lds0 = (unsigned)(size_t)(__attribute__((address_space(3))) unsigned char *)smem;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = lane >> 5;
    const int col = lane & 31;

    int bh, qt;
    map_workgroup<CAUSAL>(p, bh, qt);
    const int b = bh / p.H;
    const int h = bh - b * p.H;
    const int S = p.S;

    const T *qg = (const T *)p.q + b * p.q_sb + h * p.q_sh;
    const T *kg = (const T *)p.k + b * p.k_sb + h * p.k_sh;
    const T *vg = (const T *)p.v + b * p.v_sb + h * p.v_sh;
    T *og = (T *)p.o + b * p.o_sb + h * p.o_sh;

    const int q0 = qt * BM;
    const int q0w = q0 + 32 * wave;
    const int qi = q0w + col;
    const int nt = (CAUSAL ? min(q0 + BM - 1, S - 1) : S - 1) / BN + 1;       // tiles of the workgroup
    const int n_w = q0w >= S ? 0 : (CAUSAL ? min(q0w + 31, S - 1) : S - 1) / BN + 1;  // tiles of this wave
    // Only a wave's last tile can straddle the diagonal or the end of the sequence.
    const bool last_mask =
        n_w > 0 && ((CAUSAL && (n_w - 1) * BN + BN - 1 > q0w) || ((n_w - 1) * BN + BN > S));
    const int lim = CAUSAL ? min(qi, S - 1) : S - 1;   // last key visible to this lane's row

    // ---- Q fragments: lane holds Q[qi][16dk + 8hi .. +7] ----
    frag qf[NDK];
    {
        const int qrow = min(qi, S - 1);
        const T *src = qg + (int64_t)qrow * p.q_ss + 8 * hi;
#pragma unroll
        for (int dk = 0; dk < NDK; ++dk) qf[dk] = __builtin_bit_cast(frag, *(const u32x4_t *)(src + 16 * dk));
    }

    // ---- LDS-DMA plan: slot s = i * NW + wave of a step (K slots, then V
    // slots, then dummies).  The per-lane byte offset into the tile's buffer
    // range is the same for every tile. ----
    int dma_off[LY::PER_WAVE];
#pragma unroll
    for (int i = 0; i < LY::PER_WAVE; ++i) {
        const int s = i * NW + wave;
        int off = 0;
        if (s < LY::K_SLOTS) {
            const int byte = s * 1024 + 16 * lane;
            const int row = byte / LY::K_STRIDE, cb = byte % LY::K_STRIDE;
            if (cb < D * 2) off = (int)((key_of_lds_row(row) * p.k_ss) * (int64_t)sizeof(T)) + cb;
        } else if (s < LY::K_SLOTS + LY::V_SLOTS) {
            const int byte = (s - LY::K_SLOTS) * 1024 + 16 * lane;
            const int row = byte / LY::V_STRIDE, cb = byte % LY::V_STRIDE;
            if (cb < D * 2) off = (int)((row * p.v_ss) * (int64_t)sizeof(T)) + cb;
        }
        dma_off[i] = off;
    }
    // Buffer range of one tile: its first key to the last key of the
    // sequence (rows past the end read as zero and are masked).
    auto tile_rsrc = [&](const T *base, int64_t ss, int t) {
        const int rows = min(BN, S - t * BN);
        return __builtin_amdgcn_make_buffer_rsrc((void *)(base + (int64_t)t * BN * ss), (short)0,
                                                 (int)(((rows - 1) * ss + D) * sizeof(T)), 0x00020000);
    };
    // Issue this wave's PER_WAVE DMAs for K tile tk and V tile tv (a tile
    // outside [0, nt) sends its slots to the dummy sink, so every wave always
    // issues the same number of DMAs per step).
    auto dma_step = [&](int tk, int tv) {
        const bool kv = tk >= 0 && tk < nt, vv = tv >= 0 && tv < nt;
        const __amdgpu_buffer_rsrc_t kr = tile_rsrc(kg, p.k_ss, kv ? tk : 0);
        const __amdgpu_buffer_rsrc_t vr = tile_rsrc(vg, p.v_ss, vv ? tv : 0);
        const unsigned kbase = lds0 + LY::K_RING + (unsigned)((kv ? tk : 0) % LY::NSTAGE) * LY::K_TILE;
        const unsigned vbase = lds0 + LY::V_RING + (unsigned)((vv ? tv : 0) % LY::NSTAGE) * LY::V_TILE;
#pragma unroll
        for (int i = 0; i < LY::PER_WAVE; ++i) {
            const int s = i * NW + wave;   // wave-uniform
            if (s < LY::K_SLOTS)
                lds_dma16(kr, dma_off[i], kv ? kbase + 1024u * s : lds0 + LY::DUMMY);
            else if (s < LY::K_SLOTS + LY::V_SLOTS)
                lds_dma16(vr, dma_off[i], vv ? vbase + 1024u * (s - LY::K_SLOTS) : lds0 + LY::DUMMY);
            else
                lds_dma16(kr, 0, lds0 + LY::DUMMY);
        }
    };
    // Wait until only the DMAs of the latest step are outstanding.
    auto dma_wait_keep_step = [&]() {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LY::PER_WAVE) : "memory");
    };

    // ---- per-lane LDS read bases (stage offsets are added per step) ----
    const int kread = LY::K_RING + col * LY::K_STRIDE + 16 * hi;
    const int g = lane >> 4, tt = lane & 15;
    const int vread = LY::V_RING + (16 * (g >> 1) + (tt >> 2)) * LY::V_STRIDE + 2 * (16 * (g & 1) + 4 * (tt & 3));

    f32x16_t acc[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
    float m_run = -INFINITY;
    float l_run = 0.f;
    const float c2 = p.scale_log2;

    // Scores of one tile from the K stage at byte offset kst (prologue only).
    auto qk = [&](int kst, f32x16_t(&s)[2]) {
        const unsigned char *kb0 = smem + kst + kread;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
#pragma unroll
            for (int dk = 0; dk < NDK; ++dk) {
                const frag a = __builtin_bit_cast(frag, *(const u32x4_t *)(kb0 + kb * 32 * LY::K_STRIDE + 32 * dk));
                s[kb] = E::mma(a, qf[dk], s[kb]);
            }
        }
    };
    // Element mask of a tile whose first key is kbase.
    auto mask = [&](f32x16_t(&s)[2], int kbase) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (kbase + 32 * kb + 16 * hi + r > lim) s[kb][r] = -INFINITY;
    };
    // Softmax of one tile: row max, alpha, probabilities packed to 16 bits.
    auto softmax_a = [&](f32x16_t(&s)[2], uint32_t(&pk)[2][8]) -> float {
        float mx = fmaxf(s[0][0], s[0][1]);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = (kb == 0 ? 2 : 0); r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
        mx = half_max(mx);
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2((m_run - m_new) * c2);   // 0 on the first tile
        m_run = m_new;
        const float moff = (m_new == -INFINITY) ? 0.f : -m_new * c2;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 8; ++r)
                pk[kb][r] = E::pack2(fast_exp2(__builtin_fmaf(s[kb][2 * r], c2, moff)),
                                     fast_exp2(__builtin_fmaf(s[kb][2 * r + 1], c2, moff)));
        return alpha;
    };
    // Rescale O and l by alpha and add the tile's probabilities (as rounded
    // for the P*V product, so O is normalised by exactly its weights) to l.
    auto softmax_b = [&](float alpha, const uint32_t(&pk)[2][8]) {
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 8; ++r) l_run = E::sum2(pk[kb][r], l_run);
    };
    typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
    typedef short s16x8_t __attribute__((ext_vector_type(8)));
    // V^T operand of P*V MFMA i from the V stage at byte offset vst:
    // key block kb = i / (2*NDB), 8-key half c = (i / NDB) % 2, d block db = i % NDB.
    auto vread2 = [&](int vst, int i) {
        const unsigned char *a0 = smem + vst + vread +
                                  (32 * (i / (2 * NDB)) + 8 * ((i / NDB) % 2)) * LY::V_STRIDE + 64 * (i % NDB);
        const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)a0);
        const s16x4_t up = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(a0 + 4 * LY::V_STRIDE));
        const s16x8_t a8 = {lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
        return __builtin_bit_cast(frag, a8);
    };
    // O^T += V^T P^T without interleave (a wave's last tile).
    auto pv = [&](int vst, const uint32_t(&pk)[2][8]) {
#pragma unroll
        for (int i = 0; i < 4 * NDB; ++i) {
            const int kb = i / (2 * NDB), c = (i / NDB) % 2, db = i % NDB;
            const u32x4_t bw = {pk[kb][4 * c], pk[kb][4 * c + 1], pk[kb][4 * c + 2], pk[kb][4 * c + 3]};
            acc[db] = E::mma(vread2(vst, i), __builtin_bit_cast(frag, bw), acc[db]);
        }
    };

    // Phase 1 of a step: the 2*NDK score MFMAs of the next tile (K stage kst)
    // with the O/l rescale by a and the sum of the current probabilities.
    // Each group is one MFMA, the LDS read of the operand two MFMAs ahead,
    // NDB*16/(2*NDK) multiplies and 16/(2*NDK) dot2 sums.
    auto phase1 = [&](int kst, f32x16_t(&s)[2], float a, const uint32_t(&pk)[2][8]) {
        constexpr int NM = 2 * NDK;
        constexpr int PF = NM < 2 ? NM : 2;
        constexpr int MUL_PER = NDB * 16 / NM;
        constexpr int DOT_PER = 16 / NM;
        const unsigned char *kb0 = smem + kst + kread;
        auto kaddr = [&](int i) { return kb0 + (i / NDK) * 32 * LY::K_STRIDE + 32 * (i % NDK); };
        frag kf[NM];
#pragma unroll
        for (int i = 0; i < PF; ++i) kf[i] = __builtin_bit_cast(frag, *(const u32x4_t *)kaddr(i));
        l_run *= a;
#pragma unroll
        for (int i = 0; i < NM; ++i) {
            const int kb = i / NDK, dk = i % NDK;
            if (i + PF < NM) kf[i + PF] = __builtin_bit_cast(frag, *(const u32x4_t *)kaddr(i + PF));
            if (dk == 0) {
#pragma unroll
                for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
            }
            s[kb] = E::mma(kf[i], qf[dk], s[kb]);
#pragma unroll
            for (int u = i * MUL_PER; u < (i + 1) * MUL_PER; ++u) acc[u / 16][u % 16] *= a;
#pragma unroll
            for (int u = i * DOT_PER; u < (i + 1) * DOT_PER; ++u) l_run = E::sum2(pk[u / 8][u % 8], l_run);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // Phase 2 of a step: the 4*NDB P*V MFMAs of the current tile (V stage
    // vst, probabilities pc) with the softmax of the next tile's scores s: the
    // row max rides on the first two MFMAs, the lane-half exchange and alpha
    // on the third, the exp2 / pack of the 16 probability pairs on the rest.
    // Returns alpha of the next tile; its packed probabilities go to pn.
    auto phase2 = [&](int vst, const uint32_t(&pc)[2][8], f32x16_t(&s)[2], uint32_t(&pn)[2][8]) -> float {
        constexpr int NM = 4 * NDB;
        constexpr int PF = NM < 2 ? NM : 2;
        constexpr int NX = NM > 3 ? NM - 3 : 1;
        frag vf[NM];
#pragma unroll
        for (int i = 0; i < PF; ++i) vf[i] = vread2(vst, i);
        float mx = -INFINITY, alpha = 0.f, moff = 0.f;
#pragma unroll
        for (int i = 0; i < NM; ++i) {
            const int kb = i / (2 * NDB), c = (i / NDB) % 2, db = i % NDB;
            if (i + PF < NM) vf[i + PF] = vread2(vst, i + PF);
            const u32x4_t bw = {pc[kb][4 * c], pc[kb][4 * c + 1], pc[kb][4 * c + 2], pc[kb][4 * c + 3]};
            acc[db] = E::mma(vf[i], __builtin_bit_cast(frag, bw), acc[db]);
            if (i < 2 || (NM < 3 && i == NM - 1)) {
#pragma unroll
                for (int kk = 0; kk < 2; ++kk)
                    if (kk == i || NM < 2)
#pragma unroll
                        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kk][r]);
            }
            if (i == (NM < 3 ? NM - 1 : 2)) {
                mx = half_max(mx);
                const float m_new = fmaxf(m_run, mx);
                alpha = fast_exp2((m_run - m_new) * c2);
                m_run = m_new;
                moff = (m_new == -INFINITY) ? 0.f : -m_new * c2;
            }
            if (i >= 3 || (NM <= 3 && i == NM - 1)) {
                const int x = NM > 3 ? i - 3 : 0;
#pragma unroll
                for (int u = x * 16 / NX; u < (x + 1) * 16 / NX; ++u) {
                    const int kk = u / 8, r = 2 * (u % 8);
                    pn[kk][u % 8] = E::pack2(fast_exp2(__builtin_fmaf(s[kk][r], c2, moff)),
                                             fast_exp2(__builtin_fmaf(s[kk][r + 1], c2, moff)));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        return alpha;
    };

    // ---- prologue: DMA K_0, K_1, V_0 (and K_2, V_1 in flight); S_0 ----
    dma_step(0, -1);
    dma_step(1, 0);
    dma_step(2, 1);
    dma_wait_keep_step();
    __syncthreads();

    f32x16_t sc[2];                  // scores of the next tile
    uint32_t pk0[2][8], pk1[2][8];   // packed probabilities, by tile parity
    float alpha = 0.f;
    if (n_w > 0) {
        qk(0, sc);
        if (n_w == 1 && last_mask) mask(sc, 0);
        alpha = softmax_a(sc, pk0);
    }
    __syncthreads();   // K stage 0 is refilled by the first step

    // Straight-line body of a step whose wave also scores tile j+1 (MASK:
    // tile j+1 needs the element mask).  alpha passes through an opaque copy
    // so the O/l rescale cannot be computed outside this region.
    auto pipelined = [&](auto mask_c, int j, int kst, int vst, uint32_t(&pc)[2][8], uint32_t(&pn)[2][8]) {
        constexpr bool MASK = decltype(mask_c)::value;
        float a1 = alpha;
        asm volatile("" : "+v"(a1));
        __builtin_amdgcn_sched_barrier(0);
        phase1(kst, sc, a1, pc);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (MASK) mask(sc, (j + 1) * BN);
        __builtin_amdgcn_sched_barrier(0);
        alpha = phase2(vst, pc, sc, pn);
        __builtin_amdgcn_sched_barrier(0);
    };
    // Step j: K_{j+1} in K stage (j+1)%3, V_j in V stage j%3, P_j in pc.
    // DMAs for K_{j+3} and V_{j+2} are issued first and waited on one step later.
    int kst = LY::K_TILE;   // byte offset of K stage (j+1) % 3 within the K ring
    int vst = 0;            // byte offset of V stage j % 3 within the V ring
    auto step = [&](int j, uint32_t(&pc)[2][8], uint32_t(&pn)[2][8]) {
        dma_step(j + 3, j + 2);
        if (j + 1 < n_w) {
            if (j + 1 == n_w - 1 && last_mask)
                pipelined(std::true_type{}, j, kst, vst, pc, pn);
            else
                pipelined(std::false_type{}, j, kst, vst, pc, pn);
        } else if (j < n_w) {
            float a1 = alpha;
            asm volatile("" : "+v"(a1));
            softmax_b(a1, pc);
            pv(vst, pc);
        }
        kst = kst == 2 * LY::K_TILE ? 0 : kst + LY::K_TILE;
        vst = vst == 2 * LY::V_TILE ? 0 : vst + LY::V_TILE;
        dma_wait_keep_step();   // K_{j+2} and V_{j+1} have landed (this wave's part)
        __syncthreads();
    };
    for (int j = 0; j < nt; j += 2) {
        step(j, pk0, pk1);
        if (j + 1 < nt) step(j + 1, pk1, pk0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // drain the sink / beyond-range DMAs

    // ---- epilogue: normalise, store O, m, l ----
    const float l_tot = half_sum(l_run);
    if (n_w > 0 && qi < S) {
        const float inv = 1.0f / l_tot;
        T *orow = og + (int64_t)qi * p.o_ss;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d = 32 * db + 8 * g4 + 4 * hi;
                u32x2_t w2 = {E::pack2(acc[db][4 * g4] * inv, acc[db][4 * g4 + 1] * inv),
                              E::pack2(acc[db][4 * g4 + 2] * inv, acc[db][4 * g4 + 3] * inv)};
                *(u32x2_t *)(orow + d) = w2;
            }
        if (hi == 0) {
            const int64_t mi = (int64_t)bh * S + qi;
            const float mval = m_run * p.scale;
            if (p.ml_f32) {
                ((float *)p.m)[mi] = mval;
                ((float *)p.l)[mi] = l_tot;
            } else {
                ((T *)p.m)[mi] = (T)mval;
                ((T *)p.l)[mi] = (T)l_tot;
            }
        }
    }
}

}  // namespace pmkl_amd
