// gfx950 (CDNA4) kernels of the fused self-attention backward (gradients of O).
//
// Reference: pmkl_pytorch_ext/fused_self_attention.cpp:66-135
// (host_self_attention_backward, reached through fused_self_attention_bw,
// :175-215, and the autograd backward of pmkl_function/__init__.py:25-32).
// For every head, query n and key j, with the m, l the forward returned:
//   P_nj  = exp(s_nj * scale - m_n) / l_n        (0 where masked)
//   dP_nj = dout_n . v_j
//   dS_nj = P_nj * (dP_nj - D_n),   D_n = sum_j P_nj dP_nj
//   dq_n  = scale * sum_j dS_nj k_j,   dk_j = scale * sum_n dS_nj q_n,
//   dv_j  = sum_n P_nj dout_n
// which is the reference's per-(n, j) sum (:101-124) regrouped.
//
// Two passes, neither with atomics:
//   attn_bwd_dq_kernel    a workgroup owns 32 query rows per wave;
//                         K and V tiles of 64 keys stream through LDS.  One
//                         loop over the keys gives D_n (skipped when the
//                         caller passes O: D_n = dout_n . o_n), a second one
//                         dS and dQ.  D_n and log2-sum-exp of every row go to
//                         the caller's workspace for the second pass.
//   attn_bwd_dkdv_kernel  a workgroup owns 32 key rows per wave; Q, dO tiles of 64
//                         queries and their two row vectors stream through
//                         LDS; dK, dV accumulate in registers.
// Both use the forward's layouts (attn_fwd_kernels.hpp): transposed products
// with the owned rows as the MFMA column, the A-row permutation key_of_arow
// so that a lane half owns 16 consecutive streamed rows, P and dS packed
// straight into the B operand of the next product, and the LDS transpose read
// ds_read_b64_tr_b16 for operands needed with the other orientation.  A
// streamed tensor read both as rows and transposed is kept in LDS twice, once
// per swizzle, so both reads are bank-conflict free.
#pragma once

#include "attn_fwd_kernels.hpp"

namespace pmkl_amd {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// The [B, H, S, D] tensors of the backward, indexing the stride arrays.
enum BwdTensor : int { BQ = 0, BK, BV, BO, BDOUT, BDQ, BDK, BDV };

struct BwdParams {
    const void *q, *k, *v, *o, *dout;   // [B, H, S, D], head_dim contiguous; o may be null
    const void *m, *l;                  // [BH, S] contiguous, the forward's outputs
    void *dq, *dk, *dv;                 // [B, H, S, D]
    float *lse2;                        // workspace [BH, S]: m * log2(e) + log2(l)
    float *drow;                        // workspace [BH, S]: D_n
    int32_t S, BH, H;
    int32_t n_qtiles, n_ktiles;         // ceil(S / owned rows per workgroup), dq and dk/dv kernels
    float scale, scale_log2;
    int32_t ml_f32;                     // m, l stored as float (else in T)
    int64_t sb[8], sh[8];               // batch and head element strides, by BwdTensor
    int32_t ss[8];                      // seq (row) element strides, by BwdTensor
};

// Row 0 of head bh (= b H + h) of tensor t.
template <typename T>
__device__ __forceinline__ T *bwd_head(const BwdParams &p, const void *base, int t, int bh) {
    const int b = bh / p.H, h = bh - b * p.H;
    return (T *)base + (int64_t)b * p.sb[t] + (int64_t)h * p.sh[t];
}

// Waves per workgroup: 8 (two per SIMD) where the registers of a wave fit in
// 256, else 4 (one per SIMD, up to 512 registers): at head_dim 128 the
// pipelined dQ loop (two score sets) and the dK/dV accumulators.
template <int D> constexpr int bwd_waves_dq() { return D >= 128 ? 4 : 8; }
template <int D> constexpr int bwd_waves_dkdv() { return D >= 128 ? 4 : 8; }

// 16-byte chunk (logical chunk pc of row `row`) staging of a 64-row tile:
// loads go to registers ahead of use (the dK/dV pass one tile ahead, the
// dQ pass's plain loop below head_dim 128), LDS writes place the chunk at its
// swizzled position in each layout the tensor is read with; the dQ pass at
// head_dim 128 moves the chunks by LDS DMA instead.
template <typename T, int D, int NW_>
struct BwdTile {
    static constexpr int NW = NW_;
    static constexpr int THREADS = NW * 64;
    static constexpr int ROWS = 32 * NW;        // owned rows per workgroup
    static constexpr int BN = 64;
    static constexpr int CPR = D / 8;
    static constexpr int CHUNKS = BN * CPR;
    static constexpr int LOADS = (CHUNKS + THREADS - 1) / THREADS;
    static constexpr bool PARTIAL = CHUNKS % THREADS != 0;
};

// Buffer resource of the rows [r0, S) of a [S, D] matrix with row stride ss
// elements: rows past S read as zero.
template <typename T, int D>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t bwd_rows_rsrc(const T *base, int r0, int S, int ss) {
    const int rows = min(64, S - r0);
    return __builtin_amdgcn_make_buffer_rsrc((void *)(base + (int64_t)r0 * ss), (short)0,
                                             (int)((rows - 1) * ss + D) * (int)sizeof(T), 0x00020000);
}

// A-operand fragment (rows) of a 32-row block from a tile stored with swz_k:
// lane reads row 32 blk + key_of_arow(col), head_dim 16 dk + 8 hi .. +7.
template <typename T, int D>
__device__ __forceinline__ typename Elt16<T>::frag bwd_row_frag(const T *tile, int blk, int dk, int arow, int hi) {
    constexpr int CPR = D / 8;
    const int row = 32 * blk + arow;
    const int x = 2 * dk + hi;
    return __builtin_bit_cast(typename Elt16<T>::frag,
                              *(const u32x4_t *)(tile + row * D + 8 * (x ^ swz_k<CPR>(row))));
}

// A-operand fragment of the transpose (head_dim x 16 streamed rows) from a
// tile stored with swz_v: 32 head-dim columns 32 db .., streamed rows of the
// 16-row block c of the 32-row block blk, in the order that matches a B
// operand packed from registers 8c .. 8c+7 of the key_of_arow layout.
template <typename T, int D>
__device__ __forceinline__ typename Elt16<T>::frag bwd_tr_frag(const T *tile, int blk, int c, int db, int vrow0,
                                                               int vcol0) {
    constexpr int CPR = D / 8;
    typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
    typedef short s16x8_t __attribute__((ext_vector_type(8)));
    const int r0 = 32 * blk + 8 * c + vrow0;
    const int cc = 32 * db + vcol0;
    const int ch = cc >> 3, part = cc & 7;
    const T *a0 = tile + r0 * D + 8 * (ch ^ swz_v<CPR>(r0)) + part;
    const T *a1 = tile + (r0 + 4) * D + 8 * (ch ^ swz_v<CPR>(r0 + 4)) + part;
    s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)a0);
    s16x4_t hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)a1);
    return __builtin_bit_cast(typename Elt16<T>::frag,
                              s16x8_t{lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]});
}

template <typename T>
__device__ __forceinline__ float bwd_load_ml(const void *base, int64_t i, bool f32) {
    return f32 ? ((const float *)base)[i] : (float)((const T *)base)[i];
}

// 16 bytes per lane from a buffer straight into LDS at M0 + 16 lane, M0 =
// lds + LOFF (the dQ pass's K/V staging).  The M0 write needs one wait state
// before the load; s_add_u32 also writes SCC, so both are declared clobbered.
template <int LOFF>
__device__ __forceinline__ void bwd_lds_dma16(__amdgpu_buffer_rsrc_t r, int off, unsigned lds) {
    asm volatile("s_add_u32 m0, %1, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds" ::"v"(off), "s"(lds),
                 "s"(r), "n"(LOFF)
                 : "memory", "scc", "m0");
}

// ---------------------------------------------------------------------------
// pass 1: dQ (and the row vectors D_n, log2-sum-exp)
// ---------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(bwd_waves_dq<D>() * 64, 1) void attn_bwd_dq_kernel(BwdParams p) {
    using E = Elt16<T>;
    using frag = typename E::frag;
    using TL = BwdTile<T, D, bwd_waves_dq<D>()>;
    constexpr int BN = TL::BN, CPR = TL::CPR, LOADS = TL::LOADS;
    constexpr int kBwdThreads = TL::THREADS, kBwdRows = TL::ROWS;
    constexpr bool PARTIAL = TL::PARTIAL;
    constexpr int NDB = D / 32, NDK = D / 16;

    // The software-pipelined loop (head_dim 128, one wave per SIMD) keeps three
    // tiles in LDS, the plain loop two.
    constexpr bool PIPE = D >= 128;
    __shared__ __attribute__((aligned(16))) T smem[PIPE ? 3 : 2][3][BN * D];   // [stage][K swz_k, K swz_v, V swz_k]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = lane >> 5;
    const int col = lane & 31;

    // Longest query tiles first (causal).
    const int bh = blockIdx.x % p.BH;
    const int qt = CAUSAL ? p.n_qtiles - 1 - (int)blockIdx.x / p.BH : (int)blockIdx.x / p.BH;
    const int S = p.S;
    const T *qg = bwd_head<const T>(p, p.q, BQ, bh);
    const T *kg = bwd_head<const T>(p, p.k, BK, bh);
    const T *vg = bwd_head<const T>(p, p.v, BV, bh);
    const T *dog = bwd_head<const T>(p, p.dout, BDOUT, bh);
    T *dqg = bwd_head<T>(p, p.dq, BDQ, bh);
    const int qss = p.ss[BQ], kss = p.ss[BK], vss = p.ss[BV], doss = p.ss[BDOUT];

    const int q0 = qt * kBwdRows;
    const int q0w = q0 + 32 * wave;
    const int qi = q0w + col;                 // this lane's query row
    const int qrow = min(qi, S - 1);
    const int last_key = CAUSAL ? min(q0 + kBwdRows - 1, S - 1) : S - 1;
    const int nt = last_key / BN + 1;
    const bool wave_active = q0w < S;

    // B-operand fragments of the owned rows: Q (for S^T = K Q^T) and dout
    // (for dP^T = V dout^T); lane holds row qi, head_dim 16 dk + 8 hi .. +7.
    frag qf[NDK], df[NDK];
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) {
        qf[dk] = __builtin_bit_cast(frag, *(const u32x4_t *)(qg + (int64_t)qrow * qss + 16 * dk + 8 * hi));
        df[dk] = __builtin_bit_cast(frag, *(const u32x4_t *)(dog + (int64_t)qrow * doss + 16 * dk + 8 * hi));
    }
    // log2-sum-exp of the row: P = exp2(s * scale * log2(e) - lse2).
    const float m_i = bwd_load_ml<T>(p.m, (int64_t)bh * S + qrow, p.ml_f32 != 0);
    const float l_i = bwd_load_ml<T>(p.l, (int64_t)bh * S + qrow, p.ml_f32 != 0);
    const float lse2 = m_i * 1.4426950408889634f + __log2f(l_i);
    const float c = p.scale_log2;

    // ---- staging of the pipelined loop by LDS DMA: tile kt lands in stage
    // kt % 3, 16 bytes per lane straight from memory.  Lane `lane` of wave
    // `wave` fills chunk slot j*THREADS + 64*wave + lane of each layout (LDS
    // bytes layout_base + 16 THREADS j + 1024 wave + 16 lane) with the logical
    // chunk that the layout's XOR swizzle places there. ----
    constexpr int TILE_BYTES = BN * D * (int)sizeof(T);
    int doffk[LOADS], doffkt[LOADS], doffv[LOADS];   // K rows, K transposed layout, V rows
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const int sl = j * kBwdThreads + tid;
        const int row = sl / CPR, pp = sl % CPR;
        doffk[j] = (row * kss + 8 * (pp ^ swz_k<CPR>(row))) * (int)sizeof(T);
        doffkt[j] = (row * kss + 8 * (pp ^ swz_v<CPR>(row))) * (int)sizeof(T);
        doffv[j] = (row * vss + 8 * (pp ^ swz_k<CPR>(row))) * (int)sizeof(T);
    }
    const unsigned lds_w = (unsigned)(uintptr_t)(__attribute__((address_space(3))) T *)&smem[0][0][0] + 1024u * wave;
    // All DMAs of tile kt into stage kt % 3 (rows past S read as zero).
    auto dma_tile = [&](int kt) __attribute__((always_inline)) {
        static_assert(!PIPE || !PARTIAL, "the DMA staging covers whole tiles");
        const auto kr = bwd_rows_rsrc<T, D>(kg, kt * BN, S, kss);
        const auto vr = bwd_rows_rsrc<T, D>(vg, kt * BN, S, vss);
        const unsigned base = lds_w + (unsigned)((kt % 3) * 3 * TILE_BYTES);
        bwd_static_for<0, LOADS>([&](auto j_c) __attribute__((always_inline)) {
            constexpr int J = decltype(j_c)::value;
            bwd_lds_dma16<0 * TILE_BYTES + 16 * kBwdThreads * J>(kr, doffk[J], base);
            bwd_lds_dma16<1 * TILE_BYTES + 16 * kBwdThreads * J>(kr, doffkt[J], base);
            bwd_lds_dma16<2 * TILE_BYTES + 16 * kBwdThreads * J>(vr, doffv[J], base);
        });
    };
    // The DMAs are inline asm: their completion is waited for explicitly,
    // before the barrier after which the tile is read.
    auto dma_wait_sync = [&]() __attribute__((always_inline)) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    };

    // ---- staging of the plain loop: two register sets, two LDS stages ----
    int goffk[LOADS], goffv[LOADS];   // lane byte offsets of its chunks in a K / V tile
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const int sl = j * kBwdThreads + tid;
        goffk[j] = ((sl / CPR) * kss + 8 * (sl % CPR)) * (int)sizeof(T);
        goffv[j] = ((sl / CPR) * vss + 8 * (sl % CPR)) * (int)sizeof(T);
    }
    u32x4_t kreg2[2][LOADS], vreg2[2][LOADS];
    auto gload2 = [&](int kt, auto set_c) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value;
        const auto kr = bwd_rows_rsrc<T, D>(kg, kt * BN, S, kss);
        const auto vr = bwd_rows_rsrc<T, D>(vg, kt * BN, S, vss);
#pragma unroll
        for (int j = 0; j < LOADS; ++j)
            if (!PARTIAL || j * kBwdThreads + tid < TL::CHUNKS) {
                kreg2[SET][j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(kr, goffk[j], 0, 0));
                vreg2[SET][j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(vr, goffv[j], 0, 0));
            }
    };
    auto swrite2 = [&](int st, auto set_c) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value;
#pragma unroll
        for (int j = 0; j < LOADS; ++j) {
            const int sl = j * kBwdThreads + tid;
            if (!PARTIAL || sl < TL::CHUNKS) {
                const int row = sl / CPR, pc = sl % CPR;
                *(u32x4_t *)(&smem[st][0][row * D + 8 * (pc ^ swz_k<CPR>(row))]) = kreg2[SET][j];
                *(u32x4_t *)(&smem[st][1][row * D + 8 * (pc ^ swz_v<CPR>(row))]) = kreg2[SET][j];
                *(u32x4_t *)(&smem[st][2][row * D + 8 * (pc ^ swz_k<CPR>(row))]) = vreg2[SET][j];
            }
        }
    };

    const int arow = key_of_arow(col);
    const int g16 = lane >> 4, tt = lane & 15;
    const int vrow0 = 16 * (g16 >> 1) + (tt >> 2);
    const int vcol0 = 16 * (g16 & 1) + 4 * (tt & 3);

    float drow_part = 0.f;      // pass A: per-lane part of D_n
    float drow = 0.f;
    f32x16_t acc[NDB];          // dQ^T (head_dim x owned rows)
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;

    // Scores S^T and dP^T of a tile: MFMA m (0 .. NSD-1) is (dk, kb, which)
    // = (m / 4, (m / 2) % 2, m % 2), i.e. four interleaved accumulator chains.
    constexpr int NSD = 4 * NDK;
    auto sd_frag = [&](int st, int m) __attribute__((always_inline)) {
        const int dk = m >> 2, kb = (m >> 1) & 1, which = m & 1;
        return bwd_row_frag<T, D>(smem[st][which ? 2 : 0], kb, dk, arow, hi);
    };
    auto sd_mma = [&](f32x16_t (&sv)[2], f32x16_t (&dpv)[2], int m, frag a) __attribute__((always_inline)) {
        const int dk = m >> 2, kb = (m >> 1) & 1, which = m & 1;
        if (which) dpv[kb] = E::mma(a, df[dk], dk == 0 ? f32x16_t{} : dpv[kb]);
        else sv[kb] = E::mma(a, qf[dk], dk == 0 ? f32x16_t{} : sv[kb]);
    };
    // All scores of tile (stage st), fragments read one MFMA ahead.
    auto sd_tile = [&](f32x16_t (&sv)[2], f32x16_t (&dpv)[2], int st) __attribute__((always_inline)) {
        frag a = sd_frag(st, 0);
#pragma unroll
        for (int m = 0; m < NSD; ++m) {
            const frag b = m + 1 < NSD ? sd_frag(st, m + 1) : a;
            sd_mma(sv, dpv, m, a);
            a = b;
        }
    };

    // One loop over the key tiles.  PASS 0: D_n; PASS 1: dS and dQ.  Software
    // pipelined by one tile: step kt starts the DMAs of tile kt+2, issues the
    // S^T, dP^T MFMAs of tile kt+1 one by one, each followed by a share of
    // tile kt's softmax VALU (P, dS), then the dQ MFMAs of tile kt, all MFMA
    // fragments read RING MFMAs ahead through one ring.  One barrier per
    // tile, after the wait for the DMAs.
    constexpr int RING = 4;
    constexpr int NUNIT = 16;   // softmax units of a tile: (kb, register pair)
    auto key_loop = [&](auto pass_c) __attribute__((always_inline)) {
        constexpr int PASS = decltype(pass_c)::value;
        dma_tile(0);
        if (nt > 1) dma_tile(1);
        dma_wait_sync();
        f32x16_t s0[2], dp0[2], s1[2], dp1[2];
        if (wave_active) sd_tile(s0, dp0, 0);

        auto step = [&](int kt, f32x16_t (&sc)[2], f32x16_t (&dpc)[2], f32x16_t (&sn)[2], f32x16_t (&dpn)[2])
                        __attribute__((always_inline)) {
            const int st = kt % 3, st1 = (kt + 1) % 3;
            // tile kt+2 into the stage of tile kt-1, which every wave finished
            // reading before the last barrier
            if (kt + 2 < nt) dma_tile(kt + 2);
            const int kbase = kt * BN;
            const bool wave_needed = wave_active && (!CAUSAL || kbase <= q0w + 31);
            // Two copies of the tile's work, with and without the mask (a
            // wave masks only its last tile, and the one past S): written
            // per score, the mask's compare and select cost ~130 scalar and
            // vector instructions on every tile.
            const bool need_mask = (CAUSAL && kbase + BN - 1 > q0w) || (kbase + BN > S);
            auto work = [&](auto mask_c) __attribute__((always_inline)) {
                constexpr bool MASK = decltype(mask_c)::value;
                const int lim = CAUSAL ? min(qi, S - 1) : S - 1;
                uint32_t dsk[2][8];
                // One stream of fragments through the ring: the S^T, dP^T
                // row fragments of tile kt+1, then (dQ pass) the transposed K
                // fragments of tile kt, so the first dQ MFMAs find theirs read.
                const T *Kv = smem[st][1];
                constexpr int NQ = PASS == 1 ? 4 * NDB : 0;
                static_assert(NSD % RING == 0, "the dQ MFMAs continue the ring");
                // dQ MFMA m is (kb, cc, db) = (m / (2 NDB), (m / NDB) % 2, m % NDB)
                auto kt_frag = [&](int m) __attribute__((always_inline)) {
                    return bwd_tr_frag<T, D>(Kv, m / (2 * NDB), (m / NDB) & 1, m % NDB, vrow0, vcol0);
                };
                auto next_frag = [&](int n) __attribute__((always_inline)) {
                    return n < NSD ? sd_frag(st1, n) : kt_frag(n - NSD);
                };
                frag ring[RING];
#pragma unroll
                for (int i = 0; i < RING; ++i) ring[i] = sd_frag(st1, i);
                // Softmax unit u of tile kt (registers 2u, 2u+1 of block u / 8)
                // in two halves, one behind each MFMA: the exponentials behind
                // MFMA 2u, the products behind MFMA 2u+1, so no two MFMAs issue
                // back to back and the exponentials' latency passes under an
                // MFMA.
                static_assert(2 * NUNIT == NSD, "one half-unit per MFMA");
                float pv[2];
#pragma unroll
                for (int m = 0; m < NSD; ++m) {
                    __builtin_amdgcn_sched_barrier(0);
                    sd_mma(sn, dpn, m, ring[m % RING]);
                    if (m + RING < NSD + NQ) ring[m % RING] = next_frag(m + RING);
                    const int u = m >> 1, kb = u >> 3, r = 2 * (u & 7);
                    if ((m & 1) == 0) {
#pragma unroll
                        for (int e = 0; e < 2; ++e) {
                            const int key = kbase + 32 * kb + 16 * hi + r + e;
                            const float sv = MASK && key > lim ? -INFINITY : sc[kb][r + e];
                            pv[e] = fast_exp2(__builtin_fmaf(sv, c, -lse2));
                        }
                    } else if (PASS == 0) {
                        drow_part = __builtin_fmaf(pv[0], dpc[kb][r], drow_part);
                        drow_part = __builtin_fmaf(pv[1], dpc[kb][r + 1], drow_part);
                    } else {
                        dsk[kb][r >> 1] = E::pack2(pv[0] * (dpc[kb][r] - drow), pv[1] * (dpc[kb][r + 1] - drow));
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                if (PASS == 1) {
                    // dQ^T += K^T dS^T over the 4 blocks of 16 keys, the
                    // transposed K fragments continuing the ring
#pragma unroll
                    for (int m = 0; m < NQ; ++m) {
                        __builtin_amdgcn_sched_barrier(0);
                        const int kb = m / (2 * NDB), cc = (m / NDB) & 1, db = m % NDB;
                        const u32x4_t bw = {dsk[kb][4 * cc], dsk[kb][4 * cc + 1], dsk[kb][4 * cc + 2], dsk[kb][4 * cc + 3]};
                        acc[db] = E::mma(ring[m % RING], __builtin_bit_cast(frag, bw), acc[db]);
                        if (m + RING < NQ) ring[m % RING] = kt_frag(m + RING);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            };
            if (wave_needed) {
                if (need_mask) work(std::true_type{});
                else work(std::false_type{});
            }
            dma_wait_sync();
        };
        for (int kt = 0; kt < nt; kt += 2) {
            step(kt, s0, dp0, s1, dp1);
            if (kt + 1 < nt) step(kt + 1, s1, dp1, s0, dp0);
        }
    };

    // The plain loop (head_dim < 128, two waves per SIMD): per tile S^T and
    // dP^T, then P / dS, then dQ, the other wave of the SIMD overlapping.
    auto key_loop_plain = [&](auto pass_c) __attribute__((always_inline)) {
        constexpr int PASS = decltype(pass_c)::value;
        gload2(0, std::integral_constant<int, 0>{});
        swrite2(0, std::integral_constant<int, 0>{});
        __builtin_amdgcn_s_waitcnt(0);
        gload2(min(1, nt - 1), std::integral_constant<int, 1>{});
        __syncthreads();
        auto tile_step = [&](auto set_c, int kt) __attribute__((always_inline)) {
            constexpr int SET = decltype(set_c)::value;
            gload2(min(kt + 2, nt - 1), set_c);
            const int kbase = kt * BN;
            const bool wave_needed = wave_active && (!CAUSAL || kbase <= q0w + 31);
            // masked and unmasked copies, as in the pipelined loop
            const bool need_mask = (CAUSAL && kbase + BN - 1 > q0w) || (kbase + BN > S);
            auto work = [&](auto mask_c) __attribute__((always_inline)) {
                constexpr bool MASK = decltype(mask_c)::value;
                const T *Kk = smem[SET][0];
                const T *Kv = smem[SET][1];
                const T *Vk = smem[SET][2];
                f32x16_t s[2], dp[2];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[kb][r] = dp[kb][r] = 0.f;
#pragma unroll
                    for (int dk = 0; dk < NDK; ++dk) {
                        s[kb] = E::mma(bwd_row_frag<T, D>(Kk, kb, dk, arow, hi), qf[dk], s[kb]);
                        dp[kb] = E::mma(bwd_row_frag<T, D>(Vk, kb, dk, arow, hi), df[dk], dp[kb]);
                    }
                }
                // register r of block kb holds key kbase + 32 kb + 16 hi + r
                const int lim = CAUSAL ? min(qi, S - 1) : S - 1;
                uint32_t dsk[2][8];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; r += 2) {
                        float pv[2];
#pragma unroll
                        for (int e = 0; e < 2; ++e) {
                            const int key = kbase + 32 * kb + 16 * hi + r + e;
                            const float sv = MASK && key > lim ? -INFINITY : s[kb][r + e];
                            pv[e] = fast_exp2(__builtin_fmaf(sv, c, -lse2));
                        }
                        if (PASS == 0) {
                            drow_part = __builtin_fmaf(pv[0], dp[kb][r], drow_part);
                            drow_part = __builtin_fmaf(pv[1], dp[kb][r + 1], drow_part);
                        } else {
                            dsk[kb][r >> 1] = E::pack2(pv[0] * (dp[kb][r] - drow), pv[1] * (dp[kb][r + 1] - drow));
                        }
                    }
                if (PASS == 1) {
                    // dQ^T += K^T dS^T over the 4 blocks of 16 keys
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                        for (int cc = 0; cc < 2; ++cc) {
                            u32x4_t bw = {dsk[kb][4 * cc], dsk[kb][4 * cc + 1], dsk[kb][4 * cc + 2], dsk[kb][4 * cc + 3]};
                            const frag bfr = __builtin_bit_cast(frag, bw);
#pragma unroll
                            for (int db = 0; db < NDB; ++db)
                                acc[db] = E::mma(bwd_tr_frag<T, D>(Kv, kb, cc, db, vrow0, vcol0), bfr, acc[db]);
                        }
                }
            };
            if (wave_needed) {
                if (need_mask) work(std::true_type{});
                else work(std::false_type{});
            }
            if (kt + 1 < nt) swrite2(SET ^ 1, std::integral_constant<int, SET ^ 1>{});
            __syncthreads();
        };
        for (int kt = 0; kt < nt; kt += 2) {
            tile_step(std::integral_constant<int, 0>{}, kt);
            if (kt + 1 < nt) tile_step(std::integral_constant<int, 1>{}, kt + 1);
        }
    };

    if (p.o != nullptr) {
        // D_n = dout_n . o_n straight from O (same lane split as the fragments)
        const T *og = bwd_head<const T>(p, p.o, BO, bh);
        float part = 0.f;
#pragma unroll
        for (int dk = 0; dk < NDK; ++dk) {
            const frag of = __builtin_bit_cast(frag, *(const u32x4_t *)(og + (int64_t)qrow * p.ss[BO] + 16 * dk + 8 * hi));
#pragma unroll
            for (int e = 0; e < 8; ++e) part = __builtin_fmaf((float)of[e], (float)df[dk][e], part);
        }
        drow = half_sum(part);
    } else {
        if constexpr (PIPE) key_loop(std::integral_constant<int, 0>{});
        else key_loop_plain(std::integral_constant<int, 0>{});
        drow = half_sum(drow_part);
    }
    if (hi == 0 && qi < S) {
        p.lse2[(int64_t)bh * S + qi] = lse2;
        p.drow[(int64_t)bh * S + qi] = drow;
    }
    if constexpr (PIPE) key_loop(std::integral_constant<int, 1>{});
    else key_loop_plain(std::integral_constant<int, 1>{});

    // ---- epilogue: dq = scale * dQ^T, lane = query column ----
    if (wave_active && qi < S) {
        T *row = dqg + (int64_t)qi * p.ss[BDQ];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d = 32 * db + 8 * g4 + 4 * hi;
                u32x2_t w2 = {E::pack2(acc[db][4 * g4] * p.scale, acc[db][4 * g4 + 1] * p.scale),
                              E::pack2(acc[db][4 * g4 + 2] * p.scale, acc[db][4 * g4 + 3] * p.scale)};
                *(u32x2_t *)(row + d) = w2;
            }
    }
}

// ---------------------------------------------------------------------------
// pass 2: dK, dV
// ---------------------------------------------------------------------------
// f(integral_constant<int, I>) for I = B .. E-1, unrolled at compile time.
template <int B, int E, typename F>
__device__ __forceinline__ void bwd_static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        bwd_static_for<B + 1, E>(f);
    }
}

// Causal mask of a dK/dV tile as one threshold per lane: query
// qbase + 32 qb + 16 hi + r is visible to the lane's key kj iff
// 32 qb + r >= kj - qbase - 16 hi, one compare against a constant per score.
// Tiles wholly at or past the wave's last key get a threshold every register
// passes.  Queries past S need no mask: their lse2 is +inf and their Q and
// dout rows read as zero, so P = exp2(0 * c - inf) = 0 and dS = 0 exactly.
template <bool CAUSAL>
__device__ __forceinline__ int bwd_dkdv_mlim(int qbase, int k0w, int kj, int hi) {
    return CAUSAL && qbase < k0w + 31 ? kj - qbase - 16 * hi : -64;
}

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(bwd_waves_dkdv<D>() * 64, 1) void attn_bwd_dkdv_kernel(BwdParams p) {
    using E = Elt16<T>;
    using frag = typename E::frag;
    using TL = BwdTile<T, D, bwd_waves_dkdv<D>()>;
    constexpr int BN = TL::BN, CPR = TL::CPR, LOADS = TL::LOADS;
    constexpr int kBwdThreads = TL::THREADS, kBwdRows = TL::ROWS;
    constexpr bool PARTIAL = TL::PARTIAL;
    constexpr int NDB = D / 32, NDK = D / 16;

    // [stage][Q swz_k, Q swz_v, dout swz_k, dout swz_v]; row vectors [stage][lse2, D_n]
    __shared__ __attribute__((aligned(16))) T smem[2][4][BN * D];
    __shared__ __attribute__((aligned(16))) float svec[2][2][BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = lane >> 5;
    const int col = lane & 31;

    // Key tiles with the most queries first (causal: the first keys).
    const int bh = blockIdx.x % p.BH;
    const int ktile = (int)blockIdx.x / p.BH;
    const int S = p.S;
    const T *qg = bwd_head<const T>(p, p.q, BQ, bh);
    const T *kg = bwd_head<const T>(p, p.k, BK, bh);
    const T *vg = bwd_head<const T>(p, p.v, BV, bh);
    const T *dog = bwd_head<const T>(p, p.dout, BDOUT, bh);
    const float *lse2g = p.lse2 + (int64_t)bh * S;
    const float *drowg = p.drow + (int64_t)bh * S;
    T *dkg = bwd_head<T>(p, p.dk, BDK, bh);
    T *dvg = bwd_head<T>(p, p.dv, BDV, bh);
    const int qss = p.ss[BQ], doss = p.ss[BDOUT];

    const int k0 = ktile * kBwdRows;
    const int k0w = k0 + 32 * wave;
    const int kj = k0w + col;                 // this lane's key row
    const int krow = min(kj, S - 1);
    const bool wave_active = k0w < S;
    const int t0 = CAUSAL ? k0 / BN : 0;      // first query tile with a visible query
    const int nq = (S + BN - 1) / BN;

    // B-operand fragments of the owned rows: K (for S = Q K^T) and V (for
    // dP = dout V^T); lane holds row kj, head_dim 16 dk + 8 hi .. +7.
    frag kf[NDK], vf[NDK];
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) {
        kf[dk] = __builtin_bit_cast(frag, *(const u32x4_t *)(kg + (int64_t)krow * p.ss[BK] + 16 * dk + 8 * hi));
        vf[dk] = __builtin_bit_cast(frag, *(const u32x4_t *)(vg + (int64_t)krow * p.ss[BV] + 16 * dk + 8 * hi));
    }
    const float c = p.scale_log2;

    // ---- staging of Q, dout (two layouts each) and the row vectors ----
    u32x4_t qreg[LOADS], oreg[LOADS];
    float vreg;      // one row-vector element per thread (threads 0..127)
    int goffq[LOADS], goffo[LOADS];   // lane byte offsets of its chunks in a Q / dout tile
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const int sl = j * kBwdThreads + tid;
        goffq[j] = ((sl / CPR) * qss + 8 * (sl % CPR)) * (int)sizeof(T);
        goffo[j] = ((sl / CPR) * doss + 8 * (sl % CPR)) * (int)sizeof(T);
    }
    auto gload = [&](int qtl) __attribute__((always_inline)) {
        const auto qr = bwd_rows_rsrc<T, D>(qg, qtl * BN, S, qss);
        const auto orr = bwd_rows_rsrc<T, D>(dog, qtl * BN, S, doss);
#pragma unroll
        for (int j = 0; j < LOADS; ++j)
            if (!PARTIAL || j * kBwdThreads + tid < TL::CHUNKS) {
                qreg[j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(qr, goffq[j], 0, 0));
                oreg[j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(orr, goffo[j], 0, 0));
            }
        if (tid < 2 * BN) {
            const int row = qtl * BN + (tid & (BN - 1));
            // rows past S: lse2 = +inf gives P = 0 (their scores are masked too)
            vreg = row < S ? ((tid < BN) ? lse2g[row] : drowg[row]) : ((tid < BN) ? INFINITY : 0.f);
        }
    };
    auto swrite = [&](int st) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < LOADS; ++j) {
            const int sl = j * kBwdThreads + tid;
            if (!PARTIAL || sl < TL::CHUNKS) {
                const int row = sl / CPR, pc = sl % CPR;
                *(u32x4_t *)(&smem[st][0][row * D + 8 * (pc ^ swz_k<CPR>(row))]) = qreg[j];
                *(u32x4_t *)(&smem[st][1][row * D + 8 * (pc ^ swz_v<CPR>(row))]) = qreg[j];
                *(u32x4_t *)(&smem[st][2][row * D + 8 * (pc ^ swz_k<CPR>(row))]) = oreg[j];
                *(u32x4_t *)(&smem[st][3][row * D + 8 * (pc ^ swz_v<CPR>(row))]) = oreg[j];
            }
        }
        if (tid < 2 * BN) svec[st][tid >> 6][tid & (BN - 1)] = vreg;
    };

    const int arow = key_of_arow(col);
    const int g16 = lane >> 4, tt = lane & 15;
    const int vrow0 = 16 * (g16 >> 1) + (tt >> 2);
    const int vcol0 = 16 * (g16 & 1) + 4 * (tt & 3);

    f32x16_t dk_acc[NDB], dv_acc[NDB];   // dK^T, dV^T (head_dim x owned keys)
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) dk_acc[db][r] = dv_acc[db][r] = 0.f;

    const int ntl = nq - t0;   // query tiles of the workgroup
    if (ntl > 0) {
        gload(t0);
        swrite(0);
        __builtin_amdgcn_s_waitcnt(0);
        gload(min(t0 + 1, nq - 1));
        __syncthreads();
    }
    auto tile_step = [&](auto set_c, int it) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value;
        const int qtl = t0 + it;
        // Tile it+1 goes from registers to the LDS stage that tile it-1 used
        // (free since the barrier that ended tile it-1), then tile it+2 is
        // loaded into the same registers: one register set, a tile of latency.
        if (it + 1 < ntl) swrite(SET ^ 1);
        gload(min(qtl + 2, nq - 1));
        const int qbase = qtl * BN;
        // causal: the tile holds a query at or past the wave's first key
        const bool wave_needed = wave_active && (!CAUSAL || qbase + BN - 1 >= k0w);
        if (wave_needed) {
            const T *Qk = smem[SET][0];
            const T *Qv = smem[SET][1];
            const T *Ok = smem[SET][2];
            const T *Ov = smem[SET][3];
            const float *lse2s = svec[SET][0];
            const float *drows = svec[SET][1];
            if constexpr (D >= 128) {
                // Half-tile pipeline over the two 32-query blocks qb: one stream of
                // NMM MFMAs in four phases,
                //   0  S, dP of block 0
                //   1  S, dP of block 1        + P, dS of block 0 behind the MFMAs
                //   2  dV^T, dK^T of block 0   + P, dS of block 1 behind the MFMAs
                //   3  dV^T, dK^T of block 1
                // so the softmax VALU of one block runs under the other block's
                // MFMAs.  S, dP MFMA j of a block is (dk, which) = (j / 2, j % 2);
                // dV^T, dK^T MFMA j is (cc, db, which) = (j / (2 NDB),
                // (j / 2) % NDB, j % 2).  Fragments are read RING MFMAs ahead.
                constexpr int RING = 2, NSQ = 2 * NDK, NGQ = 4 * NDB, NMM = 2 * (NSQ + NGQ);
                auto frag_at = [&](int n) __attribute__((always_inline)) {
                    if (n < 2 * NSQ) {
                        const int qb = n / NSQ, j = n % NSQ;
                        return bwd_row_frag<T, D>((j & 1) ? Ok : Qk, qb, j >> 1, arow, hi);
                    }
                    const int m = n - 2 * NSQ, qb = m / NGQ, j = m % NGQ;
                    return bwd_tr_frag<T, D>((j & 1) ? Qv : Ov, qb, j / (2 * NDB), (j >> 1) % NDB, vrow0, vcol0);
                };
                // register r of block qb holds query qbase + 32 qb + 16 hi + r;
                // the causal mask keeps it iff 32 qb + r >= mlim (bwd_dkdv_mlim)
                const int mlim = bwd_dkdv_mlim<CAUSAL>(qbase, k0w, kj, hi);
                f32x16_t s[2], dp[2];
                uint32_t pp[2][8], dsp[2][8];
                f32x4_t l4[2][4], d4[2][4];
                auto load_vec = [&](int qb) __attribute__((always_inline)) {
                    const int rb = 32 * qb + 16 * hi;
    #pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        l4[qb][i] = *(const f32x4_t *)(lse2s + rb + 4 * i);
                        d4[qb][i] = *(const f32x4_t *)(drows + rb + 4 * i);
                    }
                };
                // P and dS of registers 2u, 2u + 1 of block qb
                auto unit = [&](int qb, int u) __attribute__((always_inline)) {
                    const int r = 2 * u;
                    float pv[2], dsv[2];
    #pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const float sv = !CAUSAL || 32 * qb + r + e >= mlim ? s[qb][r + e] : -INFINITY;
                        pv[e] = fast_exp2(__builtin_fmaf(sv, c, -l4[qb][(r + e) >> 2][(r + e) & 3]));
                        dsv[e] = pv[e] * (dp[qb][r + e] - d4[qb][(r + e) >> 2][(r + e) & 3]);
                    }
                    pp[qb][u] = E::pack2(pv[0], pv[1]);
                    dsp[qb][u] = E::pack2(dsv[0], dsv[1]);
                };
                auto mma_at = [&](int n, frag a) __attribute__((always_inline)) {
                    if (n < 2 * NSQ) {
                        const int qb = n / NSQ, j = n % NSQ, dk = j >> 1;
                        if (j & 1) dp[qb] = E::mma(a, vf[dk], dk == 0 ? f32x16_t{} : dp[qb]);
                        else s[qb] = E::mma(a, kf[dk], dk == 0 ? f32x16_t{} : s[qb]);
                    } else {
                        const int m = n - 2 * NSQ, qb = m / NGQ, j = m % NGQ;
                        const int db = (j >> 1) % NDB, cc = j / (2 * NDB);
                        if (j & 1) {
                            const u32x4_t bs = {dsp[qb][4 * cc], dsp[qb][4 * cc + 1], dsp[qb][4 * cc + 2], dsp[qb][4 * cc + 3]};
                            dk_acc[db] = E::mma(a, __builtin_bit_cast(frag, bs), dk_acc[db]);
                        } else {
                            const u32x4_t bp = {pp[qb][4 * cc], pp[qb][4 * cc + 1], pp[qb][4 * cc + 2], pp[qb][4 * cc + 3]};
                            dv_acc[db] = E::mma(a, __builtin_bit_cast(frag, bp), dv_acc[db]);
                        }
                    }
                };
                frag ring[RING];
    #pragma unroll
                for (int i = 0; i < RING; ++i) ring[i] = frag_at(i);
                // a block's row vectors are read from LDS a few MFMAs before its
                // first softmax unit
                constexpr int VLEAD = NSQ < 4 ? NSQ : 4;
                bwd_static_for<0, NMM>([&](auto n_c) __attribute__((always_inline)) {
                    constexpr int n = decltype(n_c)::value;
                    __builtin_amdgcn_sched_barrier(0);
                    if constexpr (n == NSQ - VLEAD) load_vec(0);
                    if constexpr (n == 2 * NSQ - VLEAD) load_vec(1);
                    mma_at(n, ring[n % RING]);
                    if constexpr (n + RING < NMM) ring[n % RING] = frag_at(n + RING);
                    // phase 1 carries block 0's units, phase 2 block 1's
                    constexpr int ph = n < NSQ ? 0 : n < 2 * NSQ ? 1 : n < 2 * NSQ + NGQ ? 2 : 3;
                    if constexpr (ph == 1 || ph == 2) {
                        constexpr int len = ph == 1 ? NSQ : NGQ, k = n - (ph == 1 ? NSQ : 2 * NSQ);
    #pragma unroll
                        for (int u = (k * 8) / len; u < ((k + 1) * 8) / len; ++u) unit(ph - 1, u);
                    }
                });
                __builtin_amdgcn_sched_barrier(0);
            } else {
                // Plain tile (the half-tile pipeline spills at 8 waves):
                // S = Q K^T, dP = dout V^T: MFMA m is (dk, qb, which) = (m / 4,
                // (m / 2) % 2, m % 2), four interleaved chains, row fragments read
                // RING MFMAs ahead
                constexpr int RING = 2, NSD = 4 * NDK;
                auto sd_frag = [&](int m) __attribute__((always_inline)) {
                    return bwd_row_frag<T, D>((m & 1) ? Ok : Qk, (m >> 1) & 1, m >> 2, arow, hi);
                };
                f32x16_t s[2], dp[2];
                {
                    frag ring[RING];
    #pragma unroll
                    for (int i = 0; i < RING; ++i) ring[i] = sd_frag(i);
    #pragma unroll
                    for (int m = 0; m < NSD; ++m) {
                        const int dk = m >> 2, qb = (m >> 1) & 1;
                        if (m & 1) dp[qb] = E::mma(ring[m % RING], vf[dk], dk == 0 ? f32x16_t{} : dp[qb]);
                        else s[qb] = E::mma(ring[m % RING], kf[dk], dk == 0 ? f32x16_t{} : s[qb]);
                        if (m + RING < NSD) ring[m % RING] = sd_frag(m + RING);
                    }
                }
                // register r of block qb holds query qbase + 32 qb + 16 hi + r;
                // the causal mask keeps it iff 32 qb + r >= mlim (bwd_dkdv_mlim)
                const int mlim = bwd_dkdv_mlim<CAUSAL>(qbase, k0w, kj, hi);
                uint32_t pp[2][8], dsp[2][8];
    #pragma unroll
                for (int qb = 0; qb < 2; ++qb) {
                    const int rb = 32 * qb + 16 * hi;
                    f32x4_t l4[4], d4[4];
    #pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        l4[i] = *(const f32x4_t *)(lse2s + rb + 4 * i);
                        d4[i] = *(const f32x4_t *)(drows + rb + 4 * i);
                    }
    #pragma unroll
                    for (int r = 0; r < 16; r += 2) {
                        float pv[2], dsv[2];
    #pragma unroll
                        for (int e = 0; e < 2; ++e) {
                            const float sv = !CAUSAL || 32 * qb + r + e >= mlim ? s[qb][r + e] : -INFINITY;
                            pv[e] = fast_exp2(__builtin_fmaf(sv, c, -l4[(r + e) >> 2][(r + e) & 3]));
                            dsv[e] = pv[e] * (dp[qb][r + e] - d4[(r + e) >> 2][(r + e) & 3]);
                        }
                        pp[qb][r >> 1] = E::pack2(pv[0], pv[1]);
                        dsp[qb][r >> 1] = E::pack2(dsv[0], dsv[1]);
                    }
                }
                // dV^T += dout^T P,  dK^T += Q^T dS over the 4 blocks of 16 queries:
                // MFMA m is (qb, cc, db, which), transposed fragments read RING
                // MFMAs ahead
                constexpr int NGR = 8 * NDB;
                auto gr_frag = [&](int m) __attribute__((always_inline)) {
                    const int db = (m >> 1) % NDB, cc = (m / (2 * NDB)) & 1, qb = m / (4 * NDB);
                    return bwd_tr_frag<T, D>((m & 1) ? Qv : Ov, qb, cc, db, vrow0, vcol0);
                };
                {
                    frag ring[RING];
    #pragma unroll
                    for (int i = 0; i < RING; ++i) ring[i] = gr_frag(i);
    #pragma unroll
                    for (int m = 0; m < NGR; ++m) {
                        const int db = (m >> 1) % NDB, cc = (m / (2 * NDB)) & 1, qb = m / (4 * NDB);
                        if (m & 1) {
                            const u32x4_t bs = {dsp[qb][4 * cc], dsp[qb][4 * cc + 1], dsp[qb][4 * cc + 2], dsp[qb][4 * cc + 3]};
                            dk_acc[db] = E::mma(ring[m % RING], __builtin_bit_cast(frag, bs), dk_acc[db]);
                        } else {
                            const u32x4_t bp = {pp[qb][4 * cc], pp[qb][4 * cc + 1], pp[qb][4 * cc + 2], pp[qb][4 * cc + 3]};
                            dv_acc[db] = E::mma(ring[m % RING], __builtin_bit_cast(frag, bp), dv_acc[db]);
                        }
                        if (m + RING < NGR) ring[m % RING] = gr_frag(m + RING);
                    }
                }
            }
        }
        __syncthreads();
    };
    for (int it = 0; it < ntl; it += 2) {
        tile_step(std::integral_constant<int, 0>{}, it);
        if (it + 1 < ntl) tile_step(std::integral_constant<int, 1>{}, it + 1);
    }

    // ---- epilogue: dk = scale * dK^T, dv = dV^T; lane = key column ----
    if (wave_active && kj < S) {
        T *rk = dkg + (int64_t)kj * p.ss[BDK];
        T *rv = dvg + (int64_t)kj * p.ss[BDV];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d = 32 * db + 8 * g4 + 4 * hi;
                u32x2_t wk = {E::pack2(dk_acc[db][4 * g4] * p.scale, dk_acc[db][4 * g4 + 1] * p.scale),
                              E::pack2(dk_acc[db][4 * g4 + 2] * p.scale, dk_acc[db][4 * g4 + 3] * p.scale)};
                u32x2_t wv = {E::pack2(dv_acc[db][4 * g4], dv_acc[db][4 * g4 + 1]),
                              E::pack2(dv_acc[db][4 * g4 + 2], dv_acc[db][4 * g4 + 3])};
                *(u32x2_t *)(rk + d) = wk;
                *(u32x2_t *)(rv + d) = wv;
            }
    }
}

}  // namespace pmkl_amd
