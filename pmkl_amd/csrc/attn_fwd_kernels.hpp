// gfx950 (CDNA4) kernels of the fused causal self-attention forward.
//
// Reference path: pmkl/nlp/causal_attention.h:145-256 (GPU kernel) and
// pmkl_pytorch_ext/fused_self_attention.cpp:5-64 (CPU operator).  The
// reference kernel is scalar fp32 with ~2,250 block barriers per key tile; the
// kernels here are written for wave64 MFMA instead:
//
//  * Scores are computed transposed, S^T = K * Q^T, with
//    v_mfma_f32_32x32x16_{bf16,f16} (v_mfma_f32_32x32x2f32 for fp32).  In the
//    32x32 accumulator layout a lane owns one query column and 16 key rows, so
//    the row max and row sum of the softmax are in-lane reductions plus one
//    v_permlane32_swap between the two lane halves.
//  * K rows are fed to the MFMA A operand in a permuted order (pi below) so
//    that lane half h ends up owning 16 consecutive keys.  Those 16 fp32
//    probabilities, converted to bf16/fp16, are exactly the B operand of the
//    P*V MFMA (O^T = V^T * P^T): P never goes through LDS.
//  * V^T is read from a row-major V tile with ds_read_b64_tr_b16 (the gfx950
//    LDS transpose read), so K and V share one staging scheme.
//  * K/V tiles are double buffered in LDS with XOR swizzles chosen so that the
//    MFMA operand reads are bank-conflict free; Q stays in VGPRs.
//  * Key tiles wholly above the diagonal are never loaded or computed; the
//    mask is applied element-wise only on tiles that straddle the diagonal or
//    the end of the sequence (in the causal resident form at head_dim 32 it
//    is the accumulator input of the diagonal block's score MFMA instead).
//    Workgroups are issued longest-first.
//  * Softmax is FA2-style: running max and per-lane partial sum, exp2 with
//    scale*log2(e) folded into one FMA, normalisation once in the epilogue.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace pmkl_amd {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));

// Kernel parameters.  Strides are in elements; head_dim is contiguous.
struct AttnParams {
    const void *q;
    const void *k;
    const void *v;
    void *o;
    void *m;
    void *l;
    int64_t q_sb, q_sh, q_ss;
    int64_t k_sb, k_sh, k_ss;
    int64_t v_sb, v_sh, v_ss;
    int64_t o_sb, o_sh, o_ss;
    int32_t H;           // heads
    int32_t S;           // sequence length
    int32_t BH;          // batch * heads
    int32_t n_qtiles;    // ceil(S / BLOCK_M)
    float scale;         // multiplies raw dot products
    float scale_log2;    // scale * log2(e)
    int32_t ml_f32;      // 1: m/l stored as float, 0: stored in the tensor dtype
    int32_t xcd_order;   // 1: workgroup index read as (XCD, head group, q-tile), see map_workgroup
    float lazy_raw;      // kLazyLog2 / scale_log2: the 16-bit kernels' rescale threshold in raw
                         // dot-product units (divided once on the host, not per wave)
};

constexpr int kWaves = 4;                // waves per workgroup of the fp32 kernel
constexpr int kThreads = kWaves * 64;    // 256
constexpr int kBlockM = 32 * kWaves;     // query rows per workgroup (32 per wave)
constexpr float kLazyLog2 = 8.0f;        // rescale threshold of the 16-bit kernel (log2 units)

// ---------------------------------------------------------------------------
// small device helpers
// ---------------------------------------------------------------------------

// Value of x in the other half of the wave (lane ^ 32), combined with op.
// v_permlane32_swap(old=x, src=x) returns {x_lo|x_lo, x_hi|x_hi}; so
// max/sum of the two results is max/sum of x and its partner in every lane.
__device__ __forceinline__ float half_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// f(integral_constant<int, I>) for I = 0 .. N-1, unrolled at compile time.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

// Row of the K tile fed to MFMA A-row i (0..31) of a 32-key block.  A-row
// i = 8g + 4h + t lands in accumulator register 4g + t of lane half h, so
// feeding it key 16h + 4g + t gives lane half h the keys 16h .. 16h+15 in
// register order.
__device__ __forceinline__ int key_of_arow(int i) {
    return ((i >> 2) & 1) * 16 + (i >> 3) * 4 + (i & 3);
}

// 16-bit element traits: MFMA, and fp32 -> T packing.
template <typename T> struct Elt16;
template <> struct Elt16<__bf16> {
    typedef bf16x8_t frag;
    static __device__ __forceinline__ f32x16_t mma(frag a, frag b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float a, float b) {
        bf16x2_t v = {(__bf16)a, (__bf16)b};
        return __builtin_bit_cast(uint32_t, v);
    }
    // acc + lo + hi of a packed pair (v_dot2_f32_bf16 against {1, 1}).
    static __device__ __forceinline__ float sum2(uint32_t packed, float acc) {
        const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, packed), one, acc, false);
    }
    // c + the lane's own four packed values, in every register of c: 16
    // blocks of 4x4x4 with an all-ones A operand (lane 4i + j of block i
    // holds column j of B and receives column j of the product).
    static __device__ __forceinline__ f32x4_t sum4(u32x2_t packed, f32x4_t c) {
        const s16x4_t one = {0x3f80, 0x3f80, 0x3f80, 0x3f80};   // bf16 1.0
        return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(one, __builtin_bit_cast(s16x4_t, packed), c, 0, 0, 0);
    }
};
template <> struct Elt16<_Float16> {
    typedef f16x8_t frag;
    static __device__ __forceinline__ f32x16_t mma(frag a, frag b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float a, float b) {
        f16x2_t v = {(_Float16)a, (_Float16)b};
        return __builtin_bit_cast(uint32_t, v);
    }
    static __device__ __forceinline__ float sum2(uint32_t packed, float acc) {
        const f16x2_t one = {(_Float16)1.0f, (_Float16)1.0f};
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, packed), one, acc, false);
    }
    static __device__ __forceinline__ f32x4_t sum4(u32x2_t packed, f32x4_t c) {
        const f16x4_t one = {(_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f};
        return __builtin_amdgcn_mfma_f32_4x4x4f16(one, __builtin_bit_cast(f16x4_t, packed), c, 0, 0, 0);
    }
};

// XOR swizzles of the 16-byte chunks of a K / V tile row (CPR chunks per
// row).  K is read with ds_read_b128 by the 32 A-rows in key_of_arow order;
// V is read with ds_read_b64_tr_b16 by groups of 4 consecutive rows.
template <int CPR> __device__ __forceinline__ int swz_k(int row) {
    if constexpr (CPR >= 16) {
        return (row & 3) | (((row >> 4) & 1) << 2) | (((row >> 2) & 1) << 3);
    } else if constexpr (CPR == 8) {
        return ((row >> 1) & 1) | (((row >> 4) & 1) << 1) | (((row >> 2) & 1) << 2);
    } else {
        return ((row >> 4) & 1) | (((row >> 2) & 1) << 1);
    }
}
template <int CPR> __device__ __forceinline__ int swz_v(int row) {
    if constexpr (CPR >= 16) {
        return ((row & 3) << 1) | ((row & 1) << 3);
    } else if constexpr (CPR == 8) {
        return ((row >> 1) & 1) << 2;
    } else {
        return 0;
    }
}

// Work item (workgroup) index L -> (head bh, query tile qt).  Default: L walks all heads
// of one query tile at a time, longest tiles first when causal.  With
// p.xcd_order (host sets it when B*H allows), L is read the way the
// dispatcher places workgroups, round-robin over the 8 XCDs (XCD = L % 8):
// each XCD walks its heads in pairs, longest query tile first within the pair
// (causal), or one head at a time (non-causal).  An XCD's L2 then holds the K/V
// of about two heads at a time while the longest tiles still start first.
template <bool CAUSAL>
__device__ __forceinline__ void map_index(const AttnParams &p, int L, int &bh, int &qt) {
    const int NQT = p.n_qtiles;
    if (p.xcd_order) {
        const int xcd = L & 7, k = L >> 3;
        if (CAUSAL) {
            const int grp = k / (2 * NQT), pos = k - grp * 2 * NQT;
            qt = NQT - 1 - (pos >> 1);
            bh = xcd + 8 * (2 * grp + (pos & 1));
        } else {
            bh = xcd + 8 * (k / NQT);
            qt = k % NQT;
        }
    } else {
        bh = L % p.BH;
        qt = CAUSAL ? (NQT - 1 - L / p.BH) : (L / p.BH);
    }
}
template <bool CAUSAL>
__device__ __forceinline__ void map_workgroup(const AttnParams &p, int &bh, int &qt) {
    map_index<CAUSAL>(p, (int)blockIdx.x, bh, qt);
}

// ---------------------------------------------------------------------------
// 16-bit kernel (bf16 / fp16), head_dim D in {32, 64, 128}
//
// NTR = 0: K/V tiles stream through a two-stage LDS ring, one barrier per
// tile.  NTR > 0 (short sequences, host guarantees ceil(S / 64) <= NTR): the
// loads of every key tile of the workgroup are issued at once, each tile gets
// its own LDS stage, and after one barrier the waves run their tiles with no
// further barrier, so a work item waits for memory once instead of once per
// tile.
// ---------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL, int NW, int NTR = 0>
__global__ __launch_bounds__(NW * 64, 8 / NW) void attn_fwd_mfma16_kernel(AttnParams p) {
    using E = Elt16<T>;
    using frag = typename E::frag;
    constexpr int kThreads = NW * 64;
    constexpr int kBlockM = 32 * NW;        // query rows per workgroup (32 per wave)
    constexpr int BN = 64;                  // keys per tile
    constexpr int CPR = D / 8;              // 16-byte chunks per row
    constexpr int TILE_CHUNKS = BN * CPR;   // chunks per K (or V) tile
    constexpr int LOADS = (TILE_CHUNKS + kThreads - 1) / kThreads;
    constexpr bool PARTIAL = TILE_CHUNKS % kThreads != 0;   // some threads idle in the last load
    constexpr int NDB = D / 32;             // 32-wide blocks of head_dim
    constexpr int NDK = D / 16;             // 16-deep MFMA steps over head_dim
    constexpr int NST = NTR > 0 ? NTR : 2;  // LDS stages (and register sets)

    __shared__ __attribute__((aligned(16))) T smem[NST][2][BN * D];  // [stage][K,V]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = lane >> 5;          // lane half
    const int col = lane & 31;         // query column owned by this lane

    // Longest-first order: blockIdx.x walks all heads of the last query tile
    // first.  Consecutive blocks of one head are BH apart, which keeps one
    // head on one XCD when BH is a multiple of 8.
    int bh, qt;
    map_workgroup<CAUSAL>(p, bh, qt);
    const int b = bh / p.H;
    const int h = bh - b * p.H;
    const int S = p.S;

    const T *qg = (const T *)p.q + b * p.q_sb + h * p.q_sh;
    const T *kg = (const T *)p.k + b * p.k_sb + h * p.k_sh;
    const T *vg = (const T *)p.v + b * p.v_sb + h * p.v_sh;
    T *og = (T *)p.o + b * p.o_sb + h * p.o_sh;

    const int q0 = qt * kBlockM;
    // 32-row block of this wave.  Resident form (one query tile; nb blocks
    // hold rows, block b needs b / 2 + 1 key tiles): waves w and w + 4 share
    // a SIMD, and with no barrier between tiles the SIMD with the most tiles
    // sets the time.  With P = nb - 4 SIMDs that must take two blocks, the
    // 2P shortest blocks are paired short with long (0 with 2P - 1, 1 with
    // 2P - 2, ...) and the longest ones run alone: at S = 256, 5 tiles per
    // SIMD instead of up to 6.
    int rb = wave;
    if constexpr (NTR > 0 && CAUSAL && NW == 8) {
        const int P = max(0, min(8, (S + 31) >> 5) - 4);
        if (wave < 4)
            rb = wave < P ? wave : P + wave;
        else if (wave - 4 < P)
            rb = 2 * P - 1 - (wave - 4);
    }
    const int q0w = q0 + 32 * rb;
    const int qi = q0w + col;                         // this lane's query row
    const int last_key = CAUSAL ? min(q0 + kBlockM - 1, S - 1) : S - 1;
    const int nt = last_key / BN + 1;                 // key tiles for the workgroup
    const bool wave_active = q0w < S;

    // Q fragments (B operand of S^T = K Q^T): lane holds Q[qi][16dk + 8hi .. +7].
    frag qf[NDK];
    {
        const int qrow = min(qi, S - 1);
        const T *src = qg + (int64_t)qrow * p.q_ss + 8 * hi;
#pragma unroll
        for (int dk = 0; dk < NDK; ++dk)
            qf[dk] = __builtin_bit_cast(frag, *(const u32x4_t *)(src + 16 * dk));
    }

    // Global -> register staging of one K/V tile with buffer loads.  Thread
    // tid owns physical chunk slots j*256 + tid and fetches the logical chunk
    // that the swizzle places there.  The buffer resource of each tile starts
    // at its first key and ends at the last key of the sequence, so rows past
    // the end read as zero (those keys are masked) and the per-thread byte
    // offsets are the same for every tile.
    // Streaming: two register sets; the loads of tile t go to set t & 1 two
    // tiles ahead of use, so a load has two steps to land before its LDS
    // write.  Resident: one set per tile.
    u32x4_t kreg[NST][LOADS], vreg[NST][LOADS];
    int koff[LOADS], voff[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const int sl = j * kThreads + tid;
        const int row = sl / CPR;
        const int pc = sl % CPR;
        koff[j] = (int)((row * p.k_ss + 8 * (pc ^ swz_k<CPR>(row))) * (int64_t)sizeof(T));
        voff[j] = (int)((row * p.v_ss + 8 * (pc ^ swz_v<CPR>(row))) * (int64_t)sizeof(T));
    }
    auto gload = [&](int kt, auto set_c) {
        constexpr int SET = decltype(set_c)::value;
        const int kbase = kt * BN;
        const int rows = min(BN, S - kbase);
        const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(kg + (int64_t)kbase * p.k_ss), (short)0, (int)(((rows - 1) * p.k_ss + D) * sizeof(T)),
            0x00020000);
        const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(vg + (int64_t)kbase * p.v_ss), (short)0, (int)(((rows - 1) * p.v_ss + D) * sizeof(T)),
            0x00020000);
#pragma unroll
        for (int j = 0; j < LOADS; ++j) {
            if (!PARTIAL || j * kThreads + tid < TILE_CHUNKS) {
                kreg[SET][j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(kr, koff[j], 0, 0));
                vreg[SET][j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(vr, voff[j], 0, 0));
            }
        }
    };
    auto swrite = [&](int st, auto set_c) {
        constexpr int SET = decltype(set_c)::value;
#pragma unroll
        for (int j = 0; j < LOADS; ++j) {
            const int sl = j * kThreads + tid;
            if (!PARTIAL || sl < TILE_CHUNKS) {
                *(u32x4_t *)(&smem[st][0][sl * 8]) = kreg[SET][j];
                *(u32x4_t *)(&smem[st][1][sl * 8]) = vreg[SET][j];
            }
        }
    };

    f32x16_t acc[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
    // Row max bookkeeping in raw dot-product units.  m_true is the exact
    // running max (the m output); m_use is the offset of the exponentials,
    // moved up to the running max only when some row of the wave outgrows it
    // by more than kLazyLog2 in log2 units, so O and l are rescaled on a few
    // tiles instead of every tile with a new max.  Probabilities then stay
    // below 2^kLazyLog2, which bf16 / fp16 and the fp32 accumulators hold
    // with their usual relative precision.
    float m_true = -INFINITY;
    float m_use = -INFINITY;
    // Per-lane partial row sums relative to m_use, accumulated by 4x4x4
    // MFMAs (sum4) into component 0 .. 3 alike; two accumulators alternate so
    // that consecutive row-sum MFMAs do not wait on each other.
    f32x4_t lsum[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    const float lazy_raw = p.lazy_raw;

    // Per-lane constant parts of the LDS addresses.
    const int arow = key_of_arow(col);        // K tile row read by this lane (per 32-key block)
    const int g = lane >> 4, tt = lane & 15;  // 16-lane group for the V transpose read
    const int vrow0 = 16 * (g >> 1) + (tt >> 2);
    const int vcol0 = 16 * (g & 1) + 4 * (tt & 3);

    // Causal resident form at head_dim 32: a wave's rows start on a 32-key
    // block boundary, so each 32-key block is wholly visible, wholly masked,
    // or the diagonal block, whose mask is the same for every wave: lane
    // half hi, register r holds key 16 hi + r of the block against query col.
    // The diagonal block takes its mask as the accumulator input of its first
    // score MFMA (0 where visible, -inf where not), which costs no VALU work
    // (a compare and a select per score otherwise); the masked block after it
    // is skipped.  The mask lives in LDS (dtab[j][lane] = registers 4j ..
    // 4j+3 of lane; wave 0 writes it before the workgroup's barrier), read
    // with four conflict-free 16-byte reads: kept in VGPRs it is rebuilt by
    // the compiler on every use.  Only at head_dim 32 (107 VGPRs, four waves
    // per SIMD): with the five tile bodies of this form (KIND 1-3, FIRST or
    // not) the head_dim-64 kernel needs 159, three waves per SIMD.
    constexpr bool BIAS = CAUSAL && NTR > 0 && D == 32;
    __shared__ __attribute__((aligned(16))) f32x4_t dtab[BIAS ? 4 * 64 : 1];

    // One key tile kt of this wave from LDS stage st: scores, mask, online
    // softmax, O update.  KIND 0: element-wise mask where the tile straddles
    // the diagonal or the end of the sequence; 1: no mask; 2: diagonal block
    // second (BIAS only); 3: diagonal block first, second block masked
    // (BIAS only).  + FIRST (BIAS only): the wave's first tile, whose row
    // sums and O start from zero MFMA accumulators and need no rescale.
    constexpr int FIRST = 4;
    auto compute_tile = [&](int st, int kt, auto kind_c) __attribute__((always_inline)) {
        constexpr int KIND = decltype(kind_c)::value & 3;
        constexpr bool IS_FIRST = (decltype(kind_c)::value & FIRST) != 0;
        constexpr int NKB = KIND == 3 ? 1 : 2;   // 32-key blocks computed
        const int kbase = kt * BN;
        {
            const T *Ks = smem[st][0];
            const T *Vs = smem[st][1];
            // ---- S^T = K Q^T for two 32-key blocks ----
            f32x16_t sacc[2];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                if constexpr (BIAS && (KIND == 2 || KIND == 3)) {
                    if (kb == (KIND == 2 ? 1 : 0)) {
                        const f32x4_t b0 = dtab[lane], b1 = dtab[64 + lane], b2 = dtab[128 + lane], b3 = dtab[192 + lane];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            sacc[kb][e] = b0[e];
                            sacc[kb][4 + e] = b1[e];
                            sacc[kb][8 + e] = b2[e];
                            sacc[kb][12 + e] = b3[e];
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
                }
                const int row = 32 * kb + arow;
                const T *krow = Ks + row * D;
                const int sw = swz_k<CPR>(row);
#pragma unroll
                for (int dk = 0; dk < NDK; ++dk) {
                    const int x = 2 * dk + hi;
                    frag a = __builtin_bit_cast(frag, *(const u32x4_t *)(krow + 8 * (x ^ sw)));
                    sacc[kb] = E::mma(a, qf[dk], sacc[kb]);
                }
            }
            // ---- mask (only tiles that straddle the diagonal or the end) ----
            const bool need_mask = (CAUSAL && kbase + BN - 1 > q0w) || (kbase + BN > S);
            if (KIND == 0 && need_mask) {
                const int lim = CAUSAL ? min(qi, S - 1) : S - 1;   // last visible key
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    // register r holds key kbase + 32kb + 16hi + r: visible iff r <= d
                    const int d = lim - (kbase + 32 * kb + 16 * hi);
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (r > d) sacc[kb][r] = -INFINITY;
                }
            }
            // ---- online softmax ----
            // Row max as a tree (v_max3, depth 3 per block) rather than a
            // 16-deep chain: the chain's latency sits between the score
            // MFMAs and the exponentials of every tile.
            float bm[NKB];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                float t5[5];
#pragma unroll
                for (int i = 0; i < 5; ++i) t5[i] = fmaxf(fmaxf(sacc[kb][3 * i], sacc[kb][3 * i + 1]), sacc[kb][3 * i + 2]);
                bm[kb] = fmaxf(fmaxf(fmaxf(t5[0], t5[1]), t5[2]), fmaxf(fmaxf(t5[3], t5[4]), sacc[kb][15]));
            }
            float mx = NKB == 1 ? bm[0] : fmaxf(bm[0], bm[NKB - 1]);
            mx = half_max(mx);
            // Rescale O and l only when some row max of this wave grew (a
            // wave-uniform branch); the offset is always the exact running max.
            m_true = fmaxf(m_true, mx);
            if (IS_FIRST) {
                m_use = mx;   // finite: every row has a visible key in its first tile
            } else if (__builtin_amdgcn_ballot_w64(mx > m_use + lazy_raw)) {
                const float m_new = fmaxf(m_use, mx);
                const float alpha = fast_exp2((m_use - m_new) * p.scale_log2);  // 0 on the first tile
                m_use = m_new;
                if (kt > 0) {   // tile 0 is every wave's first: O and l are still zero
                    lsum[0] *= alpha;
                    lsum[1] *= alpha;
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
                }
            }
            const float moff = (m_use == -INFINITY) ? 0.f : -m_use * p.scale_log2;
            uint32_t pk[2][8];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    const float p0 = fast_exp2(__builtin_fmaf(sacc[kb][r], p.scale_log2, moff));
                    const float p1 = fast_exp2(__builtin_fmaf(sacc[kb][r + 1], p.scale_log2, moff));
                    pk[kb][r >> 1] = E::pack2(p0, p1);
                }
            // l sums the probabilities as rounded for the PV product, so O is
            // normalised by exactly the weights it was built from.
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const u32x2_t pair = {pk[kb][2 * c], pk[kb][2 * c + 1]};
                    lsum[c & 1] = E::sum4(pair, (IS_FIRST && kb == 0 && c < 2) ? f32x4_t{0.f, 0.f, 0.f, 0.f} : lsum[c & 1]);
                }
            // ---- O^T += V^T P^T ----
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    u32x4_t bw = {pk[kb][4 * c], pk[kb][4 * c + 1], pk[kb][4 * c + 2], pk[kb][4 * c + 3]};
                    const frag bfr = __builtin_bit_cast(frag, bw);
                    const int r0 = 32 * kb + 8 * c + vrow0;      // rows r0 .. (elements 0-3), r0+4 .. (4-7)
#pragma unroll
                    for (int db = 0; db < NDB; ++db) {
                        const int cc = 32 * db + vcol0;             // element column of this lane's 4-wide read
                        const int ch = cc >> 3, part = cc & 7;
                        const T *a0 = Vs + r0 * D + 8 * (ch ^ swz_v<CPR>(r0)) + part;
                        const T *a1 = Vs + (r0 + 4) * D + 8 * (ch ^ swz_v<CPR>(r0 + 4)) + part;
                        typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
                        s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)a0);
                        s16x4_t hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)a1);
                        typedef short s16x8_t __attribute__((ext_vector_type(8)));
                        s16x8_t a8 = {lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                        acc[db] = E::mma(__builtin_bit_cast(frag, a8), bfr,
                                         (IS_FIRST && kb == 0 && c == 0) ? f32x16_t{} : acc[db]);
                    }
                }
        }
    };
    auto wave_needs = [&](int kt) __attribute__((always_inline)) { return wave_active && (!CAUSAL || kt * BN <= q0w + 31); };

    if constexpr (NTR > 0) {
        // All key tiles of the workgroup at once (nt <= NTR): issue every
        // load, wait once, write each tile to its own stage, one barrier.
        static_for<NTR>([&](auto t_c) {
            constexpr int t = decltype(t_c)::value;
            if (t < nt) gload(t, t_c);
        });
        __builtin_amdgcn_s_waitcnt(0);
        static_for<NTR>([&](auto t_c) {
            constexpr int t = decltype(t_c)::value;
            if (t < nt) swrite(t, t_c);
        });
        if constexpr (BIAS) {
            if (wave == 0) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    f32x4_t v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = (16 * hi + 4 * j + e <= col) ? 0.f : -INFINITY;
                    dtab[64 * j + lane] = v;
                }
            }
        }
        __syncthreads();
        // No barrier from here on: each wave runs its own tiles and leaves.
        if constexpr (BIAS) {
            if (wave_active) {
                const int kdiag = q0w / BN;   // tile of the wave's diagonal block (kdiag < nt)
                if (kdiag == 0) {
                    if (q0w % BN)
                        compute_tile(0, 0, std::integral_constant<int, 2 | FIRST>{});
                    else
                        compute_tile(0, 0, std::integral_constant<int, 3 | FIRST>{});
                } else {
                    compute_tile(0, 0, std::integral_constant<int, 1 | FIRST>{});
                    for (int kt = 1; kt < kdiag; ++kt) compute_tile(kt, kt, std::integral_constant<int, 1>{});
                    if (q0w % BN)
                        compute_tile(kdiag, kdiag, std::integral_constant<int, 2>{});
                    else
                        compute_tile(kdiag, kdiag, std::integral_constant<int, 3>{});
                }
            }
        } else {
            for (int kt = 0; kt < nt && wave_needs(kt); ++kt) compute_tile(kt, kt, std::integral_constant<int, 0>{});
        }
    } else {
        gload(0, std::integral_constant<int, 0>{});
        swrite(0, std::integral_constant<int, 0>{});
        // Q fragments and tile 0 have landed before the loop, so no vmcnt wait is
        // needed before the score MFMAs of a tile; tile 1 is left in flight.
        __builtin_amdgcn_s_waitcnt(0);
        gload(min(1, nt - 1), std::integral_constant<int, 1>{});
        __syncthreads();

        // Tile kt: LDS stage kt & 1; its registers (set kt & 1) are refilled with
        // tile kt + 2, and tile kt + 1 (set (kt+1) & 1) goes to the other stage.
        auto tile_step = [&](auto set_c, int kt) __attribute__((always_inline)) {
            constexpr int SET = decltype(set_c)::value;
            // Issued on every step (a clamped tile near the end) so that the
            // number of loads in flight, and hence the vmcnt wait before the LDS
            // write below, is the same on every path.
            gload(min(kt + 2, nt - 1), set_c);
            if (wave_needs(kt)) compute_tile(SET, kt, std::integral_constant<int, 0>{});
            if (kt + 1 < nt) swrite(SET ^ 1, std::integral_constant<int, SET ^ 1>{});
            __syncthreads();
        };
        for (int kt = 0; kt < nt; kt += 2) {
            tile_step(std::integral_constant<int, 0>{}, kt);
            if (kt + 1 < nt) tile_step(std::integral_constant<int, 1>{}, kt + 1);
        }
    }

    // ---- epilogue: normalise, store O, m, l ----
    const float l_sum = half_sum(lsum[0][0] + lsum[1][0]);   // relative to m_use
    // Streaming form: O goes out through LDS.  A lane holds 8-byte pieces of
    // its row, and stores of those (16 bytes of each of 32 rows per
    // instruction) write partial lines; each wave instead writes its 32 x D
    // block to its own slice of the K/V stages (free: the loop ends on a
    // barrier), 16-byte chunks XOR-swizzled by row, and stores whole rows,
    // 64 / CPR rows per instruction (measured 5-16% faster at S 300-1,000,
    // head_dim 64 and 128; no gain at 32, whose 64-byte rows the direct
    // stores already fill in four instructions).  The resident form keeps the
    // direct stores: its waves end at different times and a barrier before
    // the stores cost more than it saved.
    const float inv = __builtin_amdgcn_rcpf(l_sum);   // v_rcp_f32 (1 ulp); not stored where l_sum is 0
    if constexpr (NTR == 0 && D >= 64) {
        static_assert(NST * 2 * BN >= NW * 32, "O staging must fit in the K/V stages");
        T *ost = &smem[0][0][0] + wave * 32 * D;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int c = 4 * db + g4;   // 16-byte chunk of the row
                u32x2_t w2 = {E::pack2(acc[db][4 * g4] * inv, acc[db][4 * g4 + 1] * inv),
                              E::pack2(acc[db][4 * g4 + 2] * inv, acc[db][4 * g4 + 3] * inv)};
                *(u32x2_t *)(ost + col * D + 8 * (c ^ (col % CPR)) + 4 * hi) = w2;
            }
        // LDS operations of one wave complete in order; this keeps the
        // compiler from moving the reads above the other lanes' writes.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        constexpr int RPI = 64 / CPR;   // rows per store instruction
        const int c = lane % CPR;
#pragma unroll
        for (int it = 0; it < 32 / RPI; ++it) {
            const int r = it * RPI + lane / CPR;
            const u32x4_t val = *(const u32x4_t *)(ost + r * D + 8 * (c ^ (r % CPR)));
            if (wave_active && q0w + r < S) *(u32x4_t *)(og + (int64_t)(q0w + r) * p.o_ss + 8 * c) = val;
        }
    } else if (wave_active && qi < S) {
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
    }
    if (wave_active && qi < S) {
        // l of the output is relative to the exact row max
        const float l_tot = l_sum * fast_exp2((m_use - m_true) * p.scale_log2);
        if (hi == 0) {
            const int64_t mi = (int64_t)bh * S + qi;
            const float mval = m_true * p.scale;
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

// ---------------------------------------------------------------------------
// fp32 kernel (true fp32 arithmetic on v_mfma_f32_32x32x2f32), D in {32,64,128}
// ---------------------------------------------------------------------------
template <int D, bool CAUSAL>
__global__ __launch_bounds__(kThreads, 1) void attn_fwd_f32_kernel(AttnParams p) {
    constexpr int BN = 32;           // keys per tile
    constexpr int LD = D + 1;        // padded LDS row (floats)
    constexpr int NDB = D / 32;
    constexpr int NDK = D / 2;
    __shared__ float Ks[BN * LD];
    __shared__ float Vs[BN * LD];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = lane >> 5;
    const int col = lane & 31;

    const int L = blockIdx.x;
    const int bh = L % p.BH;
    const int qt = CAUSAL ? (p.n_qtiles - 1 - L / p.BH) : (L / p.BH);
    const int b = bh / p.H;
    const int h = bh - b * p.H;
    const int S = p.S;

    const float *qg = (const float *)p.q + b * p.q_sb + h * p.q_sh;
    const float *kg = (const float *)p.k + b * p.k_sb + h * p.k_sh;
    const float *vg = (const float *)p.v + b * p.v_sb + h * p.v_sh;
    float *og = (float *)p.o + b * p.o_sb + h * p.o_sh;

    const int q0 = qt * kBlockM;
    const int q0w = q0 + 32 * wave;
    const int qi = q0w + col;
    const int last_key = CAUSAL ? min(q0 + kBlockM - 1, S - 1) : S - 1;
    const int nt = last_key / BN + 1;
    const bool wave_active = q0w < S;

    float qf[NDK];
    {
        const int qrow = min(qi, S - 1);
        const float *src = qg + (int64_t)qrow * p.q_ss + hi;
#pragma unroll
        for (int dk = 0; dk < NDK; ++dk) qf[dk] = src[2 * dk];
    }

    f32x16_t acc[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    const int arow = key_of_arow(col);

    // K/V tile staging: tile kt+1 is loaded into registers while tile kt is
    // computed, and written to LDS at the top of the next iteration.
    constexpr int NE = BN * D / kThreads;   // elements per thread per tensor
    static_assert(BN * D % kThreads == 0, "whole tile per pass");
    float kreg[NE], vreg[NE];
    auto load_tile = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NE; ++j) {
            const int i = j * kThreads + tid;
            const int r = i / D, c = i % D;
            const int key = min(kt * BN + r, S - 1);
            kreg[j] = kg[(int64_t)key * p.k_ss + c];
            vreg[j] = vg[(int64_t)key * p.v_ss + c];
        }
    };
    load_tile(0);
    for (int kt = 0; kt < nt; ++kt) {
        const int kbase = kt * BN;
#pragma unroll
        for (int j = 0; j < NE; ++j) {
            const int i = j * kThreads + tid;
            const int r = i / D, c = i % D;
            Ks[r * LD + c] = kreg[j];
            Vs[r * LD + c] = vreg[j];
        }
        __syncthreads();
        if (kt + 1 < nt) load_tile(kt + 1);
        const bool wave_needed = wave_active && (!CAUSAL || kbase <= q0w + 31);
        if (wave_needed) {
            f32x16_t sacc;
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
#pragma unroll
            for (int dk = 0; dk < NDK; ++dk)
                sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[arow * LD + 2 * dk + hi], qf[dk], sacc, 0, 0, 0);
            const bool need_mask = (CAUSAL && kbase + BN - 1 > q0w) || (kbase + BN > S);
            if (need_mask) {
                const int lim = CAUSAL ? min(qi, S - 1) : S - 1;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (kbase + 16 * hi + r > lim) sacc[r] = -INFINITY;
            }
            float mx = sacc[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sacc[r]);
            mx = half_max(mx);
            const float m_new = fmaxf(m_run, mx);
            const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
            const float alpha = fast_exp2((m_run - m_use) * p.scale_log2);
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
            const float moff = -m_use * p.scale_log2;
            float pr[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                pr[r] = fast_exp2(__builtin_fmaf(sacc[r], p.scale_log2, moff));
                l_run += pr[r];
            }
#pragma unroll
            for (int c = 0; c < 16; ++c)
#pragma unroll
                for (int db = 0; db < NDB; ++db)
                    acc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[(16 * hi + c) * LD + 32 * db + col], pr[c],
                                                                    acc[db], 0, 0, 0);
        }
        __syncthreads();
    }

    const float l_tot = half_sum(l_run);
    if (wave_active && qi < S) {
        const float inv = 1.0f / l_tot;
        float *orow = og + (int64_t)qi * p.o_ss;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d = 32 * db + 8 * g4 + 4 * hi;
                float4 w4 = {acc[db][4 * g4] * inv, acc[db][4 * g4 + 1] * inv, acc[db][4 * g4 + 2] * inv,
                             acc[db][4 * g4 + 3] * inv};
                *(float4 *)(orow + d) = w4;
            }
        if (hi == 0) {
            const int64_t mi = (int64_t)bh * S + qi;
            ((float *)p.m)[mi] = m_run * p.scale;
            ((float *)p.l)[mi] = l_tot;
        }
    }
}

// ---------------------------------------------------------------------------
// fp32, small problems: one workgroup per (head, 32-row query block); its
// NSPL waves split the block's key tiles (wave w takes tiles w, w + NSPL,
// ...), each staging its own tiles in LDS (no workgroup barrier in the loop),
// then the partial (O, m, l) of the waves are combined by the log-sum-exp
// rule.  The rows' longest chain of dependent tiles shrinks NSPL-fold, which
// is what bounds a launch of a few workgroups.  Same arithmetic per tile as
// attn_fwd_f32_kernel (v_mfma_f32_32x32x2f32, exact rescale).
// ---------------------------------------------------------------------------
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void attn_fwd_f32_split_kernel(AttnParams p) {
    constexpr int BN = 32;            // keys per tile (= query rows per workgroup)
    constexpr int NSPL = 4;           // waves, each a share of the key tiles
    constexpr int LD = D + 1;         // padded LDS row (floats)
    constexpr int NDB = D / 32;
    constexpr int NDK = D / 2;
    constexpr int NE = BN * D / 64;   // elements per lane per tensor per tile
    // Per wave: K and V tile; after the loop the same memory holds the
    // partials (NDB * 16 accumulators + m + l per lane and wave).
    constexpr int PW = NDB * 16 * 64 + 2 * 64;
    static_assert(NSPL * PW <= NSPL * 2 * BN * LD, "partials fit the staging memory");
    __shared__ float smem[NSPL * 2 * BN * LD];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = lane >> 5;
    const int col = lane & 31;

    const int L = blockIdx.x;
    const int bh = L % p.BH;
    const int rb = CAUSAL ? (p.n_qtiles - 1 - L / p.BH) : (L / p.BH);
    const int b = bh / p.H;
    const int h = bh - b * p.H;
    const int S = p.S;

    const float *qg = (const float *)p.q + b * p.q_sb + h * p.q_sh;
    const float *kg = (const float *)p.k + b * p.k_sb + h * p.k_sh;
    const float *vg = (const float *)p.v + b * p.v_sb + h * p.v_sh;
    float *og = (float *)p.o + b * p.o_sb + h * p.o_sh;

    const int q0 = rb * BN;
    const int qi = q0 + col;
    // Every row of the block sees at least the first key of each tile up to
    // its block's diagonal tile (rows and key tiles are both 32 wide).
    const int last_key = CAUSAL ? min(q0 + BN - 1, S - 1) : S - 1;
    const int nt = last_key / BN + 1;

    float qf[NDK];
    {
        const int qrow = min(qi, S - 1);
        const float *src = qg + (int64_t)qrow * p.q_ss + hi;
#pragma unroll
        for (int dk = 0; dk < NDK; ++dk) qf[dk] = src[2 * dk];
    }
    f32x16_t acc[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    const int arow = key_of_arow(col);
    float *Ks = smem + wave * 2 * BN * LD;
    float *Vs = Ks + BN * LD;

    for (int kt = wave; kt < nt; kt += NSPL) {
        const int kbase = kt * BN;
        float kreg[NE], vreg[NE];
#pragma unroll
        for (int j = 0; j < NE; ++j) {
            const int i = j * 64 + lane;
            const int r = i / D, c = i % D;
            const int key = min(kbase + r, S - 1);
            kreg[j] = kg[(int64_t)key * p.k_ss + c];
            vreg[j] = vg[(int64_t)key * p.v_ss + c];
        }
        // The wave's own LDS region: its earlier reads of the previous tile
        // are issued before these writes, and the LDS executes one wave's
        // instructions in order, so neither side needs a barrier.
        asm volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < NE; ++j) {
            const int i = j * 64 + lane;
            const int r = i / D, c = i % D;
            Ks[r * LD + c] = kreg[j];
            Vs[r * LD + c] = vreg[j];
        }
        asm volatile("" ::: "memory");
        f32x16_t sacc;
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
#pragma unroll
        for (int dk = 0; dk < NDK; ++dk)
            sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[arow * LD + 2 * dk + hi], qf[dk], sacc, 0, 0, 0);
        const bool need_mask = (CAUSAL && kbase + BN - 1 > q0) || (kbase + BN > S);
        if (need_mask) {
            const int lim = CAUSAL ? min(qi, S - 1) : S - 1;
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (kbase + 16 * hi + r > lim) sacc[r] = -INFINITY;
        }
        float mx = sacc[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sacc[r]);
        mx = half_max(mx);
        const float m_new = fmaxf(m_run, mx);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = fast_exp2((m_run - m_use) * p.scale_log2);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
        const float moff = -m_use * p.scale_log2;
        float pr[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            pr[r] = fast_exp2(__builtin_fmaf(sacc[r], p.scale_log2, moff));
            l_run += pr[r];
        }
#pragma unroll
        for (int c = 0; c < 16; ++c)
#pragma unroll
            for (int db = 0; db < NDB; ++db)
                acc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[(16 * hi + c) * LD + 32 * db + col], pr[c], acc[db],
                                                                0, 0, 0);
        asm volatile("" ::: "memory");
    }

    // Partials to LDS (the staging memory, once every wave is past its loop),
    // then wave 0 combines them: O = sum_w 2^((m_w - M) c) O_w over the
    // block's running maxima M = max_w m_w, l likewise.  A wave without
    // tiles holds m = -inf, l = 0, O = 0 and weighs 0.
    __syncthreads();
    float *part = smem + wave * PW;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) part[(db * 16 + r) * 64 + lane] = acc[db][r];
    part[NDB * 1024 + lane] = m_run;
    part[NDB * 1024 + 64 + lane] = l_run;
    __syncthreads();
    if (wave != 0) return;
    float mw[NSPL];
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NSPL; ++w) {
        mw[w] = smem[w * PW + NDB * 1024 + lane];
        M = fmaxf(M, mw[w]);
    }
    float l_sum = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
#pragma unroll
    for (int w = 0; w < NSPL; ++w) {
        const float f = fast_exp2((mw[w] - M) * p.scale_log2);   // 0 for a wave without tiles
        const float *pw = smem + w * PW;
        l_sum += f * pw[NDB * 1024 + 64 + lane];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[db][r] += f * pw[(db * 16 + r) * 64 + lane];
    }
    const float l_tot = half_sum(l_sum);
    if (qi < S) {
        const float inv = 1.0f / l_tot;
        float *orow = og + (int64_t)qi * p.o_ss;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d = 32 * db + 8 * g4 + 4 * hi;
                float4 w4 = {acc[db][4 * g4] * inv, acc[db][4 * g4 + 1] * inv, acc[db][4 * g4 + 2] * inv,
                             acc[db][4 * g4 + 3] * inv};
                *(float4 *)(orow + d) = w4;
            }
        if (hi == 0) {
            const int64_t mi = (int64_t)bh * S + qi;
            ((float *)p.m)[mi] = M * p.scale;
            ((float *)p.l)[mi] = l_tot;
        }
    }
}

}  // namespace pmkl_amd
