// Slot-scheduled variant of the 16-bit attention kernel (gfx950).
//
// Same layouts and arithmetic as attn_fwd_mfma16_kernel (transposed scores
// S^T = K Q^T, P kept in registers as the B operand of O^T = V^T P^T, V^T from
// ds_read_b64_tr_b16, lazy rescale).  256 query rows per workgroup, in one of
// two layouts (template parameters QB, NW):
//  * QB = 2, NW = 4: one wave per SIMD, each owning two 32-row blocks; every
//    K or V fragment read from LDS feeds one MFMA of each block, which halves
//    the LDS operand reads per MFMA;
//  * QB = 1, NW = 8: two waves per SIMD, 32 rows each, both running the same
//    schedule: when one wave waits (barrier, LDS, a dependency), the other
//    issues.  A wave that issues an MFMA while the matrix core is busy blocks
//    the SIMD's vector issue of the other wave too, so the waves do not split
//    into an MFMA wave and a softmax wave: each keeps its own vector work
//    between its own MFMAs.
//
// Software pipeline: iteration t issues, one MFMA per slot,
//   slots 0 .. QKS-1       QK of tile t+1 (every block, score set (t+1) & 1)
//   slots QKS .. NSLOT-1   PV of tile t (every block), each group of PV
//                          MFMAs followed by the row-sum MFMAs of its
//                          probabilities (an all-ones A operand)
// and behind every MFMA a share of the VALU work, placed at compile time
// (W64Sched): the exponentials and packing of tile t, finished a slot before
// the PV MFMA that reads them, then the row maxima of tile t+1 once its QK is
// done.  The wave issues in order, so what stands between two
// MFMAs must fit under one MFMA (~32 clocks of the matrix core): an MFMA
// issued straight behind another stalls the wave, and its VALU share with it.
// sched_barrier fences pin every slot; asm-volatile register pins keep the
// IR optimizer from sinking VALU work towards its consumers.
//
// Operands: K fragments of tile t+1 then V^T fragments of tile t form one
// stream of NF fragments per iteration, read from LDS RING fragments ahead of
// their MFMAs into a ring of registers (NF % RING == 0, so the ring position
// of a fragment is the same in every iteration); the last RING reads of an
// iteration already fetch the first K fragments of the next one.
//
// Registers: O^T accumulators (QB x D/32 x 16), row sums (QB x 16) and the
// Q fragments live in AGPRs, used only by MFMAs issued from inline asm;
// scores, P and operands live in VGPRs.  The compiler cannot see inside those MFMAs, so the kernel
// keeps the MFMA -> VALU hazard distances itself (w64_mfma_drain before the
// first VALU access of an MFMA result, and P written a full slot before the
// MFMA that reads it).
//
// LDS: K/V tiles reach LDS by LDS-DMA (buffer_load ... lds) into four slots
// each, K(t) and V(t) in slot t % 4; an item's stream positions are rounded
// up to a multiple of four, so every item starts in slot 0 and the unrolled
// loop addresses the slots at compile time.  Iteration t issues the DMAs of
// K(t+3) and V(t+2) in the slots right before its barrier (BARS), which
// follows the wave's last LDS read of K(t+1) and V(t) and a wait for the
// DMAs of iteration t-1 (K(t+2), V(t+1)).  So a DMA only overwrites a slot
// all waves have finished reading (K(t-1), V(t-2), read before the previous
// barrier), and a tile is read only after the barrier that follows its
// arrival.  At head_dim 64 (PAIR below) barriers come at odd positions only,
// with the same DMAs issued in each position's first slots.
#pragma once

#include "attn_fwd_kernels.hpp"

namespace pmkl_amd {

// One LDS-DMA of 16 bytes per lane: bytes [off + so, off + so + 16) of
// buffer r (off per lane, so wave-uniform) land at LDS byte address
// lds + LOFF + 16 * lane.  Inline asm, so the compiler neither waits for it
// before unrelated LDS reads nor counts it; the kernel waits itself.  M0 is
// formed here from the wave's LDS base and the compile-time slot offset (so
// the compiler does not keep one SGPR per slot).  An SALU write of M0 needs
// one wait state before an LDS-DMA reads it.  The add writes SCC as well as
// M0, and both are declared clobbered: the compiler must not keep a
// comparison result in SCC across a DMA (it did, once code was added around
// the loop, and a flag tested before a DMA and used after it read as 0).
template <int LOFF>
__device__ __forceinline__ void w64_lds_dma16(__amdgpu_buffer_rsrc_t r, int off, int so, unsigned lds) {
    asm volatile("s_add_u32 m0, %1, %4\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %2, %3 offen lds" ::"v"(off), "s"(lds),
                 "s"(r), "s"(so), "n"(LOFF)
                 : "memory", "scc", "m0");
}

// MFMAs with operands pinned to register files:
//   pv    c (AGPRs) += a * b
//   qk0   d (VGPRs)  = a * b (b in AGPRs)
//   qk    d (VGPRs) += a * b (b in AGPRs)
template <typename T> struct W64Mma;
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
template <> struct W64Mma<__bf16> {
    typedef bf16x4_t half_frag;
    // c (AGPRs) += a * b over 16 blocks of 4x4x4: lane 4 i + j of block i
    // holds column j of b, so with a = 1 every register of a lane receives the
    // sum of the lane's own four values of b.
    static __device__ __forceinline__ void sum4(f32x4_t &c, bf16x4_t a, bf16x4_t b) {
        asm volatile("v_mfma_f32_4x4x4_16b_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
    }
    static __device__ __forceinline__ void pv(f32x16_t &c, bf16x8_t a, bf16x8_t b) {
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
    }
    static __device__ __forceinline__ void qk0(f32x16_t &d, bf16x8_t a, bf16x8_t b) {
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "a"(b));
    }
    static __device__ __forceinline__ void qk(f32x16_t &d, bf16x8_t a, bf16x8_t b) {
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "a"(b));
    }
};
template <> struct W64Mma<_Float16> {
    typedef f16x4_t half_frag;
    static __device__ __forceinline__ void sum4(f32x4_t &c, f16x4_t a, f16x4_t b) {
        asm volatile("v_mfma_f32_4x4x4_16b_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
    }
    static __device__ __forceinline__ void pv(f32x16_t &c, f16x8_t a, f16x8_t b) {
        asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
    }
    static __device__ __forceinline__ void qk0(f32x16_t &d, f16x8_t a, f16x8_t b) {
        asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "a"(b));
    }
    static __device__ __forceinline__ void qk(f32x16_t &d, f16x8_t a, f16x8_t b) {
        asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "a"(b));
    }
};
// 24 wait states: enough between an MFMA writing registers and VALU reading
// or writing them, for every MFMA used here.  The MFMAs are inline asm, so
// the compiler inserts no wait states of its own and does not know that the
// drain guards their results: every drain is followed (and, where VALU
// writes feed a later MFMA, preceded) by w64_fence on the registers it
// guards, an empty asm that redefines them, so no read of them is scheduled
// above the drain and no write below it.
__device__ __forceinline__ void w64_mfma_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }
__device__ __forceinline__ void w64_fence_a(f32x16_t &x) { asm volatile("" : "+a"(x)); }
__device__ __forceinline__ void w64_fence_a(f32x4_t &x) { asm volatile("" : "+a"(x)); }
__device__ __forceinline__ void w64_fence_v(f32x16_t &x) { asm volatile("" : "+v"(x)); }

// s = (R <= d) ? s : -inf, through VCC: left to itself the compiler computes
// all compares of a tile into separate SGPR pairs first, and that pressure
// spills long-lived SGPRs for the whole loop.  A VALU write of VCC needs two
// wait states before v_cndmask reads it as the lane mask (the compiler keeps
// the same distance in its own code for gfx950), hence the s_nop 1.
template <int R>
__device__ __forceinline__ float w64_mask_key(float s, int d) {
    asm volatile("v_cmp_le_i32 vcc, %1, %2\n\ts_nop 1\n\tv_cndmask_b32 %0, %3, %0, vcc"
                 : "+v"(s) : "n"(R), "v"(d), "v"(-INFINITY) : "vcc");
    return s;
}
// Row-max steps as single instructions: fmaxf on MFMA results (opaque to the
// compiler) is lowered with a canonicalising v_max of each input first, 8
// extra VALU instructions per 32x64 score tile.
__device__ __forceinline__ float w64_max3(float a, float b, float c) {
    float d;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}
__device__ __forceinline__ float w64_max(float a, float b) {
    float d;
    asm("v_max_f32 %0, %1, %2" : "=v"(d) : "v"(a), "v"(b));
    return d;
}
// f(integral_constant<int, I>) for I = B .. E-1, unrolled at compile time.
template <int B, int E, typename F>
__device__ __forceinline__ void w64_static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        w64_static_for<B + 1, E>(f);
    }
}

// Compile-time slot schedule of one iteration (head_dim D, QB 32-row query
// blocks per wave), one MFMA per slot:
//   slots 0 .. QKS-1      QK of tile t+1: fragment s / QB, block s % QB
//   then 4 groups (kb, c) of GS slots: the NDB QB PV MFMAs of the group
//   (fragment, block), then 2 QB row-sum MFMAs (4x4x4, all-ones A operand),
//   each adding half of a block's packed probabilities of the group into the
//   row sums.
template <int D, int QB> struct W64Sched {
    static constexpr int NDB = D / 32;            // 32-wide blocks of head_dim
    static constexpr int NDK = D / 16;            // 16-deep MFMA steps over head_dim
    static constexpr int NKF = 2 * NDK;           // K fragments per tile: (dk, kb)
    static constexpr int NVF = 4 * NDB;           // V^T fragments per tile: (kb, c, db)
    static constexpr int NF = NKF + NVF;          // fragments per iteration
    static constexpr int QKS = QB * NKF;          // first PV slot
    static constexpr int GS = QB * (NDB + 2);     // slots per PV group
    static constexpr int NSLOT = QKS + 4 * GS;    // MFMAs per iteration
    static constexpr int RING = 4;                // fragments read ahead
    enum { QK = 0, PV = 1, SUM = 2 };
    static constexpr int kind(int s) { return s < QKS ? QK : (s - QKS) % GS < NDB * QB ? PV : SUM; }
    // fragment of a QK / PV slot, block of any slot, group of a PV / SUM slot
    static constexpr int frag_of(int s) {
        return s < QKS ? s / QB : NKF + ((s - QKS) / GS) * NDB + ((s - QKS) % GS) / QB;
    }
    static constexpr int qb_of(int s) {
        return s < QKS ? s % QB : (s - QKS) % GS < NDB * QB ? ((s - QKS) % GS) % QB : ((s - QKS) % GS - NDB * QB) % QB;
    }
    static constexpr int sum_half(int s) { return ((s - QKS) % GS - NDB * QB) / QB; }   // SUM slots
    static constexpr int group_of(int s) { return (s - QKS) / GS; }
    // slot of fragment g's last-block MFMA, after which its ring entry is refilled
    static constexpr int last_slot(int g) {
        return g < NKF ? QB * g + QB - 1 : QKS + ((g - NKF) / NDB) * GS + ((g - NKF) % NDB) * QB + QB - 1;
    }
    // Barrier slot: the slot whose refill is the first read of a next-tile
    // fragment (fragment NF - RING).
    static constexpr int BARS = last_slot(NF - RING);
    static_assert(NF % RING == 0, "ring position must repeat every iteration");

    // Exponential pairs in the order the PV MFMAs read them: pair i covers
    // score registers 2 r2 and 2 r2 + 1 of block qb, key block kb; the PV
    // fragments (kb, c, *) read pairs 4c .. 4c+3 of (qb, kb).
    static constexpr int NP = 16 * QB;            // pairs per tile
    static constexpr int pair_c(int i) { return (i / (4 * QB)) & 1; }
    static constexpr int pair_kb(int i) { return i / (8 * QB); }
    static constexpr int pair_qb(int i) { return (i >> 2) % QB; }
    static constexpr int pair_r2(int i) { return 4 * pair_c(i) + (i & 3); }
    static constexpr int pair_need(int i) { return QKS + GS * (2 * pair_kb(i) + pair_c(i)); }

    // Exponential units, three per pair: A (first exp), B (second), C
    // (pack), in the stream A0 B0 A1 B1 C0 A2 B2 C1 ... A(NP-1) B(NP-1)
    // C(NP-2) C(NP-1), spread evenly over slots 0 .. ES-1. ES is the widest
    // spread (at most QKS + 3 GS - 2 QB - 1) that packs every pair a full slot
    // before the row-sum slots preceding its PV group (those are short 4x4x4
    // MFMAs); at head_dim 32 the groups are short and the spread narrows.
    static constexpr int NU = 3 * NP;
    static constexpr int c_unit(int i) { return i == NP - 1 ? NU - 1 : 3 * i + 4; }
    static constexpr bool packs_in_time(int es) {
        for (int i = 0; i < NP; ++i)
            if (c_unit(i) * es / NU > pair_need(i) - 2 * QB - 2) return false;
        return true;
    }
    static constexpr int widest_spread(int es) { return es <= 1 || packs_in_time(es) ? es : widest_spread(es - 1); }
    static constexpr int ES = widest_spread(QKS + 3 * GS - 2 * QB - 1);
    static constexpr int unit_slot(int n) { return n * ES / NU; }
    static constexpr int unit_first(int s) { return (s * NU + ES - 1) / ES; }   // first unit of slot s
    static constexpr int unit_kind(int n) { return n < 2 ? n : n == NU - 1 ? 2 : (n - 2) % 3; }
    static constexpr int unit_pair(int n) {
        return n < 2 ? 0 : n == NU - 1 ? NP - 1 : (n - 2) % 3 == 2 ? (n - 2) / 3 : (n - 2) / 3 + 1;
    }

    // Maxima of tile t+1: drain and mask at slot MS0, then 4 QB partial maxima
    // (qb, kb, half), the QB block maxima and the QB block updates.
    static constexpr int NMU = 6 * QB;
    static constexpr int MS0 = QKS + 2;
    static constexpr int max_slot(int k) { return MS0 + k * (NSLOT - 1 - MS0) / (NMU - 1); }

    // DMAs of the iteration, in the n slots right before the barrier (measured
    // ~1% faster than spreading them over the slots before it).
    static constexpr int dma_slot(int j, int n) { return BARS - n + j; }

    static constexpr bool valid() {
        for (int n = 0; n < NU; ++n)
            if (unit_slot(n) < 0 || unit_slot(n) >= ES || unit_first(unit_slot(n)) > n ||
                unit_first(unit_slot(n) + 1) <= n)
                return false;
        if (!packs_in_time(ES)) return false;
        // The block updates change the exponent offsets: after every exponential.
        if (max_slot(5 * QB) < ES) return false;
        if (max_slot(NMU - 1) != NSLOT - 1) return false;
        for (int s = 0; s < NSLOT; ++s)   // slot decoding is consistent
            if (kind(s) != SUM && last_slot(frag_of(s)) < s) return false;
        return BARS > QKS && kind(BARS) == PV;
    }
    static_assert(valid(), "slot schedule");
};

// QB 32-row query blocks per wave, NW waves per workgroup, 32 QB NW query
// rows per workgroup: (QB, NW) = (2, 4) is one wave of 64 rows per SIMD;
// (1, 8) two waves of 32 rows per SIMD, each running the same slot schedule,
// so that one wave issues while the other waits; (1, 4) the same two waves
// per SIMD from two workgroups of 128 rows on one CU (head_dim 64: 64 KiB of
// LDS each), which halves the work item for problems with few items.
template <typename T, int D, bool CAUSAL, int QB = 2, int NW = 4>
__global__ __launch_bounds__(64 * NW, (QB == 1 && NW == 4) ? 2 : 1)
__attribute__((amdgpu_waves_per_eu(QB == 1 ? 2 : NW / 4, QB == 1 ? 2 : NW / 4)))
void attn_fwd_w64_kernel(AttnParams p) {
    using E = Elt16<T>;
    using M = W64Mma<T>;
    using Sch = W64Sched<D, QB>;
    using frag = typename E::frag;
    constexpr int NT = 64 * NW;             // threads per workgroup
    constexpr int kBlockM = 32 * QB * NW;   // query rows per workgroup
    static_assert(kBlockM == 256 || (kBlockM == 128 && QB == 1), "work items are 256- or 128-row query tiles");
    constexpr int BN = 64;                  // keys per tile
    constexpr int CPR = D / 8;              // 16-byte chunks per row
    constexpr int TILE_CHUNKS = BN * CPR;   // chunks per K (or V) tile
    constexpr int LOADS = TILE_CHUNKS / NT;   // DMAs per thread per tensor per tile
    static_assert(Sch::BARS >= 2 * LOADS, "the DMAs of an iteration issue before its barrier");
    constexpr int TILE_BYTES = BN * D * (int)sizeof(T);
    constexpr int NDB = Sch::NDB, NDK = Sch::NDK, NKF = Sch::NKF, NF = Sch::NF;
    constexpr int NSLOT = Sch::NSLOT, RING = Sch::RING;
    static_assert(TILE_CHUNKS % NT == 0, "tile must split evenly over the workgroup's threads");

    // LDS slots: tile x of the stream (K and V) lives in slot x % NSL.  Four
    // slots, so that with NSL-aligned item lengths every item starts at slot
    // 0 and score set 0, and the unrolled loop below addresses the slots with
    // compile-time offsets.
    constexpr int NSL = 4;
    __shared__ __attribute__((aligned(1024))) T smem[2 * NSL][BN * D];   // K slots 0..NSL-1, V slots NSL..2 NSL-1
    const unsigned lds0 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) T *)smem[0];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = lane >> 5;
    const int col = lane & 31;

    const int S = p.S;
    const int n_items = p.n_qtiles * p.BH;
    // Work items (head bh, query tile qt) of this workgroup, one after the
    // other: round r takes item index r * G + c, c running forwards in even
    // rounds and backwards in odd ones.  Items come longest first, so the
    // causal work evens out over the workgroups.  With p.xcd_order the snake
    // runs over the workgroups of each XCD, keeping item index % 8 = XCD.
    const int G = gridDim.x;
    auto item_index = [&](int r) __attribute__((always_inline)) {
        const int wg = blockIdx.x;
        if (p.xcd_order && (G & 7) == 0) {
            const int C = G >> 3, c = wg >> 3;
            return 8 * (r * C + ((r & 1) ? C - 1 - c : c)) + (wg & 7);
        }
        return r * G + ((r & 1) ? G - 1 - wg : wg);
    };
    auto item_tiles = [&](int qt_) __attribute__((always_inline)) {
        const int last_key = CAUSAL ? min(qt_ * kBlockM + kBlockM - 1, S - 1) : S - 1;
        return last_key / BN + 1;   // key tiles of the item
    };

    // Current item.
    int bh = 0, qt = 0, q0w = 0, nt = 1, npos = NSL, ntw = 0;
    bool wave_active = false;
    const T *kg = nullptr, *vg = nullptr;
    // Next item: its first tiles are loaded during the current item's last
    // iterations.
    bool has_next = false;
    int nt_n = 1, bh_nx = 0, q0w_nx = 0;   // next item: tiles, head, first row of the wave
    const T *kg_n = nullptr, *vg_n = nullptr;
    auto head_ptrs = [&](int bh_, const T *&kp, const T *&vp) __attribute__((always_inline)) {
        const int b_ = bh_ / p.H, h_ = bh_ - b_ * p.H;
        kp = (const T *)p.k + b_ * p.k_sb + h_ * p.k_sh;
        vp = (const T *)p.v + b_ * p.v_sb + h_ * p.v_sh;
    };
    // Rows of the wave within the item.  With two waves per SIMD (waves w and
    // w + 4 share a SIMD), wave w < 4 takes rows 32 w and wave w >= 4 rows
    // 32 (11 - w), so each SIMD holds one block of the upper and one of the
    // lower half of the tile and the SIMDs see equal causal work.
    const int wave_row = NW == 4 ? 32 * QB * wave : 32 * (wave < 4 ? wave : 11 - wave);
    auto set_item = [&](int L) __attribute__((always_inline)) {
        map_index<CAUSAL>(p, L, bh, qt);
        q0w = qt * kBlockM + wave_row;    // first row of the wave
        nt = item_tiles(qt);
        npos = (nt + NSL - 1) & ~(NSL - 1);   // stream positions of the item, run by every wave
        wave_active = q0w < S;
        // Tiles this wave computes: 0 .. ntw-1; only tile ntw-1 can hold keys
        // past a row of the wave (causal diagonal) or past S.
        ntw = !wave_active ? 0 : CAUSAL ? min(nt, (q0w + 32 * QB - 1) / BN + 1) : nt;
        head_ptrs(bh, kg, vg);
    };
    auto set_next = [&](int L) __attribute__((always_inline)) {
        has_next = L < n_items;
        if (has_next) {
            int qt_n;
            map_index<CAUSAL>(p, L, bh_nx, qt_n);
            nt_n = item_tiles(qt_n);
            q0w_nx = qt_n * kBlockM + wave_row;
            head_ptrs(bh_nx, kg_n, vg_n);
        }
    };

    // Q fragments of the current item (B operand of S^T = K Q^T, AGPRs):
    // block qb, lane holds Q[q0w + 32 qb + col][16 dk + 8 hi .. +7].
    frag qf[QB][NDK];
    auto load_q_of = [&](int bh_q, int q0w_q) __attribute__((always_inline)) {
        const int b_ = bh_q / p.H, h_ = bh_q - b_ * p.H;
        const T *qg = (const T *)p.q + b_ * p.q_sb + h_ * p.q_sh;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const int qrow = min(q0w_q + 32 * qb + col, S - 1);
            const T *src = qg + (int64_t)qrow * p.q_ss + 8 * hi;
#pragma unroll
            for (int dk = 0; dk < NDK; ++dk)
                qf[qb][dk] = __builtin_bit_cast(frag, *(const u32x4_t *)(src + 16 * dk));
        }
    };
    // Q defined in AGPRs, where the QK MFMAs read them (otherwise the register
    // allocator may keep them in VGPRs and copy before each use).  The pin
    // waits for the loads, so it sits after the previous item's O stores:
    // the load latency overlaps them.
    auto load_q = [&]() __attribute__((always_inline)) { load_q_of(bh, q0w); };
    auto pin_q = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int dk = 0; dk < NDK; ++dk) asm volatile("" : "+a"(qf[qb][dk]));
    };

    // ---- DMA staging: lane `lane` of wave `wave` fills chunk slot
    // j*NT + 64*wave + lane, i.e. LDS bytes slot_base + 16 NT j + 1024 wave
    // + 16 lane, with the logical chunk the XOR swizzle places there.
    int koff[LOADS], voff[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const int sl = j * NT + tid;
        const int row = sl / CPR;
        const int pc = sl % CPR;
        koff[j] = (int)((row * p.k_ss + 8 * (pc ^ swz_k<CPR>(row))) * (int64_t)sizeof(T));
        voff[j] = (int)((row * p.v_ss + 8 * (pc ^ swz_v<CPR>(row))) * (int64_t)sizeof(T));
    }
    // Buffer resource of one head's K or V, from key 0 to the last key of
    // the sequence: rows past S read as zero (those keys are masked).  The
    // host keeps (S - 1) * stride + D elements within 2^31 bytes.
    const int k_records = (int)(((S - 1) * p.k_ss + D) * sizeof(T));
    const int v_records = (int)(((S - 1) * p.v_ss + D) * sizeof(T));
    const int k_tile_bytes = (int)(BN * p.k_ss * sizeof(T));
    const int v_tile_bytes = (int)(BN * p.v_ss * sizeof(T));
    const unsigned lds_w = lds0 + (unsigned)(wave * 1024);
    // The K and V streams run one tile per stream position: position kt of
    // an item is its tile min(kt, nt - 1) (copies past the last tile are never
    // read), and positions npos, npos + 1, ... are the next item's tiles 0, 1,
    // ...  Each stream keeps its source as it goes: the buffer resource of the
    // head its next tile comes from, the tile's byte offset (the DMAs'
    // soffset) and the offset of that head's last tile of the item.  A stream
    // moves to the next item's head after its DMAs of position npos - 1
    // (sw_at = npos with a next item; never without).
    __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(nullptr, (short)0, 0, 0x00020000);
    __amdgpu_buffer_rsrc_t vrs = krs;
    int kso = 0, vso = 0, klast = 0, vlast = 0, sw_at = -1;
    auto stream_start = [&]() __attribute__((always_inline)) {
        krs = __builtin_amdgcn_make_buffer_rsrc((void *)kg, (short)0, k_records, 0x00020000);
        vrs = __builtin_amdgcn_make_buffer_rsrc((void *)vg, (short)0, v_records, 0x00020000);
        kso = vso = 0;
        klast = (nt - 1) * k_tile_bytes;
        vlast = (nt - 1) * v_tile_bytes;
    };
    // after the K (V) DMAs of position kt: move on to position kt + 1
    auto next_k = [&](int kt, bool may_switch) __attribute__((always_inline)) {
        if (may_switch && __builtin_expect(kt + 1 == sw_at, 0)) {
            krs = __builtin_amdgcn_make_buffer_rsrc((void *)kg_n, (short)0, k_records, 0x00020000);
            kso = 0;
            klast = (nt_n - 1) * k_tile_bytes;
        } else {
            kso = min(kso + k_tile_bytes, klast);
        }
    };
    auto next_v = [&](int kt, bool may_switch) __attribute__((always_inline)) {
        if (may_switch && __builtin_expect(kt + 1 == sw_at, 0)) {
            vrs = __builtin_amdgcn_make_buffer_rsrc((void *)vg_n, (short)0, v_records, 0x00020000);
            vso = 0;
            vlast = (nt_n - 1) * v_tile_bytes;
        } else {
            vso = min(vso + v_tile_bytes, vlast);
        }
    };
    // DMA j of the stream's current tile into LDS slot SL (= kt % NSL).
    auto dma_k = [&](auto sl_c, auto j_c) __attribute__((always_inline)) {
        constexpr int SL = decltype(sl_c)::value, J = decltype(j_c)::value;
        w64_lds_dma16<SL * TILE_BYTES + J * 16 * NT>(krs, koff[J], kso, lds_w);
    };
    auto dma_v = [&](auto sl_c, auto j_c) __attribute__((always_inline)) {
        constexpr int SL = decltype(sl_c)::value, J = decltype(j_c)::value;
        w64_lds_dma16<(NSL + SL) * TILE_BYTES + J * 16 * NT>(vrs, voff[J], vso, lds_w);
    };
    // DMA i of position t: K(t+3) into slot (t+3) % NSL (slk), then V(t+2)
    // into slot (t+2) % NSL (slv).  The slots hold K(t-1) and V(t-2), last
    // read before the previous position's barrier.  npos is a multiple of
    // NSL, so the K stream can only switch at positions t = 0 (mod NSL) and
    // the V stream at t = 1 (mod NSL): PH (t mod NSL, or -1 when not known at
    // compile time) skips the test elsewhere.
    // Slots as compile-time constants: SLK = (t + 3) % NSL, SLV = (t + 2) % NSL.
    auto dma_step_c = [&](int t, auto slk_c, auto slv_c, auto i_c, auto ph_c) __attribute__((always_inline)) {
        constexpr int PH = decltype(ph_c)::value, I = decltype(i_c)::value;
        if constexpr (I < LOADS) {
            dma_k(slk_c, std::integral_constant<int, I>{});
            if constexpr (I == LOADS - 1) next_k(t + 3, PH < 0 || PH == 0);
        } else {
            dma_v(slv_c, std::integral_constant<int, I - LOADS>{});
            if constexpr (I == 2 * LOADS - 1) next_v(t + 2, PH < 0 || PH == 1);
        }
    };
    // All DMAs of position t, the slots known at run time only (t mod NSL).
    auto dma_position = [&](int t) __attribute__((always_inline)) {
        w64_static_for<0, NSL>([&](auto ph_c) __attribute__((always_inline)) {
            constexpr int PH = decltype(ph_c)::value;
            if ((t & (NSL - 1)) == PH)
                w64_static_for<0, 2 * LOADS>([&](auto i_c) __attribute__((always_inline)) {
                    dma_step_c(t, std::integral_constant<int, (PH + 3) % NSL>{},
                               std::integral_constant<int, (PH + 2) % NSL>{}, i_c, std::integral_constant<int, -1>{});
                });
        });
    };
    // Barrier placement.  Head_dim 128 (and 32): one barrier per stream
    // position, at BARS, waiting until only the position's own DMAs (2 LOADS,
    // issued in the slots right before it) may be in flight.  Head_dim 64
    // (PAIR): one barrier per two positions, at the odd ones; position t
    // issues its DMAs (K(t+3) into K(t-1)'s slot, V(t+2) into V(t-2)'s) in
    // its first slots, both read before the last barrier, and each barrier
    // waits for all of them (measured 2.8% faster at C2, 1.1% slower at C3).
    // Either way a tile is read only after a barrier that follows its DMA.
    constexpr bool PAIR = D == 64;
    auto sync_tiles = [&]() __attribute__((always_inline)) {
        if constexpr (PAIR)
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        else
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(2 * LOADS) : "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    // Softmax state of the current item (reset per item).
    f32x16_t acc[QB][NDB];     // O^T accumulators, AGPRs
    f32x16_t sc[2][QB][2];     // [set][qb][kb] scores; tile t uses set t & 1
    uint32_t pk[QB][2][8];     // [qb][kb][pair] probabilities of the tile in PV
    float pe[2][2];            // exponentials of a pair until packed, by pair parity
    float m_true[QB], m_use[QB];
    float moff[QB];            // -m_use * scale_log2 (0 while m_use is -inf)
    float alpha[QB];
    bool rescale[QB];
    // Row sums: 4x4x4 MFMAs of an all-ones A operand with the packed
    // probabilities add each lane's own rounded P to every register of its
    // lsum (AGPRs; the two lane halves are combined at the end), so O is
    // normalised by exactly the weights the PV product used, and the sums cost
    // no vector instructions.  One accumulator per (block, half of a group's
    // P): the row-sum MFMAs of a group run back to back, and a 4x4x4 result
    // is not ready for the SrcC read of the very next MFMA; on one
    // accumulator they are a whole group apart.
    using half_frag = typename M::half_frag;
    f32x4_t lsum[QB][2];
    half_frag ones;
#pragma unroll
    for (int i = 0; i < 4; ++i) ones[i] = (T)1.0f;
    // Opaque from here on: kept in four VGPRs instead of being rebuilt from
    // SGPRs by VALU moves right before each MFMA that reads it (the MFMAs
    // are inline asm, so the compiler inserts no wait states for them).
    asm volatile("" : "+v"(ones));
    const float lazy_raw = p.lazy_raw;
    auto reset_state = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[qb][db][r] = 0.f;
            m_true[qb] = m_use[qb] = -INFINITY;
            moff[qb] = 0.f;
            alpha[qb] = 1.f;
            rescale[qb] = false;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r) lsum[qb][h][r] = 0.f;
        }
    };

    const int arow = key_of_arow(col);
    const int g16 = lane >> 4, tt = lane & 15;
    const int vrow0 = 16 * (g16 >> 1) + (tt >> 2);
    const int vcol0 = 16 * (g16 & 1) + 4 * (tt & 3);
    const uint32_t krow_off = (uint32_t)(arow * D * sizeof(T));
    const uint32_t kx16 = (uint32_t)((hi ^ swz_k<CPR>(arow)) * 16);
    typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
    typedef __attribute__((address_space(3))) u32x4_t lds_u32x4;
    typedef short s16x8_t __attribute__((ext_vector_type(8)));

    // Lane part of the LDS byte address of K fragment (dk, *): row
    // key_of_arow(col), 16-byte chunk 2 dk + hi through the swizzle.
    uint32_t kaddr[NDK];
#pragma unroll
    for (int dk = 0; dk < NDK; ++dk) kaddr[dk] = krow_off + (((uint32_t)(32 * dk)) ^ kx16);
    // K fragment f = (dk, kb) = (f >> 1, f & 1) of the tile in the LDS slot
    // starting at byte kslot_b.
    auto kfrag = [&](uint32_t kslot_b, int f) __attribute__((always_inline)) {
        const int dk = f >> 1, kb = f & 1;
        const uint32_t addr = kaddr[dk] + kslot_b + (uint32_t)(kb * 32 * D * sizeof(T));
        return __builtin_bit_cast(frag, *(const lds_u32x4 *)(uintptr_t)addr);
    };
    // V^T fragment f = (kb, c, db): 32 head-dim columns x 16 keys.
    auto vfrag = [&](const T *Vs, int f) __attribute__((always_inline)) {
        const int kb = f / (2 * NDB), c = (f / NDB) % 2, db = f % NDB;
        const int r0 = 32 * kb + 8 * c + vrow0;
        const int cc = 32 * db + vcol0;
        const int ch = cc >> 3, part = cc & 7;
        const T *a0 = Vs + r0 * D + 8 * (ch ^ swz_v<CPR>(r0)) + part;
        const T *a1 = Vs + (r0 + 4) * D + 8 * (ch ^ swz_v<CPR>(r0 + 4)) + part;
        s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)a0);
        s16x4_t hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)a1);
        return __builtin_bit_cast(frag, s16x8_t{lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]});
    };
    auto k_slot_base = [&](int sl) __attribute__((always_inline)) { return lds0 + (uint32_t)(sl * TILE_BYTES); };

    // ---- softmax pieces ----
    // Mask of tile kt (score set SET): tile ntw-1 against the diagonal / S,
    // later tiles entirely (a fully masked tile changes nothing).
    auto sm_mask = [&](int kt, auto set_c) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value;
        if (__builtin_expect(kt >= ntw - 1, 0)) {
            const int kbase = kt * BN;
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                const int qi = q0w + 32 * qb + col;
                const int lim = kt == ntw - 1 ? (CAUSAL ? min(qi, S - 1) : S - 1) : -1;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    // register r holds key kbase + 32 kb + 16 hi + r: kept iff r <= d
                    const int d = lim - (kbase + 32 * kb + 16 * hi);
                    w64_static_for<0, 16>([&](auto r_c) __attribute__((always_inline)) {
                        constexpr int r = decltype(r_c)::value;
                        sc[SET][qb][kb][r] = w64_mask_key<r>(sc[SET][qb][kb][r], d);
                    });
                }
            }
        }
    };
    float mx[QB];
    bool upv[QB];
    // Max unit k of score set SET: k < 4 QB partial row max (qb, kb, half) of
    // the lane's own keys; k in [4 QB, 5 QB) for block k - 4 QB the lane's
    // running max (m_true holds each lane's half of a row; the two halves
    // are combined once per item, in the epilogue) and whether its tile max
    // passes the lazy threshold; k in [5 QB, 6 QB) the rescale decision for
    // block k - 5 QB (a wave-uniform branch, taken rarely): the row max over
    // both lane halves, the new offset and the factor for O and l (the O
    // rescale itself waits for the PV MFMAs in flight).  Split so that no
    // dependency chain stalls the in-order issue for long.
    auto max_unit = [&](auto set_c, int k) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value;
        if (k < 4 * QB) {
            const int qb = k >> 2, kb = (k >> 1) & 1, r0 = 8 * (k & 1);
            const auto &sv = sc[SET][qb][kb];
            float m;
            // Each unit is one asm block: the compiler puts a wait state after
            // every inline-asm VALU instruction whose result the next one
            // reads (it cannot rule out a transcendental), so a chain of
            // separate statements would carry one s_nop per step.
            if ((k & 3) == 0) {   // first unit of the block: 8 values, 4 instructions
                asm("v_max3_f32 %0, %1, %2, %3\n\tv_max3_f32 %0, %0, %4, %5\n\t"
                    "v_max3_f32 %0, %0, %6, %7\n\tv_max_f32 %0, %0, %8"
                    : "=&v"(m)
                    : "v"(sv[r0]), "v"(sv[r0 + 1]), "v"(sv[r0 + 2]), "v"(sv[r0 + 3]), "v"(sv[r0 + 4]),
                      "v"(sv[r0 + 5]), "v"(sv[r0 + 6]), "v"(sv[r0 + 7]));
            } else {
                m = mx[qb];
                asm("v_max3_f32 %0, %0, %1, %2\n\tv_max3_f32 %0, %0, %3, %4\n\t"
                    "v_max3_f32 %0, %0, %5, %6\n\tv_max3_f32 %0, %0, %7, %8"
                    : "+v"(m)
                    : "v"(sv[r0]), "v"(sv[r0 + 1]), "v"(sv[r0 + 2]), "v"(sv[r0 + 3]), "v"(sv[r0 + 4]),
                      "v"(sv[r0 + 5]), "v"(sv[r0 + 6]), "v"(sv[r0 + 7]));
            }
            asm volatile("" : "+v"(m));
            mx[qb] = m;
        } else if (k < 5 * QB) {
            const int qb = k - 4 * QB;
            m_true[qb] = w64_max(m_true[qb], mx[qb]);
            upv[qb] = mx[qb] > m_use[qb] + lazy_raw;
        } else {
            const int qb = k - 5 * QB;
            if (__builtin_amdgcn_ballot_w64(upv[qb]) != 0) {
                const float mh = half_max(mx[qb]);
                const float m_new = fmaxf(m_use[qb], mh);
                alpha[qb] = fast_exp2((m_use[qb] - m_new) * p.scale_log2);   // 0 on the first tile
                moff[qb] = m_new == -INFINITY ? 0.f : -m_new * p.scale_log2;
                m_use[qb] = m_new;
                rescale[qb] = true;
            }
        }
    };
    // The O^T accumulators and row sums of block qb at a drain.
    auto fence_block = [&](int qb) __attribute__((always_inline)) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) w64_fence_a(acc[qb][db]);
        w64_fence_a(lsum[qb][0]);
        w64_fence_a(lsum[qb][1]);
    };
    auto apply_rescale = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
            if (__builtin_expect(rescale[qb], 0)) {
                w64_mfma_drain();
                fence_block(qb);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    lsum[qb][0][r] *= alpha[qb];
                    lsum[qb][1][r] *= alpha[qb];
                }
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[qb][db][r] *= alpha[qb];
                fence_block(qb);
                w64_mfma_drain();
                rescale[qb] = false;
            }
    };
    // Exponential unit n of score set SET (see W64Sched).  Every result is
    // pinned where it is computed: without a use there, IR-level sinking
    // moves the work next to the PV MFMAs that consume P, in one clump.
    auto exp_unit = [&](auto set_c, auto n_c) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value;
        constexpr int n = decltype(n_c)::value;
        constexpr int kind = Sch::unit_kind(n), i = Sch::unit_pair(n);
        constexpr int qb = Sch::pair_qb(i), kb = Sch::pair_kb(i), r = 2 * Sch::pair_r2(i);
        if constexpr (kind < 2) {
            pe[i & 1][kind] = fast_exp2(__builtin_fmaf(sc[SET][qb][kb][r + kind], p.scale_log2, moff[qb]));
            asm volatile("" : "+v"(pe[i & 1][kind]));
        } else {
            pk[qb][kb][r >> 1] = E::pack2(pe[i & 1][0], pe[i & 1][1]);
            asm volatile("" : "+v"(pk[qb][kb][r >> 1]));
        }
    };

    frag ring[RING];
    // Iteration t (PH = t % NSL, tile scores in set SET = t & 1): QK of tile
    // t+1 into set SET ^ 1 and PV of tile t, with the VALU work of the
    // schedule.  LDS slots, compile-time: V(t) in PH, K(t+1) in PH + 1, K(t+2)
    // (the next iteration's first fragments) in PH + 2 (mod NSL).
    auto iteration = [&](int t, auto ph_c) __attribute__((always_inline)) {
        constexpr int PH = decltype(ph_c)::value;
        constexpr int SET = PH & 1;
        constexpr int SL0 = PH, SL1 = (PH + 1) % NSL, SL2 = (PH + 2) % NSL, SL3 = (PH + 3) % NSL;
        using NSET = std::integral_constant<int, SET ^ 1>;
        using CSET = std::integral_constant<int, SET>;
        const uint32_t kcur = k_slot_base(SL1);
        const uint32_t knext = k_slot_base(SL2);
        const T *Vs = smem[NSL + SL0];
        w64_static_for<0, NSLOT>([&](auto s_c) __attribute__((always_inline)) {
            constexpr int s = decltype(s_c)::value;
            constexpr int kd = Sch::kind(s), qb = Sch::qb_of(s);
            constexpr int g = kd == Sch::SUM ? 0 : Sch::frag_of(s);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (kd == Sch::QK) {
                constexpr int dk = g >> 1, kb = g & 1;
                if constexpr (dk == 0) M::qk0(sc[SET ^ 1][qb][kb], ring[g % RING], qf[qb][0]);
                else M::qk(sc[SET ^ 1][qb][kb], ring[g % RING], qf[qb][dk]);
            } else if constexpr (kd == Sch::PV) {
                constexpr int f = g - NKF;
                constexpr int kb = f / (2 * NDB), c = (f / NDB) % 2, db = f % NDB;
                u32x4_t bw = {pk[qb][kb][4 * c], pk[qb][kb][4 * c + 1], pk[qb][kb][4 * c + 2], pk[qb][kb][4 * c + 3]};
                M::pv(acc[qb][db], ring[g % RING], __builtin_bit_cast(frag, bw));
            } else {
                constexpr int grp = Sch::group_of(s), kb = grp >> 1, c = grp & 1, h = Sch::sum_half(s);
                u32x2_t bw = {pk[qb][kb][4 * c + 2 * h], pk[qb][kb][4 * c + 2 * h + 1]};
                M::sum4(lsum[qb][h], ones, __builtin_bit_cast(half_frag, bw));
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (s == Sch::BARS && (!PAIR || (PH & 1))) sync_tiles();
            if constexpr (kd != Sch::SUM && qb == QB - 1) {   // fragment g is done: refill its ring entry
                constexpr int gn = g + RING;
                if constexpr (gn < NKF) ring[g % RING] = kfrag(kcur, gn);
                else if constexpr (gn < NF) ring[g % RING] = vfrag(Vs, gn - NKF);
                else ring[g % RING] = kfrag(knext, gn - NF);
            }
            w64_static_for<0, 2 * LOADS>([&](auto j_c) __attribute__((always_inline)) {
                constexpr int j = decltype(j_c)::value;
                if constexpr ((PAIR ? j + 1 : Sch::dma_slot(j, 2 * LOADS)) == s)
                    dma_step_c(t, std::integral_constant<int, SL3>{}, std::integral_constant<int, SL2>{}, j_c,
                               std::integral_constant<int, PH>{});
            });
            if constexpr (s == Sch::MS0) {
                w64_mfma_drain();   // the QK MFMAs of tile t+1 have written the scores
#pragma unroll
                for (int qb = 0; qb < QB; ++qb)
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb) w64_fence_v(sc[SET ^ 1][qb][kb]);
                sm_mask(t + 1, NSET{});
            }
            if constexpr (s < Sch::ES)
                w64_static_for<Sch::unit_first(s), Sch::unit_first(s + 1)>(
                    [&](auto n_c) __attribute__((always_inline)) { exp_unit(CSET{}, n_c); });
            w64_static_for<0, Sch::NMU>([&](auto k_c) __attribute__((always_inline)) {
                constexpr int k = decltype(k_c)::value;
                if constexpr (Sch::max_slot(k) == s) max_unit(NSET{}, k);
            });
            __builtin_amdgcn_sched_barrier(0);
        });
        apply_rescale();   // decided for tile t+1; the PV MFMAs of tile t are issued
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;

    // Epilogue of an item: normalise, store O, m, l.  In the O^T accumulator
    // lane (col, hi) holds dims 32 db + 8 g4 + 4 hi + 0..3 of query row col;
    // one v_permlane32_swap per packed pair hands lane col the partner's
    // dims +4..7 of g4 = 2j and lane col + 32 lane col's dims +8..11 of
    // g4 = 2j + 1, so each lane stores 8 consecutive dims (16 bytes) and a
    // row's 32-byte piece is written by two lanes of one store instruction.
    auto store_item = [&](int bh_e, int q0w_e, bool active_e) __attribute__((always_inline)) {
        const int b_ = bh_e / p.H, h_ = bh_e - b_ * p.H;
        T *og = (T *)p.o + b_ * p.o_sb + h_ * p.o_sh;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const float l_sum = half_sum(lsum[qb][0][0] + lsum[qb][1][0]);   // relative to m_use
            const int qi = q0w_e + 32 * qb + col;
            const bool ok = active_e && qi < S;
            const float inv = 1.0f / l_sum;                    // not stored where !ok
            T *orow = og + (int64_t)(ok ? qi : 0) * p.o_ss;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const f32x16_t &c = acc[qb][db];
                    const uint32_t a0 = E::pack2(c[8 * j] * inv, c[8 * j + 1] * inv);
                    const uint32_t a1 = E::pack2(c[8 * j + 2] * inv, c[8 * j + 3] * inv);
                    const uint32_t b0 = E::pack2(c[8 * j + 4] * inv, c[8 * j + 5] * inv);
                    const uint32_t b1 = E::pack2(c[8 * j + 6] * inv, c[8 * j + 7] * inv);
                    const auto r0 = __builtin_amdgcn_permlane32_swap(a0, b0, false, false);
                    const auto r1 = __builtin_amdgcn_permlane32_swap(a1, b1, false, false);
                    const u32x4_t w4 = {r0[0], r1[0], r0[1], r1[1]};
                    if (ok) *(u32x4_t *)(orow + 32 * db + 16 * j + 8 * hi) = w4;
                }
            const float m_row = half_max(m_true[qb]);   // both lane halves of the row
            if (ok) {
                const float l_tot = l_sum * fast_exp2((m_use[qb] - m_row) * p.scale_log2);
                if (hi == 0) {
                    const int64_t mi = (int64_t)bh_e * S + qi;
                    const float mval = m_row * p.scale;
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
    };

    // ---- first item: K(0), V(0), K(1) landed; K(2), V(1) in flight ----
    int r = 0;
    if (item_index(0) >= n_items) return;   // (the host launches at most n_items workgroups)
    set_item(item_index(0));
    set_next(item_index(1));
    load_q();
    stream_start();
    sw_at = has_next ? npos : -1;
    // K(0), V(0), K(1), K(2), V(1) (npos >= NSL = 4: no stream switches here)
    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, 1>;
    using C2 = std::integral_constant<int, 2>;
    w64_static_for<0, LOADS>([&](auto j_c) __attribute__((always_inline)) { dma_k(C0{}, j_c); });
    next_k(0, false);
    w64_static_for<0, LOADS>([&](auto j_c) __attribute__((always_inline)) { dma_v(C0{}, j_c); });
    next_v(0, false);
    w64_static_for<0, LOADS>([&](auto j_c) __attribute__((always_inline)) { dma_k(C1{}, j_c); });
    next_k(1, false);
    w64_static_for<0, LOADS>([&](auto j_c) __attribute__((always_inline)) { dma_k(C2{}, j_c); });
    next_k(2, false);
    w64_static_for<0, LOADS>([&](auto j_c) __attribute__((always_inline)) { dma_v(C1{}, j_c); });
    next_v(1, false);
    sync_tiles();

    // Outputs of the previous item (its O, row sums and maxima stay in acc,
    // lsum, m_true, m_use until written): stored under the next item's first
    // score MFMAs, after the wait for that item's Q, so neither the stores
    // nor their normalisation hold up the item start.
    bool have_prev = false, active_p = false;
    int bh_p = 0, q0w_p = 0;
    while (true) {
        pin_q();
        // Scores and maxima of tile 0 (slot 0; landed, see above).
        {
            const uint32_t k0 = k_slot_base(0);
#pragma unroll
            for (int f = 0; f < NKF; ++f) {
                const frag a = kfrag(k0, f);
                const int dk = f >> 1, kb = f & 1;
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    if (dk == 0) M::qk0(sc[0][qb][kb], a, qf[qb][0]);
                    else M::qk(sc[0][qb][kb], a, qf[qb][dk]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (have_prev) store_item(bh_p, q0w_p, active_p);
            reset_state();
            __builtin_amdgcn_sched_barrier(0);
            w64_mfma_drain();
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) w64_fence_v(sc[0][qb][kb]);
            sm_mask(0, S0{});
#pragma unroll
            for (int k = 0; k < Sch::NMU; ++k) max_unit(S0{}, k);
            // Tile 0 always passes the rescale test (m_use was -inf), but O
            // and the row sums were just zeroed: nothing to scale (the
            // multiply by alpha = 0 cost ~200 vector instructions per wave
            // and item, AGPR reads and writes included).
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) rescale[qb] = false;
        }
        // No barrier here with a barrier per position: iteration 0 refills
        // slots 3 and 2 (K(3), V(2)), free since the previous item's last
        // barrier, and K(0), V(0), K(1) landed before it.  (So the epilogue's
        // O stores are not waited for until iteration 0's barrier.)  With one
        // per two positions, position 1 fills K(4) into K(0)'s slot before
        // any barrier of this item, while K(0) was read above, outside the
        // iterations: every wave must be past that first.
        if constexpr (PAIR) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        }
        {
            const uint32_t k1 = k_slot_base(1);
#pragma unroll
            for (int f = 0; f < RING; ++f) ring[f] = kfrag(k1, f);
        }

        // ---- tiles the wave computes, NSL per loop iteration (phases 0..3:
        // score sets 0, 1, 0, 1 and the LDS slots as compile-time offsets) ----
        int t = 0;
        while (t < ntw) {
            iteration(t, std::integral_constant<int, 0>{});
            if (++t == ntw) break;
            iteration(t, std::integral_constant<int, 1>{});
            if (++t == ntw) break;
            iteration(t, std::integral_constant<int, 2>{});
            if (++t == ntw) break;
            iteration(t, std::integral_constant<int, 3>{});
            ++t;
        }
        // A wave with DMA-only positions left no longer reads Q: the next
        // item's Q loads go out now and land under those positions.
        const bool q_early = has_next && t < npos;
        if (q_early) load_q_of(bh_nx, q0w_nx);
        // ---- remaining positions of the item: DMAs and barriers only ----
        for (; t < npos; ++t) {
            dma_position(t);
            if (!PAIR || (t & 1)) sync_tiles();
        }
        w64_mfma_drain();   // the last PV MFMAs have written O
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) fence_block(qb);

        // Next item (its Q loads land under the DMA-only positions or the
        // next loop head); this item's outputs go out there, or now after the
        // last item.
        const int bh_e = bh, q0w_e = q0w;
        const bool active_e = wave_active, more = has_next;
        if (more) {
            ++r;
            set_item(item_index(r));
            set_next(item_index(r + 1));
            sw_at = has_next ? npos : -1;
            if (!q_early) load_q();
        }
        if (!more) {
            store_item(bh_e, q0w_e, active_e);
            break;
        }
        have_prev = true;
        bh_p = bh_e;
        q0w_p = q0w_e;
        active_p = active_e;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // no DMA outlives the workgroup
}

}  // namespace pmkl_amd
