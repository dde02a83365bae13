// C ABI of the gfx950 fused causal self-attention forward (include/pmkl_attn.h).
//
// Host side of the path: argument validation, kernel selection and launch.
// It replaces the reference launcher pmkl::nlp::causal_attention_forward
// (pmkl/nlp/causal_attention.h:258-288), which checks S % 32 and the shared
// memory size with CHECK_FAIL and submits one lambda through the CUDA/SYCL
// GpuLauncher singleton (pmkl/core/launcher/cuda_launcher.h:297-335).  Here a
// named __global__ kernel is launched directly on the caller's stream, launch
// errors are checked (the reference never calls cudaGetLastError), and errors
// come back as status codes with thread-local text instead of exceptions.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <atomic>
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <utility>

#include "pmkl_attn.h"
#include "capi_common.hpp"
#include "attn_fwd_kernels.hpp"
#include "attn_fwd_w64.hpp"
#include "attn_bwd_kernels.hpp"
#include "attn_bwd_f32.hpp"

// The 64-row forward kernels are instantiated in attn_fwd_w64_<dtype>_<mask>.hip
// (one translation unit each, compiled in parallel).
namespace pmkl_amd {
#define PMKL_W64_EXTERN(T, C)                                                            \
    extern template __global__ void attn_fwd_w64_kernel<T, 64, C, 1, 8>(AttnParams);  \
    extern template __global__ void attn_fwd_w64_kernel<T, 128, C, 1, 8>(AttnParams); \
    extern template __global__ void attn_fwd_w64_kernel<T, 32, C, 2, 4>(AttnParams);  \
    extern template __global__ void attn_fwd_w64_kernel<T, 64, C, 2, 4>(AttnParams);  \
    extern template __global__ void attn_fwd_w64_kernel<T, 128, C, 2, 4>(AttnParams);
PMKL_W64_EXTERN(__bf16, true)
PMKL_W64_EXTERN(__bf16, false)
PMKL_W64_EXTERN(_Float16, true)
PMKL_W64_EXTERN(_Float16, false)
#undef PMKL_W64_EXTERN
extern template __global__ void attn_fwd_w64_kernel<__bf16, 64, true, 1, 4>(AttnParams);
extern template __global__ void attn_fwd_w64_kernel<_Float16, 64, true, 1, 4>(AttnParams);
}  // namespace pmkl_amd

namespace {

using pmkl_capi::dtype_size;
using pmkl_capi::dtype_valid;

bool head_dim_supported(int64_t d) { return d == 32 || d == 64 || d == 128; }

using pmkl_amd::AttnParams;
typedef void (*kernel_fn)(AttnParams);

// A kernel and its launch shape: threads per workgroup and query rows per
// workgroup; family and t1, t2 (its template parameters after the mask, -1
// if none) name it for pmkl_attn_fwd_kernel_name.
struct KernelChoice {
    kernel_fn fn;
    int threads;
    int block_m;
    int per_cu = 1;   // persistent workgroups per CU (64-row kernel)
    const char *family = "";
    int t1 = -1, t2 = -1;
};

// PMKL_ATTN_WAVES=4 or 8 pins the waves of the 16-bit MFMA kernel; 0 if unset.
int waves16_env() {
    static const int w = [] {
        const char *e = getenv("PMKL_ATTN_WAVES");
        return e ? (atoi(e) == 4 ? 4 : 8) : 0;
    }();
    return w;
}

// Waves of the 16-bit MFMA kernel where the 64-row kernel is not used:
// measured per shape, 4 waves (128-row workgroups, finer causal load
// balance) for causal head_dim 64 at 512 < S <= 2048, else 8.
int waves16(int64_t D, int64_t S, bool causal) {
    if (const int e = waves16_env()) return e;
    return (causal && D == 64 && S > 512 && S <= 2048) ? 4 : 8;
}

template <typename T, int D, int NW, int NTR = 0>
KernelChoice pick16w(bool causal) {
    return {causal ? (kernel_fn)pmkl_amd::attn_fwd_mfma16_kernel<T, D, true, NW, NTR>
                   : (kernel_fn)pmkl_amd::attn_fwd_mfma16_kernel<T, D, false, NW, NTR>,
            NW * 64, NW * 32, 1, "attn_fwd_mfma16_kernel", NW, NTR};
}
// Key tiles (of 64) the resident form of the 8-wave kernel holds in LDS:
// NTR * 2 * 64 * D * 2 bytes, 32 KiB at head_dim 32, 64 KiB at 64 and 128.
constexpr int resident_tiles(int64_t D) { return D == 128 ? 2 : 4; }

// Resident form (all key tiles loaded at once, no barrier per tile) for
// sequences of at most resident_tiles(D) key tiles, unless
// PMKL_ATTN_RESIDENT=0 (read once).
bool resident_enabled() {
    static const bool on = [] {
        const char *e = getenv("PMKL_ATTN_RESIDENT");
        return !(e && atoi(e) == 0);
    }();
    return on;
}
// 64-row kernel choice: PMKL_ATTN_W64=0 never, =1 wherever it applies,
// unset: for head_dim 128, and for causal head_dim 64 from S = 512 on (in its
// two-wave layout, measured 5-35% faster there; non-causal and at S <= 384
// the 8-wave kernel is faster, as at head_dim 32).
int w64_mode() {
    static const int v = [] {
        const char *e = getenv("PMKL_ATTN_W64");
        return e ? (atoi(e) == 1 ? 1 : 0) : -1;
    }();
    return v;
}

// XCD-aware work order unless PMKL_ATTN_NOXCD is set (read once).
bool xcd_order_enabled() {
    static const bool on = getenv("PMKL_ATTN_NOXCD") == nullptr;
    return on;
}

// CUs of the current device (cached per device; 0 if it cannot be read).
int cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev < 64) {
        const int c = cache[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

// Layout of the 64-row kernel at head_dim 64 and 128: by default two waves
// of 32 rows per SIMD (8 waves per workgroup, measured 4-6% faster at C3,
// equal at C4, 15% faster at C2); PMKL_ATTN_W32=0 keeps one wave of 64 rows
// per SIMD.
int w32_mode() {
    static const int v = [] {
        const char *e = getenv("PMKL_ATTN_W32");
        return e ? (atoi(e) == 0 ? 0 : 1) : 1;
    }();
    return v;
}

template <typename T, int D>
KernelChoice pick_w32(bool causal) {
    return {causal ? (kernel_fn)pmkl_amd::attn_fwd_w64_kernel<T, D, true, 1, 8>
                   : (kernel_fn)pmkl_amd::attn_fwd_w64_kernel<T, D, false, 1, 8>,
            512, 256, 1, "attn_fwd_w64_kernel", 1, 8};
}
// Two 128-row workgroups per CU for small causal head_dim-64 problems unless
// PMKL_ATTN_SPLIT=0 (read once).
bool split_enabled() {
    static const bool on = [] {
        const char *e = getenv("PMKL_ATTN_SPLIT");
        return !(e && atoi(e) == 0);
    }();
    return on;
}
// fp32 problems too small to fill the CUs take the key-split kernel unless
// PMKL_ATTN_F32SPLIT=0 (read once).
bool f32split_enabled() {
    static const bool on = [] {
        const char *e = getenv("PMKL_ATTN_F32SPLIT");
        return !(e && atoi(e) == 0);
    }();
    return on;
}

// split: causal head_dim 64 with fewer 256-row work items than two per CU
// runs two 128-row workgroups per CU instead (measured same-box: B1 H8 S8192
// 129 -> 102 us, B3 H5 S700 16.4 -> 13.0 us; equal at C2, 1-2% slower with
// two or more 256-row items per CU).
template <typename T>
KernelChoice pick_w32(int64_t D, bool causal, bool split) {
    if (D == 64 && causal && split)
        return {(kernel_fn)pmkl_amd::attn_fwd_w64_kernel<T, 64, true, 1, 4>, 256, 128, 2, "attn_fwd_w64_kernel", 1, 4};
    return D == 64 ? pick_w32<T, 64>(causal) : pick_w32<T, 128>(causal);
}

template <typename T, int D>
KernelChoice pick16(bool causal, bool w64, int waves, bool resident) {
    if (w64)
        return {causal ? (kernel_fn)pmkl_amd::attn_fwd_w64_kernel<T, D, true>
                       : (kernel_fn)pmkl_amd::attn_fwd_w64_kernel<T, D, false>,
                256, 256, 1, "attn_fwd_w64_kernel", 2, 4};
    if (resident) return pick16w<T, D, 8, resident_tiles(D)>(causal);
    return waves == 4 ? pick16w<T, D, 4>(causal) : pick16w<T, D, 8>(causal);
}
template <int D>
KernelChoice pick32(bool causal) {
    return {causal ? (kernel_fn)pmkl_amd::attn_fwd_f32_kernel<D, true>
                   : (kernel_fn)pmkl_amd::attn_fwd_f32_kernel<D, false>,
            pmkl_amd::kThreads, pmkl_amd::kBlockM, 1, "attn_fwd_f32_kernel"};
}

template <int D>
KernelChoice pick32split(bool causal) {
    return {causal ? (kernel_fn)pmkl_amd::attn_fwd_f32_split_kernel<D, true>
                   : (kernel_fn)pmkl_amd::attn_fwd_f32_split_kernel<D, false>,
            256, 32, 1, "attn_fwd_f32_split_kernel"};
}
KernelChoice pick32split(int64_t d, bool causal) {
    if (d == 32) return pick32split<32>(causal);
    if (d == 64) return pick32split<64>(causal);
    if (d == 128) return pick32split<128>(causal);
    return {nullptr, 0, 0};
}

KernelChoice select_kernel(int32_t dt, int64_t d, bool causal, bool w64, int waves, bool resident) {
    switch (dt) {
        case PMKL_DTYPE_BF16:
            if (d == 32) return pick16<__bf16, 32>(causal, w64, waves, resident);
            if (d == 64) return pick16<__bf16, 64>(causal, w64, waves, resident);
            if (d == 128) return pick16<__bf16, 128>(causal, w64, waves, resident);
            break;
        case PMKL_DTYPE_F16:
            if (d == 32) return pick16<_Float16, 32>(causal, w64, waves, resident);
            if (d == 64) return pick16<_Float16, 64>(causal, w64, waves, resident);
            if (d == 128) return pick16<_Float16, 128>(causal, w64, waves, resident);
            break;
        case PMKL_DTYPE_F32:
            if (d == 32) return pick32<32>(causal);
            if (d == 64) return pick32<64>(causal);
            if (d == 128) return pick32<128>(causal);
            break;
        default:
            break;
    }
    return {nullptr, 0, 0};
}

// Fills the three strides with the contiguous [B, H, S, D] ones when all are zero.
void default_strides(int64_t st[3], const int64_t in[3], int64_t H, int64_t S, int64_t D) {
    if (in[0] == 0 && in[1] == 0 && in[2] == 0) {
        st[0] = H * S * D;
        st[1] = S * D;
        st[2] = D;
    } else {
        st[0] = in[0];
        st[1] = in[1];
        st[2] = in[2];
    }
}

int check_tensor(const char *name, const void *ptr, const int64_t st[3], int64_t B, int64_t H, int64_t S,
                 int64_t D, size_t esize) {
    const size_t vec = 16 / esize;  // elements per 16-byte access
    PMKL_REQUIRE(ptr != nullptr, PMKL_EINVAL, "%s is a null pointer", name);
    PMKL_REQUIRE(((uintptr_t)ptr % 16) == 0, PMKL_EINVAL, "%s must be 16-byte aligned", name);
    PMKL_REQUIRE(st[0] >= 0 && st[1] >= 0 && st[2] >= D, PMKL_EINVAL,
                 "%s strides (%lld, %lld, %lld) must be non-negative with seq stride >= head_dim %lld", name,
                 (long long)st[0], (long long)st[1], (long long)st[2], (long long)D);
    PMKL_REQUIRE(st[0] % vec == 0 && st[1] % vec == 0 && st[2] % vec == 0, PMKL_EINVAL,
                 "%s strides (%lld, %lld, %lld) must be multiples of %zu elements (16 bytes)", name,
                 (long long)st[0], (long long)st[1], (long long)st[2], vec);
    // A 64-key tile is addressed by one 32-bit buffer range (bytes).
    PMKL_REQUIRE(st[2] * (int64_t)esize * 64 < (1LL << 31), PMKL_EINVAL,
                 "%s seq stride %lld is too large (a 64-row tile must span < 2 GiB)", name, (long long)st[2]);
    // The largest element offset must stay addressable with 64-bit arithmetic.
    const double span = (double)(B - 1) * st[0] + (double)(H - 1) * st[1] + (double)(S - 1) * st[2] + D;
    PMKL_REQUIRE(span < 9.0e18, PMKL_EINVAL, "%s spans too many elements", name);
    return PMKL_OK;
}

// An output must not alias itself: distinct (b, h, s) rows of a [B, H, S, D]
// tensor (head_dim contiguous) must not share an element, or workgroups
// writing different rows race on the same bytes.  Sufficient test: with the
// dimensions of size > 1 sorted by stride, each stride is at least the extent
// of the dimensions inside it (D elements for the innermost).
int check_no_self_overlap(const char *name, const int64_t st[3], int64_t B, int64_t H, int64_t S, int64_t D) {
    std::pair<int64_t, int64_t> dims[3] = {{st[0], B}, {st[1], H}, {st[2], S}};   // (stride, size)
    std::sort(dims, dims + 3);
    double extent = (double)D;
    for (const auto &d : dims) {
        if (d.second <= 1) continue;
        PMKL_REQUIRE((double)d.first >= extent, PMKL_EINVAL,
                     "%s strides (%lld, %lld, %lld) make distinct rows of the output overlap", name,
                     (long long)st[0], (long long)st[1], (long long)st[2]);
        extent = (double)d.first * (double)(d.second - 1) + extent;
    }
    return PMKL_OK;
}

using pmkl_amd::BwdParams;
typedef void (*bwd_kernel_fn)(BwdParams);

struct BwdKernels {
    bwd_kernel_fn dq, dkdv;
    int dq_threads, dq_rows;       // threads and owned rows per workgroup
    int dkdv_threads, dkdv_rows;
    bool flat;                     // grid over the B*H*S rows, else (row tile, head)
};

template <typename T, int D>
BwdKernels pick_bwd(bool causal) {
    using TQ = pmkl_amd::BwdTile<T, D, pmkl_amd::bwd_waves_dq<D>()>;
    using TK = pmkl_amd::BwdTile<T, D, pmkl_amd::bwd_waves_dkdv<D>()>;
    if (causal)
        return {pmkl_amd::attn_bwd_dq_kernel<T, D, true>, pmkl_amd::attn_bwd_dkdv_kernel<T, D, true>, TQ::THREADS,
                TQ::ROWS, TK::THREADS, TK::ROWS, false};
    return {pmkl_amd::attn_bwd_dq_kernel<T, D, false>, pmkl_amd::attn_bwd_dkdv_kernel<T, D, false>, TQ::THREADS,
            TQ::ROWS, TK::THREADS, TK::ROWS, false};
}

template <int D>
BwdKernels pick_bwd_f32(bool causal) {
    constexpr int W = pmkl_amd::kBwdF32Waves;
    if (causal)
        return {pmkl_amd::attn_bwd_f32_dq_kernel<D, true>, pmkl_amd::attn_bwd_f32_dkdv_kernel<D, true>, 64 * W, W,
                64 * W, W, true};
    return {pmkl_amd::attn_bwd_f32_dq_kernel<D, false>, pmkl_amd::attn_bwd_f32_dkdv_kernel<D, false>, 64 * W, W,
            64 * W, W, true};
}

BwdKernels select_bwd(int32_t dt, int64_t d, bool causal) {
    if (dt == PMKL_DTYPE_BF16) {
        if (d == 32) return pick_bwd<__bf16, 32>(causal);
        if (d == 64) return pick_bwd<__bf16, 64>(causal);
        if (d == 128) return pick_bwd<__bf16, 128>(causal);
    } else if (dt == PMKL_DTYPE_F16) {
        if (d == 32) return pick_bwd<_Float16, 32>(causal);
        if (d == 64) return pick_bwd<_Float16, 64>(causal);
        if (d == 128) return pick_bwd<_Float16, 128>(causal);
    } else if (dt == PMKL_DTYPE_F32) {
        if (d == 32) return pick_bwd_f32<32>(causal);
        if (d == 64) return pick_bwd_f32<64>(causal);
        if (d == 128) return pick_bwd_f32<128>(causal);
    }
    return {nullptr, nullptr, 0, 0, 0, 0, false};
}

// One [B, H, S, D] tensor of a backward call, for the checks and the launch.
struct BwdTensorArg {
    const char *name;
    const void *ptr;
    const int64_t *strides;
    bool optional;   // may be null (o)
    bool output;     // written by the call (dq, dk, dv)
};

// Validates a backward call except for the workspace.  *empty is set for a
// problem with no rows (nothing to launch).
int check_bwd(const pmkl_attn_bwd_args *a, bool *empty) {
    PMKL_REQUIRE(a != nullptr, PMKL_EINVAL, "args is a null pointer");
    PMKL_REQUIRE(dtype_valid(a->dtype), PMKL_EUNSUPPORTED,
                 "backward dtype %d has no device kernel (supported: F32, F16, BF16)", (int)a->dtype);
    PMKL_REQUIRE(a->ml_dtype == a->dtype || a->ml_dtype == PMKL_DTYPE_F32, PMKL_EINVAL,
                 "ml_dtype %d must equal dtype %d or be F32", (int)a->ml_dtype, (int)a->dtype);
    PMKL_REQUIRE(a->batch >= 0 && a->heads >= 0 && a->seq_len >= 0, PMKL_EINVAL,
                 "negative shape (batch %lld, heads %lld, seq %lld)", (long long)a->batch, (long long)a->heads,
                 (long long)a->seq_len);
    PMKL_REQUIRE(head_dim_supported(a->head_dim), PMKL_EUNSUPPORTED,
                 "head_dim %lld has no compiled kernel (supported: 32, 64, 128)", (long long)a->head_dim);
    PMKL_REQUIRE(std::isfinite(a->scale) && a->scale >= 0.f, PMKL_EINVAL, "scale must be finite and >= 0");
    *empty = a->batch * a->heads * a->seq_len == 0;
    if (*empty) return PMKL_OK;

    const int64_t B = a->batch, H = a->heads, S = a->seq_len, D = a->head_dim;
    PMKL_REQUIRE(S <= (1LL << 30) && B * H <= (1LL << 30), PMKL_EINVAL, "shape too large (B*H %lld, S %lld)",
                 (long long)(B * H), (long long)S);
    PMKL_REQUIRE(B * H * S * D < (1LL << 62), PMKL_EINVAL, "tensors span too many elements");
    const size_t es = dtype_size(a->dtype);
    const BwdTensorArg tensors[] = {
        {"dout", a->dout, a->dout_strides, false, false}, {"q", a->q, a->q_strides, false, false},
        {"k", a->k, a->k_strides, false, false},          {"v", a->v, a->v_strides, false, false},
        {"o", a->o, a->o_strides, true, false},           {"dq", a->dq, a->dq_strides, false, true},
        {"dk", a->dk, a->dk_strides, false, true},        {"dv", a->dv, a->dv_strides, false, true}};
    int rc;
    for (const auto &t : tensors) {
        if (t.ptr == nullptr && t.optional) continue;
        int64_t st[3];
        default_strides(st, t.strides, H, S, D);
        if ((rc = check_tensor(t.name, t.ptr, st, B, H, S, D, es)) != PMKL_OK) return rc;
        if (t.output && (rc = check_no_self_overlap(t.name, st, B, H, S, D)) != PMKL_OK) return rc;
    }
    PMKL_REQUIRE(a->m != nullptr && a->l != nullptr, PMKL_EINVAL, "m / l must not be null");
    const size_t ml_es = dtype_size(a->ml_dtype);
    PMKL_REQUIRE((uintptr_t)a->m % ml_es == 0 && (uintptr_t)a->l % ml_es == 0, PMKL_EINVAL,
                 "m / l must be aligned to their element size");
    const BwdKernels kc = select_bwd(a->dtype, D, a->is_causal != 0);
    PMKL_REQUIRE(kc.dq != nullptr, PMKL_EUNSUPPORTED, "no backward kernel for dtype %d head_dim %lld",
                 (int)a->dtype, (long long)D);
    const int64_t nq = (S + kc.dq_rows - 1) / kc.dq_rows, nk = (S + kc.dkdv_rows - 1) / kc.dkdv_rows;
    const int64_t gq = kc.flat ? (B * H * S + kc.dq_rows - 1) / kc.dq_rows : nq * B * H;
    const int64_t gk = kc.flat ? (B * H * S + kc.dkdv_rows - 1) / kc.dkdv_rows : nk * B * H;
    PMKL_REQUIRE(std::max(gq, gk) <= 0x7fffffffLL, PMKL_EINVAL, "grid too large (%lld workgroups)",
                 (long long)std::max(gq, gk));
    return PMKL_OK;
}

// Launches the two backward passes of a validated, non-empty call.  ws holds
// two floats per query row (log2-sum-exp, then sum_j P dP): the dq pass writes
// every row's pair before the dk/dv pass, on the same stream, reads it, so
// nothing in it needs clearing.
int launch_bwd(const pmkl_attn_bwd_args *a, float *ws, void *stream) {
    const int64_t B = a->batch, H = a->heads, S = a->seq_len, D = a->head_dim;
    const BwdKernels kc = select_bwd(a->dtype, D, a->is_causal != 0);
    const int64_t nq = (S + kc.dq_rows - 1) / kc.dq_rows, nk = (S + kc.dkdv_rows - 1) / kc.dkdv_rows;
    const int64_t gq = kc.flat ? (B * H * S + kc.dq_rows - 1) / kc.dq_rows : nq * B * H;
    const int64_t gk = kc.flat ? (B * H * S + kc.dkdv_rows - 1) / kc.dkdv_rows : nk * B * H;

    BwdParams p;
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.o = a->o;
    p.dout = a->dout;
    p.m = a->m;
    p.l = a->l;
    p.dq = a->dq;
    p.dk = a->dk;
    p.dv = a->dv;
    p.lse2 = ws;
    p.drow = ws + B * H * S;
    p.S = (int32_t)S;
    p.BH = (int32_t)(B * H);
    p.H = (int32_t)H;
    {
        const int64_t *in[8];
        in[pmkl_amd::BQ] = a->q_strides;
        in[pmkl_amd::BK] = a->k_strides;
        in[pmkl_amd::BV] = a->v_strides;
        in[pmkl_amd::BO] = a->o_strides;
        in[pmkl_amd::BDOUT] = a->dout_strides;
        in[pmkl_amd::BDQ] = a->dq_strides;
        in[pmkl_amd::BDK] = a->dk_strides;
        in[pmkl_amd::BDV] = a->dv_strides;
        for (int t = 0; t < 8; ++t) {
            int64_t st[3];
            default_strides(st, in[t], H, S, D);
            p.sb[t] = st[0];
            p.sh[t] = st[1];
            p.ss[t] = (int32_t)st[2];   // a 64-row tile spans < 2 GiB (checked)
        }
    }
    p.n_qtiles = (int32_t)nq;
    p.n_ktiles = (int32_t)nk;
    p.scale = a->scale > 0.f ? a->scale : 1.0f / std::sqrt((float)D);
    p.scale_log2 = p.scale * 1.4426950408889634f;
    p.ml_f32 = a->ml_dtype == PMKL_DTYPE_F32 ? 1 : 0;

    hipStream_t st = (hipStream_t)stream;
    // dQ first: it writes the row vectors the dK/dV pass reads.
    hipLaunchKernelGGL(kc.dq, dim3((unsigned)gq), dim3(kc.dq_threads), 0, st, p);
    hipError_t err = hipGetLastError();
    PMKL_REQUIRE(err == hipSuccess, PMKL_EHIP, "dq kernel launch failed: %s", hipGetErrorString(err));
    hipLaunchKernelGGL(kc.dkdv, dim3((unsigned)gk), dim3(kc.dkdv_threads), 0, st, p);
    err = hipGetLastError();
    PMKL_REQUIRE(err == hipSuccess, PMKL_EHIP, "dk/dv kernel launch failed: %s", hipGetErrorString(err));
    return PMKL_OK;
}

// Workspace of pmkl_attn_bwd_noalloc: two floats per query row for up to
// PMKL_ATTN_BWD_NOALLOC_MAX_ROWS rows (8 MiB), static device memory of this
// code object, so each GPU the library runs on holds its own copy until the
// process ends.  In host code `scratch` only names the symbol; its device
// address comes from hipGetSymbolAddress (scratch_on_device), never from the
// name itself.
static __device__ __align__(256) float scratch[2 * PMKL_ATTN_BWD_NOALLOC_MAX_ROWS];

// Device address of `scratch` on the current device, looked up on the first
// call on that device (with that device current) and cached per device.
int scratch_on_device(float **out) {
    static std::atomic<void *> cache[64];
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    PMKL_REQUIRE(err == hipSuccess && dev >= 0, PMKL_EHIP, "hipGetDevice failed: %s", hipGetErrorString(err));
    if (dev < 64) {
        if (void *p = cache[dev].load(std::memory_order_acquire)) {
            *out = (float *)p;
            return PMKL_OK;
        }
    }
    void *ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    PMKL_REQUIRE(err == hipSuccess && ptr != nullptr, PMKL_EHIP, "hipGetSymbolAddress(scratch) failed: %s",
                 hipGetErrorString(err));
    if (dev < 64) cache[dev].store(ptr, std::memory_order_release);
    *out = (float *)ptr;
    return PMKL_OK;
}

// A validated forward call: kernel, grid and parameters.
struct FwdPlan {
    KernelChoice kc;
    AttnParams p;
    int64_t grid;
    bool empty;
};

// Validates a forward call and chooses its kernel, launch shape and
// parameters (pl->empty: no rows, nothing to launch).
int plan_fwd(const pmkl_attn_fwd_args *a, FwdPlan *pl) {
    pl->empty = false;
    PMKL_REQUIRE(a != nullptr, PMKL_EINVAL, "args is a null pointer");
    PMKL_REQUIRE(dtype_valid(a->dtype), PMKL_EUNSUPPORTED, "unsupported dtype %d", (int)a->dtype);
    PMKL_REQUIRE(a->ml_dtype == a->dtype || a->ml_dtype == PMKL_DTYPE_F32, PMKL_EINVAL,
                 "ml_dtype %d must equal dtype %d or be F32", (int)a->ml_dtype, (int)a->dtype);
    PMKL_REQUIRE(a->batch >= 0 && a->heads >= 0 && a->seq_len >= 0, PMKL_EINVAL,
                 "negative shape (batch %lld, heads %lld, seq %lld)", (long long)a->batch, (long long)a->heads,
                 (long long)a->seq_len);
    PMKL_REQUIRE(head_dim_supported(a->head_dim), PMKL_EUNSUPPORTED,
                 "head_dim %lld has no compiled kernel (supported: 32, 64, 128)", (long long)a->head_dim);
    PMKL_REQUIRE(std::isfinite(a->scale) && a->scale >= 0.f, PMKL_EINVAL, "scale must be finite and >= 0");
    // Empty problem: nothing to do (reference causal_attention.h:270).
    if (a->batch * a->heads * a->seq_len == 0) {
        pl->empty = true;
        return PMKL_OK;
    }

    const int64_t B = a->batch, H = a->heads, S = a->seq_len, D = a->head_dim;
    PMKL_REQUIRE(S <= (1LL << 30) && B * H <= (1LL << 30), PMKL_EINVAL, "shape too large (B*H %lld, S %lld)",
                 (long long)(B * H), (long long)S);
    const size_t es = dtype_size(a->dtype);
    int64_t qs[3], ks[3], vs[3], os[3];
    default_strides(qs, a->q_strides, H, S, D);
    default_strides(ks, a->k_strides, H, S, D);
    default_strides(vs, a->v_strides, H, S, D);
    default_strides(os, a->o_strides, H, S, D);
    int rc;
    if ((rc = check_tensor("q", a->q, qs, B, H, S, D, es)) != PMKL_OK) return rc;
    if ((rc = check_tensor("k", a->k, ks, B, H, S, D, es)) != PMKL_OK) return rc;
    if ((rc = check_tensor("v", a->v, vs, B, H, S, D, es)) != PMKL_OK) return rc;
    if ((rc = check_tensor("o", a->o, os, B, H, S, D, es)) != PMKL_OK) return rc;
    if ((rc = check_no_self_overlap("o", os, B, H, S, D)) != PMKL_OK) return rc;

    // The 64-row kernel addresses a head's whole K / V through one buffer
    // resource with 32-bit offsets, and streams the first key tiles of its
    // next work item during the last iterations of the current one, which
    // needs at least three key tiles per item (S > 128).
    auto head_span_ok = [&](const int64_t *st) {
        return st[2] >= 0 && ((S - 1) * st[2] + D) * (int64_t)es < (1LL << 31);
    };
    const int mode = w64_mode();
    const bool causal = a->is_causal != 0;
    // Head_dim 128 with fewer 256-row work items than CUs (most CUs idle
    // under the 64-row kernel) at 128 < S <= 384 (causal: 192 < S <= 352):
    // the 4-wave MFMA kernel, whose 128-row workgroups spread the rows over
    // twice as many CUs (measured 3-16% faster there; slower once the items
    // fill the CUs, and for causal rows outside that range with very few
    // heads; PMKL_ATTN_W64=1 keeps the 64-row kernel).
    const bool small128 = mode != 1 && D == 128 && (causal ? S > 192 && S <= 352 : S > 128 && S <= 384) &&
                          B * H * ((S + 255) / 256) < (int64_t)cu_count();
    const bool w64 = mode != 0 && !small128 && (mode == 1 || D >= 128 || (D == 64 && causal && S >= 512)) &&
                     a->dtype != PMKL_DTYPE_F32 && S > 128 && head_span_ok(ks) && head_span_ok(vs);
    const bool w32 = w64 && (D == 64 || D == 128) && w32_mode() == 1;
    const bool bf = a->dtype == PMKL_DTYPE_BF16;
    const int waves = small128 && !waves16_env() ? 4 : waves16(D, S, causal);
    const bool resident = !w64 && a->dtype != PMKL_DTYPE_F32 && waves == 8 &&
                          (S + 63) / 64 <= resident_tiles(D) && resident_enabled();
    const bool split = w32 && D == 64 && causal && split_enabled() &&
                       B * H * ((S + 255) / 256) < 2 * (int64_t)cu_count();
    // fp32 with the 128-row kernel's workgroups on fewer than half the CUs
    // (C1: 4): 32-row workgroups whose four waves split the key tiles.
    const bool f32split = a->dtype == PMKL_DTYPE_F32 && f32split_enabled() && S <= 1024 &&
                          B * H * ((S + 127) / 128) * 2 < (int64_t)cu_count();
    const KernelChoice kc = w32        ? (bf ? pick_w32<__bf16>(D, causal, split) : pick_w32<_Float16>(D, causal, split))
                            : f32split ? pick32split(D, causal)
                                       : select_kernel(a->dtype, D, causal, w64, waves, resident);
    PMKL_REQUIRE(kc.fn != nullptr, PMKL_EUNSUPPORTED, "no kernel for dtype %d head_dim %lld", (int)a->dtype,
                 (long long)D);
    const int64_t n_qtiles = (S + kc.block_m - 1) / kc.block_m;
    PMKL_REQUIRE(n_qtiles * B * H <= 0x7fffffffLL, PMKL_EINVAL, "grid too large (%lld workgroups)",
                 (long long)(n_qtiles * B * H));
    PMKL_REQUIRE(a->m != nullptr && a->l != nullptr, PMKL_EINVAL, "m / l must not be null");
    const size_t ml_es = dtype_size(a->ml_dtype);
    PMKL_REQUIRE((uintptr_t)a->m % ml_es == 0 && (uintptr_t)a->l % ml_es == 0, PMKL_EINVAL,
                 "m / l must be aligned to their element size");

    AttnParams &p = pl->p;
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.o = a->o;
    p.m = a->m;
    p.l = a->l;
    p.q_sb = qs[0]; p.q_sh = qs[1]; p.q_ss = qs[2];
    p.k_sb = ks[0]; p.k_sh = ks[1]; p.k_ss = ks[2];
    p.v_sb = vs[0]; p.v_sh = vs[1]; p.v_ss = vs[2];
    p.o_sb = os[0]; p.o_sh = os[1]; p.o_ss = os[2];
    p.H = (int32_t)H;
    p.S = (int32_t)S;
    p.BH = (int32_t)(B * H);
    p.n_qtiles = (int32_t)n_qtiles;
    // Reference scale: 1.0f / std::sqrt((float)hidden_size), fused_self_attention.cpp:30.
    p.scale = a->scale > 0.f ? a->scale : 1.0f / std::sqrt((float)D);
    p.scale_log2 = p.scale * 1.4426950408889634f;
    p.lazy_raw = pmkl_amd::kLazyLog2 / p.scale_log2;   // IEEE float division, as the kernels' was
    p.ml_f32 = a->ml_dtype == PMKL_DTYPE_F32 ? 1 : 0;
    // XCD-grouped issue order needs whole head pairs (causal) or heads per XCD.
    p.xcd_order = (a->dtype != PMKL_DTYPE_F32 && xcd_order_enabled() && (B * H) % (a->is_causal ? 16 : 8) == 0) ? 1 : 0;

    // One workgroup per work item, except the 64-row kernel: one workgroup per
    // CU, each looping over its share of the items.
    int64_t grid = n_qtiles * B * H;
    if (w64) {
        const int cus = cu_count();
        PMKL_REQUIRE(cus > 0, PMKL_EHIP, "could not read the device's CU count");
        grid = std::min<int64_t>(grid, (int64_t)kc.per_cu * cus);
    }
    pl->kc = kc;
    pl->grid = grid;
    return PMKL_OK;
}

}  // namespace

extern "C" {

const char *pmkl_last_error(void) { return pmkl_capi::g_err; }

int pmkl_abi_version(void) { return PMKL_ABI_VERSION; }

int pmkl_attn_fwd_supported(int32_t dtype, int64_t head_dim) {
    return dtype_valid(dtype) && head_dim_supported(head_dim) ? 1 : 0;
}

int pmkl_attn_fwd(const pmkl_attn_fwd_args *a, void *stream) {
    pmkl_capi::g_err[0] = '\0';
    FwdPlan pl;
    const int rc = plan_fwd(a, &pl);
    if (rc != PMKL_OK || pl.empty) return rc;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(pl.kc.fn, dim3((unsigned)pl.grid), dim3(pl.kc.threads), 0, st, pl.p);
    hipError_t err = hipGetLastError();
    PMKL_REQUIRE(err == hipSuccess, PMKL_EHIP, "kernel launch failed: %s", hipGetErrorString(err));
    return PMKL_OK;
}

const char *pmkl_attn_fwd_kernel_name(const pmkl_attn_fwd_args *a) {
    pmkl_capi::g_err[0] = '\0';
    static thread_local char name[160];
    FwdPlan pl;
    if (plan_fwd(a, &pl) != PMKL_OK) return nullptr;
    if (pl.empty) return "none";
    const char *dt = a->dtype == PMKL_DTYPE_BF16 ? "bf16" : a->dtype == PMKL_DTYPE_F16 ? "fp16" : "fp32";
    const char *mask = a->is_causal ? "causal" : "full";
    const char *order = pl.p.xcd_order ? ", xcd order" : "";
    if (pl.kc.t1 >= 0)
        snprintf(name, sizeof(name), "%s<%s, %lld, %s, %d, %d> grid %lld x %d%s", pl.kc.family, dt,
                 (long long)a->head_dim, mask, pl.kc.t1, pl.kc.t2, (long long)pl.grid, pl.kc.threads, order);
    else
        snprintf(name, sizeof(name), "%s<%lld, %s> grid %lld x %d%s", pl.kc.family, (long long)a->head_dim, mask,
                 (long long)pl.grid, pl.kc.threads, order);
    return name;
}

uint64_t pmkl_attn_bwd_workspace_size(int64_t batch, int64_t heads, int64_t seq_len) {
    if (batch <= 0 || heads <= 0 || seq_len <= 0) return 0;
    return (uint64_t)(2 * batch * heads * seq_len) * sizeof(float);
}

int pmkl_attn_bwd_supported(int32_t dtype, int64_t head_dim) {
    return dtype_valid(dtype) && head_dim_supported(head_dim) ? 1 : 0;
}

int pmkl_attn_bwd(const pmkl_attn_bwd_args *a, void *stream) {
    pmkl_capi::g_err[0] = '\0';
    bool empty = false;
    int rc = check_bwd(a, &empty);
    if (rc != PMKL_OK || empty) return rc;
    const uint64_t ws = pmkl_attn_bwd_workspace_size(a->batch, a->heads, a->seq_len);
    PMKL_REQUIRE(a->workspace != nullptr && ((uintptr_t)a->workspace % 16) == 0, PMKL_EINVAL,
                 "workspace must be a 16-byte aligned device pointer");
    PMKL_REQUIRE(a->workspace_bytes >= ws, PMKL_EINVAL, "workspace of %llu bytes is too small (needs %llu)",
                 (unsigned long long)a->workspace_bytes, (unsigned long long)ws);
    return launch_bwd(a, (float *)a->workspace, stream);
}

int pmkl_attn_bwd_noalloc(const pmkl_attn_bwd_args *a, void *stream) {
    pmkl_capi::g_err[0] = '\0';
    bool empty = false;
    int rc = check_bwd(a, &empty);
    if (rc != PMKL_OK || empty) return rc;
    const int64_t rows = a->batch * a->heads * a->seq_len;
    PMKL_REQUIRE(rows <= PMKL_ATTN_BWD_NOALLOC_MAX_ROWS, PMKL_EINVAL,
                 "pmkl_attn_bwd_noalloc handles at most %d query rows (batch * heads * seq_len), got %lld; "
                 "use pmkl_attn_bwd with a workspace", (int)PMKL_ATTN_BWD_NOALLOC_MAX_ROWS, (long long)rows);
    float *ws = nullptr;
    if ((rc = scratch_on_device(&ws)) != PMKL_OK) return rc;
    return launch_bwd(a, ws, stream);
}

int pmkl_causal_attention_forward(int32_t dtype, void *out, const void *q, const void *k, const void *v,
                                  int32_t batch_size, int32_t num_heads, int32_t seq_length, int32_t hidden_size,
                                  void *out_m, void *out_l, void *stream) {
    pmkl_attn_fwd_args a;
    memset(&a, 0, sizeof(a));
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = out;
    a.m = out_m;
    a.l = out_l;
    a.dtype = dtype;
    a.ml_dtype = dtype;
    a.batch = batch_size;
    a.heads = num_heads;
    a.seq_len = seq_length;
    a.head_dim = hidden_size;
    a.scale = 0.f;
    a.is_causal = 1;
    return pmkl_attn_fwd(&a, stream);
}

}  // extern "C"
