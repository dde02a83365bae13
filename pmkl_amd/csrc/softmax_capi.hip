// C ABI of the gfx950 row softmax / log-softmax (include/pmkl_softmax.h).
//
// Replaces the reference launcher pmkl::norm::warp_softmax_forward
// (pmkl/norm/warp_softmax.h:159-201), which checks 0 <= softmax_elements <=
// 1024 with CHECK_FAIL, returns early for an empty row, and submits one of
// eleven power-of-two kernel instances (1 .. 1024 elements) through the
// GpuLauncher singleton with 128-thread blocks of 32-lane warps.  Here the
// host picks the lanes per row (G), the chunks per lane (C) and the vector
// width (W) from the row length and the pointers' alignment, and launches a
// named __global__ kernel on the caller's stream.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "capi_common.hpp"
#include "pmkl_softmax.h"
#include "softmax_kernels.hpp"

namespace {

using pmkl_amd::SoftmaxParams;
typedef void (*softmax_fn)(SoftmaxParams);

template <typename Tin, typename Tout, int W, int C>
softmax_fn pick_log(bool log) {
    return log ? pmkl_amd::softmax_fwd_kernel<Tin, Tout, W, C, true> : pmkl_amd::softmax_fwd_kernel<Tin, Tout, W, C, false>;
}

// C chunks of W elements per lane, G <= 64 lanes per row: rows of up to 1024
// elements need C <= 1024 / (64 W).
template <typename Tin, typename Tout, int W>
softmax_fn pick_c(int c, bool log) {
    constexpr int CMAX = PMKL_SOFTMAX_MAX_ELEMENTS / (64 * W);
    switch (c) {
        case 1: return pick_log<Tin, Tout, W, 1>(log);
        case 2: return pick_log<Tin, Tout, W, 2>(log);
        case 4:
            if constexpr (CMAX >= 4) return pick_log<Tin, Tout, W, 4>(log);
            return nullptr;
        case 8:
            if constexpr (CMAX >= 8) return pick_log<Tin, Tout, W, 8>(log);
            return nullptr;
        case 16:
            if constexpr (CMAX >= 16) return pick_log<Tin, Tout, W, 16>(log);
            return nullptr;
        default: return nullptr;
    }
}

template <typename Tin, typename Tout>
softmax_fn pick_w(bool vec, int c, bool log) {
    constexpr int WV = 16 / sizeof(Tin);
    return vec ? pick_c<Tin, Tout, WV>(c, log) : pick_c<Tin, Tout, 1>(c, log);
}

template <typename Tin>
softmax_fn pick_out(int32_t out_dt, bool vec, int c, bool log) {
    switch (out_dt) {
        case PMKL_DTYPE_F32: return pick_w<Tin, float>(vec, c, log);
        case PMKL_DTYPE_F16: return pick_w<Tin, _Float16>(vec, c, log);
        case PMKL_DTYPE_BF16: return pick_w<Tin, __bf16>(vec, c, log);
        default: return nullptr;
    }
}

softmax_fn pick(int32_t out_dt, int32_t in_dt, bool vec, int c, bool log) {
    switch (in_dt) {
        case PMKL_DTYPE_F32: return pick_out<float>(out_dt, vec, c, log);
        case PMKL_DTYPE_F16: return pick_out<_Float16>(out_dt, vec, c, log);
        case PMKL_DTYPE_BF16: return pick_out<__bf16>(out_dt, vec, c, log);
        default: return nullptr;
    }
}

int ceil_log2(int64_t v) {
    int r = 0;
    while ((int64_t(1) << r) < v) ++r;
    return r;
}

}  // namespace

extern "C" {

int pmkl_softmax_fwd(const pmkl_softmax_args *a, void *stream) {
    pmkl_capi::g_err[0] = '\0';
    PMKL_REQUIRE(a != nullptr, PMKL_EINVAL, "null argument block");
    PMKL_REQUIRE(a->elements >= 0 && a->elements <= PMKL_SOFTMAX_MAX_ELEMENTS, PMKL_EINVAL,
                 "softmax_elements >= 0 && softmax_elements <= %d (got %lld)", PMKL_SOFTMAX_MAX_ELEMENTS,
                 (long long)a->elements);
    PMKL_REQUIRE(pmkl_capi::dtype_valid(a->in_dtype) && pmkl_capi::dtype_valid(a->out_dtype), PMKL_EINVAL,
                 "unknown dtype (in %d, out %d)", (int)a->in_dtype, (int)a->out_dtype);
    PMKL_REQUIRE(a->batch >= 0 && a->batch <= INT32_MAX, PMKL_EINVAL, "batch_count must be in [0, 2^31) (got %lld)",
                 (long long)a->batch);
    PMKL_REQUIRE(a->stride >= a->elements, PMKL_EINVAL, "softmax_elements_stride (%lld) < softmax_elements (%lld)",
                 (long long)a->stride, (long long)a->elements);
    if (a->elements == 0 || a->batch == 0) return PMKL_OK;
    PMKL_REQUIRE(a->src != nullptr && a->dst != nullptr, PMKL_EINVAL, "null src or dst");
    PMKL_REQUIRE(a->src != a->dst || a->in_dtype == a->out_dtype, PMKL_EINVAL,
                 "in-place softmax needs the same input and output dtype");
    // Element offsets r * stride + i stay far inside int64 (and inside any
    // allocation): the span (batch - 1) * stride + elements is capped at 2^48.
    PMKL_REQUIRE(a->stride <= (int64_t(1) << 48) &&
                     (a->batch - 1) <= ((int64_t(1) << 48) - a->elements) / (a->stride > 0 ? a->stride : 1),
                 PMKL_EINVAL, "rows span more than 2^48 elements (batch %lld, stride %lld)", (long long)a->batch,
                 (long long)a->stride);

    const int64_t n = a->elements;
    const int wv = 16 / (int)pmkl_capi::dtype_size(a->in_dtype);
    const bool vec = n % wv == 0 && a->stride % wv == 0 && reinterpret_cast<uintptr_t>(a->src) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(a->dst) % 16 == 0;
    const int w = vec ? wv : 1;
    const int64_t chunks = (n + w - 1) / w;
    const int g = ceil_log2(chunks) < 6 ? ceil_log2(chunks) : 6;
    const int64_t per_lane = (chunks + (1 << g) - 1) >> g;
    const int c = 1 << ceil_log2(per_lane);
    softmax_fn fn = pick(a->out_dtype, a->in_dtype, vec, c, a->is_log != 0);
    PMKL_REQUIRE(fn != nullptr, PMKL_EUNSUPPORTED, "no softmax kernel for %lld elements (W %d, C %d)", (long long)n,
                 w, c);

    SoftmaxParams p;
    p.dst = a->dst;
    p.src = a->src;
    p.stride = a->stride;
    p.batch = a->batch;
    p.n = (int32_t)n;
    p.log2g = g;
    const int64_t rows_per_block = int64_t(pmkl_amd::kSoftmaxThreads / 64) << (6 - g);
    const int64_t blocks = (a->batch + rows_per_block - 1) / rows_per_block;
    hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(pmkl_amd::kSoftmaxThreads), 0, (hipStream_t)stream, p);
    const hipError_t err = hipGetLastError();
    PMKL_REQUIRE(err == hipSuccess, PMKL_EHIP, "softmax launch failed: %s", hipGetErrorString(err));
    return PMKL_OK;
}

int pmkl_warp_softmax_forward(int32_t out_dtype, int32_t in_dtype, int32_t is_log, void *dst, const void *src,
                              int64_t softmax_elements, int64_t softmax_elements_stride, int64_t batch_count,
                              void *stream) {
    pmkl_softmax_args a;
    a.dst = dst;
    a.src = src;
    a.out_dtype = out_dtype;
    a.in_dtype = in_dtype;
    a.elements = softmax_elements;
    a.stride = softmax_elements_stride;
    a.batch = batch_count;
    a.is_log = is_log;
    return pmkl_softmax_fwd(&a, stream);
}

}  // extern "C"
