// gfx950 row softmax / log-softmax over rows of up to 1024 elements.
//
// Replaces the kernel body of pmkl::norm::warp_softmax_forward,
// warp_softmax_forward_impl (pmkl/norm/warp_softmax.h:74-157).  Per row r
// (elements x_i = src[r*stride + i], i < n), in fp32:
//   m = max_i x_i                                   (:108-118)
//   s = sum_i exp(x_i - m)                          (:120-133)
//   softmax:     y_i = exp(x_i - m) / s, NaN if s == 0   (:147-150)
//   log-softmax: y_i = (x_i - m) - log(s)                 (:140, :146)
//
// Work layout.  A row is owned by a group of G = 2^g lanes of one wave64
// (G = 1 .. 64, so one wave holds 64/G rows; the reference fixes a 32-lane
// warp and two rows per warp for rows of <= 128 elements).  Lane j of a group
// holds C chunks of W consecutive elements, chunk c starting at element
// (c*G + j)*W: one load instruction of the wave reads G*W consecutive
// elements of each of its rows.  W is 16 bytes of the input type (4 fp32 or 8
// fp16/bf16 elements) when the row length, the stride and both base pointers
// allow 16-byte vectors, else 1.  The whole row sits in registers between the
// load and the store, so src is read once and dst written once (2 passes of
// HBM traffic in total: the kernel is HBM-bound at any row length).  The max
// and the sum are xor butterflies over the G lanes of the group.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace pmkl_amd {

struct SoftmaxParams {
    void *dst;
    const void *src;
    int64_t stride;  // elements between row starts, src and dst alike
    int64_t batch;   // rows
    int32_t n;       // elements per row, 1 .. 1024
    int32_t log2g;   // lanes per row = 1 << log2g, 0 .. 6
};

constexpr int kSoftmaxThreads = 256;  // 4 waves per workgroup

template <typename T, int W>
struct alignas(sizeof(T) * W >= 16 ? 16 : sizeof(T) * W) SoftmaxVec {
    T v[W];
};

// Streaming accesses: every element is read once and written once, so loads
// and stores carry the nontemporal hint (the "nt" bit), which keeps the
// stream from displacing other data in the caches; measured ~10% faster than
// plain accesses on 131,072 x 1,024 fp32.  A vector moves as words of up to
// 16 bytes.
template <int BYTES> struct SoftmaxWord;
template <> struct SoftmaxWord<16> { typedef __attribute__((ext_vector_type(4))) unsigned type; };
template <> struct SoftmaxWord<8> { typedef __attribute__((ext_vector_type(2))) unsigned type; };
template <> struct SoftmaxWord<4> { typedef unsigned type; };
template <> struct SoftmaxWord<2> { typedef unsigned short type; };

template <typename V>
__device__ __forceinline__ V softmax_nt_load(const V *p) {
    constexpr int WB = sizeof(V) >= 16 ? 16 : (int)sizeof(V);
    typedef typename SoftmaxWord<WB>::type U;
    struct alignas(V) Words { U w[sizeof(V) / WB]; } r;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(V) / WB); ++i) r.w[i] = __builtin_nontemporal_load(reinterpret_cast<const U *>(p) + i);
    return __builtin_bit_cast(V, r);
}
template <typename V>
__device__ __forceinline__ void softmax_nt_store(V *p, const V &v) {
    constexpr int WB = sizeof(V) >= 16 ? 16 : (int)sizeof(V);
    typedef typename SoftmaxWord<WB>::type U;
    struct alignas(V) Words { U w[sizeof(V) / WB]; };
    const Words r = __builtin_bit_cast(Words, v);
#pragma unroll
    for (int i = 0; i < (int)(sizeof(V) / WB); ++i) __builtin_nontemporal_store(r.w[i], reinterpret_cast<U *>(p) + i);
}

// exp(d) for d = x - max <= 0 on v_exp_f32 (2^t).  t = d*log2(e) is rounded
// to fp32, so 2^t alone would carry a relative error up to |t| * 2^-24; the
// rounding error of the product, recovered with an fma against a two-part
// split of log2(e) (head = log2(e) rounded to fp32, tail = the remainder), is
// put back through 2^(t + c) ~ 2^t * (1 + c ln 2).  Error: that of v_exp_f32
// plus about one rounding.  d below -120 (exp < 1e-52, zero in fp32; this
// includes the -inf of padding and of masked inputs) is clamped to -120 so the
// fma stays finite; a NaN d stays NaN (the comparison is false).
__device__ __forceinline__ float softmax_exp(float d) {
    constexpr float kLog2eHi = 1.44269502162933349609375f;   // fp32(log2 e)
    constexpr float kLog2eLo = 1.9259629911266175e-08f;      // log2 e - kLog2eHi
    constexpr float kLn2 = 0.693147180559945309f;
    d = d < -120.f ? -120.f : d;
    const float t = d * kLog2eHi;
    const float c = fmaf(d, kLog2eHi, -t) + d * kLog2eLo;
    const float e = __builtin_amdgcn_exp2f(t);
    return fmaf(e, c * kLn2, e);
}

template <typename Tin, typename Tout, int W, int C, bool LOG>
__global__ __launch_bounds__(kSoftmaxThreads) void softmax_fwd_kernel(SoftmaxParams p) {
    const int lane = threadIdx.x & 63;
    const int g = p.log2g;
    const int G = 1 << g;
    const int j = lane & (G - 1);
    const int64_t wave = (int64_t)blockIdx.x * (kSoftmaxThreads / 64) + (threadIdx.x >> 6);
    const int64_t row = (wave << (6 - g)) + (lane >> g);
    const bool live = row < p.batch;
    const int64_t base = live ? row * p.stride : 0;
    const Tin *src = static_cast<const Tin *>(p.src) + base;

    float x[C][W];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int e0 = (c * G + j) * W;
        if (live && e0 < p.n) {  // with W > 1, n % W == 0, so e0 + W <= n
            const SoftmaxVec<Tin, W> t = softmax_nt_load(reinterpret_cast<const SoftmaxVec<Tin, W> *>(src + e0));
#pragma unroll
            for (int w = 0; w < W; ++w) x[c][w] = static_cast<float>(t.v[w]);
        } else {
#pragma unroll
            for (int w = 0; w < W; ++w) x[c][w] = -INFINITY;
        }
    }

    // Row max.  A NaN element makes the sum below NaN, so every output of its
    // row is NaN whatever the max keeps (as in the reference).
    float m = -INFINITY;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int w = 0; w < W; ++w) m = fmaxf(m, x[c][w]);
    for (int off = G >> 1; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));

    // Sum of exp(x - m); softmax keeps the exponentials, log-softmax keeps x.
    // Padding elements are -inf and add exp(-inf) = 0.
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float e = softmax_exp(x[c][w] - m);
            s += e;
            if (!LOG) x[c][w] = e;
        }
    for (int off = G >> 1; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);

    if (!live) return;
    Tout *dst = static_cast<Tout *>(p.dst) + base;
    // softmax: one correctly rounded reciprocal per row, then a multiply per
    // element (the reference divides each element by the sum); s == 0 gives NaN
    // as the reference's explicit check does.  log-softmax: (x - m) - log(s).
    const float k = LOG ? logf(s) : (s == 0.f ? __builtin_nanf("") : 1.f / s);
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int e0 = (c * G + j) * W;
        if (e0 < p.n) {
            SoftmaxVec<Tout, W> t;
#pragma unroll
            for (int w = 0; w < W; ++w) t.v[w] = static_cast<Tout>(LOG ? (x[c][w] - m) - k : x[c][w] * k);
            softmax_nt_store(reinterpret_cast<SoftmaxVec<Tout, W> *>(dst + e0), t);
        }
    }
}

}  // namespace pmkl_amd
