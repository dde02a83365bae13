// C++ test of the drop-in header pmkl/norm/warp_softmax.h on the GPU.
//
// Mirrors the reference test test/test_softmax.cpp:30-60: batch 12, 1024
// elements, fp32, inputs U(-10, 10), ten calls of
// warp_softmax_forward<float, float, float, false>, then all_close (default
// atol = rtol = 1e-5) against the reference's CPU check host_softmax_forward
// (test_softmax.cpp:10-28; oracle_softmax_host_f32 restates it op for op).
// Inputs come from a seeded generator (the reference's fill_rand uses rand()).
// It also runs log-softmax, 16-bit and mixed types and a strided, ragged row
// length against the float64 oracle, and the reference's error path
// (softmax_elements > 1024 throws).
//
// Exit code 0 on success, 1 on any failure (as the reference's ctest exes).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "pmkl/pmkl.h"

extern "C" {
int oracle_softmax_f64(const double *src, int64_t n, int64_t stride, int64_t batch, int is_log, double *dst);
void oracle_softmax_host_f32(float *dst, const float *src, int softmax_elements, int softmax_elements_stride,
                             int batch_count);
}

namespace {

uint16_t to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
float from_bf16(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

template <typename T>
struct Conv;
template <>
struct Conv<float> {
    static float to(float x) { return x; }
    static float from(float x) { return x; }
    static constexpr int mant = 23;
    static constexpr int min_exp = -149;  // spacing of the subnormals
};
template <>
struct Conv<pmkl::bfloat16_t> {
    static pmkl::bfloat16_t to(float x) { return pmkl::bfloat16_t{to_bf16(x)}; }
    static float from(pmkl::bfloat16_t x) { return from_bf16(x.bits); }
    static constexpr int mant = 7;
    static constexpr int min_exp = -133;
};
template <>
struct Conv<_Float16> {
    static _Float16 to(float x) { return (_Float16)x; }
    static float from(_Float16 x) { return (float)x; }
    static constexpr int mant = 10;
    static constexpr int min_exp = -24;
};

// The reference test's exact case and criterion.
bool reference_case() {
    const int batch_size = 12, eltsize = 1024, numel = batch_size * eltsize;
    std::mt19937 gen(20240701);
    std::uniform_real_distribution<float> dist(-10.0f, 10.0f);
    std::vector<float> input_cpu(numel), output_cpu(numel), output_gpu_cpu(numel);
    for (auto &x : input_cpu) x = dist(gen);
    pmkl::DeviceBuffer input(numel * sizeof(float)), output(numel * sizeof(float));
    input.copy_from_host(input_cpu.data());
    for (int i = 0; i < 10; i++)
        pmkl::norm::warp_softmax_forward<float, float, float, false>(output.as<float>(), input.as<float>(), eltsize,
                                                                     eltsize, batch_size);
    output.copy_to_host(output_gpu_cpu.data());
    oracle_softmax_host_f32(output_cpu.data(), input_cpu.data(), eltsize, eltsize, batch_size);
    const bool ok = pmkl::utils::all_close(output_gpu_cpu.data(), output_cpu.data(), numel);
    std::printf("fp32 12x1024 softmax vs host_softmax_forward (all_close 1e-5): %s\n", ok ? "ok" : "FAILED");
    return ok;
}

// Any types, row length and stride, against the float64 oracle: at most
// 16 fp32 ulps (plus the rounding of x - max, |x - max| ulps) before the
// output rounding, and 1 ulp of a 16-bit output.
template <typename out_t, typename in_t, bool LOG>
bool oracle_case(const char *name, int n, int stride, int batch, float lo, float hi, uint32_t seed) {
    const size_t total = (size_t)batch * stride;
    std::mt19937 gen(seed);
    std::uniform_real_distribution<float> dist(lo, hi);
    std::vector<in_t> hx(total);
    std::vector<double> x64(total);
    std::vector<out_t> hy(total, Conv<out_t>::to(-7.0f));
    for (size_t i = 0; i < total; ++i) {
        hx[i] = Conv<in_t>::to(dist(gen));
        x64[i] = Conv<in_t>::from(hx[i]);
    }
    pmkl::DeviceBuffer dx(total * sizeof(in_t)), dy(total * sizeof(out_t));
    dx.copy_from_host(hx.data());
    dy.copy_from_host(hy.data());
    pmkl::norm::warp_softmax_forward<out_t, in_t, float, LOG>(dy.as<out_t>(), dx.as<in_t>(), n, stride, batch);
    dy.copy_to_host(hy.data());
    std::vector<double> ref(total, 0.0);
    oracle_softmax_f64(x64.data(), n, stride, batch, LOG ? 1 : 0, ref.data());
    double worst = 0;
    bool ok = true;
    for (int r = 0; r < batch; ++r) {
        double m = -INFINITY;
        for (int i = 0; i < n; ++i) m = std::fmax(m, x64[(size_t)r * stride + i]);
        for (int i = 0; i < stride; ++i) {
            const size_t k = (size_t)r * stride + i;
            const double y = Conv<out_t>::from(hy[k]);
            if (i >= n) {  // padding untouched
                if (y != -7.0) ok = false;
                continue;
            }
            const double d = std::fabs(x64[k] - m), w = ref[k];
            double bound = LOG ? std::ldexp(std::fabs(d) + std::fabs(w) + 16.0, -23)
                               : std::ldexp((16.0 + d) * std::fabs(w), -24) + std::ldexp(1.0, -126);
            if (Conv<out_t>::mant < 23) {
                const double a = std::fabs(w) > 0 ? std::fabs(w) : 1e-30;
                const int e = (int)std::floor(std::log2(a)) - Conv<out_t>::mant;
                bound += std::ldexp(1.0, e > Conv<out_t>::min_exp ? e : Conv<out_t>::min_exp) + std::ldexp(1.0, -126);
            }
            const double err = std::fabs(y - w);
            worst = std::fmax(worst, err / bound);
            if (!(err <= bound)) ok = false;
        }
    }
    std::printf("%s: worst err/bound %.3f: %s\n", name, worst, ok ? "ok" : "FAILED");
    return ok;
}

}  // namespace

int main() {
    std::printf("test_softmax: start\n");
    std::fflush(stdout);
    bool ok = reference_case();
    ok = oracle_case<float, float, true>("fp32 log-softmax 300x1000", 1000, 1000, 300, -10.f, 10.f, 11) && ok;
    ok = oracle_case<pmkl::bfloat16_t, pmkl::bfloat16_t, false>("bf16 softmax 1000x128", 128, 128, 1000, -4.f, 4.f,
                                                                12) && ok;
    ok = oracle_case<float, _Float16, false>("fp16->fp32 softmax 257x77 stride 80", 77, 80, 257, -6.f, 6.f, 13) && ok;
    ok = oracle_case<_Float16, float, true>("fp32->fp16 log-softmax 33x513 stride 520", 513, 520, 33, -3.f, 3.f,
                                            14) && ok;

    // Error path of the reference launcher: more than 1024 elements throws.
    bool threw = false;
    try {
        pmkl::norm::warp_softmax_forward<float, float, float, false>(nullptr, nullptr, 1025, 1025, 1);
    } catch (const pmkl::utils::Error &e) {
        threw = std::strstr(e.what(), "softmax_elements <=") != nullptr;
    }
    std::printf("softmax_elements > 1024 rejected: %s\n", threw ? "ok" : "FAILED");
    ok = ok && threw;
    // softmax_elements == 0 returns without touching the (null) pointers.
    pmkl::norm::warp_softmax_forward<float, float, float, false>(nullptr, nullptr, 0, 0, 5);
    std::printf("%s\n", ok ? "ok" : "FAILED");
    return ok ? 0 : 1;
}
