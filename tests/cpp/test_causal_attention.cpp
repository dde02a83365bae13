// C++ test of the drop-in header pmkl/nlp/causal_attention.h on the GPU.
//
// Mirrors the reference test test/test_causal_attention.cpp:143-207: shape
// {4, 16, 1024, 64}, fp32, U(-1.05, 1.05) inputs, all_close(atol = rtol = 1e-5)
// on m, l and out.  Differences: inputs come from a seeded generator (the
// reference seeds rand() with time(0)), the host side is the float64 oracle
// (oracle/liboracle.so) instead of a copy of the CPU body in the test, and the
// test also runs bf16 / fp16 at their stated tolerances and checks the
// reference's error path (seq_length % BLOCK_M != 0 throws).
//
// Exit code 0 on success, 1 on any failure (as the reference's ctest exes).
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "pmkl/pmkl.h"

extern "C" {
double oracle_default_scale(int64_t D);
int oracle_attn_fwd_rows(const float *q, const float *k, const float *v, int64_t BH, int64_t S, int64_t D,
                         int causal, double scale, const int64_t *rows, int64_t nrows, double *o, double *m,
                         double *l);
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
};
template <>
struct Conv<pmkl::bfloat16_t> {
    static pmkl::bfloat16_t to(float x) { return pmkl::bfloat16_t{to_bf16(x)}; }
    static float from(pmkl::bfloat16_t x) { return from_bf16(x.bits); }
};
template <>
struct Conv<_Float16> {
    static _Float16 to(float x) { return (_Float16)x; }
    static float from(_Float16 x) { return (float)x; }
};

// ulp of x rounded to a format with `mant` explicit mantissa bits.
double ulp_of(double x, int mant) {
    int e;
    std::frexp(std::fabs(x), &e);
    return std::ldexp(1.0, e - 1 - mant);
}

template <typename T, int D>
bool run_case(const char *name, int B, int H, int S, double tol_o, double tol_ml, bool ulp_ml, int mant,
              uint64_t seed) {
    const size_t n = (size_t)B * H * S * D, nr = (size_t)B * H * S;
    std::mt19937_64 gen(seed);
    std::uniform_real_distribution<float> dist(-1.05f, 1.05f);
    std::vector<T> hq(n), hk(n), hv(n), ho(n), hm(nr), hl(nr);
    std::vector<float> fq(n), fk(n), fv(n);
    for (size_t i = 0; i < n; ++i) {
        hq[i] = Conv<T>::to(dist(gen));
        fq[i] = Conv<T>::from(hq[i]);
    }
    for (size_t i = 0; i < n; ++i) {
        hk[i] = Conv<T>::to(dist(gen));
        fk[i] = Conv<T>::from(hk[i]);
    }
    for (size_t i = 0; i < n; ++i) {
        hv[i] = Conv<T>::to(dist(gen));
        fv[i] = Conv<T>::from(hv[i]);
    }
    std::vector<double> ro(n), rm(nr), rl(nr);
    if (oracle_attn_fwd_rows(fq.data(), fk.data(), fv.data(), (int64_t)B * H, S, D, 1, oracle_default_scale(D),
                             nullptr, 0, ro.data(), rm.data(), rl.data()) != 0) {
        std::printf("%s: oracle failed\n", name);
        return false;
    }
    pmkl::DeviceBuffer q(n * sizeof(T)), k(n * sizeof(T)), v(n * sizeof(T)), o(n * sizeof(T)), m(nr * sizeof(T)),
        l(nr * sizeof(T));
    q.copy_from_host(hq.data());
    k.copy_from_host(hk.data());
    v.copy_from_host(hv.data());
    pmkl::nlp::causal_attention_forward<T, 32, D>(o.as<T>(), q.as<T>(), k.as<T>(), v.as<T>(), B, H, S, m.as<T>(),
                                                  l.as<T>());
    o.copy_to_host(ho.data());
    m.copy_to_host(hm.data());
    l.copy_to_host(hl.data());
    std::vector<float> go(n), gm(nr), gl(nr);
    std::vector<float> tgt_o(n), tgt_m(nr), tgt_l(nr);
    double max_o = 0, max_m = 0, max_l = 0;
    bool ok = true;
    for (size_t i = 0; i < n; ++i) {
        go[i] = Conv<T>::from(ho[i]);
        tgt_o[i] = (float)ro[i];
        max_o = std::fmax(max_o, std::fabs(go[i] - ro[i]));
    }
    for (size_t i = 0; i < nr; ++i) {
        gm[i] = Conv<T>::from(hm[i]);
        gl[i] = Conv<T>::from(hl[i]);
        tgt_m[i] = (float)rm[i];
        tgt_l[i] = (float)rl[i];
        const double em = std::fabs(gm[i] - rm[i]), el = std::fabs(gl[i] - rl[i]);
        max_m = std::fmax(max_m, em);
        max_l = std::fmax(max_l, el);
        if (ulp_ml && (em > ulp_of(rm[i], mant) || el > ulp_of(rl[i], mant))) {
            if (ok) std::printf("%s: m/l beyond 1 ulp at row %zu: m %g vs %g, l %g vs %g\n", name, i, gm[i], rm[i], gl[i], rl[i]);
            ok = false;
        }
    }
    std::printf("%s: max|dO| %.3g  max|dm| %.3g  max|dl| %.3g\n", name, max_o, max_m, max_l);
    if (ulp_ml) {
        ok = ok && max_o <= tol_o;
    } else {
        std::printf("testing m ...\n");
        ok = pmkl::utils::all_close(gm.data(), tgt_m.data(), nr, tol_ml, tol_ml) && ok;
        std::printf("testing l ...\n");
        ok = pmkl::utils::all_close(gl.data(), tgt_l.data(), nr, tol_ml, tol_ml) && ok;
        std::printf("testing out ...\n");
        ok = pmkl::utils::all_close(go.data(), tgt_o.data(), n, tol_o, tol_o) && ok;
    }
    std::printf("%s: %s\n", name, ok ? "ok" : "FAILED");
    return ok;
}

}  // namespace

int main() {
    std::printf("test_causal_attention: start\n");
    std::fflush(stdout);
    bool ok = true;
    // Reference shape and criterion (test_causal_attention.cpp:146-148, 197-204).
    ok = run_case<float, 64>("fp32 4x16x1024x64", 4, 16, 1024, 1e-5, 1e-5, false, 23, 20240601) && ok;
    ok = run_case<pmkl::bfloat16_t, 128>("bf16 2x4x512x128", 2, 4, 512, 1e-2, 0, true, 7, 20240602) && ok;
    ok = run_case<_Float16, 64>("fp16 2x4x512x64", 2, 4, 512, 2e-3, 0, true, 10, 20240603) && ok;

    // Error path of the reference launcher: seq_length % BLOCK_M != 0 throws.
    bool threw = false;
    try {
        pmkl::nlp::causal_attention_forward<float, 32, 64>(nullptr, nullptr, nullptr, nullptr, 1, 1, 33, nullptr,
                                                           nullptr);
    } catch (const pmkl::utils::Error &e) {
        threw = std::strstr(e.what(), "seq_length % BLOCK_M == 0") != nullptr;
    }
    std::printf("S %% 32 != 0 rejected: %s\n", threw ? "ok" : "FAILED");
    ok = ok && threw;
    // Empty problem returns without touching the (null) pointers.
    pmkl::nlp::causal_attention_forward<float, 32, 64>(nullptr, nullptr, nullptr, nullptr, 0, 4, 128, nullptr,
                                                       nullptr);
    std::printf("%s\n", ok ? "ok" : "FAILED");
    return ok ? 0 : 1;
}
