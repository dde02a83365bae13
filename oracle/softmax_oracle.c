/*
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle for the row
 * softmax / log-softmax.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker.  The
 * product path (pmkl_amd/, include/) never links or calls it.
 *
 * oracle_softmax_f64 restates, in float64, the per-row result of the reference
 * kernel warp_softmax_forward_impl (pmkl/norm/warp_softmax.h:74-157) behind
 * pmkl::norm::warp_softmax_forward (:159-201):
 *   m = max_i x_i                                         :108-118
 *   s = sum_i exp(x_i - m)                                :120-133
 *   softmax:     y_i = exp(x_i - m) / s, NaN if s == 0    :128, :147-150
 *   log-softmax: y_i = (x_i - m) - log(s)                 :126, :140, :146
 * over the elements x_i = src[r*stride + i], i < n, of row r, which is the row
 * placement of the reference's own CPU check (test/test_softmax.cpp:14-15).
 * The only deliberate difference: double instead of acc_t = float.  A NaN
 * element makes every output of its row NaN (through s), as in the reference.
 *
 * oracle_softmax_host_f32 is the reference's CPU check itself,
 * host_softmax_forward<float, float, float> (test/test_softmax.cpp:10-28),
 * op for op in float (max from -99999999, a sequential float sum, exp per
 * element twice, a division per element); it is the CPU baseline the
 * benchmark times.
 */
#include <math.h>
#include <stdint.h>

int oracle_softmax_f64(const double *src, int64_t n, int64_t stride, int64_t batch, int is_log, double *dst) {
    if (n < 0 || batch < 0 || stride < n) return -1;
    for (int64_t r = 0; r < batch; ++r) {
        const double *x = src + r * stride;
        double *y = dst + r * stride;
        double m = -INFINITY;
        int has_nan = 0;
        for (int64_t i = 0; i < n; ++i) {
            if (isnan(x[i])) has_nan = 1;
            if (x[i] > m) m = x[i];
        }
        double s = 0.0;
        for (int64_t i = 0; i < n; ++i) s += exp(x[i] - m);
        if (has_nan) s = NAN;
        for (int64_t i = 0; i < n; ++i) {
            if (is_log)
                y[i] = (x[i] - m) - log(s);
            else
                y[i] = s == 0.0 ? NAN : exp(x[i] - m) / s;
        }
    }
    return 0;
}

void oracle_softmax_host_f32(float *dst, const float *src, int softmax_elements, int softmax_elements_stride,
                             int batch_count) {
    for (int b = 0; b < batch_count; b++) {
        const float *src_b = src + (int64_t)b * softmax_elements_stride;
        float *dst_b = dst + (int64_t)b * softmax_elements_stride;
        float max_v = -99999999;
        for (int i = 0; i < softmax_elements; i++) max_v = src_b[i] > max_v ? src_b[i] : max_v;
        float sum = 0;
        for (int i = 0; i < softmax_elements; i++) sum += expf(src_b[i] - max_v);
        for (int i = 0; i < softmax_elements; i++) dst_b[i] = expf(src_b[i] - max_v) / sum;
    }
}
