/*
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle for the causal
 * self-attention forward path.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker.  The
 * product path (pmkl_amd/, include/) never links or calls it.
 *
 * It restates, in float64 accumulation, the reference CPU algorithm
 *   pmkl_pytorch_ext/fused_self_attention.cpp:5-64   (host_self_attention_forward)
 * which is identical to the host oracle of
 *   test/test_causal_attention.cpp:11-70
 * and the output definitions of the reference GPU kernel
 *   pmkl/nlp/causal_attention.h:176-255   (m = row max of the scaled, masked
 *   logits; l = sum_j exp(s_ij - m_i), not a log-sum-exp).
 *
 * Per (head, query row i) it does what the reference does per row:
 *   s_ij = (sum_d q_id * k_jd) * scale        fused_self_attention.cpp:23-32
 *     with scale = 1.0f / sqrtf((float)D) rounded to float first (:30); the
 *     caller may pass another scale (the C ABI accepts one).
 *   s_ij = -inf for j > i when causal          :33-37
 *   m_i  = max_j s_ij                          :38-43
 *   l_i  = sum_j exp(s_ij - m_i) in double     :44-48
 *   p_ij = exp(s_ij - m_i) / l_i               :49-51
 *   o_id = sum_j p_ij * v_jd                   :53-61
 * The only deliberate difference: every operation is carried out in double
 * instead of scalar_t, which is the fp32+ accumulation reference against which
 * the tolerances of the path are stated.
 *
 * The backward (oracle_attn_bwd below) restates, in float64,
 *   pmkl_pytorch_ext/fused_self_attention.cpp:66-135 (host_self_attention_backward)
 * for the gradients of O only (as the reference's autograd backward, which
 * ignores the gradients of m and l, pmkl_function/__init__.py:25-32).  Per
 * head, query n and key j it does what the reference does:
 *   s_nj  = (q_n . k_j) * scale, -inf for j > n when causal       :88-93
 *   p_nj  = exp(s_nj - m_n) / l_n, with the m, l the forward returned   :94
 *   dv_j += p_nj * dout_n                                           :96-98
 *   acc   = scale * sum_j' dP_nj' * (j' == j ? p_nj (1 - p_nj) : -p_nj' p_nj),
 *           dP_nj' = dout_n . v_j'                                  :101-124
 *         = scale * p_nj * (dP_nj - sum_j' p_nj' dP_nj')   (same sum, regrouped)
 *   dq_n += acc * k_j;   dk_j += acc * q_n                          :126-131
 *
 * Parity of this restatement is pinned in tests/test_oracle.py against
 * closed forms (K == 0, constant V, row 0, single key), against
 * torch.nn.functional.scaled_dot_product_attention in float64 (the
 * reference's own Python oracle, test_fused_self_attention.py:6-7), against
 * brute force on tiny shapes, and against the reference's own CPU operator
 * compiled from its source into oracle/_ref when that build is present; the
 * backward against torch autograd through SDPA in float64, against central
 * differences of the forward, and against the reference's own backward
 * operator (float64) from oracle/_ref.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Reference scale: 1.0f / std::sqrt((float)hidden_size), fused_self_attention.cpp:30. */
double oracle_default_scale(int64_t D) {
    float s = 1.0f / sqrtf((float)D);
    return (double)s;
}

/*
 * q, k, v: [BH, S, D] float32 (values are exact upcasts of the test dtype).
 * rows: NULL -> all S rows of every head; otherwise nrows row indices that are
 *       evaluated in every head.
 * o:  [BH, nrows, D]  double;  m, l: [BH, nrows] double.
 * Returns 0, or -1 on bad arguments or allocation failure.
 */
int oracle_attn_fwd_rows(const float *q, const float *k, const float *v,
                         int64_t BH, int64_t S, int64_t D, int causal, double scale,
                         const int64_t *rows, int64_t nrows,
                         double *o, double *m, double *l) {
    if (BH < 0 || S < 0 || D <= 0) return -1;
    if (rows == NULL) nrows = S;
    for (int64_t r = 0; rows != NULL && r < nrows; ++r)
        if (rows[r] < 0 || rows[r] >= S) return -1;
    int bad = 0;
#pragma omp parallel
    {
        double *srow = (double *)malloc(sizeof(double) * (size_t)(S > 0 ? S : 1));
        double *acc = (double *)malloc(sizeof(double) * (size_t)D);
        if (srow == NULL || acc == NULL) {
#pragma omp atomic write
            bad = 1;
        } else {
#pragma omp for schedule(dynamic, 1) collapse(2)
            for (int64_t b = 0; b < BH; ++b) {
                for (int64_t r = 0; r < nrows; ++r) {
                    const int64_t i = rows ? rows[r] : r;
                    const float *qi = q + (b * S + i) * D;
                    const float *kb = k + b * S * D;
                    const float *vb = v + b * S * D;
                    /* scores over the full row, then the mask (reference order) */
                    for (int64_t j = 0; j < S; ++j) {
                        const float *kj = kb + j * D;
                        double sum = 0.0;
                        for (int64_t d = 0; d < D; ++d) sum += (double)qi[d] * (double)kj[d];
                        srow[j] = sum * scale;
                    }
                    if (causal)
                        for (int64_t j = i + 1; j < S; ++j) srow[j] = -INFINITY;
                    double mx = -INFINITY;
                    for (int64_t j = 0; j < S; ++j) mx = srow[j] > mx ? srow[j] : mx;
                    double e2sum = 0.0;
                    for (int64_t j = 0; j < S; ++j) e2sum += exp(srow[j] - mx);
                    memset(acc, 0, sizeof(double) * (size_t)D);
                    for (int64_t j = 0; j < S; ++j) {
                        const double p = exp(srow[j] - mx) / e2sum;
                        if (p == 0.0) continue; /* masked keys add exact zeros */
                        const float *vj = vb + j * D;
                        for (int64_t d = 0; d < D; ++d) acc[d] += p * (double)vj[d];
                    }
                    double *ob = o + (b * nrows + r) * D;
                    for (int64_t d = 0; d < D; ++d) ob[d] = acc[d];
                    m[b * nrows + r] = mx;
                    l[b * nrows + r] = e2sum;
                }
            }
        }
        free(srow);
        free(acc);
    }
    return bad ? -1 : 0;
}

/* Round-to-nearest-even float -> bfloat16 bits, as torch.Tensor.to(torch.bfloat16)
 * and c10::detail::round_to_nearest_even do (NaN -> quiet NaN 0x7fc0). */
uint16_t oracle_f32_to_bf16_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

void oracle_round_bf16(const float *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        uint32_t u = (uint32_t)oracle_f32_to_bf16_bits(src[i]) << 16;
        memcpy(&dst[i], &u, 4);
    }
}

/*
 * Backward of O (see the header).  q, k, v, dout: [BH, S, D] float32;
 * m, l: [BH, S] double, the forward's outputs (as the caller holds them).
 * heads: NULL -> every head; otherwise nheads head indices.
 * dq, dk, dv: [nheads, S, D] double.
 * Returns 0, or -1 on bad arguments or allocation failure.
 */
int oracle_attn_bwd(const float *q, const float *k, const float *v, const float *dout,
                    const double *m, const double *l, int64_t BH, int64_t S, int64_t D, int causal,
                    double scale, const int64_t *heads, int64_t nheads, double *dq, double *dk, double *dv) {
    if (BH < 0 || S < 0 || D <= 0) return -1;
    if (heads == NULL) nheads = BH;
    for (int64_t h = 0; heads != NULL && h < nheads; ++h)
        if (heads[h] < 0 || heads[h] >= BH) return -1;
    const size_t sd = (size_t)(S * D > 0 ? S * D : 1);
    int nthr = 1;
#pragma omp parallel
#pragma omp single
    nthr = omp_get_num_threads();
    /* per-thread partial sums of dk, dv, added in thread order afterwards
     * (static row schedule): the result does not depend on timing */
    double *part = (double *)calloc(2 * sd * (size_t)nthr, sizeof(double));
    if (part == NULL) return -1;
    int bad = 0;
    for (int64_t hh = 0; hh < nheads && !bad; ++hh) {
        const int64_t b = heads ? heads[hh] : hh;
        const float *qb = q + b * S * D, *kb = k + b * S * D, *vb = v + b * S * D, *ob = dout + b * S * D;
        const double *mb = m + b * S, *lb = l + b * S;
        double *dqh = dq + hh * S * D, *dkh = dk + hh * S * D, *dvh = dv + hh * S * D;
        memset(part, 0, sizeof(double) * 2 * sd * (size_t)nthr);
#pragma omp parallel num_threads(nthr)
        {
            const int tid = omp_get_thread_num();
            double *dkt = part + 2 * sd * (size_t)tid, *dvt = dkt + sd;
            double *p = (double *)malloc(sizeof(double) * (size_t)(S > 0 ? S : 1));
            double *dp = (double *)malloc(sizeof(double) * (size_t)(S > 0 ? S : 1));
            if (p == NULL || dp == NULL) {
#pragma omp atomic write
                bad = 1;
            } else {
#pragma omp for schedule(static)
                for (int64_t n = 0; n < S; ++n) {
                    const float *qn = qb + n * D, *on = ob + n * D;
                    double dsum = 0.0;
                    for (int64_t j = 0; j < S; ++j) {
                        double s = 0.0, t = 0.0;
                        const float *kj = kb + j * D, *vj = vb + j * D;
                        for (int64_t d = 0; d < D; ++d) {
                            s += (double)qn[d] * (double)kj[d];
                            t += (double)on[d] * (double)vj[d];
                        }
                        s *= scale;
                        if (causal && j > n) s = -INFINITY;
                        p[j] = exp(s - mb[n]) / lb[n];
                        dp[j] = t;
                        dsum += p[j] * t;
                    }
                    double *dqn = dqh + n * D;
                    for (int64_t d = 0; d < D; ++d) dqn[d] = 0.0;
                    for (int64_t j = 0; j < S; ++j) {
                        if (p[j] == 0.0) continue; /* masked keys add exact zeros */
                        const double ds = scale * p[j] * (dp[j] - dsum);
                        const float *kj = kb + j * D;
                        double *dkj = dkt + j * D, *dvj = dvt + j * D;
                        for (int64_t d = 0; d < D; ++d) {
                            dqn[d] += ds * (double)kj[d];
                            dkj[d] += ds * (double)qn[d];
                            dvj[d] += p[j] * (double)on[d];
                        }
                    }
                }
            }
            free(p);
            free(dp);
        }
        for (size_t i = 0; i < (size_t)(S * D); ++i) {
            double sk = 0.0, sv = 0.0;
            for (int t = 0; t < nthr; ++t) {
                sk += part[2 * sd * (size_t)t + i];
                sv += part[2 * sd * (size_t)t + sd + i];
            }
            dkh[i] = sk;
            dvh[i] = sv;
        }
    }
    free(part);
    return bad ? -1 : 0;
}
