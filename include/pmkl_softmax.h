/*
 * pmkl_softmax.h - C ABI of the MI355X (gfx950) row softmax / log-softmax.
 *
 * Interface replaced:
 *   pmkl::norm::warp_softmax_forward<output_t, input_t, acc_t, is_log_softmax>(
 *       dst, src, softmax_elements, softmax_elements_stride, batch_count)
 *       -> reference pmkl/norm/warp_softmax.h:159-201 (kernel body :74-157)
 *
 * Semantics, per row r = 0 .. batch-1 over the elements x_i = src[r*stride + i],
 * i = 0 .. elements-1, evaluated in fp32 (the reference's acc_t = float):
 *   m   = max_i x_i
 *   s   = sum_i exp(x_i - m)
 *   softmax:      dst[r*stride + i] = exp(x_i - m) / s     (NaN where s == 0)
 *   log-softmax:  dst[r*stride + i] = (x_i - m) - log(s)
 * Elements between `elements` and `stride` in a row are neither read nor
 * written.  dst may equal src (in place) when the dtypes match.
 *
 * Row addressing: the reference kernel places row first_batch + i of a warp at
 * first_batch*stride + i*elements (warp_softmax.h:88,101,146), which is row
 * r*stride only when stride == elements, its one tested layout
 * (test/test_softmax.cpp:49).  This library always places row r at r*stride;
 * both agree whenever stride == elements.
 *
 * Contract: the caller allocates src and dst in device memory; the call
 * allocates nothing and is asynchronous on the given stream (NULL = default
 * stream); re-entrant; errors leave text in pmkl_last_error().
 */
#ifndef PMKL_SOFTMAX_H_
#define PMKL_SOFTMAX_H_

#include <stdint.h>

#include "pmkl_attn.h" /* pmkl_dtype, pmkl_status, pmkl_last_error */

#ifdef __cplusplus
extern "C" {
#endif

/* The reference's CHECK_FAIL(softmax_elements >= 0 && softmax_elements <= 1024)
 * (warp_softmax.h:162). */
#define PMKL_SOFTMAX_MAX_ELEMENTS 1024

typedef struct pmkl_softmax_args {
    void *dst;           /* [batch, stride] of out_dtype                         */
    const void *src;     /* [batch, stride] of in_dtype                          */
    int32_t out_dtype;   /* pmkl_dtype of dst (output_t)                         */
    int32_t in_dtype;    /* pmkl_dtype of src (input_t)                          */
    int64_t elements;    /* softmax_elements: 0 .. PMKL_SOFTMAX_MAX_ELEMENTS     */
    int64_t stride;      /* softmax_elements_stride (elements), >= elements      */
    int64_t batch;       /* batch_count: 0 .. 2^31 - 1                           */
    int32_t is_log;      /* is_log_softmax                                       */
} pmkl_softmax_args;

/* Row softmax or log-softmax.  Returns PMKL_OK, or
 *   PMKL_EINVAL       elements outside 0..1024, stride < elements, batch out of
 *                     range, a null pointer with work to do, an unknown dtype,
 *                     or in-place with different dtypes;
 *   PMKL_EHIP         the launch failed.
 * elements == 0 or batch == 0 returns PMKL_OK without launching, as the
 * reference returns early for softmax_elements == 0 (warp_softmax.h:163-164).
 * Replaces pmkl/norm/warp_softmax.h:159-201. */
int pmkl_softmax_fwd(const pmkl_softmax_args *a, void *stream);

/* Positional form mirroring the reference template's argument order
 * (warp_softmax.h:160-161): dst, src, softmax_elements,
 * softmax_elements_stride, batch_count; the template parameters become
 * out_dtype, in_dtype and is_log. */
int pmkl_warp_softmax_forward(int32_t out_dtype, int32_t in_dtype, int32_t is_log, void *dst, const void *src,
                              int64_t softmax_elements, int64_t softmax_elements_stride, int64_t batch_count,
                              void *stream);

#ifdef __cplusplus
}
#endif

#endif /* PMKL_SOFTMAX_H_ */
