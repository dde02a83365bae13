// pmkl/norm/warp_softmax.h - drop-in C++ entry point of the row softmax, same
// name and arguments as the reference
//   pmkl::norm::warp_softmax_forward<output_t, input_t, acc_t, is_log_softmax>(
//       dst, src, softmax_elements, softmax_elements_stride, batch_count)
//   (reference pmkl/norm/warp_softmax.h:159-201).
//
// Behaviour kept from the reference:
//   * CHECK_FAIL(softmax_elements >= 0 && softmax_elements <= 1024) (:162),
//     thrown as pmkl::utils::Error;
//   * early return for softmax_elements == 0 (:163-164);
//   * the call is synchronous (the reference GpuLauncher syncs after every
//     submit, cuda_launcher.h:334);
//   * per-row results: softmax exp(x - max) / sum, NaN where the sum is 0;
//     log-softmax (x - max) - log(sum) (:120-156).
// What changes: the work runs in the gfx950 kernel behind pmkl_softmax.h on
// pmkl::current_stream(); output_t and input_t may each be float or a 16-bit
// type (pmkl/dtype.h); acc_t must be float (the kernel accumulates in fp32);
// launch errors are reported; row r always starts at r * stride (the
// reference kernel agrees with that only when stride == elements).
#pragma once

#include <type_traits>

#include "../../pmkl_softmax.h"
#include "../core.h"
#include "../dtype.h"

namespace pmkl {
namespace norm {

template <typename output_t, typename input_t, typename acc_t, bool is_log_softmax>
void warp_softmax_forward(output_t *dst, const input_t *src, int softmax_elements, int softmax_elements_stride,
                          int batch_count) {
    static_assert(dtype_code<output_t>::value >= 0 && dtype_code<input_t>::value >= 0,
                  "output_t and input_t must be float or a 16-bit float type");
    static_assert(std::is_same<acc_t, float>::value, "acc_t must be float: the kernel accumulates in fp32");
    CHECK_FAIL(softmax_elements >= 0 && softmax_elements <= PMKL_SOFTMAX_MAX_ELEMENTS);
    if (softmax_elements == 0) return;

    hipStream_t stream = current_stream();
    const int rc = pmkl_warp_softmax_forward(dtype_code<output_t>::value, dtype_code<input_t>::value,
                                             is_log_softmax ? 1 : 0, dst, src, softmax_elements,
                                             softmax_elements_stride, batch_count, (void *)stream);
    CHECK_FAIL(rc == PMKL_OK, pmkl_last_error());
    PMKL_HIP_CHECK(hipStreamSynchronize(stream));
}

}  // namespace norm
}  // namespace pmkl
