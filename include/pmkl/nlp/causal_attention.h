// pmkl/nlp/causal_attention.h - drop-in C++ entry point of the fused causal
// self-attention forward, same name and arguments as the reference
//   pmkl::nlp::causal_attention_forward<scalar_t, BLOCK_M, HIDDEN_SIZE>
//   (reference pmkl/nlp/causal_attention.h:258-288).
//
// Behaviour kept from the reference:
//   * CHECK_FAIL(seq_length % BLOCK_M == 0) and CHECK_FAIL(BLOCK_M == 32)
//     (:267-268), thrown as pmkl::utils::Error;
//   * early return for an empty problem (:270);
//   * the call is synchronous: it waits for the kernel (the reference
//     GpuLauncher syncs after every submit, cuda_launcher.h:274,334);
//   * scale 1/sqrt(HIDDEN_SIZE), m and l written in scalar_t.
// What changes: the work runs in the gfx950 kernels behind pmkl_attn.h, on
// pmkl::current_stream(); scalar_t may be float or a 16-bit type
// (pmkl::half_t / _Float16, pmkl::bfloat16_t / __bf16; other 16-bit types
// can specialise pmkl::dtype_code, pmkl/dtype.h); HIDDEN_SIZE may be 32, 64 or 128; launch
// errors are reported.  BLOCK_M is validated as in the reference but the tile
// shape is the kernel's own.
#pragma once

#include <cstdint>

#include "../../pmkl_attn.h"
#include "../core.h"
#include "../dtype.h"

namespace pmkl {
namespace nlp {

template <typename scalar_t, int BLOCK_M = 32, int HIDDEN_SIZE = 64>
void causal_attention_forward(scalar_t *out, const scalar_t *q, const scalar_t *k, const scalar_t *v,
                              const int batch_size, const int num_heads, const int seq_length, scalar_t *out_m,
                              scalar_t *out_l) {
    constexpr int WARP_SIZE = 32;  // the reference's row-tile contract, not the hardware wave size
    static_assert(dtype_code<scalar_t>::value >= 0, "scalar_t must be float or a 16-bit float type");
    static_assert(HIDDEN_SIZE == 32 || HIDDEN_SIZE == 64 || HIDDEN_SIZE == 128,
                  "HIDDEN_SIZE must be 32, 64 or 128");
    CHECK_FAIL(seq_length % BLOCK_M == 0);
    CHECK_FAIL(BLOCK_M == WARP_SIZE);

    if (batch_size * num_heads * seq_length == 0) return;

    hipStream_t stream = current_stream();
    const int rc = pmkl_causal_attention_forward(dtype_code<scalar_t>::value, out, q, k, v, batch_size, num_heads,
                                                 seq_length, HIDDEN_SIZE, out_m, out_l, (void *)stream);
    CHECK_FAIL(rc == PMKL_OK, pmkl_last_error());
    PMKL_HIP_CHECK(hipStreamSynchronize(stream));
}

}  // namespace nlp
}  // namespace pmkl
