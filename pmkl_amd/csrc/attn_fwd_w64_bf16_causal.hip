// Explicit instantiations of the 64-row forward kernel for __bf16, causal:
// compiled as a translation unit of its own so that the library's kernels
// build in parallel (attn_capi.hip declares them extern).
#include <hip/hip_runtime.h>

#include "attn_fwd_w64.hpp"

namespace pmkl_amd {
template __global__ void attn_fwd_w64_kernel<__bf16, 64, true, 1, 8>(AttnParams);
template __global__ void attn_fwd_w64_kernel<__bf16, 64, true, 1, 4>(AttnParams);
template __global__ void attn_fwd_w64_kernel<__bf16, 128, true, 1, 8>(AttnParams);
template __global__ void attn_fwd_w64_kernel<__bf16, 32, true, 2, 4>(AttnParams);
template __global__ void attn_fwd_w64_kernel<__bf16, 64, true, 2, 4>(AttnParams);
template __global__ void attn_fwd_w64_kernel<__bf16, 128, true, 2, 4>(AttnParams);
}  // namespace pmkl_amd
