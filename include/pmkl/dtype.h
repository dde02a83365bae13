// pmkl/dtype.h - element types of the C++ entry points and their pmkl_dtype
// codes (the dtype field of the C ABI, pmkl_attn.h).
//
// pmkl::dtype_code<T>::value is PMKL_DTYPE_F32 / _F16 / _BF16 for float and
// the 16-bit types below (and clang's _Float16 / __bf16), -1 otherwise.  Host
// code with another 16-bit storage type of the same bit layout can specialise
// it.
#pragma once

#include <cstdint>

#include "../pmkl_attn.h"

namespace pmkl {

// 16-bit storage types for host code that has no native half/bfloat16 type.
struct half_t {
    uint16_t bits;
};
struct bfloat16_t {
    uint16_t bits;
};

template <typename T>
struct dtype_code {
    static constexpr int value = -1;
};
template <>
struct dtype_code<float> {
    static constexpr int value = PMKL_DTYPE_F32;
};
template <>
struct dtype_code<half_t> {
    static constexpr int value = PMKL_DTYPE_F16;
};
template <>
struct dtype_code<bfloat16_t> {
    static constexpr int value = PMKL_DTYPE_BF16;
};
#if defined(__clang__)
template <>
struct dtype_code<_Float16> {
    static constexpr int value = PMKL_DTYPE_F16;
};
template <>
struct dtype_code<__bf16> {
    static constexpr int value = PMKL_DTYPE_BF16;
};
#endif

}  // namespace pmkl
