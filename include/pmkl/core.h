// pmkl/core.h - the part of pmkl's core that the attention path and its tests
// use, rebuilt for HIP on MI355X.
//
//   pmkl::utils::Error / CHECK_FAIL   <- reference pmkl/core/utils/exception.h:13-161
//   pmkl::utils::all_close            <- reference pmkl/core/utils/measure.h:10-29
//   pmkl::DeviceBuffer                <- the device-allocation role of
//                                        reference pmkl/core/tensor.h:21-60,175-206
//                                        and GpuLauncher::malloc/free/memcpy
//                                        (pmkl/core/launcher/cuda_launcher.h:157-199)
//   pmkl::set_stream / current_stream <- GpuLauncher::stream_begin/stream_end
//                                        (cuda_launcher.h:125-138)
//
// The reference's launcher is a lambda-submitting singleton over CUDA or SYCL;
// here kernels are plain HIP launches behind the C ABI (pmkl_attn.h), so only
// buffers, a per-thread stream and the error convention remain.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <exception>
#include <iostream>
#include <sstream>
#include <string>
#include <utility>

namespace pmkl {
namespace utils {

// Exception thrown by CHECK_FAIL, with the message layout of the reference
// ("[enforce fail at file:line:func] Expected <cond> to be true, but got false. <msg>").
class Error : public std::exception {
    std::string what_;

public:
    Error(const char *func, const char *file, uint32_t line, const char *cond, const std::string &msg) {
        std::ostringstream oss;
        oss << "[enforce fail at " << file << ":" << line << ":" << func << "] " << cond << ". " << msg;
        what_ = oss.str();
    }
    explicit Error(std::string msg) : what_(std::move(msg)) {}
    const char *what() const noexcept override { return what_.c_str(); }
};

inline void stream_args(std::ostringstream &) {}
template <typename A, typename... R>
inline void stream_args(std::ostringstream &os, const A &a, const R &...r) {
    os << a;
    stream_args(os, r...);
}
template <typename... Args>
inline std::string check_msg(const Args &...args) {
    std::ostringstream os;
    stream_args(os, args...);
    return os.str();
}

#define CHECK_FAIL(cond, ...)                                                                          \
    if (__builtin_expect(!(cond), 0)) {                                                                \
        throw ::pmkl::utils::Error(__func__, __FILE__, static_cast<uint32_t>(__LINE__),               \
                                   "Expected " #cond " to be true, but got false",                     \
                                   ::pmkl::utils::check_msg(__VA_ARGS__));                              \
    }

// Elementwise |input - target| <= atol + rtol * |target|, NaN in input fails.
// Prints up to max_errors_print mismatches, as the reference does in DEBUG builds.
template <typename T>
bool all_close(const T *input, const T *target, size_t len, double atol = 1e-5, double rtol = 1e-5,
               int max_errors_print = 10) {
    size_t errors = 0;
    for (size_t i = 0; i < len; ++i) {
        const double a = (double)input[i], b = (double)target[i];
        if (std::isnan(a) || std::fabs(a - b) > atol + rtol * std::fabs(b)) {
            if ((int)errors < max_errors_print)
                std::cout << "Accuracy error: index[" << i << "], input: " << a << ", target: " << b << std::endl;
            ++errors;
        }
    }
    if (errors) std::cout << "Total " << errors << " errors\n";
    return errors == 0;
}

}  // namespace utils

// Stream used by the synchronous C++ entry points of this thread (the
// reference launcher uses one stream per process and is not thread-safe).
inline hipStream_t &current_stream_ref() {
    static thread_local hipStream_t s = nullptr;
    return s;
}
inline hipStream_t current_stream() { return current_stream_ref(); }
inline void set_stream(hipStream_t s) { current_stream_ref() = s; }

#define PMKL_HIP_CHECK(expr)                                                                            \
    do {                                                                                                \
        hipError_t e_ = (expr);                                                                         \
        CHECK_FAIL(e_ == hipSuccess, #expr, ": ", hipGetErrorString(e_));                               \
    } while (0)

// Owning device allocation (move-only).
class DeviceBuffer {
    void *ptr_ = nullptr;
    size_t bytes_ = 0;

public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) : bytes_(bytes) {
        if (bytes_) PMKL_HIP_CHECK(hipMalloc(&ptr_, bytes_));
    }
    ~DeviceBuffer() {
        if (ptr_) (void)hipFree(ptr_);
    }
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    DeviceBuffer(DeviceBuffer &&o) noexcept : ptr_(o.ptr_), bytes_(o.bytes_) {
        o.ptr_ = nullptr;
        o.bytes_ = 0;
    }
    DeviceBuffer &operator=(DeviceBuffer &&o) noexcept {
        std::swap(ptr_, o.ptr_);
        std::swap(bytes_, o.bytes_);
        return *this;
    }
    void *data() const { return ptr_; }
    template <typename T>
    T *as() const {
        return static_cast<T *>(ptr_);
    }
    size_t bytes() const { return bytes_; }
    void copy_from_host(const void *src) { PMKL_HIP_CHECK(hipMemcpy(ptr_, src, bytes_, hipMemcpyHostToDevice)); }
    void copy_to_host(void *dst) const { PMKL_HIP_CHECK(hipMemcpy(dst, ptr_, bytes_, hipMemcpyDeviceToHost)); }
};

}  // namespace pmkl
