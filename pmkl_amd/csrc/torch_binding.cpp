// pmkl_pytorch_ext: the PyTorch-ROCm operators of the fused self-attention
// forward and backward, rebuilt as a binding over the C ABI in
// include/pmkl_attn.h.
//
// Replaces pmkl_pytorch_ext/fused_self_attention.cpp:139-173, :175-215 and
// :217-220 of the reference (same module name, function names, arguments,
// return tuples and TORCH_CHECK messages).  The reference has only CPU
// bodies; for the forward this binding
//   * sends tensors on a ROCm device to pmkl_attn_fwd (the gfx950 kernels), on
//     the current HIP stream, with no host synchronisation;
//   * keeps the CPU body for CPU tensors: host_attention_forward below computes
//     exactly what the reference CPU operator computes (same per-element
//     operation sequence in scalar_t, so c10 Half/BFloat16 round after every
//     operation and the softmax denominator is accumulated in double), with the
//     heads spread over at::parallel_for threads.  Device tensors never reach it.
// Outputs are allocated contiguous [B, H, S, D] (the reference uses
// empty_like(v), which keeps a strided v's layout while the body writes it as
// if it were contiguous); out_m and out_l are [B, H, S] in v's dtype.
// The backward does the same split: device tensors (fp16 / bf16) go to
// pmkl_attn_bwd with a workspace from torch's allocator, CPU tensors to
// host_attention_backward, the reference's per-element steps.
#include <torch/extension.h>

#include <ATen/Parallel.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <cmath>
#include <limits>

#include "../../include/pmkl_attn.h"

namespace {

// CPU body.  Per head b and query row i, the same steps as the reference
// (fused_self_attention.cpp:13-63): full-length score row in scalar_t,
// -inf mask, max, double denominator, p = exp(s - max) / e2sum rounded to
// scalar_t, then o_i = sum_j p_ij v_j accumulated in scalar_t in key order.
// The row is kept in a length-S buffer instead of an S x S matrix, and the PV
// sum walks keys in the outer loop; every output element still sees the same
// operations in the same order.
template <typename scalar_t>
void host_attention_forward(scalar_t *o, const scalar_t *q, const scalar_t *k, const scalar_t *v, int64_t BH,
                            int64_t S, int64_t D, bool is_causal, scalar_t *out_m, scalar_t *out_l) {
    const scalar_t neg_inf = -std::numeric_limits<scalar_t>::infinity();
    const float scale = 1.0f / std::sqrt((float)D);
    at::parallel_for(0, BH, 1, [&](int64_t begin, int64_t end) {
        std::vector<scalar_t> row((size_t)S);
        std::vector<scalar_t> acc((size_t)D);
        for (int64_t b = begin; b < end; ++b) {
            const scalar_t *qb = q + b * S * D;
            const scalar_t *kb = k + b * S * D;
            const scalar_t *vb = v + b * S * D;
            scalar_t *ob = o + b * S * D;
            for (int64_t i = 0; i < S; ++i) {
                const scalar_t *qi = qb + i * D;
                const int64_t visible = is_causal ? i + 1 : S;
                for (int64_t j = 0; j < visible; ++j) {
                    const scalar_t *kj = kb + j * D;
                    scalar_t dot = 0;
                    for (int64_t d = 0; d < D; ++d) dot += qi[d] * kj[d];
                    row[j] = dot * scale;
                }
                for (int64_t j = visible; j < S; ++j) row[j] = neg_inf;
                scalar_t mx = neg_inf;
                for (int64_t j = 0; j < S; ++j) mx = std::max(row[j], mx);
                double denom = 0;
                for (int64_t j = 0; j < S; ++j) denom += std::exp((double)row[j] - mx);
                out_m[b * S + i] = mx;
                out_l[b * S + i] = denom;
                for (int64_t d = 0; d < D; ++d) acc[d] = 0;
                for (int64_t j = 0; j < S; ++j) {
                    const scalar_t pj = std::exp(row[j] - mx) / denom;
                    const scalar_t *vj = vb + j * D;
                    for (int64_t d = 0; d < D; ++d) acc[d] += pj * vj[d];
                }
                for (int64_t d = 0; d < D; ++d) ob[i * D + d] = acc[d];
            }
        }
    });
}

// CPU body of the backward.  Per head, the reference's loops
// (fused_self_attention.cpp:66-135): key m outer, query n inner; the score and
// probability of (n, m) in scalar_t, dv_m += p dout_n, then the softmax
// Jacobian row sum acc_d over every key (recomputing each other probability,
// kept in the type `auto` gives it there), scaled, and dq_n += acc_d k_m,
// dk_m += acc_d q_n.  Same operations, types and order per output element, so
// fp16 / bf16 results round exactly as the reference's do.  O(S^3 D): for
// debugging and small problems, like the reference.
template <typename scalar_t>
void host_attention_backward(scalar_t *dq, scalar_t *dk, scalar_t *dv, const scalar_t *dout, const scalar_t *q,
                             const scalar_t *k, const scalar_t *v, const scalar_t *out_m, const scalar_t *out_l,
                             int64_t BH, int64_t S, int64_t D, bool is_causal) {
    const scalar_t neg_inf = -std::numeric_limits<scalar_t>::infinity();
    at::parallel_for(0, BH, 1, [&](int64_t begin, int64_t end) {
        for (int64_t b = begin; b < end; ++b) {
            const int64_t ob = b * S * D;
            const scalar_t *qb = q + ob, *kb = k + ob, *vb = v + ob, *gb = dout + ob;
            scalar_t *dqb = dq + ob, *dkb = dk + ob, *dvb = dv + ob;
            const scalar_t *mb = out_m + b * S, *lb = out_l + b * S;
            auto score = [&](int64_t n, int64_t key) {
                scalar_t s = 0;
                for (int64_t d = 0; d < D; ++d) s += qb[n * D + d] * kb[key * D + d];
                s = s * (1.0f / std::sqrt((float)D));
                if (is_causal) s = n >= key ? s : neg_inf;
                return s;
            };
            for (int64_t key = 0; key < S; ++key) {
                for (int64_t n = 0; n < S; ++n) {
                    const scalar_t s = score(n, key);
                    const scalar_t p = std::exp(s - mb[n]) / lb[n];
                    for (int64_t d = 0; d < D; ++d) dvb[key * D + d] += p * gb[n * D + d];
                    scalar_t acc_d = 0;
                    for (int64_t other = 0; other < S; ++other) {
                        scalar_t dpv = 0;
                        for (int64_t d = 0; d < D; ++d) dpv += gb[n * D + d] * vb[other * D + d];
                        scalar_t term;
                        if (other == key) {
                            term = dpv * p * (1 - p);
                        } else {
                            const scalar_t s2 = score(n, other);
                            auto p2 = std::exp(s2 - mb[n]) / lb[n];
                            term = -dpv * p2 * p;
                        }
                        term *= (1.0f / std::sqrt((float)D));
                        acc_d += term;
                    }
                    for (int64_t d = 0; d < D; ++d) dqb[n * D + d] += acc_d * kb[key * D + d];
                    for (int64_t d = 0; d < D; ++d) dkb[key * D + d] += acc_d * qb[n * D + d];
                }
            }
        }
    });
}

int32_t to_pmkl_dtype(at::ScalarType t) {
    switch (t) {
        case at::kFloat: return PMKL_DTYPE_F32;
        case at::kHalf: return PMKL_DTYPE_F16;
        case at::kBFloat16: return PMKL_DTYPE_BF16;
        default: return -1;
    }
}

// A device tensor the kernels can read in place: head_dim contiguous, 16-byte
// aligned base and strides.  Anything else is copied contiguous first, as the
// reference does with .contiguous() (fused_self_attention.cpp:160-162).
at::Tensor device_view(const at::Tensor &t) {
    const int64_t vec = 16 / t.element_size();
    const bool ok = t.stride(3) == 1 && t.stride(0) % vec == 0 && t.stride(1) % vec == 0 && t.stride(2) % vec == 0 &&
                    t.stride(2) >= t.size(3) && (reinterpret_cast<uintptr_t>(t.data_ptr()) % 16) == 0;
    return ok ? t : t.contiguous();
}

void fill_strides(int64_t dst[3], const at::Tensor &t) {
    dst[0] = t.stride(0);
    dst[1] = t.stride(1);
    dst[2] = t.stride(2);
}

}  // namespace

std::tuple<at::Tensor, at::Tensor, at::Tensor> fused_self_attention_fw(const at::Tensor &q, const at::Tensor &k,
                                                                       const at::Tensor &v, bool is_causal) {
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "Input tensor shapes must match");
    TORCH_CHECK(q.sizes() == k.sizes() && q.sizes() == v.sizes(), "Input tensor shapes must match");
    TORCH_CHECK(q.scalar_type() == k.scalar_type() && q.scalar_type() == v.scalar_type(),
                "Input tensor dtypes must match");
    TORCH_CHECK(q.device() == k.device() && q.device() == v.device(), "Input tensors must be on one device");

    const int64_t B = q.size(0), H = q.size(1), S = q.size(2), D = q.size(3);
    auto opts = v.options().memory_format(at::MemoryFormat::Contiguous);
    auto out = at::empty({B, H, S, D}, opts);
    auto out_m = at::empty({B, H, S}, opts);
    auto out_l = at::empty({B, H, S}, opts);

    if (q.is_cpu()) {
        AT_DISPATCH_FLOATING_TYPES_AND2(at::ScalarType::Half, at::ScalarType::BFloat16, v.scalar_type(),
                                        "fused_self_attention_fw", [&]() {
                                            auto qc = q.contiguous(), kc = k.contiguous(), vc = v.contiguous();
                                            host_attention_forward<scalar_t>(
                                                out.data_ptr<scalar_t>(), qc.data_ptr<scalar_t>(),
                                                kc.data_ptr<scalar_t>(), vc.data_ptr<scalar_t>(), B * H, S, D,
                                                is_causal, out_m.data_ptr<scalar_t>(), out_l.data_ptr<scalar_t>());
                                        });
        return std::forward_as_tuple(out, out_m, out_l);
    }

    TORCH_CHECK(q.is_cuda(), "fused_self_attention_fw: tensors must be on the CPU or a ROCm device, got ",
                q.device());
    const int32_t dt = to_pmkl_dtype(q.scalar_type());
    TORCH_CHECK(dt >= 0, "fused_self_attention_fw: device path supports float32, float16 and bfloat16, got ",
                q.scalar_type());
    TORCH_CHECK(pmkl_attn_fwd_supported(dt, D), "fused_self_attention_fw: head_dim ", D,
                " is not supported on the device (supported: 32, 64, 128)");
    if (B * H * S == 0) return std::forward_as_tuple(out, out_m, out_l);

    c10::OptionalDeviceGuard guard(q.device());
    auto qd = device_view(q), kd = device_view(k), vd = device_view(v);
    pmkl_attn_fwd_args a;
    std::memset(&a, 0, sizeof(a));
    a.q = qd.data_ptr();
    a.k = kd.data_ptr();
    a.v = vd.data_ptr();
    a.o = out.data_ptr();
    a.m = out_m.data_ptr();
    a.l = out_l.data_ptr();
    a.dtype = dt;
    a.ml_dtype = dt;
    a.batch = B;
    a.heads = H;
    a.seq_len = S;
    a.head_dim = D;
    fill_strides(a.q_strides, qd);
    fill_strides(a.k_strides, kd);
    fill_strides(a.v_strides, vd);
    fill_strides(a.o_strides, out);
    a.scale = 0.f;
    a.is_causal = is_causal ? 1 : 0;
    hipStream_t stream = c10::hip::getCurrentHIPStream(q.device().index()).stream();
    const int rc = pmkl_attn_fwd(&a, (void *)stream);
    TORCH_CHECK(rc == PMKL_OK, "fused_self_attention_fw: ", pmkl_last_error());
    return std::forward_as_tuple(out, out_m, out_l);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> fused_self_attention_bw(const at::Tensor &dout, const at::Tensor &q,
                                                                       const at::Tensor &k, const at::Tensor &v,
                                                                       const at::Tensor &out_m,
                                                                       const at::Tensor &out_l, bool is_causal) {
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "Input tensor shapes must match");
    // The CPU body indexes contiguous rows, as the reference's does (its check
    // and message, fused_self_attention.cpp:181-182); the device backward takes
    // any strides with head_dim contiguous, without copies.
    TORCH_CHECK(!q.is_cpu() || (q.is_contiguous() && k.is_contiguous() && v.is_contiguous()),
                "Input tensor must be contiguous");
    TORCH_CHECK(q.sizes() == k.sizes() && q.sizes() == v.sizes(), "Input tensor shapes must match");
    TORCH_CHECK(dout.sizes() == q.sizes(), "dout must have the shape of q");
    const int64_t B = q.size(0), H = q.size(1), S = q.size(2), D = q.size(3);
    TORCH_CHECK(out_m.numel() == B * H * S && out_l.numel() == B * H * S, "out_m / out_l must hold B*H*S elements");
    TORCH_CHECK(q.scalar_type() == k.scalar_type() && q.scalar_type() == v.scalar_type() &&
                    q.scalar_type() == dout.scalar_type(),
                "Input tensor dtypes must match");
    // Every tensor on q's device before anything is dispatched: a host
    // pointer handed to a kernel (or a device pointer to the CPU body) would
    // be dereferenced on the wrong side.
    TORCH_CHECK(dout.device() == q.device() && k.device() == q.device() && v.device() == q.device() &&
                    out_m.device() == q.device() && out_l.device() == q.device(),
                "Input tensors must be on one device");

    if (q.is_cpu()) {
        auto dq = at::zeros_like(q);
        auto dk = at::zeros_like(k);
        auto dv = at::zeros_like(v);
        auto doc = dout.contiguous();
        AT_DISPATCH_FLOATING_TYPES_AND2(at::ScalarType::Half, at::ScalarType::BFloat16, v.scalar_type(),
                                        "fused_self_attention_bw", [&]() {
                                            auto mc = out_m.contiguous().to(v.scalar_type());
                                            auto lc = out_l.contiguous().to(v.scalar_type());
                                            host_attention_backward<scalar_t>(
                                                dq.data_ptr<scalar_t>(), dk.data_ptr<scalar_t>(),
                                                dv.data_ptr<scalar_t>(), doc.data_ptr<scalar_t>(),
                                                q.data_ptr<scalar_t>(), k.data_ptr<scalar_t>(),
                                                v.data_ptr<scalar_t>(), mc.data_ptr<scalar_t>(),
                                                lc.data_ptr<scalar_t>(), B * H, S, D, is_causal);
                                        });
        return std::forward_as_tuple(dq, dk, dv);
    }

    TORCH_CHECK(q.is_cuda(), "fused_self_attention_bw: tensors must be on the CPU or a ROCm device, got ",
                q.device());
    const int32_t dt = to_pmkl_dtype(q.scalar_type());
    TORCH_CHECK(pmkl_attn_bwd_supported(dt, D), "fused_self_attention_bw: the device backward supports float32, ",
                "float16 and bfloat16 with head_dim 32, 64 or 128, got ", q.scalar_type(), " head_dim ", D);
    // Gradients come back contiguous [B, H, S, D]; the kernels write every element.
    auto gopts = q.options().memory_format(at::MemoryFormat::Contiguous);
    auto dq = at::empty({B, H, S, D}, gopts);
    auto dk = at::empty({B, H, S, D}, gopts);
    auto dv = at::empty({B, H, S, D}, gopts);
    if (B * H * S == 0) return std::forward_as_tuple(dq, dk, dv);
    const int32_t mdt = to_pmkl_dtype(out_m.scalar_type());
    TORCH_CHECK(out_m.scalar_type() == out_l.scalar_type() && (mdt == dt || mdt == PMKL_DTYPE_F32),
                "fused_self_attention_bw: out_m / out_l must be in the tensors' dtype or float32");

    c10::OptionalDeviceGuard guard(q.device());
    auto mc = out_m.contiguous(), lc = out_l.contiguous();
    // Strided views go to the kernels as they are; only a layout the kernels
    // cannot address (head_dim not contiguous, strides or base not 16-byte
    // aligned) is copied.
    auto qd = device_view(q), kd = device_view(k), vd = device_view(v), dod = device_view(dout);
    const uint64_t ws_bytes = pmkl_attn_bwd_workspace_size(B, H, S);
    auto ws = at::empty({(int64_t)((ws_bytes + 3) / 4)}, q.options().dtype(at::kFloat));
    pmkl_attn_bwd_args a;
    std::memset(&a, 0, sizeof(a));
    a.dout = dod.data_ptr();
    a.q = qd.data_ptr();
    a.k = kd.data_ptr();
    a.v = vd.data_ptr();
    fill_strides(a.dout_strides, dod);
    fill_strides(a.q_strides, qd);
    fill_strides(a.k_strides, kd);
    fill_strides(a.v_strides, vd);
    fill_strides(a.dq_strides, dq);
    fill_strides(a.dk_strides, dk);
    fill_strides(a.dv_strides, dv);
    a.o = nullptr;
    a.m = mc.data_ptr();
    a.l = lc.data_ptr();
    a.dq = dq.data_ptr();
    a.dk = dk.data_ptr();
    a.dv = dv.data_ptr();
    a.workspace = ws.data_ptr();
    a.workspace_bytes = (uint64_t)ws.numel() * 4;
    a.dtype = dt;
    a.ml_dtype = mdt;
    a.batch = B;
    a.heads = H;
    a.seq_len = S;
    a.head_dim = D;
    a.scale = 0.f;
    a.is_causal = is_causal ? 1 : 0;
    hipStream_t stream = c10::hip::getCurrentHIPStream(q.device().index()).stream();
    const int rc = pmkl_attn_bwd(&a, (void *)stream);
    TORCH_CHECK(rc == PMKL_OK, "fused_self_attention_bw: ", pmkl_last_error());
    return std::forward_as_tuple(dq, dk, dv);
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("fused_self_attention_fw", &fused_self_attention_fw, "fused_self_attention_fw",
          pybind11::arg("q"), pybind11::arg("k"), pybind11::arg("v"), pybind11::arg("is_causal"));
    m.def("fused_self_attention_bw", &fused_self_attention_bw, "fused_self_attention_bw",
          pybind11::arg("dout"), pybind11::arg("q"), pybind11::arg("k"), pybind11::arg("v"),
          pybind11::arg("out_m"), pybind11::arg("out_l"), pybind11::arg("is_causal"));
}
