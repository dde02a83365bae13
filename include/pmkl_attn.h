/*
 * pmkl_attn.h - C ABI of the MI355X (gfx950) fused causal self-attention
 * forward and its backward.
 *
 * This is the drop-in boundary for the pmkl hot path.  Every entry point takes
 * plain pointers and sizes; no C++, HIP or torch type crosses it (the stream is
 * passed as an opaque hipStream_t cast to void*).
 *
 * Interfaces replaced:
 *   pmkl::nlp::causal_attention_forward<scalar_t, BLOCK_M, HIDDEN_SIZE>(
 *       out, q, k, v, batch_size, num_heads, seq_length, out_m, out_l)
 *       -> reference pmkl/nlp/causal_attention.h:258-288
 *   fused_self_attention_fw(q, k, v, is_causal) -> (out, out_m, out_l)
 *       -> reference pmkl_pytorch_ext/fused_self_attention.cpp:139-173
 *   fused_self_attention_bw(dout, q, k, v, out_m, out_l, is_causal) -> (dq, dk, dv)
 *       -> reference pmkl_pytorch_ext/fused_self_attention.cpp:175-215
 *          (algorithm :66-135)
 *
 * Semantics (identical to the reference CPU operator,
 * fused_self_attention.cpp:5-64, evaluated with fp32 accumulation):
 *   s_ij = scale * <q_i, k_j>           (scale defaults to 1.0f/sqrtf((float)D))
 *   s_ij = -inf for j > i when causal
 *   m_i  = max_j s_ij
 *   l_i  = sum_j exp(s_ij - m_i)        (a plain sum, not a log-sum-exp)
 *   o_i  = sum_j exp(s_ij - m_i) / l_i * v_j
 * Tensors are [batch, heads, seq, head_dim] with head_dim contiguous; m and l
 * are contiguous [batch, heads, seq].
 *
 * Contract:
 *   - The caller allocates every tensor (and the backward's workspace) in
 *     device memory; the library allocates nothing per call.
 *   - Calls are asynchronous on the given stream (NULL = the default stream).
 *   - The functions are re-entrant and thread-safe, with one exception:
 *     pmkl_attn_bwd_noalloc keeps its scratch in one array per GPU, so calls
 *     of it that overlap on one GPU race (see its declaration).  Error text is
 *     thread-local.
 */
#ifndef PMKL_ATTN_H_
#define PMKL_ATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PMKL_ABI_VERSION 5

/* Element types.  The reference dispatches on float, double, half and
 * bfloat16 (fused_self_attention.cpp:152-156); the device path implements
 * float, half and bfloat16.  double stays on the CPU branch of the torch op. */
typedef enum pmkl_dtype {
    PMKL_DTYPE_F32 = 0,
    PMKL_DTYPE_F16 = 1,
    PMKL_DTYPE_BF16 = 2
} pmkl_dtype;

/* Status codes.  The reference raises pmkl::utils::Error from CHECK_FAIL
 * (pmkl/core/utils/exception.h:121-161); at the C boundary that becomes a
 * status code plus pmkl_last_error() text. */
typedef enum pmkl_status {
    PMKL_OK = 0,
    PMKL_EINVAL = 1,      /* bad shape, null pointer, misalignment, bad stride */
    PMKL_EUNSUPPORTED = 2,/* no compiled kernel for this dtype / head_dim      */
    PMKL_EHIP = 3         /* the HIP runtime reported an error at launch        */
} pmkl_status;

/* Arguments of pmkl_attn_fwd.  Strides are in elements; a zero stride triple
 * means "contiguous [B, H, S, D]".  head_dim is always contiguous. */
typedef struct pmkl_attn_fwd_args {
    const void *q;
    const void *k;
    const void *v;
    void *o;
    void *m;            /* [B, H, S] row max of the scaled, masked logits       */
    void *l;            /* [B, H, S] sum_j exp(s_ij - m_i)                       */
    int32_t dtype;      /* pmkl_dtype of q, k, v, o                              */
    int32_t ml_dtype;   /* pmkl_dtype of m and l: dtype (as the reference) or F32 */
    int64_t batch;
    int64_t heads;
    int64_t seq_len;
    int64_t head_dim;   /* 32, 64 or 128                                          */
    int64_t q_strides[3]; /* batch, head, seq strides (elements)                  */
    int64_t k_strides[3];
    int64_t v_strides[3];
    int64_t o_strides[3];
    float scale;        /* 0 -> 1.0f / sqrtf((float)head_dim)                     */
    int32_t is_causal;  /* nonzero: lower-triangular mask j <= i                  */
} pmkl_attn_fwd_args;

/* General entry point.  Replaces the device half of fused_self_attention_fw
 * (fused_self_attention.cpp:139-173): any seq_len >= 0, causal or not,
 * strided q/k/v/o.  Returns a pmkl_status. */
int pmkl_attn_fwd(const pmkl_attn_fwd_args *args, void *stream);

/* Flat form of pmkl::nlp::causal_attention_forward (causal_attention.h:258-262):
 * contiguous [B, H, S, D] tensors, causal mask, scale 1/sqrt(D), m and l in
 * the tensor dtype.  Asynchronous on `stream`. */
int pmkl_causal_attention_forward(int32_t dtype, void *out, const void *q, const void *k,
                                  const void *v, int32_t batch_size, int32_t num_heads,
                                  int32_t seq_length, int32_t hidden_size, void *out_m,
                                  void *out_l, void *stream);

/* 1 if a kernel is compiled for (dtype, head_dim), else 0. */
int pmkl_attn_fwd_supported(int32_t dtype, int64_t head_dim);

/* The kernel pmkl_attn_fwd would launch for these arguments, with its launch
 * shape and work order, e.g.
 * "attn_fwd_w64_kernel<bf16, 128, causal, 1, 8> grid 256 x 512, xcd order";
 * "none" for an empty problem; NULL (and pmkl_last_error() text) where
 * pmkl_attn_fwd would return an error.  Launches nothing.  The string lives in
 * thread-local storage until the calling thread's next call of this function.
 * No counterpart in the reference: it labels measurements (the reference's
 * launcher times each launch, pmkl/core/launcher/cuda_launcher.h:317-328,
 * without naming what it ran).  ABI version 5. */
const char *pmkl_attn_fwd_kernel_name(const pmkl_attn_fwd_args *args);

/* Arguments of pmkl_attn_bwd.  Tensors [B, H, S, D] with head_dim contiguous
 * and any batch / head / seq element strides (all three zero: contiguous), as
 * for pmkl_attn_fwd; m, l contiguous [B, H, S].  The reference operator takes
 * contiguous q, k, v only and copies dout to contiguous
 * (fused_self_attention.cpp:179-182, :201); strided views (BSHD, a packed
 * QKV) need no copies here.
 * Gradients of O only, as the reference: with the forward's m and l,
 *   P_ij  = exp(s_ij - m_i) / l_i,   dP_ij = <dout_i, v_j>,
 *   dS_ij = P_ij (dP_ij - sum_j' P_ij' dP_ij'),
 *   dq_i = scale sum_j dS_ij k_j,  dk_j = scale sum_i dS_ij q_i,
 *   dv_j = sum_i P_ij dout_i. */
typedef struct pmkl_attn_bwd_args {
    const void *dout;
    const void *q;
    const void *k;
    const void *v;
    const void *o;       /* optional forward output: with it sum_j' P dP is
                            <dout_i, o_i>; NULL computes it from the keys      */
    const void *m;       /* [B, H, S] as pmkl_attn_fwd returned it             */
    const void *l;
    void *dq;
    void *dk;
    void *dv;
    void *workspace;     /* device memory, 16-byte aligned, at least
                            pmkl_attn_bwd_workspace_size() bytes; scratch of
                            the call (two floats per query row)               */
    uint64_t workspace_bytes;
    int32_t dtype;       /* pmkl_dtype of dout, q, k, v, o, dq, dk, dv: F32, F16
                            or BF16 (F32: m and l in F32 too)                 */
    int32_t ml_dtype;    /* pmkl_dtype of m and l: dtype or F32                 */
    int64_t batch;
    int64_t heads;
    int64_t seq_len;
    int64_t head_dim;    /* 32, 64 or 128                                        */
    float scale;         /* 0 -> 1.0f / sqrtf((float)head_dim)                   */
    int32_t is_causal;
    /* batch, head, seq strides (elements) of each [B, H, S, D] tensor; all
       three zero: contiguous.  Multiples of 16 bytes, seq stride >= head_dim
       (ABI version 4). */
    int64_t dout_strides[3];
    int64_t q_strides[3];
    int64_t k_strides[3];
    int64_t v_strides[3];
    int64_t o_strides[3];
    int64_t dq_strides[3];
    int64_t dk_strides[3];
    int64_t dv_strides[3];
} pmkl_attn_bwd_args;

/* Bytes of workspace pmkl_attn_bwd needs for this shape. */
uint64_t pmkl_attn_bwd_workspace_size(int64_t batch, int64_t heads, int64_t seq_len);

/* Backward of the attention output.  Replaces the device half of
 * fused_self_attention_bw (fused_self_attention.cpp:175-215), whose
 * algorithm is :66-135.  Writes dq, dk, dv (every element).  Asynchronous on
 * `stream`; allocates nothing.  Returns a pmkl_status. */
int pmkl_attn_bwd(const pmkl_attn_bwd_args *args, void *stream);

/* 1 if a backward kernel is compiled for (dtype, head_dim), else 0. */
int pmkl_attn_bwd_supported(int32_t dtype, int64_t head_dim);

/* Largest batch * heads * seq_len that pmkl_attn_bwd_noalloc accepts. */
#define PMKL_ATTN_BWD_NOALLOC_MAX_ROWS 1048576

/* pmkl_attn_bwd without a caller workspace, and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The two floats per query row that pmkl_attn_bwd
 * keeps in args->workspace live instead in a fixed 8 MiB device array of the
 * library (one per GPU, held until the process ends), so batch * heads *
 * seq_len must not exceed PMKL_ATTN_BWD_NOALLOC_MAX_ROWS (else PMKL_EINVAL,
 * nothing launched).  args->workspace and args->workspace_bytes are ignored;
 * everything else is as for pmkl_attn_bwd, with identical results.  Every
 * call on one GPU shares that array: calls that overlap on one GPU (other
 * streams, other threads) race and must be serialised by the caller.  The
 * first call on a device looks up the array's device address (no allocation).
 * ABI version 3 (strided tensors: 4). */
int pmkl_attn_bwd_noalloc(const pmkl_attn_bwd_args *args, void *stream);

/* Thread-local text of the last error ("" if none), with the file:line of the
 * check that failed, in the style of the reference's CHECK_FAIL message. */
const char *pmkl_last_error(void);

/* PMKL_ABI_VERSION of the loaded library. */
int pmkl_abi_version(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* PMKL_ATTN_H_ */
