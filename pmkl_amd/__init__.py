"""pmkl_amd - MI355X (gfx950) fused causal self-attention forward.

Drop-in replacement for pmkl's attention path:
  * C++:    include/pmkl/nlp/causal_attention.h  (pmkl::nlp::causal_attention_forward)
  * C ABI:  include/pmkl_attn.h                  (libpmkl_attn.so)
  * torch:  pmkl_amd.pmkl_pytorch_ext.fused_self_attention_fw / _bw
  * Python: pmkl_amd.pmkl_function.fused_self_attention
and for the row softmax the fused kernel replaces:
  * C++:    include/pmkl/norm/warp_softmax.h     (pmkl::norm::warp_softmax_forward)
  * C ABI:  include/pmkl_softmax.h               (libpmkl_attn.so)

`attn_fwd`, `attn_bwd`, `warp_softmax_forward` and `softmax` below call the C
ABI directly on device tensors through ctypes; they are what the parity tests
and the benchmark use.
"""
from __future__ import annotations

from . import capi

__all__ = ["attn_fwd", "attn_bwd", "warp_softmax_forward", "softmax", "capi", "torch_dtype_to_pmkl"]


def torch_dtype_to_pmkl(dt) -> int:
    import torch

    table = {torch.float32: capi.PMKL_DTYPE_F32, torch.float16: capi.PMKL_DTYPE_F16,
             torch.bfloat16: capi.PMKL_DTYPE_BF16}
    if dt not in table:
        raise TypeError(f"unsupported dtype {dt} (float32, float16, bfloat16)")
    return table[dt]


def _check_fwd_buffers(q, out, out_m, out_l, ml_dtype):
    """Validates caller-provided output buffers of attn_fwd against q and
    returns the dtype of m and l.  out: [B, H, S, D] in q's dtype on q's
    device with head_dim contiguous (other strides are passed to the kernel);
    out_m / out_l: contiguous [B, H, S] on q's device, both in one dtype,
    which is the m/l dtype (it must agree with ml_dtype when both are given;
    with neither, q's dtype).  The kernels write these buffers assuming
    exactly that, so anything else raises ValueError before a launch."""
    import torch

    B, H, S, D = q.shape
    if out is not None:
        if tuple(out.shape) != (B, H, S, D) or out.dtype != q.dtype or out.device != q.device:
            raise ValueError(f"out must be a [{B}, {H}, {S}, {D}] {q.dtype} tensor on {q.device}")
        if out.stride(3) != 1:
            raise ValueError("out: head_dim must be contiguous")
        if _rows_overlap(_abi_strides(out), (B, H, S), D):
            raise ValueError(f"out strides {tuple(out.stride())} make distinct rows overlap "
                             "(an expanded or aliased output)")
    mdt = ml_dtype
    for name, t in (("out_m", out_m), ("out_l", out_l)):
        if t is None:
            continue
        if tuple(t.shape) != (B, H, S) or t.device != q.device or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous [{B}, {H}, {S}] tensor on {q.device}")
        if mdt is None:
            mdt = t.dtype
        elif t.dtype != mdt:
            raise ValueError(f"{name} is {t.dtype}, but the m/l dtype is {mdt}")
    if mdt is None:
        mdt = q.dtype
    if mdt not in (q.dtype, torch.float32):
        raise ValueError(f"m/l dtype must be q's dtype ({q.dtype}) or float32, got {mdt}")
    return mdt


def attn_fwd(q, k, v, is_causal: bool = True, scale: float | None = None, ml_dtype=None,
             out=None, out_m=None, out_l=None, stream=None):
    """Fused attention forward on ROCm tensors [B, H, S, D] through pmkl_attn_fwd.

    Returns (out, out_m, out_l).  out is contiguous [B, H, S, D] in q's dtype;
    out_m / out_l are [B, H, S] in `ml_dtype` (default: the dtype of a given
    out_m / out_l, else q's dtype, as the reference operator).  q, k, v and
    out may be strided as long as head_dim is contiguous; given buffers are
    validated first (_check_fwd_buffers).  Runs on `stream` (a raw hipStream_t int) or torch's current
    stream; nothing is synchronised.
    """
    import torch

    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("attn_fwd takes ROCm device tensors")
    if q.dim() != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k, v must share a 4-D shape [B, H, S, D]")
    B, H, S, D = q.shape
    dt = torch_dtype_to_pmkl(q.dtype)
    mdt = _check_fwd_buffers(q, out, out_m, out_l, ml_dtype)
    if out is None:
        out = torch.empty((B, H, S, D), dtype=q.dtype, device=q.device)
    if out_m is None:
        out_m = torch.empty((B, H, S), dtype=mdt, device=q.device)
    if out_l is None:
        out_l = torch.empty((B, H, S), dtype=mdt, device=q.device)
    if stream is None:
        stream = torch.cuda.current_stream(q.device).cuda_stream
    a = capi.make_args(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), out_m.data_ptr(),
                       out_l.data_ptr(), dtype=dt, ml_dtype=torch_dtype_to_pmkl(mdt), batch=B, heads=H,
                       seq_len=S, head_dim=D, is_causal=is_causal, scale=0.0 if scale is None else float(scale),
                       q_strides=_abi_strides(q), k_strides=_abi_strides(k), v_strides=_abi_strides(v),
                       o_strides=_abi_strides(out))
    if q.stride(3) != 1 or k.stride(3) != 1 or v.stride(3) != 1 or out.stride(3) != 1:
        raise ValueError("head_dim must be contiguous")
    rc = capi.attn_fwd_raw(a, stream)
    if rc != capi.PMKL_OK:
        raise capi.PmklError(rc, capi.last_error())
    return out, out_m, out_l


def _rows_overlap(strides, sizes, D) -> bool:
    """True unless distinct rows (b, h, s) of a [B, H, S, D] layout with these
    batch / head / seq element strides (head_dim contiguous) are sure not to
    share an element: with the dimensions of size > 1 sorted by stride, each
    stride must be at least the extent of the dimensions inside it (D
    elements for the innermost).  The C ABI applies the same rule to outputs."""
    extent = D
    for st, n in sorted(zip(strides, sizes)):
        if n <= 1:
            continue
        if st < extent:
            return True
        extent = st * (n - 1) + extent
    return False


def _abi_strides(t):
    """Batch / head / seq element strides of a [B, H, S, D] tensor for the C
    ABI.  A size-1 dimension's stride is never multiplied by a nonzero index
    (torch leaves arbitrary values there after views), so it is passed as a
    value the ABI accepts: 0 for batch / head, D for seq."""
    return tuple(t.stride(i) if t.shape[i] != 1 else (t.shape[3] if i == 2 else 0) for i in range(3))


def kernel_view(t):
    """t itself if the kernels can address it in place (head_dim contiguous,
    base and batch / head / seq strides multiples of 16 bytes, rows not
    overlapping), else a contiguous copy."""
    es = t.element_size()
    vec = 16 // es
    st = _abi_strides(t)
    ok = (t.stride(3) == 1 or t.shape[3] == 1) and all(x % vec == 0 and x >= 0 for x in st) and \
        (t.shape[2] == 1 or st[2] >= t.shape[3]) and t.data_ptr() % 16 == 0
    return t if ok else t.contiguous()


def attn_bwd(dout, q, k, v, out_m, out_l, is_causal: bool = True, scale: float | None = None, out=None,
             stream=None):
    """Backward of the attention output on ROCm tensors through pmkl_attn_bwd.

    dout, q, k, v: [B, H, S, D] (fp32 / fp16 / bf16) with head_dim contiguous
    and any batch / head / seq strides (multiples of 16 bytes; passed to the
    kernels, no copies); out_m, out_l: the forward's contiguous [B, H, S]
    outputs (in q's dtype or float32).  `out` (the forward's O, strided like
    the inputs may be) is optional: with it the row terms come from
    <dout, O>.  Returns contiguous (dq, dk, dv).  Runs on `stream` or torch's
    current stream; the workspace is allocated through torch's caching
    allocator.
    """
    import torch

    for name, t in (("dout", dout), ("q", q), ("k", k), ("v", v)) + ((("out", out),) if out is not None else ()):
        if not t.is_cuda:
            raise ValueError(f"attn_bwd takes ROCm device tensors ({name} is not)")
        if t.dim() != 4 or t.shape != q.shape:
            raise ValueError("dout, q, k, v (and out) must share a 4-D shape [B, H, S, D]")
        if t.stride(3) != 1 and t.shape[3] != 1:
            raise ValueError(f"{name}: head_dim must be contiguous")
    if out_m.shape != q.shape[:3] or out_l.shape != q.shape[:3] or not (out_m.is_contiguous() and out_l.is_contiguous()):
        raise ValueError("out_m / out_l must be contiguous [B, H, S] tensors")
    B, H, S, D = q.shape
    dt = torch_dtype_to_pmkl(q.dtype)
    mdt = torch_dtype_to_pmkl(out_m.dtype)
    lib = capi.load()
    ws_bytes = int(lib.pmkl_attn_bwd_workspace_size(B, H, S))
    ws = torch.empty((max(ws_bytes, 16) + 3) // 4, dtype=torch.float32, device=q.device)
    dq = torch.empty((B, H, S, D), dtype=q.dtype, device=q.device)
    dk = torch.empty((B, H, S, D), dtype=q.dtype, device=q.device)
    dv = torch.empty((B, H, S, D), dtype=q.dtype, device=q.device)
    if stream is None:
        stream = torch.cuda.current_stream(q.device).cuda_stream
    strides = {"dout": _abi_strides(dout), "q": _abi_strides(q), "k": _abi_strides(k), "v": _abi_strides(v)}
    if out is not None:
        strides["o"] = _abi_strides(out)
    a = capi.make_bwd_args(dout.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                           0 if out is None else out.data_ptr(), out_m.data_ptr(),
                           out_l.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                           ws.data_ptr(), ws.numel() * 4, dtype=dt, ml_dtype=mdt, batch=B, heads=H, seq_len=S,
                           head_dim=D, is_causal=is_causal, scale=0.0 if scale is None else float(scale),
                           strides=strides)
    rc = capi.attn_bwd_raw(a, stream)
    if rc != capi.PMKL_OK:
        raise capi.PmklError(rc, capi.last_error())
    return dq, dk, dv


def warp_softmax_forward(dst, src, softmax_elements: int, softmax_elements_stride: int, batch_count: int,
                         is_log_softmax: bool = False, stream=None) -> None:
    """pmkl::norm::warp_softmax_forward (pmkl/norm/warp_softmax.h:159-201) on
    ROCm tensors: row r of `src` (elements [r*stride, r*stride + n)) goes to
    the same place in `dst`.  The dtypes of dst and src (float32, float16,
    bfloat16) play the template's output_t and input_t; accumulation is fp32.
    Asynchronous on `stream` or torch's current stream."""
    import torch

    for name, t in (("dst", dst), ("src", src)):
        if not t.is_cuda:
            raise ValueError(f"warp_softmax_forward takes ROCm device tensors ({name} is not)")
    need = 0 if batch_count <= 0 or softmax_elements <= 0 else \
        (batch_count - 1) * softmax_elements_stride + softmax_elements
    for name, t in (("dst", dst), ("src", src)):
        if t.numel() < need or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous tensor of at least {need} elements")
    if stream is None:
        stream = torch.cuda.current_stream(src.device).cuda_stream
    a = capi.make_softmax_args(dst.data_ptr(), src.data_ptr(), out_dtype=torch_dtype_to_pmkl(dst.dtype),
                               in_dtype=torch_dtype_to_pmkl(src.dtype), elements=softmax_elements,
                               stride=softmax_elements_stride, batch=batch_count, is_log=is_log_softmax)
    rc = capi.softmax_raw(a, stream)
    if rc != capi.PMKL_OK:
        raise capi.PmklError(rc, capi.last_error())


def softmax(x, is_log: bool = False, out_dtype=None, stream=None):
    """Softmax (or log-softmax) over the last dimension (<= 1024 elements) of
    a ROCm tensor, through pmkl_softmax_fwd.  Rows must be evenly strided with
    the last dimension contiguous (anything else is copied first); the result
    has x's shape, in out_dtype (default x.dtype), with the same row stride."""
    import torch

    if not x.is_cuda:
        raise ValueError("softmax takes a ROCm device tensor")
    n = x.shape[-1] if x.dim() else 1
    x2 = x.reshape(-1, n)
    if x2.numel() and (x2.stride(1) != 1 or x2.stride(0) < n):
        x2 = x2.contiguous()
    rows = x2.shape[0]
    stride = x2.stride(0) if rows > 1 else n
    out_full = torch.empty((rows, max(stride, n)), dtype=out_dtype or x.dtype, device=x.device)
    out = out_full[:, :n]
    if stream is None:
        stream = torch.cuda.current_stream(x.device).cuda_stream
    a = capi.make_softmax_args(out_full.data_ptr(), x2.data_ptr(), out_dtype=torch_dtype_to_pmkl(out.dtype),
                               in_dtype=torch_dtype_to_pmkl(x.dtype), elements=n, stride=stride, batch=rows,
                               is_log=is_log)
    rc = capi.softmax_raw(a, stream)
    if rc != capi.PMKL_OK:
        raise capi.PmklError(rc, capi.last_error())
    return out.view(x.shape)
