"""CPU tests of the C ABI (include/pmkl_attn.h, include/pmkl_softmax.h,
pmkl_amd/libpmkl_attn.so).

No kernel is launched here: the library is loaded, every declared symbol is
resolved, and the argument checks are driven into each of their error paths
(all of which return before any HIP call).  The error text must carry the
file:line of the failed check, like the reference's CHECK_FAIL
(pmkl/core/utils/exception.h:153-161).
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from pmkl_amd import capi

ROOT = Path(__file__).resolve().parent.parent
HEADERS = (ROOT / "include" / "pmkl_attn.h", ROOT / "include" / "pmkl_softmax.h")


def _declared_functions():
    names = set()
    for header in HEADERS:
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(pmkl_\w+)\s*\(", header.read_text(), re.M))
    return sorted(names)


def test_header_declares_the_exported_set():
    assert _declared_functions() == sorted(capi.EXPORTED_SYMBOLS)


def test_library_loads_and_exports_every_declared_symbol():
    lib = capi.load()
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} is declared in include/ but not exported"


def test_abi_version_and_support_matrix():
    lib = capi.load()
    assert lib.pmkl_abi_version() == 5
    for dt in (capi.PMKL_DTYPE_F32, capi.PMKL_DTYPE_F16, capi.PMKL_DTYPE_BF16):
        for d in (32, 64, 128):
            assert lib.pmkl_attn_fwd_supported(dt, d) == 1
        for d in (0, 16, 80, 96, 256):
            assert lib.pmkl_attn_fwd_supported(dt, d) == 0
    assert lib.pmkl_attn_fwd_supported(7, 64) == 0


def _args(**kw):
    base = dict(q=0x1000, k=0x2000, v=0x3000, o=0x4000, m=0x5000, l=0x6000, dtype=capi.PMKL_DTYPE_BF16,
                batch=1, heads=2, seq_len=64, head_dim=64)
    base.update(kw)
    return capi.make_args(**base)


def _expect(args, code, pattern):
    rc = capi.attn_fwd_raw(args)
    msg = capi.last_error()
    assert rc == code, (rc, msg)
    assert re.search(pattern, msg), msg
    assert re.search(r"pmkl check failed at attn_capi\.hip:\d+", msg), msg


def test_error_paths():
    lib = capi.load()
    assert lib.pmkl_attn_fwd(None, None) == capi.PMKL_EINVAL
    _expect(_args(dtype=9), capi.PMKL_EUNSUPPORTED, "unsupported dtype")
    _expect(_args(ml_dtype=capi.PMKL_DTYPE_F16), capi.PMKL_EINVAL, "ml_dtype")
    _expect(_args(batch=-1), capi.PMKL_EINVAL, "negative shape")
    _expect(_args(head_dim=80), capi.PMKL_EUNSUPPORTED, "head_dim 80")
    _expect(_args(scale=float("nan")), capi.PMKL_EINVAL, "scale")
    _expect(_args(q=0), capi.PMKL_EINVAL, "q is a null pointer")
    _expect(_args(v=0x3002), capi.PMKL_EINVAL, "v must be 16-byte aligned")
    _expect(_args(k_strides=(2 * 64 * 64, 64 * 64, 32)), capi.PMKL_EINVAL, "seq stride >= head_dim")
    _expect(_args(q_strides=(2 * 64 * 64, 64 * 64, 68)), capi.PMKL_EINVAL, "multiples of 8 elements")
    _expect(_args(o_strides=(1 << 40, 1 << 30, 1 << 28)), capi.PMKL_EINVAL, "too large")
    _expect(_args(m=0), capi.PMKL_EINVAL, "m / l must not be null")
    # outputs whose rows alias (an expanded batch, heads packed closer than a head's rows)
    _expect(_args(batch=2, o_strides=(0, 64 * 64, 64)), capi.PMKL_EINVAL, "o strides .* overlap")
    _expect(_args(o_strides=(2 * 64 * 64, 32 * 64, 64)), capi.PMKL_EINVAL, "o strides .* overlap")
    # interleaved heads ([B, S, H, D] memory) do not overlap: the call plans a kernel
    assert capi.attn_fwd_kernel_name(_args(o_strides=(2 * 64 * 64, 64, 2 * 64))) is not None, capi.last_error()
    _expect(_args(dtype=capi.PMKL_DTYPE_F32, ml_dtype=capi.PMKL_DTYPE_F32, m=0x5002), capi.PMKL_EINVAL,
            "aligned to their element size")


def test_empty_problem_returns_ok_without_touching_pointers():
    """An empty problem returns before any pointer is used (causal_attention.h:270)."""
    lib = capi.load()
    for kw in (dict(seq_len=0), dict(batch=0), dict(heads=0)):
        a = _args(q=0, k=0, v=0, o=0, m=0, l=0, **kw)
        assert capi.attn_fwd_raw(a) == capi.PMKL_OK
    assert lib.pmkl_causal_attention_forward(capi.PMKL_DTYPE_F32, None, None, None, None, 0, 4, 128, 64,
                                             None, None, None) == capi.PMKL_OK


def test_flat_entry_point_validates_like_the_template():
    lib = capi.load()
    rc = lib.pmkl_causal_attention_forward(capi.PMKL_DTYPE_BF16, None, None, None, None, 1, 1, 64, 96,
                                           None, None, None)
    assert rc == capi.PMKL_EUNSUPPORTED and "head_dim 96" in capi.last_error()
    rc = lib.pmkl_causal_attention_forward(capi.PMKL_DTYPE_BF16, None, None, None, None, 1, 1, 64, 64,
                                           None, None, None)
    assert rc == capi.PMKL_EINVAL and "null pointer" in capi.last_error()


@pytest.mark.parametrize("cname,cls", [("pmkl_attn_fwd_args", "AttnFwdArgs"), ("pmkl_attn_bwd_args", "AttnBwdArgs")])
def test_args_struct_layout_matches_header(tmp_path, cname, cls):
    """Field offsets and size of the ctypes mirrors equal those of the C
    structs, as a C compiler lays them out from include/pmkl_attn.h."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    mirror = getattr(capi, cls)
    fields = [f[0] for f in mirror._fields_]
    src = tmp_path / "layout.c"
    body = "".join(f'  printf("%s %zu\\n", "{f}", offsetof({cname}, {f}));\n' for f in fields)
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "pmkl_attn.h"\nint main(void) {\n'
                   + body + f'  printf("sizeof %zu\\n", sizeof({cname}));\n  return 0;\n}}\n')
    exe = tmp_path / "layout"
    subprocess.run([cc, "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    out = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                         check=True).stdout.splitlines())
    for f in fields:
        assert int(out[f]) == getattr(mirror, f).offset, f
    assert int(out["sizeof"]) == ctypes.sizeof(mirror)


def _bwd_args(**kw):
    base = dict(dout=0x1000, q=0x2000, k=0x3000, v=0x4000, o=0, m=0x5000, l=0x6000, dq=0x7000, dk=0x8000,
                dv=0x9000, workspace=0xa000, workspace_bytes=1 << 20, dtype=capi.PMKL_DTYPE_BF16,
                batch=1, heads=2, seq_len=64, head_dim=64)
    base.update(kw)
    return capi.make_bwd_args(**base)


def _expect_bwd(args, code, pattern):
    rc = capi.attn_bwd_raw(args)
    msg = capi.last_error()
    assert rc == code, (rc, msg)
    assert re.search(pattern, msg), msg
    assert re.search(r"pmkl check failed at attn_capi\.hip:\d+", msg), msg


def test_bwd_workspace_size_and_support():
    lib = capi.load()
    assert lib.pmkl_attn_bwd_workspace_size(4, 32, 4096) == 2 * 4 * 32 * 4096 * 4
    assert lib.pmkl_attn_bwd_workspace_size(0, 32, 4096) == 0
    for dt in (capi.PMKL_DTYPE_F32, capi.PMKL_DTYPE_F16, capi.PMKL_DTYPE_BF16):
        for d in (32, 64, 128):
            assert lib.pmkl_attn_bwd_supported(dt, d) == 1
        assert lib.pmkl_attn_bwd_supported(dt, 80) == 0
    assert lib.pmkl_attn_bwd_supported(7, 64) == 0


def test_bwd_error_paths():
    lib = capi.load()
    assert lib.pmkl_attn_bwd(None, None) == capi.PMKL_EINVAL
    _expect_bwd(_bwd_args(dtype=9, ml_dtype=9), capi.PMKL_EUNSUPPORTED, "no device kernel")
    _expect_bwd(_bwd_args(dtype=capi.PMKL_DTYPE_F32, ml_dtype=capi.PMKL_DTYPE_BF16), capi.PMKL_EINVAL, "ml_dtype")
    _expect_bwd(_bwd_args(ml_dtype=capi.PMKL_DTYPE_F16), capi.PMKL_EINVAL, "ml_dtype")
    _expect_bwd(_bwd_args(seq_len=-1), capi.PMKL_EINVAL, "negative shape")
    _expect_bwd(_bwd_args(head_dim=96), capi.PMKL_EUNSUPPORTED, "head_dim 96")
    _expect_bwd(_bwd_args(dq=0), capi.PMKL_EINVAL, "dq is a null pointer")
    _expect_bwd(_bwd_args(k=0x3008), capi.PMKL_EINVAL, "k must be 16-byte aligned")
    _expect_bwd(_bwd_args(o=0x3008), capi.PMKL_EINVAL, "o must be 16-byte aligned")
    _expect_bwd(_bwd_args(l=0), capi.PMKL_EINVAL, "m / l must not be null")
    _expect_bwd(_bwd_args(workspace=0), capi.PMKL_EINVAL, "workspace must be")
    _expect_bwd(_bwd_args(workspace_bytes=100), capi.PMKL_EINVAL, "workspace of 100 bytes is too small")
    # strides: validated per tensor, as the forward's
    _expect_bwd(_bwd_args(strides={"v": (2 * 64 * 64, 64 * 64, 60)}), capi.PMKL_EINVAL,
                r"v strides \(8192, 4096, 60\) must be non-negative with seq stride >= head_dim 64")
    _expect_bwd(_bwd_args(strides={"dq": (2 * 64 * 72, 72, 2 * 72 + 4)}), capi.PMKL_EINVAL,
                r"dq strides .* must be multiples of 8 elements")
    _expect_bwd(_bwd_args(strides={"dout": (-1, 64, 128)}), capi.PMKL_EINVAL, "dout strides")
    # gradient outputs whose rows alias
    _expect_bwd(_bwd_args(strides={"dk": (2 * 64 * 64, 0, 64)}), capi.PMKL_EINVAL, "dk strides .* overlap")
    _expect_bwd(_bwd_args(strides={"dv": (2 * 64 * 64, 64 * 32, 64)}), capi.PMKL_EINVAL, "dv strides .* overlap")
    _expect_bwd(_bwd_args(batch=2, strides={"dq": (0, 64 * 64, 64)}), capi.PMKL_EINVAL, "dq strides .* overlap")
    with pytest.raises(ValueError, match="no stride field"):
        _bwd_args(strides={"m": (0, 0, 1)})
    # an empty problem succeeds without touching anything
    assert capi.attn_bwd_raw(_bwd_args(seq_len=0, dq=0, workspace=0)) == capi.PMKL_OK


def test_softmax_args_struct_layout_matches_header(tmp_path):
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    fields = [f[0] for f in capi.SoftmaxArgs._fields_]
    src = tmp_path / "layout.c"
    body = "".join(f'  printf("%s %zu\\n", "{f}", offsetof(pmkl_softmax_args, {f}));\n' for f in fields)
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "pmkl_softmax.h"\nint main(void) {\n'
                   + body + '  printf("sizeof %zu\\n", sizeof(pmkl_softmax_args));\n  return 0;\n}\n')
    exe = tmp_path / "layout"
    subprocess.run([cc, "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    out = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                         check=True).stdout.splitlines())
    for f in fields:
        assert int(out[f]) == getattr(capi.SoftmaxArgs, f).offset, f
    assert int(out["sizeof"]) == ctypes.sizeof(capi.SoftmaxArgs)


def _softmax_args(**kw):
    base = dict(dst=0x1000, src=0x2000, out_dtype=capi.PMKL_DTYPE_F32, in_dtype=capi.PMKL_DTYPE_F32,
                elements=1024, stride=1024, batch=12, is_log=False)
    base.update(kw)
    return capi.make_softmax_args(**base)


def _expect_softmax(args, code, pattern):
    rc = capi.softmax_raw(args)
    msg = capi.last_error()
    assert rc == code, (rc, msg)
    assert re.search(pattern, msg), msg
    assert re.search(r"pmkl check failed at softmax_capi\.hip:\d+", msg), msg


def test_softmax_error_paths():
    """The reference's CHECK_FAIL(softmax_elements >= 0 && <= 1024)
    (warp_softmax.h:162) and this boundary's own argument checks."""
    E = capi.PMKL_EINVAL
    _expect_softmax(_softmax_args(elements=1025, stride=1025), E, r"softmax_elements <= 1024 \(got 1025\)")
    _expect_softmax(_softmax_args(elements=-1), E, r"softmax_elements >= 0")
    _expect_softmax(_softmax_args(in_dtype=7), E, r"unknown dtype")
    _expect_softmax(_softmax_args(out_dtype=-1), E, r"unknown dtype")
    _expect_softmax(_softmax_args(batch=-1), E, r"batch_count")
    _expect_softmax(_softmax_args(batch=1 << 31), E, r"batch_count")
    _expect_softmax(_softmax_args(stride=1000), E, r"stride \(1000\) < softmax_elements \(1024\)")
    _expect_softmax(_softmax_args(src=0), E, r"null src or dst")
    _expect_softmax(_softmax_args(stride=1 << 40, batch=1 << 20), E, r"rows span more than 2\^48")
    _expect_softmax(_softmax_args(stride=(1 << 48) + 1, batch=1), E, r"rows span more than 2\^48")
    _expect_softmax(_softmax_args(dst=0x2000, out_dtype=capi.PMKL_DTYPE_BF16), E, r"in-place")
    rc = capi.load().pmkl_softmax_fwd(None, None)
    assert rc == E and "null argument block" in capi.last_error()


def test_softmax_empty_problem_returns_ok_without_touching_pointers():
    """softmax_elements == 0 returns early as in the reference
    (warp_softmax.h:163-164); so does batch_count == 0."""
    assert capi.softmax_raw(_softmax_args(dst=0, src=0, elements=0, stride=0)) == capi.PMKL_OK
    assert capi.softmax_raw(_softmax_args(dst=0, src=0, batch=0)) == capi.PMKL_OK
    lib = capi.load()
    assert lib.pmkl_warp_softmax_forward(0, 0, 0, None, None, 0, 0, 5, None) == capi.PMKL_OK
    assert lib.pmkl_warp_softmax_forward(0, 0, 0, None, None, 1025, 1025, 5, None) == capi.PMKL_EINVAL
    assert "softmax_elements" in capi.last_error()


def test_attn_fwd_rejects_bad_output_buffers():
    """Caller-provided out / out_m / out_l are validated before any launch
    (pmkl_amd._check_fwd_buffers, run here on CPU tensors)."""
    import torch

    from pmkl_amd import _check_fwd_buffers

    q = torch.empty(2, 3, 40, 64, dtype=torch.bfloat16)
    ok_o = torch.empty_like(q)
    ok_m = torch.empty(2, 3, 40, dtype=torch.bfloat16)
    assert _check_fwd_buffers(q, ok_o, ok_m, ok_m.clone(), None) == torch.bfloat16
    assert _check_fwd_buffers(q, None, None, None, None) == torch.bfloat16
    assert _check_fwd_buffers(q, None, None, None, torch.float32) == torch.float32
    m32 = ok_m.float()
    assert _check_fwd_buffers(q, None, m32, m32.clone(), None) == torch.float32   # dtype taken from out_m
    # strided out with head_dim contiguous is fine ([B, S, H, D] memory)
    assert _check_fwd_buffers(q, torch.empty(2, 40, 3, 64, dtype=q.dtype).transpose(1, 2), None, None, None)
    bad = [
        ((torch.empty(2, 3, 41, 64, dtype=q.dtype), None, None, None), "out must be"),
        ((torch.empty_like(q, dtype=torch.float16), None, None, None), "out must be"),
        ((torch.empty(2, 3, 64, 40, dtype=q.dtype).transpose(2, 3), None, None, None), "head_dim must be contiguous"),
        ((None, torch.empty(2, 3, 39, dtype=q.dtype), None, None), "out_m must be"),
        ((None, None, torch.empty(2, 40, 3, dtype=q.dtype).transpose(1, 2), None), "out_l must be"),
        ((None, ok_m, m32, None), "out_l is torch.float32"),
        ((None, ok_m, None, torch.float32), "out_m is torch.bfloat16"),
        ((None, torch.empty(2, 3, 40, dtype=torch.float16), None, None), "m/l dtype must be"),
        ((None, torch.empty(2, 3, 40, dtype=q.dtype, device="meta"), None, None), "out_m must be"),
        # outputs whose rows alias: expanded over batch, over heads, rows closer than head_dim
        ((torch.empty(1, 3, 40, 64, dtype=q.dtype).expand(2, 3, 40, 64), None, None, None), "overlap"),
        ((torch.empty(2, 1, 40, 64, dtype=q.dtype).expand(2, 3, 40, 64), None, None, None), "overlap"),
        ((torch.empty(2 * 3 * 40 * 64, dtype=q.dtype).as_strided((2, 3, 40, 64), (3 * 40 * 64, 40 * 32, 32, 1)),
          None, None, None), "overlap"),
    ]
    for (o, m, l, mdt), msg in bad:
        with pytest.raises(ValueError, match=msg):
            _check_fwd_buffers(q, o, m, l, mdt)


def test_kernel_name_query():
    """pmkl_attn_fwd_kernel_name names the kernel pmkl_attn_fwd would launch,
    or returns NULL with the same error text where the call would fail; it
    launches nothing (shapes here need no device to plan)."""
    # an invalid call: NULL and the check's text
    assert capi.attn_fwd_kernel_name(_args(head_dim=80)) is None
    assert "head_dim 80" in capi.last_error()
    assert capi.attn_fwd_kernel_name(_args(o_strides=(0, 64 * 64, 64), batch=2)) is None
    assert "overlap" in capi.last_error()
    # an empty problem launches nothing
    assert capi.attn_fwd_kernel_name(_args(seq_len=0, q=0, k=0, v=0, o=0, m=0, l=0)) == "none"
    # short 16-bit sequences: the resident form of the 8-wave MFMA kernel
    name = capi.attn_fwd_kernel_name(_args(seq_len=200))
    assert name.startswith("attn_fwd_mfma16_kernel<bf16, 64, causal, 8, 4> grid "), name
    assert capi.attn_fwd_kernel_name(_args(seq_len=200, is_causal=False)).startswith(
        "attn_fwd_mfma16_kernel<bf16, 64, full, 8, 4>")
    # fp32 with the CU count unknown (no device): the 128-row fp32 kernel
    name = capi.attn_fwd_kernel_name(_args(dtype=capi.PMKL_DTYPE_F32, ml_dtype=capi.PMKL_DTYPE_F32, seq_len=300))
    assert name == "attn_fwd_f32_kernel<64, causal> grid 6 x 256", name
