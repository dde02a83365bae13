"""In-tree build of the native parts of pmkl_amd.

Products (all next to their sources, so they travel with the tree):
  pmkl_amd/libpmkl_attn.so                 gfx950 kernels + C ABI (hipcc): attention
                                           forward/backward and row softmax
  pmkl_amd/pmkl_pytorch_ext.<ext-suffix>   torch operator over the C ABI (g++)

Every function compiles unconditionally; nothing is skipped because an output
already exists.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "pmkl_amd"
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")

# Packed fp32 VALU ops are kept off: they have given silent wrong results on
# these boxes.  The host pass warns that it does not know the feature.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

CAPI_LIB = PKG / "libpmkl_attn.so"
EXT_NAME = "pmkl_pytorch_ext"
EXT_LIB = PKG / (EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def _run(cmd: list[str], cwd: Path = ROOT) -> None:
    res = subprocess.run(cmd, cwd=str(cwd), capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}\n{err}")


CAPI_SOURCES = ("attn_capi.hip", "softmax_capi.hip", "attn_fwd_w64_bf16_causal.hip", "attn_fwd_w64_bf16_full.hip",
                "attn_fwd_w64_f16_causal.hip", "attn_fwd_w64_f16_full.hip")


def build_capi() -> Path:
    """Compiles each C ABI source to an object in parallel, then links them."""
    objs = [CAPI_LIB.parent / (Path(src).stem + ".o.tmp") for src in CAPI_SOURCES]
    procs = [subprocess.Popen([HIPCC, *HIP_FLAGS, "-I", str(INCLUDE), "-c", str(CSRC / src), "-o", str(obj)],
                              cwd=str(ROOT), stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
             for src, obj in zip(CAPI_SOURCES, objs)]
    errors = []
    for src, proc in zip(CAPI_SOURCES, procs):
        out, err = proc.communicate()
        if proc.returncode != 0:
            errors.append(f"{src} ({proc.returncode}):\n{out}\n{err}")
    try:
        if errors:
            raise RuntimeError("build step failed: " + "\n".join(errors))
        tmp = CAPI_LIB.with_suffix(".so.tmp")
        _run([HIPCC, *HIP_FLAGS, "-shared", *map(str, objs), "-o", str(tmp)])
        os.replace(tmp, CAPI_LIB)
    finally:
        for obj in objs:
            obj.unlink(missing_ok=True)
    return CAPI_LIB


def build_torch_ext() -> Path:
    import torch
    from torch.utils import cpp_extension

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    inc = [f"-I{p}" for p in cpp_extension.include_paths()]
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fopenmp",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *inc, f"-I{ROCM / 'include'}", f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}",
        str(CSRC / "torch_binding.cpp"),
        f"-L{torch_lib}", f"-L{PKG}", f"-L{ROCM / 'lib'}",
        "-lpmkl_attn", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lamdhip64",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}",
        "-o", str(EXT_LIB) + ".tmp",
    ]
    _run(cmd)
    os.replace(str(EXT_LIB) + ".tmp", EXT_LIB)
    return EXT_LIB


def build_all(verbose: bool = True) -> None:
    for step in (build_capi, build_torch_ext):
        out = step()
        if verbose:
            print(f"[pmkl_amd build] {step.__name__}: {out.relative_to(ROOT)}", flush=True)


if __name__ == "__main__":
    build_all()
    sys.exit(0)
