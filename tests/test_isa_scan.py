"""Scans the generated gfx950 code of the 64-row kernel (every instantiation of
one translation unit, compiled here with the library's flags), and of the
head_dim-128 backward kernels (whose dQ pass stages K/V by the same kind of
LDS-DMA block), for hazards that inline assembly hides from the compiler and
that tests show only by chance:

* SCC across the LDS-DMA block: the block forms M0 with s_add_u32, which writes
  SCC.  An SCC reader whose last SCC writer comes before such a block reads the
  add's carry, not the comparison (a float-m/l flag once read as 0 that way).
* Row-sum MFMA chains: a v_mfma_f32_4x4x4 result is not ready for the SrcC of
  the next one; two such MFMAs on one accumulator need three instructions
  between them (one shared accumulator once lost the first sum).

CPU only: compiles and reads assembly text, runs nothing on a GPU."""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
TU = ROOT / "pmkl_amd" / "csrc" / "attn_fwd_w64_bf16_causal.hip"

# SCC writers (SOP1/SOP2/SOPC/SOPK arithmetic, logic, compares) and readers.
SCC_WRITE = re.compile(
    r"^(s_cmp|s_cmpk|s_add_[ui]32|s_addc_u32|s_sub_[ui]32|s_subb_u32|s_and_|s_or_|s_xor_|s_andn[12]_|s_orn[12]_|"
    r"s_nand_|s_nor_|s_xnor_|s_lshl|s_lshr|s_ashr|s_bfe_|s_not_|s_min_|s_max_|s_abs|s_bitcmp|s_bcnt|s_absdiff|"
    r"s_quadmask|s_wqm)")
SCC_READ = re.compile(r"^(s_cselect|s_cbranch_scc|s_addc_u32|s_subb_u32|s_cmov)")


# The head_dim-128 backward kernels, instantiated explicitly.
BWD_TU = """#include <hip/hip_runtime.h>
#include "attn_bwd_kernels.hpp"
namespace pmkl_amd {
template __global__ void attn_bwd_dq_kernel<__bf16, 128, true>(BwdParams);
template __global__ void attn_bwd_dq_kernel<__bf16, 128, false>(BwdParams);
template __global__ void attn_bwd_dq_kernel<_Float16, 128, true>(BwdParams);
template __global__ void attn_bwd_dkdv_kernel<__bf16, 128, true>(BwdParams);
}
"""


def _asm(tmp_path: Path, tu: Path = TU) -> list[str]:
    if not Path(HIPCC).exists():
        pytest.skip("hipcc not available")
    out = tmp_path / "k.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-I", str(ROOT / "include"), "-I", str(ROOT / "pmkl_amd" / "csrc"),
           str(tu), "--cuda-device-only", "-S", "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    lines = []
    for raw in out.read_text().splitlines():
        s = raw.split(";")[0].strip()
        if s and "ASMSTART" not in raw and "ASMEND" not in raw:
            lines.append(s)
    return lines


@pytest.fixture(scope="module")
def asm_lines(tmp_path_factory):
    return _asm(tmp_path_factory.mktemp("isa"))


@pytest.fixture(scope="module")
def bwd_asm_lines(tmp_path_factory):
    d = tmp_path_factory.mktemp("isa_bwd")
    tu = d / "bwd.hip"
    tu.write_text(BWD_TU)
    return _asm(d, tu)


def test_kernels_compiled(asm_lines):
    kernels = [l for l in asm_lines if re.match(r"^_ZN8pmkl_amd19attn_fwd_w64_kernel.*:$", l)]
    assert len(kernels) >= 6, kernels


def _scc_sites(asm_lines):
    bad = []
    writer_before_dma = False   # the last SCC writer precedes a DMA block (no writer since)
    for i, l in enumerate(asm_lines):
        op = l.split()[0]
        if l.endswith(":") or op in ("s_branch", "s_endpgm") or op.startswith("s_cbranch_exec") \
                or op.startswith("s_cbranch_vcc"):
            writer_before_dma = False   # block boundary: the scan stays within straight-line code
        if op == "s_add_u32" and " m0," in l:
            writer_before_dma = True
            continue
        if SCC_READ.match(op) and writer_before_dma:
            bad.append((i, l))
        if SCC_WRITE.match(op):
            writer_before_dma = False
    return bad


def test_no_scc_read_across_lds_dma(asm_lines):
    bad = _scc_sites(asm_lines)
    assert not bad, bad[:5]


def test_backward_kernels_compiled_with_lds_dma(bwd_asm_lines):
    kernels = [l for l in bwd_asm_lines if re.match(r"^_ZN8pmkl_amd(18attn_bwd_dq|20attn_bwd_dkdv)_kernel.*:$", l)]
    assert len(kernels) == 4, kernels
    assert sum(1 for l in bwd_asm_lines if l.startswith("buffer_load_dwordx4") and l.endswith(" lds")) > 0


def test_no_scc_read_across_lds_dma_backward(bwd_asm_lines):
    bad = _scc_sites(bwd_asm_lines)
    assert not bad, bad[:5]


def test_row_sum_mfma_chains_spaced(asm_lines):
    last = {}
    bad = []
    for i, l in enumerate(asm_lines):
        if l.endswith(":"):
            last.clear()
            continue
        if l.startswith("v_mfma_f32_4x4x4"):
            acc = l.split(None, 1)[1].split(",")[3].strip()
            if acc in last and i - last[acc] < 4:
                bad.append((i - last[acc], l))
            last[acc] = i
    assert not bad, bad[:5]
