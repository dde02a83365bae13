"""The committed rocprofv3 summaries under profiles/ parse the way bench.py
reads them: every kernel trace names its kernel by the library's own name
(the text of pmkl_attn_fwd_kernel_name up to the launch shape) and carries
per-lease "lease:" lines, and every traffic summary its HBM bytes per launch.
CPU only: no GPU, no library call."""
from __future__ import annotations

import importlib.util
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PROFILES = ROOT / "profiles"
KERNEL_ID = re.compile(r"^kernel_id:\s*(.+?)\s*$", re.M)
# name<dtype, head_dim, causal|full, waves / blocks...> as the C ABI prints it
FULL_NAME = re.compile(r"^attn_fwd_[a-z0-9_]+_kernel<(bf16|fp16|fp32)?(, )?\d+, (causal|full)(, \d+)*>$")


def _bench():
    spec = importlib.util.spec_from_file_location("bench_module", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _forward_traces():
    return sorted(PROFILES.glob("attn_fwd_*_C[1-5]_kernel_trace.txt"))


def test_forward_traces_name_their_kernel_and_leases():
    traces = _forward_traces()
    assert traces, "no forward kernel traces committed"
    for path in traces:
        txt = path.read_text()
        m = KERNEL_ID.search(txt)
        if m is None:
            continue   # summaries of earlier builds without a kernel_id line are not read by bench.py
        kid = m.group(1)
        assert FULL_NAME.match(kid), (path.name, kid)
        family = kid.split("<")[0].removesuffix("_kernel")
        assert path.name.startswith(family + "_"), (path.name, family)
        leases = re.findall(r"^lease:\s*(\S+)\s+trace_mean_us\s+([0-9.]+)\s+shader_clock_GHz\s+([0-9.]+|n/a)",
                            txt, re.M)
        assert leases, path.name


def test_headline_trace_has_two_leases_with_clock():
    txt = (PROFILES / "attn_fwd_w64_C3_kernel_trace.txt").read_text()
    leases = re.findall(r"^lease:\s*(\S+)\s+trace_mean_us\s+([0-9.]+)\s+shader_clock_GHz\s+([0-9.]+)", txt, re.M)
    assert len(leases) >= 2
    for _, us, ghz in leases:
        assert 100.0 < float(us) < 5000.0
        assert 0.5 < float(ghz) < 2.5   # a shader clock, not a counter window artefact


@pytest.mark.parametrize("config", ["C2", "C3", "C4", "C5"])
def test_bench_reads_traffic_and_profile(config):
    bench = _bench()
    txt = (PROFILES / f"pmc_attn_fwd_{config}.txt").read_text()
    kid = KERNEL_ID.search(txt).group(1)
    traffic = bench.read_traffic(config, kid + " grid 1 x 64")
    assert traffic is not None and traffic > 0
    # the trace summary of the same kernel is found by its family
    prof = bench.read_profile(config, kid + " grid 1 x 64", 1.0e9, 1.0)
    assert prof is not None and prof["leases"], config
    # a different kernel name finds neither
    assert bench.read_traffic(config, "attn_fwd_other_kernel<bf16, 128, causal> grid 1 x 64") is None


def test_traffic_summaries_state_bytes_per_launch():
    for path in sorted(PROFILES.glob("pmc_attn_fwd_C*.txt")):
        txt = path.read_text()
        m = re.search(r"^hbm_bytes_per_launch:\s*([0-9.eE+]+)", txt, re.M)
        assert m is not None, path.name
        assert float(m.group(1)) > 0
        assert "rocprofv3 --pmc FETCH_SIZE" in txt and "rocprofv3 --pmc WRITE_SIZE" in txt, path.name
