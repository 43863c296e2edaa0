"""Register budgets of the HIP kernels, from the compiler's per-kernel
resource report that the build writes (grinqh/_lib/kernel_resources.json,
hipcc -Rpass-analysis=kernel-resource-usage).

A kernel that spills registers uses private-segment (scratch) memory that the
HIP runtime supplies, which the allocation-free entry point cannot vouch for,
and spill reloads near the MFMA loops can land on accumulator registers an
MFMA issued just before still reads.  Every kernel must use no scratch except
the documented ones, each within its bound: the large-batch prefill kernel's
512-row instantiations spill a few registers in the epilogue (after the MFMA
loop, all 512 registers of a lane in use).  A change that makes another
kernel spill, or these spill more, fails here.
"""
import json
import os

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPORT = os.path.join(HERE, "..", "vllm-grinqh-plugin_amd", "grinqh", "_lib", "kernel_resources.json")

# kernel family (a substring of the mangled name) -> scratch bytes per lane allowed
ALLOWED_SCRATCH = {
    "19prefill_tall_kernel": 192,
}


def _report():
    if not os.path.exists(REPORT):
        pytest.fail(f"{REPORT} missing: build the library first (python vllm-grinqh-plugin_amd/build.py)")
    with open(REPORT) as f:
        return json.load(f)


def test_report_covers_every_kernel_family():
    names = list(_report())
    for family in ("gemv_kernel", "decode_kernel", "prefill_kernel", "prefill_tall_kernel", "prefill_wide_kernel",
                   "repack_x_kernel", "splitk_reduce_kernel", "dequant_nk_kernel"):
        assert any(family in n for n in names), f"no {family} in the build's resource report"


def test_no_scratch_beyond_the_documented_spills():
    over = []
    for name, r in _report().items():
        scratch = r.get("scratch", 0)
        bound = next((b for fam, b in ALLOWED_SCRATCH.items() if fam in name), 0)
        if scratch > bound:
            over.append((name, scratch, bound))
    assert not over, "kernels using more scratch than allowed (name, bytes per lane, bound): " + repr(over[:8])
