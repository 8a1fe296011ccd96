"""Register budget of every built kernel -- CPU only.

The GEMM kernels keep their accumulators, the next K block's operands and
the epilogue's values in VGPRs at two waves per SIMD. One epilogue change
that pushes that past 256 VGPRs makes the compiler spill to scratch
memory, which costs no correctness but doubled the stage-1 prefill time in
one measured case. The build records the compiler's kernel-resource-usage
remarks (aiter_amd/_build/resource_usage.json); this test holds every
kernel to no spills and no scratch, and the GEMM kernels to at least two
waves per SIMD.
"""
import json

import pytest

from aiter_amd import build as B


def _usage():
    path = B.RESOURCE_USAGE
    if not path.exists():
        pytest.skip("no resource_usage.json: run aiter_amd.build first")
    sources = [*B.CSRC.glob("*.hip"), *B.CSRC.glob("*.h"), *(B.PKG_DIR.parent / "include").glob("*.h")]
    if any(p.stat().st_mtime > path.stat().st_mtime for p in sources):
        pytest.skip("resource_usage.json is older than the sources: rebuild first")
    return json.loads(path.read_text())


def test_every_source_reported():
    usage = _usage()
    assert set(usage) == {p.name for p in B.CSRC.glob("*.hip")}
    # the GEMM, sorting, quant and routing sources all define kernels; the two
    # C-ABI sources are host code
    for name, kernels in usage.items():
        if name not in ("abi.hip", "ctypes_ffi.hip"):
            assert kernels, name


def test_no_spills_or_scratch():
    bad = [(src, k, v) for src, ks in _usage().items() for k, v in ks.items()
           if v.get("vgpr_spill", 0) or v.get("sgpr_spill", 0) or v.get("scratch", 0)]
    assert not bad, bad[:5]


def test_gemm_kernels_keep_two_waves_per_simd():
    for src, ks in _usage().items():
        if src.startswith("moe_gemm"):
            for k, v in ks.items():
                assert v["vgpr"] + v.get("agpr", 0) <= 256 and v["occupancy"] >= 2, (src, k, v)
