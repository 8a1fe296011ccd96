"""Build libaiter_amd.so (gfx950) from aiter_amd/csrc/*.hip with hipcc.

Objects go to aiter_amd/_build/, the shared library next to this file so it
is loaded in-tree.  Each kernel's registers, spills, scratch, LDS and
occupancy, as the compiler reports them, go to
aiter_amd/_build/resource_usage.json.  Usage: ``python -m aiter_amd.build``
(or ``build()``).

``python -m aiter_amd.build --sanitize`` builds a second library,
aiter_amd/_build_san/libaiter_amd_san.so, whose host code (the C ABI's
argument checks, layouts and launch set-up) carries AddressSanitizer and
UndefinedBehaviorSanitizer; the device code is built as usual.  The CPU tests
run against it with

    ASAN_OPTIONS=detect_leaks=0 LD_PRELOAD=<clang's libclang_rt.asan-x86_64.so> \
    AITER_AMD_LIB=aiter_amd/_build_san/libaiter_amd_san.so python -m pytest tests -m "not gpu"

(``sanitizer_runtime()`` finds the runtime; the GPU tests are not run so).
"""
from __future__ import annotations

import concurrent.futures as cf
import json
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libaiter_amd.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 VALU ops stay off (only ordinary scalar fp32 code is emitted)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results straight into VGPRs: the block-scale FMA reads them there
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build aiter_amd)")


RESOURCE_USAGE = BUILD_DIR / "resource_usage.json"

_REMARKS = {
    "vgpr": re.compile(r"remark:\s+VGPRs: (\d+)"),
    "agpr": re.compile(r"remark:\s+AGPRs: (\d+)"),
    "vgpr_spill": re.compile(r"remark:\s+VGPRs Spill: (\d+)"),
    "sgpr_spill": re.compile(r"remark:\s+SGPRs Spill: (\d+)"),
    "scratch": re.compile(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)"),
    "lds": re.compile(r"remark:\s+LDS Size \[bytes/block\]: (\d+)"),
    "occupancy": re.compile(r"remark:\s+Occupancy \[waves/SIMD\]: (\d+)"),
}


def _resource_usage(stderr: str) -> dict:
    """Per-kernel register, spill, scratch, LDS and occupancy figures from
    the compiler's kernel-resource-usage remarks, keyed by mangled name."""
    out, cur = {}, None
    for line in stderr.splitlines():
        m = re.search(r"remark:\s+Function Name: (\S+)", line)
        if m:
            cur = out.setdefault(m.group(1), {})
            continue
        if cur is None:
            continue
        for key, pat in _REMARKS.items():
            m = pat.search(line)
            if m:
                cur[key] = int(m.group(1))
    return out


def _compile(src: Path, hipcc: str):
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-I", str(CSRC),
           "-I", str(PKG_DIR.parent / "include"), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj, _resource_usage(res.stderr)


SAN_DIR = PKG_DIR / "_build_san"
SAN_LIB_PATH = SAN_DIR / "libaiter_amd_san.so"
# host-only sanitizers: each -fsanitize= applies to the host pass alone
SAN_FLAGS = ["-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-omit-frame-pointer"]


def sanitizer_runtime() -> Path:
    """clang's AddressSanitizer runtime, preloaded into python for the sanitized library."""
    hipcc = Path(_hipcc()).resolve()
    for root in (hipcc.parent.parent / "lib" / "llvm" / "lib" / "clang",
                 Path("/opt/rocm/lib/llvm/lib/clang")):
        hits = sorted(root.glob("*/lib/linux/libclang_rt.asan-x86_64.so"))
        if hits:
            return hits[-1]
    raise RuntimeError("libclang_rt.asan-x86_64.so not found next to hipcc")


def build_sanitized(verbose: bool = True) -> Path:
    """The library with AddressSanitizer + UndefinedBehaviorSanitizer host code."""
    hipcc = _hipcc()
    SAN_DIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))

    def one(src: Path) -> Path:
        obj = SAN_DIR / (src.stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, *SAN_FLAGS, "-I", str(CSRC),
               "-I", str(PKG_DIR.parent / "include"), "-c", str(src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(one, srcs))
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Xarch_host", "-fsanitize=address",
           "-Xarch_host", "-fsanitize=undefined", "-o", str(SAN_LIB_PATH), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    if verbose:
        print(f"[aiter_amd] built {SAN_LIB_PATH} (host sanitizers)", file=sys.stderr)
    return SAN_LIB_PATH


def build(verbose: bool = True) -> Path:
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        done = list(ex.map(lambda s: _compile(s, hipcc), srcs))
    objs = [o for o, _ in done]
    usage = {src.name: u for src, (_, u) in zip(srcs, done)}
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    RESOURCE_USAGE.write_text(json.dumps(usage, indent=1, sort_keys=True))
    if verbose:
        print(f"[aiter_amd] built {LIB_PATH} from {len(srcs)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    if "--sanitize" in sys.argv[1:]:
        build_sanitized()
    else:
        build()
