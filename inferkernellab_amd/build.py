"""Builds libikl_paged.so (the gfx950 HIP kernels behind the C ABI of
include/ikl_paged.h) in-tree with hipcc.

Usage: ``python -m inferkernellab_amd.build`` (or ``build()`` from Python).
Each ``.hip`` file is compiled to an object in parallel, then linked into
``inferkernellab_amd/libikl_paged.so`` with an atomic rename.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR / "_build"
LIB_NAME = "libikl_paged.so"
LIB_PATH = PACKAGE_DIR / LIB_NAME
ARCH = "gfx950"

SOURCES = (
    "abi.hip",
    "append_kv.hip",
    "paged_decode.hip",
    "paged_decode_mfma.hip",
    "paged_prefill.hip",
    "rope_append.hip",
    "read_probe.hip",
)

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed fp32 VALU ops are kept out of the device code on purpose.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Per-source additions. The prefill kernels produce no NaN of their own
# (masked scores are -inf, never 0/0): without NaN handling, fmaxf skips the
# IEEE canonicalisation of its operands in the softmax. The decode MFMA
# kernels keep their matrix accumulators in VGPRs: the 32-head kernels (one
# wave per SIMD) then lose the accumulator-register copies the allocator
# otherwise places in every tile (MQA balanced split 29.7 -> 28.6 us); the
# 16-head kernels already allocate VGPRs only (two waves per SIMD) and are
# unchanged.
SOURCE_FLAGS = {
    "paged_prefill.hip": ["-fno-honor-nans"],
    "paged_decode_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def source_hash() -> str:
    """First 16 hex digits of a SHA-256 over the kernel sources and the C
    ABI header (names and contents, sorted): the library embeds it, so a
    run can tell whether the library it loaded was built from the sources
    beside it."""
    import hashlib

    h = hashlib.sha256()
    files = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.h")) + [PACKAGE_DIR.parent / "include" / "ikl_paged.h"]
    for f in files:
        h.update(f.name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


def build_info() -> str:
    """'src:<source hash>,git:<revision>[-dirty]' (no spaces: it travels as a
    preprocessor definition)."""
    rev = "unknown"
    try:
        root = PACKAGE_DIR.parent
        out = subprocess.run(["git", "rev-parse", "--short=12", "HEAD"], cwd=root, capture_output=True,
                             text=True, timeout=10)
        if out.returncode == 0:
            rev = out.stdout.strip()
            st = subprocess.run(["git", "status", "--porcelain", "--untracked-files=no"], cwd=root,
                                capture_output=True, text=True, timeout=10)
            if st.returncode == 0 and st.stdout.strip():
                rev += "-dirty"
    except (OSError, subprocess.SubprocessError):
        pass
    return f"src:{source_hash()},git:{rev}"


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; ROCm is required to build libikl_paged.so")
    return path


def _compile(hipcc: str, src: Path, obj: Path, extra: list[str]) -> None:
    cmd = [hipcc, *COMMON_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{result.stdout}\n{result.stderr}")


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compile every HIP source for gfx950 and link libikl_paged.so."""
    hipcc = _hipcc()
    extra = list(extra_flags or [])
    BUILD_DIR.mkdir(exist_ok=True)
    objs = [BUILD_DIR / (name.replace(".hip", ".o")) for name in SOURCES]
    jobs = min(len(SOURCES), max(1, os.cpu_count() or 1))
    info = [f'-DIKL_BUILD_INFO="{build_info()}"']
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        futures = [
            pool.submit(_compile, hipcc, CSRC / name, obj,
                        [*SOURCE_FLAGS.get(name, []), *(info if name == "abi.hip" else []), *extra])
            for name, obj in zip(SOURCES, objs)
        ]
        for future in futures:
            future.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stdout}\n{result.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
