"""Build libmi355x_encoder.so (gfx950) in-tree with hipcc.

Usage: ``python -m tiktoktechjam2026track3_amd.build_native`` or
``build_native.build()``.  Each ``csrc/*.hip`` file is compiled to an object in
``csrc/_build/`` in parallel, then linked into ``libmi355x_encoder.so`` next to
this file.  The library is always rebuilt when ``build()`` is called.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR / "csrc"
BUILD_DIR = CSRC_DIR / "_build"
LIBRARY_NAME = "libmi355x_encoder.so"
LIBRARY_PATH = PACKAGE_DIR / LIBRARY_NAME
OFFLOAD_ARCH = "gfx950"

SOURCES = (
    "layernorm.hip",
    "gemm.hip",
    "attention.hip",
    "attention_hd8.hip",
    "attention_hd32.hip",
    "attention_hd64.hip",
    "attention_hd128.hip",
    "attention_hd256.hip",
    "flash_attention.hip",
    "block_tail.hip",
    "capi.hip",
)

# Packed FP32 VALU ops (v_pk_fma_f32 and friends) are disabled for every device
# compile; hipcc's host pass prints a harmless "not a recognized feature" note.
COMMON_FLAGS = (
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={OFFLOAD_ARCH}",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
)


# Per-source extra flags.  The attention kernels read every score accumulator
# with VALU instructions; keeping MFMA results in VGPRs (not AGPRs) saves a
# v_accvgpr_read per score.  The GEMM keeps the compiler's choice: its large
# accumulator tiles live in AGPRs.
EXTRA_FLAGS = {
    "attention_hd8.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form"),
    "attention_hd32.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form"),
    "attention_hd64.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form"),
    "attention_hd128.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form"),
    "attention_hd256.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form"),
    "flash_attention.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form"),
}


def _hipcc() -> str:
    candidate = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(candidate).exists():
        raise RuntimeError("hipcc not found; the gfx950 HIP library cannot be built")
    return candidate


# Text of the warning clang prints for a target feature it does not know.  The
# host (x86) pass of every hipcc compile prints it for -packed-fp32-ops; the
# device pass must not (_check_device_feature_flag), and the built code is
# scanned for packed FP32 instructions as well (_check_mfma_hazards).
_UNKNOWN_FEATURE = "is not a recognized feature for this target"


def _check_device_feature_flag(hipcc: str) -> None:
    """Fail when the gfx950 device pass does not recognise -packed-fp32-ops:
    a device-only compile of a small kernel with the build's flags must be
    free of the unknown-feature warning that the host pass prints."""
    probe_dir = BUILD_DIR / "feature_probe"
    probe_dir.mkdir(parents=True, exist_ok=True)
    src = probe_dir / "probe.hip"
    src.write_text(
        "#include <hip/hip_runtime.h>\n"
        "typedef float f2 __attribute__((ext_vector_type(2)));\n"
        "__global__ void probe(f2* a, const f2* b) { a[threadIdx.x] = a[threadIdx.x] * b[threadIdx.x] + b[0]; }\n"
    )
    cmd = [hipcc, *COMMON_FLAGS, "--cuda-device-only", "-c", str(src), "-o", str(probe_dir / "probe.o")]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"device feature probe failed: {' '.join(cmd)}\n{proc.stdout}")
    if _UNKNOWN_FEATURE in proc.stdout:
        raise RuntimeError("the gfx950 device pass ignores -packed-fp32-ops:\n" + proc.stdout.strip())


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # the host pass's unknown-feature note (the device pass is checked by
    # _check_device_feature_flag before any source is compiled)
    noise = _UNKNOWN_FEATURE
    output = "\n".join(
        line for line in proc.stdout.splitlines() if noise not in line
    ).strip()
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{output}")
    if output:
        print(output, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source for gfx950 and link the shared library."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    _check_device_feature_flag(hipcc)
    include = f"-I{PACKAGE_DIR.parent / 'include'}"
    objects = []
    commands = []
    for name in SOURCES:
        src = CSRC_DIR / name
        obj = BUILD_DIR / (src.stem + ".o")
        objects.append(obj)
        extra = EXTRA_FLAGS.get(name, ())
        commands.append([hipcc, *COMMON_FLAGS, *extra, include, "-c", str(src), "-o", str(obj)])
    workers = jobs or min(len(commands), max(1, (os.cpu_count() or 2)))
    if verbose:
        for cmd in commands:
            print(" ".join(cmd))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        for future in [pool.submit(_run, cmd) for cmd in commands]:
            future.result()
    tmp = LIBRARY_PATH.with_suffix(".so.tmp")
    link = [hipcc, "-shared", "-fPIC", f"--offload-arch={OFFLOAD_ARCH}", *map(str, objects), "-o", str(tmp)]
    if verbose:
        print(" ".join(link))
    _run(link)
    _check_launch_stubs(tmp)
    _check_mfma_hazards(objects, jobs=workers)
    os.replace(tmp, LIBRARY_PATH)
    return LIBRARY_PATH


def _check_mfma_hazards(objects, jobs: int) -> None:
    """Fail the build when any path reads an MFMA result too early, or when
    packed FP32 instructions appear (hazard_check.py: the device code is
    disassembled and every path after each MFMA is walked)."""
    from . import hazard_check

    if not hazard_check.tools_available():
        print("warning: ROCm LLVM tools not found; MFMA hazard check skipped", file=sys.stderr)
        return
    report = hazard_check.check_objects(objects, jobs=jobs)
    if report.findings:
        details = "\n".join(str(f) for f in report.findings[:20])
        raise RuntimeError(f"MFMA result read with too few wait states ({len(report.findings)} finding(s)):\n{details}")
    if report.packed_fp32:
        details = "\n".join(report.packed_fp32[:20])
        raise RuntimeError(f"packed FP32 instructions in the device code (-packed-fp32-ops not honoured):\n{details}")


def _check_launch_stubs(path: Path) -> None:
    """Fail the build when a kernel's host-side launch stub is missing.

    Some kernel template bodies make clang's host pass drop the stub without a
    diagnostic; the library then links but cannot be loaded.  ``nm`` lists
    such stubs as undefined symbols.
    """
    nm = shutil.which("nm")
    if nm is None:
        return
    proc = subprocess.run([nm, "-D", "--undefined-only", str(path)], capture_output=True, text=True)
    # A dropped stub shows up either as the stub itself or as the kernel's
    # host-side handle (the kernel's own mangled name, in namespace enc).
    missing = [
        line.split()[-1]
        for line in proc.stdout.splitlines()
        if "__device_stub__" in line or "_ZN3enc" in line
    ]
    if missing:
        raise RuntimeError(f"{path.name}: {len(missing)} kernel launch stub(s) missing, e.g. {missing[0]}")


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
