"""Build liblazyrecall_hip.so (gfx950) from csrc/*.hip with hipcc, the host planner module
_plan from csrc/host_plan.cpp with g++ against torch's headers, the recall archive
liblazyrecall_archive.so from csrc/archive.cpp with g++, and the recall transport's ring
liblazyrecall_recall.so from csrc/recall_ring.cpp with g++ against the HIP runtime API.

Run as ``python -m code_for_iclr27_amd.build``. Each translation unit is compiled in parallel,
then linked into ``code_for_iclr27_amd/liblazyrecall_hip.so`` next to this file; the planner
becomes ``code_for_iclr27_amd/_plan<EXT_SUFFIX>``.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR.parent / "_build" / "hip"
LIBRARY = PACKAGE_DIR / "liblazyrecall_hip.so"
ARCH = os.environ.get("LAZYRECALL_ARCH", "gfx950")

COMPILE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    # Reproducible arithmetic: no implicit multiply-add contraction (the reference builds with
    # --fmad=false); kernels that want an FMA call it explicitly.
    "-ffp-contract=off",
    # Packed-FP32 VALU forms are kept out of generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs: the scorer epilogues read every accumulator element, and
    # the AGPR form would add one v_accvgpr_read per element.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    candidates = [shutil.which("hipcc"), "/opt/rocm/bin/hipcc"]
    for candidate in candidates:
        if candidate and os.path.exists(candidate):
            return candidate
    raise RuntimeError("hipcc not found; the HIP toolchain is required to build liblazyrecall_hip.so")


def _run(command: list[str]) -> None:
    result = subprocess.run(command, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(command)}\n{stderr}")
    if stderr.strip():
        sys.stderr.write(stderr + "\n")


def build_host_plan(verbose: bool = False) -> Path:
    """The host-side planner and launcher (a CPython extension; no GPU code: it calls the
    library's entry points on torch's current HIP stream)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    target = PACKAGE_DIR / ("_plan" + sysconfig.get_config_var("EXT_SUFFIX"))
    temporary = target.with_name(target.name + ".tmp")
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    includes = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"],
                str(PACKAGE_DIR.parent / "include"), str(rocm / "include")]
    library_dirs = cpp_extension.library_paths()
    command = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Wno-unused-function",
               f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
               "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM",
               "-DTORCH_EXTENSION_NAME=_plan", str(SOURCE_DIR / "host_plan.cpp"),
               "-o", str(temporary)]
    command += [f"-I{path}" for path in includes]
    command += [f"-L{path}" for path in library_dirs]
    command += [f"-Wl,-rpath,{path}" for path in library_dirs]
    command += ["-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
                f"-L{rocm / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{rocm / 'lib'}"]
    if verbose:
        print(" ".join(command), flush=True)
    _run(command)
    os.replace(temporary, target)
    return target


ARCHIVE = PACKAGE_DIR / "liblazyrecall_archive.so"


def build_archive(verbose: bool = False) -> Path:
    """The recall archive (host C++, no GPU code, no torch): liblazyrecall_archive.so."""
    temporary = ARCHIVE.with_suffix(".so.tmp")
    command = ["g++", "-O3", "-std=c++17", "-march=x86-64-v3", "-shared", "-fPIC", "-pthread",
               "-Wall", str(SOURCE_DIR / "archive.cpp"), "-o", str(temporary)]
    if verbose:
        print(" ".join(command), flush=True)
    _run(command)
    os.replace(temporary, ARCHIVE)
    return ARCHIVE


RECALL = PACKAGE_DIR / "liblazyrecall_recall.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def build_recall(verbose: bool = False) -> Path:
    """The recall transport's ring (host C++ against the HIP runtime API, no GPU code):
    liblazyrecall_recall.so, linked to liblazyrecall_archive.so next to it."""
    temporary = RECALL.with_suffix(".so.tmp")
    command = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-pthread", "-Wall",
               "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}",
               f"-I{PACKAGE_DIR.parent / 'include'}", str(SOURCE_DIR / "recall_ring.cpp"),
               "-o", str(temporary), f"-L{PACKAGE_DIR}", "-llazyrecall_archive",
               "-Wl,-rpath,$ORIGIN", f"-L{ROCM / 'lib'}", "-lamdhip64",
               f"-Wl,-rpath,{ROCM / 'lib'}"]
    if verbose:
        print(" ".join(command), flush=True)
    _run(command)
    os.replace(temporary, RECALL)
    return RECALL


def build_host_libraries(verbose: bool = False) -> None:
    """The archive, then the ring that links it."""
    build_archive(verbose)
    build_recall(verbose)


def build(verbose: bool = False) -> Path:
    hipcc = _hipcc()
    sources = sorted(SOURCE_DIR.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {SOURCE_DIR}")
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    objects = [BUILD_DIR / (source.stem + ".o") for source in sources]

    def compile_one(pair):
        source, obj = pair
        command = [hipcc, *COMPILE_FLAGS, "-c", str(source), "-o", str(obj)]
        if verbose:
            print(" ".join(command), flush=True)
        _run(command)
        return obj

    workers = min(len(sources) + 1, max(1, (os.cpu_count() or 4)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        planner = pool.submit(build_host_plan, verbose)
        archive = pool.submit(build_host_libraries, verbose)
        list(pool.map(compile_one, zip(sources, objects)))
        planner.result()
        archive.result()
    temporary = LIBRARY.with_suffix(".so.tmp")
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(temporary),
            *map(str, objects)]
    if verbose:
        print(" ".join(link), flush=True)
    _run(link)
    os.replace(temporary, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
