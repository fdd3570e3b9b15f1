"""Build recipe of the gfx950 kernel library.

Compiles every ``csrc/*.hip`` translation unit with ``hipcc --offload-arch=gfx950`` (in
parallel, one process per file) and links them into ``_lib/libcollab_edge_attn.so`` inside
the package, so the library travels with the source tree; then compiles the PyTorch operator
layer ``csrc/torch_ops.cpp`` (host C++) into ``_lib/libcollab_edge_torch.so``, linked against
the kernel library.  Run ``python build.py`` or call
:func:`build`.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
OBJ_DIR = PKG_DIR / "_lib" / "obj"
LIB_PATH = PKG_DIR / "_lib" / "libcollab_edge_attn.so"
OPS_PATH = PKG_DIR / "_lib" / "libcollab_edge_torch.so"
INCLUDE = REPO_DIR / "include"
ARCH = os.environ.get("CEA_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
CXX = shutil.which("g++") or "c++"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
    # keep the compiler from emitting packed-FP32 VALU instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-file extras.  The prefill kernel handles +-inf explicitly and never produces or tests
# NaN; without NaN semantics the compiler drops the quieting v_max_f32 x,x,x it otherwise
# puts on every matrix-core result before a max.
FILE_FLAGS = {
    # M0 is set by the kernel's own LDS-DMA assembly; the clobber note is expected
    "attn_prefill.hip": ["-fno-honor-nans", "-Wno-inline-asm"],
    "attn_decode.hip": ["-fno-honor-nans", "-Wno-inline-asm"],
    # the layer ops round every product to the tensor dtype before the next add, as the
    # reference's separate tensor ops do: no multiply-add contraction (without this flag
    # x*cos + rot*sin in f16 becomes an f16 fma, and f32 products fuse into the sums)
    "layers.hip": ["-ffp-contract=off"],
    # the projection's epilogue rounds like the reference's separate ops (see layers.hip);
    # M0 is set by the LDS-DMA assembly
    "gemm.hip": ["-ffp-contract=off", "-Wno-inline-asm"],
}


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def _torch_flags():
    """Include / library directories and ABI flag of the installed PyTorch (host C++ only)."""
    import torch
    import torch.utils.cpp_extension as ce

    inc = [f"-I{p}" for p in ce.include_paths()]
    libdirs = ce.library_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return inc, libdirs, abi


def _compile_ops(inc, abi) -> Path:
    """The PyTorch operator layer (csrc/torch_ops.cpp): host C++ against torch's headers."""
    obj = OBJ_DIR / "torch_ops.o"
    rocm_inc = os.environ.get("ROCM_PATH", "/opt/rocm") + "/include"
    cmd = [CXX, "-O2", "-std=c++17", "-fPIC", "-Wall", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", *inc, f"-I{rocm_inc}", f"-I{INCLUDE}", "-c",
           str(CSRC / "torch_ops.cpp"), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"torch_ops.cpp failed to compile:\n{proc.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compiles all kernels and links the kernel library, then the PyTorch operator library
    on top of it; returns the kernel library's path."""
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    inc, libdirs, abi = _torch_flags()
    jobs = jobs or min(len(sources) + 1, max(1, (os.cpu_count() or 4)), 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        ops_obj = pool.submit(_compile_ops, inc, abi)
        objs = list(pool.map(_compile, sources))
        ops_obj = ops_obj.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    tmp = OPS_PATH.with_suffix(".so.tmp")
    cmd = [CXX, "-shared", "-fPIC", "-o", str(tmp), str(ops_obj), f"-L{LIB_PATH.parent}",
           "-lcollab_edge_attn", *[f"-L{d}" for d in libdirs], "-ltorch", "-ltorch_cpu", "-lc10",
           "-lc10_hip", "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{d}" for d in libdirs]]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"operator library link failed:\n{proc.stderr}")
    os.replace(tmp, OPS_PATH)
    if verbose:
        print(f"built {LIB_PATH} and {OPS_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
