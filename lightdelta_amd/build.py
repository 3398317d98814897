"""Build liblightdelta_hip.so (gfx950) in-tree with hipcc.

Usage: python -m lightdelta_amd.build   (or __graft_entry__.build()).
Every call recompiles; objects go to lightdelta_amd/_build/, the library next to this file.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "liblightdelta_hip.so"
# torch.ops.lightdelta dispatcher kernels (host C++ over the C ABI; see csrc/torch_ops.cpp)
TORCH_LIBRARY = PACKAGE / "liblightdelta_torch.so"
SOURCES = ("abi.hip", "gdn_decode.hip", "prefill_serial.hip", "prefill_chunked.hip",
           "state_io.hip")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fno-gpu-rdc",
    "-Wall",
    "-Werror=return-type",
    # Packed fp32 VALU forms are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Atomics stay as written: the optimizer's wave-aggregated form of a returning atomic
    # consumes the result at once, which waits for every load in flight (the conv-state
    # ticket count is issued mid-kernel and first read at the end).
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


# Per-source additions.  gdn_decode.hip: its decode kernel takes the request-metadata pointers
# and the head count as its first 7 argument dwords, which the hardware then preloads into
# SGPRs at launch (kernels without such leading scalar arguments preload nothing).
EXTRA_FLAGS = {"gdn_decode.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=7"]}


def _rocm() -> Path:
    return Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the HIP library needs ROCm's hipcc to build")
    return path


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(
            "build step failed:\n" + " ".join(cmd) + "\n" + result.stdout + result.stderr
        )


def build(verbose: bool = False) -> Path:
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    objects = []
    commands = []
    for name in SOURCES:
        obj = BUILD / (Path(name).stem + ".o")
        objects.append(obj)
        commands.append([hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(name, []), "-c", str(CSRC / name),
                         "-o", str(obj)])
    workers = max(1, min(len(commands), os.cpu_count() or 1, 8))
    with ThreadPoolExecutor(workers) as pool:
        list(pool.map(_run, commands))
    tmp = LIBRARY.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          f"-Wl,-soname,{LIBRARY.name}", *map(str, objects)])
    os.replace(tmp, LIBRARY)
    build_torch_ops()
    if verbose:
        print(f"built {LIBRARY} and {TORCH_LIBRARY}", file=sys.stderr)
    return LIBRARY


def build_torch_ops() -> Path:
    """liblightdelta_torch.so: csrc/torch_ops.cpp compiled by the host compiler against
    torch's headers and libraries (c10, c10_hip, torch_cpu) and linked to
    liblightdelta_hip.so, found next to it at load time."""
    import torch

    torch_dir = Path(torch.__file__).resolve().parent
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("no host C++ compiler (g++) for the torch.ops kernels")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = TORCH_LIBRARY.with_suffix(".so.tmp")
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
          "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM", f"-I{torch_dir / 'include'}",
          f"-I{torch_dir / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
          f"-I{_rocm() / 'include'}", f"-I{ROOT / 'include'}", str(CSRC / "torch_ops.cpp"),
          "-o", str(tmp), f"-L{torch_dir / 'lib'}", "-lc10", "-lc10_hip", "-ltorch_cpu",
          f"-L{PACKAGE}", "-llightdelta_hip", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, TORCH_LIBRARY)
    return TORCH_LIBRARY


if __name__ == "__main__":
    build(verbose=True)
