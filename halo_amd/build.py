"""Build the halo_mi355x shared library (gfx950) and the CPU oracle in-tree.

The library is compiled with hipcc for gfx950 only. Flags:
  -fno-gpu-flush-denormals-to-zero   fp16/fp32 subnormal scales must survive (bit-exact dequant)
  -fhip-fp32-correctly-rounded-divide-sqrt   fp32 / and sqrtf correctly rounded (the RMS norm is
                                     bitwise the CPU's); clang's default for HIP, stated here
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed fp32 instructions
  -mcode-object-version=5            loadable by the HIP runtime torch bundles (ROCm 7.0) as well
                                     as /opt/rocm's (7.2)
  -mllvm -amdgpu-atomic-optimizer-strategy=None
                                     every atomic here is issued by one lane; the optimizer's
                                     wave scan reads the returned value at once, which waits for
                                     every load issued before it (the split-K ticket is taken after
                                     the weight loads and needed only at the workgroup's end)
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIB = PKG / "libhalo_mi355x.so"
CSRC = PKG / "csrc"
# the kernel files first: they take longest and are compiled in parallel with the rest
SOURCES = [CSRC / "k_gemv.hip", CSRC / "k_gemv_group.hip", CSRC / "k_gemm.hip", CSRC / "k_gemm_sx.hip", CSRC / "k_dequant.hip", CSRC / "k_argmax.hip", CSRC / "k_norm.hip",
           CSRC / "api.cpp", CSRC / "upload.cpp", CSRC / "host_utils.cpp", CSRC / "backend.cpp"]
OBJ_DIR = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "-O3",
    "--offload-arch=gfx950",
    "-std=c++20",
    "-fPIC",
    "-pthread",
    "-fno-gpu-flush-denormals-to-zero",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wall",
]


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: not an error.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build failed ({' '.join(cmd)}):\n{err}\n{proc.stdout}")
    if err.strip():
        sys.stderr.write(err + "\n")


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.name + ".o")
    _run([HIPCC, *HIP_FLAGS, "-c", "-o", str(obj), str(src)])
    return obj


def build_library() -> Path:
    """Every source to an object (in parallel), then one shared library."""
    OBJ_DIR.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=max(1, min(len(SOURCES), os.cpu_count() or 1))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-pthread", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> Path:
    _run(["make", "-B", "-C", str(ROOT / "oracle")])
    return ROOT / "oracle" / "liboracle.so"


CPP_TEST_SRC = ROOT / "tests" / "cpp" / "backend_pair.cpp"
CPP_TEST_BIN = ROOT / "tests" / "cpp" / "backend_pair"


def build_cpp_tests() -> Path:
    """The C++ test of the Backend adapter (host code only: g++, linked against the library
    and the oracle, found through $ORIGIN-relative run paths)."""
    _run(["g++", "-std=c++20", "-O1", "-Wall", "-o", str(CPP_TEST_BIN), str(CPP_TEST_SRC),
          "-L" + str(PKG), "-lhalo_mi355x", "-L" + str(ROOT / "oracle"), "-loracle",
          "-Wl,-rpath,$ORIGIN/../../halo_amd:$ORIGIN/../../oracle"])
    return CPP_TEST_BIN


def build_all() -> None:
    build_oracle()
    build_library()
    build_cpp_tests()


if __name__ == "__main__":
    build_all()
    print(LIB)
