"""Build libpai_hip.so in-tree (host C11 via gcc, kernels via hipcc for gfx950).

    python -m prosperoai_amd.build          # library + oracle checker

The library lands in prosperoai_amd/lib/ so it travels with the source
tree; objects go to prosperoai_amd/_build/.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "lib" / "libpai_hip.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

C_SOURCES = ["pai_hip.c", "pai_gguf.c", "pai_llama.c", "paiq.c", "pai_qref.c", "pai_v0.c", "pai_pai64.c"]
HIP_SOURCES = ["qlayout.hip", "qgemv.hip", "qgemv_mx.hip", "qgemm.hip", "qdecode.hip",
               "qscratch.hip", "qv0.hip"]
# qgemm.hip is also compiled once per block format (object name, defines):
# the four formats' GEMM kernels build in parallel
HIP_VARIANTS = [(f"qgemm_{f.lower()}.hip", "qgemm.hip",
                 [f"-DPAI_GEMM_FMT={f}", f"-DPAI_GEMM_ENTRY=paik_gemm_mfma_{f.lower()}"])
                for f in ("Q4_K", "Q6_K", "Q4_0", "Q8_0")]
HEADERS = ["paik.h", "qdev.h"]

# no floating-point contraction: the CPU twin reproduces the reference's
# separately rounded products and sums
C_FLAGS = ["-std=c11", "-O2", "-fPIC", "-ffp-contract=off", "-Wall", "-Wextra",
           "-Wno-unused-parameter",
           "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}", f"-I{ROOT / 'include'}",
           f"-I{CSRC}"]
HIP_FLAGS = ["-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}",
             # packed-FP32 VALU forms are kept out of the device code
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             f"-I{ROOT / 'include'}", f"-I{CSRC}", "-Wno-unused-result"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[0]} ... {cmd[-1]}")


def _compile(item) -> Path:
    """A C or HIP source, or (object name, HIP source, extra defines)."""
    name, src, defs = item if isinstance(item, tuple) else (item, item, [])
    out = OBJ / (name + ".o")
    if src.endswith(".c"):
        cmd = ["gcc", *C_FLAGS, "-c", str(CSRC / src), "-o", str(out)]
    else:
        cmd = [HIPCC, *HIP_FLAGS, *defs, "-c", str(CSRC / src), "-o", str(out)]
    _run(cmd)
    return out


def units() -> list:
    """Every compilation unit, longest first (so the pool starts them early)."""
    return [*HIP_VARIANTS, "qgemv.hip", "qgemv_mx.hip", "qlayout.hip", "qgemm.hip", "qdecode.hip",
            "qscratch.hip", "qv0.hip", *C_SOURCES]


def build_library(jobs: int = 6) -> Path:
    """Compile every source (always; this is also the 'does it build' check)."""
    OBJ.mkdir(parents=True, exist_ok=True)
    LIB.parent.mkdir(parents=True, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, units()))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp),
          *map(str, objs), "-lpthread", "-lm"])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> None:
    """The CPU checker (oracle/) and, where the reference tree exists, its build."""
    _run(["make", "-s", "-C", str(ROOT / "oracle")])


def main() -> None:
    if shutil.which("gcc") is None:
        raise RuntimeError("gcc not found")
    lib = build_library()
    build_oracle()
    print(f"built {lib}")


if __name__ == "__main__":
    main()
