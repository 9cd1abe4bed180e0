"""Build librfxq.so: the gfx950 code object embedded in the host library.

Steps (the counterpart of the reference's build.rs:199-252 + src/aot.rs, which
run nvcc per .cu file and embed the images as bytes):
  1. hipcc --offload-arch=gfx950 --cuda-device-only --no-gpu-bundle-output
     compiles csrc/kernels.hip to a raw code object (_build/rfxq_gfx950.co).
  2. An assembler stub .incbin's that file into .rodata (_build/embed.o).
  3. hipcc compiles csrc/scratch.hip (host code plus the fixed device scratch
     array of rfxq_gemm_no_alloc) to an ordinary object.
  4. The host C++ (csrc/rfxq.cpp, no device code) is linked with them against
     libamdhip64 into reflex_amd/librfxq.so, which hipModuleLoadData's the
     embedded image on first use.

Run: python -m reflex_amd.build
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
LIB = os.path.join(HERE, "librfxq.so")
ARCH = "gfx950"

DEVICE_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "--cuda-device-only", "--no-gpu-bundle-output",
    # packed FP32 instructions stay disabled in every HIP compile of this project
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-variable",
] + os.environ.get("RFXQ_EXTRA_DEVICE_FLAGS", "").split()


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out:
        print(out)


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    co = os.path.join(BUILD, f"rfxq_{ARCH}.co")
    _run([os.path.join(ROCM, "bin", "hipcc"), *DEVICE_FLAGS, "-c", os.path.join(CSRC, "kernels.hip"), "-o", co],
         verbose)
    embed_s = os.path.join(BUILD, "embed.S")
    with open(embed_s, "w") as f:
        f.write(
            "    .section .rodata\n"
            "    .p2align 12\n"
            "    .globl rfxq_code_object\n"
            "rfxq_code_object:\n"
            f"    .incbin \"{co}\"\n"
            "    .globl rfxq_code_object_end\n"
            "rfxq_code_object_end:\n"
            "    .byte 0\n"
            "    .section .note.GNU-stack,\"\",@progbits\n"
        )
    embed_o = os.path.join(BUILD, "embed.o")
    _run(["gcc", "-c", embed_s, "-o", embed_o], verbose)
    # the fixed scratch array of rfxq_gemm_no_alloc: host + gfx950 device code
    scratch_o = os.path.join(BUILD, "scratch.o")
    _run([os.path.join(ROCM, "bin", "hipcc"), "-x", "hip", "-O2", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall",
          "-c", os.path.join(CSRC, "scratch.hip"), "-o", scratch_o], verbose)
    tmp = LIB + ".tmp"
    _run([
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fopenmp", "-Wall", "-Wextra", "-Wno-unused-parameter",
        "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", *os.environ.get("RFXQ_EXTRA_HOST_FLAGS", "").split(),
        os.path.join(CSRC, "rfxq.cpp"), embed_o, scratch_o,
        f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-o", tmp,
    ], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
