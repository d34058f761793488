"""Compile the HIP/C++ sources of this package into libsqattn.so for gfx950.

Every source is compiled by hipcc (-x hip) into _build/, then linked into a
shared library next to this file. Flags:
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed fp32 VALU ops
  -ffp-contract=fast-honor-pragmas is hipcc's default; code that must round
  every multiply and add on its own (the q4_0 quantizer, the K/Q producer)
  says #pragma clang fp contract(off): HIP's __fmul_rn/__fadd_rn are plain
  * and + and do not stop the fusion.
"""
import concurrent.futures
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libsqattn.so")
ARCH = os.environ.get("SQA_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-x", "hip",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-I", os.path.join(ROOT, "include"),
]


def sources():
    csrc = os.path.join(HERE, "csrc")
    return sorted(glob.glob(os.path.join(csrc, "*.hip")) + glob.glob(os.path.join(csrc, "*.cpp")))


# Per-source extra flags. fa_prefill.hip: its MFMA accumulators are read and
# rescaled by VALU code, so keep every MFMA result in VGPRs (the AGPR form makes
# the register allocator copy the 128-register accumulator on every tile).
EXTRA_FLAGS = {
    "fa_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"],
}


def _compile(src, out):
    cmd = [HIPCC] + CFLAGS + EXTRA_FLAGS.get(os.path.basename(src), []) + ["-c", src, "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{errs}")
    if errs.strip():
        sys.stderr.write(errs + "\n")
    return out


def build(verbose=False):
    bdir = os.path.join(HERE, "_build")
    os.makedirs(bdir, exist_ok=True)
    srcs = sources()
    outs = [os.path.join(bdir, os.path.basename(s) + ".o") for s in srcs]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(_compile, srcs, outs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + outs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
