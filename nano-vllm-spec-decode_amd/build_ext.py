"""Builds the HIP extension libsd_attn.so (gfx950) in-tree, next to the nanovllm_amd package.

    python nano-vllm-spec-decode_amd/build_ext.py [--jobs N]

Every csrc/*.hip and csrc/*.cpp file is compiled with hipcc to an object under _build/ and linked into
nanovllm_amd/libsd_attn.so. Packed-fp32 instruction selection is switched off for the device code, and MFMA
results are selected into VGPRs.
"""
import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "nanovllm_amd", "libsd_attn.so")
ARCH = "gfx950"
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", f"-I{os.path.join(HERE, '..', 'include')}"]
# MFMA results in VGPRs (-amdgpu-mfma-vgpr-form): kernels that need more than 256 registers a wave then keep
# their accumulators where the VALU reads them and give the AGPRs what only MFMAs read, instead of moving
# values between the two files every iteration (the compiler's default AGPR form).
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-mllvm", "-amdgpu-mfma-vgpr-form=1"]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP extension)")
    return path


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON, "-c", src, "-o", obj]
    if src.endswith(".hip"):
        cmd[1:1] = DEVICE
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = [ln for ln in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n" + "\n".join(noise))
    if any("warning" in ln for ln in noise):
        print("\n".join(noise), file=sys.stderr)
    return obj


def build(jobs: int = 8, verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(sources)} sources")
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    build(ap.parse_args().jobs)
