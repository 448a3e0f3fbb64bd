"""Builds libvqk_hip.so (gfx950) from the .hip sources in this directory.

Usage: python build.py [--out PATH] [--jobs N] [--save-temps DIR]

Every translation unit is compiled with hipcc for gfx950 only, with fp contraction off
(the sampler's noise and the quantizers must match the CPU oracle bit for bit) and with
packed-FP32 instruction selection disabled.
"""
import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(os.path.dirname(HERE), "vllm_quant_kernels")
REPO = os.path.dirname(os.path.dirname(HERE))
INCLUDE = os.path.join(REPO, "include")
DEFAULT_OUT = os.path.join(PKG, "libvqk_hip.so")

SOURCES = ["vqk_device.hip", "vqk_quant.hip", "vqk_lmhead.hip", "vqk_sampler.hip", "vqk_topk.hip"]


def hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libvqk_hip.so)")


def flags():
    return [
        "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", INCLUDE, "-I", HERE,
        "-Wno-unused-command-line-argument",
    ]


def build(out=DEFAULT_OUT, jobs=4, save_temps=None, verbose=False, defines=()):
    cc = hipcc()
    objdir = os.path.join(REPO, "_build", "obj" + "".join("_" + d.replace("=", "") for d in defines))
    os.makedirs(objdir, exist_ok=True)
    os.makedirs(os.path.dirname(out), exist_ok=True)

    def compile_one(src):
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        cmd = [cc] + flags() + [f"-D{d}" for d in defines] + ["-c", os.path.join(HERE, src), "-o", obj]
        if save_temps:
            os.makedirs(save_temps, exist_ok=True)
            cmd += ["-save-temps=obj"]
            cmd[cmd.index("-o") + 1] = os.path.join(save_temps, os.path.basename(obj))
            obj = cmd[cmd.index("-o") + 1]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr[-6000:]}")
        return obj

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = out + ".tmp"
    cmd = [cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=DEFAULT_OUT)
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--save-temps", default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("-D", dest="defines", action="append", default=[], help="extra preprocessor define")
    a = ap.parse_args()
    print(build(a.out, a.jobs, a.save_temps, a.verbose, tuple(a.defines)))
    sys.exit(0)
