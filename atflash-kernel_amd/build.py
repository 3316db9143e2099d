"""Build the atflash HIP library for gfx950 in-tree.

    python atflash-kernel_amd/build.py [--verbose]

Compiles csrc/*.hip and csrc/*.cpp with hipcc (--offload-arch=gfx950) and links
atflash/libatflash_hip.so next to the Python package, so the library travels
with the source tree.  Kernel resource usage (VGPRs, AGPRs, spills, LDS) from
the compiler is written to _build/resource_usage.txt.
"""
import concurrent.futures as cf
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "atflash", "libatflash_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-x", "hip",
    # packed fp32 arithmetic stays off (v_pk_* fp32 forms are not used)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Rpass-analysis=kernel-resource-usage",
    "-Wno-unused-command-line-argument",
]


# Per-file flags.  The decode kernels take their first arguments as scalars
# that the dispatch preloads into SGPRs (kernarg preloading, gfx950): up to 14
# dwords (16 user SGPRs less the argument-block pointer).  A firmware without
# it runs the compiler's compatibility prologue, which loads them instead.
EXTRA = {"atf_decode.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=14"]}


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def compile_one(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON, *EXTRA.get(os.path.basename(src), []), "-I", CSRC, "-c", src, "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{p.stderr}")
    return obj, p.stderr


def resource_summary(logs):
    lines = []
    for src, text in logs:
        for m in re.finditer(r"remark: [^\n]*?Function Name: (\S+)", text):
            lines.append(f"{os.path.basename(src)} {m.group(1)}")
        for m in re.finditer(r"remark: [^\n]*?((?:VGPRs|AGPRs|ScratchSize|Occupancy|SGPRs|LDS Size)[^\n]*)", text):
            lines.append("    " + m.group(1))
    return "\n".join(lines)


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        results = list(ex.map(compile_one, srcs))
    objs = [o for o, _ in results]
    summary = resource_summary(list(zip(srcs, [log for _, log in results])))
    with open(os.path.join(BUILD, "resource_usage.txt"), "w") as f:
        f.write(summary + "\n")
    if verbose:
        print(summary)
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{p.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
