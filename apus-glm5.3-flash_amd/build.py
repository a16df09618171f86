"""Build libapus_ghip.so in-tree: the C host layer (gcc, C11) and the gfx950
HIP kernel units (hipcc), linked by hipcc into one shared library next to
this file. Also builds the test-only CPU checker under oracle/ (make).

Usage: python build.py   (or __graft_entry__.build())
"""
import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libapus_ghip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

C_SRCS = ["ghip_backend.c", "ghip_synth.c", "ghip_container.c"]
HIP_SRCS = ["k_linear.hip", "k_moe.hip", "k_moe_prefill.hip", "k_synth.hip"]

INC = ["-I" + os.path.join(ROOT, "include"), "-I" + CSRC]
CFLAGS = ["-std=c11", "-O2", "-Wall", "-Wextra", "-fPIC", "-ffp-contract=off",
          "-D_GNU_SOURCE", "-D__HIP_PLATFORM_AMD__",
          "-I" + os.path.join(ROCM, "include")] + INC
# gfx950 only; packed-fp32 ops disabled (the host pass warns that it does
# not know the feature: harmless); fp contraction pinned off.
HIPFLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
            "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang",
            "-packed-fp32-ops", "-Wno-unused-command-line-argument",
            "-Rpass-analysis=kernel-resource-usage"] + INC

_REMARK = re.compile(r"remark:\s+(Function Name|VGPRs Spill|ScratchSize \[bytes/lane\]"
                     r"|SGPRs Spill):\s*(\S+)")


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True)
    out = "\n".join(l for l in p.stdout.splitlines()
                    if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError("build failed: %s\n%s" % (" ".join(cmd), out))
    return out


def resource_usage(out):
    """Per-kernel {name: {"vgpr_spill", "scratch", "sgpr_spill"}} from the
    compiler's kernel-resource-usage remarks; the remark lines are dropped
    from the returned text."""
    usage, name, keep, ctx = {}, None, [], False
    for l in out.splitlines():
        m = _REMARK.search(l)
        if not m:
            if "kernel-resource-usage" in l:
                ctx = True
            elif not (ctx and re.match(r"\s*\d*\s*\|", l)):
                ctx = False
                keep.append(l)
            continue
        ctx = True
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            name = val
            usage[name] = {}
        elif name is not None:
            usage[name][{"VGPRs Spill": "vgpr_spill", "SGPRs Spill": "sgpr_spill"}
                        .get(key, "scratch")] = int(val)
    return usage, "\n".join(keep)


# kernels whose remarks must be present: if the compiler stops emitting the
# resource-usage remarks, or words them differently, the gate would see
# nothing and pass, so their absence fails the build instead
REQUIRED_KERNELS = ("k_moe_decode", "k_pf_gemm", "k_fp8_gemv_stream", "k_fp8_gemm")


def check_resources(usage, required=REQUIRED_KERNELS):
    """A kernel that spills VGPRs or uses scratch memory fails the build
    (SGPR spills go to VGPR lanes, not memory, and are allowed), and so does
    a required kernel with no parsed remarks (or no remarks at all)."""
    if not usage:
        raise RuntimeError("no kernel-resource-usage remarks parsed from the "
                           "compiler output: the spill/scratch gate cannot run")
    missing = [k for k in required if not any(k in name for name in usage)]
    if missing:
        raise RuntimeError("no resource-usage remarks for kernels: " + ", ".join(missing))
    incomplete = sorted(n for n, u in usage.items()
                        if "vgpr_spill" not in u or "scratch" not in u)
    if incomplete:
        raise RuntimeError("resource-usage remarks without spill/scratch figures: "
                           + ", ".join(incomplete))
    bad = ["%s: %d VGPR spills, %d B/lane scratch"
           % (k, u.get("vgpr_spill", 0), u.get("scratch", 0))
           for k, u in sorted(usage.items())
           if u.get("vgpr_spill", 0) or u.get("scratch", 0)]
    if bad:
        raise RuntimeError("kernels spill to scratch memory:\n  " + "\n  ".join(bad))


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    jobs = []
    objs = []
    for s in C_SRCS:
        o = os.path.join(BUILD, s + ".o")
        jobs.append(["gcc"] + CFLAGS + ["-c", os.path.join(CSRC, s), "-o", o])
        objs.append(o)
    for s in HIP_SRCS:
        o = os.path.join(BUILD, s + ".o")
        jobs.append([HIPCC] + HIPFLAGS + ["-c", os.path.join(CSRC, s), "-o", o])
        objs.append(o)
    usage = {}
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for out in ex.map(_run, jobs):
            u, out = resource_usage(out)
            usage.update(u)
            if verbose and out.strip():
                print(out)
    check_resources(usage)
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
         + ["-lm"])
    os.replace(tmp, LIB)
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle")])
    # the compiled C callers of the boundary (test programs, linked against
    # the library just built and the oracle)
    _run(["make", "-s", "-B", "-C", os.path.join(ROOT, "tests", "c")])
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
