"""Build the HIP library (libf16hip.so) in-tree for gfx950.

Compiled with hipcc straight from csrc/ (one object per source under _build/, linked into one
shared library); no torch extension machinery, no JIT cache: the .so sits next to this file so
that it travels with the repository snapshot to the GPU box.

Flags:
  -ffp-contract=off    keep every add and multiply separately rounded (parity with the
                       reference's --fmad=false build and with the CPU restatement);
  -packed-fp32-ops off no packed FP32 instructions (they are avoided on this fleet).
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libf16hip.so")
SOURCES = ["fdm_kernels.hip", "gae_kernel.hip", "obs_kernels.hip", "policy_kernels.hip",
           "ppo_kernels.hip"]
ARCH = os.environ.get("F16_OFFLOAD_ARCH", "gfx950")


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src, obj, verbose):
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-c",
           "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I", os.path.join(ROOT, "include"), "-I", CSRC, "-o", obj, src]
    if verbose:
        cmd.append("-Rpass-analysis=kernel-resource-usage")
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)


def build(verbose=False):
    """Compile every HIP source (one hipcc process per source, in parallel) and link them
    into libf16hip.so (always recompiles)."""
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    procs = [_compile(os.path.join(CSRC, s), o, verbose) for s, o in zip(SOURCES, objs)]
    failed = False
    for s, p in zip(SOURCES, procs):
        out, err = p.communicate()
        if p.returncode != 0:
            sys.stderr.write(out + err)
            failed = True
        elif verbose:
            sys.stderr.write("\n".join(l for l in err.splitlines() if "remark" in l) + "\n")
    if failed:
        raise RuntimeError("hipcc failed building libf16hip.so")
    tmp = LIB + ".tmp"
    p = subprocess.run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs,
                       capture_output=True, text=True)
    if p.returncode != 0:
        sys.stderr.write(p.stdout + p.stderr)
        raise RuntimeError("hipcc failed linking libf16hip.so")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
