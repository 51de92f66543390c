"""Build the gfx950 C-ABI library (libqlora_amd.so) from csrc/*.hip with hipcc.

Compiled in-tree, next to this file, so the library travels with the source tree. Flags:
  --offload-arch=gfx950      MI355X (CDNA4) only
  -ffp-contract=off          no implicit FMA: the NF4 dequant must round the product
                             code2 * absmax2 before adding the offset, as bitsandbytes does
  -target-feature -packed-fp32-ops   no packed fp32 VALU instructions
  -target-feature -fma-mix-insts      no v_fma_mix*: the NF4 decode's fp16(fp32(level * scale))
                             rounds twice, as bitsandbytes; the mix form rounds once
No vendor GEMM library is linked: every product runs on the package's own kernels.
Usage: python -m <package>.build  (or build() from __graft_entry__)
"""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libqlora_amd.so")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-shared", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Xclang", "-target-feature", "-Xclang", "-fma-mix-insts",
    "-fvisibility=hidden", "-Wno-unused-command-line-argument",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build(verbose=False, jobs=None):
    """Compile every csrc/*.hip to an object in parallel, then link libqlora_amd.so."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    procs = []
    objs = []
    for src in sources():
        obj = os.path.join(objdir, os.path.basename(src)[:-4] + ".o")
        objs.append(obj)
        cmd = [hipcc, *[f for f in FLAGS if f != "-shared"], "-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                            stderr=subprocess.STDOUT, text=True)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        if p.returncode != 0:
            failed.append((src, out))
        elif verbose and out.strip():
            print(out)
    if failed:
        msg = "\n".join(f"--- {s}\n{o}" for s, o in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    tmp = LIB + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
