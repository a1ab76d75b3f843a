"""Build the gfx950 kernels into hy_nomas/libhynomas_hip.so (in-tree, so the library travels with the repo).

    python comfyui-hy-nomas_amd/build.py [-v]

Every .hip file under csrc/ is compiled for gfx950 only (one object per file, in parallel) and linked
into one shared library with a plain C ABI (include/hynomas.h).  The library links the HIP runtime by
its soname, so inside a process that imported torch it binds to torch's already-loaded runtime and the
stream handles torch hands out are valid for it.
"""
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "hy_nomas", "libhynomas_hip.so")
# the benchmark's peak-rate probes (csrc/probes/): a library of their own, not part of the C ABI
PROBES_OUT = os.path.join(HERE, "hy_nomas", "libhynomas_probes.so")
ARCH = "gfx950"

# -ffp-contract=off: every fused multiply-add in the kernels is written explicitly.
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 from the auto-vectorizer.
HIPCC_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-I", os.path.join(HERE, "..", "include")]


def hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    return path if os.path.exists(path) else "hipcc"


def build(verbose=False, jobs=None):
    os.makedirs(BUILD, exist_ok=True)
    libs = {OUT: sorted(glob.glob(os.path.join(CSRC, "*.hip"))),
            PROBES_OUT: sorted(glob.glob(os.path.join(CSRC, "probes", "*.hip")))}
    sources = [src for srcs in libs.values() for src in srcs]
    jobs = jobs or min(len(sources), os.cpu_count() or 1, 16)
    objects, running = {}, []
    for src in sources:
        obj = os.path.join(BUILD, os.path.relpath(src, CSRC).replace(os.sep, "_") + ".o")
        objects[src] = obj
        cmd = [hipcc()] + HIPCC_FLAGS + ["-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        running.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        if len(running) >= jobs:
            _reap(running.pop(0), verbose)
    while running:
        _reap(running.pop(0), verbose)
    for out, srcs in libs.items():
        tmp = out + ".tmp"
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC"] + [objects[s] for s in srcs] + ["-o", tmp]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        os.replace(tmp, out)
    return OUT


def _reap(item, verbose):
    src, proc = item
    out, _ = proc.communicate()
    text = "\n".join(line for line in out.decode(errors="replace").splitlines()
                     if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{text}")
    if verbose and text.strip():
        print(text, flush=True)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
