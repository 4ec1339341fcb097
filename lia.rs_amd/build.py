"""Build recipe for liblia_hip.so (gfx950 code objects + the C ABI).

Every source under csrc/ is compiled by hipcc for gfx950 only, in-tree, and linked
into lia.rs_amd/liblia_hip.so.  Packed-FP32 instruction selection is disabled for the
device code (-packed-fp32-ops).
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "liblia_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SOURCES = ["attention.hip", "kv.hip", "transfer.hip", "sampling.hip", "hbm.hip", "host.cpp", "page_cache.cpp"]
DEVICE_FLAGS = ["--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-result"]


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    procs = []
    objs = []
    for src in SOURCES:
        path = os.path.join(CSRC, src)
        obj = os.path.join(OBJ, src + ".o")
        objs.append(obj)
        if src.endswith(".hip"):
            cmd = [HIPCC, *COMMON, *DEVICE_FLAGS, "-c", path, "-o", obj]
        else:
            cmd = [HIPCC, *COMMON, "-x", "c++", "-c", path, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = False
    for cmd, p in procs:
        out, _ = p.communicate()
        text = "\n".join(line for line in out.decode(errors="replace").splitlines()
                         if "packed-fp32-ops" not in line)
        if text.strip():
            print(text, file=sys.stderr)
        if p.returncode != 0:
            failed = True
    if failed:
        raise RuntimeError("liblia_hip build failed")
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", *objs, "-o", OUT]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return OUT


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
