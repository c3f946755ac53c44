"""Builds the HIP library (libglmmoe.so) in-tree for gfx950 with hipcc."""
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_lib")
LIB = os.path.join(OUT_DIR, "libglmmoe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # Every multiply-add that should fuse is written as an explicit fma; the
    # router's bit-exact reduction order depends on nothing else fusing.
    "-ffp-contract=off",
    # No packed-fp32 VALU instructions anywhere in this library.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def build(verbose=False, out_lib=None, defines=()):
    """Compiles csrc/ into out_lib (default: the in-tree _lib/libglmmoe.so)."""
    lib_path = out_lib or LIB
    out_dir = os.path.dirname(lib_path)
    os.makedirs(out_dir, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip"))) + sorted(
        glob.glob(os.path.join(CSRC, "*.cpp")))
    objs = []
    procs = []
    for src in srcs:
        obj = os.path.join(out_dir, os.path.basename(src) + ".o")
        lang = ["-x", "hip"] if src.endswith(".cpp") else []
        cmd = [HIPCC] + HIP_FLAGS + ["-D" + d for d in defines] + lang + ["-c", src, "-o", obj]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        objs.append(obj)
    failed = False
    for cmd, p in procs:
        out = p.communicate()[0].decode(errors="replace")
        out = "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l)
        if p.returncode != 0:
            failed = True
            sys.stderr.write(" ".join(cmd) + "\n" + out + "\n")
        elif verbose and out.strip():
            sys.stderr.write(out + "\n")
    if failed:
        raise RuntimeError("hipcc failed")
    tmp = lib_path + ".tmp"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs,
                   check=True)
    os.replace(tmp, lib_path)
    for o in objs:
        os.remove(o)
    if out_lib is None:
        # The peak-rate probe (a stand-alone program next to the library).
        probe = os.path.join(out_dir, "glmmoe_peaks")
        subprocess.run([HIPCC] + HIP_FLAGS + [os.path.join(HERE, "microbench", "peaks.hip"), "-o", probe],
                       check=True)
    return lib_path


if __name__ == "__main__":
    print(build(verbose=True))
