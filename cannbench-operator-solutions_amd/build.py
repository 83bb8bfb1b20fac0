"""Build the gfx950 HIP operator library in-tree: csrc/*.hip -> libcannbench_amd.so.

Each translation unit is compiled separately (parallel), then linked into one shared library that
exports the C ABI declared in include/cannbench_amd.h.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
OBJ_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libcannbench_amd.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed fp32 VALU ops are kept off (see the image notes on v_pk_* fp32 correctness)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # no FMA contraction: the reference's vector units round after every multiply and add, and the
    # dequant epilogues must reproduce those roundings bit for bit
    "-ffp-contract=off",
    "-Wall", "-Wno-unused-function",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src, defines=(), obj_dir=OBJ_DIR):
    obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
    cmd = [HIPCC, *HIP_FLAGS, *[f"-D{d}" for d in defines], "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = [ln for ln in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in ln]
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(msgs))
    return obj, msgs


def build(verbose=False, defines=(), out=LIB_PATH, obj_dir=OBJ_DIR):
    """Compile and link; `defines` are extra -D flags (tuning variants), `out` the library path."""
    os.makedirs(obj_dir, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        results = list(ex.map(lambda s: _compile(s, defines, obj_dir), srcs))
    objs = [o for o, _ in results]
    if verbose:
        for _, msgs in results:
            for m in msgs:
                print(m)
    tmp = out + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, out)
    return out


# Host-side AddressSanitizer + UBSan build of the same sources (the device code is unchanged: the
# sanitizers apply to the host passes only).  Test infrastructure: tests/test_sanitize.py loads it
# into a process that preloads the clang ASan runtime and runs the CPU tests (every validation
# branch of the C ABI, no GPU) against it.
SAN_DIR = os.path.join(OBJ_DIR, "san")
SAN_LIB = os.path.join(SAN_DIR, "libcannbench_amd_san.so")
SAN_FLAGS = ["-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]


def build_sanitized():
    """The sanitized library (rebuilt only when a source or header is newer than it)."""
    deps = [os.path.join(CSRC, f) for f in os.listdir(CSRC)] + [
        os.path.join(os.path.dirname(PKG_DIR), "include", "cannbench_amd.h"), os.path.abspath(__file__)]
    if os.path.exists(SAN_LIB) and os.path.getmtime(SAN_LIB) >= max(os.path.getmtime(d) for d in deps):
        return SAN_LIB
    global HIP_FLAGS
    saved = HIP_FLAGS
    HIP_FLAGS = saved + SAN_FLAGS
    try:
        return build(out=SAN_LIB, obj_dir=SAN_DIR)
    finally:
        HIP_FLAGS = saved


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
