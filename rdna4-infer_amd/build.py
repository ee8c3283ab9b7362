"""Build librdna4attn.so for gfx950 in-tree with hipcc (no torch extension).

Usage: python rdna4-infer_amd/build.py   (also called by __graft_entry__.build()).
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "librdna4attn.so")
SOURCES = ["kv.hip", "attn_generic.hip", "attn_decode_mfma.hip", "attn_prefill_mfma.hip", "prefill.hip", "misc.hip", "merge.hip", "qk_epilogue.hip", "capi.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    # packed FP32 instructions are kept out of every code object
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src):
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = [l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l]
    return src, r.returncode, obj, "\n".join(msgs)


def build(verbose=True, out=None, extra=()):
    """Compile every source and link the library (to `out`, default in-tree)."""
    global FLAGS
    flags0 = FLAGS
    FLAGS = FLAGS + list(extra)
    try:
        return _build(verbose, out or LIB)
    finally:
        FLAGS = flags0


def _build(verbose, lib_path):
    os.makedirs(OBJ, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        results = list(ex.map(_compile, SOURCES))
    bad = [r for r in results if r[1] != 0]
    for src, rc, _, msg in results:
        if msg.strip() and (verbose or rc):
            print("[%s]\n%s" % (src, msg), file=sys.stderr)
    if bad:
        raise RuntimeError("hipcc failed for: " + ", ".join(b[0] for b in bad))
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", lib_path] + [r[2] for r in results]
    subprocess.run(cmd, check=True)
    return lib_path


ROOT = os.path.dirname(HERE)
SHIM_CHECK_SRC = os.path.join(ROOT, "tests", "shim_kv_device.hip")
SHIM_CHECK_LIB = os.path.join(ROOT, "tests", "libshimkv.so")


def build_shim_check():
    """Compile the device-side check of the include/rdna4 shims (tests only)."""
    cmd = [HIPCC, *FLAGS, "-shared", "-I", os.path.join(ROOT, "include"), SHIM_CHECK_SRC,
           "-o", SHIM_CHECK_LIB]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError("hipcc failed for shim_kv_device.hip:\n" + r.stderr)
    return SHIM_CHECK_LIB


if __name__ == "__main__":
    # python build.py [out.so] [-DNAME=VALUE ...]: variant builds for experiments
    args = sys.argv[1:]
    out = next((a for a in args if a.endswith(".so")), None)
    print(build(out=out, extra=[a for a in args if a.startswith("-D")]))
