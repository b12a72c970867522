"""Build helpers for the C-level test drivers (compiled with gcc at test time
against include/ and, where needed, librlrt_amd.so)."""
import ctypes
import os
import subprocess
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
LIBDIR = os.path.join(ROOT, "gb300-rl-runtime_amd", "lib")
_TMP = tempfile.mkdtemp(prefix="rlrt_tests_")


def build(src_rel: str, shared: bool = False, link_runtime: bool = False) -> str:
    src = os.path.join(ROOT, src_rel)
    out = os.path.join(_TMP, os.path.basename(src_rel).rsplit(".", 1)[0] + (".so" if shared else ""))
    cmd = ["gcc", "-std=gnu11", "-O1", "-Wall", "-I", INC, src, "-o", out]
    if shared:
        cmd[1:1] = ["-shared", "-fPIC"]
    if link_runtime:
        cmd += ["-L", LIBDIR, "-lrlrt_amd", "-Wl,-rpath," + LIBDIR, "-lpthread"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return out


def load_shared(src_rel: str, link_runtime: bool = True) -> ctypes.CDLL:
    return ctypes.CDLL(build(src_rel, shared=True, link_runtime=link_runtime))
