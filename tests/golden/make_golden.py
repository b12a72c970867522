"""Regenerates the committed fixtures under tests/golden/.

abi_layout_ref.json  sizeof/offsetof of the reference ABI structs, printed by
                     oracle/_ref/ref_layout (oracle/ref_layout.c compiled
                     against /root/reference/include by oracle/Makefile).
philox_kat.json      Random123 Philox4x32-10 known-answer vectors (Salmon et
                     al., SC'11), cross-checked here against PyTorch's
                     independent ATen/core/PhiloxRNGEngine.h when torch's
                     headers are present.
Run from the repo root after `make -C oracle`.
"""
import json
import os
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))


def abi_layout():
    exe = os.path.join(ROOT, "oracle", "_ref", "ref_layout")
    out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    data = json.loads(out)
    with open(os.path.join(HERE, "abi_layout_ref.json"), "w") as f:
        json.dump(data, f, indent=1, sort_keys=True)


KAT = [
    {"ctr": [0, 0, 0, 0], "key": [0, 0], "out": [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]},
    {"ctr": [0xFFFFFFFF] * 4, "key": [0xFFFFFFFF] * 2, "out": [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]},
    {"ctr": [0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], "key": [0xA4093822, 0x299F31D0],
     "out": [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]},
]

TORCH_CHECK = r"""
#include <ATen/core/PhiloxRNGEngine.h>
#include <cstdio>
int main(int argc, char **argv) {
  unsigned long long s = strtoull(argv[1], 0, 16), sub = strtoull(argv[2], 0, 16), off = strtoull(argv[3], 0, 16);
  at::philox_engine e(s, sub, off);
  unsigned a = e(); unsigned b = e(); unsigned c = e(); unsigned d = e();
  printf("%08x %08x %08x %08x\n", a, b, c, d);
}
"""


def philox():
    try:
        import torch
        inc = os.path.join(os.path.dirname(torch.__file__), "include")
    except Exception:
        inc = None
    if inc and os.path.exists(os.path.join(inc, "ATen", "core", "PhiloxRNGEngine.h")):
        with tempfile.TemporaryDirectory() as d:
            src, exe = os.path.join(d, "k.cpp"), os.path.join(d, "k")
            open(src, "w").write(TORCH_CHECK)
            subprocess.run(["g++", "-std=c++17", "-O1", "-I", inc, src, "-o", exe], check=True)
            for v in KAT:
                c, k = v["ctr"], v["key"]
                seed = (k[1] << 32) | k[0]
                sub = (c[3] << 32) | c[2]
                off = (c[1] << 32) | c[0]
                got = subprocess.run([exe, "%x" % seed, "%x" % sub, "%x" % off], check=True, capture_output=True,
                                     text=True).stdout.split()
                assert [int(x, 16) for x in got] == v["out"], (v, got)
        print("philox KATs agree with torch PhiloxRNGEngine.h")
    with open(os.path.join(HERE, "philox_kat.json"), "w") as f:
        json.dump(KAT, f, indent=1)


if __name__ == "__main__":
    abi_layout()
    philox()
    sys.exit(0)
