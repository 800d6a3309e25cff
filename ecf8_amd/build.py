"""Compile libecf8.so (HIP kernels for gfx950 + host codec) in-tree.

Run ``python -m ecf8_amd.build``.  The library is built with hipcc directly
(no JIT cache) so the shared object travels with the source tree.
"""

from __future__ import annotations

import os
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libecf8.so")
SOURCES = [os.path.join(HERE, "csrc", f)
           for f in ("ecf8_decode.hip", "ecf8_table_kernel.hip", "ecf8_llm.hip", "ecf8_tile.hip",
                     "ecf8_stream.hip",
                     "ecf8_tables.cpp", "ecf8_host.cpp", "ecf8_tile_host.cpp")]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # the HIP runtime torch ships accepts code object v5
    "-mcode-object-version=5",
    # never emit packed-FP32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-I" + os.path.join(REPO, "include"),
]


def build(verbose: bool = False) -> str:
    """Compile every source into ecf8_amd/libecf8.so (atomically replaced)."""
    fd, tmp = tempfile.mkstemp(prefix=".libecf8.", suffix=".so.tmp", dir=HERE)
    os.close(fd)
    cmd = [HIPCC, *FLAGS, "-o", tmp, *SOURCES]
    try:
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + res.stdout + res.stderr)
        if verbose:
            print(" ".join(cmd))
        os.replace(tmp, LIB_PATH)
    finally:
        if os.path.exists(tmp):
            os.unlink(tmp)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
