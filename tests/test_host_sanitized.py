"""The host codec of libecf8 under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU): ``tests/asan/host_fuzz.cpp`` is built with
g++ together with the library's host sources (format validator, host table
builder, code recovery, bitstream and tiled encoders) and run on real
compressed blocks, which it then corrupts -- LUT bytes and row counts,
output positions, sizes, code tables, exponents and output capacities.
The reference validates nothing before its launch
(dfloat/run/run.py:362-364), so these entry points are the ones that parse
untrusted checkpoint contents."""

from __future__ import annotations

import os
import shutil
import struct
import subprocess

import numpy as np
import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "ecf8_amd", "csrc")
SOURCES = [os.path.join(REPO, "tests", "asan", "host_fuzz.cpp")] + [
    os.path.join(CSRC, f) for f in ("ecf8_host.cpp", "ecf8_tables.cpp", "ecf8_tile_host.cpp")]


def _blocks():
    """Compressed [rows, cols] weights: the synthetic scheme, a skewed
    histogram (1-bit code), long codes, and few symbols."""
    from dfloat.compress import compress_flat
    from ecf8_amd.synth import synthetic_fp8

    rng = np.random.default_rng(7)
    out = []
    w, _ = synthetic_fp8(128, 1024, 0.02, seed=3)
    out.append(w.view(torch.uint8).numpy())
    b = w.view(torch.uint8).numpy().copy()
    hit = rng.random(b.shape) < 0.8
    b[hit] = (b[hit] & 0x87) | (11 << 3)
    out.append(b)
    e = np.minimum(rng.geometric(0.45, b.shape) - 1, 14).astype(np.uint8)  # long codes
    out.append(((rng.integers(0, 16, b.shape, dtype=np.uint8) & 0x87) | (e << 3)).astype(np.uint8))
    out.append(((rng.integers(0, 16, (16, 128), dtype=np.uint8) & 0x87) | (12 << 3)).astype(np.uint8))
    recs = []
    for wb in out:
        rows, cols = wb.shape
        flat = torch.from_numpy(np.ascontiguousarray(wb).reshape(-1))
        res = compress_flat(flat.view(torch.float8_e4m3fn))
        luts = res["luts"].numpy()
        op = res["output_positions"].numpy().view(np.uint64)
        exps = (flat.numpy() >> 3) & 0xF
        recs.append(struct.pack("<iqqqqii", luts.shape[0], res["encoded"].numel(), flat.numel(),
                                op.size, res["gaps"].numel(), rows, cols)
                    + luts.tobytes() + res["encoded"].numpy().tobytes()
                    + res["packed_other_4bits"].numpy().tobytes() + op.tobytes()
                    + res["gaps"].numpy().tobytes() + exps.astype(np.uint8).tobytes()
                    + flat.numpy().tobytes())
    return b"".join(recs)


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not installed")
def test_host_codec_is_clean_under_address_and_ub_sanitizers(tmp_path):
    exe = str(tmp_path / "host_fuzz")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-I" + os.path.join(REPO, "include"), "-I" + CSRC, *SOURCES, "-o", exe, "-lpthread"]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-3000:]
    data = tmp_path / "blocks.bin"
    data.write_bytes(_blocks())
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=23",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    run = subprocess.run([exe, str(data)], capture_output=True, text=True, env=env, timeout=600)
    assert run.returncode == 0, (run.stdout + run.stderr)[-4000:]
    assert "blocks 4 failures 0" in run.stdout
