"""bench.py's contract on the CPU: one GPU only, and the decode line's
algorithmic byte count for the Qwen3-8B-shaped layer as its parts (format
geometry: 4 KiB format-blocks, 256 gap bytes each, one u64 position per
block plus one, the LUT stack, half a byte of sign/mantissa per element;
one FP8 byte written per element)."""

from __future__ import annotations

import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


def test_algorithmic_bytes_of_the_qwen3_layer():
    import bench

    n, n_bytes, n_luts = 192_937_984, 62_123_008, 3
    total, reads, writes = bench.algorithmic_bytes(n, n_bytes, n_luts)
    n_fb = 15_167  # 62,123,008 bitstream bytes in 4,096-byte format-blocks, rounded up
    assert (n_fb - 1) * 4096 < n_bytes <= n_fb * 4096
    parts = {"bitstream": n_bytes, "nibbles": 96_468_992, "gaps": 3_882_752,
             "positions": 121_344, "luts": 768}
    assert parts["nibbles"] * 2 == n and parts["gaps"] == n_fb * 256
    assert parts["positions"] == 8 * (n_fb + 1) and parts["luts"] == 256 * n_luts
    assert reads == sum(parts.values()) == 162_596_864
    assert writes == n and total == 355_534_848
