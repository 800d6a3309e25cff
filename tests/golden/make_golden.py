"""Write the small golden vectors under tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

Each case is a seeded FP8 block compressed by the pure-Python oracle
(oracle/codec.py, a restatement of dfloat/utils.py:207-499); the .npz holds
the input bytes and every compressed tensor, named as in the reference's
cache files (scripts/compress.py:239-247).  The reference itself ships no
vectors, so these pin regressions of the oracle, the product encoder and the
GPU decoder against one another; the oracle is pinned independently by the
brute-force and closed-form tests in tests/test_oracle_pinning.py.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import codec as oc  # noqa: E402


def _synthetic(rows, cols, sigma, seed):
    import torch

    from ecf8_amd.synth import synthetic_fp8

    w, _ = synthetic_fp8(rows, cols, sigma, seed=seed)
    return w.reshape(-1).view(torch.uint8).numpy().copy()


def _fibonacci_block(seed):
    # exponent counts 1,1,2,3,5,... give a caterpillar tree: with EOF that is
    # 17 leaves, so the longest code is exactly 16 bits, the format's limit
    # (the length limiter of utils.py:251-265 does not fire for 16
    # exponents plus EOF; its test uses a larger alphabet)
    rng = np.random.default_rng(seed)
    counts = [1, 1]
    while len(counts) < 16:
        counts.append(counts[-1] + counts[-2])
    exps = np.concatenate([np.full(c, s, np.uint8) for s, c in enumerate(counts)])
    rng.shuffle(exps)
    if exps.size % 2:
        exps = np.concatenate([exps, np.array([15], np.uint8)])
    other = rng.integers(0, 16, exps.size, dtype=np.uint8)
    return (((other & 8) << 4) | (exps << 3) | (other & 7)).astype(np.uint8)


def cases():
    rng = np.random.default_rng(1234)
    yield "synth_128x256", _synthetic(128, 256, 0.02, seed=7), 512
    yield "synth_128x256_tpb128", _synthetic(128, 256, 0.02, seed=8), 128
    yield "single_exponent", np.full(8192, 0x6A, np.uint8), 512
    yield "uniform_exponents", rng.integers(0, 256, 20000, dtype=np.uint8), 512
    yield "fibonacci_long_codes", _fibonacci_block(5), 512
    yield "two_elements", np.array([0x38, 0xC1], np.uint8), 512


def main():
    index = {}
    for name, flat, tpb in cases():
        res = oc.compress_block(flat, bytes_per_thread=8, threads_per_block=tpb)
        table = {("_EOF" if isinstance(k, oc.EndOfFile) else str(int(k))): list(v)
                 for k, v in res["table"].items()}
        np.savez_compressed(
            os.path.join(HERE, f"{name}.npz"),
            flat=flat,
            luts=res["luts"],
            encoded=res["encoded"],
            packed_other_4bits=res["packed_other_4bits"],
            output_positions=res["output_positions"].view(np.uint8),
            gaps=res["gaps"],
            threads_per_block=np.array(tpb),
        )
        index[name] = {"threads_per_block": tpb, "n_elements": int(flat.size),
                       "n_bytes": int(res["encoded"].size), "table": table}
    with open(os.path.join(HERE, "index.json"), "w") as f:
        json.dump(index, f, indent=1)


if __name__ == "__main__":
    main()
