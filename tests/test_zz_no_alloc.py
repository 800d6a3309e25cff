"""ecf8_decode_noalloc: the decode with the reference kernel's arguments
only (no table, no workspace), its derived table in the library's static
device array.  Checked through the C ABI against ecf8_decode with a table
from ecf8_build_table, and against the original FP8 bytes: two calls in a
row, the second on a smaller block, for automaton and multi-symbol LUTs.
Argument errors are returned before any HIP call (CPU tests)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

KEYS = ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps")


def _noalloc(d, out, n, max_block=0, tpb=512, bpt=8, stream=None, **over):
    from ecf8_amd._lib import lib

    a = {k: (v.data_ptr() if torch.is_tensor(v) else v) for k, v in d.items()}
    a.update(over)
    return lib().ecf8_decode_noalloc(a["luts"], a["encoded"], a["packed_other_4bits"],
                                     a["output_positions"], a["gaps"],
                                     out if isinstance(out, int) else out.data_ptr(),
                                     over.get("n_luts", d["luts"].shape[0]
                                              if torch.is_tensor(d["luts"]) else 3),
                                     over.get("n_bytes", d["encoded"].numel()
                                              if torch.is_tensor(d["encoded"]) else 100),
                                     n, max_block, tpb, bpt, stream)


_FAKE = dict(luts=0x1000, encoded=0x2000, packed_other_4bits=0x3000, output_positions=0x4000,
             gaps=0x5000)


@pytest.mark.parametrize("over,status", [
    (dict(bpt=4), 2),
    (dict(tpb=300), 2),
    (dict(n=63), 1),
    (dict(n_luts=1), 4),
    (dict(n_luts=19), 4),
    (dict(out=0x6001), 3),
    (dict(encoded=0x2008), 3),
    (dict(gaps=0), 1),
    (dict(n_bytes=2**31), 2),
])
def test_noalloc_rejects_before_any_hip_call(over, status):
    over = dict(over)
    n = over.pop("n", 64)
    out = over.pop("out", 0x6000)
    tpb = over.pop("tpb", 512)
    bpt = over.pop("bpt", 8)
    d = dict(_FAKE)
    for k in list(over):
        if k in d:
            d[k] = over.pop(k)
    assert _noalloc(d, out, n, tpb=tpb, bpt=bpt, **over) == status


def _block(seed, n_rows, skewed=False):
    from dfloat.compress import compress_flat
    from ecf8_amd.synth import synthetic_fp8

    if not skewed:
        w, _ = synthetic_fp8(n_rows, 2048, 0.02, seed=seed)
        flat = w.reshape(-1)
    else:  # a dominant exponent: a 1-bit code, the multi-symbol kernel
        rng = np.random.default_rng(seed)
        n = n_rows * 2048
        e = np.where(rng.random(n) < 0.8, 12, rng.integers(0, 16, n)).astype(np.uint8)
        o = rng.integers(0, 16, n, dtype=np.uint8)
        flat = torch.from_numpy(((o & 8) << 4 | e << 3 | (o & 7)).astype(np.uint8)).view(
            torch.float8_e4m3fn)
    return flat, compress_flat(flat)


@pytest.mark.gpu
def test_noalloc_equals_ecf8_decode_on_consecutive_calls(cuda_device):
    from ecf8_amd.decode import build_table, decode_into, largest_block, min_code_bits

    cases = [_block(1, 2048), _block(2, 640), _block(3, 896, skewed=True), _block(4, 128)]
    sizes = [f.numel() for f, _ in cases]
    assert sizes[1] < sizes[0] and sizes[3] < sizes[2]
    pad = 4096
    for i, (flat, res) in enumerate(cases):
        n = flat.numel()
        print(f"noalloc case {i}: {n} elements", flush=True)
        d = {k: res[k].contiguous().to(cuda_device) for k in KEYS}
        cap = largest_block(d["output_positions"])
        ref = torch.full((n + pad,), 0x5A, dtype=torch.uint8, device=cuda_device)
        decode_into(ref, *(d[k] for k in KEYS), table=build_table(d["luts"]), n_elements=n,
                    max_block_elements=cap, min_code_bits=min_code_bits(d["luts"]))
        got = torch.full((n + pad,), 0x5A, dtype=torch.uint8, device=cuda_device)
        stream = torch.cuda.current_stream(cuda_device).cuda_stream
        assert _noalloc(d, got, n, max_block=cap, stream=stream) == 0
        torch.cuda.synchronize()
        g, r = got.cpu(), ref.cpu()
        assert torch.equal(g, r), i
        assert torch.equal(g[:n], flat.view(torch.uint8)), i
        assert (g[n:] == 0x5A).all(), i
