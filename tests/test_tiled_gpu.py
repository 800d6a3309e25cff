"""The tiled execution layout on the GPU (include/ecf8_tile.h), on one
Qwen3-8B-shaped layer (q/k/v/o/gate/up/down, one compressed block):

* ecf8_tile_decode writes each Linear's original FP8 bytes;
* ecf8_tile_linear -- the small-M linear decoding its weight operands on the
  fly -- is bit-identical to ecf8_fp8_linear over the decoded weights, for
  the decode step's four linears (q/k/v fused, o, gate/up fused, down) and
  M = 1, 7, 16, with the same wave count as the FP8 linear;
* it follows a float64 restatement of the block-scaled product (same
  tolerance as the FP8 linear's own test);
* it refuses what it cannot run.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def layer(cuda_device):
    from dfloat.compress import compress_flat
    from ecf8_amd.decode import build_table
    from ecf8_amd.synth import flat_block, qwen3_8b_layer
    from ecf8_amd.tiled import TiledOperand, code_from_luts, tile_encode

    _say("[tiled] encoding a Qwen3-8B layer")
    weights = qwen3_8b_layer(seed=3)
    flat, _ = flat_block(weights)
    res = compress_flat(flat)
    luts = res["luts"].contiguous().to(cuda_device)
    table = build_table(luts)
    assert table.kind == 1
    bits, vals = code_from_luts(res["luts"])
    ops, dense = {}, {}
    for name, (w, s) in weights.items():
        enc = tile_encode(w, bits, vals)
        ops[name] = TiledOperand(enc, s, w.shape[0], w.shape[1], cuda_device)
        dense[name] = (w.to(cuda_device), s.to(cuda_device))
    return ops, dense, table


def test_tile_decode_writes_the_original_bytes(layer):
    from ecf8_amd.tiled import tile_decode

    ops, dense, table = layer
    for name, op in ops.items():
        out = torch.full((op.n * op.k + 64,), 0x5A, dtype=torch.uint8, device=op.device)
        tile_decode(op, table, out[: op.n * op.k])
        torch.cuda.synchronize()
        w = dense[name][0]
        assert torch.equal(out[: op.n * op.k].view(op.n, op.k), w.view(torch.uint8)), name
        assert bool((out[op.n * op.k:] == 0x5A).all()), name


LINEARS = {  # the decode step's four launches and their inputs' width
    "qkv": (["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"], 4096),
    "o": (["self_attn.o_proj"], 4096),
    "gate_up": (["mlp.gate_proj", "mlp.up_proj"], 4096),
    "down": (["mlp.down_proj"], 12288),
}


def _activations(M, K, seed, dev):
    from ecf8_amd.llm_kernels import act_quant

    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(16, K, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    aq = torch.empty(16, K, dtype=FP8, device=dev)
    as_ = torch.empty(16, K // 128, dtype=torch.float32, device=dev)
    act_quant(x, 16, aq, as_)
    return aq, as_


@pytest.mark.parametrize("which", sorted(LINEARS))
@pytest.mark.parametrize("M", [1, 7, 16])
def test_tile_linear_is_bit_identical_to_the_fp8_linear(layer, which, M, cuda_device):
    from ecf8_amd.llm_kernels import LinearPlan
    from ecf8_amd.tiled import TileLinearPlan, linear_waves

    ops, dense, table = layer
    names, K = LINEARS[which]
    aq, as_ = _activations(M, K, 11 + M, cuda_device)
    N = sum(ops[n].n for n in names)
    ref = torch.full((16, N + 8), 7.0, dtype=torch.bfloat16, device=cuda_device)
    got = ref.clone()
    LinearPlan([dense[n] for n in names], ref)(aq, as_, M)
    plan = TileLinearPlan([ops[n] for n in names], table, got)
    assert plan.waves == linear_waves(N, K, cuda_device)
    _say(f"[tiled] {which} M={M} N={N} K={K} waves={plan.waves}")
    plan(aq, as_, M)
    torch.cuda.synchronize()
    assert torch.equal(got, ref), which
    assert bool((got[M:] == 7.0).all()) and bool((got[:, N:] == 7.0).all())


def test_tile_linear_follows_an_fp64_restatement(layer, cuda_device):
    from ecf8_amd.tiled import TileLinearPlan

    ops, dense, table = layer
    M, K = 5, 4096
    aq, as_ = _activations(M, K, 3, cuda_device)
    out = torch.empty(16, 1024, dtype=torch.bfloat16, device=cuda_device)
    TileLinearPlan([ops["self_attn.k_proj"]], table, out)(aq, as_, M)
    w, s = dense["self_attn.k_proj"]
    wd = w.double().cpu() * s.double().cpu().repeat_interleave(128, 0).repeat_interleave(128, 1)
    from ecf8_amd.llm_kernels import from_tiles

    xd = (from_tiles(aq, M, K).double().cpu().view(M, K // 128, 128)
          * as_[:M].double().cpu()[..., None]).view(M, K)
    ref = xd @ wd.T
    got = out[:M].double().cpu()
    assert torch.allclose(got, ref, rtol=2 ** -7, atol=1e-3)


def test_tile_linear_refusals(layer, cuda_device):
    from ecf8_amd._lib import ECF8Error
    from ecf8_amd.tiled import TileLinearPlan

    ops, dense, table = layer
    aq, as_ = _activations(16, 4096, 1, cuda_device)
    out = torch.empty(32, 1024, dtype=torch.bfloat16, device=cuda_device)
    plan = TileLinearPlan([ops["self_attn.k_proj"]], table, out)
    with pytest.raises(ECF8Error):
        plan(aq, as_, 17)  # more than 16 rows
    with pytest.raises(ECF8Error):
        TileLinearPlan([ops["self_attn.k_proj"], ops["mlp.down_proj"]], table, out)  # K differs
    with pytest.raises(ECF8Error):
        TileLinearPlan([ops["self_attn.k_proj"]], table, out[:, :512])  # too few columns


def test_tile_kernels_turn_a_non_automaton_table_into_nans(layer, cuda_device):
    """The tile entry points cannot see on the host what kind of table a
    device-built table is.  Handed a multi-symbol table (a block whose code
    has a 1-bit symbol), the kernels read its kind word with the entries and
    write NaNs over every output they own -- bf16 0x7FC0 from the linear,
    e4m3fn 0x7F from the decode -- and nothing outside it."""
    import ctypes

    from ecf8_amd._lib import lib
    from ecf8_amd.decode import build_table
    from ecf8_amd.tiled import linear_waves

    ops, _dense, _table = layer
    # LUTs of a 1-bit code: exponent 11 for 80 % of the symbols
    from dfloat.compress import compress_flat

    rng = np.random.default_rng(1)
    b = rng.integers(0, 256, 1 << 16, dtype=np.int64).astype(np.uint8)
    hit = rng.random(b.size) < 0.8
    b[hit] = (b[hit] & 0x87) | (11 << 3)
    b[(b & 0x7F) == 0x7F] = 0x7E
    res = compress_flat(torch.from_numpy(b).view(FP8))
    multi = build_table(res["luts"].contiguous().to(cuda_device))
    assert multi.kind == 0
    stream = torch.cuda.current_stream(cuda_device).cuda_stream
    op = ops["self_attn.o_proj"]
    M = 5
    aq, as_ = _activations(M, op.k, 2, cuda_device)
    out = torch.zeros(M + 1, op.n + 128, dtype=torch.bfloat16, device=cuda_device)
    s = op.c_struct(64)
    rc = lib().ecf8_tile_linear(aq.data_ptr(), as_.data_ptr(), M, op.k, ctypes.byref(s), 1,
                                multi.data.data_ptr(), out.data_ptr(), out.shape[1],
                                linear_waves(op.n, op.k, cuda_device), stream)
    assert rc == 0
    got = out.view(torch.int16).cpu()
    assert bool((got[:M, 64:64 + op.n] == 0x7FC0).all())
    assert bool((got[:M, :64] == 0).all()) and bool((got[:M, 64 + op.n:] == 0).all())
    assert bool((got[M] == 0).all())
    dec = torch.zeros(op.n * op.k + 256, dtype=torch.uint8, device=cuda_device)
    s0 = op.c_struct()
    rc = lib().ecf8_tile_decode(ctypes.byref(s0), op.k, multi.data.data_ptr(), dec.data_ptr(),
                                stream)
    assert rc == 0
    d = dec.cpu()
    assert bool((d[: op.n * op.k] == 0x7F).all()) and bool((d[op.n * op.k:] == 0).all())
