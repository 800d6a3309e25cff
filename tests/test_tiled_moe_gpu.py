"""The tiled execution layout's grouped expert linear on the GPU
(include/ecf8_tile.h: ecf8_tile_moe_linear, ecf8_tile_decode_batch), on
Qwen3-30B-A3B-shaped experts (hidden 2048, intermediate 768), each expert
compressed as its own block and re-tiled under its own code:

* ecf8_tile_decode_batch writes every expert's original FP8 bytes;
* ecf8_tile_moe_linear -- routed experts decoding their weight operands on
  the fly -- is bit-identical to ecf8_moe_linear over the decoded experts,
  for gate/up (token rows gathered, 4 waves of 4 groups) and down (one row
  per sorted pair: 3 waves of 2 groups at K = 768, 4 at K = 1024), 1, 5
  and 16 routed tokens, any workgroup split;
  eight waves at K = 4096, with three operands per expert;
* a re-tiled small MoE model generates the FP8 model's tokens and logits,
  eager and graph-replayed;
* it refuses what it cannot run.
"""

from __future__ import annotations

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

E, H, I, TOP_K = 16, 2048, 768, 8


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def experts(cuda_device):
    from dfloat.compress import compress_flat
    from ecf8_amd.decode import build_table
    from ecf8_amd.synth import flat_block, synthetic_block
    from ecf8_amd.tiled import TiledOperand, code_from_luts, tile_encode

    shapes = {"gate_proj": (I, H, 0.02), "up_proj": (I, H, 0.02), "down_proj": (H, I, 0.02)}
    dense, ops, tables = [], [], []
    _say(f"[tiled-moe] encoding {E} experts")
    for e in range(E):
        w = synthetic_block(shapes, seed=500 + e)
        flat, _ = flat_block(w)
        res = compress_flat(flat)
        table = build_table(res["luts"].contiguous().to(cuda_device))
        assert table.kind == 1
        bits, vals = code_from_luts(res["luts"])
        ops.append({n: TiledOperand(tile_encode(wt, bits, vals), s, wt.shape[0], wt.shape[1],
                                    cuda_device) for n, (wt, s) in w.items()})
        dense.append({n: (wt.to(cuda_device), s.to(cuda_device)) for n, (wt, s) in w.items()})
        tables.append(table)
    return dense, ops, tables


def test_tile_decode_batch_writes_the_original_bytes(experts, cuda_device):
    from ecf8_amd.tiled import TileDecodeBatch

    dense, ops, tables = experts
    for name in ("gate_proj", "down_proj"):
        n, k = ops[0][name].n, ops[0][name].k
        buf = torch.full((E, n * k + 64), 0x5A, dtype=torch.uint8, device=cuda_device)
        TileDecodeBatch([o[name] for o in ops], tables, [buf[e, :n * k] for e in range(E)])()
        torch.cuda.synchronize()
        for e in range(E):
            assert torch.equal(buf[e, :n * k].view(n, k), dense[e][name][0].view(torch.uint8)), \
                (name, e)
        assert bool((buf[:, n * k:] == 0x5A).all())


def _routing(M, seed, dev):
    """Router state for M tokens with top-k distinct random experts, grouped
    by ecf8_moe_group."""
    from ecf8_amd import llm_kernels as K

    g = torch.Generator().manual_seed(seed)
    r = K.MoeRouting(16, TOP_K, E, dev)
    idx = torch.stack([torch.randperm(E, generator=g)[:TOP_K] for _ in range(M)])
    r.topk_idx[:M] = idx.to(torch.int32).to(dev)
    r.topk_w[:M] = torch.rand(M, TOP_K, generator=g).to(dev)
    K.moe_group(r, M)
    return r


def _acts(rows, K, seed, dev):
    from ecf8_amd.llm_kernels import act_quant

    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(rows, K, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    aq = torch.empty((rows + 15) // 16 * 16, K, dtype=torch.float8_e4m3fn, device=dev)  # tiles
    as_ = torch.empty(rows, K // 128, dtype=torch.float32, device=dev)
    act_quant(x, rows, aq, as_)
    return aq, as_


@pytest.mark.parametrize("splits", [0, 1, 5])
@pytest.mark.parametrize("M", [1, 5, 16])
@pytest.mark.parametrize("which", ["gate_up", "down"])
def test_tile_moe_linear_is_bit_identical_to_the_fp8_grouped_linear(experts, cuda_device, which,
                                                                       M, splits):
    from ecf8_amd.llm_kernels import MoeLinearPlan
    from ecf8_amd.tiled import TileMoePlan

    dense, ops, tables = experts
    names = ["gate_proj", "up_proj"] if which == "gate_up" else ["down_proj"]
    gather = which == "gate_up"
    K = H if gather else I
    N = sum(ops[0][n].n for n in names)
    r = _routing(M, 7 + M, cuda_device)
    P = 16 * TOP_K
    aq, as_ = _acts(16 if gather else P, K, 3 + M, cuda_device)
    ref = torch.full((P, N + 8), 7.0, dtype=torch.bfloat16, device=cuda_device)
    got = ref.clone()
    MoeLinearPlan([[dense[e][n] for n in names] for e in range(E)], ref)(aq, as_, r, gather, M=M)
    plan = TileMoePlan([[ops[e][n] for n in names] for e in range(E)], tables, got, splits=splits)
    _say(f"[tiled-moe] {which} M={M} splits={splits}")
    plan(aq, as_, r, gather, M=M)
    torch.cuda.synchronize()
    rows = M * TOP_K
    assert torch.equal(got[:rows], ref[:rows]), which
    assert bool((got[rows:] == 7.0).all()) and bool((got[:, N:] == 7.0).all())
    assert len(set(got[:rows].float().reshape(-1).tolist())) > 100


@pytest.mark.parametrize("spread", ["all", "random", "same"])
@pytest.mark.parametrize("which", ["gate_up", "down"])
def test_many_routed_experts_share_the_resident_grid(experts, cuda_device, which, spread):
    """128 expert slots (the 16 experts' operands, each reused 8 times):
    16 tokens routed to 128 distinct experts (the most a decode step can
    route: four workgroups per expert on the resident grid), to a random
    ~90 (five), or all to the same top-k (8 experts, each holding a full
    16-row tile, their split capped at one panel per group): still
    bit-identical to the FP8 grouped linear."""
    from ecf8_amd import llm_kernels as K
    from ecf8_amd.llm_kernels import MoeLinearPlan
    from ecf8_amd.tiled import TileMoePlan

    dense, ops, tables = experts
    n_slots = 128
    names = ["gate_proj", "up_proj"] if which == "gate_up" else ["down_proj"]
    gather = which == "gate_up"
    Kd = H if gather else I
    N = sum(ops[0][n].n for n in names)
    M = 16
    r = K.MoeRouting(16, TOP_K, n_slots, cuda_device)
    if spread == "all":
        idx = torch.arange(M * TOP_K).view(M, TOP_K)
    elif spread == "same":
        g = torch.Generator().manual_seed(78)
        pick = torch.randperm(n_slots, generator=g)[:TOP_K]
        idx = torch.stack([pick[torch.randperm(TOP_K, generator=g)] for _ in range(M)])
    else:
        g = torch.Generator().manual_seed(77)
        idx = torch.stack([torch.randperm(n_slots, generator=g)[:TOP_K] for _ in range(M)])
    r.topk_idx[:M] = idx.to(torch.int32).to(cuda_device)
    r.topk_w[:M] = torch.rand(M, TOP_K, generator=torch.Generator().manual_seed(5)).to(cuda_device)
    K.moe_group(r, M)
    n_active = int(r.n_active.item())
    if spread == "all":
        assert n_active == 128
    elif spread == "same":
        assert n_active == TOP_K
    else:
        assert 80 <= n_active < 128
    P = 16 * TOP_K
    aq, as_ = _acts(16 if gather else P, Kd, 9, cuda_device)
    ref = torch.full((P, N + 8), 7.0, dtype=torch.bfloat16, device=cuda_device)
    got = ref.clone()
    MoeLinearPlan([[dense[e % E][n] for n in names] for e in range(n_slots)], ref)(
        aq, as_, r, gather, M=M)
    _say(f"[tiled-moe] {which}: {n_active} of {n_slots} experts routed")
    TileMoePlan([[ops[e % E][n] for n in names] for e in range(n_slots)],
                [tables[e % E] for e in range(n_slots)], got)(aq, as_, r, gather, M=M)
    torch.cuda.synchronize()
    rows = M * TOP_K
    assert torch.equal(got[:rows], ref[:rows])
    assert bool((got[:, N:] == 7.0).all())
    assert len(set(got[:rows].float().reshape(-1).tolist())) > 100


@pytest.fixture(scope="module")
def wide_experts(cuda_device):
    """Eight experts of intermediate 1024: the down projection's K = 1024
    gives the FP8 grouped linear four waves of two groups each (K = 768's
    six groups take three waves)."""
    from dfloat.compress import compress_flat
    from ecf8_amd.decode import build_table
    from ecf8_amd.synth import flat_block, synthetic_block
    from ecf8_amd.tiled import TiledOperand, code_from_luts, tile_encode

    inter = 1024
    dense, ops, tables = [], [], []
    for e in range(8):
        w = synthetic_block({"down_proj": (H, inter, 0.02)}, seed=700 + e)
        res = compress_flat(flat_block(w)[0])
        tables.append(build_table(res["luts"].contiguous().to(cuda_device)))
        bits, vals = code_from_luts(res["luts"])
        wt, sc = w["down_proj"]
        ops.append(TiledOperand(tile_encode(wt, bits, vals), sc, wt.shape[0], wt.shape[1],
                                cuda_device))
        dense.append((wt.to(cuda_device), sc.to(cuda_device)))
    return dense, ops, tables, inter


@pytest.mark.parametrize("M", [1, 16])
def test_four_wave_down_projection_is_bit_identical(wide_experts, cuda_device, M):
    from ecf8_amd import llm_kernels as K
    from ecf8_amd.llm_kernels import MoeLinearPlan
    from ecf8_amd.tiled import TileMoePlan

    dense, ops, tables, inter = wide_experts
    n_exp, top_k = len(ops), 4
    g = torch.Generator().manual_seed(90 + M)
    r = K.MoeRouting(16, top_k, n_exp, cuda_device)
    r.topk_idx[:M] = torch.stack([torch.randperm(n_exp, generator=g)[:top_k]
                                  for _ in range(M)]).to(torch.int32).to(cuda_device)
    r.topk_w[:M] = torch.rand(M, top_k, generator=g).to(cuda_device)
    K.moe_group(r, M)
    P = 16 * top_k
    aq, as_ = _acts(P, inter, 40 + M, cuda_device)
    ref = torch.full((P, H + 8), 7.0, dtype=torch.bfloat16, device=cuda_device)
    got = ref.clone()
    MoeLinearPlan([[d] for d in dense], ref)(aq, as_, r, False, M=M)
    _say(f"[tiled-moe] four-wave down K={inter} M={M}")
    TileMoePlan([[o] for o in ops], tables, got)(aq, as_, r, False, M=M)
    torch.cuda.synchronize()
    rows = M * top_k
    assert torch.equal(got[:rows], ref[:rows])
    assert bool((got[rows:] == 7.0).all()) and bool((got[:, H:] == 7.0).all())
    assert len(set(got[:rows].float().reshape(-1).tolist())) > 100


@pytest.fixture(scope="module")
def deep_experts(cuda_device):
    """Six experts of three [256, 4096] operands each: K = 4096 gives the
    FP8 grouped linear eight waves, and three operands deal the workgroups
    to three runs."""
    from dfloat.compress import compress_flat
    from ecf8_amd.decode import build_table
    from ecf8_amd.synth import flat_block, synthetic_block
    from ecf8_amd.tiled import TiledOperand, code_from_luts, tile_encode

    names = ("a_proj", "b_proj", "c_proj")
    dense, ops, tables = [], [], []
    for e in range(6):
        w = synthetic_block({n: (256, 4096, 0.02) for n in names}, seed=800 + e)
        res = compress_flat(flat_block(w)[0])
        tables.append(build_table(res["luts"].contiguous().to(cuda_device)))
        bits, vals = code_from_luts(res["luts"])
        ops.append([TiledOperand(tile_encode(w[n][0], bits, vals), w[n][1], 256, 4096,
                                 cuda_device) for n in names])
        dense.append([(w[n][0].to(cuda_device), w[n][1].to(cuda_device)) for n in names])
    return dense, ops, tables


@pytest.mark.parametrize("splits", [0, 1, 4])
@pytest.mark.parametrize("M", [1, 16])
def test_eight_wave_three_operand_grouped_linear_is_bit_identical(deep_experts, cuda_device, M,
                                                                 splits):
    from ecf8_amd import llm_kernels as K
    from ecf8_amd.llm_kernels import MoeLinearPlan
    from ecf8_amd.tiled import TileMoePlan

    dense, ops, tables = deep_experts
    n_exp, top_k, N = len(ops), 2, 3 * 256
    g = torch.Generator().manual_seed(120 + M)
    r = K.MoeRouting(16, top_k, n_exp, cuda_device)
    r.topk_idx[:M] = torch.stack([torch.randperm(n_exp, generator=g)[:top_k]
                                  for _ in range(M)]).to(torch.int32).to(cuda_device)
    r.topk_w[:M] = torch.rand(M, top_k, generator=g).to(cuda_device)
    K.moe_group(r, M)
    aq, as_ = _acts(16, 4096, 60 + M, cuda_device)
    P = 16 * top_k
    ref = torch.full((P, N + 8), 7.0, dtype=torch.bfloat16, device=cuda_device)
    got = ref.clone()
    MoeLinearPlan(dense, ref)(aq, as_, r, True, M=M)
    _say(f"[tiled-moe] eight-wave three-operand K=4096 M={M} splits={splits}")
    TileMoePlan(ops, tables, got, splits=splits)(aq, as_, r, True, M=M)
    torch.cuda.synchronize()
    rows = M * top_k
    assert torch.equal(got[:rows], ref[:rows])
    assert bool((got[rows:] == 7.0).all()) and bool((got[:, N:] == 7.0).all())
    assert len(set(got[:rows].float().reshape(-1).tolist())) > 100


def test_tile_moe_linear_refusals(experts, cuda_device):
    from ecf8_amd._lib import ECF8Error
    from ecf8_amd import llm_kernels as K
    from ecf8_amd.tiled import TileMoePlan

    dense, ops, tables = experts
    out = torch.empty(32 * TOP_K, 2 * I, dtype=torch.bfloat16, device=cuda_device)
    plan = TileMoePlan([[o["gate_proj"], o["up_proj"]] for o in ops], tables, out)
    r = K.MoeRouting(32, TOP_K, E, cuda_device)
    aq, as_ = _acts(32, H, 1, cuda_device)
    with pytest.raises(ECF8Error):
        plan(aq, as_, r, True, M=17)  # more than 16 routed tokens
    with pytest.raises(ECF8Error):
        TileMoePlan([[o["gate_proj"], o["down_proj"]] for o in ops], tables, out)  # shapes differ
    with pytest.raises(ECF8Error):
        TileMoePlan([[o["gate_proj"]] for o in ops], tables[:-1], out)  # a table missing


SMALL_MOE = dict(hidden=2048, layers=2, heads=16, kv_heads=2, experts=16, top_k=4,
                 moe_intermediate=256, vocab=1024)


def test_retiled_moe_model_matches_fp8_exactly(cuda_device):
    """Attention blocks and experts re-tiled: the decode step's attention
    linears and grouped expert linears decode their weight operands
    themselves, the prompt decodes the tiled Linears first; eager and
    graph-replayed, the FP8 model's tokens and logits."""
    from dfloat.run.run import TensorManager
    from ecf8_amd.moe import (Qwen3MoeConfig, Qwen3MoeRunner, compress_moe_layers,
                              random_moe_model, retile_moe_layers)

    cfg = Qwen3MoeConfig(**SMALL_MOE)
    plain, drawn = random_moe_model(cfg, cuda_device, seed=4)
    tiled_model, _ = random_moe_model(cfg, cuda_device, seed=4)
    compress_moe_layers(tiled_model, drawn)
    retile_moe_layers(tiled_model, drawn)
    assert not hasattr(tiled_model.model.layers[0].mlp.experts[0], "encoded")
    B, T, new = 4, 40, 6
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(5))
    results = {}
    for name, model in (("fp8", plain), ("fused", tiled_model)):
        for graph in (False, True):
            _say(f"[tiled-moe] e2e {name} graph={graph}")
            TensorManager.clear_device()
            r = Qwen3MoeRunner(model, B, T, T + new, cuda_device,
                               prefill_chunk=512 if graph else 16)
            if graph:
                r.capture()
            for rep in range(2):
                toks = r.generate(prompt, new).cpu()
                results[(name, graph, rep)] = (toks, r.logits.float().cpu())
            del r
    base_t, base_l = results[("fp8", False, 0)]
    for key, (t, l) in results.items():
        assert torch.equal(t, base_t), key
        assert torch.equal(l, base_l), key
    assert len(set(base_t.reshape(-1).tolist())) > 1
