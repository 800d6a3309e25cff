"""The configurations at their stated size, on the GPU.

* Qwen3-30B-A3B-shaped MoE layer: the attention block and all 128 expert
  blocks decoded by ONE batched launch, bit-exact, nothing written past any
  block; then through the device-side selection with a top-8 routing of 16
  tokens (selected blocks bit-exact, the others untouched).
* Qwen3-30B-A3B-shaped model (48 layers x 128 experts, 6,192 compressed
  blocks): batch-16 greedy generate from 128-token prompts gives the FP8
  model's tokens and logits with routed batched expert decode, side-stream
  attention decode and fused (re-tiled) decode-step linears, eager and
  graph-replayed.
* Qwen3-8B-shaped model (36 layers, hidden 4096, vocab 151,936): every
  layer's forward-pre-hook injects bit-exact weights, and a batch-16 greedy
  generate from 128-token prompts gives the FP8 model's tokens and logits,
  eager and graph-replayed, with the decode in the hook, on the side
  stream, and fused into the decode step's linears (re-tiled layers).
* FLUX.1-dev-shaped DiT (19 double + 38 single blocks, hidden 3072): every
  block injects bit-exact weights, and one denoising step at 4096 image +
  512 text tokens gives the FP8 pipeline's latents.

Weights are synthetic (N(0, sigma) block-quantized per 128x128 tile); two
distinct layers (blocks) are drawn and every layer holds its own device
copy of one of them, which bounds the CPU setup time while the device
memory and traffic are those of the full model.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

KEYS = ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps")
SENTINEL = 0x3C
PAD = 256


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


# ------------------------------------------------------------- MoE layer


@pytest.fixture(scope="module")
def moe_layer(cuda_device):
    from dfloat.compress import compress_flat
    from ecf8_amd.decode import build_table
    from ecf8_amd.synth import QWEN3_MOE_ATTN, QWEN3_MOE_EXPERT, flat_block, synthetic_block

    _say("[full] MoE layer: compressing 129 blocks")
    flats = [flat_block(synthetic_block(QWEN3_MOE_ATTN, 0))[0]]
    flats += [flat_block(synthetic_block(QWEN3_MOE_EXPERT, 1 + e))[0] for e in range(128)]
    blocks, tables, bufs = [], [], []
    for f in flats:
        c = compress_flat(f)
        b = {k: c[k].contiguous().to(cuda_device) for k in KEYS}
        blocks.append(b)
        tables.append(build_table(b["luts"]))
        bufs.append(torch.full((f.numel() + PAD,), SENTINEL, dtype=torch.uint8, device=cuda_device))
    assert sum(f.numel() for f in flats) == 622_854_144
    return flats, blocks, tables, bufs


def _check(flats, bufs, selected=None):
    for i, (f, buf) in enumerate(zip(flats, bufs)):
        n = f.numel()
        want = f.view(torch.uint8).to(buf.device)
        if selected is None or selected[i]:
            assert torch.equal(buf[:n], want), f"block {i}"
        else:
            assert bool((buf[:n] == SENTINEL).all()), f"unselected block {i} was written"
        assert bool((buf[n:] == SENTINEL).all()), f"block {i} wrote past its end"


def test_moe_layer_decodes_in_one_batched_launch(moe_layer):
    from ecf8_amd.decode import decode_batched, prepare_batch

    flats, blocks, tables, bufs = moe_layer
    plan = prepare_batch(blocks, [b[: f.numel()] for b, f in zip(bufs, flats)], tables)
    assert plan.count == 129 and not plan.singles
    _say(f"[full] MoE layer: one launch, {plan.n_tasks} tasks")
    decode_batched(plan)
    torch.cuda.synchronize()
    _check(flats, bufs)


def test_moe_layer_routed_selection(moe_layer, cuda_device):
    from ecf8_amd.decode import BatchSelect, prepare_batch

    flats, blocks, tables, bufs = moe_layer
    plan = prepare_batch(blocks, [b[: f.numel()] for b, f in zip(bufs, flats)], tables)
    sel = BatchSelect(plan)
    g = torch.Generator().manual_seed(5)
    for rep in range(2):
        picked = torch.stack([torch.randperm(128, generator=g)[:8] for _ in range(16)]).unique()
        flags = torch.zeros(129, dtype=torch.int32)
        flags[0] = 1
        flags[1 + picked] = 1
        _say(f"[full] MoE layer: routed selection of {int(flags.sum()) - 1} experts")
        for b in bufs:
            b.fill_(SENTINEL)
        sel(flags.to(cuda_device))
        torch.cuda.synchronize()
        _check(flats, bufs, flags.tolist())


# --------------------------------------------------------- Qwen3-8B model


def test_qwen3_8b_model_bs16_matches_fp8(cuda_device):
    from dfloat.run.run import TensorManager
    from ecf8_amd.llm import Qwen3Config, Qwen3Runner, compress_layers, random_model, retile_layers
    from ecf8_amd.prefetch import LayerPrefetcher

    cfg = Qwen3Config()
    assert (cfg.layers, cfg.hidden, cfg.intermediate, cfg.vocab) == (36, 4096, 12288, 151936)
    _say("[full] Qwen3-8B: building")
    model, drawn = random_model(cfg, cuda_device, distinct_layers=2, seed=0)
    B, T, new = 16, 128, 4
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(1))
    results = {}

    def run(tag, graph):
        _say(f"[full] Qwen3-8B: {tag} graph={graph}")
        TensorManager.clear_device()
        r = Qwen3Runner(model, B, T, T + new, cuda_device)
        if graph:
            r.capture()
        toks = r.generate(prompt, new).cpu()
        results[(tag, graph)] = (toks, r.logits.float().cpu())
        del r
        torch.cuda.empty_cache()

    run("fp8", False)
    from ecf8_amd.llm import tile_resident_weights

    assert tile_resident_weights(model) == 7 * cfg.layers  # FP8 weights re-laid out in tiles
    run("fp8", True)
    _say("[full] Qwen3-8B: compressing")
    compress_layers(model, drawn)
    # every layer's hook injects its original weights
    for i, layer in enumerate(model.model.layers):
        for hook in layer._forward_pre_hooks.values():
            hook(layer, None)
        for name, (w, _) in drawn[i % len(drawn)].items():
            got = layer.get_submodule(name).weight.view(torch.uint8)
            assert torch.equal(got, w.view(torch.uint8).to(cuda_device)), (i, name)
    for graph in (False, True):
        run("ecf8", graph)
    pf = LayerPrefetcher(model.model.layers, cuda_device).install()
    run("ecf8_prefetch", True)
    pf.uninstall()
    _say("[full] Qwen3-8B: re-tiling")
    retile_layers(model, drawn)
    for graph in (False, True):
        run("ecf8_fused", graph)
    base_t, base_l = results[("fp8", False)]
    assert len(set(base_t.reshape(-1).tolist())) > 1
    for key, (t, l) in results.items():
        assert torch.equal(t, base_t), key
        assert torch.equal(l, base_l), key


# ----------------------------------------------------- Qwen3-30B-A3B model


def test_qwen3_moe_model_bs16_matches_fp8(cuda_device):
    """The 48-layer, 128-expert model (6,192 compressed blocks): batch 16,
    128-token prompts, greedy decode; the FP8 model's tokens and logits with
    the attention blocks decoded by their hooks and the routed experts by
    one batched launch per layer (eager and graph-replayed), with the next
    attention block on a side stream, and re-tiled (fused decode-step
    linears, eager and graph-replayed)."""
    from dfloat.run.run import TensorManager
    from ecf8_amd.moe import Qwen3MoeConfig, Qwen3MoeRunner, compress_moe_layers, \
        random_moe_model, retile_moe_layers
    from ecf8_amd.prefetch import LayerPrefetcher

    cfg = Qwen3MoeConfig()
    assert (cfg.layers, cfg.hidden, cfg.experts, cfg.top_k, cfg.moe_intermediate) == \
        (48, 2048, 128, 8, 768)
    _say("[full] Qwen3-30B-A3B: building")
    model, drawn = random_moe_model(cfg, cuda_device, distinct_layers=2, seed=0)
    B, T, new = 16, 128, 4
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(2))
    results = {}

    def run(tag, graph):
        _say(f"[full] Qwen3-30B-A3B: {tag} graph={graph}")
        TensorManager.clear_device()
        r = Qwen3MoeRunner(model, B, T, T + new, cuda_device)
        if graph:
            r.capture()
        toks = r.generate(prompt, new).cpu()
        results[(tag, graph)] = (toks, r.logits.float().cpu())
        del r
        torch.cuda.empty_cache()

    run("fp8", False)
    from ecf8_amd.llm import tile_resident_weights

    assert tile_resident_weights(model) == cfg.layers * (4 + 3 * cfg.experts)
    run("fp8", True)
    _say("[full] Qwen3-30B-A3B: compressing 6,192 blocks")
    compress_moe_layers(model, drawn)
    n_blocks = sum(1 for m in model.modules() if "encoded" in m._buffers)
    assert n_blocks == cfg.layers * (cfg.experts + 1)
    # spot-check injected weights: every expert of the first and last layer
    for i in (0, cfg.layers - 1):
        for e, ex in enumerate(model.model.layers[i].mlp.experts):
            for hook in ex._forward_pre_hooks.values():
                hook(ex, None)
            for name, (w, _) in drawn[i % len(drawn)]["experts"][e].items():
                got = ex.get_submodule(name).weight.view(torch.uint8)
                assert torch.equal(got, w.view(torch.uint8).to(cuda_device)), (i, e, name)
    for graph in (False, True):
        run("ecf8", graph)
    pf = LayerPrefetcher([layer.self_attn for layer in model.model.layers], cuda_device).install()
    run("ecf8_prefetch", True)
    pf.uninstall()
    TensorManager.clear_device()
    torch.cuda.empty_cache()
    _say("[full] Qwen3-30B-A3B: re-tiling")
    retile_moe_layers(model, drawn)
    for graph in (False, True):
        run("ecf8_fused", graph)
    base_t, base_l = results[("fp8", False)]
    assert len(set(base_t.reshape(-1).tolist())) > 1
    for key, (t, l) in results.items():
        assert torch.equal(t, base_t), key
        assert torch.equal(l, base_l), key


# -------------------------------------------------------------- FLUX DiT


def test_flux_dit_full_size_matches_fp8(cuda_device):
    from dfloat.run.run import TensorManager
    from ecf8_amd.dit import FluxConfig, compress_blocks, generate, random_pipeline

    cfg = FluxConfig()
    assert (cfg.double, cfg.single, cfg.hidden) == (19, 38, 3072)
    _say("[full] FLUX DiT: building")
    pipe, drawn = random_pipeline(cfg, cuda_device, distinct=2, seed=0)
    g = torch.Generator().manual_seed(11)
    lat = torch.randn(1, 4096, cfg.in_channels, generator=g).to(torch.bfloat16).to(cuda_device)
    txt = torch.randn(1, 512, cfg.txt_dim, generator=g).to(torch.bfloat16).to(cuda_device)
    pooled = torch.randn(1, cfg.pooled_dim, generator=g).to(torch.bfloat16).to(cuda_device)
    with torch.no_grad():
        _say("[full] FLUX DiT: FP8 step")
        ref = generate(pipe, lat, txt, pooled, steps=1)
        ref2 = generate(pipe, lat, txt, pooled, steps=1)
        torch.cuda.synchronize()
        assert torch.equal(ref.view(torch.int16), ref2.view(torch.int16)), "FP8 step not repeatable"
        _say("[full] FLUX DiT: compressing")
        compress_blocks(pipe, drawn)
        TensorManager.clear_device()
        for blocks, dr in ((pipe.dit.blocks, drawn[0]), (pipe.dit.single_blocks, drawn[1])):
            for i, blk in enumerate(blocks):
                for hook in blk._forward_pre_hooks.values():
                    hook(blk, None)
                for name, (w, _) in dr[i % len(dr)].items():
                    got = blk.get_submodule(name).weight.view(torch.uint8)
                    assert torch.equal(got, w.view(torch.uint8).to(cuda_device)), (i, name)
        _say("[full] FLUX DiT: ECF8 step")
        out = generate(pipe, lat, txt, pooled, steps=1)
        torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert bool(torch.isfinite(out.float()).all())
