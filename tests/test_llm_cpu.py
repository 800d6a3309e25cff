"""Host-side wiring of the end-to-end model (ecf8_amd/llm.py), on the CPU:
layers are compressed and registered as the reference's loader registers
them (dfloat/run/run.py:406-458), and every stored block decodes (oracle)
to the layer's original FP8 weights in the reference's sorted order."""

from __future__ import annotations

import numpy as np
import torch

from oracle import codec as oc

TINY = dict(hidden=512, intermediate=1024, layers=3, heads=4, kv_heads=1, vocab=256)


def test_compressed_layers_hold_the_original_weights():
    from ecf8_amd.llm import LINEAR_NAMES, Qwen3Config, compress_layers, random_model

    cfg = Qwen3Config(**TINY)
    model, drawn = random_model(cfg, "cpu", distinct_layers=2, seed=3)
    originals = [{n: layer.get_submodule(n).weight.detach().view(torch.uint8).clone()
                  for n in LINEAR_NAMES} for layer in model.model.layers]
    # layer 2 reuses layer 0's draw, in its own memory
    assert torch.equal(originals[2]["mlp.up_proj"], originals[0]["mlp.up_proj"])
    assert model.model.layers[2].mlp.up_proj.weight.data_ptr() != \
        model.model.layers[0].mlp.up_proj.weight.data_ptr()
    compress_layers(model, drawn)
    for i, layer in enumerate(model.model.layers):
        assert len(layer._forward_pre_hooks) == 1
        assert [type(m).__name__ for m in layer.weight_injection_modules] == ["FP8Linear"] * 7
        for n in LINEAR_NAMES:
            assert "weight" not in layer.get_submodule(n)._parameters
            assert layer.get_submodule(n).weight_scale_inv.dtype == torch.float32
        flat = oc.decode(layer.luts.numpy(), layer.encoded.numpy(), layer.packed_other_4bits.numpy(),
                         layer.output_positions.numpy(), layer.gaps.numpy())
        parts = np.split(flat, layer.split_positions)
        for n, part in zip(LINEAR_NAMES, parts):
            assert np.array_equal(part, originals[i][n].numpy().reshape(-1)), (i, n)
    assert model.model.layers[2].encoded.data_ptr() != model.model.layers[0].encoded.data_ptr()


def test_linear_shapes_follow_the_qwen3_8b_layer():
    from ecf8_amd.llm import Qwen3Config
    from ecf8_amd.synth import QWEN3_8B_LAYER

    assert Qwen3Config().linear_shapes() == QWEN3_8B_LAYER


def test_dit_blocks_compress_with_the_reference_patterns():
    """FLUX-shaped DiT blocks are compressed per dfloat/const.py's
    diffsynth-flux-fp8 patterns: 8 Linears per double block, 3 per single
    block, and each stored block decodes (oracle) to its original weights."""
    from ecf8_amd.dit import (DOUBLE_LINEARS, SINGLE_LINEARS, FluxConfig, compress_blocks,
                              random_pipeline)

    cfg = FluxConfig(hidden=256, heads=2, mlp=512, double=2, single=3, txt_dim=128,
                     pooled_dim=128)
    pipe, drawn = random_pipeline(cfg, "cpu", distinct=2, seed=5)
    groups = ((pipe.dit.blocks, DOUBLE_LINEARS), (pipe.dit.single_blocks, SINGLE_LINEARS))
    originals = [[{n: b.get_submodule(n).weight.detach().view(torch.uint8).clone() for n in names}
                  for b in blocks] for blocks, names in groups]
    compress_blocks(pipe, drawn)
    for (blocks, names), orig in zip(groups, originals):
        for blk, o in zip(blocks, orig):
            assert len(blk._forward_pre_hooks) == 1
            assert [type(m).__name__ for m in blk.weight_injection_modules] == ["_Lin"] * len(names)
            flat = oc.decode(blk.luts.numpy(), blk.encoded.numpy(), blk.packed_other_4bits.numpy(),
                             blk.output_positions.numpy(), blk.gaps.numpy())
            for n, part in zip(names, np.split(flat, blk.split_positions)):
                assert np.array_equal(part, o[n].numpy().reshape(-1)), n


def test_moe_blocks_compress_with_the_reference_patterns():
    """A Qwen3-MoE-shaped model is cut as dfloat/const.py's qwen3moe
    patterns cut it: each layer's self_attn (k, o, q, v) and each expert
    (down, gate, up) is one block, and every stored block decodes (oracle)
    to its original weights in name-sorted order."""
    from ecf8_amd.moe import (ATTN_LINEARS, EXPERT_LINEARS, Qwen3MoeConfig, compress_moe_layers,
                              random_moe_model)

    cfg = Qwen3MoeConfig(hidden=512, layers=3, heads=8, kv_heads=1, experts=4, top_k=2,
                         moe_intermediate=256, vocab=128)
    model, drawn = random_moe_model(cfg, "cpu", distinct_layers=2, seed=4)
    blocks = []
    for layer in model.model.layers:
        blocks.append((layer.self_attn, ATTN_LINEARS))
        blocks += [(ex, EXPERT_LINEARS) for ex in layer.mlp.experts]
    originals = [{n: m.get_submodule(n).weight.detach().view(torch.uint8).clone() for n in names}
                 for m, names in blocks]
    compress_moe_layers(model, drawn)
    for (m, names), orig in zip(blocks, originals):
        assert len(m._forward_pre_hooks) == 1
        assert [type(x).__name__ for x in m.weight_injection_modules] == ["FP8Linear"] * len(names)
        flat = oc.decode(m.luts.numpy(), m.encoded.numpy(), m.packed_other_4bits.numpy(),
                         m.output_positions.numpy(), m.gaps.numpy())
        for n, part in zip(names, np.split(flat, m.split_positions)):
            assert np.array_equal(part, orig[n].numpy().reshape(-1)), n
    # the router stays a dense bf16 Linear, outside every pattern
    assert model.model.layers[0].mlp.gate.weight.dtype == torch.bfloat16
    # layer 2 reuses layer 0's draw, in its own memory
    assert torch.equal(model.model.layers[2].mlp.experts[1].encoded,
                       model.model.layers[0].mlp.experts[1].encoded)
    assert (model.model.layers[2].mlp.experts[1].encoded.data_ptr()
            != model.model.layers[0].mlp.experts[1].encoded.data_ptr())


def test_dit_attention_follows_an_fp64_softmax_attention():
    """The DiT's chunked attention (bf16 operands, fp32 accumulation) against a
    float64 restatement: relative L2 <= 2e-2 (bf16 operand rounding), over
    chunk boundaries."""
    from ecf8_amd.dit import _attention

    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(1, 2, 150, 128, generator=g) for _ in range(3))
    got = _attention(q, k, v, chunk=64)
    s = (q.double() @ k.double().transpose(-1, -2)) / 128 ** 0.5
    ref = torch.softmax(s, -1) @ v.double()
    rel = ((got.double() - ref).norm() / ref.norm()).item()
    assert got.dtype == torch.float32 and rel <= 2e-2, rel
