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
