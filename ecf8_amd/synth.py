"""Seeded synthetic FP8 e4m3fn weights and the Qwen3-8B decoder-layer shapes.

Weights are N(0, sigma) fp32, quantized per 128x128 tile with scale =
448 / amax (the forward scale; weight_scale_inv = amax / 448 is what an FP8
checkpoint stores), clamped to +-448 and cast to e4m3fn -- the scheme of
transformers' block FP8 quantizer that produces the reference's FP8
checkpoints.
"""

from __future__ import annotations

import torch

FP8_MAX = 448.0
BLOCK = 128

# (out_features, in_features, sigma) of one Qwen3-8B decoder layer's linears,
# in the name-sorted order the reference flattens a block in.
QWEN3_8B_LAYER = {
    "mlp.down_proj": (4096, 12288, 0.01),
    "mlp.gate_proj": (12288, 4096, 0.02),
    "mlp.up_proj": (12288, 4096, 0.02),
    "self_attn.k_proj": (1024, 4096, 0.02),
    "self_attn.o_proj": (4096, 4096, 0.01),
    "self_attn.q_proj": (4096, 4096, 0.02),
    "self_attn.v_proj": (1024, 4096, 0.02),
}


# FLUX.1-dev-shaped DiT blocks (hidden 3072, MLP 12288, 24 heads x 128):
# the FP8 linears of one double-stream and one single-stream block.
FLUX_DOUBLE_BLOCK = {
    "attn.a_to_out": (3072, 3072, 0.02),
    "attn.a_to_qkv": (9216, 3072, 0.02),
    "attn.b_to_out": (3072, 3072, 0.02),
    "attn.b_to_qkv": (9216, 3072, 0.02),
    "ff_a.0": (12288, 3072, 0.02),
    "ff_a.2": (3072, 12288, 0.02),
    "ff_b.0": (12288, 3072, 0.02),
    "ff_b.2": (3072, 12288, 0.02),
}
FLUX_SINGLE_BLOCK = {
    "norm.linear": (9216, 3072, 0.02),
    "proj_out": (3072, 15360, 0.02),
    "to_qkv_mlp": (21504, 3072, 0.02),
}

# Qwen3-30B-A3B-shaped MoE layer (hidden 2048, 128 experts of intermediate
# 768, 32 query / 4 KV heads x 128): one expert block and the attention block.
QWEN3_MOE_EXPERT = {
    "down_proj": (2048, 768, 0.02),
    "gate_proj": (768, 2048, 0.02),
    "up_proj": (768, 2048, 0.02),
}
QWEN3_MOE_ATTN = {
    "k_proj": (512, 2048, 0.02),
    "o_proj": (2048, 4096, 0.01),
    "q_proj": (4096, 2048, 0.02),
    "v_proj": (512, 2048, 0.02),
}


def quantize_fp8_blockwise(w: torch.Tensor, block: int = BLOCK):
    """fp32 [out, in] -> (e4m3fn [out, in], weight_scale_inv fp32 [out/b, in/b])."""
    rows, cols = w.shape
    assert rows % block == 0 and cols % block == 0
    t = w.float().reshape(rows // block, block, cols // block, block)
    amax = t.abs().amax(dim=(1, 3))
    safe = torch.where(amax > 0, amax, torch.ones_like(amax))
    scale = torch.where(amax > 0, FP8_MAX / safe, torch.ones_like(amax))
    q = torch.clamp(t * scale[:, None, :, None], -FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q.reshape(rows, cols), (1.0 / scale).float()


def synthetic_fp8(rows: int, cols: int, sigma: float = 0.02, seed: int = 0,
                  generator: torch.Generator | None = None):
    """Seeded N(0, sigma) weights, block-quantized; returns (fp8, scale_inv)."""
    g = generator
    if g is None:
        g = torch.Generator().manual_seed(seed)
    w = torch.randn(rows, cols, generator=g, dtype=torch.float32) * sigma
    return quantize_fp8_blockwise(w)


def synthetic_block(shapes: dict, seed: int = 0):
    """{name: (fp8 weight, scale_inv)} for a block of linears given as
    {name: (out, in, sigma)}, drawn from one generator seeded with ``seed``
    in name-sorted order."""
    g = torch.Generator().manual_seed(seed)
    return {name: synthetic_fp8(o, i, s, generator=g) for name, (o, i, s) in sorted(shapes.items())}


def qwen3_8b_layer(seed: int = 0):
    """{name: (fp8 weight, scale_inv)} for one Qwen3-8B-shaped layer."""
    return synthetic_block(QWEN3_8B_LAYER, seed)


def flat_block(weights: dict) -> tuple[torch.Tensor, list[int]]:
    """Concatenate name-sorted fp8 weights; returns (flat e4m3fn, split positions)."""
    names = sorted(weights)
    ts = [weights[n][0] if isinstance(weights[n], tuple) else weights[n] for n in names]
    flat = torch.cat([t.reshape(-1) for t in ts])
    splits, acc = [], 0
    for t in ts[:-1]:
        acc += t.numel()
        splits.append(acc)
    return flat, splits
