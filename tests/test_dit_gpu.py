"""GPU checks of the FLUX-shaped DiT flow (ecf8_amd/dit.py): the FP8 block
dequantization is bit-exact against torch's fp32 product rounded to bf16,
and sampling with ECF8-compressed blocks (decoded by the forward-pre-hook)
gives exactly the latents of the same pipeline kept in FP8, also with the
blocks decoded on a side stream one block ahead."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_dequant_fp8_block_matches_torch(cuda_device):
    from ecf8_amd.llm_kernels import dequant_fp8_block

    g = torch.Generator().manual_seed(2)
    n, k = 384, 1024
    b = torch.randint(0, 256, (n, k), generator=g, dtype=torch.int32).to(torch.uint8)
    b[(b & 0x7F) == 0x7F] = 0x7E  # NaN codes never occur in weights
    w = b.view(torch.float8_e4m3fn)
    s = torch.rand(n // 128, k // 128, generator=g) * 1e-2 + 1e-5
    got = dequant_fp8_block(w.to(cuda_device), s.to(cuda_device)).cpu()
    ref = (w.float() * s.repeat_interleave(128, 0).repeat_interleave(128, 1)).to(torch.bfloat16)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


SMALL = dict(hidden=256, heads=2, mlp=512, double=2, single=2, txt_dim=128, pooled_dim=128)


def test_compressed_dit_samples_exactly_like_fp8(cuda_device):
    from ecf8_amd.dit import FluxConfig, compress_blocks, generate, random_pipeline
    from dfloat.run.run import TensorManager

    cfg = FluxConfig(**SMALL)
    plain, drawn = random_pipeline(cfg, cuda_device, seed=3)
    comp, _ = random_pipeline(cfg, cuda_device, seed=3)
    compress_blocks(comp, drawn)
    g = torch.Generator().manual_seed(4)
    lat = torch.randn(1, 64, cfg.in_channels, generator=g).to(torch.bfloat16).to(cuda_device)
    txt = torch.randn(1, 16, cfg.txt_dim, generator=g).to(torch.bfloat16).to(cuda_device)
    pooled = torch.randn(1, cfg.pooled_dim, generator=g).to(torch.bfloat16).to(cuda_device)
    TensorManager.clear_device()
    a = generate(plain, lat, txt, pooled, steps=3, grid=(8, 8))
    b = generate(comp, lat, txt, pooled, steps=3, grid=(8, 8))
    assert torch.isfinite(a.float()).all()
    assert not torch.equal(a, lat)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_prefetched_dit_samples_exactly_like_fp8(cuda_device):
    """Five blocks (an odd count: the last block takes the prefetcher's
    third buffer), decoded one block ahead on a side stream, over three
    sampling steps: each step's first block was decoded by the previous
    step's last pre-hook."""
    from ecf8_amd.dit import FluxConfig, compress_blocks, generate, prefetch_blocks, random_pipeline
    from dfloat.run.run import TensorManager

    cfg = FluxConfig(**dict(SMALL, single=3))
    plain, drawn = random_pipeline(cfg, cuda_device, seed=5)
    comp, _ = random_pipeline(cfg, cuda_device, seed=5)
    compress_blocks(comp, drawn)
    pf = prefetch_blocks(comp, cuda_device)
    assert pf.slot == [0, 1, 0, 1, 2]
    g = torch.Generator().manual_seed(6)
    lat = torch.randn(1, 64, cfg.in_channels, generator=g).to(torch.bfloat16).to(cuda_device)
    txt = torch.randn(1, 16, cfg.txt_dim, generator=g).to(torch.bfloat16).to(cuda_device)
    pooled = torch.randn(1, cfg.pooled_dim, generator=g).to(torch.bfloat16).to(cuda_device)
    TensorManager.clear_device()
    a = generate(plain, lat, txt, pooled, steps=3, grid=(8, 8))
    for _ in range(2):
        b = generate(comp, lat, txt, pooled, steps=3, grid=(8, 8))
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert not torch.equal(a, lat)
    pf.uninstall()
