"""ecf8_decode_bf16: one compressed block decoded straight into the bf16
weights of its block-scaled FP8 Linears.

GPU: bit-exact against the two-pass path (ecf8_decode, then
ecf8_dequant_fp8_block on each Linear's view) and against torch's fp32
product rounded to bf16, over blocks whose format-blocks start and end
inside and across Linears, every finite FP8 code, and extreme scales;
then the DiT flow with the fused hook gives the FP8 pipeline's latents.
CPU: every argument error is returned before any HIP call."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

FP8 = torch.float8_e4m3fn


def _torch_bf16(w, scale):
    """bf16(fp32(w) * scale[r / 128, c / 128]), computed by torch on the CPU."""
    s = scale.repeat_interleave(128, 0).repeat_interleave(128, 1)
    return (w.float() * s).to(torch.bfloat16)


def _compress(weights):
    from dfloat.compress import compress_flat

    flat = torch.cat([w.reshape(-1) for w, _ in weights])
    return compress_flat(flat)


def _parts(weights, dev):
    parts, start = [], 0
    for w, s in weights:
        parts.append((start, w.shape[0], w.shape[1], s.to(dev)))
        start += w.numel()
    return parts


KEYS = ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps")


def _decode_both(weights, dev):
    """(fused bf16, two-pass bf16, torch bf16) for one block of Linears."""
    from ecf8_amd.decode import build_table, decode_bf16, decode_into, largest_block
    from ecf8_amd.llm_kernels import dequant_fp8_block

    comp = _compress(weights)
    d = {k: comp[k].to(dev) for k in KEYS}
    table = build_table(d["luts"])
    assert table.kind == 1  # automaton
    n = sum(w.numel() for w, _ in weights)
    mb = largest_block(comp["output_positions"])
    parts = _parts(weights, dev)
    fused = torch.full((n + 64,), float("nan"), dtype=torch.bfloat16, device=dev)
    decode_bf16(fused, *(d[k] for k in KEYS), parts, table=table, max_block_elements=mb)
    fp8 = torch.empty(n, dtype=FP8, device=dev)
    decode_into(fp8, *(d[k] for k in KEYS), table=table, max_block_elements=mb)
    two = torch.empty(n, dtype=torch.bfloat16, device=dev)
    for st, rows, cols, sc in parts:
        dequant_fp8_block(fp8[st:st + rows * cols].view(rows, cols), sc,
                          out=two[st:st + rows * cols])
    ref = torch.cat([_torch_bf16(w, s).reshape(-1) for w, s in weights])
    torch.cuda.synchronize()
    tail = fused[n:].cpu()
    return fused[:n].cpu(), two.cpu(), ref, tail


@pytest.mark.gpu
def test_fused_bf16_equals_decode_then_dequant(cuda_device):
    from ecf8_amd.synth import synthetic_fp8

    # widths that are not powers of two, rows of one to five 128-groups; the
    # block spans dozens of format-blocks, whose edges fall inside Linears
    # and at arbitrary elements
    shapes = [(256, 384), (384, 128), (128, 640), (640, 256), (128, 3072)]
    weights = [synthetic_fp8(r, c, 0.02, seed=10 + i) for i, (r, c) in enumerate(shapes)]
    fused, two, ref, tail = _decode_both(weights, cuda_device)
    assert torch.equal(fused.view(torch.int16), two.view(torch.int16))
    assert torch.equal(fused.view(torch.int16), ref.view(torch.int16))
    assert torch.isnan(tail.float()).all()  # nothing past n_elements is written


@pytest.mark.gpu
def test_fused_bf16_every_fp8_code_and_extreme_scales(cuda_device):
    g = torch.Generator().manual_seed(3)
    codes = torch.tensor([c for c in range(256) if c & 0x7F != 0x7F], dtype=torch.uint8)
    rows, cols = 384, 512
    idx = torch.randint(0, codes.numel(), (rows * cols,), generator=g)
    idx[: codes.numel()] = torch.arange(codes.numel())  # every code at least once
    w = codes[idx].view(FP8).view(rows, cols)
    scale = torch.rand(rows // 128, cols // 128, generator=g) * 1e-2 + 1e-6
    scale[0, 0] = 1e-36   # products below the f32 normal range
    scale[1, 1] = 2.5e30  # 448 x scale near the top of the bf16 range
    scale[2, 3] = 1.0
    w2 = w[:128, :256].contiguous()
    s2 = torch.full((1, 2), 0.5)
    fused, two, ref, _ = _decode_both([(w, scale), (w2, s2)], cuda_device)
    assert torch.equal(fused.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(fused.view(torch.int16), two.view(torch.int16))


@pytest.mark.gpu
def test_fused_bf16_sixteen_small_parts(cuda_device):
    """ECF8_MAX_SCALED_PARTS Linears of 128 x 128 to 384 x 256 elements:
    format-blocks (up to 14 K elements at these dense codes) start in one part
    and end in the next, so each block's scale lookups move forward across
    a part boundary."""
    from ecf8_amd.decode import MAX_SCALED_PARTS

    g = torch.Generator().manual_seed(5)
    weights = []
    for j in range(MAX_SCALED_PARTS):
        rows, cols = 128 * (1 + j % 3), 128 * (1 + (j // 3) % 2)
        # mostly four exponents (2-bit codes): many elements per format-block
        e = torch.randint(6, 10, (rows, cols), generator=g)
        e[torch.rand(rows, cols, generator=g) < 0.05] = 3
        o = torch.randint(0, 16, (rows, cols), generator=g)
        b = ((o & 8) << 4 | e << 3 | (o & 7)).to(torch.uint8)
        sc = torch.rand(rows // 128, cols // 128, generator=g) * 1e-2 + 1e-4
        weights.append((b.view(FP8), sc))
    fused, two, ref, tail = _decode_both(weights, cuda_device)
    assert torch.equal(fused.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(fused.view(torch.int16), two.view(torch.int16))
    assert torch.isnan(tail.float()).all()


@pytest.mark.gpu
def test_fused_bf16_rejects_a_multi_symbol_table(cuda_device):
    from ecf8_amd._lib import ECF8_TABLE_MULTI, ECF8Error
    from ecf8_amd.decode import build_table, decode_bf16
    from ecf8_amd.synth import synthetic_fp8

    w, s = synthetic_fp8(128, 256, 0.02, seed=1)
    comp = _compress([(w, s)])
    d = {k: comp[k].to(cuda_device) for k in KEYS}
    table = build_table(d["luts"], kind=ECF8_TABLE_MULTI)
    out = torch.empty(w.numel(), dtype=torch.bfloat16, device=cuda_device)
    with pytest.raises(ECF8Error):
        decode_bf16(out, *(d[k] for k in KEYS), _parts([(w, s)], cuda_device), table=table)


SMALL = dict(hidden=256, heads=2, mlp=512, double=2, single=3, txt_dim=128, pooled_dim=128)


def _small_inputs(cfg, dev):
    g = torch.Generator().manual_seed(8)
    lat = torch.randn(1, 64, cfg.in_channels, generator=g).to(torch.bfloat16).to(dev)
    txt = torch.randn(1, 16, cfg.txt_dim, generator=g).to(torch.bfloat16).to(dev)
    pooled = torch.randn(1, cfg.pooled_dim, generator=g).to(torch.bfloat16).to(dev)
    return lat, txt, pooled


@pytest.mark.gpu
def test_fused_dit_samples_exactly_like_fp8(cuda_device):
    from ecf8_amd.dit import FluxConfig, compress_blocks, fuse_dequant_blocks, generate, random_pipeline

    cfg = FluxConfig(**SMALL)
    plain, drawn = random_pipeline(cfg, cuda_device, seed=7)
    comp, _ = random_pipeline(cfg, cuda_device, seed=7)
    compress_blocks(comp, drawn)
    fuse_dequant_blocks(comp)
    lat, txt, pooled = _small_inputs(cfg, cuda_device)
    a = generate(plain, lat, txt, pooled, steps=3, grid=(8, 8))
    for _ in range(2):
        b = generate(comp, lat, txt, pooled, steps=3, grid=(8, 8))
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert not torch.equal(a, lat)


@pytest.mark.gpu
def test_fused_dit_falls_back_for_tables_the_automaton_cannot_run(cuda_device, monkeypatch):
    """Blocks whose table is the multi-symbol kind decode to FP8, then
    dequantize each Linear into the same bf16 buffer."""
    import dfloat.run.run as run
    from ecf8_amd._lib import ECF8_TABLE_MULTI
    from ecf8_amd.decode import build_table
    from ecf8_amd.dit import FluxConfig, compress_blocks, fuse_dequant_blocks, generate, random_pipeline

    real = run._module_state

    def multi_state(module):
        table, max_block, min_bits = real(module)
        return build_table(module.luts, kind=ECF8_TABLE_MULTI), max_block, min_bits

    cfg = FluxConfig(**SMALL)
    plain, drawn = random_pipeline(cfg, cuda_device, seed=9)
    comp, _ = random_pipeline(cfg, cuda_device, seed=9)
    compress_blocks(comp, drawn)
    monkeypatch.setattr(run, "_module_state", multi_state)
    fuse_dequant_blocks(comp)
    lat, txt, pooled = _small_inputs(cfg, cuda_device)
    a = generate(plain, lat, txt, pooled, steps=2, grid=(8, 8))
    b = generate(comp, lat, txt, pooled, steps=2, grid=(8, 8))
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


# ------------------------------------------------------------------- CPU


_FAKE = dict(luts=0x1000, encoded=0x2000, packed=0x3000, op=0x4000, gaps=0x5000, out=0x6000,
             table=0x7000)


def _call(n=2 * 128 * 128, n_bytes=1000, kind=1, tpb=512, bpt=8, parts=None, n_parts=None,
          **ptrs):
    from ecf8_amd._lib import lib
    from ecf8_amd.decode import SCALED_PART_DTYPE

    p = dict(_FAKE)
    p.update(ptrs)
    if parts is None:
        parts = [(0x8000, 0, 128, 128), (0x9000, 128 * 128, 128, 128)]
    rec = np.zeros(max(1, len(parts)), dtype=SCALED_PART_DTYPE)
    for j, r in enumerate(parts):
        rec[j] = r
    cnt = len(parts) if n_parts is None else n_parts
    return lib().ecf8_decode_bf16(p["luts"], p["encoded"], p["packed"], p["op"], p["gaps"],
                                  p["out"], 3, n_bytes, n, 0, p["table"], kind,
                                  rec.ctypes.data_as(ctypes.c_void_p), cnt, tpb, bpt, None)


@pytest.mark.parametrize("case,status", [
    (dict(kind=0), 2),                                    # multi-symbol table
    (dict(kind=-1), 2),                                   # kind only known on the device
    (dict(tpb=256), 2),
    (dict(bpt=4), 2),
    (dict(n=2 * 128 * 128 + 1), 1),                       # odd element count
    (dict(out=0x6008), 3),                                # output not 16-byte aligned
    (dict(table=0), 1),
    (dict(parts=[]), 1),
    (dict(n_parts=17), 1),
    (dict(parts=[(0x8000, 0, 128, 128), (0x9000, 128 * 128 + 16, 128, 128)]), 1),  # gap
    (dict(parts=[(0x8000, 0, 128, 128), (0x9000, 128 * 128, 128, 192)]), 1),       # cols
    (dict(parts=[(0x8000, 0, 128, 128), (0x9000, 128 * 128, 64, 256)]), 1),        # rows
    (dict(parts=[(0x8000, 0, 128, 128)]), 1),             # parts end before n_elements
    (dict(parts=[(0x8000, 0, 128, 128), (0, 128 * 128, 128, 128)]), 1),             # no scale
    (dict(parts=[(0x8000, 0, 128, 128), (0x9002, 128 * 128, 128, 128)]), 3),        # scale align
    (dict(n=64, parts=[(0x8000, 0, 128, 128), (0x9000, 128 * 128, 128, 128)]), 1),
    (dict(n_bytes=8), 2),                                 # below the clamped vector loads
])
def test_bf16_rejects_before_any_hip_call(case, status):
    assert _call(**case) == status
