"""A FLUX.1-dev-shaped diffusion transformer whose FP8 blocks can be
ECF8-compressed: the end-to-end check and benchmark of the decode path for
the reference's DiT flow (dfloat/run/run.py:569-729, scripts/inference_dfsyn.py).

The module tree keeps DiffSynth's FLUX DiT names (``dit.blocks.N`` double-
stream blocks, ``dit.single_blocks.N`` single-stream blocks, and their
Linears ``attn.a_to_qkv`` ... ``ff_b.2``, ``norm.linear``, ``to_qkv_mlp``,
``proj_out``), so the reference's ``diffsynth-flux-fp8`` patterns
(dfloat/const.py) select exactly the Linears that are compressed, and a
compressed block decodes through the same forward-pre-hook as an LLM layer.

Architecture (public FLUX.1 design): hidden 3072, 24 heads of 128, MLP
12288, 19 double-stream blocks (image and text streams, each with its own
adaptive LayerNorm modulation, joint attention over text + image tokens)
and 38 single-stream blocks (one fused qkv + MLP projection), 3-axis rotary
embedding (16 + 56 + 56 dims), timestep / guidance / pooled-text
conditioning.  Random init.

Compute: the FP8 Linears run at thousands of rows, where the work is
matrix-bound, so each one dequantizes its e4m3fn weight with its 128x128
block scales to bf16 (ecf8_dequant_fp8_block) and calls the library bf16
GEMM; attention runs on bf16 operands with fp32 accumulation (chunked over
queries), the precision of the reference's bf16 pipeline.  The same
consumer runs for the compressed and the uncompressed model.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import llm_kernels as K
from .llm import FP8Linear

DOUBLE_REGEX = r"dit\.blocks\.\d+"
SINGLE_REGEX = r"dit\.single_blocks\.\d+"
DOUBLE_LINEARS = ("attn.a_to_out", "attn.a_to_qkv", "attn.b_to_out", "attn.b_to_qkv",
                  "ff_a.0", "ff_a.2", "ff_b.0", "ff_b.2")  # sorted, dfloat/const.py
SINGLE_LINEARS = ("norm.linear", "proj_out", "to_qkv_mlp")


@dataclass
class FluxConfig:
    """FLUX.1-dev by default."""
    hidden: int = 3072
    heads: int = 24
    head_dim: int = 128
    mlp: int = 12288
    double: int = 19
    single: int = 38
    in_channels: int = 64
    txt_dim: int = 4096
    pooled_dim: int = 768
    axes: tuple = (16, 56, 56)
    theta: float = 10000.0

    def double_shapes(self) -> dict:
        h, m = self.hidden, self.mlp
        return {"attn.a_to_out": (h, h, 0.02), "attn.a_to_qkv": (3 * h, h, 0.02),
                "attn.b_to_out": (h, h, 0.02), "attn.b_to_qkv": (3 * h, h, 0.02),
                "ff_a.0": (m, h, 0.02), "ff_a.2": (h, m, 0.02),
                "ff_b.0": (m, h, 0.02), "ff_b.2": (h, m, 0.02)}

    def single_shapes(self) -> dict:
        h, m = self.hidden, self.mlp
        return {"norm.linear": (3 * h, h, 0.02), "proj_out": (h, h + m, 0.02),
                "to_qkv_mlp": (3 * h + m, h, 0.02)}


class _Lin(FP8Linear):
    """FP8 Linear with a bf16 bias, run as dequantize + bf16 GEMM."""

    def __init__(self, in_features, out_features):
        super().__init__(in_features, out_features)
        self.bias = nn.Parameter(torch.zeros(out_features, dtype=torch.bfloat16),
                                 requires_grad=False)

    def forward(self, x):
        # bf16 weights decoded by the block's hook (fuse_dequant_blocks), or
        # the FP8 weight dequantized here
        w = self.__dict__.get("_w_bf16")
        if w is None:
            w = K.dequant_fp8_block(self.weight, self.weight_scale_inv)
        return F.linear(x, w, self.bias)


class _Norm(nn.Module):
    def __init__(self, dim):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim, dtype=torch.bfloat16), requires_grad=False)

    def forward(self, x):  # RMSNorm over the head, fp32
        x = x.float()
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * self.weight.float()


def _bf16_linear(i, o):
    return nn.Linear(i, o, dtype=torch.bfloat16)


def _modulate(x, shift, scale):
    x = F.layer_norm(x.float(), (x.shape[-1],), eps=1e-6)
    return (x * (1 + scale.float()[:, None]) + shift.float()[:, None]).to(torch.bfloat16)


def _rope(x, cos, sin):
    """Rotate interleaved pairs (2i, 2i+1) of the last dim; x fp32 [B, H, T, D]."""
    x0, x1 = x[..., 0::2], x[..., 1::2]
    out = torch.empty_like(x)
    out[..., 0::2] = x0 * cos - x1 * sin
    out[..., 1::2] = x0 * sin + x1 * cos
    return out


def _attention(q, k, v, chunk: int = 1152):
    """Softmax attention of q, k, v [B, H, T, D] (fp32 in, fp32 out), chunked
    over queries, in the precision the reference's bf16 pipeline attends
    in: bf16 operands for both products and for the softmax, every
    reduction accumulated in fp32.  Every operand of a batched product is a
    contiguous bf16 tensor."""
    scale = 1.0 / math.sqrt(q.shape[-1])
    qb = (q * scale).to(torch.bfloat16).contiguous()
    kt = k.to(torch.bfloat16).transpose(-1, -2).contiguous()
    vb = v.to(torch.bfloat16).contiguous()
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    for i in range(0, q.shape[2], chunk):
        s = torch.matmul(qb[:, :, i:i + chunk].contiguous(), kt)
        p = torch.softmax(s, dim=-1).contiguous()  # fp32 accumulation, bf16 out
        out[:, :, i:i + chunk] = torch.matmul(p, vb).float()
    return out


class _AdaNorm(nn.Module):
    """emb -> 6 modulation vectors (bf16 Linear, not compressed)."""

    def __init__(self, dim, n):
        super().__init__()
        self.linear = _bf16_linear(dim, n * dim)
        self.n = n

    def forward(self, emb):
        return self.linear(F.silu(emb)).chunk(self.n, dim=-1)


class _JointAttention(nn.Module):
    def __init__(self, cfg: FluxConfig):
        super().__init__()
        h = cfg.hidden
        self.a_to_qkv, self.b_to_qkv = _Lin(h, 3 * h), _Lin(h, 3 * h)
        self.a_to_out, self.b_to_out = _Lin(h, h), _Lin(h, h)
        self.norm_q_a, self.norm_k_a = _Norm(cfg.head_dim), _Norm(cfg.head_dim)
        self.norm_q_b, self.norm_k_b = _Norm(cfg.head_dim), _Norm(cfg.head_dim)
        self.heads = cfg.heads


def _heads(x, n_heads):
    B, T, C = x.shape
    return x.view(B, T, n_heads, C // n_heads).transpose(1, 2)


class DoubleBlock(nn.Module):
    def __init__(self, cfg: FluxConfig):
        super().__init__()
        h, m = cfg.hidden, cfg.mlp
        self.norm1_a, self.norm1_b = _AdaNorm(h, 6), _AdaNorm(h, 6)
        self.attn = _JointAttention(cfg)
        self.ff_a = nn.Sequential(_Lin(h, m), nn.GELU(approximate="tanh"), _Lin(m, h))
        self.ff_b = nn.Sequential(_Lin(h, m), nn.GELU(approximate="tanh"), _Lin(m, h))

    def forward(self, img, txt, emb, cos, sin):
        at = self.attn
        sa, ca, ga, sma, cma, gma = self.norm1_a(emb)
        sb, cb, gb, smb, cmb, gmb = self.norm1_b(emb)
        qa, ka, va = _heads(at.a_to_qkv(_modulate(img, sa, ca)), at.heads * 3).chunk(3, dim=1)
        qb, kb, vb = _heads(at.b_to_qkv(_modulate(txt, sb, cb)), at.heads * 3).chunk(3, dim=1)
        q = torch.cat([at.norm_q_b(qb), at.norm_q_a(qa)], dim=2)
        k = torch.cat([at.norm_k_b(kb), at.norm_k_a(ka)], dim=2)
        v = torch.cat([vb.float(), va.float()], dim=2)
        o = _attention(_rope(q, cos, sin), _rope(k, cos, sin), v)
        o = o.transpose(1, 2).reshape(img.shape[0], -1, img.shape[-1]).to(torch.bfloat16)
        n_txt = txt.shape[1]
        img = img + ga[:, None] * at.a_to_out(o[:, n_txt:])
        txt = txt + gb[:, None] * at.b_to_out(o[:, :n_txt])
        img = img + gma[:, None] * self.ff_a(_modulate(img, sma, cma))
        txt = txt + gmb[:, None] * self.ff_b(_modulate(txt, smb, cmb))
        return img, txt


class _SingleNorm(nn.Module):
    def __init__(self, h):
        super().__init__()
        self.linear = _Lin(h, 3 * h)  # compressed: "norm.linear"


class SingleBlock(nn.Module):
    def __init__(self, cfg: FluxConfig):
        super().__init__()
        h, m = cfg.hidden, cfg.mlp
        self.norm = _SingleNorm(h)
        self.to_qkv_mlp = _Lin(h, 3 * h + m)
        self.norm_q_a, self.norm_k_a = _Norm(cfg.head_dim), _Norm(cfg.head_dim)
        self.proj_out = _Lin(h + m, h)
        self.heads, self.hidden = cfg.heads, h

    def forward(self, x, emb, cos, sin):
        shift, scale, gate = self.norm.linear(F.silu(emb)).chunk(3, dim=-1)
        y = self.to_qkv_mlp(_modulate(x, shift, scale))
        qkv, mlp = y[..., : 3 * self.hidden], y[..., 3 * self.hidden:]
        q, k, v = _heads(qkv, self.heads * 3).chunk(3, dim=1)
        o = _attention(_rope(self.norm_q_a(q), cos, sin), _rope(self.norm_k_a(k), cos, sin),
                       v.float())
        o = o.transpose(1, 2).reshape(x.shape[0], -1, self.hidden).to(torch.bfloat16)
        out = self.proj_out(torch.cat([o, F.gelu(mlp, approximate="tanh")], dim=-1))
        return x + gate[:, None] * out


def _timestep_embedding(t: torch.Tensor, dim: int = 256) -> torch.Tensor:
    half = dim // 2
    freqs = torch.exp(-math.log(10000.0) * torch.arange(half, dtype=torch.float32,
                                                        device=t.device) / half)
    a = t.float()[:, None] * 1000.0 * freqs[None]
    return torch.cat([torch.cos(a), torch.sin(a)], dim=-1)


class FluxDiT(nn.Module):
    def __init__(self, cfg: FluxConfig):
        super().__init__()
        h = cfg.hidden
        self.cfg = cfg
        self.x_embedder = _bf16_linear(cfg.in_channels, h)
        self.context_embedder = _bf16_linear(cfg.txt_dim, h)
        self.time_embedder = nn.Sequential(_bf16_linear(256, h), nn.SiLU(), _bf16_linear(h, h))
        self.guidance_embedder = nn.Sequential(_bf16_linear(256, h), nn.SiLU(), _bf16_linear(h, h))
        self.pooled_text_embedder = nn.Sequential(_bf16_linear(cfg.pooled_dim, h), nn.SiLU(),
                                                  _bf16_linear(h, h))
        self.blocks = nn.ModuleList(DoubleBlock(cfg) for _ in range(cfg.double))
        self.single_blocks = nn.ModuleList(SingleBlock(cfg) for _ in range(cfg.single))
        self.final_norm_out = _AdaNorm(h, 2)
        self.final_proj_out = _bf16_linear(h, cfg.in_channels)

    def rope_tables(self, n_txt: int, h: int, w: int, device):
        """cos/sin [T, D/2] for text ids (0, 0, 0) then image ids (0, y, x)."""
        ids = torch.zeros(n_txt + h * w, 3, dtype=torch.float64)
        ys, xs = torch.meshgrid(torch.arange(h), torch.arange(w), indexing="ij")
        ids[n_txt:, 1] = ys.reshape(-1).double()
        ids[n_txt:, 2] = xs.reshape(-1).double()
        angles = []
        for axis, d in enumerate(self.cfg.axes):
            omega = 1.0 / self.cfg.theta ** (torch.arange(0, d, 2, dtype=torch.float64) / d)
            angles.append(ids[:, axis:axis + 1] * omega[None])
        a = torch.cat(angles, dim=-1)
        return (torch.cos(a).float().to(device)[None, None], torch.sin(a).float().to(device)[None, None])

    def forward(self, latents, txt, pooled, t, guidance, cos, sin):
        emb = (self.time_embedder(_timestep_embedding(t).to(torch.bfloat16))
               + self.guidance_embedder(_timestep_embedding(guidance).to(torch.bfloat16))
               + self.pooled_text_embedder(pooled))
        img = self.x_embedder(latents)
        txt = self.context_embedder(txt)
        for blk in self.blocks:
            img, txt = blk(img, txt, emb, cos, sin)
        x = torch.cat([txt, img], dim=1)
        for blk in self.single_blocks:
            x = blk(x, emb, cos, sin)
        img = x[:, txt.shape[1]:]
        shift, scale = self.final_norm_out(emb)
        return self.final_proj_out(_modulate(img, shift, scale))


class FluxPipeline(nn.Module):
    """Holds the DiT as ``dit`` so module paths are ``dit.blocks.N``."""

    def __init__(self, cfg: FluxConfig):
        super().__init__()
        self.dit = FluxDiT(cfg)


def _sigmas(steps: int, n_img: int):
    """Flow-matching sigmas 1 -> 0 with the resolution-dependent shift FLUX
    uses (mu interpolated between 256 and 4096 image tokens)."""
    mu = 0.5 + (1.15 - 0.5) * (n_img - 256) / (4096 - 256)
    s = torch.linspace(1.0, 1.0 / steps, steps, dtype=torch.float64)
    s = math.exp(mu) / (math.exp(mu) + (1.0 / s - 1.0))
    return torch.cat([s, torch.zeros(1, dtype=torch.float64)])


@torch.no_grad()
def generate(pipe: FluxPipeline, latents, txt, pooled, steps: int = 28, guidance: float = 3.5,
             grid=(64, 64)):
    """Euler flow-matching sampling (scripts/inference_dfsyn.py's 28 steps,
    embedded guidance 3.5, cfg 1): returns the final latents."""
    dit = pipe.dit
    dev = latents.device
    cos, sin = dit.rope_tables(txt.shape[1], grid[0], grid[1], dev)
    sig = _sigmas(steps, latents.shape[1])
    g = torch.full((latents.shape[0],), guidance, device=dev)
    x = latents
    for i in range(steps):
        t = torch.full((latents.shape[0],), float(sig[i]), device=dev)
        v = dit(x, txt, pooled, t, g, cos, sin)
        x = (x.float() + (float(sig[i + 1]) - float(sig[i])) * v.float()).to(torch.bfloat16)
    return x


# ------------------------------------------------------------ construction


def random_pipeline(cfg: FluxConfig, device, distinct: int | None = None, seed: int = 0):
    """Random-init pipeline; the compressible Linears get synthetic FP8
    weights (N(0, 0.02) block-quantized).  ``distinct`` draws that many
    double and single blocks and gives every block its own copy of one."""
    from .synth import synthetic_block

    with torch.device("meta"):
        pipe = FluxPipeline(cfg)
    pipe = pipe.to_empty(device=device)
    g = torch.Generator(device=device).manual_seed(seed)
    with torch.no_grad():
        for name, p in pipe.named_parameters():
            if p.dtype == torch.float8_e4m3fn:
                continue
            if name.endswith("norm_q_a.weight") or "norm_" in name.split(".")[-2]:
                p.fill_(1.0)
            elif name.endswith(".bias"):
                p.zero_()
            else:
                p.normal_(0.0, 0.02, generator=g)
    nd = cfg.double if distinct is None else max(1, min(distinct, cfg.double))
    ns = cfg.single if distinct is None else max(1, min(distinct, cfg.single))
    drawn_d = [synthetic_block(cfg.double_shapes(), seed=seed * 1000 + j) for j in range(nd)]
    drawn_s = [synthetic_block(cfg.single_shapes(), seed=seed * 1000 + 500 + j) for j in range(ns)]
    for blocks, drawn in ((pipe.dit.blocks, drawn_d), (pipe.dit.single_blocks, drawn_s)):
        for i, blk in enumerate(blocks):
            for name, (w, s) in drawn[i % len(drawn)].items():
                lin = blk.get_submodule(name)
                lin.weight = nn.Parameter(w.to(device, copy=True), requires_grad=False)
                lin.weight_scale_inv = s.to(device, copy=True)
    return pipe, (drawn_d, drawn_s)


def compress_blocks(pipe: FluxPipeline, drawn=None, threads_per_block: int = 512,
                    bytes_per_thread: int = 8):
    """Compress every double and single block as the reference does
    (one block per ``dit.blocks.N`` / ``dit.single_blocks.N`` match) and
    install the decode hooks through the loader's registration."""
    from dfloat.compress import compress_flat
    from dfloat.run.run import _process_compressed_tensor
    from .synth import flat_block

    groups = ((pipe.dit.blocks, "dit.blocks", DOUBLE_REGEX, DOUBLE_LINEARS,
               None if drawn is None else drawn[0]),
              (pipe.dit.single_blocks, "dit.single_blocks", SINGLE_REGEX, SINGLE_LINEARS,
               None if drawn is None else drawn[1]))
    for blocks, prefix, regex, names, dr in groups:
        pattern = {regex: list(names)}
        cache = {}
        for i, blk in enumerate(blocks):
            key = i % len(dr) if dr is not None else i
            comp = cache.get(key)
            if comp is None:
                weights = (dr[key] if dr is not None else
                           {n: blk.get_submodule(n).weight.detach().cpu() for n in names})
                flat, split = flat_block(weights)
                res = compress_flat(flat, bytes_per_thread, threads_per_block)
                comp = {k: res[k] for k in ("luts", "encoded", "packed_other_4bits",
                                            "output_positions", "gaps")}
                comp["split_positions"] = torch.tensor(split, dtype=torch.int64)
                if dr is not None:
                    cache[key] = comp
            dev = blk.get_submodule(names[0]).weight_scale_inv.device
            for attr in ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps",
                         "split_positions"):
                value = comp[attr] if attr == "split_positions" else comp[attr].to(dev).clone()
                _process_compressed_tensor(blk, attr, value, f"{prefix}.{i}.{attr}", pattern,
                                           threads_per_block, bytes_per_thread)
    return pipe


def prefetch_blocks(pipe: FluxPipeline, device=None, workgroups_per_cu: float = 2):
    """Replace the compressed blocks' decode hooks by side-stream prefetch
    (ecf8_amd/prefetch.py) over the blocks in forward order: the 19 double
    blocks, then the 38 single blocks.  A block's decode (an HBM-bound
    pass) then runs while the previous block's matrix-bound GEMMs and
    attention run, instead of between them."""
    from .prefetch import LayerPrefetcher

    blocks = list(pipe.dit.blocks) + list(pipe.dit.single_blocks)
    return LayerPrefetcher(blocks, device, workgroups_per_cu=workgroups_per_cu).install()


_BF16_BUFFERS: dict = {}


def _bf16_buffer(device, n: int) -> torch.Tensor:
    """One grow-only bf16 decode buffer per device, shared by every block
    (as the loader's TensorManager shares its FP8 buffer)."""
    buf = _BF16_BUFFERS.get(device)
    if buf is None or buf.numel() < n:
        _BF16_BUFFERS.pop(device, None)
        buf = torch.empty(n, dtype=torch.bfloat16, device=device)
        _BF16_BUFFERS[device] = buf
    return buf


def fuse_dequant_blocks(pipe: FluxPipeline):
    """Replace each compressed block's decode hook by one that decodes the
    block straight into its Linears' bf16 weights (ecf8_decode_bf16: the
    FP8 bytes times their 128x128 block scales, never written as FP8), so
    the Linears skip their own dequantization: the same bf16 weights as
    decode + dequantize, in one pass over HBM instead of two.

    All blocks decode into one shared bf16 buffer (as the loader's hooks
    share TensorManager's FP8 buffer); each Linear gets its view of that
    buffer here, once, and every call's arguments are checked and packed
    here, so a hook is one launch (the DiT's step issues thousands of small
    kernels, and host time spent in hooks shows up as GPU idle time).  Call
    after the pipeline is on its device; the blocks' FP8 ``weight`` views
    are no longer set."""
    from dfloat.run.run import TensorManager, _module_state
    from ._lib import ECF8_TABLE_DFA
    from .decode import decode_into, prepare_bf16

    blocks = list(pipe.dit.blocks) + list(pipe.dit.single_blocks)
    if not blocks:
        return pipe
    dev = blocks[0].encoded.device
    n_max = max(b.packed_other_4bits.numel() * 2 for b in blocks)
    out = _bf16_buffer(dev, n_max)
    for blk in blocks:
        lins = list(blk.weight_injection_modules)
        starts = [0] + list(blk.split_positions)
        parts = [(st, lin.out_features, lin.in_features, lin.weight_scale_inv)
                 for st, lin in zip(starts, lins)]
        n = blk.packed_other_4bits.numel() * 2
        if starts[-1] + lins[-1].out_features * lins[-1].in_features != n:
            raise ValueError("the block's Linears do not cover its compressed elements")
        for (st, rows, cols, _), lin in zip(parts, lins):
            lin.__dict__["_w_bf16"] = out[st:st + rows * cols].view(rows, cols)
        table, max_block, min_bits = _module_state(blk)
        if table.kind == ECF8_TABLE_DFA:
            call = prepare_bf16(out, blk.luts, blk.encoded, blk.packed_other_4bits,
                                blk.output_positions, blk.gaps, parts, table=table,
                                max_block_elements=max_block)

            def hook(module, _args, call=call):
                call()
        else:  # LUTs the automaton cannot run: decode, then dequantize
            def hook(module, _args, parts=parts, n=n, table=table, max_block=max_block,
                     min_bits=min_bits):
                fp8 = TensorManager.get_tensor(module.encoded.device, n)
                decode_into(fp8, module.luts, module.encoded, module.packed_other_4bits,
                            module.output_positions, module.gaps, table=table,
                            max_block_elements=max_block, min_code_bits=min_bits)
                for st, rows, cols, scale in parts:
                    K.dequant_fp8_block(fp8[st:st + rows * cols].view(rows, cols), scale,
                                        out=out[st:st + rows * cols])

        blk._forward_pre_hooks.clear()
        blk.register_forward_pre_hook(hook)
    return pipe


def timed_generate(pipe, latents, txt, pooled, steps, grid):
    dev = latents.device
    torch.cuda.synchronize(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    t0 = time.perf_counter()
    out = generate(pipe, latents, txt, pooled, steps=steps, grid=grid)
    torch.cuda.synchronize(dev)
    dt = time.perf_counter() - t0
    return {"seconds": dt, "peak_mib": torch.cuda.max_memory_allocated(dev) / 2**20,
            "latents": out.clone()}
