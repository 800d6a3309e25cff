"""A Qwen3-MoE-shaped causal LM (Qwen3-30B-A3B by default) whose attention
blocks and experts are the reference's compressed blocks: the end-to-end
check and benchmark of the batched, routed decode.

The module tree keeps Hugging Face's Qwen3-MoE names
(``model.layers.N.self_attn.q_proj``, ``model.layers.N.mlp.gate``,
``model.layers.N.mlp.experts.E.gate_proj`` ...), so the reference's
``qwen3moe`` patterns (dfloat/const.py:15-21) cut the same blocks: each
layer's ``self_attn`` (k, o, q, v) and each expert (down, gate, up).  They
are registered through the loader's path (dfloat/run/run.py:406-458).  The
attention block is decoded by its forward-pre-hook, as the reference does.
The reference also hooks every expert, and transformers runs each expert
the router picked, which decodes each picked expert in its own launch.
Here the router runs on the device, then one batched launch decodes only
the picked experts of the layer (ecf8_decode_batched_select).  The grouped
expert linears read the decoded experts from the shared expert buffer.

MoE math (transformers' Qwen3MoeSparseMoeBlock): router logits over the
bf16 normalized hidden state, softmax in fp32, top-k experts, weights
renormalized to sum 1, output = sum_k w_k * down_k(silu(gate_k(h)) *
up_k(h)), accumulated in fp32 per token in top-k order.  Expert linears
use the block-scaled FP8 math of the dense layers.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn

from . import decode as _dev
from . import llm_kernels as K
from . import tiled
from ._lib import ECF8Error
from .llm import FP8Linear, RMSNorm, _GreedyRunner, _rotary_tables, weight_layout
from .synth import QWEN3_MOE_ATTN, QWEN3_MOE_EXPERT

ATTN_LINEARS = ("k_proj", "o_proj", "q_proj", "v_proj")   # sorted
EXPERT_LINEARS = ("down_proj", "gate_proj", "up_proj")    # sorted
ATTN_REGEX = r"model\.layers\.\d+\.self_attn"
EXPERT_REGEX = r"model\.layers\.\d+\.mlp\.experts\.\d+"
_KEYS = ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps")


@dataclass
class Qwen3MoeConfig:
    """Qwen3-30B-A3B by default."""
    hidden: int = 2048
    layers: int = 48
    heads: int = 32
    kv_heads: int = 4
    head_dim: int = 128
    experts: int = 128
    top_k: int = 8
    moe_intermediate: int = 768
    vocab: int = 151936
    rope_theta: float = 1_000_000.0
    eps: float = 1e-6

    def attn_shapes(self) -> dict:
        h, q, kv = self.hidden, self.heads * self.head_dim, self.kv_heads * self.head_dim
        if (h, q, kv) == (2048, 4096, 512):
            return dict(QWEN3_MOE_ATTN)
        return {"q_proj": (q, h, 0.02), "k_proj": (kv, h, 0.02), "v_proj": (kv, h, 0.02),
                "o_proj": (h, q, 0.01)}

    def expert_shapes(self) -> dict:
        h, i = self.hidden, self.moe_intermediate
        if (h, i) == (2048, 768):
            return dict(QWEN3_MOE_EXPERT)
        return {"gate_proj": (i, h, 0.02), "up_proj": (i, h, 0.02), "down_proj": (h, i, 0.02)}


class MoeAttention(nn.Module):
    def __init__(self, cfg: Qwen3MoeConfig):
        super().__init__()
        h, q, kv = cfg.hidden, cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
        self.q_proj, self.k_proj = FP8Linear(h, q), FP8Linear(h, kv)
        self.v_proj, self.o_proj = FP8Linear(h, kv), FP8Linear(q, h)
        self.q_norm, self.k_norm = RMSNorm(cfg.head_dim), RMSNorm(cfg.head_dim)

    def forward(self, runner: "Qwen3MoeRunner", index: int, prefill: bool):
        # calling the module (not runner.attention directly) runs the decode hook
        return runner.attention(self, index, prefill)


class Expert(nn.Module):
    def __init__(self, cfg: Qwen3MoeConfig):
        super().__init__()
        self.gate_proj = FP8Linear(cfg.hidden, cfg.moe_intermediate)
        self.up_proj = FP8Linear(cfg.hidden, cfg.moe_intermediate)
        self.down_proj = FP8Linear(cfg.moe_intermediate, cfg.hidden)


class SparseMoeBlock(nn.Module):
    def __init__(self, cfg: Qwen3MoeConfig):
        super().__init__()
        self.gate = nn.Linear(cfg.hidden, cfg.experts, bias=False, dtype=torch.bfloat16)
        self.experts = nn.ModuleList(Expert(cfg) for _ in range(cfg.experts))


class MoeDecoderLayer(nn.Module):
    def __init__(self, cfg: Qwen3MoeConfig):
        super().__init__()
        self.self_attn, self.mlp = MoeAttention(cfg), SparseMoeBlock(cfg)
        self.input_layernorm = RMSNorm(cfg.hidden)
        self.post_attention_layernorm = RMSNorm(cfg.hidden)

    def forward(self, runner: "Qwen3MoeRunner", index: int, x_prev, prefill: bool):
        return runner.layer(self, index, x_prev, prefill)


class _MoeModel(nn.Module):
    def __init__(self, cfg: Qwen3MoeConfig):
        super().__init__()
        self.embed_tokens = nn.Embedding(cfg.vocab, cfg.hidden, dtype=torch.bfloat16)
        self.layers = nn.ModuleList(MoeDecoderLayer(cfg) for _ in range(cfg.layers))
        self.norm = RMSNorm(cfg.hidden)


class Qwen3MoeForCausalLM(nn.Module):
    def __init__(self, cfg: Qwen3MoeConfig):
        super().__init__()
        self.config = cfg
        self.model = _MoeModel(cfg)
        self.lm_head = nn.Linear(cfg.hidden, cfg.vocab, bias=False, dtype=torch.bfloat16)


class _LayerExperts:
    """One layer's experts as the grouped linears see them: address tables
    of (gate, up) and (down) per expert.  Compressed experts (buffers
    registered by the loader) decode into slot e of the shared expert
    buffer; ``decode_routed`` decodes the experts whose select flag is set,
    ``decode_all`` every expert (the prompt, where nearly all are picked).
    Re-tiled experts (retile_moe_layers) run the decode step's grouped
    linears on their tiled form (``tiled_gu`` / ``tiled_down``, which decode
    the routed experts' weight operands themselves); ``decode_all`` writes
    every expert's FP8 Linears into the buffer for the prompt."""

    def __init__(self, mlp: SparseMoeBlock, expert_buf, gu_out, down_out):
        experts = list(mlp.experts)
        self.compressed = hasattr(experts[0], "encoded")
        self.tiled = hasattr(experts[0], "_ecf8_tiles")
        weights = []
        layout = K.WEIGHT_ROWS  # decoded experts land row-major in the expert buffer
        if self.tiled:
            n_e = sum(lin.out_features * lin.in_features
                      for lin in (experts[0].gate_proj, experts[0].up_proj, experts[0].down_proj))
            if expert_buf is None or expert_buf.numel() < n_e * len(experts):
                raise ECF8Error("expert buffer too small for the layer's experts")
            tables = [ex._ecf8_tile_table for ex in experts]
            self._decoders = []
            views = {name: [] for name in ("gate_proj", "up_proj", "down_proj")}
            for e, ex in enumerate(experts):
                off = e * n_e
                for name in ("gate_proj", "up_proj", "down_proj"):
                    lin = ex.get_submodule(name)
                    n = lin.out_features * lin.in_features
                    views[name].append(expert_buf[off:off + n].view(lin.out_features,
                                                                    lin.in_features))
                    off += n
            for name in ("gate_proj", "up_proj", "down_proj"):
                self._decoders.append(tiled.TileDecodeBatch(
                    [ex._ecf8_tiles[name] for ex in experts], tables, views[name]))
            for e, ex in enumerate(experts):
                weights.append(tuple((views[name][e], ex.get_submodule(name).weight_scale_inv)
                                     for name in ("gate_proj", "up_proj", "down_proj")))
            self.tiled_gu = tiled.TileMoePlan(
                [[ex._ecf8_tiles["gate_proj"], ex._ecf8_tiles["up_proj"]] for ex in experts],
                tables, gu_out)
            self.tiled_down = tiled.TileMoePlan([[ex._ecf8_tiles["down_proj"]] for ex in experts],
                                                tables, down_out)
        elif self.compressed:
            n_e = experts[0].packed_other_4bits.numel() * 2
            if expert_buf is None or expert_buf.numel() < n_e * len(experts):
                raise ECF8Error("expert buffer too small for the layer's experts")
            blocks, outs, tables, largest = [], [], [], 0
            from dfloat.run.run import _module_state

            for e, ex in enumerate(experts):
                if ex.packed_other_4bits.numel() * 2 != n_e:
                    raise ECF8Error("experts of one layer must have equal sizes")
                table, max_block, _ = _module_state(ex)
                largest = max(largest, max_block)
                out = expert_buf[e * n_e:(e + 1) * n_e]
                blocks.append({k: getattr(ex, k) for k in _KEYS})
                outs.append(out)
                tables.append(table)
                # the block's Linears in flatten (name-sorted) order
                parts = torch.tensor_split(out, ex.split_positions)
                views = {id(m): p.view(m.out_features, m.in_features)
                         for m, p in zip(ex.weight_injection_modules, parts)}
                weights.append(tuple((views[id(lin)], lin.weight_scale_inv)
                                     for lin in (ex.gate_proj, ex.up_proj, ex.down_proj)))
            self.plan = _dev.prepare_batch(blocks, outs, tables, max_block_elements=largest)
            self.select = _dev.BatchSelect(self.plan)
        else:
            for ex in experts:
                weights.append(tuple((lin.weight, lin.weight_scale_inv)
                                     for lin in (ex.gate_proj, ex.up_proj, ex.down_proj)))
            layouts = {weight_layout(lin) for ex in experts
                       for lin in (ex.gate_proj, ex.up_proj, ex.down_proj)}
            if len(layouts) != 1:
                raise ECF8Error("a layer's experts must share one weight layout")
            layout = layouts.pop()
        self.gu = K.MoeLinearPlan([[g, u] for g, u, _ in weights], gu_out, layout)
        self.down = K.MoeLinearPlan([[d] for _, _, d in weights], down_out, layout)

    def decode_routed(self, flags):
        self.select(flags)

    def decode_all(self):
        if self.tiled:
            for dec in self._decoders:
                dec()
        else:
            _dev.decode_batched(self.plan)


class Qwen3MoeRunner(_GreedyRunner):
    """Prefill + greedy decode of a fixed batch on one device.  The prompt's
    MoE runs in chunks of ``prefill_chunk`` tokens (rounded down to a
    multiple of 16, the activation tile height; at most 8192 (token,
    expert) pairs per routing step)."""

    def __init__(self, model: Qwen3MoeForCausalLM, batch: int, prompt_len: int, max_len: int,
                 device=None, prefill_chunk: int = 512):
        cfg = model.config
        if cfg.hidden not in (2048, 4096) or cfg.head_dim != 128:
            raise ECF8Error("the fused kernels need hidden 2048 or 4096 and head_dim 128")
        if cfg.heads not in (4 * cfg.kv_heads, 8 * cfg.kv_heads):
            raise ECF8Error("query heads must be 4 or 8 per KV head")
        if cfg.moe_intermediate % 128 or cfg.experts > 256:
            raise ECF8Error("expert intermediate must be a multiple of 128; at most 256 experts")
        # chunks start on 16-row boundaries of the tile-layout activations
        chunk = min(prefill_chunk, 8192 // cfg.top_k) // 16 * 16
        if batch * cfg.top_k > 8192 or chunk < 16:
            raise ECF8Error("a decode step routes at most 8192 (token, expert) pairs")
        self.model, self.cfg = model, cfg
        self.dev = torch.device(device) if device is not None else model.lm_head.weight.device
        self.B, self.T, self.Lmax, self.chunk = batch, prompt_len, max_len, chunk
        dev, B = self.dev, batch
        M = B * prompt_len
        H, Hq, Hkv, D = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim
        I, E = cfg.moe_intermediate, cfg.experts
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.kc = [torch.empty(B, Hkv, max_len, D, **bf) for _ in range(cfg.layers)]
        self.vc = [torch.empty(B, Hkv, max_len, D, **bf) for _ in range(cfg.layers)]
        self.cos, self.sin = _rotary_tables(cfg, max_len, dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.step = torch.zeros(1, dtype=torch.int64, device=dev)
        self.res = torch.empty(M, H, dtype=torch.float32, device=dev)
        # quantized activations in the tile layout: rows padded to 16
        self.aqH = torch.empty(K.pad16(M), H, dtype=torch.float8_e4m3fn, device=dev)
        self.asH = torch.empty(M, H // 128, dtype=torch.float32, device=dev)
        self.aqA = torch.empty(K.pad16(M), Hq * D, dtype=torch.float8_e4m3fn, device=dev)
        self.asA = torch.empty(M, Hq * D // 128, dtype=torch.float32, device=dev)
        self.qkv = torch.empty(M, (Hq + 2 * Hkv) * D, **bf)
        self.q = torch.empty(B * Hq * prompt_len * D, **bf)
        self.attn = torch.empty(M, Hq * D, **bf)
        self.o = torch.empty(M, H, **bf)
        self.hb = torch.empty(M, H, **bf)
        self.y = torch.empty(M, H, **bf)
        self.h = torch.empty(M, H, **bf)
        self.work = K.attention_work(B, Hq, max_len, dev)
        Mr = max(B, chunk)
        P = Mr * cfg.top_k
        self.route = K.MoeRouting(Mr, cfg.top_k, E, dev)
        self.gu = torch.empty(P, 2 * I, **bf)
        self.hq = torch.empty(K.pad16(P), I, dtype=torch.float8_e4m3fn, device=dev)
        self.hs = torch.empty(P, I // 128, dtype=torch.float32, device=dev)
        self.down = torch.empty(P, H, **bf)
        layers = list(model.model.layers)
        ex0 = layers[0].mlp.experts[0]
        self.expert_buf = None
        if hasattr(ex0, "encoded") or hasattr(ex0, "_ecf8_tiles"):
            n_e = sum(lin.out_features * lin.in_features
                      for lin in (ex0.gate_proj, ex0.up_proj, ex0.down_proj))
            self.expert_buf = torch.empty(n_e * E, dtype=torch.float8_e4m3fn, device=dev)
        self.experts = [_LayerExperts(layer.mlp, self.expert_buf, self.gu, self.down)
                        for layer in layers]
        self.next_tok = torch.zeros(B, dtype=torch.int64, device=dev)
        self.tokens = torch.zeros(B, max_len, dtype=torch.int64, device=dev)
        self.graph = None
        self.logits = None
        self._plans = {}

    def _attn_linear(self, a: MoeAttention, index: int, which, names, out, M):
        """An FP8 plan over the attention block's (hook injected) weights, or
        for a re-tiled block the tiled linear (M <= 16) or its Linears
        decoded into prompt buffers first."""
        tiles = getattr(a, "_ecf8_tiles", None)
        if tiles is None:
            mods = [a.get_submodule(n) for n in names]
            return self._plan(a, index, which,
                              [(x.weight, x.weight_scale_inv, weight_layout(x)) for x in mods], out)
        if M <= 16:
            key = (index, which, "tiled")
            p = self._plans.get(key)
            if p is None:
                p = tiled.TileLinearPlan([tiles[n] for n in names], a._ecf8_tile_table, out)
                self._plans[key] = p
            return p
        weights = []
        for n in names:
            op = tiles[n]
            buf = self._tile_scratch(op.n * op.k, n)
            tiled.tile_decode(op, a._ecf8_tile_table, buf)
            weights.append((buf.view(op.n, op.k), op.weight_scale))
        return K.LinearPlan(weights, out)

    def _tile_scratch(self, numel, name):
        if not hasattr(self, "_tile_bufs"):
            self._tile_bufs = {}
        buf = self._tile_bufs.get(name)
        if buf is None or buf.numel() < numel:
            buf = torch.empty(numel, dtype=torch.float8_e4m3fn, device=self.dev)
            self._tile_bufs[name] = buf
        return buf[:numel]

    def attention(self, a: MoeAttention, index: int, prefill: bool):
        cfg = self.cfg
        B, T = self.B, (self.T if prefill else 1)
        M = B * T
        Hq, Hkv = cfg.heads, cfg.kv_heads
        self._attn_linear(a, index, "qkv", ("q_proj", "k_proj", "v_proj"), self.qkv,
                          M)(self.aqH, self.asH, M)
        if prefill:
            K.qk_norm_rope(self.qkv, B, T, Hq, Hkv, a.q_norm.weight, a.k_norm.weight, cfg.eps,
                           self.cos, self.sin, self.pos, self.q, self.kc[index], self.vc[index])
            self._prefill_attention(index, T)
            K.act_quant(self.attn, M, self.aqA, self.asA)
        else:
            K.decode_attention_fused(self.qkv, B, Hq, Hkv, a.q_norm.weight, a.k_norm.weight,
                                     cfg.eps, self.cos, self.sin, self.pos, self.kc[index],
                                     self.vc[index], self.work, self.aqA, self.asA)
        self._attn_linear(a, index, "o", ("o_proj",), self.o, M)(self.aqA, self.asA, M)

    def _moe(self, mlp: SparseMoeBlock, index: int, M: int, prefill: bool,
             quantized: bool = False):
        """Routed MLP of the normalized rows hb[:M]; ``quantized``: aqH /
        asH already hold their fp8 form (the norm wrote both)."""
        cfg, r, ex = self.cfg, self.route, self.experts[index]
        if not quantized:
            K.act_quant(self.hb, M, self.aqH, self.asH)  # the experts' input
        fused = ex.tiled and not prefill and M <= 16
        if (prefill or ex.tiled) and (ex.compressed or ex.tiled) and not fused:
            ex.decode_all()
        step = self.chunk if prefill else M
        for c0 in range(0, M, step):
            m = min(step, M - c0)
            K.moe_route(self.hb[c0:c0 + m], mlp.gate.weight, m, r)
            K.moe_group(r, m)
            if ex.compressed and not prefill:
                ex.decode_routed(r.select)
            gu, down = (ex.tiled_gu, ex.tiled_down) if fused else (ex.gu, ex.down)
            # c0 is a multiple of 16: the chunk's rows are whole activation
            # tiles, the same bytes as the row range of a [rows, H] view
            gu(self.aqH[c0:c0 + K.pad16(m)], self.asH[c0:c0 + m], r, gather=True, M=m)
            K.silu_mul_quant(self.gu, m * cfg.top_k, self.hq, self.hs)
            down(self.hq, self.hs, r, gather=False, M=m)
            K.moe_combine(self.down, r, m, self.y[c0:c0 + m])

    def time_linears(self, reps: int = 3) -> dict:
        """Decode-step (M = batch) time of each linear of a layer, on the
        inputs and the routing in the runner's buffers (those of the last
        decode step's last layer, or set by the caller: aqH/asH, aqA/asA,
        hq/hs and ``route``): the linear of every layer launched back to
        back (one HIP graph replayed between one event pair), the best of
        ``reps`` rounds divided by the layer count.
        The grouped expert linears of every layer run the same routing, so
        each reads the weights of the experts that step picked (~88 of 128
        at 16 tokens, ~0.4 GB per layer: the 48 layers stream from HBM as in
        a decode step).  Returns {linear: {"us", "bytes" (weights and scales
        read per layer), "flops"}} for qkv, o, gate_up and down.  FP8
        resident or re-tiled blocks only: blocks decoded by their hooks
        share one buffer."""
        cfg, M, r = self.cfg, self.B, self.route
        layers = list(self.model.model.layers)
        n_active = int(r.n_active.item())
        if n_active <= 0:
            raise ECF8Error("time_linears needs a routed decode step first")
        Hq, D, I = cfg.heads, cfg.head_dim, cfg.moe_intermediate

        def weight_bytes(mod, names):
            tiles = getattr(mod, "_ecf8_tiles", None)
            if tiles is not None:
                return sum(tiles[n].nbytes() + tiles[n].weight_scale.numel() * 4 for n in names)
            return sum(mod.get_submodule(n).weight.numel() +
                       mod.get_submodule(n).weight_scale_inv.numel() * 4 for n in names)

        res = {}
        for which, names, out, aq, as_, k_in in (
                ("qkv", ("q_proj", "k_proj", "v_proj"), self.qkv, self.aqH, self.asH, cfg.hidden),
                ("o", ("o_proj",), self.o, self.aqA, self.asA, Hq * D)):
            calls = []
            for i, layer in enumerate(layers):
                a = layer.self_attn
                if getattr(a, "_ecf8_tiles", None) is None and hasattr(a, "encoded"):
                    raise ECF8Error("blocks decoded by their hooks share one buffer")
                p = self._attn_linear(a, i, which, names, out, M)
                calls.append(lambda p=p: p(aq, as_, M))
            n_out = sum(layers[0].self_attn.get_submodule(n).out_features for n in names)
            res[which] = {"us": round(self._time_launches(calls, reps) * 1e3, 2),
                          "bytes": int(weight_bytes(layers[0].self_attn, names)),
                          "flops": 2 * M * n_out * k_in}
        gu_calls, down_calls = [], []
        for i in range(len(layers)):
            ex = self.experts[i]
            if ex.compressed and not ex.tiled:
                raise ECF8Error("experts decoded per step share one buffer")
            gu, down = (ex.tiled_gu, ex.tiled_down) if ex.tiled else (ex.gu, ex.down)
            gu_calls.append(lambda gu=gu: gu(self.aqH[:K.pad16(M)], self.asH[:M], r, gather=True,
                                             M=M))
            down_calls.append(lambda down=down: down(self.hq, self.hs, r, gather=False, M=M))
        ex0 = layers[0].mlp.experts[0]
        pairs = M * cfg.top_k
        for which, calls, names, flops in (
                ("gate_up", gu_calls, ("gate_proj", "up_proj"), 2 * pairs * 2 * I * cfg.hidden),
                ("down", down_calls, ("down_proj",), 2 * pairs * cfg.hidden * I)):
            res[which] = {"us": round(self._time_launches(calls, reps) * 1e3, 2),
                          "bytes": int(n_active * weight_bytes(ex0, names)), "flops": flops}
        return res

    def layer(self, layer: MoeDecoderLayer, index: int, x_prev, prefill: bool):
        cfg = self.cfg
        M = self.B * (self.T if prefill else 1)
        K.rmsnorm(self.res, layer.input_layernorm.weight, cfg.eps, M, x=x_prev, out_q=self.aqH,
                  out_scale=self.asH)
        layer.self_attn(self, index, prefill)
        # bf16 rows for the router, fp8 rows for the experts, in one pass
        K.rmsnorm(self.res, layer.post_attention_layernorm.weight, cfg.eps, M, x=self.o,
                  out_q=self.aqH, out_scale=self.asH, out_bf16=self.hb)
        self._moe(layer.mlp, index, M, prefill, quantized=True)
        return self.y


# ------------------------------------------------------------ construction


def random_moe_model(cfg: Qwen3MoeConfig, device, distinct_layers: int | None = None,
                     seed: int = 0):
    """Random-init model with synthetic FP8 attention and expert weights
    (N(0, sigma) block-quantized per 128x128 tile); ``distinct_layers``
    draws that many layers and gives every layer its own device copy of
    layer (i mod distinct_layers).  Returns (model, drawn) with drawn[j] =
    {"attn": {...}, "experts": [{...} per expert]} on the host."""
    from .synth import synthetic_block

    n_distinct = cfg.layers if distinct_layers is None else max(1, min(distinct_layers, cfg.layers))
    with torch.device("meta"):
        model = Qwen3MoeForCausalLM(cfg)
    model = model.to_empty(device=device)
    g = torch.Generator(device=device).manual_seed(seed)
    with torch.no_grad():
        model.model.embed_tokens.weight.normal_(0.0, 0.02, generator=g)
        model.lm_head.weight.normal_(0.0, 0.02, generator=g)
        for layer in model.model.layers:
            layer.mlp.gate.weight.normal_(0.0, 0.02, generator=g)
        for mod in model.modules():
            if isinstance(mod, RMSNorm):
                mod.weight.fill_(1.0)
    drawn = []
    for j in range(n_distinct):
        base = seed * 100_000 + j * 1000
        drawn.append({"attn": synthetic_block(cfg.attn_shapes(), seed=base),
                      "experts": [synthetic_block(cfg.expert_shapes(), seed=base + 1 + e)
                                  for e in range(cfg.experts)]})
    for i, layer in enumerate(model.model.layers):
        src = drawn[i % n_distinct]
        targets = [(layer.self_attn, src["attn"])]
        targets += [(ex, w) for ex, w in zip(layer.mlp.experts, src["experts"])]
        for mod, weights in targets:
            for name, (w, s) in weights.items():
                lin = mod.get_submodule(name)
                lin.weight = nn.Parameter(w.to(device, copy=True), requires_grad=False)
                lin.weight_scale_inv = s.to(device, copy=True)
    return model, drawn


def compress_moe_layers(model: Qwen3MoeForCausalLM, drawn=None, threads_per_block: int = 512,
                        bytes_per_thread: int = 8):
    """Compress each layer's attention block and each expert as one block
    (the reference's qwen3moe patterns) and register them through the
    loader's path.  ``drawn`` (from random_moe_model) lets layers that share
    weights share one compression; every layer gets its own device copy."""
    from dfloat.compress import compress_flat
    from dfloat.run.run import _process_compressed_tensor
    from .synth import flat_block

    cache = {}

    def comp_of(key, weights):
        c = cache.get(key) if key is not None else None
        if c is None:
            flat, split = flat_block(weights)
            res = compress_flat(flat, bytes_per_thread, threads_per_block)
            c = {k: res[k] for k in _KEYS}
            c["split_positions"] = torch.tensor(split, dtype=torch.int64)
            if key is not None:
                cache[key] = c
        return c

    def register(mod, path, pattern, comp):
        dev = mod.get_submodule(pattern[next(iter(pattern))][0]).weight_scale_inv.device
        for n in pattern[next(iter(pattern))]:  # the hooks inject row-major views
            mod.get_submodule(n).weight_layout = K.WEIGHT_ROWS
        for attr in (*_KEYS, "split_positions"):
            value = comp[attr] if attr == "split_positions" else comp[attr].to(dev).clone()
            _process_compressed_tensor(mod, attr, value, f"{path}.{attr}", pattern,
                                       threads_per_block, bytes_per_thread)

    for i, layer in enumerate(model.model.layers):
        key = i % len(drawn) if drawn is not None else None
        w_attn = (drawn[key]["attn"] if drawn is not None else
                  {n: layer.self_attn.get_submodule(n).weight.detach().cpu() for n in ATTN_LINEARS})
        register(layer.self_attn, f"model.layers.{i}.self_attn", {ATTN_REGEX: list(ATTN_LINEARS)},
                 comp_of(None if key is None else (key, "attn"), w_attn))
        for e, ex in enumerate(layer.mlp.experts):
            w_ex = (drawn[key]["experts"][e] if drawn is not None else
                    {n: ex.get_submodule(n).weight.detach().cpu() for n in EXPERT_LINEARS})
            register(ex, f"model.layers.{i}.mlp.experts.{e}", {EXPERT_REGEX: list(EXPERT_LINEARS)},
                     comp_of(None if key is None else (key, e), w_ex))
    return model


def retile_moe_layers(model: Qwen3MoeForCausalLM, drawn=None, n_threads: int | None = None):
    """Re-tile every compressed attention block and expert for the fused
    decode step (ecf8_amd.tiled): each block is decoded once on its device,
    its Linears re-encoded under the block's own code into the tiled layout,
    and its reference-layout buffers and decode hook removed.  The decode
    step's attention linears and grouped expert linears then decode their
    weight operands themselves; the prompt decodes the tiled Linears first.
    ``drawn`` (from random_moe_model) lets layers that hold copies of one
    block share one encoding; each layer keeps its own device copy.

    A block the tiled layout cannot hold (LUTs with a 1-bit code, or a
    Linear over 3 bits per exponent in some 16x128 segment) stays compressed
    in the reference layout: an attention block keeps its decode hook, and
    since one grouped launch serves all of a layer's experts, one refused
    expert keeps every expert of its layer on the routed batched decode
    followed by the FP8 grouped linear.  The refused blocks and their reasons
    are returned in ``model._ecf8_untiled`` and printed on stderr; every
    check of a block (or of a layer's experts) runs before any of it
    changes."""
    for i, layer in enumerate(model.model.layers):
        if not hasattr(layer.self_attn, "encoded") or not all(
                hasattr(ex, "encoded") for ex in layer.mlp.experts):
            raise ECF8Error(f"layer {i} holds blocks that are not compressed")
    cache = {}
    untiled = []
    for i, layer in enumerate(model.model.layers):
        key = i % len(drawn) if drawn is not None else None
        got = tiled.tile_block(layer.self_attn, ATTN_LINEARS, cache,
                               None if key is None else (key, "attn"), n_threads)
        if isinstance(got, str):
            untiled.append((f"model.layers.{i}.self_attn", got))
        else:
            tiled.install_tiles(layer.self_attn, ATTN_LINEARS, *got)
        experts, refused = [], None
        for e, ex in enumerate(layer.mlp.experts):
            got = tiled.tile_block(ex, EXPERT_LINEARS, cache,
                                   None if key is None else (key, e), n_threads)
            if isinstance(got, str):
                refused = (f"model.layers.{i}.mlp.experts.{e}", got)
                break
            experts.append(got)
        if refused is not None:
            untiled.append((f"model.layers.{i}.mlp.experts",
                            f"{refused[0]}: {refused[1]}; one grouped launch serves the layer's "
                            "experts, so all of them stay on the routed decode"))
            continue
        for ex, got in zip(layer.mlp.experts, experts):
            tiled.install_tiles(ex, EXPERT_LINEARS, *got)
    tiled.report_untiled(untiled)
    model.__dict__["_ecf8_untiled"] = untiled
    return model
