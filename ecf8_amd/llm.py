"""A Qwen3-shaped causal LM whose decoder layers run on the consumer kernels
(ecf8_amd.llm_kernels): the end-to-end check and benchmark of the decode
path, compressed vs uncompressed FP8.

The module tree keeps Hugging Face's Qwen3 names (``model.embed_tokens``,
``model.layers.N.self_attn.q_proj`` ...), so a layer is compressed and
hooked exactly as the reference does it for ``model.layers.N``
(scripts/compress.py:197-247, dfloat/run/run.py:84-155, 406-458): the
forward-pre-hook decodes the layer's block into the shared TensorManager
buffer and injects the seven ``.weight`` views that the layer's FP8
linears then read.  Generation follows scripts/inference_llm.py:108-142:
a batch of prompts, greedy decoding of a fixed number of new tokens,
tokens/s = batch * new tokens / latency, and peak allocated HBM.

Runtime layout: fp32 residual stream; e4m3fn activations with one fp32
scale per row and 128 columns; bf16 projection outputs; per-layer KV caches
bf16 [B, Hkv, Lmax, 128]; the prefill runs eagerly, every decode step is
one HIP graph replay (captured once per runner), with positions held in a
device counter so the same graph serves every step.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import llm_kernels as K
from . import tiled
from ._lib import ECF8Error

LINEAR_NAMES = ("mlp.down_proj", "mlp.gate_proj", "mlp.up_proj", "self_attn.k_proj",
                "self_attn.o_proj", "self_attn.q_proj", "self_attn.v_proj")  # sorted
LAYER_REGEX = r"model\.layers\.\d+"


@dataclass
class Qwen3Config:
    """Qwen3-8B by default."""
    hidden: int = 4096
    intermediate: int = 12288
    layers: int = 36
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    vocab: int = 151936
    rope_theta: float = 1_000_000.0
    eps: float = 1e-6

    def linear_shapes(self) -> dict:
        """{name: (out, in, sigma)}: sigma 0.02 for q/k/v/gate/up and 0.01
        for o/down, the synthetic weight scheme of a Qwen3-8B layer."""
        h, q, kv, i = self.hidden, self.heads * self.head_dim, self.kv_heads * self.head_dim, self.intermediate
        return {"self_attn.q_proj": (q, h, 0.02), "self_attn.k_proj": (kv, h, 0.02),
                "self_attn.v_proj": (kv, h, 0.02), "self_attn.o_proj": (h, q, 0.01),
                "mlp.gate_proj": (i, h, 0.02), "mlp.up_proj": (i, h, 0.02),
                "mlp.down_proj": (h, i, 0.01)}


class FP8Linear(nn.Module):
    """e4m3fn weight [out, in] with fp32 scale_inv per 128x128 block (the
    FP8 checkpoint layout); ``weight`` may be replaced by an injected view.
    ``weight_layout``: K.WEIGHT_ROWS (row-major, as loaded or injected) or
    K.WEIGHT_TILES (re-laid out by ``tile_resident_weights``)."""

    def __init__(self, in_features: int, out_features: int):
        super().__init__()
        self.in_features, self.out_features = in_features, out_features
        self.weight = nn.Parameter(torch.empty(out_features, in_features, dtype=torch.float8_e4m3fn),
                                   requires_grad=False)
        self.register_buffer("weight_scale_inv", torch.ones(
            math.ceil(out_features / 128), math.ceil(in_features / 128), dtype=torch.float32))
        self.weight_layout = K.WEIGHT_ROWS


def weight_layout(lin) -> int:
    """The layout of a Linear's current ``weight`` (row-major unless
    ``tile_resident_weights`` re-laid it out)."""
    return getattr(lin, "weight_layout", K.WEIGHT_ROWS)


def tile_resident_weights(model: nn.Module) -> int:
    """Re-lay every resident FP8 Linear weight of ``model`` out in the tile
    layout of include/ecf8_llm.h (in place: one copy, the same bytes
    reordered), which the FP8 linears read with 1 KB-contiguous loads;
    returns the number of Linears changed.  Compressed blocks (weights
    injected row-major by their decode hooks) are not touched."""
    count = 0
    for mod in model.modules():
        if isinstance(mod, FP8Linear) and "weight" in mod._parameters \
                and weight_layout(mod) == K.WEIGHT_ROWS:
            w = mod.weight
            if w.shape[0] % 16 or w.shape[1] % 128:
                continue
            with torch.no_grad():
                mod.weight = nn.Parameter(K.to_tiles(w.data), requires_grad=False)
            mod.weight_layout = K.WEIGHT_TILES
            count += 1
    return count


class RMSNorm(nn.Module):
    def __init__(self, dim: int):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim, dtype=torch.bfloat16), requires_grad=False)


class Attention(nn.Module):
    def __init__(self, cfg: Qwen3Config):
        super().__init__()
        h, q, kv = cfg.hidden, cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
        self.q_proj, self.k_proj = FP8Linear(h, q), FP8Linear(h, kv)
        self.v_proj, self.o_proj = FP8Linear(h, kv), FP8Linear(q, h)
        self.q_norm, self.k_norm = RMSNorm(cfg.head_dim), RMSNorm(cfg.head_dim)


class MLP(nn.Module):
    def __init__(self, cfg: Qwen3Config):
        super().__init__()
        self.gate_proj = FP8Linear(cfg.hidden, cfg.intermediate)
        self.up_proj = FP8Linear(cfg.hidden, cfg.intermediate)
        self.down_proj = FP8Linear(cfg.intermediate, cfg.hidden)


class DecoderLayer(nn.Module):
    def __init__(self, cfg: Qwen3Config):
        super().__init__()
        self.self_attn, self.mlp = Attention(cfg), MLP(cfg)
        self.input_layernorm = RMSNorm(cfg.hidden)
        self.post_attention_layernorm = RMSNorm(cfg.hidden)

    def forward(self, runner: "Qwen3Runner", index: int, x_prev, prefill: bool):
        # calling the module (not runner.layer directly) runs the decode hook
        return runner.layer(self, index, x_prev, prefill)


class _Model(nn.Module):
    def __init__(self, cfg: Qwen3Config):
        super().__init__()
        self.embed_tokens = nn.Embedding(cfg.vocab, cfg.hidden, dtype=torch.bfloat16)
        self.layers = nn.ModuleList(DecoderLayer(cfg) for _ in range(cfg.layers))
        self.norm = RMSNorm(cfg.hidden)


class Qwen3ForCausalLM(nn.Module):
    def __init__(self, cfg: Qwen3Config):
        super().__init__()
        self.config = cfg
        self.model = _Model(cfg)
        self.lm_head = nn.Linear(cfg.hidden, cfg.vocab, bias=False, dtype=torch.bfloat16)


def _rotary_tables(cfg: Qwen3Config, max_len: int, device):
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2, dtype=torch.float64) / cfg.head_dim))
    ang = torch.arange(max_len, dtype=torch.float64)[:, None] * inv[None, :]
    return (torch.cos(ang).float().to(device).contiguous(),
            torch.sin(ang).float().to(device).contiguous())


class _GreedyRunner:
    """Generation mechanics shared by the dense and the MoE runners: a
    subclass provides ``layer()`` and the buffers named here (``res``, ``h``,
    ``q``, ``kc``/``vc``, ``attn``, ``pos``, ``step``, ``tokens``,
    ``next_tok``); prefill runs eagerly, a decode step can be captured as one
    HIP graph."""

    def _plan(self, layer, index, which, weights, out):
        """Linear argument blocks are cached per (layer, which, weight
        addresses and layouts): injected views of the decode buffer keep
        their addresses from call to call."""
        key = (index, which, tuple((e[0].data_ptr(),) + tuple(e[2:]) for e in weights))
        p = self._plans.get(key)
        if p is None:
            p = K.LinearPlan(weights, out)
            self._plans[key] = p
        return p

    def _time_launches(self, launches, reps: int, warm_ms: float = 40.0) -> float:
        """Best time in ms per launch of ``launches`` (callables, each one
        kernel launch on the current stream) over ``reps`` replays of one
        HIP graph holding them all: a graph, so host launch time cannot
        starve the GPU between these short kernels (a decode step replays a
        graph too).  Before timing, one eager round and back-to-back
        replays for about ``warm_ms`` of sustained load: on MI355X the
        first ~15 ms of such load run up to 8 % slower, and a generation
        runs its steps back to back."""
        dev = self.dev
        for f in launches:
            f()
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for f in launches:
                f()
        stream = torch.cuda.current_stream(dev)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        graph.replay()
        b.record(stream)
        torch.cuda.synchronize(dev)
        for _ in range(min(1000, int(warm_ms / max(a.elapsed_time(b), 1e-3)))):
            graph.replay()
        # the timed replays follow on without a host round trip in between
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        marks[0].record(stream)
        for i in range(reps):
            graph.replay()
            marks[i + 1].record(stream)
        torch.cuda.synchronize(dev)
        del graph
        return min(marks[i].elapsed_time(marks[i + 1]) for i in range(reps)) / len(launches)

    def _prefill_attention(self, index: int, T: int):
        """Causal attention of the prompt in fp32 (torch), positions 0..T-1."""
        cfg = self.cfg
        B, Hq, Hkv = self.B, cfg.heads, cfg.kv_heads
        G = Hq // Hkv
        q = self.q[: B * Hq * T * 128].view(B, Hq, T, 128).float()
        k = self.kc[index][:, :, :T].float().repeat_interleave(G, dim=1)
        v = self.vc[index][:, :, :T].float().repeat_interleave(G, dim=1)
        s = torch.matmul(q, k.transpose(-1, -2).contiguous()) / math.sqrt(128)
        mask = torch.ones(T, T, dtype=torch.bool, device=self.dev).triu(1)
        s.masked_fill_(mask, float("-inf"))
        o = torch.matmul(torch.softmax(s, dim=-1), v)
        self.attn[: B * T].copy_(o.permute(0, 2, 1, 3).reshape(B * T, Hq * 128))

    def _forward(self, prefill: bool):
        """All layers + final norm + lm_head; returns bf16 logits [B, vocab]
        of each sequence's last position."""
        cfg, B = self.cfg, self.B
        T = self.T if prefill else 1
        x = None
        for i, layer in enumerate(self.model.model.layers):
            x = layer(self, i, x, prefill)
        K.rmsnorm(self.res, self.model.model.norm.weight, cfg.eps, B * T, x=x, out_bf16=self.h)
        last = self.h[: B * T].view(B, T, cfg.hidden)[:, T - 1]
        return F.linear(last, self.model.lm_head.weight)

    def prefill(self, prompt: torch.Tensor) -> torch.Tensor:
        """prompt int64 [B, T] -> logits of the last position; sets the
        first generated token and the position counter."""
        B, T = self.B, self.T
        if tuple(prompt.shape) != (B, T):
            raise ECF8Error(f"prompt must be [{B}, {T}]")
        self.pos.zero_()
        self.step.zero_()
        emb = F.embedding(prompt.to(self.dev).reshape(-1), self.model.model.embed_tokens.weight)
        self.res[: B * T].copy_(emb)
        logits = self._forward(True)
        self._emit(logits)
        self.pos.fill_(T)
        return logits

    def _emit(self, logits):
        tok = logits.argmax(dim=-1)
        self.tokens.index_copy_(1, self.step, tok.unsqueeze(1))
        self.next_tok.copy_(tok)
        self.step.add_(1)

    def _decode_body(self):
        emb = F.embedding(self.next_tok, self.model.model.embed_tokens.weight)
        self.res[: self.B].copy_(emb)
        logits = self._forward(False)
        self._emit(logits)
        self.pos.add_(1)
        return logits

    def decode_step(self) -> torch.Tensor:
        """One greedy step, eagerly (hooks and launches from Python)."""
        return self._decode_body()

    def capture(self):
        """Capture one decode step as a HIP graph.  Runs one eager step
        first (it initializes every lazily built state, e.g. each hooked
        layer's decode table), then restores the counters."""
        torch.cuda.synchronize(self.dev)
        pos, step = self.pos.clone(), self.step.clone()
        s = torch.cuda.Stream(self.dev)
        s.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(s):
            self._decode_body()
        torch.cuda.current_stream(self.dev).wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.logits = self._decode_body()
        torch.cuda.synchronize(self.dev)
        self.pos.copy_(pos)
        self.step.copy_(step)
        self.graph = g
        return g

    def generate(self, prompt: torch.Tensor, new_tokens: int) -> torch.Tensor:
        """Greedy generation of ``new_tokens`` tokens per sequence (the
        first from the prefill logits); returns int64 [B, new_tokens]."""
        if new_tokens < 1 or self.T + new_tokens - 1 > self.Lmax:
            raise ECF8Error("new_tokens does not fit the cache")
        self.prefill(prompt)
        for _ in range(new_tokens - 1):
            if self.graph is not None:
                self.graph.replay()  # refreshes self.logits in place
            else:
                self.logits = self._decode_body()
        return self.tokens[:, :new_tokens]


class Qwen3Runner(_GreedyRunner):
    """Prefill + greedy decode of a fixed batch on one device."""

    def __init__(self, model: Qwen3ForCausalLM, batch: int, prompt_len: int, max_len: int,
                 device=None):
        cfg = model.config
        if cfg.hidden != 4096 or cfg.head_dim != 128 or cfg.heads != 4 * cfg.kv_heads:
            raise ECF8Error("the fused kernels need hidden 4096, head_dim 128, heads = 4 kv heads")
        if cfg.intermediate % 4096:
            raise ECF8Error("intermediate size must be a multiple of 4096")
        self.model, self.cfg = model, cfg
        self.dev = torch.device(device) if device is not None else model.lm_head.weight.device
        self.B, self.T, self.Lmax = batch, prompt_len, max_len
        dev, B = self.dev, batch
        M = B * prompt_len
        Hq, Hkv, D = cfg.heads, cfg.kv_heads, cfg.head_dim
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.kc = [torch.empty(B, Hkv, max_len, D, **bf) for _ in range(cfg.layers)]
        self.vc = [torch.empty(B, Hkv, max_len, D, **bf) for _ in range(cfg.layers)]
        self.cos, self.sin = _rotary_tables(cfg, max_len, dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.step = torch.zeros(1, dtype=torch.int64, device=dev)
        self.res = torch.empty(M, cfg.hidden, dtype=torch.float32, device=dev)
        # quantized activations in the tile layout: rows padded to 16
        self.aq = {k: torch.empty(K.pad16(M), k, dtype=torch.float8_e4m3fn, device=dev)
                   for k in sorted({cfg.hidden, cfg.intermediate, Hq * D})}
        self.as_ = {k: torch.empty(M, k // 128, dtype=torch.float32, device=dev) for k in self.aq}
        self.qkv = torch.empty(M, (Hq + 2 * Hkv) * D, **bf)
        self.q = torch.empty(B * Hq * prompt_len * D, **bf)
        self.attn = torch.empty(M, Hq * D, **bf)
        self.o = torch.empty(M, cfg.hidden, **bf)
        self.gu = torch.empty(M, 2 * cfg.intermediate, **bf)
        self.down = torch.empty(M, cfg.hidden, **bf)
        self.h = torch.empty(M, cfg.hidden, **bf)
        self.work = K.attention_work(B, Hq, max_len, dev)
        self.next_tok = torch.zeros(B, dtype=torch.int64, device=dev)
        self.tokens = torch.zeros(B, max_len, dtype=torch.int64, device=dev)
        self.graph = None
        self.logits = None  # logits of the last decode step
        self._plans = {}

    # ------------------------------------------------------------ layer

    def _linear(self, layer, index, which, names, out, M):
        """The linear `which` of a layer: an FP8 plan over the layer's (hook
        injected) weights, or -- for a re-tiled layer -- the tiled linear
        that decodes its weight operands itself (M <= 16) or, for the
        prompt, its Linears decoded into the decode buffer first."""
        tiles = getattr(layer, "_ecf8_tiles", None)
        if tiles is None:
            mods = [layer.get_submodule(n) for n in names]
            return self._plan(layer, index, which,
                              [(x.weight, x.weight_scale_inv, weight_layout(x)) for x in mods], out)
        if M <= 16:
            key = (index, which, "tiled")
            p = self._plans.get(key)
            if p is None:
                p = tiled.TileLinearPlan([tiles[n] for n in names], layer._ecf8_tile_table, out)
                self._plans[key] = p
            return p
        weights = []
        for n in names:
            op = tiles[n]
            buf = self._tile_scratch(op.n * op.k, n)
            tiled.tile_decode(op, layer._ecf8_tile_table, buf)
            weights.append((buf.view(op.n, op.k), op.weight_scale))
        return K.LinearPlan(weights, out)

    def _tile_scratch(self, numel, name):
        """Prompt-time FP8 buffers for re-tiled Linears, one per Linear name
        (reused by every layer: layers run one after another)."""
        if not hasattr(self, "_tile_bufs"):
            self._tile_bufs = {}
        buf = self._tile_bufs.get(name)
        if buf is None or buf.numel() < numel:
            buf = torch.empty(numel, dtype=torch.float8_e4m3fn, device=self.dev)
            self._tile_bufs[name] = buf
        return buf[:numel]

    LINEARS = (("qkv", ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"), "qkv", "H"),
               ("o", ("self_attn.o_proj",), "o", "A"),
               ("gate_up", ("mlp.gate_proj", "mlp.up_proj"), "gu", "H"),
               ("down", ("mlp.down_proj",), "down", "I"))

    def time_linears(self, reps: int = 3, prompt: bool = False) -> dict:
        """Decode-step (M = batch) time of each linear of a layer: the
        linear of every layer launched back to back (one HIP graph replayed
        between one event pair), so the layers' weights stream from HBM as
        in a decode step (36
        Qwen3-8B layers hold 5.8-6.9 GB, far above the 256 MB MALL); the
        best of ``reps`` rounds, divided by the layer count.  Returns
        {linear: {"us": ..., "bytes": weight bytes read per layer,
        "flops": per layer}}.  Runs the FP8 linears of resident weights or
        the tiled linears of re-tiled layers; layers decoded by their hooks
        share one buffer and are not timed this way.  ``prompt``: the
        prompt's GEMMs instead (M = batch x prompt length, resident FP8
        weights only)."""
        cfg, M = self.cfg, (self.B * self.T if prompt else self.B)
        layers = list(self.model.model.layers)
        widths = {"H": cfg.hidden, "A": cfg.heads * cfg.head_dim, "I": cfg.intermediate}
        res = {}
        for which, names, out_name, kin in self.LINEARS:
            K_in = widths[kin]
            out = getattr(self, out_name)
            plans, nbytes = [], 0
            for i, layer in enumerate(layers):
                tiles = getattr(layer, "_ecf8_tiles", None)
                if tiles is None and hasattr(layer, "encoded"):
                    raise ECF8Error("layers decoded by their hooks share one buffer")
                if tiles is not None and M > 16:
                    raise ECF8Error("the prompt's GEMMs of re-tiled layers read decoded scratch")
                plans.append(self._linear(layer, i, which, names, out, M))
                if i == 0:
                    nbytes = (sum(tiles[n].nbytes() + tiles[n].weight_scale.numel() * 4
                                  for n in names) if tiles is not None else
                              sum(layer.get_submodule(n).weight.numel() +
                                  layer.get_submodule(n).weight_scale_inv.numel() * 4
                                  for n in names))
            aq, as_ = self.aq[K_in], self.as_[K_in]
            best = self._time_launches([lambda p=p: p(aq, as_, M) for p in plans], reps)
            n_out = sum(layers[0].get_submodule(n).weight.shape[0] if tiles is None else tiles[n].n
                        for n in names)
            res[which] = {"us": round(best * 1e3, 2), "bytes": int(nbytes),
                          "flops": 2 * M * n_out * K_in}
        return res

    def layer(self, layer: DecoderLayer, index: int, x_prev, prefill: bool):
        cfg = self.cfg
        B, T = self.B, (self.T if prefill else 1)
        M = B * T
        H, I, Hq, Hkv = cfg.hidden, cfg.intermediate, cfg.heads, cfg.kv_heads
        a, m = layer.self_attn, layer.mlp
        aqH, asH = self.aq[H], self.as_[H]
        K.rmsnorm(self.res, layer.input_layernorm.weight, cfg.eps, M, x=x_prev, out_q=aqH,
                  out_scale=asH)
        self._linear(layer, index, "qkv", ("self_attn.q_proj", "self_attn.k_proj",
                                           "self_attn.v_proj"), self.qkv, M)(aqH, asH, M)
        aqA, asA = self.aq[Hq * 128], self.as_[Hq * 128]
        if prefill:
            K.qk_norm_rope(self.qkv, B, T, Hq, Hkv, a.q_norm.weight, a.k_norm.weight, cfg.eps,
                           self.cos, self.sin, self.pos, self.q, self.kc[index], self.vc[index])
            self._prefill_attention(index, T)
            K.act_quant(self.attn, M, aqA, asA)
        else:
            K.decode_attention_fused(self.qkv, B, Hq, Hkv, a.q_norm.weight, a.k_norm.weight,
                                     cfg.eps, self.cos, self.sin, self.pos, self.kc[index],
                                     self.vc[index], self.work, aqA, asA)
        self._linear(layer, index, "o", ("self_attn.o_proj",), self.o, M)(aqA, asA, M)
        K.rmsnorm(self.res, layer.post_attention_layernorm.weight, cfg.eps, M, x=self.o,
                  out_q=aqH, out_scale=asH)
        self._linear(layer, index, "gu", ("mlp.gate_proj", "mlp.up_proj"), self.gu, M)(aqH, asH,
                                                                                       M)
        aqI, asI = self.aq[I], self.as_[I]
        K.silu_mul_quant(self.gu, M, aqI, asI)
        self._linear(layer, index, "down", ("mlp.down_proj",), self.down, M)(aqI, asI, M)
        return self.down


# ------------------------------------------------------------ construction


def random_model(cfg: Qwen3Config, device, distinct_layers: int | None = None, seed: int = 0):
    """A randomly initialized model with synthetic FP8 layer weights
    (N(0, sigma) block-quantized per 128x128 tile).  ``distinct_layers``
    draws that many layers and gives every layer its own copy of layer
    (i mod distinct_layers), which keeps setup time bounded for the full
    36-layer shape while every layer still owns separate memory."""
    from .synth import synthetic_block

    n_distinct = cfg.layers if distinct_layers is None else max(1, min(distinct_layers, cfg.layers))
    with torch.device("meta"):
        model = Qwen3ForCausalLM(cfg)
    model = model.to_empty(device=device)
    g = torch.Generator(device=device).manual_seed(seed)
    with torch.no_grad():
        model.model.embed_tokens.weight.normal_(0.0, 0.02, generator=g)
        model.lm_head.weight.normal_(0.0, 0.02, generator=g)
        for mod in model.modules():
            if isinstance(mod, RMSNorm):
                mod.weight.fill_(1.0)
    shapes = cfg.linear_shapes()
    drawn = [synthetic_block(shapes, seed=seed * 1000 + j) for j in range(n_distinct)]
    for i, layer in enumerate(model.model.layers):
        src = drawn[i % n_distinct]
        for name, (w, s) in src.items():
            lin = layer.get_submodule(name)
            lin.weight = nn.Parameter(w.to(device, copy=True), requires_grad=False)
            lin.weight_scale_inv = s.to(device, copy=True)
    return model, drawn


def compress_layers(model: Qwen3ForCausalLM, drawn=None, threads_per_block: int = 512,
                    bytes_per_thread: int = 8):
    """Compress every decoder layer as one block and install the decode
    hook, through the same registration the checkpoint loader uses
    (dfloat/run/run.py:406-458).  ``drawn`` (from random_model) lets layers
    that share weights share one compression; each layer still gets its own
    device copy of the compressed tensors."""
    from dfloat.compress import compress_flat
    from dfloat.run.run import _process_compressed_tensor
    from .synth import flat_block

    pattern = {LAYER_REGEX: list(LINEAR_NAMES)}
    cache = {}
    for i, layer in enumerate(model.model.layers):
        key = i % len(drawn) if drawn is not None else i
        comp = cache.get(key)
        if comp is None:
            weights = (drawn[key] if drawn is not None else
                       {n: layer.get_submodule(n).weight.detach().cpu() for n in LINEAR_NAMES})
            flat, split = flat_block(weights)  # name-sorted, as the reference flattens
            res = compress_flat(flat, bytes_per_thread, threads_per_block)
            comp = {"luts": res["luts"], "encoded": res["encoded"],
                    "packed_other_4bits": res["packed_other_4bits"],
                    "output_positions": res["output_positions"], "gaps": res["gaps"],
                    "split_positions": torch.tensor(split, dtype=torch.int64)}
            if drawn is not None:
                cache[key] = comp
        dev = layer.self_attn.q_proj.weight_scale_inv.device
        for n in LINEAR_NAMES:  # the hook injects row-major views of the decoded block
            layer.get_submodule(n).weight_layout = K.WEIGHT_ROWS
        for attr in ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps",
                     "split_positions"):
            value = comp[attr] if attr == "split_positions" else comp[attr].to(dev).clone()
            _process_compressed_tensor(layer, attr, value, f"model.layers.{i}.{attr}", pattern,
                                       threads_per_block, bytes_per_thread)
    return model


def retile_layers(model: Qwen3ForCausalLM, drawn=None, n_threads: int | None = None):
    """Re-tile every compressed layer for the fused decode + linear
    (ecf8_amd.tiled): each layer's block is decoded once on its device, each
    of its seven Linears re-encoded under the block's own code into the
    tiled layout, and the block's reference-layout buffers and decode hook
    removed -- the decode step's linears then decode their weight operands
    themselves.  ``drawn`` (from random_model) lets layers that hold copies
    of one block share one encoding; each layer keeps its own device copy.

    A block the tiled layout cannot hold -- LUTs with a 1-bit code (no
    automaton table) or a Linear with a 16x128 segment over 3 bits per
    exponent -- stays as it is, compressed in the reference layout with its
    decode hook, and its linears run decode-then-GEMM; the refused layers
    and their reasons are returned in ``model._ecf8_untiled`` and printed
    on stderr.  Every check of a block runs before any of it changes."""
    for i, layer in enumerate(model.model.layers):
        if not hasattr(layer, "encoded"):
            raise ECF8Error(f"layer {i} holds no compressed block")
    cache = {}
    untiled = []
    for i, layer in enumerate(model.model.layers):
        key = i % len(drawn) if drawn is not None else None
        got = tiled.tile_block(layer, LINEAR_NAMES, cache, key, n_threads)
        if isinstance(got, str):
            untiled.append((f"model.layers.{i}", got))
            continue
        tiled.install_tiles(layer, LINEAR_NAMES, *got)
    tiled.report_untiled(untiled)
    model.__dict__["_ecf8_untiled"] = untiled
    return model


def timed_generate(runner: Qwen3Runner, prompt: torch.Tensor, new_tokens: int):
    """Latency of one generate call (synchronized on both sides), tokens/s
    as scripts/inference_llm.py:126-152 reports it, and peak allocated HBM."""
    dev = runner.dev
    torch.cuda.synchronize(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    t0 = time.perf_counter()
    out = runner.generate(prompt, new_tokens)
    torch.cuda.synchronize(dev)
    latency = time.perf_counter() - t0
    return {"latency_s": latency,
            "tokens_per_s": runner.B * new_tokens / latency,
            "peak_mib": torch.cuda.max_memory_allocated(dev) / 2**20,
            "allocated_mib": torch.cuda.memory_allocated(dev) / 2**20,
            "tokens": out.clone()}
