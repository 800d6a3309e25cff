"""Python wrappers of the consumer kernels (include/ecf8_llm.h): the
block-scaled FP8 linear that reads decoded weights and the fused kernels of
a Qwen3-shaped decoder layer.  Every call launches on torch's current stream
of the tensors' device; shapes, dtypes and contiguity are checked here, the
library checks sizes and alignment again and returns a status."""

from __future__ import annotations

import ctypes

import torch

from ._lib import ECF8Error, check, lib

GROUP = 128
MAX_SEGS = 3
WEIGHT_ROWS, WEIGHT_TILES = 0, 1  # ECF8_WEIGHT_ROWS / ECF8_WEIGHT_TILES


class _Seg(ctypes.Structure):
    _fields_ = [("weight", ctypes.c_void_p), ("weight_scale", ctypes.c_void_p),
                ("n", ctypes.c_int64), ("out_col", ctypes.c_int64),
                ("weight_layout", ctypes.c_int64)]


def pad16(rows: int) -> int:
    """Rows of a tile-layout buffer holding ``rows`` rows."""
    return (int(rows) + 15) // 16 * 16


def to_tiles(x: torch.Tensor) -> torch.Tensor:
    """[R, K] e4m3fn/uint8 row-major -> the tile layout of include/ecf8_llm.h
    as a [pad16(R), K] tensor of the same dtype (pad rows zero): per 16
    rows and 128 columns a 2 KB block, lane l = 16 g + r holding row r's
    bytes [16 g, +16) at 16 l and [64 + 16 g, +16) at 1024 + 16 l."""
    R, K = x.shape
    if K % GROUP:
        raise ECF8Error("the tile layout needs K a multiple of 128")
    b = x.view(torch.uint8)
    Rp = pad16(R)
    if Rp != R:
        b = torch.cat([b, b.new_zeros(Rp - R, K)])
    t = b.reshape(Rp // 16, 16, K // GROUP, 2, 4, 16).permute(0, 2, 3, 4, 1, 5)
    return t.contiguous().view(Rp, K).view(x.dtype)


def from_tiles(t: torch.Tensor, R: int, K: int) -> torch.Tensor:
    """The first R rows of a tile-layout buffer, row-major [R, K]."""
    Rp = pad16(R)
    b = t.reshape(-1).view(torch.uint8)[: Rp * K]
    x = b.view(Rp // 16, K // GROUP, 2, 4, 16, 16).permute(0, 4, 1, 2, 3, 5)
    return x.contiguous().view(Rp, K)[:R].view(t.dtype)


def _act_rows(M, K, t, name):
    """A tile-layout activation buffer ``t`` holds M rows of K columns."""
    if t is not None and (t.dim() != 2 or t.shape[1] != K or t.shape[0] < pad16(M)):
        raise ECF8Error(f"{name} {tuple(t.shape)} is not a tile-layout [>= {pad16(M)}, {K}] "
                        "buffer (rows padded to 16)")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _need(t: torch.Tensor, dtype, name: str, dev=None):
    if not t.is_cuda:
        raise ECF8Error(f"{name} must be a CUDA tensor")
    if dev is not None and t.device != dev:
        raise ECF8Error(f"{name} must be on {dev}")
    if t.dtype != dtype:
        raise ECF8Error(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ECF8Error(f"{name} must be contiguous")


def _ptr(t):
    return None if t is None else t.data_ptr()


def _rows(M, K, *tensors):
    """Every given tensor is 2-D [>= M, K]."""
    for t in tensors:
        if t is not None and (t.dim() != 2 or t.shape[1] != K or t.shape[0] < M):
            raise ECF8Error(f"tensor {tuple(t.shape)} is not [>= {M}, {K}]")


class LinearPlan:
    """Precomputed argument block of one (possibly fused) FP8 linear: the
    segment table is built once, so a call costs one ctypes launch."""

    def __init__(self, weights, out: torch.Tensor):
        """``weights``: list of (weight e4m3fn [n, K], weight_scale_inv f32
        [n/128, K/128]) or (weight, scale, layout) with layout WEIGHT_ROWS
        (row-major, the default) or WEIGHT_TILES (the tile layout, e.g.
        from ``to_tiles``); outputs are written side by side into ``out``
        columns in that order."""
        if not 1 <= len(weights) <= MAX_SEGS:
            raise ECF8Error(f"1..{MAX_SEGS} weight segments per linear")
        dev = out.device
        _need(out, torch.bfloat16, "out", dev)
        K = weights[0][0].shape[1]
        segs = (_Seg * len(weights))()
        col = 0
        for i, entry in enumerate(weights):
            w, s = entry[0], entry[1]
            layout = entry[2] if len(entry) > 2 else WEIGHT_ROWS
            if layout not in (WEIGHT_ROWS, WEIGHT_TILES):
                raise ECF8Error(f"unknown weight layout {layout}")
            _need(w, torch.float8_e4m3fn, "weight", dev)
            _need(s, torch.float32, "weight_scale_inv", dev)
            n, k = w.shape
            if k != K or n % GROUP or K % GROUP:
                raise ECF8Error(f"weight {tuple(w.shape)} does not fit K={K} in 128-multiples")
            if tuple(s.shape) != (n // GROUP, K // GROUP):
                raise ECF8Error(f"weight_scale_inv {tuple(s.shape)} for weight {tuple(w.shape)}")
            segs[i] = _Seg(w.data_ptr(), s.data_ptr(), n, col, layout)
            col += n
        if out.shape[-1] < col:
            raise ECF8Error(f"out has {out.shape[-1]} columns, {col} needed")
        self.segs, self.count, self.K, self.N, self.out, self.ldo = segs, len(weights), K, col, out, out.shape[-1]
        self._keep = [t for entry in weights for t in entry[:2]]

    def __call__(self, aq: torch.Tensor, a_scale: torch.Tensor, M: int):
        """``aq``: quantized activations in the tile layout ([>= pad16(M), K])."""
        _need(aq, torch.float8_e4m3fn, "aq", self.out.device)
        _need(a_scale, torch.float32, "a_scale", self.out.device)
        if (aq.dim() != 2 or aq.shape[1] != self.K or aq.shape[0] < pad16(M)
                or tuple(a_scale.shape[1:]) != (self.K // GROUP,) or a_scale.shape[0] < M):
            raise ECF8Error("activation shape does not match the linear (tile-layout aq has "
                            "rows padded to 16)")
        if self.out.shape[0] < M:
            raise ECF8Error("out has fewer rows than M")
        check(lib().ecf8_fp8_linear(aq.data_ptr(), a_scale.data_ptr(), M, self.K, self.segs,
                                    self.count, self.out.data_ptr(), self.ldo, _stream(aq)),
              "ecf8_fp8_linear")
        return self.out


def fp8_linear(aq, a_scale, weights, out, M=None):
    """One-shot form of LinearPlan: out[:, cols] = aq @ w.T per segment."""
    return LinearPlan(weights, out)(aq, a_scale, aq.shape[0] if M is None else M)


def rmsnorm(residual, weight, eps, M, x=None, out_q=None, out_scale=None, out_bf16=None):
    """residual[:M] += x[:M] (if x); normalized rows -> bf16 and/or fp8 +
    scales (with both, the fp8 form quantizes the bf16-rounded rows)."""
    dev = residual.device
    _need(residual, torch.float32, "residual", dev)
    _need(weight, torch.bfloat16, "weight", dev)
    K = residual.shape[-1]
    if x is not None:
        _need(x, torch.bfloat16, "x", dev)
    if (out_q is None) != (out_scale is None) or (out_bf16 is None and out_q is None):
        raise ECF8Error("rmsnorm needs out_bf16, or out_q and out_scale, or all three")
    if out_bf16 is not None:
        _need(out_bf16, torch.bfloat16, "out_bf16", dev)
    if out_q is not None:
        _need(out_q, torch.float8_e4m3fn, "out_q", dev)
        _need(out_scale, torch.float32, "out_scale", dev)
    _rows(M, K, residual, x, out_bf16)
    _act_rows(M, K, out_q, "out_q")
    _rows(M, K // GROUP, out_scale)
    if weight.numel() != K:
        raise ECF8Error("norm weight shape does not match the rows")
    check(lib().ecf8_rmsnorm(_ptr(x), residual.data_ptr(), weight.data_ptr(), float(eps), M, K,
                             _ptr(out_q), _ptr(out_scale), _ptr(out_bf16), _stream(residual)),
          "ecf8_rmsnorm")


def silu_mul_quant(gate_up, M, out_q, out_scale):
    dev = gate_up.device
    _need(gate_up, torch.bfloat16, "gate_up", dev)
    _need(out_q, torch.float8_e4m3fn, "out_q", dev)
    _need(out_scale, torch.float32, "out_scale", dev)
    inter = gate_up.shape[-1] // 2
    _rows(M, 2 * inter, gate_up)
    _act_rows(M, inter, out_q, "out_q")
    _rows(M, inter // GROUP, out_scale)
    check(lib().ecf8_silu_mul_quant(gate_up.data_ptr(), M, inter, out_q.data_ptr(),
                                    out_scale.data_ptr(), _stream(gate_up)), "ecf8_silu_mul_quant")


def act_quant(x, M, out_q, out_scale):
    dev = x.device
    _need(x, torch.bfloat16, "x", dev)
    _need(out_q, torch.float8_e4m3fn, "out_q", dev)
    _need(out_scale, torch.float32, "out_scale", dev)
    _rows(M, x.shape[-1], x)
    _act_rows(M, x.shape[-1], out_q, "out_q")
    _rows(M, x.shape[-1] // GROUP, out_scale)
    check(lib().ecf8_act_quant(x.data_ptr(), M, x.shape[-1], out_q.data_ptr(), out_scale.data_ptr(),
                               _stream(x)), "ecf8_act_quant")


def qk_norm_rope(qkv, B, T, Hq, Hkv, q_norm, k_norm, eps, cos_t, sin_t, pos, q_out, k_cache,
                 v_cache):
    dev = qkv.device
    for t, n in ((qkv, "qkv"), (q_norm, "q_norm"), (k_norm, "k_norm"), (q_out, "q_out"),
                 (k_cache, "k_cache"), (v_cache, "v_cache")):
        _need(t, torch.bfloat16, n, dev)
    _need(cos_t, torch.float32, "cos", dev)
    _need(sin_t, torch.float32, "sin", dev)
    _need(pos, torch.int32, "pos", dev)
    if pos.numel() < 1 or q_norm.numel() != 128 or k_norm.numel() != 128:
        raise ECF8Error("pos must hold the position; q_norm / k_norm must be [128]")
    Lmax = k_cache.shape[2]
    if tuple(k_cache.shape) != (B, Hkv, Lmax, 128) or k_cache.shape != v_cache.shape:
        raise ECF8Error("caches must be [B, Hkv, Lmax, 128]")
    if q_out.numel() < B * Hq * T * 128 or qkv.numel() < B * T * (Hq + 2 * Hkv) * 128:
        raise ECF8Error("q_out / qkv too small")
    if cos_t.shape != (Lmax, 64) or sin_t.shape != (Lmax, 64):
        raise ECF8Error("rotary tables must be [Lmax, 64]")
    check(lib().ecf8_qk_norm_rope(qkv.data_ptr(), B, T, Hq, Hkv, q_norm.data_ptr(),
                                  k_norm.data_ptr(), float(eps), cos_t.data_ptr(), sin_t.data_ptr(),
                                  pos.data_ptr(), Lmax, q_out.data_ptr(), k_cache.data_ptr(),
                                  v_cache.data_ptr(), _stream(qkv)), "ecf8_qk_norm_rope")


def attention_work(B, Hq, Lmax, device) -> torch.Tensor:
    """Work buffer of both attention forms (split partials)."""
    n = lib().ecf8_attention_work_floats(B, Hq, Lmax)
    if n < 0:
        raise ECF8Error("bad attention work size")
    return torch.zeros(n, dtype=torch.float32, device=device)


def decode_attention(q, k_cache, v_cache, pos, work, out_q, out_scale, Hq, out_bf16=None):
    """q: the first B*Hq*128 elements of ``q`` are [B, Hq, 128]."""
    dev = q.device
    B, Hkv, Lmax, D = k_cache.shape
    if q.numel() < B * Hq * 128:
        raise ECF8Error("q too small")
    for t, n in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _need(t, torch.bfloat16, n, dev)
    _need(pos, torch.int32, "pos", dev)
    if pos.numel() < 1:
        raise ECF8Error("pos must hold the position")
    _need(work, torch.float32, "work", dev)
    _need(out_q, torch.float8_e4m3fn, "out_q", dev)
    _need(out_scale, torch.float32, "out_scale", dev)
    if out_bf16 is not None:
        _need(out_bf16, torch.bfloat16, "out_bf16", dev)
    if D != 128 or v_cache.shape != k_cache.shape:
        raise ECF8Error("caches must be [B, Hkv, Lmax, 128]")
    if (out_q.numel() < pad16(B) * Hq * 128 or out_scale.numel() < B * Hq
            or (out_bf16 is not None and out_bf16.numel() < B * Hq * 128)):
        raise ECF8Error("outputs too small (out_q: tile layout, rows padded to 16)")
    check(lib().ecf8_decode_attention(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                      pos.data_ptr(), B, Hq, Hkv, Lmax, work.data_ptr(),
                                      work.numel(), out_q.data_ptr(), out_scale.data_ptr(),
                                      _ptr(out_bf16), _stream(q)), "ecf8_decode_attention")


def decode_attention_fused(qkv, B, Hq, Hkv, q_norm, k_norm, eps, cos_t, sin_t, pos, k_cache,
                           v_cache, work, out_q, out_scale, out_bf16=None):
    """qk_norm_rope (one new token per sequence) folded into
    decode_attention, same results: q/k/v from the projection output qkv
    [>= B, (Hq + 2*Hkv) * 128], the new token's k/v written to the caches
    at pos[0]."""
    dev = qkv.device
    for t, n in ((qkv, "qkv"), (q_norm, "q_norm"), (k_norm, "k_norm"), (k_cache, "k_cache"),
                 (v_cache, "v_cache")):
        _need(t, torch.bfloat16, n, dev)
    _need(cos_t, torch.float32, "cos", dev)
    _need(sin_t, torch.float32, "sin", dev)
    _need(pos, torch.int32, "pos", dev)
    _need(work, torch.float32, "work", dev)
    _need(out_q, torch.float8_e4m3fn, "out_q", dev)
    _need(out_scale, torch.float32, "out_scale", dev)
    if out_bf16 is not None:
        _need(out_bf16, torch.bfloat16, "out_bf16", dev)
    Lmax = k_cache.shape[2]
    if (tuple(k_cache.shape) != (B, Hkv, Lmax, 128) or v_cache.shape != k_cache.shape
            or cos_t.shape != (Lmax, 64) or sin_t.shape != (Lmax, 64)):
        raise ECF8Error("caches must be [B, Hkv, Lmax, 128], rotary tables [Lmax, 64]")
    if (pos.numel() < 1 or q_norm.numel() != 128 or k_norm.numel() != 128
            or qkv.numel() < B * (Hq + 2 * Hkv) * 128):
        raise ECF8Error("pos, q_norm / k_norm [128] or qkv does not fit")
    if (out_q.numel() < pad16(B) * Hq * 128 or out_scale.numel() < B * Hq
            or (out_bf16 is not None and out_bf16.numel() < B * Hq * 128)):
        raise ECF8Error("outputs too small (out_q: tile layout, rows padded to 16)")
    check(lib().ecf8_decode_attention_fused(
        qkv.data_ptr(), B, Hq, Hkv, q_norm.data_ptr(), k_norm.data_ptr(), float(eps),
        cos_t.data_ptr(), sin_t.data_ptr(), pos.data_ptr(), Lmax, k_cache.data_ptr(),
        v_cache.data_ptr(), work.data_ptr(), work.numel(), out_q.data_ptr(), out_scale.data_ptr(),
        _ptr(out_bf16), _stream(qkv)), "ecf8_decode_attention_fused")


def dequant_fp8_block(weight, scale_inv, out=None):
    """bf16 [n, k] = e4m3fn weight x its 128x128 block scales."""
    dev = weight.device
    _need(weight, torch.float8_e4m3fn, "weight", dev)
    _need(scale_inv, torch.float32, "weight_scale_inv", dev)
    n, k = weight.shape
    if tuple(scale_inv.shape) != (n // GROUP, k // GROUP):
        raise ECF8Error("weight_scale_inv shape does not match the weight")
    if out is None:
        out = torch.empty(n, k, dtype=torch.bfloat16, device=dev)
    _need(out, torch.bfloat16, "out", dev)
    if out.numel() < n * k:
        raise ECF8Error("out too small")
    check(lib().ecf8_dequant_fp8_block(weight.data_ptr(), scale_inv.data_ptr(), n, k,
                                       out.data_ptr(), _stream(weight)), "ecf8_dequant_fp8_block")
    return out.view(-1)[: n * k].view(n, k)


# ------------------------------------------------------------------ MoE


class MoeRouting:
    """Device buffers of one routing step for up to ``M`` tokens
    (``M * top_k <= 8192``): the router's choices, the pairs grouped by
    expert, and the per-expert flags the routed decode takes."""

    def __init__(self, M: int, top_k: int, n_experts: int, device):
        if M * top_k > 8192 or n_experts > 256:
            raise ECF8Error("routing holds at most 8192 (token, expert) pairs and 256 experts")
        P = M * top_k
        i32 = dict(dtype=torch.int32, device=device)
        self.M, self.top_k, self.E = M, top_k, n_experts
        self.logits = torch.zeros(M, n_experts, dtype=torch.float32, device=device)
        self.topk_idx = torch.zeros(M, top_k, **i32)
        self.topk_w = torch.zeros(M, top_k, dtype=torch.float32, device=device)
        self.offsets = torch.zeros(n_experts + 1, **i32)
        self.active = torch.zeros(n_experts, **i32)
        self.n_active = torch.zeros(1, **i32)
        self.pair_tok = torch.zeros(P, **i32)
        self.pair_w = torch.zeros(P, dtype=torch.float32, device=device)
        self.pair_pos = torch.zeros(P, **i32)
        self.select = torch.zeros(n_experts, **i32)


def moe_route(x, router_w, M: int, r: MoeRouting):
    """Router of M tokens: x bf16 [>= M, H], router_w bf16 [E, H]."""
    dev = x.device
    _need(x, torch.bfloat16, "x", dev)
    _need(router_w, torch.bfloat16, "router_w", dev)
    H = x.shape[-1]
    _rows(M, H, x)
    if tuple(router_w.shape) != (r.E, H) or not 1 <= M <= r.M:
        raise ECF8Error(f"router_w must be [{r.E}, {H}] and 1 <= M <= {r.M}")
    check(lib().ecf8_moe_route(x.data_ptr(), router_w.data_ptr(), M, H, r.E, r.top_k,
                               r.logits.data_ptr(), r.topk_idx.data_ptr(), r.topk_w.data_ptr(),
                               _stream(x)), "ecf8_moe_route")


def moe_group(r: MoeRouting, M: int):
    """Group the routed pairs of the first M tokens by expert."""
    if not 1 <= M <= r.M:
        raise ECF8Error(f"1 <= M <= {r.M}")
    check(lib().ecf8_moe_group(r.topk_idx.data_ptr(), r.topk_w.data_ptr(), M, r.top_k, r.E,
                               r.offsets.data_ptr(), r.active.data_ptr(), r.n_active.data_ptr(),
                               r.pair_tok.data_ptr(), r.pair_w.data_ptr(), r.pair_pos.data_ptr(),
                               r.select.data_ptr(), _stream(r.topk_idx)), "ecf8_moe_group")


class MoeLinearPlan:
    """Device address tables of one grouped expert linear: ``experts`` is a
    list (one per expert) of 1..3 segments (weight e4m3fn [seg_n, K],
    weight_scale_inv f32 [seg_n/128, K/128]), e.g. (gate, up) or (down,).
    Segment s of every expert writes output columns [s*seg_n, +seg_n).
    ``weight_layout``: WEIGHT_ROWS (row-major) or WEIGHT_TILES, for every
    expert weight."""

    def __init__(self, experts, out: torch.Tensor, weight_layout: int = WEIGHT_ROWS):
        dev = out.device
        _need(out, torch.bfloat16, "out", dev)
        n_segs = len(experts[0])
        if not 1 <= n_segs <= MAX_SEGS or any(len(e) != n_segs for e in experts):
            raise ECF8Error(f"every expert needs the same 1..{MAX_SEGS} segments")
        seg_n, K = experts[0][0][0].shape
        ws, ss = [], []
        for segs in experts:
            for w, s in segs:
                _need(w, torch.float8_e4m3fn, "weight", dev)
                _need(s, torch.float32, "weight_scale_inv", dev)
                if tuple(w.shape) != (seg_n, K) or tuple(s.shape) != (seg_n // GROUP, K // GROUP):
                    raise ECF8Error(f"expert weight {tuple(w.shape)} / scale {tuple(s.shape)} "
                                    f"do not match [{seg_n}, {K}]")
                ws.append(w.data_ptr())
                ss.append(s.data_ptr())
        if seg_n % GROUP or K % GROUP or out.shape[-1] < n_segs * seg_n:
            raise ECF8Error("seg_n and K must be multiples of 128 and fit out")
        if weight_layout not in (WEIGHT_ROWS, WEIGHT_TILES):
            raise ECF8Error(f"unknown weight layout {weight_layout}")
        self.w_table = torch.tensor(ws, dtype=torch.int64).to(dev)
        self.s_table = torch.tensor(ss, dtype=torch.int64).to(dev)
        self.E, self.n_segs, self.seg_n, self.K, self.out = len(experts), n_segs, seg_n, K, out
        self.weight_layout = int(weight_layout)
        self._keep = [t for segs in experts for pair in segs for t in pair]

    def __call__(self, aq, a_scale, r: MoeRouting, gather: bool, M: int | None = None):
        """``gather``: activation rows are tokens (aq: tile layout,
        [>= pad16(M), K], row of a sorted pair = its token); otherwise aq
        has one row per sorted pair ([>= pad16(M * top_k), K]).  M: the
        tokens routed into ``r`` (default: its capacity)."""
        dev = self.out.device
        _need(aq, torch.float8_e4m3fn, "aq", dev)
        _need(a_scale, torch.float32, "a_scale", dev)
        M = r.M if M is None else M
        if not 1 <= M <= r.M:
            raise ECF8Error(f"1 <= M <= {r.M}")
        P = r.M * r.top_k
        rows = M if gather else M * r.top_k
        if (aq.dim() != 2 or aq.shape[1] != self.K or aq.shape[0] < pad16(rows)
                or tuple(a_scale.shape[1:]) != (self.K // GROUP,) or a_scale.shape[0] < rows
                or self.out.shape[0] < P or r.E != self.E):
            raise ECF8Error("activation / output shape does not match the grouped linear")
        check(lib().ecf8_moe_linear(aq.data_ptr(), a_scale.data_ptr(),
                                    r.pair_tok.data_ptr() if gather else None,
                                    r.offsets.data_ptr(), r.active.data_ptr(), r.n_active.data_ptr(),
                                    self.E, self.w_table.data_ptr(), self.s_table.data_ptr(),
                                    self.n_segs, self.seg_n, self.K, self.weight_layout,
                                    self.out.data_ptr(), self.out.shape[-1], _stream(aq)),
              "ecf8_moe_linear")
        return self.out


def moe_combine(down, r: MoeRouting, M: int, out):
    """out[m] = sum_k w * down[pair of (m, k)] (bf16 [>= M, H])."""
    dev = down.device
    _need(down, torch.bfloat16, "down", dev)
    _need(out, torch.bfloat16, "out", dev)
    H = out.shape[-1]
    if (down.dim() != 2 or down.shape[0] < M * r.top_k or down.shape[1] < H or out.shape[0] < M
            or not 1 <= M <= r.M):
        raise ECF8Error("down / out shape does not match the routing")
    check(lib().ecf8_moe_combine(down.data_ptr(), down.shape[1], r.pair_pos.data_ptr(),
                                 r.pair_w.data_ptr(), M, r.top_k, H, out.data_ptr(), _stream(down)),
          "ecf8_moe_combine")
