"""The tiled execution layout ECF8-T (include/ecf8_tile.h) from Python.

A compressed block (one layer, the reference's layout) is re-tiled at load
time, Linear by Linear, under the block's own Huffman code: the symbols of
each 16-row x 128-column tile are reordered into the lanes' MFMA operand
order and cut into 2048-symbol segments.  The decode step's small-M linears
then decode their weight operands themselves (``TileLinearPlan``, the C ABI
``ecf8_tile_linear``), bit-identical to decoding the block and running the
FP8 linear, without writing or re-reading an FP8 copy; the prompt's
large-M linears decode a tiled Linear to row-major FP8 first
(``tile_decode``).

No reference counterpart: the reference decodes every block before its
GEMMs (dfloat/run/run.py:84-155).  The checkpoint and hook layout stays the
reference's; this layout is derived from it in device memory.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

from ._lib import ECF8Error, check, lib

__all__ = ["code_from_luts", "tile_encode", "TiledOperand", "tile_decode", "TileLinearPlan",
           "linear_waves", "TileMoePlan", "TileDecodeBatch", "SEG_SYMBOLS", "tile_block",
           "install_tiles", "report_untiled"]

SEG_SYMBOLS = 2048
_GROUP = 128


class _TileOp(ctypes.Structure):
    _fields_ = [("stream", ctypes.c_void_p), ("seg_off", ctypes.c_void_p),
                ("gaps", ctypes.c_void_p), ("other", ctypes.c_void_p),
                ("weight_scale", ctypes.c_void_p), ("n", ctypes.c_int64),
                ("out_col", ctypes.c_int64)]


def _vp(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def code_from_luts(luts) -> tuple[np.ndarray, np.ndarray]:
    """(code_bits u8[16], code_vals u32[16]) of a block's Huffman code, read
    off its LUT stack (ecf8_code_from_luts)."""
    lut = np.ascontiguousarray(torch.as_tensor(luts).detach().cpu().numpy(), dtype=np.uint8)
    if lut.size % 256:
        raise ECF8Error("luts size is not a multiple of 256")
    bits = np.zeros(16, np.uint8)
    vals = np.zeros(16, np.uint32)
    check(lib().ecf8_code_from_luts(_vp(lut), lut.size // 256, _vp(bits), _vp(vals)),
          "ecf8_code_from_luts")
    return bits, vals


def tile_encode(weight, code_bits, code_vals, n_threads: int | None = None) -> dict:
    """ECF8-T encoding of one FP8 Linear (e4m3fn or uint8 [n, K], any device;
    encoded on the host): {stream, seg_off, gaps, other} as CPU tensors."""
    w = weight.detach()
    if w.dtype == torch.float8_e4m3fn:
        w = w.view(torch.uint8)
    if w.dtype != torch.uint8 or w.dim() != 2:
        raise ECF8Error("weight must be a 2-D e4m3fn or uint8 tensor")
    wn = np.ascontiguousarray(w.cpu().numpy())
    n, k = wn.shape
    bits = np.ascontiguousarray(code_bits, dtype=np.uint8)
    vals = np.ascontiguousarray(code_vals, dtype=np.uint32)
    L = lib()
    nb, ns = ctypes.c_int64(), ctypes.c_int64()
    check(L.ecf8_tile_sizes(_vp(wn), n, k, _vp(bits), ctypes.byref(nb), ctypes.byref(ns)),
          "ecf8_tile_sizes")
    stream = np.empty(nb.value, np.uint8)
    seg_off = np.empty(ns.value + 1, np.uint32)
    gaps = np.empty(ns.value * 8, np.uint32)
    other = np.empty(ns.value * 1024, np.uint8)
    threads = n_threads or min(os.cpu_count() or 1, 16)
    check(L.ecf8_tile_encode(_vp(wn), n, k, _vp(bits), _vp(vals), _vp(stream), nb.value,
                             _vp(seg_off), _vp(gaps), _vp(other), threads), "ecf8_tile_encode")
    return {"stream": torch.from_numpy(stream), "seg_off": torch.from_numpy(seg_off.view(np.int32)),
            "gaps": torch.from_numpy(gaps.view(np.int32)), "other": torch.from_numpy(other)}


class TiledOperand:
    """One tiled Linear on a device: its ECF8-T tensors, its weight scales
    and shape."""

    def __init__(self, enc: dict, weight_scale: torch.Tensor, n: int, k: int, device=None):
        dev = torch.device(device) if device is not None else weight_scale.device
        self.stream = enc["stream"].to(dev)
        self.seg_off = enc["seg_off"].to(dev)
        self.gaps = enc["gaps"].to(dev)
        self.other = enc["other"].to(dev)
        self.weight_scale = weight_scale.to(dev).contiguous()
        self.n, self.k = int(n), int(k)
        if self.n % _GROUP or self.k % _GROUP:
            raise ECF8Error("tiled Linears need 128-multiples")
        if tuple(self.weight_scale.shape) != (self.n // _GROUP, self.k // _GROUP):
            raise ECF8Error("weight_scale does not match the Linear's shape")
        n_seg = (self.n // 16) * (self.k // _GROUP)
        if (self.seg_off.numel() != n_seg + 1 or self.gaps.numel() != 8 * n_seg
                or self.other.numel() != 1024 * n_seg):
            raise ECF8Error("tiled tensors do not match the Linear's shape")
        self.device = dev

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in
                   (self.stream, self.seg_off, self.gaps, self.other))

    def c_struct(self, out_col: int = 0) -> _TileOp:
        return _TileOp(self.stream.data_ptr(), self.seg_off.data_ptr(), self.gaps.data_ptr(),
                       self.other.data_ptr(), self.weight_scale.data_ptr(), self.n, out_col)


def _table_ptr(table, dev):
    data = getattr(table, "data", table)
    if not data.is_cuda or data.device != dev:
        raise ECF8Error(f"the decode table must be on {dev}")
    if getattr(table, "kind", 1) not in (1,):
        raise ECF8Error("tiled decoding needs the block's automaton (ECF8_TABLE_DFA) table")
    return data.data_ptr()


def tile_decode(op: TiledOperand, table, out: torch.Tensor | None = None) -> torch.Tensor:
    """Row-major e4m3fn [n, K] of a tiled Linear (into ``out`` if given)."""
    dev = op.device
    if out is None:
        out = torch.empty(op.n, op.k, dtype=torch.float8_e4m3fn, device=dev)
    if (not out.is_cuda or out.device != dev or out.numel() < op.n * op.k
            or not out.is_contiguous() or out.dtype not in (torch.uint8, torch.float8_e4m3fn)):
        raise ECF8Error("out must be a contiguous e4m3fn/uint8 tensor of n*K elements on the device")
    s = op.c_struct()
    with torch.cuda.device(dev):
        check(lib().ecf8_tile_decode(ctypes.byref(s), op.k, _table_ptr(table, dev), out.data_ptr(),
                                     torch.cuda.current_stream(dev).cuda_stream), "ecf8_tile_decode")
    return out


def linear_waves(n_total: int, k: int, device) -> int:
    """The wave count the FP8 linear uses for M <= 16 at this shape (16 for
    K >= 64 groups, for at most one 16-column tile per CU, or the
    persistent K = 4096 form; else 8): the tiled linear must use the same
    one to sum in the same order."""
    if k // _GROUP >= 64:
        return 16
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    tiles = n_total // 16
    if tiles <= cus or (k == 4096 and tiles > 2 * cus):
        return 16
    return 8


class TileLinearPlan:
    """A (possibly fused) small-M linear over tiled operands written side by
    side into ``out`` (bf16 [rows, ldo]) -- the tiled counterpart of
    llm_kernels.LinearPlan."""

    def __init__(self, ops, table, out: torch.Tensor, waves: int | None = None):
        if not 1 <= len(ops) <= 3:
            raise ECF8Error("1..3 operands per linear")
        dev = out.device
        if out.dtype != torch.bfloat16 or not out.is_cuda or not out.is_contiguous():
            raise ECF8Error("out must be a contiguous bf16 CUDA tensor")
        K = ops[0].k
        arr = (_TileOp * len(ops))()
        col = 0
        for i, op in enumerate(ops):
            if op.k != K or op.device != dev:
                raise ECF8Error("operands differ in K or device")
            arr[i] = op.c_struct(col)
            col += op.n
        if out.shape[-1] < col:
            raise ECF8Error(f"out has {out.shape[-1]} columns, {col} needed")
        self.ops, self.arr, self.K, self.N, self.out = list(ops), arr, K, col, out
        self.ldo = out.shape[-1]
        self.table_ptr = _table_ptr(table, dev)
        self._table = table
        self.waves = waves if waves is not None else linear_waves(col, K, dev)

    def __call__(self, aq: torch.Tensor, a_scale: torch.Tensor, M: int):
        dev = self.out.device
        if (aq.dtype != torch.float8_e4m3fn or a_scale.dtype != torch.float32 or aq.device != dev
                or aq.dim() != 2 or aq.shape[1] != self.K or aq.shape[0] < 16
                or tuple(a_scale.shape[1:]) != (self.K // _GROUP,) or a_scale.shape[0] < M
                or not aq.is_contiguous() or not a_scale.is_contiguous()):
            raise ECF8Error("activation shape does not match the linear (aq: tile layout, "
                            "16 rows)")
        if not 1 <= M <= 16 or self.out.shape[0] < M:
            raise ECF8Error("the tiled linear runs 1..16 rows")
        check(lib().ecf8_tile_linear(aq.data_ptr(), a_scale.data_ptr(), M, self.K, self.arr,
                                     len(self.ops), self.table_ptr, self.out.data_ptr(), self.ldo,
                                     self.waves, torch.cuda.current_stream(dev).cuda_stream),
              "ecf8_tile_linear")
        return self.out


def _device_structs(structs, dev) -> torch.Tensor:
    """A ctypes struct array copied to device memory (8-byte aligned)."""
    raw = ctypes.string_at(ctypes.addressof(structs), ctypes.sizeof(structs))
    return torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(dev)


def _device_ptrs(ptrs, dev) -> torch.Tensor:
    return torch.tensor(list(ptrs), dtype=torch.int64).to(dev)


class TileMoePlan:
    """The grouped expert linear over tiled experts (``ecf8_tile_moe_linear``):
    the tiled counterpart of llm_kernels.MoeLinearPlan.  ``experts`` is a
    list (one per expert) of 1..3 TiledOperands of one shape [seg_n, K]
    (e.g. gate, up); ``tables`` one automaton table per expert (its block's
    code)."""

    def __init__(self, experts, tables, out: torch.Tensor, splits: int = 0):
        dev = out.device
        if out.dtype != torch.bfloat16 or not out.is_cuda or not out.is_contiguous():
            raise ECF8Error("out must be a contiguous bf16 CUDA tensor")
        n_segs = len(experts[0])
        if not 1 <= n_segs <= 3 or any(len(e) != n_segs for e in experts):
            raise ECF8Error("every expert needs the same 1..3 operands")
        if len(tables) != len(experts):
            raise ECF8Error("one table per expert")
        seg_n, K = experts[0][0].n, experts[0][0].k
        arr = (_TileOp * (len(experts) * n_segs))()
        for e, ops in enumerate(experts):
            for j, op in enumerate(ops):
                if (op.n, op.k) != (seg_n, K) or op.device != dev:
                    raise ECF8Error("expert operands differ in shape or device")
                arr[e * n_segs + j] = op.c_struct(j * seg_n)
        if out.shape[-1] < n_segs * seg_n:
            raise ECF8Error(f"out has {out.shape[-1]} columns, {n_segs * seg_n} needed")
        self.ops_dev = _device_structs(arr, dev)
        self.tables_dev = _device_ptrs((_table_ptr(t, dev) for t in tables), dev)
        self._keep = (list(experts), list(tables))
        self.E, self.n_segs, self.seg_n, self.K, self.out = len(experts), n_segs, seg_n, K, out
        self.splits = int(splits)

    def __call__(self, aq, a_scale, r, gather: bool, M: int | None = None):
        """As MoeLinearPlan: ``gather``: activation rows are tokens, else one
        row per sorted pair; M (<= 16): the tokens routed into ``r``."""
        dev = self.out.device
        M = r.M if M is None else M
        if not 1 <= M <= min(r.M, 16):
            raise ECF8Error("the tiled grouped linear runs 1..16 routed tokens")
        rows = M if gather else M * r.top_k
        if (aq.dtype != torch.float8_e4m3fn or a_scale.dtype != torch.float32 or aq.device != dev
                or aq.dim() != 2 or aq.shape[1] != self.K or aq.shape[0] < (rows + 15) // 16 * 16
                or tuple(a_scale.shape[1:]) != (self.K // _GROUP,) or a_scale.shape[0] < rows
                or not aq.is_contiguous() or not a_scale.is_contiguous()
                or self.out.shape[0] < r.M * r.top_k or r.E != self.E):
            raise ECF8Error("activation / output shape does not match the grouped linear")
        check(lib().ecf8_tile_moe_linear(
            aq.data_ptr(), a_scale.data_ptr(), r.pair_tok.data_ptr() if gather else None,
            r.offsets.data_ptr(), r.active.data_ptr(), r.n_active.data_ptr(), self.E,
            self.ops_dev.data_ptr(), self.tables_dev.data_ptr(), self.n_segs, self.seg_n, self.K, M,
            self.out.data_ptr(), self.out.shape[-1], self.splits,
            torch.cuda.current_stream(dev).cuda_stream), "ecf8_tile_moe_linear")
        return self.out


class TileDecodeBatch:
    """``ecf8_tile_decode_batch``: same-shape tiled operands (e.g. one
    projection of every expert) decoded into their row-major FP8 outputs
    in one launch."""

    def __init__(self, ops, tables, outs):
        if not ops or len(tables) != len(ops) or len(outs) != len(ops):
            raise ECF8Error("one table and one output per operand")
        dev = ops[0].device
        n, k = ops[0].n, ops[0].k
        arr = (_TileOp * len(ops))()
        for i, (op, o) in enumerate(zip(ops, outs)):
            if (op.n, op.k) != (n, k) or op.device != dev:
                raise ECF8Error("operands differ in shape or device")
            if (not o.is_cuda or o.device != dev or o.numel() < n * k or not o.is_contiguous()
                    or o.dtype not in (torch.uint8, torch.float8_e4m3fn) or o.data_ptr() % 16):
                raise ECF8Error("each output must be a contiguous, 16-byte aligned e4m3fn/uint8 "
                                "tensor of n*K elements on the device")
            arr[i] = op.c_struct()
        self.ops_dev = _device_structs(arr, dev)
        self.tables_dev = _device_ptrs((_table_ptr(t, dev) for t in tables), dev)
        self.outs_dev = _device_ptrs((o.data_ptr() for o in outs), dev)
        self._keep = (list(ops), list(tables), list(outs))
        self.n_ops, self.n, self.k, self.device = len(ops), n, k, dev

    def __call__(self):
        with torch.cuda.device(self.device):
            check(lib().ecf8_tile_decode_batch(
                self.ops_dev.data_ptr(), self.tables_dev.data_ptr(), self.outs_dev.data_ptr(),
                self.n_ops, self.n, self.k, torch.cuda.current_stream(self.device).cuda_stream),
                "ecf8_tile_decode_batch")


# ------------------------------------------------- re-tiling compressed blocks

_BLOCK_KEYS = ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps",
               "split_positions")


def tile_block(mod, names, cache: dict | None = None, key=None, n_threads: int | None = None):
    """Re-tile one compressed block (a module holding the reference-layout
    buffers and ``weight_injection_modules``) without changing it.

    Returns (encodings {Linear name: tile_encode result}, automaton table)
    or, when the tiled layout cannot hold the block, the reason as a string:
    LUTs with a 1-bit code (no automaton table), or a Linear whose 16x128
    segment needs more than 64 chunks (over 3 bits per exponent).
    ``cache`` / ``key``: blocks with equal contents share one encoding (or
    one refusal)."""
    from ._lib import ECF8_TABLE_DFA
    from .decode import build_table, decode

    table = build_table(mod.luts.contiguous())
    if table.kind != ECF8_TABLE_DFA:
        return "its LUTs hold a 1-bit code, which the tiled decode's automaton cannot take"
    enc = cache.get(key) if cache is not None and key is not None else None
    if enc is None:
        flat = decode(mod.luts, mod.encoded, mod.packed_other_4bits, mod.output_positions,
                      mod.gaps).cpu()
        enc = {}
        try:
            bits, vals = code_from_luts(mod.luts)
            for sub, part in zip(mod.weight_injection_modules,
                                 torch.tensor_split(flat, mod.split_positions)):
                name = next(n for n in names if mod.get_submodule(n) is sub)
                enc[name] = tile_encode(part.view(sub.out_features, sub.in_features), bits, vals,
                                        n_threads)
        except ECF8Error as e:
            enc = f"the tiled layout cannot hold a Linear of the block ({e})"
        if cache is not None and key is not None:
            cache[key] = enc
    return enc if isinstance(enc, str) else (enc, table)


def install_tiles(mod, names, enc: dict, table) -> None:
    """Give a block its tiled Linears (from ``tile_block``) on its device
    and drop its reference-layout buffers, decode hook and injected views.
    The device copies are made before anything of the block changes."""
    dev = mod.encoded.device
    tiles = {}
    for n in names:
        sub = mod.get_submodule(n)
        tiles[n] = TiledOperand(enc[n], sub.weight_scale_inv, sub.out_features, sub.in_features,
                                dev)
    mod._ecf8_tiles = tiles
    mod._ecf8_tile_table = table
    mod._forward_pre_hooks.clear()
    for n in names:  # weight views a decode hook injected earlier
        mod.get_submodule(n).__dict__.pop("weight", None)
    for attr in _BLOCK_KEYS:
        if attr in mod._buffers:
            del mod._buffers[attr]
    mod.__dict__.pop("_ecf8_state", None)
    mod.__dict__.pop("_ecf8_launch", None)


def report_untiled(untiled) -> None:
    """One stderr line per block left on decode-then-GEMM."""
    import sys

    for name, reason in untiled:
        print(f"[ecf8] {name} stays decode-then-GEMM: {reason}", file=sys.stderr)
