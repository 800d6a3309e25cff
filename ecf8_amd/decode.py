"""Device-side decode API over libecf8 (torch tensors in, torch tensors out).

Tensors supply device memory and the stream; the work runs in the HIP
kernels of libecf8.  Shapes and dtypes are checked on the host before every
launch, and any failure raises ``ECF8Error`` -- there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
from typing import NamedTuple

import numpy as np
import torch

from ._lib import (ECF8_MAX_LUTS, ECF8_TABLE_ANY, ECF8_TABLE_BYTES, ECF8_TABLE_DFA,
                   ECF8_TABLE_MULTI, ECF8Error, check, lib)

__all__ = ["DecodeTable", "build_table", "build_table_host", "decode_into", "decode",
           "decode_batched", "prepare_batch", "BatchPlan",
           "n_format_blocks", "largest_block", "min_code_bits", "validate_format", "ECF8Error",
           "ECF8_TABLE_ANY", "ECF8_TABLE_MULTI", "ECF8_TABLE_DFA"]


class DecodeTable(NamedTuple):
    """A derived decode table on the device and its kind (ECF8_TABLE_DFA or
    ECF8_TABLE_MULTI, which selects the decode kernel, or ECF8_TABLE_ANY when
    the kind is only known on the device)."""

    data: torch.Tensor
    kind: int


def _stream_handle(device: torch.device, stream=None):
    s = torch.cuda.current_stream(device) if stream is None else stream
    return s.cuda_stream


def n_format_blocks(n_bytes: int, threads_per_block: int = 512, bytes_per_thread: int = 8) -> int:
    fb = threads_per_block * bytes_per_thread
    return (int(n_bytes) + fb - 1) // fb


def _n_luts(luts: torch.Tensor) -> int:
    if luts.ndim == 2:
        if luts.shape[1] != 256:
            raise ECF8Error(f"luts must be [n_luts, 256], got {tuple(luts.shape)}")
        return int(luts.shape[0])
    if luts.numel() % 256:
        raise ECF8Error("luts size is not a multiple of 256")
    return luts.numel() // 256


def _op_entries(op: torch.Tensor) -> int:
    if op.dtype == torch.uint8:
        if op.numel() % 8:
            raise ECF8Error("output_positions byte view is not a multiple of 8")
        return op.numel() // 8
    if op.dtype in (torch.uint64, torch.int64):
        return op.numel()
    raise ECF8Error(f"output_positions must be u64 (or its u8 view), got {op.dtype}")


def largest_block(output_positions) -> int:
    """Largest output_positions[b+1] - output_positions[b] of a block (the
    quantity the reference turns into shared_mem_size, run.py:453-458).
    Reads the positions on the host; call once per block, not per decode."""
    op = torch.as_tensor(output_positions).detach().contiguous()
    if op.dtype != torch.uint8:
        op = op.view(torch.uint8)
    op = op.cpu().numpy().view(np.uint64).astype(np.int64)
    return int((op[1:] - op[:-1]).max()) if op.size > 1 else 0


def min_code_bits(luts) -> int:
    """Shortest nonzero code length in a LUT stack's length row (its last
    row); 0 if the row is empty.  Reads the LUTs on the host: call once per
    block, not per decode."""
    row = torch.as_tensor(luts).detach().reshape(-1, 256)[-1].cpu().numpy()
    nz = row[row > 0]
    return int(nz.min()) if nz.size else 0


def build_table_host(luts, kind: int = ECF8_TABLE_ANY):
    """Derived decode table for a LUT stack, built on the host: (u32 numpy
    array of ECF8_TABLE_BYTES, kind).  ``kind`` ECF8_TABLE_ANY picks the byte
    automaton when the LUTs allow it, else the multi-symbol table."""
    lut = np.ascontiguousarray(torch.as_tensor(luts).detach().cpu().numpy(), dtype=np.uint8)
    if lut.size % 256:
        raise ECF8Error("luts size is not a multiple of 256")
    n_luts = lut.size // 256
    table = np.zeros(ECF8_TABLE_BYTES // 4, np.uint32)
    got = ctypes.c_int(-1)
    check(lib().ecf8_build_table_host(lut.ctypes.data_as(ctypes.c_void_p), n_luts, int(kind),
                                      table.ctypes.data_as(ctypes.c_void_p), ctypes.byref(got)),
          "ecf8_build_table_host")
    return table, got.value


def build_table(luts: torch.Tensor, out: torch.Tensor | None = None, stream=None,
                kind: int = ECF8_TABLE_ANY, sync: bool = True) -> DecodeTable:
    """Derived decode table for ``luts`` (a CUDA tensor), built on its
    device by the table kernel (into ``out`` if given) on ``stream``.

    ``sync=True`` reads the kind back (one stream synchronization: call once
    per compressed block, at load time) so that decodes launch only the
    kernel for that kind.  ``sync=False`` stays asynchronous -- nothing
    returns to the host, so the call can be graph-captured -- and the
    table's kind is ECF8_TABLE_ANY: decodes then read it on the device."""
    if not luts.is_cuda or luts.dtype != torch.uint8 or not luts.is_contiguous():
        raise ECF8Error("luts must be a contiguous uint8 CUDA tensor")
    n_luts = _n_luts(luts)
    if not 2 <= n_luts <= ECF8_MAX_LUTS:
        raise ECF8Error(f"n_luts={n_luts} outside [2, {ECF8_MAX_LUTS}]")
    if not sync and kind == ECF8_TABLE_DFA:
        raise ECF8Error("an automaton-only table needs sync=True to report a refusal")
    if out is None:
        out = torch.empty(ECF8_TABLE_BYTES // 4, dtype=torch.int32, device=luts.device)
    elif (out.numel() * out.element_size() < ECF8_TABLE_BYTES or out.device != luts.device
          or not out.is_contiguous() or out.data_ptr() % 4):
        raise ECF8Error("table buffer too small, misaligned or on another device")
    got = ctypes.c_int(-1)
    with torch.cuda.device(luts.device):
        check(lib().ecf8_build_table(luts.data_ptr(), n_luts, int(kind), out.data_ptr(),
                                     ctypes.byref(got) if sync else None,
                                     _stream_handle(luts.device, stream)), "ecf8_build_table")
    return DecodeTable(out, got.value if sync else ECF8_TABLE_ANY)


def decode_into(out: torch.Tensor, luts: torch.Tensor, encoded: torch.Tensor,
                packed_other_4bits: torch.Tensor, output_positions: torch.Tensor,
                gaps: torch.Tensor, table: torch.Tensor | None = None,
                threads_per_block: int = 512, bytes_per_thread: int = 8,
                n_elements: int | None = None, max_block_elements: int = 0,
                min_code_bits: int = 0, stream=None) -> torch.Tensor:
    """Decode one compressed block into ``out`` (uint8 / e4m3fn, >= n elements).

    ``max_block_elements`` (see largest_block()) and ``min_code_bits`` (see
    min_code_bits()) size the kernel's LDS; 0 assumes the worst case, which
    is always correct but lowers occupancy."""
    dev = encoded.device
    tensors = {"luts": luts, "encoded": encoded, "packed_other_4bits": packed_other_4bits,
               "output_positions": output_positions, "gaps": gaps, "out": out}
    for name, t in tensors.items():
        if not t.is_cuda or t.device != dev:
            raise ECF8Error(f"{name} must be on {dev}")
        if not t.is_contiguous():
            raise ECF8Error(f"{name} must be contiguous")
    for name in ("luts", "encoded", "packed_other_4bits", "gaps"):
        if tensors[name].dtype != torch.uint8:
            raise ECF8Error(f"{name} must be uint8, got {tensors[name].dtype}")
    if out.dtype not in (torch.uint8, torch.float8_e4m3fn):
        raise ECF8Error(f"out must be uint8 or float8_e4m3fn, got {out.dtype}")
    n = packed_other_4bits.numel() * 2 if n_elements is None else int(n_elements)
    if n > packed_other_4bits.numel() * 2 or n % 2:
        raise ECF8Error("n_elements must be even and covered by packed_other_4bits")
    if out.numel() < n:
        raise ECF8Error(f"out holds {out.numel()} elements, {n} needed")
    n_bytes = encoded.numel()
    n_fb = n_format_blocks(n_bytes, threads_per_block, bytes_per_thread)
    if n_fb and gaps.numel() != n_fb * threads_per_block // 2:
        raise ECF8Error(f"gaps has {gaps.numel()} bytes, expected {n_fb * threads_per_block // 2}")
    if n_fb and _op_entries(output_positions) != n_fb + 1:
        raise ECF8Error(f"output_positions has {_op_entries(output_positions)} entries, "
                        f"expected {n_fb + 1}")
    n_luts = _n_luts(luts)
    if table is None:
        table = build_table(luts, stream=stream)
    elif not isinstance(table, DecodeTable):
        raise ECF8Error("table must be the DecodeTable returned by build_table")
    if table.data.device != dev:
        raise ECF8Error(f"table must be on {dev}")
    with torch.cuda.device(dev):
        check(lib().ecf8_decode(luts.data_ptr(), encoded.data_ptr(),
                                packed_other_4bits.data_ptr(), output_positions.data_ptr(),
                                gaps.data_ptr(), out.data_ptr(), n_luts, n_bytes, n,
                                int(max_block_elements), int(min_code_bits), table.data.data_ptr(),
                                int(table.kind), threads_per_block, bytes_per_thread,
                                _stream_handle(dev, stream)), "ecf8_decode")
    return out


# ecf8_scaled_part (include/ecf8.h): scale pointer, start, rows, cols
SCALED_PART_DTYPE = np.dtype([("scale", "<u8"), ("start", "<i8"), ("rows", "<i8"),
                              ("cols", "<i8")])
assert SCALED_PART_DTYPE.itemsize == 32
MAX_SCALED_PARTS = 16


class Bf16Decode:
    """One block's ecf8_decode_bf16 call with every argument checked and
    packed once (prepare_bf16); calling it launches the decode on the
    current stream of the block's device, or on ``stream``.  Holds the
    tensors it points to.  Valid while those tensors stay where they are."""

    def __init__(self, dev, args, keep):
        self.dev, self._args, self._keep = dev, args, keep
        self._fn = lib().ecf8_decode_bf16

    def __call__(self, stream=None):
        rc = self._fn(*self._args, _stream_handle(self.dev, stream))
        if rc:
            check(rc, "ecf8_decode_bf16")


def prepare_bf16(out: torch.Tensor, luts: torch.Tensor, encoded: torch.Tensor,
                 packed_other_4bits: torch.Tensor, output_positions: torch.Tensor,
                 gaps: torch.Tensor, parts, table: "DecodeTable | None" = None,
                 max_block_elements: int = 0) -> Bf16Decode:
    """Check and pack one ecf8_decode_bf16 call (see decode_bf16) for
    repeated launches: a hook that decodes the same block every step pays
    the checks once."""
    dev = encoded.device
    tensors = {"luts": luts, "encoded": encoded, "packed_other_4bits": packed_other_4bits,
               "output_positions": output_positions, "gaps": gaps, "out": out}
    for name, t in tensors.items():
        if not t.is_cuda or t.device != dev:
            raise ECF8Error(f"{name} must be on {dev}")
        if not t.is_contiguous():
            raise ECF8Error(f"{name} must be contiguous")
    if out.dtype != torch.bfloat16:
        raise ECF8Error(f"out must be bfloat16, got {out.dtype}")
    n = packed_other_4bits.numel() * 2
    if out.numel() < n:
        raise ECF8Error(f"out holds {out.numel()} elements, {n} needed")
    parts = list(parts)
    if not 1 <= len(parts) <= MAX_SCALED_PARTS:
        raise ECF8Error(f"1..{MAX_SCALED_PARTS} parts needed, got {len(parts)}")
    rec = np.zeros(len(parts), dtype=SCALED_PART_DTYPE)
    scales = []
    for j, (start, rows, cols, scale) in enumerate(parts):
        if scale.dtype != torch.float32 or not scale.is_contiguous() or scale.device != dev:
            raise ECF8Error("each part's scale must be a contiguous float32 tensor on the device")
        if tuple(scale.shape) != (int(rows) // 128, int(cols) // 128):
            raise ECF8Error(f"part {j}: scale shape {tuple(scale.shape)} does not match "
                            f"[{rows} / 128, {cols} / 128]")
        rec[j] = (scale.data_ptr(), int(start), int(rows), int(cols))
        scales.append(scale)
    if table is None:
        table = build_table(luts)
    elif not isinstance(table, DecodeTable):
        raise ECF8Error("table must be the DecodeTable returned by build_table")
    args = (luts.data_ptr(), encoded.data_ptr(), packed_other_4bits.data_ptr(),
            output_positions.data_ptr(), gaps.data_ptr(), out.data_ptr(), _n_luts(luts),
            encoded.numel(), n, int(max_block_elements), table.data.data_ptr(), int(table.kind),
            rec.ctypes.data, len(parts), 512, 8)
    keep = (luts, encoded, packed_other_4bits, output_positions, gaps, out, table, rec, scales)
    return Bf16Decode(dev, args, keep)


def decode_bf16(out: torch.Tensor, luts: torch.Tensor, encoded: torch.Tensor,
                packed_other_4bits: torch.Tensor, output_positions: torch.Tensor,
                gaps: torch.Tensor, parts, table: "DecodeTable | None" = None,
                max_block_elements: int = 0, stream=None) -> torch.Tensor:
    """Decode one compressed block straight into the bf16 weights of its
    block-scaled FP8 Linears (ecf8_decode_bf16): ``out`` (bfloat16, >= n
    elements) receives bf16(fp8 x scale) for every element, the bytes
    ecf8_decode followed by dequant_fp8_block on each Linear's view would
    give.  ``parts``: (start, rows, cols, weight_scale_inv) per Linear, in
    the block's element order (start = its split position).  Threads per
    block 512, automaton tables only."""
    prepare_bf16(out, luts, encoded, packed_other_4bits, output_positions, gaps, parts,
                 table=table, max_block_elements=max_block_elements)(stream)
    return out


# ecf8_block_desc (include/ecf8.h): 7 device pointers, n_bytes, n_elements,
# n_luts, task_begin
BLOCK_DESC_DTYPE = np.dtype([
    ("luts", "<u8"), ("encoded", "<u8"), ("packed_other_4bits", "<u8"),
    ("output_positions", "<u8"), ("gaps", "<u8"), ("outputs", "<u8"), ("table", "<u8"),
    ("n_bytes", "<i8"), ("n_elements", "<i8"), ("n_luts", "<i4"), ("task_begin", "<i4")])
assert BLOCK_DESC_DTYPE.itemsize == 80


class BatchPlan:
    """Device descriptors for one batched decode (ecf8_decode_batched),
    built once by prepare_batch and replayed by decode_batched: the tensors
    they point to must stay alive and in place while the plan is used."""

    def __init__(self, descs, count, n_tasks, blocks_per_task, cap, threads_per_block,
                 singles, keep, desc_blocks=()):
        self.descs = descs            # u8 device tensor of ecf8_block_desc
        self.count = count
        self.n_tasks = n_tasks
        self.blocks_per_task = blocks_per_task
        self.cap = cap
        self.threads_per_block = threads_per_block
        self.singles = singles        # decode_into argument tuples of unbatched blocks
        self.desc_blocks = list(desc_blocks)  # index (in the blocks given) of each descriptor
        self.n_blocks = count + len(singles)
        self._keep = keep             # the referenced tensors


def prepare_batch(blocks, outs, tables, threads_per_block: int = 512, bytes_per_thread: int = 8,
                  blocks_per_task: int | None = None, max_block_elements=None) -> BatchPlan:
    """Plan a batched decode of many compressed blocks on one device (e.g.
    the experts of an MoE layer): checks every block as decode_into does,
    uploads the descriptors once, and picks blocks_per_task so that the work
    splits into about eight tasks per resident workgroup.

    ``blocks``: dicts with the block tensors (``luts``, ``encoded``,
    ``packed_other_4bits``, ``output_positions``, ``gaps``); ``outs``: one
    output tensor per block; ``tables``: one DecodeTable per block.  Blocks
    whose table is not an automaton, or that are too small for the batched
    kernel, are decoded one by one with decode_into.  ``max_block_elements``
    bounds every block's largest format-block (None: read on the host)."""
    if not (len(blocks) == len(outs) == len(tables)):
        raise ECF8Error("blocks, outs and tables differ in length")
    keys = ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps")
    dev, rows, singles, largest, desc_blocks = None, [], [], 0, []
    for i, (b, out, t) in enumerate(zip(blocks, outs, tables)):
        enc = b["encoded"]
        n = b["packed_other_4bits"].numel() * 2
        dev = enc.device if dev is None else dev
        if not isinstance(t, DecodeTable):
            raise ECF8Error("tables must be DecodeTables returned by build_table")
        if (t.kind != ECF8_TABLE_DFA or enc.numel() < 12 or n < 16 or bytes_per_thread != 8):
            singles.append(((out, *(b[k] for k in keys)), t))
            continue
        _check_block(out, b, t, n, threads_per_block, bytes_per_thread, dev)
        desc_blocks.append(i)
        rows.append((b["luts"].data_ptr(), enc.data_ptr(), b["packed_other_4bits"].data_ptr(),
                     b["output_positions"].data_ptr(), b["gaps"].data_ptr(), out.data_ptr(),
                     t.data.data_ptr(), enc.numel(), n, _n_luts(b["luts"]), 0))
        if max_block_elements is None:
            largest = max(largest, largest_block(b["output_positions"]))
    descs = np.zeros(len(rows), BLOCK_DESC_DTYPE)
    for i, r in enumerate(rows):
        descs[i] = r
    n_fb = -(-descs["n_bytes"] // (threads_per_block * bytes_per_thread))
    if blocks_per_task is None:
        # Eight tasks per resident workgroup (6 format-blocks per task for a
        # Qwen3-30B-A3B-shaped layer) rather than four (12): the whole layer
        # decodes as fast (234.9 against 235.3 us on MI355X), and a routed
        # selection (BatchSelect keeps this split) fills more of the grid:
        # one token's experts 27.8 against 36.3 us, sixteen tokens' 156.9
        # against 161.3 us.  Four format-blocks per task is slower for the
        # whole layer (238.6 us: more table loads per byte decoded).
        slots = 8 * _resident_workgroups(dev) if rows else 1
        blocks_per_task = int(min(64, max(2, -(-int(n_fb.sum()) // slots))))
    if blocks_per_task < 1:
        raise ECF8Error("blocks_per_task must be >= 1")
    n_task = -(-n_fb // blocks_per_task)
    if rows:
        descs["task_begin"] = np.concatenate([[0], np.cumsum(n_task)[:-1]])
    d_descs = torch.from_numpy(descs.view(np.uint8).copy()).to(dev) if rows else None
    cap = int(max_block_elements) if max_block_elements is not None else largest
    return BatchPlan(d_descs, len(rows), int(n_task.sum()), blocks_per_task, cap,
                     threads_per_block, singles, (list(blocks), list(outs), list(tables)),
                     desc_blocks)


def _resident_workgroups(dev) -> int:
    """CUs x 4: the 512-lane automaton kernel keeps 4 workgroups per CU."""
    return torch.cuda.get_device_properties(dev).multi_processor_count * 4


def decode_batched(plan, outs=None, tables=None, stream=None, **kwargs):
    """Run a BatchPlan (one launch plus the unbatched blocks).  For
    convenience, ``decode_batched(blocks, outs, tables, ...)`` prepares the
    plan first (prepare_batch's keyword arguments apply)."""
    if not isinstance(plan, BatchPlan):
        plan = prepare_batch(plan, outs, tables, **kwargs)
    for args, t in plan.singles:
        decode_into(*args, table=t, threads_per_block=plan.threads_per_block, stream=stream)
    if plan.count:
        dev = plan.descs.device
        with torch.cuda.device(dev):
            check(lib().ecf8_decode_batched(plan.descs.data_ptr(), plan.count, plan.n_tasks,
                                            plan.blocks_per_task, plan.cap,
                                            plan.threads_per_block, _stream_handle(dev, stream)),
                  "ecf8_decode_batched")
    return plan


class BatchSelect:
    """Decode a device-chosen subset of a BatchPlan's blocks per call
    (ecf8_decode_batched_select): e.g. the experts the router picked, from a
    flags tensor (int32, one per block in the order given to prepare_batch)
    that the model writes on the device.  Allocates its work descriptors
    once; a call reads nothing back to the host, so it can be captured in a
    HIP graph and replayed with new flags.

    Blocks outside the batched kernel (a multi-symbol table, or under 16
    elements) cannot be chosen on the device without a host read: they are
    decoded on every call, selected or not, so a selected one is always
    current (an unselected one's output is rewritten with the same bytes)."""

    def __init__(self, plan: BatchPlan):
        if not plan.n_blocks:
            raise ECF8Error("empty plan")
        self.plan = plan
        dev = (plan.descs.device if plan.count else plan.singles[0][0][1].device)
        self.work = torch.empty_like(plan.descs) if plan.count else None
        self.counts = torch.zeros(2, dtype=torch.int32, device=dev)
        # flags per block -> flags per descriptor, when some blocks are not in
        # the batched launch
        self.index = (torch.tensor(plan.desc_blocks, dtype=torch.int64, device=dev)
                      if plan.singles and plan.count else None)

    def __call__(self, select: torch.Tensor, stream=None):
        p = self.plan
        dev = self.counts.device
        if (not select.is_cuda or select.device != dev or select.dtype != torch.int32
                or not select.is_contiguous() or select.numel() < p.n_blocks):
            raise ECF8Error(f"select must be a contiguous int32 tensor of >= {p.n_blocks} "
                            f"flags on {dev}")
        for args, t in p.singles:
            decode_into(*args, table=t, threads_per_block=p.threads_per_block, stream=stream)
        if not p.count:
            return
        flags = select
        if self.index is not None:
            s = torch.cuda.current_stream(dev) if stream is None else stream
            with torch.cuda.stream(s):
                flags = select.index_select(0, self.index)
        with torch.cuda.device(dev):
            check(lib().ecf8_decode_batched_select(p.descs.data_ptr(), p.count, flags.data_ptr(),
                                                   self.work.data_ptr(), self.counts.data_ptr(),
                                                   p.blocks_per_task, p.cap, p.threads_per_block,
                                                   _stream_handle(dev, stream)),
                  "ecf8_decode_batched_select")


def _check_block(out, b, t, n, threads_per_block, bytes_per_thread, dev):
    for name in ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps"):
        v = b[name]
        if not v.is_cuda or v.device != dev or not v.is_contiguous():
            raise ECF8Error(f"{name} must be a contiguous tensor on {dev}")
    if not out.is_cuda or out.device != dev or out.numel() < n or out.dtype not in (
            torch.uint8, torch.float8_e4m3fn):
        raise ECF8Error("out must be a uint8/e4m3fn tensor on the blocks' device holding n")
    if t.data.device != dev:
        raise ECF8Error(f"table must be on {dev}")
    n_fb = n_format_blocks(b["encoded"].numel(), threads_per_block, bytes_per_thread)
    if b["gaps"].numel() != n_fb * threads_per_block // 2:
        raise ECF8Error("gaps size does not match the bitstream")
    if _op_entries(b["output_positions"]) != n_fb + 1:
        raise ECF8Error("output_positions size does not match the bitstream")
    if (b["encoded"].data_ptr() & 15 or b["packed_other_4bits"].data_ptr() & 7
            or out.data_ptr() & 15 or t.data.data_ptr() & 3 or b["output_positions"].data_ptr() & 7):
        raise ECF8Error("misaligned device buffer")
    if b["encoded"].numel() > 2**31 - 65 or n > 2**31 - 65:
        raise ECF8Error("block too large for 32-bit positions")


def decode(luts, encoded, packed_other_4bits, output_positions, gaps, table=None,
           threads_per_block=512, bytes_per_thread=8, max_block_elements=None,
           min_code_bits=None, stream=None) -> torch.Tensor:
    """Decode one compressed block into a new e4m3fn tensor (derives
    max_block_elements and min_code_bits on the host when not given)."""
    n = packed_other_4bits.numel() * 2
    out = torch.empty(n, dtype=torch.float8_e4m3fn, device=encoded.device)
    if max_block_elements is None:
        max_block_elements = largest_block(output_positions)
    if min_code_bits is None:
        min_code_bits = globals()["min_code_bits"](luts)
    return decode_into(out, luts, encoded, packed_other_4bits, output_positions, gaps, table,
                       threads_per_block, bytes_per_thread,
                       max_block_elements=max_block_elements, min_code_bits=min_code_bits,
                       stream=stream)


def validate_format(luts, encoded_bytes: int, packed_other_4bits_bytes: int, output_positions,
                    gaps_bytes: int, threads_per_block: int = 512, bytes_per_thread: int = 8):
    """Host-side format check of one compressed block (libecf8
    ecf8_validate_format); raises ECF8Error with the reason."""
    luts_np = np.ascontiguousarray(torch.as_tensor(luts).cpu().numpy().reshape(-1), dtype=np.uint8)
    op = torch.as_tensor(output_positions).cpu().contiguous()
    op_np = np.ascontiguousarray(op.view(torch.uint8).numpy()).view(np.uint64)
    msg = ctypes.create_string_buffer(256)
    rc = lib().ecf8_validate_format(
        luts_np.ctypes.data_as(ctypes.c_void_p), luts_np.size // 256, int(encoded_bytes),
        int(packed_other_4bits_bytes), op_np.ctypes.data_as(ctypes.c_void_p), op_np.size,
        int(gaps_bytes), 2 * int(packed_other_4bits_bytes), threads_per_block, bytes_per_thread,
        msg, 256)
    if rc != 0:
        raise ECF8Error(f"invalid compressed block: {msg.value.decode()}")
