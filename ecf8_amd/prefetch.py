"""Double-buffered layer decode on a side stream.

The reference decodes a compressed block inside the block's own
forward-pre-hook, on the compute stream (dfloat/run/run.py:84-155), so every
layer's decode sits between two layers' compute.  On MI355X the decode-step
compute of a layer (small-M FP8 GEMMs, norms, attention) leaves most of the
HBM bandwidth idle, so the decode of layer i+1 runs on a second HIP stream
while layer i computes:

* two decode buffers; layer i reads buffer i % 2, except that with an odd
  layer count the last layer reads a third buffer, so that the decode of
  layer 0 for the next pass (buffer 0) never overwrites the running layer;
* layer i's pre-hook makes the compute stream wait for layer i's decode,
  injects its weight views, then has the side stream wait until the layer
  that last read layer i+1's buffer has released it and decode layer i+1
  into it;
* layer i's post-hook records that its buffer is free again;
* the last layer's pre-hook decodes layer 0 for the next forward pass, and
  its post-hook joins the side stream back into the compute stream, so a
  forward pass (and a HIP graph captured from one) starts and ends with
  buffer 0 holding layer 0.

The side-stream decode runs with a capped grid (``workgroups_per_cu``
resident decode workgroups per CU, through the batched launch's task
split), which leaves CU slots for the compute stream's kernels.  Stream
priorities stay at the default.
"""

from __future__ import annotations

import torch

from . import decode as _dev
from dfloat.run.run import _inject, _module_state

_KEYS = ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps")


class LayerPrefetcher:
    def __init__(self, layers, device=None, workgroups_per_cu: float = 2,
                 threads_per_block: int = 512):
        layers = list(layers)
        if len(layers) < 2:
            raise ValueError("the prefetcher alternates layers over buffers: give at least two layers")
        self.layers = layers
        self.dev = torch.device(device) if device is not None else layers[0].encoded.device
        sizes = [m.packed_other_4bits.numel() * 2 for m in layers]
        self.slot = [i % 2 for i in range(len(layers))]
        if len(layers) % 2:
            self.slot[-1] = 2
        n_bufs = max(self.slot) + 1
        self.bufs = [torch.empty(max(n for n, b in zip(sizes, self.slot) if b == k),
                                 dtype=torch.float8_e4m3fn, device=self.dev)
                     for k in range(n_bufs)]
        self.side = torch.cuda.Stream(self.dev)
        cus = torch.cuda.get_device_properties(self.dev).multi_processor_count
        # fractions below 1 leave some CUs without a decode workgroup
        slots = max(1, int(round(cus * workgroups_per_cu)))
        self.plans, self.views = [], []
        for i, (m, n) in enumerate(zip(layers, sizes)):
            m.__dict__["_ecf8_tpb"] = threads_per_block
            table, max_block, _ = _module_state(m)
            out = self.bufs[self.slot[i]][:n]
            n_fb = _dev.n_format_blocks(m.encoded.numel(), threads_per_block, 8)
            bpt = max(1, -(-n_fb // slots))
            plan = _dev.prepare_batch([{k: getattr(m, k) for k in _KEYS}], [out], [table],
                                      threads_per_block=threads_per_block, blocks_per_task=bpt,
                                      max_block_elements=max_block)
            self.plans.append(plan)
            self.views.append(out)
        self.ready = [torch.cuda.Event() for _ in layers]
        self.free = [torch.cuda.Event() for _ in range(n_bufs)]
        self._released = [False] * n_bufs
        self._handles = []
        self.primed = False

    def _decode(self, i: int):
        """Queue layer i's decode on the side stream, after the buffer it
        writes has been released by the compute stream."""
        main = torch.cuda.current_stream(self.dev)
        b = self.slot[i]
        if self._released[b]:
            self.side.wait_event(self.free[b])
        else:
            self.side.wait_stream(main)
        with torch.cuda.stream(self.side):
            _dev.decode_batched(self.plans[i])
            self.ready[i].record(self.side)

    def prime(self):
        """Decode layer 0 before the first forward pass (joined into the
        compute stream, as at the end of every pass)."""
        self._released = [False] * len(self.bufs)
        self._decode(0)
        torch.cuda.current_stream(self.dev).wait_stream(self.side)
        self.primed = True

    def _pre(self, i: int):
        def hook(module, _):
            main = torch.cuda.current_stream(self.dev)
            if i > 0:  # layer 0 was joined at the end of the previous pass
                main.wait_event(self.ready[i])
            _inject(module, self.views[i])
            nxt = i + 1 if i + 1 < len(self.layers) else 0
            self._decode(nxt)
        return hook

    def _post(self, i: int):
        def hook(module, _args, _out):
            main = torch.cuda.current_stream(self.dev)
            self.free[self.slot[i]].record(main)
            self._released[self.slot[i]] = True
            if i == len(self.layers) - 1:
                main.wait_stream(self.side)  # join: layer 0 is decoded for the next pass
                self._released = [False] * len(self.bufs)
        return hook

    def install(self):
        """Replace each layer's decode hook by the prefetching pair."""
        for i, m in enumerate(self.layers):
            m._forward_pre_hooks.clear()
            self._handles.append(m.register_forward_pre_hook(self._pre(i)))
            self._handles.append(m.register_forward_hook(self._post(i)))
        self.prime()
        return self

    def uninstall(self):
        """Remove the prefetching hooks (the layers are left without a
        decode hook; install another prefetcher or the loader's hooks)."""
        torch.cuda.current_stream(self.dev).wait_stream(self.side)
        for h in self._handles:
            h.remove()
        self._handles = []
