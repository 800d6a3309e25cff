"""ECF8 decode benchmark on one MI355X.

Default workload (--workload qwen3-8b-layer): one Qwen3-8B-shaped decoder
layer's seven FP8 e4m3fn linears (q/k/v/o/gate/up/down, 192,937,984
elements), synthetic N(0, sigma) weights block-quantized per 128x128 tile,
compressed as ONE block exactly as the reference compresses a
`model.layers.N` block.  A step is one decode of the whole layer (one kernel
launch) from HBM-resident compressed tensors into an FP8 buffer.
Inputs/outputs rotate over several copies so the 256 MB Infinity Cache
cannot serve a step from the previous one.

--workload qwen3-moe-layer: one Qwen3-30B-A3B-shaped MoE layer, the
attention block plus 128 expert blocks each compressed on its own, decoded
by ONE batched launch (ecf8_decode_batched) per step.

Prints ONE JSON line: decode GB/s of algorithmic bytes
(compressed bytes read + FP8 bytes written) over the K timed steps, the
roofline of the decode kernel against the 8 TB/s HBM peak from the
per-launch duration (launches timed one by one), the CPU decode baseline
(the C restatement of the decode rule in oracle/) timed on this host, and
-- for the default workload -- the end-to-end half of the metric in an
``e2e`` object: tokens/s and peak HBM of the Qwen3-8B-shaped model at batch
16 (128 + 1024 tokens) and of the Qwen3-30B-A3B-shaped MoE (128 + 512),
FP8 resident vs ECF8, each run in a child process after the timed region.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

HBM_PEAK_GBPS = 8000.0
FP8_PEAK_TFLOPS = 5000.0  # MI355X dense FP8 MFMA
REPO = os.path.dirname(os.path.abspath(__file__))


def algorithmic_bytes(n_elements: int, n_bytes: int, n_luts: int, tpb: int = 512, bpt: int = 8):
    """Bytes a decode must move: encoded + sign/mantissa nibbles + gaps +
    output positions + LUTs read, FP8 bytes written."""
    n_fb = -(-n_bytes // (tpb * bpt))
    reads = n_bytes + n_elements // 2 + n_fb * tpb // 2 + 8 * (n_fb + 1) + 256 * n_luts
    return reads + n_elements, reads, n_elements


def _traffic_from_profile(name):
    """HBM bytes per launch from the committed rocprofv3 counter summary
    profiles/<name>, if present (line `traffic_bytes_per_launch: <int>`)."""
    path = os.path.join(REPO, "profiles", name)
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", open(path).read())
    return int(m.group(1)) if m else None


def cpu_baseline(block, n_elements, alg_bytes, repeats=3):
    """The oracle's C decoder (single-threaded per format-block range, ranges
    spread over up to 16 host cores) on the same compressed layer."""
    import numpy as np

    from oracle import native

    # the host share of one GPU is 16 cores; never spread wider than that
    threads = min(os.cpu_count() or 1, 16)
    args = [block[k].numpy() for k in ("luts", "encoded", "packed_other_4bits",
                                        "output_positions", "gaps")]
    out = np.empty(n_elements, np.uint8)
    native.decode(*args, threads=threads, out=out)  # warm-up (page-in)
    best = float("inf")
    for _ in range(repeats):
        t0 = time.perf_counter()
        native.decode(*args, threads=threads, out=out)
        best = min(best, time.perf_counter() - t0)
    return {
        "value": round(alg_bytes / best / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"whole layer ({n_elements} elements), best of {repeats} decodes, "
                  f"C restatement of dfloat/run/decode.cu over {threads} threads",
    }


def cpu_encode(flat, seed: int = 0):
    """CPU encode timings (the reference's CPU path is its encoder,
    dfloat/utils.py:373-499): the product's C++ encoder (ecf8_encode_exponents,
    one thread) over the whole layer, and the oracle's per-symbol Python
    restatement of the reference loop over the 4096x4096 tensor the
    reference's CPU case names (seeded N(0, 0.02), 128x128 block scales),
    whose output the C decoder then checks against the original bytes."""
    import numpy as np
    import torch

    from dfloat.compress import compress_flat
    from ecf8_amd.synth import synthetic_fp8
    from oracle import codec as oc
    from oracle import native

    n = flat.numel()
    t0 = time.perf_counter()
    compress_flat(flat)  # split + counts + codebook + LUTs + C++ bitstream encoder
    full = time.perf_counter() - t0
    w, _ = synthetic_fp8(4096, 4096, 0.02, seed=seed)
    part = w.reshape(-1).view(torch.uint8).numpy()
    t0 = time.perf_counter()
    blk = oc.compress_block(part)
    py = time.perf_counter() - t0
    back = native.decode(*(blk[k] for k in ("luts", "encoded", "packed_other_4bits",
                                            "output_positions", "gaps")))
    return {
        "product_cpp": {"value": round(n / full / 1e6, 2), "unit": "M elements/s",
                        "cores": torch.get_num_threads(),
                        "sample": f"whole layer ({n} elements): split and counts (torch, "
                                  f"{torch.get_num_threads()} threads), codebook, LUTs, bitstream "
                                  f"(C++ encoder, 1 thread), {full:.2f} s"},
        "reference_loop_python": {"value": round(part.size / py / 1e6, 4), "unit": "M elements/s",
                                  "cores": 1, "kind": "port",
                                  "sample": f"4096x4096 seeded N(0, 0.02) tensor ({part.size} "
                                            f"elements), per-symbol Python restatement of "
                                            f"dfloat/utils.py:373-499, {py:.2f} s",
                                  "round_trip_bit_exact": bool(np.array_equal(back, part))},
    }


CEILING_SIZES = {  # bytes streamed by one launch, named for the decode path's launches
    "o_proj 4096x4096": 4096 * 4096,
    "qkv 6144x4096": 6144 * 4096,
    "down 4096x12288": 4096 * 12288,
    "gate_up 24576x4096": 24576 * 4096,
    "qwen3-8b layer": 192937984,
}


def stream_ceiling(steps, warmup):
    """What one launch of a plain streaming kernel reaches on this GPU, per
    size the decode path streams: a read-only sweep and a copy
    (ecf8_stream_probe) over every grid (1, 2, 4, 8 workgroups per CU),
    workgroup size (256, 512, 1024 lanes), loads in flight per lane (1, 2,
    4, 8) and load/store hint (plain, non-temporal); each size rotates over
    enough buffers (>= 2 GiB) that the 256 MB MALL cannot serve a launch
    from an earlier one.  Prints the best configuration per size and op."""
    import torch

    from ecf8_amd._lib import check, lib

    dev = torch.device("cuda", 0)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    L = lib()
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    hs = torch.cuda.current_stream(dev).cuda_stream
    results, every = {}, []
    for name, nbytes in CEILING_SIZES.items():
        n_buf = max(2, -(-(2 << 30) // nbytes))
        srcs = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(n_buf)]
        dsts = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(n_buf)]
        for t in srcs:
            t.random_(0, 256)
        per_op = {}
        for op, op_name in ((0, "read"), (1, "copy")):
            best = None
            for wpc in (1, 2, 4, 8):
                for block in (256, 512, 1024):
                    for depth in (1, 2, 4, 8):
                        for nt in (0, 1):
                            grid = cus * wpc

                            def launch(i):
                                check(L.ecf8_stream_probe(op, srcs[i % n_buf].data_ptr(),
                                                          dsts[i % n_buf].data_ptr(), nbytes,
                                                          grid, block, depth, nt,
                                                          sink.data_ptr(), hs),
                                      "ecf8_stream_probe")

                            for i in range(warmup):
                                launch(i)
                            a = torch.cuda.Event(enable_timing=True)
                            b = torch.cuda.Event(enable_timing=True)
                            torch.cuda.synchronize()
                            a.record()
                            for i in range(steps):
                                launch(warmup + i)
                            b.record()
                            torch.cuda.synchronize()
                            us = a.elapsed_time(b) / steps * 1e3
                            moved = nbytes * (1 if op == 0 else 2)
                            cand = {"us": round(us, 2), "tb_per_s": round(moved / us / 1e6, 3),
                                    "workgroups_per_cu": wpc, "block": block,
                                    "loads_in_flight_per_lane": depth,
                                    "nontemporal": bool(nt)}
                            if best is None or us < best["us"]:
                                best = cand
                            every.append([op_name, name, wpc, block, depth, nt, round(us, 2)])
            per_op[op_name] = best
            print(f"[ceiling] {name}: {op_name} best {best}", file=sys.stderr, flush=True)
        results[name] = {"bytes": nbytes, **per_op}
        del srcs, dsts
        torch.cuda.empty_cache()
    line = {"metric": "one-launch streaming ceiling per size (read-only sweep and copy)",
            "unit": "us per launch", "steps": steps, "warmup": warmup, "cus": cus,
            "ceiling": results,
            "sweep_columns": ["op", "size", "workgroups_per_cu", "block",
                              "loads_in_flight_per_lane", "nontemporal", "us"],
            "sweep": every}
    print(json.dumps(line), flush=True)


def copy_calibration(steps, warmup):
    """A plain device-to-device copy of known size (1 GiB read + 1 GiB
    written per launch): the reference point for scaling the HBM counters
    and the practical bandwidth ceiling of a streaming kernel."""
    import torch

    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(warmup):
        dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    print(json.dumps({"mode": "copy", "bytes_read": n, "bytes_written": n, "ms_per_copy": ms,
                      "GBps_read_plus_write": round(2 * n / ms / 1e6, 1)}), flush=True)


def _qwen3_layer_workload(args, dev):
    """One Qwen3-8B-shaped layer as one compressed block: returns the
    per-copy C-ABI calls, a verifier and the figures for the JSON line."""
    import torch

    from ecf8_amd._lib import lib
    from dfloat.compress import compress_flat
    from ecf8_amd.decode import build_table, decode_into, largest_block, min_code_bits
    from ecf8_amd.synth import flat_block, qwen3_8b_layer

    t0 = time.time()
    flat, _ = flat_block(qwen3_8b_layer(seed=args.seed))
    block = compress_flat(flat)
    n = flat.numel()
    print(f"[bench] compressed layer: {n} elements -> {block['encoded'].numel()} bitstream bytes "
          f"in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    n_luts = block["luts"].shape[0]
    alg, _, _ = algorithmic_bytes(n, block["encoded"].numel(), n_luts)
    keys = ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps")
    max_block = largest_block(block["output_positions"])
    min_bits = min_code_bits(block["luts"])
    sets = []
    for _ in range(args.copies):
        d = {k: block[k].contiguous().to(dev) for k in keys}
        d["table"] = build_table(d["luts"])
        d["out"] = torch.empty(n, dtype=torch.float8_e4m3fn, device=dev)
        sets.append(d)
    torch.cuda.synchronize()
    # first decode of every set through the checked API, then straight C-ABI
    # calls with the same arguments so host overhead cannot starve the queue
    for d in sets:
        decode_into(d["out"], d["luts"], d["encoded"], d["packed_other_4bits"],
                    d["output_positions"], d["gaps"], table=d["table"],
                    max_block_elements=max_block, min_code_bits=min_bits)
    L = lib()
    hstream = torch.cuda.current_stream(dev).cuda_stream
    calls = [(L.ecf8_decode, (d["luts"].data_ptr(), d["encoded"].data_ptr(),
                              d["packed_other_4bits"].data_ptr(), d["output_positions"].data_ptr(),
                              d["gaps"].data_ptr(), d["out"].data_ptr(), n_luts,
                              d["encoded"].numel(), n, max_block, min_bits,
                              d["table"].data.data_ptr(), d["table"].kind, 512, 8, hstream))
             for d in sets]
    if args.call_form == "reference":
        # each step as the reference's callers launch the kernel
        # (dfloat/run/run.py:104-119): dfloat.run._decode, which checks its
        # cached table against the LUTs on the device before the decode
        from dfloat.run.run import _decode

        def ref_call(d):
            kw = dict(grid=(-(-d["encoded"].numel() // 4096),), block=(512,),
                      shared_mem=512 * 4 + 4 + max_block,
                      args=[d["luts"].data_ptr(), d["encoded"].data_ptr(),
                            d["packed_other_4bits"].data_ptr(), d["output_positions"].data_ptr(),
                            d["gaps"].data_ptr(), d["out"].data_ptr(), n_luts,
                            d["encoded"].numel(), n])
            return lambda: (_decode(**kw), 0)[1]

        calls = [(ref_call(d), ()) for d in sets]
        for fn, _ in calls:  # each set's table cache filled before timing
            fn()
        torch.cuda.synchronize()

    def verify():
        # every rotated set: each decoded the timed launches' bytes
        want = flat.view(torch.uint8).to(dev)
        return all(torch.equal(d["out"].view(torch.uint8), want) for d in sets)

    config = {
        "workload": "qwen3-8b-layer-decode",
        "elements": n,
        "linears": "q,k,v,o,gate,up,down (one compressed block)",
        "bitstream_bytes": block["encoded"].numel(),
        "algorithmic_bytes": alg,
        "rotated_copies": args.copies,
        "threads_per_block": 512,
        "bytes_per_thread": 8,
        "table_kind": "dfa" if sets[0]["table"].kind == 1 else "multi",
    }
    if args.call_form == "reference":
        config["workload"] = "qwen3-8b-layer-decode-reference-call-form"
        config["call_form"] = ("dfloat.run._decode(grid=, block=, shared_mem=, args=[...]): "
                               "table-cache check kernel + decode kernel per step")
    return calls, verify, alg, n, config, (block, n, flat)


def _flux_block_bf16_workload(args, dev):
    """One FLUX.1-dev double block (8 Linears, 226.5 M elements) as one
    compressed block, decoded straight into its Linears' bf16 weights
    (ecf8_decode_bf16: fp8 x 128x128 block scale, round to nearest even)."""
    import torch

    from dfloat.compress import compress_flat
    from ecf8_amd.decode import build_table, largest_block, prepare_bf16
    from ecf8_amd.dit import FluxConfig
    from ecf8_amd.synth import flat_block, synthetic_block

    t0 = time.time()
    weights = synthetic_block(FluxConfig().double_shapes(), seed=args.seed + 1)
    flat, split = flat_block(weights)
    block = compress_flat(flat)
    n = flat.numel()
    names = sorted(weights)
    starts = [0] + list(split)
    print(f"[bench] compressed FLUX double block: {n} elements -> {block['encoded'].numel()} "
          f"bitstream bytes in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    n_luts = block["luts"].shape[0]
    _, reads, _ = algorithmic_bytes(n, block["encoded"].numel(), n_luts)
    scale_bytes = sum(weights[k][1].numel() * 4 for k in names)
    alg = reads + scale_bytes + 2 * n  # bf16 written
    keys = ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps")
    max_block = largest_block(block["output_positions"])
    sets = []
    for _ in range(args.copies):
        d = {k: block[k].contiguous().to(dev) for k in keys}
        d["table"] = build_table(d["luts"])
        d["out"] = torch.empty(n, dtype=torch.bfloat16, device=dev)
        parts = [(st, weights[k][0].shape[0], weights[k][0].shape[1], weights[k][1].to(dev))
                 for st, k in zip(starts, names)]
        d["call"] = prepare_bf16(d["out"], *(d[k] for k in keys), parts, table=d["table"],
                                 max_block_elements=max_block)
        sets.append(d)
    torch.cuda.synchronize()
    calls = [(lambda c=d["call"]: (c(), 0)[1], ()) for d in sets]

    def verify():
        ref = torch.cat([(w.float() * s.repeat_interleave(128, 0).repeat_interleave(128, 1))
                         .to(torch.bfloat16).reshape(-1) for w, s in (weights[k] for k in names)])
        want = ref.view(torch.int16).to(dev)
        return all(torch.equal(d["out"].view(torch.int16), want) for d in sets)

    config = {
        "workload": "flux-double-block-bf16-decode",
        "elements": n,
        "linears": ", ".join(names) + " (one compressed block)",
        "bitstream_bytes": block["encoded"].numel(),
        "algorithmic_bytes": alg,
        "rotated_copies": args.copies,
        "threads_per_block": 512,
        "bytes_per_thread": 8,
        "output": "bf16 = fp8 x 128x128 block scale (the DiT Linears' weights)",
    }
    return calls, verify, alg, n, config, None


def _qwen3_moe_layer_workload(args, dev):
    """One Qwen3-30B-A3B-shaped MoE layer: the attention block and all 128
    expert blocks (each compressed on its own, as the reference's qwen3moe
    patterns cut them), decoded by one batched launch."""
    import torch

    from ecf8_amd._lib import lib
    from dfloat.compress import compress_flat
    from ecf8_amd.decode import build_table, prepare_batch
    from ecf8_amd.synth import QWEN3_MOE_ATTN, QWEN3_MOE_EXPERT, flat_block, synthetic_block

    t0 = time.time()
    flats = [flat_block(synthetic_block(QWEN3_MOE_ATTN, args.seed))[0]]
    flats += [flat_block(synthetic_block(QWEN3_MOE_EXPERT, args.seed + 1 + e))[0]
              for e in range(128)]
    comp = [compress_flat(f) for f in flats]
    n = sum(f.numel() for f in flats)
    alg = sum(algorithmic_bytes(f.numel(), c["encoded"].numel(), c["luts"].shape[0])[0]
              for f, c in zip(flats, comp))
    print(f"[bench] compressed moe layer: {len(flats)} blocks, {n} elements in "
          f"{time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    keys = ("luts", "encoded", "packed_other_4bits", "output_positions", "gaps")
    plans, out_sets = [], []
    copies = max(1, min(args.copies, 2))
    for _ in range(copies):
        blocks = [{k: c[k].contiguous().to(dev) for k in keys} for c in comp]
        tables = [build_table(b["luts"]) for b in blocks]
        outs = [torch.empty(f.numel(), dtype=torch.float8_e4m3fn, device=dev) for f in flats]
        out_sets.append(outs)
        plans.append(prepare_batch(blocks, outs, tables))
    torch.cuda.synchronize()
    assert all(not p.singles for p in plans)
    L = lib()
    hstream = torch.cuda.current_stream(dev).cuda_stream
    calls = [(L.ecf8_decode_batched, (p.descs.data_ptr(), p.count, p.n_tasks, p.blocks_per_task,
                                      p.cap, 512, hstream)) for p in plans]
    routed = None
    if args.routed_tokens:
        # decode only the attention block and the experts a top-k router
        # picks for `routed_tokens` tokens (uniform random routing, 8
        # routings rotated), selected on the device
        from ecf8_amd.decode import BatchSelect

        rng = torch.Generator().manual_seed(args.seed + 3)
        per_block = [algorithmic_bytes(f.numel(), c["encoded"].numel(), c["luts"].shape[0])[0]
                     for f, c in zip(flats, comp)]
        sels = [BatchSelect(p) for p in plans]
        flag_sets, alg_sets, n_sel = [], [], []
        for _ in range(8):
            picked = torch.stack([torch.randperm(128, generator=rng)[: args.top_k]
                                  for _ in range(args.routed_tokens)]).unique()
            flags = torch.zeros(len(flats), dtype=torch.int32)
            flags[0] = 1
            flags[1 + picked] = 1
            flag_sets.append(flags.to(dev))
            alg_sets.append(sum(b for b, f in zip(per_block, flags.tolist()) if f))
            n_sel.append(int(flags.sum()) - 1)
        calls = []
        for i in range(8):
            sel = sels[i % len(sels)]
            calls.append((lambda f, sel=sel: (sel(f), 0)[1], (flag_sets[i],)))
        alg = sum(alg_sets) // len(alg_sets)
        routed = {"tokens": args.routed_tokens, "top_k": args.top_k,
                  "experts_decoded_mean": round(sum(n_sel) / len(n_sel), 1),
                  "algorithmic_bytes_mean": alg}

    def verify():
        wants = [f.view(torch.uint8).to(dev) for f in flats]
        if routed is not None:
            # one routed call per rotated set on sentinel-filled outputs: the
            # selected blocks decode exactly, the others are untouched
            ok = True
            for i, (outs, sel) in enumerate(zip(out_sets, sels)):
                for o in outs:
                    o.view(torch.uint8).fill_(0x3C)
                sel(flag_sets[i])
                torch.cuda.synchronize()
                for o, w, s_ in zip(outs, wants, flag_sets[i].tolist()):
                    got = o.view(torch.uint8)
                    ok &= torch.equal(got, w) if s_ else bool((got == 0x3C).all())
            return ok
        # every rotated set, each written by the timed launches
        return all(torch.equal(o.view(torch.uint8), w)
                   for outs in out_sets for o, w in zip(outs, wants))

    config = {
        "workload": "qwen3-moe-layer-decode",
        "elements": n,
        "blocks": len(flats),
        "linears": "attention q,k,v,o + 128 experts x gate,up,down (one block each)",
        "algorithmic_bytes": alg,
        "rotated_copies": copies,
        "blocks_per_task": plans[0].blocks_per_task,
        "tasks": plans[0].n_tasks,
        "threads_per_block": 512,
        "bytes_per_thread": 8,
    }
    if routed is not None:
        config["workload"] = "qwen3-moe-layer-routed-decode"
        config["routed"] = routed
        config["algorithmic_bytes"] = alg
    return calls, verify, alg, n, config, None


def e2e_generate(args):
    """Qwen3-8B-shaped causal LM (36 layers, random init, FP8 linears with
    128x128 block scales; embedding and lm_head bf16), batch 16, random
    prompts of 128 tokens, greedy decoding of --new-tokens tokens: first
    with the FP8 weights resident, then with every layer ECF8-compressed and
    decoded by its forward-pre-hook before the layer's FP8 linears run.
    Both runs use the same engine (eager prefill, one HIP graph replay per
    decode step) and must produce identical tokens."""
    import torch

    from ecf8_amd.llm import (Qwen3Config, Qwen3Runner, compress_layers, random_model,
                              retile_layers, tile_resident_weights, timed_generate)
    from ecf8_amd.prefetch import LayerPrefetcher
    from dfloat.run.run import TensorManager

    dev = torch.device("cuda", 0)
    cfg = Qwen3Config()
    B, T, new = args.batch, args.prompt_len, args.new_tokens
    t0 = time.time()
    model, drawn = random_model(cfg, dev, distinct_layers=args.distinct_layers, seed=args.seed)
    print(f"[bench] model built in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(args.seed + 7)
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=g)
    results = {}
    prefetcher = None
    # the uncompressed model's FP8 weights re-laid out at load in the tile
    # layout its linears read fastest (one copy, the same bytes)
    tile_resident_weights(model)
    for mode in ("fp8", "ecf8", "ecf8_prefetch", "ecf8_fused"):
        if mode == "ecf8":
            t0 = time.time()
            compress_layers(model, drawn)
            torch.cuda.synchronize()
            print(f"[bench] layers compressed in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
        if mode == "ecf8_prefetch":
            prefetcher = LayerPrefetcher(model.model.layers, dev,
                                         workgroups_per_cu=args.prefetch_workgroups).install()
        if mode == "ecf8_fused":
            prefetcher.uninstall()
            prefetcher = None
            TensorManager.clear_device()
            torch.cuda.empty_cache()
            t0 = time.time()
            retile_layers(model, drawn)
            torch.cuda.synchronize()
            print(f"[bench] layers re-tiled in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
        TensorManager.clear_device()
        torch.cuda.empty_cache()
        runner = Qwen3Runner(model, B, T, T + new, dev)
        runner.capture()
        runner.generate(prompt, min(new, 8))  # warm-up
        r = timed_generate(runner, prompt, new)
        print(f"[bench] {mode}: {r['tokens_per_s']:.1f} tokens/s, latency {r['latency_s']:.3f}s, "
              f"peak {r['peak_mib']:.0f} MiB", file=sys.stderr, flush=True)
        r["weights_mib"] = sum(t.numel() * t.element_size() for t in
                               list(model.parameters()) + list(model.buffers())) / 2**20
        if mode == "ecf8_fused":
            r["weights_mib"] += sum(op.nbytes() for layer in model.model.layers
                                    for op in layer._ecf8_tiles.values()) / 2**20
        if mode in ("fp8", "ecf8_fused"):
            r["linears"] = runner.time_linears()
            print(f"[bench] {mode}: decode-step linears per layer {r['linears']}",
                  file=sys.stderr, flush=True)
        if mode == "fp8":
            # the prompt's GEMMs (every mode runs the same kernel on the same bytes)
            r["prefill"] = runner.time_linears(prompt=True)
            print(f"[bench] prompt GEMMs per layer {r['prefill']}", file=sys.stderr, flush=True)
        results[mode] = r
        del runner
    ecf8_modes = ("ecf8", "ecf8_prefetch", "ecf8_fused")
    same = all(torch.equal(results["fp8"]["tokens"], results[m]["tokens"]) for m in ecf8_modes)
    fp8 = results["fp8"]
    best = max(ecf8_modes, key=lambda m: results[m]["tokens_per_s"])
    ecf8 = results[best]

    def summary(r):
        return {"tokens_per_s": round(r["tokens_per_s"], 1), "latency_s": round(r["latency_s"], 4),
                "peak_mib": round(r["peak_mib"], 1), "weights_mib": round(r["weights_mib"], 1)}

    line = {
        "metric": "e2e tokens/s, Qwen3-8B-shape bs16 (ECF8-compressed layers, fastest decode "
                  "mode; config.ecf8_decode names it)",
        "value": round(ecf8["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "higher_is_better": True,
        "vs_baseline": None,
        "dtype": "fp8",
        "data": "synthetic (random-init weights, random prompts)",
        "config": {"workload": "qwen3-8b-generate", "layers": cfg.layers, "hidden": cfg.hidden,
                   "fp8_weights": "tile layout (re-laid out at load)",
                   "intermediate": cfg.intermediate, "heads": cfg.heads, "kv_heads": cfg.kv_heads,
                   "vocab": cfg.vocab, "batch": B, "prompt_len": T, "new_tokens": new,
                   "distinct_layer_weights": args.distinct_layers, "decoding": "greedy",
                   "ecf8_decode": {
                       "ecf8": "each layer decoded in its forward-pre-hook, then FP8 GEMMs",
                       "ecf8_prefetch": "next layer decoded on a side stream (double-buffered)",
                       "ecf8_fused": "layers re-tiled at load (ECF8-T); decode-step linears "
                                     "decode their weight operands into the MFMAs"}[best]},
        "uncompressed_fp8": summary(fp8),
        "ecf8": summary(ecf8),
        "ecf8_mode": best,
        "ecf8_modes": {m: summary(results[m]) for m in ecf8_modes},
        "ratio_vs_uncompressed": round(ecf8["tokens_per_s"] / fp8["tokens_per_s"], 4),
        "identical_tokens": same,
        "linears_per_layer_step": {m: _linear_summary(results[m]["linears"])
                                   for m in ("fp8", "ecf8_fused")},
        "prompt_gemms_per_layer": _gemm_summary(results["fp8"]["prefill"]),
    }
    return line


def linears_workload(args):
    """The four decode-step linears of the Qwen3-8B-shaped model alone
    (M = --batch rows; each linear launched for all 36 layers back to back,
    so the weights stream from HBM as in a decode step): first over FP8
    weights resident in the tile layout, then over the same layers
    ECF8-compressed and re-tiled (the fused decode-into-MFMA linears).  The
    activations are one seeded random batch quantized per 1x128 group; the
    last layer's outputs of the two modes must be identical.  Also times
    the prompt's GEMMs (M = batch x --prompt-len rows, FP8 weights) as
    TFLOP/s.  Starts no child process, so a counter profile of it sees only
    these kernels."""
    import torch

    from ecf8_amd import llm_kernels as K
    from ecf8_amd.llm import (Qwen3Config, Qwen3Runner, compress_layers, random_model,
                              retile_layers, tile_resident_weights)

    dev = torch.device("cuda", 0)
    cfg = Qwen3Config()
    B = args.batch
    if B > 16:
        raise SystemExit("--batch: the decode-step linears take at most 16 rows")
    model, drawn = random_model(cfg, dev, distinct_layers=args.distinct_layers, seed=args.seed)
    g = torch.Generator(device=dev).manual_seed(args.seed + 11)
    results, outs = {}, {}
    for mode in ("fp8", "ecf8_fused"):
        if mode == "fp8":
            tile_resident_weights(model)
        else:
            compress_layers(model, drawn)
            retile_layers(model, drawn)
        T = args.prompt_len if mode == "fp8" else 1
        runner = Qwen3Runner(model, B, T, T + 1, dev)
        if mode == "fp8":
            acts = {k: torch.randn(B * T, k, generator=g, device=dev).to(torch.bfloat16)
                    for k in runner.aq}
        for k, x in acts.items():
            K.act_quant(x[: B * T], B * T, runner.aq[k], runner.as_[k])
        results[mode] = runner.time_linears(reps=args.steps)
        torch.cuda.synchronize()
        outs[mode] = {out: getattr(runner, out)[:B].clone() for _, _, out, _ in runner.LINEARS}
        if mode == "fp8":  # after the compared outputs: it rewrites the output buffers
            prompt = runner.time_linears(reps=args.steps, prompt=True)
        print(f"[bench] {mode}: decode-step linears per layer {results[mode]}", file=sys.stderr,
              flush=True)
        del runner
    same = all(torch.equal(outs["fp8"][o], outs["ecf8_fused"][o]) for o in outs["fp8"])
    fp8, fused = _linear_summary(results["fp8"]), _linear_summary(results["ecf8_fused"])
    line = {
        "metric": "decode-step linear time per Qwen3-8B-shape layer (q/k/v, o, gate/up, down)",
        "value": fused["layer"]["us"],
        "unit": "us",
        "n_gpus": 1,
        "higher_is_better": False,
        "vs_baseline": None,
        "dtype": "fp8",
        "data": "synthetic (random-init weights, random activations)",
        "config": {"workload": "qwen3-8b-decode-step-linears", "layers": cfg.layers, "rows": B,
                   "reps": args.steps, "timing": "best of reps; one graph replay of the 36 "
                                                 "layers' launches per linear"},
        "fp8": fp8,
        "ecf8_fused": fused,
        "ratio_fp8_over_fused": round(fp8["layer"]["us"] / fused["layer"]["us"], 4),
        "identical_outputs": same,
        "prompt_gemms_per_layer": dict(_gemm_summary(prompt), rows=B * args.prompt_len),
    }
    print(json.dumps(line), flush=True)
    sys.exit(0 if same else 1)


def moe_linears_workload(args):
    """The decode-step linears of the Qwen3-30B-A3B-shaped MoE model alone
    (M = --batch tokens): attention q/k/v and o, and the routed experts'
    grouped gate/up and down, each launched for all 48 layers back to back
    on one routing of seeded random activations through layer 0's router
    (top-8 of 128 experts per token; every layer runs that routing, so each
    reads the picked experts' weights, ~0.4 GB per layer), first over FP8
    weights resident in the tile layout, then over the same blocks
    ECF8-compressed and re-tiled.  The last layer's outputs of the two
    modes must be identical.  Starts no child process."""
    import torch

    from ecf8_amd import llm_kernels as K
    from ecf8_amd.llm import tile_resident_weights
    from ecf8_amd.moe import (Qwen3MoeConfig, Qwen3MoeRunner, compress_moe_layers,
                              random_moe_model, retile_moe_layers)

    dev = torch.device("cuda", 0)
    cfg = Qwen3MoeConfig()
    B = args.batch
    if B > 16:
        raise SystemExit("--batch: the decode-step linears take at most 16 rows")
    model, drawn = random_moe_model(cfg, dev, distinct_layers=args.distinct_layers, seed=args.seed)
    g = torch.Generator(device=dev).manual_seed(args.seed + 11)
    P, I, A = B * cfg.top_k, cfg.moe_intermediate, cfg.heads * cfg.head_dim
    bf = dict(dtype=torch.bfloat16, device=dev)
    x_h = torch.randn(B, cfg.hidden, generator=g, device=dev).to(torch.bfloat16)
    x_a = torch.randn(B, A, generator=g, device=dev).to(torch.bfloat16)
    x_gu = torch.randn(P, 2 * I, generator=g, device=dev).to(torch.bfloat16)
    results, outs, n_active = {}, {}, {}
    for mode in ("fp8", "ecf8_fused"):
        if mode == "fp8":
            tile_resident_weights(model)
        else:
            compress_moe_layers(model, drawn)
            retile_moe_layers(model, drawn)
        runner = Qwen3MoeRunner(model, B, 1, 2, dev)
        layer0 = model.model.layers[0]
        runner.hb[:B].copy_(x_h)
        K.act_quant(runner.hb, B, runner.aqH, runner.asH)
        K.act_quant(x_a, B, runner.aqA, runner.asA)
        K.moe_route(runner.hb[:B], layer0.mlp.gate.weight, B, runner.route)
        K.moe_group(runner.route, B)
        runner.gu[:P].copy_(x_gu)
        K.silu_mul_quant(runner.gu, P, runner.hq, runner.hs)
        n_active[mode] = int(runner.route.n_active.item())
        results[mode] = runner.time_linears(reps=args.steps)
        torch.cuda.synchronize()
        outs[mode] = {"qkv": runner.qkv[:B].clone(), "o": runner.o[:B].clone(),
                      "gate_up": runner.gu[:P].clone(), "down": runner.down[:P].clone()}
        print(f"[bench] {mode}: decode-step linears per layer {results[mode]}", file=sys.stderr,
              flush=True)
        del runner
    same = all(torch.equal(outs["fp8"][o], outs["ecf8_fused"][o]) for o in outs["fp8"])
    fp8, fused = _linear_summary(results["fp8"]), _linear_summary(results["ecf8_fused"])
    line = {
        "metric": "decode-step linear time per Qwen3-30B-A3B-shape MoE layer (q/k/v, o, routed "
                  "gate/up, routed down)",
        "value": fused["layer"]["us"],
        "unit": "us",
        "n_gpus": 1,
        "higher_is_better": False,
        "vs_baseline": None,
        "dtype": "fp8",
        "data": "synthetic (random-init weights, random activations)",
        "config": {"workload": "qwen3-moe-decode-step-linears", "layers": cfg.layers,
                   "tokens": B, "experts": cfg.experts, "top_k": cfg.top_k,
                   "experts_routed": n_active["fp8"], "reps": args.steps,
                   "timing": "best of reps; one graph replay of the 48 layers' launches per "
                             "linear"},
        "fp8": fp8,
        "ecf8_fused": fused,
        "ratio_fp8_over_fused": round(fp8["layer"]["us"] / fused["layer"]["us"], 4),
        "identical_outputs": same and n_active["fp8"] == n_active["ecf8_fused"],
    }
    print(json.dumps(line), flush=True)
    sys.exit(0 if line["identical_outputs"] else 1)


def _gemm_summary(lin: dict) -> dict:
    """Per-layer prompt GEMM times as TFLOP/s and a fraction of MI355X's
    dense FP8 MFMA peak."""
    out = {k: {"us": v["us"], "tflop_s": round(v["flops"] / (v["us"] * 1e-6) / 1e12, 1),
               "fp8_peak_frac": round(v["flops"] / (v["us"] * 1e-6) / 1e12 / FP8_PEAK_TFLOPS, 4)}
           for k, v in lin.items()}
    us = sum(v["us"] for v in lin.values())
    fl = sum(v["flops"] for v in lin.values())
    out["layer"] = {"us": round(us, 2), "gflop": round(fl / 1e9, 1),
                    "tflop_s": round(fl / (us * 1e-6) / 1e12, 1),
                    "fp8_peak_frac": round(fl / (us * 1e-6) / 1e12 / FP8_PEAK_TFLOPS, 4)}
    return out


def _linear_summary(lin: dict) -> dict:
    """Per-layer decode-step linear times with their weight bytes as a rate
    and a fraction of the HBM peak."""
    total_us = sum(v["us"] for v in lin.values())
    total_b = sum(v["bytes"] for v in lin.values())
    out = {k: {"us": v["us"], "tb_per_s": round(v["bytes"] / (v["us"] * 1e-6) / 1e12, 3)}
           for k, v in lin.items()}
    out["layer"] = {"us": round(total_us, 2), "bytes": total_b,
                    "tb_per_s": round(total_b / (total_us * 1e-6) / 1e12, 3),
                    "hbm_frac": round(total_b / (total_us * 1e-6) / (HBM_PEAK_GBPS * 1e9), 4)}
    return out


def moe_generate(args):
    """Qwen3-30B-A3B-shaped MoE causal LM (48 layers, hidden 2048, 32 query /
    4 KV heads, 128 experts of intermediate 768, top-8 routing; random init,
    FP8 attention and expert linears with 128x128 block scales, bf16 router,
    embedding and lm_head), batch 16, random prompts of 128 tokens, greedy
    decoding of --new-tokens (default 512) tokens: first with the FP8
    weights resident, then with every attention block and expert
    ECF8-compressed -- decoded by the attention block's forward-pre-hook and,
    per decode step, only the experts the router picked in one batched
    launch per layer (selected on the device), with the next layer's
    attention block on a side stream, and finally re-tiled (ECF8-T), the
    decode step's attention and grouped expert linears decoding their
    weight operands themselves.  Every run uses the same engine (eager
    prefill, one HIP graph replay per decode step) and must produce
    identical tokens."""
    import torch

    from ecf8_amd.llm import timed_generate
    from ecf8_amd.llm import tile_resident_weights
    from ecf8_amd.moe import (Qwen3MoeConfig, Qwen3MoeRunner, compress_moe_layers,
                              random_moe_model, retile_moe_layers)
    from ecf8_amd.prefetch import LayerPrefetcher
    from dfloat.run.run import TensorManager

    dev = torch.device("cuda", 0)
    cfg = Qwen3MoeConfig()
    B, T = args.batch, args.prompt_len
    new = args.new_tokens if args.new_tokens is not None else 512
    t0 = time.time()
    model, drawn = random_moe_model(cfg, dev, distinct_layers=args.distinct_layers, seed=args.seed)
    print(f"[bench] model built in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(args.seed + 7)
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=g)
    results = {}
    prefetcher = None
    tile_resident_weights(model)  # the FP8 model's weights in the tile layout
    for mode in ("fp8", "ecf8", "ecf8_prefetch", "ecf8_fused"):
        if mode == "ecf8":
            t0 = time.time()
            compress_moe_layers(model, drawn)
            torch.cuda.synchronize()
            print(f"[bench] blocks compressed in {time.time() - t0:.1f}s", file=sys.stderr,
                  flush=True)
        if mode == "ecf8_prefetch":
            # the next layer's attention block decoded on a side stream
            prefetcher = LayerPrefetcher([layer.self_attn for layer in model.model.layers], dev,
                                         workgroups_per_cu=args.prefetch_workgroups).install()
        if mode == "ecf8_fused":
            prefetcher.uninstall()
            prefetcher = None
            TensorManager.clear_device()
            torch.cuda.empty_cache()
            t0 = time.time()
            retile_moe_layers(model, drawn)
            torch.cuda.synchronize()
            print(f"[bench] blocks re-tiled in {time.time() - t0:.1f}s", file=sys.stderr,
                  flush=True)
        TensorManager.clear_device()
        torch.cuda.empty_cache()
        t0 = time.time()
        runner = Qwen3MoeRunner(model, B, T, T + new, dev)
        runner.capture()
        print(f"[bench] {mode}: runner ready in {time.time() - t0:.1f}s", file=sys.stderr,
              flush=True)
        runner.generate(prompt, min(new, 8))  # warm-up
        r = timed_generate(runner, prompt, new)
        # experts the last step's router picked, in the last layer
        r["experts_routed_last_step"] = int(runner.route.n_active.item())
        if mode in ("fp8", "ecf8_fused"):
            # on the last step's routing and inputs
            r["linears"] = runner.time_linears()
            print(f"[bench] {mode}: decode-step linears per layer {r['linears']}",
                  file=sys.stderr, flush=True)
        print(f"[bench] {mode}: {r['tokens_per_s']:.1f} tokens/s, latency {r['latency_s']:.3f}s, "
              f"peak {r['peak_mib']:.0f} MiB", file=sys.stderr, flush=True)
        r["weights_mib"] = sum(t.numel() * t.element_size() for t in
                               list(model.parameters()) + list(model.buffers())) / 2**20
        if mode == "ecf8_fused":
            r["weights_mib"] += sum(op.nbytes() for mod in model.modules()
                                    for op in getattr(mod, "_ecf8_tiles", {}).values()) / 2**20
        results[mode] = r
        del runner
    ecf8_modes = ("ecf8", "ecf8_prefetch", "ecf8_fused")
    same = all(torch.equal(results["fp8"]["tokens"], results[m]["tokens"]) for m in ecf8_modes)
    fp8 = results["fp8"]
    best = max(ecf8_modes, key=lambda m: results[m]["tokens_per_s"])
    ecf8 = results[best]

    def summary(r):
        return {"tokens_per_s": round(r["tokens_per_s"], 1), "latency_s": round(r["latency_s"], 4),
                "peak_mib": round(r["peak_mib"], 1), "weights_mib": round(r["weights_mib"], 1)}

    line = {
        "metric": "e2e tokens/s, Qwen3-30B-A3B-shape MoE bs16 (ECF8 attention blocks and "
                  "experts, fastest decode mode; config.ecf8_decode names it)",
        "value": round(ecf8["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "higher_is_better": True,
        "vs_baseline": None,
        "dtype": "fp8",
        "data": "synthetic (random-init weights, random prompts)",
        "config": {"workload": "qwen3-moe-generate", "layers": cfg.layers, "hidden": cfg.hidden,
                   "fp8_weights": "tile layout (re-laid out at load)",
                   "heads": cfg.heads, "kv_heads": cfg.kv_heads, "experts": cfg.experts,
                   "top_k": cfg.top_k, "moe_intermediate": cfg.moe_intermediate,
                   "vocab": cfg.vocab, "batch": B, "prompt_len": T, "new_tokens": new,
                   "distinct_layer_weights": args.distinct_layers, "decoding": "greedy",
                   "ecf8_decode": {
                       "ecf8": "attention block in its hook; routed experts per step "
                               "(device-side selection, one batched launch per layer)",
                       "ecf8_prefetch": "next layer's attention block on a side stream; routed "
                                        "experts per step (one batched launch per layer)",
                       "ecf8_fused": "blocks re-tiled at load (ECF8-T); decode-step attention "
                                     "and routed-expert linears decode their weight operands "
                                     "into the MFMAs"}[best]},
        "uncompressed_fp8": summary(fp8),
        "ecf8": summary(ecf8),
        "ecf8_mode": best,
        "ecf8_modes": {m: summary(results[m]) for m in ecf8_modes},
        "experts_routed_last_step": ecf8["experts_routed_last_step"],
        "ratio_vs_uncompressed": round(ecf8["tokens_per_s"] / fp8["tokens_per_s"], 4),
        "identical_tokens": same,
        "linears_per_layer_step": {m: _linear_summary(results[m]["linears"])
                                   for m in ("fp8", "ecf8_fused")},
    }
    return line


def dit_generate(args):
    """FLUX.1-dev-shaped DiT (19 double + 38 single blocks, hidden 3072),
    one 1024x1024 image: 4096 latent tokens of 64 channels and 512 text
    tokens of 4096, embedded guidance 3.5, --dit-steps Euler steps at batch
    1; first with the FP8 weights resident, then with every block
    ECF8-compressed and decoded by its forward-pre-hook, then with each
    block's decode on a side stream one block ahead, then with each block
    decoded straight into its Linears' bf16 weights (no FP8 pass, no
    per-call dequantization).  Every run must produce identical latents."""
    import torch

    from ecf8_amd.dit import (FluxConfig, compress_blocks, fuse_dequant_blocks, prefetch_blocks,
                              random_pipeline, timed_generate)
    from dfloat.run.run import TensorManager

    dev = torch.device("cuda", 0)
    cfg = FluxConfig()
    t0 = time.time()
    pipe, drawn = random_pipeline(cfg, dev, distinct=args.distinct_layers, seed=args.seed)
    print(f"[bench] DiT built in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(args.seed + 11)
    lat = torch.randn(1, 4096, cfg.in_channels, generator=g).to(torch.bfloat16).to(dev)
    txt = torch.randn(1, 512, cfg.txt_dim, generator=g).to(torch.bfloat16).to(dev)
    pooled = torch.randn(1, cfg.pooled_dim, generator=g).to(torch.bfloat16).to(dev)
    results = {}
    weights_exact = True
    prefetcher = None
    for mode in ("fp8", "ecf8", "ecf8_prefetch", "ecf8_fused"):
        if mode == "ecf8":
            t0 = time.time()
            compress_blocks(pipe, drawn)
            torch.cuda.synchronize()
            print(f"[bench] blocks compressed in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
        if mode == "ecf8_prefetch":
            prefetcher = prefetch_blocks(pipe, dev, workgroups_per_cu=args.prefetch_workgroups)
        if mode == "ecf8_fused":
            prefetcher.uninstall()
            prefetcher = None
            fuse_dequant_blocks(pipe)
        TensorManager.clear_device()
        torch.cuda.empty_cache()
        timed_generate(pipe, lat, txt, pooled, 1, (64, 64))  # warm-up
        r = timed_generate(pipe, lat, txt, pooled, args.dit_steps, (64, 64))
        r["weights_mib"] = sum(t.numel() * t.element_size() for t in
                               list(pipe.parameters()) + list(pipe.buffers())) / 2**20
        print(f"[bench] {mode}: {r['seconds']:.3f} s/image, peak {r['peak_mib']:.0f} MiB",
              file=sys.stderr, flush=True)
        results[mode] = r
        if mode == "ecf8":
            # the decode path's own claim, checked directly: every block's
            # hook injects exactly its original FP8 weights
            for blocks, dr in ((pipe.dit.blocks, drawn[0]), (pipe.dit.single_blocks, drawn[1])):
                for i, blk in enumerate(blocks):
                    for hook in blk._forward_pre_hooks.values():
                        hook(blk, None)
                    for name, (w, _) in dr[i % len(dr)].items():
                        got = blk.get_submodule(name).weight.view(torch.uint8)
                        weights_exact &= torch.equal(got, w.view(torch.uint8).to(dev))
    ecf8_modes = ("ecf8", "ecf8_prefetch", "ecf8_fused")
    fp8 = results["fp8"]
    same = all(torch.equal(fp8["latents"].view(torch.int16), results[m]["latents"].view(torch.int16))
               for m in ecf8_modes)
    diff = max((fp8["latents"].float() - results[m]["latents"].float()).abs().max().item()
               for m in ecf8_modes)
    best = min(ecf8_modes, key=lambda m: results[m]["seconds"])
    ecf8 = results[best]

    def summary(r):
        return {"seconds_per_image": round(r["seconds"], 3), "peak_mib": round(r["peak_mib"], 1),
                "weights_mib": round(r["weights_mib"], 1)}

    line = {
        "metric": "DiT s/image, FLUX.1-dev-shape 1024x1024 (ECF8-compressed blocks, fastest "
                  "decode mode; config.ecf8_decode names it)",
        "value": round(ecf8["seconds"], 3),
        "unit": "s/image",
        "n_gpus": 1,
        "higher_is_better": False,
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, random latents and text embeddings)",
        "config": {"workload": "flux-dit-generate", "double_blocks": cfg.double,
                   "single_blocks": cfg.single, "hidden": cfg.hidden, "heads": cfg.heads,
                   "mlp": cfg.mlp, "image_tokens": 4096, "text_tokens": 512, "batch": 1,
                   "steps": args.dit_steps, "guidance": 3.5,
                   "distinct_block_weights": args.distinct_layers,
                   "linears": "FP8 weights dequantized to bf16 per call + library bf16 GEMM",
                   "attention": "bf16 operands, fp32 accumulation",
                   "ecf8_decode": {
                       "ecf8": "each block decoded in its forward-pre-hook",
                       "ecf8_prefetch": "next block decoded on a side stream (two buffers, "
                                        "a third for the last of an odd count)",
                       "ecf8_fused": "each block decoded straight into its Linears' bf16 "
                                     "weights (FP8 x block scale, one pass)"}[best]},
        "uncompressed_fp8": summary(fp8),
        "ecf8": summary(ecf8),
        "ecf8_mode": best,
        "ecf8_modes": {m: summary(results[m]) for m in ecf8_modes},
        "ratio_vs_uncompressed": round(fp8["seconds"] / ecf8["seconds"], 4),
        "weights_bit_exact": bool(weights_exact),
        "identical_latents": same,
        "latents_max_abs_diff": diff,
    }
    print(json.dumps(line), flush=True)
    if not weights_exact:
        sys.exit(1)


def _child_line(extra_args, timeout_s: float):
    """Run this script with ``extra_args`` in a child process (its own HIP
    context, so its kernels stay out of this process's profile and its
    memory is returned when it ends); returns (JSON line, wall seconds) or
    ({"error": reason}, wall seconds)."""
    import subprocess

    cmd = [sys.executable, os.path.abspath(__file__), *extra_args]
    t0 = time.perf_counter()
    print(f"[bench] child: {' '.join(cmd[1:])}", file=sys.stderr, flush=True)
    try:
        res = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout_s)
    except subprocess.TimeoutExpired:
        return {"error": f"timed out after {timeout_s:.0f} s"}, time.perf_counter() - t0
    sys.stderr.write(res.stderr)
    lines = [ln for ln in res.stdout.splitlines() if ln.startswith("{")]
    if not lines:
        return ({"error": f"exit status {res.returncode}, no result line"},
                time.perf_counter() - t0)
    return json.loads(lines[-1]), time.perf_counter() - t0


def e2e_child(workload: str, seed: int, timeout_s: float):
    """Summary of an end-to-end generate workload run in a child process
    (see _child_line), or the reason it has none."""
    full, wall = _child_line(["--workload", workload, "--seed", str(seed)], timeout_s)
    if "error" in full:
        return full
    keep = ("uncompressed_fp8", "ecf8", "ecf8_mode", "ecf8_modes", "ratio_vs_uncompressed",
            "identical_tokens", "experts_routed_last_step", "linears_per_layer_step",
            "prompt_gemms_per_layer")
    out = {"workload": full["config"]["workload"], "unit": full["unit"],
           "batch": full["config"]["batch"], "prompt_len": full["config"]["prompt_len"],
           "new_tokens": full["config"]["new_tokens"],
           "ecf8_decode": full["config"]["ecf8_decode"]}
    out.update({k: full[k] for k in keep if k in full})
    out["wall_s"] = round(wall, 1)
    return out


def dit_child(seed: int, timeout_s: float):
    """Summary of the FLUX.1-dev-shaped DiT image (28 steps, every decode
    mode) run in a child process."""
    full, wall = _child_line(["--workload", "flux-dit-generate", "--seed", str(seed)], timeout_s)
    if "error" in full:
        return full
    cfg = full["config"]
    out = {"workload": cfg["workload"], "unit": full["unit"], "steps": cfg["steps"],
           "image_tokens": cfg["image_tokens"], "text_tokens": cfg["text_tokens"],
           "batch": cfg["batch"], "ecf8_decode": cfg["ecf8_decode"]}
    out.update({k: full[k] for k in ("uncompressed_fp8", "ecf8", "ecf8_mode", "ecf8_modes",
                                     "ratio_vs_uncompressed", "weights_bit_exact",
                                     "identical_latents") if k in full})
    out["wall_s"] = round(wall, 1)
    return out


BATCHED_MIN_STEPS = 200
BATCHED_MIN_WARMUP = 100


def batched_child(seed: int, steps: int, warmup: int, timeout_s: float):
    """The batched MoE-layer decode line (one Qwen3-30B-A3B-shaped layer,
    attention + 128 experts in one launch) run in a child process with at
    least BATCHED_MIN_WARMUP warm-up launches (~24 ms) and at least
    BATCHED_MIN_STEPS timed ones (~47 ms): on MI355X the first ~15 ms of
    sustained decode load run up to 8 % slower than the rest (launch times
    235 -> 255 -> 235 us, with or without a GPU-busy prime beforehand), so a
    window after 5 warm-up launches would time that onset, not the
    layer-after-layer rate of a model's decode."""
    full, wall = _child_line(["--workload", "qwen3-moe-layer", "--seed", str(seed), "--steps",
                              str(max(steps, BATCHED_MIN_STEPS)), "--warmup",
                              str(max(warmup, BATCHED_MIN_WARMUP))],
                             timeout_s)
    if "error" in full:
        return full
    cfg = full["config"]
    return {"workload": cfg["workload"], "blocks": cfg["blocks"], "elements": cfg["elements"],
            "algorithmic_bytes": cfg["algorithmic_bytes"], "value": full["value"],
            "unit": full["unit"], "steps": full["steps"], "warmup": full["warmup"],
            "ms_per_step": full["ms_per_step"], "warmup_ms_per_step": full["warmup_ms_per_step"],
            "roofline": full["roofline"],
            "bit_exact": full["bit_exact"], "wall_s": round(wall, 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--copies", type=int, default=10, help="rotated input/output sets")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=("qwen3-8b-layer", "qwen3-moe-layer", "flux-block-bf16",
                                           "qwen3-8b-generate", "qwen3-moe-generate",
                                           "flux-dit-generate", "qwen3-8b-linears",
                                           "qwen3-moe-linears"),
                    default="qwen3-8b-layer",
                    help="qwen3-moe-layer: attention + 128 experts in one batched launch; "
                         "qwen3-8b-generate: end-to-end greedy generation, FP8 vs ECF8; "
                         "qwen3-moe-generate: the same for the 30B-A3B-shaped MoE; "
                         "flux-dit-generate: one 1024x1024 DiT image, FP8 vs ECF8; "
                         "flux-block-bf16: one FLUX double block decoded straight into bf16 "
                         "weights; qwen3-8b-linears: the decode-step linears alone, FP8 vs "
                         "fused ECF8 (--steps = timing rounds); qwen3-moe-linears: the same for "
                         "the MoE's attention and routed expert linears")
    ap.add_argument("--dit-steps", type=int, default=28)
    ap.add_argument("--routed-tokens", type=int, default=0,
                    help="qwen3-moe-layer: decode only the experts a top-k router picks for "
                         "this many tokens (device-side selection)")
    ap.add_argument("--top-k", type=int, default=8)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--prompt-len", type=int, default=128)
    ap.add_argument("--new-tokens", type=int, default=None,
                    help="generate: new tokens per sequence (1024 dense, 512 MoE)")
    ap.add_argument("--prefetch-workgroups", type=float, default=2,
                    help="generate: side-stream decode workgroups per CU (fractions leave "
                         "CUs free)")
    ap.add_argument("--distinct-layers", type=int, default=2,
                    help="generate: layers drawn independently (the rest copy them)")
    ap.add_argument("--e2e", choices=("all", "dense", "none"), default="all",
                    help="qwen3-8b-layer: also run the end-to-end workloads in child processes "
                         "and report them in the line's e2e object (dense Qwen3-8B bs16; with "
                         "'all' also the MoE, the FLUX DiT image, and the batched MoE-layer "
                         "decode in the line's batched object)")
    ap.add_argument("--single-launches", type=int, default=10,
                    help="launches timed one by one (an event pair each) for the per-launch "
                         "kernel duration")
    ap.add_argument("--call-form", choices=("abi", "reference"), default="abi",
                    help="qwen3-8b-layer: 'reference' launches each step through "
                         "dfloat.run._decode, the reference's RawKernel call form")
    ap.add_argument("--mode", choices=("decode", "copy", "ceiling"), default="decode",
                    help="copy: time a plain 1 GiB device copy (HBM counter calibration); "
                         "ceiling: sweep the streaming probe kernels per size")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the decode path has no multi-GPU component)", file=sys.stderr)
        sys.exit(2)
    if args.mode == "copy":
        return copy_calibration(args.steps, args.warmup)
    if args.mode == "ceiling":
        return stream_ceiling(args.steps, args.warmup)
    if args.workload in ("qwen3-8b-generate", "qwen3-moe-generate"):
        if args.workload == "qwen3-8b-generate":
            if args.new_tokens is None:
                args.new_tokens = 1024
            line = e2e_generate(args)
        else:
            line = moe_generate(args)
        print(json.dumps(line), flush=True)
        sys.exit(0 if line["identical_tokens"] else 1)
    if args.workload == "flux-dit-generate":
        return dit_generate(args)
    if args.workload == "qwen3-8b-linears":
        return linears_workload(args)
    if args.workload == "qwen3-moe-linears":
        return moe_linears_workload(args)

    import torch

    dev = torch.device("cuda", 0)
    setup = {"qwen3-8b-layer": _qwen3_layer_workload, "qwen3-moe-layer": _qwen3_moe_layer_workload,
             "flux-block-bf16": _flux_block_bf16_workload}[args.workload]
    calls, verify, alg, n, config, cpu_case = setup(args, dev)
    pmc_profile = {"qwen3-8b-layer-decode": "decode_qwen3_layer_pmc.md",
                   "qwen3-moe-layer-decode": "decode_qwen3_moe_layer_pmc.md",
                   "flux-double-block-bf16-decode": "decode_flux_block_bf16_pmc.md"}.get(
                       config["workload"])

    def step(i):
        fn, cargs = calls[i % len(calls)]
        rc = fn(*cargs)
        if rc:
            raise RuntimeError(f"decode failed with status {rc}")

    # Warm-up straight into the timed region: the only gap between them is
    # the synchronization.  The outputs are verified after timing (so they
    # are the timed launches' own): verifying in between left the GPU idle
    # for the host copy and compare, and the timed launches then paid its
    # return from idle clocks (measured on MI355X: 72.5-73.3 us per launch
    # instead of 68).  An event pair around the warm-up launches (no
    # synchronization) reports their own average too: the first ~15 ms of
    # sustained decode load run slower on MI355X.
    stream = torch.cuda.current_stream(dev)
    w_start = torch.cuda.Event(enable_timing=True)
    w_end = torch.cuda.Event(enable_timing=True)
    w_start.record(stream)
    for i in range(args.warmup):
        step(i)
    w_end.record(stream)

    # One event pair around the K back-to-back launches on the launch stream:
    # a step is exactly one decode kernel, so the average launch duration is
    # the timed span over K (events between launches would add their own gaps).
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    start.record(stream)
    for i in range(args.steps):
        step(i)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    total_ms = start.elapsed_time(end)
    warmup_ms = w_start.elapsed_time(w_end) / args.warmup if args.warmup else None
    ms_per_step = total_ms / args.steps
    gbps = alg / (ms_per_step * 1e-3) / 1e9
    # Per-launch wall time: launches one at a time, each between its own
    # event pair on the launch stream.  Each pair also spans the dispatch of
    # its launch (~3 us on MI355X), so this is an upper bound; the roofline
    # uses the timed region's average above, which rocprofv3's kernel
    # durations of the same command match.
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(args.single_launches)]
    for i, (a, b) in enumerate(pairs):
        a.record(stream)
        step(args.steps + i)
        b.record(stream)
    torch.cuda.synchronize()
    launch_ms = [a.elapsed_time(b) for a, b in pairs]
    avg_launch_ms = sum(launch_ms) / len(launch_ms) if launch_ms else ms_per_step
    ok = verify()
    if not ok:
        print("[bench] decoded weights differ from the original FP8 bytes", file=sys.stderr)
        sys.exit(1)

    cpu = enc = None
    if not args.no_cpu_baseline and cpu_case is not None:
        cpu = cpu_baseline(cpu_case[0], cpu_case[1], alg)
        enc = cpu_encode(cpu_case[2], args.seed)
    e2e = batched = None
    if args.workload == "qwen3-8b-layer" and args.e2e != "none" and args.call_form == "abi":
        del calls, cpu_case
        torch.cuda.empty_cache()
        e2e = {"qwen3_8b_bs16": e2e_child("qwen3-8b-generate", args.seed, 420)}
        if args.e2e == "all":
            e2e["qwen3_30b_a3b_bs16"] = e2e_child("qwen3-moe-generate", args.seed, 480)
            e2e["flux_dit_1024"] = dit_child(args.seed, 420)
            batched = batched_child(args.seed, args.steps, args.warmup, 300)
    line = {
        "metric": "ECF8 decode GB/s + % HBM roofline; e2e tokens/s, Qwen3-8B-shape bs16",
        "value": round(gbps, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "kernel_ms_per_launch": round(avg_launch_ms, 5),
        "warmup_ms_per_step": round(warmup_ms, 5) if warmup_ms is not None else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8" if config["workload"] != "flux-double-block-bf16-decode" else "u8 + f32 scale",
        "data": "synthetic",
        "config": config,
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "traffic": _traffic_from_profile(pmc_profile) if pmc_profile else None,
        },
        "cpu_baseline": cpu,
        "cpu_encode": enc,
        "e2e": e2e,
        "batched": batched,
        "wall_s_timed": round(wall, 4),
        "bit_exact": ok,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
