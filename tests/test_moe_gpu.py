"""GPU numerics of the routed-expert kernels (include/ecf8_llm.h, MoE part)
against plain torch / numpy restatements: the router's top-k choice and
weights, the grouping of (token, expert) pairs, the grouped FP8 expert
linear (fp64 per-pair reference), and the weighted combine.

Tolerances: router probabilities 1e-5 absolute (fp32 dot products summed
in a different order than torch's); linear outputs 2^-7 relative plus
1e-4 of the largest magnitude (bf16 output rounding); combine 2^-7
relative (bf16)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn
MULTI = 0  # ECF8_TABLE_MULTI


def _rand_fp8(shape, gen, dev):
    b = torch.randint(0, 256, shape, generator=gen, dtype=torch.int32).to(torch.uint8)
    b[(b & 0x7F) == 0x7F] = 0x7E
    return b.view(FP8).to(dev)


def _groups_ref(idx, E):
    """Counting sort of the pairs (m, k) by expert, token order inside an
    expert: offsets, the active experts, and each pair's sorted position."""
    flat = idx.reshape(-1).tolist()
    counts = np.bincount(flat, minlength=E)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    pos, seen = [], np.zeros(E, np.int64)
    for e in flat:
        pos.append(offsets[e] + seen[e])
        seen[e] += 1
    return offsets, np.nonzero(counts)[0], np.array(pos)


@pytest.mark.parametrize("M,E,top_k,H", [(16, 128, 8, 2048), (3, 64, 4, 512), (1, 128, 8, 2048)])
def test_router_picks_the_top_k_and_renormalizes(cuda_device, M, E, top_k, H):
    from ecf8_amd.llm_kernels import MoeRouting, moe_route

    gen = torch.Generator().manual_seed(M * 100 + E)
    x = torch.randn(M, H, generator=gen).to(torch.bfloat16)
    wr = (torch.randn(E, H, generator=gen) * 0.05).to(torch.bfloat16)
    r = MoeRouting(M, top_k, E, cuda_device)
    moe_route(x.to(cuda_device), wr.to(cuda_device), M, r)
    probs = torch.softmax(x.double() @ wr.double().T, dim=-1)
    ref_p, _ = torch.topk(probs, top_k, dim=-1)
    idx = r.topk_idx.cpu().long()
    got_p = probs.gather(1, idx)
    # the chosen experts carry the top-k probabilities, in descending order
    assert torch.allclose(got_p, ref_p, atol=1e-5, rtol=0)
    assert bool((got_p[:, :-1] >= got_p[:, 1:] - 1e-6).all())
    assert all(len(set(row)) == top_k for row in idx.tolist())
    w = r.topk_w.cpu().double()
    assert torch.allclose(w, ref_p / ref_p.sum(-1, keepdim=True), atol=1e-5, rtol=0)
    assert torch.allclose(w.sum(-1), torch.ones(M, dtype=torch.float64), atol=1e-6)


@pytest.mark.parametrize("M,top_k,E", [(16, 8, 128), (5, 3, 16), (32, 8, 256), (300, 8, 128),
                                        (1024, 8, 128)])
def test_group_sorts_pairs_by_expert(cuda_device, M, top_k, E):
    from ecf8_amd.llm_kernels import MoeRouting, moe_group

    rng = np.random.default_rng(M + E)
    idx = np.stack([rng.choice(E, top_k, replace=False) for _ in range(M)]).astype(np.int32)
    w = rng.random((M, top_k)).astype(np.float32)
    r = MoeRouting(M, top_k, E, cuda_device)
    r.topk_idx.copy_(torch.from_numpy(idx))
    r.topk_w.copy_(torch.from_numpy(w))
    moe_group(r, M)
    offsets, active, pos = _groups_ref(idx, E)
    n_act = int(r.n_active.item())
    assert n_act == len(active)
    assert np.array_equal(r.offsets.cpu().numpy(), offsets)
    assert np.array_equal(r.active.cpu().numpy()[:n_act], active)
    assert np.array_equal(r.pair_pos.cpu().numpy(), pos)
    tok = np.repeat(np.arange(M), top_k)
    got_tok = r.pair_tok.cpu().numpy()
    got_w = r.pair_w.cpu().numpy()
    assert np.array_equal(got_tok[pos], tok)
    assert np.array_equal(got_w[pos], w.reshape(-1))
    sel = np.zeros(E, np.int32)
    sel[active] = 1
    assert np.array_equal(r.select.cpu().numpy(), sel)


def _pair_linear_ref(a_rows, a_s_rows, w, ws):
    """fp64 block-scaled product of the given activation rows with one
    expert's weight (the math of the dense FP8 linear)."""
    a = a_rows.cpu().double()
    M, K = a.shape
    wd = w.cpu().double()
    n = wd.shape[0]
    part = torch.einsum("mgk,ngk->mng", a.view(M, K // 128, 128), wd.view(n, K // 128, 128))
    scale = a_s_rows.cpu().double()[:, None, :] * ws.cpu().double().repeat_interleave(128, 0)[None]
    return (part * scale).sum(-1)


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("gather", [True, False])
def test_grouped_expert_linear_matches_fp64(cuda_device, gather, layout):
    """gate/up form (gather the token rows, two segments) and down form (one
    row per sorted pair, one segment, K below 16 groups); expert weights
    row-major (layout 0) or in the tile layout (1), activations in the tile
    layout."""
    from ecf8_amd.llm_kernels import MoeLinearPlan, MoeRouting, moe_group, to_tiles

    dev = cuda_device
    gen = torch.Generator().manual_seed(11 if gather else 12)
    rng = np.random.default_rng(3)
    M, top_k, E = 16, 4, 12
    K, seg_n, n_segs = (1024, 256, 2) if gather else (768, 384, 1)
    idx = np.stack([rng.choice(E, top_k, replace=False) for _ in range(M)]).astype(np.int32)
    idx[:, 0] = 5  # one expert with all 16 tokens
    r = MoeRouting(M, top_k, E, dev)
    r.topk_idx.copy_(torch.from_numpy(idx))
    r.topk_w.fill_(0.25)
    moe_group(r, M)
    P = M * top_k
    rows = M if gather else P
    aq = _rand_fp8((rows, K), gen, dev)
    a_s = (torch.rand(rows, K // 128, generator=gen) * 1e-2 + 1e-4).to(dev)
    experts = []
    for _ in range(E):
        segs = []
        for _ in range(n_segs):
            w = _rand_fp8((seg_n, K), gen, dev)
            ws = (torch.rand(seg_n // 128, K // 128, generator=gen) * 1e-3 + 1e-5).to(dev)
            segs.append((w, ws))
        experts.append(segs)
    ldo = n_segs * seg_n + 32
    out = torch.full((P, ldo), 7.0, dtype=torch.bfloat16, device=dev)
    plan_experts = [[(to_tiles(w), ws) for w, ws in segs] for segs in experts] if layout \
        else experts
    MoeLinearPlan(plan_experts, out, layout)(to_tiles(aq), a_s, r, gather=gather)
    offsets, active, _ = _groups_ref(idx, E)
    tok = r.pair_tok.cpu().long()
    got = out.double().cpu()
    for e in active:
        q = torch.arange(int(offsets[e]), int(offsets[e + 1]))
        src = tok[q] if gather else q
        ref = torch.cat([_pair_linear_ref(aq.cpu()[src], a_s.cpu()[src], w, ws)
                         for w, ws in experts[e]], dim=1)
        g = got[q, : n_segs * seg_n]
        assert bool(((g - ref).abs() <= 2 ** -7 * ref.abs() + 1e-4 * ref.abs().max()).all()), e
    assert bool((out[:, n_segs * seg_n:].cpu() == 7.0).all())


def test_combine_weights_the_pairs_in_order(cuda_device):
    from ecf8_amd.llm_kernels import MoeRouting, moe_combine, moe_group

    dev = cuda_device
    rng = np.random.default_rng(8)
    M, top_k, E, H = 16, 8, 128, 2048
    idx = np.stack([rng.choice(E, top_k, replace=False) for _ in range(M)]).astype(np.int32)
    w = rng.random((M, top_k)).astype(np.float32)
    r = MoeRouting(M, top_k, E, dev)
    r.topk_idx.copy_(torch.from_numpy(idx))
    r.topk_w.copy_(torch.from_numpy(w))
    moe_group(r, M)
    down = torch.randn(M * top_k, H, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
    moe_combine(down.to(dev), r, M, out)
    pos = torch.from_numpy(_groups_ref(idx, E)[2]).view(M, top_k)
    ref = (torch.from_numpy(w).double()[..., None] * down.double()[pos]).sum(1)
    assert torch.allclose(out.double().cpu(), ref, rtol=2 ** -7, atol=1e-3)


# ------------------------------------------------------------ end to end


SMALL_MOE = dict(hidden=2048, layers=2, heads=16, kv_heads=2, experts=16, top_k=4,
                 moe_intermediate=256, vocab=1024)


@pytest.fixture(scope="module")
def small_moe_models(cuda_device):
    from ecf8_amd.moe import Qwen3MoeConfig, compress_moe_layers, random_moe_model

    cfg = Qwen3MoeConfig(**SMALL_MOE)
    plain, drawn = random_moe_model(cfg, cuda_device, seed=2)
    comp, _ = random_moe_model(cfg, cuda_device, seed=2)
    compress_moe_layers(comp, drawn)
    return cfg, plain, comp


def test_compressed_moe_matches_uncompressed_exactly(small_moe_models, cuda_device):
    """Attention blocks decoded by their hooks, experts decoded only when
    the router picks them (prompt: every expert), eager and graph-replayed:
    the same tokens and logits as the model kept in FP8."""
    from ecf8_amd.moe import Qwen3MoeRunner
    from dfloat.run.run import TensorManager

    cfg, plain, comp = small_moe_models
    B, T, new = 4, 40, 6
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(3))
    results = {}
    for name, model in (("fp8", plain), ("ecf8", comp)):
        for graph in (False, True):
            print(f"[moe] e2e {name} graph={graph}", flush=True)
            TensorManager.clear_device()
            # the prompt's MoE in 16-token chunks (eager) or one chunk (graph):
            # per-token results do not depend on the chunking
            r = Qwen3MoeRunner(model, B, T, T + new, cuda_device,
                               prefill_chunk=512 if graph else 16)
            if graph:
                r.capture()
            for rep in range(2):
                toks = r.generate(prompt, new).cpu()
                results[(name, graph, rep)] = (toks, r.logits.float().cpu())
    from ecf8_amd.prefetch import LayerPrefetcher

    # the next layer's attention block decoded on a side stream
    LayerPrefetcher([layer.self_attn for layer in comp.model.layers], cuda_device).install()
    for graph in (False, True):
        print(f"[moe] e2e ecf8 prefetch graph={graph}", flush=True)
        r = Qwen3MoeRunner(comp, B, T, T + new, cuda_device)
        if graph:
            r.capture()
        for rep in range(2):
            toks = r.generate(prompt, new).cpu()
            results[("ecf8_prefetch", graph, rep)] = (toks, r.logits.float().cpu())
    base_t, base_l = results[("fp8", False, 0)]
    for key, (t, l) in results.items():
        assert torch.equal(t, base_t), key
        assert torch.equal(l, base_l), key
    assert len(set(base_t.reshape(-1).tolist())) > 1


def _q128(x):
    """Activation quantization of the kernels (amax / 448 per 1x128 group,
    RNE to e4m3fn), dequantized back to fp64."""
    x = x.float().cpu()
    M, K = x.shape
    g = x.view(M, K // 128, 128)
    amax = g.abs().amax(-1)
    s = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (g / s[..., None]).to(FP8).double()
    return (q * s.double()[..., None]).view(M, K)


def _wdeq(lin):
    w = lin.weight.double().cpu()
    ws = lin.weight_scale_inv.double().cpu().repeat_interleave(128, 0).repeat_interleave(128, 1)
    return w * ws


def test_moe_block_matches_a_torch_restatement(small_moe_models, cuda_device):
    """One layer's routed MLP on a random normalized hidden state against
    a float64 torch restatement of transformers' Qwen3MoeSparseMoeBlock with
    the kernels' quantization points (relative L2 <= 1e-2: bf16 outputs
    and rare fp8 rounding flips)."""
    from ecf8_amd.moe import Qwen3MoeRunner

    cfg, plain, _ = small_moe_models
    B = 12
    r = Qwen3MoeRunner(plain, B, 1, 8, cuda_device)
    gen = torch.Generator().manual_seed(9)
    hb = torch.randn(B, cfg.hidden, generator=gen).to(torch.bfloat16)
    r.hb[:B].copy_(hb)
    mlp = plain.model.layers[0].mlp
    r._moe(mlp, 0, B, prefill=False)
    got = r.y[:B].double().cpu()
    # reference
    logits = hb.double() @ mlp.gate.weight.double().cpu().T
    p = torch.softmax(logits, -1)
    w, idx = torch.topk(p, cfg.top_k, -1)
    w = w / w.sum(-1, keepdim=True)
    x = _q128(hb)
    ref = torch.zeros(B, cfg.hidden, dtype=torch.float64)
    for t in range(B):
        for k in range(cfg.top_k):
            ex = mlp.experts[int(idx[t, k])]
            g = (x[t:t + 1] @ _wdeq(ex.gate_proj).T).to(torch.bfloat16).double()
            u = (x[t:t + 1] @ _wdeq(ex.up_proj).T).to(torch.bfloat16).double()
            h = _q128((g * torch.sigmoid(g) * u).float())
            d = (h @ _wdeq(ex.down_proj).T).to(torch.bfloat16).double()
            ref[t] += w[t, k] * d[0]
    rel = ((got - ref).norm() / ref.norm()).item()
    assert rel <= 1e-2, rel
    # routing agrees with the fp64 choice
    assert torch.equal(torch.sort(r.route.topk_idx[:B].cpu().long(), -1).values,
                       torch.sort(idx, -1).values)


def test_moe_with_a_multi_symbol_expert_matches_uncompressed(cuda_device):
    """An expert whose exponents are dominated by one value gets a 1-bit
    code, so its block needs the multi-symbol table and stays outside the
    batched launch: the routed decode still covers it, and the compressed
    model gives the FP8 model's tokens and logits, eager and graph-replayed.
    Re-tiled, that expert's layer keeps all its experts on the routed decode
    (one grouped launch serves a layer's experts) while its attention block
    and the other layer are tiled, with the same tokens and logits."""
    from dfloat.run.run import TensorManager
    from ecf8_amd.decode import build_table
    from ecf8_amd.moe import Qwen3MoeConfig, Qwen3MoeRunner, compress_moe_layers, \
        random_moe_model, retile_moe_layers

    cfg = Qwen3MoeConfig(**dict(SMALL_MOE, layers=2))
    plain, drawn = random_moe_model(cfg, cuda_device, seed=6)
    comp, _ = random_moe_model(cfg, cuda_device, seed=6)
    rng = np.random.default_rng(0)
    for name, (w, s) in drawn[0]["experts"][3].items():
        b = w.view(torch.uint8).numpy()
        skew = rng.random(b.shape) < 0.8
        b[skew] = (b[skew] & 0x87) | (11 << 3)  # exponent 11, sign and mantissa kept
        plain.model.layers[0].mlp.experts[3].get_submodule(name).weight.data.copy_(
            w.to(cuda_device))
    compress_moe_layers(comp, drawn)
    ex = comp.model.layers[0].mlp.experts[3]
    assert build_table(ex.luts).kind == MULTI
    B, T, new = 4, 24, 5
    prompt = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(4))
    results = {}

    def run(name, model):
        for graph in (False, True):
            print(f"[moe multi] {name} graph={graph}", flush=True)
            TensorManager.clear_device()
            r = Qwen3MoeRunner(model, B, T, T + new, cuda_device)
            if graph:
                r.capture()
            toks = r.generate(prompt, new).cpu()
            results[(name, graph)] = (toks, r.logits.float().cpu())
            del r

    run("fp8", plain)
    run("ecf8", comp)
    retile_moe_layers(comp, drawn)
    untiled = dict(comp._ecf8_untiled)
    assert list(untiled) == ["model.layers.0.mlp.experts"], untiled
    assert "experts.3" in untiled["model.layers.0.mlp.experts"]
    l0, l1 = comp.model.layers
    assert hasattr(l0.self_attn, "_ecf8_tiles") and hasattr(l1.self_attn, "_ecf8_tiles")
    assert all(hasattr(e, "encoded") and not hasattr(e, "_ecf8_tiles") for e in l0.mlp.experts)
    assert all(hasattr(e, "_ecf8_tiles") and not hasattr(e, "encoded") for e in l1.mlp.experts)
    run("fused", comp)
    base_t, base_l = results[("fp8", False)]
    for key, (t, l) in results.items():
        assert torch.equal(t, base_t), key
        assert torch.equal(l, base_l), key
