"""transformers' ``FP8Linear`` served by the engine's block-scaled FP8 linear.

An FP8 checkpoint loaded by transformers (``quantization_config`` with
``quant_method: fp8``) holds every quantized Linear as
``transformers.integrations.finegrained_fp8.FP8Linear``: ``weight`` e4m3fn
[N, K], ``weight_scale_inv`` fp32 per 128x128 block, activations quantized
dynamically per 1x128 group.  Its forward calls a DeepGEMM or Triton kernel
fetched from the hub (``finegrained_fp8.py:182-290``), which neither exists
for gfx950 nor can be fetched offline.  The reference's inference flow
(scripts/inference_llm.py:94-137) runs ``generate`` over exactly these
modules, with each decoder layer's forward-pre-hook injecting the decoded
``weight`` views first (dfloat/run/run.py:84-155).

``bind_fp8_linears`` rebinds each such module's ``forward`` to
``engine_fp8_linear``: the activations (rounded to bf16 first when the model
runs in another dtype) are quantized per 1x128 group by ``ecf8_act_quant``
(scale = amax/448, round to nearest even), multiplied by
``ecf8_fp8_linear`` (per-group fp32 dot products scaled by both scales,
fixed summation order) and returned as bf16, cast to the input's dtype.
The same binding serves a compressed and an uncompressed model, so the two
give identical logits when the decoded weights are bit-exact.  There is no
CPU path: a CPU input raises ``ECF8Error``.
"""

from __future__ import annotations

import types

import torch

from . import llm_kernels as K
from ._lib import ECF8Error

_BOUND = "_ecf8_bound_forward"


def fp8_linear_class():
    """transformers' FP8Linear class, or None when transformers lacks it."""
    try:
        from transformers.integrations.finegrained_fp8 import FP8Linear
    except ImportError:
        return None
    return FP8Linear


def engine_fp8_linear(x: torch.Tensor, weight: torch.Tensor, scale_inv: torch.Tensor,
                      bias: torch.Tensor | None = None) -> torch.Tensor:
    """y[..., N] = x[..., K] @ dequant(weight)^T (+ bias) with the engine's
    numerics: weight e4m3fn [N, K] and scale_inv fp32 [N/128, K/128] (N and
    K multiples of 128), activations quantized per 1x128 group."""
    if not x.is_cuda:
        raise ECF8Error("engine_fp8_linear needs CUDA tensors (there is no CPU path)")
    if weight.dtype != torch.float8_e4m3fn or weight.dim() != 2:
        raise ECF8Error(f"weight must be 2-D float8_e4m3fn, got {weight.dtype} {tuple(weight.shape)}")
    n, k = weight.shape
    if x.shape[-1] != k:
        raise ECF8Error(f"input has {x.shape[-1]} features, weight expects {k}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, k)
    m = x2.shape[0]
    if m == 0:
        return x.new_empty(*lead, n)
    xb = x2.to(torch.bfloat16).contiguous()
    dev = x.device
    aq = torch.empty(K.pad16(m), k, dtype=torch.float8_e4m3fn, device=dev)  # tile layout
    a_scale = torch.empty(m, k // K.GROUP, dtype=torch.float32, device=dev)
    K.act_quant(xb, m, aq, a_scale)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    K.fp8_linear(aq, a_scale, [(weight.contiguous(), scale_inv.float().contiguous())], out, m)
    if bias is not None:
        out = out + bias.to(out.dtype)
    return out.reshape(*lead, n).to(x.dtype)


def _fp8linear_forward(self, input: torch.Tensor) -> torch.Tensor:
    """FP8Linear.forward (finegrained_fp8.py:335-350) on the engine."""
    weight = self.weight
    if weight.element_size() > 1:
        # a dequantized (bf16/fp32) weight: FP8Linear's own fallback
        return torch.nn.functional.linear(input, weight, self.bias)
    if self.block_size is None or tuple(self.block_size) != (K.GROUP, K.GROUP):
        raise ECF8Error(f"FP8Linear with block_size {self.block_size}: only 128x128 block "
                        "scales are served")
    if getattr(self, "activation_scale", None) is not None:
        raise ECF8Error("FP8Linear with a static activation scale is not served "
                        "(only the dynamic per-group scheme)")
    return engine_fp8_linear(input, weight, self.weight_scale_inv, self.bias)


def bind_fp8_linears(model: torch.nn.Module) -> int:
    """Rebind the forward of every FP8Linear under ``model`` to the engine
    (idempotent); returns how many modules are bound."""
    cls = fp8_linear_class()
    if cls is None:
        return 0
    count = 0
    for module in model.modules():
        if isinstance(module, cls):
            if not module.__dict__.get(_BOUND):
                module.forward = types.MethodType(_fp8linear_forward, module)
                module.__dict__[_BOUND] = True
            count += 1
    return count
