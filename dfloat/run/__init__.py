"""Runtime names of the reference's ``dfloat.run`` (dfloat/run/__init__.py:1-17)."""

from .run import (
    DFloatDiffSynthModelFP8,
    DFloatModel,
    TensorManager,
    _decode,
    get_dfloat_model_name_or_path,
    get_hook,
    load_and_replace_tensors,
    load_and_replace_tensors_parallel,
)

__all__ = [
    "DFloatModel",
    "_decode",
    "get_dfloat_model_name_or_path",
    "load_and_replace_tensors",
    "load_and_replace_tensors_parallel",
    "DFloatDiffSynthModelFP8",
    "TensorManager",
    "get_hook",
]
