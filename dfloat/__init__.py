"""dfloat -- the Python API of zeyuyang8/ecf8, served by the MI355X engine.

A user of the reference keeps its imports unchanged:

* ``dfloat.run``    runtime: ``_decode`` (the decode launch in the reference's
                    call form), ``TensorManager``, the forward-pre-hook,
                    the loaders, ``DFloatModel`` and ``DFloatDiffSynthModelFP8``;
* ``dfloat.utils``  codec: FP8 split, block flattening, codebook, LUTs and
                    the bitstream encoder;
* ``dfloat.const``  the block patterns per model class;
* ``dfloat.compress`` the per-block compression pipeline and checkpoint
                    writer of the reference's ``scripts/compress.py``.

Decoding runs in the gfx950 HIP kernels of ``ecf8_amd/libecf8.so`` (through
``ecf8_amd.decode``); without that library every decode raises
``ECF8Error`` -- there is no CPU path.
"""

__version__ = "0.2.0"
