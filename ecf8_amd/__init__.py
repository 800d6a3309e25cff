"""ecf8_amd -- the MI355X (gfx950) ECF8 decode engine behind ``dfloat``.

* ``libecf8.so`` (``csrc/``): the HIP decode kernels, the consumer kernels
  of the end-to-end flows and the host codec, behind the C ABI of
  ``include/ecf8.h`` and ``include/ecf8_llm.h``;
* ``decode``, ``llm_kernels``: ctypes wrappers of that ABI with argument
  checks;
* ``llm``, ``moe``, ``dit``, ``prefetch``: the Qwen3-8B-, Qwen3-30B-A3B- and
  FLUX-shaped engines that consume the decoded weights.

The reference's Python API (``dfloat.run``, ``dfloat.utils``,
``dfloat.const``) lives in the ``dfloat`` package and calls this engine.
Importing does not need the library; calling it does, and raises
``ECF8Error`` if it is missing.
"""

__version__ = "0.2.0"
