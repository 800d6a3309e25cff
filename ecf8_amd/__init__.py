"""ecf8_amd -- ECF8 (Huffman-coded FP8 exponent) decode engine for MI355X.

Mirrors the reference package ``dfloat`` (zeyuyang8/ecf8): ``ecf8_amd.run``
holds the runtime names of ``dfloat.run`` and ``ecf8_amd.utils`` the codec
names of ``dfloat.utils``.  Decoding runs in the HIP kernels of
``ecf8_amd/libecf8.so``; importing the runtime does not need the library,
calling it does, and raises ``ECF8Error`` if it is missing.
"""

__version__ = "0.1.0"
