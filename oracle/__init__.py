"""CPU oracle for the ECF8 decode path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of the reference project
(zeyuyang8/ecf8) for the ECF8 exponent codec, so that the HIP decoder shipped
in ``ecf8_amd`` can be checked against it.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and there only as the checker or as the timed CPU baseline.  The
product (``ecf8_amd``) never imports, links or calls anything in here.

Contents
--------
``codec.py``        pure-Python restatement (small inputs):
                    FP8 split/merge      dfloat/utils.py:207-227
                    Huffman code table   dahuffman HuffmanCodec.from_frequencies
                                         (third party, called at
                                         dfloat/utils.py:240,259)
                    length limiter       dfloat/utils.py:239-267
                    LUT builder          dfloat/utils.py:270-370
                    bitstream encoder    dfloat/utils.py:373-499
                    decode rule          dfloat/run/decode.cu:15-211
``ecf8_oracle.c``   the same encoder and decode rule in plain C, for large
                    inputs and as the CPU baseline (built by ``Makefile``).
``native.py``       ctypes loader for the C restatement.

Pinning status (what each function is checked against, in tests/):
  split/merge      all 256 byte values + e4m3fn value decomposition (closed form)
  Huffman table    Kraft equality, prefix-freeness, optimal cost vs textbook
                   Huffman; exact dahuffman code assignment: parity unpinned
                   (dahuffman is neither vendored nor installed, and the
                   reference ships no golden vectors)
  LUT builder      brute force over every code word x every 16-bit padding;
                   the worked example of docs/assets/figures/lookup_table.png
  encoder          bit-string brute force + closed-form gap/position
                   invariants on small inputs; C vs Python restatement
  decode rule      round trip against the original FP8 bytes (the
                   reference's own check, scripts/compress.py:126)
"""
