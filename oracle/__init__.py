"""CPU oracle for the PLaMo-3 0.8B token loop -- TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped runtime (``plamo3-0.8b-runtime_amd``) never imports,
links or executes anything here, and fails loudly when its HIP library is
missing instead of falling back to this code.

Modules (each function cites the reference file:line it restates):

* ``bf16``    -- BF16 round-to-nearest-even exactly as ``Kernels.metal:5-10``.
* ``p12``     -- the lossless ``.p12`` block packing (``scripts/pack_weights.py:19-86``),
                 the GPU decode (``Kernels.metal:23-44``) and the archive chain
                 validation (``Sources/Plamo/Packed.swift:12-91``).
* ``rope``    -- RoPE cos/sin tables shared bit-for-bit with the runtime.
* ``model``   -- the full forward pass (``Runtime.swift:327-483`` with the kernel
                 arithmetic of ``Kernels.metal``) in PyTorch-CPU FP32 with BF16
                 rounding at the reference's points, plus an independent
                 textbook forward used to pin it.
* ``sampler`` -- greedy argmax (``Kernels.metal:704-729``), ``Sampler.select`` /
                 ``forbidden`` (``Sampler.swift:9-70``) and ``decodeBatch``
                 (``BatchDecode.swift:8-37``).
* ``tokenizer`` -- the unigram tokenizer (``Tokenizer.swift:59-269``): vocabulary rules,
                 boundary segmentation, Viterbi with byte fallback, decode and stream.

Pinning status of every function is listed in each module header.
"""
