"""CPU oracle for the weight-only quantized Linear (test infrastructure only).

This package is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped path (``ondeviceinfer_amd``) never imports, links or
calls anything here, and raises when its HIP library is missing instead of
falling back to the CPU.

Modules
-------
``qdq``
    numpy restatement of the reference's explicit QDQ path
    (``ondeviceinfer/weight_quantization/backend.py:26-54``,
    ``ondeviceinfer/quantization.py:226-353``,
    ``ondeviceinfer/quantized_model.py:76-121``,
    ``benchmarks/validate_weight_reconstruction.py:20-31``) plus the parity
    metrics of ``benchmarks/validate_weight_quant_kernels.py:55-76``.
``tile_layout``
    numpy model of this build's own gfx950 tile layout (the repack target).
    It has no reference counterpart; it is pinned by bit-exact round trips and
    by decode equality with ``qdq.decode_weight``.
``synth``
    seeded synthetic inputs (AWQ-style asymmetric uint4 RTN, the INT8
    config-1 weights) used by tests and the benchmark.

Pinning status of every function is listed in each module's header.
"""
