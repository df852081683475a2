"""MI355X-native (gfx950) weight-only quantized Linear for OnDeviceInfer.

Python host on PyTorch-ROCm over a C-ABI HIP library
(``libondeviceinfer_wq.so``, interface in ``include/ondeviceinfer_wq.h``):

* ``weight_quantization.backend``: the pluggable compressed Linear
  (``CompressedLinearBackend``, ``decode_weight``, ``load_compressed_store``,
  ``CompressedResidentRuntime``);
* ``quantization``: the INT8 per-output-channel format and ops;
* ``quantized_model``: the runtime INT8 weight-only linear;
* ``runtime.quantized``: layer tensor names.
"""
__version__ = '0.1.0'
