"""Per-runtime transfer counters, the ``runtime.stats`` object of the
reference's runtimes (``ondeviceinfer/runtime/offload.py:126-144``; set by
``weight_quantization/backend.py:134-135`` and ``runtime/quantized.py:448-455``).

The resident runtimes here copy every decoder tensor to the GPU once, at
construction, so ``startup_h2d_bytes`` is the only counter they set; the
per-forward counters stay at zero and exist because the reference's harnesses
read and reset them (``benchmarks/benchmark_weight_quant_models.py:64``,
``benchmarks/benchmark_quantized.py:92``).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass
class RuntimeStats:
    startup_h2d_bytes: int = 0
    weight_h2d_bytes: int = 0
    synchronous_copy_seconds: float = 0.0
    # (start, end) event pairs of asynchronous weight copies, timed on demand
    async_copy_events: list = field(default_factory=list)

    def reset_forward_counters(self) -> None:
        """Zero what one forward accumulates; ``startup_h2d_bytes`` stays."""
        self.weight_h2d_bytes = 0
        self.synchronous_copy_seconds = 0.0
        self.async_copy_events.clear()

    def async_copy_seconds(self) -> float:
        """Summed duration of the recorded asynchronous copies, in seconds
        (synchronizes the device first when there are any)."""
        if not self.async_copy_events:
            return 0.0
        torch.cuda.synchronize()
        return sum(start.elapsed_time(end) for start, end in self.async_copy_events) / 1000.0
