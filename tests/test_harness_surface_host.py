"""The attributes the reference's own harnesses touch on the product objects
(CPU only):

* ``benchmarks/benchmark_weight_quant_models.py:52-96``: ``model.runtime.stats``
  (``startup_h2d_bytes``), ``model.dequant_scratch`` (numel x element size),
  ``model.runtime.resident_storage_bytes``, the backend's counters and
  ``marlin_*`` flags, ``model.compute_stats``, ``model.store.manifest``;
* ``benchmarks/benchmark_quantized.py:92``: ``runtime.stats.reset_forward_counters()``;
* ``benchmarks/validate_weight_quant_kernels.py:44-77``: ``backend.ops.scaled_int8_quant``,
  ``prepare`` / ``linear`` / ``fallback_count``, ``LINEAR_WEIGHT_NAMES``;
* ``ondeviceinfer/quantized_model.py:302-327``: the cache's lifecycle hooks and
  ``layer_probe_callback`` around every decoder layer
  (``benchmarks/validate_weight_quant.py:152``).
"""
import dataclasses
import inspect

import pytest
import torch
import torch.nn.functional as F

from ondeviceinfer_amd.cache import ResidentKVCache
from ondeviceinfer_amd.config import Qwen3Config
from ondeviceinfer_amd.functional import rms_norm
from ondeviceinfer_amd.quantized_model import QuantizedQwen3ForCausalLM
from ondeviceinfer_amd.runtime.quantized import (LINEAR_WEIGHT_NAMES, QuantizedCpuWeightStore,
                                                 QuantizedResidentRuntime, layer_shapes, qweight_name, scale_name,
                                                 validate_int8_layer)
from ondeviceinfer_amd.runtime.stats import RuntimeStats
from ondeviceinfer_amd.weight_quantization.backend import (CompressedLinearBackend, CompressedResidentRuntime,
                                                           NativeOps)
from ondeviceinfer_amd.weight_quantization.synthetic import random_compressed_store


def tiny_config(layers=3):
    return Qwen3Config(vocab_size=97, hidden_size=256, intermediate_size=384, num_hidden_layers=layers,
                       num_attention_heads=2, num_key_value_heads=1, head_dim=128, max_position_embeddings=64,
                       rms_norm_eps=1e-6, rope_theta=1_000_000.0, tie_word_embeddings=False)


def test_runtime_stats_semantics():
    stats = RuntimeStats(startup_h2d_bytes=123)
    stats.weight_h2d_bytes, stats.synchronous_copy_seconds = 7, 0.5
    stats.async_copy_events.append(('start', 'end'))
    stats.reset_forward_counters()
    assert (stats.startup_h2d_bytes, stats.weight_h2d_bytes, stats.synchronous_copy_seconds) == (123, 0, 0.0)
    assert stats.async_copy_events == [] and stats.async_copy_seconds() == 0.0


def test_compressed_runtime_stats_and_storage():
    cfg = tiny_config(2)
    store = random_compressed_store(cfg, seed=1)
    backend = CompressedLinearBackend('reference_int4')    # prepare keeps the raw tensors: no GPU needed
    runtime = CompressedResidentRuntime(store, backend, device='cpu', verbose=False)
    expected = sum(v.numel() * v.element_size() for layer in store.layers for v in layer.values()
                   if isinstance(v, torch.Tensor))
    assert runtime.stats.startup_h2d_bytes == expected == runtime.startup_h2d_bytes
    runtime.stats.reset_forward_counters()
    assert runtime.stats.startup_h2d_bytes == expected and runtime.stats.async_copy_seconds() == 0.0
    assert not hasattr(runtime.stats, 'h2d_bytes')            # the harness then records weight_h2d_bytes = 0
    assert runtime.resident_storage_bytes == 0                # CPU tensors are not counted (cuda only)
    assert runtime.gpu_layer_budget == 2 and runtime.weights_for(1) is runtime.resident[1]


def _int8_store(cfg):
    gen = torch.Generator().manual_seed(3)
    norms, linears = layer_shapes(cfg)
    layers = []
    for _ in range(cfg.num_hidden_layers):
        layer = {name: torch.ones(shape, dtype=torch.float16) for name, shape in norms.items()}
        for name, (n, k) in linears.items():
            layer[qweight_name(name)] = torch.randint(-127, 128, (n, k), generator=gen, dtype=torch.int8)
            layer[scale_name(name)] = torch.full((n,), 0.01, dtype=torch.float16)
        layers.append(layer)
    z = torch.zeros(cfg.vocab_size, cfg.hidden_size, dtype=torch.float16)
    return QuantizedCpuWeightStore(config=cfg, layers=layers, embed_tokens=z, final_norm=torch.ones(cfg.hidden_size,
                                   dtype=torch.float16), lm_head=z, compute_dtype=torch.float16,
                                   manifest={'source': 'synthetic'})


def test_int8_runtime_stats():
    cfg = tiny_config(2)
    store = _int8_store(cfg)
    runtime = QuantizedResidentRuntime(store, device='cpu')
    assert runtime.stats.startup_h2d_bytes == store.decoder_bytes == runtime.startup_h2d_bytes
    runtime.stats.reset_forward_counters()
    assert runtime.stats.weight_h2d_bytes == 0 and runtime.stats.startup_h2d_bytes == store.decoder_bytes
    assert runtime.resident_count == runtime.gpu_layer_budget == 2


def test_int8_layer_shapes_follow_the_reference():
    """q_proj and o_proj must be (hidden, hidden), as the reference's
    _validate_layer requires, also when a config object (built without
    Qwen3Config.validate) has heads * head_dim != hidden."""
    cfg = dataclasses.replace(tiny_config(1), num_attention_heads=4)   # 4 * 128 = 512 != hidden 256
    layer = _int8_store(tiny_config(1)).layers[0]
    validate_int8_layer(layer, 0, cfg)
    bad = dict(layer)
    bad[qweight_name('self_attn.q_proj.weight')] = torch.zeros(512, 256, dtype=torch.int8)
    bad[scale_name('self_attn.q_proj.weight')] = torch.full((512,), 0.01, dtype=torch.float16)
    with pytest.raises(ValueError, match='Invalid shape for layer 0 self_attn.q_proj.weight'):
        validate_int8_layer(bad, 0, cfg)


def test_scaled_int8_quant_surface():
    """``backend.ops.scaled_int8_quant(x)`` as the kernel harness calls it;
    static scales and asymmetric quantization are refused, CPU input too."""
    ops = CompressedLinearBackend('int8_gemm').ops
    assert isinstance(ops, NativeOps)
    params = inspect.signature(ops.scaled_int8_quant).parameters
    assert list(params)[:4] == ['x', 'scale', 'azp', 'symmetric']
    x = torch.zeros(2, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match='symmetric'):
        ops.scaled_int8_quant(x, symmetric=False)
    with pytest.raises(ValueError, match='symmetric'):
        ops.scaled_int8_quant(x, scale=torch.ones(1))
    with pytest.raises(Exception, match='GPU|cuda|device'):
        ops.scaled_int8_quant(x)


def test_backend_report_fields():
    """Every backend field the two harnesses record, with its type."""
    for name in ('marlin', 'int8_gemm', 'reference_int4', 'reference_w8a8'):
        b = CompressedLinearBackend(name)
        assert b.name == name and callable(b.prepare) and callable(b.linear)
        for field in ('calls', 'gemm_calls', 'fallback_count', 'explicit_dequant_bytes', 'activation_quantize_calls',
                      'marlin_max_rows_per_call'):
            assert isinstance(getattr(b, field), int)
        assert isinstance(b.marlin_use_fp32_reduce, bool)
    assert len(LINEAR_WEIGHT_NAMES) == 7


class _DenseBackend:
    """A linear backend over fp16 dense weights in the layer dicts, so the
    eager forward runs on the CPU (the hooks under test are host logic)."""
    name = 'dense'

    def __init__(self, dense):
        self.dense = dense
        self.calls = 0

    def prepare(self, layer, name):
        pass

    def linear(self, inputs, weights, name):
        self.calls += 1
        return F.linear(inputs.float(), weights[name].float()).half()


class _HookedCache(ResidentKVCache):
    """A resident cache with the offloaded caches' lifecycle hooks, recording
    the order they are called in."""

    def __init__(self, log, **kw):
        super().__init__(**kw)
        self.log = log

    def begin_forward(self, *, query_length):
        self.log.append(('begin_forward', query_length))

    def before_layer(self, idx):
        self.log.append(('before_layer', idx))

    def after_layer(self, idx):
        self.log.append(('after_layer', idx))

    def end_forward(self):
        self.log.append(('end_forward',))


def _dense_model(cfg):
    gen = torch.Generator().manual_seed(5)
    norms, linears = layer_shapes(cfg)
    layers = []
    for _ in range(cfg.num_hidden_layers):
        layer = {name: (1 + 0.1 * torch.randn(shape, generator=gen)).half() for name, shape in norms.items()}
        for name, (n, k) in linears.items():
            layer[name] = (torch.randn(n, k, generator=gen) * 0.05).half()
        layers.append(layer)

    class Store:
        config = cfg
        embed_tokens = (torch.randn(cfg.vocab_size, cfg.hidden_size, generator=gen) * 0.5).half()
        final_norm = torch.ones(cfg.hidden_size, dtype=torch.float16)
        lm_head = (torch.randn(cfg.vocab_size, cfg.hidden_size, generator=gen) * 0.05).half()
        compute_dtype = torch.float16
        manifest = {}
    Store.layers = layers
    backend = _DenseBackend(layers)
    runtime = CompressedResidentRuntime(Store, backend, device='cpu', verbose=False)
    return QuantizedQwen3ForCausalLM(Store, runtime, device='cpu', linear_backend=backend)


def test_cache_hooks_and_layer_probe_order():
    cfg = tiny_config(3)
    model = _dense_model(cfg)
    assert model.layer_probe_callback is None
    assert model.dequant_scratch.numel() * model.dequant_scratch.element_size() == 0
    assert model.dequant_scratch.is_contiguous()
    log, probes = [], {}
    model.layer_probe_callback = lambda idx, hidden: (log.append(('probe', idx)),
                                                      probes.__setitem__(idx, hidden.clone()))
    cache = _HookedCache(log, num_layers=3, batch_size=1, num_key_value_heads=1, max_seq_len=16, head_dim=128,
                         device='cpu', dtype=torch.float16)
    ids = torch.tensor([[3, 14, 15, 92, 65]])
    out = model(ids, cache=cache)
    layer_calls = [e for i in range(3) for e in (('before_layer', i), ('probe', i), ('after_layer', i))]
    assert log == [('begin_forward', 5), *layer_calls, ('end_forward',)]
    assert sorted(probes) == [0, 1, 2] and probes[2].shape == (1, 5, cfg.hidden_size)
    # The probe sees the hidden state the final norm and LM head consume.
    expected = F.linear(rms_norm(probes[2], model.final_norm, cfg.rms_norm_eps).float(), model.lm_head.float())
    assert torch.allclose(out.logits.float(), expected, atol=2e-2, rtol=1e-2)
    # A decode token (one more position) goes through the hooks too.
    log.clear()
    model(torch.tensor([[7]]), cache=cache)
    assert log[0] == ('begin_forward', 1) and log[-1] == ('end_forward',) and len(log) == 2 + 3 * 3
    # Without a probe nothing is called on the model side, and a cache
    # without hooks is fine.
    model.layer_probe_callback = None
    plain = ResidentKVCache(num_layers=3, batch_size=1, num_key_value_heads=1, max_seq_len=16, head_dim=128,
                            device='cpu', dtype=torch.float16)
    again = model(ids, cache=plain)
    assert torch.equal(again.logits, out.logits)
