"""Host-side behaviour of the backend and INT8 modules (CPU only).

Mirrors the reference's own host tests: row-split dispatch with a fake op
(``tests/test_weight_quant_backend.py:48-66``), scratch reuse and manifest
round trip (``tests/test_quantization.py:65-114``), loader validation
(``backend.py:69-128``), plus the no-fallback contract.
"""
import json
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from ondeviceinfer_amd import quantization as q8
from ondeviceinfer_amd.quantized_model import int8_weight_only_linear
from ondeviceinfer_amd.runtime.quantized import LINEAR_WEIGHT_NAMES, NORM_WEIGHT_NAMES
from ondeviceinfer_amd.weight_quantization import backend as wq
from oracle import synth

KAT = json.loads((Path(__file__).parent / 'golden' / 'weight_quant_kat.json').read_text())


def test_backend_names():
    with pytest.raises(ValueError):
        wq.CompressedLinearBackend('bogus')
    for name in ('reference_int4', 'reference_w8a8', 'int8_gemm', 'w8a16', 'marlin'):
        b = wq.CompressedLinearBackend(name)
        assert (b.calls, b.gemm_calls, b.fallback_count, b.explicit_dequant_bytes,
                b.activation_quantize_calls) == (0, 0, 0, 0, 0)


def test_int8_gemm_prepare_and_dispatch():
    """``prepare`` keeps the INT8 weight as stored with an fp32 scale
    (``backend.py:227-231``); ``linear`` quantizes the activations once and
    runs one scaled INT8 GEMM per call, counting both (``:249-256``)."""
    backend = wq.CompressedLinearBackend('int8_gemm')
    q = torch.randint(-127, 128, (24, 64), dtype=torch.int8)
    layer = {'mlp.up_proj.weight': q, 'mlp.up_proj.weight_scale': torch.rand(24, 1).half()}
    backend.prepare(layer, 'mlp.up_proj.weight')
    p = layer['mlp.up_proj._prepared']
    assert isinstance(p, wq.PreparedW8A8) and (p.k, p.n) == (64, 24)
    assert p.scale.dtype == torch.float32 and p.scale.shape == (24,) and torch.equal(p.qweight, q)
    seen = []

    def fake_quant(x):
        seen.append(('quant', tuple(x.shape)))
        return x.round().to(torch.int8), torch.ones(x.shape[0])

    def fake_linear(qx, sx, prepared, output=None):
        seen.append(('gemm', tuple(qx.shape)))
        return qx.float().half() @ prepared.qweight.t().float().half()

    backend.ops = SimpleNamespace(w8a8_quantize=fake_quant, w8a8_linear=fake_linear)
    out = backend.linear(torch.randn(2, 3, 64), layer, 'mlp.up_proj.weight')
    assert out.shape == (2, 3, 24)
    assert seen == [('quant', (6, 64)), ('gemm', (6, 64))]
    assert (backend.calls, backend.gemm_calls, backend.activation_quantize_calls) == (1, 1, 1)
    with pytest.raises(TypeError, match='expected INT8'):
        backend.prepare({'x.weight': q.float(), 'x.weight_scale': torch.ones(24, 1)}, 'x.weight')


def test_row_split_dispatch_preserves_shape_and_counts():
    c = KAT['kat_row_dispatch']
    backend = object.__new__(wq.CompressedLinearBackend)
    backend.name = 'marlin'
    backend.calls = backend.gemm_calls = 0
    backend.marlin_max_rows_per_call = c['max_rows']
    widths = []

    def fake(a, prepared, output=None):
        widths.append(a.shape[0])
        assert a.shape[0] <= c['max_rows']
        actual = a @ prepared.tiles.t()
        if output is not None:
            output.copy_(actual)
            return output
        return actual

    backend.ops = SimpleNamespace(w4a16_linear=fake)
    weight = torch.randn(c['n'], c['x_shape'][-1])
    x = torch.randn(*c['x_shape'])
    weights = {'mlp.up_proj._prepared': wq.PreparedW4(weight, None, None, c['x_shape'][-1], c['n'], 128)}
    out = backend.linear(x, weights, 'mlp.up_proj.weight')
    assert out.shape == (*c['x_shape'][:-1], c['n'])
    assert torch.allclose(out, x @ weight.t())
    assert widths == c['expected_widths']
    assert backend.calls == c['expected_calls'] and backend.gemm_calls == c['expected_gemm_calls']


def test_linear_epilogue_dispatch_on_the_host():
    """``linear_epilogue`` takes the fused prefill GEMM only for prepared W4
    weights on the GEMM grids that carry the epilogue (the predicate is host
    logic in the library, no GPU call); otherwise it returns None and the
    decoder runs the linear and the elementwise op as two steps."""
    from ondeviceinfer_amd import _native
    silu, res = _native.EPI_SILU_MUL, _native.EPI_RESIDUAL
    sup = _native.w4a16_epilogue_supported
    assert sup(4096, 34816, 5120, 128, silu) and sup(4096, 5120, 17408, 128, res)
    assert sup(65, 34816, 1024, 128, silu) and not sup(64, 34816, 1024, 128, silu)   # decode GEMV rows
    assert not sup(4096, 2040, 512, 128, silu)                  # n % 32: gate and up not whole tiles
    assert sup(2560, 1024, 1024, 128, res) and not sup(2560, 1024, 1024, 128, silu)   # one tile per wave
    assert not sup(200, 1024, 1024, 128, res)                   # deep-ring grid
    assert not sup(4096, 5120, 5120, 64, res) and not sup(4096, 5120, 5120, 128, 3)
    x = torch.zeros(64, 64)
    assert wq.CompressedLinearBackend('reference_int4').linear_epilogue(
        x, {}, 'mlp.down_proj.weight', res, x) is None
    backend = wq.CompressedLinearBackend('marlin')
    w8 = {'mlp.down_proj._prepared': wq.PreparedW8(None, None, 64, 64)}
    assert backend.linear_epilogue(x, w8, 'mlp.down_proj.weight', res, x) is None
    w4 = {'mlp.gate_up_proj._prepared': wq.PreparedW4(None, None, None, 5120, 34816, 128)}
    assert backend.linear_epilogue(torch.zeros(64, 5120), w4, 'mlp.gate_up_proj.weight', silu) is None
    assert backend.calls == 0 and backend.gemm_calls == 0


def test_no_cpu_path():
    weights, _ = synth.w4_case(16, 256, 1, name='p.weight')
    layer = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in weights.items()}
    with pytest.raises(ValueError, match='GPU'):
        wq.decode_weight(layer, 'p.weight')
    with pytest.raises(ValueError, match='GPU'):
        q8.quantize_linear_weight(torch.randn(4, 8))
    with pytest.raises(ValueError):          # shape checks come first, as in the reference
        q8.quantize_linear_weight(torch.randn(4))


def test_container_validation_and_manifest_round_trip():
    with pytest.raises(TypeError):
        q8.QuantizedLinearWeight(torch.zeros(2, 2, dtype=torch.int16), torch.ones(2))
    with pytest.raises(ValueError):
        q8.QuantizedLinearWeight(torch.zeros(2, 2, dtype=torch.int8), torch.ones(3))
    with pytest.raises(ValueError):
        q8.QuantizedLinearWeight(torch.zeros(2, 2, dtype=torch.int8), torch.tensor([1.0, 0.0]))
    with pytest.raises(ValueError):
        q8.QuantizedLinearWeight(torch.zeros(2, 2, dtype=torch.int8), torch.tensor([1.0, float('inf')]))
    w = q8.QuantizedLinearWeight(torch.zeros(4, 6, dtype=torch.int8), torch.ones(4, dtype=torch.float16))
    prefix = 'model.layers.0.self_attn.q_proj.weight'
    restored = q8.QuantizedLinearWeight.from_tensor_dict(w.tensor_dict(prefix), prefix)
    manifest = w.manifest_entry(prefix)
    assert restored.qweight is w.qweight and restored.scale is w.scale
    assert manifest['format'] == q8.QUANTIZATION_FORMAT and manifest['axis'] == 0
    assert manifest['shape'] == [4, 6]
    assert manifest['qweight_key'].endswith('.qweight') and manifest['scale_key'].endswith('.scale')


def test_scratch_capacity_and_reuse():
    first = q8.QuantizedLinearWeight(torch.zeros(5, 8, dtype=torch.int8), torch.ones(5))
    second = q8.QuantizedLinearWeight(torch.zeros(3, 8, dtype=torch.int8), torch.ones(3))
    scratch = q8.FP16DequantScratch.for_weights([first, second], device='cpu')
    assert scratch.capacity == 40
    assert scratch.view_for((5, 8)).data_ptr() == scratch.view_for((3, 8)).data_ptr() == scratch.buffer.data_ptr()
    with pytest.raises(ValueError, match='smaller than required'):
        scratch.view_for((6, 8))
    with pytest.raises(TypeError):
        q8.FP16DequantScratch(torch.empty(4))
    with pytest.raises(ValueError):
        q8.FP16DequantScratch.allocate(0, device='cpu')


def test_int8_runtime_linear_validation():
    weights = {'self_attn.q_proj.qweight': torch.zeros(4, 8, dtype=torch.int8),
               'self_attn.q_proj.scale': torch.ones(4, dtype=torch.float16)}
    x = torch.zeros(1, 8, dtype=torch.float16)
    with pytest.raises(KeyError):
        int8_weight_only_linear(x, weights, 'lm_head.weight', torch.empty(64, dtype=torch.float16))
    with pytest.raises(ValueError, match='Scratch has'):
        int8_weight_only_linear(x, weights, 'self_attn.q_proj.weight', torch.empty(16, dtype=torch.float16))
    with pytest.raises(ValueError, match='GPU'):
        int8_weight_only_linear(x, weights, 'self_attn.q_proj.weight', torch.empty(64, dtype=torch.float16))


# ---------------------------------------------------------------- compressed-tensors loader

TINY = dict(model_type='qwen3', vocab_size=64, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
            num_attention_heads=2, num_key_value_heads=1, head_dim=128, max_position_embeddings=128,
            rms_norm_eps=1e-6, rope_theta=1e6, tie_word_embeddings=True)


def write_tiny_checkpoint(path: Path, *, int8_layer: int | None = None, mutate=None) -> None:
    path.mkdir(parents=True, exist_ok=True)
    cfg = dict(TINY, quantization_config={'format': 'pack-quantized', 'group_size': 128})
    (path / 'config.json').write_text(json.dumps(cfg))
    h, i, kv = TINY['hidden_size'], TINY['intermediate_size'], TINY['num_key_value_heads'] * TINY['head_dim']
    shapes = {'self_attn.q_proj.weight': (h, h), 'self_attn.k_proj.weight': (kv, h),
              'self_attn.v_proj.weight': (kv, h), 'self_attn.o_proj.weight': (h, h),
              'mlp.gate_proj.weight': (i, h), 'mlp.up_proj.weight': (i, h), 'mlp.down_proj.weight': (h, i)}
    tensors = {'model.embed_tokens.weight': torch.randn(64, h, dtype=torch.float16),
               'model.norm.weight': torch.ones(h, dtype=torch.float16)}
    rng = np.random.default_rng(0)
    for layer in range(TINY['num_hidden_layers']):
        base = f'model.layers.{layer}.'
        for name in NORM_WEIGHT_NAMES:
            size = TINY['head_dim'] if 'q_norm' in name or 'k_norm' in name else h
            tensors[base + name] = torch.ones(size, dtype=torch.float16)
        for name in LINEAR_WEIGHT_NAMES:
            n, k = shapes[name]
            prefix = base + name.removesuffix('.weight')
            w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
            if layer == int8_layer:
                qw = np.clip(np.rint(w / 0.001), -127, 127).astype(np.int8)
                tensors[base + name] = torch.from_numpy(qw)
                tensors[prefix + '.weight_scale'] = torch.full((n, 1), 0.001, dtype=torch.float16)
            else:
                for key, value in synth.awq_quantize(w).items():
                    tensors[f'{prefix}.{key}'] = torch.from_numpy(np.ascontiguousarray(value))
    if mutate:
        mutate(tensors)
    save_file(tensors, str(path / 'model.safetensors'))


def test_loader_accepts_valid_checkpoint(tmp_path):
    write_tiny_checkpoint(tmp_path / 'ok', int8_layer=1)
    store = wq.load_compressed_store(tmp_path / 'ok')
    assert len(store.layers) == 2 and store.config.hidden_size == 256
    assert store.layers[0]['self_attn.k_proj.weight_packed'].shape == (128, 32)
    assert store.layers[1]['mlp.down_proj.weight'].dtype == torch.int8
    assert store.lm_head is store.embed_tokens                       # tied
    assert store.manifest['quantization_config']['format'] == 'pack-quantized'


@pytest.mark.parametrize('mutation,message', [
    (lambda t: t.__setitem__('model.layers.0.mlp.up_proj.weight_scale',
                             -t['model.layers.0.mlp.up_proj.weight_scale']), 'non-positive scale'),
    (lambda t: t.__setitem__('model.layers.0.mlp.up_proj.weight_packed',
                             t['model.layers.0.mlp.up_proj.weight_packed'][:, :-1].contiguous()), 'packed shape'),
    (lambda t: t.__setitem__('model.layers.0.mlp.up_proj.weight_zero_point',
                             t['model.layers.0.mlp.up_proj.weight_zero_point'][:-1].contiguous()), 'zero-point'),
    (lambda t: t.pop('model.layers.1.input_layernorm.weight'), 'missing layer 1 norm'),
    (lambda t: t.__setitem__('model.layers.0.self_attn.q_proj.weight_shape', torch.tensor([256, 128])),
     'logical shape'),
])
def test_loader_rejects_malformed_checkpoints(tmp_path, mutation, message):
    write_tiny_checkpoint(tmp_path / 'bad', mutate=mutation)
    with pytest.raises(ValueError, match=message):
        wq.load_compressed_store(tmp_path / 'bad')
