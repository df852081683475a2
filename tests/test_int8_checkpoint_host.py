"""INT8 v1 checkpoints on the host (CPU only): the writer and the loader of
``qwen3-int8-weight-only-v1`` (reference ``runtime/quantized.py:99-250``)
round-trip tensor for tensor, and every check the reference's loader makes
raises the reference's exception type."""
import json

import pytest
import torch
from safetensors.torch import load_file, save_file

from ondeviceinfer_amd.config import Qwen3Config
from ondeviceinfer_amd.runtime.quantized import (LINEAR_WEIGHT_NAMES, NORM_WEIGHT_NAMES, QuantizedCpuWeightStore,
                                                 layer_shapes, load_quantized_cpu_weight_store, qweight_name,
                                                 scale_name, validate_int8_layer, write_int8_checkpoint)


def tiny_config(layers=2):
    return Qwen3Config(vocab_size=101, hidden_size=256, intermediate_size=512, num_hidden_layers=layers,
                       num_attention_heads=2, num_key_value_heads=1, head_dim=128, max_position_embeddings=128,
                       rms_norm_eps=1e-6, rope_theta=1_000_000.0, tie_word_embeddings=False)


def tiny_store(cfg, seed=0):
    g = torch.Generator().manual_seed(seed)
    norms, linears = layer_shapes(cfg)
    layers = []
    for _ in range(cfg.num_hidden_layers):
        layer = {name: (1 + 0.1 * torch.randn(shape, generator=g)).half() for name, shape in norms.items()}
        for name, (n, k) in linears.items():
            layer[qweight_name(name)] = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
            layer[scale_name(name)] = (torch.rand(n, generator=g) * 1e-3 + 1e-4).half()
        layers.append(layer)
    return QuantizedCpuWeightStore(config=cfg, layers=layers,
                                   embed_tokens=torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g).half(),
                                   final_norm=torch.ones(cfg.hidden_size).half(),
                                   lm_head=torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g).half(),
                                   compute_dtype=torch.float16, manifest={})


@pytest.fixture()
def checkpoint(tmp_path):
    cfg = tiny_config()
    store = tiny_store(cfg)
    return write_int8_checkpoint(tmp_path / 'int8', store), store


def test_round_trip_and_store_accounting(checkpoint):
    path, store = checkpoint
    loaded = load_quantized_cpu_weight_store(path, pin_memory=False, progress=False, verify_checksums=True)
    assert loaded.config == store.config and loaded.compute_dtype == torch.float16
    assert loaded.manifest['format'] == 'qwen3-int8-weight-only-v1'
    assert {f['name'] for f in loaded.manifest['tensor_files']} == \
        {'layer-000.safetensors', 'layer-001.safetensors', 'global.safetensors'}
    for a, b in zip(loaded.layers, store.layers):
        assert set(a) == set(b) and all(torch.equal(a[k], b[k]) for k in a)
    for name in ('embed_tokens', 'final_norm', 'lm_head'):
        assert torch.equal(getattr(loaded, name), getattr(store, name))
    assert loaded.max_dequant_elements == 512 * 256
    assert loaded.decoder_bytes == store.decoder_bytes
    assert loaded.total_bytes == loaded.decoder_bytes + (101 * 256 * 2) * 2 + 256 * 2
    assert not loaded.all_pinned


def test_checksums_and_format_are_checked(checkpoint):
    path, _ = checkpoint
    manifest = json.loads((path / 'quantization_manifest.json').read_text())
    layer1 = path / 'layer-001.safetensors'
    raw = bytearray(layer1.read_bytes())
    raw[-1] ^= 0x01                                     # same size, different content
    layer1.write_bytes(bytes(raw))
    load_quantized_cpu_weight_store(path, pin_memory=False, progress=False)     # not verified: loads
    with pytest.raises(RuntimeError, match='SHA-256 mismatch'):
        load_quantized_cpu_weight_store(path, pin_memory=False, progress=False, verify_checksums=True)
    layer1.write_bytes(bytes(raw) + b'\0')
    with pytest.raises(RuntimeError, match='Size mismatch'):
        load_quantized_cpu_weight_store(path, pin_memory=False, progress=False, verify_checksums=True)
    manifest['format'] = 'something-else'
    (path / 'quantization_manifest.json').write_text(json.dumps(manifest))
    with pytest.raises(ValueError, match='Unsupported quantized format'):
        load_quantized_cpu_weight_store(path, pin_memory=False, progress=False)


def test_missing_layer_and_bad_globals(checkpoint):
    path, store = checkpoint
    g = load_file(path / 'global.safetensors')
    save_file({**g, 'extra.weight': torch.zeros(2)}, str(path / 'global.safetensors'))
    with pytest.raises(RuntimeError, match='Invalid global tensors'):
        load_quantized_cpu_weight_store(path, pin_memory=False, progress=False)
    save_file({**g, 'model.norm.weight': torch.zeros(255).half()}, str(path / 'global.safetensors'))
    with pytest.raises(ValueError, match='Invalid global shape for model.norm.weight'):
        load_quantized_cpu_weight_store(path, pin_memory=False, progress=False)
    save_file({k: v.float() for k, v in g.items()}, str(path / 'global.safetensors'))
    loaded = load_quantized_cpu_weight_store(path, pin_memory=False, progress=False)
    assert loaded.lm_head.dtype == torch.float16     # globals are cast to fp16
    (path / 'layer-001.safetensors').unlink()
    with pytest.raises(FileNotFoundError):
        load_quantized_cpu_weight_store(path, pin_memory=False, progress=False)


def _layer(cfg):
    return {k: v.clone() for k, v in tiny_store(cfg, seed=3).layers[0].items()}


def test_layer_validation_rules():
    cfg = tiny_config(1)
    validate_int8_layer(_layer(cfg), 0, cfg)
    cases = []
    layer = _layer(cfg)
    del layer[scale_name(LINEAR_WEIGHT_NAMES[2])]
    cases.append((layer, RuntimeError, 'missing='))
    layer = _layer(cfg)
    layer['mlp.extra'] = torch.zeros(1)
    cases.append((layer, RuntimeError, 'unexpected='))
    layer = _layer(cfg)
    layer[NORM_WEIGHT_NAMES[0]] = layer[NORM_WEIGHT_NAMES[0]].float()
    cases.append((layer, TypeError, 'must be FP16'))
    layer = _layer(cfg)
    layer['self_attn.q_norm.weight'] = torch.ones(64).half()
    cases.append((layer, ValueError, 'Invalid shape for layer 0 self_attn.q_norm.weight'))
    layer = _layer(cfg)
    layer[qweight_name('mlp.up_proj.weight')] = layer[qweight_name('mlp.up_proj.weight')].to(torch.int16)
    cases.append((layer, TypeError, 'must be INT8'))
    layer = _layer(cfg)
    layer[scale_name('mlp.up_proj.weight')] = layer[scale_name('mlp.up_proj.weight')].float()
    cases.append((layer, TypeError, 'must be FP16'))
    layer = _layer(cfg)
    layer[scale_name('mlp.up_proj.weight')] = layer[scale_name('mlp.up_proj.weight')][:-1]
    cases.append((layer, ValueError, 'Invalid qweight/scale shapes'))
    layer = _layer(cfg)
    layer[scale_name('mlp.down_proj.weight')][3] = float('nan')
    cases.append((layer, ValueError, 'Non-finite scale in layer 0 mlp.down_proj.weight'))
    layer = _layer(cfg)
    layer[scale_name('mlp.down_proj.weight')][3] = 0
    cases.append((layer, ValueError, 'Non-positive scale'))
    layer = _layer(cfg)
    name = 'self_attn.o_proj.weight'
    layer[qweight_name(name)] = layer[qweight_name(name)][:, :128].contiguous()
    cases.append((layer, ValueError, 'Invalid shape for layer 0 self_attn.o_proj.weight'))
    for layer, exc, msg in cases:
        with pytest.raises(exc, match=msg):
            validate_int8_layer(layer, 0, cfg)


def test_qweight_and_scale_names():
    assert qweight_name('mlp.up_proj.weight') == 'mlp.up_proj.qweight'
    assert scale_name('mlp.up_proj.weight') == 'mlp.up_proj.scale'
    with pytest.raises(ValueError, match='.weight suffix'):
        qweight_name('mlp.up_proj.bias')
