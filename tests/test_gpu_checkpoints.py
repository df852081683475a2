"""Checkpoints on disk through the loaders onto the GPU, against the oracle.

* compressed-tensors pack-quantized (W4A16 G=128): ``write_compressed_checkpoint``
  -> ``load_compressed_store`` -> ``CompressedResidentRuntime`` (``prepare`` =
  the startup repack) -> ``CompressedLinearBackend.linear`` for every linear
  at M in {1, 5, 100}, then the Qwen3 model (prefill + graph decode), as the
  reference's ``validate_weight_quant_kernels.py:25-56`` flow does;
* INT8 v1 (``qwen3-int8-weight-only-v1``): ``write_int8_checkpoint`` ->
  ``load_quantized_cpu_weight_store`` (checksums verified, pinned) ->
  ``QuantizedResidentRuntime`` -> ``int8_weight_only_linear`` for every linear
  and the model with ``linear_backend=None``.

The oracle reads the tensors back from the same files (safetensors, numpy).
"""
import numpy as np
import pytest
import torch
from safetensors.numpy import load_file as load_np

from oracle import qdq, qwen3

pytestmark = pytest.mark.gpu


class Cfg:
    vocab_size = 1000
    hidden_size = 512
    intermediate_size = 1024
    num_hidden_layers = 2
    num_attention_heads = 4
    num_key_value_heads = 2
    head_dim = 128
    rms_norm_eps = 1e-6
    rope_theta = 1_000_000.0


def _qcfg():
    from ondeviceinfer_amd.config import Qwen3Config
    return Qwen3Config(vocab_size=Cfg.vocab_size, hidden_size=Cfg.hidden_size,
                       intermediate_size=Cfg.intermediate_size, num_hidden_layers=Cfg.num_hidden_layers,
                       num_attention_heads=Cfg.num_attention_heads, num_key_value_heads=Cfg.num_key_value_heads,
                       head_dim=Cfg.head_dim, max_position_embeddings=4096, rms_norm_eps=Cfg.rms_norm_eps,
                       rope_theta=Cfg.rope_theta, tie_word_embeddings=False)


def _parity(got, ref, what):
    m = qdq.parity_metrics(np.asarray(got, dtype=np.float32), np.asarray(ref, dtype=np.float32))
    print(what, {k: (round(v, 8) if isinstance(v, float) else v) for k, v in m.items()}, flush=True)
    assert qdq.parity_ok(m), (what, m)


def _run_model(model, oracle_model, gpu, tag):
    prompt = np.random.default_rng(7).integers(0, Cfg.vocab_size, 64)
    cache = model.make_resident_cache(batch_size=1, max_seq_len=96)
    assert cache._decode_graph is not None
    ocache = qwen3.KVCacheOracle(Cfg.num_hidden_layers)
    out = model(torch.from_numpy(prompt)[None].to(gpu), cache=cache, logits_to_keep=1)
    _parity(out.logits[0].float().cpu().numpy(), qwen3.forward(prompt, oracle_model, Cfg, ocache, logits_to_keep=1),
            f'{tag} prefill')
    token = out.logits[:, -1].argmax(-1, keepdim=True)
    for step in range(3):
        out = model(token, cache=cache, logits_to_keep=1)
        assert out.next_token is not None
        ref = qwen3.forward(token.cpu().numpy().reshape(-1), oracle_model, Cfg, ocache, logits_to_keep=1)
        _parity(out.logits[0].float().cpu().numpy(), ref, f'{tag} decode {step}')
        token = out.next_token
    # With a layer probe set, a decode token on the graph-bound cache runs the
    # eager layers, which call the probe after each layer
    # (quantized_model.py:323-324 of the reference); same logits bar.
    seen = []
    model.layer_probe_callback = lambda idx, hidden: seen.append((idx, tuple(hidden.shape)))
    try:
        out = model(token, cache=cache, logits_to_keep=1)
    finally:
        model.layer_probe_callback = None
    assert out.next_token is None      # not the graph's output
    assert seen == [(i, (1, 1, Cfg.hidden_size)) for i in range(Cfg.num_hidden_layers)]
    ref = qwen3.forward(token.cpu().numpy().reshape(-1), oracle_model, Cfg, ocache, logits_to_keep=1)
    _parity(out.logits[0].float().cpu().numpy(), ref, f'{tag} probed decode')


def _oracle_globals(path_global):
    return {'embed_tokens': path_global['model.embed_tokens.weight'], 'final_norm': path_global['model.norm.weight'],
            'lm_head': path_global['lm_head.weight']}


def test_pack_quantized_checkpoint_from_disk(gpu, tmp_path):
    from ondeviceinfer_amd.quantized_model import QuantizedQwen3ForCausalLM
    from ondeviceinfer_amd.weight_quantization.backend import (CompressedLinearBackend, CompressedResidentRuntime,
                                                               load_compressed_store)
    from ondeviceinfer_amd.weight_quantization.synthetic import random_compressed_store, write_compressed_checkpoint
    path = write_compressed_checkpoint(tmp_path / 'w4', random_compressed_store(_qcfg(), seed=1, device=gpu))
    # The oracle's view of the files: every tensor read back with numpy.
    on_disk = {}
    for shard in sorted(path.glob('*.safetensors')):
        on_disk.update(load_np(str(shard)))
    np_layers = [{k.split('.', 3)[3]: v for k, v in on_disk.items() if k.startswith(f'model.layers.{i}.')}
                 for i in range(Cfg.num_hidden_layers)]
    store = load_compressed_store(path)
    backend = CompressedLinearBackend('marlin')
    runtime = CompressedResidentRuntime(store, backend, device=gpu, verbose=False)
    rng = np.random.default_rng(3)
    for idx, layer in enumerate(runtime.resident):
        for name in qwen3.LINEAR_NAMES:
            assert name.removesuffix('.weight') + '.weight_packed' not in layer     # prepare kept only the tiles
            k = int(np_layers[idx][name.removesuffix('.weight') + '.weight_shape'][1])
            for m in (1, 5, 100):
                x = rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)
                y = backend.linear(torch.from_numpy(x).to(gpu), layer, name)
                _parity(y.cpu().numpy(), qdq.qdq_linear(x, np_layers[idx], name), f'w4 layer {idx} {name} m={m}')
    model = QuantizedQwen3ForCausalLM(store, runtime, device=gpu, linear_backend=backend)
    oracle_model = {'layers': np_layers, **_oracle_globals(on_disk)}
    _run_model(model, oracle_model, gpu, 'w4 checkpoint')


def test_int8_v1_checkpoint_from_disk(gpu, tmp_path):
    from ondeviceinfer_amd.quantized_model import (QuantizedQwen3ForCausalLM, TiledInt8QWeight,
                                                   int8_weight_only_linear)
    from ondeviceinfer_amd.runtime.quantized import (QuantizedResidentRuntime, load_quantized_cpu_weight_store,
                                                     qweight_name, scale_name, validate_int8_layer,
                                                     write_int8_checkpoint)
    from ondeviceinfer_amd.weight_quantization.synthetic import random_int8_store
    path = write_int8_checkpoint(tmp_path / 'int8', random_int8_store(_qcfg(), seed=2, device=gpu))
    np_layers = [load_np(str(path / f'layer-{i:03d}.safetensors')) for i in range(Cfg.num_hidden_layers)]
    store = load_quantized_cpu_weight_store(path, pin_memory=True, progress=False, verify_checksums=True)
    assert store.all_pinned
    runtime = QuantizedResidentRuntime(store, device=gpu)
    assert runtime.stats.startup_h2d_bytes == store.decoder_bytes
    model = QuantizedQwen3ForCausalLM(store, runtime, device=gpu, linear_backend=None)
    # The bound model holds each weight once, as INT8 tiles; the reference's
    # keys stay, still pass the loader's per-layer checks and read back as the
    # checkpoint's row-major INT8 bit for bit.
    for idx, layer in enumerate(runtime.resident):
        validate_int8_layer({k: v for k, v in layer.items() if not k.endswith('._prepared')}, idx, store.config)
        for name in qwen3.LINEAR_NAMES:
            q = layer[qweight_name(name)]
            assert isinstance(q, TiledInt8QWeight) and q.dtype == torch.int8
            assert np.array_equal(q.cpu().numpy(), np_layers[idx][qweight_name(name)])
            assert np.array_equal(layer[scale_name(name)].cpu().numpy(), np_layers[idx][scale_name(name)])
    assert model.dequant_scratch.is_contiguous()
    assert model.dequant_scratch.numel() == store.max_dequant_elements
    rng = np.random.default_rng(4)
    linears = []
    for idx, layer in enumerate(runtime.resident):
        decoded = {}
        for name in qwen3.LINEAR_NAMES:
            q, s = np_layers[idx][qweight_name(name)], np_layers[idx][scale_name(name)]
            decoded[name] = qdq.DecodedLinear(None, weight_fp16=qdq.dequantize_linear_weight(q, s))
            for m in (1, 5, 100):
                x = rng.standard_normal((m, q.shape[1]), dtype=np.float32).astype(np.float16)
                y = int8_weight_only_linear(torch.from_numpy(x).to(gpu), layer, name, model.dequant_scratch,
                                            stats=model.compute_stats)
                _parity(y.cpu().numpy(), decoded[name](x), f'int8 layer {idx} {name} m={m}')
        linears.append(decoded)
    assert model.compute_stats.linear_calls == 3 * 7 * Cfg.num_hidden_layers
    oracle_model = {'layers': np_layers, 'linears': linears,
                    **_oracle_globals(load_np(str(path / 'global.safetensors')))}
    _run_model(model, oracle_model, gpu, 'int8 checkpoint')
