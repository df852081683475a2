"""Random Qwen3-shaped compressed-tensors models and a checkpoint writer.

There is no real checkpoint or network on the benchmark machines, so the
end-to-end benchmark and the loader tests need pack-quantized weights of the
right shapes.  ``random_compressed_store`` draws each decoder linear as fp16
``N(0, 0.02)`` and quantizes it (``awq_quantize``: asymmetric uint4, min-max
round-to-nearest per row and group along K, the range widened to include 0)
into the compressed-tensors layout that ``load_compressed_store`` validates
(``ondeviceinfer/weight_quantization/backend.py:69-128``): per linear
``weight_packed`` int32 ``[n, k/8]``, ``weight_scale`` fp16 ``[n, k/G]``,
``weight_zero_point`` int32 ``[n/8, k/G]`` (omitted for symmetric uint4b8),
``weight_shape``; fp16 norms near 1; fp16 embedding and LM head on the host,
as the reference keeps them.

``write_compressed_checkpoint`` writes such a store as safetensors shards +
``model.safetensors.index.json`` + ``config.json`` with a
``quantization_config`` of format ``pack-quantized`` (the on-disk contract of
``calibrate_weight_quant.py:97-102,150`` in the reference).
"""
from __future__ import annotations

import json
from dataclasses import asdict
from pathlib import Path

import torch

from ..config import Qwen3Config
from ..runtime.quantized import LINEAR_WEIGHT_NAMES, NORM_WEIGHT_NAMES
from .backend import CompressedStore


def linear_shapes(cfg: Qwen3Config) -> dict[str, tuple[int, int]]:
    """``name -> (n, k)`` of the seven decoder linears."""
    hidden, inter = cfg.hidden_size, cfg.intermediate_size
    kv = cfg.num_key_value_heads * cfg.head_dim
    q = cfg.num_attention_heads * cfg.head_dim
    return {
        'self_attn.q_proj.weight': (q, hidden), 'self_attn.k_proj.weight': (kv, hidden),
        'self_attn.v_proj.weight': (kv, hidden), 'self_attn.o_proj.weight': (hidden, q),
        'mlp.gate_proj.weight': (inter, hidden), 'mlp.up_proj.weight': (inter, hidden),
        'mlp.down_proj.weight': (hidden, inter),
    }


def pack_nibbles(codes: torch.Tensor, axis: int) -> torch.Tensor:
    """uint4 codes (int32 in [0, 15]) -> int32 words of 8 codes, first code in
    the lowest bits: along K (``axis=1``, ``[n, k] -> [n, k/8]``) or along N
    (``axis=0``, ``[n, g] -> [n/8, g]``), the compressed-tensors packing."""
    if axis == 0:
        return pack_nibbles(codes.t(), 1).t().contiguous()
    rows, cols = codes.shape
    shifts = torch.arange(0, 32, 4, device=codes.device, dtype=torch.int64)
    words = (codes.reshape(rows, cols // 8, 8).to(torch.int64) << shifts).sum(-1)
    return (words - ((words >> 31) << 32)).to(torch.int32)   # two's complement of the 32-bit pattern


def awq_quantize(w: torch.Tensor, group_size: int = 128, *, symmetric: bool = False) -> dict[str, torch.Tensor]:
    """fp16 ``w [n, k]`` -> unprefixed pack-quantized tensors, in fp32 on
    ``w``'s device.  Asymmetric: per (row, group) ``s = fp16((max - min) / 15)``
    over the group's range widened to include 0, ``z = clamp(round(-min / s),
    0, 15)``, ``q = clamp(round(w / s) + z, 0, 15)``.  Symmetric (uint4b8):
    ``s = fp16(absmax / 7.5)``, ``q = clamp(round(w / s) + 8, 0, 15)``.  A zero
    range gives ``s = 1``; rounding is half-to-even."""
    n, k = w.shape
    if k % group_size or n % 8:
        raise ValueError('need k % group_size == 0 and n % 8 == 0')
    g = w.float().reshape(n, k // group_size, group_size)
    if symmetric:
        s16 = (g.abs().amax(-1) / 7.5).half()
        s16 = torch.where(s16 == 0, torch.ones_like(s16), s16)
        q = torch.clamp(torch.round(g / s16.float()[..., None]) + 8, 0, 15).to(torch.int32).reshape(n, k)
        return {'weight_packed': pack_nibbles(q, 1), 'weight_scale': s16,
                'weight_shape': torch.tensor([n, k], dtype=torch.int64)}
    lo = torch.clamp(g.amin(-1), max=0.0)
    hi = torch.clamp(g.amax(-1), min=0.0)
    s16 = ((hi - lo) / 15.0).half()
    s16 = torch.where(s16 == 0, torch.ones_like(s16), s16)
    s = s16.float()
    z = torch.clamp(torch.round(-lo / s), 0, 15)
    q = torch.clamp(torch.round(g / s[..., None]) + z[..., None], 0, 15).to(torch.int32).reshape(n, k)
    return {'weight_packed': pack_nibbles(q, 1), 'weight_scale': s16,
            'weight_zero_point': pack_nibbles(z.to(torch.int32), 0),
            'weight_shape': torch.tensor([n, k], dtype=torch.int64)}


def random_compressed_store(cfg: Qwen3Config, *, seed: int = 0, device: str | torch.device = 'cpu',
                            group_size: int = 128, symmetric: bool = False, std: float = 0.02) -> CompressedStore:
    """A random W4 (G=``group_size``) Qwen3 model: every decoder linear drawn
    as ``fp16(N(0, std))`` and quantized by :func:`awq_quantize` on ``device``,
    where the decoder tensors stay; embedding / final norm / LM head
    (``fp16(N(0, 0.02))``, norms near 1) on the host."""
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    cpu_gen = torch.Generator().manual_seed(seed + 1)
    layers = []
    for _ in range(cfg.num_hidden_layers):
        layer = {}
        for name, (n, k) in linear_shapes(cfg).items():
            prefix = name.removesuffix('.weight')
            w = (torch.randn((n, k), device=device, generator=gen) * std).half()
            for key, value in awq_quantize(w, group_size, symmetric=symmetric).items():
                layer[f'{prefix}.{key}'] = value
            del w
        for name in NORM_WEIGHT_NAMES:
            size = cfg.head_dim if 'q_norm' in name or 'k_norm' in name else cfg.hidden_size
            layer[name] = (1.0 + 0.1 * torch.randn(size, device=device, generator=gen)).half()
        layers.append(layer)
    # Drawn on `device` (fast for the 151936 x 5120 tables), kept on the host.
    big = gen if device.type == 'cuda' else cpu_gen
    embed = (torch.randn(cfg.vocab_size, cfg.hidden_size, device=device, generator=big) * 0.02).half().cpu()
    lm_head = embed if cfg.tie_word_embeddings else \
        (torch.randn(cfg.vocab_size, cfg.hidden_size, device=device, generator=big) * 0.02).half().cpu()
    final_norm = (1.0 + 0.1 * torch.randn(cfg.hidden_size, generator=cpu_gen)).half()
    manifest = {'source': 'synthetic', 'seed': seed, 'weight_std': std,
                'quantization_config': quantization_config(group_size, symmetric)}
    return CompressedStore(cfg, layers, embed, final_norm, lm_head, manifest)


def random_int8_store(cfg: Qwen3Config, *, seed: int = 0, device: str | torch.device = 'cuda:0',
                      std: float = 0.02):
    """A random INT8 v1 Qwen3 model (``QuantizedCpuWeightStore``): every
    decoder linear drawn as ``fp16(N(0, std))`` and quantized per output
    channel by the GPU quantizer (``wq_w8_quantize``, the reference's
    ``quantize_linear_weight`` bit for bit); ``prefix.qweight`` /
    ``prefix.scale`` and the norms stay on ``device``, the embedding / final
    norm / LM head on the host."""
    from .. import _native
    from ..runtime.quantized import QuantizedCpuWeightStore, qweight_name, scale_name
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    cpu_gen = torch.Generator().manual_seed(seed + 1)
    layers = []
    for _ in range(cfg.num_hidden_layers):
        layer = {}
        for name, (n, k) in linear_shapes(cfg).items():
            w = (torch.randn((n, k), device=device, generator=gen) * std).half()
            layer[qweight_name(name)], layer[scale_name(name)] = _native.w8_quantize(w)
            del w
        for name in NORM_WEIGHT_NAMES:
            size = cfg.head_dim if 'q_norm' in name or 'k_norm' in name else cfg.hidden_size
            layer[name] = (1.0 + 0.1 * torch.randn(size, device=device, generator=gen)).half()
        layers.append(layer)
    embed = (torch.randn(cfg.vocab_size, cfg.hidden_size, device=device, generator=gen) * 0.02).half().cpu()
    lm_head = embed if cfg.tie_word_embeddings else \
        (torch.randn(cfg.vocab_size, cfg.hidden_size, device=device, generator=gen) * 0.02).half().cpu()
    final_norm = (1.0 + 0.1 * torch.randn(cfg.hidden_size, generator=cpu_gen)).half()
    return QuantizedCpuWeightStore(config=cfg, layers=layers, embed_tokens=embed, final_norm=final_norm,
                                   lm_head=lm_head, compute_dtype=torch.float16,
                                   manifest={'format': 'qwen3-int8-weight-only-v1', 'source': 'synthetic',
                                             'seed': seed, 'weight_std': std})


def quantization_config(group_size: int, symmetric: bool) -> dict:
    """compressed-tensors ``quantization_config`` for W4A16 pack-quantized."""
    return {
        'quant_method': 'compressed-tensors', 'format': 'pack-quantized',
        'config_groups': {'group_0': {
            'targets': ['Linear'],
            'weights': {'num_bits': 4, 'type': 'int', 'symmetric': symmetric, 'strategy': 'group',
                        'group_size': group_size, 'actorder': None, 'dynamic': False},
            'input_activations': None}},
        'ignore': ['lm_head'],
    }


def config_json(cfg: Qwen3Config) -> dict:
    raw = asdict(cfg)
    raw['model_type'] = 'qwen3'
    raw['architectures'] = ['Qwen3ForCausalLM']
    raw['torch_dtype'] = 'float16'
    return raw


def write_compressed_checkpoint(path: str | Path, store: CompressedStore, *, layers_per_shard: int = 8) -> Path:
    """Write ``store`` as a compressed-tensors checkpoint that
    ``load_compressed_store`` reads back tensor for tensor."""
    from safetensors.torch import save_file
    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    weight_map: dict[str, str] = {}
    n_layers = len(store.layers)
    shards = [list(range(i, min(i + layers_per_shard, n_layers))) for i in range(0, n_layers, layers_per_shard)]
    total = len(shards) + 1
    for s_idx, layer_ids in enumerate(shards):
        fname = f'model-{s_idx + 1:05d}-of-{total:05d}.safetensors'
        tensors = {}
        for li in layer_ids:
            for key, value in store.layers[li].items():
                if isinstance(value, torch.Tensor):
                    tensors[f'model.layers.{li}.{key}'] = value.detach().to('cpu').contiguous()
        save_file(tensors, str(path / fname))
        weight_map.update({name: fname for name in tensors})
    fname = f'model-{total:05d}-of-{total:05d}.safetensors'
    tensors = {'model.embed_tokens.weight': store.embed_tokens.cpu().contiguous(),
               'model.norm.weight': store.final_norm.cpu().contiguous()}
    if not store.config.tie_word_embeddings:
        tensors['lm_head.weight'] = store.lm_head.cpu().contiguous()
    save_file(tensors, str(path / fname))
    weight_map.update({name: fname for name in tensors})
    (path / 'model.safetensors.index.json').write_text(json.dumps({'metadata': {}, 'weight_map': weight_map}, indent=1))
    raw = config_json(store.config)
    raw['quantization_config'] = store.manifest.get('quantization_config') or quantization_config(128, False)
    (path / 'config.json').write_text(json.dumps(raw, indent=1))
    return path


__all__ = ['awq_quantize', 'linear_shapes', 'pack_nibbles', 'random_compressed_store', 'random_int8_store', 'quantization_config', 'write_compressed_checkpoint',
           'LINEAR_WEIGHT_NAMES']
