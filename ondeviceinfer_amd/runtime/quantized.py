"""INT8 weight-only (v1) checkpoints: tensor names, the CPU store, its loader
and writer, and the resident GPU runtime.

On-disk format (``qwen3-int8-weight-only-v1``, written by the reference's
``benchmarks/quantize_checkpoint.py`` and read by
``ondeviceinfer/runtime/quantized.py:174-250``): a directory with
``config.json``, ``quantization_manifest.json`` (``format``, and
``tensor_files``: name / bytes / sha256 of every ``*.safetensors``), one
``layer-XXX.safetensors`` per decoder layer holding the four fp16 norms and,
per linear, ``prefix.qweight`` int8 ``[n, k]`` + ``prefix.scale`` fp16 ``[n]``,
and ``global.safetensors`` with the fp16 embedding, final norm and LM head.

Only the resident placement is built here (every decoder tensor on the GPU
for the whole run); the reference's layer-streaming runtimes are outside
this library's scope.
"""
from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import torch
from torch import Tensor

from .stats import RuntimeStats

LINEAR_WEIGHT_NAMES = (
    'self_attn.q_proj.weight',
    'self_attn.k_proj.weight',
    'self_attn.v_proj.weight',
    'self_attn.o_proj.weight',
    'mlp.gate_proj.weight',
    'mlp.up_proj.weight',
    'mlp.down_proj.weight',
)

NORM_WEIGHT_NAMES = (
    'input_layernorm.weight',
    'post_attention_layernorm.weight',
    'self_attn.q_norm.weight',
    'self_attn.k_norm.weight',
)

CHECKPOINT_FORMAT = 'qwen3-int8-weight-only-v1'
GLOBAL_TENSOR_NAMES = ('model.embed_tokens.weight', 'model.norm.weight', 'lm_head.weight')


def _renamed(weight_name: str, leaf: str) -> str:
    if not weight_name.endswith('.weight'):
        raise ValueError(f'Expected a .weight suffix, got {weight_name!r}')
    return weight_name[:-len('weight')] + leaf


def qweight_name(weight_name: str) -> str:
    """``x.weight`` -> ``x.qweight`` (``runtime/quantized.py:45-48``)."""
    return _renamed(weight_name, 'qweight')


def scale_name(weight_name: str) -> str:
    """``x.weight`` -> ``x.scale`` (``runtime/quantized.py:51-54``)."""
    return _renamed(weight_name, 'scale')


def _nbytes(tensors) -> int:
    return sum(t.numel() * t.element_size() for t in tensors)


def quantized_layer_bytes(layer: dict[str, Tensor]) -> int:
    return _nbytes(layer.values())


def layer_shapes(config) -> tuple[dict[str, tuple[int, ...]], dict[str, tuple[int, int]]]:
    """(norm name -> shape, linear weight name -> (n, k)) of one decoder layer.
    q_proj and o_proj are ``(hidden, hidden)``, as the reference's
    ``_validate_layer`` requires (``runtime/quantized.py:135-143``);
    ``Qwen3Config.validate`` makes ``heads * head_dim == hidden`` anyway."""
    hidden, inter, d = config.hidden_size, config.intermediate_size, config.head_dim
    kv = config.num_key_value_heads * d
    norms = {'input_layernorm.weight': (hidden,), 'post_attention_layernorm.weight': (hidden,),
             'self_attn.q_norm.weight': (d,), 'self_attn.k_norm.weight': (d,)}
    linears = {'self_attn.q_proj.weight': (hidden, hidden), 'self_attn.k_proj.weight': (kv, hidden),
               'self_attn.v_proj.weight': (kv, hidden), 'self_attn.o_proj.weight': (hidden, hidden),
               'mlp.gate_proj.weight': (inter, hidden), 'mlp.up_proj.weight': (inter, hidden),
               'mlp.down_proj.weight': (hidden, inter)}
    return norms, linears


@dataclass
class QuantizedCpuWeightStore:
    """An INT8 v1 model in host memory (``runtime/quantized.py:57-96``)."""

    config: Any
    layers: list[dict[str, Tensor]]
    embed_tokens: Tensor
    final_norm: Tensor
    lm_head: Tensor
    compute_dtype: torch.dtype
    manifest: dict[str, object]

    @property
    def decoder_bytes(self) -> int:
        return sum(quantized_layer_bytes(layer) for layer in self.layers)

    @property
    def total_bytes(self) -> int:
        return self.decoder_bytes + _nbytes((self.embed_tokens, self.final_norm, self.lm_head))

    @property
    def all_pinned(self) -> bool:
        globals_ = (self.embed_tokens, self.final_norm, self.lm_head)
        return all(t.is_pinned() for t in (*globals_, *(t for layer in self.layers for t in layer.values())))

    @property
    def max_dequant_elements(self) -> int:
        """Elements of the largest decoder matrix (the reference's fp16
        dequant scratch is sized by it)."""
        return max(layer[qweight_name(name)].numel() for layer in self.layers for name in LINEAR_WEIGHT_NAMES)


def validate_int8_layer(layer: dict[str, Tensor], layer_idx: int, config) -> None:
    """The reference's per-layer checks (``runtime/quantized.py:99-163``):
    exact key set (``RuntimeError``), fp16 norms (``TypeError``) of the
    config's shapes, int8 ``qweight`` / fp16 ``scale`` (``TypeError``) of the
    config's shapes with finite, positive scales (``ValueError``)."""
    norms, linears = layer_shapes(config)
    wanted = set(norms) | {f(n) for n in LINEAR_WEIGHT_NAMES for f in (qweight_name, scale_name)}
    missing, extra = sorted(wanted - set(layer)), sorted(set(layer) - wanted)
    if missing or extra:
        raise RuntimeError(f'Invalid quantized layer {layer_idx}: missing={missing}, unexpected={extra}')
    for name, shape in norms.items():
        t = layer[name]
        if t.dtype != torch.float16:
            raise TypeError(f'{name} must be FP16, got {t.dtype}')
        if tuple(t.shape) != shape:
            raise ValueError(f'Invalid shape for layer {layer_idx} {name}: expected {shape}, got {tuple(t.shape)}')
    for name, shape in linears.items():
        q, s = layer[qweight_name(name)], layer[scale_name(name)]
        if q.dtype != torch.int8:
            raise TypeError(f'{qweight_name(name)} must be INT8')
        if s.dtype != torch.float16:
            raise TypeError(f'{scale_name(name)} must be FP16')
        if q.dim() != 2 or tuple(s.shape) != (q.shape[0],):
            raise ValueError(f'Invalid qweight/scale shapes for {name}: {tuple(q.shape)} and {tuple(s.shape)}')
        if not bool(torch.isfinite(s).all()):
            raise ValueError(f'Non-finite scale in layer {layer_idx} {name}')
        if not bool((s > 0).all()):
            raise ValueError(f'Non-positive scale in layer {layer_idx} {name}')
        if tuple(q.shape) != shape:
            raise ValueError(f'Invalid shape for layer {layer_idx} {name}: expected {shape}, got {tuple(q.shape)}')


def file_sha256(path: Path, chunk: int = 1 << 23) -> str:
    h = hashlib.sha256()
    with open(path, 'rb') as f:
        for piece in iter(lambda: f.read(chunk), b''):
            h.update(piece)
    return h.hexdigest()


def _host(t: Tensor, pin: bool) -> Tensor:
    t = t.contiguous()
    return t.pin_memory() if pin else t


def load_quantized_cpu_weight_store(checkpoint_path: str | Path, *, pin_memory: bool = True, progress: bool = True,
                                    verify_checksums: bool = False) -> QuantizedCpuWeightStore:
    """Read an INT8 v1 checkpoint into host memory with the reference's checks
    (``runtime/quantized.py:174-250``): the manifest's ``format`` must be
    ``qwen3-int8-weight-only-v1`` (``ValueError``); with ``verify_checksums``
    every listed tensor file's size and SHA-256 must match (``RuntimeError``);
    a missing layer file raises ``FileNotFoundError``; the global file must
    hold exactly the embedding, final norm and LM head (``RuntimeError``),
    which are cast to fp16 and shape-checked against the config
    (``ValueError``)."""
    from safetensors.torch import load_file
    from ..config import Qwen3Config
    root = Path(checkpoint_path)
    config = Qwen3Config.from_json(root / 'config.json')
    manifest_file = root / 'quantization_manifest.json'
    manifest = json.loads(manifest_file.read_text(encoding='utf-8'))
    if manifest.get('format') != CHECKPOINT_FORMAT:
        raise ValueError(f'Unsupported quantized format in {manifest_file}')
    if verify_checksums:
        for record in manifest.get('tensor_files', []):
            f = root / record['name']
            if f.stat().st_size != record['bytes']:
                raise RuntimeError(f'Size mismatch for {f}')
            if file_sha256(f) != record['sha256']:
                raise RuntimeError(f'SHA-256 mismatch for {f}')
    layers = []
    for idx in range(config.num_hidden_layers):
        f = root / f'layer-{idx:03d}.safetensors'
        if not f.exists():
            raise FileNotFoundError(f)
        layer = {name: _host(t, pin_memory) for name, t in load_file(f, device='cpu').items()}
        validate_int8_layer(layer, idx, config)
        layers.append(layer)
        if progress:
            print(f'loaded INT8 layer {idx + 1}/{config.num_hidden_layers} '
                  f'({quantized_layer_bytes(layer) / 2**20:.2f} MiB)', flush=True)
    found = load_file(root / 'global.safetensors', device='cpu')
    if set(found) != set(GLOBAL_TENSOR_NAMES):
        raise RuntimeError(f'Invalid global tensors: expected {sorted(GLOBAL_TENSOR_NAMES)}, got {sorted(found)}')
    shapes = dict(zip(GLOBAL_TENSOR_NAMES, ((config.vocab_size, config.hidden_size), (config.hidden_size,),
                                            (config.vocab_size, config.hidden_size))))
    g = {}
    for name in GLOBAL_TENSOR_NAMES:
        g[name] = _host(found[name].to(torch.float16), pin_memory)
        if tuple(g[name].shape) != shapes[name]:
            raise ValueError(f'Invalid global shape for {name}: expected {shapes[name]}, got {tuple(g[name].shape)}')
    return QuantizedCpuWeightStore(config=config, layers=layers, embed_tokens=g['model.embed_tokens.weight'],
                                   final_norm=g['model.norm.weight'], lm_head=g['lm_head.weight'],
                                   compute_dtype=torch.float16, manifest=manifest)


def write_int8_checkpoint(path: str | Path, store: QuantizedCpuWeightStore) -> Path:
    """Write ``store`` in the INT8 v1 layout that
    :func:`load_quantized_cpu_weight_store` reads: per-layer and global
    safetensors files, ``config.json`` and a manifest listing every tensor
    file's size and SHA-256 (the fields the loader checks, plus the
    quantization parameters of the format)."""
    from dataclasses import asdict
    from safetensors.torch import save_file
    from ..quantization import QMAX, QMIN, QUANTIZATION_FORMAT, QUANTIZATION_VERSION
    root = Path(path)
    root.mkdir(parents=True, exist_ok=True)
    for idx, layer in enumerate(store.layers):
        save_file({k: v.detach().cpu().contiguous() for k, v in layer.items()}, str(root / f'layer-{idx:03d}.safetensors'))
    save_file({'model.embed_tokens.weight': store.embed_tokens.cpu().contiguous(),
               'model.norm.weight': store.final_norm.cpu().contiguous(),
               'lm_head.weight': store.lm_head.cpu().contiguous()}, str(root / 'global.safetensors'))
    config = asdict(store.config)
    config.update(model_type='qwen3', architectures=['Qwen3ForCausalLM'], torch_dtype='float16')
    (root / 'config.json').write_text(json.dumps(config, indent=1))
    files = sorted(root.glob('*.safetensors'))
    manifest = {
        'format': CHECKPOINT_FORMAT, 'algorithm': QUANTIZATION_FORMAT, 'algorithm_version': QUANTIZATION_VERSION,
        'axis': 0, 'zero_point': 0, 'quant_min': QMIN, 'quant_max': QMAX, 'scale_dtype': 'float16',
        'compute_dtype': 'float16', 'schema_version': 1, 'num_layers': len(store.layers),
        'quantized_decoder_bytes': store.decoder_bytes,
        'tensor_files': [{'name': f.name, 'bytes': f.stat().st_size, 'sha256': file_sha256(f)} for f in files],
    }
    (root / 'quantization_manifest.json').write_text(json.dumps(manifest, indent=2) + '\n', encoding='utf-8')
    return root


class QuantizedResidentRuntime:
    """Every INT8 decoder tensor resident on one device for the whole run
    (``runtime/quantized.py:437-469``): the runtime protocol of the model
    (``begin_forward`` / ``weights_for`` / ``after_layer`` / ``end_forward``)
    with nothing to stream."""

    def __init__(self, store: QuantizedCpuWeightStore, *, device: torch.device | str) -> None:
        self.store = store
        self.device = torch.device(device)
        self.gpu_layer_budget = self.resident_count = store.config.num_hidden_layers
        self.stats = RuntimeStats()
        self.resident = [{name: t.to(self.device) for name, t in layer.items()} for layer in store.layers]
        self.stats.startup_h2d_bytes = sum(quantized_layer_bytes(layer) for layer in self.resident)

    @property
    def startup_h2d_bytes(self) -> int:
        return self.stats.startup_h2d_bytes

    def begin_forward(self) -> None:
        pass

    def weights_for(self, layer_idx: int) -> dict[str, Tensor]:
        return self.resident[layer_idx]

    def after_layer(self, layer_idx: int) -> None:
        pass

    def end_forward(self) -> None:
        pass
