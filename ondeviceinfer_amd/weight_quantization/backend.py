"""Pluggable compressed Linear over compressed-tensors INT4 and INT8 checkpoints.

MI355X counterpart of ``ondeviceinfer/weight_quantization/backend.py``.  The
interface is the reference's: ``CompressedLinearBackend(name, group_size)``
with ``prepare(layer, name)`` (once per linear, at startup, after the tensors
are on the GPU) and ``linear(inputs, weights, name)``, the same dict keys,
the same counters and the same exceptions.  What runs underneath is this
build's HIP library (``libondeviceinfer_wq.so``):

* ``'marlin'``: the W4A16 path.  The name is kept so callers that select the
  fused backend by name work unchanged; ``prepare`` repacks into the gfx950
  tile layout (``wq_w4_repack``) and ``linear`` runs the MFMA GEMV / GEMM
  (``wq_w4a16_linear``).
* ``'w8a16'``: compressed-tensors channel INT8 (``weight`` int8 + ``weight_scale
  [N,1]``) as a weight-only fused INT8 x fp16 linear (``wq_w8a16_linear``).
* ``'int8_gemm'``: W8A8 on compressed-tensors channel INT8: dynamic per-token
  symmetric INT8 activations (``wq_w8a8_quantize``) times the INT8 weight,
  int32 accumulation on the int8 matrix cores (``wq_w8a8_linear``), as the
  reference's ``scaled_int8_quant`` + ``cutlass_scaled_mm`` (``backend.py:249-256``).
* ``'reference_int4'`` / ``'reference_w8a8'``: the explicit QDQ paths, as in the
  reference: decode the whole fp16 weight (``wq_w4_decode``/``wq_w8_decode``),
  fake-quantize the activations per token for W8A8, then ``F.linear``.

There is no silent fallback (``fallback_count`` stays 0): a missing library,
an unsupported shape or a CPU tensor raises.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass
from pathlib import Path
from typing import NamedTuple

import torch
import torch.nn.functional as F

from .. import _native
from ..config import Qwen3Config
from ..profiling import nvtx_range
from ..runtime.quantized import LINEAR_WEIGHT_NAMES, NORM_WEIGHT_NAMES
from ..runtime.stats import RuntimeStats

BACKEND_NAMES = ('marlin', 'int8_gemm', 'w8a16', 'reference_int4', 'reference_w8a8')
FUSED_BACKENDS = ('marlin', 'int8_gemm', 'w8a16')


def unpack_unsigned(packed: torch.Tensor, bits: int, axis: int, length: int) -> torch.Tensor:
    """b-bit unsigned fields of int32 words, LSB first (``backend.py:26-32``).

    ``axis=1`` unpacks along columns, ``axis=0`` along rows.  Plain tensor
    arithmetic on whatever device the input lives; a utility for callers and
    diagnostics, not used by the fused path (the repack kernel reads the packed
    zero points directly).
    """
    value = packed.transpose(0, 1) if axis == 0 else packed
    shifts = torch.arange(0, 32, bits, device=value.device, dtype=torch.int32)
    unpacked = ((value.unsqueeze(-1) >> shifts) & ((1 << bits) - 1)).reshape(value.shape[0], -1)
    unpacked = unpacked[:, :length]
    return unpacked.transpose(0, 1) if axis == 0 else unpacked


def decode_weight(weights: dict, name: str, *, group_size: int = 128) -> torch.Tensor:
    """Explicit dequantization to an fp16 ``[N, K]`` weight on the GPU.

    Same contract as ``backend.py:35-54``: INT8 channel ``fp16(q * s[n])``;
    W4 ``fp16((q - z) * s)`` in fp32 with ``z = 8`` when there is no zero point
    and ``weight_g_idx`` honoured.  Runs ``wq_w8_decode`` / ``wq_w4_decode``.
    """
    prefix = name.removesuffix('.weight')
    if prefix + '.weight_packed' not in weights:
        return _native.w8_decode(weights[name], weights[prefix + '.weight_scale'])
    n, k = (int(x) for x in weights[prefix + '.weight_shape'].tolist())
    return _native.w4_decode(weights[prefix + '.weight_packed'], weights[prefix + '.weight_scale'],
                             weights.get(prefix + '.weight_zero_point'), weights.get(prefix + '.weight_g_idx'),
                             n, k, group_size)


def decode_rows(weights: dict, name: str, rows: torch.Tensor) -> torch.Tensor:
    """fp16 ``[len(rows), K]``: the explicit decode of the sampled rows of one
    weight, without decoding the rest (``benchmarks/validate_weight_reconstruction.py:20-31``;
    like the reference, W4 groups are 128 along K).  INT8 channel weights:
    ``fp16(q[rows] * s[rows])``.  Runs ``wq_w4_decode_rows`` / ``wq_w8_decode``."""
    prefix = name.removesuffix('.weight')
    if prefix + '.weight_packed' not in weights:
        q = weights[name]
        idx = rows.reshape(-1).to(device=q.device, dtype=torch.int64)
        return _native.w8_decode(q.index_select(0, idx).contiguous(),
                                 weights[prefix + '.weight_scale'].index_select(0, idx))
    n, k = (int(x) for x in weights[prefix + '.weight_shape'].tolist())
    return _native.w4_decode_rows(weights[prefix + '.weight_packed'], weights[prefix + '.weight_scale'],
                                  weights.get(prefix + '.weight_zero_point'), rows, n, k, 128)


# fused linear -> the prepared projections it concatenates along N, in order
FUSED_PROJECTIONS = {
    'self_attn.qkv_proj': ('self_attn.q_proj', 'self_attn.k_proj', 'self_attn.v_proj'),
    'mlp.gate_up_proj': ('mlp.gate_proj', 'mlp.up_proj'),
}


class PreparedW4(NamedTuple):
    """What ``prepare`` stores under ``prefix._prepared`` for the W4A16 path."""
    tiles: torch.Tensor       # uint8, gfx950 tile layout
    meta: torch.Tensor        # uint8, 40 B per (16-row tile, group)
    workspace: torch.Tensor | None
    k: int
    n: int
    group_size: int


class PreparedW8(NamedTuple):
    qweight: object           # _native.W8Tiles (k % 128 == 0), else int8 [N, K] row-major as stored
    scale: torch.Tensor       # fp16 [N]
    k: int
    n: int


class PreparedW8A8(NamedTuple):
    qweight: object           # _native.W8Tiles (k % 128 == 0), else int8 [N, K] row-major as stored
    scale: torch.Tensor       # fp32 [N]
    k: int
    n: int


def int8_streamed(q: torch.Tensor):
    """The form the INT8 kernels stream a row-major INT8 weight in: its
    tiles (``_native.w8_repack``) when k % 128 == 0, which turn every 16-byte
    lane load into one contiguous 1 KiB wave load (same values, same results),
    else the tensor itself."""
    q = q.contiguous()
    return _native.w8_repack(q) if q.shape[1] % 128 == 0 else q


class NativeOps:
    """Tensor-level calls into the HIP library; swappable for tests (the
    reference's own dispatch test swaps ``backend.ops`` the same way)."""

    @staticmethod
    def w4a16_linear(x: torch.Tensor, prepared: PreparedW4, output: torch.Tensor | None = None) -> torch.Tensor:
        # The prepared workspace is sized for the decode GEMV (M <= 4); larger
        # batches take the library's shared workspace for their own plans.
        ws = prepared.workspace if x.shape[0] <= 4 else None
        return _native.w4a16_linear(x, prepared.tiles, prepared.meta, prepared.n, prepared.group_size,
                                    out=output, workspace=ws)

    @staticmethod
    def w8a16_linear(x: torch.Tensor, prepared: PreparedW8, output: torch.Tensor | None = None) -> torch.Tensor:
        return _native.w8a16_linear(x, prepared.qweight, prepared.scale, out=output)

    @staticmethod
    def w8a8_quantize(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        return _native.w8a8_quantize(x)

    @staticmethod
    def scaled_int8_quant(x: torch.Tensor, scale: torch.Tensor | None = None, azp: torch.Tensor | None = None,
                          symmetric: bool = True) -> tuple[torch.Tensor, torch.Tensor, None]:
        """vLLM's ``ops.scaled_int8_quant`` surface as the reference's kernel
        harness calls it (``benchmarks/validate_weight_quant_kernels.py:51``):
        dynamic per-token symmetric INT8 of a 2-D fp16 ``x``, returning
        ``(qx int8 [M, K], scale fp32 [M, 1], None)`` from ``wq_w8a8_quantize``.
        Static scales and asymmetric (zero-point) quantization are not part of
        this path and raise ``ValueError``."""
        if scale is not None or azp is not None or not symmetric:
            raise ValueError('scaled_int8_quant: only dynamic per-token symmetric quantization is supported')
        qx, x_scale = _native.w8a8_quantize(x)
        return qx, x_scale.view(-1, 1), None

    @staticmethod
    def w8a8_linear(qx: torch.Tensor, x_scale: torch.Tensor, prepared: PreparedW8A8,
                    output: torch.Tensor | None = None) -> torch.Tensor:
        return _native.w8a8_linear(qx, x_scale, prepared.qweight, prepared.scale, out=output)


@dataclass
class CompressedStore:
    config: Qwen3Config
    layers: list[dict]
    embed_tokens: torch.Tensor
    final_norm: torch.Tensor
    lm_head: torch.Tensor
    manifest: dict
    compute_dtype: torch.dtype = torch.float16
    max_dequant_elements: int = 0


def _shard_names(path: Path) -> list[str]:
    index_path = path / 'model.safetensors.index.json'
    if index_path.exists():
        raw = json.loads(index_path.read_text(encoding='utf-8'))
        return sorted(set(raw['weight_map'].values()))
    files = sorted(p.name for p in path.glob('*.safetensors'))
    if len(files) != 1:
        raise FileNotFoundError(f'No safetensors index found in {path}')
    return files


def load_compressed_store(path: str | Path) -> CompressedStore:
    """Read a compressed-tensors checkpoint with the reference's validation
    (``backend.py:69-128``): per layer, all 7 linears either pack-quantized
    (``weight_packed`` int32 ``(n, k//8)``, ``weight_shape`` ``[n, k]``,
    ``weight_scale`` ``(n, k//128)`` finite and > 0, ``weight_zero_point`` int32
    ``(n//8, k//128)`` or absent) or channel INT8 (``weight`` int8 ``(n, k)`` +
    ``weight_scale`` ``(n, 1)``); fp16 finite norms; tied LM head."""
    from safetensors import safe_open
    path = Path(path)
    cfg = Qwen3Config.from_json(path / 'config.json')
    layers: list[dict] = [{} for _ in range(cfg.num_hidden_layers)]
    globals_: dict = {}
    for shard in _shard_names(path):
        with safe_open(path / shard, framework='pt', device='cpu') as handle:
            for name in handle.keys():
                tensor = handle.get_tensor(name)
                if name.startswith('model.layers.'):
                    _, _, layer_index, local = name.split('.', 3)
                    layers[int(layer_index)][local] = tensor.contiguous()
                elif name in ('model.embed_tokens.weight', 'model.norm.weight', 'lm_head.weight'):
                    globals_[name] = tensor.half().contiguous()
    hidden, intermediate = cfg.hidden_size, cfg.intermediate_size
    kv = cfg.num_key_value_heads * cfg.head_dim
    expected_shapes = {
        'self_attn.q_proj.weight': (hidden, hidden),
        'self_attn.k_proj.weight': (kv, hidden),
        'self_attn.v_proj.weight': (kv, hidden),
        'self_attn.o_proj.weight': (hidden, hidden),
        'mlp.gate_proj.weight': (intermediate, hidden),
        'mlp.up_proj.weight': (intermediate, hidden),
        'mlp.down_proj.weight': (hidden, intermediate),
    }
    for idx, layer in enumerate(layers):
        for name in NORM_WEIGHT_NAMES:
            if name not in layer:
                raise ValueError(f'missing layer {idx} norm {name}')
            layer[name] = layer[name].half()
            if not bool(torch.isfinite(layer[name]).all()):
                raise ValueError(f'non-finite layer {idx} norm {name}')
        for name in LINEAR_WEIGHT_NAMES:
            prefix = name.removesuffix('.weight')
            if prefix + '.weight_scale' not in layer:
                raise ValueError(f'missing layer {idx} scale {prefix}')
            scale = layer[prefix + '.weight_scale']
            if not bool(torch.isfinite(scale).all()) or not bool((scale > 0).all()):
                raise ValueError(f'non-finite or non-positive scale: layer {idx} {prefix}')
            n, k = expected_shapes[name]
            if prefix + '.weight_packed' in layer:
                if tuple(layer[prefix + '.weight_shape'].tolist()) != (n, k):
                    raise ValueError(f'logical shape mismatch: layer {idx} {name}')
                packed = layer[prefix + '.weight_packed']
                if packed.dtype != torch.int32 or tuple(packed.shape) != (n, k // 8):
                    raise ValueError(f'packed shape/dtype mismatch: layer {idx} {name}')
                if tuple(scale.shape) != (n, k // 128):
                    raise ValueError(f'group scale mismatch: layer {idx} {name}')
                zero = layer.get(prefix + '.weight_zero_point')
                if zero is not None and (zero.dtype != torch.int32 or tuple(zero.shape) != (n // 8, k // 128)):
                    raise ValueError(f'packed zero-point mismatch: layer {idx} {name}')
            elif name not in layer or layer[name].dtype != torch.int8 or tuple(layer[name].shape) != (n, k):
                raise ValueError(f'INT8 shape/dtype mismatch: layer {idx} {name}')
            elif tuple(scale.shape) != (n, 1):
                raise ValueError(f'INT8 channel scale mismatch: layer {idx} {name}')
    manifest_path = path / 'experiment_manifest.json'
    manifest = json.loads(manifest_path.read_text()) if manifest_path.exists() else {}
    manifest['quantization_config'] = json.loads((path / 'config.json').read_text()).get('quantization_config', {})
    if 'lm_head.weight' not in globals_ and cfg.tie_word_embeddings:
        globals_['lm_head.weight'] = globals_['model.embed_tokens.weight']
    return CompressedStore(cfg, layers, globals_['model.embed_tokens.weight'], globals_['model.norm.weight'],
                           globals_['lm_head.weight'], manifest)


class CompressedResidentRuntime:
    """All layers resident on the GPU, each linear prepared once
    (``backend.py:131-169``)."""

    def __init__(self, store: CompressedStore, backend: 'CompressedLinearBackend', device='cuda:0',
                 verbose: bool = True):
        self.store, self.backend = store, backend
        self.stats = RuntimeStats()
        self.stats.startup_h2d_bytes = sum(v.numel() * v.element_size() for layer in store.layers
                                           for v in layer.values() if isinstance(v, torch.Tensor))
        self.gpu_layer_budget = len(store.layers)
        self.resident = []
        for idx, source in enumerate(store.layers):
            layer = {name: value.to(device) if isinstance(value, torch.Tensor) else value
                     for name, value in source.items()}
            for name in LINEAR_WEIGHT_NAMES:
                backend.prepare(layer, name)
            self.resident.append(layer)
            if verbose:
                print(f'prepared layer {idx + 1}/{len(store.layers)} for {backend.name}', flush=True)

    @property
    def startup_h2d_bytes(self) -> int:
        return self.stats.startup_h2d_bytes

    @property
    def resident_storage_bytes(self) -> int:
        storages = {}

        def visit(value):
            if isinstance(value, torch.Tensor) and value.device.type == 'cuda':
                storage = value.untyped_storage()
                storages[storage.data_ptr()] = storage.nbytes()
            elif isinstance(value, dict):
                for child in value.values():
                    visit(child)
            elif isinstance(value, (list, tuple)):
                for child in value:
                    visit(child)
        visit(self.resident)
        return sum(storages.values())

    def begin_forward(self):
        pass

    def weights_for(self, layer_idx):
        return self.resident[layer_idx]

    def after_layer(self, layer_idx):
        pass

    def end_forward(self):
        pass


class CompressedLinearBackend:
    """Same surface as the reference backend (``backend.py:172-263``)."""

    def __init__(self, name: str, group_size: int = 128):
        if name not in BACKEND_NAMES:
            raise ValueError(name)
        self.name, self.group_size = name, group_size
        self.calls = 0
        self.fallback_count = 0          # never incremented: there is no fallback
        self.explicit_dequant_bytes = 0
        self.gemm_calls = 0
        self.activation_quantize_calls = 0
        # Row splitting stays an explicit diagnostic (``backend.py:182-184``).
        self.marlin_max_rows_per_call = int(os.environ.get('ONDEVICEINFER_MARLIN_MAX_ROWS', '0'))
        # Recorded for report compatibility; these kernels always reduce in fp32.
        self.marlin_use_fp32_reduce = os.environ.get('ONDEVICEINFER_MARLIN_FP32_REDUCE', '0') == '1'
        self.ops = NativeOps()
        if name in FUSED_BACKENDS:
            _native.load()   # fail at construction, like the reference's vLLM import

    # -- fused dispatch (the reference's _marlin_gemm, backend.py:195-202)
    def _fused(self, x: torch.Tensor, prepared, output: torch.Tensor | None = None) -> torch.Tensor:
        self.gemm_calls += 1
        if isinstance(prepared, PreparedW8):
            return self.ops.w8a16_linear(x, prepared, output)
        if isinstance(prepared, PreparedW8A8):
            qx, x_scale = self.ops.w8a8_quantize(x)
            self.activation_quantize_calls += 1
            return self.ops.w8a8_linear(qx, x_scale, prepared, output)
        return self.ops.w4a16_linear(x, prepared, output)

    def prepare(self, layer: dict, name: str) -> None:
        prefix = name.removesuffix('.weight')
        if self.name == 'marlin':
            n, k = (int(x) for x in layer[prefix + '.weight_shape'].tolist())
            packed = layer[prefix + '.weight_packed']
            if layer.get(prefix + '.weight_g_idx') is not None:
                raise ValueError('runtime G-index unsupported in this experiment; disable act-order')
            scale = layer[prefix + '.weight_scale'].half().contiguous()
            zero = layer.get(prefix + '.weight_zero_point')
            tiles, meta = _native.w4_repack(packed.contiguous(), scale,
                                            None if zero is None else zero.contiguous(), n, k, self.group_size)
            ws_bytes = _native.w4a16_workspace_size(1, n, k, self.group_size)
            workspace = torch.zeros(ws_bytes, dtype=torch.uint8, device=packed.device) if ws_bytes else None
            layer[prefix + '._prepared'] = PreparedW4(tiles, meta, workspace, k, n, self.group_size)
            # The fused path retains only the repacked weights (backend.py:224-226).
            for suffix in ('.weight_packed', '.weight_scale', '.weight_zero_point'):
                layer.pop(prefix + suffix, None)
        elif self.name in ('w8a16', 'int8_gemm'):
            q = layer[name]
            if q.dtype != torch.int8:
                raise TypeError(f'{name}: expected INT8, got {q.dtype}')
            n, k = q.shape
            # The raw weight stays in the dict, as in the reference (backend.py:227-231).
            if self.name == 'w8a16':
                scale = layer[prefix + '.weight_scale'].reshape(-1).half().contiguous()
                layer[prefix + '._prepared'] = PreparedW8(int8_streamed(q), scale, k, n)
            else:   # the reference keeps the scale in fp32 for the scaled GEMM (backend.py:231)
                scale = layer[prefix + '.weight_scale'].float().reshape(-1).contiguous()
                layer[prefix + '._prepared'] = PreparedW8A8(int8_streamed(q), scale, k, n)

    def fuse_projections(self, layer: dict) -> None:
        """Add ``self_attn.qkv_proj._prepared`` and ``mlp.gate_up_proj._prepared``:
        the prepared q/k/v (gate/up) weights concatenated along N, so each
        group runs as one linear whose output is ``[q | k | v]``
        (``[gate | up]``).  W4 tiles and meta and INT8 tiles are tile-major
        and row-major INT8 is row-major, so concatenation is a plain copy;
        afterwards the parts' own ``_prepared`` entries are views into the
        fused buffers (no duplicate weights).  Layers whose parts do not line
        up (mixed formats, tiles with N not a multiple of 16) are left as
        they are."""
        for fused, parts in FUSED_PROJECTIONS.items():
            preps = [layer.get(p + '._prepared') for p in parts]
            if fused + '._prepared' in layer or any(p is None for p in preps):
                continue
            if all(isinstance(p, PreparedW4) for p in preps):
                if len({(p.k, p.group_size) for p in preps}) != 1 or any(p.n % 16 for p in preps):
                    continue
                tiles = torch.cat([p.tiles for p in preps])
                meta = torch.cat([p.meta for p in preps])
                n, k, g = sum(p.n for p in preps), preps[0].k, preps[0].group_size
                ws_bytes = _native.w4a16_workspace_size(1, n, k, g)
                ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=tiles.device) if ws_bytes else None
                layer[fused + '._prepared'] = PreparedW4(tiles, meta, ws, k, n, g)
                t0 = m0 = 0
                for part, p in zip(parts, preps):
                    layer[part + '._prepared'] = p._replace(tiles=tiles[t0:t0 + p.tiles.numel()],
                                                            meta=meta[m0:m0 + p.meta.numel()])
                    t0 += p.tiles.numel()
                    m0 += p.meta.numel()
            elif all(isinstance(p, PreparedW8) for p in preps) or all(isinstance(p, PreparedW8A8) for p in preps):
                if len({p.k for p in preps}) != 1:
                    continue
                kind = type(preps[0])
                k = preps[0].k
                sc = torch.cat([p.scale for p in preps])
                n = sum(p.n for p in preps)
                if all(isinstance(p.qweight, _native.W8Tiles) for p in preps):
                    if any(p.n % 16 for p in preps):   # the tiles of a part end on a 16-row boundary
                        continue
                    tiles = torch.cat([p.qweight.tiles for p in preps])
                    layer[fused + '._prepared'] = kind(_native.W8Tiles(tiles, n, k), sc, k, n)
                    t0 = r0 = 0
                    for part, p in zip(parts, preps):
                        size = p.qweight.tiles.numel()
                        layer[part + '._prepared'] = kind(_native.W8Tiles(tiles[t0:t0 + size], p.n, k),
                                                          sc[r0:r0 + p.n], k, p.n)
                        t0 += size
                        r0 += p.n
                elif all(isinstance(p.qweight, torch.Tensor) for p in preps):
                    q = torch.cat([p.qweight for p in preps])
                    layer[fused + '._prepared'] = kind(q, sc, k, n)
                    r0 = 0
                    for part, p in zip(parts, preps):
                        layer[part + '._prepared'] = kind(q[r0:r0 + p.n], sc[r0:r0 + p.n], p.k, p.n)
                        r0 += p.n

    def linear_epilogue(self, inputs: torch.Tensor, weights: dict, name: str, mode: int,
                        residual: torch.Tensor | None = None) -> torch.Tensor | None:
        """``linear`` with the MLP's next elementwise op in the prefill GEMM's
        epilogue, bit-identical to ``linear`` followed by that op:
        ``_native.EPI_SILU_MUL`` gives ``silu(gate) * up`` of a fused
        ``[gate | up]`` weight, ``_native.EPI_RESIDUAL`` gives
        ``residual + linear``.  Returns None where no such launch exists (INT8
        weights, the decode GEMV's row counts, grids without the epilogue);
        the caller then runs ``linear`` and the op as two steps.  Row chunks
        follow ``marlin_max_rows_per_call`` as in ``linear``."""
        if self.name not in FUSED_BACKENDS:
            return None
        prepared = weights.get(name.removesuffix('.weight') + '._prepared')
        if not isinstance(prepared, PreparedW4):
            return None
        k, n, g = prepared.k, prepared.n, prepared.group_size
        x = inputs.reshape(-1, k)
        rows = x.shape[0]
        step = self.marlin_max_rows_per_call if 0 < self.marlin_max_rows_per_call < rows else rows
        if rows == 0 or not all(_native.w4a16_epilogue_supported(min(step, rows - r), n, k, g, mode)
                                for r in range(0, rows, step)):
            return None
        n_out = n // 2 if mode == _native.EPI_SILU_MUL else n
        res = residual.reshape(rows, n).contiguous() if residual is not None else None
        self.calls += 1
        with nvtx_range(f'weight_quant::{self.name}::{name}+epilogue{mode}'):
            x = x.contiguous()
            out = x.new_empty((rows, n_out))
            for r in range(0, rows, step):
                e = min(r + step, rows)
                self.gemm_calls += 1
                _native.w4a16_linear_epilogue(x[r:e], prepared.tiles, prepared.meta, n, g, mode,
                                              None if res is None else res[r:e], out=out[r:e])
        return out.reshape(*inputs.shape[:-1], n_out)

    def linear(self, inputs: torch.Tensor, weights: dict, name: str) -> torch.Tensor:
        self.calls += 1
        prefix = name.removesuffix('.weight')
        with nvtx_range(f'weight_quant::{self.name}::{name}'):
            if self.name in FUSED_BACKENDS:
                prepared = weights[prefix + '._prepared']
                k, n = prepared.k, prepared.n
                x = inputs.reshape(-1, k).contiguous()
                if self.marlin_max_rows_per_call <= 0 or x.shape[0] <= self.marlin_max_rows_per_call:
                    out = self._fused(x, prepared)
                else:
                    out = x.new_empty((x.shape[0], n))
                    for start in range(0, x.shape[0], self.marlin_max_rows_per_call):
                        end = min(start + self.marlin_max_rows_per_call, x.shape[0])
                        self._fused(x[start:end], prepared, out[start:end])
                return out.reshape(*inputs.shape[:-1], n)
            weight = decode_weight(weights, name, group_size=self.group_size)
            self.explicit_dequant_bytes += weight.numel() * weight.element_size()
            if self.name == 'reference_w8a8':
                # Per-token symmetric fake quantization (backend.py:258-261).
                x = inputs.float()
                scale = x.abs().amax(dim=-1, keepdim=True).clamp_min(1e-12) / 127
                inputs = (x.div(scale).round().clamp(-127, 127) * scale).half()
            return F.linear(inputs, weight)
