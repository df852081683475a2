"""Runtime INT8 weight-only linear for the INT8 v1 checkpoint format.

Mirrors ``int8_weight_only_linear`` and ``QuantizedComputeStats`` of
``ondeviceinfer/quantized_model.py:27-121``.  The reference dequantizes each
matrix into a shared fp16 scratch (``copy_`` + ``mul_``) and then runs an fp16
GEMM; here one fused HIP kernel (``wq_w8a16_linear``) reads the INT8 weight
once, so ``scratch`` is only validated and the dequant timing list stays
empty.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Mapping

import torch
from torch import Tensor

from . import _native
from .profiling import nvtx_range
from .runtime.quantized import LINEAR_WEIGHT_NAMES, qweight_name, scale_name


@dataclass
class QuantizedComputeStats:
    """Optional event timing of the linear kernels (``quantized_model.py:27-60``)."""

    enabled: bool = False
    dequant_events: list = field(default_factory=list)
    gemm_events: list = field(default_factory=list)
    dequantized_weight_bytes: int = 0
    linear_calls: int = 0

    def reset(self) -> None:
        self.dequant_events.clear()
        self.gemm_events.clear()
        self.dequantized_weight_bytes = 0
        self.linear_calls = 0

    @staticmethod
    def _seconds(events) -> float:
        if not events:
            return 0.0
        torch.cuda.synchronize()
        return sum(start.elapsed_time(end) for start, end in events) / 1000.0

    def dequant_seconds(self) -> float:
        return self._seconds(self.dequant_events)

    def gemm_seconds(self) -> float:
        return self._seconds(self.gemm_events)


def int8_weight_only_linear(inputs: Tensor, weights: Mapping[str, Tensor], weight_name: str, scratch: Tensor, *,
                            stats: QuantizedComputeStats | None = None) -> Tensor:
    """``inputs . (qweight * scale)^T`` for one decoder linear, fused on the GPU.

    Same keys (``prefix.qweight`` int8 ``[N, K]``, ``prefix.scale`` fp16 ``[N]``),
    same validation and errors as ``quantized_model.py:76-101``; work is queued
    on the current stream.
    """
    if weight_name not in LINEAR_WEIGHT_NAMES:
        raise KeyError(f'Unsupported quantized linear tensor {weight_name!r}')
    qweight = weights[qweight_name(weight_name)]
    scale = weights[scale_name(weight_name)]
    if qweight.device != inputs.device or scale.device != inputs.device:
        raise ValueError('INT8 weights, scales, and activations must share a device')
    if qweight.numel() > scratch.numel():
        raise ValueError(f'Scratch has {scratch.numel()} elements, but {weight_name} needs {qweight.numel()}')
    if stats is not None:
        stats.linear_calls += 1
    n, k = qweight.shape
    x = inputs.reshape(-1, k)
    scale16 = scale if scale.dtype == torch.float16 else scale.half()
    # A layer bound for the decode graph (_bind_int8_v1) holds the weight as
    # INT8 tiles, which the kernels stream faster; same results.
    prepared = weights.get(weight_name.removesuffix('.weight') + '._prepared')
    if prepared is not None and prepared.n == n and prepared.k == k:
        qweight, scale16 = prepared.qweight, prepared.scale
    elif isinstance(qweight, TiledInt8QWeight):
        qweight = qweight.w8_tiles
    with nvtx_range(f'w8a16_linear::{weight_name}'):
        if stats is not None and stats.enabled and inputs.device.type == 'cuda':
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            y = _native.w8a16_linear(x, qweight, scale16)
            end.record()
            stats.gemm_events.append((start, end))
        else:
            y = _native.w8a16_linear(x, qweight, scale16)
    return y.reshape(*inputs.shape[:-1], n)


# ============================================================================
# Qwen3 forward over the quantized linears (quantized_model.py:124-338)
# ============================================================================

import weakref  # noqa: E402

import torch.nn.functional as F  # noqa: E402

from .attention import cached_scaled_dot_product_attention  # noqa: E402
from .cache import KVCache, ResidentKVCache, kv_block  # noqa: E402
from .functional import add_rms_norm, rms_norm  # noqa: E402
from .layers import RotaryEmbedding, apply_rotary_pos_emb  # noqa: E402

QKV_FUSED = 'self_attn.qkv_proj.weight'
GATE_UP_FUSED = 'mlp.gate_up_proj.weight'


@dataclass
class CausalLMOutput:
    logits: Tensor
    cache: object | None = None
    # Greedy token of the last position ([batch, 1] int64), when the decode
    # graph computed it with the LM head (torch.argmax over the fp16 logits).
    next_token: Tensor | None = None


def _has_prepared(weights: Mapping, name: str) -> bool:
    return name.removesuffix('.weight') + '._prepared' in weights


def _int8_fused_linear(inputs: Tensor, weights: Mapping, name: str, parts: int,
                       stats: QuantizedComputeStats | None) -> Tensor | None:
    """The fused q|k|v or gate|up INT8 weight of a layer bound for the decode
    graph (``_bind_int8_v1``) as one W8A16 linear, counted as its ``parts``
    reference linears; None when the layer holds no such weight.  Each
    output column is the same sum the per-projection linear computes."""
    from .weight_quantization.backend import PreparedW8
    p = weights.get(name.removesuffix('.weight') + '._prepared')
    if not isinstance(p, PreparedW8) or not inputs.is_cuda:
        return None
    if stats is not None:
        stats.linear_calls += parts
    x = inputs.reshape(-1, p.k)
    with nvtx_range(f'w8a16_linear::{name}'):
        if stats is not None and stats.enabled:
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            y = _native.w8a16_linear(x, p.qweight, p.scale)
            end.record()
            stats.gemm_events.append((start, end))
        else:
            y = _native.w8a16_linear(x, p.qweight, p.scale)
    return y.reshape(*inputs.shape[:-1], p.n)


def _int8_epilogue(inputs: Tensor, weights: Mapping, name: str, parts: int, stats: QuantizedComputeStats | None,
                   mode: int, residual: Tensor | None = None) -> Tensor | None:
    """``_int8_fused_linear`` (or a bound per-projection INT8 weight) with the
    MLP's next elementwise op in the prefill GEMM's epilogue
    (``_native.w8a16_linear_epilogue``); None where that launch does not apply
    (rows at or below the decode GEMV's 64, grids without the epilogue)."""
    from .weight_quantization.backend import PreparedW8
    p = weights.get(name.removesuffix('.weight') + '._prepared')
    if not isinstance(p, PreparedW8) or not isinstance(p.qweight, _native.W8Tiles) or not inputs.is_cuda:
        return None
    x = inputs.reshape(-1, p.k)
    if not _native.w8a16_epilogue_supported(x.shape[0], p.n, p.k, mode):
        return None
    if stats is not None:
        stats.linear_calls += parts
    res = residual.reshape(x.shape[0], p.n).contiguous() if residual is not None else None
    with nvtx_range(f'w8a16_linear::{name}+epilogue{mode}'):
        y = _native.w8a16_linear_epilogue(x.contiguous(), p.qweight, p.scale, mode, res)
    return y.reshape(*inputs.shape[:-1], y.shape[-1])


def quantized_decoder_layer_forward(hidden_states: Tensor, weights: Mapping[str, Tensor], config: object,
                                    layer_idx: int, cos: Tensor, sin: Tensor, scratch: Tensor, *,
                                    cache: KVCache | None = None, stats: QuantizedComputeStats | None = None,
                                    linear_backend: object | None = None) -> Tensor:
    """One Qwen3 decoder layer (``quantized_model.py:124-228``).

    Same operation order and signature as the reference; when the backend
    prepared fused QKV / gate_up weights (``fuse_projections``) the three and
    the two projections run as one linear each, and ``silu(gate) * up`` runs
    as one HIP kernel; on the prefill GEMM it and the MLP's residual add run
    in the gate_up and down GEMMs' epilogues.  INT8 layers bound for the
    decode graph run their fused q|k|v and gate|up W8A16 weights the same way.  With a resident batch-1 cache the q/k norms, RoPE and
    cache append run as one HIP kernel and the causal attention as another
    (``wq_prefill_attention``, reading the cache rows in place).
    """
    def linear(inputs, name):
        if linear_backend is not None:
            return linear_backend.linear(inputs, weights, name)
        return int8_weight_only_linear(inputs, weights, name, scratch, stats=stats)

    eps = config.rms_norm_eps
    hq, hkv, d = config.num_attention_heads, config.num_key_value_heads, config.head_dim
    residual = hidden_states
    states = rms_norm(hidden_states, weights['input_layernorm.weight'], eps)
    batch_size, query_length, _ = states.shape
    qkv = None
    if linear_backend is not None and _has_prepared(weights, QKV_FUSED):
        qkv = linear(states, QKV_FUSED)
    elif linear_backend is None:
        qkv = _int8_fused_linear(states, weights, QKV_FUSED, 3, stats)
    if (qkv is not None and batch_size == 1 and d == 128 and qkv.is_cuda and qkv.dtype == torch.float16
            and isinstance(cache, ResidentKVCache) and cache.batch_size == 1
            and cos.dtype == torch.float16 and tuple(cos.shape) == (1, query_length, d)):
        # Resident batch-1 cache: q/k norm, RoPE and the cache append in one
        # launch (same per-element arithmetic as the steps below).
        start = cache.get_seq_length(layer_idx)
        end = start + query_length
        if end > cache.max_seq_len:
            raise ValueError(f'KV cache capacity exceeded: requested {end}, capacity {cache.max_seq_len}')
        # q comes back token-major [T, hq, d]; the flash attention kernel reads
        # it and the cache rows in place and writes token-major output (no
        # layout copies).
        query = _native.prefill_qk_rope(
            qkv.view(query_length, -1), hq, hkv, weights['self_attn.q_norm.weight'],
            weights['self_attn.k_norm.weight'], eps, cos[0], sin[0], start, cache.key_cache[layer_idx][0],
            cache.value_cache[layer_idx][0])
        cache.lengths[layer_idx] = end
        attention_output = _native.prefill_attention(
            query, hq, hkv, cache.key_cache[layer_idx][0], cache.value_cache[layer_idx][0], start,
            1.0 / float(d) ** 0.5).transpose(0, 1).unsqueeze(0)
    else:
        if qkv is not None:
            query, key, value = qkv.split((hq * d, hkv * d, hkv * d), dim=-1)
        else:
            query = linear(states, 'self_attn.q_proj.weight')
            key = linear(states, 'self_attn.k_proj.weight')
            value = linear(states, 'self_attn.v_proj.weight')
        query = query.reshape(batch_size, query_length, hq, d)
        key = key.reshape(batch_size, query_length, hkv, d)
        value = value.reshape(batch_size, query_length, hkv, d)
        query = rms_norm(query, weights['self_attn.q_norm.weight'], eps).transpose(1, 2)
        key = rms_norm(key, weights['self_attn.k_norm.weight'], eps).transpose(1, 2)
        value = value.transpose(1, 2)
        query, key = apply_rotary_pos_emb(query, key, cos, sin)
        attention_output = cached_scaled_dot_product_attention(query, key, value, layer_idx=layer_idx,
                                                               cache=cache, attention_mask=None, dropout_p=0.0)
    attention_output = attention_output.transpose(1, 2).contiguous().view(batch_size, query_length, hq * d)
    attention_output = linear(attention_output, 'self_attn.o_proj.weight')
    # residual + attention_output, then the post-attention RMSNorm (one launch on GPU)
    residual, states = add_rms_norm(residual, attention_output, weights['post_attention_layernorm.weight'], eps)
    # Prefill rows: silu(gate) * up in the fused gate_up GEMM's epilogue and
    # the residual add in the down GEMM's (bit-identical to the separate ops).
    epilogue = getattr(linear_backend, 'linear_epilogue', None)
    activated = None
    if linear_backend is not None and _has_prepared(weights, GATE_UP_FUSED):
        if epilogue is not None:
            activated = epilogue(states, weights, GATE_UP_FUSED, _native.EPI_SILU_MUL)
        if activated is None:
            activated = _native.silu_mul(linear(states, GATE_UP_FUSED).contiguous())
    elif linear_backend is None and (act := _int8_epilogue(states, weights, GATE_UP_FUSED, 2, stats,
                                                             _native.EPI_SILU_MUL)) is not None:
        activated = act
    elif linear_backend is None and (gate_up := _int8_fused_linear(states, weights, GATE_UP_FUSED, 2,
                                                                      stats)) is not None:
        activated = _native.silu_mul(gate_up.contiguous())
    else:
        gate = linear(states, 'mlp.gate_proj.weight')
        up = linear(states, 'mlp.up_proj.weight')
        activated = F.silu(gate) * up
    if epilogue is not None:
        out = epilogue(activated, weights, 'mlp.down_proj.weight', _native.EPI_RESIDUAL, residual)
        if out is not None:
            return out
    elif linear_backend is None:
        out = _int8_epilogue(activated, weights, 'mlp.down_proj.weight', 1, stats, _native.EPI_RESIDUAL, residual)
        if out is not None:
            return out
    mlp_output = linear(activated, 'mlp.down_proj.weight')
    return residual + mlp_output


class TiledInt8QWeight(torch.Tensor):
    """The ``prefix.qweight`` entry of an INT8 layer whose weight is held only
    as INT8 tiles (``_native.W8Tiles``): an int8 ``[N, K]`` tensor in shape,
    dtype and device, with no row-major storage of its own.  Metadata
    (``shape``, ``dtype``, ``device``, ``numel``) is answered directly, so the
    loader's and ``int8_weight_only_linear``'s checks run unchanged; any torch
    operation on it first rebuilds the row-major weight with ``wq_w8_unpack``
    (a temporary ``[N, K]`` copy, bit-exact) and runs on that."""

    @staticmethod
    def __new__(cls, tiles: '_native.W8Tiles'):
        r = torch.Tensor._make_wrapper_subclass(cls, (tiles.n, tiles.k), dtype=torch.int8,
                                                device=tiles.tiles.device, requires_grad=False)
        r.w8_tiles = tiles
        return r

    def __repr__(self) -> str:
        return f'TiledInt8QWeight(shape={tuple(self.shape)}, device={self.device})'

    def row_major(self) -> Tensor:
        return _native.w8_unpack(self.w8_tiles)

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        from torch.utils._pytree import tree_map

        def unwrap(t):
            return t.row_major() if isinstance(t, TiledInt8QWeight) else t
        return func(*tree_map(unwrap, args), **tree_map(unwrap, kwargs or {}))


def _bind_int8_v1(layer: dict, ops) -> None:
    """Give an INT8 v1 layer the prepared entries the decode graph runs:
    per linear a ``PreparedW8`` over its weight as INT8 tiles (``int8_streamed``)
    and fp16 ``scale``, then q|k|v and gate|up concatenated
    (``fuse_projections``).  The weight is then held once: each row-major
    ``qweight`` entry is replaced by a ``TiledInt8QWeight`` over the fused
    tiles (the reference's keys, shapes and dtypes stay; the row-major copy
    is freed), and ``scale`` by a view of the fused scales.  When the weights
    stay row-major (k % 128 != 0) the entries are rebound to views of the
    fused row-major copies instead."""
    from .weight_quantization.backend import PreparedW8, int8_streamed
    if not all(qweight_name(n) in layer for n in LINEAR_WEIGHT_NAMES) or QKV_FUSED.removesuffix('.weight') + \
            '._prepared' in layer:
        return
    for name in LINEAR_WEIGHT_NAMES:
        q = layer[qweight_name(name)]
        s16 = layer[scale_name(name)].reshape(-1).half().contiguous()
        layer[name.removesuffix('.weight') + '._prepared'] = PreparedW8(int8_streamed(q), s16, int(q.shape[1]),
                                                                       int(q.shape[0]))
    ops.fuse_projections(layer)
    for name in LINEAR_WEIGHT_NAMES:
        p = layer[name.removesuffix('.weight') + '._prepared']
        if isinstance(p.qweight, torch.Tensor):
            layer[qweight_name(name)] = p.qweight
        else:
            layer[qweight_name(name)] = TiledInt8QWeight(p.qweight)
        if layer[scale_name(name)].dtype == torch.float16:
            layer[scale_name(name)] = p.scale


class DecodeStepGraph:
    """One batch-1 decode token of the whole model, captured once as a HIP
    graph over model-owned buffers: embedding row -> per layer [fused QKV
    linear (RMSNorm in its prologue), attention (q/k norm, RoPE, KV append,
    GQA softmax, chunk merge), o linear (+ residual), fused gate_up linear
    (RMSNorm prologue), down linear (SiLU*up prologue, + residual)] -> final
    norm -> fp16 LM head with the greedy token picked in the same pass (or,
    with the optional W4 LM head, its GEMV and an argmax), for W4 and INT8
    (W8A16) weights alike; other formats (W8A8) take the same
    steps with the norms, residual adds and SiLU*up as separate kernels.
    Inputs are the token id and the position (device
    scalars; the step advances the position itself, a torch add at its end);
    the token's embedding row comes from the table in pinned host memory
    (``wq_embed_rows``); every other launch is a HIP kernel of this library,
    except that the LM head falls back to torch's GEMM when the hidden size
    is not a multiple of 512."""

    def __init__(self, model: 'QuantizedQwen3ForCausalLM', key_cache: list[Tensor], value_cache: list[Tensor],
                 max_seq_len: int):
        cfg, dev = model.config, model.device
        self.model = model
        self.max_seq_len = max_seq_len
        self.kc = [t[0] for t in key_cache]       # [kv_heads, max_seq, head_dim] views (batch 0)
        self.vc = [t[0] for t in value_cache]
        self.cos, self.sin = model.rotary_emb.table(max_seq_len, dev)
        hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        hidden = cfg.hidden_size
        f16 = dict(dtype=torch.float16, device=dev)
        # The logits and the greedy token share one buffer, so that one copy
        # hands both to the caller.
        vocab = cfg.vocab_size
        tok_off = (2 * vocab + 15) // 16 * 16
        self.out_buf = torch.zeros(tok_off + 16, dtype=torch.uint8, device=dev)
        self._vocab, self._tok_off = vocab, tok_off
        self.logits = self.out_buf[:2 * vocab].view(torch.float16).view(1, vocab)
        self.next_token = self.out_buf[tok_off:tok_off + 8].view(torch.long)
        self.token = torch.zeros(1, dtype=torch.long, device=dev)
        self.position = torch.zeros(1, dtype=torch.int32, device=dev)
        self.hidden = torch.empty(1, hidden, **f16)
        self.states = torch.empty(1, hidden, **f16)
        self.qkv = torch.empty(1, (hq + 2 * hkv) * d, **f16)
        self.attn = torch.empty(hq * d, **f16)
        self.delta = torch.empty(1, hidden, **f16)
        self.gate_up = torch.empty(1, 2 * cfg.intermediate_size, **f16)
        self.act = torch.empty(1, cfg.intermediate_size, **f16)
        self.lm_w4 = model.lm_head_w4
        self.argmax_ws = torch.zeros(_native.argmax_f16_workspace_size(cfg.vocab_size), dtype=torch.uint8,
                                     device=dev) if self.lm_w4 is not None else None
        self.native_lm_head = hidden % 512 == 0 and hidden <= 8192 and model.lm_head.is_contiguous()
        self.lm_ws = torch.zeros(max(_native.lm_head_workspace_size(hidden, cfg.vocab_size), 1), dtype=torch.uint8,
                                 device=dev) if self.native_lm_head else None
        self.attn_ws = torch.zeros(max(_native.decode_attention_workspace_size(hq, hkv, d, max_seq_len), 1),
                                   dtype=torch.uint8, device=dev)
        self.scale = 1.0 / float(d) ** 0.5
        self.layers = [model.runtime.weights_for(i) for i in range(cfg.num_hidden_layers)]
        ops = model.graph_ops
        calls = (ops.calls, ops.gemm_calls, model.compute_stats.linear_calls)
        for w in self.layers:
            for name in (QKV_FUSED, 'self_attn.o_proj.weight', GATE_UP_FUSED, 'mlp.down_proj.weight'):
                if not _has_prepared(w, name):
                    raise ValueError(f'decode graph needs prepared {name}')
        self.embed = model.embedding_table()
        self.lm_head_t = model.lm_head.t()
        from .weight_quantization.backend import PreparedW4, PreparedW8
        names = ('self_attn.qkv_proj', 'self_attn.o_proj', 'mlp.gate_up_proj', 'mlp.down_proj')
        prepared = [w[p + '._prepared'] for w in self.layers for p in names]
        # The fused decode linears take one weight format per step; INT8 also
        # needs k in whole 128-k blocks.
        self.fused = hidden % 16 == 0 and all(p.n % 16 == 0 for p in prepared) and (
            all(isinstance(p, PreparedW4) for p in prepared) or
            all(isinstance(p, PreparedW8) and p.k % 128 == 0 for p in prepared))
        self.sumsq_o = torch.zeros(hidden // 16, dtype=torch.float32, device=dev)
        self.sumsq_down = torch.zeros(hidden // 16, dtype=torch.float32, device=dev)
        # One eager step loads every code object and the GEMM's handles, then
        # the capture (the eager step's KV row 0 is rewritten by any prefill).
        self._step()
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()
        torch.cuda.synchronize(dev)
        ops.calls, ops.gemm_calls, model.compute_stats.linear_calls = calls   # set-up launches are not calls
        # The position the device holds for the next step (None: unknown).
        self._dev_position = None

    def _linear(self, x: Tensor, weights: Mapping, name: str, out: Tensor) -> None:
        prepared = weights[name.removesuffix('.weight') + '._prepared']
        self.model.graph_ops._fused(x, prepared, out)

    def _step(self) -> None:
        if self.fused:
            self._step_fused()
        else:
            self._step_unfused()
        self.position.add_(1)   # the next token's position, unless the caller asks for another

    @staticmethod
    def _fused_linear(x: Tensor, p, **kw) -> None:
        if hasattr(p, 'tiles'):
            _native.w4a16_decode_fused(x, p.tiles, p.meta, p.n, p.group_size, workspace=p.workspace, **kw)
        else:
            _native.w8a16_decode_fused(x, p.qweight, p.scale, **kw)

    def _step_fused(self) -> None:
        """The RMSNorms, residual adds and SiLU*up ride inside the decode
        linears (wq_w4a16_decode_fused / wq_w8a16_decode_fused): per layer one
        QKV linear, the attention, and the o, gate_up and down linears."""
        cfg = self.model.config
        eps = cfg.rms_norm_eps
        nat = _native
        lin = self._fused_linear
        # The embedding kernel also leaves the row's per-tile sums of squares,
        # so the first layer's input RMSNorm rides in its QKV linear like
        # every later layer's.
        _native.embed_rows(self.embed, self.token, out=self.hidden, sumsq_out=self.sumsq_down)
        hid = self.hidden.view(-1)
        for idx, w in enumerate(self.layers):
            qkv_p, o_p = w[QKV_FUSED.removesuffix('.weight') + '._prepared'], w['self_attn.o_proj._prepared']
            gu_p, dn_p = w[GATE_UP_FUSED.removesuffix('.weight') + '._prepared'], w['mlp.down_proj._prepared']
            lin(hid, qkv_p, x_mode=nat.X_RMSNORM, norm_weight=w['input_layernorm.weight'],
                sumsq_in=self.sumsq_down, eps=eps, out=self.qkv)
            nat.decode_attention(self.qkv.view(-1), cfg.num_attention_heads, cfg.num_key_value_heads,
                                 w['self_attn.q_norm.weight'], w['self_attn.k_norm.weight'], eps, self.cos,
                                 self.sin, self.position, self.kc[idx], self.vc[idx], self.scale, out=self.attn,
                                 workspace=self.attn_ws)
            lin(self.attn, o_p, residual=hid, sumsq_out=self.sumsq_o, out=hid)
            lin(hid, gu_p, x_mode=nat.X_RMSNORM, norm_weight=w['post_attention_layernorm.weight'],
                sumsq_in=self.sumsq_o, eps=eps, out=self.gate_up)
            lin(self.gate_up.view(-1), dn_p, x_mode=nat.X_SILU_MUL, residual=hid, sumsq_out=self.sumsq_down,
                out=hid)
        if self.lm_w4 is None and self.native_lm_head:
            # The final RMSNorm inside the LM head, from the last down
            # projection's sums of squares.
            _native.lm_head(hid, self.model.lm_head, logits=self.logits.view(-1), token=self.next_token,
                            workspace=self.lm_ws, norm_weight=self.model.final_norm, sumsq_in=self.sumsq_down,
                            eps=eps)
            return
        nat.add_rmsnorm(self.hidden, self.model.final_norm, eps, out=self.states)
        self._lm_head()

    def _lm_head(self) -> None:
        if self.lm_w4 is not None:
            p = self.lm_w4
            _native.w4a16_linear(self.states, p.tiles, p.meta, p.n, p.group_size, out=self.logits,
                                 workspace=p.workspace)
            _native.argmax_f16(self.logits.view(-1), out=self.next_token, workspace=self.argmax_ws)
        elif self.native_lm_head:
            _native.lm_head(self.states.view(-1), self.model.lm_head, logits=self.logits.view(-1),
                            token=self.next_token, workspace=self.lm_ws)
        else:
            torch.mm(self.states, self.lm_head_t, out=self.logits)
            torch.argmax(self.logits.view(-1), out=self.next_token.view(()))

    def _step_unfused(self) -> None:
        cfg = self.model.config
        eps = cfg.rms_norm_eps
        _native.embed_rows(self.embed, self.token, out=self.hidden)
        for idx, w in enumerate(self.layers):
            _native.add_rmsnorm(self.hidden, w['input_layernorm.weight'], eps, delta=None if idx == 0 else self.delta,
                                out=self.states, out_sum=self.hidden)
            self._linear(self.states, w, QKV_FUSED, self.qkv)
            _native.decode_attention(self.qkv.view(-1), cfg.num_attention_heads, cfg.num_key_value_heads,
                                     w['self_attn.q_norm.weight'], w['self_attn.k_norm.weight'], eps, self.cos,
                                     self.sin, self.position, self.kc[idx], self.vc[idx], self.scale, out=self.attn,
                                     workspace=self.attn_ws)
            self._linear(self.attn.view(1, -1), w, 'self_attn.o_proj.weight', self.delta)
            _native.add_rmsnorm(self.hidden, w['post_attention_layernorm.weight'], eps, delta=self.delta,
                                out=self.states, out_sum=self.hidden)
            self._linear(self.states, w, GATE_UP_FUSED, self.gate_up)
            _native.silu_mul(self.gate_up, out=self.act)
            self._linear(self.act, w, 'mlp.down_proj.weight', self.delta)
        _native.add_rmsnorm(self.hidden, self.model.final_norm, eps, delta=self.delta, out=self.states)
        self._lm_head()

    def run(self, token: Tensor, position: int) -> tuple[Tensor, Tensor]:
        """One decode step: the token's logits ``[1, 1, vocab]`` and its
        greedy next token ``[1, 1]``, fresh tensors (one copy of the step's
        output buffer).  The step advances the device position itself, so the
        position is written only when it differs from the one the previous
        replay left there."""
        if not 0 <= position < self.max_seq_len:
            raise ValueError(f'KV cache capacity exceeded: requested {position + 1}, capacity {self.max_seq_len}')
        self.token.copy_(token.reshape(1), non_blocking=True)
        if position != self._dev_position:
            self.position.fill_(position)
        self.graph.replay()
        self._dev_position = position + 1
        backend = self.model.linear_backend
        if backend is not None:
            backend.calls += 4 * len(self.layers)       # fused QKV, o, fused gate_up, down per layer
            backend.gemm_calls += 4 * len(self.layers)
        else:   # INT8 v1: the reference counts its 7 linears per layer
            self.model.compute_stats.linear_calls += 7 * len(self.layers)
        out = self.out_buf.clone()
        logits = out[:2 * self._vocab].view(torch.float16).view(1, 1, self._vocab)
        next_token = out[self._tok_off:self._tok_off + 8].view(torch.long).view(1, 1)
        return logits, next_token


class QuantizedQwen3ForCausalLM:
    """Qwen3 over the quantized decoder (``quantized_model.py:231-338``).

    ``store``/``runtime``/``linear_backend`` as in the reference.  Prefill and
    multi-token calls run eagerly layer by layer; single-token calls with a
    cache from ``make_resident_cache`` (batch 1) replay a captured
    ``DecodeStepGraph`` bound to that cache's storage.
    """

    def __init__(self, store, runtime, *, device: str | torch.device, profile_compute: bool = False,
                 linear_backend: object | None = None, decode_graph: bool = True,
                 quantize_lm_head: bool = False) -> None:
        self.store = store
        self.runtime = runtime
        self.config = store.config
        self.device = torch.device(device)
        self.dtype = store.compute_dtype
        self.final_norm = store.final_norm.to(self.device)
        self.lm_head = store.lm_head.to(self.device)
        self.rotary_emb = RotaryEmbedding(self.config.head_dim, self.config.rope_theta).to(self.device)
        self.linear_backend = linear_backend
        self.compute_stats = QuantizedComputeStats(enabled=profile_compute)
        # (layer_idx, hidden_states) after every decoder layer, when set
        self.layer_probe_callback = None
        self._dequant_scratch = None
        if linear_backend is None:
            # INT8 v1 weights (``prefix.qweight`` / ``prefix.scale``).  The
            # reference dequantizes into an fp16 scratch of the largest
            # matrix; the fused W8A16 kernel needs none, so the forward passes
            # a zero-stride view with that element count (only the capacity
            # check of int8_weight_only_linear reads it), and the public
            # ``dequant_scratch`` is allocated on first access.
            self._scratch_elements = store.max_dequant_elements
            self._forward_scratch = torch.empty(1, device=self.device, dtype=self.dtype).expand(
                self._scratch_elements)
            from .weight_quantization.backend import CompressedLinearBackend
            self.graph_ops = CompressedLinearBackend('w8a16')
            for idx in range(self.config.num_hidden_layers):
                _bind_int8_v1(runtime.weights_for(idx), self.graph_ops)
        else:
            self._scratch_elements = 0
            self._forward_scratch = torch.empty(0, device=self.device, dtype=self.dtype)
            self.graph_ops = linear_backend
            if hasattr(linear_backend, 'fuse_projections'):
                for idx in range(self.config.num_hidden_layers):
                    linear_backend.fuse_projections(runtime.weights_for(idx))
        self.decode_graph_enabled = decode_graph and hasattr(self.graph_ops, 'fuse_projections') and \
            self.device.type == 'cuda'
        self._embed_table = None
        self._kv_pool: dict = {}
        self.lm_head_w4 = None
        if quantize_lm_head:
            self.quantize_lm_head()

    @property
    def dequant_scratch(self) -> Tensor:
        """The reference's persistent fp16 dequantization scratch
        (``quantized_model.py:255-258``): the largest decoder matrix's element
        count for INT8 v1 weights, 0 elements with a linear backend.  A real
        contiguous buffer, allocated when first asked for (the fused kernels
        never use it)."""
        if self._dequant_scratch is None:
            self._dequant_scratch = torch.empty(self._scratch_elements, device=self.device, dtype=self.dtype)
        return self._dequant_scratch

    def quantize_lm_head(self, group_size: int = 128) -> None:
        """Optional W4 LM head (not in the reference, whose AWQ recipe keeps
        lm_head fp16): the fp16 head quantized to uint4 with per-group fp16
        scales and zero points (asymmetric min-max RTN, as the decoder
        linears) and repacked; the logits of every later call come from the
        W4 kernels.  Caches made earlier keep the decode graph they captured;
        new caches capture one with the W4 head."""
        from .weight_quantization.backend import PreparedW4
        from .weight_quantization.synthetic import awq_quantize
        vocab, hidden = self.lm_head.shape
        q = awq_quantize(self.lm_head, group_size)
        tiles, meta = _native.w4_repack(q['weight_packed'], q['weight_scale'], q['weight_zero_point'], vocab, hidden,
                                        group_size)
        del q
        ws_bytes = _native.w4a16_workspace_size(1, vocab, hidden, group_size)
        workspace = torch.zeros(ws_bytes, dtype=torch.uint8, device=self.device) if ws_bytes else None
        self.lm_head_w4 = PreparedW4(tiles, meta, workspace, hidden, vocab, group_size)
        self._kv_pool = {}

    def embedding_table(self):
        """The embedding table the decode graph gathers its token's row from.
        The reference keeps it in host memory and embeds on the CPU
        (``quantized_model.py:289-291``); here a CPU table stays there too, in
        pinned memory (the store's table is replaced by its pinned copy when
        it was not pinned), and the graph's ``wq_embed_rows`` reads the one
        row over the host link, so the 151936 x 5120 table takes no HBM.  A
        table already on the GPU is used in place."""
        if self._embed_table is None:
            table = self.store.embed_tokens
            if table.device.type == 'cpu':
                self._embed_table = _native.host_table(table.half(), self.device)
                self.store.embed_tokens = self._embed_table.tensor
            else:
                self._embed_table = table.to(self.device, torch.float16).contiguous()
        return self._embed_table

    def make_resident_cache(self, *, batch_size: int, max_seq_len: int,
                            device: str | torch.device | None = None) -> ResidentKVCache:
        """A fresh cache (lengths 0).  Its storage comes from a model-owned
        pool: a cache of the same shape whose previous owner object is gone
        is reused together with the decode graph captured for it, so repeated
        generations capture once; caches alive at the same time never share
        storage."""
        dev = torch.device(device or self.device)
        cfg = self.config
        entries = self._kv_pool.setdefault((batch_size, max_seq_len, str(dev)), [])
        entry = next((e for e in entries if e['owner']() is None), None)
        if entry is None:
            block = kv_block(cfg.num_hidden_layers, batch_size, cfg.num_key_value_heads, max_seq_len, cfg.head_dim,
                             device=dev, dtype=self.dtype, zero=True)
            entry = {'block': block, 'graph': None}
            if self.decode_graph_enabled and batch_size == 1 and dev.type == 'cuda' and \
                    max_seq_len <= _native.DECODE_ATTENTION_MAX_SEQ:
                view = ResidentKVCache.over(block)
                entry['graph'] = DecodeStepGraph(self, view.key_cache, view.value_cache, max_seq_len)
            entries.append(entry)
        cache = ResidentKVCache.over(entry['block'])
        entry['owner'] = weakref.ref(cache)
        cache._decode_graph = entry['graph']
        return cache

    @torch.inference_mode()
    def __call__(self, input_ids: Tensor, *, cache: KVCache | None = None, position_ids: Tensor | None = None,
                 logits_to_keep: int = 0, **_: object) -> CausalLMOutput:
        graph = getattr(cache, '_decode_graph', None)
        # The captured step exposes no per-layer hidden state, so a probe
        # callback sends the token through the eager layers, which call it.
        if graph is not None and position_ids is None and input_ids.shape == (1, 1) and \
                self.layer_probe_callback is None:
            past = cache.get_seq_length(0)
            if any(n != past for n in cache.lengths):
                raise RuntimeError('decode graph needs every layer of the cache at the same length')
            logits, next_token = graph.run(input_ids.to(self.device), past)
            cache.lengths[:] = [past + 1] * len(cache.lengths)
            return CausalLMOutput(logits=logits, cache=cache, next_token=next_token)

        ids_cpu = input_ids.detach().to(device='cpu')
        hidden_cpu = F.embedding(ids_cpu, self.store.embed_tokens)
        hidden_states = hidden_cpu.to(self.device)
        past_length = cache.get_seq_length(0) if cache is not None else 0
        query_length = input_ids.shape[1]
        if position_ids is None:
            position_ids = torch.arange(past_length, past_length + query_length,
                                        device=self.device).expand(input_ids.shape[0], -1)
        cos, sin = self.rotary_emb(hidden_states, position_ids)
        # The cache's lifecycle hooks and the per-layer probe, called where
        # the reference calls them (``quantized_model.py:302-327``).
        hook = lambda name: getattr(cache, name, None) if cache is not None else None  # noqa: E731
        if (begin := hook('begin_forward')) is not None:
            begin(query_length=query_length)
        self.runtime.begin_forward()
        for layer_idx in range(self.config.num_hidden_layers):
            if (before := hook('before_layer')) is not None:
                before(layer_idx)
            weights = self.runtime.weights_for(layer_idx)
            hidden_states = quantized_decoder_layer_forward(
                hidden_states, weights, self.config, layer_idx, cos, sin, self._forward_scratch, cache=cache,
                stats=self.compute_stats, linear_backend=self.linear_backend)
            if self.layer_probe_callback is not None:
                self.layer_probe_callback(layer_idx, hidden_states)
            if (after := hook('after_layer')) is not None:
                after(layer_idx)
            self.runtime.after_layer(layer_idx)
        self.runtime.end_forward()
        if (end := hook('end_forward')) is not None:
            end()
        # The norm is per row, so keeping the last rows first gives the same
        # logits as the reference's norm-then-slice without normalizing the
        # whole prompt.
        if logits_to_keep > 0:
            hidden_states = hidden_states[:, -logits_to_keep:, :].contiguous()
        hidden_states = rms_norm(hidden_states, self.final_norm, self.config.rms_norm_eps)
        if self.lm_head_w4 is not None:
            p = self.lm_head_w4
            flat = hidden_states.reshape(-1, p.k).contiguous()
            logits = _native.w4a16_linear(flat, p.tiles, p.meta, p.n, p.group_size,
                                          workspace=p.workspace if flat.shape[0] <= 4 else None)
            logits = logits.view(*hidden_states.shape[:-1], p.n)
        else:
            logits = F.linear(hidden_states, self.lm_head)
        return CausalLMOutput(logits=logits, cache=cache)
