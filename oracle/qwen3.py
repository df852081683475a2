"""numpy restatement of the reference's Qwen3 decoder forward around the
quantized linears (test oracle only).

Test infrastructure: imported only by ``tests/`` (and ``__graft_entry__.smoke()``)
as the checker of the GPU decode path; the product never imports it.

It follows the reference's operation order, including where it rounds to
fp16 (every elementwise op on fp16 tensors rounds once; reductions, softmax
and the linears accumulate in fp32).  The linears are the explicit QDQ path
(``qdq.qdq_linear``: ``decode_weight`` + fp32-accumulated ``F.linear``).

Pinning (what checks this oracle independently of its own formulas):

===========================  =================================================
function                     pinned by
===========================  =================================================
rms_norm                     float64 closed form; the reference test's recipe
                             ``test_foundations.py:36-48`` (fp32 normalize,
                             cast, scale) computed with torch on the CPU
rotary_tables / apply_rope   reference test ``test_foundations.py:51-67``
                             (position 0 is the identity, norms preserved);
                             relative-position property q_m.k_n = f(m - n);
                             torch's ``pow``/``cos``/``sin`` on the CPU
build_causal_mask            reference KAT ``test_model.py:29-38``
attention                    ``torch.nn.functional.scaled_dot_product_attention``
                             on the CPU (fp32); GQA == explicit K/V repetition
                             (``test_model.py:40-53``); a single key returns V
swiglu                       formula KAT (``test_model.py:68-74``)
decoder_layer / forward      an independent torch-CPU float32 implementation in
                             the tests (library ops: F.rms_norm, SDPA, F.silu);
                             prefill of t+1 tokens == prefill of t + one cached
                             decode step (the KV-cache invariant)
===========================  =================================================
"""
from __future__ import annotations

import numpy as np

from . import qdq

F16 = np.float16
F32 = np.float32

LINEAR_NAMES = ('self_attn.q_proj.weight', 'self_attn.k_proj.weight', 'self_attn.v_proj.weight',
                'self_attn.o_proj.weight', 'mlp.gate_proj.weight', 'mlp.up_proj.weight', 'mlp.down_proj.weight')


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """``weight * fp16(x32 * rsqrt(mean(x32^2) + eps))`` over the last axis
    (``ondeviceinfer/functional.py:17-22``)."""
    x32 = np.asarray(x).astype(F32)
    var = np.mean(x32 * x32, axis=-1, keepdims=True, dtype=F32)
    normalized = (x32 * (F32(1) / np.sqrt(var + F32(eps)))).astype(F16)
    return (np.asarray(weight).astype(F16) * normalized).astype(F16)


def rotary_tables(head_dim: int, theta: float, positions: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """fp16 ``cos``/``sin`` ``[len(positions), head_dim]``: angles in fp32 from
    ``inv_freq = 1 / theta ** (arange(0, d, 2) / d)``, duplicated halves
    (``ondeviceinfer/layers.py:36-61``)."""
    exponent = np.arange(0, head_dim, 2, dtype=F32) / F32(head_dim)
    inv_freq = (F32(1) / np.power(F32(theta), exponent, dtype=F32)).astype(F32)
    freqs = np.asarray(positions, dtype=F32)[:, None] * inv_freq[None, :]
    angles = np.concatenate([freqs, freqs], axis=-1).astype(F32)
    return np.cos(angles).astype(F16), np.sin(angles).astype(F16)


def rotate_half(x: np.ndarray) -> np.ndarray:
    """``[x1, x2] -> [-x2, x1]`` on the last axis (``layers.py:64-67``)."""
    half = x.shape[-1] // 2
    return np.concatenate([-x[..., half:], x[..., :half]], axis=-1)


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """``x * cos + rotate_half(x) * sin`` on fp16 ``x [heads, seq, d]`` with
    ``cos/sin [seq, d]``; each product and the sum round to fp16
    (``layers.py:70-80``)."""
    x = np.asarray(x).astype(F16)
    a = (x * cos[None]).astype(F16)
    b = (rotate_half(x) * sin[None]).astype(F16)
    return (a + b).astype(F16)


def build_causal_mask(query_length: int, key_length: int) -> np.ndarray:
    """Absolute-position causal mask, True = attends (``attention.py:14-32``)."""
    if query_length > key_length:
        raise ValueError('query_length cannot exceed key_length')
    past = key_length - query_length
    q = np.arange(past, key_length)[:, None]
    k = np.arange(key_length)[None, :]
    return k <= q


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask: np.ndarray | None) -> np.ndarray:
    """Grouped-query softmax attention with scale ``1/sqrt(d)``:
    ``q [Hq, S, d]``, ``k, v [Hkv, T, d]`` -> fp16 ``[Hq, S, d]``; computed in
    fp32 (``F.scaled_dot_product_attention(..., enable_gqa=True)`` as called at
    ``attention.py:78-85``)."""
    hq, hkv = q.shape[0], k.shape[0]
    group = hq // hkv
    q32, k32, v32 = (np.asarray(t).astype(F32) for t in (q, k, v))
    k32 = np.repeat(k32, group, axis=0)
    v32 = np.repeat(v32, group, axis=0)
    scores = np.einsum('hsd,htd->hst', q32, k32) * F32(1.0 / np.sqrt(q.shape[-1]))
    if mask is not None:
        scores = np.where(mask[None], scores, -np.inf)
    scores = scores - scores.max(axis=-1, keepdims=True)
    p = np.exp(scores)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.einsum('hst,htd->hsd', p, v32).astype(F16)


def silu(x: np.ndarray) -> np.ndarray:
    """fp16 ``silu`` computed in fp32 (``F.silu`` on an fp16 tensor)."""
    x32 = np.asarray(x).astype(F32)
    return (x32 / (F32(1) + np.exp(-x32))).astype(F16)


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """``F.silu(gate) * up`` in fp16 (``quantized_model.py:222-224``)."""
    return (silu(gate) * np.asarray(up).astype(F16)).astype(F16)


class KVCacheOracle:
    """Per-layer K/V rows ``[Hkv, T, d]`` appended in order
    (``ondeviceinfer/cache.py:60-80``)."""

    def __init__(self, num_layers: int):
        self.k = [None] * num_layers
        self.v = [None] * num_layers

    def length(self, layer: int = 0) -> int:
        return 0 if self.k[layer] is None else self.k[layer].shape[1]

    def update(self, layer: int, k: np.ndarray, v: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
        self.k[layer] = k if self.k[layer] is None else np.concatenate([self.k[layer], k], axis=1)
        self.v[layer] = v if self.v[layer] is None else np.concatenate([self.v[layer], v], axis=1)
        return self.k[layer], self.v[layer]


def decoder_layer(hidden: np.ndarray, weights: dict, cfg, layer_idx: int, cos: np.ndarray, sin: np.ndarray,
                  cache: KVCacheOracle | None, linear=None) -> np.ndarray:
    """One decoder layer on fp16 ``hidden [S, hidden]`` (batch 1), restating
    ``quantized_model.py:124-228`` with the QDQ linears.  ``linear(x, name)``
    defaults to ``qdq.qdq_linear`` on ``weights``."""
    if linear is None:
        def linear(x, name):
            return qdq.qdq_linear(x, weights, name)
    eps = cfg.rms_norm_eps
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    s_len = hidden.shape[0]
    residual = hidden
    states = rms_norm(hidden, weights['input_layernorm.weight'], eps)
    q = linear(states, 'self_attn.q_proj.weight').reshape(s_len, hq, d)
    k = linear(states, 'self_attn.k_proj.weight').reshape(s_len, hkv, d)
    v = linear(states, 'self_attn.v_proj.weight').reshape(s_len, hkv, d)
    q = rms_norm(q, weights['self_attn.q_norm.weight'], eps).transpose(1, 0, 2)
    k = rms_norm(k, weights['self_attn.k_norm.weight'], eps).transpose(1, 0, 2)
    v = v.transpose(1, 0, 2)
    q = apply_rope(q, cos, sin)
    k = apply_rope(k, cos, sin)
    if cache is not None:
        k, v = cache.update(layer_idx, k, v)
    t_len = k.shape[1]
    mask = build_causal_mask(s_len, t_len) if s_len > 1 else None
    attn = attention(q, k, v, mask).transpose(1, 0, 2).reshape(s_len, hq * d)
    hidden = (residual + linear(attn, 'self_attn.o_proj.weight')).astype(F16)
    residual = hidden
    states = rms_norm(hidden, weights['post_attention_layernorm.weight'], eps)
    gate = linear(states, 'mlp.gate_proj.weight')
    up = linear(states, 'mlp.up_proj.weight')
    mlp = linear(swiglu(gate, up), 'mlp.down_proj.weight')
    return (residual + mlp).astype(F16)


def forward(token_ids: np.ndarray, model: dict, cfg, cache: KVCacheOracle | None = None,
            logits_to_keep: int = 0) -> np.ndarray:
    """Logits ``[S', vocab]`` (fp16) for ``token_ids [S]`` (batch 1), restating
    ``QuantizedQwen3ForCausalLM.__call__`` (``quantized_model.py:280-338``):
    embedding, layers at positions ``past .. past + S - 1``, final norm, fp16
    LM head.  ``model``: ``embed_tokens``, ``layers`` (list of weight dicts),
    ``final_norm``, ``lm_head``; optionally ``linears`` (per layer, a dict of
    weight name -> ``qdq.DecodedLinear``) and ``lm_head_linear``, which give
    the same results with each weight decoded once."""
    ids = np.asarray(token_ids).reshape(-1)
    hidden = np.asarray(model['embed_tokens'])[ids].astype(F16)
    past = cache.length(0) if cache is not None else 0
    cos, sin = rotary_tables(cfg.head_dim, cfg.rope_theta, np.arange(past, past + ids.size))
    decoded = model.get('linears')
    for idx, weights in enumerate(model['layers']):
        linear = None
        if decoded is not None:
            def linear(x, name, _d=decoded[idx]):
                return _d[name](x)
        hidden = decoder_layer(hidden, weights, cfg, idx, cos, sin, cache, linear=linear)
    hidden = rms_norm(hidden, model['final_norm'], cfg.rms_norm_eps)
    if logits_to_keep > 0:
        hidden = hidden[-logits_to_keep:]
    if model.get('lm_head_linear') is not None:
        return model['lm_head_linear'](hidden)
    return qdq.linear_fp32(hidden, model['lm_head'])


def greedy_generate(prompt: np.ndarray, model: dict, cfg, max_new_tokens: int) -> np.ndarray:
    """Prefill then greedy decode with the cache (``generation.py:29-70``):
    the generated token ids ``[max_new_tokens]``."""
    cache = KVCacheOracle(cfg.num_hidden_layers)
    logits = forward(prompt, model, cfg, cache, logits_to_keep=1)
    out = [int(np.argmax(logits[-1].astype(F32)))]
    for _ in range(1, max_new_tokens):
        logits = forward(np.array([out[-1]]), model, cfg, cache, logits_to_keep=1)
        out.append(int(np.argmax(logits[-1].astype(F32))))
    return np.array(out, dtype=np.int64)
