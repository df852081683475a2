"""Pins for oracle/qwen3.py (CPU): the reference's own model tests restated,
library routines (torch on the CPU) and invariants."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import qdq, qwen3, synth


class Cfg:
    vocab_size = 97
    hidden_size = 256
    intermediate_size = 512
    num_hidden_layers = 2
    num_attention_heads = 2
    num_key_value_heads = 1
    head_dim = 128
    rms_norm_eps = 1e-6
    rope_theta = 1_000_000.0


def tiny_model(cfg=Cfg, seed=0):
    rng = np.random.default_rng(seed)
    layers = []
    shapes = {
        'self_attn.q_proj.weight': (cfg.num_attention_heads * cfg.head_dim, cfg.hidden_size),
        'self_attn.k_proj.weight': (cfg.num_key_value_heads * cfg.head_dim, cfg.hidden_size),
        'self_attn.v_proj.weight': (cfg.num_key_value_heads * cfg.head_dim, cfg.hidden_size),
        'self_attn.o_proj.weight': (cfg.hidden_size, cfg.num_attention_heads * cfg.head_dim),
        'mlp.gate_proj.weight': (cfg.intermediate_size, cfg.hidden_size),
        'mlp.up_proj.weight': (cfg.intermediate_size, cfg.hidden_size),
        'mlp.down_proj.weight': (cfg.hidden_size, cfg.intermediate_size),
    }
    for _ in range(cfg.num_hidden_layers):
        layer = {}
        for name, (n, k) in shapes.items():
            w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.05)).astype(np.float16)
            layer.update(synth.prefixed(synth.awq_quantize(w), name))
        for name, size in (('input_layernorm.weight', cfg.hidden_size), ('post_attention_layernorm.weight',
                                                                          cfg.hidden_size),
                           ('self_attn.q_norm.weight', cfg.head_dim), ('self_attn.k_norm.weight', cfg.head_dim)):
            layer[name] = (1 + 0.1 * rng.standard_normal(size)).astype(np.float16)
        layers.append(layer)
    return {'layers': layers,
            'embed_tokens': (rng.standard_normal((cfg.vocab_size, cfg.hidden_size)) * 0.5).astype(np.float16),
            'final_norm': (1 + 0.1 * rng.standard_normal(cfg.hidden_size)).astype(np.float16),
            'lm_head': (rng.standard_normal((cfg.vocab_size, cfg.hidden_size)) * 0.05).astype(np.float16)}


def test_causal_mask_kat():
    """Reference KAT tests/test_model.py:29-38."""
    expected = np.array([[True, True, True, True, False], [True, True, True, True, True]])
    assert np.array_equal(qwen3.build_causal_mask(2, 5), expected)
    with pytest.raises(ValueError):
        qwen3.build_causal_mask(3, 2)


def test_rms_norm_against_float64_closed_form_and_reference_recipe():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 5, 128)).astype(np.float16)
    w = rng.uniform(0.5, 1.5, 128).astype(np.float16)
    got = qwen3.rms_norm(x, w, 1e-6).astype(np.float64)
    x64 = x.astype(np.float64)
    closed = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * w.astype(np.float64)
    assert np.abs(got - closed).max() <= 4e-3 * np.abs(closed).max()
    # test_foundations.py:36-48: F.rms_norm in fp32, cast, times the weight
    recipe = (F.rms_norm(torch.from_numpy(x).float(), (128,), None, 1e-6).half() * torch.from_numpy(w)).numpy()
    assert np.abs(got - recipe.astype(np.float64)).max() <= 2 ** -9 * np.abs(closed).max()


def test_rotary_tables_match_torch_formula():
    pos = np.arange(0, 4096, 37)
    cos, sin = qwen3.rotary_tables(128, 1_000_000.0, pos)
    inv = 1.0 / (1_000_000.0 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))
    ang = torch.from_numpy(pos).float()[:, None] * inv
    ang = torch.cat((ang, ang), -1)
    assert np.abs(cos.astype(np.float32) - ang.cos().half().float().numpy()).max() <= 2 ** -10
    assert np.abs(sin.astype(np.float32) - ang.sin().half().float().numpy()).max() <= 2 ** -10


def test_rope_identity_at_position_zero_and_norm_preserving():
    """Reference test tests/test_foundations.py:51-67."""
    rng = np.random.default_rng(1)
    q = rng.standard_normal((8, 7, 128)).astype(np.float16)
    cos, sin = qwen3.rotary_tables(128, 1_000_000.0, np.arange(7))
    r = qwen3.apply_rope(q, cos, sin)
    assert np.array_equal(r[:, 0], q[:, 0])
    n0 = np.linalg.norm(q.astype(np.float64), axis=-1)
    n1 = np.linalg.norm(r.astype(np.float64), axis=-1)
    assert np.abs(n1 - n0).max() <= 2e-3 * n0.max()


def test_rope_dot_products_depend_only_on_relative_position():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 1, 128)).astype(np.float16)
    k = rng.standard_normal((1, 1, 128)).astype(np.float16)
    dots = []
    for m, n in ((10, 3), (107, 100), (1010, 1003)):
        cq, sq = qwen3.rotary_tables(128, 1_000_000.0, np.array([m]))
        ck, sk = qwen3.rotary_tables(128, 1_000_000.0, np.array([n]))
        a = qwen3.apply_rope(q, cq, sq).astype(np.float64).ravel()
        b = qwen3.apply_rope(k, ck, sk).astype(np.float64).ravel()
        dots.append(a @ b)
    assert max(dots) - min(dots) <= 0.05 * abs(dots[0]) + 0.05


def test_attention_matches_torch_sdpa_and_explicit_repetition():
    """GQA via SDPA (library) and via repeated K/V (tests/test_model.py:40-53)."""
    rng = np.random.default_rng(3)
    q = rng.standard_normal((4, 5, 16)).astype(np.float16)
    k = rng.standard_normal((2, 9, 16)).astype(np.float16)
    v = rng.standard_normal((2, 9, 16)).astype(np.float16)
    mask = qwen3.build_causal_mask(5, 9)
    got = qwen3.attention(q, k, v, mask).astype(np.float32)
    tq, tk, tv = (torch.from_numpy(a).float()[None] for a in (q, k, v))
    ref = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=torch.from_numpy(mask), enable_gqa=True)[0].numpy()
    rep = F.scaled_dot_product_attention(tq, tk.repeat_interleave(2, 1), tv.repeat_interleave(2, 1),
                                         attn_mask=torch.from_numpy(mask))[0].numpy()
    assert np.abs(got - ref).max() <= 2e-3 and np.abs(ref - rep).max() <= 1e-5
    # a single key returns its value
    one = qwen3.attention(q[:, :1], k[:, :1], v[:, :1], None)
    assert np.array_equal(one, np.repeat(v[:, :1], 2, axis=0))


def test_swiglu_formula():
    g = np.array([-2.0, -0.5, 0.0, 0.5, 3.0], dtype=np.float16)
    u = np.array([1.0, 2.0, 3.0, -1.0, 0.25], dtype=np.float16)
    expected = (F.silu(torch.from_numpy(g).float()).half() * torch.from_numpy(u)).numpy()
    assert np.array_equal(qwen3.swiglu(g, u), expected)


def _torch_layer(hidden, weights, cfg, cos, sin, past_k=None, past_v=None):
    """Independent float32 torch-CPU decoder layer (library ops only)."""
    def lin(x, name):
        return x @ torch.from_numpy(qdq.decode_weight(weights, name).astype(np.float32)).T

    def norm(x, w):
        return F.rms_norm(x, (x.shape[-1],), torch.from_numpy(w).float(), cfg.rms_norm_eps)

    def rope(x):
        c, s = torch.from_numpy(cos).float(), torch.from_numpy(sin).float()
        x1, x2 = x[..., :64], x[..., 64:]
        return x * c + torch.cat((-x2, x1), -1) * s

    h = torch.from_numpy(hidden).float()
    st = norm(h, weights['input_layernorm.weight'])
    s_len = h.shape[0]
    q = norm(lin(st, 'self_attn.q_proj.weight').view(s_len, -1, 128), weights['self_attn.q_norm.weight'])
    k = norm(lin(st, 'self_attn.k_proj.weight').view(s_len, -1, 128), weights['self_attn.k_norm.weight'])
    v = lin(st, 'self_attn.v_proj.weight').view(s_len, -1, 128)
    q, k, v = rope(q.transpose(0, 1)), rope(k.transpose(0, 1)), v.transpose(0, 1)
    if past_k is not None:
        k, v = torch.cat((past_k, k), 1), torch.cat((past_v, v), 1)
    mask = torch.from_numpy(qwen3.build_causal_mask(s_len, k.shape[1]))
    a = F.scaled_dot_product_attention(q[None], k[None], v[None], attn_mask=mask, enable_gqa=True)[0]
    h = h + lin(a.transpose(0, 1).reshape(s_len, -1), 'self_attn.o_proj.weight')
    st = norm(h, weights['post_attention_layernorm.weight'])
    h = h + lin(F.silu(lin(st, 'mlp.gate_proj.weight')) * lin(st, 'mlp.up_proj.weight'), 'mlp.down_proj.weight')
    return h.numpy(), k, v


def test_decoder_layer_matches_independent_float32_implementation():
    model = tiny_model()
    rng = np.random.default_rng(4)
    hidden = (rng.standard_normal((6, Cfg.hidden_size)) * 0.5).astype(np.float16)
    cos, sin = qwen3.rotary_tables(128, Cfg.rope_theta, np.arange(6))
    got = qwen3.decoder_layer(hidden, model['layers'][0], Cfg, 0, cos, sin, None).astype(np.float64)
    ref, _, _ = _torch_layer(hidden, model['layers'][0], Cfg, cos, sin)
    m = qdq.parity_metrics(got, ref)
    assert m['cosine'] >= 0.9999 and m['relative_l2'] <= 5e-3, m


def test_cached_decode_equals_longer_prefill():
    model = tiny_model()
    ids = np.array([5, 17, 3, 88, 41, 9, 60])
    full = qwen3.forward(ids, model, Cfg).astype(np.float64)
    cache = qwen3.KVCacheOracle(Cfg.num_hidden_layers)
    qwen3.forward(ids[:-1], model, Cfg, cache)
    step = qwen3.forward(ids[-1:], model, Cfg, cache).astype(np.float64)
    assert cache.length(0) == cache.length(1) == len(ids)
    m = qdq.parity_metrics(step[-1], full[-1])
    assert m['cosine'] >= 0.9999 and m['max_abs'] <= 2e-2 * m['ref_inf'], m


def test_greedy_generate_is_argmax_of_teacher_forced_logits():
    model = tiny_model()
    prompt = np.array([1, 2, 3, 4])
    gen = qwen3.greedy_generate(prompt, model, Cfg, 4)
    logits = qwen3.forward(np.concatenate([prompt, gen[:-1]]), model, Cfg).astype(np.float32)
    assert gen.shape == (4,)
    assert np.array_equal(np.argmax(logits[len(prompt) - 1:], axis=-1), gen)
