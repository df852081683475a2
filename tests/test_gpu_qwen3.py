"""A tiny Qwen3-shaped W4A16 model end to end on the GPU against the oracle's
forward (oracle/qwen3.py, QDQ linears): prefill through the W4 GEMM, decode
through the captured decode-step graph, and the reference's generation loop."""
import numpy as np
import pytest
import torch

from oracle import qdq, qwen3, synth

pytestmark = pytest.mark.gpu


class TinyCfg:
    vocab_size = 1000
    hidden_size = 512
    intermediate_size = 1024
    num_hidden_layers = 2
    num_attention_heads = 4
    num_key_value_heads = 2
    head_dim = 128
    rms_norm_eps = 1e-6
    rope_theta = 1_000_000.0


def numpy_model(cfg, seed=0):
    rng = np.random.default_rng(seed)
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    shapes = {'self_attn.q_proj.weight': (hq * d, cfg.hidden_size),
              'self_attn.k_proj.weight': (hkv * d, cfg.hidden_size),
              'self_attn.v_proj.weight': (hkv * d, cfg.hidden_size),
              'self_attn.o_proj.weight': (cfg.hidden_size, hq * d),
              'mlp.gate_proj.weight': (cfg.intermediate_size, cfg.hidden_size),
              'mlp.up_proj.weight': (cfg.intermediate_size, cfg.hidden_size),
              'mlp.down_proj.weight': (cfg.hidden_size, cfg.intermediate_size)}
    layers = []
    for _ in range(cfg.num_hidden_layers):
        layer = {}
        for name, (n, k) in shapes.items():
            w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.05)).astype(np.float16)
            layer.update(synth.prefixed(synth.awq_quantize(w), name))
        for name, size in (('input_layernorm.weight', cfg.hidden_size),
                           ('post_attention_layernorm.weight', cfg.hidden_size),
                           ('self_attn.q_norm.weight', d), ('self_attn.k_norm.weight', d)):
            layer[name] = (1 + 0.1 * rng.standard_normal(size)).astype(np.float16)
        layers.append(layer)
    return {'layers': layers,
            'embed_tokens': (rng.standard_normal((cfg.vocab_size, cfg.hidden_size)) * 0.5).astype(np.float16),
            'final_norm': (1 + 0.1 * rng.standard_normal(cfg.hidden_size)).astype(np.float16),
            'lm_head': (rng.standard_normal((cfg.vocab_size, cfg.hidden_size)) * 0.05).astype(np.float16)}


def build(np_model, cfg, decode_graph=True, quantize_lm_head=False):
    from ondeviceinfer_amd.config import Qwen3Config
    from ondeviceinfer_amd.quantized_model import QuantizedQwen3ForCausalLM
    from ondeviceinfer_amd.weight_quantization.backend import (CompressedLinearBackend, CompressedResidentRuntime,
                                                               CompressedStore)
    qcfg = Qwen3Config(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
                       intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_hidden_layers,
                       num_attention_heads=cfg.num_attention_heads, num_key_value_heads=cfg.num_key_value_heads,
                       head_dim=cfg.head_dim, max_position_embeddings=4096, rms_norm_eps=cfg.rms_norm_eps,
                       rope_theta=cfg.rope_theta, tie_word_embeddings=False)
    layers = []
    for layer in np_model['layers']:
        t = {}
        for key, value in layer.items():
            t[key] = torch.from_numpy(np.ascontiguousarray(value))
        layers.append(t)
    store = CompressedStore(qcfg, layers, torch.from_numpy(np_model['embed_tokens']),
                            torch.from_numpy(np_model['final_norm']), torch.from_numpy(np_model['lm_head']), {})
    backend = CompressedLinearBackend('marlin')
    runtime = CompressedResidentRuntime(store, backend, device='cuda:0', verbose=False)
    return QuantizedQwen3ForCausalLM(store, runtime, device='cuda:0', linear_backend=backend,
                                     decode_graph=decode_graph, quantize_lm_head=quantize_lm_head), backend


@pytest.fixture(scope='module')
def tiny(gpu):
    np_model = numpy_model(TinyCfg)
    model, backend = build(np_model, TinyCfg)
    return np_model, model, backend


def _ok(got, ref, what):
    m = qdq.parity_metrics(got.float().cpu().numpy(), ref.astype(np.float32))
    assert qdq.parity_ok(m), (what, m)


def test_prefill_then_graph_decode_match_oracle(tiny):
    np_model, model, backend = tiny
    cache = model.make_resident_cache(batch_size=1, max_seq_len=160)
    assert cache._decode_graph is not None
    prompt = np.random.default_rng(1).integers(0, TinyCfg.vocab_size, 100)
    ocache = qwen3.KVCacheOracle(TinyCfg.num_hidden_layers)
    print('[qwen3] prefill 100 tokens', flush=True)
    out = model(torch.from_numpy(prompt)[None].cuda(), cache=cache, logits_to_keep=1)
    ref = qwen3.forward(prompt, np_model, TinyCfg, ocache, logits_to_keep=1)
    assert out.logits.shape == (1, 1, TinyCfg.vocab_size) and cache.lengths == [100, 100]
    _ok(out.logits[0], ref, 'prefill')
    token = out.logits[:, -1].argmax(-1, keepdim=True)
    calls = backend.calls
    for step in range(6):
        print(f'[qwen3] decode step {step}', flush=True)
        out = model(token, cache=cache, logits_to_keep=1)
        ref = qwen3.forward(token.cpu().numpy().reshape(-1), np_model, TinyCfg, ocache, logits_to_keep=1)
        _ok(out.logits[0], ref, f'decode {step}')
        token = out.logits[:, -1].argmax(-1, keepdim=True)
    assert cache.lengths == [106, 106]
    assert backend.calls - calls == 6 * 4 * TinyCfg.num_hidden_layers


def test_chunked_prefill_matches_oracle(tiny):
    """A prompt in two multi-token chunks: the second chunk attends over cache
    rows it did not write (the explicit causal mask over the in-place cache
    rows), every position's logits against the oracle's forward."""
    np_model, model, _ = tiny
    cache = model.make_resident_cache(batch_size=1, max_seq_len=160)
    prompt = np.random.default_rng(2).integers(0, TinyCfg.vocab_size, 100)
    ocache = qwen3.KVCacheOracle(TinyCfg.num_hidden_layers)
    for lo, hi in ((0, 61), (61, 100)):
        print(f'[qwen3] prefill chunk {lo}..{hi}', flush=True)
        out = model(torch.from_numpy(prompt[lo:hi])[None].cuda(), cache=cache)
        ref = qwen3.forward(prompt[lo:hi], np_model, TinyCfg, ocache)
        assert out.logits.shape == (1, hi - lo, TinyCfg.vocab_size) and cache.lengths == [hi, hi]
        _ok(out.logits[0], ref, f'chunk {lo}..{hi}')


def test_graph_decode_equals_eager_decode(tiny):
    np_model, model, _ = tiny
    eager, _ = build(np_model, TinyCfg, decode_graph=False)
    prompt = torch.arange(20, 50)[None].cuda()
    ca = model.make_resident_cache(batch_size=1, max_seq_len=160)
    cb = eager.make_resident_cache(batch_size=1, max_seq_len=160)
    assert cb._decode_graph is None
    ta = model(prompt, cache=ca, logits_to_keep=1).logits[:, -1].argmax(-1, keepdim=True)
    tb = eager(prompt, cache=cb, logits_to_keep=1).logits[:, -1].argmax(-1, keepdim=True)
    for _ in range(4):
        la, lb = model(ta, cache=ca).logits, eager(ta, cache=cb).logits
        _ok(la[0], lb[0].float().cpu().numpy(), 'graph vs eager')
        ta = la[:, -1].argmax(-1, keepdim=True)


def test_pooled_graph_restarts_at_the_new_caches_position(tiny):
    """The decode step advances its device position itself, and the host
    writes the position only when the next call asks for another one: a
    pooled graph handed to a new cache (the previous owner gone) left the
    device at the old cache's next position, and the new cache's steps must
    still match the eager decoder at its own positions."""
    import gc
    np_model, model, _ = tiny
    eager, _ = build(np_model, TinyCfg, decode_graph=False)
    ca = model.make_resident_cache(batch_size=1, max_seq_len=160)
    graph = ca._decode_graph
    t = model(torch.arange(20, 50)[None].cuda(), cache=ca, logits_to_keep=1).logits[:, -1].argmax(-1, keepdim=True)
    for _ in range(3):
        t = model(t, cache=ca).logits[:, -1].argmax(-1, keepdim=True)
    assert graph._dev_position == 33                  # positions 30, 31, 32 decoded
    del ca
    gc.collect()
    cb = model.make_resident_cache(batch_size=1, max_seq_len=160)
    assert cb._decode_graph is graph
    ce = eager.make_resident_cache(batch_size=1, max_seq_len=160)
    prompt = torch.arange(100, 110)[None].cuda()
    tb = model(prompt, cache=cb, logits_to_keep=1).logits[:, -1].argmax(-1, keepdim=True)
    te = eager(prompt, cache=ce, logits_to_keep=1).logits[:, -1].argmax(-1, keepdim=True)
    assert torch.equal(tb, te)
    for step in range(3):
        lb, le = model(tb, cache=cb).logits, eager(tb, cache=ce).logits
        _ok(lb[0], le[0].float().cpu().numpy(), f'pooled graph vs eager, step {step}')
        assert graph._dev_position == 11 + step
        tb = lb[:, -1].argmax(-1, keepdim=True)


def test_greedy_generate_runs_the_reference_loop(tiny):
    from ondeviceinfer_amd.generation import greedy_generate
    np_model, model, _ = tiny
    cache = model.make_resident_cache(batch_size=1, max_seq_len=160)
    prompt = torch.arange(7, 19)[None].cuda()
    res = greedy_generate(model, prompt, max_new_tokens=8, cache=cache)
    assert res.generated_ids.shape == (1, 8) and res.token_ids.shape == (1, 20)
    assert res.decode_tokens_per_second > 0 and cache.lengths == [19, 19]
    gen = res.generated_ids[0].cpu().numpy()
    logits = qwen3.forward(np.concatenate([prompt[0].cpu().numpy(), gen[:-1]]), np_model, TinyCfg)
    logits = logits[11:].astype(np.float32)
    top2 = np.sort(logits, axis=-1)[:, -2:]
    decisive = (top2[:, 1] - top2[:, 0]) > 2e-2 * np.abs(logits).max()
    assert np.array_equal(np.argmax(logits, -1)[decisive], gen[decisive])


def test_w4_lm_head_prefill_and_graph_decode_match_oracle(tiny):
    """quantize_lm_head=True: the fp16 LM head quantized to uint4 G=128 and
    repacked at load; prefill logits through the W4 GEMV/GEMM, decode through
    the graph's W4 GEMV + wq_argmax_f16, against the oracle decoding the same
    codes (read back from the tiles with wq_w4_unpack)."""
    from ondeviceinfer_amd import _native
    np_model, _, _ = tiny
    model, _ = build(np_model, TinyCfg, quantize_lm_head=True)
    p = model.lm_head_w4
    packed, scale, zero = _native.w4_unpack(p.tiles, p.meta, p.n, p.k, p.group_size)
    head = {'lm_head.weight_packed': packed.cpu().numpy(), 'lm_head.weight_scale': scale.cpu().numpy(),
            'lm_head.weight_zero_point': zero.cpu().numpy(),
            'lm_head.weight_shape': np.array([p.n, p.k], dtype=np.int64)}
    decoded = qdq.decode_weight(head, 'lm_head.weight')
    # the quantized head is close to the fp16 one it came from (RTN, 4 bits)
    assert np.abs(decoded.astype(np.float32) - np_model['lm_head'].astype(np.float32)).max() < 0.05
    oracle_model = dict(np_model, lm_head_linear=qdq.DecodedLinear(head, 'lm_head.weight'))
    cache = model.make_resident_cache(batch_size=1, max_seq_len=160)
    assert cache._decode_graph is not None
    prompt = np.random.default_rng(3).integers(0, TinyCfg.vocab_size, 70)
    ocache = qwen3.KVCacheOracle(TinyCfg.num_hidden_layers)
    out = model(torch.from_numpy(prompt)[None].cuda(), cache=cache, logits_to_keep=5)
    _ok(out.logits[0], qwen3.forward(prompt, oracle_model, TinyCfg, ocache, logits_to_keep=5), 'w4 head prefill')
    token = out.logits[:, -1].argmax(-1, keepdim=True)
    for step in range(4):
        out = model(token, cache=cache, logits_to_keep=1)
        ref = qwen3.forward(token.cpu().numpy().reshape(-1), oracle_model, TinyCfg, ocache, logits_to_keep=1)
        _ok(out.logits[0], ref, f'w4 head decode {step}')
        assert torch.equal(out.next_token, out.logits[:, -1].argmax(-1, keepdim=True))
        token = out.next_token
