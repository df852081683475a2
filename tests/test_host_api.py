"""Host-side API of the INT8 containers, the resident cache and the greedy
generation loop (CPU only; no compute through the HIP library).  The
behaviours are the reference's (``tests/test_quantization.py:65-114``,
``ondeviceinfer/cache.py``, ``ondeviceinfer/generation.py``)."""
from dataclasses import dataclass

import pytest
import torch

from ondeviceinfer_amd.cache import ResidentKVCache, kv_block
from ondeviceinfer_amd.generation import GenerationResult, greedy_generate
from ondeviceinfer_amd.quantization import (QMAX, QMIN, QUANTIZATION_FORMAT, QUANTIZATION_VERSION,
                                            FP16DequantScratch, QuantizedLinearWeight, _scratch_view)


def _qw(rows=4, cols=6, scale=None):
    q = torch.arange(rows * cols, dtype=torch.int8).reshape(rows, cols)
    s = torch.linspace(0.5, 1.5, rows).half() if scale is None else scale
    return QuantizedLinearWeight(qweight=q, scale=s)


def test_tensor_dict_and_manifest_round_trip():
    w = _qw()
    prefix = 'model.layers.0.self_attn.q_proj.weight'
    tensors = w.tensor_dict(prefix)
    assert set(tensors) == {prefix + '.qweight', prefix + '.scale'}
    restored = QuantizedLinearWeight.from_tensor_dict(tensors, prefix)
    assert restored.qweight is w.qweight and restored.scale is w.scale
    assert w.tensor_dict() == {'qweight': w.qweight, 'scale': w.scale}
    assert set(w.tensor_dict('layer.')) == {'layer.qweight', 'layer.scale'}
    assert w.manifest_entry(prefix) == {
        'format': QUANTIZATION_FORMAT, 'version': QUANTIZATION_VERSION, 'axis': 0, 'zero_point': 0,
        'quant_min': QMIN, 'quant_max': QMAX, 'shape': [4, 6], 'qweight_key': prefix + '.qweight',
        'scale_key': prefix + '.scale', 'qweight_dtype': 'int8', 'scale_dtype': 'float16'}
    assert (QUANTIZATION_FORMAT, QUANTIZATION_VERSION, QMIN, QMAX) == \
        ('int8_per_output_channel_symmetric', 1, -127, 127)
    assert w.shape == (4, 6) and w.out_features == 4 and w.in_features == 6
    assert w.storage_nbytes == 24 + 8 and w.device.type == 'cpu'
    moved = w.to('cpu')
    assert torch.equal(moved.qweight, w.qweight) and moved.scale.dtype == torch.float16


@pytest.mark.parametrize('q,s,exc,msg', [
    (torch.zeros(4, dtype=torch.int8), torch.ones(4), ValueError, 'out_features, in_features'),
    (torch.zeros(4, 2), torch.ones(4), TypeError, 'torch.int8'),
    (torch.zeros(4, 2, dtype=torch.int8), torch.ones(3), ValueError, 'shape \\[out_features\\]'),
    (torch.zeros(4, 2, dtype=torch.int8), torch.ones(4, dtype=torch.int32), TypeError, 'floating-point'),
    (torch.zeros(4, 2, dtype=torch.int8), torch.tensor([1.0, float('inf'), 1.0, 1.0]), ValueError, 'finite'),
    (torch.zeros(4, 2, dtype=torch.int8), torch.tensor([1.0, 0.0, 1.0, 1.0]), ValueError, 'strictly positive'),
])
def test_container_validation(q, s, exc, msg):
    with pytest.raises(exc, match=msg):
        QuantizedLinearWeight(qweight=q, scale=s)


def test_container_is_frozen():
    w = _qw()
    with pytest.raises(Exception):
        w.qweight = torch.zeros(1)


def test_scratch_views_share_one_buffer():
    a, b = _qw(5, 8), _qw(3, 8)
    scratch = FP16DequantScratch.for_weights([a, b])
    assert scratch.capacity == 40 and scratch.device.type == 'cpu'
    ptr = scratch.buffer.data_ptr()
    assert scratch.view_for((5, 8)).data_ptr() == ptr and scratch.view_for([3, 8]).shape == (3, 8)
    with pytest.raises(ValueError, match='smaller than required'):
        scratch.view_for((6, 8))
    with pytest.raises(ValueError, match='at least one'):
        FP16DequantScratch.for_weights([])
    with pytest.raises(ValueError, match='positive'):
        FP16DequantScratch.allocate(0, device='cpu')
    with pytest.raises(TypeError, match='float16'):
        FP16DequantScratch(torch.zeros(4))
    with pytest.raises(ValueError, match='flat'):
        FP16DequantScratch(torch.zeros(2, 2).half())
    raw = torch.zeros(4, 10).half()
    assert _scratch_view(raw, (5, 8)).data_ptr() == raw.data_ptr()
    with pytest.raises(ValueError):
        _scratch_view(torch.zeros(10, 4).half().t(), (5, 8))
    with pytest.raises(TypeError):
        _scratch_view(torch.zeros(40), (5, 8))


def test_resident_cache_block_views_and_errors():
    cache = ResidentKVCache(num_layers=3, batch_size=2, num_key_value_heads=2, max_seq_len=5, head_dim=4,
                            device='cpu', dtype=torch.float16)
    assert len(cache.key_cache) == 3 and cache.key_cache[1].shape == (2, 2, 5, 4)
    assert cache.storage_bytes == 2 * 3 * 2 * 2 * 5 * 4 * 2
    rows = torch.randn(2, 2, 2, 4).half()
    k, v = cache.update(1, rows, -rows)
    assert k.shape == (2, 2, 2, 4) and torch.equal(v, -rows) and cache.lengths == [0, 2, 0]
    assert torch.equal(cache._block[0, 1, :, :, :2], rows)   # the views are the block
    with pytest.raises(ValueError, match='shapes differ'):
        cache.update(0, rows, rows[:, :, :1])
    with pytest.raises(ValueError, match='batch'):
        cache.update(0, rows[:1], rows[:1])
    with pytest.raises(ValueError, match='KV cache capacity exceeded: requested 6, capacity 5'):
        cache.update(1, torch.zeros(2, 2, 4, 4).half(), torch.zeros(2, 2, 4, 4).half())
    cache.reset()
    assert cache.lengths == [0, 0, 0] and cache.stats.cpu_to_gpu_bytes == 0
    with pytest.raises(ValueError, match='positive'):
        ResidentKVCache(num_layers=1, batch_size=1, num_key_value_heads=1, max_seq_len=0, head_dim=4,
                        device='cpu', dtype=torch.float16)
    block = kv_block(2, 1, 2, 7, 4, device='cpu', dtype=torch.float16, zero=True)
    over = ResidentKVCache.over(block)
    assert over.max_seq_len == 7 and over.batch_size == 1 and over.lengths == [0, 0]
    assert over.key_cache[1].data_ptr() == block[0, 1].data_ptr()
    with pytest.raises(ValueError):
        ResidentKVCache.over(torch.zeros(3, 4))


@dataclass
class _Out:
    logits: torch.Tensor
    next_token: torch.Tensor | None = None


class _CountingModel:
    """Next token = previous + 1 (mod vocab) via one-hot logits; optionally
    hands the token over as ``next_token`` like the decode graph does."""

    def __init__(self, vocab=50, device_token=False):
        self.vocab, self.device_token, self.calls = vocab, device_token, []

    def __call__(self, ids, *, cache, logits_to_keep=0):
        self.calls.append(tuple(ids.shape))
        nxt = (ids[:, -1:] + 1) % self.vocab
        logits = torch.nn.functional.one_hot(nxt, self.vocab).half()
        return _Out(logits, nxt.clone() if self.device_token else None)


@pytest.mark.parametrize('device_token', [False, True])
def test_greedy_generate_loop(device_token):
    model = _CountingModel(device_token=device_token)
    prompt = torch.tensor([[3, 4, 5]])
    res = greedy_generate(model, prompt, max_new_tokens=6, cache=None)
    assert res.generated_ids.tolist() == [[6, 7, 8, 9, 10, 11]]
    assert res.token_ids.tolist() == [[3, 4, 5, 6, 7, 8, 9, 10, 11]]
    assert model.calls == [(1, 3)] + [(1, 1)] * 5
    assert res.prefill_seconds >= 0 and res.decode_seconds > 0
    assert res.decode_tokens_per_second == pytest.approx(5 / res.decode_seconds)
    # eos: the eos token is kept, nothing after it
    res = greedy_generate(_CountingModel(device_token=device_token), prompt, max_new_tokens=6, cache=None,
                          eos_token_id=8)
    assert res.generated_ids.tolist() == [[6, 7, 8]]
    # the prefill's token always exists
    res = greedy_generate(_CountingModel(), prompt, max_new_tokens=0, cache=None)
    assert res.generated_ids.tolist() == [[6]]
    assert GenerationResult(prompt, res.generated_ids, 0.1, 0.0).decode_tokens_per_second == 0.0


def test_greedy_generate_rejects_bad_inputs():
    with pytest.raises(ValueError, match='batch, sequence'):
        greedy_generate(_CountingModel(), torch.tensor([1, 2]), max_new_tokens=2, cache=None)
    with pytest.raises(NotImplementedError, match='batch size 1'):
        greedy_generate(_CountingModel(), torch.tensor([[1], [2]]), max_new_tokens=2, cache=None)
