"""Host-side logic of the Qwen3 forward (CPU only): cache, mask, rotary
tables, projection fusion, the synthetic checkpoint writer and the decode-op
argument checks of the C ABI."""
import ctypes

import numpy as np
import pytest
import torch

from ondeviceinfer_amd import _native
from ondeviceinfer_amd.attention import build_causal_mask
from ondeviceinfer_amd.cache import ResidentKVCache
from ondeviceinfer_amd.config import Qwen3Config
from ondeviceinfer_amd.layers import RotaryEmbedding, apply_rotary_pos_emb
from ondeviceinfer_amd.weight_quantization.backend import (FUSED_PROJECTIONS, CompressedLinearBackend, PreparedW4,
                                                           PreparedW8, load_compressed_store)
from ondeviceinfer_amd.weight_quantization.synthetic import (linear_shapes, random_compressed_store,
                                                             write_compressed_checkpoint)
from oracle import qwen3


def tiny_config(layers=2):
    return Qwen3Config(vocab_size=101, hidden_size=256, intermediate_size=512, num_hidden_layers=layers,
                       num_attention_heads=2, num_key_value_heads=1, head_dim=128, max_position_embeddings=128,
                       rms_norm_eps=1e-6, rope_theta=1_000_000.0, tie_word_embeddings=False)


def test_causal_mask_kat():
    """tests/test_model.py:29-38 of the reference."""
    mask = build_causal_mask(2, 5, device=torch.device('cpu'))
    assert torch.equal(mask, torch.tensor([[True, True, True, True, False], [True, True, True, True, True]]))


def test_resident_cache_appends_without_reallocation():
    """tests/test_model.py:77-98 of the reference."""
    cache = ResidentKVCache(num_layers=2, batch_size=1, num_key_value_heads=2, max_seq_len=8, head_dim=4,
                            device='cpu', dtype=torch.float32)
    ptr = cache.key_cache[0].data_ptr()
    first, second = torch.randn(1, 2, 3, 4), torch.randn(1, 2, 1, 4)
    cache.update(0, first, first)
    keys, _ = cache.update(0, second, second)
    assert cache.get_seq_length(0) == 4 and cache.get_seq_length(1) == 0
    assert cache.key_cache[0].data_ptr() == ptr
    assert torch.equal(keys[:, :, :3], first) and torch.equal(keys[:, :, 3:], second)
    with pytest.raises(ValueError, match='capacity exceeded'):
        cache.update(0, torch.randn(1, 2, 5, 4), torch.randn(1, 2, 5, 4))
    cache.reset()
    assert cache.lengths == [0, 0]


def test_rotary_embedding_identity_at_zero_and_matches_oracle_tables():
    """tests/test_foundations.py:51-67 of the reference, plus the table the
    decode kernel reads against the oracle's numpy tables."""
    rope = RotaryEmbedding(128, 1_000_000)
    q, k = torch.randn(2, 16, 7, 128), torch.randn(2, 8, 7, 128)
    cos, sin = rope(q, torch.arange(7).expand(2, -1))
    qr, kr = apply_rotary_pos_emb(q, k, cos, sin)
    assert cos.shape == (2, 7, 128)
    assert torch.equal(qr[:, :, 0], q[:, :, 0]) and torch.equal(kr[:, :, 0], k[:, :, 0])
    assert torch.allclose(qr.norm(dim=-1), q.norm(dim=-1), atol=1e-5)
    tc, ts = rope.table(300, 'cpu')
    oc, os_ = qwen3.rotary_tables(128, 1_000_000.0, np.arange(300))
    assert tc.shape == (300, 128) and tc.dtype == torch.float16
    assert np.abs(tc.float().numpy() - oc.astype(np.float32)).max() <= 2 ** -10
    assert np.abs(ts.float().numpy() - os_.astype(np.float32)).max() <= 2 ** -10


def _fake_w4(n, k, fill):
    tb, mb = _native.w4_repack_size(n, k, 128)
    return PreparedW4(torch.full((tb,), fill, dtype=torch.uint8), torch.full((mb,), fill, dtype=torch.uint8),
                      None, k, n, 128)


def test_fuse_projections_concatenates_and_leaves_views():
    backend = CompressedLinearBackend('reference_int4')
    layer = {'self_attn.q_proj._prepared': _fake_w4(256, 256, 1), 'self_attn.k_proj._prepared': _fake_w4(128, 256, 2),
             'self_attn.v_proj._prepared': _fake_w4(128, 256, 3), 'mlp.gate_proj._prepared': _fake_w4(512, 256, 4),
             'mlp.up_proj._prepared': _fake_w4(512, 256, 5)}
    backend.fuse_projections(layer)
    qkv = layer['self_attn.qkv_proj._prepared']
    assert qkv.n == 512 and qkv.k == 256
    assert qkv.tiles.numel() == sum(_native.w4_repack_size(n, 256, 128)[0] for n in (256, 128, 128))
    q, k, v = (layer[f'self_attn.{p}_proj._prepared'] for p in 'qkv')
    assert q.tiles.data_ptr() == qkv.tiles.data_ptr()
    assert k.tiles.data_ptr() == qkv.tiles.data_ptr() + q.tiles.numel()
    assert int(v.tiles[0]) == 3 and int(v.meta[-1]) == 3
    assert layer['mlp.gate_up_proj._prepared'].n == 1024
    assert set(FUSED_PROJECTIONS) == {'self_attn.qkv_proj', 'mlp.gate_up_proj'}


def test_fuse_projections_int8_rows_and_skips_mismatched():
    backend = CompressedLinearBackend('reference_int4')
    q8 = [torch.full((n, 64), i, dtype=torch.int8) for i, n in enumerate((32, 16, 16))]
    s8 = [torch.full((n,), float(i + 1), dtype=torch.float16) for i, n in enumerate((32, 16, 16))]
    layer = {f'self_attn.{p}_proj._prepared': PreparedW8(q, s, 64, q.shape[0]) for p, q, s in zip('qkv', q8, s8)}
    layer['mlp.gate_proj._prepared'] = PreparedW8(torch.zeros(8, 64, dtype=torch.int8), torch.ones(8).half(), 64, 8)
    layer['mlp.up_proj._prepared'] = PreparedW8(torch.zeros(8, 32, dtype=torch.int8), torch.ones(8).half(), 32, 8)
    backend.fuse_projections(layer)
    fused = layer['self_attn.qkv_proj._prepared']
    assert fused.qweight.shape == (64, 64) and int(fused.qweight[40, 0]) == 1 and float(fused.scale[63]) == 3.0
    assert 'mlp.gate_up_proj._prepared' not in layer      # different k: left alone


def test_synthetic_checkpoint_round_trips_through_the_loader(tmp_path):
    cfg = tiny_config()
    store = random_compressed_store(cfg, seed=3)
    path = write_compressed_checkpoint(tmp_path / 'ckpt', store, layers_per_shard=1)
    loaded = load_compressed_store(path)
    assert loaded.config == cfg
    assert loaded.manifest['quantization_config']['format'] == 'pack-quantized'
    for a, b in zip(store.layers, loaded.layers):
        assert set(a) == set(b)
        for key in a:
            assert torch.equal(a[key].cpu(), b[key]), key
    assert torch.equal(store.lm_head, loaded.lm_head) and torch.equal(store.embed_tokens, loaded.embed_tokens)
    shapes = linear_shapes(cfg)
    assert shapes['mlp.down_proj.weight'] == (256, 512)


def test_symmetric_synthetic_store_has_no_zero_points():
    store = random_compressed_store(tiny_config(1), symmetric=True)
    assert not any(k.endswith('weight_zero_point') for k in store.layers[0])


def _status(fn, *args):
    return getattr(_native.load(), fn)(*args)


def test_decode_op_argument_checks_on_the_host():
    b = ctypes.c_size_t()
    assert _status('wq_decode_attention_workspace_size', 40, 8, 128, 4224, ctypes.byref(b)) == _native.WQ_OK
    # 264 blocks of 16 positions, 32 chunks wanted per kv head -> 10 blocks per chunk
    # (five waves x 2), 27 chunks per kv head
    ml = (8 * 27 * 5 * 2 * 4 + 255) // 256 * 256          # (max, sum) | partial outputs
    assert b.value == ml + 8 * 27 * 5 * 128 * 4
    assert _status('wq_decode_attention_workspace_size', 32, 4, 128, 9000, ctypes.byref(b)) == _native.WQ_OK
    ml = (4 * 57 * 8 * 2 * 4 + 255) // 256 * 256          # 563 blocks, 64 wanted -> 10 per chunk, 57 chunks
    assert b.value == ml + 4 * 57 * 8 * 128 * 4
    assert _status('wq_decode_attention_workspace_size', 40, 8, 128, 300, ctypes.byref(b)) == _native.WQ_OK
    ml = (8 * 4 * 5 * 2 * 4 + 255) // 256 * 256           # 19 blocks -> 5 per chunk (one per wave), 4 chunks
    assert b.value == ml + 8 * 4 * 5 * 128 * 4
    assert _status('wq_decode_attention_workspace_size', 40, 8, 128, 16384, ctypes.byref(b)) == _native.WQ_OK
    ml = (8 * 64 * 5 * 2 * 4 + 255) // 256 * 256          # 1024 blocks: four-wave split, 16 per chunk, 64 chunks
    assert b.value == ml + 8 * 64 * 5 * 128 * 4
    assert _status('wq_decode_attention_workspace_size', 40, 8, 64, 4224, ctypes.byref(b)) == _native.WQ_ERR_UNSUPPORTED
    assert b'head_dim 128' in _native.load().wq_last_error()
    assert _status('wq_decode_attention_workspace_size', 40, 3, 128, 4224, ctypes.byref(b)) == \
        _native.WQ_ERR_INVALID_ARGUMENT
    assert _status('wq_decode_attention_workspace_size', 80, 8, 128, 64, ctypes.byref(b)) == _native.WQ_ERR_UNSUPPORTED
    assert _status('wq_decode_attention_workspace_size', 8, 8, 128, 16384, ctypes.byref(b)) == _native.WQ_OK
    assert _status('wq_decode_attention_workspace_size', 8, 8, 128, 16385, ctypes.byref(b)) == \
        _native.WQ_ERR_UNSUPPORTED
    assert _status('wq_decode_attention_workspace_size', 8, 8, 128, 64, ctypes.byref(b)) == _native.WQ_OK
    assert b.value == 0        # one chunk: no cross-workgroup merge
    # missing workspace for a multi-chunk cache
    assert _status('wq_decode_attention', 16, 8, 8, 128, None, None, ctypes.c_float(1e-6), 16, 16, 16, 16, 16, 4096,
                   ctypes.c_float(0.1), 16, None, 0, None) == _native.WQ_ERR_WORKSPACE
    assert _status('wq_add_rmsnorm', None, None, None, 1, 256, ctypes.c_float(1e-6), None, None, None) == \
        _native.WQ_ERR_INVALID_ARGUMENT
    assert _status('wq_add_rmsnorm', 16, None, 16, 1, 12, ctypes.c_float(1e-6), 16, None, None) == \
        _native.WQ_ERR_INVALID_ARGUMENT
    assert _status('wq_add_rmsnorm', None, None, None, 0, 256, ctypes.c_float(1e-6), None, None, None) == _native.WQ_OK
    assert _status('wq_silu_mul', 16, 1, 12, 16, None) == _native.WQ_ERR_INVALID_ARGUMENT
