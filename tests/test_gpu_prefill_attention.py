"""Prefill causal GQA attention kernel (wq_prefill_attention) against the
oracle's softmax attention (oracle/qwen3.py), on sampled query rows at the
Qwen3-14B prompt size; cache rows past the last query's position hold NaN,
so a read of them that reached the output would show."""
import numpy as np
import pytest
import torch

from oracle import qdq, qwen3

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def nat(gpu):
    from ondeviceinfer_amd import _native
    _native.load()
    return _native


def _case(T, start, H, KV, max_seq, seed):
    rng = np.random.default_rng(seed)
    kc = np.full((KV, max_seq, 128), np.nan, dtype=np.float16)
    vc = np.full((KV, max_seq, 128), np.nan, dtype=np.float16)
    kc[:, :start + T] = rng.standard_normal((KV, start + T, 128)).astype(np.float16)
    vc[:, :start + T] = rng.standard_normal((KV, start + T, 128)).astype(np.float16)
    q = (rng.standard_normal((T, H, 128)) * 1.5).astype(np.float16)
    return q, kc, vc


def _rows(T):
    if T <= 160:
        return np.arange(T)
    picks = {0, 1, 15, 16, 31, 32, 63, 64, 127, 128, T // 2, T - 129, T - 128, T - 2, T - 1}
    return np.array(sorted(t for t in picks if 0 <= t < T))


@pytest.mark.parametrize('T,start,H,KV,max_seq', [
    (1, 0, 40, 8, 64),            # one token
    (7, 100, 8, 4, 200),          # a chunk after 100 cached rows
    (128, 0, 40, 8, 128),         # one full query block, cache exactly full
    (300, 0, 64, 8, 300),         # 8 query heads per kv head, partial last block
    (1000, 37, 8, 8, 1100),       # no grouping, odd offset
    (129, 4000, 40, 8, 4200),     # long prefix, two query blocks
    (4096, 0, 40, 8, 4119),       # Qwen3-14B 4K prompt (sampled rows)
])
def test_prefill_attention_matches_oracle(nat, T, start, H, KV, max_seq):
    print(f'[prefill_attention] T={T} start={start} H={H} KV={KV} max_seq={max_seq}', flush=True)
    q, kc, vc = _case(T, start, H, KV, max_seq, seed=T + start + H)
    out = nat.prefill_attention(torch.from_numpy(q).cuda(), H, KV, torch.from_numpy(kc).cuda(),
                                torch.from_numpy(vc).cuda(), start, 1.0 / np.sqrt(128.0))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    for t in _rows(T):
        end = start + t + 1
        ref = qwen3.attention(q[t][:, None, :], kc[:, :end], vc[:, :end], None)[:, 0, :]
        m = qdq.parity_metrics(got[t], ref)
        assert qdq.parity_ok(m), (t, m)


def test_prefill_attention_equals_across_calls_and_matches_torch_sdpa(nat):
    """Deterministic bits over repeated calls; close to torch's fused SDPA
    (the path it replaces) at the 4K prompt."""
    from ondeviceinfer_amd.attention import strided_prefill_attention
    T, H, KV, max_seq = 4096, 40, 8, 4119
    q, kc, vc = _case(T, 0, H, KV, max_seq, seed=5)
    qd, kd, vd = torch.from_numpy(q).cuda(), torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda()
    a = nat.prefill_attention(qd, H, KV, kd, vd, 0, 1.0 / np.sqrt(128.0))
    b = nat.prefill_attention(qd, H, KV, kd, vd, 0, 1.0 / np.sqrt(128.0))
    assert torch.equal(a, b)
    ref = strided_prefill_attention(qd.transpose(0, 1).unsqueeze(0), kd[None, :, :T], vd[None, :, :T])
    ref = ref[0].transpose(0, 1).float().cpu().numpy()
    m = qdq.parity_metrics(a.float().cpu().numpy(), ref)
    assert qdq.parity_ok(m), m


def test_prefill_attention_rejects_capacity_overflow(nat):
    kd = torch.zeros(8, 64, 128, dtype=torch.float16, device='cuda')
    q = torch.zeros(10, 40, 128, dtype=torch.float16, device='cuda')
    with pytest.raises(ValueError, match='exceed'):
        nat.prefill_attention(q, 40, 8, kd, kd, 60, 0.1)


def test_prefill_attention_rejects_non_positive_scale(nat):
    kd = torch.zeros(8, 64, 128, dtype=torch.float16, device='cuda')
    q = torch.zeros(10, 40, 128, dtype=torch.float16, device='cuda')
    for bad in (0.0, -0.1, float('inf')):
        with pytest.raises(ValueError, match='scale'):
            nat.prefill_attention(q, 40, 8, kd, kd, 0, bad)
