"""Decode-step operators on the GPU against the oracle (oracle/qwen3.py):
add + RMSNorm, SiLU * up, and the fused q/k-norm + RoPE + KV-append + GQA
attention kernel, through the C ABI."""
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


def _close(got, ref, rel=4e-3):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert np.isfinite(got).all()
    err = np.abs(got - ref).max()
    assert err <= rel * max(np.abs(ref).max(), 1e-3), (err, np.abs(ref).max())


@pytest.mark.parametrize('rows,n,with_delta,in_place', [(1, 5120, True, True), (1, 5120, False, False),
                                                        (37, 512, True, False), (4096, 5120, True, True)])
def test_add_rmsnorm(nat, rows, n, with_delta, in_place):
    print(f'[add_rmsnorm] rows={rows} n={n} delta={with_delta} in_place={in_place}', flush=True)
    rng = np.random.default_rng(rows + n)
    x = (rng.standard_normal((rows, n)) * 3).astype(np.float16)
    d = (rng.standard_normal((rows, n)) * 2).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float16)
    tx, td, tw = (torch.from_numpy(a).cuda() for a in (x, d, w))
    out_sum = tx if in_place else torch.empty_like(tx)
    y = nat.add_rmsnorm(tx, tw, 1e-6, delta=td if with_delta else None, out_sum=out_sum)
    torch.cuda.synchronize()
    s = (x + d).astype(np.float16) if with_delta else x
    assert np.array_equal(out_sum.cpu().numpy(), s)
    _close(y.cpu().numpy(), qwen3.rms_norm(s, w, 1e-6))


def test_functional_add_rms_norm_equals_two_steps(nat):
    """The prefill's fused residual add + RMSNorm gives the same bits as torch's
    fp16 ``+`` followed by ``rms_norm``, and leaves the residual untouched."""
    from ondeviceinfer_amd.functional import add_rms_norm, rms_norm
    print('[add_rms_norm] rows=4096 n=5120', flush=True)
    g = torch.Generator().manual_seed(11)
    r = (torch.randn(1, 4096, 5120, generator=g) * 3).half().cuda()
    d = (torch.randn(1, 4096, 5120, generator=g) * 2).half().cuda()
    w = (1 + 0.1 * torch.randn(5120, generator=g)).half().cuda()
    r_before = r.clone()
    summed, normed = add_rms_norm(r, d, w, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(r, r_before)
    assert torch.equal(summed, r + d)
    assert torch.equal(normed, rms_norm(r + d, w, 1e-6))


def test_silu_mul(nat):
    rng = np.random.default_rng(5)
    gu = (rng.standard_normal((3, 2 * 17408)) * 3).astype(np.float16)
    y = nat.silu_mul(torch.from_numpy(gu).cuda()).cpu().numpy()
    ref = qwen3.swiglu(gu[:, :17408], gu[:, 17408:])
    ulp = np.abs(y.astype(np.float64) - ref.astype(np.float64)) / np.maximum(np.abs(ref.astype(np.float64)), 2 ** -14)
    assert ulp.max() <= 2 ** -9


class AttnCase:
    """Random qkv and cache rows 0..pos-1; rows past pos hold NaN so a read
    beyond the attended range would poison the output."""

    def __init__(self, h, kv, max_seq, seed, norms=True):
        self.h, self.kv, self.max_seq = h, kv, max_seq
        rng = np.random.default_rng(seed)
        self.rng = rng
        self.qn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float16) if norms else None
        self.kn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float16) if norms else None
        self.cos, self.sin = qwen3.rotary_tables(128, 1_000_000.0, np.arange(max_seq))
        self.kc = np.full((kv, max_seq, 128), np.nan, dtype=np.float16)
        self.vc = np.full((kv, max_seq, 128), np.nan, dtype=np.float16)

    def fill(self, upto):
        self.kc[:, :upto] = self.rng.standard_normal((self.kv, upto, 128)).astype(np.float16)
        self.vc[:, :upto] = self.rng.standard_normal((self.kv, upto, 128)).astype(np.float16)

    def qkv(self):
        return (self.rng.standard_normal((self.h + 2 * self.kv) * 128) * 2).astype(np.float16)

    def expected(self, qkv, pos):
        h, kv = self.h, self.kv
        q = qkv[:h * 128].reshape(h, 1, 128)
        k = qkv[h * 128:(h + kv) * 128].reshape(kv, 1, 128)
        v = qkv[(h + kv) * 128:].reshape(kv, 1, 128)
        if self.qn is not None:
            q = qwen3.rms_norm(q, self.qn, 1e-6)
            k = qwen3.rms_norm(k, self.kn, 1e-6)
        c, s = self.cos[pos:pos + 1], self.sin[pos:pos + 1]
        q, k = qwen3.apply_rope(q, c, s), qwen3.apply_rope(k, c, s)
        keys = np.concatenate([self.kc[:, :pos], k], axis=1)
        vals = np.concatenate([self.vc[:, :pos], v], axis=1)
        return qwen3.attention(q, keys, vals, None).reshape(-1), k[:, 0], v[:, 0]

    def tensors(self):
        t = {'kc': torch.from_numpy(self.kc).cuda(), 'vc': torch.from_numpy(self.vc).cuda(),
             'cos': torch.from_numpy(self.cos).cuda(), 'sin': torch.from_numpy(self.sin).cuda()}
        t['qn'] = None if self.qn is None else torch.from_numpy(self.qn).cuda()
        t['kn'] = None if self.kn is None else torch.from_numpy(self.kn).cuda()
        return t


def _run(nat, case, t, qkv, pos, ws):
    p = torch.tensor([pos], dtype=torch.int32, device='cuda')
    out = nat.decode_attention(torch.from_numpy(qkv).cuda(), case.h, case.kv, t['qn'], t['kn'], 1e-6, t['cos'],
                               t['sin'], p, t['kc'], t['vc'], 1.0 / np.sqrt(128.0), workspace=ws)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize('h,kv,max_seq,positions', [
    (40, 8, 4224, (0, 1, 15, 16, 63, 64, 65, 1000, 4095, 4096, 4223)),   # Qwen3-14B at a 4K+128 cache
    (40, 8, 16384, (0, 255, 256, 9000, 16383)),      # largest cache: 64 workgroups of 4 sub-chunks
    (8, 4, 9000, (0, 191, 192, 8999)),                # 47 workgroups of 3 sub-chunks
    (40, 8, 64, (0, 10, 63)),                         # one chunk: no cross-workgroup merge
    (64, 8, 300, (0, 129, 299)),                      # 8 query heads per kv head
    (8, 8, 200, (5, 199)),                            # no grouping
])
def test_decode_attention_matches_oracle(nat, h, kv, max_seq, positions):
    case = AttnCase(h, kv, max_seq, seed=h + max_seq)
    # All-ones bytes (NaN floats): the workspace needs no initialization.
    ws = torch.full((max(nat.decode_attention_workspace_size(h, kv, 128, max_seq), 1),), 255, dtype=torch.uint8,
                    device='cuda')
    for pos in positions:
        print(f'[decode_attention] h={h} kv={kv} max_seq={max_seq} pos={pos}', flush=True)
        case.kc[:] = np.nan
        case.vc[:] = np.nan
        case.fill(pos)
        t = case.tensors()
        qkv = case.qkv()
        got = _run(nat, case, t, qkv, pos, ws)
        ref, k_new, v_new = case.expected(qkv, pos)
        m = qdq.parity_metrics(got, ref)
        assert qdq.parity_ok(m), (pos, m)
        kc = t['kc'].cpu().numpy()
        assert np.array_equal(t['vc'].cpu().numpy()[:, pos], v_new)
        _close(kc[:, pos], k_new)
        assert np.isnan(kc[:, pos + 1:]).all() and np.array_equal(kc[:, :pos], case.kc[:, :pos])



@pytest.mark.parametrize('tokens,start,h,kv,with_norm', [(37, 5, 40, 8, True), (1, 0, 8, 8, True),
                                                          (300, 100, 64, 8, False), (4096, 0, 40, 8, True)])
def test_prefill_qk_rope_matches_oracle(nat, tokens, start, h, kv, with_norm):
    """Multi-token q/k RMSNorm + RoPE + cache append (one launch) against the
    oracle's rms_norm / apply_rope; v copied bit for bit; other cache rows kept."""
    d, eps = 128, 1e-6
    rng = np.random.default_rng(tokens + start + h)
    max_seq = start + tokens + 3
    qkv = rng.standard_normal((tokens, (h + 2 * kv) * d), dtype=np.float32).astype(np.float16)
    qn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float16)
    kn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float16)
    cos, sin = qwen3.rotary_tables(d, 1e6, np.arange(start, start + tokens))
    kc = torch.full((kv, max_seq, d), float('nan'), dtype=torch.float16, device='cuda')
    vc = torch.full((kv, max_seq, d), float('nan'), dtype=torch.float16, device='cuda')
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    q = nat.prefill_qk_rope(dev(qkv), h, kv, dev(qn) if with_norm else None, dev(kn) if with_norm else None, eps,
                            dev(cos), dev(sin), start, kc, vc)
    torch.cuda.synchronize()
    x = qkv.reshape(tokens, h + 2 * kv, d)
    qr, kr, vr = x[:, :h], x[:, h:h + kv], x[:, h + kv:]
    if with_norm:
        qr, kr = qwen3.rms_norm(qr, qn, eps), qwen3.rms_norm(kr, kn, eps)
    q_ref = qwen3.apply_rope(qr.transpose(1, 0, 2), cos, sin)
    k_ref = qwen3.apply_rope(kr.transpose(1, 0, 2), cos, sin)
    assert tuple(q.shape) == (tokens, h, d)
    _close(q.cpu().numpy().transpose(1, 0, 2), q_ref)
    kcn, vcn = kc.cpu().numpy(), vc.cpu().numpy()
    _close(kcn[:, start:start + tokens], k_ref)
    assert np.array_equal(vcn[:, start:start + tokens], vr.transpose(1, 0, 2))
    for c in (kcn, vcn):
        assert np.isnan(c[:, :start]).all() and np.isnan(c[:, start + tokens:]).all()


def test_prefill_qk_rope_rejects_capacity_overflow(nat):
    kc = torch.zeros((8, 16, 128), dtype=torch.float16, device='cuda')
    qkv = torch.zeros((4, 56 * 128), dtype=torch.float16, device='cuda')
    cs = torch.zeros((4, 128), dtype=torch.float16, device='cuda')
    with pytest.raises(ValueError, match='capacity'):
        nat.prefill_qk_rope(qkv, 40, 8, None, None, 1e-6, cs, cs, 13, kc, kc.clone())


def test_decode_attention_without_norms(nat):
    case = AttnCase(16, 4, 500, seed=9, norms=False)
    ws = torch.zeros(nat.decode_attention_workspace_size(16, 4, 128, 500), dtype=torch.uint8, device='cuda')
    case.fill(321)
    t = case.tensors()
    qkv = case.qkv()
    got = _run(nat, case, t, qkv, 321, ws)
    ref, _, _ = case.expected(qkv, 321)
    assert qdq.parity_ok(qdq.parity_metrics(got, ref))


def test_decode_attention_out_of_range_position_leaves_cache(nat):
    case = AttnCase(16, 4, 128, seed=3)
    case.fill(128)
    t = case.tensors()
    before = t['kc'].clone()
    ws = torch.zeros(nat.decode_attention_workspace_size(16, 4, 128, 128), dtype=torch.uint8, device='cuda')
    got = _run(nat, case, t, case.qkv(), 128, ws)
    assert np.isnan(got).all()
    assert torch.equal(t['kc'], before)
    # the next in-range call still works with the same workspace
    qkv = case.qkv()
    case.kc = t['kc'].cpu().numpy()
    got = _run(nat, case, t, qkv, 100, ws)
    ref, _, _ = case.expected(qkv, 100)
    assert qdq.parity_ok(qdq.parity_metrics(got, ref))


def test_decode_attention_graph_replays_follow_the_position(nat):
    """Captured once, replayed for consecutive positions (each replay appends
    one row), with eager work and synchronizations between replays."""
    case = AttnCase(40, 8, 1024, seed=11)
    case.fill(500)
    t = case.tensors()
    ws = torch.zeros(nat.decode_attention_workspace_size(40, 8, 128, 1024), dtype=torch.uint8, device='cuda')
    pos_t = torch.zeros(1, dtype=torch.int32, device='cuda')
    qkv_t = torch.empty((40 + 16) * 128, dtype=torch.float16, device='cuda')
    out_t = torch.empty(40 * 128, dtype=torch.float16, device='cuda')

    def step():
        nat.decode_attention(qkv_t, 40, 8, t['qn'], t['kn'], 1e-6, t['cos'], t['sin'], pos_t, t['kc'], t['vc'],
                             1.0 / np.sqrt(128.0), out=out_t, workspace=ws)

    qkv_t.copy_(torch.from_numpy(case.qkv()))
    pos_t.fill_(999)
    step()                                          # eager warm-up (row 999 is not attended below)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for pos in range(500, 504):
        qkv = case.qkv()
        qkv_t.copy_(torch.from_numpy(qkv))
        pos_t.fill_(pos)
        g.replay()
        torch.cuda.synchronize()
        ref, k_new, v_new = case.expected(qkv, pos)
        assert qdq.parity_ok(qdq.parity_metrics(out_t.cpu().numpy(), ref)), pos
        case.kc[:, pos] = t['kc'][:, pos].cpu().numpy()
        case.vc[:, pos] = v_new
        _ = torch.randn(1000, device='cuda').sum().item()   # eager work between replays


@pytest.mark.parametrize('on_host', [True, False])
def test_embed_rows(nat, on_host):
    """wq_embed_rows gathers the rows of device token ids bit-exactly from a
    table in pinned host memory (the decode graph's embedding) or on the
    device; an out-of-range id gives a NaN row."""
    print(f'[embed_rows] on_host={on_host}', flush=True)
    vocab, hidden = 1000, 5120
    table = (torch.randn(vocab, hidden, generator=torch.Generator().manual_seed(1)) * 0.02).half()
    src = nat.host_table(table, 'cuda:0') if on_host else table.cuda()
    if on_host:
        assert src.tensor.is_pinned() and torch.equal(src.tensor, table)
    ids = torch.tensor([0, 999, 17, 17, 523], dtype=torch.long, device='cuda')
    out = nat.embed_rows(src, ids)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), table[ids.cpu()])
    bad = nat.embed_rows(src, torch.tensor([3, -1, 1000], dtype=torch.long, device='cuda'))
    torch.cuda.synchronize()
    bad = bad.cpu()
    assert torch.equal(bad[0], table[3]) and bool(torch.isnan(bad[1:]).all())
    # The per-16-element sums of squares the first layer's fused RMSNorm takes.
    sq = torch.full((ids.numel() * hidden // 16,), -1.0, device='cuda')
    again = nat.embed_rows(src, ids, sumsq_out=sq)
    torch.cuda.synchronize()
    assert torch.equal(again.cpu(), table[ids.cpu()])
    ref = (table[ids.cpu()].double() ** 2).view(ids.numel(), hidden // 16, 16).sum(-1).view(-1)
    assert torch.allclose(sq.cpu().double(), ref, rtol=1e-6, atol=0)
    sq_bad = torch.zeros(3 * hidden // 16, device='cuda')
    nat.embed_rows(src, torch.tensor([3, -1, 1000], dtype=torch.long, device='cuda'), sumsq_out=sq_bad)
    sq_bad = sq_bad.cpu().view(3, -1)
    assert bool(torch.isfinite(sq_bad[0]).all()) and bool(torch.isnan(sq_bad[1:]).all())
    with pytest.raises(ValueError):
        nat.embed_rows(src, ids, sumsq_out=torch.zeros(7, device='cuda'))
    with pytest.raises(ValueError):
        nat.host_table(table.cuda(), 'cuda:0')


@pytest.mark.parametrize('count', [1, 2, 3, 5, 7, 320, 512])
def test_rmsnorm_prologue_any_sumsq_count(nat, count):
    """The RMSNorm prologue sums however many partial sums of squares the
    producer left (0 < count <= 512), including counts below one float4 and
    counts that are not a multiple of 4; the output is the oracle's norm."""
    from oracle import synth
    k, n = 5120, 1024
    print(f'[rmsnorm_prologue] count={count}', flush=True)
    w, _ = synth.w4_case(n, k, 1, seed=count)
    rng = np.random.default_rng(count)
    key = 'mlp.up_proj'
    tiles, meta = nat.w4_repack(torch.from_numpy(w[f'{key}.weight_packed']).cuda(),
                                torch.from_numpy(w[f'{key}.weight_scale']).cuda(),
                                torch.from_numpy(w[f'{key}.weight_zero_point']).cuda(), n, k, 128)
    xin = (rng.standard_normal(k) * 3).astype(np.float16)
    nw = (1 + 0.1 * rng.standard_normal(k)).astype(np.float16)
    sq = xin.astype(np.float32) ** 2
    parts = np.array([c.sum(dtype=np.float64) for c in np.array_split(sq, count)], dtype=np.float32)
    out = nat.w4a16_decode_fused(torch.from_numpy(xin).cuda(), tiles, meta, n, 128, x_mode=nat.X_RMSNORM,
                                 norm_weight=torch.from_numpy(nw).cuda(), sumsq_in=torch.from_numpy(parts).cuda(),
                                 eps=1e-6)
    torch.cuda.synchronize()
    expect = qdq.qdq_linear(qwen3.rms_norm(xin, nw, 1e-6)[None], w, f'{key}.weight')[0]
    m = qdq.parity_metrics(out.cpu().numpy().astype(np.float32), expect.astype(np.float32))
    assert qdq.parity_ok(m), m


@pytest.mark.parametrize('k,n,mode', [(5120, 7168, 1), (5120, 5120, 0), (17408, 5120, 2), (5120, 34816, 1),
                                      (512, 1024, 2)])
def test_w4a16_decode_fused_matches_oracle(nat, k, n, mode):
    """RMSNorm / SiLU*up prologue, fp16 residual and per-tile sums of squares
    of wq_w4a16_decode_fused against the oracle's ops around qdq_linear."""
    from oracle import synth
    print(f'[decode_fused] k={k} n={n} mode={mode}', flush=True)
    w, _ = synth.w4_case(n, k, 1, seed=k + n + mode)
    rng = np.random.default_rng(mode)
    key = 'mlp.up_proj'
    tiles, meta = nat.w4_repack(torch.from_numpy(w[f'{key}.weight_packed']).cuda(),
                                torch.from_numpy(w[f'{key}.weight_scale']).cuda(),
                                torch.from_numpy(w[f'{key}.weight_zero_point']).cuda(), n, k, 128)
    res = (rng.standard_normal(n) * 4).astype(np.float16)
    if mode == 2:
        xin = (rng.standard_normal(2 * k) * 2).astype(np.float16)
        x_eff = qwen3.swiglu(xin[:k], xin[k:])
        kw = {}
    elif mode == 1:
        xin = (rng.standard_normal(k) * 3).astype(np.float16)
        nw = (1 + 0.1 * rng.standard_normal(k)).astype(np.float16)
        x_eff = qwen3.rms_norm(xin, nw, 1e-6)
        parts = (xin.astype(np.float32) ** 2).reshape(-1, 16).sum(-1).astype(np.float32)
        kw = {'norm_weight': torch.from_numpy(nw).cuda(), 'sumsq_in': torch.from_numpy(parts).cuda()}
    else:
        xin = rng.standard_normal(k).astype(np.float16)
        x_eff = xin
        kw = {}
    y_lin = qdq.qdq_linear(x_eff[None], w, f'{key}.weight')[0]
    expect = (res + y_lin).astype(np.float16)
    hid = torch.from_numpy(res.copy()).cuda()               # residual updated in place
    ss = torch.zeros(n // 16, dtype=torch.float32, device='cuda')
    out = nat.w4a16_decode_fused(torch.from_numpy(xin).cuda(), tiles, meta, n, 128, x_mode=mode, residual=hid,
                                 sumsq_out=ss, out=hid, **kw)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert out.data_ptr() == hid.data_ptr()
    m = qdq.parity_metrics(got.astype(np.float32) - res, expect.astype(np.float32) - res)
    assert qdq.parity_ok(m), m
    g64 = got.astype(np.float64)
    assert np.allclose(ss.cpu().numpy(), (g64 ** 2).reshape(-1, 16).sum(-1), rtol=1e-5, atol=1e-3)


@pytest.mark.parametrize('k,n,mode', [(5120, 7168, 1), (5120, 5120, 0), (17408, 5120, 2), (5120, 34816, 1),
                                      (512, 1024, 2), (256, 512, 0)])
def test_w8a16_decode_fused_matches_oracle(nat, k, n, mode):
    """wq_w8a16_decode_fused (INT8 weight, fp16 row scale) in every mode
    against the oracle: fp16(q * s) weights (the reference's
    int8_weight_only_linear), its RMSNorm / SiLU*up, the fp16 residual add and
    the per-tile sums of squares."""
    from oracle import synth
    print(f'[w8 decode_fused] k={k} n={n} mode={mode}', flush=True)
    _, q, s, _ = synth.int8_case(n, k, 1, seed=k + n + mode)
    rng = np.random.default_rng(mode + 10)
    res = (rng.standard_normal(n) * 4).astype(np.float16)
    if mode == 2:
        xin = (rng.standard_normal(2 * k) * 2).astype(np.float16)
        x_eff = qwen3.swiglu(xin[:k], xin[k:])
        kw = {}
    elif mode == 1:
        xin = (rng.standard_normal(k) * 3).astype(np.float16)
        nw = (1 + 0.1 * rng.standard_normal(k)).astype(np.float16)
        x_eff = qwen3.rms_norm(xin, nw, 1e-6)
        parts = (xin.astype(np.float32) ** 2).reshape(-1, 16).sum(-1).astype(np.float32)
        kw = {'norm_weight': torch.from_numpy(nw).cuda(), 'sumsq_in': torch.from_numpy(parts).cuda()}
    else:
        xin = rng.standard_normal(k).astype(np.float16)
        x_eff = xin
        kw = {}
    y_lin = qdq.linear_fp32(x_eff[None], qdq.dequantize_linear_weight(q, s))[0]
    expect = (res + y_lin).astype(np.float16)
    hid = torch.from_numpy(res.copy()).cuda()
    ss = torch.zeros(n // 16, dtype=torch.float32, device='cuda')
    out = nat.w8a16_decode_fused(torch.from_numpy(xin).cuda(), torch.from_numpy(q).cuda(),
                                 torch.from_numpy(s).cuda(), x_mode=mode, residual=hid, sumsq_out=ss, out=hid, **kw)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert out.data_ptr() == hid.data_ptr()
    m = qdq.parity_metrics(got.astype(np.float32) - res, expect.astype(np.float32) - res)
    assert qdq.parity_ok(m), m
    g64 = got.astype(np.float64)
    assert np.allclose(ss.cpu().numpy(), (g64 ** 2).reshape(-1, 16).sum(-1), rtol=1e-5, atol=1e-3)
    # Without the fusions the entry point is the plain INT8 linear, bit for bit.
    if mode == 0:
        xt = torch.from_numpy(xin).cuda()
        plain = nat.w8a16_decode_fused(xt, torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda())
        ref = nat.w8a16_linear(xt[None], torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda())
        assert torch.equal(plain.view(-1), ref.view(-1))


# ------------------------------------------------------------------ LM head + greedy token

def _lm_case(vocab, k, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(k) * 0.5).astype(np.float16)
    w = (rng.standard_normal((vocab, k)) * 0.05).astype(np.float16)
    return x, w


@pytest.mark.parametrize('vocab,k', [(1, 512), (3, 1024), (1000, 512), (4097, 4096), (20000, 8192),
                                     (151936, 5120)])
def test_lm_head_logits_and_token(nat, vocab, k):
    """fp16 logits against the fp32-accumulated oracle; the token is exactly
    torch.argmax of the returned logits (first index of the largest)."""
    print(f'[lm_head] vocab={vocab} k={k}', flush=True)
    x, w = _lm_case(vocab, k, seed=vocab + k)
    tx, tw = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    logits, token = nat.lm_head(tx, tw)
    torch.cuda.synchronize()
    ref = qdq.linear_fp32(x[None], w)[0]
    m = qdq.parity_metrics(logits.cpu().numpy(), ref)
    assert qdq.parity_ok(m), m
    assert token.item() == int(torch.argmax(logits).item())
    # Where the oracle's top two are apart by more than the fp16 step, the
    # token is the oracle's too.
    if vocab > 1:
        top2 = np.sort(ref.astype(np.float32))[-2:]
        if top2[1] - top2[0] > 4e-3 * max(abs(top2[1]), 1.0):
            assert token.item() == int(np.argmax(ref))


@pytest.mark.parametrize('vocab,k', [(1000, 512), (151936, 5120)])
def test_lm_head_with_final_rmsnorm(nat, vocab, k):
    """wq_lm_head_rmsnorm: the final RMSNorm formed inside the LM head from
    the residual stream and its per-16-element sums of squares, against the
    oracle's rms_norm followed by the fp32-accumulated LM head; the token is
    argmax of the returned logits."""
    from oracle import qwen3
    print(f'[lm_head_rmsnorm] vocab={vocab} k={k}', flush=True)
    rng = np.random.default_rng(vocab + k + 1)
    x = (rng.standard_normal(k) * 3.0).astype(np.float16)
    nw = (1 + 0.1 * rng.standard_normal(k)).astype(np.float16)
    w = (rng.standard_normal((vocab, k)) * 0.05).astype(np.float16)
    sq = (x.astype(np.float32) ** 2).reshape(-1, 16).sum(-1).astype(np.float32)
    eps = 1e-6
    tw = torch.from_numpy(w).cuda()
    logits, token = nat.lm_head(torch.from_numpy(x).cuda(), tw, norm_weight=torch.from_numpy(nw).cuda(),
                                sumsq_in=torch.from_numpy(sq).cuda(), eps=eps)
    torch.cuda.synchronize()
    ref = qdq.linear_fp32(qwen3.rms_norm(x[None], nw, eps), w)[0]
    m = qdq.parity_metrics(logits.cpu().numpy(), ref)
    assert qdq.parity_ok(m), m
    assert token.item() == int(torch.argmax(logits).item())
    with pytest.raises(ValueError):
        nat.lm_head(torch.from_numpy(x).cuda(), tw, norm_weight=torch.from_numpy(nw).cuda())


def test_lm_head_ties_nan_and_infinities(nat):
    k, vocab = 512, 3000
    x = np.ones(k, dtype=np.float16)
    w = np.zeros((vocab, k), dtype=np.float16)
    w[17, :] = 0.01
    w[2500, :] = 0.01           # same logit as row 17: the first index wins
    tx = torch.from_numpy(x).cuda()
    _, token = nat.lm_head(tx, torch.from_numpy(w).cuda())
    assert token.item() == 17
    w[1200, 0] = np.nan         # a NaN logit counts as the largest (torch.argmax)
    w[2900, 0] = np.nan
    logits, token = nat.lm_head(tx, torch.from_numpy(w).cuda())
    assert token.item() == 1200 == int(torch.argmax(logits).item())
    w = np.full((vocab, k), -60000, dtype=np.float16)   # every logit overflows to -inf
    logits, token = nat.lm_head(tx, torch.from_numpy(w).cuda())
    assert torch.isneginf(logits).all() and token.item() == 0


def test_lm_head_only_logits_or_only_token(nat):
    x, w = _lm_case(5000, 1024, seed=5)
    tx, tw = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    both_l, both_t = nat.lm_head(tx, tw)
    only_l, none_t = nat.lm_head(tx, tw, want_token=False)
    none_l, only_t = nat.lm_head(tx, tw, want_logits=False)
    torch.cuda.synchronize()
    assert none_t is None and none_l is None
    assert torch.equal(both_l, only_l) and torch.equal(both_t, only_t)
    with pytest.raises(ValueError, match='k % 512'):
        nat.lm_head(torch.zeros(640, dtype=torch.float16, device='cuda'),
                    torch.zeros(8, 640, dtype=torch.float16, device='cuda'))
    with pytest.raises(ValueError, match='workspace'):
        nat.lm_head(tx, tw, workspace=torch.zeros(8, dtype=torch.uint8, device='cuda'))


@pytest.mark.parametrize('n', [1, 7, 8, 9, 1000, 2048, 4097, 151936, (1 << 20) + 3])
def test_argmax_f16_matches_torch(nat, n):
    """wq_argmax_f16 against torch.argmax on the CPU: random values, a planted
    tie for the maximum (first index wins), a NaN (wins, first NaN), and all
    -inf."""
    print(f'[argmax] n={n}', flush=True)
    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, generator=g).half()
    cases = [x.clone()]
    if n > 3:
        t = x.clone()
        t[n // 3] = t[n - 1] = 60000.0
        cases.append(t)
        t = x.clone()
        t[n // 2] = float('nan')
        t[n - 1] = float('nan')
        t[0] = float('inf')
        cases.append(t)
    cases.append(torch.full((n,), float('-inf')).half())
    for c in cases:
        got = nat.argmax_f16(c.cuda())
        torch.cuda.synchronize()
        assert got.item() == int(torch.argmax(c.float()).item()), (n, got.item())
