"""GPU checks of packed variable-length sequences (fav4_bshd_forward_varlen) via the C ABI.

Sequence b's query rows are [cu_q[b], cu_q[b+1]) of the packed Q/O and its
key rows [cu_k[b], cu_k[b+1]) of the packed K/V.  Pins:
  * bitwise equality, sequence by sequence, with fav4_bshd_forward (MHA) or
    fav4_bshd_forward_gqa (GQA) at config 2 on that sequence alone: the varlen
    kernel runs the same per-wave tile loop (BN 64, 2 LDS stages; 128-row
    workgroups for max_seqlen_q <= 1024 or small grids, else 256-row ones,
    both bitwise equal to config 2), so any difference is an indexing error
    (wrong sequence, head or row);
  * the FP64 oracle on every sequence, at the reference harness's bar;
  * a sequence without keys gives O = 0 and LSE = -inf, one without queries
    writes nothing, and rows outside O / LSE are never written;
  * bottom-right causal (causal = 2) against the FP64 bottom-right reference,
    and bitwise the top-left call on sequences with as many queries as keys.
"""
import numpy as np
import pytest

from oracle import attention as orc
from tests.conftest import to_device, to_host_bits

pytestmark = pytest.mark.gpu

GUARD = 64   # extra rows after O and entries after LSE that must stay untouched

# (heads, kv_heads, [(sq, sk), ...])
CASES = [
    (4, 4, [(1, 1), (255, 300), (256, 256), (257, 2049), (1000, 64)]),
    (8, 2, [(513, 513), (7, 1000), (300, 77)]),
    (6, 1, [(129, 1500), (700, 100), (64, 65)]),
    (2, 2, [(1, 4096)]),
]


def _pack(heads, kv_heads, lens, seed=0):
    qs, ks, vs = [], [], []
    for i, (sq, sk) in enumerate(lens):
        q, _, _ = orc.make_inputs(1, heads, sq, max(sk, 1), "normal", seed=seed + 2 * i)
        _, k, v = orc.make_inputs(1, kv_heads, max(sq, 1), sk, "normal", seed=seed + 2 * i + 1)
        qs.append(q[0])
        ks.append(k[0])
        vs.append(v[0])
    cu_q = np.concatenate([[0], np.cumsum([s for s, _ in lens])]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum([s for _, s in lens])]).astype(np.int32)
    return np.concatenate(qs), np.concatenate(ks), np.concatenate(vs), cu_q, cu_k


def _run_varlen(runner, qd, kd, vd, cu_q, cu_k, max_q, max_k, causal, with_lse):
    """Run into O / LSE views that are followed by NaN guard rows; return (o, lse, o_guard, lse_guard)."""
    import torch
    dev = qd.device
    tq, h, d = qd.shape
    o_buf = torch.full((tq + GUARD, h, d), float("nan"), device=dev, dtype=torch.bfloat16)
    l_buf = torch.full((h * tq + GUARD,), float("nan"), device=dev, dtype=torch.float32)
    o = o_buf[:tq]
    lse = l_buf[:h * tq].view(h, tq) if with_lse else None
    runner.call_varlen(qd, kd, vd, o, lse, torch.from_numpy(cu_q).to(dev), torch.from_numpy(cu_k).to(dev),
                       max_q, max_k, causal)
    torch.cuda.synchronize()
    return o, (l_buf[:h * tq].view(h, tq) if with_lse else None), o_buf[tq:], l_buf[h * tq:]


def _alone(runner, q, k, v, h, kvh, causal):
    """fav4_bshd_forward(_gqa) config 2 on one sequence: (O [sq,h,d], LSE [h,sq])."""
    import torch
    dev = torch.device("cuda:0")
    qd, kd, vd = (to_device(x[None], dev) for x in (q, k, v))
    o = torch.full_like(qd, float("nan"))
    lse = torch.full((1, h, q.shape[0]), float("nan"), device=dev, dtype=torch.float32)
    if kvh == h:
        runner.call(qd, kd, vd, o, lse, causal, 2)
    else:
        runner.call_gqa(qd, kd, vd, o, lse, causal, 2)
    torch.cuda.synchronize()
    return o[0], lse[0]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "h%dkv%d_n%d" % (c[0], c[1], len(c[2])))
@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_varlen_matches_per_sequence_forward(gpu_runner, case, causal):
    import torch
    h, kvh, lens = case
    q, k, v, cu_q, cu_k = _pack(h, kvh, lens)
    dev = torch.device("cuda:0")
    qd, kd, vd = to_device(q, dev), to_device(k, dev), to_device(v, dev)
    max_q = max(s for s, _ in lens)
    max_k = max(s for _, s in lens)
    print(f"  varlen H{h} KVH{kvh} lens={lens} causal={causal}", flush=True)
    o, lse, og, lg = _run_varlen(gpu_runner, qd, kd, vd, cu_q, cu_k, max_q, max_k, causal, True)
    o2, _, og2, lg2 = _run_varlen(gpu_runner, qd, kd, vd, cu_q, cu_k, max_q, max_k, causal, False)
    assert torch.isnan(og).all().item() and torch.isnan(lg).all().item()
    assert torch.isnan(og2).all().item() and torch.isnan(lg2).all().item()
    assert torch.equal(o.view(torch.int16), o2.view(torch.int16))      # LSE on/off: same O
    group = h // kvh
    for i, (sq, sk) in enumerate(lens):
        a, b = cu_q[i], cu_q[i + 1]
        c, d = cu_k[i], cu_k[i + 1]
        o_ref, l_ref = _alone(gpu_runner, q[a:b], k[c:d], v[c:d], h, kvh, causal)
        assert torch.equal(o[a:b].view(torch.int16), o_ref.view(torch.int16)), (i, sq, sk)
        assert torch.equal(lse[:, a:b].view(torch.int32), l_ref.view(torch.int32)), (i, sq, sk)
        ke = np.repeat(k[c:d][None], group, axis=2)
        ve = np.repeat(v[c:d][None], group, axis=2)
        ref, ref_lse = orc.attention_fp64(q[a:b][None], ke, ve, orc.DEFAULT_SCALE, causal)
        e = orc.errors(to_host_bits(o[a:b])[None], lse[:, a:b].cpu().numpy()[None], ref, ref_lse)
        assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), (i, sq, sk, e)


@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_varlen_empty_sequences(gpu_runner, causal):
    """No queries: nothing written for it.  No keys: O = 0, LSE = -inf.  The
    others are unaffected by their empty neighbours."""
    import torch
    h = kvh = 4
    lens = [(0, 5), (100, 0), (64, 64), (0, 0), (300, 257), (1, 0)]
    q, k, v, cu_q, cu_k = _pack(h, kvh, lens, seed=11)
    dev = torch.device("cuda:0")
    qd, kd, vd = to_device(q, dev), to_device(k, dev), to_device(v, dev)
    o, lse, og, lg = _run_varlen(gpu_runner, qd, kd, vd, cu_q, cu_k, 300, 257, causal, True)
    assert torch.isnan(og).all().item() and torch.isnan(lg).all().item()
    assert not torch.isnan(o.float()).any().item() and not torch.isnan(lse).any().item()
    for i, (sq, sk) in enumerate(lens):
        a, b = cu_q[i], cu_q[i + 1]
        c, d = cu_k[i], cu_k[i + 1]
        if sq == 0:
            continue
        if sk == 0:
            assert (o[a:b].float() == 0).all().item(), i
            assert torch.isneginf(lse[:, a:b]).all().item(), i
            continue
        o_ref, l_ref = _alone(gpu_runner, q[a:b], k[c:d], v[c:d], h, kvh, causal)
        assert torch.equal(o[a:b].view(torch.int16), o_ref.view(torch.int16)), i
        assert torch.equal(lse[:, a:b].view(torch.int32), l_ref.view(torch.int32)), i


def test_varlen_loose_max_seqlen_and_long_sequences(gpu_runner):
    """A max_seqlen larger than any sequence changes nothing; sequences of
    several thousand rows (several q tiles) match the per-sequence forward."""
    import torch
    h, kvh = 8, 4
    lens = [(4096, 4096), (3000, 5000), (17, 8192), (2500, 1200)]
    q, k, v, cu_q, cu_k = _pack(h, kvh, lens, seed=5)
    dev = torch.device("cuda:0")
    qd, kd, vd = to_device(q, dev), to_device(k, dev), to_device(v, dev)
    for causal in (False, True):
        print(f"  varlen long causal={causal}", flush=True)
        o, lse, og, lg = _run_varlen(gpu_runner, qd, kd, vd, cu_q, cu_k, 4096, 8192, causal, True)
        o_l, lse_l, _, _ = _run_varlen(gpu_runner, qd, kd, vd, cu_q, cu_k, 9000, 20000, causal, True)
        assert torch.equal(o.view(torch.int16), o_l.view(torch.int16))
        assert torch.equal(lse.view(torch.int32), lse_l.view(torch.int32))
        assert torch.isnan(og).all().item() and torch.isnan(lg).all().item()
        for i in range(len(lens)):
            a, b = cu_q[i], cu_q[i + 1]
            c, d = cu_k[i], cu_k[i + 1]
            o_ref, l_ref = _alone(gpu_runner, q[a:b], k[c:d], v[c:d], h, kvh, causal)
            assert torch.equal(o[a:b].view(torch.int16), o_ref.view(torch.int16)), (i, causal)
            assert torch.equal(lse[:, a:b].view(torch.int32), l_ref.view(torch.int32)), (i, causal)


# (heads, kv_heads, [(sq, sk), ...]) for bottom-right causal: sq < sk (a
# prefill chunk against a cache), sq = sk, sq > sk (the first sq - sk rows see
# no key), sequences without keys or queries, several q tiles.  The first batch
# runs 128-row workgroups (max_seqlen_q <= 1024), the second 256-row ones
# (6 x 8 x 6 (sequence, head, q tile) items, more than the 256 CUs).
BR_CASES = [
    (8, 2, [(300, 3000), (129, 129), (700, 100), (64, 1), (0, 40), (5, 0), (1, 2049), (513, 1000)]),
    (8, 8, [(1500, 4000), (1100, 1100), (1300, 600), (2, 9), (1024, 1500), (257, 300)]),
]


@pytest.mark.parametrize("case", BR_CASES, ids=["bm128", "bm256"])
def test_varlen_bottom_right_causal(gpu_runner, case):
    """causal = 2: every sequence against the FP64 bottom-right reference (rows
    that see no key: O = 0, LSE = -inf exactly), nothing written past O / LSE,
    O without LSE bitwise O with it, the one-chunk split-KV packed call
    bitwise this one, and sequences with sq = sk bitwise the top-left
    (causal = 1) call."""
    import torch
    from tests.test_gpu_splitkv_paged import _check_bottom_right
    h, kvh, lens = case
    q, k, v, cu_q, cu_k = _pack(h, kvh, lens, seed=71)
    dev = torch.device("cuda:0")
    qd, kd, vd = to_device(q, dev), to_device(k, dev), to_device(v, dev)
    max_q, max_k = max(s for s, _ in lens), max(s for _, s in lens)
    print(f"  varlen bottom-right h{h} kv{kvh} max_q {max_q} max_k {max_k}", flush=True)
    o, lse, og, lg = _run_varlen(gpu_runner, qd, kd, vd, cu_q, cu_k, max_q, max_k, 2, True)
    assert torch.isnan(og).all().item() and torch.isnan(lg).all().item()
    assert not torch.isnan(o.float()).any().item() and not torch.isnan(lse).any().item()
    _check_bottom_right(o, lse, q, k, v, cu_q, cu_k, lens, h // kvh, "unsplit")
    o_nl, _, og_nl, _ = _run_varlen(gpu_runner, qd, kd, vd, cu_q, cu_k, max_q, max_k, 2, False)
    assert torch.equal(o.view(torch.int16), o_nl.view(torch.int16))
    assert torch.isnan(og_nl).all().item()
    # the split-KV packed call with one chunk takes this kernel (no workspace)
    assert gpu_runner.splitkv_varlen_workspace_size(len(lens), h, kvh, max_q, max_k, len(q), len(k), 2, 1) == 0
    o_s = torch.full_like(o, float("nan"))
    lse_s = torch.full_like(lse, float("nan"))
    gpu_runner.call_splitkv_varlen(qd, kd, vd, o_s, lse_s, torch.from_numpy(cu_q).to(dev),
                                   torch.from_numpy(cu_k).to(dev), max_q, max_k, 2, 1)
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int16), o_s.view(torch.int16))
    assert torch.equal(lse.view(torch.int32), lse_s.view(torch.int32))
    o_tl, lse_tl, _, _ = _run_varlen(gpu_runner, qd, kd, vd, cu_q, cu_k, max_q, max_k, 1, True)
    for i, (sq, sk) in enumerate(lens):
        a, b = cu_q[i], cu_q[i + 1]
        if sq == sk and sq > 0:
            assert torch.equal(o[a:b].view(torch.int16), o_tl[a:b].view(torch.int16)), i
            assert torch.equal(lse[:, a:b].view(torch.int32), lse_tl[:, a:b].view(torch.int32)), i
