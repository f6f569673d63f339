"""GPU checks of split-KV over packed sequences (fav4_bshd_forward_splitkv_varlen) via the C ABI.

The decode case of continuous batching: every sequence brings 1-32 new
queries and its own cache length.  Pins:
  * every sequence against the FP64 oracle at the reference harness's bar,
    for ragged batches (0-32 queries, 0 to ~20000 keys), MHA / GQA / MQA head
    groups, LSE on and off, Auto and explicit chunk counts;
  * a batch of equal lengths is bitwise the contiguous split-KV (GQA entry
    point) on the same data at the same chunk count (same plan, chunk bounds
    and merge), so any difference is an indexing error;
  * a sequence without queries writes nothing, one without keys gets O = 0
    and LSE = -inf, and rows after O / LSE are never written;
  * causal and max_seqlen_q > 32 run the unsplit packed forward, bitwise.
"""
import numpy as np
import pytest

from oracle import attention as orc
from tests.conftest import to_device, to_host_bits

pytestmark = pytest.mark.gpu

GUARD = 64

# (heads, kv_heads, [(sq, sk), ...], chunk counts)
CASES = [
    (32, 8, [(1, 4096), (1, 100), (1, 1), (1, 9000), (1, 33), (1, 2048)], (0, 7)),
    (8, 1, [(16, 3000), (5, 1), (32, 700), (1, 5000)], (0, 3)),
    (4, 4, [(3, 300), (32, 4096), (0, 50), (7, 0), (1, 20000)], (0, 16)),
    (6, 2, [(32, 32), (31, 64), (17, 1025)], (0, 2, 256)),
]


def _pack(heads, kv_heads, lens, seed=0):
    qs, ks, vs = [], [], []
    for i, (sq, sk) in enumerate(lens):
        q, _, _ = orc.make_inputs(1, heads, max(sq, 1), max(sk, 1), "normal", seed=seed + 2 * i)
        _, k, v = orc.make_inputs(1, kv_heads, max(sq, 1), max(sk, 1), "normal", seed=seed + 2 * i + 1)
        qs.append(q[0, :sq])
        ks.append(k[0, :sk])
        vs.append(v[0, :sk])
    cu_q = np.concatenate([[0], np.cumsum([s for s, _ in lens])]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum([s for _, s in lens])]).astype(np.int32)
    return np.concatenate(qs), np.concatenate(ks), np.concatenate(vs), cu_q, cu_k


def _run(runner, qd, kd, vd, cu_q, cu_k, max_q, max_k, causal, with_lse, splits, plain=False):
    """Split-KV (or, plain=True, the unsplit packed forward) into NaN-filled O /
    LSE followed by NaN guard rows; returns (o, lse, o_guard, lse_guard)."""
    import torch
    dev = qd.device
    tq, h, d = qd.shape
    o_buf = torch.full((tq + GUARD, h, d), float("nan"), device=dev, dtype=torch.bfloat16)
    l_buf = torch.full((h * tq + GUARD,), float("nan"), device=dev, dtype=torch.float32)
    o = o_buf[:tq]
    lse = l_buf[:h * tq].view(h, tq) if with_lse else None
    cq, ck = torch.from_numpy(cu_q).to(dev), torch.from_numpy(cu_k).to(dev)
    if plain:
        runner.call_varlen(qd, kd, vd, o, lse, cq, ck, max_q, max_k, causal)
    else:
        runner.call_splitkv_varlen(qd, kd, vd, o, lse, cq, ck, max_q, max_k, causal, splits)
    torch.cuda.synchronize()
    return o, (l_buf[:h * tq].view(h, tq) if with_lse else None), o_buf[tq:], l_buf[h * tq:]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "h%dkv%d_n%d" % (c[0], c[1], len(c[2])))
def test_splitkv_varlen_matches_oracle(gpu_runner, case):
    import torch
    h, kvh, lens, split_list = case
    q, k, v, cu_q, cu_k = _pack(h, kvh, lens, seed=3)
    dev = torch.device("cuda:0")
    qd, kd, vd = to_device(q, dev), to_device(k, dev), to_device(v, dev)
    max_q = max(s for s, _ in lens)
    max_k = max(s for _, s in lens)
    group = h // kvh
    refs = {}
    for splits in split_list:
        n = gpu_runner.splitkv_varlen_select(len(lens), h, kvh, max_q, max_k, len(q), len(k), False) \
            if splits == 0 else splits
        print(f"  splitkv varlen H{h} KVH{kvh} lens={lens} splits={splits} (Auto {n})", flush=True)
        o, lse, og, lg = _run(gpu_runner, qd, kd, vd, cu_q, cu_k, max_q, max_k, False, True, splits)
        o2, _, og2, lg2 = _run(gpu_runner, qd, kd, vd, cu_q, cu_k, max_q, max_k, False, False, splits)
        assert torch.isnan(og).all().item() and torch.isnan(lg).all().item()
        assert torch.isnan(og2).all().item() and torch.isnan(lg2).all().item()
        for i, (sq, sk) in enumerate(lens):
            a, b = cu_q[i], cu_q[i + 1]
            c, d = cu_k[i], cu_k[i + 1]
            if sq == 0:
                continue
            if sk == 0:
                assert (o[a:b].float() == 0).all().item() and (o2[a:b].float() == 0).all().item(), i
                assert torch.isneginf(lse[:, a:b]).all().item(), i
                continue
            if i not in refs:
                ke = np.repeat(k[c:d][None], group, axis=2)
                ve = np.repeat(v[c:d][None], group, axis=2)
                refs[i] = orc.attention_fp64(q[a:b][None], ke, ve, orc.DEFAULT_SCALE, False)
            ref, ref_lse = refs[i]
            e = orc.errors(to_host_bits(o[a:b])[None], lse[:, a:b].cpu().numpy()[None], ref, ref_lse)
            assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), (splits, i, sq, sk, e)
            e2 = orc.errors(to_host_bits(o2[a:b])[None], None, ref, None)
            assert orc.check_acceptance_tolerance(e2) and orc.check_reference_tolerance(e2), (splits, i, e2)


@pytest.mark.parametrize("shape", [(3, 16, 4, 4, 3000, 5), (2, 8, 8, 1, 8192, 0), (4, 8, 1, 32, 2500, 11)],
                         ids=lambda s: "b%dh%dkv%d_%dx%d_s%d" % s)
def test_splitkv_varlen_uniform_is_contiguous_splitkv(gpu_runner, shape):
    """Equal lengths: bitwise the contiguous split-KV at the same chunk count."""
    import torch
    b, h, kvh, sq, sk, splits = shape
    q, k, v, cu_q, cu_k = _pack(h, kvh, [(sq, sk)] * b, seed=9)
    dev = torch.device("cuda:0")
    qd, kd, vd = to_device(q, dev), to_device(k, dev), to_device(v, dev)
    n = splits or gpu_runner.splitkv_varlen_select(b, h, kvh, sq, sk, b * sq, b * sk, False)
    assert n == (splits or gpu_runner.splitkv_select(b, h, sq, sk, False, kv_heads=kvh)) and n > 1
    print(f"  splitkv varlen uniform {shape} chunks {n}", flush=True)
    o, lse, _, _ = _run(gpu_runner, qd, kd, vd, cu_q, cu_k, sq, sk, False, True, n)
    q4, k4, v4 = qd.view(b, sq, h, 128), kd.view(b, sk, kvh, 128), vd.view(b, sk, kvh, 128)
    oc = torch.full_like(q4, float("nan"))
    lc = torch.full((b, h, sq), float("nan"), device=dev, dtype=torch.float32)
    gpu_runner.call_splitkv(q4, k4, v4, oc, lc, False, n)
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int16), oc.view(-1, h, 128).view(torch.int16))
    assert torch.equal(lse.view(torch.int32), lc.permute(1, 0, 2).reshape(h, b * sq).view(torch.int32))


def test_splitkv_varlen_unsplit_paths(gpu_runner):
    """Causal (top-left: a decode row sees at most 32 keys) and max_seqlen_q >
    32 take one chunk: bitwise the packed forward, explicit counts included."""
    import torch
    h, kvh = 8, 2
    dev = torch.device("cuda:0")
    for lens, causal in (([(1, 3000), (32, 900), (4, 0)], True), ([(33, 2000), (1, 5000)], False),
                         ([(40, 100), (2, 700)], True)):
        q, k, v, cu_q, cu_k = _pack(h, kvh, lens, seed=21)
        qd, kd, vd = to_device(q, dev), to_device(k, dev), to_device(v, dev)
        max_q = max(s for s, _ in lens)
        max_k = max(s for _, s in lens)
        assert gpu_runner.splitkv_varlen_select(len(lens), h, kvh, max_q, max_k, len(q), len(k), causal) == 1
        assert gpu_runner.splitkv_varlen_workspace_size(len(lens), h, kvh, max_q, max_k, len(q), len(k), causal,
                                                        8) == 0
        print(f"  splitkv varlen unsplit lens={lens} causal={causal}", flush=True)
        ref = _run(gpu_runner, qd, kd, vd, cu_q, cu_k, max_q, max_k, causal, True, 0, plain=True)
        for splits in (0, 8):
            got = _run(gpu_runner, qd, kd, vd, cu_q, cu_k, max_q, max_k, causal, True, splits)
            assert torch.equal(got[0].view(torch.int16), ref[0].view(torch.int16)), (lens, splits)
            assert torch.equal(got[1].view(torch.int32), ref[1].view(torch.int32)), (lens, splits)
            assert torch.isnan(got[2]).all().item() and torch.isnan(got[3]).all().item()


def test_splitkv_varlen_graph_replay(gpu_runner):
    """Captured in a HIP graph with its workspace: every replay equals the
    eager result, with new K/V contents and eager work between replays."""
    import torch
    h, kvh = 16, 4
    lens = [(1, 6000), (2, 300), (1, 2048), (3, 4100)]
    q, k, v, cu_q, cu_k = _pack(h, kvh, lens, seed=31)
    dev = torch.device("cuda:0")
    qd, kd, vd = to_device(q, dev), to_device(k, dev), to_device(v, dev)
    cq, ck = torch.from_numpy(cu_q).to(dev), torch.from_numpy(cu_k).to(dev)
    max_q, max_k = 3, 6000
    n = gpu_runner.splitkv_varlen_select(len(lens), h, kvh, max_q, max_k, len(q), len(k), False)
    assert n > 1
    ws = torch.empty(gpu_runner.splitkv_varlen_workspace_size(len(lens), h, kvh, max_q, max_k, len(q), len(k),
                                                              False), device=dev, dtype=torch.uint8)
    o = torch.full_like(qd, float("nan"))
    lse = torch.full((h, len(q)), float("nan"), device=dev, dtype=torch.float32)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    print(f"  splitkv varlen graph chunks {n}", flush=True)
    with torch.cuda.stream(s):
        gpu_runner.call_splitkv_varlen(qd, kd, vd, o, lse, cq, ck, max_q, max_k, False, 0, workspace=ws,
                                       stream=s.cuda_stream)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            gpu_runner.call_splitkv_varlen(qd, kd, vd, o, lse, cq, ck, max_q, max_k, False, 0, workspace=ws,
                                           stream=s.cuda_stream)
    torch.cuda.synchronize()
    for rep in range(3):
        kd.copy_(to_device(np.roll(k, rep + 1, axis=0), dev))
        oe, le, _, _ = _run(gpu_runner, qd, kd, vd, cu_q, cu_k, max_q, max_k, False, True, 0)
        o.fill_(float("nan"))
        lse.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o.view(torch.int16), oe.view(torch.int16)), rep
        assert torch.equal(lse.view(torch.int32), le.view(torch.int32)), rep
