"""GPU parity of the split-KV forward (fav4_bshd_forward_splitkv) through the C ABI.

Split-KV cuts each (b, h, 256-row q tile)'s key range into chunks attended in
parallel and merged by log-sum-exp.  It must meet the same bars against the
FP64 oracle as the single-pass kernel (the reference harness's bar and the
port bar), on ragged shapes, with and without LSE, dense and top-left causal
(where some chunks hold no visible key for early rows), for explicit and Auto
chunk counts, whatever the workspace held before the call.
"""
import numpy as np
import pytest

from oracle import attention as orc
from tests.conftest import to_device, to_host_bits

pytestmark = pytest.mark.gpu

SHAPES = [(1, 2, 300, 5000), (2, 3, 257, 1000), (1, 1, 1, 4097), (1, 4, 64, 64), (2, 2, 513, 2049)]


def _run(gpu_runner, torch, q, k, v, causal, splits, with_lse, ws_fill=None):
    dev = torch.device("cuda:0")
    qd, kd, vd = to_device(q, dev), to_device(k, dev), to_device(v, dev)
    b, sq, h, _ = q.shape
    o = torch.full_like(qd, float("nan"))
    lse = torch.full((b, h, sq), float("nan"), device=dev, dtype=torch.float32) if with_lse else None
    kvh = k.shape[2]
    need = gpu_runner.splitkv_workspace_size(b, h, sq, k.shape[1], causal, splits,
                                             kv_heads=None if kvh == h else kvh)
    assert need >= 0
    ws = torch.empty(max(need, 1), device=dev, dtype=torch.uint8)
    if ws_fill is not None and need >= 4:
        ws[: need - need % 4].view(torch.float32).fill_(ws_fill)
    print(f"  splitkv B{b} H{h} {sq}x{k.shape[1]} causal={causal} splits={splits} lse={with_lse} ws={need}",
          flush=True)
    gpu_runner.call_splitkv(qd, kd, vd, o, lse, causal, splits, workspace=ws)
    torch.cuda.synchronize()
    assert not torch.isnan(o).any().item(), "unwritten output elements"
    return to_host_bits(o), (lse.cpu().numpy() if with_lse else None)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "b%dh%d_%dx%d" % s)
@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_splitkv_parity(gpu_runner, shape, causal):
    import torch
    b, h, sq, sk = shape
    q, k, v = orc.make_inputs(b, h, sq, sk, "normal")
    ref, ref_lse = orc.attention_fp64(q, k, v, orc.DEFAULT_SCALE, causal)
    for splits in (2, 3, 5, 0):
        for with_lse in (False, True):
            o, lse = _run(gpu_runner, torch, q, k, v, causal, splits, with_lse)
            e = orc.errors(o, lse, ref, ref_lse if with_lse else None)
            assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), (splits, with_lse, e)


@pytest.mark.parametrize("pattern", ["large", "late_max", "stress", "zero"])
def test_splitkv_patterns(gpu_runner, pattern):
    """The reference's value patterns: large logits move the base inside some
    chunks only, late_max puts the row max in the last chunk."""
    import torch
    q, k, v = orc.make_inputs(1, 8, 256, 3000, pattern)
    for causal in (False, True):
        ref, ref_lse = orc.attention_fp64(q, k, v, orc.DEFAULT_SCALE, causal)
        o, lse = _run(gpu_runner, torch, q, k, v, causal, 6, True)
        e = orc.errors(o, lse, ref, ref_lse)
        assert orc.check_acceptance_tolerance(e), (pattern, causal, e)


def test_splitkv_workspace_contents_do_not_matter(gpu_runner):
    import torch
    q, k, v = orc.make_inputs(1, 2, 300, 2000, "normal")
    outs = [_run(gpu_runner, torch, q, k, v, True, 4, True, ws_fill=fill) for fill in (float("nan"), 0.0, 1e30)]
    for o, lse in outs[1:]:
        assert np.array_equal(o, outs[0][0]) and np.array_equal(lse.view(np.int32), outs[0][1].view(np.int32))


def test_splitkv_single_chunk_is_the_plain_forward(gpu_runner):
    """splits resolving to 1 needs no workspace and runs fav4_bshd_forward: bitwise equal."""
    import torch
    q, k, v = orc.make_inputs(2, 4, 300, 300, "normal")
    assert gpu_runner.splitkv_workspace_size(2, 4, 300, 300, 0, 1) == 0
    dev = torch.device("cuda:0")
    qd, kd, vd = to_device(q, dev), to_device(k, dev), to_device(v, dev)
    for causal in (False, True):
        o1 = torch.empty_like(qd)
        o2 = torch.empty_like(qd)
        gpu_runner.call(qd, kd, vd, o1, None, causal, 0)
        gpu_runner.call_splitkv(qd, kd, vd, o2, None, causal, 1)
        torch.cuda.synchronize()
        assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))


@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_splitkv_long_keys_sampled_rows(gpu_runner, causal):
    """The shape split-KV is for: B1 H8 Sq1024 Sk32768 (32 q tiles; Auto -> 8 chunks
    dense; causal rows see only the first 1024 keys, where Auto keeps the
    unsplit forward, so causal runs 4 explicit chunks), checked on the
    reference's sampled rows for every head."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(11939)
    mk = lambda s: torch.randn((1, s, 8, 128), device="cuda", dtype=torch.float32, generator=g).to(torch.bfloat16)
    q, k, v = mk(1024), mk(32768), mk(32768)
    o = torch.full_like(q, float("nan"))
    lse = torch.full((1, 8, 1024), float("nan"), device="cuda", dtype=torch.float32)
    assert gpu_runner.splitkv_select(1, 8, 1024, 32768, causal) == (1 if causal else 8)
    splits = 4 if causal else 0
    print(f"  splitkv B1 H8 1024x32768 causal={causal} splits={splits}", flush=True)
    gpu_runner.call_splitkv(q, k, v, o, lse, causal, splits)
    torch.cuda.synchronize()
    assert not torch.isnan(o).any().item()
    rows = orc.sample_rows(1024)
    heads = [(0, hh) for hh in range(8)]
    ref, ref_lse = orc.attention_fp64(to_host_bits(q), to_host_bits(k), to_host_bits(v), orc.DEFAULT_SCALE, causal,
                                      rows=rows, heads=heads)
    got = to_host_bits(o[:, rows])
    got_lse = lse[:, :, rows].cpu().numpy()
    sel = lambda x: np.stack([x[0, :, hh] for _, hh in heads])
    e = orc.errors(sel(got), got_lse[0], sel(ref), ref_lse[0])
    assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), e


@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_splitkv_decode_at_scale(gpu_runner, causal):
    """Decode: B4 H8, one query against 65536 keys (Auto: the one-wave decode
    shape, 24 chunks of 86 32-key tiles), every row and head against the FP64
    oracle."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    mk = lambda s: torch.randn((4, s, 8, 128), device="cuda", dtype=torch.float32, generator=g).to(torch.bfloat16)
    q, k, v = mk(1), mk(65536), mk(65536)
    o = torch.full_like(q, float("nan"))
    lse = torch.full((4, 8, 1), float("nan"), device="cuda", dtype=torch.float32)
    splits = gpu_runner.splitkv_select(4, 8, 1, 65536, causal)
    print(f"  splitkv decode B4 H8 1x65536 causal={causal} splits={splits}", flush=True)
    assert splits == (1 if causal else 24)
    gpu_runner.call_splitkv(q, k, v, o, lse, causal, 0)
    torch.cuda.synchronize()
    ref, ref_lse = orc.attention_fp64(to_host_bits(q), to_host_bits(k), to_host_bits(v), orc.DEFAULT_SCALE, causal)
    e = orc.errors(to_host_bits(o), lse.cpu().numpy(), ref, ref_lse)
    assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), e


MANY = [((1, 2, 1, 20000), False), ((2, 3, 17, 9000), False), ((1, 2, 40, 20000), False),
        ((1, 2, 2048, 2048), True)]


@pytest.mark.parametrize("case", MANY, ids=lambda c: "b%dh%d_%dx%d" % c[0] + ("_causal" if c[1] else ""))
def test_splitkv_many_chunks(gpu_runner, case):
    """Merges of 9 to 256 chunks, where the merge spreads a row's chunks over
    2, 4 or 8 lane groups: decode (32-key tiles) and prefill (64-key tiles)
    shapes, and causal rows that see only the first chunks, against the FP64
    oracle with and without LSE."""
    import torch
    (b, h, sq, sk), causal = case
    q, k, v = orc.make_inputs(b, h, sq, sk, "normal", seed=21)
    ref, ref_lse = orc.attention_fp64(q, k, v, orc.DEFAULT_SCALE, causal)
    for splits in (9, 17, 33, 100, 256):
        for with_lse in (False, True):
            o, lse = _run(gpu_runner, torch, q, k, v, causal, splits, with_lse)
            e = orc.errors(o, lse, ref, ref_lse if with_lse else None)
            assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), (splits, with_lse, e)


GQA = [(2, 8, 2, 1, 5000), (1, 12, 3, 5, 4000), (3, 6, 2, 20, 1500), (2, 8, 1, 16, 3000), (1, 8, 4, 100, 2000),
       (1, 32, 8, 1, 40000)]


@pytest.mark.parametrize("shape", GQA, ids=lambda s: "b%dh%dkv%d_%dx%d" % s)
def test_splitkv_gqa(gpu_runner, shape):
    """fav4_bshd_forward_splitkv_gqa: decode shapes (Sq <= 32) pack the query
    heads of a K/V head into shared 32-row tiles, longer ones run one head per
    item.  Against the FP64 oracle (Auto and explicit chunks), and at an
    explicit chunk count bitwise equal to the MHA split-KV call on K/V with
    their heads repeated group-wise (per row, the packed tile computes exactly
    what a tile of that head alone does)."""
    import torch
    b, h, kvh, sq, sk = shape
    group = h // kvh
    q, _, _ = orc.make_inputs(b, h, sq, sk, "normal", seed=41)
    _, k, v = orc.make_inputs(b, kvh, sq, sk, "normal", seed=42)
    ke, ve = np.repeat(k, group, axis=2), np.repeat(v, group, axis=2)
    for causal in (False, True):
        ref, ref_lse = orc.attention_fp64(q, ke, ve, orc.DEFAULT_SCALE, causal)
        for splits in (0, 3):
            o, lse = _run(gpu_runner, torch, q, k, v, causal, splits, True)
            e = orc.errors(o, lse, ref, ref_lse)
            assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), (causal, splits, e)
            if splits:
                om, lsem = _run(gpu_runner, torch, q, ke, ve, causal, splits, True)
                assert np.array_equal(o, om), (causal, "O differs from MHA on repeated heads")
                assert np.array_equal(lse.view(np.int32), lsem.view(np.int32)), (causal, "LSE differs")
