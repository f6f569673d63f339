"""Seeded random sweep over every forward entry point through the C ABI.

Each case draws a batch, head count, K/V head grouping, query and key lengths
(1 to ~900, so tails of every residue mod 32/64/256 occur), mask, config and
LSE on/off from a fixed seed, then checks:
  * fav4_bshd_forward at the drawn config against the FP64 oracle (the
    reference harness's bar and the acceptance bar);
  * fav4_bshd_forward_gqa on the grouped K/V: bitwise equal to the MHA forward
    on K/V with their heads repeated group-wise (same config);
  * fav4_bshd_forward_strided on BHSD views of the same data: bitwise equal to
    the BSHD forward (same config);
  * fav4_bshd_forward_splitkv at a drawn chunk count (0 = Auto) against the
    FP64 oracle.
Every output buffer starts NaN-filled, so an unwritten element fails.
"""
import numpy as np
import pytest

from oracle import attention as orc
from tests.conftest import to_device, to_host_bits

pytestmark = pytest.mark.gpu

N_CASES = 24


def _draw(rng):
    b = int(rng.integers(1, 4))
    kvh = int(rng.choice([1, 2, 3]))
    group = int(rng.choice([1, 2, 4]))
    sq = int(rng.integers(1, 900))
    sk = int(rng.integers(1, 900))
    return dict(b=b, h=kvh * group, kvh=kvh, sq=sq, sk=sk, causal=bool(rng.integers(0, 2)),
                config=int(rng.integers(0, 4)), lse=bool(rng.integers(0, 2)), splits=int(rng.choice([0, 2, 3, 7, 16])))


CASES = [_draw(np.random.default_rng(1000 + i)) for i in range(N_CASES)]


def _ids(c):
    return "b{b}h{h}kv{kvh}_{sq}x{sk}_{m}_cfg{config}{l}_s{splits}".format(
        m="causal" if c["causal"] else "dense", l="_lse" if c["lse"] else "", **c)


@pytest.mark.parametrize("case", CASES, ids=_ids)
def test_random_case_all_entry_points(gpu_runner, case):
    import torch
    b, h, kvh, sq, sk = case["b"], case["h"], case["kvh"], case["sq"], case["sk"]
    causal, config, with_lse, splits = case["causal"], case["config"], case["lse"], case["splits"]
    group = h // kvh
    seed = 7 + sq * 1000 + sk
    q, _, _ = orc.make_inputs(b, h, sq, sk, "normal", seed=seed)
    _, k, v = orc.make_inputs(b, kvh, sq, sk, "normal", seed=seed + 1)
    ke, ve = np.repeat(k, group, axis=2), np.repeat(v, group, axis=2)
    dev = torch.device("cuda:0")
    qd, kd, vd, ked, ved = (to_device(x, dev) for x in (q, k, v, ke, ve))
    nan = float("nan")
    print(f"  random {_ids(case)}", flush=True)

    def lse_buf():
        return torch.full((b, h, sq), nan, device=dev, dtype=torch.float32) if with_lse else None

    # MHA forward on repeated K/V heads, against the oracle
    o = torch.full_like(qd, nan)
    lse = lse_buf()
    gpu_runner.call(qd, ked, ved, o, lse, causal, config)
    torch.cuda.synchronize()
    ref, ref_lse = orc.attention_fp64(q, ke, ve, orc.DEFAULT_SCALE, causal)
    got_lse = lse.cpu().numpy() if with_lse else None
    e = orc.errors(to_host_bits(o), got_lse, ref, ref_lse if with_lse else None)
    assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), ("forward", e)

    # GQA on the grouped K/V: bitwise the MHA result
    og = torch.full_like(qd, nan)
    lg = lse_buf()
    gpu_runner.call_gqa(qd, kd, vd, og, lg, causal, config)
    torch.cuda.synchronize()
    assert torch.equal(og.view(torch.int16), o.view(torch.int16)), "gqa O differs from MHA"
    if with_lse:
        assert torch.equal(lg.view(torch.int32), lse.view(torch.int32)), "gqa LSE differs from MHA"

    # strided forward on BHSD copies viewed as [B, S, H, D]: bitwise the BSHD result
    qs_, ks_, vs_ = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (qd, kd, vd))
    os_bhsd = torch.full((b, h, sq, 128), nan, device=dev, dtype=torch.bfloat16)
    ls = lse_buf()
    gpu_runner.call_strided(qs_, ks_, vs_, os_bhsd.transpose(1, 2), ls, causal, config)
    torch.cuda.synchronize()
    assert torch.equal(os_bhsd.transpose(1, 2).contiguous().view(torch.int16), o.view(torch.int16)), \
        "strided O differs"
    if with_lse:
        assert torch.equal(ls.view(torch.int32), lse.view(torch.int32)), "strided LSE differs"

    # split-KV (MHA) against the oracle
    osk = torch.full_like(qd, nan)
    lsk = lse_buf()
    gpu_runner.call_splitkv(qd, ked, ved, osk, lsk, causal, splits)
    torch.cuda.synchronize()
    e = orc.errors(to_host_bits(osk), lsk.cpu().numpy() if with_lse else None, ref, ref_lse if with_lse else None)
    assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), ("splitkv", splits, e)
