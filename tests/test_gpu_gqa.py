"""GPU checks of grouped-/multi-query attention (fav4_bshd_forward_gqa) via the C ABI.

Query head h reads K/V head h / (heads / kv_heads).  Two pins:
  * bitwise equality with fav4_bshd_forward on K/V whose heads are repeated
    group-wise (the same data through the same arithmetic), for every config,
    dense and top-left causal, with and without LSE;
  * the FP64 oracle on the repeated K/V at the reference harness's bar.
"""
import numpy as np
import pytest

from oracle import attention as orc
from tests.conftest import to_device, to_host_bits

pytestmark = pytest.mark.gpu

CASES = [(2, 8, 2, 257, 1000), (1, 4, 1, 300, 513), (2, 6, 3, 64, 2049), (1, 8, 8, 193, 257), (1, 2, 1, 1, 77)]


def _expand(x, group):
    """[B, S, KVH, D] -> [B, S, KVH*group, D], head h = kv head h // group."""
    return np.repeat(x, group, axis=2)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "b%dh%dkv%d_%dx%d" % c)
def test_gqa_matches_expanded_mha_bitwise_and_oracle(gpu_runner, case):
    import torch
    b, h, kvh, sq, sk = case
    group = h // kvh
    q, _, _ = orc.make_inputs(b, h, sq, sk, "normal")
    _, k, v = orc.make_inputs(b, kvh, sq, sk, "normal", seed=7)
    ke, ve = _expand(k, group), _expand(v, group)
    dev = torch.device("cuda:0")
    qd, kd, vd = to_device(q, dev), to_device(k, dev), to_device(v, dev)
    ked, ved = to_device(ke, dev), to_device(ve, dev)
    for causal in (False, True):
        ref, ref_lse = orc.attention_fp64(q, ke, ve, orc.DEFAULT_SCALE, causal)
        for config in (0, 1, 2, 3):
            print(f"  gqa B{b} H{h} KVH{kvh} {sq}x{sk} causal={causal} config={config}", flush=True)
            o_g = torch.full_like(qd, float("nan"))
            o_m = torch.full_like(qd, float("nan"))
            l_g = torch.full((b, h, sq), float("nan"), device=dev, dtype=torch.float32)
            l_m = torch.full((b, h, sq), float("nan"), device=dev, dtype=torch.float32)
            gpu_runner.call_gqa(qd, kd, vd, o_g, l_g, causal, config)
            gpu_runner.call(qd, ked, ved, o_m, l_m, causal, config)
            torch.cuda.synchronize()
            assert torch.equal(o_g.view(torch.int16), o_m.view(torch.int16)), (causal, config)
            assert torch.equal(l_g.view(torch.int32), l_m.view(torch.int32)), (causal, config)
            e = orc.errors(to_host_bits(o_g), l_g.cpu().numpy(), ref, ref_lse)
            assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), (causal, config, e)


def test_gqa_rejects_non_divisor(gpu_runner):
    import torch
    q, k, v = orc.make_inputs(1, 4, 64, 64, "normal")
    dev = torch.device("cuda:0")
    qd = to_device(q, dev)
    _, k3, v3 = orc.make_inputs(1, 3, 64, 64, "normal")
    o = torch.full_like(qd, float("nan"))
    with pytest.raises(RuntimeError, match="HIP status 1"):
        gpu_runner.call_gqa(qd, to_device(k3, dev), to_device(v3, dev), o, None, False, 0)
    torch.cuda.synchronize()
    assert torch.isnan(o).all().item()
