"""GPU checks of arbitrary-stride inputs and outputs (fav4_bshd_forward_strided) via the C ABI.

The strided entry point runs the same kernels as fav4_bshd_forward with the
addresses taken from per-tensor strides, so every layout must give O and LSE
bitwise equal to fav4_bshd_forward (or fav4_bshd_forward_gqa) on contiguous
BSHD copies of the same data.  Covered: BHSD tensors, packed QKV, K and V from
different layouts, O written into a padded buffer (the padding must stay
untouched), GQA, every config, dense and causal, LSE on and off; one FP64
oracle check per layout.
"""
import numpy as np
import pytest

from oracle import attention as orc
from tests.conftest import to_device, to_host_bits

pytestmark = pytest.mark.gpu

SHAPES = [(2, 4, 300, 700), (1, 8, 1000, 1000), (2, 2, 64, 129), (1, 3, 513, 257)]


def _bshd_reference(runner, q, k, v, causal, config, kvh):
    """Contiguous BSHD forward: (O, LSE)."""
    import torch
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    o = torch.full_like(qc, float("nan"))
    lse = torch.full((q.shape[0], q.shape[2], q.shape[1]), float("nan"), device=q.device, dtype=torch.float32)
    if kvh == q.shape[2]:
        runner.call(qc, kc, vc, o, lse, causal, config)
    else:
        runner.call_gqa(qc, kc, vc, o, lse, causal, config)
    return o, lse


def _run_strided(runner, q, k, v, o, causal, config, with_lse):
    import torch
    lse = (torch.full((q.shape[0], q.shape[2], q.shape[1]), float("nan"), device=q.device, dtype=torch.float32)
           if with_lse else None)
    runner.call_strided(q, k, v, o, lse, causal, config)
    torch.cuda.synchronize()
    return lse


def _inputs(b, h, sq, sk, kvh, seed=3):
    import torch
    dev = torch.device("cuda:0")
    q, _, _ = orc.make_inputs(b, h, sq, sk, "normal", seed=seed)
    _, k, v = orc.make_inputs(b, kvh, sq, sk, "normal", seed=seed + 1)
    return to_device(q, dev), to_device(k, dev), to_device(v, dev), (q, k, v)


def _oracle_check(host, o, lse, causal, h, kvh):
    q, k, v = host
    ke, ve = np.repeat(k, h // kvh, axis=2), np.repeat(v, h // kvh, axis=2)
    ref, ref_lse = orc.attention_fp64(q, ke, ve, orc.DEFAULT_SCALE, causal)
    e = orc.errors(to_host_bits(o), lse.cpu().numpy(), ref, ref_lse)
    assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), e


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "b%dh%d_%dx%d" % s)
def test_bhsd_layout_bitwise(gpu_runner, shape):
    """Q, K, V and O all stored [B, H, S, 128] (torch SDPA's layout)."""
    import torch
    b, h, sq, sk = shape
    qd, kd, vd, host = _inputs(b, h, sq, sk, h)
    qh, kh, vh = (x.transpose(1, 2).contiguous() for x in (qd, kd, vd))      # BHSD storage
    for causal in (False, True):
        for config in (0, 1, 2, 3):
            print(f"  bhsd {shape} causal={causal} config={config}", flush=True)
            oh = torch.full((b, h, sq, 128), float("nan"), device=qd.device, dtype=torch.bfloat16)
            lse = _run_strided(gpu_runner, qh.transpose(1, 2), kh.transpose(1, 2), vh.transpose(1, 2),
                               oh.transpose(1, 2), causal, config, True)
            o_ref, l_ref = _bshd_reference(gpu_runner, qd, kd, vd, causal, config, h)
            torch.cuda.synchronize()
            assert torch.equal(oh.transpose(1, 2).contiguous().view(torch.int16), o_ref.view(torch.int16))
            assert torch.equal(lse.view(torch.int32), l_ref.view(torch.int32))
        _oracle_check(host, oh.transpose(1, 2), lse, causal, h, h)


@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_packed_qkv_and_padded_output(gpu_runner, causal):
    """Q, K, V as views of one [B, S, 3, H, 128] buffer; O into [B, S, H+3, 128][:, :, 1:H+1]."""
    import torch
    b, h, s = 2, 4, 700
    qd, kd, vd, host = _inputs(b, h, s, s, h, seed=9)
    qkv = torch.stack([qd, kd, vd], dim=2).contiguous()
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    assert q.stride(1) == 3 * h * 128
    for config in (0, 2, 3):
        for with_lse in (False, True):
            pad = torch.full((b, s, h + 3, 128), float("nan"), device=qd.device, dtype=torch.bfloat16)
            o = pad[:, :, 1:h + 1]
            lse = _run_strided(gpu_runner, q, k, v, o, causal, config, with_lse)
            o_ref, l_ref = _bshd_reference(gpu_runner, qd, kd, vd, causal, config, h)
            torch.cuda.synchronize()
            assert torch.equal(o.contiguous().view(torch.int16), o_ref.view(torch.int16)), (config, with_lse)
            if with_lse:
                assert torch.equal(lse.view(torch.int32), l_ref.view(torch.int32))
            assert torch.isnan(pad[:, :, 0].float()).all().item() and torch.isnan(pad[:, :, h + 1:].float()).all().item()
    _oracle_check(host, o, lse, causal, h, h)


@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_gqa_mixed_layouts(gpu_runner, causal):
    """GQA (8 query heads, 2 K/V heads) with Q in BSHD, K in BHSD, V in a padded BSHD buffer."""
    import torch
    b, h, kvh, sq, sk = 2, 8, 2, 257, 1000
    qd, kd, vd, host = _inputs(b, h, sq, sk, kvh, seed=21)
    kh = kd.transpose(1, 2).contiguous()
    vpad = torch.zeros((b, sk, kvh + 1, 128), device=qd.device, dtype=torch.bfloat16)
    vpad[:, :, :kvh] = vd
    for config in (0, 1, 2, 3):
        o = torch.full_like(qd, float("nan"))
        lse = _run_strided(gpu_runner, qd, kh.transpose(1, 2), vpad[:, :, :kvh], o, causal, config, True)
        o_ref, l_ref = _bshd_reference(gpu_runner, qd, kd, vd, causal, config, kvh)
        torch.cuda.synchronize()
        assert torch.equal(o.view(torch.int16), o_ref.view(torch.int16)), config
        assert torch.equal(lse.view(torch.int32), l_ref.view(torch.int32)), config
    _oracle_check(host, o, lse, causal, h, kvh)


def test_strided_rejects_before_launch(gpu_runner):
    """A seq stride that is not a multiple of 8 elements is rejected; O stays untouched."""
    import torch
    b, h, s = 1, 2, 64
    qd, kd, vd, _ = _inputs(b, h, s, s, h)
    buf = torch.zeros((b, s, h * 128 + 4), device=qd.device, dtype=torch.bfloat16)
    qv = buf[:, :, :h * 128].unflatten(2, (h, 128))          # seq stride h*128+4 elements
    assert qv.stride(1) % 8 != 0
    o = torch.full_like(qd, float("nan"))
    with pytest.raises(RuntimeError, match="HIP status 1"):
        gpu_runner.call_strided(qv, kd, vd, o, None, False, 0)
    torch.cuda.synchronize()
    assert torch.isnan(o.float()).all().item()
