"""GPU tests at full benchmark sizes and at the edges of the contract.

Full-size shapes (B32 H8 S up to 32768) are checked like the reference
benchmark checks them (benchmarks/bshd.py:147-156): the FP64 oracle on the
sampled rows {0,1,63,64,127,128,n-1} U range(0,n,n//24), here for a few
(b, h) pairs, with NaN-prefilled outputs.  Inputs are generated on the GPU
from a seeded generator; the oracle reads the same tensors back.
"""
import math

import numpy as np
import pytest

from oracle import attention as orc
from tests.conftest import to_device, to_host_bits

pytestmark = pytest.mark.gpu
PAIRS = [(0, 0), (3, 5), (31, 7)]


def _gpu_inputs(torch, b, h, sq, sk, seed=11939):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    mk = lambda s: torch.randn((b, s, h, 128), device="cuda", dtype=torch.float32, generator=g).to(torch.bfloat16)
    return mk(sq), mk(sk), mk(sk)


def _check_sampled(runner, torch, q, k, v, causal, config, with_lse, pairs, bar="reference"):
    b, sq, h, _ = q.shape
    o = torch.full_like(q, float("nan"))
    lse = torch.full((b, h, sq), float("nan"), device="cuda", dtype=torch.float32) if with_lse else None
    print(f"  B{b} H{h} {sq}x{k.shape[1]} causal={causal} config={config} lse={with_lse}", flush=True)
    runner.call(q, k, v, o, lse, causal, config)
    torch.cuda.synchronize()
    rows = orc.sample_rows(sq)
    qb, kb, vb = to_host_bits(q), to_host_bits(k), to_host_bits(v)
    ref, ref_lse = orc.attention_fp64(qb, kb, vb, orc.DEFAULT_SCALE, causal, rows=rows, heads=pairs)
    got = to_host_bits(o[:, rows])
    got_lse = lse[:, :, rows].cpu().numpy() if with_lse else None
    sel = lambda x: np.stack([x[bb, :, hh] for bb, hh in pairs])
    sel_l = lambda x: np.stack([x[bb, hh] for bb, hh in pairs])
    e = orc.errors(sel(got), sel_l(got_lse) if with_lse else None, sel(ref), sel_l(ref_lse) if with_lse else None)
    # every output element must have been written
    assert not torch.isnan(o).any().item(), "unwritten output elements"
    ok = orc.check_acceptance_tolerance(e) and (bar != "reference" or orc.check_reference_tolerance(e))
    assert ok, e
    return e


@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_headline_b32h8s4096_all_configs(gpu_runner, causal):
    import torch
    q, k, v = _gpu_inputs(torch, 32, 8, 4096, 4096)
    for config in (0, 1, 2, 3):
        _check_sampled(gpu_runner, torch, q, k, v, causal, config, with_lse=(config == 0), pairs=PAIRS)


@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
@pytest.mark.parametrize("shape", [(2, 4, 1000, 1500), (1, 2, 257, 3000), (3, 1, 64, 64), (1, 8, 4096, 4096)],
                         ids=lambda s: "b%dh%d_%dx%d" % s)
def test_configs_1_and_2_bitwise(gpu_runner, shape, causal):
    """128-row (config 1) and 256-row (config 2) workgroups run the same
    per-wave tile loop over the same 64-key tiles, so every row's O and LSE
    are bitwise equal: Auto may pick either, and the varlen kernel (which
    follows the same choice) matches the forward at any config."""
    import torch
    b, h, sq, sk = shape
    q, k, v = _gpu_inputs(torch, b, h, sq, sk)
    outs = []
    for config in (1, 2):
        o = torch.full_like(q, float("nan"))
        lse = torch.full((b, h, sq), float("nan"), device="cuda", dtype=torch.float32)
        print(f"  config {config} B{b} H{h} {sq}x{sk} causal={causal}", flush=True)
        gpu_runner.call(q, k, v, o, lse, causal, config)
        torch.cuda.synchronize()
        outs.append((o, lse))
    assert torch.equal(outs[0][0].view(torch.int16), outs[1][0].view(torch.int16))
    assert torch.equal(outs[0][1].view(torch.int32), outs[1][1].view(torch.int32))


@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
@pytest.mark.parametrize("shape", [(8, 16, 2048, 2048), (8, 16, 1030, 1950)], ids=["even_tiles", "odd_tiles"])
def test_slices_match_isolated_launches(gpu_runner, shape, causal):
    """The result of a (b, h) slice must not depend on the rest of the launch
    (grid size, item order, XCD mapping, even or odd key-tile counts): every
    slice of a 128-head launch is bitwise equal to the same slice launched
    alone."""
    import torch
    b, h, sq, sk = shape
    q, k, v = _gpu_inputs(torch, b, h, sq, sk, seed=77)
    for config in (1, 2):
        print(f"  slices {shape} causal={causal} config={config}", flush=True)
        o = torch.full_like(q, float("nan"))
        lse = torch.full((b, h, sq), float("nan"), device="cuda", dtype=torch.float32)
        gpu_runner.call(q, k, v, o, lse, causal, config)
        for bb in range(b):
            for hh in range(h):
                qs, ks, vs = (x[bb:bb + 1, :, hh:hh + 1].contiguous() for x in (q, k, v))
                os_ = torch.full_like(qs, float("nan"))
                ls = torch.full((1, 1, sq), float("nan"), device="cuda", dtype=torch.float32)
                gpu_runner.call(qs, ks, vs, os_, ls, causal, config)
                assert torch.equal(o[bb, :, hh].view(torch.int16), os_[0, :, 0].view(torch.int16)), (bb, hh)
                assert torch.equal(lse[bb, hh].view(torch.int32), ls[0, 0].view(torch.int32)), (bb, hh)
        torch.cuda.synchronize()


@pytest.mark.parametrize("s", [512, 1024, 8192, 16384, 32768])
def test_long_sequence_sweep(gpu_runner, s):
    """B32 H8 D128, S in {512, 1024, 8192, 16384, 32768}, dense and top-left causal."""
    import torch
    q, k, v = _gpu_inputs(torch, 32, 8, s, s)
    for causal in (False, True):
        _check_sampled(gpu_runner, torch, q, k, v, causal, 0, with_lse=(s == 8192), pairs=PAIRS)
    del q, k, v
    torch.cuda.empty_cache()


def test_deterministic_and_stream(gpu_runner):
    """Same inputs give bitwise-identical O and LSE, on the default and on a side stream."""
    import torch
    q, k, v = _gpu_inputs(torch, 2, 8, 1000, 3077)
    outs = []
    side = torch.cuda.Stream()
    for use_side in (False, False, True):
        o = torch.full_like(q, float("nan"))
        lse = torch.full((2, 8, 1000), float("nan"), device="cuda", dtype=torch.float32)
        if use_side:
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                gpu_runner.call(q, k, v, o, lse, True, 0)
            torch.cuda.current_stream().wait_stream(side)
        else:
            gpu_runner.call(q, k, v, o, lse, True, 0)
        torch.cuda.synchronize()
        outs.append((o.view(torch.int16).clone(), lse.clone()))
    for o, l in outs[1:]:
        assert torch.equal(o, outs[0][0]) and torch.equal(l.view(torch.int32), outs[0][1].view(torch.int32))


@pytest.mark.parametrize("scale", [0.5, 0.01, 1.0 / 64])
def test_non_default_scale(gpu_runner, scale):
    import torch
    q, k, v = orc.make_inputs(2, 4, 193, 257, "normal")
    dev = torch.device("cuda:0")
    qd, kd, vd = to_device(q, dev), to_device(k, dev), to_device(v, dev)
    for causal in (False, True):
        o = torch.full_like(qd, float("nan"))
        lse = torch.full((2, 4, 193), float("nan"), device=dev, dtype=torch.float32)
        gpu_runner.call(qd, kd, vd, o, lse, causal, 0, scale=scale)
        torch.cuda.synchronize()
        ref, ref_lse = orc.attention_fp64(q, k, v, scale, causal)
        e = orc.errors(to_host_bits(o), lse.cpu().numpy(), ref, ref_lse)
        assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), (scale, causal, e)


@pytest.mark.parametrize("shape", [(1, 2, 1, 4099), (1, 2, 4099, 1), (3, 1, 70, 70), (1, 64, 300, 300),
                                   (2, 3, 257, 255)], ids=lambda s: "b%dh%d_%dx%d" % s)
def test_edge_shapes_and_no_out_of_bounds_writes(gpu_runner, shape):
    """Odd shapes; O and LSE are embedded in larger buffers whose tails must stay untouched."""
    import torch
    b, h, sq, sk = shape
    q, k, v = orc.make_inputs(b, h, sq, sk, "normal")
    dev = torch.device("cuda:0")
    qd, kd, vd = to_device(q, dev), to_device(k, dev), to_device(v, dev)
    n_o, n_l = b * sq * h * 128, b * h * sq
    o_buf = torch.full((n_o + 4096,), 7.0, device=dev, dtype=torch.bfloat16)
    l_buf = torch.full((n_l + 1024,), 7.0, device=dev, dtype=torch.float32)
    o = o_buf[:n_o].view(b, sq, h, 128)
    lse = l_buf[:n_l].view(b, h, sq)
    for causal in (False, True):
        o.fill_(float("nan"))
        lse.fill_(float("nan"))
        gpu_runner.call(qd, kd, vd, o, lse, causal, 0)
        torch.cuda.synchronize()
        assert torch.all(o_buf[n_o:] == 7.0).item() and torch.all(l_buf[n_l:] == 7.0).item(), "wrote past O/LSE"
        ref, ref_lse = orc.attention_fp64(q, k, v, orc.DEFAULT_SCALE, causal)
        e = orc.errors(to_host_bits(o), lse.cpu().numpy(), ref, ref_lse)
        assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), (shape, causal, e)


def test_bad_arguments_return_status(gpu_runner):
    """A rejected call returns hipErrorInvalidValue through the binding and launches nothing."""
    import torch
    q, k, v = _gpu_inputs(torch, 1, 1, 64, 64)
    o = torch.full_like(q, float("nan"))
    with pytest.raises(RuntimeError, match="HIP status 1"):
        gpu_runner.call(q, k, v, o, None, 2, 0)
    with pytest.raises(RuntimeError, match="HIP status 1"):
        gpu_runner.call(q, k, v, o, None, 0, 0, scale=float("nan"))
    torch.cuda.synchronize()
    assert torch.isnan(o).all().item()


def test_tensors_past_4gib(gpu_runner):
    """B16 H32 Sq=Sk=32768: every tensor is 4 GiB, so the last (b, h) slices sit
    past 2^32 bytes (64-bit row offsets, 32-bit buffer bounds per head)."""
    import torch
    b, h, s = 16, 32, 32768
    q, k, v = _gpu_inputs(torch, b, h, s, s)
    assert q.numel() * 2 == 1 << 32
    _check_sampled(gpu_runner, torch, q, k, v, True, 0, with_lse=True, pairs=[(15, 31), (15, 0), (8, 17)],
                   bar="acceptance")
    del q, k, v
    torch.cuda.empty_cache()
