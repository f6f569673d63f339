"""Rows past sq must not store, whatever their 32-bit row offsets wrap to.

A q tile covers rows [q0, q0 + BM); the kernels address row r of a slice at
the 32-bit offset (r - q0) * row_stride.  When the row stride is large (a huge
head count, or a strided view whose sequence stride spans the batch), a row
past sq can wrap past 2^32 onto offset 0 -- row q0 -- and, in a causal call, it
sees more keys than row q0 does.  These tests use such strides with sq = 1, so
rows 64 (128-row tiles) and 128 (256-row tiles) wrap onto row 0: row 0 sees
key 0 only, so O must equal V's key 0 exactly (its weight is exp2(0) = 1) and
LSE = scale * q.k0.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SK = 16


def _kv(torch, dev, shape, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.randn(shape, device=dev, dtype=torch.float32, generator=g).to(torch.bfloat16)


def _check_row0(torch, o, lse, q, k0, v0):
    """O[..., h, :] == v0 bitwise and LSE == scale * q.k0 for every (b, h)."""
    assert torch.equal(o.view(torch.int16), v0.expand_as(o).view(torch.int16))
    if lse is not None:
        ref = (q.double() * k0.double()).sum(-1) / np.sqrt(128)          # [B, 1, H]
        err = (lse.double() - ref.permute(0, 2, 1)).abs().max().item()
        assert err <= 1e-3, err


@pytest.mark.parametrize("config", [1, 2, 3])
def test_gqa_huge_head_count(gpu_runner, config):
    """B1 H262144 with one K/V head, sq 1, sk 16, causal: Q/O rows are 64 MiB
    apart, so row 64 of every tile sits 2^32 bytes past row 0."""
    import torch
    dev = torch.device("cuda:0")
    h = 1 << 18
    print(f"gqa B1 H{h} KVH1 sq1 sk{SK} causal config {config}", flush=True)
    q = _kv(torch, dev, (1, 1, h, 128), 1)
    k, v = _kv(torch, dev, (1, SK, 1, 128), 2), _kv(torch, dev, (1, SK, 1, 128), 3)
    o = torch.full_like(q, float("nan"))
    lse = torch.full((1, h, 1), float("nan"), device=dev, dtype=torch.float32)
    gpu_runner.call_gqa(q, k, v, o, lse, True, config)
    torch.cuda.synchronize()
    _check_row0(torch, o, lse, q, k[:, :1], v[:, :1])


@pytest.mark.parametrize("config", [1, 2, 3])
def test_strided_sbhd_view(gpu_runner, config):
    """Q/O stored [Sq=1, B=4096, H=64, 128] and K/V [Sk, B, 1, 128], passed as
    [B, S, H, 128] views: the Q/O sequence stride is 64 MiB."""
    import torch
    dev = torch.device("cuda:0")
    b, h = 4096, 64
    print(f"strided SBHD B{b} H{h} KVH1 sq1 sk{SK} causal config {config}", flush=True)
    q = _kv(torch, dev, (1, b, h, 128), 4).transpose(0, 1)
    k = _kv(torch, dev, (SK, b, 1, 128), 5).transpose(0, 1)
    v = _kv(torch, dev, (SK, b, 1, 128), 6).transpose(0, 1)
    o = torch.full((1, b, h, 128), float("nan"), device=dev, dtype=torch.bfloat16).transpose(0, 1)
    assert o.stride(1) == b * h * 128
    lse = torch.full((b, h, 1), float("nan"), device=dev, dtype=torch.float32)
    gpu_runner.call_strided(q, k, v, o, lse, True, config)
    torch.cuda.synchronize()
    _check_row0(torch, o, lse, q, k[:, :1], v[:, :1])


def test_varlen_huge_head_count(gpu_runner):
    """Packed sequences with H262144 and one K/V head (token rows 64 MiB apart):
    two sequences of one query each, 16 and 5 keys, causal."""
    import torch
    dev = torch.device("cuda:0")
    h = 1 << 18
    print(f"varlen H{h} KVH1 two sequences of one query, causal", flush=True)
    q = _kv(torch, dev, (2, h, 128), 7)
    k, v = _kv(torch, dev, (SK + 5, 1, 128), 8), _kv(torch, dev, (SK + 5, 1, 128), 9)
    cu_q = torch.tensor([0, 1, 2], device=dev, dtype=torch.int32)
    cu_k = torch.tensor([0, SK, SK + 5], device=dev, dtype=torch.int32)
    o = torch.full_like(q, float("nan"))
    lse = torch.full((h, 2), float("nan"), device=dev, dtype=torch.float32)
    gpu_runner.call_varlen(q, k, v, o, lse, cu_q, cu_k, 1, SK, True)
    torch.cuda.synchronize()
    for i, k0 in enumerate((0, SK)):
        _check_row0(torch, o[i][None, None], lse[:, i][None, :, None], q[i][None, None], k[k0][None, None],
                    v[k0][None, None])
