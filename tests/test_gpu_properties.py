"""Size-independent properties of the forward at the headline size (B32 H8
Sq=Sk=4096 D128), checked on every output element without the oracle.

* Constant values. When every V row of a (batch, head) slice is the same
  BF16 vector c, every output row is c bitwise. This holds dense and causal,
  on every config. The weights, the O rescale and the final division by the
  weight sum cancel exactly within BF16 rounding.
* Causal prefix. With top-left causal masking, row i depends only on keys
  j <= i. Rewriting the K/V rows from key m on leaves every row < m
  bitwise unchanged, O and LSE, where m lies inside a q tile and a key
  tile. This also holds when a wave's other rows move their softmax base:
  a row whose base did not move is rescaled by exactly 1.
* Slice independence. Rewriting one (batch, head) slice's Q, K and V
  leaves every other slice bitwise unchanged.
* Key and query tails. The strided entry point runs on views whose
  sequence stride leaves spare rows between batches, and those rows hold
  NaN. Sq = Sk = 4000 is not a multiple of any tile. O and LSE must be
  bitwise the contiguous call's and finite. A NaN reaching a masked PV
  product would show, since 0 * NaN = NaN. The O rows past sq keep their
  sentinel.
* The other entry points, each on one exact property:
  - constant V through the GQA forward (B32 H8, 2 K/V heads, S4096);
  - constant V through split-KV with Auto chunks: the bench's split-KV
    prefill (B1 H8 Sq1024 Sk32768, dense and causal), its GQA decode
    (B4 H32 with 8 K/V heads, one query against 32768 keys) and a
    single-head causal prefill of 16384 tokens;
  - constant V through the bench's packed and paged decode batch (32
    sequences x 1 query, 1949-31077 keys), dense and bottom-right causal;
  - independence of the sequences of the bench's packed batch (32
    sequences of 1237-6743 tokens): rewriting one leaves the others' O
    and LSE bitwise unchanged, dense, top-left and bottom-right causal.
"""
import pytest

pytestmark = pytest.mark.gpu
B, H, S = 32, 8, 4096


def _inputs(torch, b, h, sq, sk, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    mk = lambda s: torch.randn((b, s, h, 128), device="cuda", dtype=torch.float32, generator=g).to(torch.bfloat16)
    return mk(sq), mk(sk), mk(sk)


def _run(torch, runner, q, k, v, causal, config):
    o = torch.full_like(q, float("nan"))
    lse = torch.full((q.shape[0], q.shape[2], q.shape[1]), float("nan"), device="cuda", dtype=torch.float32)
    runner.call(q, k, v, o, lse, causal, config)
    torch.cuda.synchronize()
    return o, lse


def _same(torch, x, y):
    bits = torch.int16 if x.dtype == torch.bfloat16 else torch.int32
    return torch.equal(x.contiguous().view(bits), y.contiguous().view(bits))


@pytest.mark.parametrize("config", [0, 1, 2, 3])
@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_constant_values_give_that_value(gpu_runner, causal, config):
    import torch
    q, k, _ = _inputs(torch, B, H, S, S, seed=101)
    g = torch.Generator(device="cuda")
    g.manual_seed(102)
    c = torch.randn((B, 1, H, 128), device="cuda", dtype=torch.float32, generator=g).to(torch.bfloat16)
    v = c.expand(B, S, H, 128).contiguous()
    print(f"  constant V B{B} H{H} S{S} causal={causal} config={config}", flush=True)
    o, lse = _run(torch, gpu_runner, q, k, v, causal, config)
    assert _same(torch, o, c.expand_as(o)), "O differs from the constant V row"
    assert torch.isfinite(lse).all().item()


@pytest.mark.parametrize("config", [0, 1, 2, 3])
def test_causal_prefix_ignores_later_keys(gpu_runner, config):
    import torch
    q, k, v = _inputs(torch, B, H, S, S, seed=201)
    m = 2048 + 100
    print(f"  causal prefix B{B} H{H} S{S} config={config} rewrite keys >= {m}", flush=True)
    o1, l1 = _run(torch, gpu_runner, q, k, v, True, config)
    k2, v2 = k.clone(), v.clone()
    g = torch.Generator(device="cuda")
    g.manual_seed(202)
    # Larger logits past m make the rows >= m of the shared waves move their base.
    k2[:, m:] = (4 * torch.randn(k2[:, m:].shape, device="cuda", generator=g)).to(torch.bfloat16)
    v2[:, m:] = torch.randn(v2[:, m:].shape, device="cuda", generator=g).to(torch.bfloat16)
    o2, l2 = _run(torch, gpu_runner, q, k2, v2, True, config)
    assert _same(torch, o1[:, :m], o2[:, :m]), "rows before the rewritten keys changed"
    assert _same(torch, l1[:, :, :m], l2[:, :, :m]), "LSE of rows before the rewritten keys changed"
    assert not _same(torch, o1[:, m:], o2[:, m:]), "rows after the rewritten keys did not change"


@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_slices_are_independent(gpu_runner, causal):
    import torch
    q, k, v = _inputs(torch, B, H, S, S, seed=301)
    bb, hh = 17, 5
    print(f"  slice independence B{B} H{H} S{S} causal={causal} rewrite (b={bb}, h={hh})", flush=True)
    o1, l1 = _run(torch, gpu_runner, q, k, v, causal, 0)
    q2, k2, v2 = q.clone(), k.clone(), v.clone()
    g = torch.Generator(device="cuda")
    g.manual_seed(302)
    for x in (q2, k2, v2):
        x[bb, :, hh] = torch.randn(x[bb, :, hh].shape, device="cuda", generator=g).to(torch.bfloat16)
    o2, l2 = _run(torch, gpu_runner, q2, k2, v2, causal, 0)
    keep = torch.ones((B, H), dtype=torch.bool, device="cuda")
    keep[bb, hh] = False
    assert _same(torch, o1.permute(0, 2, 1, 3)[keep], o2.permute(0, 2, 1, 3)[keep])
    assert _same(torch, l1[keep], l2[keep])
    assert not _same(torch, o1[bb, :, hh], o2[bb, :, hh])


@pytest.mark.parametrize("config", [0, 1, 2, 3])
@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_nan_rows_past_the_tails_are_never_used(gpu_runner, causal, config):
    import torch
    s, pad = 4000, 96
    q, k, v = _inputs(torch, B, H, s, s, seed=401)
    print(f"  tails B{B} H{H} {s}x{s} in {s + pad}-row buffers causal={causal} config={config}", flush=True)
    o_ref, l_ref = _run(torch, gpu_runner, q, k, v, causal, config)
    bufs = []
    for x in (q, k, v):
        full = torch.full((B, s + pad, H, 128), float("nan"), device="cuda", dtype=torch.bfloat16)
        full[:, :s] = x
        bufs.append(full)
    o_full = torch.full((B, s + pad, H, 128), 7.0, device="cuda", dtype=torch.bfloat16)
    lse = torch.full((B, H, s), float("nan"), device="cuda", dtype=torch.float32)
    gpu_runner.call_strided(bufs[0][:, :s], bufs[1][:, :s], bufs[2][:, :s], o_full[:, :s], lse, causal, config)
    torch.cuda.synchronize()
    assert torch.isfinite(o_full[:, :s].float()).all().item(), "a NaN row past a tail reached the output"
    assert _same(torch, o_full[:, :s], o_ref)
    assert _same(torch, lse, l_ref)
    assert (o_full[:, s:] == 7.0).all().item(), "rows past sq were written"


# The other entry points, each on one exact property.

def _const_v(torch, b, s, kvh, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    c = torch.randn((b, 1, kvh, 128), device="cuda", dtype=torch.float32, generator=g).to(torch.bfloat16)
    return c, c.expand(b, s, kvh, 128).contiguous()


@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_constant_values_gqa(gpu_runner, causal):
    """B32 H8 with 2 K/V heads, S4096: every query head gets its K/V head's row."""
    import torch
    kvh = 2
    q, _, _ = _inputs(torch, B, H, S, S, seed=501)
    _, k, _ = _inputs(torch, B, kvh, S, S, seed=502)
    c, v = _const_v(torch, B, S, kvh, seed=503)
    print(f"  constant V gqa B{B} H{H} KVH{kvh} S{S} causal={causal}", flush=True)
    o = torch.full_like(q, float("nan"))
    gpu_runner.call_gqa(q, k, v, o, None, causal, 0)
    torch.cuda.synchronize()
    want = c.repeat_interleave(H // kvh, dim=2).expand_as(o)
    assert _same(torch, o, want)


@pytest.mark.parametrize("shape", [(1, 8, 8, 1024, 32768, False), (1, 8, 8, 1024, 32768, True),
                                   (4, 32, 8, 1, 32768, False), (1, 1, 1, 16384, 16384, True)],
                         ids=["prefill_dense", "prefill_causal", "gqa_decode", "single_head_causal"])
def test_constant_values_splitkv(gpu_runner, shape):
    """Split-KV with Auto chunks (the bench's split-KV and decode shapes): the
    FP32 chunk partials and their merge reproduce the constant row exactly."""
    import torch
    b, h, kvh, sq, sk, causal = shape
    q, _, _ = _inputs(torch, b, h, sq, sq, seed=601)
    _, k, _ = _inputs(torch, b, kvh, sk, sk, seed=602)
    c, v = _const_v(torch, b, sk, kvh, seed=603)
    splits = gpu_runner.splitkv_select(b, h, sq, sk, causal, kv_heads=kvh)
    print(f"  constant V split-KV B{b} H{h} KVH{kvh} {sq}x{sk} causal={causal} splits={splits}", flush=True)
    o = torch.full_like(q, float("nan"))
    lse = torch.full((b, h, sq), float("nan"), device="cuda", dtype=torch.float32)
    gpu_runner.call_splitkv(q, k, v, o, lse, causal, 0)
    torch.cuda.synchronize()
    assert _same(torch, o, c.repeat_interleave(h // kvh, dim=2).expand_as(o))
    assert torch.isfinite(lse).all().item()


@pytest.mark.parametrize("causal", [0, 1, 2], ids=["dense", "causal", "bottom_right"])
def test_varlen_sequences_are_independent(gpu_runner, causal):
    """The bench's packed batch (32 sequences of 1237-6743 tokens, H8):
    rewriting one sequence's Q/K/V leaves every other sequence's O and LSE
    bitwise unchanged."""
    import numpy as np
    import torch
    lens = np.random.default_rng(11939).integers(S // 4, 7 * S // 4 + 1, size=B)
    cu_h = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total, maxlen = int(cu_h[-1]), int(lens.max())
    cu = torch.from_numpy(cu_h).cuda()
    g = torch.Generator(device="cuda")
    g.manual_seed(701)
    mk = lambda: torch.randn((total, H, 128), device="cuda", dtype=torch.float32, generator=g).to(torch.bfloat16)
    q, k, v = mk(), mk(), mk()
    sel = 7
    a, e = int(cu_h[sel]), int(cu_h[sel + 1])
    print(f"  varlen independence {B} sequences ({total} tokens) causal={causal} rewrite sequence {sel}", flush=True)

    def run(q, k, v):
        o = torch.full_like(q, float("nan"))
        lse = torch.full((H, total), float("nan"), device="cuda", dtype=torch.float32)
        gpu_runner.call_varlen(q, k, v, o, lse, cu, cu, maxlen, maxlen, causal)
        torch.cuda.synchronize()
        return o, lse

    o1, l1 = run(q, k, v)
    q2, k2, v2 = q.clone(), k.clone(), v.clone()
    for x in (q2, k2, v2):
        x[a:e] = torch.randn(x[a:e].shape, device="cuda", generator=g).to(torch.bfloat16)
    o2, l2 = run(q2, k2, v2)
    keep = torch.ones(total, dtype=torch.bool, device="cuda")
    keep[a:e] = False
    assert _same(torch, o1[keep], o2[keep])
    assert _same(torch, l1[:, keep], l2[:, keep])
    assert not _same(torch, o1[a:e], o2[a:e])


@pytest.mark.parametrize("causal", [0, 2], ids=["dense", "bottom_right"])
def test_constant_values_packed_and_paged_decode(gpu_runner, causal):
    """The bench's continuous-batching decode (32 sequences x 1 query, cache
    lengths 1949-31077, H32 with 8 K/V heads, Auto chunks): with every V row
    of a K/V head equal, every output row is that row, contiguous and from
    64-key pages in random order."""
    import numpy as np
    import torch
    vb, vh, vkvh, ps = 32, 32, 8, 64
    klens = np.random.default_rng(4242).integers(1024, 32768 + 1, size=vb)
    cuk_h = np.concatenate([[0], np.cumsum(klens)]).astype(np.int32)
    tk, maxk = int(cuk_h[-1]), int(klens.max())
    cuq = torch.arange(vb + 1, dtype=torch.int32, device="cuda")
    cuk = torch.from_numpy(cuk_h).cuda()
    g = torch.Generator(device="cuda")
    g.manual_seed(801)
    q = torch.randn((vb, vh, 128), device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn((tk, vkvh, 128), device="cuda", generator=g).to(torch.bfloat16)
    c = torch.randn((1, vkvh, 128), device="cuda", generator=g).to(torch.bfloat16)
    v = c.expand(tk, vkvh, 128).contiguous()
    want = c.repeat_interleave(vh // vkvh, dim=1).expand(vb, vh, 128)
    print(f"  constant V packed decode {vb} sequences, {tk} keys, causal={causal}", flush=True)
    o = torch.full_like(q, float("nan"))
    gpu_runner.call_splitkv_varlen(q, k, v, o, None, cuq, cuk, 1, maxk, causal)
    torch.cuda.synchronize()
    assert _same(torch, o, want), "packed decode"

    npg = [-(-int(n) // ps) for n in klens]
    perm = torch.randperm(sum(npg), generator=torch.Generator().manual_seed(5)).cuda()
    kc = torch.zeros((sum(npg), ps, vkvh, 128), device="cuda", dtype=torch.bfloat16)
    vc = c.expand(sum(npg), ps, vkvh, 128).contiguous()
    table = torch.zeros((vb, max(npg)), device="cuda", dtype=torch.int32)
    at = 0
    for i, n in enumerate(npg):
        ids = perm[at:at + n]
        at += n
        table[i, :n] = ids.to(torch.int32)
        ks, ke = int(cuk_h[i]), int(cuk_h[i + 1])
        pad = torch.zeros((n * ps, vkvh, 128), device="cuda", dtype=torch.bfloat16)
        pad[:ke - ks] = k[ks:ke]
        kc[ids] = pad.view(n, ps, vkvh, 128)
    seqlens = torch.from_numpy(klens.astype(np.int32)).cuda()
    o.fill_(float("nan"))
    gpu_runner.call_splitkv_paged(q, kc, vc, o, None, cuq, seqlens, table, 1, maxk, 0, total_k=tk, causal=causal)
    torch.cuda.synchronize()
    assert _same(torch, o, want), "paged decode"
