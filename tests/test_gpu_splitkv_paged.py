"""GPU checks of split-KV decode over paged K/V caches (fav4_bshd_forward_splitkv_paged) via the C ABI.

Each sequence's keys are scattered over randomly chosen pages of the caches;
the pages no sequence uses hold NaN, and block-table entries past a
sequence's pages hold out-of-range numbers (which the kernel clamps and never
reads through), so a wrong page, slot or head shows up.  Pins:
  * bitwise equality with fav4_bshd_forward_splitkv_varlen on the same keys
    stored contiguously, at the same explicit chunk count (same plan, chunk
    bounds and merge), for page sizes 32, 64 and 256 and MHA / GQA / MQA;
  * every sequence against the FP64 oracle at the reference harness's bar,
    Auto and explicit chunk counts, LSE on and off;
  * a sequence without queries writes nothing, one without keys gets O = 0
    and LSE = -inf, and rows after O / LSE are never written.
"""
import numpy as np
import pytest

from oracle import attention as orc
from tests.conftest import to_device, to_host_bits

pytestmark = pytest.mark.gpu

GUARD = 64
NAN_BF16 = 0x7FC0

# (heads, kv_heads, page_size, [(sq, sk), ...], explicit chunk count)
CASES = [
    (32, 8, 32, [(1, 4096), (1, 100), (1, 1), (1, 9000), (1, 33), (1, 2048)], 7),
    (8, 1, 64, [(16, 3000), (5, 1), (32, 700), (1, 5000)], 5),
    (4, 4, 256, [(3, 300), (32, 4096), (0, 50), (7, 0), (1, 20000)], 16),
    (6, 2, 32, [(32, 32), (31, 64), (17, 1025)], 2),
]


def _build(heads, kv_heads, page_size, lens, seed):
    """Packed Q, contiguous packed K/V, and paged caches holding the same keys."""
    rng = np.random.default_rng(seed)
    qs, ks, vs = [], [], []
    for i, (sq, sk) in enumerate(lens):
        q, _, _ = orc.make_inputs(1, heads, max(sq, 1), max(sk, 1), "normal", seed=seed + 2 * i)
        _, k, v = orc.make_inputs(1, kv_heads, max(sq, 1), max(sk, 1), "normal", seed=seed + 2 * i + 1)
        qs.append(q[0, :sq])
        ks.append(k[0, :sk])
        vs.append(v[0, :sk])
    npages = [-(-sk // page_size) for _, sk in lens]
    max_pages = max(max(npages), 1)
    num_pages = sum(npages) + 7                       # 7 pages nobody uses
    perm = rng.permutation(num_pages)
    kc = np.full((num_pages, page_size, kv_heads, 128), NAN_BF16, dtype=np.uint16)
    vc = np.full_like(kc, NAN_BF16)
    table = rng.choice([-3, num_pages, 1 << 30], size=(len(lens), max_pages)).astype(np.int32)
    nxt = 0
    for i, (_, sk) in enumerate(lens):
        for p in range(npages[i]):
            page = perm[nxt]
            nxt += 1
            table[i, p] = page
            rows = slice(p * page_size, min(sk, (p + 1) * page_size))
            n = rows.stop - rows.start
            kc[page, :n] = ks[i][rows]
            vc[page, :n] = vs[i][rows]
    cu_q = np.concatenate([[0], np.cumsum([s for s, _ in lens])]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum([s for _, s in lens])]).astype(np.int32)
    seqlens_k = np.array([s for _, s in lens], dtype=np.int32)
    return (np.concatenate(qs), np.concatenate(ks), np.concatenate(vs), kc, vc, cu_q, cu_k, seqlens_k, table)


def _out(torch, dev, tq, h, with_lse):
    o_buf = torch.full((tq + GUARD, h, 128), float("nan"), device=dev, dtype=torch.bfloat16)
    l_buf = torch.full((h * tq + GUARD,), float("nan"), device=dev, dtype=torch.float32)
    return o_buf, l_buf, o_buf[:tq], (l_buf[:h * tq].view(h, tq) if with_lse else None)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "h%dkv%d_p%d_n%d" % (c[0], c[1], c[2], len(c[3])))
def test_splitkv_paged(gpu_runner, case):
    import torch
    h, kvh, ps, lens, splits = case
    q, k, v, kc, vc, cu_q, cu_k, seqlens_k, table = _build(h, kvh, ps, lens, seed=17)
    dev = torch.device("cuda:0")
    qd, kd, vd, kcd, vcd = (to_device(x, dev) for x in (q, k, v, kc, vc))
    cq, ck, sk_d, tb = (torch.from_numpy(x).to(dev) for x in (cu_q, cu_k, seqlens_k, table))
    max_q = max(s for s, _ in lens)
    max_k = max(s for _, s in lens)
    tq, group = len(q), h // kvh
    print(f"  splitkv paged H{h} KVH{kvh} page {ps} lens={lens} splits={splits}", flush=True)

    # bitwise against the contiguous packed split-KV at the same chunk count
    ob, lb, o, lse = _out(torch, dev, tq, h, True)
    gpu_runner.call_splitkv_paged(qd, kcd, vcd, o, lse, cq, sk_d, tb, max_q, max_k, splits, total_k=len(k))
    ob2, lb2, o2, lse2 = _out(torch, dev, tq, h, True)
    gpu_runner.call_splitkv_varlen(qd, kd, vd, o2, lse2, cq, ck, max_q, max_k, False, splits)
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int16), o2.view(torch.int16))
    assert torch.equal(lse.view(torch.int32), lse2.view(torch.int32))
    assert torch.isnan(ob[tq:]).all().item() and torch.isnan(lb[h * tq:]).all().item()

    # Auto, LSE off, against the oracle (and the explicit run's empty rows)
    ob3, lb3, o3, _ = _out(torch, dev, tq, h, False)
    gpu_runner.call_splitkv_paged(qd, kcd, vcd, o3, None, cq, sk_d, tb, max_q, max_k, 0, total_k=len(k))
    torch.cuda.synchronize()
    assert torch.isnan(ob3[tq:]).all().item() and torch.isnan(lb3).all().item()
    for i, (sq, sk) in enumerate(lens):
        a, b = cu_q[i], cu_q[i + 1]
        c, d = cu_k[i], cu_k[i + 1]
        if sq == 0:
            continue
        if sk == 0:
            assert (o[a:b].float() == 0).all().item() and (o3[a:b].float() == 0).all().item(), i
            assert torch.isneginf(lse[:, a:b]).all().item(), i
            continue
        ke = np.repeat(k[c:d][None], group, axis=2)
        ve = np.repeat(v[c:d][None], group, axis=2)
        ref, ref_lse = orc.attention_fp64(q[a:b][None], ke, ve, orc.DEFAULT_SCALE, False)
        e = orc.errors(to_host_bits(o[a:b])[None], lse[:, a:b].cpu().numpy()[None], ref, ref_lse)
        assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), (i, sq, sk, e)
        e3 = orc.errors(to_host_bits(o3[a:b])[None], None, ref, None)
        assert orc.check_acceptance_tolerance(e3) and orc.check_reference_tolerance(e3), ("auto", i, e3)


def test_splitkv_paged_single_chunk_and_long_cache(gpu_runner):
    """One chunk (max_seqlen_k <= 64 key tiles: still the split kernels and the
    merge), and a cache long enough that the 64-tile chunk cap raises an
    explicit count of 2 (2188 key tiles -> 35 chunks)."""
    import torch
    h, kvh, ps = 16, 4, 128
    dev = torch.device("cuda:0")
    group = h // kvh
    for lens, max_k, splits, want in (([(2, 2048), (1, 700), (3, 0)], 2048, 1, 1),
                                      ([(2, 70000), (1, 5000)], 70000, 2, 35)):
        q, k, v, kc, vc, cu_q, cu_k, seqlens_k, table = _build(h, kvh, ps, lens, seed=23)
        qd, kcd, vcd = (to_device(x, dev) for x in (q, kc, vc))
        cq, sk_d, tb = (torch.from_numpy(x).to(dev) for x in (cu_q, seqlens_k, table))
        max_q = max(s for s, _ in lens)
        need = gpu_runner.splitkv_paged_workspace_size(len(lens), h, kvh, max_q, max_k, len(q), len(k), ps,
                                                       table.shape[1], len(kc), splits)
        assert need == want * len(lens) * h * max_q * 520, (lens, need)
        print(f"  splitkv paged lens={lens} splits={splits} -> {want} chunks", flush=True)
        ob, lb, o, lse = _out(torch, dev, len(q), h, True)
        gpu_runner.call_splitkv_paged(qd, kcd, vcd, o, lse, cq, sk_d, tb, max_q, max_k, splits)
        torch.cuda.synchronize()
        assert torch.isnan(ob[len(q):]).all().item() and torch.isnan(lb[h * len(q):]).all().item()
        for i, (sq, sk) in enumerate(lens):
            a, b = cu_q[i], cu_q[i + 1]
            c, d = cu_k[i], cu_k[i + 1]
            if sk == 0:
                assert (o[a:b].float() == 0).all().item() and torch.isneginf(lse[:, a:b]).all().item(), i
                continue
            ke = np.repeat(k[c:d][None], group, axis=2)
            ve = np.repeat(v[c:d][None], group, axis=2)
            ref, ref_lse = orc.attention_fp64(q[a:b][None], ke, ve, orc.DEFAULT_SCALE, False)
            e = orc.errors(to_host_bits(o[a:b])[None], lse[:, a:b].cpu().numpy()[None], ref, ref_lse)
            assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), (splits, i, e)


def _draw(rng):
    kvh = int(rng.choice([1, 2, 4]))
    group = int(rng.choice([1, 2, 4, 8]))
    b = int(rng.integers(1, 7))
    sq_max = int(rng.choice([1, 4, 32]))
    lens = [(int(rng.integers(0, sq_max + 1)), int(rng.integers(0, 6000))) for _ in range(b)]
    lens[0] = (max(lens[0][0], 1), max(lens[0][1], 40))        # at least one row with keys past one tile
    return dict(h=kvh * group, kvh=kvh, ps=int(rng.choice([32, 64, 128, 512])), lens=lens,
                splits=int(rng.choice([2, 3, 8, 33, 200])), lse=bool(rng.integers(0, 2)))


RANDOM = [_draw(np.random.default_rng(500 + i)) for i in range(12)]


@pytest.mark.parametrize("case", RANDOM, ids=lambda c: "h%dkv%d_p%d_b%d_s%d" % (c["h"], c["kvh"], c["ps"],
                                                                                len(c["lens"]), c["splits"]))
def test_splitkv_paged_random(gpu_runner, case):
    """Seeded random batches: bitwise the contiguous packed split-KV at the same
    explicit chunk count, and the FP64 oracle on every sequence."""
    import torch
    h, kvh, ps, lens, splits, with_lse = case["h"], case["kvh"], case["ps"], case["lens"], case["splits"], case["lse"]
    q, k, v, kc, vc, cu_q, cu_k, seqlens_k, table = _build(h, kvh, ps, lens, seed=31)
    dev = torch.device("cuda:0")
    qd, kd, vd, kcd, vcd = (to_device(x, dev) for x in (q, k, v, kc, vc))
    cq, ck, sk_d, tb = (torch.from_numpy(x).to(dev) for x in (cu_q, cu_k, seqlens_k, table))
    max_q = max(s for s, _ in lens)
    max_k = max(s for _, s in lens)
    tq, group = len(q), h // kvh
    print(f"  splitkv paged random H{h} KVH{kvh} page {ps} lens={lens} splits={splits}", flush=True)
    ob, lb, o, lse = _out(torch, dev, tq, h, with_lse)
    gpu_runner.call_splitkv_paged(qd, kcd, vcd, o, lse, cq, sk_d, tb, max_q, max_k, splits, total_k=len(k))
    torch.cuda.synchronize()
    assert torch.isnan(ob[tq:]).all().item() and torch.isnan(lb[h * tq:]).all().item()
    # Same plan (the paged one caps chunks at 64 key tiles, which only ever
    # raises the count): same workspace size.
    ws_v = gpu_runner.splitkv_varlen_workspace_size(len(lens), h, kvh, max_q, max_k, tq, len(k), False, splits)
    ws_p = gpu_runner.splitkv_paged_workspace_size(len(lens), h, kvh, max_q, max_k, tq, len(k), ps, table.shape[1],
                                                   len(kc), splits)
    if ws_v == ws_p:
        _, _, o2, lse2 = _out(torch, dev, tq, h, with_lse)
        gpu_runner.call_splitkv_varlen(qd, kd, vd, o2, lse2, cq, ck, max_q, max_k, False, splits)
        torch.cuda.synchronize()
        assert torch.equal(o.view(torch.int16), o2.view(torch.int16))
        if with_lse:
            assert torch.equal(lse.view(torch.int32), lse2.view(torch.int32))
    for i, (sq, sk) in enumerate(lens):
        a, b = cu_q[i], cu_q[i + 1]
        c, d = cu_k[i], cu_k[i + 1]
        if sq == 0:
            continue
        if sk == 0:
            assert (o[a:b].float() == 0).all().item(), i
            continue
        ke = np.repeat(k[c:d][None], group, axis=2)
        ve = np.repeat(v[c:d][None], group, axis=2)
        ref, ref_lse = orc.attention_fp64(q[a:b][None], ke, ve, orc.DEFAULT_SCALE, False)
        got_lse = lse[:, a:b].cpu().numpy()[None] if with_lse else None
        e = orc.errors(to_host_bits(o[a:b])[None], got_lse, ref, ref_lse if with_lse else None)
        assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), (i, sq, sk, e)


def _bottom_right_ref(q, k, v, group):
    """FP64 bottom-right causal (query i sees keys j <= sk - sq + i) from the
    top-left oracle: queries padded in front to sk rows when sq <= sk, else
    the rows that see keys are the last sk, top-left against all keys."""
    sq, sk = len(q), len(k)
    ke = np.repeat(k[None], group, axis=2)
    ve = np.repeat(v[None], group, axis=2)
    h = q.shape[1]
    o = np.zeros((1, sq, h, 128))
    lse = np.full((1, h, sq), -np.inf)
    if sk == 0:
        return o, lse
    if sq <= sk:
        qp = np.concatenate([np.zeros((sk - sq,) + q.shape[1:], dtype=q.dtype), q])[None]
        ref, ref_lse = orc.attention_fp64(qp, ke, ve, orc.DEFAULT_SCALE, True)
        return ref[:, sk - sq:], ref_lse[:, :, sk - sq:]
    ref, ref_lse = orc.attention_fp64(q[sq - sk:][None], ke, ve, orc.DEFAULT_SCALE, True)
    o[:, sq - sk:] = ref
    lse[:, :, sq - sk:] = ref_lse
    return o, lse


@pytest.mark.parametrize("ps", [32, 128])
def test_splitkv_bottom_right_causal(gpu_runner, ps):
    """causal = 2 on the packed and the paged decode calls: the FP64 oracle
    (bottom-right, including sequences with more queries than keys, whose
    first rows see no key), and paged bitwise the packed call at the same
    chunk count."""
    import torch
    h, kvh = 8, 2
    lens = [(4, 3000), (1, 700), (32, 5000), (17, 17), (20, 9), (5, 0), (0, 40), (32, 65)]
    q, k, v, kc, vc, cu_q, cu_k, seqlens_k, table = _build(h, kvh, ps, lens, seed=41)
    dev = torch.device("cuda:0")
    qd, kd, vd, kcd, vcd = (to_device(x, dev) for x in (q, k, v, kc, vc))
    cq, ck, sk_d, tb = (torch.from_numpy(x).to(dev) for x in (cu_q, cu_k, seqlens_k, table))
    max_q, max_k, tq, group = 32, 5000, len(q), h // kvh
    for splits in (0, 1, 6):
        print(f"  bottom-right causal page {ps} splits={splits}", flush=True)
        ob, lb, o, lse = _out(torch, dev, tq, h, True)
        gpu_runner.call_splitkv_varlen(qd, kd, vd, o, lse, cq, ck, max_q, max_k, 2, splits)
        ob2, lb2, o2, lse2 = _out(torch, dev, tq, h, True)
        gpu_runner.call_splitkv_paged(qd, kcd, vcd, o2, lse2, cq, sk_d, tb, max_q, max_k, splits, total_k=len(k),
                                      causal=2)
        torch.cuda.synchronize()
        assert torch.isnan(ob[tq:]).all().item() and torch.isnan(lb[h * tq:]).all().item()
        assert torch.isnan(ob2[tq:]).all().item() and torch.isnan(lb2[h * tq:]).all().item()
        ws_v = gpu_runner.splitkv_varlen_workspace_size(len(lens), h, kvh, max_q, max_k, tq, len(k), 2, splits)
        ws_p = gpu_runner.splitkv_paged_workspace_size(len(lens), h, kvh, max_q, max_k, tq, len(k), ps,
                                                       table.shape[1], len(kc), splits, causal=2)
        if ws_v == ws_p:      # same plan (one explicit chunk over 157 key tiles: the paged cap makes 3)
            assert torch.equal(o.view(torch.int16), o2.view(torch.int16)), splits
            assert torch.equal(lse.view(torch.int32), lse2.view(torch.int32)), splits
        for out_o, out_lse in ((o, lse), (o2, lse2)):
            _check_bottom_right(out_o, out_lse, q, k, v, cu_q, cu_k, lens, group, splits)


def _check_bottom_right(o, lse, q, k, v, cu_q, cu_k, lens, group, splits):
    """Every sequence of a bottom-right causal output against the FP64 reference."""
    for i, (sq, sk) in enumerate(lens):
        a, b = cu_q[i], cu_q[i + 1]
        c, d = cu_k[i], cu_k[i + 1]
        if sq == 0:
            continue
        ref, ref_lse = _bottom_right_ref(q[a:b], k[c:d], v[c:d], group)
        got, got_lse = to_host_bits(o[a:b])[None], lse[:, a:b].cpu().numpy()[None]
        seen = np.isfinite(ref_lse[0, 0])                       # rows that see at least one key
        assert (got_lse[:, :, ~seen] == -np.inf).all() and (orc.bf16_to_f32(got[:, ~seen]) == 0).all(), i
        if seen.any():
            e = orc.errors(got[:, seen], got_lse[:, :, seen], ref[:, seen], ref_lse[:, :, seen])
            assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), (splits, i, e)


@pytest.mark.parametrize("ps", [64, 256])
def test_splitkv_paged_prefill(gpu_runner, ps):
    """Queries longer than 32 over paged caches (the 8-wave shape): dense and
    bottom-right causal against the FP64 oracle on ragged batches (several q
    tiles, q tiles past short sequences, sq > sk), and a uniform batch bitwise
    the contiguous split-KV at the same chunk count."""
    import torch
    h, kvh = 8, 2
    group = h // kvh
    dev = torch.device("cuda:0")
    lens = [(600, 3000), (33, 700), (300, 300), (64, 20), (0, 100), (1, 4100)]
    q, k, v, kc, vc, cu_q, cu_k, seqlens_k, table = _build(h, kvh, ps, lens, seed=61)
    qd, kcd, vcd = (to_device(x, dev) for x in (q, kc, vc))
    cq, sk_d, tb = (torch.from_numpy(x).to(dev) for x in (cu_q, seqlens_k, table))
    max_q, max_k, tq = 600, 4100, len(q)
    for causal, splits in ((0, 0), (0, 5), (2, 0), (2, 3)):
        print(f"  paged prefill page {ps} causal={causal} splits={splits}", flush=True)
        ob, lb, o, lse = _out(torch, dev, tq, h, True)
        gpu_runner.call_splitkv_paged(qd, kcd, vcd, o, lse, cq, sk_d, tb, max_q, max_k, splits, total_k=len(k),
                                      causal=causal)
        torch.cuda.synchronize()
        assert torch.isnan(ob[tq:]).all().item() and torch.isnan(lb[h * tq:]).all().item()
        if causal == 2:
            _check_bottom_right(o, lse, q, k, v, cu_q, cu_k, lens, group, splits)
            # the contiguous packed call: the same rows, bitwise when the plans agree
            kd, vd = to_device(k, dev), to_device(v, dev)
            _, _, o2, lse2 = _out(torch, dev, tq, h, True)
            gpu_runner.call_splitkv_varlen(qd, kd, vd, o2, lse2, cq, torch.from_numpy(cu_k).to(dev), max_q, max_k,
                                           2, splits)
            torch.cuda.synchronize()
            _check_bottom_right(o2, lse2, q, k, v, cu_q, cu_k, lens, group, splits)
            ws_v = gpu_runner.splitkv_varlen_workspace_size(len(lens), h, kvh, max_q, max_k, tq, len(k), 2, splits)
            ws_p = gpu_runner.splitkv_paged_workspace_size(len(lens), h, kvh, max_q, max_k, tq, len(k), ps,
                                                           table.shape[1], len(kc), splits, causal=2)
            if ws_v == ws_p:
                assert torch.equal(o.view(torch.int16), o2.view(torch.int16)), splits
                assert torch.equal(lse.view(torch.int32), lse2.view(torch.int32)), splits
            continue
        for i, (sq, sk) in enumerate(lens):
            a, b = cu_q[i], cu_q[i + 1]
            c, d = cu_k[i], cu_k[i + 1]
            if sq == 0:
                continue
            ke = np.repeat(k[c:d][None], group, axis=2)
            ve = np.repeat(v[c:d][None], group, axis=2)
            ref, ref_lse = orc.attention_fp64(q[a:b][None], ke, ve, orc.DEFAULT_SCALE, False)
            e = orc.errors(to_host_bits(o[a:b])[None], lse[:, a:b].cpu().numpy()[None], ref, ref_lse)
            assert orc.check_acceptance_tolerance(e) and orc.check_reference_tolerance(e), (splits, i, e)

    # uniform batch: bitwise the contiguous (BSHD) split-KV at the same chunk count
    b, sq, sk, splits = 3, 300, 2500, 4
    q, k, v, kc, vc, cu_q, cu_k, seqlens_k, table = _build(h, kvh, ps, [(sq, sk)] * b, seed=62)
    qd, kd, vd, kcd, vcd = (to_device(x, dev) for x in (q, k, v, kc, vc))
    cq, sk_d, tb = (torch.from_numpy(x).to(dev) for x in (cu_q, seqlens_k, table))
    _, _, o, lse = _out(torch, dev, b * sq, h, True)
    gpu_runner.call_splitkv_paged(qd, kcd, vcd, o, lse, cq, sk_d, tb, sq, sk, splits, total_k=b * sk)
    oc = torch.full((b, sq, h, 128), float("nan"), device=dev, dtype=torch.bfloat16)
    lc = torch.full((b, h, sq), float("nan"), device=dev, dtype=torch.float32)
    gpu_runner.call_splitkv(qd.view(b, sq, h, 128), kd.view(b, sk, kvh, 128), vd.view(b, sk, kvh, 128), oc, lc,
                            False, splits)
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int16), oc.view(-1, h, 128).view(torch.int16))
    assert torch.equal(lse.view(torch.int32), lc.permute(1, 0, 2).reshape(h, b * sq).view(torch.int32))


def test_splitkv_paged_presized_workspace_bottom_right(gpu_runner):
    """A caller that sizes the workspace with the helper for the mask it will
    use (as for graph capture) and passes exactly that buffer: the bottom-right
    plan of B1 H8 Sq=Sk=4096 has more chunks than the dense one, so a
    dense-sized buffer would be rejected.  The call succeeds and matches the
    call that allocates its own workspace, bitwise."""
    import torch
    h, kvh, ps = 8, 8, 64
    dev = torch.device("cuda:0")
    lens = [(4096, 4096)]
    q, k, v, kc, vc, cu_q, cu_k, seqlens_k, table = _build(h, kvh, ps, lens, seed=71)
    qd, kcd, vcd = (to_device(x, dev) for x in (q, kc, vc))
    cq, sk_d, tb = (torch.from_numpy(x).to(dev) for x in (cu_q, seqlens_k, table))
    args = (1, h, kvh, 4096, 4096, len(q), len(k), ps, table.shape[1], len(kc))
    need_dense = gpu_runner.splitkv_paged_workspace_size(*args, 0, causal=0)
    need_br = gpu_runner.splitkv_paged_workspace_size(*args, 0, causal=2)
    print(f"  workspace dense {need_dense} B, bottom-right {need_br} B", flush=True)
    ws = torch.empty(need_br, device=dev, dtype=torch.uint8)
    _, _, o, lse = _out(torch, dev, len(q), h, True)
    gpu_runner.call_splitkv_paged(qd, kcd, vcd, o, lse, cq, sk_d, tb, 4096, 4096, 0, workspace=ws, total_k=len(k),
                                  causal=2)
    _, _, o2, lse2 = _out(torch, dev, len(q), h, True)
    gpu_runner.call_splitkv_paged(qd, kcd, vcd, o2, lse2, cq, sk_d, tb, 4096, 4096, 0, total_k=len(k), causal=2)
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int16), o2.view(torch.int16))
    assert torch.equal(lse.view(torch.int32), lse2.view(torch.int32))
