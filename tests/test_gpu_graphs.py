"""HIP-graph capture of every entry point (via torch.cuda.CUDAGraph).

Serving loops capture the forward once and replay it.  Each entry point is
captured on a side stream, then replayed three times with unrelated eager work
(other launches of the library, a NaN refill of the outputs) between the
replays; every replay must reproduce the eager result bitwise.  The library
records only kernel launches (no memset or copy nodes), so the replays are
pure kernel graphs.
"""
import pytest

pytestmark = pytest.mark.gpu


def _inputs(torch, b, h, sq, sk, kvh=None, seed=3):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    mk = lambda s, hh: torch.randn((b, s, hh, 128), device="cuda", dtype=torch.float32, generator=g).to(torch.bfloat16)
    return mk(sq, h), mk(sk, kvh or h), mk(sk, kvh or h)


def _check_graph(torch, run, outs, noise):
    """run(): enqueue the call on the current stream writing `outs`.  Eager result
    first, then capture, then 3 replays separated by eager noise."""
    for x in outs:
        x.fill_(float("nan"))
    run()
    torch.cuda.synchronize()
    ref = [x.clone() for x in outs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        run()                       # warm-up on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            run()
    torch.cuda.synchronize()
    for rep in range(3):
        for x in outs:
            x.fill_(float("nan"))
        noise()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for x, r in zip(outs, ref):
            same = torch.equal(x.view(torch.int32) if x.dtype == torch.float32 else x.view(torch.int16),
                               r.view(torch.int32) if r.dtype == torch.float32 else r.view(torch.int16))
            assert same, f"replay {rep} differs"
    del graph


@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_graph_forward_and_gqa(gpu_runner, causal):
    import torch
    q, k, v = _inputs(torch, 2, 8, 1000, 1500)
    _, kg, vg = _inputs(torch, 2, 8, 1000, 1500, kvh=2, seed=4)
    o = torch.empty_like(q)
    og = torch.empty_like(q)
    lse = torch.empty((2, 8, 1000), device="cuda", dtype=torch.float32)
    on = torch.empty_like(q)
    noise = lambda: gpu_runner.call(k[:, :1000].contiguous(), q, q, on, None, not causal, 1)
    print(f"  graph forward causal={causal}", flush=True)
    _check_graph(torch, lambda: gpu_runner.call(q, k, v, o, lse, causal, 0), [o, lse], noise)
    print(f"  graph gqa causal={causal}", flush=True)
    _check_graph(torch, lambda: gpu_runner.call_gqa(q, kg, vg, og, None, causal, 0), [og], noise)


@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_graph_splitkv(gpu_runner, causal):
    import torch
    q, k, v = _inputs(torch, 1, 4, 300, 9000)
    o = torch.empty_like(q)
    lse = torch.empty((1, 4, 300), device="cuda", dtype=torch.float32)
    need = gpu_runner.splitkv_workspace_size(1, 4, 300, 9000, causal, 6)
    ws = torch.empty(max(need, 256), device="cuda", dtype=torch.uint8)
    on = torch.empty_like(q)
    # the noise reuses the same workspace with another split count between replays
    noise = lambda: gpu_runner.call_splitkv(q, k, v, on, None, causal, 3, workspace=ws)
    print(f"  graph splitkv causal={causal}", flush=True)
    _check_graph(torch, lambda: gpu_runner.call_splitkv(q, k, v, o, lse, causal, 6, workspace=ws), [o, lse], noise)


def test_graph_splitkv_gqa_decode(gpu_runner):
    """The packed GQA decode (one-wave partial kernel + grouped merge)."""
    import torch
    q, _, _ = _inputs(torch, 2, 16, 3, 5000)
    _, k, v = _inputs(torch, 2, 16, 3, 5000, kvh=4, seed=7)
    o = torch.empty_like(q)
    lse = torch.empty((2, 16, 3), device="cuda", dtype=torch.float32)
    need = gpu_runner.splitkv_workspace_size(2, 16, 3, 5000, False, 40, kv_heads=4)
    ws = torch.empty(max(need, 256), device="cuda", dtype=torch.uint8)
    on = torch.empty_like(q)
    noise = lambda: gpu_runner.call_splitkv(q, k, v, on, None, False, 9, workspace=ws)
    print("  graph splitkv gqa decode", flush=True)
    _check_graph(torch, lambda: gpu_runner.call_splitkv(q, k, v, o, lse, False, 40, workspace=ws), [o, lse], noise)


@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
def test_graph_varlen_and_strided(gpu_runner, causal):
    import torch
    h = 4
    lens = [700, 33, 1500, 256]
    cu = torch.tensor([0, 700, 733, 2233, 2489], device="cuda", dtype=torch.int32)
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    mk = lambda: torch.randn((2489, h, 128), device="cuda", generator=g).to(torch.bfloat16)
    q, k, v = mk(), mk(), mk()
    o = torch.empty_like(q)
    lse = torch.empty((h, 2489), device="cuda", dtype=torch.float32)
    qb, kb, vb = _inputs(torch, 2, h, 600, 900, seed=10)
    ob = torch.empty((2, h, 600, 128), device="cuda", dtype=torch.bfloat16)        # BHSD output
    on = torch.empty_like(qb)
    noise = lambda: gpu_runner.call(qb, kb, vb, on, None, causal, 2)
    print(f"  graph varlen causal={causal}", flush=True)
    _check_graph(torch, lambda: gpu_runner.call_varlen(q, k, v, o, lse, cu, cu, max(lens), max(lens), causal),
                 [o, lse], noise)
    print(f"  graph strided causal={causal}", flush=True)
    _check_graph(torch, lambda: gpu_runner.call_strided(qb, kb, vb, ob.transpose(1, 2), None, causal, 0), [ob],
                 noise)



def test_graph_paged_decode_bottom_right(gpu_runner):
    """Split-KV decode over paged caches with the bottom-right mask: the page
    lookup and both kernels replay to the eager result."""
    import numpy as np
    import torch
    from tests.conftest import to_device
    from tests.test_gpu_splitkv_paged import _build
    h, kvh, ps = 16, 4, 64
    lens = [(3, 2500), (1, 700), (8, 4100), (2, 0)]
    q, k, _, kc, vc, cu_q, _, seqlens_k, table = _build(h, kvh, ps, lens, seed=51)
    dev = torch.device("cuda:0")
    qd, kcd, vcd = (to_device(x, dev) for x in (q, kc, vc))
    cq, sk_d, tb = (torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in (cu_q, seqlens_k, table))
    o = torch.empty_like(qd)
    lse = torch.empty((h, len(q)), device="cuda", dtype=torch.float32)
    on = torch.empty_like(qd)
    need = max(gpu_runner.splitkv_paged_workspace_size(len(lens), h, kvh, 8, 4100, len(q), len(k), ps,
                                                       table.shape[1], len(kc), s) for s in (7, 3))
    ws = torch.empty(need, device="cuda", dtype=torch.uint8)

    def call(out, out_lse, splits):
        gpu_runner.call_splitkv_paged(qd, kcd, vcd, out, out_lse, cq, sk_d, tb, 8, 4100, splits, workspace=ws,
                                      total_k=len(k), causal=2)

    print("  graph paged decode bottom-right", flush=True)
    _check_graph(torch, lambda: call(o, lse, 7), [o, lse], lambda: call(on, None, 3))
