"""fav4_bshd_forward_splitkv_gqa_noalloc against fav4_bshd_forward_splitkv_gqa.

The no-workspace entry point runs the same plan and kernels as the workspace
one, with the chunk partials in the library's own per-device array, so on the
same inputs and chunk count O and LSE must be bitwise equal.  Each case makes
two calls in a row, the second on a smaller problem (the array keeps the first
call's partials, which must not leak into the second), and checks both.
"""
import pytest

from oracle import attention as orc
from tests.conftest import to_host_bits

pytestmark = pytest.mark.gpu

# (label, [(B, H, KVH, Sq, Sk, causal, splits), smaller second call])
CASES = [
    ("decode_gqa", [(4, 32, 8, 1, 32768, False, 0), (2, 16, 4, 1, 5000, False, 0)]),
    ("prefill_mha", [(1, 8, 8, 1024, 32768, False, 0), (1, 4, 4, 300, 4100, False, 3)]),
    ("prefill_causal", [(2, 4, 2, 2048, 2048, True, 4), (1, 2, 1, 700, 900, True, 2)]),
]


def _inputs(torch, dev, b, h, kvh, sq, sk, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    mk = lambda *s: torch.randn(s, device=dev, dtype=torch.float32, generator=g).to(torch.bfloat16)
    return mk(b, sq, h, 128), mk(b, sk, kvh, 128), mk(b, sk, kvh, 128)


@pytest.mark.parametrize("label,calls", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_workspace_call(gpu_runner, label, calls):
    import torch
    dev = torch.device("cuda:0")
    for i, (b, h, kvh, sq, sk, causal, splits) in enumerate(calls):
        print(f"{label} call {i}: B{b} H{h} KVH{kvh} Sq{sq} Sk{sk} causal={causal} splits={splits}", flush=True)
        q, k, v = _inputs(torch, dev, b, h, kvh, sq, sk, 100 + i)
        need = gpu_runner.splitkv_workspace_size(b, h, sq, sk, causal, splits, kv_heads=kvh)
        assert 0 < need <= 64 << 20, need            # the case exercises the array
        outs = []
        for noalloc in (False, True):
            o = torch.full_like(q, float("nan"))
            lse = torch.full((b, h, sq), float("nan"), device=dev, dtype=torch.float32)
            if noalloc:
                gpu_runner.call_splitkv_noalloc(q, k, v, o, lse, causal, splits)
            else:
                gpu_runner.call_splitkv(q, k, v, o, lse, causal, splits)
            torch.cuda.synchronize()
            outs.append((o, lse))
        (o0, l0), (o1, l1) = outs
        assert torch.equal(o0.view(torch.int16), o1.view(torch.int16)), (label, i)
        assert torch.equal(l0.view(torch.int32), l1.view(torch.int32)), (label, i)
        # and the result itself is right, on the reference's sampled rows of two (b, h) slices
        pairs = [(0, 0), (b - 1, h - 1)]
        rows = orc.sample_rows(sq)
        grp = h // kvh
        qh, kh, vh = (to_host_bits(x) for x in (q, k.repeat_interleave(grp, dim=2), v.repeat_interleave(grp, dim=2)))
        ref, ref_lse = orc.attention_fp64(qh, kh, vh, orc.DEFAULT_SCALE, causal, rows=rows, heads=pairs)
        got, lse_h = to_host_bits(o1)[:, rows], l1.cpu().numpy()[:, :, rows]
        for bb, hh in pairs:
            e = orc.errors(got[bb:bb + 1, :, hh:hh + 1], lse_h[bb:bb + 1, hh:hh + 1],
                           ref[bb:bb + 1, :, hh:hh + 1], ref_lse[bb:bb + 1, hh:hh + 1])
            assert orc.check_acceptance_tolerance(e), (label, i, bb, hh, e)


_CAPTURE_SCRIPT = r"""
import sys
sys.path.insert(0, sys.argv[1])
import torch
import __graft_entry__
pkg = __graft_entry__.import_package()
r = pkg.Runner()
dev = torch.device("cuda:0")
g = torch.Generator(device=dev)
g.manual_seed(7)
mk = lambda *s: torch.randn(s, device=dev, dtype=torch.float32, generator=g).to(torch.bfloat16)
b, h, kvh, sq, sk, causal, splits = 2, 16, 4, 1, 9000, False, 0
q, k, v = mk(b, sq, h, 128), mk(b, sk, kvh, 128), mk(b, sk, kvh, 128)
# eager workspace call first (loads the library's code object), then the
# process's first no-alloc call inside a capture
ref_o = torch.full_like(q, float("nan"))
ref_l = torch.full((b, h, sq), float("nan"), device=dev, dtype=torch.float32)
r.call_splitkv(q, k, v, ref_o, ref_l, causal, splits)
torch.cuda.synchronize()
o = torch.full_like(q, float("nan"))
lse = torch.full((b, h, sq), float("nan"), device=dev, dtype=torch.float32)
s = torch.cuda.Stream()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=s):
    r.call_splitkv_noalloc(q, k, v, o, lse, causal, splits, stream=s.cuda_stream)
for rep in range(3):
    o.fill_(float("nan"))
    lse.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    same = torch.equal(o.view(torch.int16), ref_o.view(torch.int16)) and \
        torch.equal(lse.view(torch.int32), ref_l.view(torch.int32))
    print(f"replay {rep}: bitwise equal to the workspace call: {same}", flush=True)
    if not same:
        sys.exit(3)
    # eager work between replays, on the same array
    o2 = torch.empty_like(q)
    r.call_splitkv_noalloc(q, k, v, o2, None, causal, splits)
    torch.cuda.synchronize()
    if not torch.equal(o2.view(torch.int16), ref_o.view(torch.int16)):
        sys.exit(4)
print("ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture():
    """In a fresh process, the first no-alloc call (the one that looks up the
    per-device array's address) is made while a stream is being captured; the
    graph is replayed three times, with eager no-alloc calls in between, and
    every replay is bitwise the workspace call."""
    import subprocess
    import sys
    from tests.conftest import ROOT
    r = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, str(ROOT)], capture_output=True, text=True,
                       timeout=180)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.returncode
