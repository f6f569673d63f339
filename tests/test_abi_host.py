"""Host-only checks of the C ABI (no GPU needed, no compute call is made).

The library must export the two entry points of the reference header
(include/fav4_bshd.h:19-20) plus the split-KV, GQA, varlen and strided additions, lay
out Fav4Args byte for byte like the reference (include/fav4_bshd.h:4-10), and
reject bad arguments with hipErrorInvalidValue before touching HIP, as
src/bshd.hip:27-34 does.  The split-KV size / plan queries are checked
against their closed forms.
"""
import ctypes as C
import math
import shutil
import subprocess
from pathlib import Path

import pytest

from tests.conftest import ROOT, load_package

HIP_ERROR_INVALID_VALUE = 1
HEADER = ROOT / "include" / "fav4_bshd.h"

# Offsets of the reference argument block (5 pointers, 4 ints, 1 float).
LAYOUT = dict(q=0, k=8, v=16, o=24, lse=32, batch=40, heads=44, sq=48, sk=52, scale=56)


@pytest.fixture(scope="module")
def lib():
    pkg = load_package()
    if not pkg.LIB_PATH.exists():
        pkg.build_library()
    return pkg.load_library()


@pytest.fixture(scope="module")
def Args():
    return load_package().Args


def test_exports_exactly_the_c_abi():
    pkg = load_package()
    if not pkg.LIB_PATH.exists():
        pkg.build_library()
    out = subprocess.run(["nm", "-D", "--defined-only", str(pkg.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    names = {line.split()[-1] for line in out.splitlines() if line.strip()}
    public = {n for n in names if not n.startswith("_")}
    assert public == {"fav4_bshd_forward", "fav4_bshd_select_config", "fav4_bshd_forward_splitkv",
                      "fav4_bshd_splitkv_workspace_size", "fav4_bshd_splitkv_select", "fav4_bshd_forward_gqa",
                      "fav4_bshd_forward_varlen", "fav4_bshd_forward_strided", "fav4_bshd_forward_splitkv_gqa",
                      "fav4_bshd_splitkv_gqa_workspace_size", "fav4_bshd_splitkv_gqa_select",
                      "fav4_bshd_forward_splitkv_varlen", "fav4_bshd_splitkv_varlen_workspace_size",
                      "fav4_bshd_splitkv_varlen_select", "fav4_bshd_forward_splitkv_paged",
                      "fav4_bshd_splitkv_paged_workspace_size", "fav4_bshd_splitkv_paged_select",
                      "fav4_bshd_forward_splitkv_gqa_noalloc", "fav4_bshd_select_config_masked"}, public


def test_ctypes_layout_matches_reference(Args):
    assert C.sizeof(Args) == 64
    for name, offset in LAYOUT.items():
        assert getattr(Args, name).offset == offset, name


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_header_layout_compiled(tmp_path):
    """Compile the public header with the host compiler and read the layout."""
    src = tmp_path / "layout.cpp"
    fields = ", ".join(f'offsetof(Fav4Args, {n})' for n in LAYOUT)
    src.write_text(
        '#include <cstddef>\n#include <cstdio>\n#include "fav4_bshd.h"\n'
        'int main() { size_t o[] = {' + fields + '};\n'
        '  std::printf("%zu", sizeof(Fav4Args)); for (size_t x : o) std::printf(" %zu", x); }\n')
    exe = tmp_path / "layout"
    subprocess.run(["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{HEADER.parent}", "-I/opt/rocm/include",
                    str(src), "-o", str(exe)], check=True, capture_output=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got == [64] + list(LAYOUT.values())


def _good(Args):
    # Distinct, 16-byte aligned fake device addresses; never dereferenced here
    # because every call below carries exactly one invalid field.
    return dict(q=0x10000, k=0x20000, v=0x30000, o=0x40000, lse=None, batch=2, heads=4, sq=256, sk=256,
                scale=1 / math.sqrt(128))


BAD = [
    ("q_null", dict(q=None)), ("k_null", dict(k=None)), ("v_null", dict(v=None)), ("o_null", dict(o=None)),
    ("batch0", dict(batch=0)), ("heads0", dict(heads=0)), ("sq0", dict(sq=0)), ("sk0", dict(sk=0)),
    ("batch_neg", dict(batch=-3)), ("sk_neg", dict(sk=-1)),
    ("scale0", dict(scale=0.0)), ("scale_neg", dict(scale=-0.5)), ("scale_nan", dict(scale=float("nan"))),
    ("scale_inf", dict(scale=float("inf"))),
    ("bh_overflow", dict(batch=1 << 16, heads=1 << 16)), ("heads_overflow", dict(heads=1 << 24)),
    ("sq_overflow", dict(heads=8, sq=1 << 21)), ("sk_overflow", dict(heads=8, sk=1 << 21)),
    ("q_misaligned", dict(q=0x10002)), ("k_misaligned", dict(k=0x20008)), ("v_misaligned", dict(v=0x30004)),
    ("o_misaligned", dict(o=0x40001)),
]


@pytest.mark.parametrize("name,change", BAD, ids=[b[0] for b in BAD])
def test_rejects_bad_arguments(lib, Args, name, change):
    fields = _good(Args)
    fields.update(change)
    a = Args(**fields)
    assert lib.fav4_bshd_forward(C.byref(a), 0, 0, None) == HIP_ERROR_INVALID_VALUE
    # the split-KV and GQA entry points apply the same checks first (GQA with
    # kv_heads = heads: the MHA limits)
    assert lib.fav4_bshd_forward_splitkv(C.byref(a), 0, 4, 0x100000, 1 << 30, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fav4_bshd_forward_gqa(C.byref(a), max(a.heads, 1), 0, 0, None) == HIP_ERROR_INVALID_VALUE


@pytest.mark.parametrize("sk", [131072, 200000, (1 << 31) // (8 * 128) - 1])
def test_gqa_key_limit_counts_kv_heads(lib, Args, sk):
    """H128 with 8 K/V heads: the key-side limit is sk * kv_heads * 128 < 2^31
    (K/V rows are kv_heads * 256 bytes apart), so long caches are accepted by
    the split-KV queries, for prefill and decode shapes alike, while the MHA
    form of the same shape (kv_heads = heads) is rejected."""
    for sq in (1, 4096):
        fields = _good(Args)
        fields.update(batch=1, heads=128, sq=sq, sk=sk)
        a = Args(**fields)
        splits = lib.fav4_bshd_splitkv_gqa_select(C.byref(a), 8, 0)
        assert splits >= 1, (sq, sk, splits)
        ws = lib.fav4_bshd_splitkv_gqa_workspace_size(C.byref(a), 8, 0, 0)
        assert ws == (0 if splits == 1 else splits * 128 * sq * (128 * 4 + 8)), (sq, sk, ws)
        assert lib.fav4_bshd_splitkv_gqa_select(C.byref(a), 128, 0) == -1
        assert lib.fav4_bshd_splitkv_gqa_workspace_size(C.byref(a), 128, 0, 0) == -1
    # one past the limit is rejected with 8 K/V heads too
    fields.update(sk=(1 << 31) // (8 * 128))
    assert lib.fav4_bshd_splitkv_gqa_select(C.byref(Args(**fields)), 8, 0) == -1


@pytest.mark.parametrize("causal,config", [(-1, 0), (2, 0), (0, -1), (0, 4), (1, 7)])
def test_rejects_bad_causal_or_config(lib, Args, causal, config):
    a = Args(**_good(Args))
    assert lib.fav4_bshd_forward(C.byref(a), causal, config, None) == HIP_ERROR_INVALID_VALUE


def test_rejects_null_args(lib):
    assert lib.fav4_bshd_forward(None, 0, 0, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fav4_bshd_select_config(None) == -1
    assert lib.fav4_bshd_select_config_masked(None, 0) == -1


@pytest.mark.parametrize("b,h,sq,want", [
    (2, 4, 1, 1), (2, 4, 127, 1), (32, 8, 256, 1), (32, 8, 768, 1),   # Sq <= 768: config 1
    (32, 8, 769, 2), (32, 8, 1000, 2), (32, 8, 1024, 2), (4, 16, 1024, 2), (2, 4, 1000, 1),
    (32, 8, 1025, 2), (32, 8, 4096, 2), (32, 8, 32768, 2), (2, 8, 4096, 2), (1, 32, 4096, 2),
    (1, 8, 4096, 1), (1, 8, 8192, 2), (2, 4, 4096, 1), (1, 1, 32768, 1)])   # fewer q tiles than 256 CUs: config 1
def test_select_config(lib, Args, b, h, sq, want):
    """Closed form of Auto for a dense call on 256 CUs (the library's value
    when no device is visible): config 1 for Sq <= 768 or fewer than 256
    q tiles of 256 rows, else config 2."""
    fields = _good(Args)
    fields.update(batch=b, heads=h, sq=sq)
    got = lib.fav4_bshd_select_config(C.byref(Args(**fields)))
    assert got == want and 1 <= got <= 3
    assert lib.fav4_bshd_select_config_masked(C.byref(Args(**fields)), 0) == got


@pytest.mark.parametrize("b,h,sq,want", [
    (32, 8, 768, 1), (32, 8, 1024, 1), (32, 8, 4096, 2), (1, 32, 4096, 2), (1, 64, 4096, 2), (2, 16, 4096, 2),
    (1, 16, 4096, 1), (1, 8, 8192, 1), (1, 8, 16384, 2), (1, 1, 32768, 1)])
def test_select_config_masked_causal(lib, Args, b, h, sq, want):
    """Closed form of Auto for a causal call on 256 CUs: config 1 for
    Sq <= 1024 or fewer than 256 q-tile pairs (B*H*ceil(ceil(Sq/256)/2)),
    else config 2.  The masks disagree at B1 H16 S4096 and B1 H8 S8192: 256
    q tiles (dense: config 2) but 128 pairs (causal: config 1); and at
    B32 H8 S1024, where the dense cut-off (Sq 768) gives config 2."""
    fields = _good(Args)
    fields.update(batch=b, heads=h, sq=sq)
    tiles = (sq + 255) // 256
    pairs = b * h * ((tiles + 1) // 2)
    assert want == (1 if sq <= 1024 or pairs < 256 else 2)
    assert lib.fav4_bshd_select_config_masked(C.byref(Args(**fields)), 1) == want
    if (b, h, sq) in ((1, 16, 4096), (1, 8, 8192), (32, 8, 1024)):
        assert lib.fav4_bshd_select_config(C.byref(Args(**fields))) == 2


@pytest.mark.parametrize("causal", [-1, 2, 3])
def test_select_config_masked_rejects_other_masks(lib, Args, causal):
    assert lib.fav4_bshd_select_config_masked(C.byref(Args(**_good(Args))), causal) == -1


def test_runner_rejects_host_tensors():
    torch = pytest.importorskip("torch")
    pkg = load_package()
    runner = pkg.Runner.__new__(pkg.Runner)  # no library needed for the argument checks
    q = torch.zeros(1, 4, 1, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        runner.args(q, q, q, q, None)
    with pytest.raises(AssertionError):
        runner.args(q.float(), q, q, q, None)


# ---- split-KV queries -------------------------------------------------------

def _split_plan(b, h, sq, sk, splits, cus=None, causal=False, kvh=None):
    """Closed form of the split plan: key tiles over the keys a row can see
    (min(sk, sq) for top-left causal); 256-row q tiles of one head and 64-key
    tiles, one workgroup per CU and at most 64 Auto chunks -- or, for sq <= 32
    (decode), 32-row tiles of a K/V head's packed (h / kvh) * sq query rows,
    32-key tiles, three workgroups per CU and at most 128; splits=0 picks
    ceil(CUs * per_cu / items) capped by min(max, ktiles // 4); then
    tiles-per-chunk and the final count so that no chunk is empty."""
    kvh = h if kvh is None else kvh
    bm, bn, per_cu, amax = (32, 32, 3, 128) if sq <= 32 else (256, 64, 1, 64)
    ktiles = -(-(min(sk, sq) if causal else sk) // bn)
    if splits == 0:
        items = b * kvh * -(-(h // kvh) * sq // bm) if sq <= 32 else b * h * -(-sq // bm)
        if sq <= 32 and items <= 2:     # one or two decode tiles: up to 256 chunks
            amax = 256
        splits = min(-(-(cus * per_cu) // items), min(amax, max(1, ktiles // 4)))
        if sq > 32 and splits > 1:
            splits = _prefill_auto(b, h, sq, sk, causal, splits, ktiles, cus)
    splits = max(1, min(splits, ktiles))
    tps = -(-ktiles // splits)
    return -(-ktiles // tps), tps


def _prefill_auto(b, h, sq, sk, causal, max_splits, ktiles, cus, br=False, br_unsplit=False):
    """Prefill Auto: the count in 1..max_splits with the lowest predicted time --
    unsplit: rounds of 128-row q tiles (causal: tile pairs), 2 per CU, x (9 +
    c per 64-key tile of a q tile, c = 0.9 with <= 1 workgroup per CU else 1.0;
    causal: 1.0 per tile of the heaviest pair); split: rounds of (256-row q
    tile, chunk) items, 1 per CU, x (19 + 1.8 per tile of a chunk; causal 18 +
    1.5) + 5."""
    keys = min(sk, sq) if causal else sk
    vis = lambda end: -(-min(keys, end if causal else keys) // 64)
    if br:      # bottom-right: the rows ending at `end` see keys up to end - 1 + sk - sq
        vis = lambda end: -(-min(keys, max(0, min(end, sq) + sk - sq)) // 64)
    nt128 = -(-sq // 128)
    if br and br_unsplit:
        # packed (varlen) bottom-right, one chunk: the unsplit packed kernel,
        # one item per (sequence, head, q tile), no pairs
        small = sq <= 1024 or b * h * -(-sq // 256) < cus
        bm = 128 if small else 256
        nt = -(-sq // bm)
        slots = 2 * cus if small else cus
        work = [vis(bm * (i + 1)) for i in range(nt)]
        best = -(-(b * h * nt) // slots) * 9.0 + max(b * h * sum(work) / slots, max(work))
    elif causal:
        npairs = (nt128 + 1) // 2
        heavy = max(vis(128 * (i + 1)) + (vis(128 * (nt128 - i)) if nt128 - 1 - i != i else 0)
                    for i in range(npairs))
        best = -(-(b * h * npairs) // (2 * cus)) * (9.0 + heavy)
    else:
        items = b * h * nt128
        best = -(-items // (2 * cus)) * (9.0 + (0.9 if items <= cus else 1.0) * ktiles)
    fixed, per_tile = (18.0, 1.5) if causal or br else (19.0, 1.8)
    if br and not br_unsplit:   # paged bottom-right: one chunk runs the split kernels too
        tps = ktiles
        items = sum(-(-vis(256 * (i + 1)) // tps) for i in range(-(-sq // 256)))
        best = -(-(b * h * items) // cus) * (fixed + per_tile * tps) + 5.0
    pick = 1
    for s in range(2, max_splits + 1):
        tps = -(-ktiles // s)
        items = sum(-(-vis(256 * (i + 1)) // tps) for i in range(-(-sq // 256)))
        t = -(-(b * h * items) // cus) * (fixed + per_tile * tps) + 5.0
        if t < best:
            best, pick = t, s
    return pick


@pytest.mark.parametrize("shape,splits", [((2, 3, 300, 5000), 5), ((1, 8, 1024, 32768), 16), ((1, 1, 1, 64), 8),
                                          ((4, 2, 257, 1000), 3), ((1, 2, 100, 129), 256), ((3, 1, 70, 4097), 7)])
def test_splitkv_workspace_size_closed_form(lib, Args, shape, splits):
    b, h, sq, sk = shape
    a = Args(None, None, None, None, None, b, h, sq, sk, 1 / math.sqrt(128))
    for causal in (0, 1):
        n, _ = _split_plan(b, h, sq, sk, splits, causal=bool(causal))
        want = 0 if n == 1 else n * b * h * sq * (128 * 4 + 8)
        assert lib.fav4_bshd_splitkv_workspace_size(C.byref(a), causal, splits) == want


@pytest.mark.parametrize("shape", [(1, 8, 1024, 32768), (32, 8, 4096, 4096), (1, 1, 256, 65536), (2, 4, 512, 2048),
                                   (1, 1, 100, 100), (1, 8, 2048, 32768), (1, 8, 4096, 32768), (1, 16, 2048, 2048),
                                   (1, 2, 8192, 4000), (1, 1, 16384, 16384), (3, 2, 1500, 60000)])
def test_splitkv_auto_plan(lib, Args, shape):
    """Auto chunk count, for the CU count the library sees (256 on MI355X; the
    same fallback when no device is visible)."""
    b, h, sq, sk = shape
    a = Args(None, None, None, None, None, b, h, sq, sk, 1 / math.sqrt(128))
    for causal in (0, 1):
        n, _ = _split_plan(b, h, sq, sk, 0, cus=256, causal=bool(causal))
        assert lib.fav4_bshd_splitkv_select(C.byref(a), causal) == n
        want = 0 if n == 1 else n * b * h * sq * (128 * 4 + 8)
        assert lib.fav4_bshd_splitkv_workspace_size(C.byref(a), causal, 0) == want


def test_splitkv_plan_examples():
    # B1 H8 Sq1024 Sk32768 (32 items, 512 key tiles): 8 chunks of 64 tiles;
    # the headline B32 H8 S4096 needs no split; 79 key tiles in 5 chunks of 16.
    assert _split_plan(1, 8, 1024, 32768, 0, cus=256) == (8, 64)
    # decode, B32 H8 Sq1 Sk8192 (one-wave shape, 256 items, 256 32-key tiles):
    # 3 chunks of 86 tiles fill three workgroups per CU
    assert _split_plan(32, 8, 1, 8192, 0, cus=256) == (3, 86)
    # decode, B1 H8 Sq1 Sk65536: 2048 key tiles, 96 chunks wanted -> 94 of 22
    assert _split_plan(1, 8, 1, 65536, 0, cus=256) == (94, 22)
    assert _split_plan(32, 8, 4096, 4096, 0, cus=256)[0] == 1
    assert _split_plan(2, 3, 300, 5000, 5) == (5, 16)
    assert _split_plan(1, 1, 256, 65536, 0, cus=256) == (64, 16)
    # causal prefill: the model keeps the unsplit forward where splitting
    # measured slower (Sq1024 H8, Sq2048 H16, Sq512) and splits where it won
    # (Sq2048 H8: 4 chunks, 36 vs 43 us; Sq4096 H8: 2 chunks, 70 vs 75 us)
    assert _split_plan(1, 8, 1024, 32768, 0, cus=256, causal=True)[0] == 1
    assert _split_plan(1, 16, 2048, 2048, 0, cus=256, causal=True)[0] == 1
    assert _split_plan(1, 8, 512, 65536, 0, cus=256, causal=True)[0] == 1
    assert _split_plan(1, 8, 2048, 32768, 0, cus=256, causal=True) == (4, 8)
    assert _split_plan(1, 8, 4096, 32768, 0, cus=256, causal=True) == (2, 32)
    # GQA decode B4 H32 KVH8 Sq1 Sk32768: 4 heads of a group share one 32-row
    # tile, 32 items, 1024 key tiles -> 24 chunks of 43
    assert _split_plan(4, 32, 1, 32768, 0, cus=256, kvh=8) == (24, 43)
    # MQA decode, 16 queries x 8 heads = 128 packed rows = 4 tiles per batch:
    # 96 chunks wanted over 512 key tiles -> 86 of 6
    assert _split_plan(2, 8, 16, 16384, 0, cus=256, kvh=1) == (86, 6)
    # one decode tile (B1 MQA, 6250 key tiles): 256 chunks of 25 tiles
    assert _split_plan(1, 8, 1, 200000, 0, cus=256, kvh=1) == (250, 25)


@pytest.mark.parametrize("shape", [(4, 32, 8, 1, 32768), (2, 8, 1, 16, 16384), (1, 12, 3, 5, 4000),
                                   (3, 6, 2, 100, 9000), (1, 8, 8, 1, 65536)])
def test_splitkv_gqa_plan(lib, Args, shape):
    """GQA split plan (decode packs a group's query heads into shared tiles)
    and its workspace, plus the rejected K/V head counts."""
    b, h, kvh, sq, sk = shape
    a = Args(None, None, None, None, None, b, h, sq, sk, 1 / math.sqrt(128))
    for causal in (0, 1):
        n, _ = _split_plan(b, h, sq, sk, 0, cus=256, causal=bool(causal), kvh=kvh)
        assert lib.fav4_bshd_splitkv_gqa_select(C.byref(a), kvh, causal) == n
        want = 0 if n == 1 else n * b * h * sq * (128 * 4 + 8)
        assert lib.fav4_bshd_splitkv_gqa_workspace_size(C.byref(a), kvh, causal, 0) == want
        for bad in (0, -1, h + 1, 5 if h % 5 else 7):
            if bad > 0 and h % bad == 0:
                continue
            assert lib.fav4_bshd_splitkv_gqa_select(C.byref(a), bad, causal) == -1
            assert lib.fav4_bshd_splitkv_gqa_workspace_size(C.byref(a), bad, causal, 0) == -1


def test_splitkv_gqa_rejects_oversized_groups(lib, Args):
    """Decode packs (heads / kv_heads) * sq rows of 512 partial bytes into one
    4 GiB-bounded buffer: 2^23 rows is one too many."""
    a = Args(None, None, None, None, None, 1, 1 << 18, 32, 64, 1 / math.sqrt(128))
    assert lib.fav4_bshd_splitkv_gqa_select(C.byref(a), 1, 0) == -1
    a.heads = (1 << 18) - 8
    assert lib.fav4_bshd_splitkv_gqa_select(C.byref(a), 1, 0) >= 1


@pytest.mark.parametrize("causal,splits,sq", [(2, 4, 256), (-1, 4, 256), (0, -1, 256), (0, 257, 256),
                                              (0, 4, (1 << 22) + 1)])
def test_splitkv_queries_reject(lib, Args, causal, splits, sq):
    a = Args(None, None, None, None, None, 1, 1, sq, 4096, 1 / math.sqrt(128))
    assert lib.fav4_bshd_splitkv_workspace_size(C.byref(a), causal, splits) == -1
    assert lib.fav4_bshd_splitkv_workspace_size(None, 0, 0) == -1
    assert lib.fav4_bshd_splitkv_select(None, 0) == -1


@pytest.mark.parametrize("ws,nbytes", [(None, 1 << 30), (0x100010, 1 << 30), (0x100000, 1000)],
                         ids=["null", "misaligned", "too_small"])
def test_splitkv_rejects_workspace(lib, Args, ws, nbytes):
    fields = _good(Args)
    fields.update(sq=256, sk=8192)
    a = Args(**fields)
    assert lib.fav4_bshd_forward_splitkv(C.byref(a), 0, 8, ws, nbytes, None) == HIP_ERROR_INVALID_VALUE


@pytest.mark.parametrize("kv_heads", [0, -1, 5, 3, 8])
def test_gqa_rejects_bad_kv_heads(lib, Args, kv_heads):
    """heads = 4: kv_heads must be a positive divisor of it."""
    a = Args(**_good(Args))
    assert lib.fav4_bshd_forward_gqa(C.byref(a), kv_heads, 0, 0, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fav4_bshd_forward_gqa(C.byref(a), 2, 2, 0, None) == HIP_ERROR_INVALID_VALUE   # bad causal
    assert lib.fav4_bshd_forward_gqa(None, 2, 0, 0, None) == HIP_ERROR_INVALID_VALUE


# ---- packed variable-length sequences --------------------------------------
VLAYOUT = dict(q=0, k=8, v=16, o=24, lse=32, cu_seqlens_q=40, cu_seqlens_k=48, batch=56, heads=60, kv_heads=64,
               max_seqlen_q=68, max_seqlen_k=72, total_q=76, total_k=80, scale=84)


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_varlen_layout_ctypes_and_header(tmp_path):
    VarlenArgs = load_package().VarlenArgs
    assert C.sizeof(VarlenArgs) == 88
    for name, offset in VLAYOUT.items():
        assert getattr(VarlenArgs, name).offset == offset, name
    src = tmp_path / "vlayout.cpp"
    fields = ", ".join(f'offsetof(Fav4VarlenArgs, {n})' for n in VLAYOUT)
    src.write_text(
        '#include <cstddef>\n#include <cstdio>\n#include "fav4_bshd.h"\n'
        'int main() { size_t o[] = {' + fields + '};\n'
        '  std::printf("%zu", sizeof(Fav4VarlenArgs)); for (size_t x : o) std::printf(" %zu", x); }\n')
    exe = tmp_path / "vlayout"
    subprocess.run(["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{HEADER.parent}", "-I/opt/rocm/include",
                    str(src), "-o", str(exe)], check=True, capture_output=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got == [88] + list(VLAYOUT.values())


def _vgood():
    return dict(q=0x10000, k=0x20000, v=0x30000, o=0x40000, lse=None, cu_seqlens_q=0x50000, cu_seqlens_k=0x60000,
                batch=3, heads=4, kv_heads=2, max_seqlen_q=300, max_seqlen_k=500, total_q=600, total_k=900,
                scale=1 / math.sqrt(128))


VBAD = [
    ("q_null", dict(q=None)), ("k_null", dict(k=None)), ("v_null", dict(v=None)), ("o_null", dict(o=None)),
    ("cuq_null", dict(cu_seqlens_q=None)), ("cuk_null", dict(cu_seqlens_k=None)),
    ("batch0", dict(batch=0)), ("heads0", dict(heads=0)), ("kv0", dict(kv_heads=0)), ("kv3", dict(kv_heads=3)),
    ("kv8", dict(kv_heads=8)), ("maxq0", dict(max_seqlen_q=0)), ("maxk0", dict(max_seqlen_k=0)),
    ("totq0", dict(total_q=0)), ("totk_neg", dict(total_k=-5)),
    ("scale0", dict(scale=0.0)), ("scale_nan", dict(scale=float("nan"))), ("scale_inf", dict(scale=float("inf"))),
    ("q_overflow", dict(max_seqlen_q=1 << 22)), ("k_overflow", dict(kv_heads=4, max_seqlen_k=1 << 22)),
    ("q_misaligned", dict(q=0x10008)), ("o_misaligned", dict(o=0x40002)), ("cu_misaligned", dict(cu_seqlens_k=0x60002)),
    ("lse_misaligned", dict(lse=0x70001)),
    ("grid_overflow", dict(batch=1 << 20, heads=1 << 10, kv_heads=1, max_seqlen_q=1 << 10)),
]


@pytest.mark.parametrize("name,change", VBAD, ids=[b[0] for b in VBAD])
def test_varlen_rejects_bad_arguments(lib, name, change):
    VarlenArgs = load_package().VarlenArgs
    f = _vgood()
    f.update(change)
    a = VarlenArgs(**f)
    assert lib.fav4_bshd_forward_varlen(C.byref(a), 0, None) == HIP_ERROR_INVALID_VALUE


@pytest.mark.parametrize("causal", [-1, 3])
def test_varlen_rejects_bad_causal(lib, causal):
    a = load_package().VarlenArgs(**_vgood())
    assert lib.fav4_bshd_forward_varlen(C.byref(a), causal, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fav4_bshd_forward_varlen(None, 0, None) == HIP_ERROR_INVALID_VALUE


# ---- split-KV of packed sequences --------------------------------------------
def _varlen_split_plan(batch, h, kvh, max_q, max_k, total_k, splits, causal=False, cus=256):
    """Closed form of the packed-batch plan: one chunk for max_q > 32; explicit
    counts as the contiguous plan at the max lengths; Auto takes the chunk size
    (key tiles) of the contiguous Auto plan at the mean key length, at most 64
    tiles when the mean is below 3/4 of the longest, enlarged to keep the
    longest sequence within 256 chunks."""
    if max_q > 32:
        return 1, 1
    if splits:
        return _split_plan(batch, h, max_q, max_k, splits, causal=causal, kvh=kvh)
    mean = max(1, min(max_k, -(-total_k // batch)))
    ktiles = -(-(min(max_k, max_q) if causal else max_k) // 32)
    tps = _split_plan(batch, h, max_q, mean, 0, cus=cus, causal=causal, kvh=kvh)[1]
    if 4 * mean < 3 * max_k:        # ragged: chunks of at most 64 key tiles
        tps = min(tps, 64)
    tps = max(tps, -(-ktiles // 256))
    return -(-ktiles // tps), tps


def _vshape(batch, h, kvh, max_q, max_k, total_q, total_k):
    f = _vgood()
    f.update(q=None, k=None, v=None, o=None, cu_seqlens_q=None, cu_seqlens_k=None, batch=batch, heads=h,
             kv_heads=kvh, max_seqlen_q=max_q, max_seqlen_k=max_k, total_q=total_q, total_k=total_k)
    return load_package().VarlenArgs(**f)


@pytest.mark.parametrize("shape", [(8, 32, 8, 1, 32768, 8 * 4096), (4, 8, 8, 1, 65536, 4 * 65536),
                                   (3, 12, 3, 5, 4000, 5000), (16, 8, 1, 32, 9000, 16 * 300),
                                   (2, 4, 2, 33, 8192, 8192), (1, 2, 2, 1, 31, 31), (5, 6, 2, 17, 2048, 3)])
def test_splitkv_varlen_plan(lib, shape):
    """Select and workspace queries of the packed-batch split-KV (shape only,
    no buffers) against the closed form; explicit counts too."""
    b, h, kvh, mq, mk, tk = shape
    a = _vshape(b, h, kvh, mq, mk, b * mq, tk)
    for causal in (0, 1):
        n, _ = _varlen_split_plan(b, h, kvh, mq, mk, tk, 0, causal=bool(causal))
        assert lib.fav4_bshd_splitkv_varlen_select(C.byref(a), causal) == n
        want = 0 if n == 1 else n * b * h * mq * (128 * 4 + 8)
        assert lib.fav4_bshd_splitkv_varlen_workspace_size(C.byref(a), causal, 0) == want
        for req in (1, 3, 200, 256):
            n, _ = _varlen_split_plan(b, h, kvh, mq, mk, tk, req, causal=bool(causal))
            want = 0 if n == 1 else n * b * h * mq * (128 * 4 + 8)
            assert lib.fav4_bshd_splitkv_varlen_workspace_size(C.byref(a), causal, req) == want


def test_splitkv_varlen_plan_examples():
    # 8 sequences of 4096 keys on average, one as long as 32768, 32 query heads
    # over 8 K/V heads: 12 chunks of 11 tiles fill the CUs at the mean length,
    # and the longest sequence needs 94 of them.
    assert _varlen_split_plan(8, 32, 8, 1, 32768, 8 * 4096, 0, cus=256) == (94, 11)
    # uniform lengths: the contiguous plan
    for sk in (32768, 9 * 32 * 4, 1000, 77777):
        assert _varlen_split_plan(4, 32, 8, 1, sk, 4 * sk, 0) == _split_plan(4, 32, 1, sk, 0, cus=256, kvh=8)
    # one sequence far longer than the mean: chunks grow to stay within 256
    assert _varlen_split_plan(64, 8, 8, 1, 1 << 20, 64 * 2048, 0, cus=256) == (256, 128)
    assert _varlen_split_plan(2, 4, 2, 33, 8192, 8192, 0) == (1, 1)


@pytest.mark.parametrize("name,change", VBAD + [("splits_neg", dict()), ("splits_big", dict())],
                         ids=[b[0] for b in VBAD] + ["splits_neg", "splits_big"])
def test_splitkv_varlen_rejects_bad_arguments(lib, name, change):
    VarlenArgs = load_package().VarlenArgs
    f = _vgood()
    f["max_seqlen_q"] = 16          # the decode shape that splits
    f.update(change)
    if name == "grid_overflow":     # 2^35 partial rows
        f.update(max_seqlen_q=32, max_seqlen_k=64)
    splits = -1 if name == "splits_neg" else 257 if name == "splits_big" else 4
    a = VarlenArgs(**f)
    assert lib.fav4_bshd_forward_splitkv_varlen(C.byref(a), 0, splits, 0x100000, 1 << 40, None) == \
        HIP_ERROR_INVALID_VALUE
    assert lib.fav4_bshd_forward_splitkv_varlen(None, 0, splits, 0x100000, 1 << 40, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fav4_bshd_forward_splitkv_varlen(C.byref(a), 3, 4, 0x100000, 1 << 40, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fav4_bshd_splitkv_varlen_select(None, 0) == -1
    assert lib.fav4_bshd_splitkv_varlen_workspace_size(None, 0, 0) == -1


def test_splitkv_varlen_bottom_right(lib):
    """causal = 2 (bottom-right) is planned like a dense call; decode always
    splits (one chunk needs a workspace too); longer queries take the dense
    prefill plan, and with one chunk the unsplit packed forward (no
    workspace)."""
    f = _vgood()
    f.update(q=None, k=None, v=None, o=None, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=4, max_seqlen_k=5000)
    a = load_package().VarlenArgs(**f)
    assert lib.fav4_bshd_splitkv_varlen_select(C.byref(a), 2) == lib.fav4_bshd_splitkv_varlen_select(C.byref(a), 0)
    for splits in (0, 3):
        dense = lib.fav4_bshd_splitkv_varlen_workspace_size(C.byref(a), 0, splits)
        assert dense > 0 and lib.fav4_bshd_splitkv_varlen_workspace_size(C.byref(a), 2, splits) == dense
    # one chunk: the dense call needs no workspace, bottom-right does
    assert lib.fav4_bshd_splitkv_varlen_workspace_size(C.byref(a), 0, 1) == 0
    assert lib.fav4_bshd_splitkv_varlen_workspace_size(C.byref(a), 2, 1) == 3 * 4 * 4 * 520
    # prefill: the contiguous dense prefill plan at the max lengths, with a workspace
    a.max_seqlen_q = 600
    n, _ = _split_plan(3, 4, 600, 5000, 0, cus=256, kvh=2)
    assert lib.fav4_bshd_splitkv_varlen_select(C.byref(a), 2) == n
    assert lib.fav4_bshd_splitkv_varlen_workspace_size(C.byref(a), 2, 0) == n * 3 * 4 * 600 * 520
    assert lib.fav4_bshd_splitkv_varlen_workspace_size(C.byref(a), 2, 1) == 0
    assert lib.fav4_bshd_splitkv_varlen_select(C.byref(a), 0) == 1
    p = _pgood(q=None, k_cache=None, v_cache=None, o=None, cu_seqlens_q=None, seqlens_k=None, block_table=None)
    assert lib.fav4_bshd_splitkv_paged_select(C.byref(p), 2) == lib.fav4_bshd_splitkv_paged_select(C.byref(p), 0) > 0
    assert lib.fav4_bshd_splitkv_paged_select(C.byref(p), 1) == -1


@pytest.mark.parametrize("ws,nbytes", [(None, 1 << 30), (0x100010, 1 << 30), (0x100000, 1000)],
                         ids=["null", "misaligned", "too_small"])
def test_splitkv_varlen_rejects_workspace(lib, ws, nbytes):
    VarlenArgs = load_package().VarlenArgs
    f = _vgood()
    f.update(max_seqlen_q=1, max_seqlen_k=8192, total_q=3, total_k=9000)
    a = VarlenArgs(**f)
    assert lib.fav4_bshd_forward_splitkv_varlen(C.byref(a), 0, 8, ws, nbytes, None) == HIP_ERROR_INVALID_VALUE


# ---- split-KV decode over paged K/V caches -------------------------------------
PLAYOUT = dict(q=0, k_cache=8, v_cache=16, o=24, lse=32, cu_seqlens_q=40, seqlens_k=48, block_table=56, batch=64,
               heads=68, kv_heads=72, max_seqlen_q=76, max_seqlen_k=80, total_q=84, total_k=88, num_pages=92,
               page_size=96, max_pages_per_seq=100, scale=104)


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_paged_layout_ctypes_and_header(tmp_path):
    PagedArgs = load_package().PagedArgs
    assert C.sizeof(PagedArgs) == 112
    for name, offset in PLAYOUT.items():
        assert getattr(PagedArgs, name).offset == offset, name
    src = tmp_path / "playout.cpp"
    fields = ", ".join(f'offsetof(Fav4PagedArgs, {n})' for n in PLAYOUT)
    src.write_text(
        '#include <cstddef>\n#include <cstdio>\n#include "fav4_bshd.h"\n'
        'int main() { size_t o[] = {' + fields + '};\n'
        '  std::printf("%zu", sizeof(Fav4PagedArgs)); for (size_t x : o) std::printf(" %zu", x); }\n')
    exe = tmp_path / "playout"
    subprocess.run(["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{HEADER.parent}", "-I/opt/rocm/include",
                    str(src), "-o", str(exe)], check=True, capture_output=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got == [112] + list(PLAYOUT.values())


def _pgood(**kw):
    f = dict(q=0x10000, k_cache=0x20000, v_cache=0x30000, o=0x40000, lse=None, cu_seqlens_q=0x50000,
             seqlens_k=0x60000, block_table=0x70000, batch=3, heads=8, kv_heads=2, max_seqlen_q=4,
             max_seqlen_k=5000, total_q=12, total_k=9000, num_pages=400, page_size=64, max_pages_per_seq=80,
             scale=1 / math.sqrt(128))
    f.update(kw)
    return load_package().PagedArgs(**f)


def _paged_plan(b, h, kvh, mq, mk, tk, splits):
    """Decode: the packed-batch plan at these sizes; prefill (mq > 32): the
    contiguous dense plan at the max lengths; chunks capped at 64 key tiles
    (32 keys decode, 64 prefill)."""
    if mq > 32:
        n, tps = _split_plan(b, h, mq, mk, splits, cus=256, kvh=kvh)
        bn = 64
    else:
        n, tps = _varlen_split_plan(b, h, kvh, mq, mk, tk, splits)
        bn = 32
    if tps > 64:
        tps = 64
        n = -(-(-(-mk // bn)) // 64)
    return n, tps


@pytest.mark.parametrize("shape", [(8, 32, 8, 1, 32768, 8 * 4096), (1, 8, 8, 1, 65536, 65536), (3, 8, 2, 4, 5000, 9000),
                                   (16, 32, 4, 16, 2048, 16 * 1000), (1, 1, 1, 1, 524288, 524288),
                                   (2, 4, 4, 32, 100, 3), (1, 8, 2, 1000, 32768, 32768), (3, 4, 4, 300, 5000, 9000),
                                   (1, 1, 1, 4096, 524288, 524288)])
def test_splitkv_paged_plan(lib, shape):
    b, h, kvh, mq, mk, tk = shape
    ps = 32 if mq <= 32 else 64
    a = _pgood(batch=b, heads=h, kv_heads=kvh, max_seqlen_q=mq, max_seqlen_k=mk, total_k=tk, total_q=b * mq,
               page_size=ps, max_pages_per_seq=-(-mk // ps), q=None, k_cache=None, v_cache=None, o=None,
               cu_seqlens_q=None, seqlens_k=None, block_table=None)
    n, tps = _paged_plan(b, h, kvh, mq, mk, tk, 0)
    assert tps <= 64
    assert lib.fav4_bshd_splitkv_paged_select(C.byref(a), 0) == n
    assert lib.fav4_bshd_splitkv_paged_workspace_size(C.byref(a), 0, 0) == n * b * h * mq * (128 * 4 + 8)
    for req in (1, 3, 256):
        n, tps = _paged_plan(b, h, kvh, mq, mk, tk, req)
        assert tps <= 64
        assert lib.fav4_bshd_splitkv_paged_workspace_size(C.byref(a), 0, req) == n * b * h * mq * (128 * 4 + 8)


PBAD = [("q_null", dict(q=None)), ("k_null", dict(k_cache=None)), ("v_null", dict(v_cache=None)),
        ("o_null", dict(o=None)), ("cuq_null", dict(cu_seqlens_q=None)), ("seqk_null", dict(seqlens_k=None)),
        ("table_null", dict(block_table=None)), ("batch0", dict(batch=0)), ("heads0", dict(heads=0)),
        ("kv3", dict(kv_heads=3)), ("maxq0", dict(max_seqlen_q=0)), ("prefill_page32", dict(max_seqlen_q=33, page_size=32)),
        ("maxq_2p22", dict(max_seqlen_q=(1 << 22) + 1, heads=2, kv_heads=2, total_q=1 << 23)),
        ("maxk0", dict(max_seqlen_k=0)), ("totq0", dict(total_q=0)), ("totk_neg", dict(total_k=-1)),
        ("pages0", dict(num_pages=0)), ("page16", dict(page_size=16)), ("page48", dict(page_size=48)),
        ("maxpages0", dict(max_pages_per_seq=0)), ("table_short", dict(max_pages_per_seq=78)),
        ("keys_2p19", dict(max_seqlen_k=524289, max_pages_per_seq=9000)),
        ("page_huge", dict(page_size=1 << 21, kv_heads=8, max_pages_per_seq=1)),
        ("group_rows", dict(heads=1 << 18, kv_heads=1, max_seqlen_q=32)),
        ("scale0", dict(scale=0.0)), ("scale_nan", dict(scale=float("nan"))),
        ("q_misaligned", dict(q=0x10008)), ("k_misaligned", dict(k_cache=0x20004)),
        ("table_misaligned", dict(block_table=0x70002)), ("lse_misaligned", dict(lse=0x80001))]


@pytest.mark.parametrize("name,change", PBAD, ids=[b[0] for b in PBAD])
def test_splitkv_paged_rejects_bad_arguments(lib, name, change):
    a = _pgood(**change)
    assert lib.fav4_bshd_forward_splitkv_paged(C.byref(a), 0, 4, 0x100000, 1 << 40, None) == HIP_ERROR_INVALID_VALUE


def test_splitkv_paged_rejects_causal_splits_and_workspace(lib):
    a = _pgood()
    assert lib.fav4_bshd_forward_splitkv_paged(C.byref(a), 1, 4, 0x100000, 1 << 40, None) == HIP_ERROR_INVALID_VALUE
    for splits in (-1, 257):
        assert lib.fav4_bshd_forward_splitkv_paged(C.byref(a), 0, splits, 0x100000, 1 << 40, None) == \
            HIP_ERROR_INVALID_VALUE
        assert lib.fav4_bshd_splitkv_paged_workspace_size(C.byref(a), 0, splits) == -1
    for ws, nbytes in ((None, 1 << 30), (0x100010, 1 << 30), (0x100000, 1000)):
        assert lib.fav4_bshd_forward_splitkv_paged(C.byref(a), 0, 4, ws, nbytes, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fav4_bshd_forward_splitkv_paged(None, 0, 4, 0x100000, 1 << 40, None) == HIP_ERROR_INVALID_VALUE
    assert lib.fav4_bshd_splitkv_paged_select(None, 0) == -1
    assert lib.fav4_bshd_splitkv_paged_select(C.byref(a), 1) == -1
    assert lib.fav4_bshd_splitkv_paged_workspace_size(None, 0, 0) == -1


# ---- arbitrary strides -------------------------------------------------------
def _strided_call(lib, a, kv_heads, strides, causal=0, config=0):
    S = load_package().Strides
    st = [C.byref(S(*x)) if x is not None else None for x in strides]
    return lib.fav4_bshd_forward_strided(C.byref(a) if a is not None else None, kv_heads, *st, causal, config, None)


def _bshd_strides(b, s, h):
    return (s * h * 128, h * 128, 128)


def test_strides_struct_layout():
    S = load_package().Strides
    assert C.sizeof(S) == 24 and S.batch.offset == 0 and S.seq.offset == 8 and S.head.offset == 16


SBAD = [
    ("q_seq_odd", 0, (4096 * 4 * 128, 4 * 128 + 4, 128)),
    ("k_head_neg", 1, (4096 * 4 * 128, 4 * 128, -128)),
    ("v_seq_zero", 2, (4096 * 4 * 128, 0, 128)),
    ("o_batch_neg", 3, (-8, 4 * 128, 128)),
    ("q_head_odd", 0, (4096 * 4 * 128, 4 * 128, 129)),
    ("o_span_2p48", 3, (1 << 47, 4 * 128, 128)),   # 2 batches 2^48 bytes apart
]


@pytest.mark.parametrize("name,which,bad", SBAD, ids=[x[0] for x in SBAD])
def test_strided_rejects_bad_strides(lib, Args, name, which, bad):
    a = Args(**_good(Args))
    strides = [_bshd_strides(2, 256, 4)] * 4
    strides[which] = bad
    assert _strided_call(lib, a, 4, strides) == HIP_ERROR_INVALID_VALUE


def test_strided_rejects_oversized_slice_and_nulls(lib, Args):
    a = Args(**_good(Args))                           # sq = sk = 256
    ok = [_bshd_strides(2, 256, 4)] * 4
    # 255 rows x 2^24 elements x 2 bytes > 4 GiB for one (batch, head) slice
    for which in range(4):
        st = list(ok)
        st[which] = (0, 1 << 24, 128)
        assert _strided_call(lib, a, 4, st) == HIP_ERROR_INVALID_VALUE, which
        st[which] = None
        assert _strided_call(lib, a, 4, st) == HIP_ERROR_INVALID_VALUE, which
    assert _strided_call(lib, None, 4, ok) == HIP_ERROR_INVALID_VALUE
    for kvh in (0, 3, 8, -1):
        assert _strided_call(lib, a, kvh, ok) == HIP_ERROR_INVALID_VALUE, kvh
    assert _strided_call(lib, a, 4, ok, causal=2) == HIP_ERROR_INVALID_VALUE
    assert _strided_call(lib, a, 4, ok, config=4) == HIP_ERROR_INVALID_VALUE


@pytest.mark.parametrize("name,change", BAD[:14] + BAD[18:], ids=[x[0] for x in BAD[:14] + BAD[18:]])
def test_strided_applies_forward_checks(lib, Args, name, change):
    """The pointer / dimension / scale / alignment checks of fav4_bshd_forward apply too."""
    f = _good(Args)
    f.update(change)
    a = Args(**f)
    st = [_bshd_strides(2, 256, 4)] * 4
    assert _strided_call(lib, a, max(1, min(4, a.heads if a.heads > 0 else 1)), st) == HIP_ERROR_INVALID_VALUE


def test_noalloc_rejects_plans_past_its_array(lib, Args):
    """The no-workspace split-KV call keeps its partials in a 64 MiB array per
    device: a plan needing more is rejected before any HIP call, as are the
    arguments the workspace call rejects."""
    lib.fav4_bshd_forward_splitkv_gqa_noalloc.argtypes = [C.POINTER(Args), C.c_int, C.c_int, C.c_int, C.c_void_p]
    fields = _good(Args)
    fields.update(batch=32, heads=8, sq=4096, sk=32768)
    a = Args(**fields)
    need = lib.fav4_bshd_splitkv_gqa_workspace_size(C.byref(a), 8, 0, 8)
    assert need == 8 * 32 * 8 * 4096 * (128 * 4 + 8) > 64 << 20
    assert lib.fav4_bshd_forward_splitkv_gqa_noalloc(C.byref(a), 8, 0, 8, None) == HIP_ERROR_INVALID_VALUE
    for kvh, causal, splits in ((0, 0, 0), (3, 0, 0), (8, 2, 0), (8, 0, 257), (8, 0, -1)):
        assert lib.fav4_bshd_forward_splitkv_gqa_noalloc(C.byref(a), kvh, causal, splits, None) == \
            HIP_ERROR_INVALID_VALUE, (kvh, causal, splits)
    assert lib.fav4_bshd_forward_splitkv_gqa_noalloc(None, 8, 0, 0, None) == HIP_ERROR_INVALID_VALUE


def test_mfma_ceiling_probe_library():
    """The measurement library behind `bench.py --mfma-ceiling` exports its one
    entry point and rejects arguments outside its ranges before any HIP call."""
    import ctypes as C
    import subprocess
    pkg = load_package()
    if not pkg.CEILING_LIB_PATH.exists():
        pkg.build_library()
    syms = subprocess.run(["nm", "-D", "--defined-only", str(pkg.CEILING_LIB_PATH)], capture_output=True,
                          text=True, check=True).stdout
    assert sorted(ln.split()[-1] for ln in syms.splitlines() if " T " in ln) == ["fav4_probe_mfma_ceiling"]
    import torch  # noqa: F401  (torch's HIP runtime first, as the package's loader does)
    probe = C.CDLL(str(pkg.CEILING_LIB_PATH))
    probe.fav4_probe_mfma_ceiling.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    probe.fav4_probe_mfma_ceiling.restype = C.c_int
    for shape, grid, iters, out in [(2, 256, 16, 0x1000), (-1, 256, 16, 0x1000), (0, 0, 16, 0x1000),
                                    (0, 65537, 16, 0x1000), (0, 256, 0, 0x1000), (1, 256, (1 << 20) + 1, 0x1000),
                                    (0, 256, 16, None), (1, 256, 16, 0x1002)]:
        assert probe.fav4_probe_mfma_ceiling(shape, grid, iters, out, None) == 1, (shape, grid, iters, out)


def test_paged_helpers_forward_the_mask(lib):
    """Runner.splitkv_paged_select / _workspace_size size the plan of the mask
    the caller will run: bottom-right prefill of B1 H8 KVH8 Sq=Sk=4096 plans
    more chunks than dense, so a workspace sized for the dense mask would be
    too small for a causal=2 call."""
    pkg = load_package()
    runner = pkg.Runner()
    args = (1, 8, 8, 4096, 4096, 4096, 4096, 64, 64, 64)
    a = pkg.PagedArgs(None, None, None, None, None, None, None, None, 1, 8, 8, 4096, 4096, 4096, 4096, 64, 64, 64,
                      1 / math.sqrt(128))
    for causal in (0, 2):
        assert runner.splitkv_paged_select(*args, causal=causal) == lib.fav4_bshd_splitkv_paged_select(C.byref(a),
                                                                                                      causal)
        assert runner.splitkv_paged_workspace_size(*args, causal=causal) == \
            lib.fav4_bshd_splitkv_paged_workspace_size(C.byref(a), causal, 0)
    dense = runner.splitkv_paged_workspace_size(*args, causal=0)
    br = runner.splitkv_paged_workspace_size(*args, causal=2)
    assert runner.splitkv_paged_select(*args, causal=2) > runner.splitkv_paged_select(*args, causal=0)
    assert br > dense > 0



@pytest.mark.parametrize("shape", [(1, 8, 4096), (1, 8, 2048), (1, 8, 8192), (2, 4, 3000), (1, 16, 1500),
                                   (4, 8, 700), (1, 1, 16384)])
def test_bottom_right_prefill_plans(lib, shape):
    """Bottom-right prefill Auto: the packed (varlen) call prices one chunk as
    its unsplit kernel, the paged call as one split-kernel chunk; both then
    keep the cheapest count of the closed-form model (max_seqlen_q = max_seqlen_k)."""
    b, h, s_ = shape
    pkg = load_package()
    runner = pkg.Runner()
    cus = 256
    ktiles = -(-s_ // 64)
    cap = min(-(-cus // (b * h * -(-s_ // 256))), min(64, max(1, ktiles // 4)))
    want_v = _prefill_auto(b, h, s_, s_, False, cap, ktiles, cus, br=True, br_unsplit=True) if cap > 1 else 1
    want_p = _prefill_auto(b, h, s_, s_, False, cap, ktiles, cus, br=True) if cap > 1 else 1
    tps_v, tps_p = -(-ktiles // want_v), -(-ktiles // want_p)
    assert runner.splitkv_varlen_select(b, h, h, s_, s_, b * s_, b * s_, 2) == -(-ktiles // tps_v)
    pages = -(-s_ // 64)
    assert runner.splitkv_paged_select(b, h, h, s_, s_, b * s_, b * s_, 64, pages, b * pages, causal=2) == \
        -(-ktiles // min(tps_p, 64))
