"""Pins for the FP64 oracle (CPU only).

The oracle restates benchmarks/bshd.py:90-100.  It is checked against
independent evidence, never against a retyped copy of its own formula:
  * golden vectors from a pure-Python brute force (tests/golden/),
  * closed forms of the reference's special input patterns
    (bshd.py:81-86: zero, negative, late_max) and of 1x1 / causal row 0,
  * invariants of exact attention (key permutation, logit shift, linearity
    in V, scale folding, Sq > Sk causal rows),
  * and planted mutants of the oracle that those checks must reject.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import attention as orc

GOLDEN = Path(__file__).resolve().parent / "golden" / "bruteforce.npz"
S = orc.DEFAULT_SCALE


def _golden_cases():
    z = np.load(GOLDEN, allow_pickle=False)
    meta = json.loads(bytes(z["meta"]).decode())
    return [(m, z[f"c{n}_q"], z[f"c{n}_k"], z[f"c{n}_v"], z[f"c{n}_o"], z[f"c{n}_lse"])
            for n, m in enumerate(meta)]


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


# ----------------------------------------------------------------------------
# The pin suite, reused against planted mutants below
# ----------------------------------------------------------------------------
def pin_failures(o) -> list:
    """Run every pin against oracle module `o`; return the names that fail."""
    fails = []

    def check(name, ok):
        if not ok:
            fails.append(name)

    def close(a, b, tol):
        a, b = np.asarray(a), np.asarray(b)
        return a.shape == b.shape and bool(np.all(np.isfinite(a))) and float(np.max(np.abs(a - b))) <= tol

    with np.errstate(all="ignore"):
        for n, (m, q, k, v, ref_o, ref_lse) in enumerate(_golden_cases()):
            got_o, got_lse = o.attention_fp64(q, k, v, m["scale"], m["causal"])
            check(f"golden{n}", close(got_o, ref_o, 1e-12) and close(got_lse, ref_lse, 1e-12))

        # zero pattern: all logits 0 -> O_i = mean of visible V, LSE_i = ln |visible|
        for causal in (False, True):
            q, k, v = orc.make_inputs(1, 2, 9, 6, "zero")
            got_o, got_lse = o.attention_fp64(q, k, v, S, causal)
            vf = orc.bf16_to_f32(v).reshape(v.shape).astype(np.float64)
            n_vis = np.array([min(i + 1, 6) if causal else 6 for i in range(9)])
            exp_o = np.stack([vf[:, :n].mean(axis=1) for n in n_vis], axis=1)
            check(f"zero_o_{causal}", close(got_o, exp_o, 1e-12))
            check(f"zero_lse_{causal}", close(got_lse, np.broadcast_to(np.log(n_vis), got_lse.shape), 1e-12))

            # negative pattern (q=8, k=-8): every logit is -8192*scale
            q, k, v = orc.make_inputs(1, 2, 9, 6, "negative")
            got_o, got_lse = o.attention_fp64(q, k, v, S, causal)
            vf = orc.bf16_to_f32(v).reshape(v.shape).astype(np.float64)
            exp_o = np.stack([vf[:, :n].mean(axis=1) for n in n_vis], axis=1)
            check(f"negative_o_{causal}", close(got_o, exp_o, 1e-10))
            check(f"negative_lse_{causal}",
                  close(got_lse, np.broadcast_to(-8192.0 * S + np.log(n_vis), got_lse.shape), 1e-9))

        # late_max pattern (q=1, k_j=floor(j/64)): logit_j = 128*S*floor(j/64)
        q, k, v = orc.make_inputs(1, 1, 3, 200, "late_max")
        got_o, got_lse = o.attention_fp64(q, k, v, S, False)
        vf = orc.bf16_to_f32(v).reshape(v.shape).astype(np.float64)[0, :, 0]
        groups = np.arange(200) // 64
        c = 128 * S
        gsum = np.array([vf[groups == g].sum(axis=0) for g in range(4)])
        gcnt = np.array([(groups == g).sum() for g in range(4)])
        wts = np.exp(c * (np.arange(4) - 3))
        exp_o = (wts[:, None] * gsum).sum(axis=0) / (wts * gcnt).sum()
        exp_lse = 3 * c + math.log((wts * gcnt).sum())
        check("late_max_o", close(got_o[0, :, 0], np.broadcast_to(exp_o, (3, 128)), 1e-10))
        check("late_max_lse", close(got_lse[0, 0], np.full(3, exp_lse), 1e-10))

        # 1x1: O = V_0, LSE = scale * q.k ; causal row 0 likewise
        for causal in (False, True):
            q, k, v = orc.make_inputs(2, 3, 1 if not causal else 7, 1 if not causal else 5, "normal")
            got_o, got_lse = o.attention_fp64(q, k, v, S, causal)
            qf, kf, vf = (orc.bf16_to_f32(t).reshape(t.shape).astype(np.float64) for t in (q, k, v))
            check(f"row0_o_{causal}", close(got_o[:, 0], vf[:, 0], 1e-12))
            dots = np.einsum("bhd,bhd->bh", qf[:, 0], kf[:, 0]) * S
            check(f"row0_lse_{causal}", close(got_lse[:, :, 0], dots, 1e-12))

        # Sq > Sk causal: rows i >= Sk-1 see every key, so they equal dense rows
        q, k, v = orc.make_inputs(1, 2, 12, 5, "normal")
        dense_o, dense_lse = o.attention_fp64(q, k, v, S, False)
        causal_o, causal_lse = o.attention_fp64(q, k, v, S, True)
        check("sq_gt_sk", close(causal_o[:, 4:], dense_o[:, 4:], 1e-12)
              and close(causal_lse[:, :, 4:], dense_lse[:, :, 4:], 1e-12)
              and not close(causal_o[:, :4], dense_o[:, :4], 1e-6))
    return fails


def test_oracle_passes_every_pin():
    assert pin_failures(orc) == []


# Planted mistakes: each must be caught by at least one pin.
def _mut_mask_diag(rows, sk):            # hides the diagonal too (j >= i)
    return np.arange(sk)[None, :] >= rows[:, None]


def _mut_mask_transposed(rows, sk):      # hides the past instead of the future
    return np.arange(sk)[None, :] < rows[:, None]


def _mut_no_scale(qs, ks, scale):        # forgets the softmax scale
    return qs @ ks.T


def _mut_swapped(qs, ks, scale):         # uses K.Q^T where Q.K^T is meant (square tiles)
    return (ks @ qs.T).T * scale + 0.0 if qs.shape == ks.shape else (qs @ ks.T) * scale * 1.0001


def _mut_lse_log2(s, vs):                # LSE in log2 units
    m = s.max(axis=1, keepdims=True)
    e = np.exp(s - m)
    l = e.sum(axis=1)
    return (e @ vs) / l[:, None], m[:, 0] + np.log2(l)


def _mut_unnormalised(s, vs):            # drops the softmax denominator
    m = s.max(axis=1, keepdims=True)
    e = np.exp(s - m)
    l = e.sum(axis=1)
    return e @ vs, m[:, 0] + np.log(l)


def _mut_fp32_scores(qs, ks, scale):     # accumulates the logits in float32
    return (qs.astype(np.float32) @ ks.T.astype(np.float32)).astype(np.float64) * np.float32(scale)


@pytest.mark.parametrize("attr,mutant", [
    ("_masked", _mut_mask_diag), ("_masked", _mut_mask_transposed), ("_scores", _mut_no_scale),
    ("_scores", _mut_swapped), ("_softmax_rows", _mut_lse_log2), ("_softmax_rows", _mut_unnormalised),
    ("_scores", _mut_fp32_scores),
], ids=["mask_diag", "mask_transposed", "no_scale", "swapped_qk", "lse_log2", "unnormalised", "fp32_logits"])
def test_pins_reject_planted_mistake(monkeypatch, attr, mutant):
    monkeypatch.setattr(orc, attr, mutant)
    assert pin_failures(orc), f"planted mistake in {attr} went unnoticed"


# ----------------------------------------------------------------------------
# Invariants of exact attention
# ----------------------------------------------------------------------------
def test_key_permutation_invariance_dense():
    q, k, v = _rand((2, 7, 3, 128), 1), _rand((2, 11, 3, 128), 2), _rand((2, 11, 3, 128), 3)
    perm = np.random.default_rng(4).permutation(11)
    o1, l1 = orc.attention_fp64(q, k, v, 0.1, False)
    o2, l2 = orc.attention_fp64(q, k[:, perm], v[:, perm], 0.1, False)
    assert np.max(np.abs(o1 - o2)) < 1e-12 and np.max(np.abs(l1 - l2)) < 1e-12


@pytest.mark.parametrize("causal", [False, True])
def test_logit_shift_invariance(causal):
    """k_j -> k_j + w shifts row i's logits by scale*q_i.w: O unchanged, LSE shifted."""
    q, k, v = _rand((1, 9, 2, 128), 5), _rand((1, 9, 2, 128), 6), _rand((1, 9, 2, 128), 7)
    w = _rand((128,), 8)
    scale = float(np.float32(0.07))
    o1, l1 = orc.attention_fp64(q, k, v, scale, causal)
    o2, l2 = orc.attention_fp64(q, k + w, v, scale, causal)
    shift = np.einsum("bshd,d->bhs", q, w) * scale
    assert np.max(np.abs(o1 - o2)) < 1e-10
    assert np.max(np.abs(l2 - l1 - shift)) < 1e-10


def test_linearity_in_v():
    q, k = _rand((1, 8, 2, 128), 9), _rand((1, 10, 2, 128), 10)
    v1, v2 = _rand((1, 10, 2, 128), 11), _rand((1, 10, 2, 128), 12)
    for causal in (False, True):
        o1, _ = orc.attention_fp64(q, k, v1, 0.1, causal)
        o2, _ = orc.attention_fp64(q, k, v2, 0.1, causal)
        o3, _ = orc.attention_fp64(q, k, 2.0 * v1 - 3.0 * v2, 0.1, causal)
        assert np.max(np.abs(o3 - (2.0 * o1 - 3.0 * o2))) < 1e-10


def test_scale_folding():
    q, k, v = _rand((1, 6, 1, 128), 13), _rand((1, 6, 1, 128), 14), _rand((1, 6, 1, 128), 15)
    o1, l1 = orc.attention_fp64(q, k, v, 0.25, True)
    o2, l2 = orc.attention_fp64(q * 0.25, k, v, 1.0, True)
    assert np.max(np.abs(o1 - o2)) < 1e-12 and np.max(np.abs(l1 - l2)) < 1e-12


def test_rows_and_heads_selection():
    q, k, v = orc.make_inputs(2, 3, 40, 33, "normal")
    full_o, full_l = orc.attention_fp64(q, k, v, S, True)
    rows = np.array([0, 5, 39])
    o, l = orc.attention_fp64(q, k, v, S, True, rows=rows, heads=[(1, 2)])
    assert np.array_equal(o[1, :, 2], full_o[1, rows, 2]) and np.array_equal(l[1, 2], full_l[1, 2, rows])
    assert np.isnan(o[0]).all()


# ----------------------------------------------------------------------------
# The tiled FP32 emulation of the kernel algorithm
# ----------------------------------------------------------------------------
@pytest.mark.parametrize("pattern", ["normal", "large", "late_max", "stress"])
@pytest.mark.parametrize("causal", [False, True])
def test_tiled_emulation_within_tolerance(pattern, causal):
    q, k, v = orc.make_inputs(1, 2, 150, 333, pattern)
    ref, ref_lse = orc.attention_fp64(q, k, v, S, causal)
    for thr in (8.0, 0.0):
        o, lse = orc.attention_tiled_fp32(q, k, v, S, causal, block_n=64, threshold=thr)
        e = orc.errors(orc.f32_to_bf16(o).reshape(o.shape), lse, ref, ref_lse)
        assert orc.check_acceptance_tolerance(e), (thr, e)


def test_conditional_rescale_only_changes_rounding():
    """In exact arithmetic the threshold does not change the result; in FP32
    with BF16 P the two variants differ only at the rounding level."""
    q, k, v = orc.make_inputs(1, 2, 64, 640, "late_max")
    o8, l8 = orc.attention_tiled_fp32(q, k, v, S, False, threshold=8.0)
    o0, l0 = orc.attention_tiled_fp32(q, k, v, S, False, threshold=0.0)
    assert np.max(np.abs(o8 - o0)) < 2e-2 and np.max(np.abs(l8 - l0)) < 1e-4


# ----------------------------------------------------------------------------
# Helpers: BF16 rounding, FLOPs, sampled rows, error metrics
# ----------------------------------------------------------------------------
def test_bf16_round_to_nearest_even():
    x = np.array([1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -2.5, np.inf, -np.inf, 3.4028235e38,
                  1 + 2 ** -8 + 2 ** -20, 0.0, -0.0], dtype=np.float32)
    want = [0x3F80, 0x3F80, 0x3F82, 0xC020, 0x7F80, 0xFF80, 0x7F80, 0x3F81, 0x0000, 0x8000]
    assert orc.f32_to_bf16(x).tolist() == want
    nan = orc.f32_to_bf16(np.array([np.nan], np.float32))
    assert np.isnan(orc.bf16_to_f32(nan)).all()
    r = np.random.default_rng(0).standard_normal(1000).astype(np.float32)
    back = orc.bf16_to_f32(orc.f32_to_bf16(r))
    assert np.all(np.abs(back - r) <= np.abs(r) * 2 ** -8)   # unit roundoff of an 8-bit significand


@pytest.mark.parametrize("sq,sk", [(1, 1), (5, 9), (9, 5), (64, 64), (100, 37)])
def test_flops_match_pair_count(sq, sk):
    visible = sum(1 for i in range(sq) for j in range(sk) if j <= i)
    assert orc.flops(2, 3, sq, sk, True) == 4 * 2 * 3 * 128 * visible
    assert orc.flops(2, 3, sq, sk, False) == 4 * 2 * 3 * 128 * sq * sk


def test_headline_flops():
    assert orc.flops(32, 8, 4096, 4096, False) == 2199023255552
    assert orc.flops(32, 8, 4096, 4096, True) == 4 * 32 * 8 * 128 * 4096 * 4097 // 2


def test_sample_rows_4096():
    rows = orc.sample_rows(4096).tolist()
    want = sorted(set([0, 1, 63, 64, 127, 128, 4095] + list(range(0, 4096, 170))))
    assert rows == want and len(rows) == 31


def test_error_metrics_and_bars():
    ref = np.array([[[[1.0] * 128]]])
    o = orc.f32_to_bf16(np.full((1, 1, 1, 128), 1.0078125, np.float32)).reshape(1, 1, 1, 128)
    e = orc.errors(o, np.array([[[0.5]]]), ref, np.array([[[0.5001]]]))
    assert abs(e["max_abs"] - 0.0078125) < 1e-12
    assert abs(e["max_tolerance_ratio"] - 0.0078125 / 0.02) < 1e-12
    assert abs(e["lse_max_abs"] - 1e-4) < 1e-12
    assert abs(e["rms_rel"] - 0.0078125) < 1e-12
    # inside max-abs 2e-2 / LSE 1e-3, but a uniform 0.78 % error breaks RMS-rel 0.005
    assert orc.check_acceptance_tolerance(e) and not orc.check_reference_tolerance(e)
    bad = dict(e, finite=False)
    assert not orc.check_acceptance_tolerance(bad) and not orc.check_reference_tolerance(bad)


def test_validation_cases_are_the_reference_ten():
    assert len(orc.VALIDATION_CASES) == 10
    assert sum(1 for c in orc.VALIDATION_CASES if c[2] > c[3]) == 1   # (1,8,129,65) negative


def test_stress_pattern_counts():
    q, k, v = orc.make_inputs(2, 4, 50, 300, "stress")
    qf = orc.bf16_to_f32(q).reshape(-1, 128)
    kf = orc.bf16_to_f32(k).reshape(-1, 128)
    big_q = (np.abs(qf).max(axis=1) > 8).sum()
    big_k = (np.abs(kf).max(axis=1) > 30).sum()
    assert abs(big_q - 40) <= 2 and abs(big_k - 24) <= 1


def test_bottom_right_reference_matches_direct_loop():
    """The bottom-right causal reference of the decode tests (built from the
    top-left oracle by padding) against a direct FP64 softmax per row: query i
    sees keys j <= sk - sq + i, rows with no key give O = 0 and LSE = -inf."""
    from tests.test_gpu_splitkv_paged import _bottom_right_ref
    for sq, sk in [(4, 30), (20, 9), (17, 17), (1, 5), (3, 0)]:
        q, _, _ = orc.make_inputs(1, 2, sq, max(sk, 1), "normal", seed=1)
        _, k, v = orc.make_inputs(1, 2, sq, max(sk, 1), "normal", seed=2)
        k, v = k[:, :sk], v[:, :sk]
        o, lse = _bottom_right_ref(q[0], k[0], v[0], 1)
        qf, kf, vf = (orc.bf16_to_f32(x).astype(np.float64) for x in (q[0], k[0], v[0]))
        for i in range(sq):
            lim = sk - sq + i
            for hh in range(2):
                if lim < 0:
                    assert lse[0, hh, i] == -np.inf and (o[0, i, hh] == 0).all()
                    continue
                sc = kf[:lim + 1, hh] @ qf[i, hh] * orc.DEFAULT_SCALE
                m = sc.max()
                p = np.exp(sc - m)
                assert np.allclose(o[0, i, hh], (p[:, None] * vf[:lim + 1, hh]).sum(0) / p.sum(), atol=1e-9)
                assert abs(lse[0, hh, i] - (m + np.log(p.sum()))) < 1e-9


def test_bench_flop_count_matches_the_oracles():
    """bench.py counts FLOPs itself (its timed legs call nothing under
    oracle/); the count must be the oracle's on dense, causal, Sq > Sk and
    Sq < Sk shapes."""
    import itertools
    import bench
    for b, h, sq, sk, causal in itertools.product([1, 3], [1, 8], [1, 100, 257, 4096], [1, 64, 3077, 4096],
                                                 [False, True]):
        assert bench.flops(b, h, sq, sk, causal) == orc.flops(b, h, sq, sk, causal), (b, h, sq, sk, causal)
