"""CPU oracle for the BF16 BSHD D=128 attention forward (TEST INFRASTRUCTURE ONLY).

This module checks results and is never the product: only ``tests/``, the package's
``smoke`` check and ``bench.py``'s ``cpu_baseline`` leg may import it.  The
product path (``libfav4_bshd.so``) never calls into it and has no CPU fallback.

What it restates, and from where (paths relative to the reference repo):

* ``attention_fp64``  -- FP64 textbook attention exactly as the reference
  harness validates it, ``benchmarks/bshd.py:90-100``: scores = Q.K^T * scale,
  ``-inf`` where key j > query i (top-left causal, ``bshd.py:96``, independent
  of Sq != Sk), ``lse = logsumexp(scores)`` (natural log), ``O = softmax.V``.
  The reference divides by ``math.sqrt(128)``; the ABI carries the scale as a
  float32, so the oracle multiplies by that float32 value in FP64.  For
  1/sqrt(128) the two differ by < 3e-8 relative.
* ``errors`` / ``check_reference_tolerance`` / ``check_acceptance_tolerance``
  -- the error metrics and BF16 tolerances of ``benchmarks/bshd.py:22-32``
  (elementwise |o-ref| <= 0.01 + 0.01|ref|, RMS-relative <= 0.005, LSE
  max-abs <= 2e-4, all finite) and the looser acceptance bar of the port
  (max-abs <= 2e-2, LSE max-abs <= 1e-3, finite).
* ``make_inputs``     -- the input patterns of ``benchmarks/bshd.py:77-87``
  (normal, zero, large, negative, late_max) plus the large-logit ``stress``
  pattern (10 % of Q rows x16, 1 % of K rows x64).
* ``flops``           -- the FLOP convention of ``benchmarks/bshd.py:169-170``
  and ``README.md:59`` (useful QK+PV only), generalised to Sq != Sk.
* ``sample_rows``     -- the benchmark's sampled check rows, ``bshd.py:147-148``.
* ``VALIDATION_CASES``-- the ten validation cases of ``bshd.py:112-115``.
* ``attention_tiled_fp32`` -- an FP32 emulation of the kernel algorithm of
  ``src/bshd_kernel.hpp:107,148-208``: log2-domain online softmax with the
  FA4 conditional rescale (threshold 8), P rounded to BF16 before the PV
  product, FP32 row sums, ``LSE = m*ln2 + ln(l)``.  Used to show that the
  threshold does not change the result beyond rounding and to bound the
  error the BF16 P rounding contributes.

How each function is pinned (tests/test_oracle.py, tests/golden/):
closed forms (zero / negative / late_max / 1x1 / causal row 0), an
independent pure-Python brute force on tiny shapes committed as golden
vectors, invariants (key permutation, logit shift, linearity in V), and
planted mutants of this module that those checks must reject.
"""
from __future__ import annotations

import math

import numpy as np

D = 128
LOG2E = 1.4426950408889634
LN2 = 0.6931471805599453

# benchmarks/bshd.py:112-115: (batch, heads, sq, sk, pattern)
VALIDATION_CASES = [
    (1, 1, 1, 1, "normal"), (2, 3, 17, 31, "normal"), (2, 3, 63, 65, "normal"),
    (1, 8, 127, 129, "normal"), (3, 8, 193, 257, "normal"), (1, 8, 256, 512, "zero"),
    (1, 8, 256, 512, "large"), (1, 8, 256, 512, "late_max"), (1, 8, 129, 65, "negative"),
    (2, 8, 512, 512, "normal"),
]

SEED = 11939  # benchmarks/bshd.py:201
DEFAULT_SCALE = float(np.float32(1.0 / math.sqrt(D)))


# ----------------------------------------------------------------------------
# BF16 helpers (numpy has no bfloat16; BF16 tensors are carried as uint16 bits)
# ----------------------------------------------------------------------------
def f32_to_bf16(x) -> np.ndarray:
    """Round float32 to BF16 bits with round-to-nearest-even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    out = rounded.astype(np.uint16)
    if nan.any():
        out[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return out


def bf16_to_f32(b) -> np.ndarray:
    """Widen BF16 bits (uint16) to float32 exactly."""
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


# ----------------------------------------------------------------------------
# Inputs (benchmarks/bshd.py:77-87) and the large-logit stress pattern
# ----------------------------------------------------------------------------
def make_inputs(b: int, h: int, sq: int, sk: int, pattern: str = "normal", seed: int = SEED):
    """Return BF16 bits (uint16) for Q [b,sq,h,128], K and V [b,sk,h,128].

    Values are N(0,1) float32 from a seeded PCG64 generator rounded to BF16,
    then overwritten per ``pattern`` as in ``benchmarks/bshd.py:81-86``.
    ``stress`` scales a seeded exact 10 % of Q (b,s,h) rows by 16 and 1 % of
    K rows by 64 (the ragged large-logit validation shape)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    q = rng.standard_normal((b, sq, h, D), dtype=np.float32)
    k = rng.standard_normal((b, sk, h, D), dtype=np.float32)
    v = rng.standard_normal((b, sk, h, D), dtype=np.float32)
    q, k, v = (bf16_to_f32(f32_to_bf16(t)).reshape(t.shape) for t in (q, k, v))
    if pattern == "normal":
        pass
    elif pattern == "zero":
        q[:] = 0
        k[:] = 0
    elif pattern == "large":
        q *= 4
        k *= 4
    elif pattern == "negative":
        q[:] = 8
        k[:] = -8
    elif pattern == "late_max":
        q[:] = 1
        k[:] = (np.arange(sk) // 64).astype(np.float32)[None, :, None, None]
    elif pattern == "stress":
        qrows = q.reshape(-1, D)
        krows = k.reshape(-1, D)
        qi = rng.choice(qrows.shape[0], size=max(1, qrows.shape[0] // 10), replace=False)
        ki = rng.choice(krows.shape[0], size=max(1, krows.shape[0] // 100), replace=False)
        qrows[qi] *= 16
        krows[ki] *= 64
    else:
        raise ValueError(f"unknown pattern {pattern!r}")
    return f32_to_bf16(q).reshape(q.shape), f32_to_bf16(k).reshape(k.shape), f32_to_bf16(v).reshape(v.shape)


# ----------------------------------------------------------------------------
# FP64 oracle (benchmarks/bshd.py:90-100)
# ----------------------------------------------------------------------------
def _scores(qs: np.ndarray, ks: np.ndarray, scale: float) -> np.ndarray:
    """[rows, D] x [Sk, D] -> [rows, Sk] scaled logits in FP64."""
    return (qs @ ks.T) * scale


def _masked(rows: np.ndarray, sk: int) -> np.ndarray:
    """True where key j is hidden from query row i: j > i (top-left causal)."""
    return np.arange(sk)[None, :] > rows[:, None]


def _softmax_rows(s: np.ndarray, vs: np.ndarray):
    """Row softmax of FP64 logits times V; returns (O [rows,D], natural-log LSE [rows])."""
    m = s.max(axis=1, keepdims=True)
    e = np.exp(s - m)
    l = e.sum(axis=1)
    return (e @ vs) / l[:, None], m[:, 0] + np.log(l)


def _as_f64(x) -> np.ndarray:
    x = np.asarray(x)
    if x.dtype == np.uint16:
        x = bf16_to_f32(x).reshape(x.shape)
    return x.astype(np.float64, copy=False)


def attention_fp64(q, k, v, scale: float = DEFAULT_SCALE, causal: bool = False, rows=None,
                   heads=None):
    """FP64 attention forward on BSHD tensors.

    q: [B,Sq,H,D], k/v: [B,Sk,H,D] (BF16 bits as uint16, or float arrays).
    ``rows`` selects query rows (default all); ``heads`` optionally restricts
    the computed (b, h) pairs to a list (others are left NaN).
    Returns (O [B,len(rows),H,D] float64, LSE [B,H,len(rows)] float64)."""
    bq, sq, hq, dq = np.shape(q)
    sk = np.shape(k)[1]
    assert dq == D and np.shape(k) == np.shape(v) and np.shape(k)[0] == bq and np.shape(k)[2] == hq
    rows = np.arange(sq) if rows is None else np.asarray(rows, dtype=np.int64)
    pairs = [(b, h) for b in range(bq) for h in range(hq)] if heads is None else list(heads)
    out = np.full((bq, len(rows), hq, D), np.nan)
    lse = np.full((bq, hq, len(rows)), np.nan)
    hidden = _masked(rows, sk) if causal else None
    for b, h in pairs:
        qs = _as_f64(np.asarray(q)[b, rows, h])
        ks = _as_f64(np.asarray(k)[b, :, h])
        vs = _as_f64(np.asarray(v)[b, :, h])
        s = _scores(qs, ks, float(np.float32(scale)))
        if causal:
            s[hidden] = -np.inf
        o_bh, lse_bh = _softmax_rows(s, vs)
        out[b, :, h] = o_bh
        lse[b, h] = lse_bh
    return out, lse


# ----------------------------------------------------------------------------
# FP32 emulation of the tiled kernel algorithm (src/bshd_kernel.hpp:148-208)
# ----------------------------------------------------------------------------
def attention_tiled_fp32(q, k, v, scale: float = DEFAULT_SCALE, causal: bool = False,
                         block_n: int = 64, threshold: float = 8.0):
    """Online-softmax forward in FP32 with the FA4 conditional rescale.

    Per key tile: row max of raw logits, ``candidate = max(m, rowmax*scale2)``
    (log2 units), the base moves only on the first tile or when
    ``candidate > m + threshold`` (``threshold=0`` gives the classic rescale
    on every increase), ``alpha = exp2(m - next)``, ``p = exp2(s*scale2 -
    next)`` in FP32, P rounded to BF16 for the PV product, the row sum kept in
    FP32, ``O = acc / l`` and ``LSE = m*ln2 + ln(l)``.  Fully-masked tiles are
    skipped as the kernel's causal loop bound does.  Returns float32 O and LSE
    with the same shapes as ``attention_fp64``."""
    qf = _as_f64(q).astype(np.float32)
    kf = _as_f64(k).astype(np.float32)
    vf = _as_f64(v).astype(np.float32)
    bq, sq, hq, _ = qf.shape
    sk = kf.shape[1]
    scale2 = np.float32(np.float32(scale) * np.float32(LOG2E))
    out = np.empty((bq, sq, hq, D), np.float32)
    lse = np.empty((bq, hq, sq), np.float32)
    rows = np.arange(sq)
    for b in range(bq):
        for h in range(hq):
            qs, ks, vs = qf[b, :, h], kf[b, :, h], vf[b, :, h]
            m = np.full(sq, -np.inf, np.float32)
            l = np.zeros(sq, np.float32)
            acc = np.zeros((sq, D), np.float32)
            end = min(sk, sq) if causal else sk
            for start in range(0, end, block_n):
                stop = min(start + block_n, sk)
                s = (qs @ ks[start:stop].T).astype(np.float32)
                cols = np.arange(start, stop)
                if causal:
                    s[cols[None, :] > rows[:, None]] = -np.inf
                rowmax = s.max(axis=1)
                with np.errstate(invalid="ignore"):
                    cand = np.maximum(m, rowmax * scale2)
                    first = start == 0
                    update = np.ones(sq, bool) if first else cand > m + np.float32(threshold)
                    nxt = np.where(update, cand, m).astype(np.float32)
                    alpha = np.zeros(sq, np.float32) if first else np.exp2(m - nxt).astype(np.float32)
                    # Rows whose whole tile is masked keep nxt = m = -inf only if
                    # no earlier key was visible; top-left causal always shows key 0.
                    p = np.exp2(s * scale2 - nxt[:, None]).astype(np.float32)
                pb = bf16_to_f32(f32_to_bf16(p)).reshape(p.shape)
                acc = acc * alpha[:, None] + pb @ vs[start:stop]
                l = l * alpha + p.sum(axis=1, dtype=np.float32)
                m = nxt
            out[b, :, h] = acc / l[:, None]
            lse[b, h] = m * np.float32(LN2) + np.log(l)
    return out, lse


# ----------------------------------------------------------------------------
# Error metrics and tolerances (benchmarks/bshd.py:22-32)
# ----------------------------------------------------------------------------
def errors(o, lse, ref, ref_lse) -> dict:
    """Error metrics of a BF16 output against the FP64 oracle.

    ``o`` / ``ref``: [B,rows,H,D]; ``lse`` / ``ref_lse``: [B,H,rows] or None."""
    o = _as_f64(o)
    ref = np.asarray(ref, np.float64)
    diff = np.abs(o - ref)
    ratio = diff / (0.01 + 0.01 * np.abs(ref))
    rms_rel = math.sqrt(float(np.mean(diff ** 2))) / max(math.sqrt(float(np.mean(ref ** 2))), 1e-30)
    lse_err = None
    if lse is not None:
        lse_err = float(np.max(np.abs(np.asarray(lse, np.float64) - ref_lse)))
        if not np.all(np.isfinite(lse)):
            lse_err = float("inf")
    return dict(max_abs=float(diff.max()) if diff.size else 0.0, rms_rel=rms_rel,
                max_tolerance_ratio=float(ratio.max()) if ratio.size else 0.0,
                lse_max_abs=lse_err, finite=bool(np.all(np.isfinite(o))))


def check_reference_tolerance(e: dict) -> bool:
    """The reference harness's BF16 bar (benchmarks/bshd.py:25,30-31)."""
    return (e["finite"] and e["max_tolerance_ratio"] <= 1 and e["rms_rel"] <= 0.005
            and (e["lse_max_abs"] is None or e["lse_max_abs"] <= 2e-4))


def check_acceptance_tolerance(e: dict) -> bool:
    """The port's acceptance bar: max-abs <= 2e-2, LSE max-abs <= 1e-3, finite."""
    return (e["finite"] and e["max_abs"] <= 2e-2
            and (e["lse_max_abs"] is None or e["lse_max_abs"] <= 1e-3))


# ----------------------------------------------------------------------------
# FLOP convention and sampled rows
# ----------------------------------------------------------------------------
def flops(b: int, h: int, sq: int, sk: int, causal: bool) -> int:
    """Useful QK+PV FLOPs (benchmarks/bshd.py:169-170, README.md:59).

    Dense: 4*B*H*D*Sq*Sk.  Causal (top-left): 4*B*H*D*sum_{i<Sq} min(i+1, Sk),
    which is 4*B*H*D*S(S+1)/2 when Sq == Sk == S."""
    if not causal:
        return 4 * b * h * D * sq * sk
    full = min(sq, sk)                      # rows 0..full-1 see i+1 keys
    area = full * (full + 1) // 2 + max(0, sq - sk) * sk
    return 4 * b * h * D * area


def sample_rows(n: int) -> np.ndarray:
    """Rows the benchmark checks at each timed shape (benchmarks/bshd.py:147-148)."""
    rows = {0, 1, 63, 64, 127, 128, n - 1} | set(range(0, n, max(1, n // 24)))
    return np.array(sorted(r for r in rows if 0 <= r < n), dtype=np.int64)
