#pragma once
// Public C ABI of the MI355X (gfx950) BF16 BSHD D=128 attention forward.
//
// Drop-in for the reference interface include/fav4_bshd.h:1-20: the argument
// block and both exported symbols keep the same layout, names, argument
// meaning and return codes, so callers built against the reference (C/C++ or
// the ctypes binding of benchmarks/bshd.py:56-74) run unchanged.
#include <hip/hip_runtime.h>

// 64-byte argument block (offsets: q 0, k 8, v 16, o 24, lse 32, batch 40,
// heads 44, sq 48, sk 52, scale 56).  Replaces include/fav4_bshd.h:4-10.
struct Fav4Args {
    const void *q, *k, *v;   // BF16 [batch, sq|sk, heads, 128], contiguous
    void *o;                 // BF16 [batch, sq, heads, 128], contiguous
    float *lse;              // optional FP32 [batch, heads, sq]; NULL = not written
    int batch, heads, sq, sk;
    float scale;             // softmax scale applied to Q.K^T (positive, finite)
};

// Contract (same as include/fav4_bshd.h:12-18):
//  * Q/K/V/O are device-resident, 16-byte aligned, non-overlapping and
//    contiguous in the native [batch, sequence, heads, 128] layout; Q, K and V
//    have the same number of heads; sq and sk may differ.
//  * causal = 1 is top-left causal: key j is visible to query i iff j <= i.
//  * The call only enqueues work on `stream` (which must belong to the calling
//    thread's current device); it allocates nothing and never synchronizes.
//  * Returns 0 on success, hipErrorInvalidValue (1) for rejected arguments
//    (checked before any HIP call), otherwise the launch status.
//
// Config IDs (gfx950 tile shapes; BM = query rows per workgroup, BN = keys per
// K/V tile, 32 query rows per wave64):
//  0: Auto (fav4_bshd_select_config)
//  1: BM 128 / BN 64, 4 waves, 2 LDS stages  -- short query lengths, small grids
//  2: BM 256 / BN 64, 8 waves, 2 LDS stages  -- default for sq >= 256
//  3: BM 256 / BN 64, 8 waves, 3 LDS stages with QK^T(t+1) pipelined
//     beside softmax(t)
//
// Replaces include/fav4_bshd.h:19 (fav4_bshd_forward).
extern "C" int fav4_bshd_forward(const Fav4Args* args, int causal, int config, hipStream_t stream);
// Replaces include/fav4_bshd.h:20 (fav4_bshd_select_config): the config ID
// that config 0 resolves to for these arguments (-1 for a NULL pointer).
extern "C" int fav4_bshd_select_config(const Fav4Args* args);
