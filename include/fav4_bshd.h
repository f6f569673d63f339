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
//  0: Auto: config 1 for sq <= 768 (dense) or sq <= 1024 (causal), or when
//     config 2 would have fewer work items than the device has CUs (items:
//     B*H*ceil(sq/256) q tiles; causal: B*H*ceil(ceil(sq/256)/2) q-tile
//     pairs), else config 2
//  1: BM 128 / BN 64, 4 waves, 2 LDS stages
//  2: BM 256 / BN 64, 8 waves, 2 LDS stages
//  3: BM 256 / BN 64, 8 waves, 3 LDS stages with QK^T(t+1) pipelined
//     beside softmax(t)
//
// Replaces include/fav4_bshd.h:19 (fav4_bshd_forward).
extern "C" int fav4_bshd_forward(const Fav4Args* args, int causal, int config, hipStream_t stream);
// Replaces include/fav4_bshd.h:20 (fav4_bshd_select_config): the config ID
// that config 0 resolves to for these arguments in a dense call (the mask is
// not an argument here; a causal call counts q-tile pairs, see above, and
// fav4_bshd_select_config_masked reports its choice), -1 for a NULL pointer.
extern "C" int fav4_bshd_select_config(const Fav4Args* args);
// No counterpart in the reference: the config ID config 0 resolves to for a
// call with this mask (causal 0 or 1), for callers that label causal runs;
// -1 for a NULL pointer or another mask value.
extern "C" int fav4_bshd_select_config_masked(const Fav4Args* args, int causal);

// ---- Split-KV forward --------------------------------------------------------
// No counterpart in the reference.  It is for callers whose B * H * ceil(Sq/256)
// work items are too few to fill the GPU while Sk is long: each item's key
// range is cut into `splits` chunks attended in parallel, then merged by their
// log-sum-exp.  Results match fav4_bshd_forward within the same tolerances
// (not bitwise: the chunks' BF16 weights are rounded against their own base).
// Same argument contract as fav4_bshd_forward (config is always Auto), plus:
//  * splits: 0 = library choice (enough chunks to fill every CU once, >= 4
//    key tiles per chunk, at most 64 chunks; for Sq <= 32 one-wave
//    workgroups over 32-key tiles, three per CU, at most 128 chunks, 256
//    when there are only one or two (batch, K/V head) tiles; for
//    Sq > 32 then the count up to that one, 1 included, with the lowest
//    time predicted by a cost model fitted on MI355X), else 1..256 (clamped
//    to the key tiles);
//    splits resolving to 1 run fav4_bshd_forward and need no workspace;
//  * workspace: caller-owned device memory, 256-byte aligned, at least
//    fav4_bshd_splitkv_workspace_size() bytes, not shared with a concurrent
//    call; its contents on entry do not matter and are scratch afterwards;
//  * Sq <= 2^22.
// Returns 0, hipErrorInvalidValue (1) for rejected arguments or a missing /
// small / misaligned workspace, else the launch status.  Allocates nothing.
extern "C" int fav4_bshd_forward_splitkv(const Fav4Args* args, int causal, int splits, void* workspace,
                                         size_t workspace_bytes, hipStream_t stream);
// Workspace bytes fav4_bshd_forward_splitkv needs for these arguments and
// `splits` (0 when it needs none), or -1 for rejected arguments.
extern "C" long long fav4_bshd_splitkv_workspace_size(const Fav4Args* args, int causal, int splits);
// The chunk count that splits = 0 resolves to (1 = no split), or -1.
extern "C" int fav4_bshd_splitkv_select(const Fav4Args* args, int causal);

// Split-KV with grouped K/V heads (GQA / MQA); no counterpart in the
// reference.  K and V are [B, Sk, kv_heads, 128] with kv_heads dividing
// args->heads (query head h reads K/V head h / (heads / kv_heads)), as in
// fav4_bshd_forward_gqa; otherwise the contract of the split-KV calls above,
// which are these with kv_heads = heads.  For Sq <= 32 (decode) the query
// heads that share a K/V head are packed into one 32-row tile (row =
// head-in-group * Sq + query), so each K/V head is streamed once per group
// instead of once per query head.  Per row the result is bitwise that of the
// MHA split-KV call on K/V with their heads repeated group-wise at the same
// explicit chunk count.  Splits resolving to 1 run fav4_bshd_forward_gqa.
// For Sq <= 32, (heads / kv_heads) * Sq must stay below 2^23 (one group's
// partial rows within a 4 GiB buffer bound).
extern "C" int fav4_bshd_forward_splitkv_gqa(const Fav4Args* args, int kv_heads, int causal, int splits,
                                             void* workspace, size_t workspace_bytes, hipStream_t stream);
extern "C" long long fav4_bshd_splitkv_gqa_workspace_size(const Fav4Args* args, int kv_heads, int causal,
                                                          int splits);
extern "C" int fav4_bshd_splitkv_gqa_select(const Fav4Args* args, int kv_heads, int causal);

// Split-KV with grouped K/V heads and no workspace argument.  No counterpart
// in the reference: it is for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).  Exactly fav4_bshd_forward_splitkv_gqa (same checks, plan,
// kernels and results, bitwise) except that the chunk partials live in a
// 64 MiB array inside the library, one copy per GPU, held until the process
// ends.  Plans whose workspace (fav4_bshd_splitkv_gqa_workspace_size) exceeds
// 64 MiB = 67108864 bytes return hipErrorInvalidValue; splits resolving to 1
// run fav4_bshd_forward_gqa.  Every call on one GPU shares that GPU's array:
// calls that overlap on one GPU (other streams, other host threads) race and
// give undefined results; calls ordered on one stream are safe.  The first
// call on a device looks the array's address up (hipGetSymbolAddress) and
// returns that lookup's error if it fails; the address is kept for the life
// of the process, so after hipDeviceReset of a GPU (which frees the array)
// this entry point must not be called on that GPU again.  The array belongs
// to the library's code object: any process that runs this library's
// kernels on a GPU holds its 64 MiB there, whichever entry points it calls.
// Allocates nothing.
extern "C" int fav4_bshd_forward_splitkv_gqa_noalloc(const Fav4Args* args, int kv_heads, int causal, int splits,
                                                     hipStream_t stream);

// ---- Grouped-query / multi-query attention ----------------------------------
// No counterpart in the reference (its README lists GQA as unsupported).  The
// same contract as fav4_bshd_forward, except that K and V are
// [batch, sk, kv_heads, 128] with kv_heads dividing heads: query head h reads
// K/V head h / (heads / kv_heads).  kv_heads == heads is exactly
// fav4_bshd_forward.  Returns hipErrorInvalidValue also for kv_heads <= 0,
// kv_heads > heads or heads % kv_heads != 0.  The key-side overflow limit
// counts the K/V heads: sk * kv_heads * 128 must stay below 2^31 (the
// split-KV calls below keep the same limit).
extern "C" int fav4_bshd_forward_gqa(const Fav4Args* args, int kv_heads, int causal, int config,
                                     hipStream_t stream);

// ---- Variable-length (packed) sequences ---------------------------------------
// No counterpart in the reference.  `batch` sequences are packed along the
// row axis: sequence b's queries are rows [cu_seqlens_q[b], cu_seqlens_q[b+1])
// of Q/O and its keys rows [cu_seqlens_k[b], cu_seqlens_k[b+1]) of K/V; each
// sequence is attended on its own (top-left causal within the sequence when
// causal = 1), exactly as fav4_bshd_forward would on that sequence alone
// (bitwise, for sequences of at least one key).  A sequence with no keys gets
// O = 0 and LSE = -inf.  GQA as in fav4_bshd_forward_gqa.  causal = 2:
// bottom-right causal, query i of a sequence with sq queries and sk keys sees
// keys j <= sk - sq + i (a prefill chunk against a cache); with sq > sk the
// first sq - sk rows see none and get O = 0, LSE = -inf.  For sq = sk it is
// bitwise the causal = 1 result.
struct Fav4VarlenArgs {
    const void *q, *k, *v;             // BF16 [total_q | total_k, heads | kv_heads, 128], contiguous
    void *o;                           // BF16 [total_q, heads, 128], contiguous
    float *lse;                        // optional FP32 [heads, total_q]; NULL = not written
    const int *cu_seqlens_q;           // device int32 [batch + 1], non-decreasing from 0
    const int *cu_seqlens_k;           // device int32 [batch + 1], non-decreasing from 0
    int batch, heads, kv_heads;        // kv_heads divides heads
    int max_seqlen_q, max_seqlen_k;    // bounds of every sequence's length
    int total_q, total_k;              // rows of Q/O and of K/V
    float scale;
};
// The offsets are read on the device and clamped to [0, total] and to the
// maximum lengths (so malformed offsets cannot move an access outside the
// buffers; they do give undefined results).  Returns 0, hipErrorInvalidValue
// (1) for rejected arguments (checked before any HIP call: NULL pointers,
// sizes < 1, kv_heads not dividing heads, bad causal / scale, misalignment,
// max_seqlen * heads * 256 >= 2^32), else the launch status.  Allocates
// nothing and never synchronizes.
extern "C" int fav4_bshd_forward_varlen(const Fav4VarlenArgs* args, int causal, hipStream_t stream);

// Split-KV of packed sequences (no counterpart in the reference): the decode
// step of continuous batching, each sequence with 1-32 new queries and its own
// cache length.  For max_seqlen_q <= 32 and causal = 0 the query heads that
// share a K/V head are packed into 32-row tiles (row = head-in-group *
// max_seqlen_q + query) and every sequence's keys are cut into chunks of one
// common number of key tiles (a sequence gets as many chunks as its keys
// need), merged by their log-sum-exp as in fav4_bshd_forward_splitkv_gqa;
// with equal lengths the result is bitwise that call's on the same data at
// the same chunk count.  Otherwise, for causal 0 or 1 (max_seqlen_q > 32,
// or causal = 1: top-left causal decode sees at most 32 keys), the call takes
// one chunk, i.e. runs fav4_bshd_forward_varlen, and needs no workspace.
// causal = 2 (these calls and the paged ones only): bottom-right causal,
// query i of a sequence with sq queries and sk keys sees keys j <= sk - sq + i
// (the last query sees them all; with sq > sk the first sq - sk rows see
// none: O = 0, LSE = -inf).  Decode (max_seqlen_q <= 32) is planned like a
// dense call; prefill (max_seqlen_q > 32, 8-wave kernels) with the contiguous
// prefill plan at the max lengths, counting for each 256-row q tile only the
// keys up to its last row's diagonal (chunks past it are empty and end at
// once).  Decode always runs the split kernels, one chunk included (with a
// workspace); prefill with one chunk runs fav4_bshd_forward_varlen, which
// takes the same mask, and needs none.  Same argument contract
// as fav4_bshd_forward_varlen (O and LSE rows, empty sequences, offset
// clamping), plus:
//  * splits: 0 = library choice (the chunk size the contiguous split-KV Auto
//    plan gives at the mean key length total_k / batch, at most 64 key tiles
//    when that mean is below 3/4 of max_seqlen_k, enlarged so that the
//    longest sequence needs at most 256 chunks), else 1..256 chunks of the
//    longest sequence (clamped to its key tiles);
//  * workspace as for fav4_bshd_forward_splitkv, of
//    fav4_bshd_splitkv_varlen_workspace_size() bytes;
//  * (heads / kv_heads) * max_seqlen_q < 2^23.
// The two queries read only the sizes (pointers may be NULL) and return -1
// for rejected arguments.
extern "C" int fav4_bshd_forward_splitkv_varlen(const Fav4VarlenArgs* args, int causal, int splits,
                                                void* workspace, size_t workspace_bytes, hipStream_t stream);
extern "C" long long fav4_bshd_splitkv_varlen_workspace_size(const Fav4VarlenArgs* args, int causal, int splits);
extern "C" int fav4_bshd_splitkv_varlen_select(const Fav4VarlenArgs* args, int causal);

// ---- Paged K/V caches ---------------------------------------------------------
// No counterpart in the reference.  Attention over paged K/V caches: packed
// sequences of new queries (Q/O/LSE as in Fav4VarlenArgs; decode when
// max_seqlen_q <= 32, else chunked prefill), each with its own number of
// cached keys, stored in fixed-size pages.  Key j of
// sequence b is row block_table[b * max_pages_per_seq + j / page_size] *
// page_size + j % page_size of the caches.  causal is 0 (dense) or 2
// (bottom-right, as for fav4_bshd_forward_splitkv_varlen); top-left (1) is
// rejected, since a top-left decode row would see only its cache's first keys.
// Decode runs the packed split-KV kernels (query heads of a K/V head share
// 32-row tiles; chunks of a common number of key tiles, merged by
// log-sum-exp), so per row the result is bitwise that of
// fav4_bshd_forward_splitkv_varlen on the same keys stored contiguously, at
// the same chunk count.  Prefill runs the 8-wave split-KV kernels (256-row q
// tiles, 64-key tiles) with the contiguous prefill plan at the max lengths,
// bitwise fav4_bshd_forward_splitkv_gqa's on a batch of equal lengths.
struct Fav4PagedArgs {
    const void *q;                     // BF16 [total_q, heads, 128], contiguous
    const void *k_cache, *v_cache;     // BF16 [num_pages, page_size, kv_heads, 128], contiguous
    void *o;                           // BF16 [total_q, heads, 128], contiguous
    float *lse;                        // optional FP32 [heads, total_q]; NULL = not written
    const int *cu_seqlens_q;           // device int32 [batch + 1], non-decreasing from 0
    const int *seqlens_k;              // device int32 [batch]: cached keys per sequence
    const int *block_table;            // device int32 [batch, max_pages_per_seq]: page numbers
    int batch, heads, kv_heads;        // kv_heads divides heads
    int max_seqlen_q, max_seqlen_k;    // bounds of every sequence's query / key count
    int total_q, total_k;              // rows of Q/O; cached keys over the batch (Auto only)
    int num_pages, page_size, max_pages_per_seq;
    float scale;
};
// Checks (before any HIP call; hipErrorInvalidValue otherwise): the pointers,
// sizes >= 1 (total_k >= 0), kv_heads dividing heads, causal 0 or 2, a finite
// positive scale, max_seqlen_q <= 2^22, page_size a multiple of 32 (decode)
// or 64 (prefill), max_seqlen_k <= max_pages_per_seq * page_size and <= 2^19
// (a chunk spans at most 64 key tiles), page_size * kv_heads * 256 < 2^32,
// max_seqlen_q * heads * 256 < 2^32, for decode (heads / kv_heads) *
// max_seqlen_q < 2^23, 16-byte aligned Q/O/caches and 4-byte aligned int
// arrays and LSE.
// Device-read values are clamped (query offsets to [0, total_q], key counts to
// [0, max_seqlen_k], page numbers to [0, num_pages)), so malformed tables give
// undefined results but no access outside the buffers.  A sequence with no
// keys gets O = 0 and LSE = -inf; one with no queries writes nothing.
//  * splits: 0 = the Auto count of fav4_bshd_forward_splitkv_varlen on these
//    sizes, else 1..256; either is raised if needed so that no chunk spans
//    more than 64 key tiles.  One chunk still runs the split kernels.
//  * workspace as for fav4_bshd_forward_splitkv, of
//    fav4_bshd_splitkv_paged_workspace_size() bytes (never 0).
// The two queries read only the sizes (pointers may be NULL) and return -1
// for rejected arguments.
extern "C" int fav4_bshd_forward_splitkv_paged(const Fav4PagedArgs* args, int causal, int splits,
                                               void* workspace, size_t workspace_bytes, hipStream_t stream);
extern "C" long long fav4_bshd_splitkv_paged_workspace_size(const Fav4PagedArgs* args, int causal, int splits);
extern "C" int fav4_bshd_splitkv_paged_select(const Fav4PagedArgs* args, int causal);

// ---- Arbitrary strides -----------------------------------------------------
// No counterpart in the reference.  Q / O are read as [B, Sq, H, 128] and K /
// V as [B, Sk, kv_heads, 128] views with the element (BF16) strides given per
// tensor; the 128 head dims must be contiguous.  Covers BHSD
// ([B, H, S, 128]: batch = H*S*128, seq = 128, head = S*128), packed QKV
// ([B, S, 3, H, 128]: seq = 3*H*128) and other views.  LSE stays [B, H, Sq].
// Query head h reads K/V head h / (heads / kv_heads).  O rows must not
// overlap each other or Q/K/V (results are undefined otherwise).
struct Fav4Strides {
    long long batch, seq, head;
};
// Returns 0, hipErrorInvalidValue (1) before any HIP call for the checks of
// fav4_bshd_forward (except the contiguous-BSHD overflow limits) plus: NULL
// strides, a negative batch / head stride, a seq stride <= 0, a stride that
// is not a multiple of 8 elements, kv_heads not dividing heads, one
// (batch, head) slice spanning 4 GiB or more, or a view spanning more than
// 2^48 bytes; else the launch status.  Same
// configs and numerics as fav4_bshd_forward (bitwise equal on the same data).
extern "C" int fav4_bshd_forward_strided(const Fav4Args* args, int kv_heads, const Fav4Strides* q,
                                         const Fav4Strides* k, const Fav4Strides* v, const Fav4Strides* o,
                                         int causal, int config, hipStream_t stream);
