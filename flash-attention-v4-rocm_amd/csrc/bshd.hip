// C-ABI host dispatch for the gfx950 attention forward.
//
// Mirrors the reference dispatch src/bshd.hip:1-38: the same argument checks
// in the same order (all before any HIP call), config 0 -> auto selection,
// config -> kernel instantiation, and hipGetLastError() after the launch.
#include "fav4_bshd.h"
#include "bshd_kernel.hpp"

#include <algorithm>
#include <atomic>
#include <climits>
#include <cmath>
#include <cstdint>

namespace {

// Upper bound on launched workgroups; larger problems loop inside the kernel.
constexpr int64_t MAX_GRID = int64_t(1) << 22;

template <int WAVES, int BN, int STAGES, bool PIPE, bool CAUSAL>
int launch(const Fav4Args& a, const fav4::Layout& L, hipStream_t stream) {
    constexpr int BM = WAVES * 32;
    const int tiles = (a.sq + BM - 1) / BM;
    const int64_t total = int64_t(fav4::items_per_head<CAUSAL>(tiles)) * a.batch * a.heads;
    if (total > INT_MAX) return hipErrorInvalidValue;
    const int grid = int(total < MAX_GRID ? total : MAX_GRID);
    if (a.lse)
        hipLaunchKernelGGL((fav4::fwd_kernel<WAVES, BN, CAUSAL, true, STAGES, PIPE>), dim3(grid),
                           dim3(WAVES * 64), 0, stream, a, L, tiles, int(total));
    else
        hipLaunchKernelGGL((fav4::fwd_kernel<WAVES, BN, CAUSAL, false, STAGES, PIPE>), dim3(grid),
                           dim3(WAVES * 64), 0, stream, a, L, tiles, int(total));
    return hipGetLastError();
}

template <bool CAUSAL>
int dispatch(const Fav4Args& a, const fav4::Layout& L, int config, hipStream_t stream) {
    switch (config) {
    case 1: return launch<4, 64, 2, false, CAUSAL>(a, L, stream);
    case 2: return launch<8, 64, 2, false, CAUSAL>(a, L, stream);
    case 3: return launch<8, 64, 3, true, CAUSAL>(a, L, stream);
    default: return hipErrorInvalidValue;
    }
}

// Argument checks of src/bshd.hip:27-34, in the same order, before any HIP call.
// kv_heads: heads of K/V (0 = heads, the reference's case); the key-side
// overflow limit counts those, as K/V rows are kv_heads * 256 bytes apart.
int validate(const Fav4Args* a, int causal, int config, int kv_heads = 0) {
    if (!a || !a->q || !a->k || !a->v || !a->o || a->batch <= 0 || a->heads <= 0 || a->sq <= 0 ||
        a->sk <= 0 || (causal != 0 && causal != 1) || config < 0 || config > 3 ||
        !std::isfinite(a->scale) || a->scale <= 0)
        return hipErrorInvalidValue;
    if (kv_heads == 0) kv_heads = a->heads;
    if (kv_heads < 0 || kv_heads > a->heads || a->heads % kv_heads != 0) return hipErrorInvalidValue;
    if (a->batch > INT_MAX / a->heads || a->heads > INT_MAX / 128 ||
        a->sq > INT_MAX / (a->heads * 128) || a->sk > INT_MAX / (kv_heads * 128) ||
        ((reinterpret_cast<uintptr_t>(a->q) | reinterpret_cast<uintptr_t>(a->k) |
          reinterpret_cast<uintptr_t>(a->v) | reinterpret_cast<uintptr_t>(a->o)) & 15))
        return hipErrorInvalidValue;
    return hipSuccess;
}

// Contiguous BSHD Q/O [B, Sq, H, 128] and K/V [B, Sk, kv_heads, 128].
fav4::Layout bshd_layout(const Fav4Args& a, int kv_heads) {
    fav4::Layout L;
    const int64_t row = int64_t(a.heads) * fav4::ROW_BYTES, kvrow = int64_t(kv_heads) * fav4::ROW_BYTES;
    L.qr = L.orow = uint32_t(row);
    L.kr = L.vr = uint32_t(kvrow);
    L.qb = L.ob = row * a.sq;
    L.kb = L.vb = kvrow * a.sk;
    L.qh = L.oh = L.kh = L.vh = fav4::ROW_BYTES;
    L.group = a.heads / kv_heads;
    return L;
}

// One tensor's element strides, checked: non-negative, multiples of 8
// elements (every row starts 16-byte aligned), the rows of one (batch, head)
// slice within a 4 GiB buffer bound, and the whole view within 2^48 bytes (so
// no address computation can overflow).
bool stride_ok(const Fav4Strides* st, int batch, int heads, int rows) {
    if (!st || st->batch < 0 || st->seq <= 0 || st->head < 0 || ((st->batch | st->seq | st->head) & 7))
        return false;
    if ((int64_t(rows) - 1) * static_cast<__int128>(st->seq) * 2 + fav4::ROW_BYTES > int64_t(UINT32_MAX))
        return false;
    const __int128 span = static_cast<__int128>(batch - 1) * st->batch + static_cast<__int128>(heads - 1) * st->head +
                          static_cast<__int128>(rows - 1) * st->seq + fav4::D;
    return span * 2 <= (static_cast<__int128>(1) << 48);
}

// ---- split-KV -------------------------------------------------------------
constexpr int MIN_TILES_PER_SPLIT = 4;   // Auto keeps >= 4 key tiles per chunk
constexpr int MAX_SPLIT_SQ = 1 << 22;    // keeps a chunk's O rows under a 4 GiB buffer bound
constexpr int DECODE_SQ = 32;            // up to this many queries: the one-wave decode shape

// Tile shape of the partial kernel: 8 waves x 256-row q tiles x 64-key tiles
// (one workgroup fills a CU), or for decode 1 wave x 32 rows x 32-key tiles
// (three workgroups per CU, each with 48 KiB of LDS).
struct SplitShape {
    int bm, bn, wgs_per_cu, auto_max;
};
SplitShape split_shape(const Fav4Args& a) {
    return a.sq <= DECODE_SQ ? SplitShape{32, 32, 3, 128} : SplitShape{256, 64, 1, 64};
}

struct SplitPlan {
    int splits, tps;   // chunks and key tiles per chunk
    SplitShape shape;
    int tiles;         // q tiles per item
    int64_t items;     // (batch, head) items, or (batch, K/V head) groups for decode
};

// CU count of the current device (256 if it cannot be read), cached per
// device after the first query.
int device_cus() {
    static std::atomic<int> cache[64];
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    const bool slot = dev >= 0 && dev < 64;
    if (slot && (cus = cache[dev].load(std::memory_order_relaxed)) > 0) return cus;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (slot) cache[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

// Auto for prefill (Sq > 32).  Filling the CUs is not enough: on the small
// grids where splitting is considered, the unsplit forward runs 128-row q
// tiles two per CU (causal: a heavy tile paired with a light one), while the
// split kernel runs 256-row (q tile, chunk) items one per CU with higher fixed
// costs.  Auto therefore keeps, among 1..max_splits chunks, the count with
// the lowest predicted time.  The model (microseconds; fitted to graph-timed
// MI355X runs of 23 shapes, B1-4, H1-64, Sq 256-16384, Sk up to 65536, where
// it picks the fastest measured choice or one within 2% of it):
//  * unsplit: rounds * (9 + c per 64-key tile of an item), an item being a
//    q tile (dense; c = 0.9 with at most one workgroup per CU, else 1.0) or
//    the heaviest tile pair (causal; c = 1.0);
//  * split: rounds * (F + c per 64-key tile of a chunk) + 5 for the merge,
//    F = 19 and c = 1.8 dense, F = 18 and c = 1.5 causal;
// where rounds = work items / resident workgroups, rounded up.
// Bottom-right causal (br): the packed (varlen) entry point runs one chunk
// on its unsplit kernel, one item per (sequence, head, q tile) and no pairs
// (br_unsplit; priced as rounds * 9 plus the larger of the average work per
// workgroup slot and the heaviest item); the paged entry point runs one chunk
// on the split kernels (priced as split_time(1)).
int prefill_auto_splits(const Fav4Args& a, int causal, int max_splits, int ktiles, bool br, bool br_unsplit) {
    const int64_t cus = device_cus();
    const int64_t bh = int64_t(a.batch) * a.heads;
    const int keys = causal ? std::min(a.sk, a.sq) : a.sk;
    // Key tiles visible to a q tile whose rows end at rows_end (bottom-right:
    // the last row sees keys up to rows_end - 1 + sk - sq).
    auto vis_tiles = [&](int64_t rows_end) {
        int64_t vis = causal ? std::min<int64_t>(keys, rows_end) : keys;
        if (br) vis = std::min<int64_t>(keys, std::max<int64_t>(0, std::min<int64_t>(rows_end, a.sq) + a.sk - a.sq));
        return int((vis + 63) / 64);
    };
    const int nt128 = (a.sq + 127) / 128;
    double best;
    if (causal) {
        const int npairs = (nt128 + 1) / 2;
        int heavy = 0;
        for (int i = 0; i < npairs; ++i) {
            const int j = nt128 - 1 - i;
            heavy = std::max(heavy, vis_tiles(128LL * (i + 1)) + (j != i ? vis_tiles(128LL * (j + 1)) : 0));
        }
        best = double((bh * npairs + 2 * cus - 1) / (2 * cus)) * (9.0 + 1.0 * heavy);
    } else {
        const int64_t items = bh * nt128;
        best = double((items + 2 * cus - 1) / (2 * cus)) * (9.0 + (items <= cus ? 0.9 : 1.0) * ktiles);
    }
    const double fixed = causal || br ? 18.0 : 19.0, per_tile = causal || br ? 1.5 : 1.8;
    const int nt256 = (a.sq + 255) / 256;
    auto split_time = [&](int s) {
        const int tps = (ktiles + s - 1) / s;
        int64_t items = 0;
        for (int i = 0; i < nt256; ++i) items += (vis_tiles(256LL * (i + 1)) + tps - 1) / tps;
        return double((bh * items + cus - 1) / cus) * (fixed + per_tile * tps) + 5.0;
    };
    if (br && br_unsplit) {
        // fwd_kernel_varlen's tile rule: 128-row tiles for sq <= 1024 or when
        // 256-row tiles would leave CUs idle (two workgroups per CU), else 256.
        const bool small = a.sq <= 1024 || bh * ((a.sq + 255) / 256) < cus;
        const int bm = small ? 128 : 256;
        const int nt = (a.sq + bm - 1) / bm;
        const int64_t slots = small ? 2 * cus : cus;
        int64_t sum = 0;
        int heavy = 0;
        for (int i = 0; i < nt; ++i) {
            const int w = vis_tiles(int64_t(bm) * (i + 1));
            sum += w;
            heavy = std::max(heavy, w);
        }
        const int64_t rounds = (bh * nt + slots - 1) / slots;
        best = double(rounds) * 9.0 + std::max(double(bh * sum) / double(slots), double(heavy));
    } else if (br) {
        best = split_time(1);
    }
    int pick = 1;
    for (int s = 2; s <= max_splits; ++s) {
        const double t = split_time(s);
        if (t < best) best = t, pick = s;
    }
    return pick;
}

// Chunking of the key range a row can see (top-left causal never shows a key
// past sq - 1); `req` = 0 picks enough chunks to fill the CUs once (the
// shape's resident workgroups per CU; more chunks only add merge traffic and
// per-chunk pipeline fill), for prefill then the model above.  The
// count is then rounded so that no chunk starts past that range.
// The decode shape packs the query heads that share a K/V head into one row
// space of (heads / kv_heads) * sq rows per (batch, K/V head).
SplitPlan split_plan(const Fav4Args& a, int kv_heads, int causal, int req, bool br = false, bool br_unsplit = false) {
    const SplitShape sh = split_shape(a);
    const bool pack = sh.bm == 32;
    const int rows = pack ? (a.heads / kv_heads) * a.sq : a.sq;
    const int tiles = (rows + sh.bm - 1) / sh.bm;
    const int64_t items = int64_t(a.batch) * (pack ? kv_heads : a.heads);
    const int keys = causal ? std::min(a.sk, a.sq) : a.sk;
    const int ktiles = (keys + sh.bn - 1) / sh.bn;
    int64_t splits = req;
    if (splits == 0) {
        const int64_t units = items * tiles;
        // Decode with one or two (batch, K/V head) tiles (B1 MQA / two K/V
        // heads, long caches) runs faster on up to 256 chunks (measured on
        // MI355X, 128 -> 256: B1 H8 KVH1 Sk200000 52.6 -> 39.9 us, B1 H8 KVH2
        // Sk262144 65.6 -> 59.6 us; with four tiles 256 lost, 54.3 -> 62.4 us).
        const int auto_max = pack && units <= 2 ? fav4::MAX_SPLITS : sh.auto_max;
        splits = (int64_t(device_cus()) * sh.wgs_per_cu + units - 1) / units;
        splits = std::min<int64_t>(splits, std::min(auto_max, std::max(1, ktiles / MIN_TILES_PER_SPLIT)));
        if (!pack && splits > 1) splits = prefill_auto_splits(a, causal, int(splits), ktiles, br, br_unsplit);
    }
    splits = std::max<int64_t>(1, std::min<int64_t>(splits, ktiles));
    const int tps = int((ktiles + splits - 1) / splits);
    return {(ktiles + tps - 1) / tps, tps, sh, tiles, items};
}

int64_t split_workspace(const Fav4Args& a, const SplitPlan& p) {
    if (p.splits <= 1) return 0;
    return int64_t(p.splits) * a.batch * a.heads * a.sq * (fav4::D * 4 + 2 * 4);
}

// Shape-only checks for the split-KV queries (no buffers needed yet).
int split_shape_ok(const Fav4Args* a, int kv_heads, int causal, int splits) {
    if (!a || a->batch <= 0 || a->heads <= 0 || a->sq <= 0 || a->sk <= 0 || (causal != 0 && causal != 1) ||
        kv_heads <= 0 || kv_heads > a->heads || a->heads % kv_heads != 0 ||
        a->batch > INT_MAX / a->heads || a->heads > INT_MAX / 128 || a->sq > INT_MAX / (a->heads * 128) ||
        a->sk > INT_MAX / (kv_heads * 128) || splits < 0 || splits > fav4::MAX_SPLITS || a->sq > MAX_SPLIT_SQ)
        return hipErrorInvalidValue;
    // Decode packs a group's (heads / kv_heads) * sq rows into one row space,
    // whose FP32 partial rows must fit a 4 GiB buffer bound.
    if (a->sq <= DECODE_SQ && int64_t(a->heads / kv_heads) * a->sq * fav4::D * 4 > int64_t(UINT32_MAX))
        return hipErrorInvalidValue;
    return hipSuccess;
}

int split_args_ok(const Fav4Args* a, int kv_heads, int causal, int splits) {
    if (kv_heads <= 0) return hipErrorInvalidValue;
    const int st = validate(a, causal, 0, kv_heads);
    return st != hipSuccess ? st : split_shape_ok(a, kv_heads, causal, splits);
}

// VARLEN: `a` holds the packed batch's shape (max lengths) and `sp` its
// sequence offsets; decode shape only.  PAGED: the same over paged K/V caches.
// Top-left causal decode (sq <= 32) sees at most 32 keys, one tile, so the
// plan never splits it: causal launches use the prefill shape only.
// BR (packed decode only): bottom-right causal, the one causal mask a decode
// splits.
template <bool CAUSAL, bool VARLEN = false, bool PAGED = false, bool BR = false>
int launch_split(const Fav4Args& a, int kv_heads, const SplitPlan& p, void* ws, fav4::SplitArgs sp,
                 hipStream_t stream) {
    static_assert(!(CAUSAL && VARLEN) || BR, "top-left causal decode never splits");
    static_assert(!BR || (CAUSAL && VARLEN), "bottom-right causal is for packed decode");
    static_assert(!PAGED || VARLEN, "paged caches hold packed sequences");
    const int tiles = p.tiles;
    const int64_t total = p.items * tiles * p.splits;
    const int64_t rows = int64_t(a.batch) * a.heads * a.sq;
    const bool decode = p.shape.bm == 32;
    if (total > INT_MAX || rows > INT_MAX || (VARLEN && !PAGED && !BR && !decode) || (CAUSAL && !BR && decode))
        return hipErrorInvalidValue;
    sp.o_part = static_cast<float*>(ws);
    sp.lse_part = sp.o_part + int64_t(p.splits) * rows * fav4::D;
    sp.splits = p.splits;
    sp.tps = p.tps;
    const int grid = int(total < MAX_GRID ? total : MAX_GRID);
    // The FP32 sums only feed an LSE output.
    auto go = [&](auto kernel, int threads) {
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(threads), 0, stream, a, sp, kv_heads, tiles, int(total));
    };
    if constexpr (VARLEN) {
        if (decode && a.lse) go(fav4::fwd_kernel_split<32, BR, 1, true, true, PAGED, BR>, 64);
        else if (decode) go(fav4::fwd_kernel_split<32, BR, 1, false, true, PAGED, BR>, 64);
        if constexpr (PAGED || BR) {  // prefill over paged caches or with the bottom-right mask: 8 waves
            if (!decode && a.lse) go(fav4::fwd_kernel_split<64, BR, 8, true, true, PAGED, BR>, 512);
            else if (!decode) go(fav4::fwd_kernel_split<64, BR, 8, false, true, PAGED, BR>, 512);
        }
    } else if constexpr (CAUSAL) {
        if (a.lse) go(fav4::fwd_kernel_split<64, true, 8, true>, 512);
        else go(fav4::fwd_kernel_split<64, true, 8, false>, 512);
    } else {
        if (decode && a.lse) go(fav4::fwd_kernel_split<32, false, 1, true>, 64);
        else if (decode) go(fav4::fwd_kernel_split<32, false, 1, false>, 64);
        else if (a.lse) go(fav4::fwd_kernel_split<64, false, 8, true>, 512);
        else go(fav4::fwd_kernel_split<64, false, 8, false>, 512);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // Lane groups per merged row: one per 8 chunks, at most 8 (one workgroup).
    const int per = p.splits <= 8 ? 1 : p.splits <= 16 ? 2 : p.splits <= 32 ? 4 : 8;
    const int64_t row_blocks = (rows * per + 7) / 8;
    const unsigned blocks = unsigned(row_blocks < MAX_GRID ? row_blocks : MAX_GRID);
    if (per == 1) hipLaunchKernelGGL((fav4::combine_kernel<1, VARLEN>), dim3(blocks), dim3(256), 0, stream, a, sp);
    else if (per == 2) hipLaunchKernelGGL((fav4::combine_kernel<2, VARLEN>), dim3(blocks), dim3(256), 0, stream, a, sp);
    else if (per == 4) hipLaunchKernelGGL((fav4::combine_kernel<4, VARLEN>), dim3(blocks), dim3(256), 0, stream, a, sp);
    else hipLaunchKernelGGL((fav4::combine_kernel<8, VARLEN>), dim3(blocks), dim3(256), 0, stream, a, sp);
    return hipGetLastError();
}

// causal = 2 on the packed calls: bottom-right causal (query i of a sequence
// with sq queries and sk keys sees keys j <= sk - sq + i).
constexpr int BOTTOM_RIGHT = 2;

template <int WAVES>
void launch_varlen(const Fav4VarlenArgs& a, int causal, int tiles, int total, int grid, hipStream_t stream) {
    const dim3 block(WAVES * 64);
    if (causal == BOTTOM_RIGHT && a.lse)
        hipLaunchKernelGGL((fav4::fwd_kernel_varlen<64, true, true, WAVES, true>), dim3(grid), block, 0, stream, a,
                           tiles, total);
    else if (causal == BOTTOM_RIGHT)
        hipLaunchKernelGGL((fav4::fwd_kernel_varlen<64, true, false, WAVES, true>), dim3(grid), block, 0, stream, a,
                           tiles, total);
    else if (causal && a.lse)
        hipLaunchKernelGGL((fav4::fwd_kernel_varlen<64, true, true, WAVES>), dim3(grid), block, 0, stream, a, tiles, total);
    else if (causal)
        hipLaunchKernelGGL((fav4::fwd_kernel_varlen<64, true, false, WAVES>), dim3(grid), block, 0, stream, a, tiles, total);
    else if (a.lse)
        hipLaunchKernelGGL((fav4::fwd_kernel_varlen<64, false, true, WAVES>), dim3(grid), block, 0, stream, a, tiles, total);
    else
        hipLaunchKernelGGL((fav4::fwd_kernel_varlen<64, false, false, WAVES>), dim3(grid), block, 0, stream, a, tiles, total);
}

// Checks of the packed-sequence arguments (before any HIP call); the shape
// checks alone serve the queries that take no buffers.  causal 0, 1 or
// BOTTOM_RIGHT.
int varlen_shape_ok(const Fav4VarlenArgs* a, int causal) {
    if (!a || a->batch <= 0 || a->heads <= 0 || a->kv_heads <= 0 || a->heads % a->kv_heads != 0 ||
        a->max_seqlen_q <= 0 || a->max_seqlen_k <= 0 || a->total_q <= 0 || a->total_k <= 0 ||
        causal < 0 || causal > BOTTOM_RIGHT || !std::isfinite(a->scale) || a->scale <= 0)
        return hipErrorInvalidValue;
    if (a->batch > INT_MAX - 1 || a->heads > INT_MAX / 256 ||
        int64_t(a->max_seqlen_q) * a->heads * 256 > int64_t(UINT32_MAX) ||
        int64_t(a->max_seqlen_k) * a->kv_heads * 256 > int64_t(UINT32_MAX))
        return hipErrorInvalidValue;
    return hipSuccess;
}

int varlen_ok(const Fav4VarlenArgs* a, int causal) {
    if (varlen_shape_ok(a, causal) != hipSuccess || !a->q || !a->k || !a->v || !a->o || !a->cu_seqlens_q ||
        !a->cu_seqlens_k ||
        ((reinterpret_cast<uintptr_t>(a->q) | reinterpret_cast<uintptr_t>(a->k) |
          reinterpret_cast<uintptr_t>(a->v) | reinterpret_cast<uintptr_t>(a->o)) & 15) ||
        ((reinterpret_cast<uintptr_t>(a->cu_seqlens_q) | reinterpret_cast<uintptr_t>(a->cu_seqlens_k)) & 3) ||
        (a->lse && (reinterpret_cast<uintptr_t>(a->lse) & 3)))
        return hipErrorInvalidValue;
    return hipSuccess;
}

// The packed batch as the split-KV kernels see it: sq / sk are the longest
// sequence's lengths, LSE is [heads, total_q].
Fav4Args varlen_shape(const Fav4VarlenArgs& v) {
    Fav4Args a{};
    a.q = v.q; a.k = v.k; a.v = v.v; a.o = v.o; a.lse = v.lse;
    a.batch = v.batch; a.heads = v.heads; a.sq = v.max_seqlen_q; a.sk = v.max_seqlen_k;
    a.scale = v.scale;
    return a;
}

// Split-KV of packed decode batches (max_seqlen_q <= 32; longer queries take
// one chunk, the plain packed forward).  Chunks are a fixed number of key
// tiles for every sequence, so a sequence has as many non-empty chunks as its
// keys need.  Auto takes the chunk size of the contiguous-batch Auto plan at
// the mean key length (total_k / batch), so a uniform batch gets exactly the
// contiguous plan.  A ragged batch (mean below 3/4 of the longest) gets
// chunks of at most RAGGED_TPS key tiles: its chunks differ in length, and
// more, shorter ones even out the CUs' finishing times (measured on MI355X,
// against the uncapped plan: +0.7%, +2% and +13% on three ragged batches;
// the same cap on uniform batches lost 3-25%).  Either is enlarged if the
// longest sequence would need more than MAX_SPLITS chunks.
constexpr int RAGGED_TPS = 64;

// `a` is the packed batch's shape (max lengths), total_k its key count.
SplitPlan packed_split_plan(const Fav4Args& a, int kv_heads, int64_t total_k, int causal, int req) {
    if (a.sq > DECODE_SQ) return {1, 1, split_shape(a), 1, 1};
    SplitPlan p = split_plan(a, kv_heads, causal, req == 0 ? 1 : req);
    if (req == 0) {
        Fav4Args mean = a;
        mean.sk = int(std::max<int64_t>(1, std::min<int64_t>(a.sk, (total_k + a.batch - 1) / a.batch)));
        const int keys = causal ? std::min(a.sk, a.sq) : a.sk;
        const int ktiles = (keys + p.shape.bn - 1) / p.shape.bn;
        int tps = split_plan(mean, kv_heads, causal, 0).tps;
        if (4 * int64_t(mean.sk) < 3 * int64_t(a.sk)) tps = std::min(tps, RAGGED_TPS);
        p.tps = std::max(tps, (ktiles + fav4::MAX_SPLITS - 1) / fav4::MAX_SPLITS);
        p.splits = (ktiles + p.tps - 1) / p.tps;
    }
    return p;
}

// Bottom-right causal in the split-KV packed calls sees as many keys as a
// dense call, so it is planned like one.  Decode always runs the split
// kernels, also for one chunk (their one-wave shape streams a K/V head once
// for its whole query group); prefill with one chunk runs the unsplit packed
// forward, which takes this mask directly.

SplitPlan varlen_split_plan(const Fav4VarlenArgs& v, int causal, int req) {
    const Fav4Args a = varlen_shape(v);
    // Bottom-right prefill: the contiguous prefill plan at the max lengths.
    if (causal == BOTTOM_RIGHT && a.sq > DECODE_SQ) return split_plan(a, v.kv_heads, 0, req, true, true);
    return packed_split_plan(a, v.kv_heads, v.total_k, causal == BOTTOM_RIGHT ? 0 : causal, req);
}

int varlen_split_ok(const Fav4VarlenArgs* v, int causal, int splits, bool buffers) {
    const bool br = causal == BOTTOM_RIGHT;
    const int st = buffers ? varlen_ok(v, br ? 0 : causal) : varlen_shape_ok(v, br ? 0 : causal);
    if (st != hipSuccess) return st;
    if (splits < 0 || splits > fav4::MAX_SPLITS) return hipErrorInvalidValue;
    if (v->max_seqlen_q > DECODE_SQ && !br) return hipSuccess;
    const Fav4Args a = varlen_shape(*v);
    return split_shape_ok(&a, v->kv_heads, br ? 0 : causal, splits);
}

// Workspace of a packed plan; bottom-right decode needs it for one chunk too.
int64_t varlen_workspace(const Fav4VarlenArgs& v, const SplitPlan& p, int causal) {
    if (p.splits <= 1 && (causal != BOTTOM_RIGHT || v.max_seqlen_q > DECODE_SQ)) return 0;
    return int64_t(p.splits) * v.batch * v.heads * v.max_seqlen_q * (fav4::D * 4 + 2 * 4);
}

// ---- paged K/V caches ----------------------------------------------------
constexpr int PAGED_MAX_TPS = 64;          // key tiles per chunk: one page number per lane
constexpr int PAGED_MAX_KEYS = fav4::MAX_SPLITS * PAGED_MAX_TPS * 32;

// Decode (max_seqlen_q <= 32) needs page_size % 32 == 0 (one 32-key tile per
// page), prefill page_size % 64 == 0 (the 8-wave shape's 64-key tiles).
int paged_shape_ok(const Fav4PagedArgs* a, int causal, int splits) {
    if (!a || a->batch <= 0 || a->heads <= 0 || a->kv_heads <= 0 || a->heads % a->kv_heads != 0 ||
        a->max_seqlen_q <= 0 || a->max_seqlen_q > MAX_SPLIT_SQ || a->max_seqlen_k <= 0 || a->total_q <= 0 ||
        a->total_k < 0 || a->num_pages <= 0 || a->page_size <= 0 ||
        a->page_size % (a->max_seqlen_q > DECODE_SQ ? 64 : 32) != 0 ||
        a->max_pages_per_seq <= 0 || (causal != 0 && causal != BOTTOM_RIGHT) || !std::isfinite(a->scale) ||
        a->scale <= 0 || splits < 0 ||
        splits > fav4::MAX_SPLITS)
        return hipErrorInvalidValue;
    if (a->batch > INT_MAX - 1 || a->heads > INT_MAX / 256 || a->max_seqlen_k > PAGED_MAX_KEYS ||
        int64_t(a->max_seqlen_k) > int64_t(a->max_pages_per_seq) * a->page_size ||
        int64_t(a->page_size) * a->kv_heads * 256 > int64_t(UINT32_MAX) ||
        int64_t(a->max_seqlen_q) * a->heads * 256 > int64_t(UINT32_MAX) ||
        (a->max_seqlen_q <= DECODE_SQ ? int64_t(a->heads / a->kv_heads) : 1) * a->max_seqlen_q * fav4::D * 4 >
            int64_t(UINT32_MAX) ||
        int64_t(a->batch) * a->heads * a->max_seqlen_q > INT_MAX)
        return hipErrorInvalidValue;
    return hipSuccess;
}

int paged_ok(const Fav4PagedArgs* a, int causal, int splits) {
    if (paged_shape_ok(a, causal, splits) != hipSuccess || !a->q || !a->k_cache || !a->v_cache || !a->o ||
        !a->cu_seqlens_q || !a->seqlens_k || !a->block_table ||
        ((reinterpret_cast<uintptr_t>(a->q) | reinterpret_cast<uintptr_t>(a->k_cache) |
          reinterpret_cast<uintptr_t>(a->v_cache) | reinterpret_cast<uintptr_t>(a->o)) & 15) ||
        ((reinterpret_cast<uintptr_t>(a->cu_seqlens_q) | reinterpret_cast<uintptr_t>(a->seqlens_k) |
          reinterpret_cast<uintptr_t>(a->block_table)) & 3) ||
        (a->lse && (reinterpret_cast<uintptr_t>(a->lse) & 3)))
        return hipErrorInvalidValue;
    return hipSuccess;
}

Fav4Args paged_shape(const Fav4PagedArgs& v) {
    Fav4Args a{};
    a.q = v.q; a.k = v.k_cache; a.v = v.v_cache; a.o = v.o; a.lse = v.lse;
    a.batch = v.batch; a.heads = v.heads; a.sq = v.max_seqlen_q; a.sk = v.max_seqlen_k;
    a.scale = v.scale;
    return a;
}

// The packed-batch plan, with chunks capped at 64 key tiles (a chunk's page
// numbers fit the lanes of one wave); one chunk still runs the split kernels.
SplitPlan paged_plan(const Fav4PagedArgs& v, int causal, int req) {
    const Fav4Args a = paged_shape(v);
    // Prefill: the contiguous prefill plan at the max lengths (bottom-right
    // causal with the key count its q tiles see).
    SplitPlan p = a.sq > DECODE_SQ ? split_plan(a, v.kv_heads, 0, req, causal == BOTTOM_RIGHT)
                                   : packed_split_plan(a, v.kv_heads, v.total_k, 0, req);
    if (p.tps > PAGED_MAX_TPS) {
        const int ktiles = (v.max_seqlen_k + p.shape.bn - 1) / p.shape.bn;
        p.tps = PAGED_MAX_TPS;
        p.splits = (ktiles + p.tps - 1) / p.tps;
    }
    return p;
}

int64_t paged_workspace(const Fav4PagedArgs& v, const SplitPlan& p) {
    return int64_t(p.splits) * v.batch * v.heads * v.max_seqlen_q * (fav4::D * 4 + 2 * 4);
}

// Auto: 128-row workgroups (config 1; two per CU, so one's prologue and
// epilogue overlap the other's key loop) for query lengths up to 768 (dense)
// or 1024 (causal), and wherever 256-row workgroups (config 2) would leave
// CUs without a work item (items: q tiles; causal: q-tile pairs); else
// config 2.  Measured on MI355X (graph-timed, config 1 vs 2, row-contiguous
// O stores): dense Sq 512 config 1 wins by 5%, Sq 768 they are equal, Sq 1024
// config 2 wins by 1.7-6.5% (B32 H8, B16 H8, B8 H8, B4 H16); causal config 1
// wins or ties up to Sq 1024 (by 26% at B8 H8 and B4 H16 Sq 1024, 17% at B32
// H8 Sq 768).  With fewer config-2 items than CUs config 1 wins by 28-46%
// (B1 H8 S2048..S4096, causal B1 H8 S8192, B2 H8 S4096); with one item per
// CU or more config 2 wins by 6-8% (dense B2 H8 S4096, B1 H32 S4096, causal
// B1 H32 S4096).
int auto_config(const Fav4Args& a, int causal) {
    if (a.sq <= (causal ? 1024 : 768)) return 1;
    const int64_t tiles = (int64_t(a.sq) + 255) / 256;
    const int64_t items = int64_t(a.batch) * a.heads * (causal ? (tiles + 1) / 2 : tiles);
    return items < device_cus() ? 1 : 2;
}

}  // namespace

// Replaces src/bshd.hip:23-25 (the dense choice; the forward calls
// auto_config with its mask).
extern "C" __attribute__((visibility("default"))) int fav4_bshd_select_config(const Fav4Args* a) {
    if (!a) return -1;
    return auto_config(*a, 0);
}

// The same for a call with this mask (no counterpart in the reference, whose
// Auto ignores the mask): the config fav4_bshd_forward runs for config 0.
extern "C" __attribute__((visibility("default"))) int fav4_bshd_select_config_masked(const Fav4Args* a,
                                                                             int causal) {
    if (!a || (causal != 0 && causal != 1)) return -1;
    return auto_config(*a, causal);
}

// Replaces src/bshd.hip:26-38.
extern "C" __attribute__((visibility("default"))) int fav4_bshd_forward(const Fav4Args* a, int causal, int config,
                                                                hipStream_t stream) {
    const int st = validate(a, causal, config);
    if (st != hipSuccess) return st;
    if (config == 0) config = auto_config(*a, causal);
    const fav4::Layout L = bshd_layout(*a, a->heads);
    return causal ? dispatch<true>(*a, L, config, stream) : dispatch<false>(*a, L, config, stream);
}

// Arbitrary strides (no counterpart in the reference).
extern "C" __attribute__((visibility("default"))) int fav4_bshd_forward_strided(
    const Fav4Args* a, int kv_heads, const Fav4Strides* q, const Fav4Strides* k, const Fav4Strides* v,
    const Fav4Strides* o, int causal, int config, hipStream_t stream) {
    if (!a || !a->q || !a->k || !a->v || !a->o || a->batch <= 0 || a->heads <= 0 || a->sq <= 0 || a->sk <= 0 ||
        (causal != 0 && causal != 1) || config < 0 || config > 3 || !std::isfinite(a->scale) || a->scale <= 0 ||
        kv_heads <= 0 || kv_heads > a->heads || a->heads % kv_heads != 0 || a->batch > INT_MAX / a->heads ||
        ((reinterpret_cast<uintptr_t>(a->q) | reinterpret_cast<uintptr_t>(a->k) |
          reinterpret_cast<uintptr_t>(a->v) | reinterpret_cast<uintptr_t>(a->o)) & 15) ||
        (a->lse && (reinterpret_cast<uintptr_t>(a->lse) & 3)) ||
        !stride_ok(q, a->batch, a->heads, a->sq) || !stride_ok(o, a->batch, a->heads, a->sq) ||
        !stride_ok(k, a->batch, kv_heads, a->sk) || !stride_ok(v, a->batch, kv_heads, a->sk))
        return hipErrorInvalidValue;
    fav4::Layout L;
    L.qb = q->batch * 2; L.qh = q->head * 2; L.qr = uint32_t(q->seq * 2);
    L.kb = k->batch * 2; L.kh = k->head * 2; L.kr = uint32_t(k->seq * 2);
    L.vb = v->batch * 2; L.vh = v->head * 2; L.vr = uint32_t(v->seq * 2);
    L.ob = o->batch * 2; L.oh = o->head * 2; L.orow = uint32_t(o->seq * 2);
    L.group = a->heads / kv_heads;
    if (config == 0) config = auto_config(*a, causal);
    return causal ? dispatch<true>(*a, L, config, stream) : dispatch<false>(*a, L, config, stream);
}

// Packed variable-length sequences (no counterpart in the reference).
extern "C" __attribute__((visibility("default"))) int fav4_bshd_forward_varlen(const Fav4VarlenArgs* a, int causal,
                                                                       hipStream_t stream) {
    const int st = varlen_ok(a, causal);
    if (st != hipSuccess) return st;
    // Tile rule on the longest sequence: 128-row tiles (4 waves) for
    // max_seqlen_q <= 1024 or when 256-row tiles would give fewer
    // (sequence, head, q tile) items than CUs; else 256-row tiles.
    const int64_t tiles256 = (int64_t(a->max_seqlen_q) + 255) / 256;
    const bool small = a->max_seqlen_q <= 1024 || int64_t(a->batch) * a->heads * tiles256 < device_cus();
    const int bm = small ? 128 : 256;
    const int tiles = (a->max_seqlen_q + bm - 1) / bm;
    const int64_t total = int64_t(a->batch) * a->heads * tiles;
    if (total > INT_MAX) return hipErrorInvalidValue;
    const int grid = int(total < MAX_GRID ? total : MAX_GRID);
    if (small)
        launch_varlen<4>(*a, causal, tiles, int(total), grid, stream);
    else
        launch_varlen<8>(*a, causal, tiles, int(total), grid, stream);
    return hipGetLastError();
}

// Grouped-query / multi-query attention (no counterpart in the reference).
extern "C" __attribute__((visibility("default"))) int fav4_bshd_forward_gqa(const Fav4Args* a, int kv_heads,
                                                                    int causal, int config, hipStream_t stream) {
    if (kv_heads <= 0) return hipErrorInvalidValue;
    const int st = validate(a, causal, config, kv_heads);
    if (st != hipSuccess) return st;
    if (config == 0) config = auto_config(*a, causal);
    const fav4::Layout L = bshd_layout(*a, kv_heads);
    return causal ? dispatch<true>(*a, L, config, stream) : dispatch<false>(*a, L, config, stream);
}

// Split-KV entry points (no counterpart in the reference; see the header).
// The MHA ones are the GQA ones with kv_heads = heads.
extern "C" __attribute__((visibility("default"))) int fav4_bshd_splitkv_gqa_select(const Fav4Args* a, int kv_heads,
                                                                           int causal) {
    if (split_shape_ok(a, kv_heads, causal, 0) != hipSuccess) return -1;
    return split_plan(*a, kv_heads, causal, 0).splits;
}

extern "C" __attribute__((visibility("default"))) long long fav4_bshd_splitkv_gqa_workspace_size(const Fav4Args* a,
                                                                                              int kv_heads,
                                                                                              int causal,
                                                                                              int splits) {
    if (split_shape_ok(a, kv_heads, causal, splits) != hipSuccess) return -1;
    return split_workspace(*a, split_plan(*a, kv_heads, causal, splits));
}

extern "C" __attribute__((visibility("default"))) int fav4_bshd_forward_splitkv_gqa(const Fav4Args* a, int kv_heads,
                                                                            int causal, int splits,
                                                                            void* workspace,
                                                                            size_t workspace_bytes,
                                                                            hipStream_t stream) {
    const int st = split_args_ok(a, kv_heads, causal, splits);
    if (st != hipSuccess) return st;
    const SplitPlan p = split_plan(*a, kv_heads, causal, splits);
    if (p.splits == 1) return fav4_bshd_forward_gqa(a, kv_heads, causal, 0, stream);
    const int64_t need = split_workspace(*a, p);
    if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255) || uint64_t(need) > workspace_bytes)
        return hipErrorInvalidValue;
    const fav4::SplitArgs sp{};
    return causal ? launch_split<true>(*a, kv_heads, p, workspace, sp, stream)
                  : launch_split<false>(*a, kv_heads, p, workspace, sp, stream);
}

extern "C" __attribute__((visibility("default"))) int fav4_bshd_splitkv_select(const Fav4Args* a, int causal) {
    return a ? fav4_bshd_splitkv_gqa_select(a, a->heads, causal) : -1;
}

extern "C" __attribute__((visibility("default"))) long long fav4_bshd_splitkv_workspace_size(const Fav4Args* a,
                                                                                          int causal, int splits) {
    return a ? fav4_bshd_splitkv_gqa_workspace_size(a, a->heads, causal, splits) : -1;
}

extern "C" __attribute__((visibility("default"))) int fav4_bshd_forward_splitkv(const Fav4Args* a, int causal,
                                                                        int splits, void* workspace,
                                                                        size_t workspace_bytes,
                                                                        hipStream_t stream) {
    if (!a) return hipErrorInvalidValue;
    return fav4_bshd_forward_splitkv_gqa(a, a->heads, causal, splits, workspace, workspace_bytes, stream);
}

// Split-KV of packed variable-length batches (no counterpart in the reference).
extern "C" __attribute__((visibility("default"))) int fav4_bshd_splitkv_varlen_select(const Fav4VarlenArgs* a,
                                                                              int causal) {
    if (varlen_split_ok(a, causal, 0, false) != hipSuccess) return -1;
    return varlen_split_plan(*a, causal, 0).splits;
}

extern "C" __attribute__((visibility("default"))) long long fav4_bshd_splitkv_varlen_workspace_size(
    const Fav4VarlenArgs* a, int causal, int splits) {
    if (varlen_split_ok(a, causal, splits, false) != hipSuccess) return -1;
    return varlen_workspace(*a, varlen_split_plan(*a, causal, splits), causal);
}

extern "C" __attribute__((visibility("default"))) int fav4_bshd_forward_splitkv_varlen(const Fav4VarlenArgs* a,
                                                                               int causal, int splits,
                                                                               void* workspace,
                                                                               size_t workspace_bytes,
                                                                               hipStream_t stream) {
    const int st = varlen_split_ok(a, causal, splits, true);
    if (st != hipSuccess) return st;
    const SplitPlan p = varlen_split_plan(*a, causal, splits);
    // Top-left causal decode (max_seqlen_q <= 32) sees at most 32 keys, one
    // tile: the plan never splits it.  One-chunk bottom-right prefill needs
    // no merge either.
    const bool br = causal == BOTTOM_RIGHT;
    const bool unsplit = br ? p.splits == 1 && a->max_seqlen_q > DECODE_SQ : p.splits == 1 || causal;
    if (unsplit) return fav4_bshd_forward_varlen(a, causal, stream);
    const Fav4Args shape = varlen_shape(*a);
    const int64_t need = varlen_workspace(*a, p, causal);
    if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255) || uint64_t(need) > workspace_bytes)
        return hipErrorInvalidValue;
    fav4::SplitArgs sp{};
    sp.cu_q = a->cu_seqlens_q;
    sp.cu_k = a->cu_seqlens_k;
    sp.total_q = a->total_q;
    sp.total_k = a->total_k;
    return br ? launch_split<true, true, false, true>(shape, a->kv_heads, p, workspace, sp, stream)
              : launch_split<false, true>(shape, a->kv_heads, p, workspace, sp, stream);
}

// Split-KV decode over paged K/V caches (no counterpart in the reference).
extern "C" __attribute__((visibility("default"))) int fav4_bshd_splitkv_paged_select(const Fav4PagedArgs* a,
                                                                             int causal) {
    if (paged_shape_ok(a, causal, 0) != hipSuccess) return -1;
    return paged_plan(*a, causal, 0).splits;
}

extern "C" __attribute__((visibility("default"))) long long fav4_bshd_splitkv_paged_workspace_size(
    const Fav4PagedArgs* a, int causal, int splits) {
    if (paged_shape_ok(a, causal, splits) != hipSuccess) return -1;
    return paged_workspace(*a, paged_plan(*a, causal, splits));
}

extern "C" __attribute__((visibility("default"))) int fav4_bshd_forward_splitkv_paged(const Fav4PagedArgs* a,
                                                                              int causal, int splits,
                                                                              void* workspace,
                                                                              size_t workspace_bytes,
                                                                              hipStream_t stream) {
    const int st = paged_ok(a, causal, splits);
    if (st != hipSuccess) return st;
    const SplitPlan p = paged_plan(*a, causal, splits);
    const int64_t need = paged_workspace(*a, p);
    if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255) || uint64_t(need) > workspace_bytes)
        return hipErrorInvalidValue;
    fav4::SplitArgs sp{};
    sp.cu_q = a->cu_seqlens_q;
    sp.total_q = a->total_q;
    sp.seqlens_k = a->seqlens_k;
    sp.block_table = a->block_table;
    sp.page_size = a->page_size;
    sp.max_pages = a->max_pages_per_seq;
    sp.num_pages = a->num_pages;
    return causal == BOTTOM_RIGHT
               ? launch_split<true, true, true, true>(paged_shape(*a), a->kv_heads, p, workspace, sp, stream)
               : launch_split<false, true, true>(paged_shape(*a), a->kv_heads, p, workspace, sp, stream);
}

// ---- Split-KV without a caller workspace ------------------------------------
// For callers that cannot allocate (code under HIP graph capture, serving
// loops, harnesses that forbid it): the chunk partials live in a fixed
// device-resident array, one copy per GPU, held until the process ends.
constexpr size_t SCRATCH_BYTES = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

namespace {

// Device address of the current device's `scratch` (in host code the array's
// name is only a stand-in, never a device address), looked up once per device
// with that device current and kept per device.
hipError_t scratch_address(void** out) {
    static std::atomic<void*> cache[64];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    void* p = cache[dev].load(std::memory_order_acquire);
    if (!p) {
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        cache[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return hipSuccess;
}

}  // namespace

extern "C" __attribute__((visibility("default"))) int fav4_bshd_forward_splitkv_gqa_noalloc(const Fav4Args* a,
                                                                                    int kv_heads, int causal,
                                                                                    int splits,
                                                                                    hipStream_t stream) {
    const int st = split_args_ok(a, kv_heads, causal, splits);
    if (st != hipSuccess) return st;
    const SplitPlan p = split_plan(*a, kv_heads, causal, splits);
    if (p.splits == 1) return fav4_bshd_forward_gqa(a, kv_heads, causal, 0, stream);
    if (split_workspace(*a, p) > int64_t(SCRATCH_BYTES)) return hipErrorInvalidValue;
    void* ws = nullptr;
    const hipError_t e = scratch_address(&ws);
    if (e != hipSuccess) return e;
    // Every partial row the merge reads is written by the partial kernel
    // first, so the array needs no clearing between calls.
    const fav4::SplitArgs sp{};
    return causal ? launch_split<true>(*a, kv_heads, p, ws, sp, stream)
                  : launch_split<false>(*a, kv_heads, p, ws, sp, stream);
}
