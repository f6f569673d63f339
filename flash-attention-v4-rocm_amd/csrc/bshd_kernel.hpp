// BF16 BSHD D=128 attention forward for gfx950 (MI355X), wave64 MFMA.
//
// Semantics follow the reference kernel src/bshd_kernel.hpp:50-211 (online
// softmax in log2 units with the FA4 conditional rescale, P rounded to BF16
// before the PV product, LSE = m*ln2 + ln(l) from the FP32 row sum), but the
// machine mapping is gfx950's own:
//
//  * A workgroup owns BM = 32*WAVES query rows of one (batch, head); each wave
//    owns 32 of them.  The score tile is computed transposed, S^T = K.Q^T, on
//    v_mfma_f32_32x32x16_bf16, so lane l holds query (l % 32) and 16 keys of
//    every 32-key block; lanes l and l^32 share a query and combine their row
//    max / row sum with one v_permlane32_swap.
//  * Q stays in registers for the whole key loop (8 MFMA B operands).
//  * K and V tiles of BN keys are double-buffered in LDS and filled by
//    buffer->LDS DMA issued by all waves.  Rows past the key length read as
//    zero through the buffer descriptor's bound.  Granules are XOR-swizzled on
//    the global-address side so the MFMA operand reads are bank-conflict free.
//  * O^T += V^T.P^T: P leaves the S accumulator directly as the B operand
//    (no LDS round trip); the V operand comes from ds_read_b64_tr_b16.
//  * Key tiles that no row of the workgroup masks run a branch-free body;
//    only the causal-diagonal and key-tail tiles run the masked body, which
//    computes every 32-key block and then masks scores element by element; a
//    wave skips a causal tile entirely above its rows.  Key tiles entirely
//    above the diagonal are never loaded.
//  * O is normalised by the sum of the BF16-rounded weights that entered the
//    PV product (see the epilogue); the LSE uses the FP32 sum as the reference.
#pragma once
#include "fav4_bshd.h"
#include "gfx950.hpp"

namespace fav4 {

constexpr int D = 128;
constexpr int ROW_BYTES = D * 2;                 // one K/V/Q/O row of a head
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float RESCALE_THRESHOLD = 8.f;         // log2 units (src/bshd_kernel.hpp:157)

// LDS swizzles (16-byte granule positions inside a 256-byte tile row).
// K: granule g of row r sits at g ^ (r % 16): the 16 rows read by one quarter
//    wave of ds_read_b128 land on 16 distinct granule positions.
// V: granule g of row r sits at g ^ (4*(r % 4) + (r / 4) % 4): the 4 rows x
//    64 bytes read by each half wave of ds_read_b64_tr_b16 cover all banks.
__device__ __forceinline__ int k_swz(int r) { return r & 15; }
__device__ __forceinline__ int v_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// Work items.  The hardware deals workgroups round-robin over the 8 XCDs, so
// item ids are remapped to give each XCD a contiguous run of items: all q
// tiles of one (batch, head) then run at the same time on one XCD and share
// its L2 copy of that head's K/V.  Dense: one item = one q tile.  Causal: one
// item = the pair of q tiles (j, tiles-1-j), heavy one first, so every item
// costs tiles+1 key tiles and the grid has no tail of light items.
template <bool CAUSAL>
__host__ __device__ constexpr int items_per_head(int tiles) { return CAUSAL ? (tiles + 1) / 2 : tiles; }

template <bool CAUSAL, class F>
__device__ __forceinline__ void for_each_item(int tiles, int total, F&& process) {
    const int per_head = items_per_head<CAUSAL>(tiles);
    for (int id = blockIdx.x; id < total; id += gridDim.x) {
        const int xcd = id & 7, slot = id >> 3, per = total >> 3, rem = total & 7;
        const int logical = xcd * per + min(xcd, rem) + slot;
        const int bh = __builtin_amdgcn_readfirstlane(logical / per_head);
        const int j = __builtin_amdgcn_readfirstlane(logical - bh * per_head);
        if constexpr (CAUSAL) {
            const int n = (j == tiles - 1 - j) ? 1 : 2;
            for (int k = 0; k < n; ++k) process(bh, k == 0 ? tiles - 1 - j : j);
        } else {
            process(bh, j);
        }
    }
}

// Byte strides of Q, K, V and O seen as [B, S, H, 128] (the 128 head dims
// contiguous).  Row = one sequence position of one head.  BSHD: row stride
// heads*256 (K/V: kv_heads*256), batch stride S*row, head stride 256.
struct Layout {
    int64_t qb, qh, kb, kh, vb, vh, ob, oh;   // batch / head strides
    uint32_t qr, kr, vr, orow;                // row strides (each slice's rows fit a 4 GiB buffer bound)
    int group;                                // query heads per K/V head
};

// Per-wave running state of the online softmax for its 32 query rows.
// m: base in log2 units (identical in both lane halves); lb: sum of the BF16
// weights that entered the PV product; l: FP32 sum (only kept for the LSE).
struct RowState {
    f32x16 o[4];
    float m, lb, l;
};

// Per-lane LDS read offsets, relative to a stage's K / V tile.
struct LdsOffsets {
    uint32_t k[8];      // K operand of d-chunk c (16 dims) for key row `col`
    uint32_t v[2][4];   // V^T operand: [first/second 4-key group][32-dim block]
};

// MFMA operand read offsets of one lane.  K (A operand of S^T = K.Q^T, one
// 32-key block): lane l reads key l % 32, dims 16c + 8(l / 32) .. +7, i.e.
// granule 2c + l / 32 of its row, found at that granule ^ k_swz(row).  V^T
// (A operand of O^T += V^T.P^T, one 16-key unit): ds_read_b64_tr_b16 from
// lane l returns dim l % 32 of a 32-dim block for four keys, so source lane
// 4r + c of each 16-lane group addresses row r (+ 4 for the upper lane half,
// + 8 for the second read) and 4 dims 4c.. of the block.
__device__ __forceinline__ LdsOffsets lds_offsets(int lane) {
    const int col = lane & 31, half = lane >> 5;
    LdsOffsets off;
#pragma unroll
    for (int c = 0; c < 8; ++c) off.k[c] = col * ROW_BYTES + ((((2 * c) | half) ^ k_swz(col)) << 4);
    const int r0 = half * 4 + ((lane & 15) >> 2);             // row inside a 16-key sub-block
    const int gl = ((lane >> 4) & 1) * 2 + ((lane & 3) >> 1);  // granule inside a 32-dim block
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int r = r0 + 8 * j;
#pragma unroll
        for (int db = 0; db < 4; ++db)
            off.v[j][db] = r * ROW_BYTES + (((db * 4 + gl) ^ v_swz(r)) << 4) + ((lane & 1) << 3);
    }
    return off;
}

// Per-lane global source offsets of the tile DMA.  Each wave issues DMA ops
// i = 0..DMA-1 per matrix; op i covers tile rows 4(wave * DMA + i) .. +3, lane
// l fetching granule (l % 16) ^ swz(row) of row 4(wave * DMA + i) + l / 16, so
// that the 1 KiB the op writes contiguously to LDS holds the rows swizzled.
template <int DMA>
struct DmaOffsets {
    uint32_t k[DMA], v[DMA];
};
template <int DMA>
__device__ __forceinline__ DmaOffsets<DMA> dma_offsets(int wave, int lane, uint32_t k_row_bytes,
                                                       uint32_t v_row_bytes) {
    DmaOffsets<DMA> d;
#pragma unroll
    for (int i = 0; i < DMA; ++i) {
        const int r = (wave * DMA + i) * 4 + (lane >> 4), p = lane & 15;
        d.k[i] = r * k_row_bytes + ((p ^ k_swz(r)) << 4);
        d.v[i] = r * v_row_bytes + ((p ^ v_swz(r)) << 4);
    }
    return d;
}

// DMA of one K and one V tile (descriptors rk / rv start at the tile's first
// row) to the LDS byte addresses k_lds and v_lds: this wave's DMA ops land at
// 1 KiB slots wave * DMA + i of each tile.
// NT: nontemporal loads, for K/V that no other workgroup reads again.
template <int DMA, bool NT = false>
__device__ __forceinline__ void dma_kv(u32x4 rk, u32x4 rv, uint32_t k_lds, uint32_t v_lds, int wave,
                                       const DmaOffsets<DMA>& d) {
    const uint32_t slot = wave * DMA * 1024;
#pragma unroll
    for (int i = 0; i < DMA; ++i) {
        dma16<NT>(rk, k_lds + slot + i * 1024, d.k[i]);
        dma16<NT>(rv, v_lds + slot + i * 1024, d.v[i]);
    }
}

// The same into one LDS stage at byte address `stage`: K at +0, V at +TILE_BYTES.
template <int DMA, int TILE_BYTES, bool NT = false>
__device__ __forceinline__ void dma_tile(u32x4 rk, u32x4 rv, uint32_t stage, int wave, const DmaOffsets<DMA>& d) {
    dma_kv<DMA, NT>(rk, rv, stage, stage + TILE_BYTES, wave, d);
}

// S^T = K.Q^T for one tile: 8 MFMAs per 32-key block, K operands read ahead.
// Masked tiles compute every block too (no branch around blocks past the key
// length or above the diagonal): tile_mask then hides them, and the tile
// stays one basic block for the scheduler.  K rows past sk hold zeros (the
// DMA's bounded buffer returns 0 there), so those scores are finite.
template <int BN>
__device__ __forceinline__ void tile_qk(const unsigned char* ks, const LdsOffsets& off, const bf16x8 (&qr)[8],
                                        f32x16 (&s)[BN / 32]) {
    constexpr int KB = BN / 32;
    const f32x16 zero = {};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        bf16x8 kop[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) kop[c] = lds_read16(ks + kb * 32 * ROW_BYTES + off.k[c]);
        s[kb] = mfma32(kop[0], qr[0], zero);
#pragma unroll
        for (int c = 1; c < 8; ++c) s[kb] = mfma32(kop[c], qr[c], s[kb]);
    }
}

// Softmax values carried from the head to the tail of one tile.
struct SmCarry {
    float alpha;      // exp2(m_old - m_new) per lane (1 when the base did not move)
    float neg;        // -m_new
    float pb0, pb1;   // partial sums of the BF16 weights
    float part[4];    // partial FP32 sums (LSE only)
    bool rescale;     // some lane of the wave moved its base: O must be rescaled
};

// Masks of one tile (diagonal / tail variant only): a score is -inf past the
// key length or above the causal diagonal, one select per score and no branch.
template <int BN, bool MASKED, bool CAUSAL>
__device__ __forceinline__ void tile_mask(f32x16 (&s)[BN / 32], int start, int sk, int row, int half) {
    if constexpr (MASKED) {
        const int lim = CAUSAL ? min(sk - 1, row) : sk - 1;   // last visible key of this row
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb) {
            // Score v holds key kl + (v / 4) * 8 + v % 4: compare that small
            // constant with lim - kl, one subtraction per block.
            const int d = lim - (start + kb * 32 + half * 4);
#pragma unroll
            for (int v = 0; v < 16; ++v) s[kb][v] = (v >> 2) * 8 + (v & 3) > d ? -__builtin_inff() : s[kb][v];
        }
    }
}

// P = exp2(s*scale2 - m) for one 16-key unit (half of a 32-key block), as
// one BF16 MFMA B operand.
template <bool LSE>
__device__ __forceinline__ void exp_unit(const f32x16& s, int sub, bf16x8& p, SmCarry& c, float scale2) {
    f32x2 e[4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float x = exp2_native(fmaf(s[sub * 8 + i], scale2, c.neg));
        e[i >> 1][i & 1] = x;
        if constexpr (LSE) c.part[i & 3] += x;
    }
    const bf16x2 b0 = __builtin_convertvector(e[0], bf16x2);
    const bf16x2 b1 = __builtin_convertvector(e[1], bf16x2);
    const bf16x2 b2 = __builtin_convertvector(e[2], bf16x2);
    const bf16x2 b3 = __builtin_convertvector(e[3], bf16x2);
    c.pb0 = bf16_pair_sum(b0, c.pb0);
    c.pb1 = bf16_pair_sum(b1, c.pb1);
    c.pb0 = bf16_pair_sum(b2, c.pb0);
    c.pb1 = bf16_pair_sum(b3, c.pb1);
    p = bf16x8{b0[0], b0[1], b1[0], b1[1], b2[0], b2[1], b3[0], b3[1]};
}

// One 16-register accumulator block at a time, fenced, so the (AGPR-resident)
// accumulators need at most 16 VGPR temporaries while being scaled.
__device__ __forceinline__ void apply_rescale(RowState& st, const SmCarry& c) {
    if (c.rescale) {
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            st.o[db] *= c.alpha;
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// Row max of one tile's raw logits, combined over the two lane halves.
template <int BN>
__device__ __forceinline__ float tile_rowmax(const f32x16 (&s)[BN / 32]) {
    float mx = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kb][v]);
    return xhalf_max(mx);
}

// Softmax and PV of one key tile whose scores S^T are already in `s`, for one
// 32-row wave, software pipelined inside the tile:
//   masks, row max, base update | exp(unit 0) | [rescale O] |
//   PV(unit u-1) beside exp(unit u) ... | PV(last)
// A unit is 16 keys (one PV k-step for all four 32-dim blocks).  Keeping the
// rare O-rescale branch in front of the first PV leaves the exp/PV overlap in
// one basic block, where the scheduler can interleave the VALU work of unit u
// with the MFMAs of unit u-1.
// EMPTY: some rows may have seen no visible key yet (a split-KV key chunk
// past a causal row's diagonal).  Their base stays -inf and the weights are
// computed against 0 instead, so they come out 0 rather than NaN.
template <int BN, bool MASKED, bool CAUSAL, bool LSE, bool EMPTY = false>
__device__ __forceinline__ void attend_tail(f32x16 (&s)[BN / 32], const unsigned char* vs, const LdsOffsets& off,
                                            RowState& st, bool first, int start, int sk, int row, int half,
                                            float scale2) {
    constexpr int KB = BN / 32, U = 2 * KB;
    tile_mask<BN, MASKED, CAUSAL>(s, start, sk, row, half);
    const float mx = tile_rowmax<BN>(s);
    const float cand = fmaxf(st.m, mx * scale2);
    const bool update = first || cand > st.m + RESCALE_THRESHOLD;
    const float next = update ? cand : st.m;
    float base = next;
    if constexpr (EMPTY && MASKED) base = next == -__builtin_inff() ? 0.f : next;
    SmCarry c;
    c.alpha = exp2_native(st.m - base);
    c.rescale = !first && __builtin_amdgcn_ballot_w64(update) != 0;
    st.m = next;
    c.neg = -base;
    c.pb0 = c.pb1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) c.part[i] = 0.f;
    bf16x8 p[U];
    exp_unit<LSE>(s[0], 0, p[0], c, scale2);
    apply_rescale(st, c);
    // PV runs for every unit, masked tiles included: the weights of a hidden
    // block are exactly 0, and a branch here would split the exp/PV overlap
    // (measured: +1.5% causal over skipping hidden blocks).
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (u + 1 < U) exp_unit<LSE>(s[(u + 1) >> 1], (u + 1) & 1, p[u + 1], c, scale2);
        const unsigned char* vb = vs + u * 16 * ROW_BYTES;
        bf16x8 vop[4];
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const bf16x4 lo = lds_read_tr(vb + off.v[0][db]);
            const bf16x4 hi = lds_read_tr(vb + off.v[1][db]);
            vop[db] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int db = 0; db < 4; ++db) st.o[db] = mfma32(vop[db], p[u], st.o[db]);
    }
    st.lb = st.lb * c.alpha + xhalf_sum(c.pb0 + c.pb1);
    if constexpr (LSE) st.l = st.l * c.alpha + xhalf_sum((c.part[0] + c.part[1]) + (c.part[2] + c.part[3]));
}

// QK^T of one tile at raised issue priority, then attend_tail.  When the two
// waves of a SIMD compete, the one feeding QK^T MFMAs goes first and the
// other fills the VALU slots (measured +5% at B32H8S4096).
template <int BN, bool MASKED, bool CAUSAL, bool LSE, bool EMPTY = false>
__device__ __forceinline__ void attend_fused(const unsigned char* ks, const unsigned char* vs, const LdsOffsets& off,
                                             const bf16x8 (&qr)[8], RowState& st, bool first, int start, int sk,
                                             int row, int half, float scale2) {
    f32x16 s[BN / 32];
    __builtin_amdgcn_s_setprio(1);
    tile_qk<BN>(ks, off, qr, s);
    __builtin_amdgcn_s_setprio(0);
    attend_tail<BN, MASKED, CAUSAL, LSE, EMPTY>(s, vs, off, st, first, start, sk, row, half, scale2);
}

// Base update from a precomputed row max, then all of the tile's P units and
// the running sums.  The O rescale it decides is applied by apply_rescale.
template <int BN, bool LSE>
__device__ __forceinline__ void softmax_from_max(const f32x16 (&s)[BN / 32], float mx, bf16x8 (&p)[2 * (BN / 32)],
                                                 RowState& st, SmCarry& c, bool first, float scale2) {
    constexpr int U = 2 * (BN / 32);
    const float cand = fmaxf(st.m, mx * scale2);
    const bool update = first || cand > st.m + RESCALE_THRESHOLD;
    const float next = update ? cand : st.m;
    c.alpha = exp2_native(st.m - next);
    c.rescale = !first && __builtin_amdgcn_ballot_w64(update) != 0;
    st.m = next;
    c.neg = -next;
    c.pb0 = c.pb1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) c.part[i] = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) exp_unit<LSE>(s[u >> 1], u & 1, p[u], c, scale2);
    st.lb = st.lb * c.alpha + xhalf_sum(c.pb0 + c.pb1);
    if constexpr (LSE) st.l = st.l * c.alpha + xhalf_sum((c.part[0] + c.part[1]) + (c.part[2] + c.part[3]));
}

// O^T += V^T.P^T for an unmasked tile.
template <int BN>
__device__ __forceinline__ void pv_plain(const unsigned char* vs, const LdsOffsets& off,
                                         const bf16x8 (&p)[2 * (BN / 32)], RowState& st) {
#pragma unroll
    for (int u = 0; u < 2 * (BN / 32); ++u) {
        const unsigned char* vb = vs + u * 16 * ROW_BYTES;
        bf16x8 vop[4];
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const bf16x4 lo = lds_read_tr(vb + off.v[0][db]);
            const bf16x4 hi = lds_read_tr(vb + off.v[1][db]);
            vop[db] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int db = 0; db < 4; ++db) st.o[db] = mfma32(vop[db], p[u], st.o[db]);
    }
}

// Epilogue store of one wave's 32 rows, O = acc * inv in BF16.  The MFMA
// accumulator gives each lane 8-byte pieces of one row, so stores straight
// from it touch 32 rows (16 bytes each) per instruction, and a workgroup's
// 64 KiB q tile took 2-3.7 us to leave the CU (measured per wave with
// s_memrealtime).  Here the wave stages 32 rows x 128 bytes at a time in LDS
// and each buffer_store_dwordx4 writes 8 rows x 128 contiguous bytes.
//  * slot: byte offset in smem of 2 KiB of this wave's, plus 2 KiB at
//    slot + TILE_BYTES, that no other wave reads or writes meanwhile (the
//    wave's own DMA slots of a stage nobody reads any more).
//  * 16-byte chunks are XOR-swizzled by the row's low 3 bits; a read's 8
//    lanes cover one whole row.  Each 8-byte write lane uses the first or
//    second half of a 16-byte chunk, so 32 rows share 16 slots of a bank
//    window: a 2-way conflict, counted as 64 stall cycles per wave and q tile
//    (SQ_LDS_BANK_CONFLICT), about 0.2% of a launch.
//  * Rows r >= rows (past the sequence) store nothing: their 32-bit offsets
//    could wrap into a valid row for large row strides.
//  * LANE_OPAQUE derives the lane offsets from an opaque copy of the lane
//    id, so that the compiler does not hoist them out of the item loop and
//    keep them live through the key loop (where the LSE kernels' register
//    budget is tight; hoisted, causal LSE spilled).
template <int TILE_BYTES, bool LANE_OPAQUE>
__device__ __forceinline__ void store_o_rows(const RowState& st, float inv, unsigned char* smem, uint32_t slot,
                                             rsrc_t ro, uint32_t orow, int wrow0, int rows, int lane) {
    static_assert(TILE_BYTES >= 16 * 128, "staging rows");
    if constexpr (LANE_OPAQUE) asm volatile("" : "+v"(lane));
    const int col = lane & 31, half = lane >> 5;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int dl = 0; dl < 2; ++dl) {
#pragma unroll
            for (int vg = 0; vg < 4; ++vg) {
                const f32x16& o = st.o[2 * h + dl];
                const f32x2 x0 = {o[vg * 4 + 0] * inv, o[vg * 4 + 1] * inv};
                const f32x2 x1 = {o[vg * 4 + 2] * inv, o[vg * 4 + 3] * inv};
                const bf16x2 y0 = __builtin_convertvector(x0, bf16x2);
                const bf16x2 y1 = __builtin_convertvector(x1, bf16x2);
                // Row col, bytes 64 * db + 16 * vg + 8 * half of the row, i.e.
                // chunk 4 * dl + vg of its 128-byte half h.
                const int chunk = 4 * dl + vg;
                const uint32_t off = slot + (col >> 4) * TILE_BYTES + (col & 15) * 128 +
                                     ((chunk ^ (col & 7)) << 4) + half * 8;
                *reinterpret_cast<FAV4_LDS bf16x4*>((FAV4_LDS void*)(smem + off)) = bf16x4{y0[0], y0[1], y1[0], y1[1]};
            }
        }
        // Store i: rows 8i .. 8i+7, lane l writing chunk l % 8 of row 8i + l / 8.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 8 * i + (lane >> 3), c = lane & 7;
            const uint32_t off = slot + (r >> 4) * TILE_BYTES + (r & 15) * 128 + ((c ^ (r & 7)) << 4);
            const bf16x8 v = *reinterpret_cast<const FAV4_LDS bf16x8*>((FAV4_LDS const void*)(smem + off));
            if (r < rows) store16(ro, uint32_t(wrow0 + r) * orow + h * 128 + c * 16, __builtin_bit_cast(f32x4, v));
        }
    }
}

// WAVES waves x 32 query rows per workgroup, BN keys per tile, STAGES LDS
// buffers of K+V.  Tile t lives in stage t % STAGES; its DMA is issued
// STAGES-1 tiles ahead (right after barrier t-STAGES+1, into the stage that
// tile t-STAGES used, which every wave finished reading before that barrier).
// PIPE (3 stages): unmasked key tiles run software pipelined across tiles,
// QK^T(t+1) beside softmax(t) and PV(t) beside the row max of tile t+1, so
// each wave always has MFMA and VALU work in flight.  K(t+1) and V(t) are
// both read between barriers t and t+1; the DMA of tile t+2 goes to the third
// stage.  Masked tiles (causal diagonal, key tail) follow unpipelined.
// LDS layout: two stages are [K0 V0 K1 V1]; three are [K0 K1 K2 V0 V1 V2],
// with the V ring's base folded into the lanes' V offsets once, so that every
// operand read's constant part stays inside the 16-bit ds_read offset (a
// stage at 64 KiB or more would otherwise cost an address add per read).
template <int WAVES, int BN, bool CAUSAL, bool LSE, int STAGES, bool PIPE = false>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fwd_kernel(Fav4Args a, Layout L, int tiles, int total) {
    static_assert(PIPE ? STAGES == 3 : STAGES == 2, "two stages, or three with the cross-tile pipeline");
    constexpr int BM = WAVES * 32;
    constexpr int TILE_BYTES = BN * ROW_BYTES;
    constexpr int STAGE_BYTES = 2 * TILE_BYTES;          // K then V
    constexpr int DMA = BN / 4 / WAVES;                  // 1 KiB DMA ops per wave per matrix
    constexpr int AHEAD = STAGES - 1;                    // prefetch distance in tiles
    static_assert(BN % 32 == 0 && BN % (4 * WAVES) == 0, "tile shape");
    static_assert(STAGES == 2 || STAGES == 3, "stages");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[STAGES * STAGE_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 31, half = lane >> 5;
    const float scale2 = a.scale * LOG2E;
    const uint32_t smem_base = lds_addr(smem);

    // K / V tile of stage s: byte offsets from smem, and the pointers the
    // operand reads use (for three stages the V ring base is in off.v).
    constexpr auto k_at = [](int s) { return STAGES == 3 ? s * TILE_BYTES : s * STAGE_BYTES; };
    constexpr auto v_at = [](int s) { return STAGES == 3 ? (3 + s) * TILE_BYTES : s * STAGE_BYTES + TILE_BYTES; };
    auto kst = [&](int s) -> const unsigned char* { return smem + k_at(s); };
    auto vst = [&](int s) -> const unsigned char* { return smem + (STAGES == 3 ? s * TILE_BYTES : v_at(s)); };
    LdsOffsets off = lds_offsets(lane);
    if constexpr (STAGES == 3) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                off.v[j][db] += 3 * TILE_BYTES;
                asm volatile("" : "+v"(off.v[j][db]));   // kept whole: not re-split into base + constant
            }
    }
    const DmaOffsets<DMA> dofs = dma_offsets<DMA>(wave, lane, L.kr, L.vr);

    auto process = [&](int bh, int tile) {
        const int batch = bh / a.heads, head = bh - batch * a.heads;
        const int q0 = tile * BM, qw = q0 + wave * 32;
        const int row = qw + col;                                 // this lane's query row
        const int kvh = head / L.group;
        const char* kbase = static_cast<const char*>(a.k) + batch * L.kb + kvh * L.kh;
        const char* vbase = static_cast<const char*>(a.v) + batch * L.vb + kvh * L.vh;
        const rsrc_t rq = make_rsrc(static_cast<const char*>(a.q) + batch * L.qb + head * L.qh + int64_t(q0) * L.qr,
                                    uint32_t(a.sq - q0 - 1) * L.qr + ROW_BYTES);
        const rsrc_t ro = make_rsrc(static_cast<char*>(a.o) + batch * L.ob + head * L.oh + int64_t(q0) * L.orow,
                                    uint32_t(a.sq - q0 - 1) * L.orow + ROW_BYTES);
        // Key tiles: [0, nfull) are unmasked for every row of the workgroup,
        // [nfull, ntiles) cross the key tail or the causal diagonal.
        constexpr int BNT = BN;                           // keys per LDS tile
        const int kend = CAUSAL ? min(a.sk, q0 + BM) : a.sk;
        const int ntiles = (kend + BNT - 1) / BNT;
        const int nfull = (CAUSAL ? min(a.sk, q0 + 1) : a.sk) / BNT;

        // DMA of tile t into stage t % STAGES.  Tiles past the last one are
        // clamped to it (the copy lands in a stage nobody reads any more), so
        // the prefetch needs no branch and vmcnt bookkeeping stays uniform.
        auto issue = [&](int t) {
            const int tc = min(t, ntiles - 1);
            const int64_t first = int64_t(tc) * BNT;
            const uint32_t rows = uint32_t(a.sk - int(first) - 1);
            const u32x4 rk = make_desc(kbase + first * L.kr, rows * L.kr + ROW_BYTES);
            const u32x4 rv = make_desc(vbase + first * L.vr, rows * L.vr + ROW_BYTES);
            const int s = t % STAGES;
            dma_kv<DMA>(rk, rv, smem_base + k_at(s), smem_base + v_at(s), wave, dofs);
        };

#pragma unroll
        for (int t = 0; t < AHEAD; ++t) issue(t);   // PIPE: tiles 0 and 1
        bf16x8 qr[8];
        {
            const uint32_t qoff = uint32_t(wave * 32 + col) * L.qr + half * 16;
#pragma unroll
            for (int c = 0; c < 8; ++c) qr[c] = load16(rq, qoff + c * 32);
            // Retire the Q loads here, so that inside the key loop the only
            // outstanding vector-memory ops are K/V DMAs.
#pragma unroll
            for (int c = 0; c < 8; ++c) asm volatile("" ::"v"(qr[c]));
        }
        RowState st;
#pragma unroll
        for (int db = 0; db < 4; ++db) st.o[db] = f32x16{};
        st.m = -__builtin_inff();
        st.lb = 0.f;
        st.l = 0.f;

        // One pipeline step on a compile-time stage: wait for tile t (the
        // AHEAD-1 younger tiles may stay in flight), prefetch tile t+AHEAD,
        // then attend to tile t.
        auto step = [&](auto stage_c, auto masked_c, int t) {
            constexpr int STAGE = decltype(stage_c)::value;
            constexpr bool MASKED = decltype(masked_c)::value;
            wait_vmem_keep<2 * DMA * (AHEAD - 1)>();
            __syncthreads();
            issue(t + AHEAD);
            // A causal tile entirely above this wave's rows changes nothing
            // (tile 0 never is): the wave only keeps the DMA and barriers.
            if (!(MASKED && CAUSAL) || t * BN <= qw + 31)
                attend_fused<BN, MASKED, CAUSAL, LSE>(kst(STAGE), vst(STAGE), off, qr, st, t == 0, t * BN, a.sk,
                                                      row, half, scale2);
        };
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        using Plain = std::integral_constant<bool, false>;
        using Masked = std::integral_constant<bool, true>;
        int t = 0;
        if constexpr (PIPE) {
            if (nfull > 6) {
                f32x16 sa[BN / 32], sb[BN / 32];
                bf16x8 p[2 * (BN / 32)];
                SmCarry c;
                wait_vmem();
                __syncthreads();
                tile_qk<BN>(kst(0), off, qr, sa);
                float mx = tile_rowmax<BN>(sa);
                // Pipelined tile t (stage STAGE = t%3): S(t) in `cur`, QK^T(t+1)
                // into `nxt` from stage (t+1)%3, then PV(t).
                auto pstep = [&](auto stage_c, f32x16 (&cur)[BN / 32], f32x16 (&nxt)[BN / 32], int t) {
                    constexpr int STAGE = decltype(stage_c)::value;
                    wait_vmem();        // tile t+1 has landed (issued one tile ago)
                    __syncthreads();
                    issue(t + 2);
                    __builtin_amdgcn_s_setprio(1);
                    tile_qk<BN>(kst((STAGE + 1) % 3), off, qr, nxt);
                    __builtin_amdgcn_s_setprio(0);
                    softmax_from_max<BN, LSE>(cur, mx, p, st, c, t == 0, scale2);
                    apply_rescale(st, c);
                    pv_plain<BN>(vst(STAGE), off, p, st);
                    mx = tile_rowmax<BN>(nxt);
                };
                using P0 = std::integral_constant<int, 0>;
                using P1 = std::integral_constant<int, 1>;
                using P2 = std::integral_constant<int, 2>;
                for (; t + 6 < nfull; t += 6) {
                    pstep(P0{}, sa, sb, t);
                    pstep(P1{}, sb, sa, t + 1);
                    pstep(P2{}, sa, sb, t + 2);
                    pstep(P0{}, sb, sa, t + 3);
                    pstep(P1{}, sa, sb, t + 4);
                    pstep(P2{}, sb, sa, t + 5);
                }
                // Drain tile t (t % 3 == 0): K already consumed, V in stage 0.
                softmax_from_max<BN, LSE>(sa, mx, p, st, c, t == 0, scale2);
                apply_rescale(st, c);
                pv_plain<BN>(vst(0), off, p, st);
                ++t;
            }
            // Remaining tiles, unpipelined, prefetch distance 1 (stage t%3).
            for (; t < ntiles; ++t) {
                const int r = t % 3;
                const bool plain = t < nfull;
                auto mstep = [&](auto stage_c, auto masked_c) {
                    constexpr int STAGE = decltype(stage_c)::value;
                    wait_vmem();
                    __syncthreads();
                    issue(t + 1);
                    attend_fused<BN, decltype(masked_c)::value, CAUSAL, LSE>(kst(STAGE), vst(STAGE), off, qr, st,
                                                                             t == 0, t * BN, a.sk, row, half,
                                                                             scale2);
                };
                using M0 = std::integral_constant<int, 0>;
                using M1 = std::integral_constant<int, 1>;
                using M2 = std::integral_constant<int, 2>;
                using Pl = std::integral_constant<bool, false>;
                using Mk = std::integral_constant<bool, true>;
                if (plain) {
                    if (r == 0) mstep(M0{}, Pl{});
                    else if (r == 1) mstep(M1{}, Pl{});
                    else mstep(M2{}, Pl{});
                } else {
                    if (r == 0) mstep(M0{}, Mk{});
                    else if (r == 1) mstep(M1{}, Mk{});
                    else mstep(M2{}, Mk{});
                }
            }
        } else if constexpr (STAGES == 2) {
            if (qw >= a.sq) {
                // All 32 rows of this wave lie past sq (tail q tile): it only
                // keeps the loop's DMA and barrier sequence.  Deciding once per
                // q tile keeps the branch out of the step body.
                for (; t < ntiles; ++t) {
                    wait_vmem();
                    __syncthreads();
                    issue(t + 1);
                }
            } else {
                for (; t + 1 < nfull; t += 2) {
                    step(S0{}, Plain{}, t);
                    step(S1{}, Plain{}, t + 1);
                }
                // t is even here, so the masked tiles also run in compile-time
                // stage pairs: a runtime choice between two step bodies made
                // the register allocator give O two homes and copy it (64-128
                // moves) on every masked step.
                for (; t + 1 < ntiles; t += 2) {
                    step(S0{}, Masked{}, t);
                    step(S1{}, Masked{}, t + 1);
                }
                if (t < ntiles) step(S0{}, Masked{}, t);
            }
        }

        // Epilogue: O = acc / lb in BF16.
        // Dividing by the sum of the rounded weights keeps them normalised, so
        // the BF16 rounding of P perturbs O by sum_j w_j e_j (V_j - O) instead
        // of sum_j w_j e_j V_j (exact when one key dominates).
        // Rows >= sq store nothing.  The store bound alone does not stop them:
        // their 32-bit offsets (row - q0) * row stride can wrap past 2^32 into
        // a valid row when the row stride is large (huge head counts, strided
        // views), and they carry another row's result.
        const float inv = 1.f / st.lb;
        if constexpr (STAGES == 2) {
            // The clamped last prefetch went to stage ntiles % 2, which no wave
            // reads any more: once this wave's own part of that DMA has landed,
            // its slots there hold the O staging.
            static_assert(STAGES != 2 || DMA >= 2, "a wave's DMA slots hold 2 KiB per matrix");
            wait_vmem();
            store_o_rows<TILE_BYTES, LSE>(st, inv, smem, uint32_t((ntiles & 1) * STAGE_BYTES + wave * DMA * 1024), ro,
                                          L.orow, wave * 32, a.sq - qw, lane);
        } else {
            const uint32_t obase = uint32_t(wave * 32 + col) * L.orow + half * 8;
            if (row < a.sq) {
#pragma unroll
                for (int db = 0; db < 4; ++db) {
#pragma unroll
                    for (int vg = 0; vg < 4; ++vg) {
                        const f32x2 x0 = {st.o[db][vg * 4 + 0] * inv, st.o[db][vg * 4 + 1] * inv};
                        const f32x2 x1 = {st.o[db][vg * 4 + 2] * inv, st.o[db][vg * 4 + 3] * inv};
                        const bf16x2 y0 = __builtin_convertvector(x0, bf16x2);
                        const bf16x2 y1 = __builtin_convertvector(x1, bf16x2);
                        store8(ro, obase + (db * 32 + vg * 8) * 2, bf16x4{y0[0], y0[1], y1[0], y1[1]});
                    }
                }
            }
        }
        // An explicit FMA: every kernel rounds the LSE the same way, whatever
        // the compiler's contraction choice in its surroundings.
        if constexpr (LSE) {
            if (half == 0 && row < a.sq) a.lse[int64_t(bh) * a.sq + row] = __builtin_fmaf(st.m, LN2, logf(st.l));
        }
        wait_vmem();       // clamped prefetches and O stores have landed before the stages are reused
        __syncthreads();
    };
    for_each_item<CAUSAL>(tiles, total, process);
}

// ---------------------------------------------------------------------------
// Split-KV: the key range of every (batch, head, q tile) is cut into `splits`
// chunks of `tps` key tiles, each chunk is attended by its own workgroup (same
// tile body as fwd_kernel, 3 LDS stages), and a second kernel merges the
// chunks.  For few (b, h, q tile) items and long
// keys this fills the GPU where one workgroup per item cannot.
// Workspace (FP32, caller-owned):
//   o_part  [splits][B*H][sq][128]  O of the chunk, normalised by its own
//                                    BF16 weight sum lb_s
//   lse_part[splits][B*H][sq][2]    log2-domain sums of the chunk:
//                                    (m_s + log2 lb_s, m_s + log2 l_s)
// The merge weights chunk s by 2^(m_s) lb_s (the first log-sum), which makes
// the merged O exactly the single-pass acc / lb; the LSE output is
// ln 2 * log2(sum_s 2^(m_s) l_s) from the second, the single-pass FP32 sum.
// Rows with no visible key in a chunk (causal) carry -inf and weight 0.
// ---------------------------------------------------------------------------
struct SplitArgs {
    float* o_part;
    float* lse_part;
    int splits, tps;
    // Packed variable-length sequences (null cu_q: BSHD).  Sequence b's
    // queries are tokens [cu_q[b], cu_q[b+1]) of Q/O, its keys tokens
    // [cu_k[b], cu_k[b+1]) of K/V; the Fav4Args shape then carries the
    // sequence count and max_seqlen_q / max_seqlen_k.
    const int* cu_q;
    const int* cu_k;
    int total_q, total_k;
    // Paged K/V caches (PAGED kernels): sequence b has seqlens_k[b] keys, key
    // j in row block_table[b * max_pages + j / page_size] * page_size +
    // j % page_size of the [num_pages * page_size, kv_heads, 128] caches.
    const int* seqlens_k;
    const int* block_table;
    int page_size, max_pages, num_pages;
};

// Query / key count and first token of sequence b (the same in every lane of
// the workgroup), read on the device and clamped to [0, total] and to the max
// lengths, as fwd_kernel_varlen does.  PAGED: the key count is seqlens_k[b]
// clamped to [0, max_k] (ktok unused).
struct SeqSpan {
    int sq, sk;
    int64_t qtok, ktok;
};
template <bool PAGED>
__device__ __forceinline__ SeqSpan seq_span(const SplitArgs& sp, int b, int max_q, int max_k) {
    auto rd = [](int x) { return __builtin_amdgcn_readfirstlane(x); };
    const int qs = min(max(rd(sp.cu_q[b]), 0), sp.total_q);
    const int qe = min(max(rd(sp.cu_q[b + 1]), qs), min(sp.total_q, qs + max_q));
    if constexpr (PAGED) return {qe - qs, min(max(rd(sp.seqlens_k[b]), 0), max_k), qs, 0};
    const int ks = min(max(rd(sp.cu_k[b]), 0), sp.total_k);
    const int ke = min(max(rd(sp.cu_k[b + 1]), ks), min(sp.total_k, ks + max_k));
    return {qe - qs, ke - ks, qs, ks};
}

// Three LDS stages keep two key tiles in flight per workgroup (prefetch
// distance 2).  Long-key prefill chunks run as fast as with two; decode-like
// chunks, where one wave computes and the kernel mostly streams K/V, gain up
// to 10% (measured), since the DMA latency rather than the MFMAs bounds a tile.
// WAVES = 8, BN = 64: long-key prefill chunks (256-row q tiles).  WAVES = 1,
// BN = 32: decode (sq <= 32): one wave per workgroup and 48 KiB of LDS, so
// three workgroups share a CU and every resident wave computes.
// LSE: keep the FP32 sums for the LSE output; without it the second log-sum
// repeats the first (the merge reads it only when writing an LSE).
// VARLEN: packed sequences; a.sq / a.sk are the max lengths, rows keep the
// a.sq stride, and rows past a sequence's own length are computed on a valid
// query but never read by the merge (eight waves: q tiles past them exit).
// PAGED (with VARLEN): K/V come from paged caches.  page_size is a multiple
// of BN, so a key tile lies in one page; a chunk spans at most 64 pages, whose
// (clamped) numbers one load puts in the wave's lanes at the chunk start.
// BR (with CAUSAL and VARLEN): bottom-right causal, query i of a sequence
// with sq queries and sk keys sees keys j <= sk - sq + i (the last query sees
// all of them; with sq > sk the first sq - sk rows see none).
// The one-wave shape keeps the 8-wave shape's 256-register budget
// (waves_per_eu 2); its occupancy is set by LDS (three workgroups per CU), so
// the compiler's note that it cannot reach two waves per SIMD is expected.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wpass-failed"
template <int BN, bool CAUSAL, int WAVES, bool LSE, bool VARLEN = false, bool PAGED = false, bool BR = false>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fwd_kernel_split(Fav4Args a, SplitArgs sp, int kv_heads, int tiles, int total) {
    static_assert(!PAGED || VARLEN, "paged caches hold packed sequences");
    static_assert(!BR || (CAUSAL && VARLEN), "bottom-right causal needs per-sequence lengths");
    constexpr int BM = WAVES * 32, STAGES = 3;
    // One wave (decode): the q-tile rows are the group's query heads times
    // their sq queries, row r = (head - first head of the group) * sq + query,
    // so the heads that share a K/V head stream it once.  Eight waves: the
    // rows of one head.
    constexpr bool PACK = WAVES == 1;
    constexpr int TILE_BYTES = BN * ROW_BYTES;
    constexpr int STAGE_BYTES = 2 * TILE_BYTES;
    constexpr int DMA = BN / 4 / WAVES;
    static_assert(BN % 32 == 0 && BN % (4 * WAVES) == 0, "tile shape");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[STAGES * STAGE_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 31, half = lane >> 5;
    const uint32_t row_bytes = uint32_t(a.heads) * ROW_BYTES;
    const uint32_t kv_row_bytes = uint32_t(kv_heads) * ROW_BYTES;
    const int group = a.heads / kv_heads;
    const float scale2 = a.scale * LOG2E;
    const uint32_t smem_base = lds_addr(smem);
    const int bhs = a.batch * a.heads;

    const LdsOffsets off = lds_offsets(lane);
    const DmaOffsets<DMA> dofs = dma_offsets<DMA>(wave, lane, kv_row_bytes, kv_row_bytes);

    // Rows of one item's row space: a head's queries, or a group's.
    const int rows = PACK ? group * a.sq : a.sq;
    const int items_per_batch = PACK ? kv_heads : a.heads;
    const int npairs = a.batch * items_per_batch, full = npairs >> 3, rem8 = npairs & 7;
    for (int id = blockIdx.x; id < total; id += gridDim.x) {
        // XCD-contiguous order; within a (b, h) -- PACK: (b, K/V head) -- the
        // q tiles of one key chunk are adjacent, so they share it in L2.
        const int xcd = id & 7, slot = id >> 3, per = total >> 3, rem = total & 7;
        const int logical = xcd * per + min(xcd, rem) + slot;
        const int per_item = tiles * sp.splits;
        int it = __builtin_amdgcn_readfirstlane(logical / per_item);
        const int r = __builtin_amdgcn_readfirstlane(logical - it * per_item);
        if constexpr (VARLEN) {
            // Packed sequences differ in length: take the (sequence, head)
            // pairs column by column from an 8-wide grid (it = 8 * row + col,
            // as fwd_kernel_varlen does), so XCD x works on the pairs with
            // it % 8 == x -- a share of every sequence -- instead of a few
            // whole sequences.  With 8 K/V heads each XCD gets one head of
            // every sequence.
            const int j = it;
            int gcol, grow;
            if (j < rem8 * (full + 1)) {
                gcol = j / (full + 1);
                grow = j - gcol * (full + 1);
            } else {
                const int jj = j - rem8 * (full + 1);
                gcol = rem8 + jj / full;
                grow = jj - (gcol - rem8) * full;
            }
            it = __builtin_amdgcn_readfirstlane(grow * 8 + gcol);
        }
        const int split = r / tiles, tile = r - split * tiles;

        // it = b*heads + h, or (PACK) b*kv_heads + K/V head; head0 = the first
        // query head of the item's rows.
        const int batch = it / items_per_batch, unit = it - batch * items_per_batch;
        const int head0 = PACK ? unit * group : unit;
        const int bh = batch * a.heads + head0;
        const int q0 = tile * BM, qw = q0 + wave * 32;
        const int row = qw + col;                              // row of the item's row space
        // The sequence: its query / key counts and first tokens.
        SeqSpan span{a.sq, a.sk, int64_t(batch) * a.sq, int64_t(batch) * a.sk};
        if constexpr (VARLEN) {
            span = seq_span<PAGED>(sp, batch, a.sq, a.sk);
            // No query rows (eight waves: none from this q tile on): nothing to merge.
            if (span.sq == 0 || (!PACK && q0 >= span.sq)) continue;
        }
        const int sq = span.sq, sk = span.sk;
        // This lane's query position (causal limit) and Q byte offset inside
        // the sequence's [sq, heads] block; rows past the space (or past the
        // sequence's queries) read a valid row.
        const int prow = min(row, rows - 1);
        const int qi = PACK ? prow % a.sq : prow;
        const int qhead = PACK ? head0 + prow / a.sq : head0;
        const int qload = min(qi, sq - 1);
        const int64_t krow0 = span.ktok * kv_heads + head0 / group;
        const char* kbase = static_cast<const char*>(a.k) + krow0 * ROW_BYTES;
        const char* vbase = static_cast<const char*>(a.v) + krow0 * ROW_BYTES;
        const rsrc_t rq = make_rsrc(static_cast<const char*>(a.q) + span.qtok * row_bytes, uint32_t(sq) * row_bytes);
        // This chunk's rows of o_part: [rows - q0][128] FP32 from row q0 (a
        // group's heads are adjacent, so its rows are contiguous).
        const int64_t prow0 = (int64_t(split) * bhs + bh) * a.sq + q0;
        const rsrc_t rp = make_rsrc(sp.o_part + prow0 * D, uint32_t(rows - q0) * D * 4);
        // PACK: every q tile holds rows of query 0 and of the last query, so
        // the causal range is the whole [0, min(sk, sq)) and no tile is
        // unmasked for every row.  BR: unmasked for every row below key
        // sk - sq + 1 (query 0's first hidden key); PACK sees [0, sk) (its
        // tile holds the last query), a q tile of rows [q0, q0 + BM) only up
        // to its last row's diagonal, so chunks past it are empty.
        const int kend = !CAUSAL ? sk
                         : BR    ? (PACK ? sk : min(sk, max(0, min(sq, q0 + BM) + sk - sq)))
                                 : min(sk, PACK ? sq : q0 + BM);
        const int ntiles = (kend + BN - 1) / BN;
        const int nfull = (BR ? max(0, (PACK ? 0 : q0) + sk - sq + 1) : CAUSAL ? (PACK ? 0 : min(sk, q0 + 1)) : sk) / BN;
        const int climit = BR ? qi + sk - sq : qi;     // last visible key of this lane's row
        const int t0 = split * sp.tps, t1 = min(ntiles, t0 + sp.tps);

        RowState st;
#pragma unroll
        for (int db = 0; db < 4; ++db) st.o[db] = f32x16{};
        st.m = -__builtin_inff();
        st.lb = 0.f;
        st.l = 0.f;

        if (t0 < t1) {
            // PAGED: lane l holds the page of the chunk's l-th page slot.
            int pages = 0, page0 = 0;
            if constexpr (PAGED) {
                page0 = t0 * BN / sp.page_size;
                const int slot = min(page0 + lane, sp.max_pages - 1);
                pages = min(max(sp.block_table[int64_t(batch) * sp.max_pages + slot], 0), sp.num_pages - 1);
            }
            // DMA of key tile t into stage (t - t0) % 3.  Tiles past the chunk
            // are clamped to its last one (the copy lands in a stage no later
            // step reads), keeping the vmcnt count uniform.
            auto issue = [&](int t) {
                const int first = min(t, t1 - 1) * BN;
                int64_t row0 = first;                       // the tile's first K/V row
                int rows_left = sk - first;                 // rows the descriptor may cover
                if constexpr (PAGED) {
                    const int in_page = first % sp.page_size;
                    const int page = __builtin_amdgcn_readlane(pages, first / sp.page_size - page0);
                    row0 = int64_t(page) * sp.page_size + in_page;
                    rows_left = min(rows_left, sp.page_size - in_page);
                }
                const uint32_t bytes = uint32_t(rows_left - 1) * kv_row_bytes + ROW_BYTES;
                const u32x4 rk = make_desc(kbase + row0 * kv_row_bytes, bytes);
                const u32x4 rv = make_desc(vbase + row0 * kv_row_bytes, bytes);
                dma_tile<DMA, TILE_BYTES, PACK>(rk, rv, smem_base + ((t - t0) % STAGES) * STAGE_BYTES, wave, dofs);
            };
            issue(t0);
            issue(t0 + 1);
            bf16x8 qr[8];
            {
                const uint32_t qoff = uint32_t(qload) * row_bytes + uint32_t(qhead) * ROW_BYTES + half * 16;
#pragma unroll
                for (int c = 0; c < 8; ++c) qr[c] = load16(rq, qoff + c * 32);
#pragma unroll
                for (int c = 0; c < 8; ++c) asm volatile("" ::"v"(qr[c]));
            }
            // Wait for tile t (tile t+1 may stay in flight), then prefetch
            // tile t+2 into the stage freed by the barrier (tile t-1's).
            auto sync_and_prefetch = [&](int t) {
                wait_vmem_keep<2 * DMA>();
                __syncthreads();
                issue(t + 2);
            };
            auto step = [&](auto stage_c, auto masked_c, int t) {
                constexpr int STAGE = decltype(stage_c)::value;
                const unsigned char* cur = smem + STAGE * STAGE_BYTES;
                sync_and_prefetch(t);
                attend_fused<BN, decltype(masked_c)::value, CAUSAL, LSE, CAUSAL>(
                    cur, cur + TILE_BYTES, off, qr, st, t == t0, t * BN, sk, climit, half, scale2);
            };
            using S0 = std::integral_constant<int, 0>;
            using S1 = std::integral_constant<int, 1>;
            using S2 = std::integral_constant<int, 2>;
            using Plain = std::integral_constant<bool, false>;
            using Masked = std::integral_constant<bool, true>;
            int t = t0;
            const int tp = min(t1, nfull);
            if (qw >= (VARLEN && !PACK ? sq : rows)) {
                // Rows all past sq (decode: 7 of 8 waves): only the DMA and
                // barrier sequence of the loop below.
                for (; t < t1; ++t) sync_and_prefetch(t);
            } else {
                for (; t + 2 < tp; t += 3) {
                    step(S0{}, Plain{}, t);
                    step(S1{}, Plain{}, t + 1);
                    step(S2{}, Plain{}, t + 2);
                }
                // (t - t0) % 3 == 0 here: the masked tiles run in compile-time
                // stage triples as well, so O keeps one register home.
                for (; t + 2 < t1; t += 3) {
                    step(S0{}, Masked{}, t);
                    step(S1{}, Masked{}, t + 1);
                    step(S2{}, Masked{}, t + 2);
                }
                if (t < t1) step(S0{}, Masked{}, t);
                if (t + 1 < t1) step(S1{}, Masked{}, t + 1);
            }
        }

        // Chunk epilogue: FP32 O / lb and the two log2-domain sums.  A packed
        // sequence's chunks past its keys skip the O rows: their log-sums are
        // -inf, so the merge gives them weight 0 and never adds their O.
        const float inv = st.lb > 0.f ? 1.f / st.lb : 0.f;
        const uint32_t pbase = uint32_t(wave * 32 + col) * (D * 4) + half * 16;
#pragma unroll
        for (int db = 0; db < 4 && !(VARLEN && t0 >= t1); ++db) {
#pragma unroll
            for (int vg = 0; vg < 4; ++vg) {
                const f32x4 x = {st.o[db][vg * 4 + 0] * inv, st.o[db][vg * 4 + 1] * inv,
                                 st.o[db][vg * 4 + 2] * inv, st.o[db][vg * 4 + 3] * inv};
                store16(rp, pbase + (db * 32 + vg * 8) * 4, x);
            }
        }
        if (half == 0 && row < rows && qi < sq) {
            float* lp = sp.lse_part + ((int64_t(split) * bhs + bh) * a.sq + row) * 2;
            const float sb = st.m + __builtin_amdgcn_logf(st.lb);
            lp[0] = sb;
            lp[1] = LSE ? st.m + __builtin_amdgcn_logf(st.l) : sb;
        }
        wait_vmem();
        __syncthreads();
    }
}

#pragma clang diagnostic pop

// ---------------------------------------------------------------------------
// Varlen: packed sequences.  Q/O are [total_q, heads, 128] and K/V
// [total_k, kv_heads, 128]; sequence b owns rows [cu_seqlens_q[b],
// cu_seqlens_q[b+1]) and [cu_seqlens_k[b], cu_seqlens_k[b+1]); LSE is
// [heads, total_q].  One item per (b, h, 256-row
// q tile up to max_seqlen_q); items past a sequence's end do nothing.  The
// offsets read from device memory are clamped to [0, total] and to the
// maximum lengths, so every access stays inside the caller's buffers.
// BR (with CAUSAL): bottom-right causal, query i of a sequence with sq queries
// and sk keys sees keys j <= sk - sq + i; with sq > sk the first sq - sk rows
// see none and give O = 0, LSE = -inf.
// ---------------------------------------------------------------------------
template <int BN, bool CAUSAL, bool LSE, int WAVES, bool BR = false>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fwd_kernel_varlen(Fav4VarlenArgs a, int tiles, int total) {
    static_assert(!BR || CAUSAL, "bottom-right is a causal mask");
    constexpr int BM = WAVES * 32;
    constexpr int TILE_BYTES = BN * ROW_BYTES;
    constexpr int STAGE_BYTES = 2 * TILE_BYTES;
    constexpr int DMA = BN / 4 / WAVES;
    static_assert(BN % 32 == 0 && BN % (4 * WAVES) == 0, "tile shape");
    static_assert(DMA >= 2, "a wave's DMA slots hold 2 KiB per matrix (O staging)");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * STAGE_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 31, half = lane >> 5;
    const uint32_t row_bytes = uint32_t(a.heads) * ROW_BYTES;
    const uint32_t kv_row_bytes = uint32_t(a.kv_heads) * ROW_BYTES;
    const int group = a.heads / a.kv_heads;
    const float scale2 = a.scale * LOG2E;
    const uint32_t smem_base = lds_addr(smem);

    const LdsOffsets off = lds_offsets(lane);
    const DmaOffsets<DMA> dofs = dma_offsets<DMA>(wave, lane, kv_row_bytes, kv_row_bytes);

    // Item order.  Each XCD gets a contiguous run of logical items (all q
    // tiles of a (sequence, head) together, for its L2), but the runs are cut
    // from the (sequence, head) pairs taken column by column from an 8-wide
    // grid, bh = 8*row + col: XCD x holds mostly the pairs with bh % 8 == x,
    // i.e. a share of every sequence rather than a few whole sequences, so
    // ragged lengths do not leave XCDs idle.  Within a pair the q tiles run
    // last-to-first (causal: heaviest first).
    const int nbh = a.batch * a.heads, full = nbh >> 3, rem8 = nbh & 7;
    for (int id = blockIdx.x; id < total; id += gridDim.x) {
        const int xcd = id & 7, slot = id >> 3, per = total >> 3, rem = total & 7;
        const int logical = xcd * per + min(xcd, rem) + slot;
        const int j = __builtin_amdgcn_readfirstlane(logical / tiles);
        const int tile = __builtin_amdgcn_readfirstlane(tiles - 1 - (logical - j * tiles));
        int gcol, grow;
        if (j < rem8 * (full + 1)) {
            gcol = j / (full + 1);
            grow = j - gcol * (full + 1);
        } else {
            const int jj = j - rem8 * (full + 1);
            gcol = rem8 + jj / full;
            grow = jj - (gcol - rem8) * full;
        }
        const int bh = grow * 8 + gcol;
        const int batch = bh / a.heads, head = bh - batch * a.heads;
        const int qs = min(max(__builtin_amdgcn_readfirstlane(a.cu_seqlens_q[batch]), 0), a.total_q);
        const int qe = min(max(__builtin_amdgcn_readfirstlane(a.cu_seqlens_q[batch + 1]), qs), min(a.total_q, qs + a.max_seqlen_q));
        const int ks = min(max(__builtin_amdgcn_readfirstlane(a.cu_seqlens_k[batch]), 0), a.total_k);
        const int ke = min(max(__builtin_amdgcn_readfirstlane(a.cu_seqlens_k[batch + 1]), ks), min(a.total_k, ks + a.max_seqlen_k));
        const int sq = qe - qs, sk = ke - ks;
        const int q0 = tile * BM;
        if (q0 >= sq) continue;    // uniform over the workgroup
        const int qw = q0 + wave * 32, row = qw + col;
        const int64_t qrow0 = (int64_t(qs) + q0) * a.heads + head;
        const int64_t krow0 = int64_t(ks) * a.kv_heads + head / group;
        const char* kbase = static_cast<const char*>(a.k) + krow0 * ROW_BYTES;
        const char* vbase = static_cast<const char*>(a.v) + krow0 * ROW_BYTES;
        const rsrc_t rq = make_rsrc(static_cast<const char*>(a.q) + qrow0 * ROW_BYTES,
                                    uint32_t(sq - q0 - 1) * row_bytes + ROW_BYTES);
        const rsrc_t ro = make_rsrc(static_cast<char*>(a.o) + qrow0 * ROW_BYTES,
                                    uint32_t(sq - q0 - 1) * row_bytes + ROW_BYTES);
        // Key tiles [0, nfull) are unmasked for every row of the q tile;
        // BR: up to the last row's diagonal, and unmasked below the first
        // row's (shift = sk - sq; may be negative).
        const int shift = BR ? sk - sq : 0;
        const int kend = !CAUSAL ? sk : BR ? min(sk, max(0, min(sq, q0 + BM) + shift)) : min(sk, q0 + BM);
        const int ntiles = (kend + BN - 1) / BN;
        const int nfull = (!CAUSAL ? sk : BR ? max(0, min(sk, q0 + 1 + shift)) : min(sk, q0 + 1)) / BN;
        const int climit = row + shift;    // last visible key of this lane's row (causal)

        RowState st;
#pragma unroll
        for (int db = 0; db < 4; ++db) st.o[db] = f32x16{};
        st.m = -__builtin_inff();
        st.lb = 0.f;
        st.l = 0.f;

        if (ntiles > 0) {
            auto issue = [&](int t) {
                const int64_t first = int64_t(t) * BN;
                const uint32_t bytes = uint32_t(sk - int(first) - 1) * kv_row_bytes + ROW_BYTES;
                const u32x4 rk = make_desc(kbase + first * kv_row_bytes, bytes);
                const u32x4 rv = make_desc(vbase + first * kv_row_bytes, bytes);
                dma_tile<DMA, TILE_BYTES>(rk, rv, smem_base + (t & 1) * STAGE_BYTES, wave, dofs);
            };
            issue(0);
            bf16x8 qr[8];
            {
                const uint32_t qoff = uint32_t(wave * 32 + col) * row_bytes + half * 16;
#pragma unroll
                for (int c = 0; c < 8; ++c) qr[c] = load16(rq, qoff + c * 32);
#pragma unroll
                for (int c = 0; c < 8; ++c) asm volatile("" ::"v"(qr[c]));
            }
            auto step = [&](auto stage_c, auto masked_c, int t) {
                constexpr int STAGE = decltype(stage_c)::value;
                const unsigned char* cur = smem + STAGE * STAGE_BYTES;
                wait_vmem();
                __syncthreads();
                if (t + 1 < ntiles) issue(t + 1);
                // A causal tile entirely above this wave's rows changes nothing.
                // BR rows that see no key yet keep a -inf base (EMPTY).
                if (!(decltype(masked_c)::value && CAUSAL) || t * BN <= qw + 31 + shift)
                    attend_fused<BN, decltype(masked_c)::value, CAUSAL, LSE, BR>(
                        cur, cur + TILE_BYTES, off, qr, st, t == 0, t * BN, sk, climit, half, scale2);
            };
            using S0 = std::integral_constant<int, 0>;
            using S1 = std::integral_constant<int, 1>;
            using Plain = std::integral_constant<bool, false>;
            using Masked = std::integral_constant<bool, true>;
            int t = 0;
            if (qw >= sq) {
                // Rows all past this sequence's end: only the DMA and barrier
                // sequence of the loop below.
                for (; t < ntiles; ++t) {
                    wait_vmem();
                    __syncthreads();
                    if (t + 1 < ntiles) issue(t + 1);
                }
            } else {
                for (; t + 1 < nfull; t += 2) {
                    step(S0{}, Plain{}, t);
                    step(S1{}, Plain{}, t + 1);
                }
                // Masked tiles in compile-time stage pairs too (t is even):
                // no runtime choice of step body, so O keeps one home.
                for (; t + 1 < ntiles; t += 2) {
                    step(S0{}, Masked{}, t);
                    step(S1{}, Masked{}, t + 1);
                }
                if (t < ntiles) step(S0{}, Masked{}, t);
            }
        }

        // O = acc / lb (0 for a sequence without keys), BF16.  Rows past the
        // sequence store nothing (their 32-bit offsets can wrap into a valid
        // row when heads * 256 bytes is large).
        const float inv = st.lb > 0.f ? 1.f / st.lb : 0.f;
        // Stage ntiles % 2 receives no DMA in this q tile and its last tile
        // (ntiles - 2) was read before the last step's barrier (with fewer
        // tiles it was never used, and the previous q tile's final wait and
        // barrier retired everything): this wave's slots there hold the O
        // staging.
        store_o_rows<TILE_BYTES, LSE>(st, inv, smem, uint32_t((ntiles & 1) * STAGE_BYTES + wave * DMA * 1024), ro,
                                      row_bytes, wave * 32, sq - qw, lane);
        if constexpr (LSE) {
            if (half == 0 && row < sq) a.lse[int64_t(head) * a.total_q + qs + row] = __builtin_fmaf(st.m, LN2, logf(st.l));
        }
        wait_vmem();
        __syncthreads();
    }
}

// Merge of the split-KV chunks.  PER groups of 32 lanes share one (b, h, row),
// so a workgroup of 256 lanes merges 8 / PER rows.  The row's PER * 32 lanes
// first read the chunks' log-sums side by side (maxima, then weights into LDS
// and the two sums); group p then accumulates the O of chunks p, p + PER, ...
// (4 dims per lane) with no branch between the loads, and the groups' partial
// sums are added in LDS.  Many chunks over few rows (decode) thus take a few
// memory round trips instead of one pair of dependent loads per chunk.
// VARLEN: rows are (sequence, head, query < max_seqlen_q); rows past their
// sequence's query count are skipped, O goes to the sequence's token rows and
// LSE to [heads, total_q]; a row whose chunks saw no key gets O = 0 and
// LSE = -inf.
constexpr int MAX_SPLITS = 256;

__device__ __forceinline__ float max32(float x) {
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m, 32));
    return x;
}

__device__ __forceinline__ float sum32(float x) {
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) x += __shfl_xor(x, m, 32);
    return x;
}

template <int PER, bool VARLEN = false>
__global__ __launch_bounds__(256) void combine_kernel(Fav4Args a, SplitArgs sp) {
    constexpr int RPB = 8 / PER, NT = PER * 32, MAXV = (MAX_SPLITS + NT - 1) / NT;
    // Chunks per lane group: PER = 1, 2, 4 serve up to 8, 16, 32 chunks; 8 up to MAX_SPLITS.
    constexpr int NS = PER == 8 ? (MAX_SPLITS + 7) / 8 : 8;
    __shared__ float wsh[RPB][MAX_SPLITS];   // chunk weights 2^(lse_b,s - max)
    __shared__ float2 red_m[8], red_s[8];    // per-group maxima, then sums
    __shared__ f32x4 part_acc[8][32];
    const int grp = threadIdx.x >> 5, q4 = threadIdx.x & 31;
    const int slot = grp / PER, part = grp - slot * PER;
    const int team = part * 32 + q4;
    const int64_t rows = int64_t(a.batch) * a.heads * a.sq;
    const int64_t slab = rows;                      // rows per chunk
    const int64_t blocks = (rows + RPB - 1) / RPB;

    // Workgroup-uniform loop: every wave reaches every barrier.
    for (int64_t blk = blockIdx.x; blk < blocks; blk += gridDim.x) {
        const int64_t r = blk * RPB + slot;
        const int64_t bh = r / a.sq;
        const int qi = int(r - bh * a.sq);
        const int batch = int(bh / a.heads), head = int(bh - int64_t(batch) * a.heads);
        int64_t qtok = int64_t(batch) * a.sq + qi;       // the row's token (BSHD)
        bool live = r < rows;
        if constexpr (VARLEN) {
            if (live) {
                // Only the query side: paged batches have no key offsets.
                const int qs = min(max(sp.cu_q[batch], 0), sp.total_q);
                const int qe = min(max(sp.cu_q[batch + 1], qs), min(sp.total_q, qs + a.sq));
                live = qi < qe - qs;
                qtok = int64_t(qs) + qi;
            }
        }
        // The partial O rows do not depend on the weights: their loads go out
        // first, so that their latency overlaps the log-sum phase (one memory
        // round per row block instead of three).  Lane group `part` holds
        // chunks part, part + PER, ... (at most NS of them).
        const float* op = sp.o_part + r * D + q4 * 4;
        f32x4 xo[NS];
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const int s = part + i * PER;
            xo[i] = live && s < sp.splits ? *reinterpret_cast<const f32x4*>(op + s * slab * D) : f32x4{};
        }
        float vb[MAXV], vl[MAXV];
        float mb = -__builtin_inff(), ml = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < MAXV; ++i) {
            const int s = team + i * NT;
            vb[i] = vl[i] = -__builtin_inff();
            if (live && s < sp.splits) {
                const float2 v = *reinterpret_cast<const float2*>(sp.lse_part + (s * slab + r) * 2);
                vb[i] = v.x;
                vl[i] = v.y;
            }
            mb = fmaxf(mb, vb[i]);
            ml = fmaxf(ml, vl[i]);
        }
        mb = max32(mb);
        ml = max32(ml);
        if (q4 == 0) red_m[grp] = float2{mb, ml};
        __syncthreads();
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            mb = fmaxf(mb, red_m[slot * PER + p].x);
            ml = fmaxf(ml, red_m[slot * PER + p].y);
        }
        if constexpr (VARLEN) {
            // No key in any chunk: weights 2^-inf = 0, so O = 0, LSE = -inf.
            if (mb == -__builtin_inff()) mb = ml = 0.f;
        }
        float den = 0.f, suml = 0.f;
#pragma unroll
        for (int i = 0; i < MAXV; ++i) {
            const int s = team + i * NT;
            if (s < sp.splits) {
                const float w = live ? exp2_native(vb[i] - mb) : 0.f;
                wsh[slot][s] = w;
                den += w;
                if (live) suml += exp2_native(vl[i] - ml);
            }
        }
        den = sum32(den);
        suml = sum32(suml);
        if (q4 == 0) red_s[grp] = float2{den, suml};
        __syncthreads();
        den = suml = 0.f;
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            den += red_s[slot * PER + p].x;
            suml += red_s[slot * PER + p].y;
        }

        // Chunks without a visible key carry weight 0 and O = 0; the test on
        // the weight keeps them out of the sum exactly.
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        if (live) {
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                const int s = part + i * PER;
                if (s < sp.splits) {
                    const float w = wsh[slot][s];
                    if (w > 0.f) acc += w * xo[i];
                }
            }
        }
        if constexpr (PER > 1) {
            part_acc[grp][q4] = acc;
            __syncthreads();
#pragma unroll
            for (int p = 1; p < PER; ++p) acc += part_acc[slot * PER + p][q4];
        }
        if (live && part == 0) {
            float rden = 1.f / den;
            if constexpr (VARLEN) rden = den > 0.f ? rden : 0.f;
            const f32x4 y = acc * rden;
            const int64_t orow = qtok * a.heads + head;
            const f32x2 y0 = {y[0], y[1]}, y1 = {y[2], y[3]};
            const bf16x2 b0 = __builtin_convertvector(y0, bf16x2), b1 = __builtin_convertvector(y1, bf16x2);
            *reinterpret_cast<bf16x4*>(static_cast<char*>(a.o) + orow * ROW_BYTES + q4 * 8) =
                bf16x4{b0[0], b0[1], b1[0], b1[1]};
            if (a.lse && q4 == 0) {
                const int64_t li = VARLEN ? int64_t(head) * sp.total_q + qtok : r;
                a.lse[li] = (ml + __builtin_amdgcn_logf(suml)) * LN2;
            }
        }
        __syncthreads();   // LDS of this row block is reused by the next
    }
}

}  // namespace fav4
