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
//    only the causal-diagonal and key-tail tiles run the masked body, where
//    32-key blocks entirely hidden from a wave are skipped and the rest get
//    the element mask.  Key tiles entirely above the diagonal are never loaded.
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

// Work item -> (bh, q tile).  Dense: the hardware deals workgroups round-robin
// over the 8 XCDs, so remap ids to give each XCD a contiguous run of items and
// keep one head's K/V hot in that XCD's L2.  Causal: heaviest q tiles first.
template <bool CAUSAL>
__device__ __forceinline__ void map_work(int id, int tiles, int bh_count, int& bh, int& tile) {
    if constexpr (CAUSAL) {
        tile = tiles - 1 - id / bh_count;
        bh = id - (id / bh_count) * bh_count;
    } else {
        const int total = tiles * bh_count;
        const int xcd = id & 7, slot = id >> 3;
        const int per = total >> 3, rem = total & 7;
        const int logical = xcd * per + min(xcd, rem) + slot;
        bh = logical / tiles;
        tile = logical - bh * tiles;
    }
}

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

// One key tile: S^T = K.Q^T, online softmax, O^T += V^T.P^T.
// MASKED selects the diagonal / tail variant.
template <int BN, bool MASKED, bool CAUSAL, bool LSE>
__device__ __forceinline__ void attend_tile(const unsigned char* ks, const unsigned char* vs,
                                            const LdsOffsets& off, const bf16x8 (&qr)[8], RowState& st,
                                            bool first, int start, int sk, int qw, int row, int half,
                                            float scale2) {
    constexpr int KB = BN / 32;
    const f32x16 zero = {};
    bool active[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
        active[kb] = !MASKED || (start + kb * 32 < sk && (!CAUSAL || start + kb * 32 <= qw + 31));

    // ---- S^T = K . Q^T (8 MFMAs per 32-key block, K operands prefetched) ----
    f32x16 s[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        s[kb] = zero;
        if (!MASKED || active[kb]) {
            bf16x8 kop[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) kop[c] = lds_read16(ks + kb * 32 * ROW_BYTES + off.k[c]);
            s[kb] = mfma32(kop[0], qr[0], zero);
#pragma unroll
            for (int c = 1; c < 8; ++c) s[kb] = mfma32(kop[c], qr[c], s[kb]);
        }
    }

    // ---- masks (key index of element v of lane (col, half) in block kb) ----
    if constexpr (MASKED) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            const int k0 = start + kb * 32;
            if (!active[kb]) {
#pragma unroll
                for (int v = 0; v < 16; ++v) s[kb][v] = -__builtin_inff();
            } else if (k0 + 32 > sk || (CAUSAL && k0 + 31 > qw)) {
                const int kl = k0 + half * 4;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int key = kl + (v >> 2) * 8 + (v & 3);
                    if (key >= sk || (CAUSAL && key > row)) s[kb][v] = -__builtin_inff();
                }
            }
        }
    }

    // ---- online softmax with the conditional rescale (log2 units) ----
    float mx = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kb][v]);
    mx = xhalf_max(mx);
    const float cand = fmaxf(st.m, mx * scale2);
    const bool update = first || cand > st.m + RESCALE_THRESHOLD;
    const float next = update ? cand : st.m;
    const float alpha = exp2_native(st.m - next);   // 0 on the first tile, 1 if no update
    if (!first && __builtin_amdgcn_ballot_w64(update)) {
#pragma unroll
        for (int db = 0; db < 4; ++db) st.o[db] *= alpha;
    }
    st.m = next;
    const float neg = -next;
    float part[4] = {0.f, 0.f, 0.f, 0.f};
    float pb0 = 0.f, pb1 = 0.f;
    bf16x8 p[KB][2];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            f32x2 e[4];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float x = exp2_native(fmaf(s[kb][sub * 8 + i], scale2, neg));
                e[i >> 1][i & 1] = x;
                if constexpr (LSE) part[i & 3] += x;
            }
            const bf16x2 b0 = __builtin_convertvector(e[0], bf16x2);
            const bf16x2 b1 = __builtin_convertvector(e[1], bf16x2);
            const bf16x2 b2 = __builtin_convertvector(e[2], bf16x2);
            const bf16x2 b3 = __builtin_convertvector(e[3], bf16x2);
            pb0 = bf16_pair_sum(b0, pb0);
            pb1 = bf16_pair_sum(b1, pb1);
            pb0 = bf16_pair_sum(b2, pb0);
            pb1 = bf16_pair_sum(b3, pb1);
            p[kb][sub] = bf16x8{b0[0], b0[1], b1[0], b1[1], b2[0], b2[1], b3[0], b3[1]};
        }
    }
    st.lb = st.lb * alpha + xhalf_sum(pb0 + pb1);
    if constexpr (LSE) st.l = st.l * alpha + xhalf_sum((part[0] + part[1]) + (part[2] + part[3]));

    // ---- O^T += V^T . P^T  (S element v of lane half h is MFMA k = h*8 + v%8) ----
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        if (MASKED && !active[kb]) continue;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            const unsigned char* vb = vs + (kb * 32 + sub * 16) * ROW_BYTES;
            bf16x8 vop[4];
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const bf16x4 lo = lds_read_tr(vb + off.v[0][db]);
                const bf16x4 hi = lds_read_tr(vb + off.v[1][db]);
                vop[db] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int db = 0; db < 4; ++db) st.o[db] = mfma32(vop[db], p[kb][sub], st.o[db]);
        }
    }
}

template <int WAVES, int BN, bool CAUSAL, bool LSE>
__global__ __launch_bounds__(WAVES * 64)
void fwd_kernel(Fav4Args a, int tiles, int total) {
    constexpr int BM = WAVES * 32;
    constexpr int TILE_BYTES = BN * ROW_BYTES;
    constexpr int DMA = BN / 4 / WAVES;                  // 1 KiB DMA ops per wave per matrix
    static_assert(BN % 32 == 0 && BN % (4 * WAVES) == 0, "tile shape");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[4 * TILE_BYTES];  // K0 V0 K1 V1

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 31, half = lane >> 5;
    const uint32_t row_bytes = uint32_t(a.heads) * ROW_BYTES;   // stride between sequence positions
    const float scale2 = a.scale * LOG2E;
    const uint32_t smem_base = lds_addr(smem);

    LdsOffsets off;
#pragma unroll
    for (int c = 0; c < 8; ++c) off.k[c] = col * ROW_BYTES + ((((2 * c) | half) ^ k_swz(col)) << 4);
    {
        const int r0 = half * 4 + ((lane & 15) >> 2);             // row inside a 16-key sub-block
        const int gl = ((lane >> 4) & 1) * 2 + ((lane & 3) >> 1);  // granule inside a 32-dim block
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int r = r0 + 8 * j;
#pragma unroll
            for (int db = 0; db < 4; ++db)
                off.v[j][db] = r * ROW_BYTES + (((db * 4 + gl) ^ v_swz(r)) << 4) + ((lane & 1) << 3);
        }
    }
    // Per-lane DMA source offsets inside a tile: each op covers 4 rows x 16 granules.
    uint32_t dk[DMA], dv[DMA];
#pragma unroll
    for (int i = 0; i < DMA; ++i) {
        const int r = (wave * DMA + i) * 4 + (lane >> 4), p = lane & 15;
        dk[i] = r * row_bytes + ((p ^ k_swz(r)) << 4);
        dv[i] = r * row_bytes + ((p ^ v_swz(r)) << 4);
    }

    for (int id = blockIdx.x; id < total; id += gridDim.x) {
        int bh, tile;
        map_work<CAUSAL>(id, tiles, a.batch * a.heads, bh, tile);
        bh = __builtin_amdgcn_readfirstlane(bh);
        tile = __builtin_amdgcn_readfirstlane(tile);
        const int batch = bh / a.heads, head = bh - batch * a.heads;
        const int q0 = tile * BM, qw = q0 + wave * 32;
        const int row = qw + col;                                 // this lane's query row
        const int64_t qrow0 = (int64_t(batch) * a.sq + q0) * a.heads + head;
        const int64_t krow0 = int64_t(batch) * a.sk * a.heads + head;
        const char* kbase = static_cast<const char*>(a.k) + krow0 * ROW_BYTES;
        const char* vbase = static_cast<const char*>(a.v) + krow0 * ROW_BYTES;
        const rsrc_t rq = make_rsrc(static_cast<const char*>(a.q) + qrow0 * ROW_BYTES,
                                    uint32_t(a.sq - q0 - 1) * row_bytes + ROW_BYTES);
        const rsrc_t ro = make_rsrc(static_cast<char*>(a.o) + qrow0 * ROW_BYTES,
                                    uint32_t(a.sq - q0 - 1) * row_bytes + ROW_BYTES);
        // Key tiles: [0, nfull) are unmasked for every row of the workgroup,
        // [nfull, ntiles) cross the key tail or the causal diagonal.
        const int kend = CAUSAL ? min(a.sk, q0 + BM) : a.sk;
        const int ntiles = (kend + BN - 1) / BN;
        const int nfull = (CAUSAL ? min(a.sk, q0 + 1) : a.sk) / BN;

        auto issue = [&](int t, int stage) {
            const int64_t first = int64_t(t) * BN;
            const uint32_t bytes = uint32_t(a.sk - int(first) - 1) * row_bytes + ROW_BYTES;
            const u32x4 rk = make_desc(kbase + first * row_bytes, bytes);
            const u32x4 rv = make_desc(vbase + first * row_bytes, bytes);
            const uint32_t ks = smem_base + stage * 2 * TILE_BYTES + wave * DMA * 1024;
#pragma unroll
            for (int i = 0; i < DMA; ++i) {
                dma16(rk, ks + i * 1024, dk[i]);
                dma16(rv, ks + TILE_BYTES + i * 1024, dv[i]);
            }
        };

        issue(0, 0);
        bf16x8 qr[8];
        {
            const uint32_t qoff = uint32_t(wave * 32 + col) * row_bytes + half * 16;
#pragma unroll
            for (int c = 0; c < 8; ++c) qr[c] = load16(rq, qoff + c * 32);
            // Retire the Q loads here, so that inside the key loop the only
            // outstanding vector-memory ops are the K/V DMA of the next tile.
#pragma unroll
            for (int c = 0; c < 8; ++c) asm volatile("" ::"v"(qr[c]));
        }
        RowState st;
#pragma unroll
        for (int db = 0; db < 4; ++db) st.o[db] = f32x16{};
        st.m = -__builtin_inff();
        st.lb = 0.f;
        st.l = 0.f;

        // One pipeline step on a compile-time stage: wait for tile t, prefetch
        // tile t+1 into the other stage, then attend to tile t.
        auto step = [&](auto stage_c, auto masked_c, int t) {
            constexpr int STAGE = decltype(stage_c)::value;
            constexpr bool MASKED = decltype(masked_c)::value;
            wait_vmem();        // this wave's DMA of tile t has landed
            __syncthreads();    // ... and every other wave's; the other stage is free
            if (t + 1 < ntiles) issue(t + 1, STAGE ^ 1);
            attend_tile<BN, MASKED, CAUSAL, LSE>(smem + STAGE * 2 * TILE_BYTES,
                                                 smem + STAGE * 2 * TILE_BYTES + TILE_BYTES, off, qr, st,
                                                 t == 0, t * BN, a.sk, qw, row, half, scale2);
        };
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        using Plain = std::integral_constant<bool, false>;
        using Masked = std::integral_constant<bool, true>;
        int t = 0;
        for (; t + 1 < nfull; t += 2) {
            step(S0{}, Plain{}, t);
            step(S1{}, Plain{}, t + 1);
        }
        if (t < nfull) {
            step(S0{}, Plain{}, t);
            ++t;
        }
        for (; t < ntiles; ++t) {
            if (t & 1) step(S1{}, Masked{}, t);
            else step(S0{}, Masked{}, t);
        }

        // Epilogue: O = acc / lb in BF16; rows >= sq fall outside the store bound.
        // Dividing by the sum of the rounded weights keeps them normalised, so
        // the BF16 rounding of P perturbs O by sum_j w_j e_j (V_j - O) instead
        // of sum_j w_j e_j V_j (exact when one key dominates).
        const float inv = 1.f / st.lb;
        const uint32_t obase = uint32_t(wave * 32 + col) * row_bytes + half * 8;
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
        if constexpr (LSE) {
            if (half == 0 && row < a.sq) a.lse[int64_t(bh) * a.sq + row] = st.m * LN2 + logf(st.l);
        }
        __syncthreads();   // LDS stages are reused by the next work item
    }
}

}  // namespace fav4
