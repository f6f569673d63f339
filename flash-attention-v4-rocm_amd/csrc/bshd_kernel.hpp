// BF16 BSHD D=128 attention forward for gfx950 (MI355X), wave64 MFMA.
//
// Semantics follow the reference kernel src/bshd_kernel.hpp:50-211 (online
// softmax in log2 units with the FA4 conditional rescale, P rounded to BF16
// before the PV product, FP32 row sums, O = acc / l, LSE = m*ln2 + ln(l)),
// but the machine mapping is gfx950's own:
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
//  * Causal: key tiles entirely above the diagonal are never loaded; inside a
//    boundary tile, 32-key blocks entirely masked for a wave are skipped and
//    only boundary blocks apply the element mask.
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

template <int WAVES, int BN, bool CAUSAL, bool LSE>
__global__ __launch_bounds__(WAVES * 64)
void fwd_kernel(Fav4Args a, int tiles, int total) {
    constexpr int BM = WAVES * 32;
    constexpr int TILE_BYTES = BN * ROW_BYTES;
    constexpr int KB = BN / 32;                          // 32-key blocks per tile
    constexpr int DMA = BN / 4 / WAVES;                  // 1 KiB DMA ops per wave per matrix
    static_assert(BN % 32 == 0 && BN % (4 * WAVES) == 0, "tile shape");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[4 * TILE_BYTES];  // K0 V0 K1 V1

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 31, half = lane >> 5;
    const uint32_t row_bytes = uint32_t(a.heads) * ROW_BYTES;   // stride between sequence positions
    const float scale2 = a.scale * LOG2E;
    const uint32_t smem_base = lds_addr(smem);

    // Per-lane LDS read offsets (tile-relative; block offsets are immediates).
    uint32_t k_off[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) k_off[c] = col * ROW_BYTES + ((((2 * c) | half) ^ k_swz(col)) << 4);
    uint32_t v_off[2][4];
    {
        const int r0 = half * 4 + ((lane & 15) >> 2);             // row inside a 16-key sub-block
        const int gl = ((lane >> 4) & 1) * 2 + ((lane & 3) >> 1);  // granule inside a 32-d block
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int r = r0 + 8 * j;
#pragma unroll
            for (int db = 0; db < 4; ++db)
                v_off[j][db] = r * ROW_BYTES + (((db * 4 + gl) ^ v_swz(r)) << 4) + ((lane & 1) << 3);
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
        const int kend = CAUSAL ? min(a.sk, q0 + BM) : a.sk;
        const int ntiles = (kend + BN - 1) / BN;

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
        f32x16 o[4];
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db] = f32x16{};
        // m: running base in log2 units; lb: sum of the BF16-rounded P that
        // actually enter the PV product (normalises O); l: FP32 sum of P
        // (feeds the LSE, kept only when LSE is requested).
        float m = -__builtin_inff(), lb = 0.f, l = 0.f;

        for (int t = 0; t < ntiles; ++t) {
            const int stage = t & 1;
            wait_vmem();        // this wave's DMA of tile t has landed
            __syncthreads();    // ... and every other wave's; stage^1 is free
            if (t + 1 < ntiles) issue(t + 1, stage ^ 1);
            const unsigned char* ks = smem + stage * 2 * TILE_BYTES;
            const unsigned char* vs = ks + TILE_BYTES;
            const int start = t * BN;

            // Block activity (wave-uniform) and whether element masks are needed.
            bool active[KB], edge[KB];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                const int k0 = start + kb * 32;
                active[kb] = k0 < a.sk && (!CAUSAL || k0 <= qw + 31);
                edge[kb] = k0 + 32 > a.sk || (CAUSAL && k0 + 31 > qw);
            }

            // S^T = K . Q^T
            f32x16 s[KB];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                s[kb] = f32x16{};
                if (active[kb]) {
#pragma unroll
                    for (int c = 0; c < 8; ++c)
                        s[kb] = mfma32(lds_read16(ks + kb * 32 * ROW_BYTES + k_off[c]), qr[c], s[kb]);
                }
            }
            // Masks: key index of element v of lane (col, half) in block kb.
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                if (!active[kb]) {
#pragma unroll
                    for (int v = 0; v < 16; ++v) s[kb][v] = -__builtin_inff();
                } else if (edge[kb]) {
                    const int k0 = start + kb * 32 + half * 4;
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int key = k0 + (v >> 2) * 8 + (v & 3);
                        if (key >= a.sk || (CAUSAL && key > row)) s[kb][v] = -__builtin_inff();
                    }
                }
            }
            // Online softmax with the conditional rescale (log2 units).
            float mx = -__builtin_inff();
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kb][v]);
            mx = xhalf_max(mx);
            const float cand = fmaxf(m, mx * scale2);
            const bool update = t == 0 || cand > m + RESCALE_THRESHOLD;
            const float next = update ? cand : m;
            const float alpha = exp2_native(m - next);
            if (t > 0 && __builtin_amdgcn_ballot_w64(update)) {
#pragma unroll
                for (int db = 0; db < 4; ++db) o[db] *= alpha;
            }
            m = next;
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
            lb = lb * alpha + xhalf_sum(pb0 + pb1);
            if constexpr (LSE) l = l * alpha + xhalf_sum((part[0] + part[1]) + (part[2] + part[3]));

            // O^T += V^T . P^T  (keys of S element v map to MFMA k = half*8 + v%8)
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                if (!active[kb]) continue;
#pragma unroll
                for (int sub = 0; sub < 2; ++sub) {
                    const unsigned char* vb = vs + (kb * 32 + sub * 16) * ROW_BYTES;
#pragma unroll
                    for (int db = 0; db < 4; ++db) {
                        const bf16x4 lo = lds_read_tr(vb + v_off[0][db]);
                        const bf16x4 hi = lds_read_tr(vb + v_off[1][db]);
                        const bf16x8 vop = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                        o[db] = mfma32(vop, p[kb][sub], o[db]);
                    }
                }
            }
        }

        // Epilogue: O = acc / lb in BF16; rows >= sq fall outside the store bound.
        // Dividing by the sum of the rounded weights keeps them normalised, so
        // the BF16 rounding of P perturbs O by sum_j w_j e_j (V_j - O) instead
        // of sum_j w_j e_j V_j (exact when one key dominates).
        const float inv = 1.f / lb;
        const uint32_t obase = uint32_t(wave * 32 + col) * row_bytes + half * 8;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
#pragma unroll
            for (int vg = 0; vg < 4; ++vg) {
                const f32x2 x0 = {o[db][vg * 4 + 0] * inv, o[db][vg * 4 + 1] * inv};
                const f32x2 x1 = {o[db][vg * 4 + 2] * inv, o[db][vg * 4 + 3] * inv};
                const bf16x2 y0 = __builtin_convertvector(x0, bf16x2);
                const bf16x2 y1 = __builtin_convertvector(x1, bf16x2);
                store8(ro, obase + (db * 32 + vg * 8) * 2, bf16x4{y0[0], y0[1], y1[0], y1[1]});
            }
        }
        if constexpr (LSE) {
            if (half == 0 && row < a.sq) a.lse[int64_t(bh) * a.sq + row] = m * LN2 + logf(l);
        }
        __syncthreads();   // LDS stages are reused by the next work item
    }
}

}  // namespace fav4
