// Known-answer probe of the K/V tile loader (a test library, libfav4_loader_kat.so;
// nothing here is exported by libfav4_bshd.so).
//
// Role in the reference: tests/bshd_tdm.hip:8-45, the exact integer test of
// its gfx1250 TDM tile loader (row stride over several head counts, the last
// head's offset, zero fill past the rows).  Here the loader is gfx950's: the
// probe kernel issues the DMA of one K and one V tile with the kernels' own
// helpers (dma_offsets, dma_tile, the bounded descriptor of a tile's first
// row), then reads the tile back twice: as the raw LDS image, and through the
// MFMA operand offsets (lds_offsets) exactly as the QK^T and PV steps read
// it.  The test compares both with integer patterns, bit for bit.
#include "bshd_kernel.hpp"

#include <climits>

namespace {

struct KatArgs {
    const unsigned char *k, *v;   // 16-bit patterns, [batch, sk, heads, 128]
    int batch, heads, sk;         // tensor shape (heads = K/V heads)
    int b, h, t;                  // the (batch, head) slice and key tile probed
    unsigned short *lds;          // [2][BN][128]: the K then V tile as it sits in LDS
    unsigned short *kop;          // [WAVES][BN/32][8][64][8]: K operand of d-chunk c, per lane
    unsigned short *vop;          // [WAVES][BN/16][4][64][8]: V^T operand of 32-dim block db, per lane
};

template <int WAVES, int BN>
__global__ __launch_bounds__(WAVES * 64) void loader_probe(KatArgs a) {
    using namespace fav4;
    constexpr int TILE_BYTES = BN * ROW_BYTES;
    constexpr int DMA = BN / 4 / WAVES;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * TILE_BYTES];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t row_bytes = uint32_t(a.heads) * ROW_BYTES;

    // The kernels' tile DMA: the slice's rows are row_bytes apart, the
    // descriptor starts at the tile's first row and ends at the slice's last.
    // The one-wave shape loads nontemporally, as the split-KV decode does.
    const DmaOffsets<DMA> dofs = dma_offsets<DMA>(wave, lane, row_bytes, row_bytes);
    const int64_t slice = (int64_t(a.b) * a.sk * a.heads + a.h) * ROW_BYTES;
    const int first = a.t * BN;
    const uint32_t bound = uint32_t(a.sk - first - 1) * row_bytes + ROW_BYTES;
    const u32x4 rk = make_desc(a.k + slice + int64_t(first) * row_bytes, bound);
    const u32x4 rv = make_desc(a.v + slice + int64_t(first) * row_bytes, bound);
    dma_tile<DMA, TILE_BYTES, WAVES == 1>(rk, rv, lds_addr(smem), wave, dofs);
    wait_vmem();
    __syncthreads();

    // Raw image, 16 bytes per lane and step.
    for (int i = threadIdx.x; i < 2 * TILE_BYTES / 16; i += WAVES * 64)
        *reinterpret_cast<bf16x8*>(a.lds + i * 8) = lds_read16(smem + i * 16);

    // Operands, as every wave of the kernels reads them.
    const LdsOffsets off = lds_offsets(lane);
#pragma unroll
    for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const bf16x8 x = lds_read16(smem + kb * 32 * ROW_BYTES + off.k[c]);
            *reinterpret_cast<bf16x8*>(a.kop + ((((wave * (BN / 32) + kb) * 8 + c) * 64 + lane) * 8)) = x;
        }
    const unsigned char* vs = smem + TILE_BYTES;
#pragma unroll
    for (int u = 0; u < BN / 16; ++u)
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const bf16x4 lo = lds_read_tr(vs + u * 16 * ROW_BYTES + off.v[0][db]);
            const bf16x4 hi = lds_read_tr(vs + u * 16 * ROW_BYTES + off.v[1][db]);
            const bf16x8 x = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            *reinterpret_cast<bf16x8*>(a.vop + ((((wave * (BN / 16) + u) * 4 + db) * 64 + lane) * 8)) = x;
        }
}

}  // namespace

// waves 8 or 4: 64-key tiles (the forward's configs 2 and 1); waves 1:
// 32-key tiles (the one-wave split-KV shape).  Returns hipErrorInvalidValue
// for arguments outside the probed tensor, else the launch status.
extern "C" __attribute__((visibility("default"))) int fav4_kat_loader(const void* k, const void* v, int batch,
                                                                      int heads, int sk, int b, int h, int t,
                                                                      int waves, void* lds, void* kop, void* vop,
                                                                      hipStream_t stream) {
    const int bn = waves == 1 ? 32 : 64;
    if (!k || !v || !lds || !kop || !vop || batch <= 0 || heads <= 0 || sk <= 0 || b < 0 || b >= batch || h < 0 ||
        h >= heads || t < 0 || int64_t(t) * bn >= sk || (waves != 1 && waves != 4 && waves != 8) ||
        int64_t(sk) * heads * fav4::ROW_BYTES > int64_t(UINT32_MAX) ||
        ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(lds) |
          reinterpret_cast<uintptr_t>(kop) | reinterpret_cast<uintptr_t>(vop)) & 15))
        return hipErrorInvalidValue;
    KatArgs a{static_cast<const unsigned char*>(k), static_cast<const unsigned char*>(v), batch, heads, sk, b, h, t,
              static_cast<unsigned short*>(lds), static_cast<unsigned short*>(kop), static_cast<unsigned short*>(vop)};
    if (waves == 8) hipLaunchKernelGGL((loader_probe<8, 64>), dim3(1), dim3(512), 0, stream, a);
    else if (waves == 4) hipLaunchKernelGGL((loader_probe<4, 64>), dim3(1), dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((loader_probe<1, 32>), dim3(1), dim3(64), 0, stream, a);
    return hipGetLastError();
}
