// MFMA-only ceiling probe: a measurement library, libfav4_mfma_ceiling.so.
// Nothing here is exported by libfav4_bshd.so.
//
// One workgroup of 8 waves per CU, two waves per SIMD, the same occupancy
// as the forward's 256-row config. Every wave streams BF16 MFMAs on
// register-resident pseudo-random operands. The data are random because
// MFMA power depends on the data, and constant operands let the clock run
// higher.
// - Shape 0: v_mfma_f32_32x32x16_bf16 rotating over four accumulators.
// - Shape 1: v_mfma_f32_16x16x32_bf16 rotating over eight. Each loop
//   iteration does the same FLOPs as shape 0.
// Under the board's power limit this is the rate the MFMAs alone sustain
// at the clock that limit allows. That rate is the ceiling the forward's
// roofline fraction is read against.
#include "gfx950.hpp"

namespace {

using namespace fav4;

// Eight BF16 values in [-2, 2) from a linear congruential sequence.
__device__ __forceinline__ bf16x8 pseudo_random8(uint32_t s) {
    bf16x8 x;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        s = s * 1664525u + 1013904223u;
        x[e] = __bf16(float(int(s >> 16) - 32768) * (1.f / 16384.f));
    }
    return x;
}

template <int SHAPE>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mfma_stream(float* out, int iters) {
    const int lane = threadIdx.x & 63;
    bf16x8 a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = pseudo_random8(lane * 977u + i * 131u + blockIdx.x);
        b[i] = pseudo_random8(lane * 733u + i * 71u + threadIdx.x / 64);
    }
    float r = 0.f;
    if constexpr (SHAPE == 0) {
        f32x16 c[4] = {};
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) c[j] = mfma32(a[(i + j) & 7], b[(i + 2 * j) & 7], c[j]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) r += c[j][v];
    } else {
        f32x4 c[8] = {};
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    c[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[(i + j) & 7], b[(i + 2 * j) & 7], c[j], 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) r += c[j][v];
    }
    out[int64_t(blockIdx.x) * 512 + threadIdx.x] = r;
}

}  // namespace

// Launch `grid` workgroups of 512 threads. Each wave does iters x 32 MFMAs of
// 32x32x16 (shape 0) or iters x 64 of 16x16x32 (shape 1): 1048576 * iters
// FLOPs per wave either way. `out` holds grid * 512 floats, one per thread
// (it keeps the MFMA chains live). Returns hipErrorInvalidValue for
// arguments outside these ranges, else the launch status.
extern "C" __attribute__((visibility("default"))) int fav4_probe_mfma_ceiling(int shape, int grid, int iters,
                                                                              float* out, hipStream_t stream) {
    if (!out || (shape != 0 && shape != 1) || grid <= 0 || grid > 65536 || iters <= 0 || iters > (1 << 20) ||
        (reinterpret_cast<uintptr_t>(out) & 3))
        return hipErrorInvalidValue;
    if (shape == 0) hipLaunchKernelGGL(mfma_stream<0>, dim3(grid), dim3(512), 0, stream, out, iters);
    else hipLaunchKernelGGL(mfma_stream<1>, dim3(grid), dim3(512), 0, stream, out, iters);
    return hipGetLastError();
}
