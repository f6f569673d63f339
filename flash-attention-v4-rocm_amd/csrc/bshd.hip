// C-ABI host dispatch for the gfx950 attention forward.
//
// Mirrors the reference dispatch src/bshd.hip:1-38: the same argument checks
// in the same order (all before any HIP call), config 0 -> auto selection,
// config -> kernel instantiation, and hipGetLastError() after the launch.
#include "fav4_bshd.h"
#include "bshd_kernel.hpp"

#include <climits>
#include <cmath>
#include <cstdint>

namespace {

// Upper bound on launched workgroups; larger problems loop inside the kernel.
constexpr int64_t MAX_GRID = int64_t(1) << 22;

template <int WAVES, int BN, int STAGES, bool PIPE, bool CAUSAL>
int launch(const Fav4Args& a, hipStream_t stream) {
    constexpr int BM = WAVES * 32;
    const int tiles = (a.sq + BM - 1) / BM;
    const int64_t total = int64_t(fav4::items_per_head<CAUSAL>(tiles)) * a.batch * a.heads;
    if (total > INT_MAX) return hipErrorInvalidValue;
    const int grid = int(total < MAX_GRID ? total : MAX_GRID);
    if (a.lse)
        hipLaunchKernelGGL((fav4::fwd_kernel<WAVES, BN, CAUSAL, true, STAGES, PIPE>), dim3(grid),
                           dim3(WAVES * 64), 0, stream, a, tiles, int(total));
    else
        hipLaunchKernelGGL((fav4::fwd_kernel<WAVES, BN, CAUSAL, false, STAGES, PIPE>), dim3(grid),
                           dim3(WAVES * 64), 0, stream, a, tiles, int(total));
    return hipGetLastError();
}

template <bool CAUSAL>
int dispatch(const Fav4Args& a, int config, hipStream_t stream) {
    switch (config) {
    case 1: return launch<4, 64, 2, false, CAUSAL>(a, stream);
    case 2: return launch<8, 64, 2, false, CAUSAL>(a, stream);
    case 3: return launch<8, 64, 3, true, CAUSAL>(a, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

// Replaces src/bshd.hip:23-25.  Small query lengths use 128-row workgroups so
// short sequences still spread over the 256 CUs; everything else uses 256 rows.
extern "C" __attribute__((visibility("default"))) int fav4_bshd_select_config(const Fav4Args* a) {
    if (!a) return -1;
    return a->sq < 256 ? 1 : 2;
}

// Replaces src/bshd.hip:26-38.
extern "C" __attribute__((visibility("default"))) int fav4_bshd_forward(const Fav4Args* a, int causal, int config,
                                                                hipStream_t stream) {
    if (!a || !a->q || !a->k || !a->v || !a->o || a->batch <= 0 || a->heads <= 0 || a->sq <= 0 ||
        a->sk <= 0 || (causal != 0 && causal != 1) || config < 0 || config > 3 ||
        !std::isfinite(a->scale) || a->scale <= 0)
        return hipErrorInvalidValue;
    if (a->batch > INT_MAX / a->heads || a->heads > INT_MAX / 128 ||
        a->sq > INT_MAX / (a->heads * 128) || a->sk > INT_MAX / (a->heads * 128) ||
        ((reinterpret_cast<uintptr_t>(a->q) | reinterpret_cast<uintptr_t>(a->k) |
          reinterpret_cast<uintptr_t>(a->v) | reinterpret_cast<uintptr_t>(a->o)) & 15))
        return hipErrorInvalidValue;
    if (config == 0) config = fav4_bshd_select_config(a);
    return causal ? dispatch<true>(*a, config, stream) : dispatch<false>(*a, config, stream);
}
