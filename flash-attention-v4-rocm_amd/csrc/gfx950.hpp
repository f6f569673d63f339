// gfx950 (CDNA4, wave64) building blocks for the attention forward kernel.
//
// Role in the reference: include/gfx1250.h (TDM tile DMA, TDM wait, LDS
// transpose reads) and the WMMA / lane-swap helpers of
// src/bshd_kernel.hpp:7-17,32-47.  Everything here is written for gfx950:
//  * MFMA v_mfma_f32_32x32x16_bf16 (wave64, 32x32 fp32 tile per wave),
//  * buffer_load_dwordx4 ... lds (direct-to-LDS DMA, 1 KiB per wave
//    instruction, bounds-checked by the buffer descriptor so rows past the end
//    of a tensor read as zero),
//  * ds_read_b64_tr_b16 (transposing LDS read for the V operand),
//  * v_permlane32_swap (exchange between the two 32-lane halves of a wave).
//
// Lane layouts (measured on MI355X with an in-bounds probe):
//  * MFMA 32x32x16: A[m][k] is held by lane m + 32*(k/8), element k%8;
//    B[k][n] by lane n + 32*(k/8), element k%8; C[m][n] by lane
//    n + 32*((m/4)%2), element (m/8)*4 + m%4.
//  * ds_read_b64_tr_b16: within each 16-lane group, output lane i element j is
//    element i%4 of the 8 bytes addressed by source lane 4*j + i/4.  So if
//    source lane 4*r + c addresses row (key0 + r), columns 4c..4c+3 of a
//    row-major 16-bit matrix, output lane i receives column i, rows key0..+3.
//  * permlane32_swap(x, x): lanes l < 32 get (x[l], x[l+32]), lanes l >= 32 get
//    (x[l-32], x[l]); both halves therefore see the pair in the same order.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace fav4 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;
#define FAV4_LDS __attribute__((address_space(3)))

// Raw buffer descriptor: `bytes` is the bounds limit (num_records); loads at or
// past it return 0 and stores there are dropped.  Word 3 = 0x00020000 is the
// gfx9-family raw-buffer format (32-bit data format, no swizzle, no stride).
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Raw buffer descriptor held as four SGPRs, for inline-asm buffer ops.
__device__ __forceinline__ u32x4 make_desc(const void* base, uint32_t bytes) {
    const uint64_t addr = reinterpret_cast<uint64_t>(base);
    return u32x4{uint32_t(addr), uint32_t(addr >> 32) & 0xffffu, bytes, 0x00020000u};
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return uint32_t(reinterpret_cast<uintptr_t>((FAV4_LDS const void*)p));
}

// 16-byte direct-to-LDS load: lane i's bytes [voffset, voffset+16) of the
// buffer land at LDS address lds + 16*i; `lds` must be wave-uniform (M0).
// Written as inline asm on purpose: the compiler then does not treat every
// later LDS read as a possible alias of the in-flight DMA (it would otherwise
// wait for the next tile's loads before reading the current tile).  Callers
// retire these loads themselves with s_waitcnt vmcnt before a barrier.  M0 is
// a reserved register for the compiler, so its value is saved and restored.
// NT sets the load's nontemporal cache policy: for data read once (a decode's
// K/V stream), measured to lift MI355X's read rate over many concurrent
// 256-byte row streams from about 6.2 to 7.0 TB/s.
template <bool NT = false>
__device__ __forceinline__ void dma16(u32x4 desc, uint32_t lds, uint32_t voffset) {
    uint32_t saved;
    if constexpr (NT)
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %1\n\t"
            "s_nop 0\n\t"
            "buffer_load_dwordx4 %2, %3, 0 offen nt lds\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved) : "s"(lds), "v"(voffset), "s"(desc) : "memory");
    else
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %1\n\t"
            "s_nop 0\n\t"
            "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved) : "s"(lds), "v"(voffset), "s"(desc) : "memory");
}

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Wait until at most N vector-memory ops of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmem_keep() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ bf16x8 load16(rsrc_t r, uint32_t voffset) {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, 0, 0));
}

__device__ __forceinline__ void store8(rsrc_t r, uint32_t voffset, bf16x4 v) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, voffset, 0, 0);
}

__device__ __forceinline__ void store16(rsrc_t r, uint32_t voffset, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, voffset, 0, 0);
}

__device__ __forceinline__ bf16x8 lds_read16(const void* lds) {
    return *reinterpret_cast<const FAV4_LDS bf16x8*>((FAV4_LDS const void*)lds);
}

__device__ __forceinline__ bf16x4 lds_read_tr(const void* lds) {
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (FAV4_LDS i16x4*)(FAV4_LDS void*)lds));
}

// Value of x in lane l combined with x in lane l^32, identical in both halves.
__device__ __forceinline__ float xhalf_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float exp2_native(float x) { return __builtin_amdgcn_exp2f(x); }

// acc + x.lo + x.hi in FP32 (v_dot2c_f32_bf16 against the pair (1, 1)).
__device__ __forceinline__ float bf16_pair_sum(bf16x2 x, float acc) {
    const bf16x2 one = {__bf16(1.f), __bf16(1.f)};
    return __builtin_amdgcn_fdot2_f32_bf16(x, one, acc, false);
}

}  // namespace fav4
