// Shared device-side pieces of the fused causal attention kernels (gfx950).
//
// Fragment layouts of v_mfma_f32_32x32x2_f32 used throughout (wave64):
//   A (32 x 2):  lane l holds A[l % 32][l / 32]
//   B (2 x 32):  lane l holds B[l / 32][l % 32]
//   D (32 x 32): lane l, register r holds D[8*(r/4) + 4*(l/32) + r%4][l % 32]
// The reduction index of one instruction is split across the two lane
// halves.  The kernels choose it so that half `hf` of step (g, c) covers
// row 8g + 4hf + c of a 32-row block: then the 16 accumulator registers of
// one product are, register for register, the A or B operand of the next
// product, and no accumulator ever has to be shuffled between lanes.
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>
#include <cstdint>

namespace gptc {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kDPad = 64;          // head size the kernels are built for (D <= 64 is zero-padded)
constexpr int kLdsStride = 68;     // floats per LDS row: 64 + 4 keeps b128 row reads conflict-free
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Element (b, t, h, d) of a per-head view lives at p + b*sb + t*st + h*sh + d.
// qkv (B, T, 3C):  sb = T*3C, st = 3C, sh = D (k at +C, v at +2C).
// y / dy (B, T, C): sb = T*C,  st = C,  sh = D.
// (B, H, T, D):     sb = H*T*D, st = D, sh = T*D.
struct HeadView {
    const float *p;
    uint32_t sb, st, sh;
};
struct HeadViewW {
    float *p;
    uint32_t sb, st, sh;
};

__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x4_f32 (wave64), the shape of the 16-row kernels:
//   A (16 x 4):  lane l holds A[l % 16][l / 16]
//   B (4 x 16):  lane l holds B[l / 16][l % 16]
//   D (16 x 16): lane l, register r holds D[4*(l/16) + r][l % 16]
// Register r of a product, across the wave, is again a B operand whose
// reduction rows are 4g + r (g = l / 16): accumulators feed the next product
// without a shuffle, as with the 32 x 32 shape.
__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.0f;
    return z;
}

__device__ __forceinline__ f32x4 zero4() {
    f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    return z;
}

// row[dim .. dim+3] with elements at or beyond D read as zero.
// VEC: D % 4 == 0 and rows 16-byte aligned, so a group is all-in or all-out.
template <bool VEC>
__device__ __forceinline__ f32x4 load4(const float *row, int dim, int D) {
    if (VEC) {
        if (dim < D) return *reinterpret_cast<const f32x4 *>(row + dim);
        return zero4();
    }
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (dim + e < D) ? row[dim + e] : 0.0f;
    return v;
}

// Raw buffer resources (dword 3 of a gfx9 buffer descriptor): loads through
// them are bounds-checked by the hardware against num_records and return
// zeros past it, so tile loads need neither branches nor row tests.
constexpr int kBufferConfig = 0x00020000;
typedef int i32x4 __attribute__((ext_vector_type(4)));

// A wave-uniform value the compiler cannot prove uniform (it would otherwise
// keep it in VGPRs, and a buffer resource in VGPRs costs a waterfall loop
// around every load).
// A compile-time int argument (tile variants chosen by a uniform switch).
template <int N>
using IntC = std::integral_constant<int, N>;

__device__ __forceinline__ uint32_t uniform(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }

// An int at a uniform address of memory that no kernel writes (the work
// lists), read through the scalar data cache.  The compiler reads such an
// entry inside a loop with a vector load, and its wait for that load also
// waits for every tile load in flight (a full memory round trip at each
// block change); this waits for the scalar load alone.
__device__ __forceinline__ int load_uniform_int(const int *p) {
    int v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
    return v;
}

template <typename T>
__device__ __forceinline__ T *uniform(T *p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint64_t lo = uniform(static_cast<uint32_t>(v)), hi = uniform(static_cast<uint32_t>(v >> 32));
    return reinterpret_cast<T *>((hi << 32) | lo);
}

// Rows [0, rows) of one head (row t at t * st floats, kDPad floats used):
// a row at or past `rows` reads as zeros.  The host guarantees that the byte
// size fits in 31 bits before it selects the kernels that use this.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t head_rows(const float *base, int rows, uint32_t st) {
    const int bytes = rows > 0 ? static_cast<int>(uniform(((rows - 1) * st + kDPad) * 4u)) : 0;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(uniform(base)), 0, bytes, kBufferConfig);
}

// The LDS pointer at a wave-uniform LDS byte address: the destination of a
// buffer load that writes LDS directly (__builtin_amdgcn_raw_ptr_buffer_load_lds;
// the compiler sets M0 from it and counts the load in its own waits).
__device__ __forceinline__ __attribute__((address_space(3))) void *lds_ptr(uint32_t byte_addr) {
    return reinterpret_cast<__attribute__((address_space(3))) void *>(static_cast<uintptr_t>(uniform(byte_addr)));
}

// Four floats at float offset `off` of a buffer resource.
__device__ __forceinline__ f32x4 buffer_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off * 4u, 0, 0));
}

// The packed P' and dS blocks are written once and read once, by the next
// kernel: they go through these non-temporal accesses, so that they do not
// evict from L2 and the memory-side cache the tiles that are read again
// (the K/V prefixes of the forward, the Q/dO tiles of dk/dv, the K tiles of
// dq) or the inputs of the next kernels.
template <typename V>
__device__ __forceinline__ V stream_load(const V *p) {
    return __builtin_nontemporal_load(p);
}
template <typename V>
__device__ __forceinline__ void stream_store(V *p, V v) {
    __builtin_nontemporal_store(v, p);
}

template <bool VEC>
__device__ __forceinline__ void store4(float *row, int dim, int D, f32x4 v) {
    if (VEC) {
        if (dim < D) *reinterpret_cast<f32x4 *>(row + dim) = v;
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (dim + e < D) row[dim + e] = v[e];
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// s_waitcnt immediate that waits for vmcnt == 0 only (gfx9 encoding:
// vmcnt [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]; the others at their maxima).
constexpr int kWaitVmcnt0 = 0x0F70;

// Value held by the lane 32 positions away (the other half of the wave).
__device__ __forceinline__ float other_half(float x) { return __shfl_xor(x, 32, 64); }

// Max and sum over the four lanes l % 16 + {0, 16, 32, 48} (one query of a
// 16 x 16 accumulator), every lane receiving the result.  gfx950's
// v_permlane32_swap / v_permlane16_swap exchange lane halves / 16-lane rows
// in the VALU: with both operands equal to x, the two results hold x at the
// lane and at its partner (l ^ 32, then l ^ 16), in some order.
__device__ __forceinline__ float max4_rows(float x) {
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float sum4_rows(float x) {
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = __uint_as_float(h[0]) + __uint_as_float(h[1]);
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace gptc
