// Shared device helpers for the MI355X (gfx950) MoE-layer kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace glmmoe {

constexpr int kWave = 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// Native vector types for inline-asm register operands ("+v" needs them).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---- bf16 -----------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Round-to-nearest-even f32 -> bf16 (NaN kept quiet), the same rule as the
// reference's host conversion include/common.hpp:126-136.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    uint32_t b = __float_as_uint(f);
    if ((b & 0x7f800000u) == 0x7f800000u && (b & 0x007fffffu)) return (b >> 16) | 0x40u;
    b += 0x7fffu + ((b >> 16) & 1u);
    return b >> 16;
}

// Two f32 -> packed bf16 (a in the low half), round-to-nearest-even, one
// v_cvt_pk_bf16_f32.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

// ---- exp / sigmoid ---------------------------------------------------------
// One exp definition shared, operation for operation, with the CPU oracle:
// Cody-Waite reduction x = n*ln2 + r with ln2 split hi/lo, degree-7 Taylor
// polynomial of e^r in Horner form, scale by 2^n built from exponent bits.
// The argument is clamped to [-80, 80] so 2^n is a normal float. Every step
// is an IEEE-rounded mul/fma/rint, so sigmoid scores are bit-identical to the
// oracle's and routing decisions match it exactly.
__device__ __forceinline__ float exp_fixed(float x) {
    if (x != x) return x;
    x = x > 80.0f ? 80.0f : x;
    x = x < -80.0f ? -80.0f : x;
    const float n = __builtin_rintf(x * 1.44269504088896341f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, x);
    r = __builtin_fmaf(-n, 1.42860682030941723e-06f, r);
    float p = 1.0f / 5040.0f;
    p = __builtin_fmaf(p, r, 1.0f / 720.0f);
    p = __builtin_fmaf(p, r, 1.0f / 120.0f);
    p = __builtin_fmaf(p, r, 1.0f / 24.0f);
    p = __builtin_fmaf(p, r, 1.0f / 6.0f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float scale = __uint_as_float((uint32_t)((int)n + 127) << 23);
    return p * scale;
}

// sigmoid = 1 / (1 + exp(-x)): src/model_glm52.cpp:96, cuda/common.cuh:54.
__device__ __forceinline__ float sigmoid_fixed(float x) { return 1.0f / (1.0f + exp_fixed(-x)); }

// SiLU for the expert activations (tolerance-checked, not bit-checked): the
// hardware exp2 and reciprocal are accurate to ~1 ulp and much cheaper than
// exp_fixed and an IEEE division.
__device__ __forceinline__ float silu_fast(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.44269504088896341f));
}

// ---- int4 -> bf16 -----------------------------------------------------------
// A packed dword holds 8 int4 codes c (the stored nibble, value c - 8) for 8
// consecutive K positions e = 0..7: e = 2s in nibble s, e = 2s+1 in nibble
// s+4. OR-ing 0x4300 into a 16-bit lane holding c gives the bf16 of 128 + c
// exactly, so each pair costs one shift and one and-or. The -136 offset
// (128 + 8) is removed after the MFMA with the activation group sum:
//   sum_k (c_k - 8) x_k = sum_k (128 + c_k) x_k - 136 * sum_k x_k.
// The mask 0x000F000F and the bf16 exponent pattern 0x43004300 as opaque
// registers: with literal constants the compiler emits a separate v_and and
// v_or (a VOP3 v_and_or_b32 cannot take two literals); with register operands
// it selects one v_and_or_b32 per pair. Call once at kernel entry, before any
// MFMA: the moves are inline asm, which the hazard recognizer does not see.
struct DqConst {
    uint32_t mask, bias;
};
__device__ __forceinline__ DqConst dq_const() {
    DqConst c;
    asm volatile("v_mov_b32 %0, 0x000f000f\n v_mov_b32 %1, 0x43004300" : "=v"(c.mask), "=v"(c.bias));
    return c;
}

__device__ __forceinline__ bf16x8 dq_w4(uint32_t w, const DqConst& c) {
    u32x4 v;
    v.x = (w & c.mask) | c.bias;
    v.y = ((w >> 4) & c.mask) | c.bias;
    v.z = ((w >> 8) & c.mask) | c.bias;
    v.w = ((w >> 12) & c.mask) | c.bias;
    return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef float f32x16 __attribute__((ext_vector_type(16)));
// 32x32x16 bf16: A lane l = row l % 32, K 8 (l / 32) + [0, 8); B lane l = column
// l % 32, same K; D lane l = column l % 32, value i = row 8 (i / 4) + 4 (l / 32) + i % 4.
__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// ---- LDS-DMA streaming helpers --------------------------------------------
typedef __attribute__((address_space(3))) char lds_char;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const lds_char*)p;
}

// 64 lanes x 16 B from per-lane global addresses to lds_base + 16 * lane.
__device__ __forceinline__ void dma16(const void* g, void* lds_base) {
    __builtin_amdgcn_global_load_lds(g, (lds_char*)lds_base, 16, 0, 0);
}
// 64 lanes x 4 B to lds_base + 4 * lane.
__device__ __forceinline__ void dma4(const void* g, void* lds_base) {
    __builtin_amdgcn_global_load_lds(g, (lds_char*)lds_base, 4, 0, 0);
}

// s_waitcnt vmcnt(N) with expcnt / lgkmcnt left unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

constexpr int kTable = 32;     // item-table steps per refill
constexpr int kTabInts = 20;   // ints per step

__device__ __forceinline__ uint4 lds_bcast16(uint32_t addr) {
    uint4 v;
    asm volatile("ds_read_b128 %0, %1\n s_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr));
    return v;
}
__device__ __forceinline__ uint32_t lds_read_u32(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1\n s_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr));
    return v;
}
__device__ __forceinline__ void lds_write_f32(uint32_t addr, float v) {
    asm volatile("ds_write_b32 %0, %1\n s_waitcnt lgkmcnt(0)" : : "v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ int sgpr(uint32_t v) { return __builtin_amdgcn_readfirstlane((int)v); }


// ---- device-coherent plain loads/stores --------------------------------------
// Data handed between workgroups of one launch (a ticket decides who reads
// it) goes through device-scope relaxed atomics: on gfx950 these are plain
// loads/stores with device-scope cache bits, coherent across the XCDs' L2s
// without the L2 write-back/invalidate a device-scope fence costs. A writer
// waits for its stores to complete (vmcnt 0) before it takes its ticket.
template <class T>
__device__ __forceinline__ void st_dev(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ T ld_dev(const T* p) {
    return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned int ticket_dev(unsigned int* p) {
    return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void reset_dev(unsigned int* p) {
    __hip_atomic_store(p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until every memory operation this wave issued has completed.
__device__ __forceinline__ void drain_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// f(std::integral_constant<int, i>) for i = 0 .. N - 1, in order: loop bodies
// whose register-array indices and wait counts must be compile-time constants.
template <class F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// LDS u16 read (waits for every pending LDS operation of the wave).
__device__ __forceinline__ uint32_t lds_read_u16(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_u16 %0, %1\n s_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr));
    return v;
}

}  // namespace glmmoe
