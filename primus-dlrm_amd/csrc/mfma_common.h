// Device helpers shared by the bf16 MFMA kernels (OneTrans block, fused
// sequence tokenizer): vector types, the 32x32x16 bf16 MFMA, instruction
// schedule pinning, bf16 rounding, the erf GELU and LDS weight fragments.
#pragma once

#include "pdm_common.h"

namespace pdm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x16_t mfma32x32x16(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                 c, 0, 0, 0);
}

// 16x16x32 bf16: lane l supplies row (A) / column (B) l % 16, k = 8 (l / 16) .. +8;
// accumulator element i of lane l is row 4 (l / 16) + i, column l % 16.
__device__ __forceinline__ f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                 c, 0, 0, 0);
}

// Pins the instruction order of a fully unrolled loop of N MFMAs, each fed by
// one LDS read: the first LEAD reads are issued up front, then one MFMA and
// the next read alternate, so every read has LEAD MFMAs of latency slack.
template <int N, int LEAD>
__device__ __forceinline__ void sched_mfma_ds_pipeline() {
  __builtin_amdgcn_sched_group_barrier(0x100, LEAD, 0);  // DS reads
#pragma unroll
  for (int i = 0; i < N - LEAD; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
  }
  __builtin_amdgcn_sched_group_barrier(0x008, LEAD, 0);
}

// bf16 rounding of the block kernels: the hardware conversion (v_cvt_pk_bf16_f32,
// round to nearest even), branch free.
__device__ __forceinline__ uint32_t bf16_bits(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }

__device__ __forceinline__ float bf16_round(float v) { return (float)(__bf16)v; }

// two values in one conversion: lo in bits 0..15, hi in bits 16..31
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// GELU with the error function, 0.5 x (1 + erf(x / sqrt 2)) (the reference's
// exact-erf F.gelu), branch free.  erfc(a) for a = |x| / sqrt 2 follows
// Abramowitz & Stegun, Handbook of Mathematical Functions, formula 7.1.26
// (|error| <= 1.5e-7): erfc(a) = t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-a^2),
// t = 1 / (1 + p a).  With e = erfc(a) / 2, GELU(x) = x - x e for x >= 0 and
// x e = -|x| e for x < 0, i.e. max(x, 0) - |x| e in both cases, so the
// negative tail carries no cancellation.  After the bf16 rounding of the result
// it agrees with the exact-erf GELU except in the far negative tail (x < -3.5,
// |GELU| < 1e-3), where the two can differ by one bf16 step.
__device__ __forceinline__ float gelu_tail(float ax) {  // e = erfc(ax / sqrt 2) / 2, ax >= 0
  // p / sqrt 2 with p = 0.3275911; coefficients a_i / 2
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(ax, 0.23164189619f, 1.0f));
  const float poly = t * (0.127414796f + t * (-0.142248368f + t * (0.7107068705f + t * (-0.7265760135f + t * 0.5307027145f))));
  // exp(-x^2 / 2) = 2^(-x^2 log2(e) / 2)
  return poly * __builtin_amdgcn_exp2f((ax * ax) * -0.72134752044448170f);
}

__device__ __forceinline__ float gelu_erf(float v) {
  const float ax = fabsf(v);
  return __builtin_fmaf(-ax, gelu_tail(ax), fmaxf(v, 0.0f));
}

// GELU of a bf16 value through a table of e(|x|) = gelu_tail(|x|) over the bf16
// values 2^-16 <= |x| <= 8 (bit patterns 0x3780 .. 0x4100, 2433 floats, 9.5 KB
// of LDS).  Inside that range the result is gelu_erf(x) bit for bit (same e,
// same final FMA).  Outside it |x| is clamped to the range ends: for
// |x| < 2^-16 both e values are 1/2 to within 2^-17, so both results round to
// the bf16 value x/2; for x > 8 both round to x; for x < -8 both are below
// 1e-14 in magnitude (the exact-erf GELU's fp32 value there is -0).  The
// table replaces two transcendental and ten other VALU operations per
// element with a clamp, a shift and one LDS read.
constexpr uint32_t GELU_T_LO = 0x3780u, GELU_T_HI = 0x4100u;
constexpr int GELU_T_N = int(GELU_T_HI - GELU_T_LO) + 1;

__device__ __forceinline__ void gelu_table_fill(float* t, int tid, int nthreads) {
  for (int i = tid; i < GELU_T_N; i += nthreads)
    t[i] = gelu_tail(__builtin_bit_cast(float, (GELU_T_LO + (uint32_t)i) << 16));
}

__device__ __forceinline__ float gelu_lut(const float* t, float x) {  // x: a bf16 value held as fp32
  const float ax = fabsf(x);
  const float c = __builtin_amdgcn_fmed3f(ax, 0x1p-16f, 8.0f);
  const float e = t[(__builtin_bit_cast(uint32_t, c) >> 16) - GELU_T_LO];
  return __builtin_fmaf(-ax, e, fmaxf(x, 0.0f));
}

// G[i] = bf16(GELU(bf16(u[2i]))) | bf16(GELU(bf16(u[2i+1]))) << 16 for N values: all N table reads are
// issued before the first is used, so the LDS latency is paid once.
template <int N>
__device__ __forceinline__ void gelu_lut_pack(const float* t, const float* u, uint32_t* g) {
  float x[N], e[N];
#pragma unroll
  for (int i = 0; i < N; i += 2) {
    const uint32_t p = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{u[i], u[i + 1]}, bf16x2_t));
    x[i] = __builtin_bit_cast(float, p << 16);
    x[i + 1] = __builtin_bit_cast(float, p & 0xffff0000u);
  }
#pragma unroll
  for (int i = 0; i < N; ++i)
    e[i] = t[(__builtin_bit_cast(uint32_t, __builtin_amdgcn_fmed3f(fabsf(x[i]), 0x1p-16f, 8.0f)) >> 16) - GELU_T_LO];
#pragma unroll
  for (int i = 0; i < N; i += 2)
    g[i >> 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(
        f32x2_t{__builtin_fmaf(-fabsf(x[i]), e[i], fmaxf(x[i], 0.0f)),
                __builtin_fmaf(-fabsf(x[i + 1]), e[i + 1], fmaxf(x[i + 1], 0.0f))}, bf16x2_t));
}

// 16 bytes per lane from global memory (uniform base + per-lane 32-bit byte offset) into LDS at the
// wave-uniform address lds + 16 * lane (global_load_lds_dwordx4; M0 holds the LDS address, one wait state
// between its write and the load).  Completion is counted by vmcnt.
__device__ __forceinline__ void lds_dma16(uint64_t base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(off), "s"(base), "s"(lds) : "memory", "m0");
}

// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt bits 6:4 left at 7, lgkmcnt bits
// 11:8 left at 15), issued through the builtin so that the compiler's own wait tracking sees them.
constexpr unsigned waitcnt_vm(unsigned n) { return 0x0F70u | (n & 15u) | ((n >> 4) << 14); }
constexpr unsigned kWaitVmcnt0 = waitcnt_vm(0);

template <int D>
constexpr int w_stride() { return 2 * D + 16; }

template <int D>
__device__ __forceinline__ u32x4_t read_w_frag(const char* lds, int r, int piece) {
  return *reinterpret_cast<const u32x4_t*>(lds + r * w_stride<D>() + (piece << 4));
}

}  // namespace pdm
