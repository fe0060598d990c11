// Shared device-side helpers for the gfx950 kernels of the DSA path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dsa_abi.h"

namespace dsa {

// MFMA operand / accumulator types (bf16 inputs, fp32 accumulate).
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;

// fp32 -> bf16 with round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f2bf(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}
__device__ __forceinline__ float bf2f(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}
typedef float f32v2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16v2 __attribute__((ext_vector_type(2)));
// Two fp32 -> packed bf16x2 (lo in bits 0..15), RNE: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32v2){lo, hi}, bf16v2));
}
__device__ __forceinline__ float bf_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
// bf16(x) (round to nearest even) as an fp32 value: one v_cvt_pk_bf16_f32 with a zero
// low operand leaves bf16(x) in the high half and zeros below it. Cheaper than a
// packed conversion of two values followed by the two extractions (the low half needs
// a left shift, which issues at the slower of the gfx950 VALU rates).
__device__ __forceinline__ float bf16_as_f32(float x) { return __builtin_bit_cast(float, pack_bf2(0.f, x)); }

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ T ld_nt(const T* p) {
  return __builtin_nontemporal_load(p);
}
template <typename T>
__device__ __forceinline__ void st_nt(T* p, T v) {
  __builtin_nontemporal_store(v, p);
}

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }

// A topk slot index as int: int32 indices as stored (the kernels mask values < 0
// and >= n_kv); int64 indices (the indexer's output dtype) narrowed in the kernel,
// every value outside [0, 2^31) becoming -1 (masked) instead of wrapping.
__device__ __forceinline__ int slot_index(const int32_t* p, int64_t i) { return p[i]; }
__device__ __forceinline__ int slot_index(const int64_t* p, int64_t i) {
  const int64_t v = p[i];
  return (v >= 0 && v <= INT32_MAX) ? (int)v : -1;
}

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding:
// vmcnt[3:0] in bits 3:0 and vmcnt[5:4] in bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Buffer resource (V#) of a raw byte range: base, stride 0, num_records =
// bytes (accesses at or beyond it read as zero, stores there are dropped),
// word3 = the gfx9 raw-buffer format word. The base is made wave-uniform.
__device__ __forceinline__ i32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  return i32x4{__builtin_amdgcn_readfirstlane((int32_t)(uint32_t)a),
               __builtin_amdgcn_readfirstlane((int32_t)((a >> 32) & 0xffffu)),
               (int32_t)bytes, 0x00020000};
}

// The same range as a typed resource for the compiler's buffer intrinsics
// (__builtin_amdgcn_raw_buffer_load_b128 / _store_b128).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)(((uint64_t)hi << 32) | lo), 0,
                                           (int)bytes, 0x00020000);
}

// One buffer_load_dwordx4 ... lds: lane l copies the 16 B at byte offset voff of
// the resource to LDS byte address m0 + 16 * l (m0 is wave-uniform). It is
// issued from inline asm so that the compiler does not track it: its own
// waitcnt insertion would otherwise put a vmcnt(0) in front of every LDS read
// of the ring. The kernel waits for these copies itself (wait_vmcnt + barrier).
// M0 is an input operand (the compiler sets it); the s_nop covers the
// M0-write -> LDS-DMA hazard.
__device__ __forceinline__ void lds_dma16(i32x4 rsrc, uint32_t voff, uint32_t m0) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "{m0}"(m0)
               : "memory");
}

// One complex product of RoPE in the rounding torch uses.
//  DSA_ROPE_CPU: vectorised CPU kernel, every product rounded, no FMA.
//  DSA_ROPE_TORCH_ROCM: the broadcast elementwise kernel of torch-ROCm; its
//  unrolled loop contracts unroll slots 0..2 as re = fma(a, c, -(b*d)),
//  im = fma(b, c, a*d) and slot 3 as re = fma(-b, d, a*c), im = (a*d) + (b*c),
//  where slot = (n / 128) % 4 for the flat index n of the complex element in the
//  [b, s, h, rd/2] tensor (measured: 1.33 M of 1.33 M elements agree bit for bit).
__device__ __forceinline__ void rope_pair(float a, float b, float c, float d, int mode,
                                          int64_t n, float& re, float& im) {
  if (mode == DSA_ROPE_CPU) {
    re = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, d));
    im = __fadd_rn(__fmul_rn(a, d), __fmul_rn(b, c));
  } else if (((n >> 7) & 3) != 3) {
    re = __fmaf_rn(a, c, -__fmul_rn(b, d));
    im = __fmaf_rn(b, c, __fmul_rn(a, d));
  } else {
    re = __fmaf_rn(-b, d, __fmul_rn(a, c));
    im = __fadd_rn(__fmul_rn(a, d), __fmul_rn(b, c));
  }
}

}  // namespace dsa

// Host helpers shared by the entry points. The library's only state: the CU
// count of each device and the dynamic-LDS limits already set per kernel,
// both filled on first use and safe to call from several threads.
namespace dsa_host {
constexpr int kMaxDevices = 64;
int device_cu_count(int* out);
int ensure_dyn_lds(const void* fn, int bytes);
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
}  // namespace dsa_host
