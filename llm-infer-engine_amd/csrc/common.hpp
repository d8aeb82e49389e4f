// Shared device helpers for the gfx950 attention-path kernels.
//
// Everything here is written for CDNA4 (gfx950): 64-lane wavefronts, DPP
// row operations for intra-row reductions, 16-byte vector memory accesses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/miattn.h"

namespace mi {

typedef __bf16 bf16_t;
typedef _Float16 f16_t;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Floor for running maxima (log2 domain).  Keeps "empty" state finite so the
// online-softmax rescale never evaluates (-inf) - (-inf).
constexpr float kNegBig = -1.0e30f;

// ---------------------------------------------------------------- host side
void set_last_error(const char* fmt, ...);
// compute units of the current device (cached per device; 256 if unknown)
int device_cu_count();
// XCDs (XCCs) of the current device, over which the hardware deals workgroup
// ids round-robin (cached per device; 1 if unknown)
int device_xcc_count();

// ---------------------------------------------------------- element traits
template <typename T> struct Elem;
template <> struct Elem<bf16_t> {
  static constexpr int kBytes = 2;
  __device__ static inline float to_f32(bf16_t x) { return (float)x; }
  __device__ static inline bf16_t from_f32(float x) { return (bf16_t)x; }
};
template <> struct Elem<f16_t> {
  static constexpr int kBytes = 2;
  __device__ static inline float to_f32(f16_t x) { return (float)x; }
  // x is materialised as fp32 first: the conversion of a product or sum is
  // otherwise selected as one v_fma_mixlo_f16 (a single rounding of the exact
  // result) where the fp32 operation and the conversion round twice, as the
  // separate ops do
  __device__ static inline f16_t from_f32(float x) {
    __asm__("" : "+v"(x));
    return (f16_t)x;
  }
};
template <> struct Elem<float> {
  static constexpr int kBytes = 4;
  __device__ static inline float to_f32(float x) { return x; }
  __device__ static inline float from_f32(float x) { return x; }
};

// Unpack one 16-byte chunk into fp32 values (8 for 2-byte types, 4 for fp32).
template <typename T> struct Chunk;
template <> struct Chunk<bf16_t> {
  static constexpr int kN = 8;
  __device__ static inline void unpack(const u32x4& w, float* o) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(u[i] << 16);
      o[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
  }
};
template <> struct Chunk<f16_t> {
  static constexpr int kN = 8;
  __device__ static inline void unpack(const u32x4& w, float* o) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      union { uint32_t u; f16_t h[2]; } c;
      c.u = u[i];
      o[2 * i] = (float)c.h[0];
      o[2 * i + 1] = (float)c.h[1];
    }
  }
};
template <> struct Chunk<float> {
  static constexpr int kN = 4;
  __device__ static inline void unpack(const u32x4& w, float* o) {
    o[0] = __uint_as_float(w.x);
    o[1] = __uint_as_float(w.y);
    o[2] = __uint_as_float(w.z);
    o[3] = __uint_as_float(w.w);
  }
};

// ------------------------------------------------------------- DPP helpers
template <int CTRL>
__device__ inline float dpp_f32(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum over aligned groups of N lanes (N in {1,2,4,8,16,32}); every lane of the
// group receives the total.  Up to 16 lanes intra-row DPP only (no LDS
// traffic); 32 adds one exchange between neighbouring rows.
template <int N>
__device__ inline float group_sum(float x) {
  if constexpr (N >= 2) x += dpp_f32<0xB1>(x);   // quad_perm [1,0,3,2]
  if constexpr (N >= 4) x += dpp_f32<0x4E>(x);   // quad_perm [2,3,0,1]
  if constexpr (N >= 8) x += dpp_f32<0x141>(x);  // row_half_mirror
  if constexpr (N >= 16) x += dpp_f32<0x140>(x); // row_mirror
  if constexpr (N >= 32) x += __shfl_xor(x, 16, 64);
  return x;
}

template <int N>
__device__ inline float group_max(float x) {
  if constexpr (N >= 2) x = fmaxf(x, dpp_f32<0xB1>(x));
  if constexpr (N >= 4) x = fmaxf(x, dpp_f32<0x4E>(x));
  if constexpr (N >= 8) x = fmaxf(x, dpp_f32<0x141>(x));
  if constexpr (N >= 16) x = fmaxf(x, dpp_f32<0x140>(x));
  return x;
}

__device__ inline float shfl_xor_f32(float x, int mask) {
  return __shfl_xor(x, mask, 64);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ inline float fast_log2(float x) { return __builtin_amdgcn_logf(x); }
// silu in fp32 (x * sigmoid(x) as x / (1 + e^-x)), the form torch's silu uses
__device__ inline float silu_f32(float a) { return a / (1.0f + expf(-a)); }

__device__ inline u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// Streaming (read-once) 16-byte load: non-temporal hint so KV bytes that are
// read exactly once do not evict reusable lines from L2.
__device__ inline u32x4 load16_stream(const void* p) {
  const u32x4* q = reinterpret_cast<const u32x4*>(p);
  return __builtin_nontemporal_load(q);
}

// Raw buffer resource over [base, base + bytes).  A 16-byte load at a byte
// offset past `bytes` returns zeros and touches no memory (the hardware range
// check): padding lanes of a tile pass kOobOffset and read nothing.
typedef __amdgpu_buffer_rsrc_t buf_rsrc;
constexpr uint32_t kOobOffset = 0x7ffffff0u;
__device__ inline buf_rsrc make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
// A pointer every lane holds the same value of, moved to scalar registers.
__device__ inline const unsigned char* uniform_ptr(const unsigned char* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const unsigned char*>((uintptr_t)(((uint64_t)hi << 32) | lo));
}
__device__ inline u32x4 buf_load16(buf_rsrc r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
// non-temporal variant (read-once weight streams)
__device__ inline u32x4 buf_load16_nt(buf_rsrc r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2));
}

// ------------------------------------------------- LDS tile staging
// One wave-wide 16-byte-per-lane global->LDS copy: lane t's 16 bytes at
// base + voff land at LDS byte address lds + 16 t.  Issued as inline asm on
// purpose: the compiler does not track it, so it does not insert a wait for
// the copy before unrelated LDS reads of the other buffer; completion is
// awaited explicitly (dma_wait_all) before the barrier that publishes the tile.
// The compiler's hazard recognizer does not look inside inline asm, so the asm
// supplies the wait states itself: s_nop 4 (5 wait states) covers both a VALU
// write of the base SGPRs (v_readlane / v_readfirstlane, 5 required before a
// VMEM read) and the M0 write (1 required before an LDS DMA).
__device__ inline void lds_dma16(const unsigned char* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds)
               : "memory");
}
__device__ inline uint32_t lds_addr(const unsigned char* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)(p);
}
__device__ inline void dma_wait_all() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// One rotate-half RoPE pair (x1 = x[i], x2 = x[i + D/2], c/s = cos/sin[i]):
// y1 = x1*c - x2*s, y2 = x2*c + x1*s in fp32 with no contraction -- products
// and the sum each rounded to fp32 (an fma, or a fused fma_mix f16
// conversion, would round once and can differ in the last bit) -- then
// rounded once to T.  Shared by the RoPE kernels and the prefill kernels'
// Q prologue, so both give the same bits.
template <typename T, typename CT>
__device__ inline void rope_rotate(float x1, float x2, CT cv, CT sv, T& y1, T& y2) {
#pragma clang fp contract(off)
  const float c = Elem<CT>::to_f32(cv), s = Elem<CT>::to_f32(sv);
  const float x1c = x1 * c, x2s = x2 * s, x2c = x2 * c, x1s = x1 * s;
  const float r1 = x1c - x2s, r2 = x2c + x1s;
  y1 = Elem<T>::from_f32(r1);
  y2 = Elem<T>::from_f32(r2);
}

__device__ inline void block_sync_lds() {
  // LDS reads of this wave are complete and every wave has arrived; the
  // tile copies (vmcnt) are waited for separately where a tile is published.
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

}  // namespace mi
