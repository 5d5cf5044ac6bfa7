// Shared types and helpers for the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <string>

#include "mpx_attn.h"

namespace mpx {

typedef uint32_t u32;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

constexpr float kLog2e = 1.4426950408889634f;
// Normaliser epsilon of the reference's tiled online-softmax path:
// O / (l + 1e-6) (mlx_primitives/constants.py:110, attention/flash.py:312).
constexpr float kSoftmaxEps = 1e-6f;

// ---- error reporting -------------------------------------------------------

void set_error(const char* fmt, ...);
void clear_error();

#define MPX_CHECK_ARG(cond, ...)  \
  do {                            \
    if (!(cond)) {                \
      ::mpx::set_error(__VA_ARGS__); \
      return MPX_EINVAL;          \
    }                             \
  } while (0)

#define MPX_CHECK_HIP(expr)                                              \
  do {                                                                   \
    hipError_t _e = (expr);                                              \
    if (_e != hipSuccess) {                                              \
      ::mpx::set_error("%s failed: %s", #expr, hipGetErrorString(_e));   \
      return MPX_EHIP;                                                   \
    }                                                                    \
  } while (0)

// ---- device helpers ----------------------------------------------------------

// Raw v_exp_f32 (base-2 exponential); exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max / sum of x over the lane pair (l, l ^ 32) with v_permlane32_swap (no LDS
// round trip): after the upper half of one copy is swapped with the lower half
// of another, every lane holds both values of its pair.
__device__ __forceinline__ float pair_max32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// 16-bit storage type <-> float.
template <bool BF16>
__device__ __forceinline__ float h2f(uint16_t x) {
  if constexpr (BF16) {
    return __uint_as_float(((u32)x) << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, x);
  }
}

// Two floats -> packed pair of 16-bit values (round to nearest even).
template <bool BF16>
__device__ __forceinline__ u32 pack2(float a, float b) {
  if constexpr (BF16) {
    bf16x2 r = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(u32, r);
  } else {
    f16x2 r = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(u32, r);
  }
}

// acc + lo(x) + hi(x) for a packed pair of 16-bit values (one v_dot2c).
template <bool BF16>
__device__ __forceinline__ float dot2_sum(u32 x, float acc) {
  if constexpr (BF16) {
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x), one, acc, false);
  } else {
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x), one, acc, false);
  }
}

// 32x32x16 MFMA on 8 packed 16-bit values per lane.
template <bool BF16>
__device__ __forceinline__ f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// 16x16x32 MFMA on 8 packed 16-bit values per lane. Lane l = i + 16 q holds
// A[i][8q .. 8q+7] and B[8q .. 8q+7][i]; element r of the result is C[4q + r][i].
template <bool BF16>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

__device__ __forceinline__ f32x16 mfma32x32x2f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Half-split rotary embedding of one dimension pair (x1 = x[i], x2 = x[i + D/2])
// by the angle whose cosine and sine are c, s, in float32:
//   y1 = x1 c - x2 s,  y2 = x1 s + x2 c
// (kernels/rope.py:477-497). Written with explicit fused multiply-adds so every
// kernel that rotates rounds identically (the standalone RoPE kernel and the
// flash kernel's rotation of Q on load agree bit for bit).
__device__ __forceinline__ void rope_pair(float x1, float x2, float c, float s, float& y1,
                                          float& y2) {
  y1 = __builtin_fmaf(x1, c, -(x2 * s));
  y2 = __builtin_fmaf(x1, s, x2 * c);
}

// ---- dropout on the attention weights ------------------------------------------
// The keep mask is counter-based: a hash of (seed, row, key), so the backward
// regenerates the forward's mask without storing it. Row r = (b * H + h) * Sq + q
// (query head h, counted mod 2^32), key k. One 32-bit hash covers the key pair
// (2m, 2m + 1): its low 16 bits decide key 2m, its high 16 bits key 2m + 1, and
// a key is kept when its 16 bits are >= thresh = round(p * 65536) (at most
// 65535), i.e. with probability 1 - thresh / 65536; kept weights are scaled by
// 1 / (1 - p) (inverted dropout, attention/flash.py:570-574).
//   bits(r, m) = lowbias32((r * 0x9E3779B1 + seed0) ^ (m * 0x85EBCA77 + seed1))
// lowbias32 is C. Wellons' 32-bit integer hash (hash-prospector, 2018):
//   x ^= x >> 16; x *= 0x7feb352d; x ^= x >> 15; x *= 0x846ca68b; x ^= x >> 16.
// 0x9E3779B1 is the 32-bit golden-ratio multiplier, 0x85EBCA77 the second
// xxHash32 prime; both are odd, so distinct rows (pairs) give distinct words.
__device__ __forceinline__ u32 lowbias32(u32 x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}
__device__ __forceinline__ u32 drop_row_key(u32 row, u32 seed0) {
  return row * 0x9E3779B1u + seed0;
}
__device__ __forceinline__ u32 drop_pair_key(u32 pair, u32 seed1) {
  return pair * 0x85EBCA77u + seed1;
}
__device__ __forceinline__ u32 drop_bits(u32 row_key, u32 pair_key) {
  return lowbias32(row_key ^ pair_key);
}
// 16-bit lane mask of a key pair's packed weights: 0xffff over each kept key.
__device__ __forceinline__ u32 drop_mask2(u32 bits, u32 thresh) {
  return ((bits & 0xffffu) >= thresh ? 0xffffu : 0u) | (bits >= (thresh << 16) ? 0xffff0000u : 0u);
}
// Keep test of one key of the pair: its half of the hash is selected by
// (half_mask, half_thresh) = (0xffff, thresh) for key 2m, (0xffff0000,
// thresh << 16) for key 2m + 1.
__device__ __forceinline__ bool drop_keep(u32 bits, u32 half_mask, u32 half_thresh) {
  return (bits & half_mask) >= half_thresh;
}
// Keep threshold for dropout probability p in [0, 1): round(p * 65536), at most 65535.
inline u32 drop_threshold(float p) {
  const double t = (double)p * 65536.0 + 0.5;
  return t >= 65535.0 ? 65535u : (u32)t;
}

// ---- LDS staging helpers (gfx950) ---------------------------------------------

// Compile-time integer tag (selects a register set in the unrolled loop).
template <int N>
struct Const {
  static constexpr int value = N;
};

// Raw buffer resource flags (word 3) for gfx950 buffer loads.
constexpr int kBufferFlags = 0x00020000;

// Raw buffer descriptor words (base, stride 0, num_records, gfx950 flags).
__device__ __forceinline__ u32x4 buffer_desc(const void* base, u32 records = 0x7fffffffu) {
  const unsigned long long a = (unsigned long long)base;
  return (u32x4){(u32)a, (u32)(a >> 32) & 0xffffu, records, (u32)kBufferFlags};
}

__device__ __forceinline__ u32 lds_addr(const void* p) {
  return (u32)(unsigned long long)(__attribute__((address_space(3))) const void*)p;
}

// Workgroup barrier without the memory fence of __syncthreads (which would wait
// for every outstanding load, including DMA into a later stage); the caller
// has already waited for the loads the other waves need. The empty asm
// statements keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// One 16-byte-per-lane DMA: lane l's bytes land at LDS address lds_addr +
// 16*l. Issued as inline assembly so the compiler does not track it: its
// waitcnt pass would otherwise make LDS reads after the loop back-edge wait
// for every DMA in flight (it cannot tell their target stages apart there).
// The caller waits for completion with explicit s_waitcnt vmcnt. M0 carries
// the LDS address; nothing else in the kernels that use it touches M0.
__device__ __forceinline__ void dma16(u32x4 rsrc, unsigned lds_addr, int voff, int soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(rsrc), "s"(soff)
               : "memory", "m0");
}

// One 4-byte-per-lane DMA: lane l's dword lands at LDS address lds_addr + 4 l.
// Untracked by the compiler like dma16.
__device__ __forceinline__ void dma4(u32x4 rsrc, unsigned lds_addr, int voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(rsrc)
               : "memory", "m0");
}

// The same DMA from 64-bit addresses, for pools of 4 GiB and more (the buffer
// form's offsets are 32-bit): lane l's 16 bytes at `src` (its own address) /
// at sbase + voff (a wave-uniform base and a per-lane offset) land at LDS
// address lds_addr + 16*l.
__device__ __forceinline__ void dma16_global(unsigned lds_addr, const void* src) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds_addr), "v"(src)
               : "memory", "m0");
}
__device__ __forceinline__ void dma16_global_s(unsigned lds_addr, const void* sbase, u32 voff) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds_addr), "v"(voff), "s"(sbase)
               : "memory", "m0");
}

// 16 zero bytes in device memory: the source of rows that have no page in the
// 64-bit (large pool) loads, which have no range check to turn them into zeros.
static __device__ const u32x4 kZeroChunk = {0u, 0u, 0u, 0u};

// ds_read_b64_tr_b16: for a group of 16 lanes whose lane s addresses row
// base + s/4, columns c0 + 4*(s%4) .. +3 of a row-major 16-bit tile, lane s
// receives column c0 + s of rows base .. base + 3.
__device__ __forceinline__ u32x2 lds_read_tr16(const void* p) {
  typedef __attribute__((ext_vector_type(4))) short s16x4;
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(u32x2, r);
}

}  // namespace mpx
