// Shared device/host helpers for the gfx950 paged attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nq_attn.h"

namespace nq {

// ---------------------------------------------------------------- errors
// Record a message for nq_last_error() and return `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Turn the status of the launch just made into NQ_OK / NQ_ELAUNCH.
int check_launch(const char *what);

// ---------------------------------------------------------------- vectors
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 16-bit element kinds used as MFMA operands.
struct BF16 {
  typedef bf16x8 vec8;
  static constexpr int dtype = NQ_BF16;
  __device__ static inline uint16_t from_float(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  }
  __device__ static inline float to_float(uint16_t h) {
    return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
  }
  // two fp32 -> packed pair (lo = a)
  __device__ static inline uint32_t pack2(float a, float b) {
    return static_cast<uint32_t>(from_float(a)) | (static_cast<uint32_t>(from_float(b)) << 16);
  }
  // two fp8 e4m3 (bytes 0,1 of w, or 2,3 when HI) -> packed pair, exact
  template <bool HI>
  __device__ static inline uint32_t fp8x2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
  }
  __device__ static inline f32x4 mfma16x16x32(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

struct F16 {
  typedef f16x8 vec8;
  static constexpr int dtype = NQ_F16;
  __device__ static inline uint16_t from_float(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
  __device__ static inline float to_float(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
  }
  __device__ static inline uint32_t pack2(float a, float b) {
    return static_cast<uint32_t>(from_float(a)) | (static_cast<uint32_t>(from_float(b)) << 16);
  }
  template <bool HI>
  __device__ static inline uint32_t fp8x2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
  }
  __device__ static inline f32x4 mfma16x16x32(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// ---------------------------------------------------------------- memory
template <typename T>
__device__ inline T ldg(const T *p) {
  return __builtin_nontemporal_load(p);
}

__device__ inline u32x4 load16(const void *p) { return *reinterpret_cast<const u32x4 *>(p); }
__device__ inline void store16(void *p, const u32x4 &v) { *reinterpret_cast<u32x4 *>(p) = v; }

// Streaming (read-once) 16-byte load: slc/nt hint keeps KV out of L2 reuse sets.
__device__ inline u32x4 load16_stream(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

// Wave-level LDS ordering: make this wave's LDS writes visible to its own
// later LDS reads from other lanes (no cross-wave barrier needed).
__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ inline float xor_max(float v, int mask) {
  return fmaxf(v, __shfl_xor(v, mask, 64));
}
__device__ inline float xor_sum(float v, int mask) { return v + __shfl_xor(v, mask, 64); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

inline int elem_size(int dtype) {
  switch (dtype) {
    case NQ_F32: return 4;
    case NQ_F16: return 2;
    case NQ_BF16: return 2;
    case NQ_FP8_E4M3: return 1;
    default: return 0;
  }
}

inline bool aligned(const void *p, int a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace nq
