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
// Compute units of the current device (cached per device).
int device_cus();

// ---------------------------------------------------------------- vectors
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
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
  static constexpr uint32_t kOne2 = 0x3f803f80u;  // two 1.0
  // two fp32 -> packed pair (lo = a), one v_cvt_pk_bf16_f32 (RNE)
  __device__ static inline uint32_t pack2(float a, float b) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
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
  __device__ static inline f32x16 mfma32x32x16(const u32x4 &a, const u32x4 &b, const f32x16 &c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // 16x16x16: lane l holds row (A) / column (B) l % 16, k = 4 (l / 16) .. +3,
  // the layout of the accumulator's rows, so a result feeds the next B operand
  __device__ static inline f32x4 mfma16x16x16(const u32x2 &a, const u32x2 &b, const f32x4 &c) {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4, a), __builtin_bit_cast(bf16x4, b), c,
                                                     0, 0, 0);
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
  static constexpr uint32_t kOne2 = 0x3c003c00u;  // two 1.0
  // two fp32 -> packed pair (lo = a), one v_cvt_pk_f16_f32 (RNE)
  __device__ static inline uint32_t pack2(float a, float b) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
  }
  template <bool HI>
  __device__ static inline uint32_t fp8x2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
  }
  __device__ static inline f32x4 mfma16x16x32(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline f32x16 mfma32x32x16(const u32x4 &a, const u32x4 &b, const f32x16 &c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4 mfma16x16x16(const u32x2 &a, const u32x2 &b, const f32x4 &c) {
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0,
                                                 0);
  }
};

// ---------------------------------------------------------------- fp8 e4m3fn
// Saturate to +-448 keeping NaN (comparisons with NaN are false).
__device__ inline float sat448(float y) {
  y = y > 448.f ? 448.f : y;
  y = y < -448.f ? -448.f : y;
  return y;
}
// Four values -> four e4m3fn bytes (saturating, round to nearest even), the
// first value in the lowest byte.
__device__ inline uint32_t fp8x4(float a, float b, float c, float d) {
  int w = 0;
  w = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(a), sat448(b), w, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(c), sat448(d), w, true);
  return static_cast<uint32_t>(w);
}

// ---------------------------------------------------------------- output gate
// Qwen3.5's attention output gate (models/qwen3_5.py:141-142) as eager torch
// computes it on 16-bit tensors: out = rnd(rnd(o) * rnd(sigmoid(g))), with
// sigmoid(g) = 1 / (1 + exp(-g)) in fp32 and rnd = round to T.  The sigmoid
// uses the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32, about one
// fp32 ulp each; 1 / (1 + 2^(-g log2 e)), exact at g = +-inf): it differs
// from the correctly rounded fp32 sigmoid by a few fp32 ulps, which moves
// rnd(sigmoid) by one 16-bit ulp only for values within those few ulps of a
// rounding boundary -- about 1e-4 of the elements -- at a quarter of the
// instructions of expf and an IEEE division (the gate is evaluated for every
// output element of a fused store).  The empty asm statements keep each
// rounding separate (the compiler would otherwise fold a product and its
// narrowing into one mixed-precision instruction).
template <class T>
__device__ inline float gate_one(float o, uint32_t g16) {
  const float gf = T::to_float(static_cast<uint16_t>(g16));
  float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gf * -1.4426950408889634f));
  asm("" : "+v"(sg));
  asm("" : "+v"(o));
  const float sr = T::to_float(T::from_float(sg));
  const float orr = T::to_float(T::from_float(o));
  return orr * sr;  // exact in fp32: two 16-bit significands
}
// Four outputs of one row (fp32) with their four gate values (packed 16-bit).
template <class T>
__device__ inline u32x2 gate4(const f32x4 &v, const u32x2 &g) {
  return u32x2{T::pack2(gate_one<T>(v[0], g[0] & 0xffffu), gate_one<T>(v[1], g[0] >> 16)),
               T::pack2(gate_one<T>(v[2], g[1] & 0xffffu), gate_one<T>(v[3], g[1] >> 16))};
}

// ---------------------------------------------------------------- memory
// Load of data that no kernel writes while it runs (sequence metadata, block
// tables), through the constant address space: with a wave-uniform address
// it becomes a scalar load, which does not wait on the vector-memory counter.
template <class T>
__device__ inline T ld_const(const T *p) {
  return *(const __attribute__((address_space(4))) T *)(reinterpret_cast<uintptr_t>(p));
}
// A wave-uniform value copied into scalar registers of its own.  Kernel
// arguments arrive through wide scalar loads; the register allocator keeps
// such a load as one unit, so a loop that needs two of its fields would
// otherwise spill and reload all sixteen registers together.
template <class T>
__device__ inline T own_sgpr(T x) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values");
  uint32_t w[sizeof(T) / 4];
  __builtin_memcpy(w, &x, sizeof(T));
#pragma unroll
  for (unsigned i = 0; i < sizeof(T) / 4; ++i) {
    w[i] = __builtin_amdgcn_readfirstlane(w[i]);
    asm volatile("" : "+s"(w[i]));
  }
  __builtin_memcpy(&x, w, sizeof(T));
  return x;
}
__device__ inline u32x4 load16(const void *p) { return *reinterpret_cast<const u32x4 *>(p); }
__device__ inline void store16(void *p, const u32x4 &v) { *reinterpret_cast<u32x4 *>(p) = v; }

// Buffer resource over [base, base + num_bytes): raw buffer loads outside the
// range return 0 without touching memory.  Dword 3 is the gfx9-family raw
// (untyped, 32-bit data format) descriptor word.
// The fields are forced into scalar registers (readfirstlane): the caller
// guarantees they are wave-uniform, and a descriptor the compiler cannot
// prove uniform would be wrapped in a per-load waterfall loop.
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t num_bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32));
  const uint32_t n = __builtin_amdgcn_readfirstlane(num_bytes);
  void *ub = reinterpret_cast<void *>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, static_cast<short>(0), static_cast<int>(n), 0x00020000);
}
// 16-byte raw buffer load with the non-temporal (streaming) hint.
__device__ inline u32x4 buffer_load16_nt(__amdgpu_buffer_rsrc_t r, int voffset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, 0, 2));
}

// The four words of the raw buffer descriptor make_rsrc builds (base, stride
// 0, num_bytes, raw dword format), for inline assembly.
__device__ inline u32x4 rsrc_words(const void *base, uint32_t num_bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32));
  return u32x4{lo, hi & 0xffffu, static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(num_bytes)), 0x00020000u};
}
// Global -> LDS copy of 16 bytes per lane (buffer_load_dwordx4 ... lds) as an
// opaque instruction: lane l's 16 bytes from descriptor `rsrc` at byte offset
// `voff` land at LDS byte address lds_addr + 16 * l (lds_addr goes into M0).
// The compiler does not know that the instruction writes LDS, so it never
// drains the copies in flight before its own LDS reads; callers order them
// with wait_vmcnt() and a workgroup barrier.  Completion counts in vmcnt.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ inline void dma16_opaque(uint32_t lds_addr, const u32x4 &rsrc, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(rsrc)
               : "m0");
}
// The same for 4 bytes per lane (buffer_load_dword ... lds): lane l's dword
// lands at lds_addr + 4 * l.
__device__ inline void dma4_opaque(uint32_t lds_addr, const u32x4 &rsrc, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(rsrc)
               : "m0");
}
#pragma clang diagnostic pop
// LDS reads the compiler schedules and waits for itself, at LDS byte address
// `addr` + OFF (the constant folds into the instruction's offset).  Only for
// LDS that no compiler-visible copy writes (the copies above are opaque).
template <int OFF>
__device__ inline u32x4 lds_load_b128(uint32_t addr) {
  static_assert(OFF % 16 == 0 && OFF >= 0 && OFF < 65536, "ds offset");
  const auto *p = reinterpret_cast<const __attribute__((address_space(3))) u32x4 *>(static_cast<uintptr_t>(addr));
  return p[OFF / 16];
}
__device__ inline void lds_store_b128(uint32_t addr, const u32x4 &v) {
  *reinterpret_cast<__attribute__((address_space(3))) u32x4 *>(static_cast<uintptr_t>(addr)) = v;
}
template <int OFF>
__device__ inline u32x2 lds_load_tr16(uint32_t addr) {
  static_assert(OFF % 8 == 0 && OFF >= 0 && OFF < 65536, "ds offset");
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  auto *p = reinterpret_cast<__attribute__((address_space(3))) s16x4 *>(static_cast<uintptr_t>(addr));
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(p + OFF / 8));
}
template <int OFF>
__device__ inline u32x2 lds_load_b64(uint32_t addr) {
  static_assert(OFF % 8 == 0 && OFF >= 0 && OFF < 65536, "ds offset");
  const auto *p = reinterpret_cast<const __attribute__((address_space(3))) u32x2 *>(static_cast<uintptr_t>(addr));
  return p[OFF / 8];
}
// Transposing 8-bit read: within each group of 16 lanes, lane 2 rho + p
// addresses 8 bytes (piece p of row rho, rho < 8), and lane i receives byte
// i % 8 of the pieces of lanes i / 8, 2 + i / 8, ..., 14 + i / 8 -- column i
// of the group's 16-column block over its 8 rows (checked on gfx950).
__device__ inline u32x2 lds_load_tr8(uint32_t addr) {
  typedef int i32x2 __attribute__((ext_vector_type(2)));
  auto *p = reinterpret_cast<__attribute__((address_space(3))) i32x2 *>(static_cast<uintptr_t>(addr));
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32(p));
}
// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ inline void wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// Workgroup barrier without the memory-model fence __syncthreads() implies
// (which would wait for every outstanding load, including in-flight DMA).
__device__ inline void raw_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Wave-level LDS ordering between lanes of ONE wave.  The LDS executes a
// wave's DS instructions in issue order, so a read issued after a write (by
// any lane of the same wave) sees it; only the compiler must be kept from
// reordering across this point.  (A memory-model fence here makes the
// backend wait for every outstanding global load, which would serialize the
// prefetch pipeline.)
__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
}

// Butterflies across lane l and l^16 / l^32 with gfx950 permlane swaps (one
// VALU op each, no LDS round trip).  With both operands = v, the swap returns
// {v, partner} in some order on every lane.
__device__ inline float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ inline uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ inline float max16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(f2u(v), f2u(v), false, false);
  const uint32_t a = r[0], b = r[1];
  return fmaxf(u2f(a), u2f(b));
}
__device__ inline float max32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(f2u(v), f2u(v), false, false);
  const uint32_t a = r[0], b = r[1];
  return fmaxf(u2f(a), u2f(b));
}
__device__ inline float sum16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(f2u(v), f2u(v), false, false);
  const uint32_t a = r[0], b = r[1];
  return u2f(a) + u2f(b);
}
__device__ inline float sum32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(f2u(v), f2u(v), false, false);
  const uint32_t a = r[0], b = r[1];
  return u2f(a) + u2f(b);
}

// The same maxima with a plain v_max_f32 after the swap: no NaN quieting of
// the swapped value (the inputs are finite or -inf).
__device__ inline float vmax_raw(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ inline float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ inline float max16_raw(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(f2u(v), f2u(v), false, false);
  const uint32_t a = r[0], b = r[1];
  return vmax_raw(u2f(a), u2f(b));
}
__device__ inline float max32_raw(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(f2u(v), f2u(v), false, false);
  const uint32_t a = r[0], b = r[1];
  return vmax_raw(u2f(a), u2f(b));
}

// Wave-wide inclusive prefix sum of an int through DPP: shifts by 1, 2, 4, 8
// within each 16-lane row, then each row's running total broadcast into the
// rows after it (row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2
// and 3).  Lanes whose source is out of range add 0 (the `old` operand).
__device__ __forceinline__ int wave_iscan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}
// Sum of an int over the 64 lanes, in every lane.
__device__ __forceinline__ int wave_sum_i32(int v) { return __builtin_amdgcn_readlane(wave_iscan(v), 63); }

// Transposing LDS read (ds_read_b64_tr_b16).  Within each 16-lane group,
// lanes 4k..4k+3 address the four 8-byte pieces of "row" k (16 consecutive
// 16-bit elements); lane i receives element i of rows 0..3, packed in order.
__device__ inline u32x2 lds_read_tr16(const uint16_t *p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4 *)(p));
  return __builtin_bit_cast(u32x2, v);
}
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
