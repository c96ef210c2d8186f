// Shared device helpers for the gfx950 (CDNA4) attention kernels.
//
// Layout conventions (wave64, 32x32 MFMA tiles):
//   * v_mfma_f32_32x32x16_{bf16,f16}: lane l holds A[i = l%32][k = 8*(l/32) + s]
//     and B[k = 8*(l/32) + s][j = l%32] for s = 0..7.
//   * v_mfma_f32_32x32x2_f32: lane l holds A[l%32][l/32] and B[l/32][l%32].
//   * accumulator C[i][j] of a 32x32 tile: lane l, register r holds
//     i = 8*(r/4) + 4*(l/32) + r%4, j = l%32.
// The attention kernels compute transposed score tiles S^T = K Q^T so that a
// lane owns one query row (j = l%32) and 16 keys of it; row reductions are
// then in-lane plus one exchange with the other half of the wave.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace st {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();
// Lazy online-softmax rescaling threshold (log2 units): the running row max
// is only raised when a new score exceeds it by more than this, so the
// exponentials of stale-max rows stay below 2^8 (far from fp32/bf16 overflow).
constexpr float kLazyLog2 = 8.f;

// Element-type traits: the MFMA used for this element type and how many
// elements of an operand one lane holds per instruction.
template <typename T> struct Mma;

template <> struct Mma<bf16> {
  static constexpr int KW = 16;   // contraction length of one instruction
  static constexpr int VEC = 8;   // operand elements per lane
  typedef bf16x8 Frag;
  static __device__ __forceinline__ f32x16 mma(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mma<f16> {
  static constexpr int KW = 16;
  static constexpr int VEC = 8;
  typedef f16x8 Frag;
  static __device__ __forceinline__ f32x16 mma(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mma<float> {
  static constexpr int KW = 2;
  static constexpr int VEC = 1;
  typedef float Frag;
  static __device__ __forceinline__ f32x16 mma(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

// 16x16x32 MFMA (gfx950), 16-bit inputs: lane l holds A[l%16][8*(l/16)+s],
// B[8*(l/16)+s][l%16] (s = 0..7) and C[4*(l/16)+r][l%16] (r = 0..3).
template <typename T> struct Mma16;
template <> struct Mma16<bf16> {
  typedef bf16x8 Frag;
  static __device__ __forceinline__ f32x4 mma(Frag a, Frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma16<f16> {
  typedef f16x8 Frag;
  static __device__ __forceinline__ f32x4 mma(Frag a, Frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// ST_DTYPE_* code of an element type (launch records).
template <typename T> constexpr int dtype_code() {
  return sizeof(T) == 4 ? 0 : (__is_same(T, f16) ? 1 : 2);
}

// (the library is built without the mixed-precision v_fma_mix* forms, so an
// fp16 result is a separate v_cvt_f16_f32 of a full fp32 value)
template <typename T> __device__ __forceinline__ T from_float(float x) { return (T)x; }
template <typename T> __device__ __forceinline__ float to_float(T x) { return (float)x; }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Row (within a 32x32 C tile) of accumulator register r in a lane of half h.
__device__ __forceinline__ int c_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// Value held by the lane 32 positions away (the other half of the wave), via
// gfx950's v_permlane32_swap rather than the LDS crossbar.
__device__ __forceinline__ float other_half(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// Wave-wide integer max / min (butterfly over the 64 lanes). Workgroup-wide
// ranges are built from these plus one LDS slot per wave: LDS atomics from
// every lane on one address serialise (about 8 us for 256 lanes x 4 values).
__device__ __forceinline__ int wave_max(int x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = max(x, __shfl_xor(x, o, 64));
  return x;
}
__device__ __forceinline__ int wave_min(int x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = min(x, __shfl_xor(x, o, 64));
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Natural-log helpers that keep -inf for zero mass.
__device__ __forceinline__ float log_mass(float m2, float mass) {
  // m2 is a running max in log2 units, mass the sum at that scale.
  return mass > 0.f ? (m2 + fast_log2(mass)) * kLn2 : kNegInf;
}

__device__ __forceinline__ float logaddexp(float a, float b) {
  float m = fmaxf(a, b);
  if (m == kNegInf) return kNegInf;
  return m + __logf(__expf(a - m) + __expf(b - m));
}

// Asynchronous 16-byte global -> LDS copy (gfx950 global_load_lds): lane l of
// the wave writes its 16 bytes to lds_base + 16*l, so one instruction fills
// 1 KiB of LDS in lane order. lds_base must be wave-uniform. Completion is
// tracked by vmcnt: wait_vm() before the data is read.
__device__ __forceinline__ void async_copy16(const void* g, void* lds_base) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds_base, 16, 0, 0);
}
__device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt(0);
  __asm__ volatile("" ::: "memory");
}

// 16-byte global load / store helpers.
template <typename V> __device__ __forceinline__ V load_vec(const void* p) {
  return *reinterpret_cast<const V*>(p);
}

}  // namespace st
