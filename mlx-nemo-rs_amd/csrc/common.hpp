// Shared device helpers for the gfx950 (CDNA4) rel-pos MHSA kernels.
//
// Operand fragments are 16 bytes per lane: 8 bf16 or 4 fp32 values along the
// contraction index. A 16x16 output tile is produced by one
// v_mfma_f32_16x16x32_bf16 (bf16) or four v_mfma_f32_16x16x4_f32 (fp32):
//
//   A operand  lane l: row  l%16, k-chunk l/16  (A[row][kc*EPL + e])
//   B operand  lane l: col  l%16, k-chunk l/16  (B[kc*EPL + e][col])
//   C/D        lane l: col  l%16, rows 4*(l/16) + r, r = 0..3
//
// For fp32 the four MFMAs take element e = 0..3 of both fragments, so a
// fragment pair covers 16 contraction indices; for bf16 one MFMA covers 32.
// (Layouts verified on gfx950 with an all-integer probe against a CPU GEMM.)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
// 16- and 8-byte chunks as native vectors (HIP's uint4/uint2 are wrapper
// structs that keep staging arrays from being promoted to registers).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

namespace mhsa {

constexpr int kWave = 64;

template <typename T> struct Frag;
template <> struct Frag<float> {
  using type = floatx4;
  static constexpr int EPL = 4;    // elements per lane per fragment
  static constexpr int KSTEP = 16; // contraction indices per fragment pair
};
template <> struct Frag<bf16> {
  using type = bf16x8;
  static constexpr int EPL = 8;
  static constexpr int KSTEP = 32;
};

__device__ __forceinline__ floatx4 mma16(const floatx4 a, const floatx4 b, floatx4 c) {
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], c, 0, 0, 0);
  return c;
}
__device__ __forceinline__ floatx4 mma16(const bf16x8 a, const bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 32x32 output tile, K = 16: lane l holds A[l%32][8*(l/32) + e],
// B[8*(l/32) + e][l%32] and C rows 8*(r/4) + 4*(l/32) + r%4 of column l%32.
typedef float floatx16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ floatx16 mma32(const bf16x8 a, const bf16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Round an fp32 value to the storage type and back (identity for fp32).
// bf16: one packed conversion with 0 as its low input leaves bf16(v) (round
// to nearest even) in the high half, and the word read as fp32 is that
// value; the element-wise form compiles to the conversion into the low half
// and a shift. The s_nop gives an input that a transcendental instruction
// (exp, rcp) has just written its wait state: the compiler does not look
// into inline assembly for that hazard.
template <typename T> __device__ __forceinline__ float round_to(float v);
template <> __device__ __forceinline__ float round_to<float>(float v) { return v; }
template <> __device__ __forceinline__ float round_to<bf16>(float v) {
  float r;
  asm("s_nop 0\n\tv_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(v));
  return r;
}

template <typename T> __device__ __forceinline__ T from_float(float v) { return (T)v; }

// sigmoid(v) = 1 / (1 + e^-v) stored in T, and nn::silu as the reference
// evaluates it: the sigmoid stored, then the product stored (conformer.rs:2069).
// e^-v is the hardware exp2 of -v log2(e) and the division a hardware
// reciprocal (each ~1 ulp, as the fast-math transcendentals of MLX's GPU
// kernels): e^-v = inf for v < -88 gives 0, e^-v = 0 gives 1.
template <typename T>
__device__ __forceinline__ float sigmoid_value(float v) {
  return round_to<T>(__builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(v * -1.4426950408889634f)));
}
template <typename T>
__device__ __forceinline__ float silu_value(float v) {
  return round_to<T>(v * sigmoid_value<T>(v));
}

template <typename T> __device__ __forceinline__ typename Frag<T>::type zero_frag();
template <> __device__ __forceinline__ floatx4 zero_frag<float>() { return floatx4{0.f, 0.f, 0.f, 0.f}; }
template <> __device__ __forceinline__ bf16x8 zero_frag<bf16>() {
  bf16x8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (bf16)0.0f;
  return z;
}

// 16-byte global load with a zero fill when `ok` is false.
template <typename V> __device__ __forceinline__ V load16(const void* p, bool ok) {
  if (ok) return *reinterpret_cast<const V*>(p);
  V z;
  __builtin_memset(&z, 0, sizeof(V));
  return z;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / kWave; }

// Max / sum over the 4 lanes that share a column (l, l^16, l^32, l^48).
__device__ __forceinline__ float col_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  v = fmaxf(v, __shfl_xor(v, 32, kWave));
  return v;
}
__device__ __forceinline__ float col_sum(float v) {
  v += __shfl_xor(v, 16, kWave);
  v += __shfl_xor(v, 32, kWave);
  return v;
}

}  // namespace mhsa
