// Shared device helpers for the LTX-2 denoise-path HIP kernels (gfx950 / CDNA4).
//
// Every kernel in this library is written for 64-wide wavefronts.  bf16 values
// are carried as clang's native __bf16; float -> bf16 conversion lowers to the
// hardware v_cvt_pk_bf16_f32 (round-to-nearest-even), which is the rounding
// mode of every `.astype(mx.bfloat16)` on the reference path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ltx_hip.h"

namespace ltx {

typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf2f(bf16 v) { return (float)v; }
__device__ __forceinline__ bf16 f2bf(float v) { return (bf16)v; }
// Round an fp32 value to the nearest bf16 (RNE) and return it widened again.
// The empty asm hides where `v` comes from: without it LLVM narrows a product
// of two bf16-exact operands, round_bf(a * b), to a bf16 multiply whose
// promoted form then fuses with a following add into one fma -- dropping
// exactly the intermediate rounding the reference performs.  It emits no
// instruction, so the compiler still sees (and guards) every real one.
__device__ __forceinline__ float round_bf(float v) {
  asm("" : "+v"(v));
  return (float)(bf16)v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Non-contractible fp32 arithmetic, used where the reference evaluates a
// product and a sum as two separately rounded operations.
// `#pragma clang fp contract(off)` keeps the backend from fusing these into
// an FMA after inlining (HIP compiles with -ffp-contract=fast by default).
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}

// Correctly rounded 1/sqrt(v): the reference uses a precise rsqrt for the
// RMSNorm normalizer.
__device__ __forceinline__ float rsqrt_rn(float v) { return __frsqrt_rn(v); }

// MXFP8 (OCP MX v1.0, E4M3 elements, E8M0 block scale) encoding of four
// values of one block whose exponent is X = floor(log2(block max)) - 8:
// code = E4M3(v / 2^X), rounded to nearest even and saturated to +-448.
// The hardware conversion divides by its scale operand (2^X) and rounds the
// same way but turns values past 448 into NaN, so they are clamped to
// +-448 * 2^X first (NaN passes the clamp and stays NaN).  Measured on the
// device: for every finite bf16 value and every X in [-127, 127] the codes
// equal the rule's, bit for bit.  s = 2^X, lim = 448 * s.
__device__ __forceinline__ uint32_t e4m3x4_ocp(float v0, float v1, float v2, float v3, float s, float lim) {
  auto cl = [lim](float v) { return fabsf(v) >= lim ? __builtin_copysignf(lim, v) : v; };
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  s16x2 w = {0, 0};
  w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, cl(v0), cl(v1), s, false);
  w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, cl(v2), cl(v3), s, true);
  return __builtin_bit_cast(uint32_t, w);
}

// The block exponent of the MXFP8 rule for a block maximum amax >= 0:
// floor(log2(amax)) - 8 clamped to [-127, 127]; -127 for an all-zero block.
__device__ __forceinline__ int mxfp8_block_exponent(float amax) {
  if (!(amax > 0.0f)) return -127;
  int e;
  frexpf(amax, &e);
  const int X = (e - 1) - 8;
  return X < -127 ? -127 : (X > 127 ? 127 : X);
}

}  // namespace ltx

// Launch-status helper shared by the C entry points.
static inline int ltx_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? LTX_OK : LTX_ERR_HIP;
}
