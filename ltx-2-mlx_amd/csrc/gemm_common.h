// Device helpers shared by the projection GEMM kernels (gemm.hip: the 4- and
// 8-wave tile kernels; gemm_rows.hip: the few-row split-K kernel): epilogue
// arithmetic, E8M0 decoding, LDS-DMA / buffer-load helpers and wait counters.
#pragma once

#include "ltx_common.h"

namespace ltx {

// B_MX: MXFP8 weights and MXFP8 activations (E4M3 codes + E8M0 scale per 32
// along K on both operands), multiplied by the scaled fp8 MFMA -- an opt-in
// path with quantised activations, only on the 8-wave kernel.
enum BKind { B_BF16 = 0, B_INT8 = 1, B_MXFP8 = 2, B_MX = 3 };

// workgroups are dealt to the 8 XCDs round-robin (block b runs on XCD b % 8)
constexpr int kNumXcd = 8;

// bf16 rounding of two values with one conversion: the same bits as
// round_bf on each
__device__ __forceinline__ void round_bf2(float& x, float& y) {
  asm("" : "+v"(x), "+v"(y));
  const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x, y}, bf16x2));
  x = __uint_as_float(u << 16);
  y = __uint_as_float(u & 0xffff0000u);
}

// GELU with the tanh approximation (feed_forward.py:8-14).  tanh(u) is
// evaluated as 1 - 2 / (exp(2u) + 1) with the hardware exp2 and reciprocal
// a few instructions instead of the libm tanh and an IEEE division, absolute
// error ~2e-7, far below the bf16 rounding of the result; saturates correctly
// at +-inf.
__device__ __forceinline__ float gelu_tanh(float x) {
  // 0.5 x (1 + tanh(u)) with u = sqrt(2/pi) (x + 0.044715 x^3) is
  // x sigmoid(2u) = x / (1 + 2^t), t = -2u log2(e) = x (A + B x^2):
  // five VALU instructions and two transcendentals per element
  constexpr float A = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
  constexpr float B = A * 0.044715f;
  const float t = x * fmaf(B, x * x, A);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

// 2 * bf16(sigmoid(y)) -- the head gate of attention.py:586-590 -- with the
// hardware exp2 and reciprocal (relative error ~2e-7 before the bf16 rounding).
__device__ __forceinline__ float sigmoid2_bf(float y) {
  const float e = __builtin_amdgcn_exp2f(-1.4426950408889634f * y);
  return 2.0f * round_bf(__builtin_amdgcn_rcpf(1.0f + e));
}

__device__ __forceinline__ float e8m0_to_f32(uint32_t s) {
  // 2^(s-127): s << 23 is the float for 1 <= s <= 254; s = 0 (2^-127) and
  // s = 255 (NaN) set the top mantissa bit as well.  Branch-free: s differs
  // per lane.
  const uint32_t special = (s == 0u || s == 0xffu) ? 0x00400000u : 0u;
  return __uint_as_float((s << 23) | special);
}

// The same value in vector instructions only (no lane-mask round trip):
// 2^-127 * 2^s by ldexp -- exact, 2^-127 itself a denormal (denormals are
// kept) -- and s = 255 (+inf from ldexp) turned into NaN by x + (x - x).
__device__ __forceinline__ float e8m0_to_f32_valu(uint32_t s) {
  const float x = __builtin_amdgcn_ldexpf(__uint_as_float(0x00400000u), (int)s);
  return x + (x - x);
}


// LDS-DMA helpers: each lane of a wave writes the 16 bytes it loads to
// `lds_wave_base + 16 * lane`; the per-lane source address implements the
// swizzle (the data a lane fetches is the data its LDS slot must hold).
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(1))) const void* gbl_ptr_t;

__device__ __forceinline__ void dma16(const void* src, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)lds_wave_base, 16, 0, 0);
}

// s_waitcnt through the builtin (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt_hi[15:14]) so the compiler's own wait insertion
// sees it.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x70 | 0xF00);
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }


// dword 3 of a raw buffer descriptor on gfx9-class GPUs (untyped, 32-bit
// data format so that dwordx4 loads are not format-converted)
constexpr int kBufferRsrcWord3 = 0x00020000;

// 16 bytes per lane from base + voff + soff (bounded by num_records bytes) to
// LDS at lds_dst + 16 * lane: a buffer load with the lds modifier.  The
// descriptor is built from wave-uniform values (scalar registers; the
// compiler hoists it out of loops).  Kept out of the kernel bodies, whose
// host-side launch stubs are not emitted when they name the descriptor type.
__device__ __forceinline__ void buffer_dma16(const void* base, int num_records, uint32_t voff, int soff,
                                             char* lds_dst) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, num_records, kBufferRsrcWord3);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds_dst, 16, voff, soff, 0, 0);
}

// Workgroup barrier without the memory fence of __syncthreads(): the fence
// would wait for every outstanding global->LDS load of the wave (they count as
// LDS writes), including the ones meant to stay in flight across the barrier.
// Callers wait for exactly what the barrier has to publish.
__device__ __forceinline__ void barrier_nofence() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}


}  // namespace ltx
