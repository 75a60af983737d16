// Weight formats of the quantised projections: encoders and bf16 decoders.
//
// MXFP8 (OCP Microscaling v1.0, element E4M3, block 32 along K, scale E8M0):
//   the storage of LTX_2_MLX's `mx.quantize(W, 32, 8, mode="mxfp8")`
//   (loader/transformer_cache.py:1255-1267): codes (N, K) uint8 -- the same
//   bytes as the reference's (N, K/4) uint32 words -- and scales (N, K/32).
//   The reference's encoder is MLX-internal; this one follows the OCP rule:
//     X = floor(log2(max|w|)) - 8 (8 = E4M3 emax), clamped to [-127, 127],
//     scale byte = X + 127, code = E4M3(w / 2^X) rounded to nearest-even and
//     saturated to +-448.  An all-zero block gets X = -127.
// FP8 checkpoints (loader/transformer_cache.py:658-708): E4M3 codes with an
//   optional per-tensor fp32 weight_scale, dequantised at load time as
//   from_fp8(w) * scale in fp32 and rounded once to the cache dtype.
// int8 W8A16 (per output channel, symmetric):
//     s[n] = max_k |w[n,k]| / 127 (fp32), q = clamp(rint(w / s), -127, 127);
//     a zero row has s = 0 and q = 0.  Decode: w' = bf16(fp32(q) * s).
#include <type_traits>

#include "ltx_common.h"

namespace ltx {

// Rows of 32-element blocks: one wave per 512-element chunk of a row, lane l
// holding elements 8l..8l+7 (one 16-byte load), lanes 4b..4b+3 forming block
// b; the block maximum takes two lane exchanges, the codes leave as one
// 8-byte store per lane (512 contiguous bytes per wave) and lane 4b writes the
// block's scale byte.  Chunks past K (K % 512 != 0) leave their lanes idle.
// Used for weights (at load) and for activation rows (the opt-in MX path).
__global__ __launch_bounds__(256) void mxfp8_quantize_kernel(const bf16* __restrict__ W, int64_t ldw, int64_t N,
                                                             int64_t K, uint8_t* __restrict__ q, int64_t ldq,
                                                             uint8_t* __restrict__ sc, int64_t lds) {
  const int lane = threadIdx.x & 63;
  const int64_t chunks = (K + 511) / 512;
  const int64_t task = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (task >= N * chunks) return;  // whole waves: the exchanges below see all 64 lanes
  const int64_t n = task / chunks;
  const int64_t col = (task % chunks) * 512 + lane * 8;
  const bool in = col < K;  // K % 32 == 0: a block's four lanes agree
  float v[8];
  float amax = 0.0f;
  if (in) {
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(W + n * ldw + col);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] = (float)x[e];
      amax = fmaxf(amax, fabsf(v[e]));
    }
  }
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
  if (!in) return;
  const int X = mxfp8_block_exponent(amax);
  if ((lane & 3) == 0) sc[n * lds + col / 32] = (uint8_t)(X + 127);
  const float s = ldexpf(1.0f, X), lim = 448.0f * s;
  const uint32_t w0 = e4m3x4_ocp(v[0], v[1], v[2], v[3], s, lim);
  const uint32_t w1 = e4m3x4_ocp(v[4], v[5], v[6], v[7], s, lim);
  *reinterpret_cast<u32x2*>(q + n * ldq + col) = u32x2{w0, w1};
}

__global__ void mxfp8_dequantize_kernel(const uint8_t* __restrict__ q, int64_t ldq,
                                        const uint8_t* __restrict__ sc, int64_t lds, int64_t N,
                                        int64_t K, bf16* __restrict__ out, int64_t ldo) {
  const int64_t per_row = K / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= N * per_row) return;
  const int64_t n = idx / per_row, c = idx % per_row;
  const u32x2 raw = *reinterpret_cast<const u32x2*>(q + n * ldq + c * 8);
  const uint32_t s = sc[n * lds + (c * 8) / 32];
  const float scale = s == 0xffu ? __uint_as_float(0x7fc00000u)
                                 : (s == 0u ? __uint_as_float(0x00400000u) : __uint_as_float(s << 23));
  uint32_t o[4];
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    o[2 * d] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[d], scale, false));
    o[2 * d + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[d], scale, true));
  }
  *reinterpret_cast<u32x4*>(out + n * ldo + c * 8) = u32x4{o[0], o[1], o[2], o[3]};
}

// One wave per row.
__global__ __launch_bounds__(256) void w8_quantize_kernel(const bf16* __restrict__ W, int64_t ldw,
                                                          int64_t N, int64_t K,
                                                          int8_t* __restrict__ q, int64_t ldq,
                                                          float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const bf16* row = W + n * ldw;
  float amax = 0.0f;
  for (int64_t k = lane * 8; k < K; k += 512) {
    bf16x8 x = *reinterpret_cast<const bf16x8*>(row + k);
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf((float)x[e]));
  }
  amax = wave_max(amax);
  const float s = __fdiv_rn(amax, 127.0f);
  if (lane == 0) scale[n] = s;
  int8_t* qrow = q + n * ldq;
  for (int64_t k = lane * 8; k < K; k += 512) {
    bf16x8 x = *reinterpret_cast<const bf16x8*>(row + k);
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float r = s > 0.0f ? rintf(__fdiv_rn((float)x[e], s)) : 0.0f;
      r = fminf(fmaxf(r, -127.0f), 127.0f);
      const uint32_t b = (uint32_t)((int32_t)r & 0xff);
      if (e < 4) w0 |= b << (8 * e); else w1 |= b << (8 * (e - 4));
    }
    *reinterpret_cast<u32x2*>(qrow + k) = u32x2{w0, w1};
  }
}

__global__ void w8_dequantize_kernel(const int8_t* __restrict__ q, int64_t ldq,
                                     const float* __restrict__ scale, int64_t N, int64_t K,
                                     bf16* __restrict__ out, int64_t ldo) {
  const int64_t per_row = K / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= N * per_row) return;
  const int64_t n = idx / per_row, c = idx % per_row;
  const u32x2 raw = *reinterpret_cast<const u32x2*>(q + n * ldq + c * 8);
  const float s = scale[n];
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int32_t v = (int32_t)(int8_t)((raw[e / 4] >> (8 * (e % 4))) & 0xffu);
    o[e] = (bf16)mul_rn((float)v, s);
  }
  *reinterpret_cast<bf16x8*>(out + n * ldo + c * 8) = o;
}

// E4M3 code -> float, exact: (-1)^s 2^(e-7) (1 + m/8), subnormals (e = 0)
// m 2^-9, 0x7F / 0xFF NaN, no infinities.  The subnormals are formed from
// the integer m rather than an fp32 denormal, so the decode does not depend on
// the denormal mode.
__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
  const uint32_t e = (c >> 3) & 0xFu, m = c & 7u;
  const float mag = e == 0u ? (float)m * 0.001953125f : __uint_as_float(((e + 120u) << 23) | (m << 20));
  const float v = (c & 0x7Fu) == 0x7Fu ? __builtin_nanf("") : mag;
  return (c & 0x80u) ? -v : v;
}

// FP8 checkpoint dequantisation: out[i] = OUT(e4m3(codes[i]) * scale) with the
// product in fp32 (scale = 1 without a weight_scale: exact).  16 codes per
// thread; the tail (n % 16) one code per thread.
template <typename OUT>
__global__ __launch_bounds__(256) void fp8_dequant_kernel(const uint8_t* __restrict__ codes, int64_t n,
                                                          const float* __restrict__ scale,
                                                          OUT* __restrict__ out) {
  const float sc = scale ? *scale : 1.0f;
  const int64_t groups = n / 16;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < groups) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(codes + t * 16);
    float v[16];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int b = 0; b < 4; ++b) v[4 * q + b] = e4m3_to_f32((w[q] >> (8 * b)) & 0xFFu) * sc;
    if constexpr (std::is_same_v<OUT, bf16>) {
      bf16x8 o0, o1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        o0[e] = (bf16)v[e];
        o1[e] = (bf16)v[8 + e];
      }
      *reinterpret_cast<bf16x8*>(out + t * 16) = o0;
      *reinterpret_cast<bf16x8*>(out + t * 16 + 8) = o1;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        *reinterpret_cast<f32x4*>(out + t * 16 + 4 * e) = f32x4{v[4 * e], v[4 * e + 1], v[4 * e + 2], v[4 * e + 3]};
    }
  } else if (t < groups + n % 16) {
    const int64_t i = groups * 16 + (t - groups);
    out[i] = (OUT)(e4m3_to_f32(codes[i]) * sc);
  }
}

}  // namespace ltx

using namespace ltx;

static inline bool a16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

extern "C" int ltx_quantize_mxfp8_bf16(const void* W, int64_t ldw, int64_t N, int64_t K,
                                       uint8_t* q, int64_t ldq, uint8_t* scales, int64_t ld_scale,
                                       void* stream) {
  if (!W || !q || !scales || N < 0 || K < 0) return LTX_ERR_INVALID_ARG;
  if (K % 32) return LTX_ERR_UNSUPPORTED;
  if (ldw < K || ldq < K || ld_scale < K / 32) return LTX_ERR_INVALID_ARG;
  if (!a16(W) || !a16(q) || ldw % 8 || ldq % 8) return LTX_ERR_ALIGNMENT;
  const int64_t tasks = N * ((K + 511) / 512);  // one wave each, four per workgroup
  if (tasks == 0) return LTX_OK;
  if ((tasks + 3) / 4 > INT32_MAX) return LTX_ERR_UNSUPPORTED;
  mxfp8_quantize_kernel<<<(int)((tasks + 3) / 4), 256, 0, (hipStream_t)stream>>>(
      (const bf16*)W, ldw, N, K, q, ldq, scales, ld_scale);
  return ltx_launch_status();
}

extern "C" int ltx_dequantize_mxfp8_bf16(const uint8_t* q, int64_t ldq, const uint8_t* scales,
                                         int64_t ld_scale, int64_t N, int64_t K, void* out,
                                         int64_t ldo, void* stream) {
  if (!q || !scales || !out || N < 0 || K < 0) return LTX_ERR_INVALID_ARG;
  if (K % 32) return LTX_ERR_UNSUPPORTED;
  if (ldq < K || ldo < K || ld_scale < K / 32) return LTX_ERR_INVALID_ARG;
  if (!a16(out) || (uintptr_t)q % 8 || ldq % 8 || ldo % 8) return LTX_ERR_ALIGNMENT;
  const int64_t total = N * (K / 8);
  if (total == 0) return LTX_OK;
  mxfp8_dequantize_kernel<<<(int)((total + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      q, ldq, scales, ld_scale, N, K, (bf16*)out, ldo);
  return ltx_launch_status();
}

extern "C" int ltx_quantize_w8_bf16(const void* W, int64_t ldw, int64_t N, int64_t K, int8_t* q,
                                    int64_t ldq, float* scale, void* stream) {
  if (!W || !q || !scale || N < 0 || K < 0) return LTX_ERR_INVALID_ARG;
  if (K % 8) return LTX_ERR_UNSUPPORTED;
  if (ldw < K || ldq < K) return LTX_ERR_INVALID_ARG;
  if (!a16(W) || (uintptr_t)q % 8 || ldw % 8 || ldq % 8) return LTX_ERR_ALIGNMENT;
  if (N == 0) return LTX_OK;
  w8_quantize_kernel<<<(int)((N + 3) / 4), 256, 0, (hipStream_t)stream>>>((const bf16*)W, ldw, N,
                                                                        K, q, ldq, scale);
  return ltx_launch_status();
}

extern "C" int ltx_dequantize_w8_bf16(const int8_t* q, int64_t ldq, const float* scale, int64_t N,
                                      int64_t K, void* out, int64_t ldo, void* stream) {
  if (!q || !scale || !out || N < 0 || K < 0) return LTX_ERR_INVALID_ARG;
  if (K % 8) return LTX_ERR_UNSUPPORTED;
  if (ldq < K || ldo < K) return LTX_ERR_INVALID_ARG;
  if (!a16(out) || (uintptr_t)q % 8 || ldq % 8 || ldo % 8) return LTX_ERR_ALIGNMENT;
  const int64_t total = N * (K / 8);
  if (total == 0) return LTX_OK;
  w8_dequantize_kernel<<<(int)((total + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      q, ldq, scale, N, K, (bf16*)out, ldo);
  return ltx_launch_status();
}

// FP8 E4M3 checkpoint tensor -> bf16 (out_dtype 0) or fp32 (out_dtype 1).
extern "C" int ltx_dequantize_fp8_e4m3(const uint8_t* codes, int64_t n, const float* scale, void* out,
                                       int out_dtype, void* stream) {
  if (!codes || !out || n < 0) return LTX_ERR_INVALID_ARG;
  if (out_dtype != 0 && out_dtype != 1) return LTX_ERR_UNSUPPORTED;
  if (!a16(codes) || !a16(out) || ((uintptr_t)scale & 3u)) return LTX_ERR_ALIGNMENT;
  const int64_t threads = n / 16 + n % 16;
  if (threads == 0) return LTX_OK;
  if ((threads + 255) / 256 > INT32_MAX) return LTX_ERR_UNSUPPORTED;
  const int blocks = (int)((threads + 255) / 256);
  if (out_dtype == 0)
    fp8_dequant_kernel<bf16><<<blocks, 256, 0, (hipStream_t)stream>>>(codes, n, scale, (bf16*)out);
  else
    fp8_dequant_kernel<float><<<blocks, 256, 0, (hipStream_t)stream>>>(codes, n, scale, (float*)out);
  return ltx_launch_status();
}
