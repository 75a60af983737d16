// Guided sampling on gfx950: the denoised (X0) prediction of a transformer
// pass, the guidance combinations of CFG / CFG-star / STG / modality
// guidance, the GE velocity correction and the Euler step from a denoised
// latent.  Replaces the elementwise math of pipelines/av_pipeline.py:625-757
// and two_stage.py:306-388 around the transformer passes:
//   X0Model.denoise            model/transformer/model.py:1519-1525
//   CFGGuider / CFGStarRescalingGuider / STGGuider / MultiModalGuider
//                              components/guiders.py:10-190
//   GE correction              av_pipeline.py:722-728
//   EulerDiffusionStep.step    components/diffusion_steps.py:19-69
//
// Every operation is an IEEE fp32 operation rounded on its own, in the
// reference's order (python scalars enter as fp32, as MLX casts a weakly typed
// scalar to the array dtype), so the elementwise kernels reproduce the
// reference bit for bit.  The two global reductions (the CFG-star projection
// coefficient and the std-ratio rescale) accumulate exact fp32 products in
// fp64 and round the result once; the reference's fp32 tree sum differs from
// it by its own summation error only.
//
// The latents are small ((T, 128) per modality: 0.4 M elements for 3456
// video tokens), so these are plain grid-stride kernels over 8-element
// vectors; the reductions run in one workgroup (no atomics, deterministic).

#include "ltx_common.h"

namespace ltx {

constexpr int kGuideThreads = 256;
constexpr int kStatsThreads = 1024;

__device__ __forceinline__ float div_rn(float a, float b) {
#pragma clang fp contract(off)
  return __fdiv_rn(a, b);
}

__device__ __forceinline__ void load8f(const float* p, float* v) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = a[i];
    v[4 + i] = b[i];
  }
}

__device__ __forceinline__ void store8f(float* p, const float* v) {
  *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
}

__device__ __forceinline__ void load8b(const bf16* p, float* v) {
  const bf16x8 a = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)a[i];
}

__device__ __forceinline__ void store8b(bf16* p, const float* v) {
  bf16x8 a;
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = (bf16)v[i];
  *reinterpret_cast<bf16x8*>(p) = a;
}

// ---- X0: latent - sigma * velocity -----------------------------------------
__global__ __launch_bounds__(kGuideThreads) void x0_kernel(const bf16* latent, const bf16* velocity,
                                                           float sigma, float* out, int64_t n) {
  const int64_t nvec = n / 8;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nvec; i += stride) {
    float x[8], v[8], o[8];
    load8b(latent + i * 8, x);
    load8b(velocity + i * 8, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = sub_rn(x[e], mul_rn(sigma, v[e]));
    store8f(out + i * 8, o);
  }
  if (blockIdx.x == 0 && threadIdx.x < (n & 7)) {
    const int64_t e = nvec * 8 + threadIdx.x;
    out[e] = sub_rn((float)latent[e], mul_rn(sigma, (float)velocity[e]));
  }
}

// ---- guidance combination ---------------------------------------------------
struct GuideArgs {
  const float* base;
  const float* term[3];
  float c[3];
  const float* coef0;   // device scalar multiplying term[0] (CFG-star), or null
  const float* factor;  // device scalar multiplying the result (std rescale), or null
  int delta_only;       // out = c0 * (base - coef0 * term0)
  float* out;
  int64_t n;
};

__device__ __forceinline__ float guide_one(const GuideArgs& g, float base, const float* t, float coef,
                                           float factor) {
  if (g.delta_only) {
    const float u = g.coef0 ? mul_rn(coef, t[0]) : t[0];
    return mul_rn(g.c[0], sub_rn(base, u));
  }
  float pred = base;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    if (!g.term[k]) continue;
    const float u = (k == 0 && g.coef0) ? mul_rn(coef, t[k]) : t[k];
    pred = add_rn(pred, mul_rn(g.c[k], sub_rn(base, u)));
  }
  if (g.factor) pred = mul_rn(pred, factor);
  return pred;
}

__global__ __launch_bounds__(kGuideThreads) void guide_kernel(GuideArgs g) {
  const float coef = g.coef0 ? *g.coef0 : 1.0f;
  const float factor = g.factor ? *g.factor : 1.0f;
  const int64_t nvec = g.n / 8;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nvec; i += stride) {
    float b[8], t[3][8] = {}, o[8];
    load8f(g.base + i * 8, b);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      if (g.term[k]) load8f(g.term[k] + i * 8, t[k]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float te[3] = {t[0][e], t[1][e], t[2][e]};
      o[e] = guide_one(g, b[e], te, coef, factor);
    }
    store8f(g.out + i * 8, o);
  }
  if (blockIdx.x == 0 && threadIdx.x < (g.n & 7)) {
    const int64_t e = nvec * 8 + threadIdx.x;
    float te[3] = {0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 3; ++k)
      if (g.term[k]) te[k] = g.term[k][e];
    g.out[e] = guide_one(g, g.base[e], te, coef, factor);
  }
}

// ---- global statistics --------------------------------------------------------
// mode LTX_GUIDE_STATS_PROJECTION: out = sum(a*b) / (sum(b*b) + 1e-8)
//   (projection_coef(to_project=a, project_onto=b), guiders.py:175-190)
// mode LTX_GUIDE_STATS_STD_RATIO: out = r * (std(a) / std(b)) + rc, rc = 1 - r
//   rounded once from double on the host, std(x) = sqrt(var(x) + 1e-8)
//   (MultiModalGuider rescale, guiders.py:155-161)
__device__ __forceinline__ double block_sum(double v, double* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  double s = 0.0;
  for (int w = 0; w < (int)(blockDim.x / kWave); ++w) s += red[w];
  return s;
}

__global__ __launch_bounds__(kStatsThreads) void guide_stats_kernel(const float* a, const float* b, int64_t n,
                                                                   int mode, float r, float rc, float* out) {
  __shared__ double red[kStatsThreads / kWave];
  double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    const float x = a[i], y = b[i];
    if (mode == LTX_GUIDE_STATS_PROJECTION) {
      s0 += (double)mul_rn(x, y);
      s1 += (double)mul_rn(y, y);
    } else {
      s0 += (double)x;
      s1 += (double)x * (double)x;
      s2 += (double)y;
      s3 += (double)y * (double)y;
    }
  }
  s0 = block_sum(s0, red);
  s1 = block_sum(s1, red);
  if (mode == LTX_GUIDE_STATS_PROJECTION) {
    if (threadIdx.x == 0) out[0] = div_rn((float)s0, add_rn((float)s1, 1e-8f));
    return;
  }
  s2 = block_sum(s2, red);
  s3 = block_sum(s3, red);
  if (threadIdx.x == 0) {
    const double inv = 1.0 / (double)n;
    const double ma = s0 * inv, mb = s2 * inv;
    const float va = (float)fmax(s1 * inv - ma * ma, 0.0);
    const float vb = (float)fmax(s3 * inv - mb * mb, 0.0);
    const float sa = sqrtf(add_rn(va, 1e-8f));
    const float sb = sqrtf(add_rn(vb, 1e-8f));
    const float f = div_rn(sa, sb);
    out[0] = add_rn(mul_rn(r, f), rc);
  }
}

// ---- GE velocity correction (in place on the denoised latent) ---------------
__global__ __launch_bounds__(kGuideThreads) void ge_kernel(const bf16* latent, float* denoised, float* prev,
                                                           int prev_valid, float sigma, float gamma,
                                                           int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float x = (float)latent[i];
    const float d = denoised[i];
    const float cur = div_rn(sub_rn(x, d), sigma);
    if (prev_valid) {
      const float p = prev[i];
      const float total = add_rn(mul_rn(gamma, sub_rn(cur, p)), p);
      denoised[i] = sub_rn(x, mul_rn(total, sigma));
    }
    prev[i] = cur;
  }
}

// ---- Euler step from a denoised latent ----------------------------------------
__global__ __launch_bounds__(kGuideThreads) void euler_denoised_kernel(const bf16* sample, const float* denoised,
                                                                       float ratio, bf16* out, int64_t n) {
  const int64_t nvec = n / 8;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nvec; i += stride) {
    float x[8], d[8], o[8];
    load8b(sample + i * 8, x);
    load8f(denoised + i * 8, d);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = add_rn(d[e], mul_rn(ratio, sub_rn(x[e], d[e])));
    store8b(out + i * 8, o);
  }
  if (blockIdx.x == 0 && threadIdx.x < (n & 7)) {
    const int64_t e = nvec * 8 + threadIdx.x;
    const float x = (float)sample[e], d = denoised[e];
    out[e] = (bf16)add_rn(d, mul_rn(ratio, sub_rn(x, d)));
  }
}

static int grid_for(int64_t n) {
  int64_t blocks = (n / 8 + kGuideThreads - 1) / kGuideThreads;
  if (blocks > 2048) blocks = 2048;
  return blocks < 1 ? 1 : (int)blocks;
}

}  // namespace ltx

using namespace ltx;

static inline bool a16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

extern "C" int ltx_x0_from_velocity_f32(const void* latent, const void* velocity, float sigma, float* out,
                                        int64_t n, void* stream) {
  if (n < 0 || !latent || !velocity || !out) return LTX_ERR_INVALID_ARG;
  if (!a16(latent) || !a16(velocity) || !a16(out)) return LTX_ERR_ALIGNMENT;
  if (n == 0) return LTX_OK;
  x0_kernel<<<grid_for(n), kGuideThreads, 0, (hipStream_t)stream>>>((const bf16*)latent, (const bf16*)velocity,
                                                                    sigma, out, n);
  return ltx_launch_status();
}

extern "C" int ltx_guidance_f32(const float* base, const float* term0, const float* term1, const float* term2,
                                float c0, float c1, float c2, const float* coef0, const float* factor,
                                float* out, int64_t n, int flags, void* stream) {
  if (n < 0 || !base || !out) return LTX_ERR_INVALID_ARG;
  if (flags & ~LTX_GUIDE_DELTA_ONLY) return LTX_ERR_INVALID_ARG;
  if ((flags & LTX_GUIDE_DELTA_ONLY) && (!term0 || term1 || term2 || factor)) return LTX_ERR_INVALID_ARG;
  if (coef0 && !term0) return LTX_ERR_INVALID_ARG;
  const float* ts[3] = {term0, term1, term2};
  if (!a16(base) || !a16(out)) return LTX_ERR_ALIGNMENT;
  for (const float* t : ts)
    if (t && !a16(t)) return LTX_ERR_ALIGNMENT;
  if ((coef0 && ((uintptr_t)coef0 & 3u)) || (factor && ((uintptr_t)factor & 3u))) return LTX_ERR_ALIGNMENT;
  if (n == 0) return LTX_OK;
  GuideArgs g;
  g.base = base;
  for (int k = 0; k < 3; ++k) g.term[k] = ts[k];
  g.c[0] = c0;
  g.c[1] = c1;
  g.c[2] = c2;
  g.coef0 = coef0;
  g.factor = factor;
  g.delta_only = (flags & LTX_GUIDE_DELTA_ONLY) != 0;
  g.out = out;
  g.n = n;
  guide_kernel<<<grid_for(n), kGuideThreads, 0, (hipStream_t)stream>>>(g);
  return ltx_launch_status();
}

extern "C" int ltx_guidance_stats_f32(const float* a, const float* b, int64_t n, int mode, float rescale,
                                      float one_minus_rescale, float* out, void* stream) {
  if (n <= 0 || !a || !b || !out) return LTX_ERR_INVALID_ARG;
  if (mode != LTX_GUIDE_STATS_PROJECTION && mode != LTX_GUIDE_STATS_STD_RATIO) return LTX_ERR_INVALID_ARG;
  if (((uintptr_t)a & 3u) || ((uintptr_t)b & 3u) || ((uintptr_t)out & 3u)) return LTX_ERR_ALIGNMENT;
  guide_stats_kernel<<<1, kStatsThreads, 0, (hipStream_t)stream>>>(a, b, n, mode, rescale,
                                                                   one_minus_rescale, out);
  return ltx_launch_status();
}

extern "C" int ltx_ge_correct_f32(const void* latent, float* denoised, float* prev_velocity, int prev_valid,
                                  float sigma, float gamma, int64_t n, void* stream) {
  if (n < 0 || !latent || !denoised || !prev_velocity) return LTX_ERR_INVALID_ARG;
  if (!(sigma > 0.0f)) return LTX_ERR_INVALID_ARG;
  if (n == 0) return LTX_OK;
  int64_t blocks = (n + kGuideThreads - 1) / kGuideThreads;
  if (blocks > 2048) blocks = 2048;
  ge_kernel<<<(int)blocks, kGuideThreads, 0, (hipStream_t)stream>>>((const bf16*)latent, denoised, prev_velocity,
                                                                    prev_valid, sigma, gamma, n);
  return ltx_launch_status();
}

extern "C" int ltx_euler_step_bf16(const void* sample, const float* denoised, float ratio, void* out, int64_t n,
                                   void* stream) {
  if (n < 0 || !sample || !denoised || !out) return LTX_ERR_INVALID_ARG;
  if (!a16(sample) || !a16(denoised) || !a16(out)) return LTX_ERR_ALIGNMENT;
  if (n == 0) return LTX_OK;
  euler_denoised_kernel<<<grid_for(n), kGuideThreads, 0, (hipStream_t)stream>>>(
      (const bf16*)sample, denoised, ratio, (bf16*)out, n);
  return ltx_launch_status();
}
