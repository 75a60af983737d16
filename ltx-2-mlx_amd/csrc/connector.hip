// Text-conditioning features for the LTX-2.3 connectors
// (model/text_encoder/feature_extractor.py:9-79, GemmaFeaturesExtractorV2):
// per token and per Gemma layer, the hidden state (D = 3840) is RMS-normalised
// over D, padding tokens are zeroed, and the result is scaled by
// sqrt(inner_dim / D) for the video and the audio aggregate embedding.  The
// reference evaluates this in bf16 array arithmetic, so every step rounds to
// bf16 (the python-float constants 1e-6 and the two scales enter as bf16):
//   sq   = bf16(x * x)              mean = bf16(sum(sq) / D)      (fp32 sum)
//   r    = bf16(1 / sqrt(bf16(mean + eps)))
//   y    = mask ? bf16(x * r) : 0
//   out  = bf16(y * scale)          (one output per scale)
// Output rows are written layer-major, feature index l * D + d; the aggregate
// embedding weights are permuted to that order once at load time (the
// reference's index is d * L + l), so each workgroup writes D contiguous
// values per output instead of a stride-L scatter.
//
// One workgroup per (token, layer); D / 8 vector lanes of work for 256
// threads, one block reduction.

#include "ltx_common.h"

namespace {

using namespace ltx;

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void gemma_features_kernel(
    const bf16* hidden, int64_t layer_stride, int64_t row_stride, int L, int D, const int32_t* mask,
    float eps_bf, float scale_v, float scale_a, bf16* out_v, bf16* out_a, int64_t out_stride) {
  __shared__ float red[kThreads / kWave];
  const int l = blockIdx.x % L;
  const int64_t t = blockIdx.x / L;
  const bf16* x = hidden + (int64_t)l * layer_stride + t * row_stride;
  const int nvec = D / 8;
  float s = 0.0f;
  for (int i = threadIdx.x; i < nvec; i += kThreads) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(x + i * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float xf = (float)v[e];
      s += round_bf(mul_rn(xf, xf));
    }
  }
  s = wave_sum(s);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = s;
  __syncthreads();
  float sum = 0.0f;
#pragma unroll
  for (int w = 0; w < kThreads / kWave; ++w) sum += red[w];
  const float mean = round_bf(__fdiv_rn(sum, (float)D));
  const float var = round_bf(add_rn(mean, eps_bf));
  const float r = round_bf(__fdiv_rn(1.0f, sqrtf(var)));
  const bool keep = mask == nullptr || mask[t] != 0;
  bf16* ov = out_v + t * out_stride + (int64_t)l * D;
  bf16* oa = out_a + t * out_stride + (int64_t)l * D;
  for (int i = threadIdx.x; i < nvec; i += kThreads) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(x + i * 8);
    bf16x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float y = keep ? round_bf(mul_rn((float)v[e], r)) : 0.0f;
      a[e] = (bf16)mul_rn(y, scale_v);
      b[e] = (bf16)mul_rn(y, scale_a);
    }
    *reinterpret_cast<bf16x8*>(ov + i * 8) = a;
    *reinterpret_cast<bf16x8*>(oa + i * 8) = b;
  }
}

}  // namespace

extern "C" int ltx_gemma_features_bf16(const void* hidden, int64_t layers, int64_t tokens, int64_t dim,
                                       int64_t layer_stride, int64_t row_stride, const int32_t* mask,
                                       float eps, float scale_video, float scale_audio, void* out_video,
                                       void* out_audio, int64_t out_stride, void* stream) {
  if (!hidden || !out_video || !out_audio || layers <= 0 || tokens < 0 || dim <= 0) return LTX_ERR_INVALID_ARG;
  if (dim % 8 || dim > 65536) return LTX_ERR_UNSUPPORTED;
  if (row_stride < dim || layer_stride < tokens * row_stride || out_stride < layers * dim)
    return LTX_ERR_INVALID_ARG;
  if (((uintptr_t)hidden | (uintptr_t)out_video | (uintptr_t)out_audio) & 15u) return LTX_ERR_ALIGNMENT;
  if ((row_stride | layer_stride | out_stride) & 7) return LTX_ERR_ALIGNMENT;
  if ((uintptr_t)mask & 3u) return LTX_ERR_ALIGNMENT;
  if (tokens == 0) return LTX_OK;
  if (tokens * layers > INT32_MAX) return LTX_ERR_UNSUPPORTED;
  gemma_features_kernel<<<(int)(tokens * layers), kThreads, 0, (hipStream_t)stream>>>(
      (const bf16*)hidden, layer_stride, row_stride, (int)layers, (int)dim, mask, eps, scale_video, scale_audio,
      (bf16*)out_video, (bf16*)out_audio, out_stride);
  return ltx_launch_status();
}
