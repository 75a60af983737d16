// Latent layout conversions at the loop's I/O boundary: the reference's
// patchifiers (components/patchifiers.py:52-124, :327-374) between the VAE's
// latent layouts and the transformer's token rows, batch 1:
//   video  (C, F, H, W)  <-> (F*H*W, C)        swap of (C, N) with N = F*H*W
//   audio  (C, T, M)     <-> (T, C*M)          swap of (C, T) keeping M inner
// Both are the swap of the two outer axes of an (A, B, R) array:
//   out[b, a, r] = in[a, b, r].
// The latents are at most a few MB and convert once per generation, so the
// kernel is a plain grid-stride loop over output elements (coalesced writes,
// strided reads).

#include "ltx_common.h"

namespace {

template <typename T>
__global__ __launch_bounds__(256) void swap_axes_kernel(const T* in, int64_t A, int64_t B, int64_t R, T* out) {
  const int64_t n = A * B * R;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < n; o += stride) {
    const int64_t r = o % R;
    const int64_t ba = o / R;
    const int64_t a = ba % A;
    const int64_t b = ba / A;
    out[o] = in[(a * B + b) * R + r];
  }
}

}  // namespace

extern "C" int ltx_swap_axes(const void* in, int64_t A, int64_t B, int64_t R, int elem_bytes, void* out,
                             void* stream) {
  if (!in || !out || A < 0 || B < 0 || R < 0) return LTX_ERR_INVALID_ARG;
  if (in == out) return LTX_ERR_INVALID_ARG;
  if (elem_bytes != 2 && elem_bytes != 4) return LTX_ERR_UNSUPPORTED;
  if (((uintptr_t)in | (uintptr_t)out) & (uintptr_t)(elem_bytes - 1)) return LTX_ERR_ALIGNMENT;
  const int64_t n = A * B * R;
  if (n == 0) return LTX_OK;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (elem_bytes == 2)
    swap_axes_kernel<uint16_t><<<(int)blocks, 256, 0, (hipStream_t)stream>>>((const uint16_t*)in, A, B, R,
                                                                            (uint16_t*)out);
  else
    swap_axes_kernel<uint32_t><<<(int)blocks, 256, 0, (hipStream_t)stream>>>((const uint32_t*)in, A, B, R,
                                                                            (uint32_t*)out);
  return ltx_launch_status();
}
