// Host-side checks of the C ABI, built against the library compiled with
// AddressSanitizer on its host code (build.py).  The first part drives every
// entry point through its argument-validation paths, which return before any
// device work -- null pointers, unsupported shapes, misaligned pointers or
// strides, empty problems, workspace and padding helpers.  The second part,
// run only where no GPU is present, makes valid calls at the workloads'
// shapes: each entry point then runs all of its host code -- tile and kernel
// choice, split counts, workspace and scratch arithmetic, launch geometry --
// up to the kernel launch, which the HIP runtime refuses for want of a
// device (LTX_ERR_HIP), so AddressSanitizer sees the launch planning too.
// Device pointers are fake, 16-byte aligned addresses that the library must
// never dereference on the host.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <initializer_list>

#include "../../include/ltx_hip.h"

// the HIP runtime's device count (C ABI of libamdhip64, which the library links)
extern "C" int hipGetDeviceCount(int* count);

static int failures = 0;

static void expect(const char* what, int64_t got, int64_t want) {
  if (got != want) {
    std::printf("FAIL %s: got %lld, want %lld\n", what, (long long)got, (long long)want);
    ++failures;
  }
}
#define EXPECT(call, want) expect(#call, (int64_t)(call), (int64_t)(want))

int main(int argc, char** argv) {
  if (argc > 1 && std::strcmp(argv[1], "--overflow-selftest") == 0) {
    // proves the sanitizer is live: one byte past a heap block
    volatile char* p = new char[8];
    const int r = p[argc + 6];
    delete[] p;
    return r;
  }
  void* d = reinterpret_cast<void*>(uintptr_t(0x10000));   // aligned fake device address
  void* m = reinterpret_cast<void*>(uintptr_t(0x10008));   // 8-byte aligned only
  const float* fd = static_cast<const float*>(d);
  float* fo = static_cast<float*>(d);
  const int32_t* id = static_cast<const int32_t*>(d);

  // status strings and version
  for (int s = -6; s <= 1; ++s) EXPECT(std::strlen(ltx_status_string(s)) > 0, 1);
  EXPECT(std::strcmp(ltx_status_string(LTX_OK), "ok"), 0);
  EXPECT(ltx_version() > 0, 1);
  EXPECT(ltx_device_clock_stamp(nullptr, nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_device_clock_stamp(reinterpret_cast<uint64_t*>(static_cast<char*>(m) + 4), nullptr), LTX_ERR_ALIGNMENT);

  // row kernels
  EXPECT(ltx_adaln_norm_fused_bf16(nullptr, 4096, fd, fd, d, 4096, 4, 4096, 1e-6f, 0, nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_adaln_norm_fused_bf16(d, 3584, fd, fd, d, 3584, 4, 3584, 1e-6f, 0, nullptr), LTX_ERR_UNSUPPORTED);
  EXPECT(ltx_adaln_norm_fused_bf16(m, 4096, fd, fd, d, 4096, 4, 4096, 1e-6f, 0, nullptr), LTX_ERR_ALIGNMENT);
  EXPECT(ltx_adaln_norm_fused_bf16(d, 4096, fd, fd, d, 4096, 0, 4096, 1e-6f, 0, nullptr), LTX_OK);
  EXPECT(ltx_adaln_norm_fused2_bf16(d, 4096, fd, fd, d, 4096, fd, fd, nullptr, 4096, 4, 4096, 1e-6f, 0, nullptr),
         LTX_ERR_INVALID_ARG);
  EXPECT(ltx_adaln_norm_fused2_bf16(d, 4096, fd, fd, d, 4096, fd, nullptr, d, 4096, 4, 4096, 1e-6f, 0, nullptr),
         LTX_ERR_INVALID_ARG);
  EXPECT(ltx_adaln_norm_fused2_bf16(d, 4096, fd, fd, d, 4096, fd, fd, m, 4096, 4, 4096, 1e-6f, 0, nullptr),
         LTX_ERR_ALIGNMENT);
  EXPECT(ltx_adaln_norm_fused2_bf16(d, 4096, fd, fd, d, 4096, fd, fd, d, 4096, 0, 4096, 1e-6f, 0, nullptr), LTX_OK);
  EXPECT(ltx_gated_add_fused_bf16(nullptr, 4096, d, 4096, fd, d, 4096, 4, 4096, 0, nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_gated_add_fused_bf16(d, 4096, d, 4096, fd, d, 4096, 4, 1000, 0, nullptr), LTX_ERR_UNSUPPORTED);
  EXPECT(ltx_gated_add_fused_bf16(d, 4096, d, 4096, fd, d, 4096, 0, 4096, 0, nullptr), LTX_OK);
  EXPECT(ltx_qknorm_rope_bf16(nullptr, 4096, 4, fd, fd, fd, d, 4096, 4, fd, fd, fd, 4096, 128, 1e-6f, nullptr),
         LTX_ERR_INVALID_ARG);
  EXPECT(ltx_qknorm_rope_bf16(d, 4096, 4, fd, fd, fd, d, 4096, 4, fd, fd, fd, 1536, 128, 1e-6f, nullptr),
         LTX_ERR_UNSUPPORTED);
  EXPECT(ltx_qknorm_rope_bf16(d, 4096, 4, fd, fd, nullptr, d, 4096, 4, fd, fd, fd, 4096, 128, 1e-6f, nullptr),
         LTX_ERR_INVALID_ARG);
  EXPECT(ltx_qknorm_rope_bf16(d, 4096, 0, fd, fd, fd, d, 4096, 0, fd, fd, fd, 4096, 128, 1e-6f, nullptr), LTX_OK);
  EXPECT(ltx_qknorm_rope_axes_bf16(d, 4096, 4, fd, fd, fd, id, 4, 49, d, 4096, 4, fd, fd, fd, id, 3, 49, 4096, 128,
                                   1e-6f, nullptr), LTX_ERR_INVALID_ARG);  // 4 axes
  EXPECT(ltx_qknorm_rope_axes_bf16(d, 4096, 4, fd, nullptr, nullptr, id, 3, 49, d, 4096, 4, fd, fd, fd, id, 3, 49,
                                   4096, 128, 1e-6f, nullptr), LTX_ERR_INVALID_ARG);  // index without tables
  EXPECT(ltx_qknorm_rope_axes_bf16(d, 4096, 0, fd, fd, fd, id, 3, 49, d, 4096, 0, fd, fd, fd, id, 3, 49, 4096, 128,
                                   1e-6f, nullptr), LTX_OK);
  EXPECT(ltx_output_norm_modulate_bf16(nullptr, 4096, fd, fd, d, 4096, 4, 4096, 1e-6f, nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_euler_x0_step_bf16(nullptr, d, 1.0f, 0.5f, d, 16, nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_timestep_embedding_f32(nullptr, 4, 1000.0f, fo, 256, nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_gemv_f32_bf16w(nullptr, 1, 256, d, fd, fo, 64, 0, nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_broadcast_add_f32(nullptr, fd, fo, 2, 64, nullptr), LTX_ERR_INVALID_ARG);

  // GEMMs
  EXPECT(ltx_gemm_bf16(nullptr, 64, d, 64, fd, d, 64, 4, 64, 64, 0, nullptr, 0, nullptr, 64, nullptr),
         LTX_ERR_INVALID_ARG);
  EXPECT(ltx_gemm_bf16(d, 96, d, 96, nullptr, d, 64, 4, 64, 96, 0, nullptr, 0, nullptr, 64, nullptr),
         LTX_ERR_UNSUPPORTED);  // K % 64
  EXPECT(ltx_gemm_bf16(m, 64, d, 64, nullptr, d, 64, 4, 64, 64, 0, nullptr, 0, nullptr, 64, nullptr),
         LTX_ERR_ALIGNMENT);
  EXPECT(ltx_gemm_bf16(d, 64, d, 64, nullptr, d, 64, 0, 64, 64, 0, nullptr, 0, nullptr, 64, nullptr), LTX_OK);
  EXPECT(ltx_gemm_bf16(d, 64, d, 64, nullptr, d, 64, 4, 64, 64, 2, nullptr, 0, nullptr, 64, nullptr),
         LTX_ERR_INVALID_ARG);  // residual epilogue without residual
  EXPECT(ltx_gemm_w8a16_bf16(d, 64, static_cast<const int8_t*>(d), 64, nullptr, nullptr, d, 64, 4, 64, 64, 0,
                             nullptr, 0, nullptr, 64, nullptr), LTX_ERR_INVALID_ARG);  // no scales
  EXPECT(ltx_gemm_mxfp8_bf16(d, 128, static_cast<const uint8_t*>(d), 128, static_cast<const uint8_t*>(d), 5,
                             nullptr, d, 64, 4, 64, 128, 0, nullptr, 0, nullptr, 64, nullptr),
         LTX_ERR_ALIGNMENT);  // scale rows not 4-byte multiples
  EXPECT(ltx_gemm_splitk_workspace_bytes(68, 2048, 4), 4ll * 68 * 2048 * 4);
  EXPECT(ltx_gemm_splitk_bf16(d, 2048, d, 2048, nullptr, d, 2048, 4, 2048, 2048, 0, nullptr, 0, nullptr, 2048, 4,
                              fo, 16, nullptr), LTX_ERR_INVALID_ARG);  // workspace too small
  EXPECT(ltx_gemm_splitk_w8a16_bf16(d, 2048, static_cast<const int8_t*>(d), 2048, fd, nullptr, d, 2048, 4, 2048,
                                    2048, 0, nullptr, 0, nullptr, 2048, 0, fo, 1 << 20, nullptr),
         LTX_ERR_INVALID_ARG);  // zero splits
  EXPECT(ltx_gemm_splitk_mxfp8_bf16(nullptr, 2048, static_cast<const uint8_t*>(d), 2048,
                                    static_cast<const uint8_t*>(d), 64, nullptr, d, 2048, 4, 2048, 2048, 0, nullptr,
                                    0, nullptr, 2048, 4, fo, 1 << 20, nullptr), LTX_ERR_INVALID_ARG);

  // weight formats
  EXPECT(ltx_quantize_mxfp8_bf16(nullptr, 64, 4, 64, static_cast<uint8_t*>(d), 64, static_cast<uint8_t*>(d), 4,
                                 nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_dequantize_mxfp8_bf16(nullptr, 64, static_cast<const uint8_t*>(d), 4, 4, 64, d, 64, nullptr),
         LTX_ERR_INVALID_ARG);
  EXPECT(ltx_quantize_w8_bf16(nullptr, 64, 4, 64, static_cast<int8_t*>(d), 64, fo, nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_dequantize_w8_bf16(nullptr, 64, fd, 4, 64, d, 64, nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_dequantize_fp8_e4m3(nullptr, 16, nullptr, d, 0, nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_dequantize_fp8_e4m3(static_cast<const uint8_t*>(d), 16, nullptr, d, 2, nullptr), LTX_ERR_UNSUPPORTED);
  EXPECT(ltx_dequantize_fp8_e4m3(static_cast<const uint8_t*>(d), 0, nullptr, d, 0, nullptr), LTX_OK);

  // guidance, sidecar layout, text features
  EXPECT(ltx_x0_from_velocity_f32(nullptr, d, 0.5f, fo, 16, nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_guidance_f32(nullptr, fd, nullptr, nullptr, 1.0f, 0.0f, 0.0f, nullptr, nullptr, fo, 16, 0, nullptr),
         LTX_ERR_INVALID_ARG);
  EXPECT(ltx_guidance_stats_f32(nullptr, fd, 16, 0, 0.7f, 0.3f, fo, nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_ge_correct_f32(nullptr, fo, fo, 0, 0.5f, 0.5f, 16, nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_euler_step_bf16(nullptr, fd, 0.5f, d, 16, nullptr), LTX_ERR_INVALID_ARG);
  EXPECT(ltx_gemma_features_bf16(nullptr, 49, 16, 3840, 16 * 3840, 3840, id, 1e-6f, 1.0f, 1.0f, d, d, 3840, nullptr),
         LTX_ERR_INVALID_ARG);
  EXPECT(ltx_swap_axes(nullptr, 2, 3, 4, 2, d, nullptr), LTX_ERR_INVALID_ARG);

  // attention
  EXPECT(ltx_attn_vt_padded_len(1), 64);
  EXPECT(ltx_attn_vt_padded_len(3456), 3456);
  EXPECT(ltx_attn_vt_padded_len(3457), 3520);
  EXPECT(ltx_flash_attn_v_bf16(d, 4096, d, 4096, d, 4096, d, 4096, nullptr, 0, 4, 4, 32, 96, 0.1f, nullptr),
         LTX_ERR_UNSUPPORTED);
  EXPECT(ltx_flash_attn_v_bf16(d, 4096, d, 4096, d, 2048, d, 4096, nullptr, 0, 4, 4, 32, 128, 0.1f, nullptr),
         LTX_ERR_INVALID_ARG);
  EXPECT(ltx_flash_attn_v_bf16(d, 4096, d, 4096, m, 4096, d, 4096, nullptr, 0, 4, 4, 32, 128, 0.1f, nullptr),
         LTX_ERR_ALIGNMENT);
  EXPECT(ltx_flash_attn_v_bf16(d, 4096, d, 4096, d, 4096, d, 4096, nullptr, 0, 0, 4, 32, 128, 0.1f, nullptr),
         LTX_OK);
  EXPECT(ltx_flash_attn_bf16(d, 4096, d, 4096, d, 32, d, 4096, nullptr, 0, 4, 4, 32, 128, 0.1f, nullptr),
         LTX_ERR_INVALID_ARG);  // tk_pad below the padded length
  EXPECT(ltx_attn_transpose_v_bf16(d, 4096, 4, 32, 96, d, 64, nullptr), LTX_ERR_UNSUPPORTED);
  EXPECT(ltx_attn_splitkv_workspace_bytes(68, 32, 64, 16) > 0, 1);
  // query norm inside the attention kernel: row statistics and table forms
  EXPECT(ltx_flash_attn_qnorm_v_bf16(d, 4096, d, 4096, d, 4096, d, 4096, nullptr, 0, 4, 4, 32, 128, 0.1f, nullptr,
                                     64, 64, fd, 1e-6f, nullptr, nullptr, nullptr, 1, 0, nullptr),
         LTX_ERR_INVALID_ARG);  // no row statistics
  EXPECT(ltx_flash_attn_qnorm_v_bf16(d, 4096, d, 4096, d, 4096, d, 4096, nullptr, 0, 4, 4, 32, 128, 0.1f, fd, 68,
                                     68, fd, 1e-6f, nullptr, nullptr, nullptr, 1, 0, nullptr),
         LTX_ERR_INVALID_ARG);  // more than 64 partials
  EXPECT(ltx_flash_attn_qnorm_v_bf16(d, 4096, d, 4096, d, 4096, d, 4096, nullptr, 0, 4, 4, 32, 128, 0.1f,
                                     static_cast<const float*>(m), 64, 64, fd, 1e-6f, nullptr, nullptr, nullptr, 1, 0,
                                     nullptr),
         LTX_ERR_ALIGNMENT);
  EXPECT(ltx_flash_attn_qnorm_v_bf16(d, 4096, d, 4096, d, 4096, d, 4096, nullptr, 0, 4, 4, 32, 128, 0.1f, fd, 64,
                                     64, fd, 1e-6f, fd, nullptr, nullptr, 1, 0, nullptr),
         LTX_ERR_INVALID_ARG);  // cos without sin
  EXPECT(ltx_flash_attn_qnorm_v_bf16(d, 4096, d, 4096, d, 4096, d, 4096, nullptr, 0, 4, 4, 32, 128, 0.1f, fd, 64,
                                     64, fd, 1e-6f, fd, fd, nullptr, 1, 3, nullptr),
         LTX_ERR_INVALID_ARG);  // per-query table shorter than Tq
  EXPECT(ltx_flash_attn_qnorm_v_bf16(d, 4096, d, 4096, d, 4096, d, 4096, nullptr, 0, 4, 4, 32, 128, 0.1f, fd, 64,
                                     64, fd, 1e-6f, fd, fd, id, 4, 10, nullptr),
         LTX_ERR_INVALID_ARG);  // more than three axes
  EXPECT(ltx_flash_attn_qnorm_v_bf16(d, 4096, d, 4096, d, 4096, d, 4096, nullptr, 0, 0, 4, 32, 128, 0.1f, fd, 64,
                                     64, fd, 1e-6f, nullptr, nullptr, nullptr, 1, 0, nullptr),
         LTX_OK);
  EXPECT(ltx_gemm_rowss_bf16(3, d, 4096, d, 4096, nullptr, 0, fd, d, 4128, 4, 4128, 4096, 0, 4096, fo, 64, 4096,
                             nullptr), LTX_ERR_INVALID_ARG);  // no such weight format
  EXPECT(ltx_gemm_rowss_bf16(0, d, 4096, d, 4096, nullptr, 0, fd, d, 4128, 4, 4128, 4096, 1, 4096, fo, 64, 4096,
                             nullptr), LTX_ERR_INVALID_ARG);  // GELU epilogue
  EXPECT(ltx_gemm_rowss_bf16(0, d, 4096, d, 4096, nullptr, 0, fd, d, 4128, 4, 4128, 4096, 1 << 8, 4096, fo, 64,
                             4096, nullptr), LTX_ERR_UNSUPPORTED);  // a 4-wave tile
  EXPECT(ltx_gemm_rowss_bf16(0, d, 4096, d, 4096, nullptr, 0, fd, d, 4128, 4, 4128, 4096, 0, 4096, fo, 64, 4000,
                             nullptr), LTX_ERR_INVALID_ARG);  // not whole 64-column slices
  EXPECT(ltx_gemm_rowss_bf16(0, d, 4096, d, 4096, nullptr, 0, fd, d, 4128, 4, 4128, 4096, 0, 4096, fo, 32, 4096,
                             nullptr), LTX_ERR_INVALID_ARG);  // row stride below the slice count
  EXPECT(ltx_gemm_rowss_bf16(0, d, 4096, d, 4096, nullptr, 0, fd, d, 4128, 4, 4128, 4096, 0, 4096,
                             reinterpret_cast<float*>(static_cast<char*>(m) + 2), 64, 4096, nullptr),
         LTX_ERR_ALIGNMENT);
  EXPECT(ltx_gemm_rowss_bf16(2, d, 4096, d, 4096, nullptr, 128, fd, d, 4128, 4, 4128, 4096, 0, 4096, fo, 64, 4096,
                             nullptr), LTX_ERR_INVALID_ARG);  // MXFP8 without scales
  EXPECT(ltx_gemm_rowss_bf16(0, d, 4096, d, 4096, nullptr, 0, fd, d, 4128, 0, 4128, 4096, 0, 4096, fo, 64, 4096,
                             nullptr), LTX_OK);
  EXPECT(ltx_attn_splitkv_workspace_bytes(68, 0, 64, 16), -1);
  EXPECT(ltx_flash_attn_splitkv_v_bf16(d, 2048, d, 2048, d, 2048, d, 2048, nullptr, 0, 68, 3456, 32, 64, 0.125f, 0,
                                       d, 1 << 20, nullptr), LTX_ERR_INVALID_ARG);  // zero splits
  EXPECT(ltx_flash_attn_splitkv_bf16(d, 2048, d, 2048, d, 3456, d, 2048, nullptr, 0, 68, 3456, 32, 64, 0.125f, 16,
                                     d, 16, nullptr), LTX_ERR_INVALID_ARG);  // workspace too small
  EXPECT(ltx_flash_attn_splitkv_noalloc_bf16(d, 2048, d, 2048, d, 3456, d, 2048, nullptr, 0, 68, 3456, 32, 64,
                                             0.125f, 300, nullptr), LTX_ERR_INVALID_ARG);  // splits > 256
  EXPECT(ltx_flash_attn_splitkv_noalloc_bf16(d, 4096, d, 4096, d, 65536, d, 4096, nullptr, 0, 65536, 65536, 32,
                                             128, 0.1f, 256, nullptr), LTX_ERR_SCRATCH_LIMIT);
  // oversize arguments: refused by the operand checks before the scratch need
  // is computed, and the size helper reports -1 rather than a wrapped count
  const int64_t hh = int64_t(1) << 40;
  EXPECT(ltx_attn_splitkv_workspace_bytes(int64_t(1) << 40, hh, 128, 256), -1);
  EXPECT(ltx_attn_splitkv_workspace_bytes(INT64_MAX, 1, 1, 1), -1);
  EXPECT(ltx_flash_attn_splitkv_noalloc_bf16(d, hh * 128, d, hh * 128, d, 64, d, hh * 128, nullptr, 0, 1 << 30, 1,
                                             hh, 128, 0.1f, 256, nullptr), LTX_ERR_UNSUPPORTED);
  EXPECT(ltx_flash_attn_splitkv_noalloc_bf16(d, 4096, d, 4096, d, 32, d, 4096, nullptr, 0, 68, 3456, 32, 128,
                                             0.1f, 16, nullptr), LTX_ERR_INVALID_ARG);  // tk_pad below Tk

  // ---- launch planning: valid calls, refused at the launch (no device).
  // Never with a device present: the fake addresses would reach a kernel.
  int ndev = 0;
  const int dev_status = hipGetDeviceCount(&ndev);  // 100: hipErrorNoDevice
  if (ndev != 0 || (dev_status != 0 && dev_status != 100)) {
    std::printf("launch-planning checks skipped: a device is present\n");
  } else {
    const uint8_t* q8 = static_cast<const uint8_t*>(d);
    const int8_t* i8 = static_cast<const int8_t*>(d);
    float* ws = fo;
    uint32_t* cnt = static_cast<uint32_t*>(d);
    const int64_t big = int64_t(1) << 30;
    // row kernels at the step's shapes (video 3456 x 4096, audio 68 x 2048, the
    // reference's T = 14640 test shape)
    for (int64_t rows : {int64_t(68), int64_t(3456), int64_t(14640)}) {
      for (int64_t c : {int64_t(2048), int64_t(4096)}) {
        EXPECT(ltx_adaln_norm_fused_bf16(d, c, fd, fd, d, c, rows, c, 1e-6f, 0, nullptr), LTX_ERR_HIP);
        EXPECT(ltx_adaln_norm_fused2_bf16(d, c, fd, fd, d, c, fd, fd, d, c, rows, c, 1e-6f, 0, nullptr),
               LTX_ERR_HIP);
        EXPECT(ltx_gated_add_fused_bf16(d, c, d, c, fd, d, c, rows, c, 0, nullptr), LTX_ERR_HIP);
        EXPECT(ltx_qknorm_rope_bf16(d, 3 * c, rows, fd, fd, fd, d, 3 * c, rows, fd, fd, fd, c, c == 4096 ? 128 : 64,
                                    1e-6f, nullptr), LTX_ERR_HIP);
        EXPECT(ltx_qknorm_rope_axes_bf16(d, 3 * c, rows, fd, fd, fd, id, 3, 49, d, 3 * c, rows / 2, fd, fd, fd, id, 3,
                                         49, c, c == 4096 ? 128 : 64, 1e-6f, nullptr), LTX_ERR_HIP);
        EXPECT(ltx_output_norm_modulate_bf16(d, c, fd, fd, d, c, rows, c, 1e-6f, nullptr), LTX_ERR_HIP);
      }
    }
    // GEMMs: every tile choice on the block's shapes, the 68-row audio shapes
    // and the text-context shapes, every epilogue code
    struct Shape { int64_t m, n, k; };
    const Shape shapes[] = {{3456, 16384, 4096}, {3456, 4096, 16384}, {3456, 12320, 4096}, {3456, 2080, 4096},
                            {3456, 4096, 2048}, {68, 6176, 2048}, {68, 2048, 8192}, {256, 8192, 4096},
                            {10368, 4096, 4096}, {1, 1024, 4096}};
    for (const Shape& sh : shapes) {
      for (int tile = 0; tile <= 6; ++tile) {
        for (int epi = 0; epi <= 4; ++epi) {
          const int flags = epi | (tile << 8);
          const void* r = epi == 2 || epi == 3 ? d : nullptr;
          const float* g = epi == 2 || epi == 3 ? fd : nullptr;
          EXPECT(ltx_gemm_bf16(d, sh.k, d, sh.k, fd, d, sh.n, sh.m, sh.n, sh.k, flags, r, sh.n, g, sh.n - 32,
                               nullptr), LTX_ERR_HIP);
          EXPECT(ltx_gemm_w8a16_bf16(d, sh.k, i8, sh.k, fd, fd, d, sh.n, sh.m, sh.n, sh.k, flags, r, sh.n, g,
                                     sh.n - 32, nullptr), LTX_ERR_HIP);
          EXPECT(ltx_gemm_mxfp8_bf16(d, sh.k, q8, sh.k, q8, sh.k / 32, fd, d, sh.n, sh.m, sh.n, sh.k,
                                     flags | LTX_GEMM_ROUND_THEN_BIAS, r, sh.n, g, sh.n - 32, nullptr),
                 LTX_ERR_HIP);
        }
      }
      for (int splits : {1, 2, 4, 8, 16}) {
        if (sh.k % (128 * splits) != 0) continue;
        const int64_t need = ltx_gemm_splitk_workspace_bytes(sh.m, sh.n, splits);
        const int64_t rneed = ltx_gemm_rows_workspace_bytes(sh.m, sh.n, splits);
        const int64_t words = ltx_gemm_rows_counter_words(sh.m, sh.n);
        EXPECT(need > 0 && rneed == need && words > 0, 1);
        EXPECT(ltx_gemm_splitk_bf16(d, sh.k, d, sh.k, fd, d, sh.n, sh.m, sh.n, sh.k, 0, nullptr, 0, nullptr, sh.n,
                                    splits, ws, need, nullptr), sh.m * sh.n * 4 * splits >= big ? LTX_ERR_HIP : LTX_ERR_HIP);
        EXPECT(ltx_gemm_splitk_mxfp8_bf16(d, sh.k, q8, sh.k, q8, sh.k / 32, fd, d, sh.n, sh.m, sh.n, sh.k, 3, d,
                                          sh.n, fd, sh.n, splits, ws, need, nullptr), LTX_ERR_HIP);
        EXPECT(ltx_gemm_splitk_w8a16_bf16(d, sh.k, i8, sh.k, fd, fd, d, sh.n, sh.m, sh.n, sh.k, 1, nullptr, 0,
                                          nullptr, sh.n, splits, ws, need, nullptr), LTX_ERR_HIP);
        if (sh.m <= 256) {
          EXPECT(ltx_gemm_rows_bf16(d, sh.k, d, sh.k, fd, d, sh.n, sh.m, sh.n, sh.k, 2, d, sh.n, fd, sh.n, splits,
                                    ws, rneed, cnt, words, nullptr), LTX_ERR_HIP);
          EXPECT(ltx_gemm_rows_w8a16_bf16(d, sh.k, i8, sh.k, fd, fd, d, sh.n, sh.m, sh.n, sh.k, 1, nullptr, 0,
                                          nullptr, sh.n, splits, ws, rneed, cnt, words, nullptr), LTX_ERR_HIP);
          EXPECT(ltx_gemm_rows_mxfp8_bf16(d, sh.k, q8, sh.k, q8, sh.k / 32, fd, d, sh.n, sh.m, sh.n, sh.k,
                                          4 | LTX_GEMM_ROUND_THEN_BIAS, nullptr, 0, nullptr, sh.n - 32, splits, ws,
                                          rneed, cnt, words, nullptr), LTX_ERR_HIP);
        }
      }
      if (sh.k % 512 == 0 && sh.m >= 256) {
        // the query projections' row statistics, every weight format
        const int64_t ssc = (sh.n >= 4096 ? 4096 : sh.n) / 64 * 64;
        EXPECT(ltx_gemm_rowss_bf16(0, d, sh.k, d, sh.k, nullptr, 0, fd, d, sh.n, sh.m, sh.n, sh.k, 0, ssc, fo,
                                   ssc / 64, ssc, nullptr), LTX_ERR_HIP);
        EXPECT(ltx_gemm_rowss_bf16(1, d, sh.k, i8, sh.k, fd, 0, fd, d, sh.n, sh.m, sh.n, sh.k, 0, ssc, fo, ssc / 64,
                                   ssc, nullptr), LTX_ERR_HIP);
        EXPECT(ltx_gemm_rowss_bf16(2, d, sh.k, q8, sh.k, q8, sh.k / 32, fd, d, sh.n, sh.m, sh.n, sh.k,
                                   LTX_GEMM_ROUND_THEN_BIAS, ssc, fo, ssc / 64, ssc, nullptr), LTX_ERR_HIP);
        EXPECT(ltx_gemm_mx_bf16(q8, sh.k, q8, sh.k / 32, q8, sh.k, q8, sh.k / 32, fd, d, sh.n, sh.m, sh.n, sh.k, 2, d,
                                sh.n, fd, sh.n, nullptr), LTX_ERR_HIP);
        EXPECT(ltx_gemm_mx_gelu_mxfp8(q8, sh.k, q8, sh.k / 32, q8, sh.k, q8, sh.k / 32, fd,
                                      static_cast<uint8_t*>(d), sh.n, static_cast<uint8_t*>(d), sh.n / 32, sh.m,
                                      sh.n, sh.k, LTX_GEMM_ROUND_THEN_BIAS, nullptr), LTX_ERR_HIP);
      }
    }
    // weight formats at the block's shapes
    EXPECT(ltx_quantize_mxfp8_bf16(d, 4096, 16384, 4096, static_cast<uint8_t*>(d), 4096, static_cast<uint8_t*>(d),
                                   128, nullptr), LTX_ERR_HIP);
    EXPECT(ltx_dequantize_mxfp8_bf16(q8, 4096, q8, 128, 16384, 4096, d, 4096, nullptr), LTX_ERR_HIP);
    EXPECT(ltx_quantize_w8_bf16(d, 4096, 16384, 4096, static_cast<int8_t*>(d), 4096, fo, nullptr), LTX_ERR_HIP);
    EXPECT(ltx_dequantize_w8_bf16(i8, 4096, fd, 16384, 4096, d, 4096, nullptr), LTX_ERR_HIP);
    EXPECT(ltx_dequantize_fp8_e4m3(q8, int64_t(16384) * 4096, fd, d, 0, nullptr), LTX_ERR_HIP);
    // attention: every call shape of the block, both V layouts, split-KV with
    // its workspace, the no-allocation form (which resolves its scratch first)
    struct Attn { int64_t tq, tk, h, dh; };
    const Attn calls[] = {{3456, 3456, 32, 128}, {6144, 6144, 32, 128}, {3456, 256, 32, 128}, {3456, 68, 32, 64},
                          {68, 3456, 32, 64}, {68, 68, 32, 64}, {68, 256, 32, 64}, {1, 1, 1, 64}};
    for (const Attn& a : calls) {
      const int64_t rs = a.h * a.dh, tkp = ltx_attn_vt_padded_len(a.tk);
      EXPECT(ltx_flash_attn_v_bf16(d, rs, d, rs, d, rs, d, rs, d, a.h, a.tq, a.tk, a.h, a.dh, 0.1f, nullptr),
             LTX_ERR_HIP);
      EXPECT(ltx_flash_attn_bf16(d, rs, d, rs, d, tkp, d, rs, nullptr, 0, a.tq, a.tk, a.h, a.dh, 0.1f, nullptr),
             LTX_ERR_HIP);
      EXPECT(ltx_attn_transpose_v_bf16(d, rs, a.tk, a.h, a.dh, d, tkp, nullptr), LTX_ERR_HIP);
      if (rs % 256 == 0 && rs / 64 <= 64) {  // query norm in the kernel: no RoPE, per-query and 3-axis tables
        EXPECT(ltx_flash_attn_qnorm_v_bf16(d, rs, d, rs, d, rs, d, rs, d, a.h, a.tq, a.tk, a.h, a.dh, 0.1f, fd,
                                           rs / 64, rs / 64, fd, 1e-6f, nullptr, nullptr, nullptr, 1, 0, nullptr),
               LTX_ERR_HIP);
        EXPECT(ltx_flash_attn_qnorm_v_bf16(d, rs, d, rs, d, rs, d, rs, d, a.h, a.tq, a.tk, a.h, a.dh, 0.1f, fd,
                                           rs / 64, rs / 64, fd, 1e-6f, fd, fd, nullptr, 1, a.tq, nullptr),
               LTX_ERR_HIP);
        EXPECT(ltx_flash_attn_qnorm_v_bf16(d, rs, d, rs, d, rs, d, rs, d, a.h, a.tq, a.tk, a.h, a.dh, 0.1f, fd,
                                           rs / 64, rs / 64, fd, 1e-6f, fd, fd, id, 3, 49, nullptr),
               LTX_ERR_HIP);
      }
      for (int64_t splits : {int64_t(2), int64_t(16), int64_t(54)}) {
        const int64_t need = ltx_attn_splitkv_workspace_bytes(a.tq, a.h, a.dh, splits);
        EXPECT(need > 0, 1);
        EXPECT(ltx_flash_attn_splitkv_v_bf16(d, rs, d, rs, d, rs, d, rs, d, a.h, a.tq, a.tk, a.h, a.dh, 0.1f, splits,
                                             d, need, nullptr), LTX_ERR_HIP);
        EXPECT(ltx_flash_attn_splitkv_bf16(d, rs, d, rs, d, tkp, d, rs, nullptr, 0, a.tq, a.tk, a.h, a.dh, 0.1f,
                                           splits, d, need, nullptr), LTX_ERR_HIP);
        if (need <= (int64_t(32) << 20))
          EXPECT(ltx_flash_attn_splitkv_noalloc_bf16(d, rs, d, rs, d, tkp, d, rs, nullptr, 0, a.tq, a.tk, a.h, a.dh,
                                                     0.1f, splits, nullptr), LTX_ERR_HIP);
      }
    }
    // step glue, guidance, latents, text features at the workloads' sizes
    EXPECT(ltx_euler_x0_step_bf16(d, d, 1.0f, 0.5f, d, 3456 * 128, nullptr), LTX_ERR_HIP);
    EXPECT(ltx_timestep_embedding_f32(fd, 4, 1000.0f, fo, 256, nullptr), LTX_ERR_HIP);
    EXPECT(ltx_gemv_f32_bf16w(fd, 2, 4096, d, fd, fo, 9 * 4096, 1, nullptr), LTX_ERR_HIP);
    EXPECT(ltx_broadcast_add_f32(fd, fd, fo, 48 * 16, 4096, nullptr), LTX_ERR_HIP);
    EXPECT(ltx_x0_from_velocity_f32(d, d, 0.5f, fo, 3456 * 128, nullptr), LTX_ERR_HIP);
    EXPECT(ltx_guidance_f32(fd, fd, fd, fd, 3.0f, 1.0f, 0.0f, fd, fd, fo, 3456 * 128, 0, nullptr), LTX_ERR_HIP);
    EXPECT(ltx_guidance_stats_f32(fd, fd, 3456 * 128, LTX_GUIDE_STATS_STD_RATIO, 0.7f, 0.3f, fo, nullptr),
           LTX_ERR_HIP);
    EXPECT(ltx_ge_correct_f32(fd, fo, fo, 0, 0.5f, 0.5f, 3456 * 128, nullptr), LTX_ERR_HIP);
    EXPECT(ltx_euler_step_bf16(d, fd, 0.5f, d, 3456 * 128, nullptr), LTX_ERR_HIP);
    EXPECT(ltx_swap_axes(d, 9, 128, 384, 2, static_cast<char*>(d) + (1 << 24), nullptr), LTX_ERR_HIP);
    EXPECT(ltx_gemma_features_bf16(d, 49, 1024, 3840, 1024 * 3840, 3840, id, 1e-6f, 1.0f, 1.0f, d, d, 49 * 3840,
                                   nullptr), LTX_ERR_HIP);
  }

  std::printf("%s: %d failure(s)\n", failures ? "FAIL" : "ok", failures);
  return failures ? 1 : 0;
}
