// Host-side checks of the C ABI, built against the library compiled with
// AddressSanitizer on its host code (build.sh).  Every call takes an
// argument-validation path that returns before any device work -- null
// pointers, unsupported shapes, misaligned pointers or strides, empty
// problems, workspace and padding helpers -- so the program runs without a
// GPU and AddressSanitizer sees all the host code those paths execute.
// Device pointers are fake, 16-byte aligned addresses that the library must
// never dereference on the host.
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "../../include/ltx_hip.h"

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

  std::printf("%s: %d failure(s)\n", failures ? "FAIL" : "ok", failures);
  return failures ? 1 : 0;
}
