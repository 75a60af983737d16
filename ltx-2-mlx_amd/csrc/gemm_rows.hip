// Few-row projection GEMMs on CDNA4 matrix cores, in one launch:
//
//   C[m, n] = epilogue( sum_k A[m, k] * W[n, k] + bias[n] ),  M <= 128 per tile
//
// The products of the 68-token audio stream (and other row counts up to a few
// hundred) have too few rows for the tile kernels of gemm.hip: a 256x256 or
// 128x128 tile is mostly padding, and their K loops are long serial chains.
// These products are bound by the weight bytes (a 2048 x 8192 MXFP8 weight is
// 17 MB; the activations are 68 x 8192 bf16 = 1.1 MB), so this kernel streams
// each weight byte from HBM exactly once, with the products split along K
// over enough workgroups to keep many weight loads in flight, and sums the
// splits and applies the epilogue inside the same launch:
//
//   * workgroup = 4 waves = one output tile of BM = 32 * TMF rows (all rows of
//     a 68-row product, TMF = 3) x 128 columns (32 per wave), over one K range
//     (split) of Ks = K / splits.  Grid = row tiles x column tiles x splits.
//   * K steps of 128 (8-bit weights) or 64 (bf16) per stage.  The activation
//     rows, the weight rows and (MXFP8) the E8M0 scales of a stage reach LDS
//     by direct buffer loads (no staging registers), RING stages deep, so
//     RING - 1 stages are in flight while one is multiplied.
//   * Within a stage the k order of the MFMA slots is permuted so that a lane
//     reads its weight row's codes as one contiguous 64-byte run: MFMA k-step
//     t, lane half h covers k = (KS/2) h + 8 t + [0, 8) on both operands; the
//     stage's sum is the same set of products.  The weight fragment is the
//     MFMA "A" operand (each lane then holds 4 consecutive output columns);
//     8-bit weights are dequantised per fragment with the exact format
//     arithmetic (v_cvt_scalef32_pk_bf16_fp8 for MXFP8; bf16(fp32(q) * s) for
//     int8), so the bf16 MFMA sees bit-exact weights.
//   * Each split writes its fp32 partial tile to the workspace with
//     device-coherent stores (sc1: coherent across the XCDs' L2 caches) and,
//     once they are complete, takes a ticket from the tile's counter (a
//     device-scope atomic).  The workgroup that draws the last ticket resets
//     the counter to zero, reads the partials back with device-coherent loads,
//     sums them in split order -- the result does not depend on which split
//     finished last -- and applies the epilogue of the tile kernels (bias,
//     quantised-linear rounding, GELU-tanh, 2*sigmoid head gate, gated
//     residual) with the same rounding points.
//   * blockIdx -> (split, tile): consecutive workgroups of one XCD share a
//     split and a row tile, i.e. one activation slice, which its L2 then
//     serves to all of them.
#include "gemm_common.h"

namespace ltx {

struct RowsArgs {
  const bf16* A;
  int64_t lda;
  const void* B;        // (N, K) weights: bf16, int8 or E4M3 codes; row stride ldb elements
  int64_t ldb;
  const void* bscale;   // int8: fp32 (N); MXFP8: uint8 (N, K/32), row stride ld_scale bytes
  int64_t ld_scale;
  const float* bias;    // fp32 (N) or null
  bf16* C;
  int64_t ldc;
  const bf16* R;        // residual (gated epilogues), may alias C
  int64_t ldr;
  const float* gate;    // fp32 (N)
  float* partial;       // [split][M][N] fp32
  uint32_t* counters;   // one ticket counter per output tile, zero between launches
  int sig_from;         // columns n >= sig_from get the 2*sigmoid head gate (EPI_BIAS)
  int round_then_bias;  // bias added to the bf16-rounded product (quantised-linear form)
  int M, N, Ks;         // Ks: K depth of one split
  int tiles_m, tiles_n, splits;
};

constexpr int kRowsThreads = 256;

template <int BKIND, int TMF>
struct RowsCfg {
  static constexpr bool B8 = BKIND != B_BF16;
  static constexpr bool MXS = BKIND == B_MXFP8;
  static constexpr int KS = B8 ? 128 : 64;  // k per stage
  static constexpr int ES = B8 ? 1 : 2;     // weight bytes per element
  static constexpr int KSTEPS = KS / 16;
  static constexpr int BM = 32 * TMF, BN = 128;
  // activation rows: 2 KS bytes = 16 (8-bit weights) or 8 (bf16) chunks
  static constexpr int A_ROWB = 2 * KS, A_CH = A_ROWB / 16;
  static constexpr int A_BYTES = BM * A_ROWB;
  // weight rows: KS codes or KS / 2 ... always 128 bytes = 8 chunks
  static constexpr int W_ROWB = KS * ES;
  static constexpr int W_BYTES = BN * W_ROWB;
  // MXFP8: 4 E8M0 bytes per column and stage (k-blocks of 32); four waves
  // write 256 bytes each, waves 2 and 3 a copy that nobody reads
  static constexpr int SC_BYTES = MXS ? 1024 : 0;
  static constexpr int STAGE = A_BYTES + W_BYTES + SC_BYTES;
  static constexpr int RING = 4 * STAGE <= 150 * 1024 ? 4 : 3;
  // direct-load instructions (1 KiB each, one 16-byte slot per lane) per wave
  // and stage, plus one 4-byte scale load for MXFP8
  static constexpr int A_DMA = A_BYTES / 1024 / 4, W_DMA = W_BYTES / 1024 / 4;
  static constexpr int L = A_DMA + W_DMA + (MXS ? 1 : 0);
  static constexpr int RING_BYTES = RING * STAGE;
  // after the ring: int8 column scales (4 waves x 256 bytes), the last-ticket flag
  static constexpr int I8_OFF = RING_BYTES, FLAG_OFF = I8_OFF + 1024;
  // epilogue column values (bias, gate): inside the ring, free by then
  static constexpr int COL_OFF = 0;
  static constexpr int LDS_BYTES = FLAG_OFF + 16;
  static_assert(W_ROWB == 128, "weight rows of 128 bytes");
  static_assert(A_BYTES % 4096 == 0, "whole direct-load instructions per wave");
  static_assert((RING - 2) * L < 64, "vmcnt range");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS");
};

// XOR of the 16-byte chunk of LDS row r that keeps 16 lanes reading one
// chunk of 16 consecutive rows on distinct banks: 256-byte rows r % 16,
// 128-byte rows (r / 2) % 8 (two rows share a bank offset 128 bytes apart).
template <int CH>
__device__ __forceinline__ int rows_swz(int r) {
  if constexpr (CH == 16) return r & 15;
  else return (r >> 1) & 7;
}

// 4-byte direct load (one dword per lane to lds_dst + 4 * lane)
__device__ __forceinline__ void buffer_dma4(const void* base, int num_records, uint32_t voff, int soff,
                                            char* lds_dst) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, num_records, kBufferRsrcWord3);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds_dst, 4, voff, soff, 0, 0);
}

// 16-byte store / load with the sc1 cache policy: device-scope coherence
// (what the compiler emits for agent-scope atomic accesses on this target),
// so a partial written on one XCD is read correctly on another.
constexpr int kAuxSc1 = 16;
__device__ __forceinline__ void store_dev16(float* base, int num_records, uint32_t voff, f32x4 v) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, num_records, kBufferRsrcWord3);
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, voff, 0, kAuxSc1);
}
__device__ __forceinline__ f32x4 load_dev16(const float* base, int num_records, uint32_t voff) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, num_records, kBufferRsrcWord3);
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, kAuxSc1));
}

template <int BKIND, int TMF, int EPI>
__global__ __launch_bounds__(kRowsThreads, 1) void gemm_rows_kernel(RowsArgs p) {
  using Cfg = RowsCfg<BKIND, TMF>;
  constexpr int KS = Cfg::KS, ES = Cfg::ES, KSTEPS = Cfg::KSTEPS, BM = Cfg::BM, BN = Cfg::BN;
  constexpr int A_ROWB = Cfg::A_ROWB, A_CH = Cfg::A_CH, A_BYTES = Cfg::A_BYTES, W_BYTES = Cfg::W_BYTES;
  constexpr int STAGE = Cfg::STAGE, RING = Cfg::RING, L = Cfg::L;
  constexpr bool MXS = Cfg::MXS;
  constexpr bool RESID = EPI == LTX_GEMM_EPI_RESIDUAL || EPI == LTX_GEMM_EPI_RESIDUAL_ROUND;
  __shared__ __attribute__((aligned(1024))) char lds[Cfg::LDS_BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // block -> (split, row tile, column tile), column tile fastest, numbered
  // XCD-contiguously (the hardware sends block b to XCD b % 8)
  int logical;
  {
    const int nb = (int)gridDim.x, b = (int)blockIdx.x;
    const int q = nb / kNumXcd, r = nb % kNumXcd;
    const int xcd = b % kNumXcd, idx = b / kNumXcd;
    logical = xcd * q + (xcd < r ? xcd : r) + idx;
  }
  const int tiles = p.tiles_m * p.tiles_n;
  const int z = logical / tiles, tile = logical % tiles;
  const int tm = tile / p.tiles_n, tn = tile % p.tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int64_t kb = (int64_t)z * p.Ks;  // first k of the split
  const int KT = p.Ks / KS;
  // a wave whose 32 columns all lie past N moves its share of every stage and
  // meets every barrier, but reads no fragments and issues no MFMAs
  const int live = __builtin_amdgcn_readfirstlane(n0 + 32 * wave < p.N ? 1 : 0);

  // ---- direct-load sources.  Instruction d of wave w fills LDS block 4d + w
  // (1 KiB); lane j its 16-byte slot j, which holds logical chunk
  // slot ^ swizzle(row).  Rows past M / N re-read the last row.  The
  // descriptors' record counts are the operand extents (checked < 2^31).
  const int a_records = (int)((int64_t)p.M * p.lda * 2);
  const int w_records = (int)((int64_t)p.N * p.ldb * ES);
  uint32_t a_src[Cfg::A_DMA];
#pragma unroll
  for (int d = 0; d < Cfg::A_DMA; ++d) {
    const int r = (1024 / A_ROWB) * (4 * d + wave) + lane / A_CH;
    int gm = m0 + r;
    gm = gm < p.M ? gm : p.M - 1;
    const int chunk = (lane % A_CH) ^ rows_swz<A_CH>(r);
    a_src[d] = (uint32_t)(((int64_t)gm * p.lda + kb) * 2) + chunk * 16;
  }
  uint32_t w_src[Cfg::W_DMA];
#pragma unroll
  for (int d = 0; d < Cfg::W_DMA; ++d) {
    const int r = 8 * (4 * d + wave) + (lane >> 3);
    int gn = n0 + r;
    gn = gn < p.N ? gn : p.N - 1;
    const int chunk = (lane & 7) ^ rows_swz<8>(r);
    w_src[d] = (uint32_t)(((int64_t)gn * p.ldb + kb) * ES) + chunk * 16;
  }
  // scale / int8-scale loads: wave w moves columns 64 (w % 2) + lane
  int sc_col = n0 + 64 * (wave & 1) + lane;
  sc_col = sc_col < p.N ? sc_col : p.N - 1;
  const int sc_records = MXS ? (int)((int64_t)p.N * p.ld_scale) : 0;
  const uint32_t sc_src = MXS ? (uint32_t)((int64_t)sc_col * p.ld_scale + kb / 32) : 0u;

  auto stage_base = [&](int buf) -> char* { return lds + buf * STAGE; };
  // blocks of rows wholly past M move 4 bytes per lane instead of 16 (the
  // rows are never stored; one instruction either way keeps the wait counts)
  int a_full[Cfg::A_DMA];
#pragma unroll
  for (int d = 0; d < Cfg::A_DMA; ++d)
    a_full[d] = __builtin_amdgcn_readfirstlane(m0 + (1024 / A_ROWB) * (4 * d + wave) < p.M ? 1 : 0);
  auto issue = [&](int kt, int buf) __attribute__((always_inline)) {
    char* As = stage_base(buf);
    char* Ws = As + A_BYTES;
#pragma unroll
    for (int d = 0; d < Cfg::A_DMA; ++d) {
      if (a_full[d]) buffer_dma16(p.A, a_records, a_src[d], kt * A_ROWB, As + (4 * d + wave) * 1024);
      else buffer_dma4(p.A, a_records, a_src[d], kt * A_ROWB, As + (4 * d + wave) * 1024);
    }
#pragma unroll
    for (int d = 0; d < Cfg::W_DMA; ++d)
      buffer_dma16(p.B, w_records, w_src[d], kt * KS * ES, Ws + (4 * d + wave) * 1024);
    if constexpr (MXS) buffer_dma4(p.bscale, sc_records, sc_src, kt * (KS / 32), Ws + W_BYTES + wave * 256);
  };

  // ---- per-lane fragment addresses (relative to a stage): lane (fr, h)
  const int fr = lane & 31, h = lane >> 5;
  int a_off[KSTEPS];
#pragma unroll
  for (int t = 0; t < KSTEPS; ++t) a_off[t] = fr * A_ROWB + ((((KS / 16) * h + t) ^ rows_swz<A_CH>(fr)) * 16);
  const int wr = 32 * wave + fr;  // weight row (output column) of the lane
  int w_off[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) w_off[j] = A_BYTES + wr * 128 + (((4 * h + j) ^ rows_swz<8>(wr)) * 16);
  const int sc_off = A_BYTES + W_BYTES + wr * 4;

  f32x16 acc[TMF];
#pragma unroll
  for (int i = 0; i < TMF; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;

  // ---- epilogue column values (bias; gate of the residual forms), one
  // column per thread, requested before the first direct load so that the
  // loop's wait counts stay exact; staged in LDS after the loop
  float col_bias = 0.0f, col_gate = 0.0f;
  if (tid < BN && n0 + tid < p.N) {
    if (p.bias) col_bias = p.bias[n0 + tid];
    if (RESID) col_gate = p.gate[n0 + tid];
  }

  // ---- prologue: int8 column scales, stages 0 .. RING-2 in flight
  if constexpr (BKIND == B_INT8) {
    buffer_dma4(p.bscale, p.N * 4, (uint32_t)sc_col * 4, 0, lds + Cfg::I8_OFF + wave * 256);
    wait_vmcnt<0>();
  }
#pragma unroll
  for (int s = 0; s < RING - 1; ++s) issue(s < KT ? s : KT - 1, s);
  float s_i8 = 0.0f;

  auto compute = [&](int buf) __attribute__((always_inline)) {
    const char* S = stage_base(buf);
    u32x4 q[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) q[j] = *reinterpret_cast<const u32x4*>(S + w_off[j]);
    uint32_t scw = 0;
    if constexpr (MXS) scw = *reinterpret_cast<const uint32_t*>(S + sc_off);
    bf16x8 af[KSTEPS][TMF];
#pragma unroll
    for (int t = 0; t < KSTEPS; ++t)
#pragma unroll
      for (int i = 0; i < TMF; ++i)
        af[t][i] = *reinterpret_cast<const bf16x8*>(S + a_off[t] + i * 32 * A_ROWB);
    // every fragment read of the stage is issued before the first MFMA (one
    // wave per SIMD: nothing else hides the LDS latency)
    __builtin_amdgcn_sched_barrier(0);
    float scf[2] = {0.0f, 0.0f};
    if constexpr (MXS) {
      scf[0] = e8m0_to_f32_valu(__builtin_amdgcn_ubfe(scw, 16 * h, 8));
      scf[1] = e8m0_to_f32_valu(__builtin_amdgcn_ubfe(scw, 16 * h + 8, 8));
    }
#pragma unroll
    for (int t = 0; t < KSTEPS; ++t) {
      bf16x8 wf;
      if constexpr (BKIND == B_BF16) {
        wf = __builtin_bit_cast(bf16x8, q[t]);
      } else {
        const uint32_t w0 = q[t >> 1][2 * (t & 1)], w1 = q[t >> 1][2 * (t & 1) + 1];
        uint32_t o[4];
        if constexpr (BKIND == B_MXFP8) {
          const float sc = scf[t >> 2];
          o[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, sc, false));
          o[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, sc, true));
          o[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, sc, false));
          o[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, sc, true));
        } else {
          // bf16(fp32(q) * s): one fp32 product, a single rounding
          const uint32_t ws[2] = {w0, w1};
#pragma unroll
          for (int d = 0; d < 2; ++d) {
            const uint32_t u = ws[d];
            bf16x2 p0, p1;
            p0[0] = (bf16)((float)(int8_t)u * s_i8);
            p0[1] = (bf16)((float)(int8_t)(u >> 8) * s_i8);
            p1[0] = (bf16)((float)(int8_t)(u >> 16) * s_i8);
            p1[1] = (bf16)((float)((int32_t)u >> 24) * s_i8);
            o[2 * d] = __builtin_bit_cast(uint32_t, p0);
            o[2 * d + 1] = __builtin_bit_cast(uint32_t, p1);
          }
        }
        wf = __builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]});
      }
#pragma unroll
      for (int i = 0; i < TMF; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, af[t][i], acc[i], 0, 0, 0);
    }
  };

  // ---- main loop: wait for stage kt (this wave's loads; RING - 2 later
  // stages may stay in flight), one barrier (every wave's loads of stage kt
  // have landed and every wave has finished reading stage kt - 1), refill the
  // buffer of stage kt - 1 with stage kt + RING - 1 (past the end: the last
  // stage again, so every iteration issues the same loads and the waits stay
  // exact), multiply stage kt.
  auto step = [&](int kt, int buf) __attribute__((always_inline)) {
    wait_vmcnt<(RING - 2) * L>();
    barrier_nofence();
    if (BKIND == B_INT8 && kt == 0) s_i8 = *reinterpret_cast<const float*>(lds + Cfg::I8_OFF + 256 * (wr >> 6) + 4 * (wr & 63));
    const int nk = kt + RING - 1;
    issue(nk < KT ? nk : KT - 1, (buf + RING - 1) % RING);
    if (live) compute(buf);
  };
  int kt = 0;
  for (; kt + RING <= KT; kt += RING) {
#pragma unroll
    for (int b = 0; b < RING; ++b) step(kt + b, b);
  }
#pragma unroll
  for (int b = 0; b < RING - 1; ++b)
    if (kt + b < KT) step(kt + b, b);
  wait_vmcnt<0>();

  // column values to LDS, into the ring once every wave's direct loads have
  // landed and its last stage has been read
  __syncthreads();
  float* col_lds = reinterpret_cast<float*>(lds + Cfg::COL_OFF);
  if (tid < BN) {
    col_lds[tid] = col_bias;
    col_lds[BN + tid] = col_gate;
  }
  __syncthreads();

  // ---- the epilogue of the tile kernels for one fp32 sum a of column n:
  // bias (after the bf16 product for the quantised-linear form), GELU or the
  // head gate, bf16 rounding; then the gated residual forms
  const bool rtb = p.round_then_bias != 0;
  auto finish = [&](float a, int n) -> float {
    float y = (rtb ? round_bf(a) : a) + col_lds[n - n0];
    if (EPI == LTX_GEMM_EPI_GELU) y = gelu_tanh(round_bf(y));
    if (EPI == LTX_GEMM_EPI_SIGMOID2) y = sigmoid2_bf(round_bf(y));
    if (EPI == LTX_GEMM_EPI_BIAS && n >= p.sig_from) y = sigmoid2_bf(round_bf(y));
    return round_bf(y);
  };
  auto residual = [&](float y, int n, float r) -> float {
    const float g = col_lds[BN + n - n0];
    return EPI == LTX_GEMM_EPI_RESIDUAL ? fmaf(g, y, r) : round_bf(y * g) + r;
  };

  // ---- one split: the epilogue straight from the accumulators.  Lane (fr, h)
  // holds row m0 + 32 i + fr, columns n0 + 32 wave + 8 g + 4 h + [0, 4).
  if (p.splits == 1) {
    if (!live) return;
    // every residual value is fetched before the first store (a store may
    // alias a later fetch as far as the compiler knows, which would order
    // each fetch behind the stores before it)
    bf16x4 rr[TMF][4];
    if constexpr (RESID) {
#pragma unroll
      for (int i = 0; i < TMF; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int m = m0 + 32 * i + fr, n = n0 + 32 * wave + 8 * g + 4 * h;
          if (m < p.M && n < p.N) rr[i][g] = *reinterpret_cast<const bf16x4*>(p.R + (int64_t)m * p.ldr + n);
        }
    }
#pragma unroll
    for (int i = 0; i < TMF; ++i) {
      const int m = m0 + 32 * i + fr;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + 32 * wave + 8 * g + 4 * h;
        if (m < p.M && n < p.N) {
          bf16x4 v;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float y = finish(acc[i][4 * g + j], n + j);
            if constexpr (RESID) y = residual(y, n + j, (float)rr[i][g][j]);
            v[j] = (bf16)y;
          }
          *reinterpret_cast<bf16x4*>(p.C + (int64_t)m * p.ldc + n) = v;
        }
      }
    }
    return;
  }

  // ---- partial tile -> workspace (device-coherent stores)
  const int MN = p.M * p.N;
  const int p_records = (int)((int64_t)p.splits * MN * 4);
  if (live) {
#pragma unroll
    for (int i = 0; i < TMF; ++i) {
      const int m = m0 + 32 * i + fr;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + 32 * wave + 8 * g + 4 * h;
        if (m < p.M && n < p.N) {
          const f32x4 v = {acc[i][4 * g], acc[i][4 * g + 1], acc[i][4 * g + 2], acc[i][4 * g + 3]};
          store_dev16(p.partial, p_records, (uint32_t)((z * MN + m * p.N + n) * 4), v);
        }
      }
    }
  }
  // the stores are complete (device-coherent) before the ticket is taken
  wait_vmcnt<0>();
  __syncthreads();
  int* flag = reinterpret_cast<int*>(lds + Cfg::FLAG_OFF);
  if (tid == 0) {
    const uint32_t t = __hip_atomic_fetch_add(p.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = t == (uint32_t)(p.splits - 1);
    if (last) __hip_atomic_store(p.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last;
  }
  __syncthreads();
  if (!*flag) return;

  // ---- last split of the tile: sum the partials in split order and apply
  // the epilogue.  Element group e = (row e / 16, 8 columns); thread t takes
  // groups t + 256 j, RC at a time, with the loads of ZB splits of all RC
  // groups in flight together (a dependent chain of loads per group would
  // cost one memory round trip per split).
  constexpr int RC = 4, ZB = 4;
  const int rows = (p.M - m0) < BM ? (p.M - m0) : BM;
  const int groups = rows * 16;
  for (int e0 = tid; e0 < groups; e0 += kRowsThreads * RC) {
    int off[RC], rowm[RC], coln[RC];
    bool ok[RC];
    bf16x8 rres[RC];
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      const int e = e0 + c * kRowsThreads;
      rowm[c] = m0 + (e >> 4);
      coln[c] = n0 + 8 * (e & 15);
      ok[c] = e < groups && coln[c] < p.N;
      off[c] = ok[c] ? (rowm[c] * p.N + coln[c]) * 4 : 0;
    }
    f32x4 s[RC][2];
    for (int zb = 0; zb < p.splits; zb += ZB) {
      f32x4 y[ZB][RC][2];
#pragma unroll
      for (int zi = 0; zi < ZB; ++zi)
#pragma unroll
        for (int c = 0; c < RC; ++c) {
          if (ok[c] && zb + zi < p.splits) {
            const uint32_t o = (uint32_t)(off[c] + (zb + zi) * MN * 4);
            y[zi][c][0] = load_dev16(p.partial, p_records, o);
            y[zi][c][1] = load_dev16(p.partial, p_records, o + 16);
          } else {
            y[zi][c][0] = y[zi][c][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          }
        }
      if (RESID && zb == 0) {
#pragma unroll
        for (int c = 0; c < RC; ++c)
          if (ok[c]) rres[c] = *reinterpret_cast<const bf16x8*>(p.R + (int64_t)rowm[c] * p.ldr + coln[c]);
      }
#pragma unroll
      for (int zi = 0; zi < ZB; ++zi)
#pragma unroll
        for (int c = 0; c < RC; ++c)
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            if (zb + zi == 0) s[c][q] = y[zi][c][q];
            else if (zb + zi < p.splits) s[c][q] += y[zi][c][q];
          }
    }
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      if (!ok[c]) continue;
      const int m = rowm[c], n = coln[c];
      bf16x8 v;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float y = finish(s[c][j >> 2][j & 3], n + j);
        if constexpr (RESID) y = residual(y, n + j, (float)rres[c][j]);
        v[j] = (bf16)y;
      }
      *reinterpret_cast<bf16x8*>(p.C + (int64_t)m * p.ldc + n) = v;
    }
  }
}

template <int BKIND, int EPI>
static void launch_rows_epi(RowsArgs p, int tmf, hipStream_t s) {
  const dim3 grid((unsigned)(p.tiles_m * p.tiles_n * p.splits));
  if (tmf == 2) gemm_rows_kernel<BKIND, 2, EPI><<<grid, kRowsThreads, 0, s>>>(p);
  else if (tmf == 3) gemm_rows_kernel<BKIND, 3, EPI><<<grid, kRowsThreads, 0, s>>>(p);
  else gemm_rows_kernel<BKIND, 4, EPI><<<grid, kRowsThreads, 0, s>>>(p);
}

// Row-tile height: 64, 96 or 128 rows (the smallest that holds M, else 128).
static inline int rows_tmf(int64_t M) { return M <= 64 ? 2 : (M <= 96 ? 3 : 4); }

template <int BKIND>
static int launch_rows(RowsArgs p, int epilogue, hipStream_t s) {
  const int tmf = rows_tmf(p.M);
  p.tiles_m = (int)((p.M + 32 * tmf - 1) / (32 * tmf));
  p.tiles_n = (p.N + 127) / 128;
  p.round_then_bias = (epilogue & LTX_GEMM_ROUND_THEN_BIAS) != 0;
  switch (epilogue & 0xff) {
    case LTX_GEMM_EPI_BIAS: launch_rows_epi<BKIND, LTX_GEMM_EPI_BIAS>(p, tmf, s); break;
    case LTX_GEMM_EPI_GELU: launch_rows_epi<BKIND, LTX_GEMM_EPI_GELU>(p, tmf, s); break;
    case LTX_GEMM_EPI_RESIDUAL: launch_rows_epi<BKIND, LTX_GEMM_EPI_RESIDUAL>(p, tmf, s); break;
    case LTX_GEMM_EPI_RESIDUAL_ROUND: launch_rows_epi<BKIND, LTX_GEMM_EPI_RESIDUAL_ROUND>(p, tmf, s); break;
    case LTX_GEMM_EPI_SIGMOID2: launch_rows_epi<BKIND, LTX_GEMM_EPI_SIGMOID2>(p, tmf, s); break;
    default: return LTX_ERR_INVALID_ARG;
  }
  return ltx_launch_status();
}

}  // namespace ltx

using namespace ltx;

static inline bool rows_al(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

extern "C" int64_t ltx_gemm_rows_workspace_bytes(int64_t M, int64_t N, int64_t splits) {
  if (M < 0 || N < 0 || splits < 1) return -1;
  return splits * M * N * 4;
}

extern "C" int64_t ltx_gemm_rows_counter_words(int64_t M, int64_t N) {
  if (M < 0 || N < 0) return -1;
  const int tmf = rows_tmf(M);
  return ((M + 32 * tmf - 1) / (32 * tmf)) * ((N + 127) / 128);
}

// Shared validation; es = weight element bytes, ks = K depth of one stage.
static int rows_check(const void* A, int64_t lda, const void* W, int64_t ldw, int es, const void* C, int64_t ldc,
                      int64_t M, int64_t N, int64_t K, int epilogue, const void* R, int64_t ldr, const float* gate,
                      int splits, const float* ws, int64_t ws_bytes, const uint32_t* counters,
                      int64_t counter_words) {
  if (!A || !W || !C || M < 0 || N < 0 || K < 0) return LTX_ERR_INVALID_ARG;
  if (epilogue & ~(0xff | LTX_GEMM_ROUND_THEN_BIAS)) return LTX_ERR_INVALID_ARG;
  const int epi = epilogue & 0xff;
  if (epi > LTX_GEMM_EPI_SIGMOID2) return LTX_ERR_INVALID_ARG;
  if ((epi == LTX_GEMM_EPI_RESIDUAL || epi == LTX_GEMM_EPI_RESIDUAL_ROUND) && (!R || !gate || ldr < N))
    return LTX_ERR_INVALID_ARG;
  if (splits < 1 || splits > 64) return LTX_ERR_INVALID_ARG;
  if (lda < K || ldw < K || ldc < N) return LTX_ERR_INVALID_ARG;
  const int64_t ks = es == 1 ? 128 : 64;
  if (K == 0 || K % (ks * splits) != 0 || N % 8 != 0) return LTX_ERR_UNSUPPORTED;
  if (!rows_al(A, 16) || !rows_al(W, 16) || !rows_al(C, 16) || lda % 8 || ldc % 8 || (ldw * es) % 16 ||
      (R && (!rows_al(R, 16) || ldr % 8)))
    return LTX_ERR_ALIGNMENT;
  // buffer-descriptor extents are 31-bit byte counts
  const int64_t lim = (int64_t)1 << 31;
  if (M * lda * 2 >= lim || N * ldw * es >= lim || splits * M * N * 4 >= lim) return LTX_ERR_UNSUPPORTED;
  if (M == 0 || N == 0) return LTX_OK;
  if (!ws || !rows_al(ws, 16) || ws_bytes < splits * M * N * 4) return LTX_ERR_INVALID_ARG;
  if (splits > 1 && (!counters || !rows_al(counters, 4) || counter_words < ltx_gemm_rows_counter_words(M, N)))
    return LTX_ERR_INVALID_ARG;
  return LTX_OK;
}

static RowsArgs rows_args(const void* A, int64_t lda, const void* W, int64_t ldw, const void* scale,
                          int64_t ld_scale, const float* bias, void* C, int64_t ldc, int64_t M, int64_t N,
                          int64_t K, const void* R, int64_t ldr, const float* gate, int64_t sigmoid_from,
                          int splits, float* ws, uint32_t* counters) {
  RowsArgs p;
  p.A = (const bf16*)A;
  p.lda = lda;
  p.B = W;
  p.ldb = ldw;
  p.bscale = scale;
  p.ld_scale = ld_scale;
  p.bias = bias;
  p.C = (bf16*)C;
  p.ldc = ldc;
  p.R = (const bf16*)R;
  p.ldr = ldr;
  p.gate = gate;
  p.partial = ws;
  p.counters = counters;
  p.sig_from = (int)(sigmoid_from < N ? (sigmoid_from < 0 ? 0 : sigmoid_from) : N);
  p.round_then_bias = 0;
  p.M = (int)M;
  p.N = (int)N;
  p.Ks = (int)(K / splits);
  p.tiles_m = p.tiles_n = 0;
  p.splits = splits;
  return p;
}

extern "C" int ltx_gemm_rows_bf16(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias,
                                  void* C, int64_t ldc, int64_t M, int64_t N, int64_t K, int epilogue,
                                  const void* residual, int64_t ldr, const float* gate, int64_t sigmoid_from,
                                  int splits, float* workspace, int64_t workspace_bytes, uint32_t* counters,
                                  int64_t counter_words, void* stream) {
  int st = rows_check(A, lda, W, ldw, 2, C, ldc, M, N, K, epilogue, residual, ldr, gate, splits, workspace,
                      workspace_bytes, counters, counter_words);
  if (st != LTX_OK || M == 0 || N == 0) return st;
  RowsArgs p = rows_args(A, lda, W, ldw, nullptr, 0, bias, C, ldc, M, N, K, residual, ldr, gate, sigmoid_from,
                         splits, workspace, counters);
  return launch_rows<B_BF16>(p, epilogue, (hipStream_t)stream);
}

extern "C" int ltx_gemm_rows_w8a16_bf16(const void* A, int64_t lda, const int8_t* Wq, int64_t ldw,
                                        const float* w_scale, const float* bias, void* C, int64_t ldc, int64_t M,
                                        int64_t N, int64_t K, int epilogue, const void* residual, int64_t ldr,
                                        const float* gate, int64_t sigmoid_from, int splits, float* workspace,
                                        int64_t workspace_bytes, uint32_t* counters, int64_t counter_words,
                                        void* stream) {
  int st = rows_check(A, lda, Wq, ldw, 1, C, ldc, M, N, K, epilogue, residual, ldr, gate, splits, workspace,
                      workspace_bytes, counters, counter_words);
  if (st != LTX_OK || M == 0 || N == 0) return st;
  if (!w_scale || !rows_al(w_scale, 4)) return LTX_ERR_INVALID_ARG;
  RowsArgs p = rows_args(A, lda, Wq, ldw, w_scale, 0, bias, C, ldc, M, N, K, residual, ldr, gate, sigmoid_from,
                         splits, workspace, counters);
  return launch_rows<B_INT8>(p, epilogue, (hipStream_t)stream);
}

extern "C" int ltx_gemm_rows_mxfp8_bf16(const void* A, int64_t lda, const uint8_t* Wq, int64_t ldw,
                                        const uint8_t* w_scale, int64_t ld_scale, const float* bias, void* C,
                                        int64_t ldc, int64_t M, int64_t N, int64_t K, int epilogue,
                                        const void* residual, int64_t ldr, const float* gate,
                                        int64_t sigmoid_from, int splits, float* workspace,
                                        int64_t workspace_bytes, uint32_t* counters, int64_t counter_words,
                                        void* stream) {
  int st = rows_check(A, lda, Wq, ldw, 1, C, ldc, M, N, K, epilogue, residual, ldr, gate, splits, workspace,
                      workspace_bytes, counters, counter_words);
  if (st != LTX_OK || M == 0 || N == 0) return st;
  // 4-byte scale loads per stage: aligned rows, K / 32 scales per row
  if (!w_scale || !rows_al(w_scale, 4) || ld_scale % 4 || ld_scale < K / 32) return LTX_ERR_ALIGNMENT;
  if (N * ld_scale >= ((int64_t)1 << 31)) return LTX_ERR_UNSUPPORTED;
  RowsArgs p = rows_args(A, lda, Wq, ldw, w_scale, ld_scale, bias, C, ldc, M, N, K, residual, ldr, gate,
                         sigmoid_from, splits, workspace, counters);
  return launch_rows<B_MXFP8>(p, epilogue, (hipStream_t)stream);
}
