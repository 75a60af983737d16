// Projection GEMMs of the DiT block on CDNA4 matrix cores.
//
//   C[m, n] = epilogue( sum_k A[m, k] * W[n, k] + bias[n] )
//
// A: bf16 activations (M, K) row-major.  W: the weight in its storage layout
// (N, K) row-major -- nn.Linear's layout -- in one of three formats:
//   bf16                          (reference: nn.Linear / mx.addmm,
//                                  attention.py:425-437, feed_forward.py:91-112)
//   int8 + fp32 per-row scale     (W8A16: w = bf16(fp32(q) * s))
//   MXFP8: E4M3 codes + E8M0 scale per 32 consecutive k
//                                 (loader/transformer_cache.py:1255-1267; the
//                                  reference dequantises to bf16 and runs a bf16
//                                  MMA, docs/PERFORMANCE_NOTES.md:1450-1470)
// Both operands are K-contiguous, which is what the MFMA fragments want.
//
// Kernel structure (one 256-thread workgroup = 4 waves in a 2x2 grid):
//   * block tile BM x BN (256x256 or 128x128), K step 64, two LDS stages plus
//     a third stage in flight, by one of two loaders:
//       - registers (default): the global loads of stage k+2 go to VGPRs while
//         stage k computes; during stage k each lane writes its registers of
//         stage k+1 to LDS and reloads them with stage k+2, one pair every
//         few MFMAs, so loads and LDS writes never idle the matrix pipe;
//       - LDS DMA (global_load_lds_dwordx4) straight into the freed buffer,
//         spread over the last k-step's MFMAs.
//     One barrier per K step.
//   * quantised weights travel to LDS as their 8-bit codes (half the bytes)
//     and are dequantised to bf16 as each lane reads its MFMA fragment, with
//     the exact format arithmetic, so the bf16 MFMA sees bit-exact weights.
//   * LDS rows are 128 bytes (64 bf16; 64 codes for 8-bit weights); 16-byte
//     chunks are XOR-swizzled ((row/2)%8, or (row/4)%4 for 64-byte rows) so
//     the fragment reads of consecutive rows spread over the banks.  The load
//     source address of each lane implements the swizzle.
//   * fragments of k-step kk+1 are read from LDS before the MFMAs of kk issue,
//     across the stage boundary too.
//   * v_mfma_f32_32x32x16_bf16 with the weight fragment as the MFMA "A"
//     operand: each lane then holds 4 consecutive output columns, so the
//     epilogue packs 4 bf16 per LDS write and streams the tile out through LDS
//     in coalesced 16-byte chunks, fusing bias, GELU-tanh, the 2*sigmoid head
//     gate or the gated residual add (fused_ops.py:345-348 semantics).  Bias
//     and gate columns come from LDS and residual rows are fetched before the
//     tile is staged, so the epilogue never waits on memory per element.
//   * blockIdx -> tile: consecutive tiles go to the same XCD (the hardware
//     round-robins workgroups over the 8 XCDs), grouped 4 tile-rows at a
//     time: the 32 concurrent tiles of an XCD form 4 x 8, the fewest distinct
//     activation and weight bytes per K step.
#include <type_traits>

#include "gemm_common.h"

namespace ltx {

// How stage tiles reach LDS: LDS DMA (global_load_lds), or global loads into
// registers one stage ahead that are written to LDS during the next stage.
enum Loader { LOAD_DMA = 0, LOAD_REG = 1 };

struct GemmArgs {
  const bf16* A;
  int64_t lda;
  const void* B;
  int64_t ldb;
  const void* bscale;  // int8: fp32 (N); mxfp8: uint8 (N, K/32)
  int64_t ld_scale;    // mxfp8 scale row stride (bytes)
  const float* bias;   // fp32 (N) or null
  bf16* C;
  int64_t ldc;
  const bf16* R;       // residual (gated epilogues), may alias C
  int64_t ldr;
  const float* gate;   // fp32 (N)
  int sig_from;        // columns n >= sig_from get the 2*sigmoid head-gate epilogue
  int round_then_bias; // bias added to the bf16-rounded product (quantised-linear form)
  float* partial;      // split-K: fp32 partial products [split][M][ldc], no epilogue
  const uint8_t* ascale;  // B_MX: activation E8M0 scales (M, K/32)
  int64_t ld_ascale;      // B_MX: their row stride (bytes)
  uint8_t* cscale;        // kEpiGeluMx: output E8M0 scales (M, N/32); C holds the codes
  int64_t ld_cscale;
  int M, N, K;         // split-K: K is the per-split depth
  int tiles_m, tiles_n;
  // 8-wave bias epilogue: per-row sums of squares of the bf16 outputs of
  // columns [0, ss_cols), one fp32 partial per 64-column slice at
  // rowss[row * ld_rowss + col / 64] (null: none)
  float* rowss = nullptr;
  int64_t ld_rowss = 0;
  int ss_cols = 0;
};

constexpr int kGemmThreads = 256;
// EPI value of the split-K pass: the accumulators go to the fp32 partial
// buffer as they are, the epilogue runs in splitk_epilogue_kernel.
constexpr int kEpiPartial = 16;
// EPI value of the MX kernel's FF up-projection: the GELU epilogue whose
// bf16 result leaves as MXFP8 rows (codes in C, E8M0 scales in cscale) --
// the next product's quantised activations, written by this one.
constexpr int kEpiGeluMx = 5;
constexpr int kGroupM = 4;

__device__ __forceinline__ void tile_coords(int bid, int nblocks, int tiles_m, int tiles_n, int& tm,
                                            int& tn) {
  // XCD-contiguous renumbering: hardware sends block b to XCD b % 8.
  const int q = nblocks / kNumXcd, r = nblocks % kNumXcd;
  const int xcd = bid % kNumXcd, idx = bid / kNumXcd;
  const int logical = xcd * q + (xcd < r ? xcd : r) + idx;
  // grouped ordering: kGroupM tile-rows sweep the tile-columns together
  const int per_group = kGroupM * tiles_n;
  const int group = logical / per_group;
  const int first_m = group * kGroupM;
  const int gsize = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int in_group = logical % per_group;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

template <int BM, int BN, int BK, int STAGES_, int BKIND, int EPI, int SWZ, int LOADER>
struct GemmCfg {
  static constexpr int WM = BM / 2, WN = BN / 2;    // wave tile (2 x 2 waves)
  static constexpr int TM = WM / 32, TN = WN / 32;  // 32x32 MFMA tiles per wave
  static constexpr bool B8 = BKIND != B_BF16;
  // 8-bit weights stay 8-bit in LDS with the DMA loader (dequantised per
  // fragment); the register loader dequantises them once, on the way to LDS.
  static constexpr bool B_RAW = B8 && LOADER == LOAD_DMA;
  static constexpr int KSTEPS = BK / 16;             // MFMA k-steps per stage
  static constexpr int A_ROWB = BK * 2;              // bytes per LDS row
  static constexpr int B_ROWB = B_RAW ? BK : BK * 2;
  static constexpr int B_GROWB = B8 ? BK : BK * 2;   // global bytes per weight row per stage
  static constexpr int A_BYTES = BM * A_ROWB, B_BYTES = BN * B_ROWB;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int STAGES = STAGES_;
  // per-lane 16-byte loads per stage (each wave instruction moves 1 KiB)
  static constexpr int A_DMA = A_BYTES / 1024 / 4;
  static constexpr int B_DMA = BN * B_GROWB / 1024 / 4;
  static constexpr int L = A_DMA + B_DMA;
  static constexpr int EPI_ROWB = WN * 2 + 16;  // padded epilogue row
  static constexpr int EPI_WAVE = WM * EPI_ROWB;
  static constexpr int EPI_BYTES = 4 * EPI_WAVE;
  static constexpr int LDS_BYTES = (STAGES * STAGE > EPI_BYTES) ? STAGES * STAGE : EPI_BYTES;
  static_assert(BK == 32 || BK == 64, "K step");
  static_assert(!B8 || BK == 64, "8-bit weights use 64-byte rows");
  static_assert(!B_RAW || BKIND != B_MXFP8 || STAGES == 2, "MXFP8 scales ride one stage ahead");
  static_assert(LOADER == LOAD_DMA || STAGES == 2, "register staging is the third stage");
  static constexpr int COL_BYTES = 2 * BN * 4;  // epilogue bias + gate columns
  static_assert(LDS_BYTES + COL_BYTES <= 160 * 1024, "LDS");
  static_assert((STAGES - 1) * L < 64, "vmcnt range");
};

// 16-byte chunk XOR of an LDS row.  128-byte rows: SWZ 0 uses (row/2)%8
// (conflict-free per 16 lanes over 256 bytes of banks), SWZ 1 uses row%8.
// 64-byte rows: (row/4)%4.
template <int ROWB, int SWZ>
__device__ __forceinline__ int chunk_xor(int r) {
  if constexpr (ROWB == 128) return SWZ == 0 ? ((r >> 1) & 7) : (r & 7);
  else return (r >> 2) & 3;
}

template <int BM, int BN, int BK, int STAGES_, int BKIND, int EPI, int SWZ, int LOADER>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_kernel(GemmArgs p) {
  using Cfg = GemmCfg<BM, BN, BK, STAGES_, BKIND, EPI, SWZ, LOADER>;
  constexpr bool REG = LOADER == LOAD_REG;
  constexpr int WM = Cfg::WM, WN = Cfg::WN, TM = Cfg::TM, TN = Cfg::TN;
  constexpr bool B8 = Cfg::B8, B_RAW = Cfg::B_RAW;
  constexpr bool B_CONV = B8 && !B_RAW;  // 8-bit weights dequantised by the loader
  constexpr int STAGES = Cfg::STAGES, KSTEPS = Cfg::KSTEPS;
  constexpr int STAGE = Cfg::STAGE;
  constexpr int A_BYTES = Cfg::A_BYTES;
  constexpr int A_ROWB = Cfg::A_ROWB, B_ROWB = Cfg::B_ROWB;
  constexpr int A_DMA = Cfg::A_DMA, B_DMA = Cfg::B_DMA, L = Cfg::L;
  constexpr int EPI_ROWB = Cfg::EPI_ROWB, EPI_WAVE = Cfg::EPI_WAVE;
  __shared__ __attribute__((aligned(1024))) char lds[Cfg::LDS_BYTES + Cfg::COL_BYTES];
  constexpr bool RESID = EPI == LTX_GEMM_EPI_RESIDUAL || EPI == LTX_GEMM_EPI_RESIDUAL_ROUND;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  int tmi, tni;
  // split-K: block b works on split b / tiles of tile b % tiles, the split's
  // k range starting at kz * K
  constexpr bool PARTIAL = EPI == kEpiPartial;
  const int tiles = p.tiles_m * p.tiles_n;
  const int kz = PARTIAL ? (int)blockIdx.x / tiles : 0;
  tile_coords(PARTIAL ? (int)blockIdx.x % tiles : (int)blockIdx.x, PARTIAL ? tiles : (int)gridDim.x,
              p.tiles_m, p.tiles_n, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;
  const int KT = p.K / BK;
  const int64_t k0 = (int64_t)kz * p.K;

  // The epilogue's per-column vectors (bias; gate of the residual forms) are
  // loaded once here, one column per thread, and reach the epilogue through
  // LDS, so no column group waits on global memory there.
  float col_bias = 0.0f, col_gate = 0.0f;
  if (tid < BN && n0 + tid < p.N) {
    if (p.bias) col_bias = p.bias[n0 + tid];
    if (RESID) col_gate = p.gate[n0 + tid];
  }
  float* col_lds = reinterpret_cast<float*>(lds + Cfg::LDS_BYTES);

  // ---- DMA source addresses (k = 0).  Wave instruction i of a tile covers
  // its 1 KiB block 4*i + wave: rows (1024 / ROWB) * (4*i + wave) + lane / LPR
  // with LPR = ROWB / 16 lanes per row; lane slot lane % LPR holds logical
  // chunk slot ^ chunk_xor(row).  Rows past M / N re-read the last row.
  constexpr int A_LPR = A_ROWB / 16, B_LPR = B_ROWB / 16;
  const char* a_src[A_DMA];
#pragma unroll
  for (int i = 0; i < A_DMA; ++i) {
    const int r = (1024 / A_ROWB) * (4 * i + wave) + lane / A_LPR;
    int gm = m0 + r;
    gm = gm < p.M ? gm : p.M - 1;
    const int chunk = (lane % A_LPR) ^ chunk_xor<A_ROWB, SWZ>(r);
    a_src[i] = (const char*)(p.A + (int64_t)gm * p.lda + k0) + chunk * 16;
  }
  const char* b_src[B_DMA];
  int b_dst[B_CONV ? B_DMA : 1];            // loader dequant: LDS byte offset of the row
  int b_c16[B_CONV ? B_DMA : 1];            // ... and the 16-code chunk of it
  const uint8_t* b_scr[B_CONV ? B_DMA : 1];  // MXFP8 scale row
  float b_s8[B_CONV ? B_DMA : 1];           // int8 row scale
#pragma unroll
  for (int i = 0; i < B_DMA; ++i) {
    if constexpr (!B_CONV) {
      const int r = (1024 / B_ROWB) * (4 * i + wave) + lane / B_LPR;
      const int chunk = (lane % B_LPR) ^ chunk_xor<B_ROWB, SWZ>(r);
      int gn = n0 + r;
      gn = gn < p.N ? gn : p.N - 1;
      b_src[i] = (const char*)p.B + ((int64_t)gn * p.ldb + k0) * (B8 ? 1 : 2) + chunk * 16;
    } else {
      // 64-byte code rows, 16 per wave instruction: lane -> row +lane/4,
      // codes 16*(lane%4) .. +16 (no swizzle: it applies to the bf16 writes)
      const int r = 16 * (4 * i + wave) + (lane >> 2);
      int gn = n0 + r;
      gn = gn < p.N ? gn : p.N - 1;
      b_c16[i] = lane & 3;
      b_dst[i] = r * B_ROWB;
      b_src[i] = (const char*)p.B + (int64_t)gn * p.ldb + k0 + b_c16[i] * 16;
      if (BKIND == B_MXFP8) b_scr[i] = (const uint8_t*)p.bscale + (int64_t)gn * p.ld_scale + k0 / 32;
      if (BKIND == B_INT8) b_s8[i] = ((const float*)p.bscale)[gn];
    }
  }

  // Per-lane weight rows of the B fragments and their scales.
  const int frag_r = lane & 31;
  const int frag_c = lane >> 5;
  float s_i8[TN];
  const uint8_t* sc_row[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    int gn = n0 + wn * WN + j * 32 + frag_r;
    gn = gn < p.N ? gn : p.N - 1;
    if (B_RAW && BKIND == B_INT8) s_i8[j] = ((const float*)p.bscale)[gn];
    if (B_RAW && BKIND == B_MXFP8) sc_row[j] = (const uint8_t*)p.bscale + (int64_t)gn * p.ld_scale + k0 / 32;
  }
  // MXFP8 scales of one stage: 2 E8M0 bytes (k blocks 0/1 of the 64) per row.
  uint32_t sc_cur[TN], sc_next[TN];

  // DMA instruction d (0 <= d < L) of stage kt into buffer buf.  Every stage
  // issues all L instructions; stages past the last one re-read stage KT-1
  // into a buffer that is never read again, so the number of outstanding
  // instructions per stage is the same everywhere.
  auto dma_op = [&](int d, int kt, int buf) {
    char* As = lds + buf * STAGE;
    if (d < A_DMA) {
      dma16(a_src[d] + (int64_t)kt * (BK * 2), As + (4 * d + wave) * 1024);
    } else {
      const int i = d - A_DMA;
      dma16(b_src[i] + (int64_t)kt * (B8 ? BK : BK * 2), As + A_BYTES + (4 * i + wave) * 1024);
    }
  };
  // Register-staged loader: load d of stage kt into rg[d], and its LDS write.
  // 8-bit weight loads carry 16 codes (and, for MXFP8, the E8M0 scale of
  // their 32-block), written to LDS as 16 dequantised bf16 in two chunks.
  typedef __attribute__((address_space(1))) const u32x4* g16_t;
  typedef __attribute__((address_space(1))) const uint32_t* g4_t;
  u32x4 rg[REG ? L : 1];
  // MXFP8: the aligned 4-byte scale word holding this load's E8M0 byte, and
  // the byte's bit offset in it (ld_scale % 4 == 0)
  uint32_t rsc[(REG && BKIND == B_MXFP8) ? B_DMA : 1], rsh[(REG && BKIND == B_MXFP8) ? B_DMA : 1];
  auto gload = [&](int d, int kt) {
    if constexpr (REG) {
      if (d < A_DMA) {
        rg[d] = *(g16_t)(a_src[d] + (int64_t)kt * (BK * 2));
      } else {
        rg[d] = *(g16_t)(b_src[d - A_DMA] + (int64_t)kt * (B8 ? BK : BK * 2));
        if constexpr (BKIND == B_MXFP8) {
          const int byte = kt * (BK / 32) + (b_c16[d - A_DMA] >> 1);
          rsc[d - A_DMA] = *(g4_t)(b_scr[d - A_DMA] + (byte & ~3));
          rsh[d - A_DMA] = 8 * (byte & 3);
        }
      }
    }
  };
  // LDS write of load d, in NPART pieces (part = 0 .. NPART-1) issued in
  // consecutive MFMA slots: an 8-bit weight load is dequantised a quarter at
  // a time (its ~16 VALU instructions in one slot would idle the matrix pipe
  // for two MFMAs), the last piece writes the 16 bf16 to LDS.
  float b_sc[B_CONV ? B_DMA : 1];      // dequantisation scale of the load in flight
  uint32_t b_o[B_CONV ? B_DMA : 1][8];  // its bf16 pairs
  auto lwrite = [&](int d, int buf, int part, int nparts) {
    if constexpr (REG) {
      char* As = lds + buf * STAGE;
      if (!B_CONV || d < A_DMA) {
        if (part != nparts - 1) return;
        char* dst = d < A_DMA ? As + (4 * d + wave) * 1024 : As + A_BYTES + (4 * (d - A_DMA) + wave) * 1024;
        *reinterpret_cast<u32x4*>(dst + lane * 16) = rg[d];
      } else {
        const int i = d - A_DMA;
        if (part == 0 && (b_dst[i] / B_ROWB) & 1) {
          // odd rows convert their upper 8 codes first, so their first LDS
          // write fills the chunks the even row above leaves free
          const u32x4 v = rg[d];
          rg[d] = u32x4{v[2], v[3], v[0], v[1]};
        }
        const u32x4 w = rg[d];
        // pieces of a load in four slots: the odd-row swap (part 0), the scale
        // and the first code word (1), two words (2), the last word and the
        // LDS writes (3) -- at most ~8 VALU instructions under one MFMA
        const int dec_part = nparts == 4 ? 1 : 0;
        if (part == dec_part) {
          if constexpr (BKIND == B_MXFP8) {
            // The loaded word goes straight into the empty asm, which pins the
            // byte extraction and decode here: hoisted to the top of the loop
            // they made every iteration wait for the previous stage's loads.
            uint32_t e = rsc[i];
            asm volatile("" : "+v"(e));
            b_sc[i] = e8m0_to_f32((e >> rsh[i]) & 0xffu);
          } else {
            b_sc[i] = b_s8[i];
          }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int q_part = nparts == 4 ? (q == 0 ? 1 : (q == 3 ? 3 : 2)) : q * nparts / 4;
          if (q_part != part) continue;
          const float sc = b_sc[i];
          if constexpr (BKIND == B_MXFP8) {
            b_o[i][2 * q] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[q], sc, false));
            b_o[i][2 * q + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[q], sc, true));
          } else {
            const float nb = -128.0f * sc;
            const uint32_t u = w[q] ^ 0x80808080u;
            bf16x2 p0, p1;
            p0[0] = (bf16)fmaf((float)(u & 0xffu), sc, nb);
            p0[1] = (bf16)fmaf((float)((u >> 8) & 0xffu), sc, nb);
            p1[0] = (bf16)fmaf((float)((u >> 16) & 0xffu), sc, nb);
            p1[1] = (bf16)fmaf((float)(u >> 24), sc, nb);
            b_o[i][2 * q] = __builtin_bit_cast(uint32_t, p0);
            b_o[i][2 * q + 1] = __builtin_bit_cast(uint32_t, p1);
          }
          // keep this piece in its slot (pure arithmetic would otherwise be
          // sunk to the LDS write)
          asm volatile("" : "+v"(b_o[i][2 * q]), "+v"(b_o[i][2 * q + 1]));
        }
        if (part == nparts - 1) {
          // rows 2m and 2m+1 share their chunk swizzle: the even row writes
          // its even chunks first, the odd row its odd chunks, so each write
          // instruction covers every chunk position of the two rows once
          const int r = b_dst[i] / B_ROWB, odd = r & 1;
          char* row = As + A_BYTES + b_dst[i];
          const int x = chunk_xor<B_ROWB, SWZ>(r);
          *reinterpret_cast<u32x4*>(row + ((2 * b_c16[i] + odd) ^ x) * 16) =
              u32x4{b_o[i][0], b_o[i][1], b_o[i][2], b_o[i][3]};
          *reinterpret_cast<u32x4*>(row + ((2 * b_c16[i] + 1 - odd) ^ x) * 16) =
              u32x4{b_o[i][4], b_o[i][5], b_o[i][6], b_o[i][7]};
        }
      }
    }
  };
  auto load_scales = [&](int kt) {
#pragma unroll
    for (int j = 0; j < TN; ++j) sc_next[j] = *reinterpret_cast<const uint16_t*>(sc_row[j] + kt * 2);
  };
  // Stage kt+1 landed while the (STAGES-2) younger stages stay in flight.
  auto wait_next_stage = [&]() {
    if constexpr (REG) return;  // the compiler tracks register loads itself
    else if constexpr (B_RAW && BKIND == B_MXFP8) wait_vmcnt<0>();  // scale loads share the counter
    else wait_vmcnt<(STAGES - 2) * L>();
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  int a_off[TM], b_off[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) a_off[i] = (wm * WM + i * 32 + frag_r) * A_ROWB;
#pragma unroll
  for (int j = 0; j < TN; ++j) b_off[j] = (wn * WN + j * 32 + frag_r) * B_ROWB;
  const int a_swz = chunk_xor<A_ROWB, SWZ>(frag_r);  // same for rows i*32+frag_r
  const int b_swz = chunk_xor<B_ROWB, SWZ>(frag_r);

  // Fragment reads of k-step kk of the stage in buffer `buf`.  8-bit weights
  // are read as their raw codes and dequantised only as their MFMAs issue
  // (conv), so no MFMA waits for a conversion that waits for LDS.
  using BFrag = std::conditional_t<B_RAW, u32x2, bf16x8>;
  auto read_frags = [&](int buf, int kk, bf16x8* fa, BFrag* fb) {
    const char* As = lds + buf * STAGE;
    const char* Bs = As + A_BYTES;
    const int ca = ((kk * 2 + frag_c) ^ a_swz) * 16;
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[i] = *reinterpret_cast<const bf16x8*>(As + a_off[i] + ca);
    if constexpr (!B_RAW) {
      const int cbf = ((kk * 2 + frag_c) ^ b_swz) * 16;
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = *reinterpret_cast<const bf16x8*>(Bs + b_off[j] + cbf);
    } else {
      const int c8 = kk * 2 + frag_c;  // 8-byte chunk of the 64-byte row
      const int cb = ((c8 >> 1) ^ b_swz) * 16 + (c8 & 1) * 8;
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = *reinterpret_cast<const u32x2*>(Bs + b_off[j] + cb);
    }
  };
  // fragment f of k-step kk: A fragments 0..TM-1, then B fragments
  auto read_frag = [&](int buf, int kk, int f, bf16x8* fa, BFrag* fb) {
    const char* As = lds + buf * STAGE;
    const char* Bs = As + A_BYTES;
    if (f < TM) {
      const int ca = ((kk * 2 + frag_c) ^ a_swz) * 16;
      fa[f] = *reinterpret_cast<const bf16x8*>(As + a_off[f] + ca);
    } else if constexpr (!B_RAW) {
      const int cbf = ((kk * 2 + frag_c) ^ b_swz) * 16;
      fb[f - TM] = *reinterpret_cast<const bf16x8*>(Bs + b_off[f - TM] + cbf);
    } else {
      const int c8 = kk * 2 + frag_c;
      const int cb = ((c8 >> 1) ^ b_swz) * 16 + (c8 & 1) * 8;
      fb[f - TM] = *reinterpret_cast<const u32x2*>(Bs + b_off[f - TM] + cb);
    }
  };
  // B fragment j of k-step kk as bf16 (MXFP8 scales of the current stage in
  // sc_cur; int8 per-row scales in s_i8).
  auto conv = [&](const BFrag* fb, int j, int kk) -> bf16x8 {
    if constexpr (!B_RAW) {
      return fb[j];
    } else {
      const u32x2 raw = fb[j];
      uint32_t o[4];
      if constexpr (BKIND == B_INT8) {
        const float sc = s_i8[j], nb = -128.0f * sc;
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          const uint32_t u = raw[d] ^ 0x80808080u;
          bf16x2 p0, p1;
          p0[0] = (bf16)fmaf((float)(u & 0xffu), sc, nb);
          p0[1] = (bf16)fmaf((float)((u >> 8) & 0xffu), sc, nb);
          p1[0] = (bf16)fmaf((float)((u >> 16) & 0xffu), sc, nb);
          p1[1] = (bf16)fmaf((float)(u >> 24), sc, nb);
          o[2 * d] = __builtin_bit_cast(uint32_t, p0);
          o[2 * d + 1] = __builtin_bit_cast(uint32_t, p1);
        }
      } else {
        const float sc = e8m0_to_f32((sc_cur[j] >> (8 * (kk >> 1))) & 0xffu);
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          o[2 * d] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[d], sc, false));
          o[2 * d + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[d], sc, true));
        }
      }
      return __builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]});
    }
  };
  // MFMAs of k-step kk, weight-fragment-major, with memory instructions spread
  // between them: op(m) issues what belongs after MFMA m.  Issuing loads or
  // LDS writes this way never idles the matrix pipe, and the dequantisation
  // of weight fragment j+1 runs under the MFMAs of fragment j.
  auto mfmas_with = [&](const bf16x8* fa, const BFrag* fb, int kk, auto&& op) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const bf16x8 b = conv(fb, j, kk);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, fa[i], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);  // the MFMA issues first; op runs under it
        op(j * TM + i);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  auto mfmas = [&](const bf16x8* fa, const BFrag* fb, int kk) { mfmas_with(fa, fb, kk, [](int) {}); };
  // the L loads of stage kt_src, spread over the NM MFMAs of one k-step
  auto loads_at = [&](int kt_src, int buf) {
    return [&, kt_src, buf](int m) {
      constexpr int NM = TM * TN;
#pragma unroll
      for (int d = 0; d < L; ++d)
        if ((d * NM) / L == m) {
          dma_op(d, kt_src, buf);
        }
    };
  };

  // Software pipeline: all STAGES buffers are filled ahead; fragments of the
  // next k-step are read while the MFMAs of the current one run, including
  // across the stage boundary, whose barrier sits between the fragment reads
  // of the last k-step and its MFMAs.
  bf16x8 fa[2][TM];
  BFrag fb[2][TN];
  if constexpr (REG) {
#pragma unroll
    for (int d = 0; d < L; ++d) gload(d, 0);
#pragma unroll
    for (int d = 0; d < L; ++d) lwrite(d, 0, 0, 1);
#pragma unroll
    for (int d = 0; d < L; ++d) gload(d, KT > 1 ? 1 : 0);
  } else {
#pragma unroll
    for (int st = 0; st < STAGES; ++st)
#pragma unroll
      for (int d = 0; d < L; ++d) dma_op(d, st < KT ? st : KT - 1, st);
  }
  if (B_RAW && BKIND == B_MXFP8) {
    load_scales(0);
    wait_vmcnt<0>();
#pragma unroll
    for (int j = 0; j < TN; ++j) sc_cur[j] = sc_next[j];
    load_scales(KT > 1 ? 1 : 0);
  } else if constexpr (!REG) {
    wait_vmcnt<(STAGES - 1) * L>();
  }
  __syncthreads();
  read_frags(0, 0, fa[0], fb[0]);
  wait_lgkmcnt0();

  // k-steps 0..KSTEPS-2 of the stage in `buf`: read k-step kk+1, then MFMAs of
  // kk.  The fragments of kk were issued one MFMA block earlier; waiting for
  // them before issuing the next reads keeps at most one group (TM+TN <= 8
  // reads) in flight, which the 4-bit LDS counter can track exactly.
  // With the register loader, the fragment reads of k-step kk+1 go one after
  // each of the first TM+TN MFMAs of kk, and the LDS writes of the next stage
  // (into wbuf), each followed one MFMA later by the global load of the stage
  // after it into the same registers (kt_load), are spread evenly over these
  // k-steps' MFMAs: no burst of LDS traffic queues up behind the other waves'.
  auto leading_ksteps = [&](int buf, int wbuf, bool write, int kt_load) {
#pragma unroll
    for (int kk = 0; kk < KSTEPS - 1; ++kk) {
      wait_lgkmcnt0();
      if constexpr (REG) {
        constexpr int NM = TM * TN, SLOTS = (KSTEPS - 1) * NM;
        // slots of a dequantising (8-bit weight) load: up to 4, within its share
        constexpr int BPARTS = (SLOTS / L) < 4 ? (SLOTS / L) : 4;
        static_assert(!B_CONV || BPARTS >= 1, "slots per load");
        mfmas_with(fa[kk & 1], fb[kk & 1], kk, [&](int m) {
          if (m < TM + TN) read_frag(buf, kk + 1, m, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
#pragma unroll
          for (int d = 0; d < L; ++d) {
            const int np = (B_CONV && d >= A_DMA) ? BPARTS : 1;
            const int slot0 = (d * SLOTS) / L;
#pragma unroll
            for (int part = 0; part < np; ++part)
              if (slot0 + part == kk * NM + m && write) lwrite(d, wbuf, part, np);
            // the reload into the same registers goes one slot after the LDS
            // write that reads them (issued right behind it, it waits for the
            // write to take its data: 3 % of a bf16 GEMM)
            const int reload = slot0 + np < SLOTS ? slot0 + np : SLOTS - 1;
            if (reload == kk * NM + m && write) gload(d, kt_load);
          }
        });
      } else {
        read_frags(buf, kk + 1, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(fa[kk & 1], fb[kk & 1], kk);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  constexpr int LASTF = (KSTEPS - 1) & 1;  // fragment set of the last k-step
  int buf = 0;
  for (int kt = 0; kt < KT - 1; ++kt) {
    const int nbuf = buf + 1 == STAGES ? 0 : buf + 1;
    leading_ksteps(buf, nbuf, true, kt + 2 < KT ? kt + 2 : KT - 1);
    wait_next_stage();
    __syncthreads();  // stage kt+1 visible to all waves; stage kt's buffer free
    read_frags(nbuf, 0, fa[0], fb[0]);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (REG) {
      mfmas(fa[LASTF], fb[LASTF], KSTEPS - 1);
    } else {  // DMA of stage kt+STAGES into the freed buffer
      const int kt_src = kt + STAGES < KT ? kt + STAGES : KT - 1;
      mfmas_with(fa[LASTF], fb[LASTF], KSTEPS - 1, loads_at(kt_src, buf));
    }
    if (B_RAW && BKIND == B_MXFP8) {  // the next stage's scales (the last k-step used this one's)
#pragma unroll
      for (int j = 0; j < TN; ++j) sc_cur[j] = sc_next[j];
      load_scales(kt + 2 < KT ? kt + 2 : KT - 1);
    }
    buf = nbuf;
  }
  leading_ksteps(buf, buf, false, 0);
  wait_lgkmcnt0();
  __builtin_amdgcn_sched_barrier(0);
  mfmas(fa[LASTF], fb[LASTF], KSTEPS - 1);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (PARTIAL) {
    // acc[i][j] reg 4g+e holds C[m][n], m = i*32 + lane%32, n = j*32 + 8g +
    // 4*(lane/32) + e (wave-local): four consecutive columns per store
    float* P = p.partial + (int64_t)kz * p.M * p.ldc;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int gm = m0 + wm * WM + i * 32 + frag_r;
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int gn = n0 + wn * WN + j * 32 + 8 * g + 4 * frag_c;
          if (gm < p.M && gn < p.N)
            *reinterpret_cast<f32x4*>(P + (int64_t)gm * p.ldc + gn) =
                f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        }
    }
    return;
  }
  wait_vmcnt<0>();  // the re-read stages land before the epilogue reuses LDS
  if (tid < BN) {
    col_lds[tid] = col_bias;
    col_lds[BN + tid] = col_gate;
  }
  __syncthreads();  // all waves done with the stage buffers; columns visible

  // ---- epilogue: registers -> bf16 tile in LDS (per wave), then coalesced
  // 16-byte row stores.  Phase-2 lane mapping: 16-byte chunk ch of rows
  // it * ROWS_PER_IT + rsub of the wave tile.
  constexpr int CHUNKS = WN / 8;  // 16-byte chunks per wave-tile row
  constexpr int ROWS_PER_IT = 64 / CHUNKS;
  constexpr int ITS = WM / ROWS_PER_IT;
  const int ch = lane % CHUNKS;
  const int rsub = lane / CHUNKS;
  const int gn2 = n0 + wn * WN + ch * 8;
  const bool col_ok = gn2 < p.N;  // N % 8 == 0: a chunk is all in or all out
  // Residual rows (rows past M re-read row M-1, columns past N read column
  // 0; neither is stored) are fetched once phase 1 has moved the
  // accumulators to LDS: fetched any earlier, next to the 256 live
  // accumulators, part of the tile spills to scratch (measured 6-15 % of the
  // residual GEMMs' time).  Their latency overlaps the barrier after phase 1.
  // The residual may alias C: every residual element of this tile is read
  // before any of its outputs is written.
  bf16x8 res[RESID ? ITS : 1];
  auto fetch_res = [&]() {
    if constexpr (RESID) {
      const int gnc = col_ok ? gn2 : 0;
#pragma unroll
      for (int it = 0; it < ITS; ++it) {
        int gm = m0 + wm * WM + it * ROWS_PER_IT + rsub;
        gm = gm < p.M ? gm : p.M - 1;
        res[it] = *reinterpret_cast<const bf16x8*>(p.R + (int64_t)gm * p.ldr + gnc);
      }
    }
  };

  // phase 1: acc[i][j] reg 4g+e holds C[m][n] with m = i*32 + lane%32 and
  // n = j*32 + 8g + 4*(lane/32) + e (wave-local coordinates).  Whether any
  // column of this wave tile takes the head-gate sigmoid is wave-uniform, so
  // the common case runs without it.
  char* E = lds + wave * EPI_WAVE;
  // sig_tag / rtb_tag: compile-time forms of two block-uniform conditions
  // (gate columns in this wave tile; bias added to the rounded product), so
  // the per-element code has no branches
  auto phase1 = [&](auto sig_tag, auto rtb_tag) {
    constexpr bool SIG = decltype(sig_tag)::value;
    constexpr bool RTB = decltype(rtb_tag)::value;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int nl = j * 32 + 8 * g + 4 * frag_c;
        const int gn = n0 + wn * WN + nl;
        const f32x4 bias4 = *reinterpret_cast<const f32x4*>(col_lds + wn * WN + nl);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float a = acc[i][j][4 * g + e];
            y[e] = (RTB ? round_bf(a) : a) + bias4[e];
            if (EPI == LTX_GEMM_EPI_GELU) y[e] = gelu_tanh(round_bf(y[e]));
            if (EPI == LTX_GEMM_EPI_SIGMOID2) y[e] = sigmoid2_bf(round_bf(y[e]));
            if (SIG && gn + e >= p.sig_from) y[e] = sigmoid2_bf(round_bf(y[e]));
          }
          bf16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (bf16)y[e];
          *reinterpret_cast<bf16x4*>(E + (i * 32 + frag_r) * EPI_ROWB + nl * 2) = v;
        }
      }
    }
  };
  const bool sig = EPI == LTX_GEMM_EPI_BIAS && n0 + wn * WN + WN > p.sig_from;
  if (p.round_then_bias) {
    if (sig) phase1(std::true_type{}, std::true_type{});
    else phase1(std::false_type{}, std::true_type{});
  } else {
    if (sig) phase1(std::true_type{}, std::false_type{});
    else phase1(std::false_type{}, std::false_type{});
  }
  fetch_res();
  __syncthreads();

  // phase 2: coalesced 16-byte stores (+ gated residual)
  float g8[8];
  if constexpr (RESID) {
    const f32x4 ga = *reinterpret_cast<const f32x4*>(col_lds + BN + wn * WN + ch * 8);
    const f32x4 gb = *reinterpret_cast<const f32x4*>(col_lds + BN + wn * WN + ch * 8 + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      g8[e] = ga[e];
      g8[4 + e] = gb[e];
    }
  }
#pragma unroll
  for (int it = 0; it < ITS; ++it) {
    const int ml = it * ROWS_PER_IT + rsub;
    const int gm = m0 + wm * WM + ml;
    bf16x8 v = *reinterpret_cast<const bf16x8*>(E + ml * EPI_ROWB + ch * 16);
    if constexpr (RESID) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = (float)v[e];
        float o;
        if (EPI == LTX_GEMM_EPI_RESIDUAL)
          o = fmaf(g8[e], y, (float)res[it][e]);
        else
          o = round_bf(y * g8[e]) + (float)res[it][e];
        v[e] = (bf16)o;
      }
    }
    if (gm < p.M && col_ok) *reinterpret_cast<bf16x8*>(p.C + (int64_t)gm * p.ldc + gn2) = v;
  }
}

// ---- 8-wave ping-pong kernel (8-bit weights; bf16 weights in 32-deep stages) --
// 256x256 tile, K step 64, eight waves (two per SIMD) in two groups of four:
// group 0 (waves 0-3) owns output rows 0-127 of the tile, group 1 (waves 4-7)
// rows 128-255; wave w & 3 owns 64 output columns.  The groups run half a
// stage apart: while one group issues its memory cluster (LDS fragment reads
// of a stage, its share of the direct global->LDS loads two stages ahead, the
// scale loads), the other group's compute cluster (the stage's 64 16x16x32
// MFMAs with the weight dequantisation of fragments 2-7 interleaved) keeps
// the SIMD's matrix pipe busy.  The memory cluster ends, once its fragment
// reads have landed, by decoding the stage's E8M0 scales and dequantising
// fragments 0 and 1, so the compute cluster's first MFMAs issue right after
// the barrier (FF up 402 -> 382 us: the dependent decode -> convert chain had
// left the matrix pipe idle at the start of every compute cluster).
// A workgroup barrier separates the clusters.  Both operands reach LDS by
// global_load_lds (no staging registers, no LDS write instructions): three
// 48 KB stages of bf16 activations (256 x 128 B) and raw weight codes
// (256 x 64 B).  The MXFP8 / int8 codes are dequantised per fragment with the
// exact format arithmetic, so the bf16 MFMA sees bit-exact weights.  bf16
// weights: five 32 KB stages of 32-deep bf16 rows of both operands, the
// direct loads four stages ahead, 32 MFMAs per cluster, no dequantisation.
// MX (8-bit codes of both operands): 16 scaled 32x32x64 MFMAs per cluster.
//
// Inside a stage the k order of the MFMA slots is permuted so that a lane
// reads the codes of both k-steps of the stage with one 16-byte LDS read:
// k-step s, lane quarter q covers k = 16q + 8s + [0, 8) for both operands
// (the E8M0 block of that k range is q / 2).  MX: k-step pair p of the
// scaled MFMA, lane half h, k = 32p + 16h + [0, 16).  The sum over the stage
// is the same set of products.
constexpr int kG8Threads = 512;
// the automatic tile choice uses the 8-wave kernel for 8-bit weights (MXFP8
// and int8) on problems of at least 100 256x256 tiles, and for bf16 weights on
// problems of at least 160

// f(integral_constant<int, I>) for I = I0 .. N-1, in order
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// 16-byte chunk XOR of row r in the 8-wave kernel's stages, 64-byte rows (4
// chunks) and 128-byte rows (8 chunks).  ds_read_b128 services a wave's lanes
// 16 at a time, in the lane-octet pairs (0, 3), (1, 2), (4, 7), (5, 6)
// (probed: two octets reading the same banks at other addresses conflict only
// in those pairs), and its conflicts were probed per read pattern (rocprofv3
// SQ_LDS_BANK_CONFLICT of a one-read kernel over 290 lane -> address tables):
// the 32x32 fragment reads (lane = row 0-31, lane / 32 = chunk half) are
// conflict-free under chunk ^ ((r / 4) % 4) and chunk ^ ((r / 2) % 8), but the
// 16x16 reads (lane % 16 = row, lane / 16 = chunk quarter) conflict under
// those (the FF up-projection: 36-39 M conflict cycles per launch) and not
// under chunk ^ (r bit 0 | r bit 2 << 1) and chunk ^ (r bit 1 | r bit 0 << 1
// | r bit 2 << 2).
__device__ __forceinline__ int g8_swz64(int r, bool s16) { return s16 ? ((r & 1) | ((r >> 1) & 2)) : ((r >> 2) & 3); }
__device__ __forceinline__ int g8_swz128(int r, bool s16) {
  return s16 ? (((r >> 1) & 1) | ((r & 1) << 1) | (r & 4)) : ((r >> 1) & 7);
}

template <int BKIND, int BM_ = 256, int BF_STAGES = 5>
struct G8Cfg {
  static constexpr bool MX = BKIND == B_MX;
  // bf16 weights: a 64-deep stage of both bf16 operands (64 KB) leaves room
  // for only two stages, so the stages are 32 deep (64-byte rows of both
  // operands, laid out like the 8-bit code rows) in a ring of BF_STAGES, the
  // direct loads running BF_STAGES - 1 stages ahead
  static constexpr bool BF = BKIND == B_BF16;
  static constexpr int BM = BM_, BN = 256, BK = BF ? 32 : 64;
  static constexpr int STAGES = BF ? BF_STAGES : 3;
  // 128x64 wave tiles: each weight fragment is dequantised by the two waves
  // that share its columns rather than four (64x128 tiles read fewer LDS
  // bytes per MFMA, but MXFP8 measured 2.5 % slower with them: the
  // conversions cost more power than the extra fragment reads).  Tiles of
  // 128 rows (BM_ = 128: 64x64 wave tiles) for products whose 256-row tiles
  // fill only part of one round.
  static constexpr int WM = BM / 2, WN = 64;
  static constexpr int TM = WM / 32, TN = WN / 32;
  static constexpr int WAVES_M = BM / WM;
  // bf16 MFMAs (bf16 or dequantised 8-bit weights) in the 16x16x32 shape:
  // same flops per cycle as 32x32x16, but the chip holds a ~12 % higher clock
  // under it at full load (2.0 vs 1.7-1.8 GHz in a register-only loop of
  // either shape on all 256 CUs); the wave tile, hence the LDS reads and the
  // accumulator registers, is unchanged.  MX keeps the scaled 32x32x64.
  static constexpr bool S16 = !MX;
  static constexpr int TM16 = WM / 16, TN16 = WN / 16;
  // bf16 activations (MX: 8-bit codes like the weights), 8-bit weight codes
  // (BF: bf16 weights)
  static constexpr int A_ROWB = MX ? BK : BK * 2, B_ROWB = BF ? BK * 2 : BK;
  static constexpr int A_BYTES = BM * A_ROWB, B_BYTES = BN * B_ROWB;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  // LDS: the A stages, then the B stages (every fragment read is then a fixed
  // per-lane register plus an immediate offset below 64 KiB)
  static constexpr int B_REGION = STAGES * A_BYTES;
  static constexpr int A_DMA = A_BYTES / 1024 / 8, B_DMA = B_BYTES / 1024 / 8;  // per wave per stage
  // epilogue staging rows: 16x16 accumulators, 128-byte rows with their
  // 16-byte chunks XORed by (row / 2) % 8 (conflict-free for both the 8-byte
  // accumulator writes and the 16-byte row reads, probed); 32x32 (MX), rows
  // padded to 144 bytes
  static constexpr int EPI_ROWB = S16 ? WN * 2 : WN * 2 + 16;
  static constexpr int EPI_WAVE = WM * EPI_ROWB;
  static constexpr int EPI_BYTES = 8 * EPI_WAVE;
  static constexpr int COL_BYTES = 2 * BN * 4;
  // the column values (bias, gate) follow the epilogue's staging area; they
  // are written after the main loop, so they may lie inside the stage ring
  static constexpr int COL_OFF = EPI_BYTES;
  static constexpr int RING = STAGES * STAGE;
  static constexpr bool COL_IN_RING = COL_OFF < RING;
  static constexpr int LDS_BYTES = (RING > EPI_BYTES + COL_BYTES) ? RING : EPI_BYTES + COL_BYTES;
  // MXFP8 scales of eight stages (256 rows x 16 E8M0 bytes), double buffered;
  // MX: the weights' then the activations' octets
  static constexpr int SC_OCT = BN * 16;
  static constexpr int SC_BYTES = BKIND == B_MXFP8 ? 2 * SC_OCT : (MX ? 4 * SC_OCT : 0);
  // the scale octets after the column values, or (MX) right after the
  // stages, inside the epilogue's staging area (dead by then: every scale
  // load has landed before the epilogue's first barrier)
  static constexpr int SC_OFF = MX ? RING : LDS_BYTES;
  static constexpr int TOTAL = MX ? LDS_BYTES : LDS_BYTES + SC_BYTES;
  static_assert(!MX || SC_OFF + SC_BYTES <= EPI_BYTES, "MX scales inside the staging area");
  static_assert(TOTAL <= 160 * 1024, "LDS");
  static_assert(BM == 256 || (BM == 128 && !MX), "256-row tiles, or 128 without MX activations");
};

template <int BKIND, int EPI, int BM_ = 256>
__global__ __launch_bounds__(kG8Threads, 1) void gemm8_kernel(GemmArgs p) {
  using Cfg = G8Cfg<BKIND, BM_>;
  constexpr int BN = Cfg::BN, WM = Cfg::WM, WN = Cfg::WN, TM = Cfg::TM, TN = Cfg::TN;
  constexpr int A_ROWB = Cfg::A_ROWB, B_ROWB = Cfg::B_ROWB, A_BYTES = Cfg::A_BYTES, B_BYTES = Cfg::B_BYTES;
  constexpr int B_REGION = Cfg::B_REGION;
  constexpr int A_DMA = Cfg::A_DMA, B_DMA = Cfg::B_DMA;
  constexpr int EPI_ROWB = Cfg::EPI_ROWB, EPI_WAVE = Cfg::EPI_WAVE;
  constexpr bool RESID = EPI == LTX_GEMM_EPI_RESIDUAL || EPI == LTX_GEMM_EPI_RESIDUAL_ROUND;
  constexpr bool MX = Cfg::MX, BF = Cfg::BF, S16 = Cfg::S16;
  constexpr int TM16 = Cfg::TM16, TN16 = Cfg::TN16;
  constexpr int STAGES = Cfg::STAGES, AHEAD = STAGES - 1;
  __shared__ __attribute__((aligned(1024))) char lds[Cfg::TOTAL];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform values live in scalar registers: the memory clusters then
  // compute their LDS destinations and load bases with scalar instructions
  // (vector instructions of one wave take matrix-pipe slots from the other)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;  // waves w and w + 4 share a SIMD
  const int wm = wave % Cfg::WAVES_M, wn = wave / Cfg::WAVES_M;

  int tmi, tni;
  tile_coords((int)blockIdx.x, (int)gridDim.x, p.tiles_m, p.tiles_n, tmi, tni);
  const int m0 = tmi * Cfg::BM, n0 = tni * BN;
  const int KT = p.K / Cfg::BK;
  // a wave whose 128 x 64 sub-tile lies wholly past M or N (the last row or
  // column of tiles) reads no fragments and issues no MFMAs: it still moves
  // its share of every stage and meets every barrier
  // (an int from a scalar register: a bool kept across the loop becomes a lane
  // mask whose tests cost vector instructions in every cluster)
  const int live = __builtin_amdgcn_readfirstlane((m0 + wm * WM < p.M && n0 + wn * WN < p.N) ? 1 : 0);

  float* col_lds = reinterpret_cast<float*>(lds + Cfg::COL_OFF);

  // ---- direct-load sources.  A wave instruction fills one contiguous 1 KiB
  // block of LDS, lane j its 16-byte slot j; the lane's source address picks
  // the logical chunk that the slot holds under the XOR swizzle of its row
  // (g8_swz128 for the 128-byte A rows, 8 per block; g8_swz64 for the 64-byte
  // rows, 16 per block), the one under which this kernel's fragment reads are
  // conflict-free.  Rows past M / N re-read the last row.
  // Direct loads as buffer loads: a buffer descriptor per operand (scalar
  // registers), a fixed 32-bit per-lane byte offset in one vector register,
  // the stage's advance as the scalar offset and the LDS destination in M0
  // -- no vector instructions per load (vector instructions of one wave take
  // matrix-pipe slots from the other).  The descriptors' record counts bound
  // every load to its operand (g8_ok checks the 32-bit extents).
  const int a_records = (int)((int64_t)p.M * p.lda * (MX ? 1 : 2)),
            b_records = (int)((int64_t)p.N * p.ldb * (BF ? 2 : 1));
  uint32_t a_src[A_DMA];
#pragma unroll
  for (int d = 0; d < A_DMA; ++d) {
    if constexpr (MX || BF) {
      // activation codes (MX) or 32-deep bf16 rows (BF): 64-byte rows laid
      // out like the weight codes
      const int r = 16 * (8 * d + wave) + (lane >> 2);
      int gm = m0 + r;
      gm = gm < p.M ? gm : p.M - 1;
      const int chunk = (lane & 3) ^ g8_swz64(r, S16);
      a_src[d] = (uint32_t)((int64_t)gm * p.lda * (MX ? 1 : 2)) + chunk * 16;
    } else {
      const int r = 8 * (8 * d + wave) + (lane >> 3);
      int gm = m0 + r;
      gm = gm < p.M ? gm : p.M - 1;
      const int chunk = (lane & 7) ^ g8_swz128(r, S16);
      a_src[d] = (uint32_t)((int64_t)gm * p.lda * 2) + chunk * 16;
    }
  }
  uint32_t b_src[B_DMA];
#pragma unroll
  for (int d = 0; d < B_DMA; ++d) {
    const int r = 16 * (8 * d + wave) + (lane >> 2);
    int gn = n0 + r;
    gn = gn < p.N ? gn : p.N - 1;
    const int chunk = (lane & 3) ^ g8_swz64(r, S16);
    b_src[d] = (uint32_t)((int64_t)gn * p.ldb * (BF ? 2 : 1)) + chunk * 16;
  }
  auto dma_stage = [&](int kt, int buf) __attribute__((always_inline)) {
    char* As = lds + buf * A_BYTES;
    char* Bs = lds + B_REGION + buf * B_BYTES;
#pragma unroll
    for (int d = 0; d < A_DMA; ++d)
      buffer_dma16(p.A, a_records, a_src[d], kt * Cfg::A_ROWB, As + (8 * d + wave) * 1024);
#pragma unroll
    for (int d = 0; d < B_DMA; ++d)
      buffer_dma16(p.B, b_records, b_src[d], kt * Cfg::B_ROWB, Bs + (8 * d + wave) * 1024);
  };

  // ---- per-lane fragment read bases: LDS byte addresses of the lane's first
  // fragment per XOR pattern, so that every fragment read is base + immediate.
  // MX (32x32x64): lane (row fr, half h) reads chunk 2 pp + h of its 64-byte
  // code rows for the stage's k-step pair pp, both operands.
  const int fr = lane & 31, h = lane >> 5;
  const int b_swz = g8_swz64(fr, false);
  int b_base[2], a_mx[2];
#pragma unroll
  for (int pp = 0; pp < 2; ++pp) {
    b_base[pp] = B_REGION + (wn * WN + fr) * B_ROWB + (((2 * pp + h) ^ b_swz) * 16);
    a_mx[pp] = (wm * WM + fr) * A_ROWB + (((2 * pp + h) ^ b_swz) * 16);
  }
  // 16x16x32 fragments: lane (r16, q) = row r16 of a 16-row block, k-quarter
  // q.  Weights: one 16-byte read per block and stage, chunk q of the 64-byte
  // row (8-bit codes: k = 16 q + [0, 16), both k-steps; BF: bf16 k = 8 q +
  // [0, 8) of the 32-deep stage).  8-bit codes: k-step s of the stage is
  // k = 16 q + 8 s + [0, 8) in lane q for both operands -- the activation
  // fragment is chunk 2 q + s of the 128-byte row -- so the E8M0 block of a
  // lane's codes is q / 2 in both k-steps.  Every 16 lanes read 16
  // consecutive rows of one logical chunk (conflict-free under g8_swz64 /
  // g8_swz128 of the 16x16 form; the row's bits 0-3 are those of r16).
  // The activation bases come as a low / high pair (stage buffers 0-1 / 1-2
  // of the 8-bit-code ring) so that the offsets fit the 16-bit immediate.
  const int r16 = lane & 15, q = lane >> 4;
  const int w16 = B_REGION + (wn * WN + r16) * B_ROWB + ((q ^ g8_swz64(r16, true)) * 16);
  int x16_lo[2], x16_hi[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    x16_lo[s] = BF ? (wm * WM + r16) * A_ROWB + ((q ^ g8_swz64(r16, true)) * 16)
                   : (wm * WM + r16) * A_ROWB + (((2 * q + s) ^ g8_swz128(r16, true)) * 16);
    x16_hi[s] = x16_lo[s] + A_BYTES;
  }
  // MXFP8 scales reach LDS by direct loads too, eight stages at a time: the
  // loop then holds no register-destined global load, whose first use would
  // make the compiler wait for every load in flight (its wait counting does
  // not see the direct loads).  Octet o of a tile is 256 weight rows x 16
  // bytes (the E8M0 of k-blocks 16o..16o+15, i.e. stages 8o..8o+7), laid out
  // [row][16]; waves 0-3 each move 64 rows per octet.  int8: the row scale
  // in a register.
  // MX: group 0 moves the weights' octets, group 1 the activations' (256
  // activation rows x 16 bytes, after the weights' two octet buffers).
  char* const sc_lds = lds + Cfg::SC_OFF;
  constexpr bool SCALED = BKIND == B_MXFP8 || MX;
  const int sc_records = SCALED ? (int)((int64_t)p.N * p.ld_scale) : 0;
  const int asc_records = MX ? (int)((int64_t)p.M * p.ld_ascale) : 0;
  const int sc_read = Cfg::SC_OFF + (wn * WN + (S16 ? r16 : fr)) * 16;
  const int asc_read = Cfg::SC_OFF + 2 * Cfg::SC_OCT + (wm * WM + fr) * 16;
  uint32_t sc_src = 0;
  if (grp == 0 || !MX) {
    int gn = n0 + (wave & 3) * 64 + lane;
    gn = gn < p.N ? gn : p.N - 1;
    sc_src = (uint32_t)((int64_t)gn * p.ld_scale);
  } else {
    int gm = m0 + (wave & 3) * 64 + lane;
    gm = gm < p.M ? gm : p.M - 1;
    sc_src = (uint32_t)((int64_t)gm * p.ld_ascale);
  }
  const int noct = KT >> 3;
  auto dma_scales = [&](int oct) {
    if constexpr (SCALED) {
      oct = oct < noct ? oct : noct - 1;  // past the end: re-read the last octet
      if (grp == 0)
        buffer_dma16(p.bscale, sc_records, sc_src, oct * 16, sc_lds + (oct & 1) * Cfg::SC_OCT + wave * 1024);
      else if (MX)
        buffer_dma16(p.ascale, asc_records, sc_src, oct * 16,
                     sc_lds + (2 + (oct & 1)) * Cfg::SC_OCT + (wave & 3) * 1024);
    }
  };
  // weight row blocks of a wave: TN of 32 rows, or (S16) TN16 of 16
  constexpr int NWB = S16 ? TN16 : TN, WB_ROWS = S16 ? 16 : 32;
  float s_i8[NWB];
#pragma unroll
  for (int j = 0; j < NWB; ++j) {
    int gn = n0 + wn * WN + j * WB_ROWS + (S16 ? r16 : fr);
    gn = gn < p.N ? gn : p.N - 1;
    if (BKIND == B_INT8) s_i8[j] = ((const float*)p.bscale)[gn];
  }
  uint32_t scw[NWB];  // this stage pair's E8M0 bytes of the lane's weight rows
  // global memory instructions of a stage's first memory cluster: the direct
  // loads of stage kt+2, plus (group 0, MXFP8) the scales in the first stage
  // of an octet
  constexpr int VM_DMA = A_DMA + B_DMA;
  constexpr int VM_SCALES = SCALED ? 1 : 0;

  // MX: the scaled 32x32x64 fragments
  u32x4 fb[2][MX ? TN : 1];   // weight codes of the stage's two k-step pairs (16 per lane)
  u32x4 fa8[2][MX ? TM : 1];  // activation codes, read like the weight codes
  uint32_t sca[MX ? TM : 1];  // this stage pair's E8M0 bytes of the lane's activation rows
  // 16x16x32: the stage's weight fragments (codes, or bf16 weights) and its
  // activation fragments per k-step
  constexpr int XS = BF ? 1 : 2;
  u32x4 w16f[S16 ? TN16 : 1];
  bf16x8 x16f[XS][S16 ? TM16 : 1];
  // fragment reads of stage kt, which sits in buffer BUF (compile-time)
  auto read_stage = [&](int kt, auto bufc) __attribute__((always_inline)) {
    constexpr int BUF = decltype(bufc)::value;
    if constexpr (SCALED) {
      const int sa = sc_read + ((kt >> 3) & 1) * Cfg::SC_OCT + ((kt & 7) >> 1) * 4;
#pragma unroll
      for (int j = 0; j < NWB; ++j) scw[j] = *reinterpret_cast<const uint32_t*>(lds + sa + j * WB_ROWS * 16);
    }
    if constexpr (MX) {
      const int sa = asc_read + ((kt >> 3) & 1) * Cfg::SC_OCT + ((kt & 7) >> 1) * 4;
#pragma unroll
      for (int i = 0; i < TM; ++i) sca[i] = *reinterpret_cast<const uint32_t*>(lds + sa + i * 32 * 16);
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
          fb[pp][j] = *reinterpret_cast<const u32x4*>(lds + b_base[pp] + BUF * B_BYTES + j * 32 * B_ROWB);
#pragma unroll
        for (int i = 0; i < TM; ++i)
          fa8[pp][i] = *reinterpret_cast<const u32x4*>(lds + a_mx[pp] + BUF * A_BYTES + i * 32 * A_ROWB);
      }
    } else {
#pragma unroll
      for (int jb = 0; jb < TN16; ++jb)
        w16f[jb] = *reinterpret_cast<const u32x4*>(lds + w16 + BUF * B_BYTES + jb * 16 * B_ROWB);
      const int* base = BUF == 0 ? x16_lo : x16_hi;
      constexpr int rel = (BUF == 0 ? 0 : BUF - 1) * A_BYTES;
#pragma unroll
      for (int s = 0; s < XS; ++s)
#pragma unroll
        for (int ib = 0; ib < TM16; ++ib)
          x16f[s][ib] = *reinterpret_cast<const bf16x8*>(lds + base[s] + rel + ib * 16 * A_ROWB);
    }
  };

  // accumulators: (32x32) TM x TN blocks of 16 values, or (16x16) TM16 x TN16
  // blocks of 4 -- the same 128 per lane
  constexpr int AM = S16 ? TM16 : TM, AN = S16 ? TN16 : TN, AE = S16 ? 4 : 16;
  using AccT = std::conditional_t<S16, f32x4, f32x16>;
  AccT acc[AM][AN];
#pragma unroll
  for (int i = 0; i < AM; ++i)
#pragma unroll
    for (int j = 0; j < AN; ++j)
#pragma unroll
      for (int e = 0; e < AE; ++e) acc[i][j][e] = 0.0f;

  // codes of one k-step (two 4-byte words) -> bf16 fragment
  auto dequant = [&](uint32_t w0, uint32_t w1, float sc) -> bf16x8 {
    uint32_t o[4];
    if constexpr (BKIND == B_MXFP8) {
      o[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, sc, false));
      o[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, sc, true));
      o[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, sc, false));
      o[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, sc, true));
    } else {
      // bf16(fp32(q * s)): each signed byte converted by one sign-extending
      // byte-select conversion, one fp32 product (a single rounding), then
      // two values per bf16 conversion
      const uint32_t ws[2] = {w0, w1};
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const uint32_t u = ws[d];
        bf16x2 p0, p1;
        p0[0] = (bf16)((float)(int8_t)u * sc);
        p0[1] = (bf16)((float)(int8_t)(u >> 8) * sc);
        p1[0] = (bf16)((float)(int8_t)(u >> 16) * sc);
        p1[1] = (bf16)((float)((int32_t)u >> 24) * sc);
        o[2 * d] = __builtin_bit_cast(uint32_t, p0);
        o[2 * d + 1] = __builtin_bit_cast(uint32_t, p1);
      }
    }
    return __builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]});
  };

  // Weight fragment f of a stage (k-step f / TN16, row block f % TN16) in two
  // alternating register sets; the scale of each row block (its E8M0 byte of
  // the lane's k-block q / 2, or the int8 row scale) set once per stage.
  float scf[NWB];
  bf16x8 bq[2];
  constexpr int NF = XS * TN16;
  const int q_sh = 8 * (q >> 1);
  auto frag_dequant = [&](int f) -> bf16x8 {
    const int s = f / TN16, jb = f % TN16;
    return dequant(w16f[jb][2 * s], w16f[jb][2 * s + 1], scf[jb]);
  };
  // end of the memory cluster of stage kt (its fragment reads have landed):
  // the stage's scales and fragments 0 and 1 (MX, bf16: nothing to decode)
  auto prep_stage = [&](int kt) __attribute__((always_inline)) {
    if constexpr (MX || BF) return;
#pragma unroll
    for (int j = 0; j < NWB; ++j) {
      if constexpr (BKIND == B_MXFP8)
        scf[j] = e8m0_to_f32_valu(__builtin_amdgcn_ubfe(scw[j], 16 * (kt & 1) + q_sh, 8));
      else
        scf[j] = s_i8[j];
    }
    bq[0] = frag_dequant(0);
    bq[1] = frag_dequant(1);
  };
  // compute cluster of stage kt.  8-bit codes: 2 k-steps x TN16 weight
  // fragments x TM16 MFMAs; fragment f+1 (f >= 1) is dequantised while the
  // MFMAs of fragment f run.  bf16: TN16 x TM16 MFMAs of the stage's 32 k.
  // MX: TN x TM scaled fp8 MFMAs of 64 k.  Their operand contract (probed on
  // the device): lane (row r, half h) holds k = 16h + [0, 16) in bytes 0-15
  // and k = 32 + 16h + [0, 16) in bytes 16-31 -- the two 16-byte code chunks
  // h and 2 + h of the row, as read above -- and lane r + 32b carries the
  // E8M0 scale of row r's k-block b (opsel 0: bits 0-7).  The stage's two
  // blocks are bytes 2 (kt & 1) + b of the octet word.
  auto compute_stage = [&](int kt) __attribute__((always_inline)) {
    if constexpr (MX) {
      const int sh = 16 * (kt & 1) + 8 * h;
      int ws[TN], as[TM];
#pragma unroll
      for (int j = 0; j < TN; ++j) ws[j] = (int)(scw[j] >> sh);
#pragma unroll
      for (int i = 0; i < TM; ++i) as[i] = (int)(sca[i] >> sh);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const i32x8 w = __builtin_bit_cast(i32x8, __builtin_shufflevector(fb[0][j], fb[1][j], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const i32x8 a =
              __builtin_bit_cast(i32x8, __builtin_shufflevector(fa8[0][i], fa8[1][i], 0, 1, 2, 3, 4, 5, 6, 7));
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, a, acc[i][j], 0, 0, 0, ws[j], 0, as[i]);
        }
      }
    } else if constexpr (BF) {
#pragma unroll
      for (int jb = 0; jb < TN16; ++jb)
#pragma unroll
        for (int ib = 0; ib < TM16; ++ib)
          acc[ib][jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, w16f[jb]), x16f[0][ib],
                                                                acc[ib][jb], 0, 0, 0);
    } else {
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const int s = f / TN16, jb = f % TN16;
        if (f >= 1 && f + 1 < NF) bq[(f + 1) & 1] = frag_dequant(f + 1);
#pragma unroll
        for (int ib = 0; ib < TM16; ++ib)
          acc[ib][jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bq[f & 1], x16f[s][ib], acc[ib][jb], 0, 0, 0);
      }
    }
  };

  // ---- prologue: scales of octet 0, stages 0 .. AHEAD-1 in flight, then one
  // barrier for all waves
  dma_scales(0);
  dma_stage(0, 0);
  if (KT > 1) dma_stage(1, 1);
  static_for<2, AHEAD>([&](auto ic) {
    if (KT > decltype(ic)::value) dma_stage(decltype(ic)::value, decltype(ic)::value);
  });
  wait_vmcnt<0>();
  __syncthreads();
  if (grp == 1) barrier_nofence();  // group 1 runs half a stage behind

  // Clusters are whole stages.  Stage s is first read by group 0's memory
  // cluster of stage s (global half-stage 2s), so its data must be in LDS by
  // the barrier before it.  The direct loads of stage s are issued in the
  // memory clusters of stage s-AHEAD; each group waits for them in its last
  // cluster before that barrier -- group 0 at the end of its compute cluster
  // of stage s-1, group 1 at the end of its memory cluster of stage s-1 --
  // leaving only the loads of the AHEAD-1 later stages in flight.  Past the last stage the
  // direct loads re-read stage KT-1 into the buffer nobody reads any more,
  // so every stage issues the same loads and the waits are exact.  The scales
  // of octet o+1 go out (group 0) with stage 8o's loads.
  // SUB = kt % 8 (compile-time in the unrolled loop).
  // The loop is compiled once per group (GRP), so the group-specific waits
  // and scale loads are resolved at compile time.
  auto stage_iter = [&](int kt, auto bufc, auto grpc) __attribute__((always_inline)) {
    constexpr int BUF = decltype(bufc)::value;
    constexpr int GRP = decltype(grpc)::value;
    const bool oct_start = SCALED && (kt & 7) == 0;
    // memory cluster (MX: group 1 moves the activations' scale octets)
    if ((GRP == 0 || MX) && oct_start) dma_scales((kt >> 3) + 1);
    dma_stage(kt + AHEAD < KT ? kt + AHEAD : KT - 1, (BUF + AHEAD) % STAGES);
    if (live) read_stage(kt, bufc);
    wait_lgkmcnt0();
    if (live) prep_stage(kt);
    if (GRP == 1) {
      if (MX && oct_start) wait_vmcnt<VM_DMA + VM_SCALES>();
      else wait_vmcnt<(AHEAD - 1) * VM_DMA>();
    }
    barrier_nofence();
    // compute cluster
    __builtin_amdgcn_s_setprio(1);
    if (live) compute_stage(kt);
    __builtin_amdgcn_s_setprio(0);
    if (GRP == 0) {
      if (oct_start) wait_vmcnt<VM_DMA + VM_SCALES>();
      else wait_vmcnt<(AHEAD - 1) * VM_DMA>();
    }
    barrier_nofence();
  };
  // the loop unrolled over one turn of the ring, then the remainder (stage
  // kt + i sits in buffer i)
  auto main_loop = [&](auto grpc) __attribute__((always_inline)) {
    int kt = 0;
    for (; kt + STAGES - 1 < KT; kt += STAGES)
      static_for<0, STAGES>([&](auto ic) { stage_iter(kt + decltype(ic)::value, ic, grpc); });
    static_for<0, STAGES - 1>([&](auto ic) {
      if (kt + decltype(ic)::value < KT) stage_iter(kt + decltype(ic)::value, ic, grpc);
    });
  };
  if (grp == 0) main_loop(std::integral_constant<int, 0>{});
  else main_loop(std::integral_constant<int, 1>{});
  if (grp == 0) barrier_nofence();
  wait_vmcnt<0>();
  // column values inside the ring: every wave's last direct loads have landed
  if constexpr (Cfg::COL_IN_RING) __syncthreads();

  // ---- epilogue (every wave is past its last LDS fragment read)
  if (tid < BN) {
    float col_bias = 0.0f, col_gate = 0.0f;
    if (n0 + tid < p.N) {
      if (p.bias) col_bias = p.bias[n0 + tid];
      if (RESID) col_gate = p.gate[n0 + tid];
    }
    col_lds[tid] = col_bias;
    col_lds[BN + tid] = col_gate;
  }
  __syncthreads();
  constexpr int CHUNKS = WN / 8;
  constexpr int ROWS_PER_IT = 64 / CHUNKS;
  constexpr int ITS = WM / ROWS_PER_IT;
  const int ch = lane % CHUNKS;
  const int rsub = lane / CHUNKS;
  const int gn2 = n0 + wn * WN + ch * 8;
  const bool col_ok = gn2 < p.N;
  char* E = lds + wave * EPI_WAVE;
  auto phase1 = [&](auto sig_tag, auto rtb_tag) {
    constexpr bool SIG = decltype(sig_tag)::value;
    constexpr bool RTB = decltype(rtb_tag)::value;
    // accumulator block (i, j), values 4 g .. 4 g + 3: output columns nl ..
    // nl + 3 of tile row (32x32) i * 32 + fr, or (16x16) i * 16 + r16
#pragma unroll
    for (int j = 0; j < AN; ++j) {
#pragma unroll
      for (int g = 0; g < AE / 4; ++g) {
        const int nl = S16 ? j * 16 + 4 * q : j * 32 + 8 * g + 4 * h;
        const int gn = n0 + wn * WN + nl;
        const f32x4 bias4 = *reinterpret_cast<const f32x4*>(col_lds + wn * WN + nl);
#pragma unroll
        for (int i = 0; i < AM; ++i) {
          // bf16 roundings two at a time (one conversion per pair)
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = acc[i][j][4 * g + e];
          if (RTB) {
            round_bf2(y[0], y[1]);
            round_bf2(y[2], y[3]);
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] += bias4[e];
          if (EPI == LTX_GEMM_EPI_GELU || EPI == kEpiGeluMx || EPI == LTX_GEMM_EPI_SIGMOID2 || SIG) {
            float r[4] = {y[0], y[1], y[2], y[3]};
            round_bf2(r[0], r[1]);
            round_bf2(r[2], r[3]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (EPI == LTX_GEMM_EPI_GELU || EPI == kEpiGeluMx) y[e] = gelu_tanh(r[e]);
              if (EPI == LTX_GEMM_EPI_SIGMOID2) y[e] = sigmoid2_bf(r[e]);
              if (SIG && gn + e >= p.sig_from) y[e] = sigmoid2_bf(r[e]);
            }
          }
          bf16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (bf16)y[e];
          if constexpr (S16) {
            const int row = i * 16 + r16;
            *reinterpret_cast<bf16x4*>(E + row * EPI_ROWB + ((((nl >> 3) ^ (row >> 1)) & 7) << 4) + (nl & 7) * 2) = v;
          } else {
            *reinterpret_cast<bf16x4*>(E + (i * 32 + fr) * EPI_ROWB + nl * 2) = v;
          }
        }
      }
    }
  };
  const bool sig = EPI == LTX_GEMM_EPI_BIAS && n0 + wn * WN + WN > p.sig_from;
  if (p.round_then_bias) {
    if (sig) phase1(std::true_type{}, std::true_type{});
    else phase1(std::false_type{}, std::true_type{});
  } else {
    if (sig) phase1(std::true_type{}, std::false_type{});
    else phase1(std::false_type{}, std::false_type{});
  }
  // residual rows after the accumulators are in LDS (fewer live registers);
  // every residual element of the tile is read before its output is written
  bf16x8 res[RESID ? ITS : 1];
  if constexpr (RESID) {
    const int gnc = col_ok ? gn2 : 0;
#pragma unroll
    for (int it = 0; it < ITS; ++it) {
      int gm = m0 + wm * WM + it * ROWS_PER_IT + rsub;
      gm = gm < p.M ? gm : p.M - 1;
      res[it] = *reinterpret_cast<const bf16x8*>(p.R + (int64_t)gm * p.ldr + gnc);
    }
  }
  __syncthreads();
  float g8[8];
  if constexpr (RESID) {
    const f32x4 ga = *reinterpret_cast<const f32x4*>(col_lds + BN + wn * WN + ch * 8);
    const f32x4 gb = *reinterpret_cast<const f32x4*>(col_lds + BN + wn * WN + ch * 8 + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      g8[e] = ga[e];
      g8[4 + e] = gb[e];
    }
  }
#pragma unroll
  for (int it = 0; it < ITS; ++it) {
    const int ml = it * ROWS_PER_IT + rsub;
    const int gm = m0 + wm * WM + ml;
    bf16x8 v = *reinterpret_cast<const bf16x8*>(E + ml * EPI_ROWB + (S16 ? ((ch ^ (ml >> 1)) & 7) : ch) * 16);
    if constexpr (RESID) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = (float)v[e];
        float o;
        if (EPI == LTX_GEMM_EPI_RESIDUAL)
          o = fmaf(g8[e], y, (float)res[it][e]);
        else
          o = round_bf(y * g8[e]) + (float)res[it][e];
        v[e] = (bf16)o;
      }
    }
    if constexpr (EPI == kEpiGeluMx) {
      // the row's 32-column block spans lanes ch & ~3 .. ch | 3 (N % 32 == 0:
      // a block lies wholly inside or outside the output); its maximum takes
      // two lane exchanges, then 8 codes per lane and one scale byte per block
      float f[8], amax = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        f[e] = (float)v[e];
        amax = fmaxf(amax, fabsf(f[e]));
      }
      amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
      amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
      const int X = mxfp8_block_exponent(amax);
      const float sx = ldexpf(1.0f, X), lim = 448.0f * sx;
      const uint32_t w0 = e4m3x4_ocp(f[0], f[1], f[2], f[3], sx, lim);
      const uint32_t w1 = e4m3x4_ocp(f[4], f[5], f[6], f[7], sx, lim);
      if (gm < p.M && col_ok) {
        uint8_t* cq = reinterpret_cast<uint8_t*>(p.C);
        *reinterpret_cast<u32x2*>(cq + (int64_t)gm * p.ldc + gn2) = u32x2{w0, w1};
        if ((ch & 3) == 0) p.cscale[(int64_t)gm * p.ld_cscale + gn2 / 32] = (uint8_t)(X + 127);
      }
    } else {
      if (gm < p.M && col_ok) *reinterpret_cast<bf16x8*>(p.C + (int64_t)gm * p.ldc + gn2) = v;
    }
    if constexpr (EPI == LTX_GEMM_EPI_BIAS) {
      // the row's sum of squares over this wave's 64 columns: eight per lane,
      // then over the row's eight lanes (consecutive: lane = 8 rsub + ch)
      if (p.rowss != nullptr && n0 + wn * WN < p.ss_cols) {
        float q = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = (float)v[e];
          q = fmaf(f, f, q);
        }
        q += __shfl_xor(q, 1, 64);
        q += __shfl_xor(q, 2, 64);
        q += __shfl_xor(q, 4, 64);
        if (ch == 0 && gm < p.M) p.rowss[(int64_t)gm * p.ld_rowss + (n0 + wn * WN) / WN] = q;
      }
    }
  }
}

template <int BKIND, int EPI, int BM = 256>
static void launch_g8(GemmArgs p, hipStream_t s) {
  p.tiles_m = (p.M + BM - 1) / BM;
  p.tiles_n = (p.N + 255) / 256;
  gemm8_kernel<BKIND, EPI, BM><<<p.tiles_m * p.tiles_n, kG8Threads, 0, s>>>(p);
}

template <int BM, int BN, int BK, int STAGES, int BKIND, int EPI, int SWZ = 0, int LOADER = LOAD_DMA>
static void launch_tile(GemmArgs p, hipStream_t s) {
  p.tiles_m = (p.M + BM - 1) / BM;
  p.tiles_n = (p.N + BN - 1) / BN;
  gemm_kernel<BM, BN, BK, STAGES, BKIND, EPI, SWZ, LOADER><<<p.tiles_m * p.tiles_n, kGemmThreads, 0, s>>>(p);
}

// Whether the 8-wave kernel takes a problem: operand extents within its 31-bit
// buffer record counts; for MXFP8 whole eight-stage scale octets (K % 512) in
// 16-byte aligned pieces.
template <int BKIND>
static bool g8_ok(const GemmArgs& p) {
  // operand extents are 31-bit buffer record counts in the kernel
  if ((int64_t)p.M * p.lda * (BKIND == B_MX ? 1 : 2) >= ((int64_t)1 << 31) ||
      (int64_t)p.N * p.ldb * (BKIND == B_BF16 ? 2 : 1) >= ((int64_t)1 << 31) ||
      (int64_t)p.N * p.ld_scale >= ((int64_t)1 << 31))
    return false;
  if (BKIND == B_MX)
    return p.K % 512 == 0 && p.ld_scale % 16 == 0 && ((uintptr_t)p.bscale & 15u) == 0 &&
           p.ld_ascale % 16 == 0 && ((uintptr_t)p.ascale & 15u) == 0 &&
           (int64_t)p.M * p.ld_ascale < ((int64_t)1 << 31);
  if (BKIND == B_MXFP8)
    return p.K % 512 == 0 && p.ld_scale % 16 == 0 && ((uintptr_t)p.bscale & 15u) == 0;
  return true;
}

// Automatic 8-wave launches split M when that shortens a partial last round:
// rows [0, r0) in 256-row tiles, rows [r0, M) in 128-row tiles by a second
// launch of the 128-row form (same per-element arithmetic, bit-identical
// outputs).  Cost model in rounds of one workgroup per CU on the MI355X's
// 256 CUs: a round of 128-row tiles takes 0.67 of a 256-row round (FF up
// alone: 1728 tiles of 128 rows in 7 rounds, 436 us, against 896 of 256 rows
// in 4 rounds, 373 us).  At M = 3456 the FF up-projection (14 x 64 tiles =
// 3.5 rounds, i.e. 4) runs 12 tile rows of 256 (3 rounds) plus 3 of 128
// (one partial round): 392.5 -> 373.1 us alone.  A split must model >= 3 %
// faster; r0 = M means one launch.
constexpr int kG8Cus = 256;
static int g8_split_rows(int M, int N) {
  const int64_t tn = (N + 255) / 256, tm = (M + 255) / 256;
  auto rounds = [](int64_t tiles) { return (double)((tiles + kG8Cus - 1) / kG8Cus); };
  const double one = rounds(tm * tn);
  double best = one;
  int r0 = M;
  for (int64_t b = tm - 1; b >= 1 && b >= tm - 8; --b) {
    const int64_t small = (M - 256 * b + 127) / 128;
    const double t = rounds(b * tn) + 0.67 * rounds(small * tn);
    if (t < best && t < 0.97 * one) {
      best = t;
      r0 = (int)(256 * b);
    }
  }
  return r0;
}
// The rows [r0, M) of a product: the same operands from row r0 on.
static GemmArgs rows_from(const GemmArgs& p, int r0) {
  GemmArgs q = p;
  q.A = p.A + (int64_t)r0 * p.lda;
  q.C = p.C + (int64_t)r0 * p.ldc;
  if (p.R) q.R = p.R + (int64_t)r0 * p.ldr;
  if (p.rowss) q.rowss = p.rowss + (int64_t)r0 * p.ld_rowss;
  q.M = p.M - r0;
  return q;
}

// Tile shapes (all K step 64): 256x256 and 128x128 with the register-staged
// loader (1 and 2; 128x128 runs two workgroups per CU), 256x256 with the
// LDS-DMA loader (3), 256x128 register-staged (4), and the 8-wave kernel with
// 256x256 (5) or 128x256 tiles (6).
template <int BKIND, int EPI>
static int launch_epi_w(const GemmArgs& p, int tile, hipStream_t s) {
  const bool auto_tile = tile == 0;
  if (tile == 0) {
    // Large tiles when they still give most CUs a tile; 128x128 otherwise.
    // 8-bit weights take the 8-wave kernel from 100 tiles of 256x256: the A2V
    // query projection (3456 x 4096 -> 2048, 112 tiles) runs in 76 instead of
    // 86 us alone, and the step gains 0.6-0.7 ms (the CUs its single round
    // leaves free take the audio stream's work).  (256x128 tiles, 14 % faster
    // on that projection alone, were 0.25 ms slower per step: explicit only.)
    // int8 measured faster there than on the 4-wave kernel on every block
    // shape (4096^2 109 vs 134 us, FF up 428 vs 472, FF down 405 vs 435).
    // (128-row tiles for the A2V query projection, 126 -> 243 tiles: 79 ->
    // 61 us alone, but the step 1.0-1.6 ms slower in two A/B pairs -- 48 %
    // more CU time per launch, which the audio stream's work beside it then
    // lacks: explicit only, LTX_GEMM_TILE_G8_128.)
    // bf16 weights (32-deep stages) take it where it measured faster at
    // M = 3456 (16x16x32 MFMAs, one box): products at least as wide as deep
    // (FF up 396 vs 422 us on the 4-wave kernel, QKV 291 vs 302, 4096^2 98.8
    // vs 103.7, A2V out 57.5 vs 59.9) and the partial round of the A2V query
    // projection (81 vs 87 us); the FF down product stays on the 4-wave
    // kernel (393 vs 402 us).
    const int64_t big = (int64_t)((p.M + 255) / 256) * ((p.N + 255) / 256);
    const bool g8 = (BKIND == B_MXFP8 || BKIND == B_INT8 || (BKIND == B_BF16 && (p.N >= p.K || big < 160))) &&
                    g8_ok<BKIND>(p);
    tile = big >= 160 ? (g8 ? 5 : 1) : (big >= 100 && g8 ? 5 : 2);
    // row sums of squares come from the 8-wave kernel's epilogue only
    if (p.rowss && tile != 5) tile = 5;
  }
  if (p.rowss && tile != 5 && tile != 6) return LTX_ERR_UNSUPPORTED;
  if (tile == 5 || tile == 6) {
    if (!g8_ok<BKIND>(p)) return LTX_ERR_UNSUPPORTED;
    const int r0 = (tile == 5 && auto_tile) ? g8_split_rows(p.M, p.N) : p.M;
    if (tile == 6) {
      launch_g8<BKIND, EPI, 128>(p, s);
    } else if (r0 < p.M) {
      GemmArgs top = p;
      top.M = r0;
      launch_g8<BKIND, EPI>(top, s);
      launch_g8<BKIND, EPI, 128>(rows_from(p, r0), s);
    } else {
      launch_g8<BKIND, EPI>(p, s);
    }
    return LTX_OK;
  }
  if (tile == 1)
    launch_tile<256, 256, 64, 2, BKIND, EPI, 0, LOAD_REG>(p, s);
  else if (tile == 2)
    launch_tile<128, 128, 64, 2, BKIND, EPI, 0, LOAD_REG>(p, s);
  else if (tile == 4)
    launch_tile<256, 128, 64, 2, BKIND, EPI, 0, LOAD_REG>(p, s);
  else
    launch_tile<256, 256, 64, 2, BKIND, EPI, 0, LOAD_DMA>(p, s);
  return LTX_OK;
}

template <int BKIND, int EPI>
static int launch_epi(const GemmArgs& p, int tile, hipStream_t s) {
  if constexpr (BKIND == B_MX) {
    // quantised activations: the 8-wave kernel only
    if (tile != 0 && tile != 5) return LTX_ERR_UNSUPPORTED;
    if (!g8_ok<BKIND>(p)) return LTX_ERR_UNSUPPORTED;
    launch_g8<BKIND, EPI>(p, s);
    return LTX_OK;
  } else {
    return launch_epi_w<BKIND, EPI>(p, tile, s);
  }
}

template <int BKIND>
static int launch_kind(const GemmArgs& p, int epilogue, hipStream_t s) {
  const int epi = epilogue & 0xff;
  const int tile = (epilogue >> 8) & 0xf;
  if (tile > 6) return LTX_ERR_INVALID_ARG;
  GemmArgs q = p;
  q.round_then_bias = (epilogue & LTX_GEMM_ROUND_THEN_BIAS) != 0;
  int st;
  switch (epi) {
    case LTX_GEMM_EPI_BIAS: st = launch_epi<BKIND, LTX_GEMM_EPI_BIAS>(q, tile, s); break;
    case LTX_GEMM_EPI_GELU: st = launch_epi<BKIND, LTX_GEMM_EPI_GELU>(q, tile, s); break;
    case LTX_GEMM_EPI_RESIDUAL: st = launch_epi<BKIND, LTX_GEMM_EPI_RESIDUAL>(q, tile, s); break;
    case LTX_GEMM_EPI_RESIDUAL_ROUND: st = launch_epi<BKIND, LTX_GEMM_EPI_RESIDUAL_ROUND>(q, tile, s); break;
    case LTX_GEMM_EPI_SIGMOID2: st = launch_epi<BKIND, LTX_GEMM_EPI_SIGMOID2>(q, tile, s); break;
    case kEpiGeluMx:
      if constexpr (BKIND == B_MX) {
        st = launch_epi<BKIND, kEpiGeluMx>(q, tile, s);
        break;
      } else {
        return LTX_ERR_INVALID_ARG;
      }
    default: return LTX_ERR_INVALID_ARG;
  }
  if (st != LTX_OK) return st;
  return ltx_launch_status();
}

// ---- split-K ---------------------------------------------------------------
// Few-row products (the 68-token audio stream, the 256-token text contexts)
// give too few output tiles to fill 256 CUs, and each tile's K loop is a
// serial latency chain.  Split-K runs `splits` K ranges as separate blocks
// writing fp32 partial tiles; this kernel sums them in a fixed order (so the
// result is deterministic) and applies the same epilogue as the single-pass
// kernel's phases 1 and 2, eight columns per thread.
template <int EPI>
__global__ __launch_bounds__(256) void splitk_epilogue_kernel(GemmArgs p, int splits) {
  constexpr bool RESID = EPI == LTX_GEMM_EPI_RESIDUAL || EPI == LTX_GEMM_EPI_RESIDUAL_ROUND;
  const int nvec = p.N / 8;
  const int64_t total = (int64_t)p.M * nvec;
  const int64_t plane = (int64_t)p.M * p.N;
  const bool rtb = p.round_then_bias != 0;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int m = (int)(idx / nvec);
    const int n = (int)(idx % nvec) * 8;
    float a[8];
    {
      const float* P = p.partial + (int64_t)m * p.N + n;
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(P);
      const f32x4 x1 = *reinterpret_cast<const f32x4*>(P + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a[e] = x0[e];
        a[4 + e] = x1[e];
      }
      for (int z = 1; z < splits; ++z) {
        const f32x4 y0 = *reinterpret_cast<const f32x4*>(P + z * plane);
        const f32x4 y1 = *reinterpret_cast<const f32x4*>(P + z * plane + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          a[e] += y0[e];
          a[4 + e] += y1[e];
        }
      }
    }
    bf16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float b = p.bias ? p.bias[n + e] : 0.0f;
      float y = (rtb ? round_bf(a[e]) : a[e]) + b;
      if (EPI == LTX_GEMM_EPI_GELU) y = gelu_tanh(round_bf(y));
      if (EPI == LTX_GEMM_EPI_SIGMOID2) y = sigmoid2_bf(round_bf(y));
      if (EPI == LTX_GEMM_EPI_BIAS && n + e >= p.sig_from) y = sigmoid2_bf(round_bf(y));
      v[e] = (bf16)y;
    }
    if constexpr (RESID) {
      const bf16x8 r = *reinterpret_cast<const bf16x8*>(p.R + (int64_t)m * p.ldr + n);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = (float)v[e], g = p.gate[n + e];
        const float o = EPI == LTX_GEMM_EPI_RESIDUAL ? fmaf(g, y, (float)r[e]) : round_bf(y * g) + (float)r[e];
        v[e] = (bf16)o;
      }
    }
    *reinterpret_cast<bf16x8*>(p.C + (int64_t)m * p.ldc + n) = v;
  }
}

template <int BKIND>
static int launch_splitk(const GemmArgs& p0, int epilogue, int splits, float* workspace, hipStream_t s) {
  const int epi = epilogue & 0xff;
  const int tile = (epilogue >> 8) & 0xf;
  if (tile != 0 && tile != 2) return LTX_ERR_UNSUPPORTED;  // 128x128 register-staged tiles
  GemmArgs p = p0;
  p.round_then_bias = (epilogue & LTX_GEMM_ROUND_THEN_BIAS) != 0;
  // pass 1: partial products, per-split depth K / splits, row stride N
  GemmArgs q = p;
  q.K = p.K / splits;
  q.partial = workspace;
  q.ldc = p.N;
  q.tiles_m = (p.M + 127) / 128;
  q.tiles_n = (p.N + 127) / 128;
  gemm_kernel<128, 128, 64, 2, BKIND, kEpiPartial, 0, LOAD_REG>
      <<<q.tiles_m * q.tiles_n * splits, kGemmThreads, 0, s>>>(q);
  // pass 2: sum + epilogue
  p.partial = workspace;
  const int64_t vecs = (int64_t)p.M * (p.N / 8);
  int blocks = (int)((vecs + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  switch (epi) {
    case LTX_GEMM_EPI_BIAS: splitk_epilogue_kernel<LTX_GEMM_EPI_BIAS><<<blocks, 256, 0, s>>>(p, splits); break;
    case LTX_GEMM_EPI_GELU: splitk_epilogue_kernel<LTX_GEMM_EPI_GELU><<<blocks, 256, 0, s>>>(p, splits); break;
    case LTX_GEMM_EPI_RESIDUAL:
      splitk_epilogue_kernel<LTX_GEMM_EPI_RESIDUAL><<<blocks, 256, 0, s>>>(p, splits);
      break;
    case LTX_GEMM_EPI_RESIDUAL_ROUND:
      splitk_epilogue_kernel<LTX_GEMM_EPI_RESIDUAL_ROUND><<<blocks, 256, 0, s>>>(p, splits);
      break;
    case LTX_GEMM_EPI_SIGMOID2:
      splitk_epilogue_kernel<LTX_GEMM_EPI_SIGMOID2><<<blocks, 256, 0, s>>>(p, splits);
      break;
    default: return LTX_ERR_INVALID_ARG;
  }
  return ltx_launch_status();
}

}  // namespace ltx

using namespace ltx;

static inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

static int gemm_check(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                      int64_t M, int64_t N, int64_t K, int epilogue, const void* R, int64_t ldr,
                      const float* gate, int b_elem_bytes) {
  if (!A || !B || !C || M < 0 || N < 0 || K < 0) return LTX_ERR_INVALID_ARG;
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > INT32_MAX / 2) return LTX_ERR_UNSUPPORTED;
  const int epi = epilogue & 0xff;
  if (epilogue & ~(0xfff | LTX_GEMM_ROUND_THEN_BIAS)) return LTX_ERR_INVALID_ARG;
  if ((epi == LTX_GEMM_EPI_RESIDUAL || epi == LTX_GEMM_EPI_RESIDUAL_ROUND) && (!R || !gate || ldr < N))
    return LTX_ERR_INVALID_ARG;
  if (K % 64 != 0 || N % 8 != 0) return LTX_ERR_UNSUPPORTED;
  if (lda < K || ldb < K || ldc < N) return LTX_ERR_INVALID_ARG;
  if (!al16(A) || !al16(B) || !al16(C) || lda % 8 || ldc % 8 || (ldb * b_elem_bytes) % 16 ||
      (R && (!al16(R) || ldr % 8)))
    return LTX_ERR_ALIGNMENT;
  return LTX_OK;
}

static GemmArgs make_args(const void* A, int64_t lda, const void* B, int64_t ldb, const void* bscale,
                          int64_t ld_scale, const float* bias, void* C, int64_t ldc, int64_t M,
                          int64_t N, int64_t K, const void* R, int64_t ldr, const float* gate,
                          int64_t sigmoid_from) {
  GemmArgs p;
  p.A = (const bf16*)A;
  p.lda = lda;
  p.B = B;
  p.ldb = ldb;
  p.bscale = bscale;
  p.ld_scale = ld_scale;
  p.bias = bias;
  p.C = (bf16*)C;
  p.ldc = ldc;
  p.R = (const bf16*)R;
  p.ldr = ldr;
  p.gate = gate;
  p.sig_from = (int)(sigmoid_from < N ? (sigmoid_from < 0 ? 0 : sigmoid_from) : N);
  p.round_then_bias = 0;
  p.partial = nullptr;
  p.ascale = nullptr;
  p.ld_ascale = 0;
  p.cscale = nullptr;
  p.ld_cscale = 0;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.tiles_m = p.tiles_n = 0;
  return p;
}

extern "C" int ltx_gemm_bf16(const void* A, int64_t lda, const void* W, int64_t ldw,
                             const float* bias, void* C, int64_t ldc, int64_t M, int64_t N,
                             int64_t K, int epilogue, const void* residual, int64_t ldr,
                             const float* gate, int64_t sigmoid_from, void* stream) {
  int st = gemm_check(A, lda, W, ldw, C, ldc, M, N, K, epilogue, residual, ldr, gate, 2);
  if (st != LTX_OK) return st;
  if (M == 0 || N == 0) return LTX_OK;
  if (K == 0) return LTX_ERR_UNSUPPORTED;
  GemmArgs p = make_args(A, lda, W, ldw, nullptr, 0, bias, C, ldc, M, N, K, residual, ldr, gate,
                         sigmoid_from);
  return launch_kind<B_BF16>(p, epilogue, (hipStream_t)stream);
}

extern "C" int ltx_gemm_w8a16_bf16(const void* A, int64_t lda, const int8_t* Wq, int64_t ldw,
                                   const float* w_scale, const float* bias, void* C, int64_t ldc,
                                   int64_t M, int64_t N, int64_t K, int epilogue,
                                   const void* residual, int64_t ldr, const float* gate,
                                   int64_t sigmoid_from, void* stream) {
  int st = gemm_check(A, lda, Wq, ldw, C, ldc, M, N, K, epilogue, residual, ldr, gate, 1);
  if (st != LTX_OK) return st;
  if (!w_scale) return LTX_ERR_INVALID_ARG;
  if (M == 0 || N == 0) return LTX_OK;
  if (K == 0) return LTX_ERR_UNSUPPORTED;
  GemmArgs p = make_args(A, lda, Wq, ldw, w_scale, 0, bias, C, ldc, M, N, K, residual, ldr, gate,
                         sigmoid_from);
  return launch_kind<B_INT8>(p, epilogue, (hipStream_t)stream);
}

extern "C" int ltx_gemm_mxfp8_bf16(const void* A, int64_t lda, const uint8_t* Wq, int64_t ldw,
                                   const uint8_t* w_scale, int64_t ld_scale, const float* bias,
                                   void* C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                                   int epilogue, const void* residual, int64_t ldr,
                                   const float* gate, int64_t sigmoid_from, void* stream) {
  int st = gemm_check(A, lda, Wq, ldw, C, ldc, M, N, K, epilogue, residual, ldr, gate, 1);
  if (st != LTX_OK) return st;
  if (!w_scale || ld_scale < K / 32) return LTX_ERR_INVALID_ARG;
  if (ld_scale % 4 || ((uintptr_t)w_scale & 3u)) return LTX_ERR_ALIGNMENT;  // scale words
  if (M == 0 || N == 0) return LTX_OK;
  if (K == 0) return LTX_ERR_UNSUPPORTED;
  GemmArgs p = make_args(A, lda, Wq, ldw, w_scale, ld_scale, bias, C, ldc, M, N, K, residual, ldr,
                         gate, sigmoid_from);
  return launch_kind<B_MXFP8>(p, epilogue, (hipStream_t)stream);
}

// The bias-epilogue product of one of the three weight formats (wformat 0:
// bf16 as ltx_gemm_bf16, 1: int8 as ltx_gemm_w8a16_bf16, 2: MXFP8 as
// ltx_gemm_mxfp8_bf16) with the per-row sums of squares of its bf16 outputs in
// columns [0, ss_cols): rowss[m * ld_rowss + j] = sum of C[m, n]^2 over
// n in [64 j, 64 j + 64).  Always the 8-wave kernel (its epilogue computes
// them); C is bit-identical to the plain entry point's on that kernel.
extern "C" int ltx_gemm_rowss_bf16(int wformat, const void* A, int64_t lda, const void* W, int64_t ldw,
                                   const void* w_scale, int64_t ld_scale, const float* bias, void* C,
                                   int64_t ldc, int64_t M, int64_t N, int64_t K, int epilogue,
                                   int64_t sigmoid_from, float* rowss, int64_t ld_rowss, int64_t ss_cols,
                                   void* stream) {
  if (wformat < 0 || wformat > 2) return LTX_ERR_INVALID_ARG;
  if ((epilogue & 0xff) != LTX_GEMM_EPI_BIAS) return LTX_ERR_INVALID_ARG;
  const int tile = (epilogue >> 8) & 0xf;
  if (tile != 0 && tile != 5 && tile != 6) return LTX_ERR_UNSUPPORTED;
  int st = gemm_check(A, lda, W, ldw, C, ldc, M, N, K, epilogue, nullptr, 0, nullptr, wformat == 0 ? 2 : 1);
  if (st != LTX_OK) return st;
  if (!rowss || ss_cols <= 0 || ss_cols % 64 || ss_cols > N || ss_cols > sigmoid_from || ld_rowss < ss_cols / 64)
    return LTX_ERR_INVALID_ARG;
  if (((uintptr_t)rowss & 3u) != 0) return LTX_ERR_ALIGNMENT;
  if (M > 0 && ld_rowss > (INT64_MAX / M)) return LTX_ERR_UNSUPPORTED;
  if (wformat == 1 && !w_scale) return LTX_ERR_INVALID_ARG;
  if (wformat == 2) {
    if (!w_scale || ld_scale < K / 32) return LTX_ERR_INVALID_ARG;
    if (ld_scale % 4 || ((uintptr_t)w_scale & 3u)) return LTX_ERR_ALIGNMENT;
  }
  if (M == 0 || N == 0) return LTX_OK;
  if (K == 0) return LTX_ERR_UNSUPPORTED;
  GemmArgs p = make_args(A, lda, W, ldw, wformat == 0 ? nullptr : w_scale, wformat == 2 ? ld_scale : 0, bias, C,
                         ldc, M, N, K, nullptr, 0, nullptr, sigmoid_from);
  p.rowss = rowss;
  p.ld_rowss = ld_rowss;
  p.ss_cols = (int)ss_cols;
  if (wformat == 0) return launch_kind<B_BF16>(p, epilogue, (hipStream_t)stream);
  if (wformat == 1) return launch_kind<B_INT8>(p, epilogue, (hipStream_t)stream);
  return launch_kind<B_MXFP8>(p, epilogue, (hipStream_t)stream);
}

// ---- split-K entry points ------------------------------------------------------
// MXFP8 activations x MXFP8 weights on the scaled fp8 MFMA (opt-in; no
// counterpart in the reference, whose MXFP8 path dequantises the weights and
// multiplies bf16 activations).  A: E4M3 codes (M, K) with row stride lda
// bytes and E8M0 scales (M, K/32) with row stride ld_ascale, as written by
// ltx_quantize_mxfp8_bf16 on the activation rows; W, w_scale as
// ltx_gemm_mxfp8_bf16.  Same epilogues and quantised-linear rounding flag.
extern "C" int ltx_gemm_mx_bf16(const uint8_t* A, int64_t lda, const uint8_t* a_scale, int64_t ld_ascale,
                                const uint8_t* Wq, int64_t ldw, const uint8_t* w_scale, int64_t ld_scale,
                                const float* bias, void* C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                                int epilogue, const void* residual, int64_t ldr, const float* gate,
                                int64_t sigmoid_from, void* stream) {
  if (!A || !a_scale || !Wq || !w_scale || !C || M < 0 || N < 0 || K < 0) return LTX_ERR_INVALID_ARG;
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > INT32_MAX / 2) return LTX_ERR_UNSUPPORTED;
  const int epi = epilogue & 0xff;
  if (epilogue & ~(0xfff | LTX_GEMM_ROUND_THEN_BIAS)) return LTX_ERR_INVALID_ARG;
  if (epi > LTX_GEMM_EPI_SIGMOID2) return LTX_ERR_INVALID_ARG;
  if ((epi == LTX_GEMM_EPI_RESIDUAL || epi == LTX_GEMM_EPI_RESIDUAL_ROUND) && (!residual || !gate || ldr < N))
    return LTX_ERR_INVALID_ARG;
  if (lda < K || ldw < K || ldc < N || ld_ascale < K / 32 || ld_scale < K / 32) return LTX_ERR_INVALID_ARG;
  if (K % 512 != 0 || N % 8 != 0) return LTX_ERR_UNSUPPORTED;
  if (!al16(A) || !al16(Wq) || !al16(C) || !al16(a_scale) || !al16(w_scale) || lda % 16 || ldw % 16 ||
      ldc % 8 || ld_ascale % 16 || ld_scale % 16 || (residual && (!al16(residual) || ldr % 8)))
    return LTX_ERR_ALIGNMENT;
  if (M == 0 || N == 0) return LTX_OK;
  GemmArgs p = make_args(A, lda, Wq, ldw, w_scale, ld_scale, bias, C, ldc, M, N, K, residual, ldr, gate,
                         sigmoid_from);
  p.ascale = a_scale;
  p.ld_ascale = ld_ascale;
  return launch_kind<B_MX>(p, epilogue, (hipStream_t)stream);
}

// The MX path's feed-forward up-projection: GELU epilogue whose bf16 result
// is written as MXFP8 rows -- codes (M, N) with row stride ldcq bytes, E8M0
// scales (M, N/32) -- the quantised input of the down-projection, bit for bit
// what ltx_quantize_mxfp8_bf16 makes of the bf16 GELU output.
extern "C" int ltx_gemm_mx_gelu_mxfp8(const uint8_t* A, int64_t lda, const uint8_t* a_scale, int64_t ld_ascale,
                                      const uint8_t* Wq, int64_t ldw, const uint8_t* w_scale, int64_t ld_scale,
                                      const float* bias, uint8_t* Cq, int64_t ldcq, uint8_t* c_scale,
                                      int64_t ld_cscale, int64_t M, int64_t N, int64_t K, int flags,
                                      void* stream) {
  if (!A || !a_scale || !Wq || !w_scale || !Cq || !c_scale || M < 0 || N < 0 || K < 0)
    return LTX_ERR_INVALID_ARG;
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > INT32_MAX / 2) return LTX_ERR_UNSUPPORTED;
  if (flags & ~LTX_GEMM_ROUND_THEN_BIAS) return LTX_ERR_INVALID_ARG;
  if (lda < K || ldw < K || ldcq < N || ld_ascale < K / 32 || ld_scale < K / 32 || ld_cscale < N / 32)
    return LTX_ERR_INVALID_ARG;
  if (K % 512 != 0 || N % 32 != 0) return LTX_ERR_UNSUPPORTED;
  if (!al16(A) || !al16(Wq) || !al16(Cq) || !al16(a_scale) || !al16(w_scale) || lda % 16 || ldw % 16 ||
      ldcq % 8 || ld_ascale % 16 || ld_scale % 16)
    return LTX_ERR_ALIGNMENT;
  if (M == 0 || N == 0) return LTX_OK;
  GemmArgs p = make_args(A, lda, Wq, ldw, w_scale, ld_scale, bias, Cq, ldcq, M, N, K, nullptr, 0, nullptr, N);
  p.ascale = a_scale;
  p.ld_ascale = ld_ascale;
  p.cscale = c_scale;
  p.ld_cscale = ld_cscale;
  return launch_kind<B_MX>(p, kEpiGeluMx | flags, (hipStream_t)stream);
}

extern "C" int64_t ltx_gemm_splitk_workspace_bytes(int64_t M, int64_t N, int64_t splits) {
  if (M < 0 || N < 0 || splits < 1) return -1;
  return splits * M * N * 4;
}

static int splitk_check(int64_t M, int64_t N, int64_t K, int splits, const float* workspace,
                        int64_t workspace_bytes) {
  if (splits < 1 || splits > 64) return LTX_ERR_INVALID_ARG;
  if (K % (64 * (int64_t)splits)) return LTX_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < ltx_gemm_splitk_workspace_bytes(M, N, splits)) return LTX_ERR_INVALID_ARG;
  if (!al16(workspace)) return LTX_ERR_ALIGNMENT;
  return LTX_OK;
}

extern "C" int ltx_gemm_splitk_bf16(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias,
                                    void* C, int64_t ldc, int64_t M, int64_t N, int64_t K, int epilogue,
                                    const void* residual, int64_t ldr, const float* gate, int64_t sigmoid_from,
                                    int splits, float* workspace, int64_t workspace_bytes, void* stream) {
  int st = gemm_check(A, lda, W, ldw, C, ldc, M, N, K, epilogue, residual, ldr, gate, 2);
  if (st != LTX_OK) return st;
  if (M == 0 || N == 0) return LTX_OK;
  if (K == 0) return LTX_ERR_UNSUPPORTED;
  if ((st = splitk_check(M, N, K, splits, workspace, workspace_bytes)) != LTX_OK) return st;
  GemmArgs p = make_args(A, lda, W, ldw, nullptr, 0, bias, C, ldc, M, N, K, residual, ldr, gate, sigmoid_from);
  return launch_splitk<B_BF16>(p, epilogue, splits, workspace, (hipStream_t)stream);
}

extern "C" int ltx_gemm_splitk_w8a16_bf16(const void* A, int64_t lda, const int8_t* Wq, int64_t ldw,
                                          const float* w_scale, const float* bias, void* C, int64_t ldc,
                                          int64_t M, int64_t N, int64_t K, int epilogue, const void* residual,
                                          int64_t ldr, const float* gate, int64_t sigmoid_from, int splits,
                                          float* workspace, int64_t workspace_bytes, void* stream) {
  int st = gemm_check(A, lda, Wq, ldw, C, ldc, M, N, K, epilogue, residual, ldr, gate, 1);
  if (st != LTX_OK) return st;
  if (!w_scale) return LTX_ERR_INVALID_ARG;
  if (M == 0 || N == 0) return LTX_OK;
  if (K == 0) return LTX_ERR_UNSUPPORTED;
  if ((st = splitk_check(M, N, K, splits, workspace, workspace_bytes)) != LTX_OK) return st;
  GemmArgs p = make_args(A, lda, Wq, ldw, w_scale, 0, bias, C, ldc, M, N, K, residual, ldr, gate, sigmoid_from);
  return launch_splitk<B_INT8>(p, epilogue, splits, workspace, (hipStream_t)stream);
}

extern "C" int ltx_gemm_splitk_mxfp8_bf16(const void* A, int64_t lda, const uint8_t* Wq, int64_t ldw,
                                          const uint8_t* w_scale, int64_t ld_scale, const float* bias, void* C,
                                          int64_t ldc, int64_t M, int64_t N, int64_t K, int epilogue,
                                          const void* residual, int64_t ldr, const float* gate,
                                          int64_t sigmoid_from, int splits, float* workspace,
                                          int64_t workspace_bytes, void* stream) {
  int st = gemm_check(A, lda, Wq, ldw, C, ldc, M, N, K, epilogue, residual, ldr, gate, 1);
  if (st != LTX_OK) return st;
  if (!w_scale || ld_scale < K / 32) return LTX_ERR_INVALID_ARG;
  if (ld_scale % 4 || ((uintptr_t)w_scale & 3u)) return LTX_ERR_ALIGNMENT;
  if (M == 0 || N == 0) return LTX_OK;
  if (K == 0) return LTX_ERR_UNSUPPORTED;
  if ((st = splitk_check(M, N, K, splits, workspace, workspace_bytes)) != LTX_OK) return st;
  if (K % (128 * (int64_t)splits)) return LTX_ERR_UNSUPPORTED;  // each split's scale words stay 4-byte aligned
  GemmArgs p = make_args(A, lda, Wq, ldw, w_scale, ld_scale, bias, C, ldc, M, N, K, residual, ldr, gate,
                         sigmoid_from);
  return launch_splitk<B_MXFP8>(p, epilogue, splits, workspace, (hipStream_t)stream);
}
