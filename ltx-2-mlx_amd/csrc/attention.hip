// Flash attention for the DiT block on CDNA4 matrix cores.
//
//   out[q, h*dh:(h+1)*dh] = gate[q, h] * softmax(Q_h K_h^T / sqrt(dh)) V_h
//
// Replaces the attention core of the reference (model/transformer/
// attention.py:170-302 -> kernels/steel_attention.py:251-280 STEEL kernel or
// mx.fast.scaled_dot_product_attention), fused with the per-head output gate
// of attention.py:594-598 (out = bf16(bf16(O) * gate)).  bf16 inputs, fp32
// scores / online softmax / accumulators, bf16 P for the second product (as
// the STEEL kernel, metal/steel_attention_ltx_body.metal:113-177), no mask.
//
// Layouts (token-major, as produced by the projections):
//   Q: (Tq, H*dh) with row stride q_rs; K: (Tk, H*dh) with row stride k_rs;
//   V is consumed pre-transposed by ltx_attn_transpose_v_bf16 into
//   Vt (H, dh, Tk_pad), Tk_pad = ceil(Tk/64)*64, zero-padded, with the keys of
//   every 16-key group permuted so that each lane's 8 keys of a P.V fragment
//   are contiguous (see vt_position).
//
// Kernel structure: one workgroup = 4 waves = 256 queries of one head; each
// wave owns 64 queries.  Scores are computed transposed, S^T = K Q^T, with
// v_mfma_f32_32x32x16_bf16: each lane then holds one query's scores in
// registers, so the row max / row sum are lane-local plus one cross-half
// shuffle, and P^T feeds the P.V MFMA straight from registers
// (O^T += Vt . P^T).  K and Vt stream through LDS in 64-key stages by direct
// global->LDS DMA, double buffered.  Workgroups of one head are numbered
// contiguously per XCD so its K/V stay in that XCD's L2.
#include "ltx_common.h"

namespace ltx {

constexpr int kAttnThreads = 256;
constexpr int kAttnQ = 256;      // queries per workgroup
constexpr int kAttnKB = 64;      // keys per stage
constexpr int kNumXcdAttn = 8;

typedef __attribute__((address_space(3))) void* lds_ptr_a;
typedef __attribute__((address_space(1))) const void* gbl_ptr_a;

__device__ __forceinline__ void adma16(const void* src, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((gbl_ptr_a)src, (lds_ptr_a)lds_wave_base, 16, 0, 0);
}

// Position of key j (0..15 within its 16-key group) in the permuted Vt row:
// MFMA k index 8h+e of a P.V step covers key 8*(e/4) + 4h + e%4.
__host__ __device__ __forceinline__ int vt_position(int j) {
  const int hi8 = j >> 3, h = (j >> 2) & 1, e4 = j & 3;
  return 8 * h + 4 * hi8 + e4;
}

template <int DH>
struct AttnCfg {
  static constexpr int DSTEPS = DH / 16;   // k-steps of S = K Q^T
  static constexpr int DTILES = DH / 32;   // 32-row tiles of O^T
  static constexpr int K_ROWB = DH * 2;    // bytes per K row in LDS
  static constexpr int K_BYTES = kAttnKB * K_ROWB;
  static constexpr int V_ROWB = kAttnKB * 2;  // 128 B per Vt row (64 keys)
  static constexpr int V_BYTES = DH * V_ROWB;
  static constexpr int STAGE = K_BYTES + V_BYTES;
  static constexpr int K_DMA = K_BYTES / 1024 / 4;  // per-lane DMA instructions per stage
  static constexpr int V_DMA = V_BYTES / 1024 / 4;
};

template <int DH, bool GATED>
__global__ __launch_bounds__(kAttnThreads, 1) void flash_attn_kernel(
    const bf16* __restrict__ Q, int64_t q_rs, const bf16* __restrict__ K, int64_t k_rs,
    const bf16* __restrict__ Vt, int64_t tk_pad, bf16* __restrict__ O, int64_t o_rs,
    const bf16* __restrict__ G, int64_t g_rs, int Tq, int Tk, int H, float scale_log2) {
  using Cfg = AttnCfg<DH>;
  constexpr int DSTEPS = Cfg::DSTEPS, DTILES = Cfg::DTILES;
  constexpr int K_ROWB = Cfg::K_ROWB, K_BYTES = Cfg::K_BYTES, V_ROWB = Cfg::V_ROWB;
  constexpr int STAGE = Cfg::STAGE, K_DMA = Cfg::K_DMA, V_DMA = Cfg::V_DMA;
  __shared__ __attribute__((aligned(1024))) char lds[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hh = lane >> 5, l32 = lane & 31;

  // workgroup -> (head, query tile); a head's tiles are contiguous per XCD
  const int qtiles = (Tq + kAttnQ - 1) / kAttnQ;
  const int nwg = gridDim.x;
  const int qd = nwg / kNumXcdAttn, rm = nwg % kNumXcdAttn;
  const int xcd = blockIdx.x % kNumXcdAttn, idx = blockIdx.x / kNumXcdAttn;
  const int logical = xcd * qd + (xcd < rm ? xcd : rm) + idx;
  const int head = logical / qtiles;
  const int q0 = (logical % qtiles) * kAttnQ + wave * 64;

  const bf16* Kh = K + (int64_t)head * DH;
  const bf16* Vh = Vt + (int64_t)head * DH * tk_pad;

  // ---- Q^T fragments: lane holds Q[q][dstep*16 + hh*8 .. +8] for its query
  bf16x8 qf[2][DSTEPS];
#pragma unroll
  for (int qa = 0; qa < 2; ++qa) {
    int q = q0 + qa * 32 + l32;
    q = q < Tq ? q : Tq - 1;
    const bf16* qrow = Q + (int64_t)q * q_rs + (int64_t)head * DH + hh * 8;
#pragma unroll
    for (int s = 0; s < DSTEPS; ++s) qf[qa][s] = *reinterpret_cast<const bf16x8*>(qrow + s * 16);
  }

  // ---- DMA sources.  K: 1 KiB per wave instruction = 1024/K_ROWB rows.
  constexpr int K_ROWS_PER = 1024 / K_ROWB;      // 4 (dh 128) or 8 (dh 64)
  constexpr int K_CH = K_ROWB / 16;               // 16-byte chunks per row
  const char* k_src[K_DMA];
  int k_row[K_DMA];
#pragma unroll
  for (int i = 0; i < K_DMA; ++i) {
    const int r = K_ROWS_PER * (4 * i + wave) + lane / K_CH;
    const int slot = lane % K_CH;
    const int chunk = (K_CH == 16) ? (slot ^ (r & 15)) : (slot ^ ((r >> 1) & 7));
    k_row[i] = r;
    k_src[i] = (const char*)(Kh) + chunk * 16;
  }
  // Vt: rows of 128 B (64 keys), 8 rows per wave instruction.
  const char* v_src[V_DMA];
#pragma unroll
  for (int i = 0; i < V_DMA; ++i) {
    const int r = 8 * (4 * i + wave) + (lane >> 3);
    const int chunk = (lane & 7) ^ ((r >> 1) & 7);
    v_src[i] = (const char*)(Vh + (int64_t)r * tk_pad) + chunk * 16;
  }

  const int nblocks = (Tk + kAttnKB - 1) / kAttnKB;
  auto issue = [&](int kb, int buf) {
    char* Ks = lds + buf * STAGE;
    char* Vs = Ks + K_BYTES;
#pragma unroll
    for (int i = 0; i < K_DMA; ++i) {
      int key = kb * kAttnKB + k_row[i];
      key = key < Tk ? key : Tk - 1;
      adma16(k_src[i] + (int64_t)key * k_rs * 2, Ks + (4 * i + wave) * 1024);
    }
#pragma unroll
    for (int i = 0; i < V_DMA; ++i) adma16(v_src[i] + (int64_t)kb * kAttnKB * 2, Vs + (4 * i + wave) * 1024);
  };

  f32x16 acc[2][DTILES];
#pragma unroll
  for (int qa = 0; qa < 2; ++qa)
#pragma unroll
    for (int t = 0; t < DTILES; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[qa][t][e] = 0.0f;
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.0f, 0.0f};

  // fragment-read offsets
  int k_off[2];
#pragma unroll
  for (int sb = 0; sb < 2; ++sb) k_off[sb] = (sb * 32 + l32) * K_ROWB;
  const int k_swz = (K_CH == 16) ? (l32 & 15) : ((l32 >> 1) & 7);  // rows sb*32+l32 share it
  int v_off[DTILES];
#pragma unroll
  for (int t = 0; t < DTILES; ++t) v_off[t] = (t * 32 + l32) * V_ROWB;
  const int v_swz = (l32 >> 1) & 7;

  issue(0, 0);
  for (int kb = 0; kb < nblocks; ++kb) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (kb + 1 < nblocks) issue(kb + 1, (kb + 1) & 1);
    const char* Ks = lds + (kb & 1) * STAGE;
    const char* Vs = Ks + K_BYTES;

    // ---- S^T = K Q^T for two 32-key sub-blocks x two 32-query tiles
    f32x16 s[2][2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int qa = 0; qa < 2; ++qa)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[sb][qa][e] = 0.0f;
#pragma unroll
    for (int ds = 0; ds < DSTEPS; ++ds) {
      const int c = ((ds * 2 + hh) ^ k_swz) * 16;
      bf16x8 kf[2];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) kf[sb] = *reinterpret_cast<const bf16x8*>(Ks + k_off[sb] + c);
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int qa = 0; qa < 2; ++qa)
          s[sb][qa] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[sb], qf[qa][ds], s[sb][qa], 0, 0, 0);
    }

    // ---- online softmax (log2 domain); lane owns one query per qa
    const bool tail = (kb + 1) * kAttnKB > Tk;
#pragma unroll
    for (int qa = 0; qa < 2; ++qa) {
      float mx = -INFINITY;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v = s[sb][qa][r] * scale_log2;
          if (tail) {
            const int key = kb * kAttnKB + sb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
            if (key >= Tk) v = -INFINITY;
          }
          s[sb][qa][r] = v;
          mx = fmaxf(mx, v);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run[qa], mx);
      const float alpha = exp2f(m_run[qa] - m_new);
      float rs = 0.0f;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = exp2f(s[sb][qa][r] - m_new);
          s[sb][qa][r] = p;
          rs += p;
        }
      rs += __shfl_xor(rs, 32, 64);
      l_run[qa] = l_run[qa] * alpha + rs;
      m_run[qa] = m_new;
#pragma unroll
      for (int t = 0; t < DTILES; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[qa][t][e] *= alpha;
    }

    // ---- O^T += Vt . P^T  (P^T fragment of step (sb, st) = S regs 8st..8st+7)
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        bf16x8 pf[2];
#pragma unroll
        for (int qa = 0; qa < 2; ++qa)
#pragma unroll
          for (int e = 0; e < 8; ++e) pf[qa][e] = (bf16)s[sb][qa][8 * st + e];
        const int chunk = sb * 4 + st * 2 + hh;  // 16-byte chunk of the 64-key row
#pragma unroll
        for (int t = 0; t < DTILES; ++t) {
          const bf16x8 vf = *reinterpret_cast<const bf16x8*>(Vs + v_off[t] + ((chunk ^ v_swz) * 16));
#pragma unroll
          for (int qa = 0; qa < 2; ++qa)
            acc[qa][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[qa], acc[qa][t], 0, 0, 0);
        }
      }
    }
  }

  // ---- epilogue: O = O^T / l, optional per-head gate, 4 bf16 per store
#pragma unroll
  for (int qa = 0; qa < 2; ++qa) {
    const int q = q0 + qa * 32 + l32;
    if (q >= Tq) continue;
    const float inv_l = 1.0f / l_run[qa];
    float g = 1.0f;
    if (GATED) g = (float)G[(int64_t)q * g_rs + head];
    bf16* orow = O + (int64_t)q * o_rs + (int64_t)head * DH;
#pragma unroll
    for (int t = 0; t < DTILES; ++t)
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float o = round_bf(acc[qa][t][4 * grp + e] * inv_l);
          if (GATED) o = o * g;
          v[e] = (bf16)o;
        }
        *reinterpret_cast<bf16x4*>(orow + t * 32 + 8 * grp + 4 * hh) = v;
      }
  }
}

// V (Tk, H*dh) token-major -> Vt (H, dh, Tk_pad), keys permuted per 16-group,
// padded keys zero.  One workgroup transposes a 64-key x dh tile of one head
// through LDS.
template <int DH>
__global__ __launch_bounds__(256) void transpose_v_kernel(const bf16* __restrict__ V, int64_t v_rs,
                                                          bf16* __restrict__ Vt, int64_t tk_pad, int Tk,
                                                          int H) {
  __shared__ bf16 tile[64][DH + 2];
  const int kb = blockIdx.x, head = blockIdx.y;
  const int tid = threadIdx.x;
  // load 64 rows x DH (8 bf16 per thread per step)
  constexpr int CH = DH / 8;
  for (int i = tid; i < 64 * CH; i += 256) {
    const int r = i / CH, c = i % CH;
    const int key = kb * 64 + r;
    bf16x8 v;
    if (key < Tk) {
      v = *reinterpret_cast<const bf16x8*>(V + (int64_t)key * v_rs + (int64_t)head * DH + c * 8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (bf16)0.0f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[r][c * 8 + e] = v[e];
  }
  __syncthreads();
  // write DH rows x 64 keys; element (d, pos) takes key group*16 + j with
  // vt_position(j) == pos%16
  for (int i = tid; i < DH * 8; i += 256) {
    const int d = i / 8, c = i % 8;  // chunk c = positions 8c .. 8c+7
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int pos = c * 8 + e;
      const int grp = pos >> 4, p16 = pos & 15;
      // invert vt_position: p16 = 8h + 4*hi8 + e4
      const int h = p16 >> 3, hi8 = (p16 >> 2) & 1, e4 = p16 & 3;
      const int j = 8 * hi8 + 4 * h + e4;
      o[e] = tile[grp * 16 + j][d];
    }
    *reinterpret_cast<bf16x8*>(Vt + ((int64_t)head * DH + d) * tk_pad + (int64_t)kb * 64 + c * 8) = o;
  }
}

}  // namespace ltx

using namespace ltx;

static inline bool al16a(const void* p) { return ((uintptr_t)p & 15u) == 0; }

extern "C" int64_t ltx_attn_vt_padded_len(int64_t Tk) { return (Tk + 63) / 64 * 64; }

extern "C" int ltx_attn_transpose_v_bf16(const void* V, int64_t v_rs, int64_t Tk, int64_t H,
                                         int64_t head_dim, void* Vt, int64_t tk_pad, void* stream) {
  if (!V || !Vt || Tk <= 0 || H <= 0) return LTX_ERR_INVALID_ARG;
  if (head_dim != 64 && head_dim != 128) return LTX_ERR_UNSUPPORTED;
  if (tk_pad < ltx_attn_vt_padded_len(Tk) || tk_pad % 64 || v_rs < H * head_dim) return LTX_ERR_INVALID_ARG;
  if (!al16a(V) || !al16a(Vt) || v_rs % 8) return LTX_ERR_ALIGNMENT;
  if (Tk > INT32_MAX || H > 65535) return LTX_ERR_UNSUPPORTED;
  dim3 grid((unsigned)(tk_pad / 64), (unsigned)H);
  if (head_dim == 128)
    transpose_v_kernel<128><<<grid, 256, 0, (hipStream_t)stream>>>((const bf16*)V, v_rs, (bf16*)Vt, tk_pad, (int)Tk, (int)H);
  else
    transpose_v_kernel<64><<<grid, 256, 0, (hipStream_t)stream>>>((const bf16*)V, v_rs, (bf16*)Vt, tk_pad, (int)Tk, (int)H);
  return ltx_launch_status();
}

extern "C" int ltx_flash_attn_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs,
                                   const void* Vt, int64_t tk_pad, void* O, int64_t o_rs,
                                   const void* gate, int64_t gate_rs, int64_t Tq, int64_t Tk,
                                   int64_t H, int64_t head_dim, float scale, void* stream) {
  if (!Q || !K || !Vt || !O || Tq < 0 || Tk <= 0 || H <= 0) return LTX_ERR_INVALID_ARG;
  if (head_dim != 64 && head_dim != 128) return LTX_ERR_UNSUPPORTED;
  if (tk_pad < ltx_attn_vt_padded_len(Tk) || tk_pad % 64) return LTX_ERR_INVALID_ARG;
  if (q_rs < H * head_dim || k_rs < H * head_dim || o_rs < H * head_dim) return LTX_ERR_INVALID_ARG;
  if (gate && gate_rs < H) return LTX_ERR_INVALID_ARG;
  if (!al16a(Q) || !al16a(K) || !al16a(Vt) || !al16a(O) || q_rs % 8 || k_rs % 8 || o_rs % 8)
    return LTX_ERR_ALIGNMENT;
  if (Tq > INT32_MAX || Tk > INT32_MAX) return LTX_ERR_UNSUPPORTED;
  if (Tq == 0) return LTX_OK;
  const int64_t qtiles = (Tq + kAttnQ - 1) / kAttnQ;
  const int64_t nwg = qtiles * H;
  if (nwg > INT32_MAX) return LTX_ERR_UNSUPPORTED;
  const float scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = (hipStream_t)stream;
#define LTX_FA(DH, G)                                                                        \
  flash_attn_kernel<DH, G><<<(int)nwg, kAttnThreads, 0, s>>>(                                \
      (const bf16*)Q, q_rs, (const bf16*)K, k_rs, (const bf16*)Vt, tk_pad, (bf16*)O, o_rs,    \
      (const bf16*)gate, gate_rs, (int)Tq, (int)Tk, (int)H, scale_log2)
  if (head_dim == 128) {
    if (gate) LTX_FA(128, true); else LTX_FA(128, false);
  } else {
    if (gate) LTX_FA(64, true); else LTX_FA(64, false);
  }
#undef LTX_FA
  return ltx_launch_status();
}
