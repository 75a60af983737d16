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
// Kernel structure: one workgroup = 8 waves = 256 queries of one head; each
// wave owns 32 queries, two waves share a SIMD, so one wave's softmax (VALU,
// transcendental) overlaps the other's matrix work.  Scores are computed
// transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16: each lane then
// holds one query's scores in registers, so the row max / row sum are
// lane-local plus one cross-half shuffle, and P^T feeds the P.V MFMA straight
// from registers (O^T += Vt . P^T).  K and Vt stream through LDS in 64-key
// stages by direct global->LDS DMA, double buffered.  The running max is
// raised only when a block's max exceeds it by more than 2^8 (P then stays
// <= 256, exact in fp32 and bf16-relative as any other P), so the O^T
// rescale runs in the first blocks and then almost never.  Workgroups of one
// head are numbered contiguously per XCD so its K/V stay in that XCD's L2.
#include "ltx_common.h"

namespace ltx {

constexpr int kAttnWaves = 8;            // full-size tiles: 8 waves = 256 queries
constexpr int kAttnSplitWaves = 4;       // split-KV tiles: 4 waves = 128 queries
constexpr int kAttnKB = 64;              // keys per stage
constexpr int kNumXcdAttn = 8;
constexpr float kLazyMax = 8.0f;         // log2 headroom before the max is raised

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

template <int DH, int WAVES>
struct AttnCfg {
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int QT = 32 * WAVES;    // queries per workgroup
  static constexpr int DSTEPS = DH / 16;   // k-steps of S = K Q^T
  static constexpr int DTILES = DH / 32;   // 32-row tiles of O^T
  static constexpr int K_ROWB = DH * 2;    // bytes per K row in LDS
  static constexpr int K_BYTES = kAttnKB * K_ROWB;
  static constexpr int V_ROWB = kAttnKB * 2;  // 128 B per Vt row (64 keys)
  static constexpr int V_BYTES = DH * V_ROWB;
  static constexpr int STAGE = K_BYTES + V_BYTES;
  // per-lane DMA instructions per stage (a wave instruction moves 1 KiB)
  static constexpr int K_DMA = K_BYTES / 1024 / WAVES;
  static constexpr int V_DMA = V_BYTES / 1024 / WAVES;
  static_assert(K_DMA >= 1 && V_DMA >= 1, "stage split over the waves");
};

// Split-KV partial results: key range `split` of (query, head) leaves its
// unnormalised O (fp32, scaled by 2^-m), running max m (log2 domain) and
// running sum l, combined by attn_combine_kernel.
struct SplitOut {
  float* o;  // (splits, Tq, H, dh)
  float* m;  // (splits, Tq, H)
  float* l;  // (splits, Tq, H)
  int splits;
};

template <int DH, bool GATED, int WAVES, bool SPLIT>
__global__ __launch_bounds__(64 * WAVES, 1) void flash_attn_kernel(
    const bf16* __restrict__ Q, int64_t q_rs, const bf16* __restrict__ K, int64_t k_rs,
    const bf16* __restrict__ Vt, int64_t tk_pad, bf16* __restrict__ O, int64_t o_rs,
    const bf16* __restrict__ G, int64_t g_rs, int Tq, int Tk, int H, float scale_log2, SplitOut so) {
  using Cfg = AttnCfg<DH, WAVES>;
  constexpr int kAttnQ = Cfg::QT;
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
  const int nsplit = SPLIT ? so.splits : 1;
  const int split = SPLIT ? logical % nsplit : 0;
  const int work = SPLIT ? logical / nsplit : logical;
  const int head = work / qtiles;
  const int q0 = (work % qtiles) * kAttnQ + wave * 32;

  const bf16* Kh = K + (int64_t)head * DH;
  const bf16* Vh = Vt + (int64_t)head * DH * tk_pad;

  // ---- Q^T fragments: lane holds Q[q][dstep*16 + hh*8 .. +8] for its query
  bf16x8 qf[DSTEPS];
  {
    int q = q0 + l32;
    q = q < Tq ? q : Tq - 1;
    const bf16* qrow = Q + (int64_t)q * q_rs + (int64_t)head * DH + hh * 8;
#pragma unroll
    for (int s = 0; s < DSTEPS; ++s) qf[s] = *reinterpret_cast<const bf16x8*>(qrow + s * 16);
  }

  // ---- DMA sources.  Wave instruction i fills the 1 KiB LDS block
  // kAttnWaves*i + wave.  K: 1024/K_ROWB rows per block.
  constexpr int K_ROWS_PER = 1024 / K_ROWB;      // 4 (dh 128) or 8 (dh 64)
  constexpr int K_CH = K_ROWB / 16;               // 16-byte chunks per row
  const char* k_src[K_DMA];
  int k_row[K_DMA];
#pragma unroll
  for (int i = 0; i < K_DMA; ++i) {
    const int r = K_ROWS_PER * (WAVES * i + wave) + lane / K_CH;
    const int slot = lane % K_CH;
    const int chunk = (K_CH == 16) ? (slot ^ (r & 15)) : (slot ^ ((r >> 1) & 7));
    k_row[i] = r;
    k_src[i] = (const char*)(Kh) + chunk * 16;
  }
  // Vt: rows of 128 B (64 keys), 8 rows per block.
  const char* v_src[V_DMA];
#pragma unroll
  for (int i = 0; i < V_DMA; ++i) {
    const int r = 8 * (WAVES * i + wave) + (lane >> 3);
    const int chunk = (lane & 7) ^ ((r >> 1) & 7);
    v_src[i] = (const char*)(Vh + (int64_t)r * tk_pad) + chunk * 16;
  }

  const int nblocks_all = (Tk + kAttnKB - 1) / kAttnKB;
  // key blocks [kb0, kb1) of this workgroup
  const int per_split = (nblocks_all + nsplit - 1) / nsplit;
  const int kb0 = split * per_split;
  const int kb1 = (kb0 + per_split) < nblocks_all ? (kb0 + per_split) : nblocks_all;
  auto issue = [&](int kb, int buf) {
    char* Ks = lds + buf * STAGE;
    char* Vs = Ks + K_BYTES;
#pragma unroll
    for (int i = 0; i < K_DMA; ++i) {
      int key = kb * kAttnKB + k_row[i];
      key = key < Tk ? key : Tk - 1;
      adma16(k_src[i] + (int64_t)key * k_rs * 2, Ks + (WAVES * i + wave) * 1024);
    }
#pragma unroll
    for (int i = 0; i < V_DMA; ++i)
      adma16(v_src[i] + (int64_t)kb * kAttnKB * 2, Vs + (WAVES * i + wave) * 1024);
  };

  f32x16 acc[DTILES];
#pragma unroll
  for (int t = 0; t < DTILES; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[t][e] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  // fragment-read offsets
  int k_off[2];
#pragma unroll
  for (int sb = 0; sb < 2; ++sb) k_off[sb] = (sb * 32 + l32) * K_ROWB;
  const int k_swz = (K_CH == 16) ? (l32 & 15) : ((l32 >> 1) & 7);  // rows sb*32+l32 share it
  int v_off[DTILES];
#pragma unroll
  for (int t = 0; t < DTILES; ++t) v_off[t] = (t * 32 + l32) * V_ROWB;
  const int v_swz = (l32 >> 1) & 7;

  if (kb0 < kb1) issue(kb0, 0);
  for (int kb = kb0; kb < kb1; ++kb) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (kb + 1 < kb1) issue(kb + 1, (kb + 1 - kb0) & 1);
    const char* Ks = lds + ((kb - kb0) & 1) * STAGE;
    const char* Vs = Ks + K_BYTES;

    // ---- S^T = K Q^T for two 32-key sub-blocks
    f32x16 s[2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int e = 0; e < 16; ++e) s[sb][e] = 0.0f;
#pragma unroll
    for (int ds = 0; ds < DSTEPS; ++ds) {
      const int c = ((ds * 2 + hh) ^ k_swz) * 16;
      bf16x8 kf[2];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) kf[sb] = *reinterpret_cast<const bf16x8*>(Ks + k_off[sb] + c);
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) s[sb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[sb], qf[ds], s[sb], 0, 0, 0);
    }

    // ---- online softmax (log2 domain); the lane owns one query
    if ((kb + 1) * kAttnKB > Tk) {
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb * kAttnKB + sb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (key >= Tk) s[sb][r] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[sb][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * scale_log2;
    float alpha = 1.0f;
    if (mx > m_run + kLazyMax) {
      alpha = __builtin_amdgcn_exp2f(m_run - mx);  // 0 on the first block (m_run = -inf)
      m_run = mx;
    }
    if (__any(alpha != 1.0f)) {
      l_run *= alpha;
#pragma unroll
      for (int t = 0; t < DTILES; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[t][e] *= alpha;
    }
    float rs = 0.0f;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        // hardware exp2: P below 2^-126 of the running max flushes to zero
        const float pr = __builtin_amdgcn_exp2f(fmaf(s[sb][r], scale_log2, -m_run));
        s[sb][r] = pr;
        rs += pr;
      }
    l_run += rs + __shfl_xor(rs, 32, 64);

    // ---- O^T += Vt . P^T  (P^T fragment of step (sb, st) = S regs 8st..8st+7)
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        bf16x8 pf;
#pragma unroll
        for (int e = 0; e < 8; ++e) pf[e] = (bf16)s[sb][8 * st + e];
        const int chunk = sb * 4 + st * 2 + hh;  // 16-byte chunk of the 64-key row
#pragma unroll
        for (int t = 0; t < DTILES; ++t) {
          const bf16x8 vf = *reinterpret_cast<const bf16x8*>(Vs + v_off[t] + ((chunk ^ v_swz) * 16));
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, acc[t], 0, 0, 0);
        }
      }
    }
  }

  const int q = q0 + l32;
  if (SPLIT) {
    // ---- partial result of this key range (an empty range leaves m = -inf,
    // l = 0, O = 0, which the combine weighs to zero)
    if (q < Tq) {
      const int64_t row = ((int64_t)split * Tq + q) * H + head;
      float* orow = so.o + row * DH;
#pragma unroll
      for (int t = 0; t < DTILES; ++t)
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {
          f32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[t][4 * grp + e];
          *reinterpret_cast<f32x4*>(orow + t * 32 + 8 * grp + 4 * hh) = v;
        }
      if (hh == 0) {
        so.m[row] = m_run;
        so.l[row] = l_run;
      }
    }
    return;
  }
  // ---- epilogue: O = O^T / l, optional per-head gate, 4 bf16 per store
  if (q < Tq) {
    const float inv_l = 1.0f / l_run;
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
          float o = round_bf(acc[t][4 * grp + e] * inv_l);
          if (GATED) o = o * g;
          v[e] = (bf16)o;
        }
        *reinterpret_cast<bf16x4*>(orow + t * 32 + 8 * grp + 4 * hh) = v;
      }
  }
}

// Combine of the split-KV partials: one thread per (query, head, 8 outputs).
// O = sum_s 2^(m_s - m) O_s / sum_s 2^(m_s - m) l_s, m = max_s m_s; then the
// same rounding and gate as the single-pass epilogue.
template <int DH, bool GATED>
__global__ __launch_bounds__(256) void attn_combine_kernel(SplitOut so, bf16* __restrict__ O, int64_t o_rs,
                                                           const bf16* __restrict__ G, int64_t g_rs,
                                                           int Tq, int H) {
  constexpr int CH = DH / 8;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)Tq * H * CH) return;
  const int c = (int)(i % CH);
  const int64_t qh = i / CH;  // q * H + head
  const int q = (int)(qh / H), head = (int)(qh % H);
  const int64_t plane = (int64_t)Tq * H;
  float m = -INFINITY;
  for (int sp = 0; sp < so.splits; ++sp) m = fmaxf(m, so.m[sp * plane + qh]);
  float l = 0.0f, o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.0f;
  for (int sp = 0; sp < so.splits; ++sp) {
    const float ms = so.m[sp * plane + qh];
    const float w = ms == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms - m);
    l = fmaf(w, so.l[sp * plane + qh], l);
    const float* src = so.o + (sp * plane + qh) * DH + c * 8;
    const f32x4 a = *reinterpret_cast<const f32x4*>(src);
    const f32x4 b = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = fmaf(w, a[e], o[e]);
      o[4 + e] = fmaf(w, b[e], o[4 + e]);
    }
  }
  const float inv_l = 1.0f / l;
  float g = 1.0f;
  if (GATED) g = (float)G[(int64_t)q * g_rs + head];
  bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float r = round_bf(o[e] * inv_l);
    if (GATED) r = r * g;
    v[e] = (bf16)r;
  }
  *reinterpret_cast<bf16x8*>(O + (int64_t)q * o_rs + (int64_t)head * DH + c * 8) = v;
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

static int attn_check(const void* Q, int64_t q_rs, const void* K, int64_t k_rs, const void* Vt,
                      int64_t tk_pad, const void* O, int64_t o_rs, const void* gate, int64_t gate_rs,
                      int64_t Tq, int64_t Tk, int64_t H, int64_t head_dim, float scale) {
  if (!Q || !K || !Vt || !O || Tq < 0 || Tk <= 0 || H <= 0) return LTX_ERR_INVALID_ARG;
  if (head_dim != 64 && head_dim != 128) return LTX_ERR_UNSUPPORTED;
  if (tk_pad < ltx_attn_vt_padded_len(Tk) || tk_pad % 64) return LTX_ERR_INVALID_ARG;
  if (q_rs < H * head_dim || k_rs < H * head_dim || o_rs < H * head_dim) return LTX_ERR_INVALID_ARG;
  if (gate && gate_rs < H) return LTX_ERR_INVALID_ARG;
  if (!(scale > 0.0f)) return LTX_ERR_INVALID_ARG;  // the running max is taken before scaling
  if (!al16a(Q) || !al16a(K) || !al16a(Vt) || !al16a(O) || q_rs % 8 || k_rs % 8 || o_rs % 8)
    return LTX_ERR_ALIGNMENT;
  if (Tq > INT32_MAX || Tk > INT32_MAX) return LTX_ERR_UNSUPPORTED;
  return LTX_OK;
}

extern "C" int ltx_flash_attn_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs,
                                   const void* Vt, int64_t tk_pad, void* O, int64_t o_rs,
                                   const void* gate, int64_t gate_rs, int64_t Tq, int64_t Tk,
                                   int64_t H, int64_t head_dim, float scale, void* stream) {
  int st = attn_check(Q, q_rs, K, k_rs, Vt, tk_pad, O, o_rs, gate, gate_rs, Tq, Tk, H, head_dim, scale);
  if (st != LTX_OK) return st;
  if (Tq == 0) return LTX_OK;
  constexpr int QT = AttnCfg<64, kAttnWaves>::QT;
  const int64_t nwg = (Tq + QT - 1) / QT * H;
  if (nwg > INT32_MAX) return LTX_ERR_UNSUPPORTED;
  const float scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = (hipStream_t)stream;
  const SplitOut none{nullptr, nullptr, nullptr, 1};
#define LTX_FA(DH, G)                                                                              \
  flash_attn_kernel<DH, G, kAttnWaves, false><<<(int)nwg, 64 * kAttnWaves, 0, s>>>(                \
      (const bf16*)Q, q_rs, (const bf16*)K, k_rs, (const bf16*)Vt, tk_pad, (bf16*)O, o_rs,          \
      (const bf16*)gate, gate_rs, (int)Tq, (int)Tk, (int)H, scale_log2, none)
  if (head_dim == 128) {
    if (gate) LTX_FA(128, true); else LTX_FA(128, false);
  } else {
    if (gate) LTX_FA(64, true); else LTX_FA(64, false);
  }
#undef LTX_FA
  return ltx_launch_status();
}

extern "C" int64_t ltx_attn_splitkv_workspace_bytes(int64_t Tq, int64_t H, int64_t head_dim, int64_t splits) {
  if (Tq < 0 || H <= 0 || head_dim <= 0 || splits <= 0) return -1;
  const int64_t rows = splits * Tq * H;
  return rows * head_dim * 4 + 2 * ((rows * 4 + 255) / 256 * 256);
}

extern "C" int ltx_flash_attn_splitkv_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs,
                                           const void* Vt, int64_t tk_pad, void* O, int64_t o_rs,
                                           const void* gate, int64_t gate_rs, int64_t Tq, int64_t Tk,
                                           int64_t H, int64_t head_dim, float scale, int64_t splits,
                                           void* workspace, int64_t workspace_bytes, void* stream) {
  int st = attn_check(Q, q_rs, K, k_rs, Vt, tk_pad, O, o_rs, gate, gate_rs, Tq, Tk, H, head_dim, scale);
  if (st != LTX_OK) return st;
  if (splits < 1 || splits > 256 || !workspace) return LTX_ERR_INVALID_ARG;
  if (workspace_bytes < ltx_attn_splitkv_workspace_bytes(Tq, H, head_dim, splits)) return LTX_ERR_INVALID_ARG;
  if (!al16a(workspace)) return LTX_ERR_ALIGNMENT;
  if (Tq == 0) return LTX_OK;
  constexpr int QT = AttnCfg<64, kAttnSplitWaves>::QT;
  const int64_t nwg = (Tq + QT - 1) / QT * H * splits;
  const int64_t rows = splits * Tq * H;
  if (nwg > INT32_MAX || rows * head_dim / 8 > INT32_MAX) return LTX_ERR_UNSUPPORTED;
  const int64_t m_off = rows * head_dim * 4, l_off = m_off + (rows * 4 + 255) / 256 * 256;
  const SplitOut so{(float*)workspace, (float*)((char*)workspace + m_off), (float*)((char*)workspace + l_off),
                    (int)splits};
  const float scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = (hipStream_t)stream;
  const int64_t cthreads = Tq * H * (head_dim / 8);
  const int cblocks = (int)((cthreads + 255) / 256);
#define LTX_FAS(DH, G)                                                                              \
  do {                                                                                              \
    flash_attn_kernel<DH, false, kAttnSplitWaves, true><<<(int)nwg, 64 * kAttnSplitWaves, 0, s>>>(  \
        (const bf16*)Q, q_rs, (const bf16*)K, k_rs, (const bf16*)Vt, tk_pad, nullptr, 0, nullptr,   \
        0, (int)Tq, (int)Tk, (int)H, scale_log2, so);                                               \
    attn_combine_kernel<DH, G><<<cblocks, 256, 0, s>>>(so, (bf16*)O, o_rs, (const bf16*)gate,       \
                                                       gate_rs, (int)Tq, (int)H);                    \
  } while (0)
  if (head_dim == 128) {
    if (gate) LTX_FAS(128, true); else LTX_FAS(128, false);
  } else {
    if (gate) LTX_FAS(64, true); else LTX_FAS(64, false);
  }
#undef LTX_FAS
  return ltx_launch_status();
}
