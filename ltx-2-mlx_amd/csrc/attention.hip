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
//   V either token-major like K (its P.V fragments come from transposing LDS
//   reads) or pre-transposed by ltx_attn_transpose_v_bf16 into Vt (H, dh,
//   Tk_pad), Tk_pad = ceil(Tk/64)*64, zero-padded, with the keys of every
//   16-key group permuted so that each lane's 8 keys of a P.V fragment are
//   contiguous (see vt_position).  Both forms give the same bits.
//
// Kernel structure: one workgroup = 8 waves = 256 queries of one head; each
// wave owns 32 queries and two waves share a SIMD.  Scores are computed
// transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16: each lane then
// holds one query's scores in registers, so the row max / row sum are
// lane-local plus one cross-half exchange (v_permlane32_swap), and P^T feeds
// the P.V MFMA straight from registers (O^T += Vt . P^T).  K and V stream
// through LDS in 64-key stages by direct global->LDS buffer loads, in rings
// of 4 stages (a workgroup sync every other stage; 2 for the split-KV tiles);
// a key range that fits the ring (text contexts, the audio tokens) is loaded
// whole before the first block, with one sync.
// Key blocks are software-pipelined inside each wave, because VALU work only
// overlaps the issuing wave's own MFMAs: the softmax of block b is cut into
// one piece per MFMA slot (row max, running-max update, then exp2 / row sum
// / bf16 pack) spread over the P.V MFMAs of block b-1 and the S^T MFMAs of
// block b+1.  The stage barrier sits after a wave's last V read of a P.V
// half, so the K fragments of the next block are read behind the remaining
// MFMAs.  The running max is raised only when a block's max exceeds it by
// more than 2^8 (P then stays <= 256, exact in fp32 and bf16-relative as any
// other P), so the O^T rescale runs in the first blocks and then almost
// never.  Workgroups of one head are numbered contiguously per XCD so its
// K/V stay in that XCD's L2.
#include <mutex>
#include <type_traits>

#include "ltx_common.h"

namespace ltx {

constexpr int kAttnWaves = 8;            // full-size tiles: 8 waves = 256 queries
constexpr int kAttnSplitWaves = 4;       // split-KV tiles: 4 waves = 128 queries
constexpr int kAttnSmallTk = 256;        // single-pass key ranges up to this take 4-wave tiles
constexpr int kAttnKB = 64;              // keys per stage
constexpr int kNumXcdAttn = 8;
constexpr float kLazyMax = 8.0f;         // log2 headroom before the max is raised

typedef __attribute__((address_space(3))) char* lds_cptr_a;

// 16 bytes per lane from base + voff to LDS at lds_dst + 16 * lane: a buffer
// load with the lds modifier; a per-lane offset voff at or past num_records
// loads zeros.  The range check covers the vector offset only (a scalar
// offset is added after it, unchecked), so a key block's advance goes into
// the descriptor's base and record count, never into the scalar offset.  The
// descriptor (untyped: base, stride 0, record count, word 3 as for every
// buffer load of this library) is built from wave-uniform values in scalar
// registers; M0 holds the wave's LDS destination (a byte address in LDS).
// Issued as inline asm: the compiler's wait insertion treats the transposing
// LDS reads (ds_read_b64_tr_b16) as aliasing every LDS load in flight and put
// a full vmcnt(0) before the first V read after each stage's loads -- a wait
// for loads meant for the stages after it.  The kernel orders these loads
// itself: every stage sync waits vmcnt(0) before its barrier, and a block is
// read only after the sync that follows its loads.  s_nop 0: one wait state
// between the M0 write and the LDS-destination load.
__device__ __forceinline__ uint64_t uniform_addr(const void* p) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a), hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ void attn_dma16(uint64_t base, int num_records, uint32_t voff, uint32_t lds_dst) {
  i32x4 rsrc;
  rsrc[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)base);
  rsrc[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)((base >> 32) & 0xffffu));
  rsrc[2] = __builtin_amdgcn_readfirstlane(num_records);
  rsrc[3] = 0x00020000;
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_dst);
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(m0));
}

// Position of key j (0..15 within its 16-key group) in the permuted Vt row:
// MFMA k index 8h+e of a P.V step covers key 8*(e/4) + 4h + e%4.
__host__ __device__ __forceinline__ int vt_position(int j) {
  const int hi8 = j >> 3, h = (j >> 2) & 1, e4 = j & 3;
  return 8 * h + 4 * hi8 + e4;
}

// 16-byte chunk XOR of key row r of a row-major V stage in LDS (DH * 2 bytes
// per row).  The transposing fragment reads of one instruction cover, per
// 32-lane half, four rows 16j + 8rr + 4hh + e (e = 0..3) at the same 64-byte
// column range; the XOR spreads them over all 64 banks: rows e = 0..3 take
// chunk groups c ^ 4e (256-byte rows), and with 128-byte rows (two rows per
// bank sweep) rows e and e + 2 take c and c ^ 4.
template <int DH>
__host__ __device__ __forceinline__ int vrow_swz(int r) {
  return DH == 128 ? 4 * (r & 3) : 4 * ((r >> 1) & 1);
}

template <int DH, int WAVES, bool VROW = false>
struct AttnCfg {
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int QT = 32 * WAVES;    // queries per workgroup
  static constexpr int DSTEPS = DH / 16;   // k-steps of S = K Q^T
  static constexpr int DTILES = DH / 32;   // 32-row tiles of O^T
  static constexpr int K_ROWB = DH * 2;    // bytes per K row in LDS
  static constexpr int K_BYTES = kAttnKB * K_ROWB;
  // V stage: Vt rows of 128 B (64 keys) or, row-major, 64 key rows of DH * 2 B
  static constexpr int V_ROWB = VROW ? DH * 2 : kAttnKB * 2;
  static constexpr int V_BYTES = kAttnKB * DH * 2;
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

// Q's RMS norm and split RoPE applied as the kernel loads Q (the rows hold
// the projection's raw output).  ss: per-row partial sums of squares over the
// whole inner dim (Tq rows of `parts` fp32 values, row stride ld_ss); w: the
// norm weights (H * dh); cos / sin: RoPE tables of (H * dh / 2) columns, one
// row per query (idx null) or `axes` factored rows per query at
// idx[q * axes + a] (clamped to tab_rows); cos null: no RoPE.  ss null: Q is
// used as given.
struct QNorm {
  const float* ss;
  int64_t ld_ss;
  int parts;
  const float* w;
  float inv_d;
  float eps;
  const float* cos;
  const float* sin;
  const int* idx;
  int axes;
  int64_t tab_rows;
};

__device__ __forceinline__ void attn_load8f(const float* p, float* out) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[i] = a[i];
    out[4 + i] = b[i];
  }
}

// Softmax schedule of one key block over the MFMA slots of the pipeline:
// slots 0..NP-1 are the P.V half that follows the block's S^T (row max in
// slots < F, running-max update in slot F, exps after it), slots NP.. are the
// next S^T half (remaining exps).  Element e = 16*sb + r of the block's S^T.
template <int NP, int NQ, int DTILES>
struct AttnSched {
  static constexpr int F = NP / 2 - 1;
  static constexpr int NE = NP + NQ - F - 1;  // slots that carry exps
  static constexpr int exp_slot(int e) { return F + 1 + e * NE / 32; }
  static constexpr int max_slot(int e) { return e * F / 32; }
  // element e is written into P^T fragment e/8, which the previous block's
  // P.V reads in half-2 slots [(e/8)*DTILES, (e/8+1)*DTILES)
  static constexpr bool valid() {
    for (int e = 0; e < 32; ++e)
      if (exp_slot(e) < NP && exp_slot(e) < (e / 8 + 1) * DTILES) return false;
    for (int e = 0; e < 32; e += 2)
      if (exp_slot(e) > exp_slot(e + 1)) return false;
    return F >= 1 && exp_slot(31) < NP + NQ;
  }
};

// VROW: V is read row-major (Tk rows of stride v_ld elements, head h at
// columns h*DH ..) and its P.V fragments come from transposing LDS reads;
// otherwise V arrives as Vt (H, DH, v_ld = Tk_pad) from transpose_v_kernel.
template <int DH, bool GATED, int WAVES, bool SPLIT, bool VROW>
__global__ __launch_bounds__(64 * WAVES, 8 / WAVES) void flash_attn_kernel(
    const bf16* __restrict__ Q, int64_t q_rs, const bf16* __restrict__ K, int64_t k_rs,
    const bf16* __restrict__ V, int64_t v_ld, bf16* __restrict__ O, int64_t o_rs,
    const bf16* __restrict__ G, int64_t g_rs, int Tq, int Tk, int H, float scale_log2, SplitOut so,
    QNorm qn) {
  using Cfg = AttnCfg<DH, WAVES, VROW>;
  constexpr int kAttnQ = Cfg::QT;
  constexpr int DSTEPS = Cfg::DSTEPS, DTILES = Cfg::DTILES;
  constexpr int K_ROWB = Cfg::K_ROWB, K_BYTES = Cfg::K_BYTES, V_ROWB = Cfg::V_ROWB;
  constexpr int V_BYTES = Cfg::V_BYTES, K_DMA = Cfg::K_DMA, V_DMA = Cfg::V_DMA;
  constexpr int NQ = 2 * DSTEPS;  // MFMAs of S^T = K Q^T per key block (one per slot)
  constexpr int NP = 4 * DTILES;  // MFMAs of O^T += Vt P^T per key block
  constexpr int EPS = 32 / NQ;    // softmax elements per S^T slot
  constexpr int PF = 4;           // fragment reads in flight ahead of their MFMA
  static_assert(NQ >= PF && NP >= PF && 32 % NQ == 0, "slot schedule");
  // K ring (RING x K_BYTES) followed by the V ring (RING x V_BYTES): a ring of
  // 4 lets the workgroup synchronise every other key block (the split-KV
  // tiles, two workgroups per CU, keep 2)
  constexpr int RING = (SPLIT || WAVES == kAttnSplitWaves) ? 2 : 4;
  __shared__ __attribute__((aligned(1024))) char lds[RING * (K_BYTES + V_BYTES)];
  char* const Ks0 = lds;
  // LDS byte addresses of the rings (the direct loads' destinations)
  const uint32_t ks_lds = (uint32_t)(uintptr_t)(lds_cptr_a)lds, vs_lds = ks_lds + RING * K_BYTES;

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
  const int live = __builtin_amdgcn_readfirstlane(q0 < Tq ? 1 : 0);

  const bf16* Kh = K + (int64_t)head * DH;
  const bf16* Vh = VROW ? V + (int64_t)head * DH : V + (int64_t)head * DH * v_ld;
  // the head's K / V base addresses in scalar registers (the direct loads'
  // descriptors are built from them per key block)
  const uint64_t kh_addr = uniform_addr(Kh), vh_addr = uniform_addr(Vh);

  // ---- Q^T fragments: lane holds Q[q][dstep*16 + hh*8 .. +8] for its query
  bf16x8 qf[DSTEPS];
  {
    int q = q0 + l32;
    q = q < Tq ? q : Tq - 1;
    const bf16* qrow = Q + (int64_t)q * q_rs + (int64_t)head * DH + hh * 8;
#pragma unroll
    for (int s = 0; s < DSTEPS; ++s) qf[s] = *reinterpret_cast<const bf16x8*>(qrow + s * 16);
  }
  // Q's norm and RoPE (QNorm), applied after this workgroup's first K / V
  // loads are issued, so that the latency of its own loads (row statistics,
  // weights, tables) overlaps theirs.  Every load is unconditional (clamped
  // indices), so each batch of them goes out at once.
  auto apply_qnorm = [&]() __attribute__((always_inline)) {
    int q = q0 + l32;
    q = q < Tq ? q : Tq - 1;
    // sum of the row's partials: lane hh takes the 4-value chunks c with
    // c % 2 == hh, the pair adds both halves in the same order
    const float* sp = qn.ss + (int64_t)q * qn.ld_ss;
    const int nch = qn.parts >> 2;
    f32x4 pv[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int ch = 2 * c + hh;
      pv[c] = *reinterpret_cast<const f32x4*>(sp + 4 * (ch < nch ? ch : 0));
    }
    const bool rope = qn.cos != nullptr;
    const int naxes = !rope ? 0 : (qn.idx != nullptr ? qn.axes : 1);
    const int64_t tw = (int64_t)H * (DH / 2);
    constexpr int NS = DSTEPS / 2;
    // weights of every pair (independent of the table rows)
    float wa[NS][8], wb[NS][8];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int c1 = head * DH + s * 16 + hh * 8;  // weight of x1; x2's is c1 + DH / 2
      attn_load8f(qn.w + c1, wa[s]);
      attn_load8f(qn.w + c1 + DH / 2, wb[s]);
    }
    int64_t rows[3] = {(int64_t)q * tw, (int64_t)q * tw, (int64_t)q * tw};
    if (qn.idx != nullptr) {
      const int* ip = qn.idx + (int64_t)q * qn.axes;
      int r[3];
#pragma unroll
      for (int a = 0; a < 3; ++a) r[a] = ip[a < qn.axes ? a : 0];
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        const int64_t row = r[a] < 0 ? 0 : (r[a] < qn.tab_rows ? r[a] : qn.tab_rows - 1);
        rows[a] = row * tw;
      }
    }
    float half = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float v4 = (pv[c][0] + pv[c][1]) + (pv[c][2] + pv[c][3]);
      half += (2 * c + hh < nch) ? v4 : 0.0f;
    }
    // after the swap, element 0 holds the hh = 0 lane's half, element 1 the
    // hh = 1 lane's: both lanes add them in that order
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(half), __float_as_uint(half), false, false);
    const float ss = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    const float inv = rsqrt_rn(ss * qn.inv_d + qn.eps);
    float x1[NS][8], x2[NS][8];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        x1[s][i] = round_bf((float)qf[s][i] * inv * wa[s][i]);
        x2[s][i] = round_bf((float)qf[s + NS][i] * inv * wb[s][i]);
      }
    if (rope) {
      // two pairs' table entries per batch of loads; factored rows combine
      // as cos = c0 c1 c2, sin = s0 + s1 + s2
#pragma unroll
      for (int s0 = 0; s0 < NS; s0 += 2) {
        float c[2][3][8], sn[2][3][8];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int t1 = head * (DH / 2) + (s0 + u) * 16 + hh * 8;  // table column of the pair
#pragma unroll
          for (int a = 0; a < 3; ++a) {
            attn_load8f(qn.cos + rows[a] + t1, c[u][a]);
            attn_load8f(qn.sin + rows[a] + t1, sn[u][a]);
          }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int s = s0 + u;
#pragma unroll
          for (int a = 1; a < 3; ++a)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              c[u][0][i] = a < naxes ? c[u][0][i] * c[u][a][i] : c[u][0][i];
              sn[u][0][i] = a < naxes ? sn[u][0][i] + sn[u][a][i] : sn[u][0][i];
            }
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float o1 = x1[s][i] * c[u][0][i] - x2[s][i] * sn[u][0][i];
            const float o2 = x1[s][i] * sn[u][0][i] + x2[s][i] * c[u][0][i];
            x1[s][i] = o1;
            x2[s][i] = o2;
          }
        }
      }
    }
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        qf[s][i] = (bf16)x1[s][i];
        qf[s + NS][i] = (bf16)x2[s][i];
      }
  };

  // ---- DMA sources.  Wave instruction i fills the 1 KiB LDS block
  // WAVES*i + wave.  K: 1024/K_ROWB rows per block.  Buffer loads: per key
  // block a descriptor (scalar registers) whose base is the block's first
  // key row and whose record count ends at the last key row of this head,
  // and one fixed 32-bit per-lane offset within the block.  Rows past Tk in
  // the last block then lie past the record count and load as zeros (their
  // scores are masked, their P is 0); no load leaves the operand.
  constexpr int K_ROWS_PER = 1024 / K_ROWB;      // 4 (dh 128) or 8 (dh 64)
  constexpr int K_CH = K_ROWB / 16;               // 16-byte chunks per row
  const int k_records = (int)((int64_t)(Tk - 1) * k_rs * 2 + DH * 2);
  uint32_t k_voff[K_DMA];
#pragma unroll
  for (int i = 0; i < K_DMA; ++i) {
    const int r = K_ROWS_PER * (WAVES * i + wave) + lane / K_CH;
    const int slot = lane % K_CH;
    const int chunk = (K_CH == 16) ? (slot ^ (r & 15)) : (slot ^ ((r >> 1) & 7));
    k_voff[i] = (uint32_t)(r * k_rs * 2 + chunk * 16);
  }
  // Vt: rows of 128 B (64 keys), 8 rows per block.  Row-major V: key rows
  // like K's, chunks XORed by vrow_swz.
  const int v_records = VROW ? (int)((int64_t)(Tk - 1) * v_ld * 2 + DH * 2) : (int)(DH * v_ld * 2);
  uint32_t v_voff[V_DMA];
#pragma unroll
  for (int i = 0; i < V_DMA; ++i) {
    if constexpr (VROW) {
      const int r = K_ROWS_PER * (WAVES * i + wave) + lane / K_CH;
      const int chunk = (lane % K_CH) ^ vrow_swz<DH>(r);
      v_voff[i] = (uint32_t)(r * v_ld * 2 + chunk * 16);
    } else {
      const int r = 8 * (WAVES * i + wave) + (lane >> 3);
      const int chunk = (lane & 7) ^ ((r >> 1) & 7);
      v_voff[i] = (uint32_t)(r * v_ld * 2 + chunk * 16);
    }
  }

  const int nblocks_all = (Tk + kAttnKB - 1) / kAttnKB;
  // key blocks [kb0, kb0 + nb) of this workgroup
  const int per_split = (nblocks_all + nsplit - 1) / nsplit;
  const int kb0 = split * per_split;
  const int kb1 = (kb0 + per_split) < nblocks_all ? (kb0 + per_split) : nblocks_all;
  const int nb = kb1 > kb0 ? kb1 - kb0 : 0;
  // a key range that fits the K / V rings is loaded whole before the first block
  const int pre = __builtin_amdgcn_readfirstlane(nb <= RING ? 1 : 0);
  // byte advance per key block; every issued block kb < nblocks_all starts at
  // or before key row Tk - 1 (Vt: column Tk_pad - 64), so the remaining
  // record count kb_records - kb * step stays positive
  const int k_step = (int)(kAttnKB * k_rs * 2);
  const int v_step = VROW ? (int)(kAttnKB * v_ld * 2) : kAttnKB * 2;
  auto issue_k = [&](int kb, int buf) {
    const uint32_t Ks = ks_lds + buf * K_BYTES;
    const uint64_t base = kh_addr + (uint64_t)((int64_t)kb * k_step);
    const int rec = k_records - kb * k_step;
#pragma unroll
    for (int i = 0; i < K_DMA; ++i) attn_dma16(base, rec, k_voff[i], Ks + (WAVES * i + wave) * 1024);
  };
  auto issue_v = [&](int kb, int buf) {
    const uint32_t Vs = vs_lds + buf * V_BYTES;
    const uint64_t base = vh_addr + (uint64_t)((int64_t)kb * v_step);
    const int rec = v_records - kb * v_step;
#pragma unroll
    for (int i = 0; i < V_DMA; ++i) attn_dma16(base, rec, v_voff[i], Vs + (WAVES * i + wave) * 1024);
  };

  // Loop-invariant fragment-read offsets; ring buffer, 32-row sub-block and
  // O^T tile enter as immediates.  K row sb*32+l32, 16-byte chunk 2*ds+hh;
  // Vt row t*32+l32, chunk 2*j+hh for P.V step j = 2*sb + st.
  const int k_swz = (K_CH == 16) ? (l32 & 15) : ((l32 >> 1) & 7);
  const int v_swz = (l32 >> 1) & 7;
  int k_addr[DSTEPS], v_addr[4];
#pragma unroll
  for (int ds = 0; ds < DSTEPS; ++ds) k_addr[ds] = l32 * K_ROWB + (((2 * ds + hh) ^ k_swz) * 16);
  if constexpr (!VROW) {
#pragma unroll
    for (int j = 0; j < 4; ++j) v_addr[j] = RING * K_BYTES + l32 * V_ROWB + (((2 * j + hh) ^ v_swz) * 16);
  } else {
    // Transposing reads (ds_read_b64_tr_b16): in each 16-lane group, lane i
    // receives element i % 4 of the 8 bytes that lane 4e + i / 4 addressed,
    // as its element e.  Lane 16g + 4e + q of a P.V fragment (j, t)
    // addresses 4 columns 32t + 16(g % 2) + 4q of key row 16j + 8rr + 4hh + e
    // (rr = 0, 1: the fragment's two reads), so lane (d, hh) receives keys
    // 16j + 8rr + 4hh + 0..3 of column d -- the P^T key order of its
    // elements 4rr..4rr+3.  v_addr[t]: the lane's byte offset for rr = j = 0.
    const int g = lane >> 4, e = (lane >> 2) & 3, q = lane & 3;
#pragma unroll
    for (int t = 0; t < DTILES; ++t) {
      const int chunk = (4 * t + 2 * (g & 1) + (q >> 1)) ^ vrow_swz<DH>(4 * hh + e);
      v_addr[t] = RING * K_BYTES + (4 * hh + e) * V_ROWB + chunk * 16 + 8 * (q & 1);
    }
  }
  // P.V fragment (j, t) of the Vt / V stage in ring slot `slot`.  v_addr holds
  // LDS byte offsets from the start of the array, V ring base included, so
  // every slot / fragment offset fits a read's 16-bit immediate.
  auto read_v = [&](int slot, int j, int t) -> bf16x8 {
    if constexpr (!VROW) {
      return *reinterpret_cast<const bf16x8*>(lds + v_addr[j] + slot * V_BYTES + t * 32 * V_ROWB);
    } else {
      typedef short v4s __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) v4s* lds_v4s;
      const char* base = lds + v_addr[t] + slot * V_BYTES + 16 * j * V_ROWB;
      const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(base));
      const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(base + 8 * V_ROWB));
      return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };

  f32x16 acc[DTILES];
#pragma unroll
  for (int t = 0; t < DTILES; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[t][e] = 0.0f;
  f32x16 s[2][2];        // S^T of two consecutive key blocks (ping-pong by block parity)
  uint32_t pw[4][4];     // P^T fragments (bf16 pairs) of one block
  bf16x8 vf[4][DTILES];  // Vt fragments in flight
  bf16x8 kf[DSTEPS][2];  // K fragments in flight
  float pe[32];          // exps of a block (an even element waits for its pair)
  float m_run = -INFINITY, l_run = 0.0f, neg_m = INFINITY, alpha_pend = 1.0f;
  float rs = 0.0f;       // row sum of the block whose exps are in flight

  // Software pipeline.  Iteration b = [half 1: S^T MFMAs of block b] then
  // [half 2: P.V MFMAs of block b-1].  Per 32-query wave a 64-key block costs
  // NQ + NP MFMAs and ~110 VALU instructions (max, scale fma, exp2, sum, bf16
  // pack); VALU work overlaps only the issuing wave's own MFMAs, so the
  // softmax of block b is spread one piece per MFMA slot over half 2 of
  // iteration b (row max, then the max update, then the first exps) and half 1
  // of iteration b+1 (the remaining exps).  A P^T fragment of block b is
  // written only after the last P.V MFMA of block b-1 that reads it.
  using Sch = AttnSched<NP, NQ, DTILES>;
  static_assert(Sch::valid(), "softmax slot schedule");
  auto half_sum = [](float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  };
  auto half_max = [](float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  };
  // exps of the block in s[X] that fall in slot G (counted from its half 2)
  auto do_exps = [&](auto xc, int G) {
    constexpr int X = decltype(xc)::value;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      if (Sch::exp_slot(e) == G) {
        // hardware exp2: P below 2^-126 of the running max flushes to zero
        pe[e] = __builtin_amdgcn_exp2f(fmaf(s[X][e >> 4][e & 15], scale_log2, neg_m));
        rs += pe[e];
        if (e & 1) {
          uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){pe[e - 1], pe[e]}, bf16x2));
          // keep the pack and the sum in this slot (pure arithmetic would
          // otherwise be sunk to its first use, past the MFMAs)
          asm volatile("" : "+v"(w));
          pw[e >> 3][(e & 7) >> 1] = w;
        }
      }
    }
    asm volatile("" : "+v"(rs));
  };
  auto read_k = [&](int buf, int k) {  // K fragment of S^T slot k
    kf[k >> 1][k & 1] =
        *reinterpret_cast<const bf16x8*>(Ks0 + buf * K_BYTES + (k & 1) * 32 * K_ROWB + k_addr[k >> 1]);
  };
  // Iteration b runs with Q = b % RING (compile-time): block b sits in ring
  // slot Q of K and V, its S^T in s[P], P = b & 1.
  // Half 1 of iteration b: S^T of block b from K slot Q into s[P] (its first
  // PF K fragments already in flight); remaining exps of block b-1 (s[1-P]);
  // first V reads of half 2 (block b-1, slot Q-1).
  auto half1 = [&](auto qc, auto qkc, auto expc, auto livec) __attribute__((always_inline)) {
    constexpr int Q = decltype(qc)::value, P = Q & 1;
    constexpr bool LV = decltype(livec)::value;
    constexpr bool QK = decltype(qkc)::value && LV, EXP = decltype(expc)::value && LV;
    constexpr int VSLOT = (Q + RING - 1) % RING;
    if (QK) {
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[P][sb][e] = 0.0f;
    }
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
      const int ds = k >> 1, sb = k & 1;
      if (QK) s[P][sb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ds][sb], qf[ds], s[P][sb], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (EXP) do_exps(std::integral_constant<int, 1 - P>(), NP + k);
      const int kn = k + PF;
      if (QK && kn < NQ) {
        read_k(Q, kn);
      } else if (EXP && kn >= NQ) {
        const int n = kn - NQ;  // first PF Vt fragments of half 2
        vf[n / DTILES][n % DTILES] = read_v(VSLOT, n / DTILES, n % DTILES);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (EXP) {
      l_run += half_sum(rs);
      rs = 0.0f;
    }
  };
  // keys past Tk in the last block score -inf
  auto mask_tail = [&](auto pc, int kb) {
    constexpr int P = decltype(pc)::value;
    if ((kb + 1) * kAttnKB > Tk) {
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb * kAttnKB + sb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (key >= Tk) s[P][sb][r] = -INFINITY;
        }
    }
  };
  auto sync_stage = [&]() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };
  // Half 2 of iteration b: P.V of block b-1 from V slot Q-1; row max of
  // block b (s[P]), the running-max update, first exps of block b.  The
  // running max (log2 domain) is raised only when a block's max exceeds it by
  // more than 2^kLazyMax; O^T is rescaled just before the next P.V.
  // Stage sync (NEW only), once this wave has issued its last V read of the
  // half: every wave is done with K_b and V_{b-1} (and all older blocks), and
  // every load issued before it is resident.  RING 2 syncs every iteration
  // and then loads K_{b+2} and V_{b+1} into the slots just freed.  RING 4
  // syncs at b = 0, loading K_2, K_3, V_1, V_2, and at every odd b, loading
  // K_{b+3}, K_{b+4}, V_{b+2}, V_{b+3} into the slots of K_{b-1}, K_b,
  // V_{b-2}, V_{b-1}: each block is loaded before the sync that precedes its
  // first read.  The remaining slots read the first K fragments of block b+1.
  auto half2 = [&](auto qc, auto pvc, auto newc, int b, auto livec) __attribute__((always_inline)) {
    constexpr int Q = decltype(qc)::value, P = Q & 1;
    constexpr bool LV = decltype(livec)::value;
    // NEW_STAGE: the stage syncs and loads, which every wave runs; NEW: the
    // block's own softmax work, which a wave without queries skips
    constexpr bool NEW_STAGE = decltype(newc)::value;
    constexpr bool PV = decltype(pvc)::value && LV, NEW = NEW_STAGE && LV;
    constexpr int VSLOT = (Q + RING - 1) % RING;
    const int kb = kb0 + b;
    if (PV && __any(alpha_pend != 1.0f)) {
#pragma unroll
      for (int t = 0; t < DTILES; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[t][e] *= alpha_pend;
    }
    if (NEW) mask_tail(std::integral_constant<int, P>(), kb);
    float mx = -INFINITY;
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      const int j = n / DTILES, t = n % DTILES;
      if (PV) {
        const bf16x8 pj = __builtin_bit_cast(bf16x8, (u32x4){pw[j][0], pw[j][1], pw[j][2], pw[j][3]});
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[j][t], pj, acc[t], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      const int nn = n + PF;
      if (PV && nn < NP) vf[nn / DTILES][nn % DTILES] = read_v(VSLOT, nn / DTILES, nn % DTILES);
      if (NEW_STAGE && nn == NP && !pre) {
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (RING == 2) {
          sync_stage();
          if (b + 2 < nb) issue_k(kb + 2, Q);
          if (b + 1 < nb) issue_v(kb + 1, (Q + 1) % RING);
        } else if constexpr ((Q & 1) == 1) {
          sync_stage();
          if (b + 3 < nb) issue_k(kb + 3, (Q + 3) % RING);
          if (b + 4 < nb) issue_k(kb + 4, Q);
          if (b + 2 < nb) issue_v(kb + 2, (Q + 2) % RING);
          if (b + 3 < nb) issue_v(kb + 3, (Q + 3) % RING);
        } else if (b == 0) {
          sync_stage();
          if (2 < nb) issue_k(kb0 + 2, 2);
          if (3 < nb) issue_k(kb0 + 3, 3);
          if (1 < nb) issue_v(kb0 + 1, 1);
          if (2 < nb) issue_v(kb0 + 2, 2);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (NEW && nn >= NP && b + 1 < nb) read_k((Q + 1) % RING, nn - NP);
      if (NEW) {
        if (n < Sch::F) {
#pragma unroll
          for (int e = 0; e < 32; ++e)
            if (Sch::max_slot(e) == n) mx = fmaxf(mx, s[P][e >> 4][e & 15]);
          asm volatile("" : "+v"(mx));
        } else if (n == Sch::F) {
          mx = half_max(mx) * scale_log2;
          float alpha = 1.0f;
          if (mx > m_run + kLazyMax) {
            alpha = __builtin_amdgcn_exp2f(m_run - mx);  // 0 on the first block (m_run = -inf)
            m_run = mx;
          }
          l_run *= alpha;
          alpha_pend = alpha;
          neg_m = -m_run;
        } else {
          do_exps(std::integral_constant<int, P>(), n);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2 % RING>;
  using I3 = std::integral_constant<int, 3 % RING>;
  using BT = std::integral_constant<bool, true>;
  using BF = std::integral_constant<bool, false>;
  // iteration b in [1, nb), Q = b % RING
  auto body = [&](auto qc, int b, auto livec) __attribute__((always_inline)) {
    half1(qc, BT(), BT(), livec);
    half2(qc, BT(), BT(), b, livec);
  };
  // drain (iteration nb): last exps and P.V of block nb-1
  auto drain = [&](auto qc, auto livec) __attribute__((always_inline)) {
    half1(qc, BF(), BT(), livec);
    half2(qc, BT(), BF(), 0, livec);
  };

  if (nb > 0) {
    if (pre) {
      // every key block fits the ring: all of K and V in flight at once, one
      // sync, no further stage syncs
      for (int i = 0; i < nb; ++i) {
        issue_k(kb0 + i, i);
        issue_v(kb0 + i, i);
      }
      if (qn.ss != nullptr && live) apply_qnorm();
      sync_stage();
    } else {
      issue_k(kb0, 0);
      if (qn.ss != nullptr && live) apply_qnorm();
      sync_stage();
      if (nb > 1) issue_k(kb0 + 1, 1);
      issue_v(kb0, 0);
    }
    // a wave whose 32 queries all lie past Tq (the last query tile of a head)
    // issues no MFMAs and no softmax work; it still moves its share of every
    // K / V stage and meets every stage sync, at the same points of the loop
    auto run_blocks = [&](auto lv) __attribute__((always_inline)) {
      if (decltype(lv)::value) {
#pragma unroll
        for (int k = 0; k < PF; ++k) read_k(0, k);
      }
      half1(I0(), BT(), BF(), lv);
      half2(I0(), BF(), BT(), 0, lv);
      int b = 1;
      if constexpr (RING == 2) {
        for (; b + 1 < nb; b += 2) {
          body(I1(), b, lv);
          body(I0(), b + 1, lv);
        }
        if (b < nb) body(I1(), b, lv);
        if (nb & 1) drain(I1(), lv); else drain(I0(), lv);
      } else {
        for (; b + 3 < nb; b += 4) {
          body(I1(), b, lv);
          body(I2(), b + 1, lv);
          body(I3(), b + 2, lv);
          body(I0(), b + 3, lv);
        }
        // b % 4 == 1 here; up to three more iterations
        if (b < nb) body(I1(), b++, lv);
        if (b < nb) body(I2(), b++, lv);
        if (b < nb) body(I3(), b++, lv);
        switch (nb % 4) {
          case 0: drain(I0(), lv); break;
          case 1: drain(I1(), lv); break;
          case 2: drain(I2(), lv); break;
          default: drain(I3(), lv); break;
        }
      }
    };
    if (live) run_blocks(BT());
    else run_blocks(BF());
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

static int attn_check(const void* Q, int64_t q_rs, const void* K, int64_t k_rs, const void* O, int64_t o_rs,
                      const void* gate, int64_t gate_rs, int64_t Tq, int64_t Tk, int64_t H, int64_t head_dim,
                      float scale) {
  if (!Q || !K || !O || Tq < 0 || Tk <= 0 || H <= 0) return LTX_ERR_INVALID_ARG;
  if (head_dim != 64 && head_dim != 128) return LTX_ERR_UNSUPPORTED;
  if (q_rs < H * head_dim || k_rs < H * head_dim || o_rs < H * head_dim) return LTX_ERR_INVALID_ARG;
  if (gate && gate_rs < H) return LTX_ERR_INVALID_ARG;
  if (!(scale > 0.0f)) return LTX_ERR_INVALID_ARG;  // the running max is taken before scaling
  if (!al16a(Q) || !al16a(K) || !al16a(O) || q_rs % 8 || k_rs % 8 || o_rs % 8) return LTX_ERR_ALIGNMENT;
  if (Tq > INT32_MAX || Tk > INT32_MAX) return LTX_ERR_UNSUPPORTED;
  // K (and token-major V) are addressed by 32-bit buffer offsets
  if ((Tk + 64) * k_rs * 2 > INT32_MAX) return LTX_ERR_UNSUPPORTED;
  return LTX_OK;
}
// V operand: Vt (H, dh, tk_pad) or row-major V (Tk rows of stride v_rs)
static int attn_check_vt(const void* Vt, int64_t tk_pad, int64_t Tk) {
  if (!Vt || tk_pad < ltx_attn_vt_padded_len(Tk) || tk_pad % 64) return LTX_ERR_INVALID_ARG;
  if (128 * tk_pad * 2 > INT32_MAX) return LTX_ERR_UNSUPPORTED;
  return al16a(Vt) ? LTX_OK : LTX_ERR_ALIGNMENT;
}
static int attn_check_v(const void* V, int64_t v_rs, int64_t Tk, int64_t H, int64_t head_dim) {
  if (!V || v_rs < H * head_dim) return LTX_ERR_INVALID_ARG;
  if ((Tk + 64) * v_rs * 2 > INT32_MAX) return LTX_ERR_UNSUPPORTED;
  return (al16a(V) && v_rs % 8 == 0) ? LTX_OK : LTX_ERR_ALIGNMENT;
}

template <bool VROW>
static int launch_attn(const void* Q, int64_t q_rs, const void* K, int64_t k_rs, const void* V, int64_t v_ld,
                       void* O, int64_t o_rs, const void* gate, int64_t gate_rs, int64_t Tq, int64_t Tk,
                       int64_t H, int64_t head_dim, float scale, hipStream_t s,
                       const QNorm& qn = QNorm{}) {
  if (Tq == 0) return LTX_OK;
  // Short key ranges (text contexts, audio keys) leave a workgroup mostly
  // waiting on its loads and its epilogue: 128-query workgroups with rings of
  // two key blocks (64 KB of LDS at dh 128) put two of them on a CU, so one
  // computes while the other waits.
  const bool small = Tk <= kAttnSmallTk;
  const int QT = small ? AttnCfg<64, kAttnSplitWaves>::QT : AttnCfg<64, kAttnWaves>::QT;
  const int64_t nwg = (Tq + QT - 1) / QT * H;
  if (nwg > INT32_MAX) return LTX_ERR_UNSUPPORTED;
  const float scale_log2 = scale * 1.4426950408889634f;
  const SplitOut none{nullptr, nullptr, nullptr, 1};
#define LTX_FA(DH, G, W)                                                                           \
  flash_attn_kernel<DH, G, W, false, VROW><<<(int)nwg, 64 * W, 0, s>>>(                            \
      (const bf16*)Q, q_rs, (const bf16*)K, k_rs, (const bf16*)V, v_ld, (bf16*)O, o_rs,             \
      (const bf16*)gate, gate_rs, (int)Tq, (int)Tk, (int)H, scale_log2, none, qn)
  if (small) {
    if (head_dim == 128) {
      if (gate) LTX_FA(128, true, kAttnSplitWaves); else LTX_FA(128, false, kAttnSplitWaves);
    } else {
      if (gate) LTX_FA(64, true, kAttnSplitWaves); else LTX_FA(64, false, kAttnSplitWaves);
    }
  } else {
    if (head_dim == 128) {
      if (gate) LTX_FA(128, true, kAttnWaves); else LTX_FA(128, false, kAttnWaves);
    } else {
      if (gate) LTX_FA(64, true, kAttnWaves); else LTX_FA(64, false, kAttnWaves);
    }
  }
#undef LTX_FA
  return ltx_launch_status();
}

extern "C" int ltx_flash_attn_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs,
                                   const void* Vt, int64_t tk_pad, void* O, int64_t o_rs,
                                   const void* gate, int64_t gate_rs, int64_t Tq, int64_t Tk,
                                   int64_t H, int64_t head_dim, float scale, void* stream) {
  int st = attn_check(Q, q_rs, K, k_rs, O, o_rs, gate, gate_rs, Tq, Tk, H, head_dim, scale);
  if (st == LTX_OK) st = attn_check_vt(Vt, tk_pad, Tk);
  if (st != LTX_OK) return st;
  return launch_attn<false>(Q, q_rs, K, k_rs, Vt, tk_pad, O, o_rs, gate, gate_rs, Tq, Tk, H, head_dim, scale,
                            (hipStream_t)stream);
}

extern "C" int ltx_flash_attn_v_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs, const void* V,
                                     int64_t v_rs, void* O, int64_t o_rs, const void* gate, int64_t gate_rs,
                                     int64_t Tq, int64_t Tk, int64_t H, int64_t head_dim, float scale,
                                     void* stream) {
  int st = attn_check(Q, q_rs, K, k_rs, O, o_rs, gate, gate_rs, Tq, Tk, H, head_dim, scale);
  if (st == LTX_OK) st = attn_check_v(V, v_rs, Tk, H, head_dim);
  if (st != LTX_OK) return st;
  return launch_attn<true>(Q, q_rs, K, k_rs, V, v_rs, O, o_rs, gate, gate_rs, Tq, Tk, H, head_dim, scale,
                           (hipStream_t)stream);
}

// ltx_flash_attn_v_bf16 on the raw query projection: the kernel applies the
// query's RMS norm and split RoPE as it loads Q (QNorm above), from the
// per-row partial sums of squares that ltx_gemm_rowss_bf16 writes next to
// the projection.
extern "C" int ltx_flash_attn_qnorm_v_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs,
                                           const void* V, int64_t v_rs, void* O, int64_t o_rs, const void* gate,
                                           int64_t gate_rs, int64_t Tq, int64_t Tk, int64_t H, int64_t head_dim,
                                           float scale, const float* ss, int64_t ld_ss, int64_t ss_parts,
                                           const float* wq, float eps, const float* cos, const float* sin,
                                           const int* idx, int64_t axes, int64_t tab_rows, void* stream) {
  int st = attn_check(Q, q_rs, K, k_rs, O, o_rs, gate, gate_rs, Tq, Tk, H, head_dim, scale);
  if (st == LTX_OK) st = attn_check_v(V, v_rs, Tk, H, head_dim);
  if (st != LTX_OK) return st;
  if (!ss || !wq || ss_parts < 4 || ss_parts > 64 || ss_parts % 4 || ld_ss < ss_parts || !(eps >= 0.0f))
    return LTX_ERR_INVALID_ARG;
  if ((cos == nullptr) != (sin == nullptr)) return LTX_ERR_INVALID_ARG;
  if (idx != nullptr && (cos == nullptr || axes < 1 || axes > 3 || tab_rows < 1)) return LTX_ERR_INVALID_ARG;
  if (cos != nullptr && idx == nullptr && tab_rows < Tq) return LTX_ERR_INVALID_ARG;
  if (!al16a(ss) || ld_ss % 4 || !al16a(wq) || (cos && (!al16a(cos) || !al16a(sin)))) return LTX_ERR_ALIGNMENT;
  if (Tq > 0 && ld_ss > INT64_MAX / Tq) return LTX_ERR_UNSUPPORTED;
  QNorm qn{};
  qn.ss = ss;
  qn.ld_ss = ld_ss;
  qn.parts = (int)ss_parts;
  qn.w = wq;
  qn.inv_d = 1.0f / (float)(H * head_dim);
  qn.eps = eps;
  qn.cos = cos;
  qn.sin = sin;
  qn.idx = idx;
  qn.axes = idx ? (int)axes : 1;
  qn.tab_rows = tab_rows;
  return launch_attn<true>(Q, q_rs, K, k_rs, V, v_rs, O, o_rs, gate, gate_rs, Tq, Tk, H, head_dim, scale,
                           (hipStream_t)stream, qn);
}

extern "C" int64_t ltx_attn_splitkv_workspace_bytes(int64_t Tq, int64_t H, int64_t head_dim, int64_t splits) {
  if (Tq < 0 || H <= 0 || head_dim <= 0 || splits <= 0) return -1;
  // -1 for sizes whose byte count does not fit an int64 (no wrapped result)
  int64_t rows = 0, obytes = 0, total = 0;
  if (__builtin_mul_overflow(splits, Tq, &rows) || __builtin_mul_overflow(rows, H, &rows)) return -1;
  if (rows > (INT64_MAX / 16) || __builtin_mul_overflow(rows, head_dim * 4, &obytes)) return -1;
  if (__builtin_add_overflow(obytes, 2 * ((rows * 4 + 255) / 256 * 256), &total)) return -1;
  return total;
}

template <bool VROW>
static int launch_attn_splitkv(const void* Q, int64_t q_rs, const void* K, int64_t k_rs, const void* V,
                               int64_t v_ld, void* O, int64_t o_rs, const void* gate, int64_t gate_rs,
                               int64_t Tq, int64_t Tk, int64_t H, int64_t head_dim, float scale,
                               int64_t splits, void* workspace, int64_t workspace_bytes, hipStream_t s) {
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
  const int64_t cthreads = Tq * H * (head_dim / 8);
  const int cblocks = (int)((cthreads + 255) / 256);
#define LTX_FAS(DH, G)                                                                              \
  do {                                                                                              \
    flash_attn_kernel<DH, false, kAttnSplitWaves, true, VROW><<<(int)nwg, 64 * kAttnSplitWaves, 0, s>>>( \
        (const bf16*)Q, q_rs, (const bf16*)K, k_rs, (const bf16*)V, v_ld, nullptr, 0, nullptr,      \
        0, (int)Tq, (int)Tk, (int)H, scale_log2, so, QNorm{});                                      \
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

extern "C" int ltx_flash_attn_splitkv_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs,
                                           const void* Vt, int64_t tk_pad, void* O, int64_t o_rs,
                                           const void* gate, int64_t gate_rs, int64_t Tq, int64_t Tk,
                                           int64_t H, int64_t head_dim, float scale, int64_t splits,
                                           void* workspace, int64_t workspace_bytes, void* stream) {
  int st = attn_check(Q, q_rs, K, k_rs, O, o_rs, gate, gate_rs, Tq, Tk, H, head_dim, scale);
  if (st == LTX_OK) st = attn_check_vt(Vt, tk_pad, Tk);
  if (st != LTX_OK) return st;
  return launch_attn_splitkv<false>(Q, q_rs, K, k_rs, Vt, tk_pad, O, o_rs, gate, gate_rs, Tq, Tk, H, head_dim,
                                    scale, splits, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int ltx_flash_attn_splitkv_v_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs,
                                             const void* V, int64_t v_rs, void* O, int64_t o_rs,
                                             const void* gate, int64_t gate_rs, int64_t Tq, int64_t Tk,
                                             int64_t H, int64_t head_dim, float scale, int64_t splits,
                                             void* workspace, int64_t workspace_bytes, void* stream) {
  int st = attn_check(Q, q_rs, K, k_rs, O, o_rs, gate, gate_rs, Tq, Tk, H, head_dim, scale);
  if (st == LTX_OK) st = attn_check_v(V, v_rs, Tk, H, head_dim);
  if (st != LTX_OK) return st;
  return launch_attn_splitkv<true>(Q, q_rs, K, k_rs, V, v_rs, O, o_rs, gate, gate_rs, Tq, Tk, H, head_dim,
                                   scale, splits, workspace, workspace_bytes, (hipStream_t)stream);
}

// ---- split-KV attention without allocation --------------------------------
// The partials of the split-KV pass live in `scratch`, device memory that the
// code object itself holds (one copy per GPU, kept until the process ends).
// Every (split, query, head) row of a call is written by the pass before the
// combine reads it, so nothing has to start at zero; calls that overlap on one
// GPU share the array and race.  The host never passes `scratch` itself to a
// kernel: its name is a host-side stand-in, and the device address comes from
// hipGetSymbolAddress, resolved once per device with that device current, on
// the first call on that device: that first call must be made outside HIP
// graph capture; later calls enqueue only the two kernels and can be captured.
static __device__ __align__(256) unsigned char scratch[LTX_ATTN_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

int scratch_on_stream_device(hipStream_t stream, void** out) {
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess) return LTX_ERR_HIP;
  int dev = cur;
  if (stream && hipStreamGetDevice(stream, &dev) != hipSuccess) return LTX_ERR_HIP;
  if (dev < 0 || dev >= kMaxDevices) return LTX_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    if (dev != cur && hipSetDevice(dev) != hipSuccess) return LTX_ERR_HIP;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur && hipSetDevice(cur) != hipSuccess) return LTX_ERR_HIP;
    if (e != hipSuccess || !p) return LTX_ERR_HIP;
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return LTX_OK;
}
}  // namespace

extern "C" int ltx_flash_attn_splitkv_noalloc_bf16(const void* Q, int64_t q_rs, const void* K, int64_t k_rs,
                                                   const void* Vt, int64_t tk_pad, void* O, int64_t o_rs,
                                                   const void* gate, int64_t gate_rs, int64_t Tq, int64_t Tk,
                                                   int64_t H, int64_t head_dim, float scale, int64_t splits,
                                                   void* stream) {
  if (splits < 1 || splits > 256) return LTX_ERR_INVALID_ARG;
  // the operands are validated before the scratch need is computed from them
  int st = attn_check(Q, q_rs, K, k_rs, O, o_rs, gate, gate_rs, Tq, Tk, H, head_dim, scale);
  if (st == LTX_OK) st = attn_check_vt(Vt, tk_pad, Tk);
  if (st != LTX_OK) return st;
  const int64_t need = ltx_attn_splitkv_workspace_bytes(Tq, H, head_dim, splits);
  if (need < 0) return LTX_ERR_INVALID_ARG;
  if (need > LTX_ATTN_NOALLOC_SCRATCH_BYTES) return LTX_ERR_SCRATCH_LIMIT;
  void* ws = nullptr;
  st = scratch_on_stream_device((hipStream_t)stream, &ws);
  if (st != LTX_OK) return st;
  return ltx_flash_attn_splitkv_bf16(Q, q_rs, K, k_rs, Vt, tk_pad, O, o_rs, gate, gate_rs, Tq, Tk, H,
                                     head_dim, scale, splits, ws, LTX_ATTN_NOALLOC_SCRATCH_BYTES, stream);
}
