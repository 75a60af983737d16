// Bandwidth-bound fused row kernels of the DiT block: AdaLN (RMSNorm +
// shift/scale), gated residual add, QK-RMSNorm + split RoPE and the output
// head's LayerNorm modulation.
//
// Layout: one 64-lane wavefront owns one token row at a time.  Lane L reads
// the 16-byte vectors L, L+64, L+128, ... of the row, so every load and store
// instruction of a wave moves one contiguous 1 KiB span of HBM.  The
// per-channel parameters (1+scale, shift, gate) depend only on the lane's
// channels: the gated add keeps its gate in registers across the rows a wave
// visits, AdaLN keeps 1+scale and shift in LDS shared by the block's waves.
// Rows are held packed (bf16) in registers and widened where used.  Row
// reductions are wave-local shuffles; no barriers inside the row loop, no
// atomics.
#include "ltx_common.h"

namespace ltx {

constexpr int kRowBlock = 256;          // 4 waves per workgroup
constexpr int kWavesPerBlock = kRowBlock / kWave;
constexpr int64_t kMaxRowBlocks = 2048;  // 256 CUs x 8 waves / 4 waves per block... x4 headroom

__device__ __forceinline__ void load8(const bf16* p, float* out) {
  bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = (float)v[i];
}

__device__ __forceinline__ void store8(bf16* p, const float* in) {
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (bf16)in[i];
  *reinterpret_cast<bf16x8*>(p) = v;
}

// Streaming forms for the row kernels' activations: nontemporal loads and
// stores (read once, written once) leave the caches to the data that is
// reused; +8-10 % of HBM bandwidth on the 14640 x 4096 rows.
__device__ __forceinline__ bf16x8 load8_stream(const bf16* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(p));
}

__device__ __forceinline__ void store8_stream(bf16* p, const float* in) {
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (bf16)in[i];
  __builtin_nontemporal_store(v, reinterpret_cast<bf16x8*>(p));
}

__device__ __forceinline__ void load8f(const float* p, float* out) {
  f32x4 a = *reinterpret_cast<const f32x4*>(p);
  f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
  out[0] = a[0]; out[1] = a[1]; out[2] = a[2]; out[3] = a[3];
  out[4] = b[0]; out[5] = b[1]; out[6] = b[2]; out[7] = b[3];
}

// ---------------------------------------------------------------------------
// AdaLN: out = bf16(rms(x) * (1 + scale) + shift)
// VPL = vectors (8 bf16) per lane = C / 512.
// THREADS: workgroup size.  Every workgroup first copies the modulation rows
// (2 x C fp32) into LDS, so a launch of few rows uses large workgroups (fewer
// copies per row); a launch of many rows, small ones (more workgroups
// resident per CU).
// NOUT = 2: one read of each row, two modulations of the same norm (scale2,
// shift2 into out2) -- the A2V and V2A inputs of one stream.
template <int VPL, int THREADS, int NOUT = 1>
__global__ __launch_bounds__(THREADS) void adaln_kernel(
    const bf16* __restrict__ x, int64_t x_stride, const float* __restrict__ scale,
    const float* __restrict__ shift, bf16* out, int64_t out_stride, const float* __restrict__ scale2,
    const float* __restrict__ shift2, bf16* out2, int64_t out2_stride, int64_t rows, float eps, int flags) {
  constexpr int C = VPL * 512;
  constexpr int WAVES = THREADS / kWave;
  // 1 + scale and shift of the whole row live in LDS (shared by the block's
  // waves) rather than in registers: ~100 fewer VGPRs per lane, twice the
  // waves in flight per SIMD.
  __shared__ __attribute__((aligned(16))) float s_onep[NOUT][C], s_shift[NOUT][C];
  for (int i = threadIdx.x; i < C; i += THREADS) {
    s_onep[0][i] = 1.0f + scale[i];
    s_shift[0][i] = shift[i];
    if constexpr (NOUT == 2) {
      s_onep[NOUT - 1][i] = 1.0f + scale2[i];
      s_shift[NOUT - 1][i] = shift2[i];
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave0 = (int64_t)blockIdx.x * WAVES + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * WAVES;
  const float inv_c = 1.0f / (float)C;
  const bool round_norm = (flags & LTX_ADALN_ROUND_NORM) != 0;
  const bool no_norm = (flags & LTX_ADALN_NO_NORM) != 0;

  for (int64_t r = wave0; r < rows; r += nwaves) {
    // An opaque zero offset keeps the LDS reads in the row loop (hoisted,
    // they would pin the modulation in registers again).
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    const bf16* xr = x + r * x_stride;
    // the row stays packed (bf16) in registers and is widened where used:
    // half the VGPRs of a float copy, more rows in flight per SIMD
    bf16x8 xv[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      xv[j] = load8_stream(xr + (lane + j * kWave) * 8);
    float inv = 1.0f;
    if (!no_norm) {
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < VPL; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float v = (float)xv[j][i];
          ss = fmaf(v, v, ss);
        }
      ss = wave_sum(ss);
      inv = rsqrt_rn(ss * inv_c + eps);
    }
#pragma unroll
    for (int k = 0; k < NOUT; ++k) {
      const float* onep = s_onep[k] + z;
      const float* shp = s_shift[k] + z;
      bf16* orow = k == 0 ? out + r * out_stride : out2 + r * out2_stride;
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        const int c0 = (lane + j * kWave) * 8;
        float op[8], sh[8], o[8];
        load8f(onep + c0, op);
        load8f(shp + c0, sh);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float n = (float)xv[j][i] * inv;
          if (round_norm) n = round_bf(n);
          o[i] = n * op[i] + sh[i];
        }
        store8_stream(orow + c0, o);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Gated residual add: out = bf16(gate * branch + residual)
// One-wave workgroups: the hardware spreads them over the CUs one by one, so
// 3456 rows put 13-14 on every CU (four-wave workgroups: up to 16 on some
// while others hold 12): 17.2 -> 16.7 us at 3456 x 4096, 9.0 -> 8.0 us at
// 1296 x 4096, 61.0 -> 60.4 us at 14640 x 4096.
constexpr int kGatedAddThreads = kWave;
template <int VPL>
__global__ __launch_bounds__(kGatedAddThreads) void gated_add_kernel(
    const bf16* residual, int64_t res_stride, const bf16* __restrict__ branch,
    int64_t br_stride, const float* __restrict__ gate, bf16* out, int64_t out_stride,
    int64_t rows, int flags) {
  constexpr int WAVES = kGatedAddThreads / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave0 = (int64_t)blockIdx.x * WAVES + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * WAVES;
  const bool round_prod = (flags & LTX_GATED_ROUND_PRODUCT) != 0;

  float g[VPL][8];
#pragma unroll
  for (int j = 0; j < VPL; ++j) load8f(gate + (lane + j * kWave) * 8, g[j]);

  for (int64_t r = wave0; r < rows; r += nwaves) {
    bf16x8 rv[VPL], bv[VPL];  // packed, widened where used
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int c0 = (lane + j * kWave) * 8;
      rv[j] = load8_stream(residual + r * res_stride + c0);
      bv[j] = load8_stream(branch + r * br_stride + c0);
    }
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float b = (float)bv[j][i], rr = (float)rv[j][i];
        if (round_prod)
          o[i] = round_bf(b * g[j][i]) + rr;
        else
          o[i] = fmaf(g[j][i], b, rr);
      }
      store8_stream(out + r * out_stride + (lane + j * kWave) * 8, o);
    }
  }
}

// ---------------------------------------------------------------------------
// QK-RMSNorm + split RoPE, in place.
//
// Lane L owns PPL = D/1024 "pairs" p = L + 64*j.  A pair is two 8-channel
// vectors of one head that rotate together: v1 in the first half of the head,
// v2 = v1 + head_dim/16 in the second half.  Its RoPE angles are the 8
// consecutive table entries [8p, 8p+8) of the token's (D/2)-wide table row, so
// each lane reads its own cos/sin with two 16-byte loads per table.  The norm
// weights live in LDS (read once per workgroup).
//
// A token's table row may also be factored over position axes: n rows of
// stacked per-axis tables whose entries combine as cos = c_0 * c_1 * ...,
// sin = s_0 + s_1 + ...  Each column belongs to one axis; every other axis
// holds exactly 1 and -0 there, so the combination reproduces that axis'
// entry bit for bit (x * 1 = x and x + -0 = x for every float x).
struct RopeRows {
  const float* c[3];
  const float* s[3];
  int n;  // 0: no RoPE
};

// One row in place: its values stay in registers for the reduction; the
// RoPE table entries of chunk j are loaded while chunk j-1 is written (the
// first chunk's during the reduction), so at most two chunks' tables are live.
template <int PPL, int HALF_VECS>
__device__ __forceinline__ void qknorm_rope_row(bf16* row, const float* w_lds, const RopeRows& tr, float eps,
                                                int lane) {
  constexpr int D = PPL * 1024;
  bf16x8 a[PPL], b[PPL];  // packed; widened where used
  int v1[PPL];
#pragma unroll
  for (int j = 0; j < PPL; ++j) {
    const int p = lane + j * kWave;
    v1[j] = (p / HALF_VECS) * (2 * HALF_VECS) + (p % HALF_VECS);
    a[j] = *reinterpret_cast<const bf16x8*>(row + v1[j] * 8);
    b[j] = *reinterpret_cast<const bf16x8*>(row + (v1[j] + HALF_VECS) * 8);
  }
  auto load_tab = [&](int j, float (&c)[8], float (&s)[8]) {
    const int p = lane + j * kWave;
    load8f(tr.c[0] + p * 8, c);
    load8f(tr.s[0] + p * 8, s);
#pragma unroll
    for (int ax = 1; ax < 3; ++ax) {
      if (ax < tr.n) {
        float c2[8], s2[8];
        load8f(tr.c[ax] + p * 8, c2);
        load8f(tr.s[ax] + p * 8, s2);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          c[i] *= c2[i];
          s[i] += s2[i];
        }
      }
    }
  };
  float cs[2][8], sn[2][8];
  if (tr.n > 0) load_tab(0, cs[0], sn[0]);
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < PPL; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float fa = (float)a[j][i], fb = (float)b[j][i];
      ss = fmaf(fa, fa, fmaf(fb, fb, ss));
    }
  ss = wave_sum(ss);
  const float inv = rsqrt_rn(ss * (1.0f / (float)D) + eps);
#pragma unroll
  for (int j = 0; j < PPL; ++j) {
    // keep the table loads of chunk j+1 here (not hoisted above the
    // reduction, which would hold every chunk's table in registers)
    __builtin_amdgcn_sched_barrier(0);
    if (tr.n > 0 && j + 1 < PPL) load_tab(j + 1, cs[(j + 1) & 1], sn[(j + 1) & 1]);
    float wa[8], wb[8];
    load8f(w_lds + v1[j] * 8, wa);
    load8f(w_lds + (v1[j] + HALF_VECS) * 8, wb);
    float oa[8], ob[8];
    // re-widen the packed values here (the widened copies of the reduction
    // are not kept alive until now)
    bf16x8 aj = a[j], bj = b[j];
    asm volatile("" : "+v"(aj), "+v"(bj));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x1 = round_bf((float)aj[i] * inv * wa[i]);
      const float x2 = round_bf((float)bj[i] * inv * wb[i]);
      if (tr.n > 0) {
        oa[i] = x1 * cs[j & 1][i] - x2 * sn[j & 1][i];
        ob[i] = x1 * sn[j & 1][i] + x2 * cs[j & 1][i];
      } else {
        oa[i] = x1;
        ob[i] = x2;
      }
    }
    store8(row + v1[j] * 8, oa);
    store8(row + (v1[j] + HALF_VECS) * 8, ob);
  }
}

// THREADS: workgroup size, chosen per launch as for adaln_kernel (each
// workgroup copies both norm weight rows into LDS first).
// Table of one operand: per-token rows (idx null: row t of cos / sin), or
// `axes` factored rows per token, idx[t * axes + a] into the stacked tables of
// `tab_rows` rows (indices clamped into range); cos null: no RoPE.
struct RopeTable {
  const float* cos;
  const float* sin;
  const int* idx;
  int axes;
  int64_t tab_rows;
};

__device__ __forceinline__ RopeRows rope_rows(const RopeTable& t, int64_t tok, int64_t half) {
  RopeRows r;
  r.n = t.cos == nullptr ? 0 : (t.idx == nullptr ? 1 : t.axes);
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    int64_t row = tok;
    if (t.idx != nullptr && a < t.axes) {
      row = t.idx[tok * t.axes + a];
      row = row < 0 ? 0 : (row < t.tab_rows ? row : t.tab_rows - 1);
    }
    r.c[a] = t.cos + row * half;
    r.s[a] = t.sin + row * half;
  }
  return r;
}

// One wave per row: task 2t is Q row t and task 2t+1 is K row t while both
// operands have rows, so a token's two rows run side by side and its table
// rows are fetched once from memory and once from cache.  At most 128
// registers per lane: 4 waves per SIMD (the earlier layout needed 183, 2 per
// SIMD).
template <int PPL, int HALF_VECS, int THREADS>
__global__ __launch_bounds__(THREADS, 4) void qknorm_rope_kernel(
    bf16* q, int64_t q_stride, int64_t rows_q, const float* __restrict__ wq, RopeTable tq, bf16* k,
    int64_t k_stride, int64_t rows_k, const float* __restrict__ wk, RopeTable tk, float eps) {
  constexpr int D = PPL * 1024;
  constexpr int WAVES = THREADS / kWave;
  __shared__ float w_lds[2 * D];
  for (int i = threadIdx.x; i < D; i += THREADS) {
    w_lds[i] = rows_q > 0 ? wq[i] : 0.0f;
    w_lds[D + i] = rows_k > 0 ? wk[i] : 0.0f;
  }
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1);
  // 16-wave workgroups (at most one per CU, at most 256 of them) number the
  // tasks across the grid: wave pair i of workgroup b takes tasks 2 (i G +
  // b) + {0, 1} (G = grid size) and then every 16 G-th after them, so a
  // second pass over the tasks is spread over every CU instead of filling
  // the first workgroups' waves; 8-wave ones take consecutive tasks
  const int64_t lw = threadIdx.x >> 6;
  const int64_t wave0 = THREADS == 1024 ? 2 * ((lw >> 1) * gridDim.x + blockIdx.x) + (lw & 1)
                                        : (int64_t)blockIdx.x * WAVES + lw;
  const int64_t nwaves = (int64_t)gridDim.x * WAVES;
  const int64_t half = D / 2;
  // tasks [0, 2 mn) pair the operands' rows; the rest are the larger
  // operand's remaining rows
  const int64_t mn = rows_q < rows_k ? rows_q : rows_k;
  const int64_t tasks = rows_q + rows_k;
  for (int64_t r = wave0; r < tasks; r += nwaves) {
    const int64_t t = r < 2 * mn ? (r >> 1) : mn + (r - 2 * mn);
    const bool is_k = r < 2 * mn ? (r & 1) != 0 : rows_k > rows_q;
    if (!is_k) {
      if (t < rows_q) qknorm_rope_row<PPL, HALF_VECS>(q + t * q_stride, w_lds, rope_rows(tq, t, half), eps, lane);
    } else if (t < rows_k) {
      qknorm_rope_row<PPL, HALF_VECS>(k + t * k_stride, w_lds + D, rope_rows(tk, t, half), eps, lane);
    }
  }
}

// ---------------------------------------------------------------------------
// Output head: bf16 LayerNorm + bf16-arithmetic modulation.
template <int VPL>
__global__ __launch_bounds__(kRowBlock) void output_norm_kernel(
    const bf16* __restrict__ x, int64_t x_stride, const float* __restrict__ table,
    const float* __restrict__ emb, bf16* out, int64_t out_stride, int64_t rows, float eps) {
  constexpr int C = VPL * 512;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave0 = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
  float shf[VPL][8], ops[VPL][8];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int c0 = (lane + j * kWave) * 8;
    float t0[8], t1[8], e[8];
    load8f(table + c0, t0);
    load8f(table + C + c0, t1);
    load8f(emb + c0, e);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      shf[j][i] = round_bf(t0[i] + e[i]);
      ops[j][i] = round_bf(1.0f + round_bf(t1[i] + e[i]));
    }
  }
  for (int64_t r = wave0; r < rows; r += nwaves) {
    float xv[VPL][8];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      load8(x + r * x_stride + (lane + j * kWave) * 8, xv[j]);
#pragma unroll
      for (int i = 0; i < 8; ++i) s += xv[j][i];
    }
    const float mean = wave_sum(s) * (1.0f / (float)C);
    float v = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float d = xv[j][i] - mean;
        v = fmaf(d, d, v);
      }
    const float inv = rsqrt_rn(wave_sum(v) * (1.0f / (float)C) + eps);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float n = round_bf((xv[j][i] - mean) * inv);
        o[i] = round_bf(n * ops[j][i]) + shf[j][i];
      }
      store8(out + r * out_stride + (lane + j * kWave) * 8, o);
    }
  }
}

// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void euler_kernel(const bf16* latent, const bf16* velocity,
                                                    float sigma, float ratio, bf16* out,
                                                    int64_t n) {
  const int64_t nvec = n / 8;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nvec; i += stride) {
    float l[8], v[8], o[8];
    load8(latent + i * 8, l);
    load8(velocity + i * 8, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x0 = sub_rn(l[e], mul_rn(sigma, v[e]));
      o[e] = add_rn(x0, mul_rn(ratio, sub_rn(l[e], x0)));
    }
    store8(out + i * 8, o);
  }
  // scalar tail (n not a multiple of 8)
  if (blockIdx.x == 0 && threadIdx.x < (n & 7)) {
    const int64_t e = nvec * 8 + threadIdx.x;
    const float l = (float)latent[e], v = (float)velocity[e];
    const float x0 = sub_rn(l, mul_rn(sigma, v));
    out[e] = (bf16)add_rn(x0, mul_rn(ratio, sub_rn(l, x0)));
  }
}

__global__ void timestep_embedding_kernel(const float* values, int64_t count, float mult,
                                          float* out, int64_t dim) {
  const int64_t half = dim / 2;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= count * dim) return;
  const int64_t b = idx / dim, c = idx % dim;
  if (c >= 2 * half) {  // odd dim: zero pad
    out[idx] = 0.0f;
    return;
  }
  const int64_t i = c < half ? c : c - half;
  // exponent = (-ln(10000) * i) / half, each step rounded to fp32 as in the
  // reference's fp32 array arithmetic.
  const float expo = __fdiv_rn(__fmul_rn(-9.210340371976184f, (float)i), (float)half);
  const float t = __fmul_rn(values[b], mult);
  const float arg = __fmul_rn(t, expf(expo));
  out[idx] = c < half ? cosf(arg) : sinf(arg);
}

// GEMV: each wave computes kGemvRowsPerWave outputs for every batch entry;
// x is staged in LDS once per workgroup (batch * K floats of dynamic LDS, so
// small batches leave room for many workgroups per CU).  A wave first issues
// every weight load of its rows (KIT 16-byte loads per lane and row, K <=
// 512 * KIT), then accumulates them in k order: one round trip to memory per
// wave instead of one per 512 columns.  Lane l accumulates columns l*8 + i +
// 512 j in the order j, i; the wave sum closes the row.
constexpr int kGemvRowsPerWave = 2;
constexpr int kGemvMaxK = 4096;
constexpr int kGemvMaxBatch = 4;

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

template <int KIT>
__global__ __launch_bounds__(256) void gemv_kernel(const float* __restrict__ x, int batch,
                                                   int K, const bf16* __restrict__ W,
                                                   const float* __restrict__ bias,
                                                   float* __restrict__ y, int64_t N, int flags) {
  extern __shared__ float xs[];  // batch * K
  for (int i = threadIdx.x; i < batch * K; i += blockDim.x) {
    float v = x[i];
    if (flags & LTX_GEMV_SILU_INPUT) v = silu(v);
    xs[i] = v;
  }
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x / kWave) + (threadIdx.x >> 6);
  const int64_t n0 = wave * kGemvRowsPerWave;
  bf16x8 wv[kGemvRowsPerWave][KIT];
#pragma unroll
  for (int rr = 0; rr < kGemvRowsPerWave; ++rr) {
    const int64_t n = n0 + rr < N ? n0 + rr : N - 1;
#pragma unroll
    for (int j = 0; j < KIT; ++j) {
      const int k0 = lane * 8 + j * kWave * 8;
      if (k0 < K) wv[rr][j] = *reinterpret_cast<const bf16x8*>(W + n * (int64_t)K + k0);
    }
  }
#pragma unroll
  for (int rr = 0; rr < kGemvRowsPerWave; ++rr) {
    const int64_t n = n0 + rr;
    if (n >= N) break;
    float acc[kGemvMaxBatch] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KIT; ++j) {
      const int k0 = lane * 8 + j * kWave * 8;
      if (k0 < K) {
        for (int b = 0; b < batch; ++b) {
          const float* xb = xs + b * K + k0;
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[b] = fmaf((float)wv[rr][j][i], xb[i], acc[b]);
        }
      }
    }
    for (int b = 0; b < batch; ++b) {
      float v = wave_sum(acc[b]);
      if (lane == 0) {
        if (bias) v += bias[n];
        if (flags & LTX_GEMV_SILU_OUTPUT) v = silu(v);
        y[(int64_t)b * N + n] = v;
      }
    }
  }
}

// out[b, i] = table[b, i] + vec[i]  (per-block AdaLN modulation rows)
__global__ void broadcast_add_kernel(const float* __restrict__ table, const float* __restrict__ vec,
                                     float* __restrict__ out, int64_t nb, int64_t n) {
  const int64_t total = nb * n;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride)
    out[i] = table[i] + vec[i % n];
}

}  // namespace ltx

// ===========================================================================
// C ABI
// ===========================================================================
using namespace ltx;

static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// AdaLN and the gated add: up to one row per wave, so at 14640 rows every
// row's loads are issued by the first wave that owns it (no grid-stride
// second pass behind a wave's stores).
constexpr int64_t kMaxStreamRowBlocks = 4096;

// Row launches of at most this many rows use the large-workgroup forms.
constexpr int64_t kFewRows = 8192;

static inline int row_grid(int64_t rows, int64_t cap = kMaxRowBlocks, int waves = kWavesPerBlock) {
  int64_t blocks = (rows + waves - 1) / waves;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  return (int)blocks;
}

extern "C" const char* ltx_status_string(int status) {
  switch (status) {
    case LTX_OK: return "ok";
    case LTX_ERR_INVALID_ARG: return "invalid argument";
    case LTX_ERR_UNSUPPORTED: return "unsupported shape";
    case LTX_ERR_HIP: return "HIP launch error";
    case LTX_ERR_ALIGNMENT: return "pointer or stride not 16-byte aligned";
    case LTX_ERR_SCRATCH_LIMIT: return "request exceeds the fixed scratch of a no-allocation entry point";
    default: return "unknown status";
  }
}

extern "C" int ltx_version(void) { return 100; }

// Device clock stamp: one lane writes the GPU's constant-rate real-time
// counter into dst[0].  Stream-ordered like any kernel (and recorded as a
// kernel node under graph capture), so two stamps bracket the work between
// them on that stream.
__global__ void clock_stamp_kernel(uint64_t* dst) {
  if (threadIdx.x == 0) dst[0] = __builtin_amdgcn_s_memrealtime();
}

extern "C" int ltx_device_clock_stamp(uint64_t* dst, void* stream) {
  if (!dst) return LTX_ERR_INVALID_ARG;
  if (((uintptr_t)dst & 7u) != 0) return LTX_ERR_ALIGNMENT;
  clock_stamp_kernel<<<1, 64, 0, (hipStream_t)stream>>>(dst);
  return ltx_launch_status();
}

static int adaln_launch(const void* x, int64_t x_stride, const float* scale, const float* shift, void* out,
                        int64_t out_stride, const float* scale2, const float* shift2, void* out2,
                        int64_t out2_stride, int64_t rows, int64_t C, float eps, int flags, void* stream) {
  const bool dual = out2 != nullptr;
  if (rows < 0 || !x || !scale || !shift || !out || (dual && (!scale2 || !shift2))) return LTX_ERR_INVALID_ARG;
  if (C <= 0 || C % 512 != 0 || C > 4096) return LTX_ERR_UNSUPPORTED;
  if (x_stride < C || out_stride < C || (dual && out2_stride < C)) return LTX_ERR_INVALID_ARG;
  if (!aligned16(x) || !aligned16(out) || !aligned16(scale) || !aligned16(shift) || x_stride % 8 ||
      out_stride % 8 || (dual && (!aligned16(out2) || !aligned16(scale2) || !aligned16(shift2) || out2_stride % 8)))
    return LTX_ERR_ALIGNMENT;
  if (rows == 0) return LTX_OK;
  hipStream_t s = (hipStream_t)stream;
  const bf16* xp = (const bf16*)x;
  bf16* op = (bf16*)out;
  bf16* op2 = (bf16*)out2;
  // few rows: large workgroups (one LDS copy of the modulation per
  // workgroup), W waves: from 1024 to 4096 rows the smallest of 8, 12, 14
  // and 16 that needs at most 256 workgroups -- at most one per CU of the
  // MI355X, every CU holding about the same rows (3456 rows: 14 waves, 247
  // workgroups, 11.8 vs 11.9 us at C = 4096 and 6.3 vs 6.6 us at C = 2048
  // against 216 of 16; 1296 rows: 8 waves, 5.7 vs 8.4 us against 81 of 16);
  // 16 below and above that range.
  const bool few = rows <= kFewRows;
  int W = 16;
  if (rows > 1024 && rows <= 4096) {
    const int64_t need = (rows + 255) / 256;
    W = need <= 8 ? 8 : need <= 12 ? 12 : need <= 14 ? 14 : 16;
  }
  const int grid = few ? row_grid(rows, kMaxStreamRowBlocks, W) : row_grid(rows, kMaxStreamRowBlocks);
#define LTX_ADALN_ARGS xp, x_stride, scale, shift, op, out_stride, scale2, shift2, op2, out2_stride, rows, eps, flags
#define LTX_ADALN_FEW(V, N)                                                                         \
  (W == 8    ? adaln_kernel<V, 512, N><<<grid, 512, 0, s>>>(LTX_ADALN_ARGS)                         \
   : W == 12 ? adaln_kernel<V, 768, N><<<grid, 768, 0, s>>>(LTX_ADALN_ARGS)                         \
   : W == 14 ? adaln_kernel<V, 896, N><<<grid, 896, 0, s>>>(LTX_ADALN_ARGS)                         \
             : adaln_kernel<V, 1024, N><<<grid, 1024, 0, s>>>(LTX_ADALN_ARGS))
#define LTX_ADALN_LAUNCH(V)                                                                                   \
  (dual ? (few ? LTX_ADALN_FEW(V, 2) : (adaln_kernel<V, kRowBlock, 2><<<grid, kRowBlock, 0, s>>>(LTX_ADALN_ARGS))) \
        : (few ? LTX_ADALN_FEW(V, 1) : (adaln_kernel<V, kRowBlock, 1><<<grid, kRowBlock, 0, s>>>(LTX_ADALN_ARGS))))
  switch (C / 512) {
    case 1: LTX_ADALN_LAUNCH(1); break;
    case 2: LTX_ADALN_LAUNCH(2); break;
    case 4: LTX_ADALN_LAUNCH(4); break;
    case 8: LTX_ADALN_LAUNCH(8); break;
    default: return LTX_ERR_UNSUPPORTED;
  }
#undef LTX_ADALN_LAUNCH
#undef LTX_ADALN_FEW
#undef LTX_ADALN_ARGS
  return ltx_launch_status();
}

extern "C" int ltx_adaln_norm_fused_bf16(const void* x, int64_t x_stride, const float* scale,
                                         const float* shift, void* out, int64_t out_stride,
                                         int64_t rows, int64_t C, float eps, int flags,
                                         void* stream) {
  return adaln_launch(x, x_stride, scale, shift, out, out_stride, nullptr, nullptr, nullptr, 0, rows, C, eps, flags,
                      stream);
}

extern "C" int ltx_adaln_norm_fused2_bf16(const void* x, int64_t x_stride, const float* scale,
                                          const float* shift, void* out, int64_t out_stride,
                                          const float* scale2, const float* shift2, void* out2,
                                          int64_t out2_stride, int64_t rows, int64_t C, float eps, int flags,
                                          void* stream) {
  if (!out2) return LTX_ERR_INVALID_ARG;
  return adaln_launch(x, x_stride, scale, shift, out, out_stride, scale2, shift2, out2, out2_stride, rows, C, eps,
                      flags, stream);
}

extern "C" int ltx_gated_add_fused_bf16(const void* residual, int64_t residual_stride,
                                        const void* branch, int64_t branch_stride,
                                        const float* gate, void* out, int64_t out_stride,
                                        int64_t rows, int64_t C, int flags, void* stream) {
  if (rows < 0 || !residual || !branch || !gate || !out) return LTX_ERR_INVALID_ARG;
  if (C <= 0 || C % 512 != 0 || C > 4096) return LTX_ERR_UNSUPPORTED;
  if (residual_stride < C || branch_stride < C || out_stride < C) return LTX_ERR_INVALID_ARG;
  if (!aligned16(residual) || !aligned16(branch) || !aligned16(gate) || !aligned16(out) ||
      residual_stride % 8 || branch_stride % 8 || out_stride % 8)
    return LTX_ERR_ALIGNMENT;
  if (rows == 0) return LTX_OK;
  hipStream_t s = (hipStream_t)stream;
  const bf16* rp = (const bf16*)residual;
  const bf16* bp = (const bf16*)branch;
  bf16* op = (bf16*)out;
  const int grid = row_grid(rows, kMaxStreamRowBlocks * kWavesPerBlock, kGatedAddThreads / kWave);
  switch (C / 512) {
    case 1: gated_add_kernel<1><<<grid, kGatedAddThreads, 0, s>>>(rp, residual_stride, bp, branch_stride, gate, op, out_stride, rows, flags); break;
    case 2: gated_add_kernel<2><<<grid, kGatedAddThreads, 0, s>>>(rp, residual_stride, bp, branch_stride, gate, op, out_stride, rows, flags); break;
    case 4: gated_add_kernel<4><<<grid, kGatedAddThreads, 0, s>>>(rp, residual_stride, bp, branch_stride, gate, op, out_stride, rows, flags); break;
    case 8: gated_add_kernel<8><<<grid, kGatedAddThreads, 0, s>>>(rp, residual_stride, bp, branch_stride, gate, op, out_stride, rows, flags); break;
    default: return LTX_ERR_UNSUPPORTED;
  }
  return ltx_launch_status();
}

static int qknorm_rope_launch(void* q, int64_t q_stride, int64_t rows_q, const float* wq, RopeTable tq,
                              void* k, int64_t k_stride, int64_t rows_k, const float* wk, RopeTable tk,
                              int64_t D, int64_t head_dim, float eps, void* stream) {
  if (rows_q < 0 || rows_k < 0) return LTX_ERR_INVALID_ARG;
  if (rows_q > 0 && (!q || !wq || q_stride < D)) return LTX_ERR_INVALID_ARG;
  if (rows_k > 0 && (!k || !wk || k_stride < D)) return LTX_ERR_INVALID_ARG;
  for (const RopeTable* t : {&tq, &tk}) {
    if ((t->cos == nullptr) != (t->sin == nullptr)) return LTX_ERR_INVALID_ARG;
    if (t->idx != nullptr && (t->cos == nullptr || t->axes < 1 || t->axes > 3 || t->tab_rows < 1))
      return LTX_ERR_INVALID_ARG;
  }
  if (D <= 0 || D % 1024 != 0 || D > 4096) return LTX_ERR_UNSUPPORTED;
  if (head_dim != 64 && head_dim != 128) return LTX_ERR_UNSUPPORTED;
  if ((rows_q > 0 && (!aligned16(q) || q_stride % 8 || (tq.cos && (!aligned16(tq.cos) || !aligned16(tq.sin))))) ||
      (rows_k > 0 && (!aligned16(k) || k_stride % 8 || (tk.cos && (!aligned16(tk.cos) || !aligned16(tk.sin))))))
    return LTX_ERR_ALIGNMENT;
  const int64_t rows = rows_q > rows_k ? rows_q : rows_k;
  if (rows == 0) return LTX_OK;
  hipStream_t s = (hipStream_t)stream;
  const int64_t tasks = rows_q + rows_k;
  // 16-wave workgroups for 1024 < tasks <= 8192 (the step's 3456-row
  // launches; one LDS copy of the norm weights per 16 rows), 8-wave
  // workgroups otherwise, in a grid of at most 2048 (measured
  // fastest for each: 3456-row Q + K 42.2 -> 39.9 us, 2 x 14640 rows 149.7 ->
  // 142.6 us against 4-wave workgroups; 68 + 68 rows 7.9 against 10.9 us in
  // 16-wave ones)
  // Past 4096 tasks the 16-wave grid stops at one workgroup per CU (256 on
  // the MI355X): the 6912 tasks of the step's Q + K rows then run as 27 per
  // CU (at most 28: 16 in the first pass, 10-12 in the second) rather than 32
  // on 176 CUs and 16 on the other 80 (432 workgroups of 16 tasks).
  const bool wide = tasks > 1024 && tasks <= kFewRows;
  const int grid = wide ? row_grid(tasks, 256, 16) : row_grid(tasks, kMaxRowBlocks, 8);
  bf16* qp = (bf16*)q;
  bf16* kp = (bf16*)k;
#define LTX_QK_LAUNCH(PPL, HV)                                                                            \
  (wide ? (qknorm_rope_kernel<PPL, HV, 1024><<<grid, 1024, 0, s>>>(qp, q_stride, rows_q, wq, tq, kp, k_stride,   \
                                                                 rows_k, wk, tk, eps))                          \
       : (qknorm_rope_kernel<PPL, HV, 512><<<grid, 512, 0, s>>>(qp, q_stride, rows_q, wq, tq, kp, k_stride,     \
                                                               rows_k, wk, tk, eps)))
  const int ppl = (int)(D / 1024);
  if (head_dim == 128) {
    switch (ppl) {
      case 1: LTX_QK_LAUNCH(1, 8); break;
      case 2: LTX_QK_LAUNCH(2, 8); break;
      case 4: LTX_QK_LAUNCH(4, 8); break;
      default: return LTX_ERR_UNSUPPORTED;
    }
  } else {
    switch (ppl) {
      case 1: LTX_QK_LAUNCH(1, 4); break;
      case 2: LTX_QK_LAUNCH(2, 4); break;
      case 4: LTX_QK_LAUNCH(4, 4); break;
      default: return LTX_ERR_UNSUPPORTED;
    }
  }
#undef LTX_QK_LAUNCH
  return ltx_launch_status();
}

extern "C" int ltx_qknorm_rope_bf16(void* q, int64_t q_stride, int64_t rows_q, const float* wq,
                                    const float* cos_q, const float* sin_q, void* k,
                                    int64_t k_stride, int64_t rows_k, const float* wk,
                                    const float* cos_k, const float* sin_k, int64_t D,
                                    int64_t head_dim, float eps, void* stream) {
  const RopeTable tq{cos_q, sin_q, nullptr, 1, 0}, tk{cos_k, sin_k, nullptr, 1, 0};
  return qknorm_rope_launch(q, q_stride, rows_q, wq, tq, k, k_stride, rows_k, wk, tk, D, head_dim, eps, stream);
}

extern "C" int ltx_qknorm_rope_axes_bf16(void* q, int64_t q_stride, int64_t rows_q, const float* wq,
                                         const float* cos_q, const float* sin_q, const int32_t* idx_q,
                                         int64_t axes_q, int64_t tab_rows_q, void* k, int64_t k_stride,
                                         int64_t rows_k, const float* wk, const float* cos_k,
                                         const float* sin_k, const int32_t* idx_k, int64_t axes_k,
                                         int64_t tab_rows_k, int64_t D, int64_t head_dim, float eps,
                                         void* stream) {
  if (axes_q < 1 || axes_q > 3 || axes_k < 1 || axes_k > 3) return LTX_ERR_INVALID_ARG;
  const RopeTable tq{cos_q, sin_q, idx_q, (int)axes_q, tab_rows_q};
  const RopeTable tk{cos_k, sin_k, idx_k, (int)axes_k, tab_rows_k};
  return qknorm_rope_launch(q, q_stride, rows_q, wq, tq, k, k_stride, rows_k, wk, tk, D, head_dim, eps, stream);
}

extern "C" int ltx_output_norm_modulate_bf16(const void* x, int64_t x_stride, const float* table,
                                             const float* emb, void* out, int64_t out_stride,
                                             int64_t rows, int64_t C, float eps, void* stream) {
  if (rows < 0 || !x || !table || !emb || !out) return LTX_ERR_INVALID_ARG;
  if (C <= 0 || C % 512 != 0 || C > 4096) return LTX_ERR_UNSUPPORTED;
  if (x_stride < C || out_stride < C) return LTX_ERR_INVALID_ARG;
  if (!aligned16(x) || !aligned16(out) || !aligned16(table) || !aligned16(emb) ||
      x_stride % 8 || out_stride % 8)
    return LTX_ERR_ALIGNMENT;
  if (rows == 0) return LTX_OK;
  hipStream_t s = (hipStream_t)stream;
  const int grid = row_grid(rows);
  const bf16* xp = (const bf16*)x;
  bf16* op = (bf16*)out;
  switch (C / 512) {
    case 1: output_norm_kernel<1><<<grid, kRowBlock, 0, s>>>(xp, x_stride, table, emb, op, out_stride, rows, eps); break;
    case 2: output_norm_kernel<2><<<grid, kRowBlock, 0, s>>>(xp, x_stride, table, emb, op, out_stride, rows, eps); break;
    case 4: output_norm_kernel<4><<<grid, kRowBlock, 0, s>>>(xp, x_stride, table, emb, op, out_stride, rows, eps); break;
    case 8: output_norm_kernel<8><<<grid, kRowBlock, 0, s>>>(xp, x_stride, table, emb, op, out_stride, rows, eps); break;
    default: return LTX_ERR_UNSUPPORTED;
  }
  return ltx_launch_status();
}

extern "C" int ltx_euler_x0_step_bf16(const void* latent, const void* velocity, float sigma,
                                      float ratio, void* out, int64_t n, void* stream) {
  if (n < 0 || !latent || !velocity || !out) return LTX_ERR_INVALID_ARG;
  if (!aligned16(latent) || !aligned16(velocity) || !aligned16(out)) return LTX_ERR_ALIGNMENT;
  if (n == 0) return LTX_OK;
  int64_t blocks = (n / 8 + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  euler_kernel<<<(int)blocks, 256, 0, (hipStream_t)stream>>>(
      (const bf16*)latent, (const bf16*)velocity, sigma, ratio, (bf16*)out, n);
  return ltx_launch_status();
}

extern "C" int ltx_timestep_embedding_f32(const float* values, int64_t count, float multiplier,
                                          float* out, int64_t dim, void* stream) {
  if (count < 0 || dim < 2 || !values || !out) return LTX_ERR_INVALID_ARG;
  if (count == 0) return LTX_OK;
  const int64_t total = count * dim;
  timestep_embedding_kernel<<<(int)((total + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      values, count, multiplier, out, dim);
  return ltx_launch_status();
}

extern "C" int ltx_gemv_f32_bf16w(const float* x, int64_t batch, int64_t K, const void* W,
                                  const float* bias, float* y, int64_t N, int flags,
                                  void* stream) {
  if (!x || !W || !y || batch < 0 || N < 0) return LTX_ERR_INVALID_ARG;
  if (batch > kGemvMaxBatch || K <= 0 || K > kGemvMaxK || K % 8) return LTX_ERR_UNSUPPORTED;
  if (!aligned16(W)) return LTX_ERR_ALIGNMENT;
  if (batch == 0 || N == 0) return LTX_OK;
  const int64_t waves = (N + kGemvRowsPerWave - 1) / kGemvRowsPerWave;
  const int64_t blocks = (waves + 3) / 4;
  if (blocks > INT32_MAX) return LTX_ERR_UNSUPPORTED;
  const size_t lds = (size_t)batch * K * sizeof(float);
  hipStream_t s = (hipStream_t)stream;
  const bf16* w = (const bf16*)W;
  if (K <= 512)
    gemv_kernel<1><<<(int)blocks, 256, lds, s>>>(x, (int)batch, (int)K, w, bias, y, N, flags);
  else if (K <= 1024)
    gemv_kernel<2><<<(int)blocks, 256, lds, s>>>(x, (int)batch, (int)K, w, bias, y, N, flags);
  else if (K <= 2048)
    gemv_kernel<4><<<(int)blocks, 256, lds, s>>>(x, (int)batch, (int)K, w, bias, y, N, flags);
  else
    gemv_kernel<8><<<(int)blocks, 256, lds, s>>>(x, (int)batch, (int)K, w, bias, y, N, flags);
  return ltx_launch_status();
}

extern "C" int ltx_broadcast_add_f32(const float* table, const float* vec, float* out, int64_t nb,
                                     int64_t n, void* stream) {
  if (!table || !vec || !out || nb < 0 || n < 0) return LTX_ERR_INVALID_ARG;
  const int64_t total = nb * n;
  if (total == 0) return LTX_OK;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  broadcast_add_kernel<<<(int)blocks, 256, 0, (hipStream_t)stream>>>(table, vec, out, nb, n);
  return ltx_launch_status();
}
