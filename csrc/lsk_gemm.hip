// Projection / LM-head GEMMs over the packed token rows (solutions/packed.py:175,182,183-185;
// common/model.py:330):  C[m][n] = epilogue( sum_k A[m][k] * W[n][k] )   (F.linear, W = [out, in]).
//
// bf16 path (gfx950 MFMA v_mfma_f32_16x16x32_bf16, fp32 accumulation).  Decode GEMMs are skinny
// (M = 1..~300 tokens against 6k-128k weight rows), so the kernel is a weight stream.
//
// Weight storage (bf16): fragment-major, written once by lsk_pack_weight.  Fragment (g, j) holds rows
// 16g .. 16g+15 and k = 32j .. 32j+31 of W as 1 KiB in MFMA lane order: lane l's 16 bytes are
// W[16g + l % 16][32j + 8 (l / 16) .. +7], fragments ordered [g][j].  A wave's fragment load is then one
// contiguous 1 KiB request stream, and the k-steps of a row group follow each other in memory; the
// row-major [out, in] layout instead makes every load touch 16 rows 64 bytes at a time (an 8 KiB
// stride at K = 4096), which measured ~25 % slower on MI355X.  Weights are read with non-temporal
// loads (each byte is used once per launch); the activations use ordinary loads (re-read from L2 by
// every row tile).
//
// A workgroup of 4 waves owns a tile of (16*NS weight rows) x (16*MS tokens); every lane fetches its
// MFMA fragments with 16-byte loads (no LDS staging); the waves split K into 128-element chunks (wave
// w takes chunks w, w+4, ... of its K slice, with the next pipeline unit in flight) and their partial
// sums are added in wave order through LDS.  Weight matrices with few rows (qkv, o, w2 of the 8B
// shape) use a fixed split of K into KS slices whose fp32 partial sums the NEXT kernel reduces in
// slice order (RoPE + append, add + RMSNorm), because a cross-workgroup reduction inside the GEMM
// needs device-scope fences that cost more than the split saves on MI355X.
//
// Batch invariance: KS is chosen from the weight shape (N, K) only (lsk_gemm_plan) and the reduction
// order of every output element is fixed by (K, KS): chunks in order within a wave, waves in order,
// slices in order.  It does not depend on M or on which rows share a tile, so a token's result is
// bitwise the same whether it is decoded alone or inside a packed verify batch.
//
// Epilogues (the reference's dtype rounding points):
//   NONE      C = rnd(acc)
//   RESIDUAL  C = rnd(R + rnd(acc))                       x + F.linear(...)
//   SILU_MUL  C = rnd(rnd(silu(rnd(g))) * rnd(u))         g, u = rows n and ffn + n of W (w13)
//   PARTIAL   P[s][m][n] = acc over K slice s (fp32), reduced later in slice order
//   ARGMAX    per (token, 16*NS-row tile): max of rnd(acc) and its first index (LM head + greedy pick)
#include <type_traits>

#include "lsk_common.h"
#include "../include/lsk.h"

#define EPI_PARTIAL 3
#define EPI_ARGMAX 4
#define EPI_QKV 5

// Fused qkv epilogue (EPI_QKV): the qkv projection's output goes straight to RoPE and the caches instead of through
// K-slice partials and the RoPE + append kernel.  The weight is packed with its q and k row groups RoPE-paired
// (lsk_pack_weight_qkv): within each head of D rows (G = D / 16 groups) packed group 2 j holds dims 16 j .. 16 j + 15
// and packed group 2 j + 1 dims D / 2 + 16 j .. (the rotation partners), so a tile of two (or four) row groups holds
// whole rotation pairs and one lane owns both values of a pair.  v rows keep their order.
struct QkvRope {
  uint16_t* q;            // [N, Hq, D] RoPE-rotated queries
  uint16_t* kc;           // K cache, fragment-major 32-position blocks (k_cache_offset)
  uint16_t* vc;           // V cache, transposed 32-position blocks
  const float* cos_tab;   // [tab_len, D] fp32
  const float* sin_tab;
  const int32_t* rows;    // [N] cache row of each token
  const int32_t* pos;     // [N] position of each token
  int hq, hkv, d, max_batch, max_seq, tab_len;
};

// Token m's values x_lo, x_hi of packed row groups G (even) and G + 1, row w16 of each: a RoPE pair for q / k (stored
// rotated to q or the K cache), two v dims 16 apart otherwise (stored to the V cache), with the RoPE + append
// kernel's arithmetic (rope_pair) and indexing.
__device__ __forceinline__ void qkv_rope_store(const QkvRope& qa, int m, int G, int w16, float x_lo, float x_hi) {
  const int D = qa.d, GH = D >> 4, half = D >> 1;
  const int row = qa.rows[m], p = qa.pos[m];
  if (row < 0 || row >= qa.max_batch || p < 0 || p >= qa.max_seq || p >= qa.tab_len) return;  // host validates too
  const int kg = (qa.hq + qa.hkv) * GH;
  if (G < kg) {
    const int h = G / GH, d1 = 16 * ((G - h * GH) >> 1) + w16;
    float o1, o2;
    rope_pair<uint16_t>(x_lo, x_hi, qa.cos_tab + (long)p * D, qa.sin_tab + (long)p * D, d1, half, o1, o2);
    if (h < qa.hq) {
      uint16_t* dst = qa.q + ((long)m * qa.hq + h) * D;
      dst[d1] = f2bf(o1);
      dst[d1 + half] = f2bf(o2);
    } else {
      uint16_t* dst = qa.kc + ((long)row * qa.hkv + (h - qa.hq)) * (long)qa.max_seq * D;
      dst[k_cache_offset<uint16_t>(p, d1, D)] = f2bf(o1);
      dst[k_cache_offset<uint16_t>(p, d1 + half, D)] = f2bf(o2);
    }
  } else {
    const int gv = G - kg, h = gv / GH, d1 = 16 * (gv - h * GH) + w16;
    uint16_t* dst = qa.vc + ((long)row * qa.hkv + h) * (long)D * qa.max_seq + (long)(p >> 5) * 32 * D + (p & 31);
    dst[(long)d1 * 32] = f2bf(x_lo);
    dst[(long)(d1 + 16) * 32] = f2bf(x_hi);
  }
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + lsk_exp(-x)); }

// One lane's 16 bytes of a weight fragment, non-temporal (streamed once per launch).
__device__ __forceinline__ lsk_bf16x8 ld_w(const uint16_t* p) {
  const lsk_i32x4 v = __builtin_nontemporal_load((const lsk_i32x4*)p);
  return __builtin_bit_cast(lsk_bf16x8, v);
}

// Two workgroups per CU where the tile's registers fit 256 VGPRs (two fragment buffers of 32 VGPRs
// per weight row group and per token group, plus 4 accumulators per pair), else one.
// k-steps of 32 per pipeline unit: half chunks (64 k) for large tiles, whole 128-k chunks otherwise.
// A unit is the granularity of the register double buffer only; every accumulator still sees the
// k-steps in the same order (chunk by chunk, 32 at a time), so the result does not depend on it.
template <int NS, int MS, int EPI>
constexpr int gemm_unit() {
  constexpr int NT = EPI == LSK_EPI_SILU_MUL ? 2 * NS : NS;
  return NT + MS > 6 ? 2 : 4;
}

template <int NS, int MS, int EPI, int CK>
constexpr int gemm_occupancy() {
  constexpr int NT = EPI == LSK_EPI_SILU_MUL ? 2 * NS : NS;
  return 8 * CK * (NT + MS) + 4 * NT * MS <= 240 ? 2 : 1;
}

// AF: A is fragment-major (lsk_frag_off, whole 16-token groups).
template <int NS, int MS, int EPI, int CK = gemm_unit<NS, MS, EPI>(), bool AF = false>
__global__ __launch_bounds__(256, (gemm_occupancy<NS, MS, EPI, CK>())) void gemm_bf16_kernel(const uint16_t* __restrict__ A, long lda,
                                                        const uint16_t* __restrict__ W, long ldw,
                                                        uint16_t* __restrict__ C, long ldc,
                                                        const uint16_t* __restrict__ R, long ldr,
                                                        float* __restrict__ P, float* __restrict__ amax_v,
                                                        int* __restrict__ amax_i, int M, int N, int K, int ffn,
                                                        int kslice, int n_tiles, int m_tiles, int m_lo,
                                                        int c_nks, QkvRope qa) {
  constexpr int NT = (EPI == LSK_EPI_SILU_MUL) ? 2 * NS : NS;
  static_assert(!AF || EPI == EPI_PARTIAL || EPI == EPI_ARGMAX || EPI == LSK_EPI_SILU_MUL || EPI == EPI_QKV,
                "fragment-major A: split-K partial, silu-mul, LM head and the fused qkv");
  static_assert(EPI != EPI_QKV || (AF && NS % 2 == 0), "fused qkv: fragment-major A, whole rotation pairs per tile");
  constexpr int E = NT * MS * 256;  // partial-sum floats per wave
  __shared__ __attribute__((aligned(16))) float red[4 * E];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: loop bounds and branches are scalar
  const int l16 = lane & 15, lg = lane >> 4;
  // workgroup -> (row tile, token tile).  With several token tiles, the token tiles of one row tile
  // take launch slots 8 apart: consecutive slots go to different XCDs, so they run side by side on one
  // XCD and the second and later reads of the weight tile hit that XCD's L2 instead of HBM.
  int tn = blockIdx.x, tm = 0;
  if (m_tiles > 1) {
    const int slot = blockIdx.x >> 3;
    tm = slot % m_tiles;
    tn = (slot / m_tiles) * 8 + (blockIdx.x & 7);
    if (tn >= n_tiles) return;  // padding slot of the last group of 8
  }
  const int n0 = tn * 16 * NS;
  const int m0 = m_lo + tm * 16 * MS;  // the launch covers rows [m_lo, M) (m_lo: rows a wide-tier launch covered)
  const int s = blockIdx.z;
  const int k0 = s * kslice;
  const int k1 = min(K, k0 + kslice);

  // fragment-major weights: row group g, k-step j at W + (g * nks + j) * 512 (+ 8 * lane for this lane)
  const int nks = K >> 5;
  const uint16_t* wrow[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int gi = (t < NS) ? (n0 / 16 + t) : ((ffn + n0) / 16 + (t - NS));
    const int gmax = (EPI == LSK_EPI_SILU_MUL) ? (t < NS ? ffn / 16 - 1 : 2 * ffn / 16 - 1) : N / 16 - 1;
    gi = gi < gmax ? gi : gmax;  // clamp: padded row groups load a valid group, results discarded
    wrow[t] = W + ((long)gi * nks + (k0 >> 5)) * 512 + 8 * lane;
  }
  const uint16_t* arow[MS];
#pragma unroll
  for (int t = 0; t < MS; ++t) {
    if constexpr (AF) {
      // whole 16-token groups up to (M + 15) / 16; groups past it (last token tile) read the last one
      const int grp = min(m0 / 16 + t, (M + 15) / 16 - 1);
      arow[t] = A + ((long)grp * nks + (k0 >> 5)) * 512 + 8 * lane;  // k-step j at + j * 512
    } else {
      int m = m0 + 16 * t + l16;
      m = m < M - 1 ? m : M - 1;
      arow[t] = A + (long)m * lda + k0 + 8 * lg;
    }
  }
  constexpr long AK = AF ? 16 : 1;  // A elements per k (fragment-major: 512 per 32-k step)

  lsk_f32x4 acc[NT][MS];
#pragma unroll
  for (int a = 0; a < NT; ++a)
#pragma unroll
    for (int t = 0; t < MS; ++t) acc[a][t] = (lsk_f32x4){0.f, 0.f, 0.f, 0.f};

  const int nk32 = (k1 - k0) / 32;
  const int nfull = nk32 / 4;                                 // full 128-element chunks of the slice
  const int my_n = nfull > wave ? (nfull - wave + 3) / 4 : 0;  // this wave's chunks: wave, wave + 4, ...
  constexpr int UPC = 4 / CK;                                 // units per chunk
  const int my_u = my_n * UPC;
  lsk_bf16x8 wA[CK][NT], aA[CK][MS], wB[CK][NT], aB[CK][MS];
  // unit u of this wave: chunk wave + 4 * (u / UPC), k-steps (u % UPC) * CK ...
  auto load = [&](lsk_bf16x8 (&wf)[CK][NT], lsk_bf16x8 (&af)[CK][MS], int u) {
    const int kb = (wave + 4 * (u / UPC)) * 128 + (u % UPC) * CK * 32;
#pragma unroll
    for (int ks = 0; ks < CK; ++ks) {
      const int k = kb + ks * 32;
#pragma unroll
      for (int a = 0; a < NT; ++a) wf[ks][a] = ld_w(wrow[a] + (long)k * 16);
#pragma unroll
      for (int t = 0; t < MS; ++t) af[ks][t] = *(const lsk_bf16x8*)(arow[t] + AK * k);
    }
  };
  auto comp = [&](lsk_bf16x8 (&wf)[CK][NT], lsk_bf16x8 (&af)[CK][MS]) {
#pragma unroll
    for (int ks = 0; ks < CK; ++ks)
#pragma unroll
      for (int a = 0; a < NT; ++a)
#pragma unroll
        for (int t = 0; t < MS; ++t)
          acc[a][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[ks][a], af[ks][t], acc[a][t], 0, 0, 0);
  };
  // two register buffers: the next unit is in flight while the current one is multiplied.  (A branch-free form of
  // this loop -- every load unconditional, the last units peeled off, scheduling barriers keeping each unit's loads
  // ahead of the previous unit's MFMAs -- gets exact wait counts but measured 1-2 % slower per layer stack.)
  if (my_u > 0) load(wA, aA, 0);
  int i = 0;
  for (; i + 2 <= my_u; i += 2) {
    load(wB, aB, i + 1);
    comp(wA, aA);
    if (i + 2 < my_u) load(wA, aA, i + 2);
    comp(wB, aB);
  }
  if (i < my_u) comp(wA, aA);
  // tail chunk (slice length % 128 != 0): owned by wave nfull % 4, k-steps in order
  if (wave == (nfull & 3)) {
    for (int kk = nfull * 4; kk < nk32; ++kk) {
      const int k = kk * 32;
      lsk_bf16x8 w1[NT], a1[MS];
#pragma unroll
      for (int a = 0; a < NT; ++a) w1[a] = ld_w(wrow[a] + (long)k * 16);
#pragma unroll
      for (int t = 0; t < MS; ++t) a1[t] = *(const lsk_bf16x8*)(arow[t] + AK * k);
#pragma unroll
      for (int a = 0; a < NT; ++a)
#pragma unroll
        for (int t = 0; t < MS; ++t)
          acc[a][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1[a], a1[t], acc[a][t], 0, 0, 0);
    }
  }

  // partial sums -> LDS, element ((a*MS + t)*64 + lane)*4 + i  <->  row 16a + 4lg + i, token 16t + l16
  float* my = red + wave * E;
#pragma unroll
  for (int a = 0; a < NT; ++a)
#pragma unroll
    for (int t = 0; t < MS; ++t)
      *(float4*)(my + ((a * MS + t) * 64 + lane) * 4) = make_float4(acc[a][t][0], acc[a][t][1], acc[a][t][2], acc[a][t][3]);
  __syncthreads();

  constexpr int TN = 16 * NS, TM = 16 * MS;
  auto reduced = [&](int a, int ml, int w16) {
    const int e = ((a * MS + (ml >> 4)) * 64 + (w16 >> 2) * 16 + (ml & 15)) * 4 + (w16 & 3);
    return ((red[e] + red[E + e]) + red[2 * E + e]) + red[3 * E + e];
  };
  if constexpr (EPI == EPI_ARGMAX) {
    // reduced, bf16-rounded logits back into wave 0's region, then one thread per token scans the tile
    float vals[TN * TM / 256];
#pragma unroll
    for (int j = 0; j < TN * TM / 256; ++j) {
      const int o = tid + 256 * j;
      const int ml = o / TN, nl = o - ml * TN;
      vals[j] = rbf(reduced(nl >> 4, ml, nl & 15));
      const int m = m0 + ml, n = n0 + nl;
      if (C != nullptr && m < M && n < N) C[(long)m * ldc + n] = f2bf(vals[j]);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TN * TM / 256; ++j) red[tid + 256 * j] = vals[j];
    __syncthreads();
    if (tid < TM) {
      const int m = m0 + tid;
      if (m < M) {
        float best = -INFINITY;
        int bi = -1;
        for (int nl = 0; nl < TN; ++nl) {
          const int n = n0 + nl;
          if (n >= N) break;
          const float v = red[tid * TN + nl];
          if (bi < 0 || v > best) {
            best = v;
            bi = n;
          }
        }
        amax_v[(long)m * n_tiles + tn] = best;
        amax_i[(long)m * n_tiles + tn] = bi;
      }
    }
    return;
  } else if constexpr (EPI == EPI_QKV) {
    // a thread per (row-group pair, token, row of the group): one RoPE pair (q / k) or two v values.  q / k tiles:
    // consecutive threads take consecutive rows (dims) of a token; v tiles (a 32-row tile never straddles the q / k
    // to v boundary): consecutive tokens of a row, so a verify block's positions land side by side in the
    // transposed V block
    const bool vtile = n0 / 16 >= (qa.hq + qa.hkv) * (qa.d >> 4);
    for (int o = tid; o < (NS / 2) * TM * 16; o += 256) {
      int w16, ml, pp;
      if (vtile) {
        ml = o % TM;
        const int r2 = o / TM;
        w16 = r2 & 15;
        pp = r2 >> 4;
      } else {
        w16 = o & 15;
        const int r2 = o >> 4;
        ml = r2 % TM;
        pp = r2 / TM;
      }
      const int m = m0 + ml;
      if (m >= M) continue;
      qkv_rope_store(qa, m, n0 / 16 + 2 * pp, w16, rbf(reduced(2 * pp, ml, w16)), rbf(reduced(2 * pp + 1, ml, w16)));
    }
  } else if (EPI == LSK_EPI_SILU_MUL && NS >= 2 && N % 8 == 0 && (ldc % 8 == 0 || c_nks > 0)) {
    // 8 outputs per lane, one 16-byte store: a wave covers 16 tokens x 32 columns per pass (lane l: token
    // 16 g + l % 16, columns 32 c + 8 (l / 16) .. +7), 8x fewer stores than one element per lane.  c_nks > 0:
    // C is fragment-major (the w2 launch's A operand); the 8 columns are one 16-byte slice of a fragment there.
    constexpr int FC = TN / 32;
    const int wv = tid >> 6;
    for (int f = wv; f < MS * FC; f += 4) {
      const int ml = 16 * (f / FC) + l16, nl0 = 32 * (f % FC) + 8 * lg;
      const int m = m0 + ml, n = n0 + nl0;
      if (m >= M || n >= N) continue;  // N % 8 == 0: the 8 columns are all in range or all out
      uint32_t pk[4];
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        const int a0 = (nl0 + i) >> 4, w0 = (nl0 + i) & 15;
        const float o0 = rbf(silu_f(rbf(reduced(a0, ml, w0)))) * rbf(reduced(a0 + NS, ml, w0));
        const float o1 = rbf(silu_f(rbf(reduced(a0, ml, w0 + 1)))) * rbf(reduced(a0 + NS, ml, w0 + 1));
        pk[i >> 1] = (uint32_t)f2bf(o0) | ((uint32_t)f2bf(o1) << 16);
      }
      *(uint4*)(C + (c_nks > 0 ? lsk_frag_off(m, n, c_nks) : (long)m * ldc + n)) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
  } else {
    for (int o = tid; o < TN * TM; o += 256) {
      const int ml = o / TN, nl = o - ml * TN;
      const int m = m0 + ml, n = n0 + nl;
      if (m >= M || n >= N) continue;
      const float v = reduced(nl >> 4, ml, nl & 15);
      if constexpr (EPI == EPI_PARTIAL) {
        P[((long)s * M + m) * N + n] = v;
      } else {
        float outv;
        if constexpr (EPI == LSK_EPI_SILU_MUL) {
          const float u = reduced((nl >> 4) + NS, ml, nl & 15);
          outv = rbf(silu_f(rbf(v))) * rbf(u);
        } else if constexpr (EPI == LSK_EPI_RESIDUAL) {
          outv = bf2f(R[(long)m * ldr + n]) + rbf(v);
        } else {
          outv = v;
        }
        C[c_nks > 0 ? lsk_frag_off(m, n, c_nks) : (long)m * ldc + n] = f2bf(outv);
      }
    }
  }
}

// ----------------------------------------------------------------------------- wide-M tier
// For many token rows the decode kernel re-reads every weight tile once per 16*MS-token tile.  This kernel
// reads it once per 16*MSW*NWV tokens: the NT x 4 weight fragments of a 128-k chunk are staged in LDS (through
// PF chunks of register prefetch) and NWV waves multiply them with their own MSW token groups.
//
// Exactly the decode kernel's arithmetic: the decode kernel's wave c % 4 accumulates chunks c, c + 4, ... of
// its K slice in order (then, for wave nfull % 4, the tail k-steps) and the four waves are summed in order.
// Here the chunks are visited class by class (class 0: chunks 0, 4, 8, ...; then class 1; ...), each class into
// a fresh accumulator `cur` that is folded into the running sum `tot` (tot = p0, tot + p1, tot + p2, tot + p3),
// so every output sees the same MFMA sequence and the same three adds: results are bitwise those of the
// decode kernel, which keeps the batch invariance of the GEMM.  Covered shapes (launch_wide): N % 64 == 0 and
// K slices of whole 128-k chunks (no tail k-steps).
//
// Token groups: block mb of a launch covers the 16-token groups [mb tbg, min((mb + 1) tbg, ceil(M / 16))), dealt
// to the NWV waves in order, the first (count % NWV) waves one more (waves w and w + 4 share a SIMD, so the extra
// groups land on different SIMDs).  MSW is the most groups a wave holds (tbg <= NWV MSW); a wave multiplies only
// its own groups, so a block's MFMA work follows its real token count.
template <int NS, int MSW, int EPI, int NWV, int PF, bool AF = false>
__global__ __launch_bounds__(64 * NWV, 1) void gemm_wide_kernel(const uint16_t* __restrict__ A, long lda,
                                                                const uint16_t* __restrict__ W,
                                                                uint16_t* __restrict__ C, long ldc,
                                                                const uint16_t* __restrict__ R, long ldr,
                                                                float* __restrict__ P, float* __restrict__ amax_v,
                                                                int* __restrict__ amax_i, int M, int N, int K, int ffn,
                                                                int kslice, int n_tiles, int m_blocks, int n_slices,
                                                                int c_nks, int tbg, QkvRope qa) {
  static_assert(EPI != EPI_QKV || (AF && NS % 2 == 0), "fused qkv: fragment-major A, whole rotation pairs per tile");
  constexpr int NT = (EPI == LSK_EPI_SILU_MUL) ? 2 * NS : NS;
  constexpr int NTH = 64 * NWV;
  constexpr int CHUNK_E = NT * 4 * 512;  // bf16 elements of one staged chunk (NT row groups x 4 k-steps)
  constexpr int LPT = CHUNK_E / (NTH * 8);
  static_assert(LPT >= 1 && CHUNK_E % (NTH * 8) == 0, "staging split");
  __shared__ __attribute__((aligned(16))) uint16_t wl[2][CHUNK_E];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  // id -> (row tile, K slice, token block): the token blocks of one (row tile, slice) take consecutive slots
  // of one XCD, so they run side by side and share each weight chunk through that XCD's L2
  const int xcd = blockIdx.x & 7, qid = blockIdx.x >> 3;
  const int mb = qid % m_blocks, rest = qid / m_blocks;
  const int s = rest % n_slices, tg = rest / n_slices;
  const int tn = tg * 8 + xcd;
  if (tn >= n_tiles) return;
  const int n0 = tn * 16 * NS;
  const int k0 = s * kslice, k1 = min(K, k0 + kslice);
  const int nks = K >> 5;
  const int nfull = (k1 - k0) / 128;
  auto group_of = [&](int g) { return (g < NS) ? (n0 / 16 + g) : ((ffn + n0) / 16 + (g - NS)); };
  // staging: piece p = tid + NTH j -> row group p / 256, k-step (p / 64) % 4, lane p % 64 of the chunk
  const uint16_t* wsrc[LPT];
  int wdst[LPT];
#pragma unroll
  for (int j = 0; j < LPT; ++j) {
    const int pc = tid + NTH * j;
    const int g = pc >> 8, ks = (pc >> 6) & 3, l = pc & 63;
    wsrc[j] = W + ((long)group_of(g) * nks + (k0 >> 5) + ks) * 512 + 8 * l;
    wdst[j] = (g * 4 + ks) * 512 + 8 * l;
  }
  // this wave's token groups [g0, g0 + ng) (ng <= MSW); group slots t >= ng load a valid group and store nothing
  const int gtot = (M + 15) / 16, gb0 = mb * tbg;
  const int gb = min(tbg, gtot - gb0);
  const int ng = __builtin_amdgcn_readfirstlane(gb / NWV + (wave < gb % NWV ? 1 : 0));
  const int g0 = gb0 + wave * (gb / NWV) + min(wave, gb % NWV);
  const uint16_t* arow[MSW];
  int mrow[MSW];
#pragma unroll
  for (int t = 0; t < MSW; ++t) {
    const int grp = min(g0 + min(t, max(ng - 1, 0)), gtot - 1);
    mrow[t] = t < ng ? (g0 + t) * 16 + l16 : INT_MAX;
    if constexpr (AF) {
      // fragment-major A holds whole 16-token groups up to (M + 15) / 16
      arow[t] = A + ((long)grp * nks + (k0 >> 5)) * 512 + 8 * lane;
    } else {
      const int m = grp * 16 + l16;
      arow[t] = A + (long)(m < M - 1 ? m : M - 1) * lda + k0 + 8 * lg;
    }
  }
  lsk_f32x4 cur[NT][MSW], tot[NT][MSW];
#pragma unroll
  for (int a = 0; a < NT; ++a)
#pragma unroll
    for (int t = 0; t < MSW; ++t) cur[a][t] = tot[a][t] = (lsk_f32x4){0.f, 0.f, 0.f, 0.f};
  // visiting order: chunk class q = 0..3 holds chunks q, q + 4, ...; n_q of them; sequence index i -> chunk
  int cum[5];
  cum[0] = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) cum[q + 1] = cum[q] + (nfull > q ? (nfull - q + 3) / 4 : 0);
  auto chunk_at = [&](int i) {
    const int q = (i >= cum[1]) + (i >= cum[2]) + (i >= cum[3]);
    return q + 4 * (i - cum[q]);
  };
  lsk_i32x4 stg[PF][LPT];
  auto issue = [&](lsk_i32x4 (&r)[LPT], int c) {
#pragma unroll
    for (int j = 0; j < LPT; ++j) r[j] = __builtin_nontemporal_load((const lsk_i32x4*)(wsrc[j] + (long)c * 4 * 512));
  };
  auto put = [&](lsk_i32x4 (&r)[LPT], int b) {
#pragma unroll
    for (int j = 0; j < LPT; ++j) *(lsk_i32x4*)(&wl[b][wdst[j]]) = r[j];
  };
  lsk_bf16x8 af[2][4][MSW];
  // na_c: std::integral_constant holding this wave's group count (the loops below are unrolled per count)
  auto load_a = [&](lsk_bf16x8 (&a)[4][MSW], int c, auto na_c) {
    constexpr int NA = decltype(na_c)::value;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int t = 0; t < NA; ++t)
        a[ks][t] = *(const lsk_bf16x8*)(arow[t] + (AF ? (long)(c * 4 + ks) * 512 : (long)(c * 128 + ks * 32)));
  };
  auto comp = [&](const lsk_bf16x8 (&a)[4][MSW], int b, auto na_c) {
    constexpr int NA = decltype(na_c)::value;
    if constexpr (NA > 0) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        lsk_bf16x8 wf[NT];
#pragma unroll
        for (int g = 0; g < NT; ++g) wf[g] = *(const lsk_bf16x8*)(&wl[b][(g * 4 + ks) * 512 + 8 * lane]);
#pragma unroll
        for (int g = 0; g < NT; ++g)
#pragma unroll
          for (int t = 0; t < NA; ++t)
            cur[g][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[g], a[ks][t], cur[g][t], 0, 0, 0);
      }
    }
  };
  int cls = 0;
  auto fold = [&]() {  // close class cls, start the next one
#pragma unroll
    for (int g = 0; g < NT; ++g)
#pragma unroll
      for (int t = 0; t < MSW; ++t) {
        if (cls == 0) {
          tot[g][t] = cur[g][t];
        } else {
          tot[g][t][0] = tot[g][t][0] + cur[g][t][0];
          tot[g][t][1] = tot[g][t][1] + cur[g][t][1];
          tot[g][t][2] = tot[g][t][2] + cur[g][t][2];
          tot[g][t][3] = tot[g][t][3] + cur[g][t][3];
        }
        cur[g][t] = (lsk_f32x4){0.f, 0.f, 0.f, 0.f};
      }
    ++cls;
  };
  // Every wave stages weights and meets every barrier; the group count only selects how many token groups it
  // loads and multiplies (a wave-uniform branch around whole copies of the loop, same barriers in each).
  auto run = [&](auto na_c) {
    // prologue: chunks 0 .. PF-1 of the sequence in flight, chunk 0 in LDS buffer 0
#pragma unroll
    for (int j = 0; j < PF; ++j)
      if (j < nfull) issue(stg[j], chunk_at(j));
    if (nfull > 0) {
      load_a(af[0], chunk_at(0), na_c);
      put(stg[0], 0);
    }
    __syncthreads();
    // sequence index i (i0 a multiple of 2 PF, so i % 2 == u % 2 and i % PF == u % PF): fold the classes that
    // ended before i, multiply chunk i from LDS buffer i % 2, refill register slot i % PF with chunk i + PF, move
    // chunk i + 1 from its register slot into the other LDS buffer.  The prefetches past the last chunk reload the
    // last one (in bounds, never used): every iteration issues the same loads, so the compiler's wait counts stay
    // exact (a conditional prefetch made it wait for the next chunk's loads before this chunk's MFMAs; measured
    // 6-28 % slower).  The 64 + 64-row silu-mul tile at 2 groups per wave keeps the conditional form: it is at the
    // register limit, and the earlier loads of the unconditional form spill.
    constexpr bool exact = !(NT * MSW >= 16);
    for (int i0 = 0; i0 < nfull; i0 += 2 * PF) {
#pragma unroll
      for (int u = 0; u < 2 * PF; ++u) {
        const int i = i0 + u;
        if (i < nfull) {
          while (cls < 3 && i >= cum[cls + 1]) fold();
          if (exact || i + 1 < nfull) load_a(af[(u + 1) & 1], chunk_at(min(i + 1, nfull - 1)), na_c);
          comp(af[u & 1], u & 1, na_c);
          if (exact || i + PF < nfull) issue(stg[u % PF], chunk_at(min(i + PF, nfull - 1)));
          if (exact || i + 1 < nfull) put(stg[(u + 1) % PF], (u + 1) & 1);
          __syncthreads();
        }
      }
    }
  };
  static_assert(MSW >= 1 && MSW <= 3, "group counts per wave");
  if (ng == MSW) run(std::integral_constant<int, MSW>{});
  else if (ng == MSW - 1) run(std::integral_constant<int, (MSW > 1 ? MSW - 1 : 0)>{});
  else if (MSW == 3 && ng == 1) run(std::integral_constant<int, 1>{});
  else run(std::integral_constant<int, 0>{});
  while (cls < 4) fold();
  // epilogue: lane holds rows 16 g + 4 lg + i of its token group t, token l16
  if constexpr (EPI == EPI_ARGMAX) {
    // per token, the largest bf16-rounded logit of the tile's 64 rows and its first index: each lane scans its 16
    // rows in increasing order, then the four lanes of the token (lg = 0..3) combine, larger value first and the
    // smaller index on ties -- the decode kernel's in-order scan over the same rounded values
#pragma unroll
    for (int t = 0; t < MSW; ++t) {
      const int m = mrow[t];
      float best = -INFINITY;
      int bi = -1;
#pragma unroll
      for (int g = 0; g < NS; ++g) {
        const int n = n0 + 16 * g + 4 * lg;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = rbf(tot[g][t][i]);
        if (n < N) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (bi < 0 || v[i] > best) {
              best = v[i];
              bi = n + i;
            }
          if (C != nullptr && m < M) {
            uint2 pk;
            pk.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
            pk.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
            *(uint2*)(C + (long)m * ldc + n) = pk;
          }
        }
      }
#pragma unroll
      for (int o = 16; o <= 32; o <<= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (oi >= 0 && (bi < 0 || ov > best || (ov == best && oi < bi))) {
          best = ov;
          bi = oi;
        }
      }
      if (lg == 0 && m < M) {
        amax_v[(long)m * n_tiles + tn] = best;
        amax_i[(long)m * n_tiles + tn] = bi;
      }
    }
    return;
  }
  if constexpr (EPI == EPI_QKV) {
    // lane: rows 4 lg + i of row groups 2 pp (low half of each RoPE pair) and 2 pp + 1 (high half), token mrow[t]
#pragma unroll
    for (int t = 0; t < MSW; ++t) {
      const int m = mrow[t];
      if (m >= M) continue;
#pragma unroll
      for (int pp = 0; pp < NS / 2; ++pp)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          qkv_rope_store(qa, m, n0 / 16 + 2 * pp, 4 * lg + i, rbf(tot[2 * pp][t][i]), rbf(tot[2 * pp + 1][t][i]));
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < MSW; ++t) {
    const int m = mrow[t];
    if (m >= M) continue;
#pragma unroll
    for (int g = 0; g < NS; ++g) {
      const int n = n0 + 16 * g + 4 * lg;
      if (n >= N) continue;
      if constexpr (EPI == EPI_PARTIAL) {
        *(float4*)(P + ((long)s * M + m) * N + n) = make_float4(tot[g][t][0], tot[g][t][1], tot[g][t][2], tot[g][t][3]);
      } else {
        uint16_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = tot[g][t][i];
          float outv;
          if constexpr (EPI == LSK_EPI_SILU_MUL) {
            outv = rbf(silu_f(rbf(v))) * rbf(tot[g + NS][t][i]);
          } else if constexpr (EPI == LSK_EPI_RESIDUAL) {
            outv = bf2f(R[(long)m * ldr + n + i]) + rbf(v);
          } else {
            outv = v;
          }
          o[i] = f2bf(outv);
        }
        uint2 pk;
        pk.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
        pk.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
        // c_nks > 0: fragment-major C; columns n .. n + 3 (n % 4 == 0) stay within one 8-column slice
        *(uint2*)(C + (c_nks > 0 ? lsk_frag_off(m, n, c_nks) : (long)m * ldc + n)) = pk;
      }
    }
  }
}

// Final greedy pick over the per-tile maxima: larger value wins, ties keep the smaller index
// (torch.argmax semantics over the bf16 logits).  out[dst ? dst[m] : m] = index.
__global__ __launch_bounds__(256) void argmax_tiles_kernel(const float* __restrict__ v, const int* __restrict__ idx,
                                                           int ntiles, int64_t* __restrict__ out,
                                                           const int64_t* __restrict__ dst) {
  const int m = blockIdx.x;
  float best = -INFINITY;
  int bi = -1;
  for (int j = threadIdx.x; j < ntiles; j += 256) {
    const float x = v[(long)m * ntiles + j];
    const int xi = idx[(long)m * ntiles + j];
    if (bi < 0 || x > best || (x == best && xi < bi)) {
      best = x;
      bi = xi;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (bi < 0 || (oi >= 0 && (ov > best || (ov == best && oi < bi)))) {
      best = ov;
      bi = oi;
    }
  }
  __shared__ float sv[4];
  __shared__ int si[4];
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = best;
    si[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sv[0];
    int i = si[0];
    for (int w = 1; w < 4; ++w)
      if (i < 0 || (si[w] >= 0 && (sv[w] > b || (sv[w] == b && si[w] < i)))) {
        b = sv[w];
        i = si[w];
      }
    out[dst ? dst[m] : m] = (int64_t)i;
  }
}

// fp32 path (parity runs): one wave per output row of W, 16 token rows per workgroup row-block.
// Lane l sums k = l, l + 64, ... in order, then a fixed xor tree over the 64 lanes.
template <int EPI>
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ A, long lda,
                                                       const float* __restrict__ W, long ldw, float* __restrict__ C,
                                                       long ldc, const float* __restrict__ R, long ldr, int M, int N,
                                                       int K, int ffn) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + wave;
  if (n >= N) return;
  const int m0 = blockIdx.y * 16;
  const int mc = min(16, M - m0);
  float acc[16], accu[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = accu[r] = 0.f;
  const float* wg = W + (long)n * ldw;
  const float* wu = W + (long)(ffn + n) * ldw;
  for (int k = lane; k < K; k += 64) {
    const float wv = wg[k];
    const float uv = (EPI == LSK_EPI_SILU_MUL) ? wu[k] : 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if (r < mc) {
        const float a = A[(long)(m0 + r) * lda + k];
        acc[r] += a * wv;
        if (EPI == LSK_EPI_SILU_MUL) accu[r] += a * uv;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      acc[r] += __shfl_xor(acc[r], o, 64);
      if (EPI == LSK_EPI_SILU_MUL) accu[r] += __shfl_xor(accu[r], o, 64);
    }
  }
  if (lane < mc) {
    float v = 0.f, u = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (r == lane) {
        v = acc[r];
        u = accu[r];
      }
    const int m = m0 + lane;
    float outv;
    if (EPI == LSK_EPI_SILU_MUL) outv = silu_f(v) * u;
    else if (EPI == LSK_EPI_RESIDUAL) outv = R[(long)m * ldr + n] + v;
    else outv = v;
    C[(long)m * ldc + n] = outv;
  }
}

// ----------------------------------------------------------------------------- weight packing
// One thread per 16-byte lane slice: packed element offset 8 * o, o = (g * nks + j) * 64 + l  <->  row
// 16 g + l % 16, columns 32 j + 8 (l / 16) .. +7 of the row-major matrix.  Both directions are pure copies.
// gh > 0 (a fused qkv weight, lsk_pack_weight_qkv): within each of the first paired_groups row groups' heads of gh
// groups, packed group 2 r holds source group r and packed group 2 r + 1 source group gh / 2 + r (RoPE partners).
template <bool PACK>
__global__ __launch_bounds__(256) void pack_weight_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                          long ld, int nks, long n_slices, int gh, int paired_groups) {
  const long o = (long)blockIdx.x * 256 + threadIdx.x;
  if (o >= n_slices) return;
  const int l = (int)(o & 63);
  const long f = o >> 6;
  const long g = f / nks, j = f - g * nks;
  long sg = g;  // source row group
  if (gh > 0 && g < paired_groups) {
    const long h = g / gh, r = g - h * gh;
    sg = h * gh + ((r & 1) ? gh / 2 + (r >> 1) : (r >> 1));
  }
  const long rm = (16 * sg + (l & 15)) * ld + 32 * j + 8 * (l >> 4);  // row-major element offset
  if (PACK)
    *(uint4*)(dst + 8 * o) = *(const uint4*)(src + rm);
  else
    *(uint4*)(dst + rm) = *(const uint4*)(src + 8 * o);
}

// ----------------------------------------------------------------------------- host side

// K-split plan of a weight shape (N rows x K); it fixes the reduction order of every output.  KS = 1
// when the matrix has >= 256 row tiles of 64; otherwise KS = the smallest power of two giving >= 512
// (32-row tile, slice) pairs, K / KS a multiple of 128.  ns_out is the row-tile width (in 16-row groups)
// of that rule.  Depends on (N, K) only, never on M; a launch's own tile width (tile_ns) may follow M.
extern "C" int lsk_gemm_plan(int N, int K, int* ns_out, int* ks_out) {
  LSK_REQUIRE(ns_out && ks_out && N > 0 && K > 0, LSK_EARG, "lsk_gemm_plan: bad arguments");
  int ns, ks = 1;
  if (N % 64 == 0 && N / 64 >= 256) {
    ns = 4;
  } else if (N % 32 == 0) {
    ns = 2;
    while (N / 32 * ks < 512 && K % (2 * ks) == 0 && (K / (2 * ks)) % 128 == 0) ks *= 2;
  } else {
    ns = 1;
  }
  *ns_out = ns;
  *ks_out = ks;
  return 0;
}

// Token tile (16 * MS tokens) of the decode kernel: the smallest of 16 / 32 / 48 / 64 that holds M.  Measured on
// MI355X at the 8B shapes (graph replay, distinct weights per launch): at 33-48 tokens the 48-token tile is
// 2-5 % faster than a half-empty 64-token tile for w13, w2, qkv and o; splitting the tokens over several
// token tiles (each re-reading the weights, mostly from L2) is 10-70 % slower.
static int ms_for(int M) { return M <= 16 ? 1 : (M <= 32 ? 2 : (M <= 48 ? 3 : 4)); }

// Tile width of a launch (16 * NS weight rows per workgroup; n = output columns, ffn for silu-mul).
// Every row tile reads the whole M x K-slice activation block, so wide tiles cut those re-reads;
// measured on MI355X at the 8B shapes, 64-row tiles win for w2, w13 (4 + 4 row groups, gate and up) and
// the head at every M, and for qkv / o from 33 tokens on.  A split-K launch with short slices (<= 1024 k)
// and fewer than two 64-row workgroups per CU is latency-bound per workgroup: up to 32 tokens, 32-row
// tiles (twice the workgroups) measured faster for qkv (13.2 vs 14.7 us at 32 tokens); with fragment-major
// activations (cheaper activation loads per workgroup) up to 48 tokens (qkv -0.35 us, o -0.24 us per launch).  The reduction
// order of an output does not depend on NS or MS (only on K and the plan's KS), so the tile follows M
// without breaking batch invariance.
// Without a K split (silu-mul, plain and residual epilogues), a shape whose 64-row tiles would leave more than a
// third of the CUs idle (fewer than 160 workgroups: the 1B MLP's 128) runs 32-row tiles instead.  Measured on
// MI355X (back-to-back launches, cold weights): 1B w13 -12 % at 8 tokens to -26 % at 64; the 7B MLP (172
// workgroups) ran 9-13 % slower with 32-row tiles, so it keeps 64.
static int tile_ns(int n, int M, int epi, int kslice = 0, int ks = 1, int short_max = 32) {
  int ns = 4;
  while (ns > 1 && n % (16 * ns) != 0) ns >>= 1;
  if (ns == 4 && epi == EPI_PARTIAL && M <= short_max && kslice <= 1024 && (long)(n / 64) * ks < 512) ns = 2;
  if (ns == 4 && epi != EPI_PARTIAL && epi != EPI_ARGMAX && n / 64 < 160 && n % 32 == 0) ns = 2;
  return ns;
}

template <int NS, int MS>
static void launch_bf16(int epi, dim3 grid, hipStream_t s, const uint16_t* A, long lda, const uint16_t* W, long ldw,
                        uint16_t* C, long ldc, const uint16_t* R, long ldr, float* P, float* av, int* ai, int M,
                        int N, int K, int ffn, int kslice, int nt, int mt, int m_lo) {
  if (epi == LSK_EPI_RESIDUAL)
    gemm_bf16_kernel<NS, MS, LSK_EPI_RESIDUAL><<<grid, 256, 0, s>>>(A, lda, W, ldw, C, ldc, R, ldr, P, av, ai, M, N, K,
                                                                    ffn, kslice, nt, mt, m_lo, 0, QkvRope{});
  else if (epi == LSK_EPI_SILU_MUL) {
    gemm_bf16_kernel<NS, MS, LSK_EPI_SILU_MUL><<<grid, 256, 0, s>>>(A, lda, W, ldw, C, ldc, R, ldr, P, av, ai, M, N,
                                                                      K, ffn, kslice, nt, mt, m_lo, 0, QkvRope{});
  } else if (epi == EPI_PARTIAL)
    gemm_bf16_kernel<NS, MS, EPI_PARTIAL><<<grid, 256, 0, s>>>(A, lda, W, ldw, C, ldc, R, ldr, P, av, ai, M, N, K, ffn,
                                                               kslice, nt, mt, m_lo, 0, QkvRope{});
  else if (epi == EPI_ARGMAX)
    gemm_bf16_kernel<NS, MS, EPI_ARGMAX><<<grid, 256, 0, s>>>(A, lda, W, ldw, C, ldc, R, ldr, P, av, ai, M, N, K, ffn,
                                                              kslice, nt, mt, m_lo, 0, QkvRope{});
  else
    gemm_bf16_kernel<NS, MS, LSK_EPI_NONE><<<grid, 256, 0, s>>>(A, lda, W, ldw, C, ldc, R, ldr, P, av, ai, M, N, K,
                                                                ffn, kslice, nt, mt, m_lo, 0, QkvRope{});
}

// Fragment-major A: split-K partials, silu-mul (C row-major, or fragment-major with c_nks > 0), the LM head and
// the fused qkv + RoPE + KV append.
template <int NS, int MS>
static void launch_bf16_af(int epi, dim3 grid, hipStream_t s, const uint16_t* A, const uint16_t* W, long ldw,
                           uint16_t* C, long ldc, int c_nks, float* P, float* av, int* ai, int M, int N, int K, int ffn,
                           int kslice, int nt, int mt, int m_lo, const QkvRope& qa) {
  if (epi == LSK_EPI_SILU_MUL)
    gemm_bf16_kernel<NS, MS, LSK_EPI_SILU_MUL, gemm_unit<NS, MS, LSK_EPI_SILU_MUL>(), true><<<grid, 256, 0, s>>>(
        A, 0, W, ldw, C, ldc, nullptr, 0, nullptr, nullptr, nullptr, M, N, K, ffn, kslice, nt, mt, m_lo, c_nks,
        QkvRope{});
  else if (epi == EPI_ARGMAX)
    gemm_bf16_kernel<NS, MS, EPI_ARGMAX, gemm_unit<NS, MS, EPI_ARGMAX>(), true><<<grid, 256, 0, s>>>(
        A, 0, W, ldw, C, ldc, nullptr, 0, nullptr, av, ai, M, N, K, 0, kslice, nt, mt, m_lo, 0, QkvRope{});
  else if (epi == EPI_QKV) {
    if constexpr (NS % 2 == 0)
      gemm_bf16_kernel<NS, MS, EPI_QKV, gemm_unit<NS, MS, EPI_QKV>(), true><<<grid, 256, 0, s>>>(
          A, 0, W, ldw, nullptr, 0, nullptr, 0, nullptr, nullptr, nullptr, M, N, K, 0, kslice, nt, mt, m_lo, 0, qa);
  } else
    gemm_bf16_kernel<NS, MS, EPI_PARTIAL, gemm_unit<NS, MS, EPI_PARTIAL>(), true><<<grid, 256, 0, s>>>(
        A, 0, W, ldw, nullptr, 0, nullptr, 0, P, nullptr, nullptr, M, N, K, 0, kslice, nt, mt, m_lo, 0, QkvRope{});
}

// Launch over nt row tiles x mt token tiles x ks K slices (the tile mapping is in the kernel).  af: a split-K
// partial launch with a fragment-major A.
static void dispatch_bf16(int ns, int ms, int epi, int nt, int mt, int ks, hipStream_t s, const void* A, long lda,
                          const void* W, long ldw, void* C, long ldc, const void* R, long ldr, float* P, float* av,
                          int* ai, int M, int N, int K, int ffn, int kslice, bool af = false, int m_lo = 0,
                          int c_nks = 0, const QkvRope& qa = QkvRope{}) {
  const dim3 grid(mt > 1 ? (unsigned)(((nt + 7) / 8) * 8 * mt) : (unsigned)nt, 1, (unsigned)ks);
  const uint16_t* a = (const uint16_t*)A;
  const uint16_t* w = (const uint16_t*)W;
  uint16_t* c = (uint16_t*)C;
  const uint16_t* r = (const uint16_t*)R;
#define LSK_GEMM_CASE(NS_, MS_)                                                                                  \
  if (ns == NS_ && ms == MS_) {                                                                                  \
    if (af)                                                                                                      \
      launch_bf16_af<NS_, MS_>(epi, grid, s, a, w, ldw, c, ldc, c_nks, P, av, ai, M, N, K, ffn, kslice, nt, mt, m_lo, qa); \
    else                                                                                                         \
      launch_bf16<NS_, MS_>(epi, grid, s, a, lda, w, ldw, c, ldc, r, ldr, P, av, ai, M, N, K, ffn, kslice, nt, mt, \
                            m_lo);                                                                               \
  }
  LSK_GEMM_CASE(1, 1) LSK_GEMM_CASE(1, 2) LSK_GEMM_CASE(1, 3) LSK_GEMM_CASE(1, 4)
  LSK_GEMM_CASE(2, 1) LSK_GEMM_CASE(2, 2) LSK_GEMM_CASE(2, 3) LSK_GEMM_CASE(2, 4)
  LSK_GEMM_CASE(4, 1) LSK_GEMM_CASE(4, 2) LSK_GEMM_CASE(4, 3) LSK_GEMM_CASE(4, 4)
#undef LSK_GEMM_CASE
}

// Wide-M tier selection.  Above 64 tokens every row goes through the wide tier in one launch.  A configuration
// is a tile width (64 rows; silu-mul also 32 + 32) and a block count nb: the token groups are dealt evenly to nb
// blocks of tbg groups, and within a block to the 8 waves, so a wave holds at most msw = ceil(tbg / 8) groups
// (register budget: 3, or 2 for the 64 + 64-row silu-mul tile, whose gate and up accumulators take twice the
// registers).  Each weight tile is streamed from HBM once per launch; the blocks of a tile run side by side on
// one XCD and re-read it from that XCD's L2.
//
// The configuration minimises a cost fitted to MI355X measurements at the 8B layer shapes (M = 66..512, qkv /
// o / w2 / w13 / LM head): workgroup rounds ceil(WGs / 256) x max(2.5, 0.83 + g) x rows / 64, where g is the most
// token groups the two waves of one SIMD hold (MFMA work) and 2.5 the floor a workgroup's weight stream sets;
// x 0.9 when a msw = 1 kernel fits two workgroups per CU (more memory parallelism), x 1.1 for the 32 + 32-row
// silu-mul tile (twice the activation reads), x 1.5 for the 32-row fused qkv tile (its rope epilogue and the
// doubled activation reads; refitted over the 1B, 8B and 7B shapes at 96-512 tokens).  The launch needs >= 192
// workgroups to stream the weights.  Returns the rows the tier took: M, or 0 where it does not apply (M <= 64,
// N % 64 != 0, K slices that are not whole 128-k chunks, or too few weight tiles to spread).  Both tiers give bitwise the same sums, so neither
// the tier nor the configuration ever changes a result.
struct WideCfg {
  int ns, m_blocks, tbg, msw;
};

static WideCfg wide_config(int epi, int M, int N, int ks) {
  const bool silu = epi == LSK_EPI_SILU_MUL;
  const int gtot = (M + 15) / 16;
  WideCfg best{0, 0, 0, 0};
  double best_cost = 0.0;
  for (int ns = 4; ns >= 2; ns -= 2) {
    if (ns == 2 && !silu && epi != EPI_QKV) break;
    const int msw_max = (silu && ns == 4) ? 2 : 3;
    const int nb_min = (gtot + 8 * msw_max - 1) / (8 * msw_max);
    for (int nb = nb_min; nb <= nb_min + 2; ++nb) {
      const int tbg = (gtot + nb - 1) / nb, m_blocks = (gtot + tbg - 1) / tbg, msw = (tbg + 7) / 8;
      const int q = tbg / 8, r = tbg % 8;
      const int g = 2 * q + (r > 0) + (r > 4);
      const long wgs = (long)(N / (16 * ns)) * m_blocks * ks;
      // >= 192 workgroups; the 64 + 64-row silu-mul tile only at msw = 2 (at msw = 1 the 32 + 32 tile, two
      // workgroups per CU, always costs less)
      if (wgs < 192 || (silu && ns == 4 && msw == 1)) continue;
      const bool two_per_cu = msw == 1 && wgs > 256;
      double cost = (double)((wgs + 255) / 256) * fmax(2.5, 0.83 + g) * ns / 4.0;
      if (two_per_cu) cost *= 0.9;
      if (ns == 2) cost *= epi == EPI_QKV ? 1.5 : 1.1;
      if (best.ns == 0 || cost < best_cost) {
        best = WideCfg{ns, m_blocks, tbg, msw};
        best_cost = cost;
      }
    }
  }
  return best;
}

template <int NS, int MSW, int EPI>
static void launch_wide_kernel(dim3 grid, hipStream_t s, bool af, const uint16_t* A, long lda, const uint16_t* W,
                               uint16_t* C, long ldc, const uint16_t* R, long ldr, float* P, float* av, int* ai, int M,
                               int N, int K, int ffn, int kslice, int n_tiles, int m_blocks, int ks, int c_nks,
                               int tbg, const QkvRope& qa) {
  if constexpr (EPI == EPI_PARTIAL || EPI == EPI_ARGMAX || EPI == LSK_EPI_SILU_MUL || EPI == EPI_QKV) {
    if (af) {
      gemm_wide_kernel<NS, MSW, EPI, 8, 2, true><<<grid, 512, 0, s>>>(A, lda, W, C, ldc, R, ldr, P, av, ai, M, N, K, ffn,
                                                                      kslice, n_tiles, m_blocks, ks, c_nks, tbg, qa);
      return;
    }
  }
  if constexpr (EPI != EPI_QKV)
    gemm_wide_kernel<NS, MSW, EPI, 8, 2><<<grid, 512, 0, s>>>(A, lda, W, C, ldc, R, ldr, P, av, ai, M, N, K, ffn,
                                                              kslice, n_tiles, m_blocks, ks, 0, tbg, QkvRope{});
}

// Whether the wide tier takes a launch (ns == 0: no) and its configuration.  c_ok: the output's row stride
// allows the tier's 4-element stores.
static WideCfg wide_plan(int epi, int M, int N, int K, int ks, bool af, bool c_ok) {
  const WideCfg none{0, 0, 0, 0};
  if (M <= 64 || ks <= 0) return none;
  if (N % 64 != 0 || !c_ok || K % ks != 0 || (K / ks) % 128 != 0) return none;
  if (af && (epi == LSK_EPI_RESIDUAL || epi == LSK_EPI_NONE)) return none;
  if (epi == EPI_QKV && !af) return none;
  // too few weight tiles to spread: the narrowest tile (32 rows for the fused qkv and the silu-mul, 64 otherwise)
  // x blocks of up to 24 row groups x K slices under 128 leaves the decode tier faster (measured over the 1B, 8B
  // and 7B projections at 96-512 tokens)
  const int gtot = (M + 15) / 16;
  const int narrow = (epi == EPI_QKV || epi == LSK_EPI_SILU_MUL) ? 32 : 64;
  if ((long)(N / narrow) * ((gtot + 23) / 24) * ks < 128) return none;
  return wide_config(epi, M, N, ks);
}

extern "C" int lsk_gemm_wide_config(int epilogue, int M, int N, int K, int ks, int af, int* cfg) {
  LSK_REQUIRE(cfg != nullptr, LSK_EARG, "lsk_gemm_wide_config: null pointer");
  LSK_REQUIRE(epilogue >= LSK_EPI_NONE && epilogue <= EPI_QKV, LSK_EARG, "lsk_gemm_wide_config: epilogue %d",
              epilogue);
  const WideCfg c = wide_plan(epilogue, M, N, K, ks, af != 0, true);
  cfg[0] = c.ns;
  cfg[1] = c.m_blocks;
  cfg[2] = c.tbg;
  cfg[3] = c.msw;
  return 0;
}

static int launch_wide(int epi, hipStream_t s, const uint16_t* A, long lda, const uint16_t* W, uint16_t* C, long ldc,
                       const uint16_t* R, long ldr, float* P, float* av, int* ai, int M, int N, int K, int ffn, int ks,
                       bool af = false, int c_nks = 0, const QkvRope& qa = QkvRope{}) {
  const WideCfg cfg = wide_plan(epi, M, N, K, ks, af, epi == EPI_PARTIAL || C == nullptr || ldc % 4 == 0);
  if (cfg.ns == 0) return 0;
  const int n_tiles = N / (16 * cfg.ns);
  const dim3 grid((unsigned)(((n_tiles + 7) / 8) * 8 * cfg.m_blocks * ks));
  const int kslice = K / ks;
#define LSK_WIDE(NS_, MSW_, EPI_)                                                                                  \
  launch_wide_kernel<NS_, MSW_, EPI_>(grid, s, af, A, lda, W, C, ldc, R, ldr, P, av, ai, M, N, K, ffn, kslice, n_tiles, \
                                      cfg.m_blocks, ks, c_nks, cfg.tbg, qa)
#define LSK_WIDE_MSW(NS_, EPI_)                 \
  do {                                          \
    if (cfg.msw == 1)                           \
      LSK_WIDE(NS_, 1, EPI_);                   \
    else if (cfg.msw == 2)                      \
      LSK_WIDE(NS_, 2, EPI_);                   \
    else                                        \
      LSK_WIDE(NS_, 3, EPI_);                   \
  } while (0)
  if (epi == LSK_EPI_SILU_MUL) {
    if (cfg.ns == 2) LSK_WIDE_MSW(2, LSK_EPI_SILU_MUL);
    else LSK_WIDE(4, 2, LSK_EPI_SILU_MUL);
  } else if (epi == EPI_PARTIAL) {
    LSK_WIDE_MSW(4, EPI_PARTIAL);
  } else if (epi == LSK_EPI_RESIDUAL) {
    LSK_WIDE_MSW(4, LSK_EPI_RESIDUAL);
  } else if (epi == LSK_EPI_NONE) {
    LSK_WIDE_MSW(4, LSK_EPI_NONE);
  } else if (epi == EPI_ARGMAX) {
    LSK_WIDE_MSW(4, EPI_ARGMAX);
  } else if (epi == EPI_QKV) {
    if (cfg.ns == 2) LSK_WIDE_MSW(2, EPI_QKV);
    else LSK_WIDE_MSW(4, EPI_QKV);
  } else {
    return 0;
  }
#undef LSK_WIDE_MSW
#undef LSK_WIDE
  return M;
}

extern "C" int lsk_gemm(int dtype, const void* A, long lda, const void* W, long ldw, void* C, long ldc,
                        const void* R, long ldr, int M, int N, int K, int epilogue, int ffn, void* stream) {
  LSK_REQUIRE(A && W && C, LSK_EARG, "lsk_gemm: null pointer");
  LSK_REQUIRE(M >= 0 && N > 0 && K > 0 && lda >= K && ldw >= K && ldc >= N, LSK_ESHAPE,
              "lsk_gemm: bad shape M=%d N=%d K=%d lda=%ld ldw=%ld ldc=%ld", M, N, K, lda, ldw, ldc);
  LSK_REQUIRE(epilogue >= LSK_EPI_NONE && epilogue <= LSK_EPI_SILU_MUL, LSK_EARG, "lsk_gemm: epilogue %d", epilogue);
  LSK_REQUIRE(epilogue != LSK_EPI_RESIDUAL || (R != nullptr && ldr >= N), LSK_EARG, "lsk_gemm: residual missing");
  LSK_REQUIRE(epilogue != LSK_EPI_SILU_MUL || ffn == N, LSK_EARG, "lsk_gemm: silu-mul needs ffn == N (got %d, %d)",
              ffn, N);
  if (M == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == LSK_DTYPE_BF16) {
    LSK_REQUIRE(K % 32 == 0 && lda % 8 == 0 && ldw == K, LSK_ESHAPE,
                "lsk_gemm: bf16 needs K %% 32 == 0, 16-byte aligned A rows and a packed W (ldw == K; K=%d ldw=%ld)", K,
                ldw);
    LSK_REQUIRE(N % 16 == 0, LSK_ESHAPE, "lsk_gemm: bf16 needs N %% 16 == 0 (N=%d)", N);
    const int mw = launch_wide(epilogue, s, (const uint16_t*)A, lda, (const uint16_t*)W, (uint16_t*)C, ldc,
                               (const uint16_t*)R, ldr, nullptr, nullptr, nullptr, M, N, K, ffn, 1);
    if (mw > 0) {
      const int rc = lsk_check_launch("lsk_gemm(bf16, wide)");
      if (rc || mw == M) return rc;
    }
    // whole-K workgroups over rows [mw, M)
    const int mr = M - mw;
    const int ns = tile_ns(N, mr, epilogue);
    const int ms = ms_for(mr);
    dispatch_bf16(ns, ms, epilogue, N / (16 * ns), (mr + 16 * ms - 1) / (16 * ms), 1, s, A, lda, W, ldw, C, ldc, R, ldr,
                  nullptr, nullptr, nullptr, M, N, K, ffn, K, false, mw);
    return lsk_check_launch("lsk_gemm(bf16)");
  }
  if (dtype == LSK_DTYPE_F32) {
    dim3 grid((N + 3) / 4, (M + 15) / 16);
    const float* a = (const float*)A;
    const float* w = (const float*)W;
    float* c = (float*)C;
    const float* r = (const float*)R;
    if (epilogue == LSK_EPI_RESIDUAL)
      gemm_f32_kernel<LSK_EPI_RESIDUAL><<<grid, 256, 0, s>>>(a, lda, w, ldw, c, ldc, r, ldr, M, N, K, ffn);
    else if (epilogue == LSK_EPI_SILU_MUL)
      gemm_f32_kernel<LSK_EPI_SILU_MUL><<<grid, 256, 0, s>>>(a, lda, w, ldw, c, ldc, r, ldr, M, N, K, ffn);
    else
      gemm_f32_kernel<LSK_EPI_NONE><<<grid, 256, 0, s>>>(a, lda, w, ldw, c, ldc, r, ldr, M, N, K, ffn);
    return lsk_check_launch("lsk_gemm(f32)");
  }
  LSK_REQUIRE(false, LSK_EUNSUPPORTED, "lsk_gemm: dtype %d", dtype);
  return LSK_EUNSUPPORTED;
}

extern "C" int lsk_gemm_partial(const void* A, long lda, const void* W, long ldw, float* P, int M, int N, int K, int ks,
                                void* stream) {
  LSK_REQUIRE(A && W && P, LSK_EARG, "lsk_gemm_partial: null pointer");
  LSK_REQUIRE(M >= 0 && N > 0 && K > 0 && lda >= K && ldw == K && ks >= 1 && K % ks == 0 && (K / ks) % 32 == 0 &&
                  N % 16 == 0 && lda % 8 == 0,
              LSK_ESHAPE, "lsk_gemm_partial: bad shape M=%d N=%d K=%d ks=%d", M, N, K, ks);
  if (M == 0) return 0;
  const int mw = launch_wide(EPI_PARTIAL, (hipStream_t)stream, (const uint16_t*)A, lda, (const uint16_t*)W, nullptr, 0,
                             nullptr, 0, P, nullptr, nullptr, M, N, K, 0, ks);
  if (mw > 0) {
    const int rc = lsk_check_launch("lsk_gemm_partial(wide)");
    if (rc || mw == M) return rc;
  }
  const int mr = M - mw;
  const int ns = tile_ns(N, mr, EPI_PARTIAL, K / ks, ks);
  const int ms = ms_for(mr);
  dispatch_bf16(ns, ms, EPI_PARTIAL, N / (16 * ns), (mr + 16 * ms - 1) / (16 * ms), ks, (hipStream_t)stream, A, lda, W,
                ldw, nullptr, 0, nullptr, 0, P, nullptr, nullptr, M, N, K, 0, K / ks, false, mw);
  return lsk_check_launch("lsk_gemm_partial");
}

// Fragment-major A (lsk_frag_off, whole 16-token groups): above 64 rows the wide tier takes its full token blocks
// and the decode kernel the rest, exactly as lsk_gemm / lsk_gemm_partial / lsk_head_argmax split a row-major A,
// with the same tiles (so the same sums).  c_nks > 0 (silu-mul): C fragment-major too.
static void gemm_af(int epi, hipStream_t s, const void* A, const void* W, void* C, long ldc, int c_nks, float* P,
                    float* av, int* ai, int M, int N, int K, int ffn, int ks) {
  const int mw = launch_wide(epi, s, (const uint16_t*)A, 0, (const uint16_t*)W, (uint16_t*)C, ldc, nullptr, 0, P, av,
                             ai, M, N, K, ffn, ks, true, c_nks);
  if (mw == M) return;
  const int mr = M - mw;
  const int ms = ms_for(mr);
  const int ns = epi == EPI_PARTIAL ? tile_ns(N, mr, EPI_PARTIAL, K / ks, ks, 48) : (epi == EPI_ARGMAX ? 4 : tile_ns(N, mr, epi));
  dispatch_bf16(ns, ms, epi, N / (16 * ns), (mr + 16 * ms - 1) / (16 * ms), ks, s, A, 0, W, K, C, ldc, nullptr, 0, P,
                av, ai, M, N, K, ffn, K / ks, true, mw, c_nks);
}

int lsk_gemm_partial_af(const void* A, const void* W, float* P, int M, int N, int K, int ks, void* stream) {
  LSK_REQUIRE(A && W && P, LSK_EARG, "lsk_gemm_partial_af: null pointer");
  LSK_REQUIRE(M >= 0 && N > 0 && N % 16 == 0 && K > 0 && ks >= 1 && K % ks == 0 && (K / ks) % 32 == 0, LSK_ESHAPE,
              "lsk_gemm_partial_af: bad shape M=%d N=%d K=%d ks=%d", M, N, K, ks);
  if (M == 0) return 0;
  gemm_af(EPI_PARTIAL, (hipStream_t)stream, A, W, nullptr, 0, 0, P, nullptr, nullptr, M, N, K, 0, ks);
  return lsk_check_launch("lsk_gemm_partial_af");
}

int lsk_gemm_silu_af(const void* A, const void* W, void* H, int h_frag, int M, int ffn, int K, void* stream) {
  LSK_REQUIRE(A && W && H, LSK_EARG, "lsk_gemm_silu_af: null pointer");
  LSK_REQUIRE(M >= 0 && ffn > 0 && ffn % 32 == 0 && K > 0 && K % 32 == 0, LSK_ESHAPE,
              "lsk_gemm_silu_af: bad shape M=%d ffn=%d K=%d", M, ffn, K);
  if (M == 0) return 0;
  gemm_af(LSK_EPI_SILU_MUL, (hipStream_t)stream, A, W, H, ffn, h_frag ? ffn / 32 : 0, nullptr, nullptr, nullptr, M,
          ffn, K, ffn, 1);
  return lsk_check_launch("lsk_gemm_silu_af");
}

extern "C" int lsk_gemm_partial_frag(const void* A, const void* W, float* P, int M, int N, int K, int ks, void* stream) {
  return lsk_gemm_partial_af(A, W, P, M, N, K, ks, stream);
}

extern "C" int lsk_gemm_silu_frag(const void* A, const void* W, void* H, int h_frag, int M, int ffn, int K,
                                  void* stream) {
  return lsk_gemm_silu_af(A, W, H, h_frag, M, ffn, K, stream);
}

extern "C" size_t lsk_head_workspace_bytes(int M, int N) {
  const size_t nt = (size_t)(N + 63) / 64;
  return lsk_align_up((size_t)M * nt * 4, 256) * 2;
}

extern "C" int lsk_head_argmax(int dtype, const void* A, long lda, const void* W, long ldw, int M, int N, int K,
                               void* logits, long ldl, int64_t* out, const int64_t* dst_idx, void* workspace,
                               size_t ws_bytes, void* stream) {
  LSK_REQUIRE(A && W && out, LSK_EARG, "lsk_head_argmax: null pointer");
  LSK_REQUIRE(M >= 0 && N > 0 && K > 0 && lda >= K && ldw >= K && (logits == nullptr || ldl >= N), LSK_ESHAPE,
              "lsk_head_argmax: bad shape");
  if (M == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  LSK_REQUIRE(dtype == LSK_DTYPE_BF16, LSK_EUNSUPPORTED, "lsk_head_argmax: bf16 only (fp32 uses lsk_gemm + lsk_argmax)");
  LSK_REQUIRE(K % 32 == 0 && N % 64 == 0 && lda % 8 == 0 && ldw == K, LSK_ESHAPE,
              "lsk_head_argmax: needs K %% 32 == 0, N %% 64 == 0 and a packed W (ldw == K; N=%d K=%d)", N, K);
  const int nt = N / 64;
  const size_t half = lsk_align_up((size_t)M * nt * 4, 256);
  LSK_REQUIRE(workspace != nullptr && ws_bytes >= 2 * half, LSK_EWORKSPACE, "lsk_head_argmax: workspace %zu < %zu",
              ws_bytes, 2 * half);
  float* av = (float*)workspace;
  int* ai = (int*)((char*)workspace + half);
  // above 64 rows the wide tier (weights staged in LDS, 128 tokens per workgroup) takes every row
  if (launch_wide(EPI_ARGMAX, s, (const uint16_t*)A, lda, (const uint16_t*)W, (uint16_t*)logits, ldl, nullptr, 0,
                  nullptr, av, ai, M, N, K, 0, 1) != M) {
    const int ms = ms_for(M);
    dispatch_bf16(4, ms, EPI_ARGMAX, nt, (M + 16 * ms - 1) / (16 * ms), 1, s, A, lda, W, ldw, logits, ldl, nullptr, 0,
                  nullptr, av, ai, M, N, K, 0, K);
  }
  int rc = lsk_check_launch("lsk_head_argmax(gemm)");
  if (rc) return rc;
  argmax_tiles_kernel<<<M, 256, 0, s>>>(av, ai, nt, out, dst_idx);
  return lsk_check_launch("lsk_head_argmax(pick)");
}

extern "C" size_t lsk_head_norm_workspace_bytes(int M, int N, int K) {
  const size_t m16 = (size_t)(M + 15) / 16 * 16;
  return lsk_align_up(m16 * (size_t)K * 2, 256) + lsk_head_workspace_bytes(M, N);
}

// Final norm into the workspace (fragment-major), then the head GEMM with its per-tile argmax and the pick, as
// lsk_head_argmax.
extern "C" int lsk_head_norm_argmax(int dtype, const void* h, long ldh, const void* norm_w, float eps, const void* W,
                                    long ldw, int M, int N, int K, void* logits, long ldl, int64_t* out,
                                    const int64_t* dst_idx, void* workspace, size_t ws_bytes, void* stream) {
  LSK_REQUIRE(h && norm_w && W && out, LSK_EARG, "lsk_head_norm_argmax: null pointer");
  LSK_REQUIRE(dtype == LSK_DTYPE_BF16, LSK_EUNSUPPORTED, "lsk_head_norm_argmax: bf16 only");
  LSK_REQUIRE(M >= 0 && N > 0 && K > 0 && ldh >= K && ldw == K && K % 32 == 0 && N % 64 == 0 &&
                  (logits == nullptr || ldl >= N),
              LSK_ESHAPE, "lsk_head_norm_argmax: bad shape M=%d N=%d K=%d (packed W, N %% 64 == 0, K %% 32 == 0)", M,
              N, K);
  if (M == 0) return 0;
  const size_t need = lsk_head_norm_workspace_bytes(M, N, K);
  LSK_REQUIRE(workspace != nullptr && ws_bytes >= need, LSK_EWORKSPACE,
              "lsk_head_norm_argmax: workspace %zu < %zu", ws_bytes, need);
  const size_t xn_bytes = lsk_align_up((size_t)(M + 15) / 16 * 16 * (size_t)K * 2, 256);
  uint16_t* xn = (uint16_t*)workspace;
  char* hw = (char*)workspace + xn_bytes;
  int rc = lsk_add_rmsnorm_impl(dtype, h, ldh, nullptr, 0, norm_w, eps, nullptr, 0, xn, K, 1, M, K, stream);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  const int nt = N / 64;
  const size_t half = lsk_align_up((size_t)M * nt * 4, 256);
  float* av = (float*)hw;
  int* ai = (int*)(hw + half);
  gemm_af(EPI_ARGMAX, s, xn, W, logits, ldl, 0, nullptr, av, ai, M, N, K, 0, 1);
  rc = lsk_check_launch("lsk_head_norm_argmax(gemm)");
  if (rc) return rc;
  argmax_tiles_kernel<<<M, 256, 0, s>>>(av, ai, nt, out, dst_idx);
  return lsk_check_launch("lsk_head_norm_argmax(pick)");
}

static int pack_common(bool pack, const void* src, void* dst, long ld, int N, int K, void* stream, int gh = 0,
                       int paired_groups = 0) {
  const char* what = pack ? "lsk_pack_weight" : "lsk_unpack_weight";
  LSK_REQUIRE(src && dst && src != dst, LSK_EARG, "%s: null or aliased pointers", what);
  LSK_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 32 == 0 && ld >= K && ld % 8 == 0, LSK_ESHAPE,
              "%s: needs N %% 16 == 0, K %% 32 == 0, ld >= K, ld %% 8 == 0 (N=%d K=%d ld=%ld)", what, N, K, ld);
  const long n_slices = (long)N * K / 8;
  const unsigned grid = (unsigned)((n_slices + 255) / 256);
  if (pack)
    pack_weight_kernel<true><<<grid, 256, 0, (hipStream_t)stream>>>((const uint16_t*)src, (uint16_t*)dst, ld, K / 32,
                                                                    n_slices, gh, paired_groups);
  else
    pack_weight_kernel<false><<<grid, 256, 0, (hipStream_t)stream>>>((const uint16_t*)src, (uint16_t*)dst, ld, K / 32,
                                                                     n_slices, gh, paired_groups);
  return lsk_check_launch(what);
}

extern "C" int lsk_pack_weight(const void* W, long ldw, void* Wp, int N, int K, void* stream) {
  return pack_common(true, W, Wp, ldw, N, K, stream);
}

extern "C" int lsk_unpack_weight(const void* Wp, void* W, long ldw, int N, int K, void* stream) {
  return pack_common(false, Wp, W, ldw, N, K, stream);
}

// Fused qkv weight [q (n_heads D rows); k (n_kv_heads D); v (n_kv_heads D)] x K: fragment-major with the q and k row
// groups RoPE-paired (see QkvRope), the storage lsk_gemm_qkv_rope reads.
static int qkv_pack_args(const char* what, int n_heads, int n_kv_heads, int head_dim, int* N, int* gh, int* paired) {
  LSK_REQUIRE(n_heads > 0 && n_kv_heads > 0 && head_dim > 0 && head_dim % 32 == 0, LSK_ESHAPE,
              "%s: head_dim %d must be a multiple of 32 (whole RoPE-paired row groups)", what, head_dim);
  *N = (n_heads + 2 * n_kv_heads) * head_dim;
  *gh = head_dim / 16;
  *paired = (n_heads + n_kv_heads) * *gh;
  return 0;
}

extern "C" int lsk_pack_weight_qkv(const void* W, long ldw, void* Wp, int n_heads, int n_kv_heads, int head_dim, int K,
                                   void* stream) {
  int N, gh, paired;
  const int rc = qkv_pack_args("lsk_pack_weight_qkv", n_heads, n_kv_heads, head_dim, &N, &gh, &paired);
  if (rc) return rc;
  return pack_common(true, W, Wp, ldw, N, K, stream, gh, paired);
}

extern "C" int lsk_unpack_weight_qkv(const void* Wp, void* W, long ldw, int n_heads, int n_kv_heads, int head_dim,
                                     int K, void* stream) {
  int N, gh, paired;
  const int rc = qkv_pack_args("lsk_unpack_weight_qkv", n_heads, n_kv_heads, head_dim, &N, &gh, &paired);
  if (rc) return rc;
  return pack_common(false, Wp, W, ldw, N, K, stream, gh, paired);
}

// qkv projection + RoPE + KV append in one GEMM (bf16).  A: the normalised rows fragment-major (lsk_frag_off,
// whole 16-token groups); W: lsk_pack_weight_qkv storage.  No K split: each output's sum runs over all of K in the
// decode kernel's chunk-class order in both tiers (batch invariant).  Writes q_out [M, n_heads, head_dim] (rotated),
// the K cache (rotated) and the V cache at (rows[m], pos[m]), with the RoPE + append kernel's arithmetic.
extern "C" int lsk_gemm_qkv_rope(const void* A, const void* W, int M, int n_heads, int n_kv_heads, int head_dim, int K,
                                 void* q_out, void* kcache, void* vcache, const float* cos_tab, const float* sin_tab,
                                 int tab_len, const int32_t* rows, const int32_t* pos, int max_batch, int max_seq,
                                 void* stream) {
  LSK_REQUIRE(A && W && q_out && kcache && vcache && cos_tab && sin_tab && rows && pos, LSK_EARG,
              "lsk_gemm_qkv_rope: null pointer");
  int N, gh, paired;
  int rc = qkv_pack_args("lsk_gemm_qkv_rope", n_heads, n_kv_heads, head_dim, &N, &gh, &paired);
  if (rc) return rc;
  LSK_REQUIRE(M >= 0 && K > 0 && K % 32 == 0 && max_batch > 0 && max_seq > 0 && max_seq % 32 == 0 && tab_len > 0,
              LSK_ESHAPE, "lsk_gemm_qkv_rope: bad shape M=%d K=%d max_seq=%d", M, K, max_seq);
  if (M == 0) return 0;
  const QkvRope qa{(uint16_t*)q_out, (uint16_t*)kcache, (uint16_t*)vcache, cos_tab, sin_tab, rows, pos, n_heads,
                   n_kv_heads, head_dim, max_batch, max_seq, tab_len};
  hipStream_t s = (hipStream_t)stream;
  const int mw = launch_wide(EPI_QKV, s, (const uint16_t*)A, 0, (const uint16_t*)W, nullptr, 0, nullptr, 0, nullptr,
                             nullptr, nullptr, M, N, K, 0, 1, true, 0, qa);
  if (mw < M) {
    // one K slice, 32-row tiles: a weight with fewer than 192 tiles (the 1B shape's 96) splits the tokens over
    // two or more token tiles, so every CU streams (the weights are re-read from the XCD's L2): 1B qkv at 64
    // tokens 11.9 -> 10.0 us on MI355X
    const int mr = M - mw;
    int ms = ms_for(mr);
    while (ms > 1 && (long)(N / 32) * ((mr + 16 * ms - 1) / (16 * ms)) < 192) --ms;
    dispatch_bf16(2, ms, EPI_QKV, N / 32, (mr + 16 * ms - 1) / (16 * ms), 1, s, A, 0, W, K, nullptr, 0, nullptr, 0,
                  nullptr, nullptr, nullptr, M, N, K, 0, K, true, mw, 0, qa);
  }
  return lsk_check_launch("lsk_gemm_qkv_rope");
}
