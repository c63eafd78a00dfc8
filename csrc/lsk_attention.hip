// Ragged verify / decode attention over the static KV cache (solutions/packed.py:142-166).
//
// Rule (solutions/packed.py:6-8): a query token at position p of cache row r attends to the
// cached positions 0..p of row r (this call's K/V already appended), for every block kind:
// decode (T = 1), verification (T = d + 1) and prefill chunks.
//
// Layouts
//   q      [N, Hq, D]            (packed token axis; RoPE applied)
//   K      bf16: [B, Hkv, S/32, 2 D/32, 64, 8] fragment-major blocks (k_cache_offset in lsk_common.h);
//          fp32: [B, Hkv, S, D] (the KVCache layout of common/model.py:171-183)
//   V      [B, Hkv, S/32, D, 32] (stored in 32-position blocks, each block transposed: element (pos, d)
//                                 at ((pos / 32) * D + d) * 32 + pos % 32 within a (row, head) stripe)
//   out    [N, Hq * D]
//   blocks int32 [nb][4] = {q_start, pos0, T, row}
//   works  int32 [n_work][8] = {q_start, row0, nrows, kv_lo, kv_hi, part, pos0, row} (the block's fields
//                                 copied in; the fp32 kernel reads them directly)
//   recs   int32 [n_slots][n_rounds][8]: the bf16 kernel's static schedule, one record per (work, KV head)
//                                 = the work record with nrows | kvh << 8 in field 2; slot s runs its records
//                                 in order and stops at the first with nrows = 0, so a workgroup's first
//                                 load depends on nothing but its own index
//   groups int32 [n_group][8] = {blk, row0, nrows, part_first, n_split, 0, 0, 0}
// The G query heads of a KV head are folded into query rows: row = t * G + g (t = token of the
// block, g = head within the group); a work item serves up to ATTN_ROWS = 48 rows, so one KV read serves
// G*T <= 48 rows.
//
// Long contexts are split into fixed, position-aligned chunks of LSK_ATTN_SPLIT positions
// (flash-decoding).  Split boundaries, tile boundaries, the wave that owns a tile and both merge
// orders depend only on absolute positions, so the result for a query never depends on which other
// tokens share its block or batch (batch invariance: a T = 1 decode query and the same query inside a
// T = 9 verify block give bitwise identical outputs).
#include <algorithm>
#include <functional>
#include <mutex>
#include <vector>

#include "lsk_common.h"
#include "../include/lsk.h"

#define ATTN_TILE 64   // work ranges are split at multiples of this (planner granularity)
#define ATTN_STEP 32   // KV positions per step of a wave
#define ATTN_QT 3      // 16-row MFMA column tiles per work item
#define ATTN_ROWS (16 * ATTN_QT)  // query rows per work item: a T <= 12 block of a 4-head group in one item
#define ATTN_MERGE_TILES 2  // column tiles merged per LDS pass of the wave merge
#define ATTN_MAX_SPLITS 128
#define ATTN_WAVES 8   // waves per work item; fixed, because it fixes which wave accumulates which step


__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max / sum over the four 16-lane rows of a wave, result in every lane (the xor-16 then xor-32 butterfly),
// with gfx950's row swaps: v_permlane16_swap(x, x) yields rows {0,0,2,2} and {1,1,3,3},
// v_permlane32_swap(x, x) the lower and the upper half in every lane.  Plain VALU, no LDS round trip;
// a + b == b + a, so every lane ends with the same bits.
__device__ __forceinline__ float rows_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// bf16 path.  Cache layouts: K in fragment-major 32-position blocks (k_cache_offset), V in transposed
// 32-position blocks (V^T per block), so both MFMA operands come straight from HBM as 16-byte vectors and
// every K or V^T fragment load of a wave is 1 KiB contiguous (read non-temporally: each byte once per launch):
//   S^T[pos][q] = K Q^T        v_mfma_f32_16x16x32_bf16, A = K rows (16 positions x 32 d), B = Q^T
//   O^T[d][q]  += V^T P^T      v_mfma_f32_16x16x32_bf16, A = V^T (16 d x 32 positions), B = P^T
// Each lane owns one query column (l16) of each column tile, so the running max / row sum are lane-local
// up to a butterfly over the four 16-lane rows (rows_max / rows_sum).  A 32-position step uses two S^T
// sub-tiles whose MFMA rows are mapped to positions so that lane group g holds positions 8g .. 8g+7 of the
// step: exactly the 8 consecutive positions its P^T fragment and its 16-byte V^T load need.
// QT column tiles of 16 query rows share every K / V fragment of a work item.  QT = 3 (items of up to 48 rows):
// the KV of a (block, KV head) is read by one workgroup for blocks of up to 48 / G tokens (a 9-token verify
// block of a 4-head group is 36 rows); the item's Q sits in LDS (rows padded by 16 bytes: the 16-byte reads of
// 16 rows hit distinct banks), which keeps three tiles' accumulators within 256 VGPRs.  QT = 1 (items of up to
// 16 rows, for launches whose rows-per-item cap is 16): Q stays in registers.  A row's arithmetic is the same
// in both, so they give bitwise equal outputs.  The 8 waves take the
// 32-position steps of the item's KV range round robin (step index within the split mod 8), keep the next
// step's K and V loads in flight while they compute, and are merged in wave order through LDS, two column
// tiles per pass; 8 waves keep the chain of dependent steps short when a decode batch has few
// (block, KV head) pairs.
template <int D, int QT>
__global__ __launch_bounds__(64 * ATTN_WAVES, 1) void attn_bf16_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vt,
    const int32_t* __restrict__ recs, int n_rounds, uint16_t* __restrict__ out, float* __restrict__ o_part,
    float* __restrict__ ml_part, int G, int Hkv, int S, float scale_log2, int out_nks) {
  constexpr int KSTEPS = D / 32;
  constexpr int CT = D / 16;
  constexpr int NW = ATTN_WAVES;
  constexpr int ROWS = 16 * QT;                      // rows per item
  constexpr bool QREG = QT == 1;                     // one tile: Q fragments in registers, no s_q
  constexpr int MT = QT < ATTN_MERGE_TILES ? QT : ATTN_MERGE_TILES;
  constexpr int MR = 16 * MT;                        // rows per merge pass
  constexpr int QLD = D + 8;                         // s_q row stride in bf16 elements
  constexpr int QCH = D / 8;                         // 16-byte chunks per Q row
  constexpr int QPT = (ROWS * QCH + 64 * NW - 1) / (64 * NW);  // Q chunks staged per thread
  __shared__ float s_ml[NW][2][ROWS];
  __shared__ __attribute__((aligned(16))) float s_o[NW][MR][D + 4];
  __shared__ __attribute__((aligned(16))) uint16_t s_q[QREG ? 1 : ROWS][QLD];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int Hq = Hkv * G;
  const int32_t* my_recs = recs + (long)blockIdx.x * n_rounds * 8;

  struct Item {
    int q_start, row0, nrows, kv_lo, kv_hi, part, pos0, crow, kvh;
  };
  // record r of this slot (nrows = 0 past the slot's last item)
  auto fetch = [&](int r) {
    Item it;
    if (r >= n_rounds) {
      it.nrows = 0;
      return it;
    }
    const int32_t* wk = my_recs + (long)r * 8;
    it.q_start = wk[0]; it.row0 = wk[1]; it.nrows = wk[2] & 255; it.kvh = wk[2] >> 8; it.kv_lo = wk[3];
    it.kv_hi = wk[4]; it.part = wk[5]; it.pos0 = wk[6]; it.crow = wk[7];
    return it;
  };
  auto kbase_of = [&](const Item& it) { return kc + ((long)it.crow * Hkv + it.kvh) * (long)S * D; };
  auto vbase_of = [&](const Item& it) { return vt + ((long)it.crow * Hkv + it.kvh) * (long)D * S; };

  // Q of an item: global -> registers (in flight during the previous item's merge) -> LDS; rows >= nrows are 0.
  // One tile (QREG): each lane loads its own column's fragments straight into qreg.
  lsk_bf16x8 qst[QPT];
  lsk_bf16x8 qreg[KSTEPS];
  auto q_load = [&](const Item& it) {
    if constexpr (QREG) {
      const bool valid = l16 < it.nrows;
      const int r = it.row0 + (valid ? l16 : 0);
      const int t = r / G, g = r - t * G;
      const uint16_t* qrow = q + ((long)(it.q_start + t) * Hq + it.kvh * G + g) * D;
#pragma unroll
      for (int j = 0; j < KSTEPS; ++j)
        qreg[j] = valid ? *(const lsk_bf16x8*)(qrow + 32 * j + 8 * lg) : (lsk_bf16x8){};
      return;
    }
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int c = tid + i * 64 * NW;
      const int r = c / QCH, c8 = c - r * QCH;
      lsk_bf16x8 v = {};
      if (r < it.nrows) {
        const int rr = it.row0 + r, t = rr / G, g = rr - t * G;
        v = *(const lsk_bf16x8*)(q + ((long)(it.q_start + t) * Hq + it.kvh * G + g) * D + 8 * c8);
      }
      qst[i] = v;
    }
  };
  auto q_store = [&]() {
    if constexpr (!QREG) {
#pragma unroll
      for (int i = 0; i < QPT; ++i) {
        const int c = tid + i * 64 * NW;
        const int r = c / QCH, c8 = c - r * QCH;
        if (r < ROWS) *(lsk_bf16x8*)(&s_q[r][8 * c8]) = qst[i];
      }
    }
  };
  // K / V fragments come through buffer loads over the item's (row, KV head) stripe: the descriptor and every
  // uniform offset live in SGPRs, a lane adds one 32-bit offset, so no 64-bit per-lane addresses occupy VGPRs.
  // Non-temporal (aux 2): each byte is read once per launch.  The descriptor's range ends at the 32-position block
  // holding the item's last position (kv_hi - 1): a step past it reads as zeros without touching memory, so the
  // next step's loads are issued unconditionally -- with them under `if (more)` the compiler's wait counts merged
  // the two paths and every step's K.Q waited for the next step's V loads too.
  auto stripe = [&](const uint16_t* base, int hi) {
    const int blocks_end = min(S, (hi + ATTN_STEP - 1) / ATTN_STEP * ATTN_STEP);
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, blocks_end * D * 2, LSK_BUFFER_RSRC_WORD3);
  };
  auto ldkv = [&](__amdgpu_buffer_rsrc_t rs, int vo, int so) -> lsk_bf16x8 {
    return __builtin_bit_cast(lsk_bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, vo, so, 2));
  };
  const int k_vo = 16 * lane;                       // bytes: lane l's 8 elements of a 1 KiB K fragment
  const int v_vo = 2 * (32 * l16 + 8 * lg);         // bytes: column l16's positions 8 lg .. 8 lg + 7 of a V^T row
  constexpr int STRIDE = ATTN_STEP * NW;  // positions between a wave's consecutive steps
  lsk_bf16x8 kf[2][KSTEPS];
  lsk_bf16x8 vf[CT];
  // fragment-major K cache: fragment (a, j) of the step's 32-position block is 1 KiB in lane order
  auto load_k = [&](__amdgpu_buffer_rsrc_t kr, int sb) {
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int j = 0; j < KSTEPS; ++j) kf[a][j] = ldkv(kr, k_vo, 2 * (sb * D + (a * KSTEPS + j) * 512));
  };
  auto load_v = [&](__amdgpu_buffer_rsrc_t vr, int sb) {
#pragma unroll
    for (int c = 0; c < CT; ++c) vf[c] = ldkv(vr, v_vo, 2 * (sb * D + 16 * c * 32));
  };
  // a wave's steps of an item: 32-position steps wave, wave + NW, ... of the item's range, in order
  auto first_step = [&](const Item& it) { return it.kv_lo + ATTN_STEP * wave; };
  auto issue_first = [&](const Item& it) {
    q_load(it);
    const int sb = first_step(it);
    const auto kr = stripe(kbase_of(it), it.kv_hi), vr = stripe(vbase_of(it), it.kv_hi);
    load_k(kr, sb);  // (a wave with no step in the item reads zeros past the range)
    load_v(vr, sb);
  };

  Item cur = fetch(0);
  if (cur.nrows == 0) return;
  issue_first(cur);
  Item nxt = fetch(1);  // the next record is read while this item streams
  if constexpr (!QREG) {
    q_store();
    __syncthreads();
  }
  for (int r = 0; cur.nrows > 0; ++r) {
    const int nq = (cur.nrows + 15) >> 4;  // column tiles in use (wave-uniform)
    const int kv_hi = cur.kv_hi;
    const auto kb = stripe(kbase_of(cur), kv_hi), vb = stripe(vbase_of(cur), kv_hi);
    int qpos[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int rl = 16 * qt + l16;
      qpos[qt] = rl < cur.nrows ? cur.pos0 + (cur.row0 + rl) / G : -1;  // invalid rows: every score masked
    }
    // positions every valid row of the item may read without masking: <= the first row's position, < kv_hi
    const int full_lim = min(kv_hi - 1, cur.pos0 + cur.row0 / G);
    lsk_f32x4 oacc[QT][CT];
    float m_run[QT], l_run[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      m_run[qt] = -INFINITY;
      l_run[qt] = 0.f;
#pragma unroll
      for (int c = 0; c < CT; ++c) oacc[qt][c] = (lsk_f32x4){0.f, 0.f, 0.f, 0.f};
    }
    for (int sb = first_step(cur); sb < kv_hi; sb += STRIDE) {
      const int sn = sb + STRIDE;
      const bool full = sb + ATTN_STEP - 1 <= full_lim;  // wave-uniform: no position of the step is masked
      lsk_bf16x8 pb[QT];
      float alpha[QT];
      // per column tile: S^T = K Q^T, then the online-softmax update of its 16 query columns
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        if (qt < nq) {
          lsk_bf16x8 qf[KSTEPS];
#pragma unroll
          for (int j = 0; j < KSTEPS; ++j)
            qf[j] = QREG ? qreg[j] : *(const lsk_bf16x8*)(&s_q[16 * qt + l16][32 * j + 8 * lg]);
          lsk_f32x4 sacc[2];
#pragma unroll
          for (int a = 0; a < 2; ++a) {
            sacc[a] = (lsk_f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < KSTEPS; ++j)
              sacc[a] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[a][j], qf[j], sacc[a], 0, 0, 0);
          }
          // sacc[a][e] <-> position sb + 8 lg + 4 a + e, query column l16 of tile qt
          float sv[8];
          float mt = -INFINITY;
#pragma unroll
          for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float sc = sacc[a][e] * scale_log2;
              if (!full) {
                const int kp = sb + 8 * lg + 4 * a + e;
                sc = (kp < kv_hi && kp <= qpos[qt]) ? sc : -INFINITY;
              }
              sv[4 * a + e] = sc;
              mt = fmaxf(mt, sc);
            }
          mt = rows_max(mt);
          const float m_new = fmaxf(m_run[qt], mt);
          alpha[qt] = (m_new == m_run[qt]) ? 1.f : fast_exp2(m_run[qt] - m_new);
          float rs = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float pe = (sv[e] == -INFINITY) ? 0.f : fast_exp2(sv[e] - m_new);
            rs += pe;
            pb[qt][e] = static_cast<__bf16>(pe);
          }
          rs = rows_sum(rs);
          l_run[qt] = l_run[qt] * alpha[qt] + rs;
          m_run[qt] = m_new;
        }
      }
      load_k(kb, sn);  // the next step's K streams in during this step's P.V (zeros past the range)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        if (qt < nq) {
#pragma unroll
          for (int c = 0; c < CT; ++c) {
            oacc[qt][c][0] *= alpha[qt];
            oacc[qt][c][1] *= alpha[qt];
            oacc[qt][c][2] *= alpha[qt];
            oacc[qt][c][3] *= alpha[qt];
            oacc[qt][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[c], pb[qt], oacc[qt][c], 0, 0, 0);
          }
        }
      }
      load_v(vb, sn);
    }
    // the next item's Q and first K / V loads fly while this item is merged
    const Item done = cur;
    cur = nxt;
    if (cur.nrows > 0) {
      issue_first(cur);
      nxt = fetch(r + 2);
    }
    // ---- merge the waves in order: M = max m_w, e_w = exp2(m_w - M), L = sum e_w l_w, O = sum e_w O_w
    //      (ATTN_MERGE_TILES column tiles per pass through s_o; the pass loop is unrolled, so a tile's
    //      accumulators are dead after its pass)
#pragma unroll
    for (int p0 = 0; p0 < QT; p0 += MT) {
      if (p0 >= nq) break;
#pragma unroll
      for (int qt = p0; qt < p0 + MT && qt < QT; ++qt) {
        if (qt < nq) {
          if (lg == 0) {
            s_ml[wave][0][16 * qt + l16] = m_run[qt];
            s_ml[wave][1][16 * qt + l16] = l_run[qt];
          }
#pragma unroll
          for (int c = 0; c < CT; ++c)
            *(float4*)(&s_o[wave][16 * (qt - p0) + l16][16 * c + 4 * lg]) =
                make_float4(oacc[qt][c][0], oacc[qt][c][1], oacc[qt][c][2], oacc[qt][c][3]);
        }
      }
      __syncthreads();
      // 4 consecutive d of one row per thread: the row's weights are formed once per 4 outputs, s_o is read as
      // float4 (consecutive lanes, consecutive 16 bytes), each output keeps the order O = ((e_0 O_0 + e_1 O_1) + ...)
      const int pr = min(done.nrows - 16 * p0, MR);
      for (int e = tid; e < pr * (D / 4); e += 64 * NW) {
        const int ql = e / (D / 4), d = 4 * (e - ql * (D / 4));
        const int qr = 16 * p0 + ql;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, s_ml[w][0][qr]);
        float L = 0.f;
        float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const float mw = s_ml[w][0][qr];
          const float ew = (mw == -INFINITY) ? 0.f : ((mw == M) ? 1.f : fast_exp2(mw - M));
          L = L + ew * s_ml[w][1][qr];
          const float4 ow = *(const float4*)(&s_o[w][ql][d]);
          O.x = O.x + ew * ow.x;
          O.y = O.y + ew * ow.y;
          O.z = O.z + ew * ow.z;
          O.w = O.w + ew * ow.w;
        }
        const int rr = done.row0 + qr;
        const int tt = rr / G, gg = rr - tt * G;
        if (done.part < 0) {
          uint2 pk;
          pk.x = (uint32_t)f2bf(O.x / L) | ((uint32_t)f2bf(O.y / L) << 16);
          pk.y = (uint32_t)f2bf(O.z / L) | ((uint32_t)f2bf(O.w / L) << 16);
          // out_nks > 0: fragment-major output (the o projection's input); 4 columns stay one 8-byte piece
          const int ot = done.q_start + tt, oc = (done.kvh * G + gg) * D + d;
          *(uint2*)(out + (out_nks > 0 ? lsk_frag_off(ot, oc, out_nks) : (long)ot * Hq * D + oc)) = pk;
        } else {
          const long slot = ((long)done.part * Hkv + done.kvh) * ATTN_ROWS + qr;
          *(float4*)(o_part + slot * D + d) = O;
          if (d == 0) {
            ml_part[slot * 2 + 0] = M;
            ml_part[slot * 2 + 1] = L;
          }
        }
      }
      // every wave is past its steps, so s_q takes the next item's Q (its loads have landed during the merge)
      if (p0 == 0 && cur.nrows > 0) q_store();
      __syncthreads();  // the merge has read s_o / s_ml before they are written again; s_q is visible
    }
  }
}

// Merge the splits of one query group in split order:
//   M = max_s m_s, w_s = exp2(m_s - M) (0 for an empty split, 1 when m_s == M),
//   out = (sum_s w_s O_s) / (sum_s w_s l_s).
// A group with a single non-empty split reduces to O_0 / l_0, exactly what the direct path stores.
// The per-row weights and denominators are computed once into LDS; the O partials stream as float4.
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(const int32_t* __restrict__ blocks,
                                                           const int32_t* __restrict__ groups,
                                                           const float* __restrict__ o_part,
                                                           const float* __restrict__ ml_part, T* __restrict__ out,
                                                           int G, int Hkv, int out_nks) {
  __shared__ float s_w[ATTN_ROWS][ATTN_MAX_SPLITS];
  __shared__ float s_L[ATTN_ROWS];
  const int32_t* gp = groups + (long)blockIdx.x * 8;
  const int blk = gp[0], row0 = gp[1], nrows = gp[2], pf = gp[3], ns = gp[4];
  const int kvh = blockIdx.y;
  const int Hq = Hkv * G;
  const int q_start = blocks[(long)blk * 4 + 0];
  const int tid = threadIdx.x;
  if (tid < nrows) {
    const int rl = tid;
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, ml_part[(((long)(pf + s) * Hkv + kvh) * ATTN_ROWS + rl) * 2]);
    float L = 0.f;
    for (int s = 0; s < ns; ++s) {
      const long slot = ((long)(pf + s) * Hkv + kvh) * ATTN_ROWS + rl;
      const float ms = ml_part[slot * 2], ls = ml_part[slot * 2 + 1];
      const float w = (ms == -INFINITY) ? 0.f : ((ms == M) ? 1.f : fast_exp2(ms - M));
      s_w[rl][s] = w;
      L = L + w * ls;
    }
    s_L[rl] = L;
  }
  __syncthreads();
  for (int e = tid; e < nrows * (D / 4); e += 256) {
    const int rl = e / (D / 4), d4 = e - rl * (D / 4);
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < ns; ++s) {
      const float w = s_w[rl][s];
      const float4 v = *(const float4*)(o_part + (((long)(pf + s) * Hkv + kvh) * ATTN_ROWS + rl) * D + 4 * d4);
      O.x = O.x + w * v.x;
      O.y = O.y + w * v.y;
      O.z = O.z + w * v.z;
      O.w = O.w + w * v.w;
    }
    const float L = s_L[rl];
    const int r = row0 + rl;
    const int t = r / G, g = r - t * G;
    const int ot = q_start + t, oc = (kvh * G + g) * D + 4 * d4;
    T* o = out + (out_nks > 0 ? lsk_frag_off(ot, oc, out_nks) : (long)ot * Hq * D + oc);
    Elem<T>::st(o + 0, O.x / L);
    Elem<T>::st(o + 1, O.y / L);
    Elem<T>::st(o + 2, O.z / L);
    Elem<T>::st(o + 3, O.w / L);
  }
}

// ----------------------------------------------------------------------------- fp32 path
// Straightforward per-query kernel for fp32 models (parity runs; V cache in the same blocked transposed
// layout as the bf16 path): one wave per query row, the
// row's positions 0..qpos in 64-position chunks (lane = position), online softmax with lsk_exp,
// O[d] accumulated over the chunk's positions in order.  Fixed order per query -> batch invariant.
template <int D>
__global__ __launch_bounds__(256) void attn_f32_kernel(const float* __restrict__ q, const float* __restrict__ kc,
                                                       const float* __restrict__ vc,
                                                       const int32_t* __restrict__ works, float* __restrict__ out,
                                                       int G, int Hkv, int S, float scale) {
  constexpr int DPL = (D + 63) / 64;  // d values per lane
  __shared__ float sp[4][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kvh = blockIdx.y;
  const int Hq = Hkv * G;
  const int32_t* wk = works + (long)blockIdx.x * 8;
  const int q_start = wk[0], row0 = wk[1], nrows = wk[2], pos0 = wk[6], crow = wk[7];
  const long head_base = ((long)crow * Hkv + kvh) * (long)S * D;
  for (int rl = wave; rl < nrows; rl += 4) {
    const int r = row0 + rl;
    const int t = r / G, g = r - t * G;
    const int qpos = pos0 + t;
    const float* qv = q + ((long)(q_start + t) * Hq + kvh * G + g) * D;
    float m_run = -INFINITY, l_run = 0.f;
    float o[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) o[i] = 0.f;
    for (int base = 0; base <= qpos; base += 64) {
      const int kp = base + lane;
      float s = -INFINITY;
      if (kp <= qpos) {
        const float* kr = kc + head_base + (long)kp * D;
        float acc = 0.f;
        for (int d = 0; d < D; ++d) acc += qv[d] * kr[d];
        s = acc * scale;
      }
      float mt = s;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) mt = fmaxf(mt, __shfl_xor(mt, off, 64));
      const float m_new = fmaxf(m_run, mt);
      const float alpha = (m_new == m_run) ? 1.f : lsk_exp(m_run - m_new);
      const float p = (s == -INFINITY) ? 0.f : lsk_exp(s - m_new);
      float rs = p;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) rs += __shfl_xor(rs, off, 64);
      l_run = l_run * alpha + rs;
      m_run = m_new;
      sp[wave][lane] = p;
      __builtin_amdgcn_wave_barrier();
      const int nvalid = min(64, qpos + 1 - base);
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        const int d = lane + 64 * i;
        if (d < D) {
          float acc = o[i] * alpha;
          for (int j = 0; j < nvalid; ++j) acc += sp[wave][j] * vc[head_base + (long)base * D + d * 32 + j % 32 + (j / 32) * 32 * D];
          o[i] = acc;
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
    float* orow = out + (long)(q_start + t) * Hq * D + (long)(kvh * G + g) * D;
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      const int d = lane + 64 * i;
      if (d < D) orow[d] = o[i] / l_run;
    }
  }
}

// ----------------------------------------------------------------------------- host planner

// Work order: a "family" is the set of query tiles of one (block, split); its tiles read the same K/V.
// Families are sorted by size and dealt in chunks of 8 launch slots; slots of shorter families in a chunk are
// padding items (nrows = 0), so sibling tiles sit 8 slots apart.  Output appended to `works` / `groups`.
static int plan_into(const int32_t* blocks, int nb, int group, int split, int rows_cap, std::vector<int32_t>& works,
                     std::vector<int32_t>& groups, int* n_parts) {
  LSK_REQUIRE(nb >= 0 && group > 0 && split >= ATTN_TILE && split % ATTN_TILE == 0, LSK_ESHAPE,
              "lsk_attn_plan: bad arguments (split must be a positive multiple of %d)", ATTN_TILE);
  LSK_REQUIRE(rows_cap > 0 && rows_cap % 16 == 0 && rows_cap <= ATTN_ROWS, LSK_ESHAPE,
              "lsk_attn_plan: rows per item %d (a multiple of 16 up to %d)", rows_cap, ATTN_ROWS);
  const int R = rows_cap;
  struct Item { int b, row0, nrows, lo, hi, part; };  // b: block index (its fields are copied into the record)
  thread_local std::vector<Item> items;               // families back to back
  thread_local std::vector<int> fam_off, fam_order, part_first, ns_of;
  items.clear();
  fam_off.clear();
  works.clear();
  groups.clear();
  int ng = 0, np = 0;
  for (int b = 0; b < nb; ++b) {
    const int pos0 = blocks[b * 4 + 1], T = blocks[b * 4 + 2];
    LSK_REQUIRE(T >= 0 && pos0 >= 0, LSK_ESHAPE, "lsk_attn_plan: block %d has T=%d pos0=%d", b, T, pos0);
    const int rows = T * group;
    const int nq = (rows + R - 1) / R;
    if (nq == 0) continue;
    // KV range of the family = the longest tile's range; each tile uses its own end
    int ns_max = 0;
    for (int qt = 0; qt < nq; ++qt) {
      const int row0 = qt * R, nrows = rows - row0 < R ? rows - row0 : R;
      const long kv_end = (long)pos0 + (row0 + nrows - 1) / group + 1;
      const int ns = (int)((kv_end + split - 1) / split);
      LSK_REQUIRE(ns <= ATTN_MAX_SPLITS || split >= (1 << 29), LSK_ESHAPE,
                  "lsk_attn_plan: %d splits of %d positions exceed %d", ns, split, ATTN_MAX_SPLITS);
      ns_max = ns > ns_max ? ns : ns_max;
    }
    part_first.resize(nq);
    ns_of.resize(nq);
    for (int qt = 0; qt < nq; ++qt) {
      const int row0 = qt * R, nrows = rows - row0 < R ? rows - row0 : R;
      const long kv_end = (long)pos0 + (row0 + nrows - 1) / group + 1;
      ns_of[qt] = (int)((kv_end + split - 1) / split);
      if (ns_of[qt] > 1) {
        const int32_t g[8] = {b, row0, nrows, np, ns_of[qt], 0, 0, 0};
        groups.insert(groups.end(), g, g + 8);
        ++ng;
        part_first[qt] = np;
        np += ns_of[qt];
      } else {
        part_first[qt] = -1;
      }
    }
    for (int sidx = 0; sidx < ns_max; ++sidx) {
      fam_off.push_back((int)items.size());
      for (int qt = 0; qt < nq; ++qt) {
        if (sidx >= ns_of[qt]) continue;
        const int row0 = qt * R, nrows = rows - row0 < R ? rows - row0 : R;
        const long kv_end = (long)pos0 + (row0 + nrows - 1) / group + 1;
        const long lo = (long)sidx * split;
        const long hi = (lo + split < kv_end) ? lo + split : kv_end;
        items.push_back({b, row0, nrows, (int)lo, (int)hi, part_first[qt] >= 0 ? part_first[qt] + sidx : -1});
      }
    }
  }
  const int nf = (int)fam_off.size();
  fam_off.push_back((int)items.size());
  fam_order.resize(nf);
  for (int f = 0; f < nf; ++f) fam_order[f] = f;
  auto fsize = [&](int f) { return fam_off[f + 1] - fam_off[f]; };
  std::stable_sort(fam_order.begin(), fam_order.end(), [&](int a, int b) { return fsize(a) > fsize(b); });
  auto emit = [&](const Item* it) {
    int32_t w[8] = {0, 0, 0, 0, 0, -1, 0, 0};
    if (it) {
      const int32_t* bm = blocks + (long)it->b * 4;
      w[0] = bm[0]; w[1] = it->row0; w[2] = it->nrows; w[3] = it->lo; w[4] = it->hi; w[5] = it->part;
      w[6] = bm[1]; w[7] = bm[3];
    }
    works.insert(works.end(), w, w + 8);
  };
  for (int c0 = 0; c0 < nf; c0 += 8) {
    const int c1 = c0 + 8 < nf ? c0 + 8 : nf;
    int depth = 0;
    for (int f = c0; f < c1; ++f) depth = fsize(fam_order[f]) > depth ? fsize(fam_order[f]) : depth;
    for (int k = 0; k < depth; ++k)
      for (int f = c0; f < c0 + 8; ++f) {
        const bool real = f < c1 && k < fsize(fam_order[f]);
        if (!real && (depth == 1 || f >= c1)) continue;  // no sibling to align: skip the padding
        emit(real ? &items[fam_off[fam_order[f]] + k] : nullptr);
      }
  }
  *n_parts = np;
  (void)ng;
  return 0;
}

extern "C" int lsk_attn_plan(const int32_t* blocks, int nb, int group, int split, int rows_cap, int32_t* works,
                             int max_works, int32_t* groups, int max_groups, int* n_works, int* n_groups,
                             int* n_parts) {
  LSK_REQUIRE(blocks && works && n_works && n_groups && n_parts, LSK_EARG, "lsk_attn_plan: null pointer");
  thread_local std::vector<int32_t> w, g;
  int np = 0;
  const int rc = plan_into(blocks, nb, group, split, rows_cap, w, g, &np);
  if (rc) return rc;
  const int nw = (int)(w.size() / 8), ng = (int)(g.size() / 8);
  LSK_REQUIRE(nw <= max_works, LSK_EWORKSPACE, "lsk_attn_plan: too many work items (max %d)", max_works);
  LSK_REQUIRE(ng == 0 || (groups != nullptr && ng <= max_groups), LSK_EWORKSPACE,
              "lsk_attn_plan: too many combine groups");
  std::copy(w.begin(), w.end(), works);
  if (ng) std::copy(g.begin(), g.end(), groups);
  *n_works = nw;
  *n_groups = ng;
  *n_parts = np;
  return 0;
}

// Rows per work item for one launch over n_slots persistent workgroups (one per CU).  The cap never changes a
// result: a row's scores, softmax and P.V depend only on its own column, its position and the fixed splits.
// It trades parallelism against KV re-reads: with few (block, KV head) pairs a launch is latency-bound and
// splitting a block's rows over more workgroups shortens the longest item (16-row items run the one-tile
// kernel, Q in registers; wider items the three-tile kernel, whose extra tiles cost every step and the merge);
// once the items fill the chip, every extra item re-reads its block's KV and the launch is bandwidth-bound.
// Estimate per cap = max(longest-first makespan of the items, KV bytes / sustained bandwidth) with item time
//   one-tile kernel:   steps * c
//   three-tile kernel: a + b (nq - 1) + steps (c + d [nq = 3])
// (steps = 32-position steps per wave, 8 waves), constants fitted to graph-timed decode-shaped launches on
// MI355X (contexts 300-1400, 1-9 query tokens of a 4-head group, 10-64 requests); equal estimates go to
// the shorter makespan, then to the larger cap.
#define ATTN_COST_ITEM_US 1.0
#define ATTN_COST_TILE_US 3.5
#define ATTN_COST_STEP_US 2.9
#define ATTN_COST_STEP3_US 0.6
#define ATTN_COST_BW_BYTES_PER_US 6.0e6
static int rows_cap_for(const int32_t* blocks, int nb, int group, int split, int n_kv_heads, int head_dim,
                        int n_slots) {
  LSK_REQUIRE(nb >= 0 && group > 0 && split >= ATTN_TILE && n_kv_heads > 0 && head_dim > 0 && n_slots > 0,
              LSK_ESHAPE, "lsk_attn_rows_cap: bad arguments");
  auto items_at = [&](int R) {
    long n = 0;
    for (int b = 0; b < nb; ++b) {
      const long rows = (long)blocks[b * 4 + 2] * group, end = (long)blocks[b * 4 + 1] + blocks[b * 4 + 2];
      n += (rows + R - 1) / R * ((end + split - 1) / split);
    }
    return n * n_kv_heads;
  };
  if (items_at(ATTN_ROWS) >= 2L * n_slots) return ATTN_ROWS;  // several items per workgroup: fewest bytes wins
  // every block fits one 16-row item: all caps give the same items, and the one-tile kernel's estimate is the
  // smallest (the wider kernels add a per-item cost), so the loop below would pick 16
  bool small = true;
  for (int b = 0; b < nb && small; ++b) small = (long)blocks[b * 4 + 2] * group <= 16;
  if (small) return 16;
  thread_local std::vector<double> cost;
  thread_local std::vector<double> load;
  const double pos_bytes = 4.0 * head_dim;  // K and V, bf16, one KV head
  int best = ATTN_ROWS;
  double best_t = 1e300, best_span = 1e300;
  for (int R = ATTN_ROWS; R >= 16; R -= 16) {
    cost.clear();
    double bytes = 0.0;
    for (int b = 0; b < nb; ++b) {
      const int pos0 = blocks[b * 4 + 1], T = blocks[b * 4 + 2], rows = T * group;
      for (int row0 = 0; row0 < rows; row0 += R) {
        const int nrows = rows - row0 < R ? rows - row0 : R, nq = (nrows + 15) / 16;
        const long kv_end = (long)pos0 + (row0 + nrows - 1) / group + 1;
        for (long lo = 0; lo < kv_end; lo += split) {
          const long len = (lo + split < kv_end ? lo + split : kv_end) - lo;
          const long steps = (len + ATTN_STEP * ATTN_WAVES - 1) / (ATTN_STEP * ATTN_WAVES);
          const double c = R == 16 ? steps * ATTN_COST_STEP_US
                                   : ATTN_COST_ITEM_US + ATTN_COST_TILE_US * (nq - 1) +
                                         steps * (ATTN_COST_STEP_US + (nq == 3 ? ATTN_COST_STEP3_US : 0.0));
          for (int h = 0; h < n_kv_heads; ++h) cost.push_back(c);
          bytes += (double)len * pos_bytes * n_kv_heads;
        }
      }
    }
    double span = 0.0;
    if ((long)cost.size() <= n_slots) {
      for (double c : cost) span = c > span ? c : span;
    } else {
      std::sort(cost.begin(), cost.end(), [](double a, double b) { return a > b; });
      load.assign(n_slots, 0.0);  // min-heap of slot loads
      for (double c : cost) {
        std::pop_heap(load.begin(), load.end(), std::greater<double>());
        load.back() += c;
        std::push_heap(load.begin(), load.end(), std::greater<double>());
      }
      for (double l : load) span = l > span ? l : span;
    }
    const double bw = bytes / ATTN_COST_BW_BYTES_PER_US;
    const double t = span > bw ? span : bw;
    // equal estimates (bandwidth-bound, same bytes): the shorter makespan, i.e. the faster kernel
    if (t < best_t * (1 - 1e-9) || (t <= best_t * (1 + 1e-9) && span < best_span)) {
      best_t = t;
      best_span = span;
      best = R;
    }
  }
  return best;
}

extern "C" int lsk_attn_rows_cap(const int32_t* blocks, int nb, int group, int split, int n_kv_heads, int head_dim,
                                 int n_slots) {
  LSK_REQUIRE(blocks || nb == 0, LSK_EARG, "lsk_attn_rows_cap: null pointer");
  return rows_cap_for(blocks, nb, group, split, n_kv_heads, head_dim, n_slots);
}

// Static schedule of a plan over n_slots persistent workgroups (one per CU): items are (work, KV head) pairs
// of non-padding works, costed by their KV steps per wave plus a fixed per-item overhead, and dealt longest
// first to the least-loaded slot (ties: lowest slot; equal costs keep plan order).  Output: records
// recs[slot][round][8] (the work record with nrows | kvh << 8 in field 2), each slot's items in processing
// order from round 0, padded with nrows = 0 records up to n_rounds = the largest item count of a slot.
// Which workgroup computes an item never changes its result.
static int schedule_into(const int32_t* works, int n_works, int n_kv_heads, int n_slots, std::vector<int32_t>& recs,
                         int* n_rounds) {
  LSK_REQUIRE(n_works >= 0 && n_kv_heads > 0 && n_kv_heads < (1 << 23) && n_slots > 0, LSK_ESHAPE,
              "lsk_attn_schedule: bad arguments");
  struct It { int id, cost; };
  thread_local std::vector<It> items;
  thread_local std::vector<std::pair<long, int>> heap;
  thread_local std::vector<int> slot_of, count, rank;
  items.clear();
  for (int w = 0; w < n_works; ++w) {
    const int32_t* wp = works + (long)w * 8;
    if (wp[2] <= 0) continue;
    LSK_REQUIRE(wp[2] <= ATTN_ROWS, LSK_ESHAPE, "lsk_attn_schedule: work %d has %d rows", w, wp[2]);
    // cost in tenths of a wave step: the steps (a three-tile item's 1.2x as long), plus the per-item overhead and
    // 1.2 steps per extra column tile (the per-item terms of the rows-per-item estimate, in step units)
    const int steps = (wp[4] - wp[3] + ATTN_STEP * ATTN_WAVES - 1) / (ATTN_STEP * ATTN_WAVES);
    const int nq = (wp[2] + 15) / 16;
    const int cost = steps * (nq == 3 ? 12 : 10) + 20 + 12 * (nq - 1);
    for (int h = 0; h < n_kv_heads; ++h) items.push_back({w * n_kv_heads + h, cost});
  }
  std::stable_sort(items.begin(), items.end(), [](const It& a, const It& b) { return a.cost > b.cost; });
  heap.clear();
  for (int sl = 0; sl < n_slots; ++sl) heap.push_back({0, sl});
  auto cmp = [](const std::pair<long, int>& a, const std::pair<long, int>& b) {
    return a.first > b.first || (a.first == b.first && a.second > b.second);
  };
  std::make_heap(heap.begin(), heap.end(), cmp);
  const int n = (int)items.size();
  slot_of.resize(n);
  rank.resize(n);
  count.assign(n_slots, 0);
  int R = 0;
  for (int i = 0; i < n; ++i) {
    std::pop_heap(heap.begin(), heap.end(), cmp);
    auto& top = heap.back();
    slot_of[i] = top.second;
    rank[i] = count[top.second]++;
    R = count[top.second] > R ? count[top.second] : R;
    top.first += items[i].cost;
    std::push_heap(heap.begin(), heap.end(), cmp);
  }
  recs.assign((size_t)n_slots * R * 8, 0);
  for (int i = 0; i < n; ++i) {
    const int id = items[i].id, w = id / n_kv_heads, h = id - w * n_kv_heads;
    const int32_t* wp = works + (long)w * 8;
    int32_t* rp = recs.data() + ((size_t)slot_of[i] * R + rank[i]) * 8;
    rp[0] = wp[0]; rp[1] = wp[1]; rp[2] = wp[2] | (h << 8); rp[3] = wp[3];
    rp[4] = wp[4]; rp[5] = wp[5]; rp[6] = wp[6]; rp[7] = wp[7];
  }
  *n_rounds = R;
  return 0;
}

// With recs == NULL only n_rounds is computed.
extern "C" int lsk_attn_schedule(const int32_t* works, int n_works, int n_kv_heads, int n_slots, int32_t* recs,
                                 int max_recs, int* n_rounds) {
  LSK_REQUIRE(n_rounds && (works || n_works == 0), LSK_EARG, "lsk_attn_schedule: null pointer");
  thread_local std::vector<int32_t> r;
  int R = 0;
  const int rc = schedule_into(works, n_works, n_kv_heads, n_slots, r, &R);
  if (rc) return rc;
  *n_rounds = R;
  if (recs == nullptr) return 0;
  LSK_REQUIRE((long)n_slots * R <= max_recs, LSK_EWORKSPACE, "lsk_attn_schedule: %ld records > %d",
              (long)n_slots * R, max_recs);
  std::copy(r.begin(), r.end(), recs);
  return 0;
}

// One packed segment's kernel metadata from its blocks in packed order (host only; see include/lsk.h).
extern "C" int lsk_pack_segment(const int64_t* rows, const int64_t* pos0, const int64_t* T, int nb, int group,
                                int split, int n_kv_heads, int head_dim, int n_slots, int bucketing, int max_batch,
                                int max_seq, int rope_len, int32_t* meta, long meta_cap, long* counts) {
  LSK_REQUIRE(counts && (nb == 0 || (rows && pos0 && T)), LSK_EARG, "lsk_pack_segment: null pointer");
  LSK_REQUIRE(nb >= 0 && (bucketing == 0 || bucketing == 1), LSK_EARG, "lsk_pack_segment: bad arguments");
  long N = 0;
  for (int b = 0; b < nb; ++b) {
    LSK_REQUIRE(rows[b] >= 0 && rows[b] < max_batch, LSK_ESHAPE, "block row %ld outside the cache's %d rows",
                (long)rows[b], max_batch);
    LSK_REQUIRE(T[b] >= 1 && pos0[b] >= 0 && pos0[b] + T[b] <= max_seq, LSK_ESHAPE,
                "block positions [%ld, %ld) outside max_seq=%d", (long)pos0[b], (long)(pos0[b] + T[b]), max_seq);
    LSK_REQUIRE(pos0[b] + T[b] <= rope_len, LSK_ESHAPE, "positions beyond the RoPE table");
    N += T[b];
  }
  LSK_REQUIRE(N < (1L << 30), LSK_ESHAPE, "lsk_pack_segment: %ld tokens", N);
  thread_local std::vector<int32_t> blk, works, groups, recs;
  blk.resize((size_t)nb * 4);
  long off = 0;
  for (int b = 0; b < nb; ++b) {
    blk[b * 4 + 0] = (int32_t)off;
    blk[b * 4 + 1] = (int32_t)pos0[b];
    blk[b * 4 + 2] = (int32_t)T[b];
    blk[b * 4 + 3] = (int32_t)rows[b];
    off += T[b];
  }
  int np = 0, R = 0;
  const int cap = rows_cap_for(blk.data(), nb, group, split, n_kv_heads, head_dim, n_slots);
  if (cap < 0) return cap;
  int rc = plan_into(blk.data(), nb, group, split, cap, works, groups, &np);
  if (rc) return rc;
  const int nw = (int)(works.size() / 8), ng = (int)(groups.size() / 8);
  rc = schedule_into(works.data(), nw, n_kv_heads, n_slots, recs, &R);
  if (rc) return rc;
  const long len = 2 * N + 4L * nb + 8L * nw + 8L * ng + (long)recs.size();
  // reference accounting (solutions/packed.py:109-138): buckets = runs of equal T ("exact") or all blocks ("pad")
  long kv_read = 0, kv_padded = 0, kv_gathered = 0, pairs = 0;
  for (int a = 0; a < nb;) {
    int e = a + 1;
    if (bucketing == 0)
      while (e < nb && T[e] == T[a]) ++e;
    else
      e = nb;
    long mx = 0;
    bool contiguous = true;
    for (int j = a; j < e; ++j) {
      mx = pos0[j] + T[j] > mx ? pos0[j] + T[j] : mx;
      kv_read += pos0[j] + T[j];
      contiguous = contiguous && rows[j] == rows[a] + (j - a);
    }
    const long L = std::min((mx + 63) / 64 * 64, (long)max_seq);
    kv_padded += (long)(e - a) * L;
    if (!contiguous) kv_gathered += (long)(e - a) * L;
    a = e;
  }
  for (int b = 0; b < nb; ++b) pairs += T[b] * pos0[b] + T[b] * (T[b] + 1) / 2;
  counts[0] = N; counts[1] = nw; counts[2] = ng; counts[3] = np; counts[4] = R; counts[5] = len;
  counts[6] = kv_read; counts[7] = kv_padded; counts[8] = kv_gathered; counts[9] = pairs; counts[10] = cap;
  if (meta == nullptr) return 0;
  LSK_REQUIRE(len <= meta_cap, LSK_EWORKSPACE, "lsk_pack_segment: %ld metadata words > %ld", len, meta_cap);
  int32_t* o = meta;
  for (int b = 0; b < nb; ++b)
    for (long t = 0; t < T[b]; ++t) *o++ = (int32_t)rows[b];
  for (int b = 0; b < nb; ++b)
    for (long t = 0; t < T[b]; ++t) *o++ = (int32_t)(pos0[b] + t);
  o = std::copy(blk.begin(), blk.end(), o);
  o = std::copy(works.begin(), works.end(), o);
  o = std::copy(groups.begin(), groups.end(), o);
  std::copy(recs.begin(), recs.end(), o);
  return 0;
}

extern "C" size_t lsk_attn_workspace_bytes(int n_parts, int n_kv_heads, int head_dim) {
  // o_part [n_parts][Hkv][ATTN_ROWS][D] fp32, ml_part [n_parts][Hkv][ATTN_ROWS][2] fp32
  const size_t rows = (size_t)n_parts * n_kv_heads * ATTN_ROWS;
  return lsk_align_up(rows * head_dim * sizeof(float), 256) + lsk_align_up(rows * 2 * sizeof(float), 256);
}

extern "C" int lsk_ragged_attn(int dtype, const void* q, const void* kcache, const void* vcache,
                               const int32_t* blocks, const int32_t* works, int n_works, const int32_t* groups,
                               int n_groups, int n_parts, const int32_t* recs, int n_rounds, int n_slots,
                               int rows_cap, void* out,
                               int n_heads, int n_kv_heads, int head_dim, int max_seq, float scale, void* workspace,
                               size_t ws_bytes, void* stream) {
  return lsk_ragged_attn_impl(dtype, q, kcache, vcache, blocks, works, n_works, groups, n_groups, n_parts, recs,
                              n_rounds, n_slots, rows_cap, out, 0, n_heads, n_kv_heads, head_dim, max_seq, scale,
                              workspace, ws_bytes, stream);
}

int lsk_ragged_attn_impl(int dtype, const void* q, const void* kcache, const void* vcache, const int32_t* blocks,
                         const int32_t* works, int n_works, const int32_t* groups, int n_groups, int n_parts,
                         const int32_t* recs, int n_rounds, int n_slots, int rows_cap, void* out, int out_frag,
                         int n_heads, int n_kv_heads, int head_dim, int max_seq, float scale, void* workspace,
                         size_t ws_bytes, void* stream) {
  LSK_REQUIRE(q && kcache && vcache && blocks && works && out, LSK_EARG, "lsk_ragged_attn: null pointer");
  LSK_REQUIRE(!out_frag || (dtype == LSK_DTYPE_BF16 && (n_heads * head_dim) % 32 == 0), LSK_EARG,
              "lsk_ragged_attn: a fragment-major output needs bf16 and n_heads * head_dim %% 32 == 0");
  const int out_nks = out_frag ? n_heads * head_dim / 32 : 0;
  LSK_REQUIRE(dtype != LSK_DTYPE_BF16 || n_works == 0 || (recs && n_rounds > 0 && n_slots > 0), LSK_EARG,
              "lsk_ragged_attn: the bf16 path needs a schedule (lsk_attn_schedule)");
  LSK_REQUIRE(rows_cap > 0 && rows_cap % 16 == 0 && rows_cap <= ATTN_ROWS, LSK_EARG,
              "lsk_ragged_attn: rows_cap %d (the plan's rows per item: 16, 32 or %d)", rows_cap, ATTN_ROWS);
  LSK_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0 && max_seq > 0 && n_works >= 0,
              LSK_ESHAPE, "lsk_ragged_attn: bad shape");
  if (n_works == 0) return 0;
  const int G = n_heads / n_kv_heads;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid(n_works, n_kv_heads);
  if (dtype == LSK_DTYPE_BF16) {
    LSK_REQUIRE(head_dim == 64 || head_dim == 128, LSK_EUNSUPPORTED,
                "lsk_ragged_attn: bf16 head_dim %d (supported: 64, 128)", head_dim);
    LSK_REQUIRE(max_seq % ATTN_TILE == 0, LSK_ESHAPE, "lsk_ragged_attn: max_seq must be a multiple of %d", ATTN_TILE);
    float* o_part = nullptr;
    float* ml_part = nullptr;
    if (n_parts > 0) {
      const size_t need = lsk_attn_workspace_bytes(n_parts, n_kv_heads, head_dim);
      LSK_REQUIRE(workspace != nullptr && ws_bytes >= need && groups != nullptr, LSK_EWORKSPACE,
                  "lsk_ragged_attn: workspace of %zu bytes needed, %zu given", need, ws_bytes);
      const size_t rows = (size_t)n_parts * n_kv_heads * ATTN_ROWS;
      o_part = (float*)workspace;
      ml_part = (float*)((char*)workspace + lsk_align_up(rows * head_dim * sizeof(float), 256));
    }
    const float scale_log2 = scale * 1.4426950408889634f;
    const dim3 pgrid(n_slots);
    // one column tile (items of <= 16 rows): Q in registers; otherwise three tiles with Q staged in LDS
#define LSK_ATTN_LAUNCH(DD, QT)                                                                               \
  attn_bf16_kernel<DD, QT><<<pgrid, 64 * ATTN_WAVES, 0, s>>>((const uint16_t*)q, (const uint16_t*)kcache,     \
                                                              (const uint16_t*)vcache, recs, n_rounds,         \
                                                              (uint16_t*)out, o_part, ml_part, G, n_kv_heads,  \
                                                              max_seq, scale_log2, out_nks)
    if (head_dim == 128) {
      if (rows_cap == 16) LSK_ATTN_LAUNCH(128, 1); else LSK_ATTN_LAUNCH(128, ATTN_QT);
    } else {
      if (rows_cap == 16) LSK_ATTN_LAUNCH(64, 1); else LSK_ATTN_LAUNCH(64, ATTN_QT);
    }
#undef LSK_ATTN_LAUNCH
    int rc = lsk_check_launch("lsk_ragged_attn");
    if (rc) return rc;
    if (n_groups > 0) {
      dim3 cg(n_groups, n_kv_heads);
      if (head_dim == 128)
        attn_combine_kernel<uint16_t, 128><<<cg, 256, 0, s>>>(blocks, groups, o_part, ml_part, (uint16_t*)out, G,
                                                               n_kv_heads, out_nks);
      else
        attn_combine_kernel<uint16_t, 64><<<cg, 256, 0, s>>>(blocks, groups, o_part, ml_part, (uint16_t*)out, G,
                                                              n_kv_heads, out_nks);
      return lsk_check_launch("lsk_ragged_attn(combine)");
    }
    return 0;
  }
  if (dtype == LSK_DTYPE_F32) {
    LSK_REQUIRE(n_parts == 0, LSK_EARG, "lsk_ragged_attn: the fp32 path takes unsplit plans");
    switch (head_dim) {
      case 16: attn_f32_kernel<16><<<grid, 256, 0, s>>>((const float*)q, (const float*)kcache, (const float*)vcache, works, (float*)out, G, n_kv_heads, max_seq, scale); break;
      case 32: attn_f32_kernel<32><<<grid, 256, 0, s>>>((const float*)q, (const float*)kcache, (const float*)vcache, works, (float*)out, G, n_kv_heads, max_seq, scale); break;
      case 64: attn_f32_kernel<64><<<grid, 256, 0, s>>>((const float*)q, (const float*)kcache, (const float*)vcache, works, (float*)out, G, n_kv_heads, max_seq, scale); break;
      case 128: attn_f32_kernel<128><<<grid, 256, 0, s>>>((const float*)q, (const float*)kcache, (const float*)vcache, works, (float*)out, G, n_kv_heads, max_seq, scale); break;
      default: LSK_REQUIRE(false, LSK_EUNSUPPORTED, "lsk_ragged_attn: fp32 head_dim %d", head_dim);
    }
    return lsk_check_launch("lsk_ragged_attn(f32)");
  }
  LSK_REQUIRE(false, LSK_EUNSUPPORTED, "lsk_ragged_attn: dtype %d", dtype);
  return LSK_EUNSUPPORTED;
}

// ----------------------------------------------------------------------------- allocation-free entry point
// lsk_ragged_attn_static keeps the split partials in this file-scope device array instead of a caller workspace,
// for callers that cannot allocate device memory.  Each GPU the library runs on holds its own copy (at its own
// address) until the process ends.  In host code `scratch` names the symbol only: its device address comes from
// hipGetSymbolAddress with the device current, looked up once per device and kept in scratch_dev; kernels are
// always given that address, never the array's name.  Every call on a GPU shares that GPU's array: calls that
// overlap on one GPU (other streams, other host threads) race on it.  The partial slots need no clearing: every
// slot a combine group reads is written by its work item in the same call before the combine launch reads it.
static __device__ __align__(256) unsigned char scratch[LSK_ATTN_SCRATCH_BYTES];

#define LSK_MAX_DEVICES 64
static std::mutex scratch_mu;
static void* scratch_dev[LSK_MAX_DEVICES];

// Device address of the current device's scratch array (looked up on the first call per device).
static int attn_scratch_address(void** out, hipStream_t stream) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  LSK_REQUIRE(e == hipSuccess, (int)e, "lsk_ragged_attn_static: hipGetDevice: %s", hipGetErrorString(e));
  LSK_REQUIRE(dev >= 0 && dev < LSK_MAX_DEVICES, LSK_EUNSUPPORTED, "lsk_ragged_attn_static: device %d", dev);
  if (stream != nullptr) {
    int sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    LSK_REQUIRE(e == hipSuccess, (int)e, "lsk_ragged_attn_static: hipStreamGetDevice: %s", hipGetErrorString(e));
    LSK_REQUIRE(sdev == dev, LSK_EARG,
                "lsk_ragged_attn_static: the stream belongs to device %d but device %d is current (the scratch "
                "array used is the current device's)", sdev, dev);
  }
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_dev[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    LSK_REQUIRE(e == hipSuccess && ptr != nullptr, e != hipSuccess ? (int)e : LSK_EUNSUPPORTED,
                "lsk_ragged_attn_static: hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    scratch_dev[dev] = ptr;
  }
  *out = scratch_dev[dev];
  return 0;
}

extern "C" size_t lsk_ragged_attn_static_scratch_bytes(void) { return LSK_ATTN_SCRATCH_BYTES; }

extern "C" int lsk_ragged_attn_static(int dtype, const void* q, const void* kcache, const void* vcache,
                                      const int32_t* blocks, const int32_t* works, int n_works,
                                      const int32_t* groups, int n_groups, int n_parts, const int32_t* recs,
                                      int n_rounds, int n_slots, int rows_cap, void* out, int n_heads,
                                      int n_kv_heads, int head_dim, int max_seq, float scale, void* stream) {
  LSK_REQUIRE(n_parts >= 0 && n_kv_heads > 0 && head_dim > 0, LSK_ESHAPE, "lsk_ragged_attn_static: bad shape");
  const size_t need = n_parts > 0 ? lsk_attn_workspace_bytes(n_parts, n_kv_heads, head_dim) : 0;
  LSK_REQUIRE(need <= LSK_ATTN_SCRATCH_BYTES, LSK_EWORKSPACE,
              "lsk_ragged_attn_static: %d split partial slots x %d KV heads need %zu bytes of scratch, more than the "
              "%u-byte static array; use lsk_ragged_attn with a workspace", n_parts, n_kv_heads, need,
              (unsigned)LSK_ATTN_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = attn_scratch_address(&ws, (hipStream_t)stream);
    if (rc) return rc;
  }
  return lsk_ragged_attn_impl(dtype, q, kcache, vcache, blocks, works, n_works, groups, n_groups, n_parts, recs,
                              n_rounds, n_slots, rows_cap, out, 0, n_heads, n_kv_heads, head_dim, max_seq, scale, ws,
                              need, stream);
}
