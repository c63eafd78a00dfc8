// Elementwise / data-movement kernels of the packed forward and its step glue:
//   RMSNorm, RoPE + KV append, embedding gather, row copies, argmax, greedy acceptance, rollback.
//
// Compiled with -ffp-contract=off: every float expression below is evaluated with one rounding
// per operation, in the order written, so the rounding points match the reference's eager ops
// (common/model.py:148-156, solutions/packed.py:175-181) exactly.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "lsk_common.h"
#include "../include/lsk.h"

// ----------------------------------------------------------------------------- errors

static thread_local char g_err[512] = "";

void lsk_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int lsk_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    lsk_set_error("%s: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

extern "C" const char* lsk_last_error(void) { return g_err; }
extern "C" int lsk_abi_version(void) { return LSK_ABI_VERSION; }

// ----------------------------------------------------------------------------- reductions

// Sum over the 64 lanes of a wavefront with a fixed xor tree (same order for every row).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ----------------------------------------------------------------------------- RMSNorm
// out = w * (x * rsqrt(mean(x^2) + eps)).to(dtype)        (common/model.py:153-156)
// One 256-thread workgroup per row.  The sum of squares is accumulated per thread over a
// fixed stride, reduced per wave by an xor tree and across the four waves in index order,
// so a row's result never depends on the other rows of the call.
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                      T* __restrict__ out, int dim, float eps, long ldx,
                                                      long ldo) {
  const int row = blockIdx.x;
  const T* xr = x + (long)row * ldx;
  T* orow = out + (long)row * ldo;
  float ss = 0.f;
  for (int j = threadIdx.x; j < dim; j += 256) {
    float v = Elem<T>::ld(xr + j);
    ss += v * v;
  }
  ss = wave_sum(ss);
  __shared__ float red[4];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = ss;
  __syncthreads();
  const float tot = ((red[0] + red[1]) + red[2]) + red[3];
  const float mean = tot / (float)dim;
  const float r = 1.0f / sqrtf(mean + eps);
  for (int j = threadIdx.x; j < dim; j += 256) {
    float n = Elem<T>::round(Elem<T>::ld(xr + j) * r);
    Elem<T>::st(orow + j, Elem<T>::ld(w + j) * n);
  }
}

extern "C" int lsk_rmsnorm(int dtype, const void* x, const void* w, void* out, int n_rows, int dim, float eps,
                           long ldx, long ldo, void* stream) {
  LSK_REQUIRE(x && w && out, LSK_EARG, "lsk_rmsnorm: null pointer");
  LSK_REQUIRE(n_rows >= 0 && dim > 0 && ldx >= dim && ldo >= dim, LSK_ESHAPE,
              "lsk_rmsnorm: bad shape n_rows=%d dim=%d ldx=%ld ldo=%ld", n_rows, dim, ldx, ldo);
  if (n_rows == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == LSK_DTYPE_BF16)
    rmsnorm_kernel<uint16_t><<<n_rows, 256, 0, s>>>((const uint16_t*)x, (const uint16_t*)w, (uint16_t*)out, dim,
                                                    eps, ldx, ldo);
  else if (dtype == LSK_DTYPE_F32)
    rmsnorm_kernel<float><<<n_rows, 256, 0, s>>>((const float*)x, (const float*)w, (float*)out, dim, eps, ldx, ldo);
  else
    LSK_REQUIRE(false, LSK_EUNSUPPORTED, "lsk_rmsnorm: dtype %d", dtype);
  return lsk_check_launch("lsk_rmsnorm");
}

// ----------------------------------------------------------------------------- RoPE + KV append
// qkv [N, (Hq + 2 Hkv) D] = [q | k | v] per token (solutions/packed.py:175-176).
// q heads:  q_out[t, h]                       = rope(q)   (common/model.py:148-150)
// k heads:  kcache[row_t, h, pos_t]           = rope(k)   (solutions/packed.py:180)
// v heads:  vcache[row_t, h, pos_t]           = v         (solutions/packed.py:181)
// rope(x)[j]       = x[j] * c[j]       + (-x[j+D/2]) * s[j]
// rope(x)[j + D/2] = x[j+D/2] * c[j+D/2] + x[j] * s[j+D/2]
// with c, s = the fp32 tables at pos_t stored to the model dtype first (solutions/packed.py:106-107)
// and one dtype rounding after each multiply and after the add.
template <typename T>
__global__ __launch_bounds__(256) void rope_append_kernel(const T* __restrict__ qkv, T* __restrict__ q_out,
                                                          T* __restrict__ kc, T* __restrict__ vc,
                                                          const float* __restrict__ cos_tab,
                                                          const float* __restrict__ sin_tab,
                                                          const int32_t* __restrict__ rows,
                                                          const int32_t* __restrict__ pos, int Hq, int Hkv, int D,
                                                          int max_batch, int max_seq, int tab_len) {
  const int t = blockIdx.x;
  const int row = rows[t], p = pos[t];
  if (row < 0 || row >= max_batch || p < 0 || p >= max_seq || p >= tab_len) return;  // host validates too
  const int half = D >> 1;
  const int width = (Hq + 2 * Hkv) * D;
  const T* src = qkv + (long)t * width;
  const float* ct = cos_tab + (long)p * D;
  const float* st = sin_tab + (long)p * D;
  // rotated heads: Hq + Hkv heads x half pairs
  const int n_pairs = (Hq + Hkv) * half;
  for (int e = threadIdx.x; e < n_pairs; e += blockDim.x) {
    const int h = e / half, j = e - h * half;
    const T* xh = src + h * D;
    const float x1 = Elem<T>::ld(xh + j), x2 = Elem<T>::ld(xh + j + half);
    const float c1 = Elem<T>::round(ct[j]), c2 = Elem<T>::round(ct[j + half]);
    const float s1 = Elem<T>::round(st[j]), s2 = Elem<T>::round(st[j + half]);
    const float a1 = Elem<T>::round(x1 * c1), b1 = Elem<T>::round((-x2) * s1);
    const float a2 = Elem<T>::round(x2 * c2), b2 = Elem<T>::round(x1 * s2);
    const float o1 = a1 + b1, o2 = a2 + b2;
    T* dst;
    if (h < Hq) {
      dst = q_out + ((long)t * Hq + h) * D;
    } else {
      const int hk = h - Hq;
      dst = kc + (((long)row * Hkv + hk) * max_seq + p) * D;
    }
    Elem<T>::st(dst + j, o1);
    Elem<T>::st(dst + j + half, o2);
  }
  // v heads: plain copy into the cache
  const T* vsrc = src + (Hq + Hkv) * D;
  for (int e = threadIdx.x; e < Hkv * D; e += blockDim.x) {
    const int hk = e / D, d = e - hk * D;
    vc[(((long)row * Hkv + hk) * max_seq + p) * D + d] = vsrc[e];
  }
}

extern "C" int lsk_rope_append(int dtype, const void* qkv, void* q_out, void* kcache, void* vcache,
                               const float* cos_tab, const float* sin_tab, int tab_len, const int32_t* rows,
                               const int32_t* pos, int n_tokens, int n_heads, int n_kv_heads, int head_dim,
                               int max_batch, int max_seq, void* stream) {
  LSK_REQUIRE(qkv && q_out && kcache && vcache && cos_tab && sin_tab && rows && pos, LSK_EARG,
              "lsk_rope_append: null pointer");
  LSK_REQUIRE(n_tokens >= 0 && n_heads > 0 && n_kv_heads > 0 && head_dim > 0 && (head_dim % 2) == 0 &&
                  n_heads % n_kv_heads == 0 && max_batch > 0 && max_seq > 0 && tab_len > 0,
              LSK_ESHAPE, "lsk_rope_append: bad shape");
  if (n_tokens == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == LSK_DTYPE_BF16)
    rope_append_kernel<uint16_t><<<n_tokens, 256, 0, s>>>(
        (const uint16_t*)qkv, (uint16_t*)q_out, (uint16_t*)kcache, (uint16_t*)vcache, cos_tab, sin_tab, rows, pos,
        n_heads, n_kv_heads, head_dim, max_batch, max_seq, tab_len);
  else if (dtype == LSK_DTYPE_F32)
    rope_append_kernel<float><<<n_tokens, 256, 0, s>>>((const float*)qkv, (float*)q_out, (float*)kcache,
                                                       (float*)vcache, cos_tab, sin_tab, rows, pos, n_heads,
                                                       n_kv_heads, head_dim, max_batch, max_seq, tab_len);
  else
    LSK_REQUIRE(false, LSK_EUNSUPPORTED, "lsk_rope_append: dtype %d", dtype);
  return lsk_check_launch("lsk_rope_append");
}

// Plain KV append (no RoPE): kcache[row_t, h, pos_t] = k[t, h]; vcache likewise.
// Used for inputs whose RoPE is already applied (solutions/packed.py:180-181 on its own).
template <typename T>
__global__ __launch_bounds__(256) void kv_append_kernel(const T* __restrict__ k, const T* __restrict__ v,
                                                        T* __restrict__ kc, T* __restrict__ vc,
                                                        const int32_t* __restrict__ rows,
                                                        const int32_t* __restrict__ pos, int Hkv, int D,
                                                        int max_batch, int max_seq) {
  const int t = blockIdx.x;
  const int row = rows[t], p = pos[t];
  if (row < 0 || row >= max_batch || p < 0 || p >= max_seq) return;
  for (int e = threadIdx.x; e < Hkv * D; e += blockDim.x) {
    const int hk = e / D, d = e - hk * D;
    const long off = (((long)row * Hkv + hk) * max_seq + p) * D + d;
    kc[off] = k[(long)t * Hkv * D + e];
    vc[off] = v[(long)t * Hkv * D + e];
  }
}

extern "C" int lsk_kv_append(int dtype, const void* k, const void* v, void* kcache, void* vcache, const int32_t* rows,
                             const int32_t* pos, int n_tokens, int n_kv_heads, int head_dim, int max_batch,
                             int max_seq, void* stream) {
  LSK_REQUIRE(k && v && kcache && vcache && rows && pos, LSK_EARG, "lsk_kv_append: null pointer");
  LSK_REQUIRE(n_tokens >= 0 && n_kv_heads > 0 && head_dim > 0 && max_batch > 0 && max_seq > 0, LSK_ESHAPE,
              "lsk_kv_append: bad shape");
  if (n_tokens == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == LSK_DTYPE_BF16)
    kv_append_kernel<uint16_t><<<n_tokens, 256, 0, s>>>((const uint16_t*)k, (const uint16_t*)v, (uint16_t*)kcache,
                                                        (uint16_t*)vcache, rows, pos, n_kv_heads, head_dim,
                                                        max_batch, max_seq);
  else if (dtype == LSK_DTYPE_F32)
    kv_append_kernel<float><<<n_tokens, 256, 0, s>>>((const float*)k, (const float*)v, (float*)kcache,
                                                     (float*)vcache, rows, pos, n_kv_heads, head_dim, max_batch,
                                                     max_seq);
  else
    LSK_REQUIRE(false, LSK_EUNSUPPORTED, "lsk_kv_append: dtype %d", dtype);
  return lsk_check_launch("lsk_kv_append");
}

// ----------------------------------------------------------------------------- embedding
// out[t] = table[id_t], id_t = sel[t] >= 0 ? seq_buf[sel[t]] : alt[t]
// (solutions/engine.py:345-346 id assembly + common/model.py:325-326 F.embedding).
// sel == NULL -> id_t = alt[t].  An id outside [0, vocab) yields a zero row (never read out of bounds).
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t* __restrict__ table, const int64_t* __restrict__ seq_buf,
                                                    const int64_t* __restrict__ sel, const int64_t* __restrict__ alt,
                                                    uint8_t* __restrict__ out, long row_bytes, long vocab,
                                                    long seq_len) {
  const int t = blockIdx.x;
  long id;
  if (sel != nullptr && sel[t] >= 0) {
    const long si = sel[t];
    id = (si < seq_len) ? seq_buf[si] : -1;
  } else {
    id = alt[t];
  }
  uint8_t* dst = out + (long)t * row_bytes;
  if (id < 0 || id >= vocab) {
    for (long b = threadIdx.x; b < row_bytes / 4; b += blockDim.x) ((uint32_t*)dst)[b] = 0u;
    return;
  }
  const uint8_t* src = table + id * row_bytes;
  if ((row_bytes & 15) == 0) {
    for (long b = threadIdx.x; b < row_bytes / 16; b += blockDim.x) ((uint4*)dst)[b] = ((const uint4*)src)[b];
  } else {
    for (long b = threadIdx.x; b < row_bytes / 4; b += blockDim.x) ((uint32_t*)dst)[b] = ((const uint32_t*)src)[b];
  }
}

extern "C" int lsk_embed(const void* table, long vocab, long row_bytes, const int64_t* seq_buf, long seq_len,
                         const int64_t* sel, const int64_t* alt, void* out, int n_tokens, void* stream) {
  LSK_REQUIRE(table && out && alt, LSK_EARG, "lsk_embed: null pointer");
  LSK_REQUIRE(sel == nullptr || seq_buf != nullptr, LSK_EARG, "lsk_embed: sel without seq_buf");
  LSK_REQUIRE(n_tokens >= 0 && vocab > 0 && row_bytes > 0 && (row_bytes % 4) == 0, LSK_ESHAPE,
              "lsk_embed: bad shape");
  if (n_tokens == 0) return 0;
  embed_kernel<<<n_tokens, 256, 0, (hipStream_t)stream>>>((const uint8_t*)table, seq_buf, sel, alt, (uint8_t*)out,
                                                           row_bytes, vocab, seq_len);
  return lsk_check_launch("lsk_embed");
}

// ----------------------------------------------------------------------------- row copies
// dst[dst_idx[i]] = src[src_idx[i]] for i < n (NULL index = identity); rows of row_bytes bytes.
// Indices outside [0, n_dst) / [0, n_src) are skipped.  (solutions/engine.py:349-350, 453-455)
__global__ __launch_bounds__(256) void copy_rows_kernel(uint8_t* __restrict__ dst, const int64_t* __restrict__ dst_idx,
                                                        const uint8_t* __restrict__ src,
                                                        const int64_t* __restrict__ src_idx, long row_bytes,
                                                        long n_dst, long n_src) {
  const long i = blockIdx.x;
  const long di = dst_idx ? dst_idx[i] : i;
  const long si = src_idx ? src_idx[i] : i;
  if (di < 0 || di >= n_dst || si < 0 || si >= n_src) return;
  uint8_t* d = dst + di * row_bytes;
  const uint8_t* s = src + si * row_bytes;
  if ((row_bytes & 15) == 0) {
    for (long b = threadIdx.x; b < row_bytes / 16; b += blockDim.x) ((uint4*)d)[b] = ((const uint4*)s)[b];
  } else {
    for (long b = threadIdx.x; b < row_bytes / 2; b += blockDim.x) ((uint16_t*)d)[b] = ((const uint16_t*)s)[b];
  }
}

extern "C" int lsk_copy_rows(void* dst, const int64_t* dst_idx, long n_dst, const void* src, const int64_t* src_idx,
                             long n_src, long row_bytes, int n, void* stream) {
  LSK_REQUIRE(dst && src, LSK_EARG, "lsk_copy_rows: null pointer");
  LSK_REQUIRE(n >= 0 && row_bytes > 0 && (row_bytes % 2) == 0, LSK_ESHAPE, "lsk_copy_rows: bad shape");
  if (n == 0) return 0;
  copy_rows_kernel<<<n, 256, 0, (hipStream_t)stream>>>((uint8_t*)dst, dst_idx, (const uint8_t*)src, src_idx, row_bytes,
                                                        n_dst, n_src);
  return lsk_check_launch("lsk_copy_rows");
}

// ----------------------------------------------------------------------------- argmax
// Greedy pick over the dtype-rounded logits of each row, first index on ties
// (torch.argmax semantics; solutions/engine.py:227,255,352,463,478).
// out[dst_idx ? dst_idx[m] : m] = argmax(logits[m, :V]).
template <typename T>
__global__ __launch_bounds__(256) void argmax_kernel(const T* __restrict__ logits, long ld, int V,
                                                     int64_t* __restrict__ out, const int64_t* __restrict__ dst_idx) {
  const int m = blockIdx.x;
  const T* r = logits + (long)m * ld;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int j = threadIdx.x; j < V; j += 256) {
    const float v = Elem<T>::ld(r + j);
    if (v > best || (bi == 0x7fffffff)) {  // first visited element seeds the thread's best
      if (v > best || bi == 0x7fffffff) {
        best = v;
        bi = j;
      }
    }
  }
  // tie-aware reduction: larger value wins, equal values keep the smaller index
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > best || (ov == best && oi < bi)) {
      best = ov;
      bi = oi;
    }
  }
  __shared__ float sv[4];
  __shared__ int si[4];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sv[0];
    int i = si[0];
    for (int w = 1; w < 4; ++w)
      if (sv[w] > b || (sv[w] == b && si[w] < i)) {
        b = sv[w];
        i = si[w];
      }
    out[dst_idx ? dst_idx[m] : m] = (int64_t)i;
  }
}

extern "C" int lsk_argmax(int dtype, const void* logits, long ld, int n_rows, int vocab, int64_t* out,
                          const int64_t* dst_idx, void* stream) {
  LSK_REQUIRE(logits && out, LSK_EARG, "lsk_argmax: null pointer");
  LSK_REQUIRE(n_rows >= 0 && vocab > 0 && ld >= vocab, LSK_ESHAPE, "lsk_argmax: bad shape");
  if (n_rows == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == LSK_DTYPE_BF16)
    argmax_kernel<uint16_t><<<n_rows, 256, 0, s>>>((const uint16_t*)logits, ld, vocab, out, dst_idx);
  else if (dtype == LSK_DTYPE_F32)
    argmax_kernel<float><<<n_rows, 256, 0, s>>>((const float*)logits, ld, vocab, out, dst_idx);
  else
    LSK_REQUIRE(false, LSK_EUNSUPPORTED, "lsk_argmax: dtype %d", dtype);
  return lsk_check_launch("lsk_argmax");
}

// ----------------------------------------------------------------------------- greedy acceptance
// One verifier j: slot i_j, its T_j = d_j + 1 verify tokens at Yv[start_j .. start_j + T_j).
// draft(jj) = seq_buf[i*Dm1 + jj + 1] for jj < T-1, -1 for the last token (always a mismatch), so
// acc = min{jj : Yv[start+jj] != draft(jj)} <= d                       (solutions/engine.py:461-476)
// forced (optional, per verifier, -1 = natural): acc = min(forced, d), and the committed tokens are
// the drafts of positions < acc followed by Yv[start + acc] (the tokens whose KV the deep segment
// wrote).  Outputs: acc_out[j]; y_out[start + jj] = committed/verified token jj; seq_buf[i*Dm1] =
// the token at jj = acc (new last committed token); kv_len[i] += acc + 1 when kv_len != NULL.
__global__ void greedy_accept_kernel(const int64_t* __restrict__ Yv, int64_t* __restrict__ seq_buf, int Dm1,
                                     const int32_t* __restrict__ slots, const int32_t* __restrict__ starts,
                                     const int32_t* __restrict__ Ts, const int32_t* __restrict__ forced, int nv,
                                     int64_t* __restrict__ acc_out, int64_t* __restrict__ y_out,
                                     int64_t* __restrict__ kv_len) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= nv) return;
  const int i = slots[j], s = starts[j], T = Ts[j];
  const int64_t* row = seq_buf + (long)i * Dm1;
  int acc = T - 1;
  for (int jj = 0; jj < T - 1; ++jj) {
    if (Yv[s + jj] != row[jj + 1]) {
      acc = jj;
      break;
    }
  }
  const bool force = forced != nullptr && forced[j] >= 0;
  if (force) acc = min(forced[j], T - 1);
  for (int jj = 0; jj < T; ++jj) {
    int64_t y = Yv[s + jj];
    if (force && jj < acc) y = row[jj + 1];
    y_out[s + jj] = y;
  }
  const int64_t last = Yv[s + acc];
  acc_out[j] = acc;
  seq_buf[(long)i * Dm1] = last;
  if (kv_len) kv_len[i] += acc + 1;
}

extern "C" int lsk_greedy_accept(const int64_t* Yv, int64_t* seq_buf, int Dm1, const int32_t* slots,
                                 const int32_t* starts, const int32_t* Ts, const int32_t* forced, int nv,
                                 int64_t* acc_out, int64_t* y_out, int64_t* kv_len, void* stream) {
  LSK_REQUIRE(Yv && seq_buf && slots && starts && Ts && acc_out && y_out, LSK_EARG,
              "lsk_greedy_accept: null pointer");
  LSK_REQUIRE(nv >= 0 && Dm1 > 0, LSK_ESHAPE, "lsk_greedy_accept: bad shape");
  if (nv == 0) return 0;
  greedy_accept_kernel<<<(nv + 63) / 64, 64, 0, (hipStream_t)stream>>>(Yv, seq_buf, Dm1, slots, starts, Ts, forced,
                                                                        nv, acc_out, y_out, kv_len);
  return lsk_check_launch("lsk_greedy_accept");
}

// ----------------------------------------------------------------------------- rollback
// Pointer rollback (solutions/engine.py:12-14, 381-384): the committed length of slot i becomes
// kv_len[i] + acc_j + 1; the KV of the rejected suffix stays where it is (never read: a query reads
// positions <= its own) and is overwritten by the next round.  No KV is moved.
__global__ void kv_rollback_kernel(int64_t* __restrict__ kv_len, const int32_t* __restrict__ slots,
                                   const int64_t* __restrict__ acc, int nv) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j < nv) kv_len[slots[j]] += acc[j] + 1;
}

extern "C" int lsk_kv_rollback(int64_t* kv_len, const int32_t* slots, const int64_t* accepted, int nv, void* stream) {
  LSK_REQUIRE(kv_len && slots && accepted, LSK_EARG, "lsk_kv_rollback: null pointer");
  LSK_REQUIRE(nv >= 0, LSK_ESHAPE, "lsk_kv_rollback: bad shape");
  if (nv == 0) return 0;
  kv_rollback_kernel<<<(nv + 63) / 64, 64, 0, (hipStream_t)stream>>>(kv_len, slots, accepted, nv);
  return lsk_check_launch("lsk_kv_rollback");
}
