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

// ----------------------------------------------------------------------------- RMSNorm (+ residual add)
// x_new = rnd(x + rnd(sum_s P[s]))   (x + F.linear(...) with the GEMM's K-slice partials, s in order;
//                                     KS = 0: x_new = x)
// out   = w * (x_new * rsqrt(mean(x_new^2) + eps)).to(dtype)      (common/model.py:153-156)
// One workgroup per row: NW waves, EPT consecutive elements per thread per pass (pass p, thread t: elements
// (p * 64 NW + t) EPT .. + EPT - 1), NP passes.  The sum of squares is accumulated per thread in element order,
// reduced per wave by an xor tree and across the waves in index order, so a row's result never depends on the
// other rows of the call.  fp32: 4 waves x 8 elements (the order the fp32 oracle restates); bf16: 8 waves x 4
// elements, twice the waves streaming the row (a row of 4096 with four fp32 partials: 4.6 -> 3.6 us per launch
// at 16-48 rows, graph-timed on MI355X).  The pass count, the partial count and which outputs exist are
// template arguments, so every load of a row is issued before the first add.
template <typename T, int N>
struct VecN;
template <>
struct VecN<uint16_t, 4> {
  static __device__ __forceinline__ void ld(const uint16_t* p, float* v) {
    const uint2 u = *(const uint2*)p;
    v[0] = __uint_as_float(u.x << 16);
    v[1] = __uint_as_float(u.x & 0xffff0000u);
    v[2] = __uint_as_float(u.y << 16);
    v[3] = __uint_as_float(u.y & 0xffff0000u);
  }
  static __device__ __forceinline__ void st(uint16_t* p, const float* v) {
    uint2 u;
    u.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
    u.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
    *(uint2*)p = u;
  }
};
template <>
struct VecN<float, 4> {
  static __device__ __forceinline__ void ld(const float* p, float* v) {
    const float4 a = *(const float4*)p;
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  }
  static __device__ __forceinline__ void st(float* p, const float* v) { *(float4*)p = make_float4(v[0], v[1], v[2], v[3]); }
};
template <typename T>
struct VecN<T, 8> {
  static __device__ __forceinline__ void ld(const T* p, float* v) {
    VecN<T, 4>::ld(p, v);
    VecN<T, 4>::ld(p + 4, v + 4);
  }
  static __device__ __forceinline__ void st(T* p, const float* v) {
    VecN<T, 4>::st(p, v);
    VecN<T, 4>::st(p + 4, v + 4);
  }
};

template <typename T> struct NormShape;
template <> struct NormShape<float> { static constexpr int NW = 4, EPT = 8; };
template <> struct NormShape<uint16_t> { static constexpr int NW = 8, EPT = 4; };
#define NORM_PASS_ELEMS 2048  // 64 NW EPT for both shapes
#define NORM_MAX_DIM 8192     // 4 passes

// KSC: the number of K-slice partials (0: none), or -1 for a run-time count KS.  XO / NO: x_out / out are written.
// x and x_out may be the same rows (the layer runner updates the residual stream in place), so neither is
// declared __restrict__; every thread reads its elements of a row before it writes them.
template <typename T, int KSC, int NP, bool XO, bool NO>
__global__ __launch_bounds__(64 * NormShape<T>::NW) void add_rmsnorm_kernel(
    const T* x, long ldx, const float* __restrict__ P, int KS, long pstride, const T* __restrict__ w, T* x_out,
    long ldxo, T* __restrict__ out, long ldo, int out_nks, int dim, float eps) {
  constexpr int NW = NormShape<T>::NW, EPT = NormShape<T>::EPT, NTH = 64 * NW;
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  float v[NP][EPT], wv[NP][EPT];
  float ss = 0.f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int j = (p * NTH + tid) * EPT;
    if (j < dim) {
      if constexpr (NO) VecN<T, EPT>::ld(w + j, wv[p]);  // issued with the row's loads: no second round trip
      VecN<T, EPT>::ld(x + (long)row * ldx + j, v[p]);
      if constexpr (KSC != 0) {
        float acc[EPT];
        const float* pr = P + (long)row * dim + j;
        if constexpr (KSC > 0) {
          float pv[KSC][EPT];
#pragma unroll
          for (int s2 = 0; s2 < KSC; ++s2) VecN<float, EPT>::ld(pr + s2 * pstride, pv[s2]);
#pragma unroll
          for (int i = 0; i < EPT; ++i) acc[i] = pv[0][i];
#pragma unroll
          for (int s2 = 1; s2 < KSC; ++s2)
#pragma unroll
            for (int i = 0; i < EPT; ++i) acc[i] = acc[i] + pv[s2][i];
        } else {
          VecN<float, EPT>::ld(pr, acc);
          for (int s2 = 1; s2 < KS; ++s2) {
            float pv[EPT];
            VecN<float, EPT>::ld(pr + s2 * pstride, pv);
#pragma unroll
            for (int i = 0; i < EPT; ++i) acc[i] = acc[i] + pv[i];
          }
        }
#pragma unroll
        for (int i = 0; i < EPT; ++i) v[p][i] = Elem<T>::round(v[p][i] + Elem<T>::round(acc[i]));
      }
      if constexpr (XO) VecN<T, EPT>::st(x_out + (long)row * ldxo + j, v[p]);  // x_new (= x when KS == 0)
#pragma unroll
      for (int i = 0; i < EPT; ++i) ss += v[p][i] * v[p][i];
    }
  }
  if constexpr (NO) {
    ss = wave_sum(ss);
    __shared__ float red[NW];
    const int wave = tid >> 6;
    if ((tid & 63) == 0) red[wave] = ss;
    __syncthreads();
    float tot = red[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) tot = tot + red[i];
    const float mean = tot / (float)dim;
    const float r = 1.0f / sqrtf(mean + eps);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int j = (p * NTH + tid) * EPT;
      if (j < dim) {
        float o[EPT];
#pragma unroll
        for (int i = 0; i < EPT; ++i) o[i] = wv[p][i] * Elem<T>::round(v[p][i] * r);
        // out_nks > 0: fragment-major output (EPT elements at j stay inside one 16-byte slice of 8)
        VecN<T, EPT>::st(out + (out_nks > 0 ? lsk_frag_off(row, j, out_nks) : (long)row * ldo + j), o);
      }
    }
  }
}

template <typename T, int KSC, int NP>
static void launch_add_rmsnorm_np(const void* x, long ldx, const float* P, int KS, long pstride, const void* w,
                                  void* x_out, long ldxo, void* out, long ldo, int out_nks, int n_rows, int dim,
                                  float eps, hipStream_t s) {
  const dim3 grid(n_rows), block(64 * NormShape<T>::NW);
  if (x_out == nullptr && out == nullptr) return;  // nothing to write
#define LSK_NORM_LAUNCH(XO_, NO_)                                                                                   \
  add_rmsnorm_kernel<T, KSC, NP, XO_, NO_><<<grid, block, 0, s>>>((const T*)x, ldx, P, KS, pstride, (const T*)w,  \
                                                                  (T*)x_out, ldxo, (T*)out, ldo, out_nks, dim, eps)
  if (x_out != nullptr && out != nullptr) LSK_NORM_LAUNCH(true, true);
  else if (out != nullptr) LSK_NORM_LAUNCH(false, true);
  else LSK_NORM_LAUNCH(true, false);
#undef LSK_NORM_LAUNCH
}

template <typename T, int KSC>
static void launch_add_rmsnorm_ks(const void* x, long ldx, const float* P, int KS, long pstride, const void* w,
                                  void* x_out, long ldxo, void* out, long ldo, int out_nks, int n_rows, int dim,
                                  float eps, hipStream_t s) {
  const int np = (dim + NORM_PASS_ELEMS - 1) / NORM_PASS_ELEMS;
  if (np == 1) launch_add_rmsnorm_np<T, KSC, 1>(x, ldx, P, KS, pstride, w, x_out, ldxo, out, ldo, out_nks, n_rows, dim, eps, s);
  else if (np == 2) launch_add_rmsnorm_np<T, KSC, 2>(x, ldx, P, KS, pstride, w, x_out, ldxo, out, ldo, out_nks, n_rows, dim, eps, s);
  else launch_add_rmsnorm_np<T, KSC, 4>(x, ldx, P, KS, pstride, w, x_out, ldxo, out, ldo, out_nks, n_rows, dim, eps, s);
}

template <typename T>
static void launch_add_rmsnorm(const void* x, long ldx, const float* P, int KS, long pstride, const void* w,
                               void* x_out, long ldxo, void* out, long ldo, int out_nks, int n_rows, int dim,
                               float eps, hipStream_t s) {
#define LSK_NORM_KS(KSC_) \
  launch_add_rmsnorm_ks<T, KSC_>(x, ldx, P, KS, pstride, w, x_out, ldxo, out, ldo, out_nks, n_rows, dim, eps, s)
  if (KS == 0) LSK_NORM_KS(0);
  else if (KS == 4) LSK_NORM_KS(4);
  else if (KS == 2) LSK_NORM_KS(2);
  else if (KS == 8) LSK_NORM_KS(8);
  else if (KS == 1) LSK_NORM_KS(1);
  else LSK_NORM_KS(-1);
#undef LSK_NORM_KS
}

extern "C" int lsk_add_rmsnorm(int dtype, const void* x, long ldx, const float* partials, int ks, const void* w,
                               float eps, void* x_out, long ldxo, void* out, long ldo, int n_rows, int dim,
                               void* stream) {
  return lsk_add_rmsnorm_impl(dtype, x, ldx, partials, ks, w, eps, x_out, ldxo, out, ldo, 0, n_rows, dim, stream);
}

int lsk_add_rmsnorm_impl(int dtype, const void* x, long ldx, const float* partials, int ks, const void* w, float eps,
                         void* x_out, long ldxo, void* out, long ldo, int out_frag, int n_rows, int dim,
                         void* stream) {
  LSK_REQUIRE(x != nullptr && (ks == 0 || partials != nullptr) && (out == nullptr || w != nullptr), LSK_EARG,
              "lsk_add_rmsnorm: null pointer");
  LSK_REQUIRE(n_rows >= 0 && dim > 0 && dim % 8 == 0 && dim <= NORM_MAX_DIM && ldx >= dim && ks >= 0 &&
                  ldx % 8 == 0 && (out == nullptr || (ldo >= dim && ldo % 8 == 0)) &&
                  (x_out == nullptr || (ldxo >= dim && ldxo % 8 == 0)),
              LSK_ESHAPE, "lsk_add_rmsnorm: bad shape n_rows=%d dim=%d", n_rows, dim);
  LSK_REQUIRE(!out_frag || (dtype == LSK_DTYPE_BF16 && out != nullptr && dim % 32 == 0), LSK_EARG,
              "lsk_add_rmsnorm: a fragment-major output needs bf16, an output and dim %% 32 == 0");
  if (n_rows == 0) return 0;
  const long pstride = (long)n_rows * dim;
  const int out_nks = out_frag ? dim / 32 : 0;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == LSK_DTYPE_BF16)
    launch_add_rmsnorm<uint16_t>(x, ldx, partials, ks, pstride, w, x_out, ldxo, out, ldo, out_nks, n_rows, dim, eps,
                                 s);
  else if (dtype == LSK_DTYPE_F32)
    launch_add_rmsnorm<float>(x, ldx, partials, ks, pstride, w, x_out, ldxo, out, ldo, 0, n_rows, dim, eps, s);
  else
    LSK_REQUIRE(false, LSK_EUNSUPPORTED, "lsk_add_rmsnorm: dtype %d", dtype);
  return lsk_check_launch("lsk_add_rmsnorm");
}

extern "C" int lsk_rmsnorm(int dtype, const void* x, const void* w, void* out, int n_rows, int dim, float eps,
                           long ldx, long ldo, void* stream) {
  LSK_REQUIRE(x && w && out, LSK_EARG, "lsk_rmsnorm: null pointer");
  return lsk_add_rmsnorm(dtype, x, ldx, nullptr, 0, w, eps, nullptr, 0, out, ldo, n_rows, dim, stream);
}

// ----------------------------------------------------------------------------- RoPE + KV append
// qkv [N, (Hq + 2 Hkv) D] = [q | k | v] per token (solutions/packed.py:175-176); from_p: the values are
// rnd(sum_s P[s][t][:]) (the QKV GEMM's K-slice partials, s in order) instead of a materialised qkv.
// q heads:  q_out[t, h]                       = rope(q)   (common/model.py:148-150)
// k heads:  kcache[row_t, h, pos_t]           = rope(k)   (solutions/packed.py:180)
// v heads:  V cache (row_t, h, pos_t)          = v         (solutions/packed.py:181; V stored in
//                                                        transposed 32-position blocks [B, Hkv, S/32, D, 32])
// rope(x)[j]       = x[j] * c[j]       + (-x[j+D/2]) * s[j]
// rope(x)[j + D/2] = x[j+D/2] * c[j+D/2] + x[j] * s[j+D/2]
// with c, s = the fp32 tables at pos_t stored to the model dtype first (solutions/packed.py:106-107)
// and one dtype rounding after each multiply and after the add.
// Grid: (token, head); a thread owns one rotation pair (j, j + D/2) or, for v heads, two elements.
// KSC as for add_rmsnorm_kernel: a compile-time slice count issues every partial load before the first add.
template <typename T, int KSC>
__device__ __forceinline__ float qkv_val(const T* qkv, const float* P, int KS, long pstride, long idx) {
  if (P == nullptr) return Elem<T>::ld(qkv + idx);
  if constexpr (KSC > 0) {
    float pv[KSC];
#pragma unroll
    for (int s = 0; s < KSC; ++s) pv[s] = P[s * pstride + idx];
    float a = pv[0];
#pragma unroll
    for (int s = 1; s < KSC; ++s) a = a + pv[s];
    return Elem<T>::round(a);
  } else {
    float a = P[idx];
    for (int s = 1; s < KS; ++s) a = a + P[s * pstride + idx];
    return Elem<T>::round(a);
  }
}

template <typename T, int KSC>
__global__ void rope_append_kernel(const T* __restrict__ qkv, const float* __restrict__ P, int KS, long pstride,
                                   T* __restrict__ q_out, T* __restrict__ kc, T* __restrict__ vc,
                                   const float* __restrict__ cos_tab, const float* __restrict__ sin_tab,
                                   const int32_t* __restrict__ rows, const int32_t* __restrict__ pos, int Hq, int Hkv,
                                   int D, int max_batch, int max_seq, int tab_len) {
  const int t = blockIdx.x, h = blockIdx.y;
  const int half = D >> 1;
  const long width = (long)(Hq + 2 * Hkv) * D;
  const long base = (long)t * width + (long)h * D;
  for (int j = threadIdx.x; j < half; j += blockDim.x) {
    // the token's values do not depend on its row / position: their loads go out with the row / position
    // loads instead of after them
    const float x1 = qkv_val<T, KSC>(qkv, P, KS, pstride, base + j);
    const float x2 = qkv_val<T, KSC>(qkv, P, KS, pstride, base + j + half);
    const int row = rows[t], p = pos[t];
    if (row < 0 || row >= max_batch || p < 0 || p >= max_seq || p >= tab_len) return;  // host validates too
    if (h < Hq + Hkv) {
      float o1, o2;
      rope_pair<T>(x1, x2, cos_tab + (long)p * D, sin_tab + (long)p * D, j, half, o1, o2);
      if (h < Hq) {
        T* dst = q_out + ((long)t * Hq + h) * D;
        Elem<T>::st(dst + j, o1);
        Elem<T>::st(dst + j + half, o2);
      } else {
        T* dst = kc + ((long)row * Hkv + (h - Hq)) * (long)max_seq * D;
        Elem<T>::st(dst + k_cache_offset<T>(p, j, D), o1);
        Elem<T>::st(dst + k_cache_offset<T>(p, j + half, D), o2);
      }
    } else {
      // V cache: 32-position blocks, each transposed ([B, Hkv, S/32, D, 32])
      T* dst = vc + ((long)row * Hkv + (h - Hq - Hkv)) * (long)D * max_seq + (long)(p >> 5) * 32 * D + (p & 31);
      Elem<T>::st(dst + (long)j * 32, x1);
      Elem<T>::st(dst + (long)(j + half) * 32, x2);
    }
  }
}

template <typename T>
static void launch_rope(const void* qkv, const float* P, int KS, long pstride, void* q_out, void* kc, void* vc,
                        const float* ct, const float* st, const int32_t* rows, const int32_t* pos, int N, int Hq,
                        int Hkv, int D, int B, int S, int tab_len, hipStream_t s) {
  dim3 grid(N, Hq + 2 * Hkv);
  const int threads = (D / 2 + 63) / 64 * 64;
#define LSK_ROPE_LAUNCH(KSC_)                                                                                   \
  rope_append_kernel<T, KSC_><<<grid, threads, 0, s>>>((const T*)qkv, P, KS, pstride, (T*)q_out, (T*)kc, (T*)vc, \
                                                       ct, st, rows, pos, Hq, Hkv, D, B, S, tab_len)
  if (P != nullptr && KS == 4) LSK_ROPE_LAUNCH(4);
  else if (P != nullptr && KS == 2) LSK_ROPE_LAUNCH(2);
  else if (P != nullptr && KS == 8) LSK_ROPE_LAUNCH(8);
  else LSK_ROPE_LAUNCH(-1);
#undef LSK_ROPE_LAUNCH
}

static int rope_common(int dtype, const void* qkv, const float* P, int KS, void* q_out, void* kcache, void* vcache,
                       const float* cos_tab, const float* sin_tab, int tab_len, const int32_t* rows,
                       const int32_t* pos, int n_tokens, int n_heads, int n_kv_heads, int head_dim, int max_batch,
                       int max_seq, void* stream) {
  LSK_REQUIRE((qkv || P) && q_out && kcache && vcache && cos_tab && sin_tab && rows && pos, LSK_EARG,
              "lsk_rope_append: null pointer");
  LSK_REQUIRE(n_tokens >= 0 && n_heads > 0 && n_kv_heads > 0 && head_dim > 0 && (head_dim % 2) == 0 &&
                  head_dim <= 512 && n_heads % n_kv_heads == 0 && max_batch > 0 && max_seq > 0 && tab_len > 0 &&
                  KS >= 1 && max_seq % 32 == 0 && (dtype != LSK_DTYPE_BF16 || head_dim % 32 == 0),
              LSK_ESHAPE, "lsk_rope_append: bad shape");
  if (n_tokens == 0) return 0;
  const long pstride = (long)n_tokens * (n_heads + 2 * n_kv_heads) * head_dim;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == LSK_DTYPE_BF16)
    launch_rope<uint16_t>(qkv, P, KS, pstride, q_out, kcache, vcache, cos_tab, sin_tab, rows, pos, n_tokens, n_heads,
                          n_kv_heads, head_dim, max_batch, max_seq, tab_len, s);
  else if (dtype == LSK_DTYPE_F32)
    launch_rope<float>(qkv, P, KS, pstride, q_out, kcache, vcache, cos_tab, sin_tab, rows, pos, n_tokens, n_heads,
                       n_kv_heads, head_dim, max_batch, max_seq, tab_len, s);
  else
    LSK_REQUIRE(false, LSK_EUNSUPPORTED, "lsk_rope_append: dtype %d", dtype);
  return lsk_check_launch("lsk_rope_append");
}

extern "C" int lsk_rope_append(int dtype, const void* qkv, void* q_out, void* kcache, void* vcache,
                               const float* cos_tab, const float* sin_tab, int tab_len, const int32_t* rows,
                               const int32_t* pos, int n_tokens, int n_heads, int n_kv_heads, int head_dim,
                               int max_batch, int max_seq, void* stream) {
  LSK_REQUIRE(qkv != nullptr, LSK_EARG, "lsk_rope_append: null qkv");
  return rope_common(dtype, qkv, nullptr, 1, q_out, kcache, vcache, cos_tab, sin_tab, tab_len, rows, pos, n_tokens,
                     n_heads, n_kv_heads, head_dim, max_batch, max_seq, stream);
}

extern "C" int lsk_rope_append_partial(int dtype, const float* partials, int ks, void* q_out, void* kcache,
                                       void* vcache, const float* cos_tab, const float* sin_tab, int tab_len,
                                       const int32_t* rows, const int32_t* pos, int n_tokens, int n_heads,
                                       int n_kv_heads, int head_dim, int max_batch, int max_seq, void* stream) {
  LSK_REQUIRE(partials != nullptr, LSK_EARG, "lsk_rope_append_partial: null partials");
  return rope_common(dtype, nullptr, partials, ks, q_out, kcache, vcache, cos_tab, sin_tab, tab_len, rows, pos,
                     n_tokens, n_heads, n_kv_heads, head_dim, max_batch, max_seq, stream);
}

// Plain KV append (no RoPE): kcache[row_t, h, pos_t] = k[t, h]; V cache (row_t, h, pos_t) = v[t, h]
// (V in transposed 32-position blocks, [B, Hkv, S/32, D, 32]).
// Used for inputs whose RoPE is already applied (solutions/packed.py:180-181 on its own).
#define KV_APPEND_TOKENS 16
template <typename T>
__global__ __launch_bounds__(256) void kv_append_kernel(const T* __restrict__ k, const T* __restrict__ v,
                                                        T* __restrict__ kc, T* __restrict__ vc,
                                                        const int32_t* __restrict__ rows,
                                                        const int32_t* __restrict__ pos, int N, int Hkv, int D,
                                                        int max_batch, int max_seq) {
  // A workgroup per (KV_APPEND_TOKENS tokens, KV head).  K: consecutive threads take consecutive d of one token
  // (16-byte runs of the fragment-major block).  V^T: consecutive threads take consecutive tokens of one d row, so
  // the positions of a verify block land side by side in the transposed 32-position block instead of one 2-byte
  // write per 64-byte row (the input rows are re-read from L2, where the previous kernel left them).
  const int t0 = blockIdx.x * KV_APPEND_TOKENS, hk = blockIdx.y;
  const int nt = min(KV_APPEND_TOKENS, N - t0);
  const int HD = Hkv * D;
  for (int e = threadIdx.x; e < nt * D; e += blockDim.x) {
    const int j = e / D, d = e - j * D;
    const int t = t0 + j, row = rows[t], p = pos[t];
    if (row < 0 || row >= max_batch || p < 0 || p >= max_seq) continue;
    kc[((long)row * Hkv + hk) * (long)max_seq * D + k_cache_offset<T>(p, d, D)] = k[(long)t * HD + hk * D + d];
  }
  for (int e = threadIdx.x; e < nt * D; e += blockDim.x) {
    const int d = e / nt, j = e - d * nt;
    const int t = t0 + j, row = rows[t], p = pos[t];
    if (row < 0 || row >= max_batch || p < 0 || p >= max_seq) continue;
    vc[((long)row * Hkv + hk) * (long)D * max_seq + (long)(p >> 5) * 32 * D + d * 32 + (p & 31)] =
        v[(long)t * HD + hk * D + d];
  }
}

extern "C" int lsk_kv_append(int dtype, const void* k, const void* v, void* kcache, void* vcache, const int32_t* rows,
                             const int32_t* pos, int n_tokens, int n_kv_heads, int head_dim, int max_batch,
                             int max_seq, void* stream) {
  LSK_REQUIRE(k && v && kcache && vcache && rows && pos, LSK_EARG, "lsk_kv_append: null pointer");
  LSK_REQUIRE(n_tokens >= 0 && n_kv_heads > 0 && head_dim > 0 && max_batch > 0 && max_seq > 0 && max_seq % 32 == 0 &&
                  (dtype != LSK_DTYPE_BF16 || head_dim % 32 == 0),
              LSK_ESHAPE, "lsk_kv_append: bad shape (bf16 needs head_dim %% 32 == 0; max_seq %% 32 == 0)");
  if (n_tokens == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((n_tokens + KV_APPEND_TOKENS - 1) / KV_APPEND_TOKENS, n_kv_heads);
  if (dtype == LSK_DTYPE_BF16)
    kv_append_kernel<uint16_t><<<grid, 256, 0, s>>>((const uint16_t*)k, (const uint16_t*)v, (uint16_t*)kcache,
                                                    (uint16_t*)vcache, rows, pos, n_tokens, n_kv_heads, head_dim,
                                                    max_batch, max_seq);
  else if (dtype == LSK_DTYPE_F32)
    kv_append_kernel<float><<<grid, 256, 0, s>>>((const float*)k, (const float*)v, (float*)kcache,
                                                 (float*)vcache, rows, pos, n_tokens, n_kv_heads, head_dim, max_batch,
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

// ----------------------------------------------------------------------------- M2 probe agreement
// pred [nc][nvt]: greedy tokens of the nc candidate exits on the nvt verify tokens; Yv [nvt]: the full model's
// tokens; acc [nv] accepted counts; blk [nvt] / jl [nvt]: verifier and position within its block of each verify
// token.  out[c] = #{t : jl[t] <= acc[blk[t]] and pred[c][t] == Yv[t]}, out[nc] = #{t : jl[t] <= acc[blk[t]]}
// (solutions/engine.py:491-514: agreement on the positions whose prefix is correct).  One workgroup per output;
// integer sums, so the order of the additions does not matter.
__global__ __launch_bounds__(256) void probe_matches_kernel(const int64_t* __restrict__ pred,
                                                            const int64_t* __restrict__ Yv,
                                                            const int64_t* __restrict__ acc,
                                                            const int32_t* __restrict__ blk,
                                                            const int32_t* __restrict__ jl, int nc, int nvt,
                                                            int64_t* __restrict__ out) {
  const int c = blockIdx.x;
  int cnt = 0;
  for (int t = threadIdx.x; t < nvt; t += 256) {
    const bool valid = jl[t] <= acc[blk[t]];
    cnt += (c == nc) ? (int)valid : (int)(valid && pred[(long)c * nvt + t] == Yv[t]);
  }
  for (int o = 32; o >= 1; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
  __shared__ int part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) out[c] = (int64_t)(part[0] + part[1] + part[2] + part[3]);
}

extern "C" int lsk_probe_matches(const int64_t* pred, const int64_t* Yv, const int64_t* acc, const int32_t* blk,
                                 const int32_t* jl, int nc, int nvt, int64_t* out, void* stream) {
  LSK_REQUIRE(out && (nvt == 0 || (pred && Yv && acc && blk && jl)), LSK_EARG, "lsk_probe_matches: null pointer");
  LSK_REQUIRE(nc >= 0 && nvt >= 0, LSK_ESHAPE, "lsk_probe_matches: bad shape");
  probe_matches_kernel<<<nc + 1, 256, 0, (hipStream_t)stream>>>(pred, Yv, acc, blk, jl, nc, nvt, out);
  return lsk_check_launch("lsk_probe_matches");
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

// ----------------------------------------------------------------------------- segment planned ahead of acceptance
// A decode segment planned before the previous step's acceptance is known: every block in cache row vslots[j]
// was planned at the position it has if all vdrafts[j] drafts of that verifier are accepted, and acc[j] (the
// greedy acceptance's output, still on the device) is the accepted count, so the block's actual position is
// acc[j] - vdrafts[j] (<= 0) away.  The kernel moves those blocks in the segment's metadata (lsk_pack_segment's
// layout): each token's position, each block's pos0, and each work record's pos0 and, for the record that ends
// at its rows' last position (the last KV split), kv_hi.  Valid when the shift never changes a block's number
// of KV splits; the caller checks that when it plans.  One workgroup: a decode segment's metadata is small.
__global__ __launch_bounds__(256) void shift_positions_kernel(int32_t* __restrict__ meta, int N, int nb, int nw,
                                                              int ng, int n_recs, int group,
                                                              const int64_t* __restrict__ acc,
                                                              const int32_t* __restrict__ vslots,
                                                              const int32_t* __restrict__ vdrafts, int nv) {
  // per-row shifts in LDS (rows below SHIFT_TAB; a row beyond it, which no cache this large holds, scans the list)
  constexpr int SHIFT_TAB = 4096;
  __shared__ int tab[SHIFT_TAB];
  for (int i = threadIdx.x; i < SHIFT_TAB; i += blockDim.x) tab[i] = 0;
  __syncthreads();
  for (int j = threadIdx.x; j < nv; j += blockDim.x) {
    const int row = vslots[j];
    if (row >= 0 && row < SHIFT_TAB) tab[row] = (int)acc[j] - vdrafts[j];
  }
  __syncthreads();
  auto delta_of = [&](int row) {
    if (row >= 0 && row < SHIFT_TAB) return tab[row];
    for (int j = 0; j < nv; ++j)
      if (vslots[j] == row) return (int)acc[j] - vdrafts[j];
    return 0;
  };
  auto fix = [&](int32_t* r) {  // [q_start, row0, nrows | kvh << 8, kv_lo, kv_hi, part, pos0, crow]
    const int dl = delta_of(r[7]);
    if (dl == 0) return;
    const int end_old = r[6] + (r[1] + (r[2] & 255) - 1) / group + 1;
    if (r[4] == end_old) r[4] += dl;
    r[6] += dl;
  };
  const int32_t* rows_h = meta;
  int32_t* pos_h = meta + N;
  int32_t* blk = meta + 2L * N;
  int32_t* works = blk + 4L * nb;
  int32_t* recs = works + 8L * nw + 8L * ng;
  for (int t = threadIdx.x; t < N; t += blockDim.x) pos_h[t] += delta_of(rows_h[t]);
  for (int b = threadIdx.x; b < nb; b += blockDim.x) blk[4L * b + 1] += delta_of(blk[4L * b + 3]);
  for (int w = threadIdx.x; w < nw; w += blockDim.x) fix(works + 8L * w);
  for (int r = threadIdx.x; r < n_recs; r += blockDim.x)
    if ((recs[8L * r + 2] & 255) > 0) fix(recs + 8L * r);
}

extern "C" int lsk_shift_segment_positions(int32_t* meta, int n_tokens, int nb, int n_works, int n_groups,
                                           int n_recs, int group, const int64_t* accepted, const int32_t* vslots,
                                           const int32_t* vdrafts, int nv, void* stream) {
  LSK_REQUIRE(n_tokens >= 0 && nb >= 0 && n_works >= 0 && n_groups >= 0 && n_recs >= 0 && group > 0 && nv >= 0,
              LSK_ESHAPE, "lsk_shift_segment_positions: bad shape");
  LSK_REQUIRE((meta != nullptr || n_tokens == 0) && (nv == 0 || (accepted && vslots && vdrafts)), LSK_EARG,
              "lsk_shift_segment_positions: null pointer");
  if (nv == 0 || n_tokens == 0) return 0;
  shift_positions_kernel<<<1, 256, 0, (hipStream_t)stream>>>(meta, n_tokens, nb, n_works, n_groups, n_recs, group,
                                                             accepted, vslots, vdrafts, nv);
  return lsk_check_launch("lsk_shift_segment_positions");
}
