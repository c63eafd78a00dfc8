// Projection / LM-head GEMMs over the packed token rows (solutions/packed.py:175,182,183-185;
// common/model.py:330):  C[m][n] = epilogue( sum_k A[m][k] * W[n][k] )   (F.linear, W = [out, in]).
//
// bf16 path (gfx950 MFMA v_mfma_f32_16x16x32_bf16, fp32 accumulation).  Both operands are
// K-contiguous, so every lane fetches its MFMA fragment with one 16-byte load straight from HBM/L2
// (no LDS staging: at decode sizes the weights are streamed exactly once and the activation rows
// are L2-resident).  A workgroup = 4 waves computes a (16*NS features) x (16*MS tokens) tile; the
// waves split K into 128-element chunks (wave w takes chunks w, w+4, ...) and their partial sums
// are added in wave order through LDS.  The reduction order of every output element is therefore
// fixed by K alone: it does not depend on M, on the tile shape, or on which rows share a tile, so a
// token's logits are bitwise identical whether it is decoded alone or inside a packed verify batch.
//
// Epilogues (the reference's dtype rounding points):
//   NONE      C = rnd(acc)
//   RESIDUAL  C = rnd(R + rnd(acc))                       x + F.linear(...)
//   SILU_MUL  C = rnd(rnd(silu(rnd(g))) * rnd(u))         g, u = rows n and ffn + n of W (w13)
#include "lsk_common.h"
#include "../include/lsk.h"

#define KCHUNK 128

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

template <int NS, int MS, int EPI>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(const uint16_t* __restrict__ A, long lda,
                                                        const uint16_t* __restrict__ W, long ldw,
                                                        uint16_t* __restrict__ C, long ldc,
                                                        const uint16_t* __restrict__ R, long ldr, int M, int N,
                                                        int K, int ffn) {
  constexpr int NT = (EPI == LSK_EPI_SILU_MUL) ? 2 * NS : NS;
  constexpr int E = NT * MS * 256;  // partial-sum floats per wave
  __shared__ __attribute__((aligned(16))) float red[4 * E];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * 16 * NS;
  const int m0 = blockIdx.y * 16 * MS;

  const uint16_t* wrow[NT];
#pragma unroll
  for (int s = 0; s < NT; ++s) {
    int n = (s < NS) ? (n0 + 16 * s + l16) : (ffn + n0 + 16 * (s - NS) + l16);
    const int nmax = (EPI == LSK_EPI_SILU_MUL) ? (s < NS ? ffn - 1 : 2 * ffn - 1) : N - 1;
    n = n < nmax ? n : nmax;  // clamp: padded features load a valid row, results discarded
    wrow[s] = W + (long)n * ldw + 8 * lg;
  }
  const uint16_t* arow[MS];
#pragma unroll
  for (int t = 0; t < MS; ++t) {
    int m = m0 + 16 * t + l16;
    m = m < M - 1 ? m : M - 1;
    arow[t] = A + (long)m * lda + 8 * lg;
  }

  lsk_f32x4 acc[NT][MS];
#pragma unroll
  for (int s = 0; s < NT; ++s)
#pragma unroll
    for (int t = 0; t < MS; ++t) acc[s][t] = (lsk_f32x4){0.f, 0.f, 0.f, 0.f};

  const int nk32 = K / 32;
  for (int c = wave; c * 4 < nk32; c += 4) {
    const int kk0 = c * 4;
    if (kk0 + 4 <= nk32) {
      lsk_bf16x8 wf[4][NT], af[4][MS];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int k = (kk0 + ks) * 32;
#pragma unroll
        for (int s = 0; s < NT; ++s) wf[ks][s] = *(const lsk_bf16x8*)(wrow[s] + k);
#pragma unroll
        for (int t = 0; t < MS; ++t) af[ks][t] = *(const lsk_bf16x8*)(arow[t] + k);
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int s = 0; s < NT; ++s)
#pragma unroll
          for (int t = 0; t < MS; ++t)
            acc[s][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[ks][s], af[ks][t], acc[s][t], 0, 0, 0);
    } else {
      for (int kk = kk0; kk < nk32; ++kk) {
        const int k = kk * 32;
        lsk_bf16x8 wf[NT], af[MS];
#pragma unroll
        for (int s = 0; s < NT; ++s) wf[s] = *(const lsk_bf16x8*)(wrow[s] + k);
#pragma unroll
        for (int t = 0; t < MS; ++t) af[t] = *(const lsk_bf16x8*)(arow[t] + k);
#pragma unroll
        for (int s = 0; s < NT; ++s)
#pragma unroll
          for (int t = 0; t < MS; ++t)
            acc[s][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[s], af[t], acc[s][t], 0, 0, 0);
      }
    }
  }

  // partial sums -> LDS, element ((s*MS + t)*64 + lane)*4 + i  <->  feature 16s + 4lg + i, token 16t + l16
  float* my = red + wave * E;
#pragma unroll
  for (int s = 0; s < NT; ++s)
#pragma unroll
    for (int t = 0; t < MS; ++t)
      *(float4*)(my + ((s * MS + t) * 64 + lane) * 4) = make_float4(acc[s][t][0], acc[s][t][1], acc[s][t][2], acc[s][t][3]);
  __syncthreads();

  constexpr int TN = 16 * NS, TM = 16 * MS;
  for (int o = tid; o < TN * TM; o += 256) {
    const int ml = o / TN, nl = o - ml * TN;
    const int m = m0 + ml, n = n0 + nl;
    if (m >= M || n >= N) continue;
    const int t = ml >> 4, ll = ml & 15;
    const int s = nl >> 4, w16 = nl & 15;
    const int ln = (w16 >> 2) * 16 + ll, i = w16 & 3;
    const int e = ((s * MS + t) * 64 + ln) * 4 + i;
    const float v = ((red[e] + red[E + e]) + red[2 * E + e]) + red[3 * E + e];
    float outv;
    if constexpr (EPI == LSK_EPI_SILU_MUL) {
      const int eu = (((s + NS) * MS + t) * 64 + ln) * 4 + i;
      const float u = ((red[eu] + red[E + eu]) + red[2 * E + eu]) + red[3 * E + eu];
      outv = rbf(silu_f(rbf(v))) * rbf(u);
    } else if constexpr (EPI == LSK_EPI_RESIDUAL) {
      outv = bf2f(R[(long)m * ldr + n]) + rbf(v);
    } else {
      outv = v;
    }
    C[(long)m * ldc + n] = f2bf(outv);
  }
}

// fp32 path (parity runs): one wave per output feature, 16 token rows per workgroup row-block.
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

template <int NS, int MS>
static void launch_bf16(int epi, dim3 grid, hipStream_t s, const uint16_t* A, long lda, const uint16_t* W, long ldw,
                        uint16_t* C, long ldc, const uint16_t* R, long ldr, int M, int N, int K, int ffn) {
  if (epi == LSK_EPI_RESIDUAL)
    gemm_bf16_kernel<NS, MS, LSK_EPI_RESIDUAL><<<grid, 256, 0, s>>>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, ffn);
  else if (epi == LSK_EPI_SILU_MUL) {
    if constexpr (NS <= 2)
      gemm_bf16_kernel<NS, MS, LSK_EPI_SILU_MUL><<<grid, 256, 0, s>>>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, ffn);
  } else
    gemm_bf16_kernel<NS, MS, LSK_EPI_NONE><<<grid, 256, 0, s>>>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, ffn);
}

// Tile choice: MS from M, then the widest NS that still gives >= 1024 workgroups (bandwidth needs
// many waves in flight).  Every choice shares the same K order, so the choice never changes results.
extern "C" int lsk_gemm_tile(int M, int N, int* ns_out, int* ms_out) {
  const int ms = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const int mt = (M + 16 * ms - 1) / (16 * ms);
  int ns = 1;
  if (N % 64 == 0 && (long)(N / 64) * mt >= 1024) ns = 4;
  else if (N % 32 == 0 && (long)(N / 32) * mt >= 1024) ns = 2;
  *ns_out = ns;
  *ms_out = ms;
  return 0;
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
    LSK_REQUIRE(K % 32 == 0 && lda % 8 == 0 && ldw % 8 == 0, LSK_ESHAPE,
                "lsk_gemm: bf16 needs K %% 32 == 0 and 16-byte aligned rows (K=%d)", K);
    LSK_REQUIRE(N % 16 == 0, LSK_ESHAPE, "lsk_gemm: bf16 needs N %% 16 == 0 (N=%d)", N);
    int ns, ms;
    lsk_gemm_tile(M, N, &ns, &ms);
    if (epilogue == LSK_EPI_SILU_MUL && ns == 4) ns = 2;  // keeps the LDS reduction buffer <= 64 KiB
    dim3 grid(N / (16 * ns), (M + 16 * ms - 1) / (16 * ms));
    const uint16_t* a = (const uint16_t*)A;
    const uint16_t* w = (const uint16_t*)W;
    uint16_t* c = (uint16_t*)C;
    const uint16_t* r = (const uint16_t*)R;
#define LSK_GEMM_CASE(NS_, MS_) \
  if (ns == NS_ && ms == MS_) launch_bf16<NS_, MS_>(epilogue, grid, s, a, lda, w, ldw, c, ldc, r, ldr, M, N, K, ffn);
    LSK_GEMM_CASE(1, 1) LSK_GEMM_CASE(1, 2) LSK_GEMM_CASE(1, 4)
    LSK_GEMM_CASE(2, 1) LSK_GEMM_CASE(2, 2) LSK_GEMM_CASE(2, 4)
    LSK_GEMM_CASE(4, 1) LSK_GEMM_CASE(4, 2) LSK_GEMM_CASE(4, 4)
#undef LSK_GEMM_CASE
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
