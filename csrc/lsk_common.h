// Shared device/host helpers for the packed ragged LayerSkip-Llama kernels (gfx950).
//
// Storage types: bf16 is carried as uint16_t (torch.bfloat16 bit layout), fp32 as float.
// Every conversion float -> bf16 rounds to nearest even with NaN -> 0x7FC0, which is the rule
// torch's CPU kernels apply when a float intermediate is stored into a bfloat16 tensor; the
// elementwise kernels rely on it to reproduce the reference's rounding points bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define LSK_DTYPE_F32 0
#define LSK_DTYPE_BF16 1

typedef __bf16 lsk_bf16x8 __attribute__((ext_vector_type(8)));
typedef short lsk_s16x4 __attribute__((ext_vector_type(4)));
typedef float lsk_f32x4 __attribute__((ext_vector_type(4)));
typedef int lsk_i32x4 __attribute__((ext_vector_type(4)));

// Word 3 of a raw buffer descriptor on gfx9-family parts (gfx950): 32-bit data format, no swizzle, no stride;
// loads of 16 bytes at byte offsets read the memory as is.
#define LSK_BUFFER_RSRC_WORD3 0x00020000

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Round a float through bf16 and back (value of the float once stored in a bf16 tensor).
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// exp(x) in fp32 (Cody and Waite's range reduction): x = n ln2 + r with n = rint(x log2(e)) and ln2 split into
// a 16-bit head (n * head is exact for the |n| <= 128 reached here) and a tail; exp(r) = sum_{k<=7} r^k / k!
// by Horner on |r| <= ln2 / 2 (truncation below 6e-9 relative); then 2^n by ldexp.  Results below 2^-124
// (x < -86) are flushed to 0 so no subnormal is ever produced; x > 89 gives +inf.  Each step is one IEEE fp32
// operation and the build contracts nothing into FMAs, so a host restatement of the same steps (the fp32
// oracle's) produces the same bits.  Used by the fp32 attention softmax and by SiLU.
__device__ __forceinline__ float lsk_exp(float x) {
  if (x != x) return x;
  if (x < -86.0f) return 0.0f;
  if (x > 89.0f) return __builtin_huge_valf();
  const float n = __builtin_rintf(x * 1.4426950216293335f);
  const float r = (x - n * 0.693145751953125f) - n * 1.428606765330187e-06f;
  float p = 0.00019841270113829523f;
  p = p * r + 0.0013888889225199819f;
  p = p * r + 0.008333333767950535f;
  p = p * r + 0.0416666679084301f;
  p = p * r + 0.1666666716337204f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  return __builtin_ldexpf(p, (int)n);
}

// Offset of K cache element (position p, dim d) within one (row, KV head) stripe of S positions x D.
// bf16: fragment-major 32-position blocks of 32 D elements, each block 2 (D / 32) MFMA fragments of 1 KiB:
//   fragment (a, j), lane l = 16 lg + l16 holds positions 8 (l16 / 4) + 4 a + l16 % 4 of the block and
//   d = 32 j + 8 lg .. +7, so a wave's K fragment load is one contiguous 1 KiB request (D % 32 == 0).
// fp32: the reference's row-major [S, D].
template <typename T>
__device__ __forceinline__ long k_cache_offset(int p, int d, int D);
template <>
__device__ __forceinline__ long k_cache_offset<uint16_t>(int p, int d, int D) {
  const int pp = p & 31;
  const int a = (pp >> 2) & 1, l16 = ((pp >> 3) << 2) | (pp & 3);
  const int j = d >> 5, lg = (d >> 3) & 3;
  return (long)(p >> 5) * 32 * D + (long)((a * (D >> 5) + j) * 64 + lg * 16 + l16) * 8 + (d & 7);
}
template <>
__device__ __forceinline__ long k_cache_offset<float>(int p, int d, int D) {
  return (long)p * D + d;
}

// Loads/stores of "dtype T" elements expressed as float.
template <typename T> struct Elem;
template <> struct Elem<float> {
  static __device__ __forceinline__ float ld(const float* p) { return *p; }
  static __device__ __forceinline__ void st(float* p, float v) { *p = v; }
  // value after being stored in a tensor of this dtype
  static __device__ __forceinline__ float round(float v) { return v; }
};
template <> struct Elem<uint16_t> {
  static __device__ __forceinline__ float ld(const uint16_t* p) { return bf2f(*p); }
  static __device__ __forceinline__ void st(uint16_t* p, float v) { *p = f2bf(v); }
  static __device__ __forceinline__ float round(float v) { return rbf(v); }
};

// One RoPE rotation pair (common/model.py:143-150 with the cos / sin rows cast to the model dtype first,
// solutions/packed.py:106-107): x1 = x[j], x2 = x[j + half] of one head at the position whose fp32 table rows are
// ct / st;  o1 = rnd(x1 c1) + rnd(-x2 s1),  o2 = rnd(x2 c2) + rnd(x1 s2)  with c, s rounded to T and one T rounding
// after each multiply (the caller's store rounds the add).  Shared by the RoPE + append kernel and the qkv GEMM's
// fused epilogue, so both give the same bits.
template <typename T>
__device__ __forceinline__ void rope_pair(float x1, float x2, const float* ct, const float* st, int j, int half,
                                          float& o1, float& o2) {
  const float c1 = Elem<T>::round(ct[j]), c2 = Elem<T>::round(ct[j + half]);
  const float s1 = Elem<T>::round(st[j]), s2 = Elem<T>::round(st[j + half]);
  const float a1 = Elem<T>::round(x1 * c1), b1 = Elem<T>::round((-x2) * s1);
  const float a2 = Elem<T>::round(x2 * c2), b2 = Elem<T>::round(x1 * s2);
  o1 = a1 + b1;
  o2 = a2 + b2;
}

// ----------------------------------------------------------------------------- host side
// Error reporting: every C-ABI entry returns 0 on success, a negative code for an argument
// error detected on the host before any launch, or a positive hipError_t.  The text of the
// last error of the calling thread is kept for lsk_last_error().
#define LSK_EARG -1
#define LSK_ESHAPE -2
#define LSK_EUNSUPPORTED -3
#define LSK_EWORKSPACE -4

void lsk_set_error(const char* fmt, ...);
int lsk_check_launch(const char* what);

#define LSK_REQUIRE(cond, code, ...)      \
  do {                                    \
    if (!(cond)) {                        \
      lsk_set_error(__VA_ARGS__);         \
      return (code);                      \
    }                                     \
  } while (0)

static inline size_t lsk_align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// ----------------------------------------------------------------------------- fragment-major activations
// The layer loop keeps GEMM inputs in the packed weights' fragment-major order: 16-token groups, each 16 x 32
// block one 1 KiB fragment in MFMA lane order, so a wave's activation load is one contiguous 1 KiB (8 full cache
// lines) instead of 16 half lines of 16 token rows.  Every row tile of a GEMM re-reads its activations from L2,
// and there a row-major fragment reads at about a third of the contiguous rate (measured on MI355X: ~9.5 vs
// ~27 TB/s over all CUs).  Used for the qkv input (the attention RMSNorm output) and the o input (the attention
// output) at every token count, for the head's normalised rows, and for the w13 input and the w2 input (w13's
// silu-mul output) above LSK_AF_MAX_TOKENS tokens, where the wide tier's many row tiles re-read them; at up to
// LSK_AF_MAX_TOKENS tokens those two measured faster row-major (the fragment-major stores cost more there).
// Element (token r, column c) of a matrix of nks = columns / 32 k-steps sits at lsk_frag_off(r, c, nks).
// Buffers hold whole 16-token groups; the padding tokens' values only reach discarded output columns.
// Both layouts hold the same values, so every result is bitwise the same as with row-major activations.
#define LSK_AF_MAX_TOKENS 64
__host__ __device__ __forceinline__ long lsk_frag_off(int r, int c, int nks) {
  return ((long)((r >> 4) * nks + (c >> 5)) * 64 + (r & 15) + 16 * ((c & 31) >> 3)) * 8 + (c & 7);
}
// Internal to liblsk (used by lsk_forward_layers; same arguments and errors as the exported entry points,
// with the fragment-major operands described above).
int lsk_add_rmsnorm_impl(int dtype, const void* x, long ldx, const float* partials, int ks, const void* w, float eps,
                         void* x_out, long ldxo, void* out, long ldo, int out_frag, int n_rows, int dim, void* stream);
int lsk_gemm_partial_af(const void* A, const void* W, float* P, int M, int N, int K, int ks, void* stream);
// w13 with silu-mul over a fragment-major A; H row-major ([M, ffn]) or, with h_frag, fragment-major (whole
// 16-token groups) for the w2 launch.
int lsk_gemm_silu_af(const void* A, const void* W, void* H, int h_frag, int M, int ffn, int K, void* stream);
int lsk_ragged_attn_impl(int dtype, const void* q, const void* kcache, const void* vcache, const int32_t* blocks,
                         const int32_t* works, int n_works, const int32_t* groups, int n_groups, int n_parts,
                         const int32_t* recs, int n_rounds, int n_slots, int rows_cap, void* out, int out_frag,
                         int n_heads, int n_kv_heads, int head_dim, int max_seq, float scale, void* workspace,
                         size_t ws_bytes, void* stream);
