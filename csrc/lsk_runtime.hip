// Native layer-range runner of the packed forward (solutions/packed.py:169-196: packed_layer /
// packed_layers).  One call issues every kernel of layers [start, end) on one stream, so the host
// pays one C call per segment instead of ~8 launches per layer from Python.
//
// Per layer (same op order and rounding points as solutions/packed.py:175-185):
//   xn   = rmsnorm(x, attn_norm)                      lsk_rmsnorm
//   qkv  = xn Wqkv^T                                  lsk_gemm NONE            (fp32)
//   q, cache[k, v] = rope(q), rope(k), v              lsk_rope_append          (fp32)
//   q, cache[k, v] = rope / append of xn Wqkv^T       lsk_gemm_qkv_rope        (bf16: one launch)
//   attn = ragged attention(q, cache)                 lsk_ragged_attn (+ split combine)
//   x    = x + attn Wo^T                              lsk_gemm RESIDUAL
//   xn   = rmsnorm(x, ffn_norm)                       lsk_rmsnorm
//   h    = silu(g) * u, [g; u] = xn W13^T             lsk_gemm SILU_MUL
//   x    = x + h W2^T                                 lsk_gemm RESIDUAL (in place)
#include <math.h>
#include <mutex>
#include <vector>

#include "lsk_common.h"
#include "../include/lsk.h"

namespace {

struct Model {
  int dtype, n_layers, dim, n_heads, n_kv_heads, head_dim, ffn, vocab;
  int ks_qkv, ks_o, ks_w2;  // canonical K splits of the bf16 projections (lsk_gemm_plan)
  float eps;
  std::vector<const void*> wqkv, wo, w13, w2, attn_norm, ffn_norm;
  std::vector<void*> kc, vc;
  int max_batch, max_seq;
  const float* cos_tab;
  const float* sin_tab;
  int tab_len;
};

std::mutex g_mu;
std::vector<Model*> g_models;  // handle = index + 1

Model* get(long h) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (h <= 0 || h > (long)g_models.size()) return nullptr;
  return g_models[h - 1];
}

size_t elem_size(int dtype) { return dtype == LSK_DTYPE_BF16 ? 2 : 4; }

// ---- optional per-launch profiling: a pair of HIP events around each launch, tagged with its kernel
// class and ALGORITHMIC bytes / flops (the figures a roofline is computed from), summed at collect time.
struct ProfRec {
  int cls;
  double bytes, flops;
  hipEvent_t e0, e1;
};
std::vector<ProfRec> g_prof;
std::vector<hipEvent_t> g_event_pool;
bool g_prof_on = false;

hipEvent_t pool_event() {
  if (!g_event_pool.empty()) {
    hipEvent_t e = g_event_pool.back();
    g_event_pool.pop_back();
    return e;
  }
  hipEvent_t e;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

struct Layout {
  size_t xn, qkv, q, attn, h, part, gpart, total;
};

Layout layout(const Model& m, int N, int n_parts) {
  const size_t es = elem_size(m.dtype);
  const int qd = m.n_heads * m.head_dim, kvd = m.n_kv_heads * m.head_dim;
  Layout L;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off += lsk_align_up(bytes, 256);
    return o;
  };
  const size_t n16 = (size_t)(N + 15) / 16 * 16;  // xn, attn: whole 16-token groups (fragment-major use)
  L.xn = take(n16 * m.dim * es);
  L.qkv = take(m.dtype == LSK_DTYPE_BF16 ? 0 : (size_t)N * (qd + 2 * kvd) * es);  // bf16: fused into the qkv GEMM
  L.q = take((size_t)N * qd * es);
  L.attn = take(n16 * qd * es);
  L.h = take(n16 * m.ffn * es);  // whole 16-token groups (fragment-major above LSK_AF_MAX_TOKENS)
  L.part = take(n_parts > 0 ? lsk_attn_workspace_bytes(n_parts, m.n_kv_heads, m.head_dim) : 0);
  size_t gp = 0;
  if (m.dtype == LSK_DTYPE_BF16) {
    const size_t a = (size_t)m.ks_qkv * (qd + 2 * kvd), b = (size_t)m.ks_o * m.dim, c = (size_t)m.ks_w2 * m.dim;
    gp = (size_t)N * sizeof(float) * (a > b ? (a > c ? a : c) : (b > c ? b : c));
  }
  L.gpart = take(gp);
  L.total = off;
  return L;
}

}  // namespace

extern "C" int lsk_prof_enable(int on) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_prof_on = on != 0;
  return 0;
}

extern "C" int lsk_prof_start(int cls, double bytes, double flops, void* stream) {
  if (!g_prof_on) return 0;
  ProfRec r{cls, bytes, flops, pool_event(), pool_event()};
  LSK_REQUIRE(r.e0 && r.e1, LSK_EARG, "lsk_prof_start: event creation failed");
  (void)hipEventRecord(r.e0, (hipStream_t)stream);
  g_prof.push_back(r);
  return 0;
}

extern "C" int lsk_prof_stop(void* stream) {
  if (!g_prof_on || g_prof.empty()) return 0;
  (void)hipEventRecord(g_prof.back().e1, (hipStream_t)stream);
  return 0;
}

// Sums per class c < n_classes: ms[c], bytes[c], flops[c], count[c]; synchronises; clears the records.
extern "C" int lsk_prof_collect(int n_classes, double* ms, double* bytes, double* flops, long* count) {
  for (int c = 0; c < n_classes; ++c) { ms[c] = bytes[c] = flops[c] = 0.0; count[c] = 0; }
  for (auto& r : g_prof) {
    hipError_t e = hipEventSynchronize(r.e1);
    if (e != hipSuccess) { lsk_set_error("lsk_prof_collect: %s", hipGetErrorString(e)); return (int)e; }
    float t = 0.f;
    (void)hipEventElapsedTime(&t, r.e0, r.e1);
    if (r.cls >= 0 && r.cls < n_classes) {
      ms[r.cls] += t; bytes[r.cls] += r.bytes; flops[r.cls] += r.flops; count[r.cls] += 1;
    }
    g_event_pool.push_back(r.e0);
    g_event_pool.push_back(r.e1);
  }
  g_prof.clear();
  return 0;
}

extern "C" long lsk_model_create(int dtype, int n_layers, int dim, int n_heads, int n_kv_heads, int head_dim, int ffn,
                                 int vocab, float eps, const void* const* wqkv, const void* const* wo,
                                 const void* const* w13, const void* const* w2, const void* const* attn_norm,
                                 const void* const* ffn_norm, void* const* kcache, void* const* vcache, int max_batch,
                                 int max_seq, const float* cos_tab, const float* sin_tab, int tab_len) {
  LSK_REQUIRE(dtype == LSK_DTYPE_BF16 || dtype == LSK_DTYPE_F32, LSK_EUNSUPPORTED, "lsk_model_create: dtype %d", dtype);
  LSK_REQUIRE(n_layers > 0 && dim > 0 && n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0 && head_dim > 0 &&
                  ffn > 0 && vocab > 0 && max_batch > 0 && max_seq > 0 && tab_len > 0,
              LSK_ESHAPE, "lsk_model_create: bad dimensions");
  LSK_REQUIRE(wqkv && wo && w13 && w2 && attn_norm && ffn_norm && kcache && vcache && cos_tab && sin_tab, LSK_EARG,
              "lsk_model_create: null pointer");
  Model* m = new Model();
  m->dtype = dtype; m->n_layers = n_layers; m->dim = dim; m->n_heads = n_heads; m->n_kv_heads = n_kv_heads;
  m->head_dim = head_dim; m->ffn = ffn; m->vocab = vocab; m->eps = eps;
  m->wqkv.assign(wqkv, wqkv + n_layers); m->wo.assign(wo, wo + n_layers);
  m->w13.assign(w13, w13 + n_layers); m->w2.assign(w2, w2 + n_layers);
  m->attn_norm.assign(attn_norm, attn_norm + n_layers); m->ffn_norm.assign(ffn_norm, ffn_norm + n_layers);
  m->kc.assign(kcache, kcache + n_layers); m->vc.assign(vcache, vcache + n_layers);
  m->max_batch = max_batch; m->max_seq = max_seq;
  m->cos_tab = cos_tab; m->sin_tab = sin_tab; m->tab_len = tab_len;
  int ns;
  m->ks_qkv = m->ks_o = m->ks_w2 = 1;
  if (dtype == LSK_DTYPE_BF16) {
    // bf16: the qkv projection runs fused with RoPE + append (lsk_gemm_qkv_rope, no K split, wqkv in
    // lsk_pack_weight_qkv storage); o and w2 leave K-slice partials for the next add + RMSNorm
    const int qd = n_heads * head_dim;
    if (dim % 32 != 0 || head_dim % 32 != 0) {
      delete m;
      LSK_REQUIRE(false, LSK_EUNSUPPORTED, "lsk_model_create: bf16 needs dim and head_dim multiples of 32 (got %d, %d)",
                  dim, head_dim);
    }
    m->ks_qkv = 0;
    lsk_gemm_plan(dim, qd, &ns, &m->ks_o);
    lsk_gemm_plan(dim, ffn, &ns, &m->ks_w2);
  }
  std::lock_guard<std::mutex> lk(g_mu);
  g_models.push_back(m);
  return (long)g_models.size();
}

extern "C" int lsk_model_destroy(long handle) {
  std::lock_guard<std::mutex> lk(g_mu);
  LSK_REQUIRE(handle > 0 && handle <= (long)g_models.size() && g_models[handle - 1], LSK_EARG,
              "lsk_model_destroy: bad handle %ld", handle);
  delete g_models[handle - 1];
  g_models[handle - 1] = nullptr;
  return 0;
}

extern "C" size_t lsk_segment_workspace_bytes(long handle, int n_tokens, int n_parts) {
  Model* m = get(handle);
  if (!m) return 0;
  return layout(*m, n_tokens, n_parts).total;
}

// meta (device int32): [rows N][pos N][blocks nb*4][works n_works*8][groups n_groups*8]
// [recs n_slots*n_rounds*8] (lsk_attn_plan with rows_cap, lsk_attn_schedule)
// capture (host array of n_layers device pointers or NULL): capture[i] != NULL receives the output of
// layer i (the hidden state entering exit layer i + 1; solutions/packed.py:190-195).
extern "C" int lsk_forward_layers(long handle, const void* x_in, void* x_out, int n_tokens, int start, int end,
                                  const int32_t* meta, int nb, int n_works, int n_groups, int n_parts, int n_rounds,
                                  int n_slots, int rows_cap, void* workspace, size_t ws_bytes, void* const* capture,
                                  double attn_bytes, double attn_flops, void* stream) {
  Model* m = get(handle);
  LSK_REQUIRE(m != nullptr, LSK_EARG, "lsk_forward_layers: bad handle %ld", handle);
  LSK_REQUIRE(0 <= start && start <= end && end <= m->n_layers, LSK_ESHAPE, "lsk_forward_layers: bad range [%d, %d)",
              start, end);
  LSK_REQUIRE(x_in && x_out && x_in != x_out, LSK_EARG, "lsk_forward_layers: x_in / x_out");
  const int N = n_tokens;
  const size_t es = elem_size(m->dtype);
  hipStream_t s = (hipStream_t)stream;
  if (N == 0) return 0;
  if (start == end) {
    hipError_t e = hipMemcpyAsync(x_out, x_in, (size_t)N * m->dim * es, hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) { lsk_set_error("lsk_forward_layers: copy %s", hipGetErrorString(e)); return (int)e; }
    return 0;
  }
  LSK_REQUIRE(meta != nullptr, LSK_EARG, "lsk_forward_layers: meta missing");
  const Layout L = layout(*m, N, n_parts);
  LSK_REQUIRE(workspace != nullptr && ws_bytes >= L.total, LSK_EWORKSPACE,
              "lsk_forward_layers: workspace of %zu bytes needed, %zu given", L.total, ws_bytes);
  char* ws = (char*)workspace;
  void* xn = ws + L.xn;
  void* qkv = ws + L.qkv;
  void* q = ws + L.q;
  void* attn = ws + L.attn;
  void* h = ws + L.h;
  void* part = n_parts > 0 ? (void*)(ws + L.part) : nullptr;
  const size_t part_bytes = n_parts > 0 ? lsk_attn_workspace_bytes(n_parts, m->n_kv_heads, m->head_dim) : 0;
  const int32_t* rows = meta;
  const int32_t* pos = meta + N;
  const int32_t* blocks = pos + N;
  const int32_t* works = blocks + (size_t)nb * 4;
  const int32_t* groups = works + (size_t)n_works * 8;
  const int32_t* recs = groups + (size_t)n_groups * 8;
  const int qd = m->n_heads * m->head_dim, kvd = m->n_kv_heads * m->head_dim;
  const float scale = (float)(1.0 / sqrt((double)m->head_dim));
  int rc;
  const double es_d = (double)es, Nd = N, dimd = m->dim, qkvd = qd + 2 * kvd, ffd = m->ffn;
  if (m->dtype == LSK_DTYPE_BF16) {
    // bf16 flow: the qkv projection is one launch with RoPE and the KV append in its epilogue (no K split);
    // the o and w2 projections leave fp32 K-slice partials in P that the next add + RMSNorm reduces in slice
    // order (it also materialises the residual stream x).  Same rounding points as the unfused sequence.
    float* P = (float*)(ws + L.gpart);
    // GEMM inputs kept fragment-major (1 KiB contiguous per MFMA fragment; every row tile re-reads them from
    // L2, where a row-major fragment -- 16 rows x 64 bytes -- reads at a third of the rate): the qkv input
    // (attention RMSNorm output) and the o input (attention output) always; the w13 input (MLP RMSNorm output)
    // and the w2 input (w13's silu-mul output) above LSK_AF_MAX_TOKENS tokens, where the wide tier re-reads
    // them (at up to 64 tokens row-major measured faster for those two).
    const int af = m->dim % 32 == 0;
    const int af_o = qd % 32 == 0;
    const int af_h = N > LSK_AF_MAX_TOKENS && m->dim % 32 == 0 && m->ffn % 64 == 0;
    const double norm_bytes_b = es_d * (2.0 * Nd * dimd + dimd);
    auto pbytes = [&](int ks, double width) { return 4.0 * ks * Nd * width; };
#define LSK_PROF2(cls, b, f, call)                               \
  do {                                                           \
    lsk_prof_start((cls), (b), (f), stream);                     \
    if ((rc = (call))) return rc;                                \
    lsk_prof_stop(stream);                                       \
  } while (0)
    for (int i = start; i < end; ++i) {
      if (i == start) {
        LSK_PROF2(LSK_PROF_NORM, norm_bytes_b, 4.0 * Nd * dimd,
                  lsk_add_rmsnorm_impl(m->dtype, x_in, m->dim, nullptr, 0, m->attn_norm[i], m->eps, nullptr, 0, xn,
                                       m->dim, af, N, m->dim, stream));
      } else {
        LSK_PROF2(LSK_PROF_NORM, norm_bytes_b + es_d * Nd * dimd + pbytes(m->ks_w2, dimd), 4.0 * Nd * dimd,
                  lsk_add_rmsnorm_impl(m->dtype, x_out, m->dim, P, m->ks_w2, m->attn_norm[i], m->eps, x_out, m->dim,
                                       xn, m->dim, af, N, m->dim, stream));
        if (capture && capture[i - 1]) {
          hipError_t e = hipMemcpyAsync(capture[i - 1], x_out, (size_t)N * m->dim * es, hipMemcpyDeviceToDevice, s);
          if (e != hipSuccess) { lsk_set_error("lsk_forward_layers: capture %s", hipGetErrorString(e)); return (int)e; }
        }
      }
      // qkv projection, RoPE and the KV append in one launch (q rotated into `q`, K / V into this layer's cache)
      LSK_PROF2(LSK_PROF_GEMM_QKV, es_d * (qkvd * dimd + Nd * dimd + Nd * qkvd) + 8.0 * Nd * m->head_dim,
                2.0 * Nd * dimd * qkvd,
                lsk_gemm_qkv_rope(xn, m->wqkv[i], N, m->n_heads, m->n_kv_heads, m->head_dim, m->dim, q, m->kc[i],
                                  m->vc[i], m->cos_tab, m->sin_tab, m->tab_len, rows, pos, m->max_batch, m->max_seq,
                                  stream));
      LSK_PROF2(LSK_PROF_ATTN, attn_bytes, attn_flops,
                lsk_ragged_attn_impl(m->dtype, q, m->kc[i], m->vc[i], blocks, works, n_works, groups, n_groups,
                                     n_parts, recs, n_rounds, n_slots, rows_cap, attn, af_o, m->n_heads,
                                     m->n_kv_heads, m->head_dim, m->max_seq, scale, part, part_bytes, stream));
      LSK_PROF2(LSK_PROF_GEMM_O, es_d * (dimd * qd + Nd * qd) + pbytes(m->ks_o, dimd), 2.0 * Nd * qd * dimd,
                af_o ? lsk_gemm_partial_af(attn, m->wo[i], P, N, m->dim, qd, m->ks_o, stream)
                     : lsk_gemm_partial(attn, qd, m->wo[i], qd, P, N, m->dim, qd, m->ks_o, stream));
      const void* xi = (i == start) ? x_in : x_out;
      LSK_PROF2(LSK_PROF_NORM, norm_bytes_b + es_d * Nd * dimd + pbytes(m->ks_o, dimd), 4.0 * Nd * dimd,
                lsk_add_rmsnorm_impl(m->dtype, xi, m->dim, P, m->ks_o, m->ffn_norm[i], m->eps, x_out, m->dim, xn,
                                     m->dim, af_h, N, m->dim, stream));
      LSK_PROF2(LSK_PROF_GEMM_W13, es_d * (2.0 * ffd * dimd + Nd * dimd + Nd * ffd), 4.0 * Nd * dimd * ffd,
                af_h ? lsk_gemm_silu_af(xn, m->w13[i], h, 1, N, m->ffn, m->dim, stream)
                     : lsk_gemm(m->dtype, xn, m->dim, m->w13[i], m->dim, h, m->ffn, nullptr, 0, N, m->ffn, m->dim,
                                LSK_EPI_SILU_MUL, m->ffn, stream));
      LSK_PROF2(LSK_PROF_GEMM_W2, es_d * (dimd * ffd + Nd * ffd) + pbytes(m->ks_w2, dimd), 2.0 * Nd * ffd * dimd,
                af_h ? lsk_gemm_partial_af(h, m->w2[i], P, N, m->dim, m->ffn, m->ks_w2, stream)
                     : lsk_gemm_partial(h, m->ffn, m->w2[i], m->ffn, P, N, m->dim, m->ffn, m->ks_w2, stream));
    }
    LSK_PROF2(LSK_PROF_NORM, 2.0 * es_d * Nd * dimd + pbytes(m->ks_w2, dimd), Nd * dimd,
              lsk_add_rmsnorm(m->dtype, x_out, m->dim, P, m->ks_w2, nullptr, m->eps, x_out, m->dim, nullptr, 0, N,
                              m->dim, stream));
    if (capture && capture[end - 1]) {
      hipError_t e = hipMemcpyAsync(capture[end - 1], x_out, (size_t)N * m->dim * es, hipMemcpyDeviceToDevice, s);
      if (e != hipSuccess) { lsk_set_error("lsk_forward_layers: capture %s", hipGetErrorString(e)); return (int)e; }
    }
#undef LSK_PROF2
    return 0;
  }
  const double norm_bytes = es_d * (2.0 * Nd * dimd + dimd);
  auto gemm_bytes = [&](double M_, double Nw, double K_, double Nout, bool res) {
    return es_d * (K_ * Nw + M_ * K_ + M_ * Nout * (res ? 2.0 : 1.0));
  };
#define LSK_PROF(cls, b, f, call)                                \
  do {                                                           \
    lsk_prof_start((cls), (b), (f), stream);                     \
    if ((rc = (call))) return rc;                                \
    lsk_prof_stop(stream);                                       \
  } while (0)
  for (int i = start; i < end; ++i) {
    const void* xi = (i == start) ? x_in : x_out;
    LSK_PROF(LSK_PROF_NORM, norm_bytes, 4.0 * Nd * dimd,
             lsk_rmsnorm(m->dtype, xi, m->attn_norm[i], xn, N, m->dim, m->eps, m->dim, m->dim, stream));
    LSK_PROF(LSK_PROF_GEMM_QKV, gemm_bytes(Nd, qkvd, dimd, qkvd, false), 2.0 * Nd * dimd * qkvd,
             lsk_gemm(m->dtype, xn, m->dim, m->wqkv[i], m->dim, qkv, qd + 2 * kvd, nullptr, 0, N, qd + 2 * kvd, m->dim,
                      LSK_EPI_NONE, 0, stream));
    LSK_PROF(LSK_PROF_ROPE, es_d * 2.0 * Nd * qkvd, 6.0 * Nd * (qd + kvd),
             lsk_rope_append(m->dtype, qkv, q, m->kc[i], m->vc[i], m->cos_tab, m->sin_tab, m->tab_len, rows, pos, N,
                             m->n_heads, m->n_kv_heads, m->head_dim, m->max_batch, m->max_seq, stream));
    LSK_PROF(LSK_PROF_ATTN, attn_bytes, attn_flops,
             lsk_ragged_attn(m->dtype, q, m->kc[i], m->vc[i], blocks, works, n_works, groups, n_groups, n_parts, recs,
                             n_rounds, n_slots, rows_cap, attn, m->n_heads, m->n_kv_heads, m->head_dim, m->max_seq, scale,
                             part, part_bytes, stream));
    LSK_PROF(LSK_PROF_GEMM_O, gemm_bytes(Nd, dimd, qd, dimd, true), 2.0 * Nd * qd * dimd,
             lsk_gemm(m->dtype, attn, qd, m->wo[i], qd, x_out, m->dim, xi, m->dim, N, m->dim, qd, LSK_EPI_RESIDUAL, 0,
                      stream));
    LSK_PROF(LSK_PROF_NORM, norm_bytes, 4.0 * Nd * dimd,
             lsk_rmsnorm(m->dtype, x_out, m->ffn_norm[i], xn, N, m->dim, m->eps, m->dim, m->dim, stream));
    LSK_PROF(LSK_PROF_GEMM_W13, gemm_bytes(Nd, 2.0 * ffd, dimd, ffd, false), 4.0 * Nd * dimd * ffd,
             lsk_gemm(m->dtype, xn, m->dim, m->w13[i], m->dim, h, m->ffn, nullptr, 0, N, m->ffn, m->dim,
                      LSK_EPI_SILU_MUL, m->ffn, stream));
    LSK_PROF(LSK_PROF_GEMM_W2, gemm_bytes(Nd, dimd, ffd, dimd, true), 2.0 * Nd * ffd * dimd,
             lsk_gemm(m->dtype, h, m->ffn, m->w2[i], m->ffn, x_out, m->dim, x_out, m->dim, N, m->dim, m->ffn,
                      LSK_EPI_RESIDUAL, 0, stream));
#undef LSK_PROF
    if (capture && capture[i]) {
      hipError_t e = hipMemcpyAsync(capture[i], x_out, (size_t)N * m->dim * es, hipMemcpyDeviceToDevice, s);
      if (e != hipSuccess) { lsk_set_error("lsk_forward_layers: capture %s", hipGetErrorString(e)); return (int)e; }
    }
  }
  return 0;
}
