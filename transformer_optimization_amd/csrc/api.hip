// C-ABI entry points: host-side validation, then one launch on the caller's
// stream.  Nothing here allocates, frees or synchronises.
#include <mutex>

#include "tx_internal.hpp"

namespace tx {

int device_cu_count() {
  // Per-device cache; filled outside any stream capture (attribute queries
  // are not stream operations, so they are legal during capture as well).
  static int cache[64];
  static std::once_flag once[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  std::call_once(once[dev], [dev]() {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) v = 0;
    cache[dev] = v;
  });
  return cache[dev];
}

int64_t device_shared_mem_per_block() {
  static int64_t cache[64];
  static std::once_flag once[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  std::call_once(once[dev], [dev]() {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) v = 0;
    cache[dev] = v;
  });
  return cache[dev];
}

static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
static inline bool is16(int dt) { return dt == TX_F16 || dt == TX_BF16; }
static inline bool isdt(int dt) { return dt == TX_F32 || dt == TX_F16 || dt == TX_BF16; }

}  // namespace tx

using namespace tx;

extern "C" {

int tx_abi_version(void) { return TX_ABI_VERSION; }

const char* tx_status_string(int code) {
  switch (code) {
    case TX_OK:
      return "ok";
    case TX_EINVAL:
      return "invalid argument (null pointer, non-positive size or bad stride)";
    case TX_EUNSUPPORTED:
      return "unsupported configuration (dtype combination, alignment or head_dim)";
    case TX_EHIP:
      return "HIP launch error";
    case TX_ESCRATCH:
      return "problem exceeds the fixed scratch buffer of the no-allocation entry point "
             "(batch * heads * seq > TX_NOALLOC_MAX_STAT_ROWS)";
    default:
      return "unknown tx status";
  }
}

int tx_device_cu_count(void) { return device_cu_count(); }

int tx_eager_softmax_supported(int64_t seq, int64_t shared_mem_per_block) {
  if (shared_mem_per_block <= 0) shared_mem_per_block = device_shared_mem_per_block();
  if (shared_mem_per_block <= 0) return -1;
  return eager_softmax_mirrorable(seq, shared_mem_per_block) ? 1 : 0;
}

int tx_layernorm_residual(const void* x, const void* delta, void* x_out, void* y,
                          const void* gamma, const void* beta, const uint8_t* row_valid,
                          float* mean_out, float* rstd_out,
                          int64_t rows, int64_t d, float eps, int x_dt, int delta_dt, int y_dt,
                          int param_dt, uint32_t flags, void* stream) {
  if (!x || !y || !gamma || !beta || rows <= 0 || d <= 0 || !(eps >= 0.f)) return TX_EINVAL;
  if ((flags & TX_LN_HAS_DELTA) && !delta) return TX_EINVAL;
  if ((flags & TX_LN_WRITE_X) && !x_out) return TX_EINVAL;
  if (flags & ~63u) return TX_EINVAL;
  if (!isdt(x_dt) || !isdt(y_dt) || !isdt(param_dt)) return TX_EINVAL;
  if ((flags & TX_LN_HAS_DELTA) && delta_dt != x_dt) return TX_EUNSUPPORTED;
  if (d % 8 != 0 || d > 8192) return TX_EUNSUPPORTED;
  if (!aligned16(x) || !aligned16(y) || !aligned16(gamma) || !aligned16(beta) ||
      (delta && !aligned16(delta)) || (x_out && !aligned16(x_out)) ||
      ((uintptr_t)mean_out & 3u) || ((uintptr_t)rstd_out & 3u))
    return TX_EUNSUPPORTED;
  LayerNormArgs a{x, delta, x_out, y, gamma, beta,
                  (flags & (TX_LN_MASK_DELTA | TX_LN_MASK_X | TX_LN_MASK_OUT)) ? row_valid : nullptr,
                  mean_out, rstd_out, rows, d, eps, x_dt, y_dt, param_dt, flags};
  return launch_layernorm(a, (hipStream_t)stream);
}

int tx_gemm(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias,
            const void* residual, int64_t ldr, void* c, int64_t ldc, int64_t m, int64_t n,
            int64_t k, int ab_dt, int c_dt, int bias_dt, int res_dt, uint32_t epilogue,
            const uint8_t* row_valid, void* stream) {
  if (!a || !w || !c || m <= 0 || n <= 0 || k <= 0) return TX_EINVAL;
  if (epilogue & ~63u) return TX_EINVAL;
  if ((epilogue & TX_EPI_SPLIT_OUT) &&
      (epilogue & (TX_EPI_RESIDUAL | TX_EPI_MASK_DELTA | TX_EPI_MASK_OUT)))
    return TX_EINVAL;
  if ((epilogue & TX_EPI_SPLIT_OUT) && (ldc < 2 * n || c_dt != ab_dt)) return TX_EINVAL;
  if ((epilogue & TX_EPI_BIAS) && !bias) return TX_EINVAL;
  if ((epilogue & TX_EPI_RESIDUAL) && (!residual || ldr < n)) return TX_EINVAL;
  if (lda < k || ldw < k || ldc < n) return TX_EINVAL;
  if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff) return TX_EUNSUPPORTED;
  if (!is16(ab_dt) || !isdt(c_dt) || !isdt(bias_dt) || !isdt(res_dt)) return TX_EINVAL;
  if (k % 8 || lda % 8 || ldw % 8) return TX_EUNSUPPORTED;
  if (!aligned16(a) || !aligned16(w)) return TX_EUNSUPPORTED;
  GemmArgs g{};
  g.a = a;
  g.w = w;
  g.bias = bias;
  g.res = residual;
  g.c = c;
  g.row_valid = (epilogue & (TX_EPI_MASK_DELTA | TX_EPI_MASK_OUT)) ? row_valid : nullptr;
  g.lda = lda;
  g.ldw = ldw;
  g.ldr = ldr;
  g.ldc = ldc;
  g.m = (int)m;
  g.n = (int)n;
  g.k = (int)k;
  g.epi = epilogue;
  return launch_gemm(g, ab_dt, c_dt, bias_dt, res_dt, false, (hipStream_t)stream);
}

int tx_qkv_proj(const void* a, const void* w_qkv, const void* b_qkv, void* qk, void* vt,
                int64_t ldvt, int64_t batch, int64_t seq, int64_t d_model, int64_t heads, int dt,
                void* stream) {
  if (!a || !w_qkv || !b_qkv || !qk || !vt) return TX_EINVAL;
  if (batch <= 0 || seq <= 0 || d_model <= 0 || heads <= 0 || d_model % heads) return TX_EINVAL;
  if (ldvt < seq) return TX_EINVAL;
  if (!is16(dt)) return TX_EUNSUPPORTED;
  if (ldvt % 8 || d_model % 64) return TX_EUNSUPPORTED;
  if (batch > 0x7fffffff || seq > 0x7fffffff || d_model > 0x7fffffff) return TX_EUNSUPPORTED;
  if (batch * seq > 0x7fffffff || 3 * d_model > 0x7fffffff || batch * heads > 0x7fffffff)
    return TX_EUNSUPPORTED;
  if (!aligned16(a) || !aligned16(w_qkv) || !aligned16(vt)) return TX_EUNSUPPORTED;
  GemmArgs g{};
  g.a = a;
  g.w = w_qkv;
  g.bias = b_qkv;
  g.c = qk;
  g.lda = d_model;
  g.ldw = d_model;
  g.ldc = 2 * d_model;
  g.m = (int)(batch * seq);
  g.n = (int)(3 * d_model);
  g.k = (int)d_model;
  g.epi = TX_EPI_BIAS;
  g.vt = vt;
  g.ldvt = ldvt;
  g.qk_cols = (int)(2 * d_model);
  g.seq = (int)seq;
  g.heads = (int)heads;
  g.head_dim = (int)(d_model / heads);
  return launch_gemm(g, dt, dt, dt, dt, true, (hipStream_t)stream);
}

int tx_flash_attn_fwd_noalloc(const void* qk, const void* vt, int64_t ldvt, void* o,
                              const uint8_t* key_valid, int64_t batch, int64_t seq, int64_t heads,
                              int64_t head_dim, float scale, int causal, int softmax_mode, int dt,
                              void* stream) {
  if (batch <= 0 || seq <= 0 || heads <= 0) return TX_EINVAL;
  if (softmax_mode != TX_SOFTMAX_EAGER)  // the online softmax uses no workspace
    return tx_flash_attn_fwd(qk, vt, ldvt, o, key_valid, batch, seq, heads, head_dim, scale, causal,
                             softmax_mode, nullptr, dt, stream);
  // Each factor is bounded first, so the products cannot overflow.
  if (batch > TX_NOALLOC_MAX_STAT_ROWS || heads > TX_NOALLOC_MAX_STAT_ROWS ||
      seq > TX_NOALLOC_MAX_STAT_ROWS || batch * heads > TX_NOALLOC_MAX_STAT_ROWS ||
      batch * heads * seq > TX_NOALLOC_MAX_STAT_ROWS)
    return TX_ESCRATCH;
  float* stats = scratch_device_ptr();
  if (!stats) return TX_EHIP;
  return tx_flash_attn_fwd(qk, vt, ldvt, o, key_valid, batch, seq, heads, head_dim, scale, causal,
                           softmax_mode, stats, dt, stream);
}

int tx_flash_attn_fwd(const void* qk, const void* vt, int64_t ldvt, void* o,
                      const uint8_t* key_valid, int64_t batch, int64_t seq, int64_t heads,
                      int64_t head_dim, float scale, int causal, int softmax_mode,
                      float* row_stats, int dt, void* stream) {
  if (!qk || !vt || !o) return TX_EINVAL;
  if (batch <= 0 || seq <= 0 || heads <= 0 || head_dim <= 0 || ldvt < seq) return TX_EINVAL;
  if (!(scale > 0.f) || !(scale < 3.0e38f)) return TX_EINVAL;
  if (softmax_mode != TX_SOFTMAX_EAGER && softmax_mode != TX_SOFTMAX_ONLINE) return TX_EINVAL;
  if (softmax_mode == TX_SOFTMAX_EAGER && (!row_stats || ((uintptr_t)row_stats & 7u)))
    return TX_EINVAL;
  if (!is16(dt)) return TX_EUNSUPPORTED;
  if (head_dim != 64 && head_dim != 128) return TX_EUNSUPPORTED;
  if (ldvt % 8) return TX_EUNSUPPORTED;
  if (batch > 0x7fffffff || seq > 0x7fffffff || heads > 0x7fffffff) return TX_EUNSUPPORTED;
  if (batch * seq > 0x7fffffff || batch * heads > 0x7fffffff) return TX_EUNSUPPORTED;
  if (!aligned16(qk) || !aligned16(vt) || ((uintptr_t)o & 7u)) return TX_EUNSUPPORTED;
  // The packed layouts as strided views: q = qk[:, :D], k = qk[:, D:],
  // heads at stride head_dim; V^T rows of ldvt keys; o = [B*S, D].
  const int64_t d = heads * head_dim;
  // The K and V^T tile loaders form per-lane byte offsets within a tile in
  // 32 bits: 64 key rows of 2D elements, head_dim V^T rows of ldvt.
  if (d >= (int64_t)1 << 24 || head_dim * ldvt * 2 + 256 > (int64_t)0xffffffff) return TX_EUNSUPPORTED;
  // o is written while other workgroups still read q, k and v.
  {
    const int64_t qk_bytes = batch * seq * 2 * d * 2, vt_bytes = batch * heads * head_dim * ldvt * 2;
    const int64_t o_bytes = batch * seq * d * 2;
    if (spans_overlap((uintptr_t)o, o_bytes, (uintptr_t)qk, qk_bytes) ||
        spans_overlap((uintptr_t)o, o_bytes, (uintptr_t)vt, vt_bytes))
      return TX_EINVAL;
  }
  AttnArgs at{};
  at.q = qk;
  at.k = (const char*)qk + d * 2;  // 16-bit elements
  at.v = vt;
  at.o = o;
  at.q_sb = at.k_sb = seq * 2 * d;
  at.q_sh = at.k_sh = head_dim;
  at.q_ss = at.k_ss = 2 * d;
  at.v_sb = heads * head_dim * ldvt;
  at.v_sh = head_dim * ldvt;
  at.v_ss = 0;
  at.o_sb = seq * d;
  at.o_sh = head_dim;
  at.o_ss = d;
  at.key_valid = key_valid;
  at.kv_sb = seq;
  at.vnat = 0;
  at.ldvt = ldvt;
  at.batch = (int)batch;
  at.seq = (int)seq;
  at.heads = (int)heads;
  at.head_dim = (int)head_dim;
  at.scale = scale;
  at.causal = causal ? 1 : 0;
  at.softmax_mode = softmax_mode;
  at.row_stats = row_stats;
  return launch_attention(at, dt, (hipStream_t)stream);
}

int tx_flash_attn_fwd_strided(const void* q, const void* k, const void* v, void* o,
                              const int64_t* q_strides, const int64_t* k_strides,
                              const int64_t* v_strides, const int64_t* o_strides,
                              const uint8_t* key_valid, int64_t key_valid_sb, int64_t batch,
                              int64_t heads, int64_t seq, int64_t head_dim, float scale, int causal,
                              int softmax_mode, float* row_stats, int dt, void* stream) {
  if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides) return TX_EINVAL;
  if (batch <= 0 || seq <= 0 || heads <= 0 || head_dim <= 0) return TX_EINVAL;
  if (!(scale > 0.f) || !(scale < 3.0e38f)) return TX_EINVAL;
  if (softmax_mode != TX_SOFTMAX_EAGER && softmax_mode != TX_SOFTMAX_ONLINE) return TX_EINVAL;
  if (softmax_mode == TX_SOFTMAX_EAGER && (!row_stats || ((uintptr_t)row_stats & 7u)))
    return TX_EINVAL;
  if (key_valid && key_valid_sb < seq) return TX_EINVAL;
  const int64_t* in_strides[3] = {q_strides, k_strides, v_strides};
  for (int t = 0; t < 3; ++t) {
    const int64_t* st = in_strides[t];
    if (st[0] < 0 || st[1] < 0 || st[2] < 0) return TX_EINVAL;
    if (st[3] != 1) return TX_EUNSUPPORTED;  // head_dim must be contiguous
    // 16-byte rows for the 128-bit loads and the DMA; row offsets of a tile
    // are 32-bit byte offsets (64 rows).
    if (st[0] % 8 || st[1] % 8 || st[2] % 8 || st[2] >= (1 << 24)) return TX_EUNSUPPORTED;
  }
  if (o_strides[0] < 0 || o_strides[1] < 0 || o_strides[2] < head_dim) return TX_EINVAL;
  if (o_strides[3] != 1 || o_strides[0] % 4 || o_strides[1] % 4 || o_strides[2] % 4)
    return TX_EUNSUPPORTED;
  if (!is16(dt)) return TX_EUNSUPPORTED;
  if (head_dim != 64 && head_dim != 128) return TX_EUNSUPPORTED;
  if (batch > 0x7fffffff || seq > 0x7fffffff || heads > 0x7fffffff) return TX_EUNSUPPORTED;
  if (batch * seq > 0x7fffffff || batch * heads > 0x7fffffff) return TX_EUNSUPPORTED;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || ((uintptr_t)o & 7u)) return TX_EUNSUPPORTED;
  // Every (b, h, s) output row is written by one workgroup: distinct rows
  // may not share elements (o_strides[1] = 0 would make every head's
  // workgroups race on one row), and o may not share memory with q, k or v,
  // which other workgroups still read while it is written.
  if (!view_is_nonoverlapping(o_strides, batch, heads, seq, head_dim)) return TX_EINVAL;
  {
    const int64_t* views[4] = {q_strides, k_strides, v_strides, o_strides};
    const void* ptrs[4] = {q, k, v, o};
    int64_t bytes[4];
    for (int t = 0; t < 4; ++t) {
      const int64_t mo = view_max_offset(views[t], batch, heads, seq, head_dim);
      if (mo < 0) return TX_EUNSUPPORTED;
      bytes[t] = (mo + 1) * 2;
    }
    for (int t = 0; t < 3; ++t)
      if (spans_overlap((uintptr_t)o, bytes[3], (uintptr_t)ptrs[t], bytes[t])) return TX_EINVAL;
  }
  AttnArgs at{};
  at.q = q;
  at.k = k;
  at.v = v;
  at.o = o;
  at.q_sb = q_strides[0];
  at.q_sh = q_strides[1];
  at.q_ss = q_strides[2];
  at.k_sb = k_strides[0];
  at.k_sh = k_strides[1];
  at.k_ss = k_strides[2];
  at.v_sb = v_strides[0];
  at.v_sh = v_strides[1];
  at.v_ss = v_strides[2];
  at.o_sb = o_strides[0];
  at.o_sh = o_strides[1];
  at.o_ss = o_strides[2];
  at.key_valid = key_valid;
  at.kv_sb = key_valid_sb;
  at.vnat = 1;
  at.ldvt = 0;
  at.batch = (int)batch;
  at.seq = (int)seq;
  at.heads = (int)heads;
  at.head_dim = (int)head_dim;
  at.scale = scale;
  at.causal = causal ? 1 : 0;
  at.softmax_mode = softmax_mode;
  at.row_stats = row_stats;
  return launch_attention(at, dt, (hipStream_t)stream);
}

}  // extern "C"
