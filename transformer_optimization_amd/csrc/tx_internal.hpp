// Internal launcher interface between the C-ABI layer (api.hip) and the
// kernel translation units.  Arguments arrive here already validated.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "limits.hpp"
#include "tx_api.h"

namespace tx {

struct LayerNormArgs {
  const void* x;
  const void* delta;
  void* x_out;
  void* y;
  const void* gamma;
  const void* beta;
  const uint8_t* row_valid;
  float* mean_out;
  float* rstd_out;
  int64_t rows;
  int64_t d;
  float eps;
  int x_dt, y_dt, param_dt;
  uint32_t flags;
};

struct GemmArgs {
  const void* a;
  const void* w;
  const void* bias;
  const void* res;
  void* c;
  const uint8_t* row_valid;
  int64_t lda, ldw, ldr, ldc;
  int m, n, k;
  uint32_t epi;
  // Packed-QKV split store (tx_qkv_proj): columns >= qk_cols go to vt.
  void* vt;
  int64_t ldvt;
  int qk_cols;  // 2 * d_model
  int seq;
  int heads;
  int head_dim;
  int group;  // tile rows per band of the tile order (set by launch_gemm)
  int stage16;  // 1: gemm_hp_kernel's 16-byte staged epilogue (set by launch_hp)
};

// Attention operands as strided [batch, head, seq, head_dim] views (element
// strides sb / sh / ss; head_dim contiguous).  V is either natural
// (vnat = 1: v[b, h, s, d] = v + b*v_sb + h*v_sh + s*v_ss + d) or head-
// transposed (vnat = 0: v[b, h, s, d] = v + b*v_sb + h*v_sh + d*ldvt + s).
struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  const uint8_t* key_valid;  // key_valid[b * kv_sb + s]; nullptr = all valid
  int64_t kv_sb;
  int vnat;
  int64_t ldvt;              // vnat = 0: keys per transposed row
  int batch, seq, heads, head_dim;
  float scale;
  int causal;
  int softmax_mode;   // TX_SOFTMAX_EAGER or TX_SOFTMAX_ONLINE
  float* row_stats;   // eager mode: [B*H*S][2] (max, sum) workspace
};

int launch_layernorm(const LayerNormArgs& a, hipStream_t st);
int launch_gemm(const GemmArgs& g, int ab_dt, int c_dt, int bias_dt, int res_dt, bool qkv,
                hipStream_t st);
int launch_attention(const AttnArgs& a, int dt, hipStream_t st);
int device_cu_count();
// Shared memory per block of the current device, as the HIP runtime reports
// it to every library on the device (0 if it cannot be queried).
int64_t device_shared_mem_per_block();
// Device address of the current device's fixed attention scratch
// (2 * TX_NOALLOC_MAX_STAT_ROWS floats); nullptr if it cannot be resolved.
float* scratch_device_ptr();

}  // namespace tx
