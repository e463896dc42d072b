/*
 * tx_api.h -- C ABI of the MI355X (gfx950) transformer-block forward library
 * (libtx_hip.so).  Plain pointers, sizes and a hipStream_t passed as void*;
 * no torch types.  The Python host (transformer_optimization_amd/_C.py)
 * binds these with ctypes.
 *
 * The reference (namsengi11/transformer_optimization) is pure Python; its hot
 * path calls Triton kernels through Python wrappers.  Each entry point below
 * replaces one such wrapper (or an ATen call site) and names it.
 * TTB = torch_transformer_benchmark.py.
 *
 * Contract shared by every entry point:
 *  - the caller owns every buffer; the library never allocates or frees
 *    device memory and never synchronises;
 *  - work is enqueued on `stream` (a hipStream_t; NULL = legacy default
 *    stream) and is capturable into a hipGraph;
 *  - arguments are validated on the host before anything is enqueued:
 *    TX_EINVAL for null pointers / non-positive sizes / bad strides,
 *    TX_EUNSUPPORTED for valid arguments outside what the kernels implement
 *    (dtype combination, alignment, head_dim), TX_EHIP when a launch fails;
 *  - no C++ exception crosses the ABI.
 */
#ifndef TX_API_H
#define TX_API_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TX_ABI_VERSION 4

typedef enum {
  TX_OK = 0,
  TX_EINVAL = 1,
  TX_EUNSUPPORTED = 2,
  TX_EHIP = 3,
  TX_ESCRATCH = 4 /* larger than the fixed scratch of tx_flash_attn_fwd_noalloc */
} tx_status;
typedef enum { TX_F32 = 0, TX_F16 = 1, TX_BF16 = 2 } tx_dtype;

/* tx_layernorm_residual flags (mirror the reference's MASK_DELTA / MASK_X /
 * MASK_OUT / WRITE_X constexpr flags, TTB:884-962). */
#define TX_LN_HAS_DELTA  1u  /* x' = round_x(x + delta)                     */
#define TX_LN_MASK_DELTA 2u  /* invalid rows: delta treated as 0             */
#define TX_LN_MASK_X     4u  /* invalid rows: x' := 0                        */
#define TX_LN_MASK_OUT   8u  /* invalid rows: y := 0                         */
#define TX_LN_WRITE_X   16u  /* store x' into x_out                          */
#define TX_LN_SPLIT_Y   32u  /* y rows hold 2d values: hi = round_y(v) in
                                 [0, d), lo = round_y(v - hi) in [d, 2d)     */

/* tx_gemm epilogue flags. */
#define TX_EPI_BIAS       1u  /* v = acc + bias[n], rounded to the C dtype          */
#define TX_EPI_GELU_ERF   2u  /* v = round(gelu_erf(float(v)))  (after the bias)    */
#define TX_EPI_RESIDUAL   4u  /* v = round(residual[m,n] + float(v))                */
#define TX_EPI_MASK_DELTA 8u  /* row_valid[m]==0: the GEMM term is dropped          */
#define TX_EPI_MASK_OUT  16u  /* row_valid[m]==0: the stored value is 0             */
#define TX_EPI_SPLIT_OUT 32u  /* no intermediate rounding: v = [gelu](acc + bias) in
                                 fp32, stored as hi = round(v) at [m, n] and
                                 lo = round(v - hi) at [m, n + N] (ldc >= 2N)    */

/* Library version; bumped whenever a signature or flag meaning changes. */
int tx_abi_version(void);

/* Static, human-readable text for a tx_status value. */
const char* tx_status_string(int code);

/* Number of compute units of the current device (0 on error); used by the
 * host to size launches.  No reference counterpart. */
int tx_device_cu_count(void);

/*
 * Whether tx_flash_attn_fwd / _strided / _noalloc with TX_SOFTMAX_EAGER serve
 * rows of `seq` keys: 1 yes, 0 no (they return TX_EUNSUPPORTED), -1 when the
 * device cannot be queried.  The eager chain's fp32 softmax (TTB:187) runs
 * ATen's wave softmax for rows of up to 2048 keys (always reproduced) and
 * its 512-thread block softmax above; the block softmax's reduction order is
 * reproduced for seq a multiple of 4 up to 65536 that fits the block's
 * shared-memory row copy (seq < (shared_mem_per_block - 32) / 4), or whose
 * uncached pass maps threads to keys the same way (seq a multiple of 2048).
 * shared_mem_per_block <= 0: the current device's value.  Used by the host
 * to pick the numeric policy per sequence length (the reference picks its
 * route per call, TTB:3509-3611); no direct reference counterpart.
 */
int tx_eager_softmax_supported(int64_t seq, int64_t shared_mem_per_block);

/*
 * Residual add + LayerNorm over `rows` contiguous rows of `d` elements.
 * Replaces _triton_add_layernorm / _add_ln_kernel (TTB:1038-1108, 884-962)
 * and the ATen fallback of _ln_site (TTB:3940-4001):
 *   x' = [MASK_X] ( round_x( x + [MASK_DELTA] delta ) )      (HAS_DELTA)
 *   x' = x                                                    (otherwise)
 *   y  = [MASK_OUT] round_y( (x' - mean) * rstd * gamma + beta ),
 * with fp32 moments and rstd = 1/sqrt(var + eps) (biased variance), reduced
 * in the order of ATen's vectorized LayerNorm so that results are bitwise
 * those of nn.LayerNorm.  mean_out / rstd_out (nullable, fp32 [rows]) receive
 * the row statistics, as torch.native_layer_norm returns them.
 * Pointers must be 16-byte aligned and d a multiple of 8.
 * row_valid may be NULL (all rows valid); it is read only when a MASK flag
 * is set.  dtypes: x/x_out x_dt, delta delta_dt, y y_dt, gamma/beta param_dt
 * (param_dt = y_dt when x is fp32 and y is 16-bit).  SPLIT_Y writes y as a
 * [rows, 2d] hi/lo pair for the two-term GEMM operand of the fp32-residual
 * policy.
 */
int tx_layernorm_residual(const void* x, const void* delta, void* x_out, void* y,
                          const void* gamma, const void* beta, const uint8_t* row_valid,
                          float* mean_out, float* rstd_out,
                          int64_t rows, int64_t d, float eps,
                          int x_dt, int delta_dt, int y_dt, int param_dt,
                          uint32_t flags, void* stream);

/*
 * C[m, n] = epilogue( sum_k A[m, k] * W[n, k] )   for m < M, n < N.
 * A is row-major [M, K] with row stride lda; W is nn.Linear storage [N, K]
 * with row stride ldw; C and residual are row-major with strides ldc / ldr.
 * Replaces F.linear on the hot path (TTB:4067-4068, 4169, 4192-4194,
 * 4221, 4296, 4311-4312) and _triton_linear / _triton_gemm_gelu
 * (TTB:1860-1880, 1754-1803): bf16/fp16 operands on MFMA with fp32
 * accumulation; the accumulator is rounded to the C dtype after the bias and
 * before GELU and the residual add, as the eager chain rounds.
 * Supported (ab_dt, c_dt, bias_dt, res_dt): all four equal to bf16 or to
 * fp16 (the eager rounding chain); and, for the fp32-residual policy,
 * c_dt = res_dt = fp32 or c_dt = fp32 with res_dt = ab_dt (fp32 residual
 * stream, no rounding of the GEMM term), and c_dt = ab_dt with SPLIT_OUT.
 * bias_dt = ab_dt.  K, lda, ldw multiples of 8; A and W 16-byte aligned.
 * Any lda / ldw >= K is accepted: shapes whose 256-row tile offsets exceed
 * 32 bits ((255 * max(lda, ldw) + 56) * element size > 2^31 - 1) run on the
 * kernel with 64-bit addressing instead of the 256-row one (same bits).
 */
int tx_gemm(const void* a, int64_t lda, const void* w, int64_t ldw,
            const void* bias, const void* residual, int64_t ldr,
            void* c, int64_t ldc, int64_t m, int64_t n, int64_t k,
            int ab_dt, int c_dt, int bias_dt, int res_dt, uint32_t epilogue,
            const uint8_t* row_valid, void* stream);

/*
 * Packed Q/K/V projection: [M, 3D] = A[M, D] * W_qkv[3D, D]^T + b_qkv, with
 * M = batch*seq, W_qkv = cat(Wq, Wk, Wv) and b_qkv = cat(bq, bk, bv).
 * Replaces _get_fused_qkv_weights + _lin(normed, W_qkv, b_qkv)
 * (TTB:440-504, 4220-4222) and _split_heads_3 (TTB:507-597): q and k are
 * stored row-major into qk[M, 2D] (q in columns [0, D), k in [D, 2D));
 * v is stored head-transposed into vt[batch][heads][head_dim][ldvt]
 * (sequence index contiguous), the layout the attention kernel reads.
 * Each value is round(acc + bias) in dt, as F.linear produces.
 * ldvt >= seq and a multiple of 8; d_model a multiple of 64.
 */
int tx_qkv_proj(const void* a, const void* w_qkv, const void* b_qkv,
                void* qk, void* vt, int64_t ldvt,
                int64_t batch, int64_t seq, int64_t d_model, int64_t heads,
                int dt, void* stream);

/*
 * Flash-attention forward over the tx_qkv_proj layouts:
 *   o[b*seq + i, h*hd + :] = sum_j P[i, j] * v[b, h, j, :]
 *   s = round(round(q_i . k_j) * scale); masked -> -inf;  P = softmax_j(s).
 * Replaces BaselineSelfAttention's matmul/scale/mask/softmax/matmul chain
 * (TTB:161-194), the reference's _flash_attn_kernel / _dispatch_attn
 * (TTB:1313-1418, 1596-1693) and its manual bit-exact route
 * (TTB:4257-4295).  Masks: causal (key j > query i) and key_valid[b*seq+j]==0
 * (NULL = all valid).  A query row with no admissible key gets 0.
 * head_dim in {64, 128}; o is row-major [batch*seq, heads*head_dim] and
 * must not overlap qk or vt (TX_EINVAL); heads*head_dim < 2^24 and
 * head_dim * ldvt * 2 + 256 <= 2^32 - 1 (32-bit tile offsets), else
 * TX_EUNSUPPORTED.
 *
 * softmax_mode TX_SOFTMAX_EAGER reproduces the eager fp32 softmax bit for bit
 * (row max, then the row sum of expf(s - max) in ATen's reduction order,
 * p = round(softmax), o = round(P V) accumulated in key order); it needs
 * row_stats, an fp32 workspace of 2*batch*heads*seq floats (scratch for the
 * row max and sum; its contents on return are unspecified: the kernels that
 * keep a row in registers do not write it).  TX_SOFTMAX_ONLINE is a one-pass
 * online softmax over fp32 scores (o = round(sum exp(s-m) v / sum exp(s-m)),
 * p rounded to dt only as the MFMA operand) and ignores row_stats.
 * TX_SOFTMAX_EAGER serves the lengths tx_eager_softmax_supported accepts
 * (every seq <= 2048; above, multiples of 4 up to 65536 under the rule given
 * there); other lengths return TX_EUNSUPPORTED.
 */
#define TX_SOFTMAX_EAGER  0
#define TX_SOFTMAX_ONLINE 1
int tx_flash_attn_fwd(const void* qk, const void* vt, int64_t ldvt, void* o,
                      const uint8_t* key_valid,
                      int64_t batch, int64_t seq, int64_t heads, int64_t head_dim,
                      float scale, int causal, int softmax_mode, float* row_stats,
                      int dt, void* stream);

/*
 * Attention over strided [batch, heads, seq, head_dim] views, the contract of
 * the reference's _triton_short_attention(q, k, v, scale, causal,
 * mask_active, valid_token_mask) / _dispatch_attn (TTB:1596-1620, 1641-1668),
 * which receives q / k / v as column slices of the packed [B, S, 3D]
 * projection and returns merged heads.  Element (b, h, s, d) of q is
 * q[b*q_strides[0] + h*q_strides[1] + s*q_strides[2] + d] (likewise k, v, o;
 * strides in elements, strides[3] must be 1).  Same computation, masks,
 * softmax modes, row_stats workspace and results as tx_flash_attn_fwd
 * (o = merged-head context when o_strides describe [B, S, H, hd]).
 * key_valid[b * key_valid_sb + j] == 0 marks key j of batch b invalid (NULL =
 * all valid).  q / k / v: 16-byte aligned, strides[0..2] multiples of 8 and
 * strides[2] < 2^24; o: 8-byte aligned, strides multiples of 4,
 * o_strides[2] >= head_dim; o's rows may not share elements (with its
 * extent-1 dimensions dropped and the rest in ascending stride order, each
 * stride reaches past what the smaller ones cover) and o must not overlap
 * q, k or v (all TX_EINVAL).
 */
int tx_flash_attn_fwd_strided(const void* q, const void* k, const void* v, void* o,
                              const int64_t q_strides[4], const int64_t k_strides[4],
                              const int64_t v_strides[4], const int64_t o_strides[4],
                              const uint8_t* key_valid, int64_t key_valid_sb,
                              int64_t batch, int64_t heads, int64_t seq, int64_t head_dim,
                              float scale, int causal, int softmax_mode, float* row_stats,
                              int dt, void* stream);

/*
 * tx_flash_attn_fwd without a caller-provided workspace: the same
 * computation, arguments and results as tx_flash_attn_fwd, with the eager
 * softmax's row statistics kept in a fixed device array of the library
 * (2 * TX_NOALLOC_MAX_STAT_ROWS floats, 8 MiB, one copy per device, held from
 * module load to process end).  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under hipGraph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  It calls no
 * allocating routine.  batch * heads * seq above TX_NOALLOC_MAX_STAT_ROWS
 * returns TX_ESCRATCH without launching.  All calls on one device share the
 * array: calls that overlap on one device (concurrent streams or threads)
 * race and must be serialised by the caller.  TX_SOFTMAX_ONLINE needs no
 * workspace and is forwarded unchanged.
 */
#define TX_NOALLOC_MAX_STAT_ROWS (1 << 20)
int tx_flash_attn_fwd_noalloc(const void* qk, const void* vt, int64_t ldvt, void* o,
                              const uint8_t* key_valid,
                              int64_t batch, int64_t seq, int64_t heads, int64_t head_dim,
                              float scale, int causal, int softmax_mode, int dt, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TX_API_H */
