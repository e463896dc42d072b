// Flash-attention forward for gfx950 on v_mfma_f32_32x32x16_{bf16,f16}.
//
// Replaces BaselineSelfAttention's eager chain (TTB:161-194), the reference's
// _flash_attn_kernel (TTB:1313-1418) and its bit-exact manual route
// (TTB:4257-4295).  Inputs are the layouts tx_qkv_proj writes: q and k
// row-major in qk[B*S, 2D] (q columns [0,D), k columns [D,2D)), v
// head-transposed in vt[B][H][hd][ldvt].  Output o[B*S, D] with heads merged.
//
// Common structure: a workgroup of 4 waves owns 128 query rows of one
// (batch, head); each wave owns 32 of them.  Key tiles of 64 rows stream
// through two LDS stages (K as [key][d], V^T as [d][key], 16-byte chunks
// XOR-swizzled by row); the next tile is fetched from HBM into registers
// while the current one is consumed.  Scores are computed transposed,
// S^T = K Q^T (keys = MFMA rows, queries = MFMA columns), so every lane holds
// 32 of the 64 scores of one query row and row reductions need one exchange
// with lane ^ 32.  Probabilities become the B operand of O^T = V^T P^T after a
// v_permlane32_swap that gives lane half g the keys 8g..8g+7 of each 16-key
// step (the MFMA sums k in 8-element groups, in group order, so keys stay in
// their natural order and the product equals an in-order K loop).
//
// Two softmax modes:
//
// * TX_SOFTMAX_EAGER (bit-exact with the eager chain, TTB:173-188):
//     s = round(round(q.k) * scale), masked -> -inf,
//     p = round(softmax_fp32(s)), o = round(sum_j p_j v_j).
//   attn_stats_kernel computes per row the max m and the sum l of expf(s - m)
//   in exactly the reduction order of ATen's fp32 softmax on ROCm (the wave
//   softmax for S <= 1024: per-lane sums of keys j = lane + 64*it, then an
//   xor butterfly; the 512-thread block softmax for longer rows: per-thread
//   sums over 4-key vectors, shuffle-down trees per wave and across waves).
//   attn_pv_kernel then forms p exactly as ATen does (expf(s-m)/l, or
//   __expf(s-m) * (1/l) for the block softmax) and accumulates P V in key
//   order.  Three passes of QK^T per row block instead of one.
//
// * TX_SOFTMAX_ONLINE (one pass): the running max is re-based only when it
//   grows by more than 2^8 in p; p = exp(s - m_running) is rounded for the
//   MFMA and o = round(sum p v / sum p).  Used where no eager baseline exists.
#include <cstdlib>
#include <type_traits>

#include "common.hpp"
#include "tx_internal.hpp"

namespace tx {

constexpr int ATT_BQ = 128;   // query rows per workgroup
constexpr int ATT_BN = 64;    // keys per tile
constexpr int ATT_THREADS = 256;

__device__ __forceinline__ int swz8(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int swz16(int r) { return r & 15; }

// Workgroup -> (batch*head, query block), XCD-aware: each XCD receives a
// contiguous run of work so blocks sharing a head's K/V share an L2.
__device__ __forceinline__ void attn_work_of(int nq, int causal, int& bh, int& qb) {
  int pid = blockIdx.x;
  const int nwg = gridDim.x;
  const int x = pid & 7, i = pid >> 3, q = nwg >> 3, r = nwg & 7;
  pid = x * q + (x < r ? x : r) + i;
  bh = pid / nq;
  qb = pid - bh * nq;
  if (causal) qb = nq - 1 - qb;  // longest rows first
}

// Per-workgroup context shared by the kernels.
template <typename T, int HD>
struct AttnTile {
  typedef typename Mfma<T>::vec vec;
  static constexpr int KCH = HD / 8;                       // 16-byte chunks per K row
  static constexpr int K_LD = ATT_BN * KCH / ATT_THREADS;  // K chunks per thread per tile
  static constexpr int V_LD = HD * 8 / ATT_THREADS;        // V^T chunks per thread per tile
  static constexpr int NDT = HD / 32;
  static constexpr int NKS = HD / 16;

  const T* kbase;
  const T* vbase;
  int64_t ldqk, ldvt;
  int S;
  u32x4 rk[K_LD], rv[V_LD];

  __device__ __forceinline__ void gload_k(int kt, int tid) {
    const int kt0 = kt * ATT_BN;
#pragma unroll
    for (int i = 0; i < K_LD; ++i) {
      const int idx = tid + i * ATT_THREADS, key = idx / KCH, cc = idx % KCH;
      rk[i] = (kt0 + key < S) ? ld128(kbase + (int64_t)(kt0 + key) * ldqk + cc * 8)
                              : u32x4{0u, 0u, 0u, 0u};
    }
  }
  __device__ __forceinline__ void gload_v(int kt, int tid) {
    const int kt0 = kt * ATT_BN;
#pragma unroll
    for (int i = 0; i < V_LD; ++i) {
      const int idx = tid + i * ATT_THREADS, d = idx >> 3, cc = idx & 7;
      const int k0 = kt0 + cc * 8;
      u32x4 v = u32x4{0u, 0u, 0u, 0u};
      if (k0 < S) {
        // In bounds: ldvt >= S is a multiple of 8, so a chunk that starts
        // below S ends inside the row.  Keys >= S are zeroed (p = 0 there,
        // and 0 * garbage could be NaN).
        v = ld128(vbase + (int64_t)d * ldvt + k0);
        if (k0 + 8 > S) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int kk = k0 + 2 * e;
            uint32_t w = v[e];
            if (kk >= S) w &= 0xffff0000u;
            if (kk + 1 >= S) w &= 0x0000ffffu;
            v[e] = w;
          }
        }
      }
      rv[i] = v;
    }
  }
  __device__ __forceinline__ void lstore_k(T* Ks, int tid) {
#pragma unroll
    for (int i = 0; i < K_LD; ++i) {
      const int idx = tid + i * ATT_THREADS, key = idx / KCH, cc = idx % KCH;
      const int phys = (KCH >= 16) ? (cc ^ swz16(key)) : (cc ^ swz8(key));
      st128(Ks + key * HD + phys * 8, rk[i]);
    }
  }
  __device__ __forceinline__ void lstore_v(T* Vs, int tid) {
#pragma unroll
    for (int i = 0; i < V_LD; ++i) {
      const int idx = tid + i * ATT_THREADS, d = idx >> 3, cc = idx & 7;
      st128(Vs + d * ATT_BN + ((cc ^ swz8(d)) << 3), rv[i]);
    }
  }
};

// S^T for the 64 keys of a tile: s[t] holds keys 32t + mfma32_row(r, lane)
// for query column lane & 31 (raw fp32 accumulators).
template <typename T, int HD>
__device__ __forceinline__ void scores_tile(const T* Ks, const typename Mfma<T>::vec* qf, int lane,
                                            f32x16* s) {
  typedef typename Mfma<T>::vec vec;
  constexpr int KCH = HD / 8, NKS = HD / 16;
  const int col = lane & 31, half = lane >> 5;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[t][r] = 0.f;
    const int key = 32 * t + col;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int ch = 2 * ks + half;
      const int phys = (KCH >= 16) ? (ch ^ swz16(key)) : (ch ^ swz8(key));
      vec kf = *reinterpret_cast<const vec*>(Ks + key * HD + phys * 8);
      s[t] = Mfma<T>::mma32(kf, qf[ks], s[t]);
    }
  }
}

// The eager score: round(round(acc) * scale); the second rounding is exact
// and skipped when scale is a power of two.
template <typename T, bool EXACT_SCALE>
__device__ __forceinline__ float eager_score(float acc, float scale) {
  const float v = round_to<T>(acc);
  return EXACT_SCALE ? v * scale : round_to<T>(v * scale);
}

// Key-validity bits of a tile (bit k = key kt0 + k exists and is valid).
__device__ __forceinline__ uint64_t tile_key_mask(const uint8_t* kv, int kt0, int S, int lane) {
  return __ballot((kt0 + lane < S) && (kv == nullptr || kv[kt0 + lane] != 0));
}

// P^T operand for MFMA step u (keys 16u..16u+15 of the tile) from eight
// probabilities of this lane (keys 32t + 8(r>>2) + 4g + (r&3), r in [8h, 8h+8),
// t = u>>1, h = u&1).  After the swap lane half g holds keys 8g..8g+7.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::vec pack_p(const float* p8) {
  const uint32_t a0 = pack2<T>(p8[0], p8[1]), a1 = pack2<T>(p8[2], p8[3]);  // keys +0..3 (+4 for g=1)
  const uint32_t b0 = pack2<T>(p8[4], p8[5]), b1 = pack2<T>(p8[6], p8[7]);  // keys +8..11 (+12 for g=1)
  // Swap lanes 32-63 of the first operand with lanes 0-31 of the second.
  auto s0 = __builtin_amdgcn_permlane32_swap(a0, b0, false, false);
  auto s1 = __builtin_amdgcn_permlane32_swap(a1, b1, false, false);
  // g=0: s0[0] = keys 0,1  s1[0] = 2,3  s0[1] = 4,5  s1[1] = 6,7
  // g=1: s0[0] = keys 8,9  s1[0] = 10,11 s0[1] = 12,13 s1[1] = 14,15
  u32x4 pk = u32x4{(uint32_t)s0[0], (uint32_t)s1[0], (uint32_t)s0[1], (uint32_t)s1[1]};
  return __builtin_bit_cast(typename Mfma<T>::vec, pk);
}

template <typename T, int HD>
__device__ __forceinline__ void load_q(const T* qk, int64_t ldqk, int64_t tok0, int myq, int S, int h,
                                       int half, typename Mfma<T>::vec* qf) {
  typedef typename Mfma<T>::vec vec;
  const T* qrow = qk + (tok0 + myq) * ldqk + h * HD + 8 * half;
#pragma unroll
  for (int ks = 0; ks < HD / 16; ++ks) {
    u32x4 v = myq < S ? ld128(qrow + 16 * ks) : u32x4{0u, 0u, 0u, 0u};
    qf[ks] = __builtin_bit_cast(vec, v);
  }
}

template <typename T, int HD>
__device__ __forceinline__ void store_o(const f32x16* o_acc, float scale_out, T* orow, int half) {
#pragma unroll
  for (int dt = 0; dt < HD / 32; ++dt) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d0 = 32 * dt + 8 * q4 + 4 * half;
      u32x2 pk;
      pk[0] = pack2<T>(o_acc[dt][4 * q4 + 0] * scale_out, o_acc[dt][4 * q4 + 1] * scale_out);
      pk[1] = pack2<T>(o_acc[dt][4 * q4 + 2] * scale_out, o_acc[dt][4 * q4 + 3] * scale_out);
      st64(orow + d0, pk);
    }
  }
}

__device__ __forceinline__ int attn_n_tiles(int S, int causal, int q0) {
  int n = (S + ATT_BN - 1) / ATT_BN;
  if (causal) {
    const int last_q = (q0 + ATT_BQ - 1) < (S - 1) ? (q0 + ATT_BQ - 1) : (S - 1);
    const int need = last_q / ATT_BN + 1;
    n = need < n ? need : n;
  }
  return n;
}

// =========================================================== online (1 pass)
template <typename T, int HD, bool EXACT_SCALE>
__global__ __launch_bounds__(ATT_THREADS) void attn_online_kernel(AttnArgs a) {
  typedef typename Mfma<T>::vec vec;
  typedef AttnTile<T, HD> Tile;
  __shared__ __attribute__((aligned(16))) T ks_lds[2][ATT_BN * HD];
  __shared__ __attribute__((aligned(16))) T vs_lds[2][HD * ATT_BN];

  const int S = a.seq, H = a.heads, D = H * HD;
  const int nq = (S + ATT_BQ - 1) / ATT_BQ;
  int bh, qb;
  attn_work_of(nq, a.causal, bh, qb);
  const int b = bh / H, h = bh - b * H;
  const int q0 = qb * ATT_BQ;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5;
  const int q0w = q0 + wave * 32, myq = q0w + (lane & 31);
  const int64_t tok0 = (int64_t)b * S;

  Tile tl;
  tl.S = S;
  tl.ldqk = 2 * (int64_t)D;
  tl.ldvt = a.ldvt;
  tl.kbase = (const T*)a.qk + tok0 * tl.ldqk + D + h * HD;
  tl.vbase = (const T*)a.vt + (int64_t)bh * HD * a.ldvt;

  vec qf[HD / 16];
  load_q<T, HD>((const T*)a.qk, tl.ldqk, tok0, myq, S, h, half, qf);

  const int n_tiles = attn_n_tiles(S, a.causal, q0);
  f32x16 o_acc[HD / 32];
#pragma unroll
  for (int t = 0; t < HD / 32; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[t][r] = 0.f;

  const float NEG_INF = -__builtin_inff();
  const float LOG2E = 1.4426950408889634f;
  const float TAU = 5.545177444479562f;  // 8 ln 2: p stays <= 2^8
  float m_run = NEG_INF, l_part = 0.f;
  const uint8_t* kv = a.key_valid ? a.key_valid + tok0 : nullptr;

  if (n_tiles > 0) {
    tl.gload_k(0, tid);
    tl.gload_v(0, tid);
    tl.lstore_k(ks_lds[0], tid);
    tl.lstore_v(vs_lds[0], tid);
  }
  __syncthreads();
  for (int kt = 0; kt < n_tiles; ++kt) {
    const int st = kt & 1, kt0 = kt * ATT_BN;
    if (kt + 1 < n_tiles) {
      tl.gload_k(kt + 1, tid);
      tl.gload_v(kt + 1, tid);
    }
    f32x16 s[2];
    scores_tile<T, HD>(ks_lds[st], qf, lane, s);

    const uint64_t kmask = tile_key_mask(kv, kt0, S, lane);
    const bool need_mask = (a.causal && (kt0 + ATT_BN - 1 > q0w)) || (kmask != ~0ull);
    float mx = NEG_INF;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = eager_score<T, EXACT_SCALE>(s[t][r], a.scale);
        if (need_mask) {
          const int kr = 32 * t + mfma32_row(r, lane);
          const bool ok = ((kmask >> kr) & 1ull) && !(a.causal && kt0 + kr > myq);
          v = ok ? v : NEG_INF;
        }
        s[t][r] = v;
        mx = fmaxf(mx, v);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (__any(mx > m_run + TAU)) {
      const float m_new = fmaxf(m_run, mx);
      const float corr = (m_new == NEG_INF) ? 1.f : exp2f((m_run - m_new) * LOG2E);
      l_part *= corr;
#pragma unroll
      for (int t = 0; t < HD / 32; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o_acc[t][r] *= corr;
      m_run = m_new;
    }
    const float m2 = (m_run == NEG_INF) ? 0.f : m_run * LOG2E;

    const T* Vs = vs_lds[st];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = u >> 1, hh = u & 1;
      float p8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p8[e] = exp2f(__builtin_fmaf(s[t][8 * hh + e], LOG2E, -m2));
        l_part += p8[e];
      }
      const vec pf = pack_p<T>(p8);
#pragma unroll
      for (int dt = 0; dt < HD / 32; ++dt) {
        const int d = 32 * dt + (lane & 31);
        vec vf = *reinterpret_cast<const vec*>(Vs + d * ATT_BN + (((2 * u + half) ^ swz8(d)) << 3));
        o_acc[dt] = Mfma<T>::mma32(vf, pf, o_acc[dt]);
      }
    }
    if (kt + 1 < n_tiles) {
      tl.lstore_k(ks_lds[st ^ 1], tid);
      tl.lstore_v(vs_lds[st ^ 1], tid);
    }
    __syncthreads();
  }

  const float l_tot = l_part + __shfl_xor(l_part, 32, 64);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (myq < S) store_o<T, HD>(o_acc, inv, (T*)a.o + (tok0 + myq) * (int64_t)D + h * HD, half);
}

// ======================================================= eager-exact: stats
// SMK: 0 = wave softmax (S <= 1024), 1 = 512-thread block softmax.
template <typename T, int HD, bool EXACT_SCALE, int SMK>
__global__ __launch_bounds__(ATT_THREADS, 2) void attn_stats_kernel(AttnArgs a) {
  typedef typename Mfma<T>::vec vec;
  typedef AttnTile<T, HD> Tile;
  __shared__ __attribute__((aligned(16))) T ks_lds[2][ATT_BN * HD];

  const int S = a.seq, H = a.heads, D = H * HD;
  const int nq = (S + ATT_BQ - 1) / ATT_BQ;
  int bh, qb;
  attn_work_of(nq, a.causal, bh, qb);
  const int b = bh / H, h = bh - b * H;
  const int q0 = qb * ATT_BQ;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5;
  const int q0w = q0 + wave * 32, myq = q0w + (lane & 31);
  const int64_t tok0 = (int64_t)b * S;

  Tile tl;
  tl.S = S;
  tl.ldqk = 2 * (int64_t)D;
  tl.ldvt = a.ldvt;
  tl.kbase = (const T*)a.qk + tok0 * tl.ldqk + D + h * HD;
  tl.vbase = nullptr;

  vec qf[HD / 16];
  load_q<T, HD>((const T*)a.qk, tl.ldqk, tok0, myq, S, h, half, qf);
  const int n_tiles = attn_n_tiles(S, a.causal, q0);
  const float NEG_INF = -__builtin_inff();
  const uint8_t* kv = a.key_valid ? a.key_valid + tok0 : nullptr;

  // ---------------- pass A: row max.  max commutes with the monotone
  // rounding and scaling, so it runs on the raw accumulators.
  float mx = NEG_INF;
  if (n_tiles > 0) {
    tl.gload_k(0, tid);
    tl.lstore_k(ks_lds[0], tid);
  }
  __syncthreads();
  for (int kt = 0; kt < n_tiles; ++kt) {
    const int st = kt & 1, kt0 = kt * ATT_BN;
    if (kt + 1 < n_tiles) tl.gload_k(kt + 1, tid);
    f32x16 s[2];
    scores_tile<T, HD>(ks_lds[st], qf, lane, s);
    const uint64_t kmask = tile_key_mask(kv, kt0, S, lane);
    const bool need_mask = (a.causal && (kt0 + ATT_BN - 1 > q0w)) || (kmask != ~0ull);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = s[t][r];
        if (need_mask) {
          const int kr = 32 * t + mfma32_row(r, lane);
          const bool ok = ((kmask >> kr) & 1ull) && !(a.causal && kt0 + kr > myq);
          v = ok ? v : NEG_INF;
        }
        mx = fmaxf(mx, v);
      }
    }
    if (kt + 1 < n_tiles) tl.lstore_k(ks_lds[st ^ 1], tid);
    __syncthreads();
  }
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float m = (mx == NEG_INF) ? NEG_INF : eager_score<T, EXACT_SCALE>(mx, a.scale);

  // ---------------- pass B: row sum of expf(s - m) in ATen's order.
  // Tile visiting order: natural for the wave softmax; for the block softmax
  // thread tau of 512 owns keys 4*tau + 2048*i + j, so visit, per wave w of
  // that softmax (64 threads = 256 consecutive keys mod 2048), its four
  // 64-key blocks bb and their repetitions i.
  const int n_all = (S + ATT_BN - 1) / ATT_BN;
  const int n_rep = (SMK == 1) ? (n_all + 31) / 32 : 1;
  auto tile_at = [&](int step) -> int {
    if (SMK == 0) return step;
    const int per_w = 4 * n_rep;
    const int w = step / per_w, rem = step - w * per_w;
    const int bb = rem / n_rep, i = rem - bb * n_rep;
    return (4 * w + bb) + 32 * i;
  };
  const int n_steps = (SMK == 0) ? n_tiles : 32 * n_rep;
  auto tile_live = [&](int kt) { return kt < n_tiles; };

  float part[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) part[i] = 0.f;
  float wsum[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) wsum[i] = 0.f;

  // Advance to the first live step, prefetch it.
  int step = 0;
  while (step < n_steps && !tile_live(tile_at(step))) ++step;
  __syncthreads();
  if (step < n_steps) {
    tl.gload_k(tile_at(step), tid);
    tl.lstore_k(ks_lds[0], tid);
  }
  __syncthreads();
  int st = 0;
  // For the block softmax the per-wave trees run when a wave's steps end.
  for (int cur = step; cur < n_steps;) {
    int nxt = cur + 1;
    while (nxt < n_steps && !tile_live(tile_at(nxt))) ++nxt;
    const int kt = tile_at(cur), kt0 = kt * ATT_BN;
    if (nxt < n_steps) tl.gload_k(tile_at(nxt), tid);
    f32x16 s[2];
    scores_tile<T, HD>(ks_lds[st], qf, lane, s);
    const uint64_t kmask = tile_key_mask(kv, kt0, S, lane);
    const bool need_mask = (a.causal && (kt0 + ATT_BN - 1 > q0w)) || (kmask != ~0ull);
    const int bb = (SMK == 1) ? ((kt & 31) & 3) : 0;
    float ev[2][16];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = eager_score<T, EXACT_SCALE>(s[t][r], a.scale);
        if (need_mask) {
          const int kr = 32 * t + mfma32_row(r, lane);
          const bool ok = ((kmask >> kr) & 1ull) && !(a.causal && kt0 + kr > myq);
          v = ok ? v : NEG_INF;
        }
        // The wave softmax sums expf terms; the block softmax sums the
        // hardware exponential (__expf), as its epilogue does.
        const float e = (m == NEG_INF) ? 0.f : (SMK == 1 ? __expf(v - m) : expf(v - m));
        if (SMK == 0) {
          part[16 * t + r] += e;
        } else {
          ev[t][r] = e;
        }
      }
    }
    if (SMK == 1) {
      // Slot of softmax thread tau: (bb, t, r>>2); j = r & 3 runs in key
      // order.  bb is uniform per tile: one branch, no per-score selects.
      auto acc_bb = [&](auto bbc) {
        constexpr int B = decltype(bbc)::value;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) part[8 * B + 4 * t + (r >> 2)] += ev[t][r];
      };
      if (bb == 0) acc_bb(std::integral_constant<int, 0>{});
      else if (bb == 1) acc_bb(std::integral_constant<int, 1>{});
      else if (bb == 2) acc_bb(std::integral_constant<int, 2>{});
      else acc_bb(std::integral_constant<int, 3>{});
    }
    if (SMK == 1) {
      // End of a wave of the block softmax: shuffle-down tree over its 64
      // threads tau (bits: bb1 bb0 t r3 r2 g, high to low), then keep the sum.
      const int wcur = cur / (4 * n_rep);
      const bool wave_done = (nxt >= n_steps) || (nxt / (4 * n_rep) != wcur);
      if (wave_done) {
        // part[8*bb + 4*t + q] is thread lambda = 16bb + 8t + 2q + g of the
        // softmax wave; levels: bb bit 1, bb bit 0, t, q bit 1, q bit 0, g.
        float f[2][4];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            f[tt][q] = (part[0 + 4 * tt + q] + part[16 + 4 * tt + q]) +
                       (part[8 + 4 * tt + q] + part[24 + 4 * tt + q]);
        float g4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) g4[q] = f[0][q] + f[1][q];          // bit t
        float g2[2] = {g4[0] + g4[2], g4[1] + g4[3]};                   // bit q1
        float g1 = g2[0] + g2[1];                                       // bit q0
        g1 = g1 + __shfl_xor(g1, 32, 64);                                // bit g
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (i == wcur) wsum[i] = g1;
#pragma unroll
        for (int i = 0; i < 32; ++i) part[i] = 0.f;
      }
    }
    if (nxt < n_steps) tl.lstore_k(ks_lds[st ^ 1], tid);
    __syncthreads();
    st ^= 1;
    cur = nxt;
  }

  float l;
  if (SMK == 0) {
    // xor butterfly of the 64 lanes of ATen's wave: t = 32tt + 8(r>>2) + 4g + (r&3);
    // offsets 32 (tt), 16 (r bit 3), 8 (r bit 2), 4 (g), 2 (r bit 1), 1 (r bit 0).
    float v16[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) v16[r] = part[r] + part[16 + r];
    float v8[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) v8[r] = v16[r] + v16[r + 8];
    float v4[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v4[r] = v8[r] + v8[r + 4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v4[r] = v4[r] + __shfl_xor(v4[r], 32, 64);
    const float v2a = v4[0] + v4[2], v2b = v4[1] + v4[3];
    l = v2a + v2b;
  } else {
    // Across the 8 waves of the block softmax: shuffle-down tree on lanes
    // 0..7 (zeros above): pairs (w, w+4), then (w, w+2), then (0, 1).
    const float a0 = wsum[0] + wsum[4], a1 = wsum[1] + wsum[5];
    const float a2 = wsum[2] + wsum[6], a3 = wsum[3] + wsum[7];
    l = (a0 + a2) + (a1 + a3);
  }
  if (myq < S && half == 0) {
    float* stats = a.row_stats + ((int64_t)bh * S + myq) * 2;
    stats[0] = m;
    stats[1] = l;
  }
}

// ========================================================== eager-exact: PV
template <typename T, int HD, bool EXACT_SCALE, int SMK>
__global__ __launch_bounds__(ATT_THREADS, 2) void attn_pv_kernel(AttnArgs a) {
  typedef typename Mfma<T>::vec vec;
  typedef AttnTile<T, HD> Tile;
  __shared__ __attribute__((aligned(16))) T ks_lds[2][ATT_BN * HD];
  __shared__ __attribute__((aligned(16))) T vs_lds[2][HD * ATT_BN];

  const int S = a.seq, H = a.heads, D = H * HD;
  const int nq = (S + ATT_BQ - 1) / ATT_BQ;
  int bh, qb;
  attn_work_of(nq, a.causal, bh, qb);
  const int b = bh / H, h = bh - b * H;
  const int q0 = qb * ATT_BQ;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5;
  const int q0w = q0 + wave * 32, myq = q0w + (lane & 31);
  const int64_t tok0 = (int64_t)b * S;

  Tile tl;
  tl.S = S;
  tl.ldqk = 2 * (int64_t)D;
  tl.ldvt = a.ldvt;
  tl.kbase = (const T*)a.qk + tok0 * tl.ldqk + D + h * HD;
  tl.vbase = (const T*)a.vt + (int64_t)bh * HD * a.ldvt;

  vec qf[HD / 16];
  load_q<T, HD>((const T*)a.qk, tl.ldqk, tok0, myq, S, h, half, qf);
  const float NEG_INF = -__builtin_inff();
  float m = NEG_INF, l = 1.f;
  if (myq < S) {
    const float* stats = a.row_stats + ((int64_t)bh * S + myq) * 2;
    m = stats[0];
    l = stats[1];
  }
  const float rinv = 1.0f / l;  // block softmax multiplies by the reciprocal
  const int n_tiles = attn_n_tiles(S, a.causal, q0);
  const uint8_t* kv = a.key_valid ? a.key_valid + tok0 : nullptr;

  f32x16 o_acc[HD / 32];
#pragma unroll
  for (int t = 0; t < HD / 32; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[t][r] = 0.f;

  if (n_tiles > 0) {
    tl.gload_k(0, tid);
    tl.gload_v(0, tid);
    tl.lstore_k(ks_lds[0], tid);
    tl.lstore_v(vs_lds[0], tid);
  }
  __syncthreads();
  for (int kt = 0; kt < n_tiles; ++kt) {
    const int st = kt & 1, kt0 = kt * ATT_BN;
    if (kt + 1 < n_tiles) {
      tl.gload_k(kt + 1, tid);
      tl.gload_v(kt + 1, tid);
    }
    f32x16 s[2];
    scores_tile<T, HD>(ks_lds[st], qf, lane, s);
    const uint64_t kmask = tile_key_mask(kv, kt0, S, lane);
    const bool need_mask = (a.causal && (kt0 + ATT_BN - 1 > q0w)) || (kmask != ~0ull);
    const T* Vs = vs_lds[st];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = u >> 1, hh = u & 1;
      float p8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int r = 8 * hh + e;
        float v = eager_score<T, EXACT_SCALE>(s[t][r], a.scale);
        if (need_mask) {
          const int kr = 32 * t + mfma32_row(r, lane);
          const bool ok = ((kmask >> kr) & 1ull) && !(a.causal && kt0 + kr > myq);
          v = ok ? v : NEG_INF;
        }
        float p;
        if (m == NEG_INF) {
          p = 0.f;
        } else if (SMK == 0) {
          p = expf(v - m) / l;
        } else {
          p = __expf(v - m) * rinv;
        }
        p8[e] = p;
      }
      const vec pf = pack_p<T>(p8);
#pragma unroll
      for (int dt = 0; dt < HD / 32; ++dt) {
        const int d = 32 * dt + (lane & 31);
        vec vf = *reinterpret_cast<const vec*>(Vs + d * ATT_BN + (((2 * u + half) ^ swz8(d)) << 3));
        o_acc[dt] = Mfma<T>::mma32(vf, pf, o_acc[dt]);
      }
    }
    if (kt + 1 < n_tiles) {
      tl.lstore_k(ks_lds[st ^ 1], tid);
      tl.lstore_v(vs_lds[st ^ 1], tid);
    }
    __syncthreads();
  }
  if (myq < S) store_o<T, HD>(o_acc, 1.0f, (T*)a.o + (tok0 + myq) * (int64_t)D + h * HD, half);
}

// ------------------------------------------------------------------ launch
template <typename T, int HD, bool EXACT>
static int launch_attn_hd(const AttnArgs& a, dim3 grid, hipStream_t st) {
  dim3 block(ATT_THREADS);
  if (a.softmax_mode == TX_SOFTMAX_ONLINE) {
    attn_online_kernel<T, HD, EXACT><<<grid, block, 0, st>>>(a);
  } else if (a.seq <= 1024) {
    attn_stats_kernel<T, HD, EXACT, 0><<<grid, block, 0, st>>>(a);
    attn_pv_kernel<T, HD, EXACT, 0><<<grid, block, 0, st>>>(a);
  } else {
    attn_stats_kernel<T, HD, EXACT, 1><<<grid, block, 0, st>>>(a);
    attn_pv_kernel<T, HD, EXACT, 1><<<grid, block, 0, st>>>(a);
  }
  return hipGetLastError() == hipSuccess ? TX_OK : TX_EHIP;
}

template <typename T>
static int launch_attn_typed(const AttnArgs& a, hipStream_t st) {
  const int nq = (a.seq + ATT_BQ - 1) / ATT_BQ;
  const long total = (long)nq * a.batch * a.heads;
  if (total > 0x7fffffffL) return TX_EUNSUPPORTED;
  dim3 grid((unsigned)total);
  // Power-of-two scale: the second eager rounding (of s * scale) is exact.
  int e2 = 0;
  const bool exact = (frexpf(a.scale, &e2) == 0.5f);
  if (a.head_dim == 64)
    return exact ? launch_attn_hd<T, 64, true>(a, grid, st) : launch_attn_hd<T, 64, false>(a, grid, st);
  if (a.head_dim == 128)
    return exact ? launch_attn_hd<T, 128, true>(a, grid, st) : launch_attn_hd<T, 128, false>(a, grid, st);
  return TX_EUNSUPPORTED;
}

int launch_attention(const AttnArgs& a, int dt, hipStream_t st) {
  if (!getenv("TX_ATTN_OLD")) return launch_attention_exact(a, dt, st);
  if (dt == TX_BF16) return launch_attn_typed<bf16>(a, st);
  if (dt == TX_F16) return launch_attn_typed<f16>(a, st);
  return TX_EUNSUPPORTED;
}

}  // namespace tx
