// Flash-attention forward for gfx950: S^T = K Q^T and O^T = V^T P^T on
// v_mfma_f32_32x32x16_{bf16,f16}, online softmax in registers.
//
// Replaces BaselineSelfAttention's eager chain (TTB:161-194) and the
// reference's _flash_attn_kernel (TTB:1313-1418).  Inputs are the layouts
// tx_qkv_proj writes: q and k row-major in qk[B*S, 2D] (q columns [0,D),
// k columns [D,2D)), v head-transposed in vt[B][H][hd][ldvt].  The output is
// row-major o[B*S, D] with heads merged, so no split/merge copies exist.
//
// Workgroup: 4 waves x 32 query rows = 128 query rows of one (batch, head).
// Key tiles of 64 rows stream through two LDS stages (K as [key][d], V^T as
// [d][key]); the next tile is fetched from HBM into registers while the
// current one is consumed.  Computing S^T (keys as MFMA rows, queries as
// columns) leaves each lane holding 32 of the 64 scores of one query row,
// so the row max / row sum need a single cross-lane exchange (lane ^ 32),
// and the packed probabilities are directly the B operand of the P*V MFMA.
//
// Rounding points of the eager chain (TTB:173-188), mirrored per score:
//   s = round(q . k)   then   s = round(s * scale)   (second rounding is
//   exact and skipped when scale is a power of two), masked -> -inf,
//   p = exp(s - m) in fp32, rounded to the model dtype for the MFMA,
//   o = round(sum p v / sum p).
// The running max is re-based only when it grows by more than 2^8 in p
// (wave-uniform branch), so most tiles skip the O rescale.
#include "common.hpp"
#include "tx_internal.hpp"

namespace tx {

constexpr int ATT_BQ = 128;   // query rows per workgroup
constexpr int ATT_BN = 64;    // keys per tile
constexpr int ATT_THREADS = 256;

// 16-byte-chunk swizzles.  Rows of 8 chunks (128 B): bijective on row&7 and
// on the parity classes of 16 rows; rows of >= 16 chunks: row & 15.
__device__ __forceinline__ int swz8(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int swz16(int r) { return r & 15; }

template <typename T, int HD, bool EXACT_SCALE>
__global__ __launch_bounds__(ATT_THREADS) void attn_fwd_kernel(AttnArgs a) {
  typedef typename Mfma<T>::vec vec;
  constexpr int KCH = HD / 8;                        // 16-byte chunks per K row
  constexpr int K_LD = ATT_BN * KCH / ATT_THREADS;   // K chunks per thread per tile
  constexpr int V_LD = HD * 8 / ATT_THREADS;         // V^T chunks per thread per tile
  constexpr int NDT = HD / 32;                       // 32-row d tiles of O^T
  constexpr int NKS = HD / 16;                       // k steps of S^T
  static_assert(K_LD >= 1 && V_LD >= 1, "tile/thread mismatch");

  __shared__ __attribute__((aligned(16))) T ks_lds[2][ATT_BN * HD];
  __shared__ __attribute__((aligned(16))) T vs_lds[2][HD * ATT_BN];

  const int S = a.seq, H = a.heads;
  const int D = H * HD;
  const int64_t ldqk = 2 * (int64_t)D;
  const int nq = (S + ATT_BQ - 1) / ATT_BQ;

  // XCD-aware order: each XCD gets a contiguous run of (head, q-block) work
  // so the blocks sharing a head's K/V run on the same L2.
  int pid = blockIdx.x;
  {
    const int nwg = gridDim.x;
    const int x = pid & 7, i = pid >> 3, q = nwg >> 3, r = nwg & 7;
    pid = x * q + (x < r ? x : r) + i;
  }
  const int bh = pid / nq;
  int qb = pid - bh * nq;
  if (a.causal) qb = nq - 1 - qb;  // longest rows first
  const int b = bh / H, h = bh - b * H;
  const int q0 = qb * ATT_BQ;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int q0w = q0 + wave * 32;
  const int myq = q0w + col;

  const T* __restrict__ qk = (const T*)a.qk;
  const T* __restrict__ vt = (const T*)a.vt;
  const int64_t tok0 = (int64_t)b * S;

  // Q^T fragments (B operand): column = query, k = d.
  vec qf[NKS];
  {
    const T* qrow = qk + (tok0 + myq) * ldqk + h * HD + 8 * half;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      u32x4 v = myq < S ? ld128(qrow + 16 * ks) : u32x4{0u, 0u, 0u, 0u};
      qf[ks] = __builtin_bit_cast(vec, v);
    }
  }

  const T* kbase = qk + tok0 * ldqk + D + h * HD;
  const T* vbase = vt + (int64_t)bh * HD * a.ldvt;

  int n_tiles = (S + ATT_BN - 1) / ATT_BN;
  if (a.causal) {
    const int last_q = (q0 + ATT_BQ - 1) < (S - 1) ? (q0 + ATT_BQ - 1) : (S - 1);
    const int need = last_q / ATT_BN + 1;
    n_tiles = need < n_tiles ? need : n_tiles;
  }

  u32x4 rk[K_LD], rv[V_LD];
  auto gload = [&](int kt) {
    const int kt0 = kt * ATT_BN;
#pragma unroll
    for (int i = 0; i < K_LD; ++i) {
      const int idx = tid + i * ATT_THREADS, key = idx / KCH, cc = idx % KCH;
      rk[i] = (kt0 + key < S) ? ld128(kbase + (int64_t)(kt0 + key) * ldqk + cc * 8)
                              : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < V_LD; ++i) {
      const int idx = tid + i * ATT_THREADS, d = idx >> 3, cc = idx & 7;
      const int k0 = kt0 + cc * 8;
      u32x4 v = u32x4{0u, 0u, 0u, 0u};
      if (k0 < S) {
        // In bounds: ldvt >= S is a multiple of 8, so a chunk that starts
        // below S ends inside the row.  Zero the keys >= S (p = 0 there,
        // and 0 * garbage could be NaN).
        v = ld128(vbase + (int64_t)d * a.ldvt + k0);
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
  };
  auto lstore = [&](int st) {
    T* Ks = ks_lds[st];
    T* Vs = vs_lds[st];
#pragma unroll
    for (int i = 0; i < K_LD; ++i) {
      const int idx = tid + i * ATT_THREADS, key = idx / KCH, cc = idx % KCH;
      const int phys = (KCH >= 16) ? (cc ^ swz16(key)) : (cc ^ swz8(key));
      st128(Ks + key * HD + phys * 8, rk[i]);
    }
#pragma unroll
    for (int i = 0; i < V_LD; ++i) {
      const int idx = tid + i * ATT_THREADS, d = idx >> 3, cc = idx & 7;
      // Keys 8cc..8cc+3 -> chunk 2(cc>>1), keys 8cc+4..8cc+7 -> chunk
      // 2(cc>>1)+1, both in half (cc&1): chunk 2u+g of a row then holds keys
      // {16u+4g..+3, 16u+8+4g..+3}, the order of the packed P operand.
      const int c0 = (cc >> 1) << 1, hf = cc & 1;
      T* row = Vs + d * ATT_BN;
      st64(row + (((c0) ^ swz8(d)) << 3) + hf * 4, u32x2{rv[i][0], rv[i][1]});
      st64(row + (((c0 + 1) ^ swz8(d)) << 3) + hf * 4, u32x2{rv[i][2], rv[i][3]});
    }
  };

  f32x16 o_acc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[t][r] = 0.f;

  const float NEG_INF = -__builtin_inff();
  const float LOG2E = 1.4426950408889634f;
  const float TAU = 5.545177444479562f;  // 8 * ln 2: p stays <= 2^8
  float m_run = NEG_INF, l_part = 0.f;
  const uint8_t* kv = a.key_valid ? a.key_valid + tok0 : nullptr;

  if (n_tiles > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();
  for (int kt = 0; kt < n_tiles; ++kt) {
    const int st = kt & 1;
    const int kt0 = kt * ATT_BN;
    if (kt + 1 < n_tiles) gload(kt + 1);

    // ---- S^T = K Q^T for the 64 keys of this tile (two 32-key blocks).
    const T* Ks = ks_lds[st];
    f32x16 s[2];
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

    // ---- eager rounding points, masks, row max.
    const uint64_t kmask =
        __ballot((kt0 + lane < S) && (kv == nullptr || kv[kt0 + lane] != 0));
    const bool need_causal = a.causal && (kt0 + ATT_BN - 1 > q0w);
    const bool need_mask = need_causal || (kmask != ~0ull);
    float mx = NEG_INF;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = round_to<T>(s[t][r]);
        v = EXACT_SCALE ? v * a.scale : round_to<T>(v * a.scale);
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

    // ---- lazy re-base of the running max (wave-uniform).
    if (__any(mx > m_run + TAU)) {
      const float m_new = fmaxf(m_run, mx);
      const float corr = (m_new == NEG_INF) ? 1.f : exp2f((m_run - m_new) * LOG2E);
      l_part *= corr;
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o_acc[t][r] *= corr;
      m_run = m_new;
    }
    const float m2 = (m_run == NEG_INF) ? 0.f : m_run * LOG2E;

    // ---- p = exp(s - m), row sums, pack to the P^T operand.
    vec pf[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = u >> 1, hh = u & 1;
      u32x4 pk;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p0 = exp2f(__builtin_fmaf(s[t][8 * hh + 2 * e], LOG2E, -m2));
        const float p1 = exp2f(__builtin_fmaf(s[t][8 * hh + 2 * e + 1], LOG2E, -m2));
        l_part += p0 + p1;
        pk[e] = pack2<T>(p0, p1);
      }
      pf[u] = __builtin_bit_cast(vec, pk);
    }

    // ---- O^T += V^T P^T.
    const T* Vs = vs_lds[st];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d = 32 * dt + col;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        vec vf = *reinterpret_cast<const vec*>(Vs + d * ATT_BN + (((2 * u + half) ^ swz8(d)) << 3));
        o_acc[dt] = Mfma<T>::mma32(vf, pf[u], o_acc[dt]);
      }
    }

    if (kt + 1 < n_tiles) lstore(st ^ 1);
    __syncthreads();
  }

  // ---- normalise and store o[b*S + q, h*HD + d].
  const float l_tot = l_part + __shfl_xor(l_part, 32, 64);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (myq < S) {
    T* orow = (T*)a.o + (tok0 + myq) * (int64_t)D + h * HD;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d0 = 32 * dt + 8 * q4 + 4 * half;
        u32x2 pk;
        pk[0] = pack2<T>(o_acc[dt][4 * q4 + 0] * inv, o_acc[dt][4 * q4 + 1] * inv);
        pk[1] = pack2<T>(o_acc[dt][4 * q4 + 2] * inv, o_acc[dt][4 * q4 + 3] * inv);
        st64(orow + d0, pk);
      }
    }
  }
}

template <typename T>
static int launch_attn_typed(const AttnArgs& a, hipStream_t st) {
  const int nq = (a.seq + ATT_BQ - 1) / ATT_BQ;
  const long total = (long)nq * a.batch * a.heads;
  if (total > 0x7fffffffL) return TX_EUNSUPPORTED;
  dim3 grid((unsigned)total), block(ATT_THREADS);
  // Power-of-two scale: the second eager rounding (of s * scale) is exact.
  int e2 = 0;
  const float mant = frexpf(a.scale, &e2);
  const bool exact = (mant == 0.5f);
  if (a.head_dim == 64) {
    if (exact)
      attn_fwd_kernel<T, 64, true><<<grid, block, 0, st>>>(a);
    else
      attn_fwd_kernel<T, 64, false><<<grid, block, 0, st>>>(a);
  } else if (a.head_dim == 128) {
    if (exact)
      attn_fwd_kernel<T, 128, true><<<grid, block, 0, st>>>(a);
    else
      attn_fwd_kernel<T, 128, false><<<grid, block, 0, st>>>(a);
  } else {
    return TX_EUNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? TX_OK : TX_EHIP;
}

int launch_attention(const AttnArgs& a, int dt, hipStream_t st) {
  if (dt == TX_BF16) return launch_attn_typed<bf16>(a, st);
  if (dt == TX_F16) return launch_attn_typed<f16>(a, st);
  return TX_EUNSUPPORTED;
}

}  // namespace tx
