// Residual add + LayerNorm.
//
// Replaces the reference's _add_ln_kernel (TTB:884-962) and the ATen chain of
// _ln_site (TTB:3988-4001).  HBM-bound: a row of D values is read once (plus
// delta when HAS_DELTA) and written once (plus x' when WRITE_X); the moments
// are computed from the register copy of the row.
#include "common.hpp"
#include "tx_internal.hpp"

namespace tx {

// One workgroup of 256 threads (4 waves) per row.  The fp32 moments use
// the reduction order of ATen's vectorized LayerNorm on ROCm, so that the
// mean and rstd (and hence every output element) are bit-identical to the
// eager nn.LayerNorm: each thread runs Welford's online update over its
// 4-element vectors (vector i goes to thread i mod 256), the 64 lanes of a
// wave are merged with shuffle-down steps 32..1, then the 4 waves with a
// two-level tree through LDS.  Output: gamma * (rstd * (x - mean)) + beta.
constexpr int LN_THREADS = 256;
constexpr int LN_VEC = 4;

struct Welford {
  float mean, m2, count;
};

// Rounding points of the ROCm build of ATen's kernel, measured against
// torch.native_layer_norm on gfx950 (mean and rstd bit-identical on every
// row of bf16/fp16/fp32 inputs, D = 256..2048): the counts' reciprocals are
// the hardware v_rcp_f32 (not a correctly rounded 1/n), the mean update is
// one fma, and the m2 update rounds the product before the add.
__device__ __forceinline__ Welford welford_push(float v, Welford w) {
  const float delta = v - w.mean;
  float n = w.count + 1.f;
  // The unrolled pushes have compile-time counts; hide them so that the
  // compiler does not fold v_rcp_f32(n) into the correctly rounded 1/n
  // (the two differ for n = 3, 6, 7, ...).
  asm volatile("" : "+v"(n));
  const float mean = __builtin_fmaf(delta, __builtin_amdgcn_rcpf(n), w.mean);
  float m2;
  {
#pragma clang fp contract(off)
    const float t = delta * (v - mean);
    m2 = w.m2 + t;
  }
  return {mean, m2, n};
}

// Merge of two partial states (b = this lane's, a = the partner's).  The
// eager kernel's compiled merges fuse one of the two mean products, and which
// one differs between its two trees (measured bit for bit against
// torch.native_layer_norm, including rows with unequal per-thread counts):
//   wave (shuffle) tree: mean = fma(na, a.mean, nb * b.mean);
//   cross-wave tree:     mean = fma(nb, b.mean, na * a.mean);
//   both:                m2 = fma(delta * delta * a.count, nb, a.m2 + b.m2).
// Spelled out here so that the compiler's own contraction choice cannot move.
template <bool WAVE_TREE>
__device__ __forceinline__ Welford welford_merge(const Welford b, const Welford a) {
#pragma clang fp contract(off)
  const float delta = b.mean - a.mean;
  const float count = a.count + b.count;
  float mean, m2;
  if (count > 0.f) {
    const float coef = __builtin_amdgcn_rcpf(count);
    const float na = a.count * coef;
    const float nb = b.count * coef;
    mean = WAVE_TREE ? __builtin_fmaf(na, a.mean, nb * b.mean) : __builtin_fmaf(nb, b.mean, na * a.mean);
    m2 = __builtin_fmaf(delta * delta * a.count, nb, a.m2 + b.m2);
  } else {
    mean = 0.f;
    m2 = 0.f;
  }
  return {mean, m2, count};
}

template <typename T> struct Vec4;
template <> struct Vec4<bf16> {
  static __device__ __forceinline__ void load(const bf16* p, float* f) {
    u32x2 v = ld64(p);
    f[0] = __builtin_bit_cast(float, v[0] << 16);
    f[1] = __builtin_bit_cast(float, v[0] & 0xffff0000u);
    f[2] = __builtin_bit_cast(float, v[1] << 16);
    f[3] = __builtin_bit_cast(float, v[1] & 0xffff0000u);
  }
  static __device__ __forceinline__ void store(bf16* p, const float* f) {
    st64(p, u32x2{pack2<bf16>(f[0], f[1]), pack2<bf16>(f[2], f[3])});
  }
};
template <> struct Vec4<f16> {
  static __device__ __forceinline__ void load(const f16* p, float* f) {
    u32x2 v = ld64(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t h = (uint16_t)(v[i >> 1] >> (16 * (i & 1)));
      f[i] = (float)__builtin_bit_cast(f16, h);
    }
  }
  static __device__ __forceinline__ void store(f16* p, const float* f) {
    st64(p, u32x2{pack2<f16>(f[0], f[1]), pack2<f16>(f[2], f[3])});
  }
};
template <> struct Vec4<float> {
  static __device__ __forceinline__ void load(const float* p, float* f) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p);
    f[0] = v[0];
    f[1] = v[1];
    f[2] = v[2];
    f[3] = v[3];
  }
  static __device__ __forceinline__ void store(float* p, const float* f) {
    *reinterpret_cast<f32x4*>(p) = f32x4{f[0], f[1], f[2], f[3]};
  }
};

// NV = vectors of 4 per thread (d <= NV * 1024).
template <typename X, typename Y, typename P, int NV>
__global__ __launch_bounds__(LN_THREADS) void layernorm_kernel(
    const X* __restrict__ x, const X* __restrict__ delta, X* __restrict__ x_out,
    Y* __restrict__ y, const P* __restrict__ gamma, const P* __restrict__ beta,
    const uint8_t* __restrict__ row_valid, float* __restrict__ mean_out,
    float* __restrict__ rstd_out, int64_t rows, int d, float eps, uint32_t flags) {
  __shared__ float red[3 * 2];
  __shared__ float stat[2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const int nvec = d / LN_VEC;
  const bool valid = (row_valid == nullptr) || (row_valid[row] != 0);

  float v[NV][4];
  const X* xr = x + row * (int64_t)d;
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int i = tid + c * LN_THREADS;
    if (i < nvec) {
      Vec4<X>::load(xr + i * LN_VEC, v[c]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[c][e] = 0.f;
    }
  }
  if (flags & TX_LN_HAS_DELTA) {
    const bool drop = (flags & TX_LN_MASK_DELTA) && !valid;
    const X* dr = delta + row * (int64_t)d;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      const int i = tid + c * LN_THREADS;
      if (i < nvec) {
        float dv[4];
        Vec4<X>::load(dr + i * LN_VEC, dv);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[c][e] = round_to<X>(v[c][e] + (drop ? 0.f : dv[e]));
      }
    }
  }
  if ((flags & TX_LN_MASK_X) && !valid) {
#pragma unroll
    for (int c = 0; c < NV; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[c][e] = 0.f;
  }
  if (flags & TX_LN_WRITE_X) {
    X* xo = x_out + row * (int64_t)d;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      const int i = tid + c * LN_THREADS;
      if (i < nvec) Vec4<X>::store(xo + i * LN_VEC, v[c]);
    }
  }

  Welford w{0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int i = tid + c * LN_THREADS;
    if (i < nvec) {
#pragma unroll
      for (int e = 0; e < 4; ++e) w = welford_push(v[c][e], w);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    Welford o{__shfl_down(w.mean, off, 64), __shfl_down(w.m2, off, 64), __shfl_down(w.count, off, 64)};
    w = welford_merge<true>(w, o);
  }
#pragma unroll
  for (int off = LN_THREADS / 128; off > 0; off >>= 1) {
    if (lane == 0 && wave >= off && wave < 2 * off) {
      const int k = wave - off;
      red[2 * k] = w.mean;
      red[2 * k + 1] = w.m2;
      red[4 + k] = w.count;
    }
    __syncthreads();
    if (lane == 0 && wave < off) {
      Welford o{red[2 * wave], red[2 * wave + 1], red[4 + wave]};
      w = welford_merge<false>(w, o);
    }
    __syncthreads();
  }
  if (tid == 0) {
    stat[0] = w.mean;
    stat[1] = w.m2 / (float)d;
  }
  __syncthreads();
  const float mean = stat[0];
  // The hardware reciprocal square root (v_rsq_f32), as the eager kernel
  // computes rstd; a correctly rounded 1/sqrt differs from it in the last bit.
  const float rstd = __builtin_amdgcn_rsqf(stat[1] + eps);
  if (tid == 0) {
    if (mean_out) mean_out[row] = mean;
    if (rstd_out) rstd_out[row] = rstd;
  }

  const bool zero_out = (flags & TX_LN_MASK_OUT) && !valid;
  const bool split = (flags & TX_LN_SPLIT_Y) != 0;
  Y* yr = y + row * (int64_t)d * (split ? 2 : 1);
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int i = tid + c * LN_THREADS;
    if (i < nvec) {
      float g[4], b[4], o[4];
      Vec4<P>::load(gamma + i * LN_VEC, g);
      Vec4<P>::load(beta + i * LN_VEC, b);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // gamma * (rstd * (x - mean)) + beta with the eager kernel's one fusion.
#pragma clang fp contract(off)
        o[e] = zero_out ? 0.f : __builtin_fmaf(g[e], rstd * (v[c][e] - mean), b[e]);
      }
      Vec4<Y>::store(yr + i * LN_VEC, o);
      if (split) {
        // Low part: the fp32 value minus its rounded copy, rounded again.
        float lo[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) lo[e] = o[e] - round_to<Y>(o[e]);
        Vec4<Y>::store(yr + d + i * LN_VEC, lo);
      }
    }
  }
}

template <typename X, typename Y, typename P>
static int launch_ln_typed(const LayerNormArgs& a, hipStream_t st) {
  const int nvec = (int)(a.d / LN_VEC);
  const int nv = (nvec + LN_THREADS - 1) / LN_THREADS;
  if (a.rows > 0x7fffffffL) return TX_EUNSUPPORTED;
  dim3 grid((unsigned)a.rows), block(LN_THREADS);
  const X* x = (const X*)a.x;
  const X* dl = (const X*)a.delta;
  X* xo = (X*)a.x_out;
  Y* y = (Y*)a.y;
  const P* g = (const P*)a.gamma;
  const P* b = (const P*)a.beta;
#define TX_LN_CASE(N)                                                                         \
  case N:                                                                                     \
    layernorm_kernel<X, Y, P, N><<<grid, block, 0, st>>>(                                    \
        x, dl, xo, y, g, b, a.row_valid, a.mean_out, a.rstd_out, a.rows, (int)a.d, a.eps, a.flags); \
    break;
  switch (nv <= 1 ? 1 : nv <= 2 ? 2 : nv <= 4 ? 4 : 8) {
    TX_LN_CASE(1)
    TX_LN_CASE(2)
    TX_LN_CASE(4)
    TX_LN_CASE(8)
  }
#undef TX_LN_CASE
  return hipGetLastError() == hipSuccess ? TX_OK : TX_EHIP;
}

int launch_layernorm(const LayerNormArgs& a, hipStream_t st) {
  if (a.x_dt == TX_BF16 && a.y_dt == TX_BF16 && a.param_dt == TX_BF16)
    return launch_ln_typed<bf16, bf16, bf16>(a, st);
  if (a.x_dt == TX_F16 && a.y_dt == TX_F16 && a.param_dt == TX_F16)
    return launch_ln_typed<f16, f16, f16>(a, st);
  if (a.x_dt == TX_F32 && a.y_dt == TX_F32 && a.param_dt == TX_F32)
    return launch_ln_typed<float, float, float>(a, st);
  if (a.x_dt == TX_F32 && a.y_dt == TX_F16 && a.param_dt == TX_F32)
    return launch_ln_typed<float, f16, float>(a, st);
  // fp32 residual stream of a bf16 / fp16 model
  if (a.x_dt == TX_F32 && a.y_dt == TX_BF16 && a.param_dt == TX_BF16)
    return launch_ln_typed<float, bf16, bf16>(a, st);
  if (a.x_dt == TX_F32 && a.y_dt == TX_F16 && a.param_dt == TX_F16)
    return launch_ln_typed<float, f16, f16>(a, st);
  return TX_EUNSUPPORTED;
}

}  // namespace tx
