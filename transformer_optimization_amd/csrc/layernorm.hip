// Residual add + LayerNorm, one wave64 per row, 128-bit loads and stores.
//
// Replaces the reference's _add_ln_kernel (TTB:884-962) and the ATen chain of
// _ln_site (TTB:3988-4001).  HBM-bound: a row of D bf16 values is read once
// (plus delta when HAS_DELTA) and written once (plus x' when WRITE_X); the
// moments are computed from registers (two passes over the register copy, no
// second HBM read).
#include "common.hpp"
#include "tx_internal.hpp"

namespace tx {

template <typename T> struct Vec8;
template <> struct Vec8<bf16> {
  static __device__ __forceinline__ void load(const bf16* p, float* f) {
    u32x4 v = ld128(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = unpack8<bf16>(v, i);
  }
  static __device__ __forceinline__ void store(bf16* p, const float* f) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = pack2<bf16>(f[2 * i], f[2 * i + 1]);
    st128(p, v);
  }
};
template <> struct Vec8<f16> {
  static __device__ __forceinline__ void load(const f16* p, float* f) {
    u32x4 v = ld128(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = unpack8<f16>(v, i);
  }
  static __device__ __forceinline__ void store(f16* p, const float* f) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = pack2<f16>(f[2 * i], f[2 * i + 1]);
    st128(p, v);
  }
};
template <> struct Vec8<float> {
  static __device__ __forceinline__ void load(const float* p, float* f) {
    u32x4 a = ld128(p), b = ld128(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[i] = __builtin_bit_cast(float, a[i]);
      f[4 + i] = __builtin_bit_cast(float, b[i]);
    }
  }
  static __device__ __forceinline__ void store(float* p, const float* f) {
    u32x4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = __builtin_bit_cast(uint32_t, f[i]);
      b[i] = __builtin_bit_cast(uint32_t, f[4 + i]);
    }
    st128(p, a);
    st128(p + 4, b);
  }
};

constexpr int LN_ROWS_PER_BLOCK = 4;

// NV = number of 8-element chunks per lane (d <= NV * 512).
template <typename X, typename Y, typename P, int NV>
__global__ __launch_bounds__(64 * LN_ROWS_PER_BLOCK) void layernorm_kernel(
    const X* __restrict__ x, const X* __restrict__ delta, X* __restrict__ x_out,
    Y* __restrict__ y, const P* __restrict__ gamma, const P* __restrict__ beta,
    const uint8_t* __restrict__ row_valid, int64_t rows, int d, float eps, uint32_t flags) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * LN_ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nchunks = d >> 3;
  const bool valid = (row_valid == nullptr) || (row_valid[row] != 0);

  float v[NV][8];
  const X* xr = x + row * (int64_t)d;
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int ch = lane + c * 64;
    if (ch < nchunks) {
      Vec8<X>::load(xr + ch * 8, v[c]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[c][i] = 0.f;
    }
  }

  if (flags & TX_LN_HAS_DELTA) {
    const bool drop = (flags & TX_LN_MASK_DELTA) && !valid;
    const X* dr = delta + row * (int64_t)d;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      const int ch = lane + c * 64;
      if (ch < nchunks) {
        float dv[8];
        Vec8<X>::load(dr + ch * 8, dv);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[c][i] = round_to<X>(v[c][i] + (drop ? 0.f : dv[i]));
      }
    }
  }
  if ((flags & TX_LN_MASK_X) && !valid) {
#pragma unroll
    for (int c = 0; c < NV; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) v[c][i] = 0.f;
  }
  if (flags & TX_LN_WRITE_X) {
    X* xo = x_out + row * (int64_t)d;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      const int ch = lane + c * 64;
      if (ch < nchunks) Vec8<X>::store(xo + ch * 8, v[c]);
    }
  }

  // fp32 moments: mean, then the biased variance about the mean.
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NV; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) s += v[c][i];
  const float inv_d = 1.0f / (float)d;
  const float mean = wave_sum(s) * inv_d;
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int ch = lane + c * 64;
    if (ch < nchunks) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float t = v[c][i] - mean;
        q += t * t;
      }
    }
  }
  const float var = wave_sum(q) * inv_d;
  const float rstd = rsqrtf(var + eps);

  const bool zero_out = (flags & TX_LN_MASK_OUT) && !valid;
  Y* yr = y + row * (int64_t)d;
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int ch = lane + c * 64;
    if (ch < nchunks) {
      float g[8], b[8], o[8];
      Vec8<P>::load(gamma + ch * 8, g);
      Vec8<P>::load(beta + ch * 8, b);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = zero_out ? 0.f : (v[c][i] - mean) * rstd * g[i] + b[i];
      Vec8<Y>::store(yr + ch * 8, o);
    }
  }
}

template <typename X, typename Y, typename P>
static int launch_ln_typed(const LayerNormArgs& a, hipStream_t st) {
  const int nchunks = (int)(a.d / 8);
  const int nv = (nchunks + 63) / 64;
  dim3 grid((unsigned)((a.rows + LN_ROWS_PER_BLOCK - 1) / LN_ROWS_PER_BLOCK));
  dim3 block(64 * LN_ROWS_PER_BLOCK);
  const X* x = (const X*)a.x;
  const X* dl = (const X*)a.delta;
  X* xo = (X*)a.x_out;
  Y* y = (Y*)a.y;
  const P* g = (const P*)a.gamma;
  const P* b = (const P*)a.beta;
#define TX_LN_CASE(N)                                                                         \
  case N:                                                                                     \
    layernorm_kernel<X, Y, P, N><<<grid, block, 0, st>>>(x, dl, xo, y, g, b, a.row_valid,     \
                                                          a.rows, (int)a.d, a.eps, a.flags); \
    break;
  switch (nv <= 1 ? 1 : nv <= 2 ? 2 : nv <= 4 ? 4 : nv <= 8 ? 8 : 16) {
    TX_LN_CASE(1)
    TX_LN_CASE(2)
    TX_LN_CASE(4)
    TX_LN_CASE(8)
    TX_LN_CASE(16)
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
  return TX_EUNSUPPORTED;
}

}  // namespace tx
