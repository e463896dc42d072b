// Residual add + LayerNorm.
//
// Replaces the reference's _add_ln_kernel (TTB:884-962) and the ATen chain of
// _ln_site (TTB:3988-4001).  HBM-bound: a row of D values is read once (plus
// delta when HAS_DELTA) and written once (plus x' when WRITE_X); the moments
// are computed from the register copy of the row.
#include "common.hpp"
#include "tx_internal.hpp"

namespace tx {

// The fp32 moments use the reduction order of ATen's vectorized LayerNorm on
// ROCm, so that the mean and rstd (and hence every output element) are
// bit-identical to the eager nn.LayerNorm: 256 thread slots each run
// Welford's online update over their 4-element vectors (vector i goes to slot
// i mod 256), the 64 slots of an eager wave are merged with shuffle-down steps
// 32..1, then the 4 eager waves with a two-level tree.  Output:
// gamma * (rstd * (x - mean)) + beta.
constexpr int LN_THREADS = 256;  // eager thread slots per row
constexpr int LN_VEC = 4;

struct Welford {
  float mean, m2, count;
};

// Welford push of v into w, the new count n and rn = v_rcp_f32(n) supplied.
// Rounding points of the ROCm build of ATen's kernel, measured against
// torch.native_layer_norm on gfx950 (mean and rstd bit-identical on every
// row of bf16/fp16/fp32 inputs, D = 256..2048): the counts' reciprocals are
// the hardware v_rcp_f32 (not a correctly rounded 1/n), the mean update is
// one fma, and the m2 update rounds the product before the add.  Every slot
// pushes its k-th element with the same count, so one reciprocal per position
// serves all of a lane's slots.
__device__ __forceinline__ Welford welford_push_r(float v, Welford w, float n, float rn) {
  const float delta = v - w.mean;
  const float mean = __builtin_fmaf(delta, rn, w.mean);
  float m2;
  {
#pragma clang fp contract(off)
    const float t = delta * (v - mean);
    m2 = w.m2 + t;
  }
  return {mean, m2, n};
}

// v_rcp_f32(k) for k = 1 .. N, the push reciprocals.  The counts are hidden
// from the compiler, which would otherwise fold them into the correctly
// rounded 1/k (the two differ for k = 3, 6, 7, ...).
template <int N> struct PushRcp {
  float r[N];
  __device__ __forceinline__ PushRcp() {
#pragma unroll
    for (int k = 0; k < N; ++k) {
      float n = (float)(k + 1);
      asm volatile("" : "+v"(n));
      r[k] = __builtin_amdgcn_rcpf(n);
    }
  }
};

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
  // Computed unconditionally and selected (no branch): an empty merge
  // (count 0) yields NaN here and takes the eager kernel's zeros instead.
  const float coef = __builtin_amdgcn_rcpf(count);
  const float na = a.count * coef;
  const float nb = b.count * coef;
  const float mean = WAVE_TREE ? __builtin_fmaf(na, a.mean, nb * b.mean) : __builtin_fmaf(nb, b.mean, na * a.mean);
  const float m2 = __builtin_fmaf(delta * delta * a.count, nb, a.m2 + b.m2);
  const bool some = count > 0.f;
  return {some ? mean : 0.f, some ? m2 : 0.f, count};
}

// Merge of two states that both hold c elements, c a power of two (every
// slot of a row whose length is a multiple of 1024 holds the same count):
// v_rcp_f32(2c) is exact, so the merge weights na = nb = c * rcp(2c) of
// welford_merge are exactly 1/2 and the result is bit-identical to it.
template <bool WAVE_TREE>
__device__ __forceinline__ Welford welford_merge_even(const Welford b, const Welford a, float c) {
#pragma clang fp contract(off)
  const float delta = b.mean - a.mean;
  const float mean = WAVE_TREE ? __builtin_fmaf(0.5f, a.mean, 0.5f * b.mean) : __builtin_fmaf(0.5f, b.mean, 0.5f * a.mean);
  const float m2 = __builtin_fmaf(delta * delta * c, 0.5f, a.m2 + b.m2);
  return {mean, m2, 2.f * c};
}

// Eight consecutive fp32 values stored as T: one 16-byte store for 16-bit
// T, two for fp32 (the pointer is aligned to 16 bytes).
template <typename T> __device__ __forceinline__ void store8(T* p, const float* f) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<f32x4*>(p) = f32x4{f[0], f[1], f[2], f[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{f[4], f[5], f[6], f[7]};
  } else {
    st128(p, u32x4{pack2<T>(f[0], f[1]), pack2<T>(f[2], f[3]), pack2<T>(f[4], f[5]), pack2<T>(f[6], f[7])});
  }
}

// Raw (unconverted) eight elements of T: one 16-byte vector for 16-bit T, two
// for fp32, so that every load of a row (x, delta, gamma, beta) is in flight
// before the first value is converted.
template <typename T> struct Raw8 {
  u32x4 v[sizeof(T) == 4 ? 2 : 1];
  __device__ __forceinline__ void load(const T* p) {
#pragma unroll
    for (int h = 0; h < (int)(sizeof(T) == 4 ? 2 : 1); ++h) v[h] = ld128(p + h * (16 / (int)sizeof(T)));
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int h = 0; h < (int)(sizeof(T) == 4 ? 2 : 1); ++h) v[h] = u32x4{0u, 0u, 0u, 0u};
  }
  __device__ __forceinline__ void unpack(float* f) const {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // Through a scalar: clang's bit_cast of a vector-element lvalue reads
        // element 0 of the vector whatever the index.
        const uint32_t w = v[e >> 2][e & 3];
        f[e] = __builtin_bit_cast(float, w);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = unpack8<T>(v[0], e);
    }
  }
};

// Residual add, masks and the x' write, shared by both kernels: v holds the
// row's x as loaded and becomes the normalised input.
struct RowFlags {
  bool has_delta, drop_delta, zero_x, write_x;
  __device__ __forceinline__ RowFlags(uint32_t flags, bool valid)
      : has_delta((flags & TX_LN_HAS_DELTA) != 0),
        drop_delta((flags & TX_LN_MASK_DELTA) && !valid),
        zero_x((flags & TX_LN_MASK_X) && !valid),
        write_x((flags & TX_LN_WRITE_X) != 0) {}
};
template <typename X> __device__ __forceinline__ void residual8(float* v, const Raw8<X>& rd, const RowFlags& f) {
  if (f.has_delta) {
    float dv[8];
    rd.unpack(dv);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = round_to<X>(v[e] + (f.drop_delta ? 0.f : dv[e]));
  }
  if (f.zero_x) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.f;
  }
}

// gamma * (rstd * (x - mean)) + beta for eight elements, stored as Y (and the
// split low part when SPLIT_Y).
template <typename Y, typename P>
__device__ __forceinline__ void output8(Y* yp, int64_t d, const float* v, const Raw8<P>& rg, const Raw8<P>& rb,
                                        float mean, float rstd, bool zero_out, bool split) {
  float g[8], b[8], o[8];
  rg.unpack(g);
  rb.unpack(b);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    // The eager kernel's one fusion: the final multiply-add.
#pragma clang fp contract(off)
    o[e] = zero_out ? 0.f : __builtin_fmaf(g[e], rstd * (v[e] - mean), b[e]);
  }
  store8<Y>(yp, o);
  if (split) {
    // Low part: the fp32 value minus its rounded copy, rounded again.
    float lo[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) lo[e] = o[e] - round_to<Y>(o[e]);
    store8<Y>(yp + d, lo);
  }
}

// ---- one wave per row (d <= 2048) ----------------------------------------------
// Lane l of the wave carries SPL of the eager kernel's 256 thread slots as
// SPL/2 pairs of adjacent slots (2s, 2s + 1); slot u owns the 4-vectors u,
// u + 256, ..., so a pair's vectors in group c are 8 consecutive elements
// (one 128-bit access for 16-bit types).  Within eager wave e (64 slots):
//   SPL = 4 (rows up to 2048 wide): e = l / 16, l' = l % 16, pairs at slots
//     64e + 2l' and 64e + 32 + 2l';
//   SPL = 2 (rows up to 512 wide, eager waves 2 and 3 empty): e = l / 32,
//     l' = l % 32, the pair at slots 64e + 2l'.
// The eager reduction maps onto the wave without LDS or barriers:
//   * per-slot Welford over the slot's 4-vectors, in order;
//   * eager wave tree, slot u <- u + off for off = 32 .. 1 (u the slot within
//     its eager wave): SPL = 4 merges off = 32 inside the lane (pair 0 <-
//     pair 1); every other off >= 2 takes the same slot of lane l + off/2 (a
//     DPP shift inside a 16-lane row, or a swizzle across the two rows of a
//     32-lane group for SPL = 2's off = 32); off = 1 merges the two slots of
//     the lane's first pair;
//   * eager cross-wave tree (wave 0 <- 2, 1 <- 3, then 0 <- 1) over the
//     eager waves' states (lanes 0, 16, 32, 48 for SPL = 4; lanes 0 and 32,
//     with waves 2 and 3 empty, for SPL = 2), read into scalars and merged by
//     every lane.
// Every merge on the path to the result has the eager tree's operands in the
// eager order, so mean, rstd and the output are bit-identical.
// DPP row shift: lane l of each 16-lane row reads lane l + N of that row
// (lanes whose source is outside the row read 0; their results are unused).
template <int N> __device__ __forceinline__ float row_down(float v) {
  if constexpr (N == 16) {
    // Across the two 16-lane rows of each 32-lane group: lane l reads l ^ 16
    // (ds_swizzle, bit mode: and 0x1f, xor 0x10); lanes 16..31 of a group
    // read 0..15, results that are unused.
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401f));
  } else {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x100 + N, 0xf, 0xf, true));
  }
}
template <int N> __device__ __forceinline__ Welford row_down(const Welford& w) {
  return {row_down<N>(w.mean), row_down<N>(w.m2), row_down<N>(w.count)};
}
__device__ __forceinline__ float lane_value(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ Welford lane_state(const Welford& w, int l) {
  return {lane_value(w.mean, l), lane_value(w.m2, l), lane_value(w.count, l)};
}

// One step of the eager wave tree at lane offset N on both slots of the
// lane's first pair; EVEN: all states hold n elements (merge_even).
template <int N, bool EVEN>
__device__ __forceinline__ void tree_step(Welford* w, float n) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const Welford o = row_down<N>(w[j]);
    w[j] = EVEN ? welford_merge_even<true>(w[j], o, n) : welford_merge<true>(w[j], o);
  }
}

// First 4-vector of pair h of group c held by lane l.
template <int SPL> __device__ __forceinline__ int pair_vec(int l, int c, int h) {
  return SPL == 4 ? 256 * c + 64 * (l >> 4) + 2 * (l & 15) + 32 * h : 256 * c + 2 * l;
}

// Four rows per 256-thread workgroup, one per wave.  NV = groups of 4*SPL
// elements per lane (d <= NV * 1024, or d <= 512 when SPL = 2); FULL: every
// slot that holds data holds NV 4-vectors (d == NV * 1024, or d == 512 when
// SPL = 2), so every merge on the result's path is of equal counts.
template <typename X, typename Y, typename P, int NV, int SPL, bool FULL>
__global__ __launch_bounds__(256) void layernorm_wave_kernel(
    const X* __restrict__ x, const X* __restrict__ delta, X* __restrict__ x_out,
    Y* __restrict__ y, const P* __restrict__ gamma, const P* __restrict__ beta,
    const uint8_t* __restrict__ row_valid, float* __restrict__ mean_out,
    float* __restrict__ rstd_out, int64_t rows, int d, float eps, uint32_t flags) {
  static_assert(SPL == 4 || (SPL == 2 && NV == 1), "slots per lane");
  constexpr int H = SPL / 2;  // 8-element halves per group and lane
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform; the kernel has no barrier
  // 4-vectors of the row; even, so 8-element halves are whole.
  const int nvec = FULL ? NV * 64 * SPL : d / LN_VEC;
  const bool split = (flags & TX_LN_SPLIT_Y) != 0;
  const bool has_delta = (flags & TX_LN_HAS_DELTA) != 0;
  const X* xr = x + row * (int64_t)d;
  const X* dr = delta + row * (int64_t)d;

  // Issue every load of the row first: the mask byte, x, delta, gamma, beta.
  // A half past the end of the row loads the row's last half instead (always
  // in bounds, no branch); its values are never pushed or stored.
  uint32_t vbyte = 1;
  if (row_valid != nullptr) vbyte = row_valid[row];
  Raw8<X> rx[NV][H], rdl[NV][H];
  Raw8<P> rg[NV][H], rb[NV][H];
#pragma unroll
  for (int c = 0; c < NV; ++c)
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const int vi = min(pair_vec<SPL>(lane, c, h), nvec - 2);
      rx[c][h].load(xr + vi * LN_VEC);
      if (has_delta) rdl[c][h].load(dr + vi * LN_VEC);
      rg[c][h].load(gamma + vi * LN_VEC);
      rb[c][h].load(beta + vi * LN_VEC);
    }
  // Consume the mask byte only here, so that its wait does not hold back the
  // row's loads.
  asm volatile("" : "+v"(vbyte));
  const bool valid = __builtin_amdgcn_readfirstlane(vbyte) != 0;  // one row per wave
  const RowFlags rf(flags, valid);

  float v[NV][8 * H];
#pragma unroll
  for (int c = 0; c < NV; ++c)
#pragma unroll
    for (int h = 0; h < H; ++h) {
      rx[c][h].unpack(&v[c][8 * h]);
      residual8<X>(&v[c][8 * h], rdl[c][h], rf);
    }
  if (rf.write_x) {
    X* xo = x_out + row * (int64_t)d;
#pragma unroll
    for (int c = 0; c < NV; ++c)
#pragma unroll
      for (int h = 0; h < H; ++h) {
        const int vi = pair_vec<SPL>(lane, c, h);
        if (vi < nvec) store8<X>(xo + vi * LN_VEC, &v[c][8 * h]);
      }
  }

  const PushRcp<4 * NV> rcp;
  Welford w[SPL];
#pragma unroll
  for (int j = 0; j < SPL; ++j) {
    w[j] = Welford{0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NV; ++c)
      if (pair_vec<SPL>(lane, c, j >> 1) + (j & 1) < nvec) {
#pragma unroll
        for (int e = 0; e < 4; ++e) w[j] = welford_push_r(v[c][4 * j + e], w[j], (float)(4 * c + e + 1), rcp.r[4 * c + e]);
      }
  }
  // Eager wave tree.  With FULL every state on the result's path holds
  // n = 4 * NV * 2^k elements at step k.
  float n = 4 * NV;
  if constexpr (SPL == 4) {
    // off 32: slots 2l', 2l' + 1 <- 2l' + 32, 2l' + 33 (the lane's second pair)
    w[0] = FULL ? welford_merge_even<true>(w[0], w[2], n) : welford_merge<true>(w[0], w[2]);
    w[1] = FULL ? welford_merge_even<true>(w[1], w[3], n) : welford_merge<true>(w[1], w[3]);
  } else {
    tree_step<16, FULL>(w, n);  // off 32
  }
  n *= 2.f;
  tree_step<8, FULL>(w, n);  // off 16
  n *= 2.f;
  tree_step<4, FULL>(w, n);  // off 8
  n *= 2.f;
  tree_step<2, FULL>(w, n);  // off 4
  n *= 2.f;
  tree_step<1, FULL>(w, n);  // off 2
  n *= 2.f;
  w[0] = FULL ? welford_merge_even<true>(w[0], w[1], n) : welford_merge<true>(w[0], w[1]);  // off 1
  n *= 2.f;
  // Eager cross-wave tree.
  Welford t;
  if constexpr (SPL == 4) {
    const Welford e0 = lane_state(w[0], 0), e1 = lane_state(w[0], 16);
    const Welford e2 = lane_state(w[0], 32), e3 = lane_state(w[0], 48);
    if constexpr (FULL)
      t = welford_merge_even<false>(welford_merge_even<false>(e0, e2, n), welford_merge_even<false>(e1, e3, n), 2.f * n);
    else
      t = welford_merge<false>(welford_merge<false>(e0, e2), welford_merge<false>(e1, e3));
  } else {
    // Eager waves 2 and 3 hold no element: merged as the empty state.
    const Welford e0 = lane_state(w[0], 0), e1 = lane_state(w[0], 32), z{0.f, 0.f, 0.f};
    t = welford_merge<false>(welford_merge<false>(e0, z), welford_merge<false>(e1, z));
  }
  const float mean = t.mean;
  // The hardware reciprocal square root (v_rsq_f32), as the eager kernel
  // computes rstd; a correctly rounded 1/sqrt differs from it in the last bit.
  const float rstd = __builtin_amdgcn_rsqf(t.m2 / (float)d + eps);
  if (lane == 0) {
    if (mean_out) mean_out[row] = mean;
    if (rstd_out) rstd_out[row] = rstd;
  }

  const bool zero_out = (flags & TX_LN_MASK_OUT) && !valid;
  Y* yr = y + row * (int64_t)d * (split ? 2 : 1);
#pragma unroll
  for (int c = 0; c < NV; ++c)
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const int vi = pair_vec<SPL>(lane, c, h);
      if (vi < nvec) output8<Y, P>(yr + vi * LN_VEC, d, &v[c][8 * h], rg[c][h], rb[c][h], mean, rstd, zero_out, split);
    }
}

// ---- two waves per row (d > 2048) -----------------------------------------------
// One workgroup of 128 threads per row, each lane carrying two of the eager
// kernel's 256 thread slots: slots 2l and 2l + 1 own the adjacent 4-vectors
// 2l + 256c and 2l + 1 + 256c, so lane l moves the 8 elements at 8l + 1024c
// with one 128-bit access (16-bit types).  The reduction is the eager one,
// remapped: each slot runs Welford over its 4-vectors in order; the eager wave
// tree merges slot u with u + off (off = 32 .. 1) -- for off >= 2 both slots
// of a lane take the state of lane + off/2 (the slots of one eager wave stay
// inside one half of our wave on every path that reaches slots 0 and 64),
// off = 1 is the merge of a lane's two slots; the eager cross-wave tree
// (wave 0 <- 2, 1 <- 3, then 0 <- 1) merges our half-waves (wave 0 lane 0 <-
// wave 1 lane 0, wave 0 lane 32 <- wave 1 lane 32, then lane 0 <- lane 32).
// NV = 8-element groups per lane (d <= NV * 1024).
template <typename X, typename Y, typename P, int NV>
__global__ __launch_bounds__(128) void layernorm_kernel(
    const X* __restrict__ x, const X* __restrict__ delta, X* __restrict__ x_out,
    Y* __restrict__ y, const P* __restrict__ gamma, const P* __restrict__ beta,
    const uint8_t* __restrict__ row_valid, float* __restrict__ mean_out,
    float* __restrict__ rstd_out, int64_t rows, int d, float eps, uint32_t flags) {
  __shared__ float red[2 * 3];
  __shared__ float stat[2];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nvec = d / LN_VEC;
  const bool split = (flags & TX_LN_SPLIT_Y) != 0;
  const bool has_delta = (flags & TX_LN_HAS_DELTA) != 0;
  const X* xr = x + row * (int64_t)d;
  const X* dr = delta + row * (int64_t)d;

  // Loads past the end of the row are clamped to its last 8 elements (in
  // bounds, no branch); their values are never pushed or stored.
  uint32_t vbyte = 1;
  if (row_valid != nullptr) vbyte = row_valid[row];
  Raw8<X> rx[NV], rdl[NV];
  Raw8<P> rg[NV], rb[NV];
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int i0 = min(2 * tid + c * 256, nvec - 2);  // slot a's 4-vector; slot b's is i0 + 1
    rx[c].load(xr + i0 * LN_VEC);
    if (has_delta) rdl[c].load(dr + i0 * LN_VEC);
    rg[c].load(gamma + i0 * LN_VEC);
    rb[c].load(beta + i0 * LN_VEC);
  }
  asm volatile("" : "+v"(vbyte));  // the mask byte's wait after the row's loads
  const bool valid = vbyte != 0;
  const RowFlags rf(flags, valid);

  float v[NV][8];
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    rx[c].unpack(v[c]);
    residual8<X>(v[c], rdl[c], rf);
  }
  if (rf.write_x) {
    X* xo = x_out + row * (int64_t)d;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      const int i0 = 2 * tid + c * 256;
      if (i0 < nvec) store8<X>(xo + i0 * LN_VEC, v[c]);
    }
  }

  const PushRcp<4 * NV> rcp;
  Welford wa{0.f, 0.f, 0.f}, wb{0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int i0 = 2 * tid + c * 256;
    if (i0 < nvec) {
#pragma unroll
      for (int e = 0; e < 4; ++e) wa = welford_push_r(v[c][e], wa, (float)(4 * c + e + 1), rcp.r[4 * c + e]);
#pragma unroll
      for (int e = 0; e < 4; ++e) wb = welford_push_r(v[c][4 + e], wb, (float)(4 * c + e + 1), rcp.r[4 * c + e]);
    }
  }
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) {
    const Welford oa{__shfl_down(wa.mean, off, 64), __shfl_down(wa.m2, off, 64), __shfl_down(wa.count, off, 64)};
    const Welford ob{__shfl_down(wb.mean, off, 64), __shfl_down(wb.m2, off, 64), __shfl_down(wb.count, off, 64)};
    wa = welford_merge<true>(wa, oa);
    wb = welford_merge<true>(wb, ob);
  }
  wa = welford_merge<true>(wa, wb);  // offset 1: slot 2l <- slot 2l + 1
  if (wave == 1 && (lane & 31) == 0) {
    const int k = lane >> 5;
    red[2 * k] = wa.mean;
    red[2 * k + 1] = wa.m2;
    red[4 + k] = wa.count;
  }
  __syncthreads();
  if (wave == 0) {
    if ((lane & 31) == 0) {
      const int k = lane >> 5;
      wa = welford_merge<false>(wa, Welford{red[2 * k], red[2 * k + 1], red[4 + k]});
    }
    const Welford o{__shfl(wa.mean, 32, 64), __shfl(wa.m2, 32, 64), __shfl(wa.count, 32, 64)};
    if (lane == 0) {
      wa = welford_merge<false>(wa, o);
      stat[0] = wa.mean;
      stat[1] = wa.m2 / (float)d;
    }
  }
  __syncthreads();
  const float mean = stat[0];
  const float rstd = __builtin_amdgcn_rsqf(stat[1] + eps);
  if (tid == 0) {
    if (mean_out) mean_out[row] = mean;
    if (rstd_out) rstd_out[row] = rstd;
  }

  const bool zero_out = (flags & TX_LN_MASK_OUT) && !valid;
  Y* yr = y + row * (int64_t)d * (split ? 2 : 1);
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int i0 = 2 * tid + c * 256;
    if (i0 < nvec) output8<Y, P>(yr + i0 * LN_VEC, d, v[c], rg[c], rb[c], mean, rstd, zero_out, split);
  }
}

template <typename X, typename Y, typename P>
static int launch_ln_typed(const LayerNormArgs& a, hipStream_t st) {
  const int nvec = (int)(a.d / LN_VEC);
  if (a.rows > 0x7fffffffL) return TX_EUNSUPPORTED;
  const X* x = (const X*)a.x;
  const X* dl = (const X*)a.delta;
  X* xo = (X*)a.x_out;
  Y* y = (Y*)a.y;
  const P* g = (const P*)a.gamma;
  const P* b = (const P*)a.beta;
  if (nvec <= 2 * LN_THREADS) {
    dim3 grid((unsigned)((a.rows + 3) / 4)), block(256);
#define TX_LN_WAVE(N, S, F)                                                                                  \
  layernorm_wave_kernel<X, Y, P, N, S, F><<<grid, block, 0, st>>>(x, dl, xo, y, g, b, a.row_valid, a.mean_out, \
                                                                  a.rstd_out, a.rows, (int)a.d, a.eps, a.flags)
    if (nvec == LN_THREADS / 2)
      TX_LN_WAVE(1, 2, true);
    else if (nvec < LN_THREADS / 2)
      TX_LN_WAVE(1, 2, false);
    else if (nvec == LN_THREADS)
      TX_LN_WAVE(1, 4, true);
    else if (nvec < LN_THREADS)
      TX_LN_WAVE(1, 4, false);
    else if (nvec == 2 * LN_THREADS)
      TX_LN_WAVE(2, 4, true);
    else
      TX_LN_WAVE(2, 4, false);
#undef TX_LN_WAVE
    return hipGetLastError() == hipSuccess ? TX_OK : TX_EHIP;
  }
  const int nv = (nvec + LN_THREADS - 1) / LN_THREADS;  // 8-element groups per lane
  dim3 grid((unsigned)a.rows), block(128);
#define TX_LN_CASE(N)                                                                         \
  case N:                                                                                     \
    layernorm_kernel<X, Y, P, N><<<grid, block, 0, st>>>(                                    \
        x, dl, xo, y, g, b, a.row_valid, a.mean_out, a.rstd_out, a.rows, (int)a.d, a.eps, a.flags); \
    break;
  switch (nv <= 4 ? 4 : 8) {
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
