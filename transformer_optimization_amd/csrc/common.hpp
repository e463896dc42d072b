// Shared device helpers for the gfx950 kernels: 16-bit float conversions,
// MFMA operand vectors, 128-bit memory helpers and wave reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace tx {

typedef __bf16 bf16;
typedef _Float16 f16;

// 8 x 16-bit operand of v_mfma_f32_32x32x16_{bf16,f16}.
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8 __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));
typedef uint32_t u32x4 __attribute__((__vector_size__(4 * sizeof(uint32_t))));
typedef uint32_t u32x2 __attribute__((__vector_size__(2 * sizeof(uint32_t))));

// static_for<N>(f): f(std::integral_constant<int, 0>{}) ... f(<N - 1>{}), each
// index a compile-time constant.  For loop bodies too large for the unroller
// to flatten, over register arrays that must only ever be indexed by
// constants (a runtime index would move the array to scratch memory).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F> __device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// ---- scalar conversions (round-to-nearest-even, as ATen's casts) ----------
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(f16 v) { return (float)v; }

// Materialise x as an fp32 register value.  Eager rounds every result to
// fp32 before converting it to 16 bits; without this the compiler may fold the
// arithmetic that produced x and the conversion into one v_fma_mix (a single
// rounding), which differs from the double rounding in rare cases.
__device__ __forceinline__ float fp32_barrier(float x) {
  asm("" : "+v"(x));
  return x;
}

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) { return (bf16)fp32_barrier(v); }
template <> __device__ __forceinline__ f16 from_f32<f16>(float v) { return (f16)fp32_barrier(v); }

// Round an fp32 value to T and back: the value an eager op materialises.
template <typename T> __device__ __forceinline__ float round_to(float v) {
  return to_f32(from_f32<T>(v));
}

// ---- MFMA -------------------------------------------------------------------
template <typename T> struct Mfma;
template <> struct Mfma<bf16> {
  typedef bf16x8 vec;
  // D(32x32) += A(32x16) * B(16x32); lane l supplies A row (l & 31) and
  // B column (l & 31), eight consecutive k values of half (l >> 5).
  static __device__ __forceinline__ f32x16 mma32(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma<f16> {
  typedef f16x8 vec;
  static __device__ __forceinline__ f32x16 mma32(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// D(16x16) += A(16x32) * B(32x16): lane l supplies A row (l & 15) and B
// column (l & 15), eight consecutive k values 8 (l >> 4) .. +7; register e of
// lane l holds D row 4 (l >> 4) + e, column l & 15.
template <typename T> struct Mfma16;
template <> struct Mfma16<bf16> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma16<f16> {
  typedef f16x8 vec;
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Accumulator layout of the 32x32 MFMA: register r of lane l holds
//   row = 8*(r/4) + 4*(l/32) + (r%4),  column = l%32.
__device__ __forceinline__ int mfma32_row(int r, int lane) {
  return ((r >> 2) << 3) + ((lane >> 5) << 2) + (r & 3);
}

// ---- memory -----------------------------------------------------------------
__device__ __forceinline__ u32x4 ld128(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st128(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ u32x2 ld64(const void* p) {
  return *reinterpret_cast<const u32x2*>(p);
}
__device__ __forceinline__ void st64(void* p, u32x2 v) { *reinterpret_cast<u32x2*>(p) = v; }

// Pack two fp32 values into two 16-bit floats of type T (low half first),
// round-to-nearest-even, with one packed conversion where the ISA has it.
template <typename T> __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef T t2 __attribute__((ext_vector_type(2)));
  const t2 v = __builtin_convertvector(f2{fp32_barrier(lo), fp32_barrier(hi)}, t2);
  return __builtin_bit_cast(uint32_t, v);
}

// The same without the fp32 barrier, for values that come straight out of an
// MFMA or a transcendental (nothing the conversion could be fused with).
template <typename T> __device__ __forceinline__ uint32_t pack2_raw(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef T t2 __attribute__((ext_vector_type(2)));
  const t2 v = __builtin_convertvector(f2{lo, hi}, t2);
  return __builtin_bit_cast(uint32_t, v);
}

// Four consecutive elements of T <-> fp32 (8-byte vector for 16-bit T,
// 16-byte vector for fp32; the pointer must be aligned to that size).
// ld_raw4 / unpack4 split the read from the conversion, so that several reads
// can be in flight before the first value is used.
template <typename T> struct Raw4 {
  typedef typename std::conditional<sizeof(T) == 4, f32x4, u32x2>::type type;
};
template <typename T> __device__ __forceinline__ typename Raw4<T>::type ld_raw4(const T* p) {
  return *reinterpret_cast<const typename Raw4<T>::type*>(p);
}
template <typename T> __device__ __forceinline__ void unpack4(typename Raw4<T>::type v, float* f) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = v[e];
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t h = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
      f[e] = to_f32(__builtin_bit_cast(T, h));
    }
  }
}
template <typename T> __device__ __forceinline__ void load4(const T* p, float* f) {
  unpack4<T>(ld_raw4(p), f);
}
template <typename T> __device__ __forceinline__ void store4(T* p, const float* f) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<f32x4*>(p) = f32x4{f[0], f[1], f[2], f[3]};
  } else {
    st64(p, u32x2{pack2<T>(f[0], f[1]), pack2<T>(f[2], f[3])});
  }
}

// Unpack element i (0..7) of eight 16-bit floats held in a u32x4.
template <typename T> __device__ __forceinline__ float unpack8(u32x4 v, int i) {
  uint32_t w = v[i >> 1];
  uint16_t h = (i & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
  return to_f32(__builtin_bit_cast(T, h));
}

// Address-space casts for __builtin_amdgcn_global_load_lds (global -> LDS
// DMA: lane l's bytes land at the wave-uniform LDS address + size * l).
#define TX_GPTR(p) ((const __attribute__((address_space(1))) void*)(p))
#define TX_LPTR(p) ((__attribute__((address_space(3))) void*)(p))

// ---- global -> LDS rings ------------------------------------------------------
// dma16: global_load_lds_dwordx4, lane l's 16 bytes from g land at the
// wave-uniform LDS address lds + 16 * l.  Issued from inline asm so that the
// compiler does not model the LDS write: it cannot tell the stages of a ring
// apart and would otherwise wait for every outstanding DMA (vmcnt(0)) before
// the first LDS read after an issue, leaving one load in flight at a time.
// The ring orders the DMA itself with ring_barrier.
__device__ __forceinline__ void dma16(const void* g, const void* lds) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds);
  // M0 holds the LDS address; the nop covers the M0-write -> LDS-DMA hazard.
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "{m0}"(l) : "memory");
}

// The same with a wave-uniform base address (SGPR pair) and a 32-bit byte
// offset per lane: no per-lane 64-bit address arithmetic at each issue.
__device__ __forceinline__ void dma16_so(const void* base, uint32_t off, const void* lds) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(base), "{m0}"(l) : "memory");
}

// The same with the LDS byte address given as a wave-uniform 32-bit value
// (M0 is then one scalar add per issue: no generic-to-LDS pointer cast).
__device__ __forceinline__ void dma16_m0(const void* base, uint32_t off, uint32_t lds_addr) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(base), "{m0}"(lds_addr) : "memory");
}

// Wait until at most N vector-memory operations of this wave are in flight
// (its DMA issues complete in order, so N = the loads issued for later
// stages), then barrier.  No release/acquire fence: __syncthreads() would add
// vmcnt(0) and drain the ring.
template <int N>
__device__ __forceinline__ void ring_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Wait for every memory operation of this wave, DMA issues included.  A ring
// issues a few loads past its last step (into stages that are never read);
// the last statement of a ring kernel drains them, so that no DMA lands in
// LDS after the workgroup has ended.  At the very end the wait overlaps
// nothing the kernel still had to do.
__device__ __forceinline__ void ring_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Complete the load that produced x here: an empty asm that reads x makes the
// compiler place its wait before this point.  Used on values loaded before a
// ring loop; a wait left for them inside the loop would be a vmcnt that also
// drains the DMA ring (the compiler does not count the DMA issues).
template <typename V> __device__ __forceinline__ void settle(V& x) { asm volatile("" : "+v"(x)); }

// ---- wave reductions (wave64) ---------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float gelu_erf(float v) {
  // F.gelu(approximate="none"): x * 0.5 * (1 + erf(x / sqrt(2))), fp32 opmath.
  return v * 0.5f * (1.0f + erff(v * 0.70710678118654752440f));
}

}  // namespace tx
