// Attention forward for gfx950 on v_mfma_f32_32x32x16_{bf16,f16}.  Q, K, V
// and O are strided [batch, head, seq, head_dim] views (head_dim contiguous):
// column slices of a packed [B*S, 3D] projection, as the reference's
// attention wrapper receives them, or the tx_qkv_proj layouts (q, k in
// qk[B*S, 2D]; v head-transposed in vt[B][H][hd][ldvt]).  K tiles and V
// tiles (natural rows, or V^T rows) move global -> LDS by DMA through a ring
// of stages; a natural-layout V tile feeds the PV MFMA through LDS transpose
// reads (ds_read_b64_tr_b16).
//
// Two softmax modes:
//   TX_SOFTMAX_EAGER  -- the stats pass (row max and softmax sum) and the PV
//                        pass below, bit-exact with the eager chain;
//   TX_SOFTMAX_ONLINE -- attn_flash_kernel, one pass with a running max.
//
// Replaces BaselineSelfAttention's matmul / scale / mask / softmax / matmul
// chain (TTB:161-194) and the reference's bit-exact manual route
// (TTB:4257-4295, 3727-3822).  Every result equals the eager chain bit for
// bit:
//     s = round(round(q.k) * scale), masked -> -inf,
//     p = round(softmax_fp32(s)),  o = round(sum_j p_j v_j)  (keys in order).
// The softmax reproduces ATen's two fp32 softmax kernels on ROCm:
//   S <= 2048 ("wave" softmax; its limit is 2048 fp32 values per row): lane
//     t of a 64-lane wave sums expf(s_j - m) over keys j = t + 64 it in
//     order of it, an xor butterfly combines the lanes, and
//     p = expf(s_j - m) / l;
//   S >  2048 ("block" softmax, 512 threads): thread tau sums __expf(s_j - m)
//     over keys j = 4 tau + 2048 i + jj (i, then jj ascending), shuffle-down
//     trees reduce each 64-thread wave and then the 8 wave sums, and
//     p = __expf(s_j - m) * (1 / l).
//
// Work split: a workgroup of 4 waves owns 128 query rows of one (batch,
// head), 32 per wave.  Scores are formed transposed, S^T = K Q^T, so lane l
// holds the 32 scores of query (l & 31) at keys 32t + 8(r>>2) + 4g + (r&3) of
// each 64-key tile (g = l >> 5, r = accumulator register, t = 32-key half).
// In that layout the 64 ATen wave lanes / 512 block threads that own the
// keys of one query map onto fixed (lane, register) slots, so each lane keeps
// the partial sums of its slots and the ATen trees become register adds plus
// one exchange with lane ^ 32.
//
// Cost per score of the exact passes is dominated by vector instructions
// (exp, the division, the roundings) rather than MFMA, so the code keeps
// that path short: rows with no admissible key use m = 0 (every score is
// -inf, so every exp is 0), the rounding of scores is one conversion per
// value, masks are applied only on tiles that need them (a wave-uniform
// branch), the wave softmax takes shortened exact expf and division
// sequences when the tile allows, and rows of one key tile (head dim 64)
// form their statistics inside the PV kernel (no stats launch).
#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "tx_internal.hpp"

namespace tx {

constexpr int AX_BQ = 128;     // query rows per workgroup
constexpr int AX_BN = 64;      // keys per tile
constexpr int AX_THREADS = 256;

// Chunk swizzle of 128-byte LDS rows (a K tile at head dim 64, a V^T tile):
// the 16 rows one ds_read_b128 cycle serves, read at one logical chunk,
// land in 16 different 16-byte bank groups.  The hardware folds address bit
// 10 (row bit 3 here) into the bank group itself, so the row's low three
// bits are the whole swizzle.
__device__ __forceinline__ int ax_swz8(int r) { return r & 7; }
template <int HD>
__device__ __forceinline__ int ax_kswz(int key) {
  if constexpr (HD == 128) return key & 15;
  else return ax_swz8(key);
}
// Chunk swizzle of a natural-layout V tile [64 keys][HD], chosen for the
// transposed PV operand reads (ds_read_b64_tr_b16): the 32 lanes of one
// read cycle cover four consecutive keys x 64 bytes, which this XOR spreads
// over all 64 banks (checked exhaustively on the host for both head dims).
template <int HD>
__device__ __forceinline__ int ax_vswz(int key) {
  if constexpr (HD == 128) return (key & 3) << 2;
  else return ((key >> 1) & 1) << 2;
}
template <int HD, bool VTILE>
__device__ __forceinline__ int ax_tile_swz(int key) {
  if constexpr (VTILE) return ax_vswz<HD>(key);
  else return ax_kswz<HD>(key);
}

// Workgroup -> (batch*head, query block); each XCD receives a contiguous run
// so the blocks of one head share K/V in its L2.  Causal: longest rows first.
__device__ __forceinline__ void ax_work_of(int nq, int causal, int& bh, int& qb) {
  int pid = blockIdx.x;
  const int nwg = gridDim.x;
  const int x = pid & 7, i = pid >> 3, q = nwg >> 3, r = nwg & 7;
  pid = x * q + (x < r ? x : r) + i;
  bh = pid / nq;
  qb = pid - bh * nq;
  if (causal) qb = nq - 1 - qb;
}

// Operand bases of one (batch, head) from the strided views.
template <typename T>
struct AxHead {
  const T* q;
  const T* k;
  const T* v;
  T* o;
  const uint8_t* kv;
  __device__ __forceinline__ void init(const AttnArgs& a, int b, int h) {
    q = (const T*)a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;
    k = (const T*)a.k + (int64_t)b * a.k_sb + (int64_t)h * a.k_sh;
    v = (const T*)a.v + (int64_t)b * a.v_sb + (int64_t)h * a.v_sh;
    o = (T*)a.o + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh;
    kv = a.key_valid ? a.key_valid + (int64_t)b * a.kv_sb : nullptr;
  }
};

// ------------------------------------------------------------ tile loaders
// K tile [64 keys][HD] and V^T tile [HD][64 keys] in LDS, 16-byte chunks
// XOR-swizzled by row.  One wave instruction fills 1 KB (64 lanes x 16 B);
// the swizzle is applied by the choice of source chunk per lane.
// VTILE: the tile holds V rows (natural layout) and uses the V swizzle.
template <typename T, int HD, bool VTILE = false>
struct AxK {
  static constexpr int CH = HD / 8;        // chunks per row (8 or 16)
  static constexpr int RPI = 64 / CH;      // rows per wave instruction (8 or 4)
  static constexpr int LD = AX_BN / RPI / 4;
  static constexpr int ELEMS = AX_BN * HD;
  const T* base;     // key 0 of this (batch, head); wave-uniform
  int64_t ld;
  uint32_t off[LD];  // byte offset of this lane's chunk within a full tile
  int rows[LD];
  int S, wv;
  __device__ __forceinline__ void init(const T* kbase, int64_t ld_, int S_, int wave, int lane) {
    base = kbase;
    ld = ld_;
    S = S_;
    wv = __builtin_amdgcn_readfirstlane(wave);
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int row = (i * 4 + wv) * RPI + lane / CH;
      const int c = (lane % CH) ^ ax_tile_swz<HD, VTILE>(row);
      rows[i] = row;
      off[i] = (uint32_t)(((int64_t)row * ld + 8 * c) * (int64_t)sizeof(T));
    }
  }
  __device__ __forceinline__ void issue(int kt, T* Ks) const {
    if ((kt + 1) * AX_BN <= S) {
      const T* tb = base + (int64_t)kt * AX_BN * ld;
#pragma unroll
      for (int i = 0; i < LD; ++i) dma16_so(tb, off[i], Ks + (i * 4 + wv) * RPI * HD);
    } else {
      // Last tile: keys >= S re-read key S - 1 (they are masked).
#pragma unroll
      for (int i = 0; i < LD; ++i) {
        const int key = min(kt * AX_BN + rows[i], S - 1);
        const uint32_t chunk = off[i] - (uint32_t)((int64_t)rows[i] * ld * (int64_t)sizeof(T));
        dma16((const char*)(base + (int64_t)key * ld) + chunk, Ks + (i * 4 + wv) * RPI * HD);
      }
    }
  }
};

template <typename T, int HD>
struct AxV {
  static constexpr int LD = HD / 8 / 4;    // 8 rows (d) per instruction
  static constexpr int ELEMS = HD * AX_BN;
  const T* base;     // V^T row 0 of this (batch, head); wave-uniform
  int ldvt, wv;
  uint32_t off[LD];  // byte offset of this lane's chunk within tile 0
  int c8[LD];
  int64_t rowoff[LD];
  __device__ __forceinline__ void init(const T* vbase, int64_t ldvt_, int wave, int lane) {
    base = vbase;
    ldvt = (int)ldvt_;
    wv = __builtin_amdgcn_readfirstlane(wave);
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int d = (i * 4 + wv) * 8 + lane / 8;
      c8[i] = 8 * ((lane % 8) ^ ax_swz8(d));
      rowoff[i] = (int64_t)d * ldvt_;
      off[i] = (uint32_t)((rowoff[i] + c8[i]) * (int64_t)sizeof(T));
    }
  }
  __device__ __forceinline__ void issue(int kt, T* Vs) const {
    if ((kt + 1) * AX_BN <= ldvt) {
      const T* tb = base + (int64_t)kt * AX_BN;
#pragma unroll
      for (int i = 0; i < LD; ++i) dma16_so(tb, off[i], Vs + (i * 4 + wv) * 8 * AX_BN);
    } else {
      // Chunks past the row end re-read its last chunk (zeroed in LDS before use).
#pragma unroll
      for (int i = 0; i < LD; ++i) {
        const int k0 = min(kt * AX_BN + c8[i], ldvt - 8);
        dma16(base + rowoff[i] + k0, Vs + (i * 4 + wv) * 8 * AX_BN);
      }
    }
  }
};

// Per-lane element offsets of the K fragments inside a K tile, one per
// 16-wide k step: key (lane & 31) (the t = 1 half adds 32 * HD), its
// swizzled chunk 2 ks + (lane >> 5).  Tile-independent, computed once.
template <int HD>
struct AxKOff {
  int off[HD / 16];
  __device__ __forceinline__ void init(int lane) {
    const int col = lane & 31, half = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) off[ks] = col * HD + (((2 * ks + half) ^ ax_kswz<HD>(col)) << 3);
  }
  // Key-permuted operand: MFMA row i reads key i with bits 2 and 3 swapped,
  // so score slot (t, r) of lane half h holds key 32 t + 16 (r >> 3) + 8 h +
  // (r & 7).  The eight slots 8 hh .. 8 hh + 7 of a lane are then eight
  // consecutive keys in the order of a 16-key P operand (lanes 0-31: keys
  // 0-7, lanes 32-63: keys 8-15), with no cross-lane exchange.  Each group of
  // 16 lanes still reads rows 0-15 (or 16-31) as a set: same LDS banks.
  __device__ __forceinline__ void init_perm(int lane) {
    const int col = lane & 31, half = lane >> 5;
    const int row = (col & ~12) | ((col & 4) << 1) | ((col & 8) >> 1);
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) off[ks] = row * HD + (((2 * ks + half) ^ ax_kswz<HD>(row)) << 3);
  }
};
// Same for the V^T fragments of a tile: row d = lane & 31 (+ 32 dt), chunk
// 2u + (lane >> 5) for the 16-key step u.
struct AxVOff {
  int off[4];
  __device__ __forceinline__ void init(int lane) {
    const int col = lane & 31, half = lane >> 5;
#pragma unroll
    for (int u = 0; u < 4; ++u) off[u] = col * AX_BN + (((2 * u + half) ^ ax_swz8(col)) << 3);
  }
};

// Natural-layout V: per-lane element offsets of the transposed operand reads.
// The PV operand of MFMA step u and head-dim block dt gives lane l the eight
// keys 16u + 8(l >> 5) .. +7 of head-dim column 32 dt + (l & 31).  Two
// ds_read_b64_tr_b16 form it: within each 16-lane group (g = l >> 4,
// j = l & 15) result element i of lane j is element j % 4 of the 8 bytes
// addressed by lane 4 i + j / 4 (layout measured on gfx950).  So lane j
// addresses key 4r + j / 4 (+ 16u + 8(g >> 1)) at head-dim column
// 32 dt + 16 (g & 1) + 4 (j % 4) for read r: lane j receives column
// 32 dt + 16 (g & 1) + j of keys 4r .. 4r + 3.  off[dt] is the element
// offset for u = 0, r = 0; step u adds 16 u HD, read r adds 4 r HD (the
// swizzle depends on key % 4 only, which u and r leave unchanged).
template <int HD>
struct AxVNatOff {
  int off[HD / 32];
  __device__ __forceinline__ void init(int lane) {
    const int g = lane >> 4, j = lane & 15;
    const int key = 8 * (g >> 1) + (j >> 2);
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt) {
      const int d = 32 * dt + 16 * (g & 1) + 4 * (j & 3);
      off[dt] = key * HD + (((d >> 3) ^ ax_vswz<HD>(key)) << 3) + (d & 7);
    }
  }
};

// The operand of step U at LDS byte address addr (read r = 0) and
// addr + 8 HD bytes (r = 1).  Issued from inline asm so that the key offsets
// are the instructions' immediate offsets (the builtin does not fold them,
// leaving two address instructions per read).  The compiler does not count
// these reads, so ax_vnat_wait must complete them before the operand is
// used; an uncounted LDS read can only make the compiler's own lgkmcnt waits
// stricter (LDS reads complete in order), never looser.
template <int HD, int U>
__device__ __forceinline__ u32x4 ax_vnat_issue(uint32_t addr) {
  u32x2 lo, hi;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(lo) : "v"(addr), "n"(2 * 16 * U * HD));
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(hi) : "v"(addr), "n"(2 * (16 * U * HD + 4 * HD)));
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}
// Wait for every LDS read of this wave, then hand the operands on (the
// in/out operands order the wait between the reads and the MFMAs).
template <int N>
__device__ __forceinline__ void ax_vnat_wait(u32x4 (&v)[N]) {
  if constexpr (N == 2) asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]));
  else asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]));
}

// V tile of either layout: its DMA loader, its PV operand read, and whether
// the key columns past S of the last tile must be zeroed in LDS (V^T: those
// chunks re-read the row's last chunk; natural V: those rows re-read key
// S - 1, finite values that meet p = 0).
template <typename T, int HD, bool VNAT>
struct AxVTile;
template <typename T, int HD>
struct AxVTile<T, HD, true> {
  typedef AxK<T, HD, true> L;
  static constexpr int LD = L::LD;
  static constexpr int ELEMS = L::ELEMS;
  static constexpr bool ZERO_TAIL = false;
  typedef typename Mfma<T>::vec vec;
  L ld;
  AxVNatOff<HD> vo;
  uint32_t va[HD / 32];     // this tile's per-lane LDS byte addresses, one per head-dim block
  u32x4 opnd[HD / 32];      // the operands of the current step
  __device__ __forceinline__ void init(const AxHead<T>& hp, const AttnArgs& a, int S, int wave, int lane) {
    ld.init(hp.v, a.v_ss, S, wave, lane);
    vo.init(lane);
  }
  __device__ __forceinline__ void issue(int kt, T* Vs) const { ld.issue(kt, Vs); }
  __device__ __forceinline__ void begin(const T* Vs) {
    const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) T*)Vs;
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt) va[dt] = base + 2u * (uint32_t)vo.off[dt];
  }
  // Step u's operands for every head-dim block: issue the reads, then wait.
  // u is a compile-time constant at every call site (unrolled loops).
  __device__ __forceinline__ void load_step(int u) {
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt) {
      switch (u) {
        case 0: opnd[dt] = ax_vnat_issue<HD, 0>(va[dt]); break;
        case 1: opnd[dt] = ax_vnat_issue<HD, 1>(va[dt]); break;
        case 2: opnd[dt] = ax_vnat_issue<HD, 2>(va[dt]); break;
        default: opnd[dt] = ax_vnat_issue<HD, 3>(va[dt]); break;
      }
    }
  }
  __device__ __forceinline__ void wait_step() { ax_vnat_wait<HD / 32>(opnd); }
  __device__ __forceinline__ vec operand(const T*, int, int dt) const {
    return __builtin_bit_cast(vec, opnd[dt]);
  }
};
template <typename T, int HD>
struct AxVTile<T, HD, false> {
  typedef AxV<T, HD> L;
  static constexpr int LD = L::LD;
  static constexpr int ELEMS = L::ELEMS;
  static constexpr bool ZERO_TAIL = true;
  L ld;
  AxVOff vo;
  __device__ __forceinline__ void init(const AxHead<T>& hp, const AttnArgs& a, int, int wave, int lane) {
    ld.init(hp.v, a.ldvt, wave, lane);
    vo.init(lane);
  }
  __device__ __forceinline__ void issue(int kt, T* Vs) const { ld.issue(kt, Vs); }
  __device__ __forceinline__ void begin(const T*) {}
  __device__ __forceinline__ void load_step(int) {}
  __device__ __forceinline__ void wait_step() {}
  __device__ __forceinline__ typename Mfma<T>::vec operand(const T* Vs, int u, int dt) const {
    return *reinterpret_cast<const typename Mfma<T>::vec*>(Vs + 32 * dt * AX_BN + vo.off[u]);
  }
};

// S^T of one tile: s[t][r] = q_(lane&31) . k_(32t + mfma32_row(r, lane)).
// init: the accumulators' starting value (zero when null).
template <typename T, int HD>
__device__ __forceinline__ void ax_scores(const T* Ks, const typename Mfma<T>::vec* qf,
                                          const AxKOff<HD>& ko, f32x16* s, const f32x16* init = nullptr) {
  typedef typename Mfma<T>::vec vec;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[t][r] = init ? (*init)[r] : 0.f;
  // The two 32-key halves alternate: consecutive MFMAs use different
  // accumulators.
#pragma unroll
  for (int ks = 0; ks < HD / 16; ++ks) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const vec kf = *reinterpret_cast<const vec*>(Ks + 32 * t * HD + ko.off[ks]);
      s[t] = Mfma<T>::mma32(kf, qf[ks], s[t]);
    }
  }
}

// Round two fp32 values to T and back (the value eager materialises), with
// one packed conversion.
// BAR = false only for values that come straight out of an MFMA (no
// arithmetic the conversion could be fused with).
template <typename T, bool BAR = true>
__device__ __forceinline__ void ax_round2(float& a, float& b) {
  if constexpr (std::is_same<T, bf16>::value) {
    // One conversion per value with a zero low half (v_cvt_pk_bf16_f32 d, 0,
    // x): the 32-bit result is the rounded value as fp32, no unpacking.
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    a = __builtin_bit_cast(float, __builtin_convertvector(f2{0.f, BAR ? fp32_barrier(a) : a}, b2));
    b = __builtin_bit_cast(float, __builtin_convertvector(f2{0.f, BAR ? fp32_barrier(b) : b}, b2));
  } else {
    a = round_to<T>(a);
    b = round_to<T>(b);
  }
}

// The 32 eager scores of this lane for one tile, as fp32 values of T:
// round(acc), then for a non-power-of-two scale round(round(acc) * scale).
// (For a power-of-two scale the product is exact and formed in ax_shift.)
template <typename T, bool EXACT_SCALE, int NT = 2>
__device__ __forceinline__ void ax_round_scores(f32x16* s, float scale) {
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      float a = s[t][r], b = s[t][r + 1];
      ax_round2<T, false>(a, b);
      if (!EXACT_SCALE) {
        a *= scale;
        b *= scale;
        ax_round2<T>(a, b);
      }
      s[t][r] = a;
      s[t][r + 1] = b;
    }
  }
}

// Masked keys (invalid, past S, or after the query when causal) -> -inf.
// PERM: the scores come from the key-permuted K operand (AxKOff::init_perm).
template <bool PERM = false>
__device__ __forceinline__ void ax_mask(float (*x)[16], uint64_t kmask, int causal, int kt0, int myq,
                                        int lane) {
  const float NEG_INF = -__builtin_inff();
  // Key of slot (t, r) = kt0 + h4 + c with a compile-time c; shift the mask
  // and the causal limit by the lane's part h4 once.
  const int h4 = (lane >> 5) << (PERM ? 3 : 2);
  const uint64_t km = kmask >> h4;
  const int lim = causal ? myq - kt0 - h4 : AX_BN;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int c = PERM ? 32 * t + ((r >> 3) << 4) + (r & 7) : 32 * t + ((r >> 2) << 3) + (r & 3);
      const bool ok = ((km >> c) & 1ull) && c <= lim;
      x[t][r] = ok ? x[t][r] : NEG_INF;
    }
  }
}

// Same with a chosen replacement value (0 for exponentials already formed).
template <bool PERM = false>
__device__ __forceinline__ void ax_mask_to(float (*x)[16], uint64_t kmask, int causal, int kt0, int myq,
                                           int lane, float val) {
  const int h4 = (lane >> 5) << (PERM ? 3 : 2);
  const uint64_t km = kmask >> h4;
  const int lim = causal ? myq - kt0 - h4 : AX_BN;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int c = PERM ? 32 * t + ((r >> 3) << 4) + (r & 7) : 32 * t + ((r >> 2) << 3) + (r & 3);
      const bool ok = ((km >> c) & 1ull) && c <= lim;
      x[t][r] = ok ? x[t][r] : val;
    }
  }
}

// ax_mask (or ax_mask_to, with val) for the 16 scores of one 32-key half t
// (wave-uniform) of a tile, unpermuted operand: slot r of lane half h holds key 32 t + 8 (r >> 2) +
// 4 h + (r & 3).
__device__ __forceinline__ void ax_mask_half(float* x, uint64_t kmask, int causal, int kt0, int q,
                                             int lane, int t, float val = -__builtin_inff()) {
  const int h4 = 32 * t + ((lane >> 5) << 2);
  const uint64_t km = kmask >> h4;
  const int lim = causal ? q - kt0 - h4 : AX_BN;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int c = ((r >> 2) << 3) + (r & 3);
    const bool ok = ((km >> c) & 1ull) && c <= lim;
    x[r] = ok ? x[r] : val;
  }
}

// ---- wave softmax (S <= 2048): expf and the division, bit for bit --------
// ATen's wave softmax calls the device library's expf and divides by the row
// sum.  When every score of the tile has x = s - m > AX_FAST_X (x <= 0
// always), both reduce to shorter sequences with identical results:
//  * expf(x): ph = x*L2E, e = rint(ph), a = (ph - e) + (fma(x, L2E, -ph) +
//    x*L2E_LO), r = ldexp(exp2(a), e), the library's sequence, without its
//    range selects (x below ~-104 -> 0, above ~88.7 -> inf), which cannot
//    fire for x in (AX_FAST_X, 0];
//  * q = e / l (l in [1, 2048], e = 0 or e > 2^-101): the correctly rounded
//    division sequence (reciprocal refined once, then two fma corrections),
//    without its operand scaling and result fix-up, which change nothing
//    for such operands; the refined reciprocal is formed once per row.
constexpr float AX_FAST_X = -70.0f;

__device__ __forceinline__ float ax_expf_inrange(float x) {
  const float L2E = __builtin_bit_cast(float, 0x3fb8aa3bu);
  const float L2E_LO = __builtin_bit_cast(float, 0x32a5705fu);
  const float ph = x * L2E;
  const float e = __builtin_rintf(ph);
  const float pl = __builtin_fmaf(x, L2E_LO, __builtin_fmaf(x, L2E, -ph));
  const float a = (ph - e) + pl;
  return __builtin_ldexpf(__builtin_amdgcn_exp2f(a), (int)e);
}

// Refined reciprocal of l, as the division sequence forms it.
__device__ __forceinline__ float ax_div_recip(float l) {
  const float r0 = __builtin_amdgcn_rcpf(l);
  return __builtin_fmaf(__builtin_fmaf(-l, r0, 1.0f), r0, r0);
}
__device__ __forceinline__ float ax_div_fast(float e, float l, float rr) {
  float q = e * rr;
  float t = __builtin_fmaf(-l, q, e);
  q = __builtin_fmaf(t, rr, q);
  t = __builtin_fmaf(-l, q, e);
  return __builtin_fmaf(t, rr, q);
}

// True when every slot of every lane has x > AX_FAST_X (wave-uniform).
__device__ __forceinline__ bool ax_wave_fast(const float (*x)[16]) {
  float mn = x[0][0];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) mn = fminf(mn, x[t][r]);
  return __builtin_amdgcn_readfirstlane((int)__all(mn > AX_FAST_X)) != 0;
}

// e[t][r] = expf(x[t][r]) of the wave softmax, 0 on masked slots; x is
// overwritten.  Returns the wave-uniform fast flag.
template <bool PERM = false>
__device__ __forceinline__ bool ax_wave_exps(float (*x)[16], bool need_mask, uint64_t kmask, int causal,
                                             int kt0, int myq, int lane) {
  const bool fast = ax_wave_fast(x);
  if (fast) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) x[t][r] = ax_expf_inrange(x[t][r]);
    if (need_mask) ax_mask_to<PERM>(x, kmask, causal, kt0, myq, lane, 0.f);
  } else {
    if (need_mask) ax_mask<PERM>(x, kmask, causal, kt0, myq, lane);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) x[t][r] = expf(x[t][r]);
  }
  return fast;
}

// x = s - m, where for an exact (power-of-two) scale s = round(acc) * scale
// is formed inside one fma (the product is exact, so this equals the eager
// subtraction).
template <bool EXACT_SCALE>
__device__ __forceinline__ float ax_shift(float v, float scale, float m) {
  return EXACT_SCALE ? __builtin_fmaf(v, scale, -m) : v - m;
}

// Key-validity bits of a tile (bit k: key kt0 + k exists and is valid).
__device__ __forceinline__ uint64_t ax_key_mask(const uint8_t* kv, int kt0, int S, int lane) {
  return __ballot((kt0 + lane < S) && (kv == nullptr || kv[kt0 + lane] != 0));
}

__device__ __forceinline__ int ax_n_tiles(int S, int causal, int q0) {
  int n = (S + AX_BN - 1) / AX_BN;
  if (causal) {
    const int last_q = min(q0 + AX_BQ - 1, S - 1);
    n = min(n, last_q / AX_BN + 1);
  }
  return n;
}

// The wave softmax's row sum from this lane's 32 per-slot partial sums
// (part[16 t + r], t = 32-key half, r = accumulator register): the xor
// butterfly of ATen's 64 lanes, lane = 32 t + 8 (r >> 2) + 4 g + (r & 3);
// offsets 32 (t), 16 (r bit 3), 8 (r bit 2), 4 (g), 2 (r bit 1), 1 (r bit 0).
// From the first level's 16 pair sums v16[r] = part[r] + part[16 + r] on.
__device__ __forceinline__ float ax_wave_softmax_sum16(const float* v16) {
  float v8[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) v8[r] = v16[r] + v16[r + 8];
  float v4[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) v4[r] = v8[r] + v8[r + 4];
#pragma unroll
  for (int r = 0; r < 4; ++r) v4[r] = v4[r] + __shfl_xor(v4[r], 32, 64);
  const float v2a = v4[0] + v4[2], v2b = v4[1] + v4[3];
  return v2a + v2b;
}
__device__ __forceinline__ float ax_wave_softmax_sum(const float* part) {
  float v16[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) v16[r] = part[r] + part[16 + r];
  return ax_wave_softmax_sum16(v16);
}

// Order in which the stats kernel visits K tiles: pass A (max) in natural
// order, then pass B (sum) in the order of ATen's per-thread sums.  For the
// block softmax, pass B walks the 8 softmax waves w; wave w owns tiles
// kt = 4w + bb + 32i (bb = 0..3, i = 0..n_rep-1), visited bb-major so that
// each thread's keys arrive in ascending order.  Tiles past the causal limit
// are skipped (their terms are exp(-inf) = 0).  The block-softmax order is
// tabulated once per workgroup in LDS: entry j = kt | bb << 16 | w << 18 |
// (last tile of its softmax wave) << 21.
constexpr int AX_MAX_TILES = 1024;  // block-softmax rows up to 65536 keys
static_assert(ATEN_SOFTMAX_BLOCK_THREADS == 512, "the block-softmax order below is for 8 waves");

// When every tile is live and n_all is a multiple of 32 the table has no
// holes: entry j = (4 w + bb) n_rep + i, which every thread can write.
__device__ __forceinline__ bool ax_order_dense(int n_live, int n_all) {
  return n_live == n_all && (n_all & 31) == 0;
}
__device__ __forceinline__ void ax_build_order_dense(uint32_t* tbl, int n_all, int tid) {
  const int n_rep = n_all / 32;
  for (int j = tid; j < n_all; j += AX_THREADS) {
    const int i = j % n_rep, wb = j / n_rep, bb = wb & 3, w = wb >> 2;
    const uint32_t end = (bb == 3 && i == n_rep - 1) ? 1u : 0u;
    tbl[j] = (uint32_t)(4 * w + bb + 32 * i) | ((uint32_t)bb << 16) | ((uint32_t)w << 18) | (end << 21);
  }
}

__device__ __forceinline__ void ax_build_order(uint32_t* tbl, int n_live, int n_all) {
  const int n_rep = (n_all + 31) / 32;
  int j = 0;
  for (int w = 0; w < 8; ++w)
    for (int bb = 0; bb < 4; ++bb)
      for (int i = 0; i < n_rep; ++i) {
        const int kt = 4 * w + bb + 32 * i;
        if (kt < n_live) tbl[j++] = (uint32_t)kt | ((uint32_t)bb << 16) | ((uint32_t)w << 18);
      }
  for (int k = 0; k < n_live; ++k) {
    const uint32_t wk = (tbl[k] >> 18) & 7u;
    if (k == n_live - 1 || ((tbl[k + 1] >> 18) & 7u) != wk) tbl[k] |= 1u << 21;
  }
}

// ======================================================================= stats
template <typename T, int HD, bool EXACT_SCALE, int SMK>
__global__ __launch_bounds__(AX_THREADS, 3) void attn_stats2_kernel(AttnArgs a) {
  typedef typename Mfma<T>::vec vec;
  typedef AxK<T, HD> KL;
  // Three workgroups per CU: LDS (K ring + order table) <= 53 KB, <= 168 VGPRs.
  constexpr int NST = (HD == 128) ? 3 : 4;
  __shared__ __attribute__((aligned(16))) T ks_lds[NST][KL::ELEMS];

  const int S = a.seq, H = a.heads;
  const int nq = (S + AX_BQ - 1) / AX_BQ;
  int bh, qb;
  ax_work_of(nq, a.causal, bh, qb);
  const int b = bh / H, h = bh - b * H;
  const int q0 = qb * AX_BQ;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5;
  const int q0w = q0 + wave * 32, myq = q0w + (lane & 31);
  const float NEG_INF = -__builtin_inff();
  AxHead<T> hp;
  hp.init(a, b, h);

  KL kl;
  kl.init(hp.k, a.k_ss, S, wave, lane);

  AxKOff<HD> ko;
  ko.init(lane);
  vec qf[HD / 16];
  {
    const T* qrow = hp.q + (int64_t)min(myq, S - 1) * a.q_ss + 8 * half;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) qf[ks] = __builtin_bit_cast(vec, ld128(qrow + 16 * ks));
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) settle(qf[ks]);
  }
  const int n_live = ax_n_tiles(S, a.causal, q0);
  const int n_all = (S + AX_BN - 1) / AX_BN;
  const uint8_t* kv = hp.kv;

  __shared__ uint32_t order[SMK == 1 ? AX_MAX_TILES : 1];
  // Tile of global step s: pass A natural, pass B in the softmax's order.
  auto tile_of = [&](int s) -> int {
    if (s < n_live) return s;
    if (SMK == 0) return s - n_live;
    return (int)(order[s - n_live] & 0xffffu);
  };
  const int n_steps = 2 * n_live;
  // Issues past the end repeat the last tile into a stage that is never
  // read, so every step issues the same number of loads.
  auto issue = [&](int s) { kl.issue(tile_of(min(s, n_steps - 1)), ks_lds[s % NST]); };
  // The first pass-A tiles need no table: their loads go out first, and the
  // table is built while they are in flight.
  const bool pre_all = n_live >= NST - 1;
#pragma unroll
  for (int s = 0; s < NST - 1; ++s)
    if (s < n_live) issue(s);
  if (SMK == 1) {
    if (ax_order_dense(n_live, n_all)) ax_build_order_dense(order, n_all, tid);
    else if (tid == 0) ax_build_order(order, n_live, n_all);
    if (pre_all) ring_barrier<KL::LD * (NST - 1)>();  // LDS table visible; DMA left in flight
    else __syncthreads();
  }
#pragma unroll
  for (int s = 0; s < NST - 1; ++s)
    if (s >= n_live) issue(s);

  float m = 0.f;           // pass B: the eager row max (0 for a row with no admissible key)
  bool dead = false;
  float part[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) part[i] = 0.f;
  float wsum[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) wsum[i] = 0.f;

  // ---- pass A (steps 0 .. n_live-1): max commutes with the monotone
  // rounding and scaling, so the raw accumulators' max is enough.  Each K
  // fragment read from LDS feeds two MFMAs: waves 2p and 2p + 1 take query
  // blocks 2p and 2p + 1 together (their own and the partner's, wave w ^ 1's),
  // wave w only the 32-key half t = w & 1 of each tile, so a wave reads half
  // the fragments it would read for its own block alone (attention at 8192
  // keys, head dim 128: 1.0% faster).  The partner's maxima go through LDS at
  // the end.
  __shared__ float pa_max[AX_THREADS / 64][32];
  float mx = NEG_INF, mx_p = NEG_INF;  // own block, partner block; key half t
  {
    const int th = wave & 1;
    const int myq_p = q0 + 32 * (wave ^ 1) + (lane & 31);
    vec qf_p[HD / 16];
    const T* qrow = hp.q + (int64_t)min(myq_p, S - 1) * a.q_ss + 8 * half;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) qf_p[ks] = __builtin_bit_cast(vec, ld128(qrow + 16 * ks));
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) settle(qf_p[ks]);
    const int q_lo = q0 + 64 * (wave >> 1);  // the pair's first query
    for (int step = 0; step < n_live; ++step) {
      ring_barrier<KL::LD * (NST - 2)>();
      issue(step + NST - 1);
      const int kt0 = step * AX_BN;
      f32x16 so, sp;
#pragma unroll
      for (int r = 0; r < 16; ++r) so[r] = sp[r] = 0.f;
      const T* kh = ks_lds[step % NST] + 32 * th * HD;
#pragma unroll
      for (int ks = 0; ks < HD / 16; ++ks) {
        const vec kf = *reinterpret_cast<const vec*>(kh + ko.off[ks]);
        so = Mfma<T>::mma32(kf, qf[ks], so);
        sp = Mfma<T>::mma32(kf, qf_p[ks], sp);
      }
      const uint64_t kmask = ax_key_mask(kv, kt0, S, lane);
      // Wave-uniform, so that unmasked tiles take a scalar branch around the masking.
      const bool need_mask = __builtin_amdgcn_readfirstlane(
          (int)((a.causal && (kt0 + AX_BN - 1 > q_lo)) || (kmask != ~0ull))) != 0;
      if (need_mask) {
        float xo[16], xp[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          xo[r] = so[r];
          xp[r] = sp[r];
        }
        ax_mask_half(xo, kmask, a.causal, kt0, myq, lane, th);
        ax_mask_half(xp, kmask, a.causal, kt0, myq_p, lane, th);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          mx = fmaxf(mx, xo[r]);
          mx_p = fmaxf(mx_p, xp[r]);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          mx = fmaxf(mx, so[r]);
          mx_p = fmaxf(mx_p, sp[r]);
        }
      }
    }
  }
  {
#pragma clang fp contract(off)
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    mx_p = fmaxf(mx_p, __shfl_xor(mx_p, 32, 64));
    if (half == 0) pa_max[wave][lane] = mx_p;
    ring_barrier<63>();  // pa_max visible; pass B's K loads stay in flight
    mx = fmaxf(mx, pa_max[wave ^ 1][lane & 31]);
    dead = (mx == NEG_INF);
    if (!dead) {
      float hi = mx, unused = 0.f;
      ax_round2<T>(hi, unused);
      if (!EXACT_SCALE) {
        hi *= a.scale;
        ax_round2<T>(hi, unused);
        m = hi;
      } else {
        m = hi * a.scale;
      }
    }
  }

  // ---- pass B (steps n_live .. 2 n_live-1): e = exp(s - m) into the ATen slots.
  for (int step = n_live; step < n_steps; ++step) {
#pragma clang fp contract(off)
    ring_barrier<KL::LD * (NST - 2)>();
    issue(step + NST - 1);
    const uint32_t ent = (SMK == 1) ? order[step - n_live] : 0u;
    const int kt = (SMK == 1) ? (int)(ent & 0xffffu) : step - n_live;
    const int kt0 = kt * AX_BN;
    f32x16 s[2];
    ax_scores<T, HD>(ks_lds[step % NST], qf, ko, s);
    const uint64_t kmask = ax_key_mask(kv, kt0, S, lane);
    const bool need_mask = __builtin_amdgcn_readfirstlane(
        (int)((a.causal && (kt0 + AX_BN - 1 > q0w)) || (kmask != ~0ull))) != 0;
    ax_round_scores<T, EXACT_SCALE>(s, a.scale);
    float ev[2][16];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) ev[t][r] = ax_shift<EXACT_SCALE>(s[t][r], a.scale, m);
    if (SMK == 1) {
      if (need_mask) ax_mask(ev, kmask, a.causal, kt0, myq, lane);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) ev[t][r] = __expf(ev[t][r]);
    } else {
      ax_wave_exps(ev, need_mask, kmask, a.causal, kt0, myq, lane);
    }
    if (SMK == 0) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) part[16 * t + r] += ev[t][r];
    } else {
      // Slot of softmax thread tau: (bb, t, r>>2); jj = r & 3 in key order.
      auto acc_bb = [&](auto bbc) {
        constexpr int B = decltype(bbc)::value;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) part[8 * B + 4 * t + (r >> 2)] += ev[t][r];
      };
      const int bb = (int)((ent >> 16) & 3u);
      if (bb == 0) acc_bb(std::integral_constant<int, 0>{});
      else if (bb == 1) acc_bb(std::integral_constant<int, 1>{});
      else if (bb == 2) acc_bb(std::integral_constant<int, 2>{});
      else acc_bb(std::integral_constant<int, 3>{});
      // End of a softmax wave: its shuffle-down tree over threads
      // lambda = 16bb + 8t + 2q + g (levels bb1, bb0, t, q1, q0, g).
      if ((ent >> 21) & 1u) {
        float f[2][4];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            f[tt][q] = (part[0 + 4 * tt + q] + part[16 + 4 * tt + q]) +
                       (part[8 + 4 * tt + q] + part[24 + 4 * tt + q]);
        float g4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) g4[q] = f[0][q] + f[1][q];
        const float g2a = g4[0] + g4[2], g2b = g4[1] + g4[3];
        float g1 = g2a + g2b;
        g1 = g1 + __shfl_xor(g1, 32, 64);
        const int wc = (int)((ent >> 18) & 7u);
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (i == wc) wsum[i] = g1;
#pragma unroll
        for (int i = 0; i < 32; ++i) part[i] = 0.f;
      }
    }
  }

  float l;
  if (SMK == 0) {
    l = ax_wave_softmax_sum(part);
  } else {
    // Across the 8 softmax waves: pairs (w, w+4), then (w, w+2), then (0, 1).
    const float a0 = wsum[0] + wsum[4], a1 = wsum[1] + wsum[5];
    const float a2 = wsum[2] + wsum[6], a3 = wsum[3] + wsum[7];
    l = (a0 + a2) + (a1 + a3);
  }
  if (myq < S && half == 0) {
    float* st = a.row_stats + ((int64_t)bh * S + myq) * 2;
    st[0] = dead ? NEG_INF : m;
    st[1] = l;
  }
  ring_drain();
}

// ========================================================================== PV
// SINGLE (rows of at most one key tile, wave softmax): the row max and sum
// are formed here from the tile's own scores, in the stats kernel's order,
// and no stats pass runs.
template <typename T, int HD, bool EXACT_SCALE, int SMK, bool SINGLE, bool VNAT>
__global__ __launch_bounds__(AX_THREADS, HD == 64 && !SINGLE ? 3 : 2) void attn_pv2_kernel(AttnArgs a) {
  typedef typename Mfma<T>::vec vec;
  typedef AxK<T, HD> KL;
  typedef AxVTile<T, HD, VNAT> VL;
  constexpr int NST = (HD == 128) ? 2 : 3;
  constexpr int LPW = KL::LD + VL::LD;
  __shared__ __attribute__((aligned(16))) T kv_lds[NST][KL::ELEMS + VL::ELEMS];

  const int S = a.seq, H = a.heads;
  const int nq = (S + AX_BQ - 1) / AX_BQ;
  int bh, qb;
  ax_work_of(nq, a.causal, bh, qb);
  const int b = bh / H, h = bh - b * H;
  const int q0 = qb * AX_BQ;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5;
  const int q0w = q0 + wave * 32, myq = q0w + (lane & 31);
  const float NEG_INF = -__builtin_inff();
  AxHead<T> hp;
  hp.init(a, b, h);

  KL kl;
  kl.init(hp.k, a.k_ss, S, wave, lane);
  VL vl;
  vl.init(hp, a, S, wave, lane);

  // Key-permuted scores (P leaves the exponentials in operand order) except
  // for the single-tile kernel, whose row sum follows ATen's lane order.
  constexpr bool PERM = !SINGLE;
  AxKOff<HD> ko;
  if constexpr (PERM) ko.init_perm(lane);
  else ko.init(lane);
  vec qf[HD / 16];
  {
    const T* qrow = hp.q + (int64_t)min(myq, S - 1) * a.q_ss + 8 * half;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) qf[ks] = __builtin_bit_cast(vec, ld128(qrow + 16 * ks));
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) settle(qf[ks]);
  }
  // Row constants.  A row with no admissible key (m = -inf) gets m = 0 and
  // l = 1: its scores are all -inf, so p = 0 and o = 0.
  float m = 0.f, l = 1.f;
  if (!SINGLE && myq < S) {
    const float* st = a.row_stats + ((int64_t)bh * S + myq) * 2;
    m = st[0];
    l = st[1];
  }
  if (m == NEG_INF) {
    m = 0.f;
    l = 1.f;
  }
  settle(m);
  settle(l);
  float rinv = 1.0f / l;  // block softmax multiplies by the reciprocal
  float rr = ax_div_recip(l);  // wave softmax: the division's refined reciprocal
  const int n_tiles = ax_n_tiles(S, a.causal, q0);
  const uint8_t* kv = hp.kv;

  f32x16 o_acc[HD / 32];
#pragma unroll
  for (int t = 0; t < HD / 32; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[t][r] = 0.f;

  auto issue = [&](int kt) {
    const int kk = min(kt, n_tiles - 1);
    T* base = kv_lds[kt % NST];
    kl.issue(kk, base);
    vl.issue(kk, base + KL::ELEMS);
  };
#pragma unroll
  for (int s = 0; s < NST - 1; ++s) issue(s);

  for (int kt = 0; kt < n_tiles; ++kt) {
    const int kt0 = kt * AX_BN;
    ring_barrier<LPW * (NST - 2)>();
    T* Ks = kv_lds[kt % NST];
    T* Vs = Ks + KL::ELEMS;
    if (VL::ZERO_TAIL && kt0 + AX_BN > S) {
      // Keys >= S of the last tile: zero V (p is 0 there, and 0 * garbage
      // could be NaN), then make the zeros visible.
      for (int idx = tid; idx < HD * AX_BN; idx += AX_THREADS) {
        const int d = idx / AX_BN, key = idx % AX_BN;
        if (kt0 + key >= S) Vs[d * AX_BN + (((key >> 3) ^ ax_swz8(d)) << 3) + (key & 7)] = (T)0.f;
      }
      __syncthreads();
    }
    issue(kt + NST - 1);
    vl.begin(Vs);

    f32x16 s[2];
    ax_scores<T, HD>(Ks, qf, ko, s);
    // Without a key mask only the last tile can hold missing keys.
    const uint64_t kmask = (kv != nullptr || kt0 + AX_BN > S) ? ax_key_mask(kv, kt0, S, lane) : ~0ull;
    // Wave-uniform, so that unmasked tiles take a scalar branch around the masking.
    const bool need_mask = __builtin_amdgcn_readfirstlane(
        (int)((a.causal && (kt0 + AX_BN - 1 > q0w)) || (kmask != ~0ull))) != 0;
    ax_round_scores<T, EXACT_SCALE>(s, a.scale);
    float x[2][16];       // this tile's exponentials (wave softmax) or shifted scores
    bool fast_e = false;  // the wave softmax's exps took the in-range sequence
    if constexpr (SINGLE) {
      // max of the rounded scores = the rounding of the raw max (monotone).
      float mv[2][16];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mv[t][r] = s[t][r];
      if (need_mask) ax_mask(mv, kmask, a.causal, kt0, myq, lane);
      float mx = NEG_INF;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, mv[t][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const bool dead = (mx == NEG_INF);
      m = dead ? 0.f : (EXACT_SCALE ? mx * a.scale : mx);
      float part[32];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mv[t][r] = ax_shift<EXACT_SCALE>(s[t][r], a.scale, m);
      fast_e = ax_wave_exps(mv, need_mask, kmask, a.causal, kt0, myq, lane);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) part[16 * t + r] = mv[t][r];
      l = dead ? 1.f : ax_wave_softmax_sum(part);
      rr = ax_div_recip(l);
      // The row's only tile: its exponentials serve the sum and p alike (as
      // ATen's softmax keeps them in registers).
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) x[t][r] = mv[t][r];
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) x[t][r] = ax_shift<EXACT_SCALE>(s[t][r], a.scale, m);
      if (SMK == 1) {
        if (need_mask) ax_mask<PERM>(x, kmask, a.causal, kt0, myq, lane);
      } else {
        fast_e = ax_wave_exps<PERM>(x, need_mask, kmask, a.causal, kt0, myq, lane);
      }
    }
    if (SMK == 0) {
      // Wave softmax: p = expf(x) / l, the correctly rounded division (a
      // reciprocal multiply with one correction differs from it in ~4e-6 of
      // fp32 quotients).
      if (fast_e) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) x[t][r] = ax_div_fast(x[t][r], l, rr);
      } else {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) x[t][r] = x[t][r] / l;
      }
    }

#pragma unroll
    for (int u = 0; u < 4; ++u) {
      // No contraction: p is rounded to fp32 and then to T, as eager does
      // (a fused multiply-and-convert would round once).
#pragma clang fp contract(off)
      const int t = u >> 1, hh = u & 1;
      vl.load_step(u);  // natural V: this step's operand reads go out first
      float p8[8];
      if (SMK == 1) {
#pragma unroll
        for (int e = 0; e < 8; ++e) p8[e] = __expf(x[t][8 * hh + e]) * rinv;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) p8[e] = x[t][8 * hh + e];
      }
      // P^T operand: half g holds keys 16u + 8g .. +7 (directly with the
      // key-permuted scores, else after the lane-half swap).
      const uint32_t a0 = pack2<T>(p8[0], p8[1]), a1 = pack2<T>(p8[2], p8[3]);
      const uint32_t b0 = pack2<T>(p8[4], p8[5]), b1 = pack2<T>(p8[6], p8[7]);
      u32x4 pk;
      if constexpr (PERM) {
        pk = u32x4{a0, a1, b0, b1};
      } else {
        auto s0 = __builtin_amdgcn_permlane32_swap(a0, b0, false, false);
        auto s1 = __builtin_amdgcn_permlane32_swap(a1, b1, false, false);
        pk = u32x4{(uint32_t)s0[0], (uint32_t)s1[0], (uint32_t)s0[1], (uint32_t)s1[1]};
      }
      const vec pf = __builtin_bit_cast(vec, pk);
      vl.wait_step();
#pragma unroll
      for (int dt = 0; dt < HD / 32; ++dt) {
        const vec vf = vl.operand(Vs, u, dt);
        o_acc[dt] = Mfma<T>::mma32(vf, pf, o_acc[dt]);
      }
    }
  }
  if (myq < S) {
    T* orow = hp.o + (int64_t)myq * a.o_ss;
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d0 = 32 * dt + 8 * q4 + 4 * half;
        u32x2 pk;
        pk[0] = pack2<T>(o_acc[dt][4 * q4 + 0], o_acc[dt][4 * q4 + 1]);
        pk[1] = pack2<T>(o_acc[dt][4 * q4 + 2], o_acc[dt][4 * q4 + 3]);
        st64(orow + d0, pk);
      }
    }
  }
  ring_drain();
}

// ============================================================ row-resident
// attn_rowres_kernel: the eager-exact path for rows of 65 .. 1024 keys at
// head dim 64 with V head-transposed (the wave softmax), taken for causal
// rows and for grids the two-kernel path would leave under-filled.  One
// workgroup per 32 query rows of one (batch, head); its four waves split
// the row's live key tiles into four consecutive runs of ceil(tiles / 4).
// Each wave forms the scores of its run once, from K fragments read
// straight from global memory, and keeps them in registers (at most 4
// tiles: 128 values a lane), as ATen's wave softmax holds its row in
// registers:
//   * row max: per-wave maxima exchanged through LDS (max is exact and
//     order-free);
//   * e = expf(s - m) once per score (the two-kernel path forms it twice);
//   * row sum in ATen's order: lane slot t of the wave softmax sums the keys
//     t + 64 it in order of it, and tile it lies in the run of wave it / run,
//     so the 32 per-lane partial sums pass from wave to wave through LDS
//     (wave 0 starts from zero, each wave adds its tiles in order), then the
//     xor butterfly of ax_wave_softmax_sum;
//   * p = e / l, rounded to T into an LDS panel of the 32 rows, and P V on
//     v_mfma_f32_16x16x32 with each wave running every key in order for 16
//     head-dim columns: 32 keys per step give the same bits as the
//     two-kernel path's 32x32x16 chain (16 keys per step).
// QK^T runs once instead of three times.
constexpr int AXR_BQ = 32;  // query rows per workgroup

template <typename T, bool EXACT_SCALE>
__global__ __launch_bounds__(AX_THREADS, 2) void attn_rowres_kernel(AttnArgs a) {
  typedef typename Mfma<T>::vec vec;
  constexpr int HD = 64;
  constexpr int TMAX = 4;  // key tiles per wave (S <= 1024)
  __shared__ float red_max[4][32];
  __shared__ float chain[32][64];  // slot sums: 32 values per lane, element-major (no bank conflicts)
  // p of the 32 rows, keys contiguous; rows padded by 16 bytes (bank spread).
  __shared__ __attribute__((aligned(16))) T p_lds[AXR_BQ][1024 + 8];

  const int S = a.seq, H = a.heads;
  const int nq = (S + AXR_BQ - 1) / AXR_BQ;
  int bh, qb;
  ax_work_of(nq, a.causal, bh, qb);
  const int b = bh / H, h = bh - b * H;
  const int q0 = qb * AXR_BQ;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, col = lane & 31;
  const int myq = q0 + col;
  const float NEG_INF = -__builtin_inff();
  AxHead<T> hp;
  hp.init(a, b, h);

  vec qf[HD / 16];
  {
    const T* qrow = hp.q + (int64_t)min(myq, S - 1) * a.q_ss + 8 * half;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) qf[ks] = __builtin_bit_cast(vec, ld128(qrow + 16 * ks));
  }
  // Live tiles of this block (causal: up to its last row) and this wave's run.
  int n_live = (S + AX_BN - 1) / AX_BN;
  if (a.causal) n_live = min(n_live, min(q0 + AXR_BQ - 1, S - 1) / AX_BN + 1);
  const int run = (n_live + 3) / 4;
  const int kt_begin = wave * run;
  const int n_mine = max(0, min(run, n_live - kt_begin));  // wave-uniform
  const uint8_t* kv = hp.kv;

  // ---- scores of the run, rounded as eager rounds them.  K fragments come
  // straight from global memory, one tile ahead of its MFMAs (scheduling
  // barriers keep the compiler from hoisting every tile's loads).
  auto kload = [&](int kt0, vec (&kf)[2][HD / 16]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      // Keys past S read key S - 1 (finite; masked below).
      const T* krow = hp.k + (int64_t)min(kt0 + 32 * t + col, S - 1) * a.k_ss + 8 * half;
#pragma unroll
      for (int ks = 0; ks < HD / 16; ++ks) kf[t][ks] = __builtin_bit_cast(vec, ld128(krow + 16 * ks));
    }
  };
  f32x16 s[TMAX][2];
  uint64_t kmask[TMAX];
  bool need_mask[TMAX];
  vec kf[2][2][HD / 16];  // two tiles' fragments: the current and the next
  if (n_mine > 0) kload(kt_begin * AX_BN, kf[0]);
#pragma unroll
  for (int j = 0; j < TMAX; ++j) {
    kmask[j] = ~0ull;
    need_mask[j] = false;
    if (j < n_mine) {
      const int kt0 = (kt_begin + j) * AX_BN;
      if (j + 1 < n_mine) kload(kt0 + AX_BN, kf[(j + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[j][t][r] = 0.f;
#pragma unroll
      for (int ks = 0; ks < HD / 16; ++ks)
#pragma unroll
        for (int t = 0; t < 2; ++t) s[j][t] = Mfma<T>::mma32(kf[j & 1][t][ks], qf[ks], s[j][t]);
      ax_round_scores<T, EXACT_SCALE>(s[j], a.scale);
      kmask[j] = ax_key_mask(kv, kt0, S, lane);
      need_mask[j] = __builtin_amdgcn_readfirstlane(
                         (int)((a.causal && (kt0 + AX_BN - 1 > q0)) || (kmask[j] != ~0ull))) != 0;
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- row max over the four runs
  float mx = NEG_INF;
#pragma unroll
  for (int j = 0; j < TMAX; ++j) {
    if (j < n_mine) {
      float mv[2][16];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mv[t][r] = s[j][t][r];
      if (need_mask[j]) ax_mask(mv, kmask[j], a.causal, (kt_begin + j) * AX_BN, myq, lane);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, mv[t][r]);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (half == 0) red_max[wave][col] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red_max[0][col], red_max[1][col]), fmaxf(red_max[2][col], red_max[3][col]));
  // A row with no admissible key: m = 0, every exponential is 0, l = 1 below.
  const bool dead = (mx == NEG_INF);
  const float m = dead ? 0.f : (EXACT_SCALE ? mx * a.scale : mx);

  // ---- e = expf(s - m), in place
  bool fast[TMAX];
#pragma unroll
  for (int j = 0; j < TMAX; ++j) {
    fast[j] = true;
    if (j < n_mine) {
      float x[2][16];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) x[t][r] = ax_shift<EXACT_SCALE>(s[j][t][r], a.scale, m);
      fast[j] = ax_wave_exps(x, need_mask[j], kmask[j], a.causal, (kt_begin + j) * AX_BN, myq, lane);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[j][t][r] = x[t][r];
    }
  }

  // ---- row sum: the per-slot partial sums pass through the runs in order
  float part[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) part[i] = 0.f;
  for (int w = 0; w < 4; ++w) {
    if (wave == w) {
      if (w > 0) {
#pragma unroll
        for (int i = 0; i < 32; ++i) part[i] = chain[i][lane];
      }
#pragma unroll
      for (int j = 0; j < TMAX; ++j)
        if (j < n_mine) {
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) part[16 * t + r] += s[j][t][r];
        }
#pragma unroll
      for (int i = 0; i < 32; ++i) chain[i][lane] = part[i];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 32; ++i) part[i] = chain[i][lane];
  const float l = dead ? 1.f : ax_wave_softmax_sum(part);
  const float rr = ax_div_recip(l);

  // The first V^T chunks of P V go out here, so that they land while the
  // divisions run (the barrier below waits for LDS only).
  typedef typename Mfma16<T>::vec vec16;
  const int r16 = lane & 15, g16 = lane >> 4;
  const T* vrow = hp.v + (int64_t)(16 * wave + r16) * a.ldvt;
  const int n_chunks = n_live * (AX_BN / 32);
  f32x4 o16[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  auto vchunk = [&](int c) -> u32x4 {
    const int k0 = 32 * c + 8 * g16;
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (k0 + 8 <= S) {
      v = ld128(vrow + k0);
    } else if (k0 < S) {
      v = ld128(vrow + k0);
      int nv = S - k0;  // valid keys of the chunk
      asm volatile("" : "+v"(nv));  // formed here only (not hoisted)
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) v[e2] &= (2 * e2 + 1 < nv) ? 0xffffffffu : (2 * e2 < nv ? 0x0000ffffu : 0u);
    }
    return v;
  };
  constexpr int VPF = 8;  // V chunks in flight
  u32x4 vq[VPF];
#pragma unroll
  for (int i = 0; i < VPF; ++i)
    if (i < n_chunks) vq[i] = vchunk(i);

  // ---- p = e / l, the correctly rounded division (ax_div_fast where the
  // in-range exponential sequence ran, as attn_pv2_kernel does), rounded to
  // T into the row panel p_lds[query][key] (keys of every run: the P V
  // chain below runs over all of them).
#pragma unroll
  for (int j = 0; j < TMAX; ++j)
    if (j < n_mine) {
      if (fast[j]) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) s[j][t][r] = ax_div_fast(s[j][t][r], l, rr);
      } else {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) s[j][t][r] = s[j][t][r] / l;
      }
      // Slot (t, r) holds key kt0 + 32 t + 8 (r >> 2) + 4 half + (r & 3):
      // four consecutive keys per r >> 2, one 8-byte write.
      const int kt0 = (kt_begin + j) * AX_BN;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const u32x2 pk = u32x2{pack2<T>(s[j][t][4 * rq + 0], s[j][t][4 * rq + 1]),
                                 pack2<T>(s[j][t][4 * rq + 2], s[j][t][4 * rq + 3])};
          st64(&p_lds[col][kt0 + 32 * t + 8 * rq + 4 * half], pk);
        }
    }
  ring_barrier<63>();  // p_lds written; the V^T loads stay in flight

  // ---- P V on v_mfma_f32_16x16x32: wave w owns head-dim columns
  // 16 w .. 16 w + 15 for both 16-query halves, and runs over every key in
  // order, 32 per MFMA (the accumulation of the two-kernel path's
  // 32x32x16 chain, 16 keys per step, gives the same bits: the library's
  // GEMMs on either instruction agree bit for bit with ours).
  // A operand: V^T row 16 w + (lane & 15), keys 32 c + 8 (lane >> 4) .. +7,
  // straight from global memory; B operand: p_lds row 16 qh + (lane & 15),
  // same keys.  Columns past S are padding of the V^T rows (a chunk that
  // starts below S ends inside ldvt = round_up(S, 8)): zeroed; chunks at or
  // past S are not read.
  for (int c0 = 0; c0 < n_chunks; c0 += VPF) {
#pragma unroll
    for (int i = 0; i < VPF; ++i) {
      const int c = c0 + i;
      if (c < n_chunks) {
        const vec16 va = __builtin_bit_cast(vec16, vq[i]);
        if (c + VPF < n_chunks) vq[i] = vchunk(c + VPF);
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) {
          const vec16 pb = __builtin_bit_cast(vec16, ld128(&p_lds[16 * qh + r16][32 * c + 8 * g16]));
          o16[qh] = Mfma16<T>::mma(va, pb, o16[qh]);
        }
      }
    }
  }
  // Lane l: query q0 + 16 qh + (l & 15), head-dim columns 16 w + 4 (l >> 4) .. +3.
#pragma unroll
  for (int qh = 0; qh < 2; ++qh) {
    const int q = q0 + 16 * qh + r16;
    if (q < S) {
      T* orow = hp.o + (int64_t)q * a.o_ss + 16 * wave + 4 * g16;
      st64(orow, u32x2{pack2<T>(o16[qh][0], o16[qh][1]), pack2<T>(o16[qh][2], o16[qh][3])});
    }
  }
}

// ================================================== one key tile, four waves
// Rows of at most one key tile (S <= 64) at head dim 64, V^T layout.  The
// eager wave softmax's chain for 32 queries (scores, max, exponentials, the
// butterfly sum, division, P V) is split over four waves, so each wave's
// vector chain is a quarter of the one-wave chain: wave w takes query half
// qh = w >> 1 (16 queries) and key half th = w & 1, on 16x16x32 MFMAs.
// Register e of lane l holds key 32 th + 16 kb + 4 (l >> 4) + e of query
// 16 qh + (l & 15) (kb: the 16-key block), so the wave softmax's butterfly
// levels are: offset 32 = th (the partner wave, through LDS; both waves of a
// pair then form the same sum), 16 = kb (in the lane), 8 and 4 = lane bits 5
// and 4, 2 and 1 = e.  The max is exchanged the same way (order-free).  p goes
// to an LDS panel [32 queries][64 keys]; each wave runs P V for its 16
// queries and 32 of the head-dim columns, 32 keys per step in order.  Q, K and
// V^T come straight from global memory (one tile, nothing to stage).  The
// results are those of attn_pv2_kernel's one-tile path: the same products in
// the same key order, roundings and reduction orders.
template <typename T, bool EXACT_SCALE>
__global__ __launch_bounds__(256) void attn_tile4_kernel(AttnArgs a) {
  typedef typename Mfma16<T>::vec vec;
  constexpr int HD = 64, PLD = 72;  // panel row stride (elements)
  __shared__ float red_max[2][32];
  __shared__ float red_e[2][2][8][64];
  __shared__ __attribute__((aligned(16))) T p_lds[32 * PLD];

  const int S = a.seq, H = a.heads;
  const int nq = (S + 31) / 32;
  const int bh = (int)blockIdx.x / nq, qb = (int)blockIdx.x - bh * nq;
  const int b = bh / H, h = bh - b * H;
  const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int th = wave & 1, qh = wave >> 1;
  const int myq = qb * 32 + 16 * qh + c16;
  const float NEG_INF = -__builtin_inff();
  AxHead<T> hp;
  hp.init(a, b, h);

  // Operands, all requested up front.  Keys >= S read key S - 1 (masked);
  // V^T chunks past the row end re-read its last chunk (zeroed below).
  vec qf[2], kf[2][2], vf[2][2];
  {
    const T* qrow = hp.q + (int64_t)min(myq, S - 1) * a.q_ss + 8 * g;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) qf[kc] = __builtin_bit_cast(vec, ld128(qrow + 32 * kc));
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const T* krow = hp.k + (int64_t)min(32 * th + 16 * kb + c16, S - 1) * a.k_ss + 8 * g;
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) kf[kb][kc] = __builtin_bit_cast(vec, ld128(krow + 32 * kc));
    }
    const int vlast = (int)a.ldvt - 8;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      const T* vrow = hp.v + (int64_t)(32 * th + 16 * db + c16) * a.ldvt;
#pragma unroll
      for (int c = 0; c < 2; ++c) vf[db][c] = __builtin_bit_cast(vec, ld128(vrow + min(32 * c + 8 * g, vlast)));
    }
  }

  // x[4 kb + e] = score of key 32 th + 16 kb + 4 g + e, rounded as eager rounds it.
  float x[8];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) acc = Mfma16<T>::mma(kf[kb][kc], qf[kc], acc);
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      float u = acc[e], v = acc[e + 1];
      ax_round2<T, false>(u, v);
      if (!EXACT_SCALE) {
        u *= a.scale;
        v *= a.scale;
        ax_round2<T>(u, v);
      }
      x[4 * kb + e] = u;
      x[4 * kb + e + 1] = v;
    }
  }
  const uint64_t kmask = ax_key_mask(hp.kv, 0, S, lane);
  const bool need_mask = __builtin_amdgcn_readfirstlane(
      (int)((a.causal && (32 * th + 31 > qb * 32 + 16 * qh)) || (kmask != ~0ull))) != 0;
  const uint32_t km = (uint32_t)(kmask >> (32 * th + 4 * g));
  const int lim = a.causal ? myq - 32 * th - 4 * g : AX_BN;
  auto mask8 = [&](float* v, float val) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = 16 * (i >> 2) + (i & 3);
      v[i] = (((km >> c) & 1u) && c <= lim) ? v[i] : val;
    }
  };

  // Row max over the query's 64 keys: 4 lanes of this wave, then the partner.
  float mx = NEG_INF;
  {
    float mv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) mv[i] = x[i];
    if (need_mask) mask8(mv, NEG_INF);
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = fmaxf(mx, mv[i]);
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (g == 0) red_max[th][16 * qh + c16] = mx;
  ring_barrier<63>();  // LDS only: nothing of this wave's memory reads waits here
  mx = fmaxf(mx, red_max[th ^ 1][16 * qh + c16]);
  const bool dead = (mx == NEG_INF);
  const float m = dead ? 0.f : (EXACT_SCALE ? mx * a.scale : mx);

  // e = expf(s - m), 0 on masked keys.
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = ax_shift<EXACT_SCALE>(x[i], a.scale, m);
  float mn = x[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) mn = fminf(mn, x[i]);
  const bool fast = __builtin_amdgcn_readfirstlane((int)__all(mn > AX_FAST_X)) != 0;
  if (fast) {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = ax_expf_inrange(x[i]);
    if (need_mask) mask8(x, 0.f);
  } else {
    if (need_mask) mask8(x, NEG_INF);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = expf(x[i]);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) red_e[th][qh][i][lane] = x[i];
  ring_barrier<63>();
  float l;
  {
    float v1[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v1[i] = x[i] + red_e[th ^ 1][qh][i][lane];  // offset 32
    float v2[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v2[e] = v1[e] + v1[4 + e];                   // offset 16
#pragma unroll
    for (int e = 0; e < 4; ++e) v2[e] = v2[e] + __shfl_xor(v2[e], 32, 64);   // offset 8
#pragma unroll
    for (int e = 0; e < 4; ++e) v2[e] = v2[e] + __shfl_xor(v2[e], 16, 64);   // offset 4
    const float v5a = v2[0] + v2[2], v5b = v2[1] + v2[3];                    // offset 2
    l = dead ? 1.f : v5a + v5b;                                              // offset 1
  }
  if (fast) {
    const float rr = ax_div_recip(l);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = ax_div_fast(x[i], l, rr);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = x[i] / l;
  }

  // p into the panel: row 16 qh + (l & 15), keys 32 th + 16 kb + 4 g .. +3.
  {
#pragma clang fp contract(off)
    T* prow = p_lds + (16 * qh + c16) * PLD + 32 * th + 4 * g;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
      *reinterpret_cast<u32x2*>(prow + 16 * kb) =
          u32x2{pack2<T>(x[4 * kb + 0], x[4 * kb + 1]), pack2<T>(x[4 * kb + 2], x[4 * kb + 3])};
  }
  // V^T values of keys >= S are zeroed (p is 0 there; 0 * a re-read value
  // must not reach the sum as NaN).
  if (S < AX_BN) {
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        u32x4 w = __builtin_bit_cast(u32x4, vf[db][c]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int k0 = 32 * c + 8 * g + 2 * j;
          const uint32_t keep = (k0 + 1 < S) ? 0xffffffffu : (k0 < S ? 0x0000ffffu : 0u);
          w[j] &= keep;
        }
        vf[db][c] = __builtin_bit_cast(vec, w);
      }
  }
  ring_barrier<63>();

  // O^T block db (16 head-dim columns x 16 queries) += V^T (16 x 32 keys) P^T,
  // keys 0..31 then 32..63.
  const T* pq = p_lds + (16 * qh + c16) * PLD + 8 * g;
  const vec pf0 = __builtin_bit_cast(vec, ld128(pq)), pf1 = __builtin_bit_cast(vec, ld128(pq + 32));
  if (myq < S) {
    T* orow = hp.o + (int64_t)myq * a.o_ss + 32 * th + 4 * g;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      f32x4 o = {0.f, 0.f, 0.f, 0.f};
      o = Mfma16<T>::mma(vf[db][0], pf0, o);
      o = Mfma16<T>::mma(vf[db][1], pf1, o);
      st64(orow + 16 * db, u32x2{pack2<T>(o[0], o[1]), pack2<T>(o[2], o[3])});
    }
  }
}

// ============================================================ online (1 pass)
// TX_SOFTMAX_ONLINE: one pass over the keys with a running row max, for
// workloads gated against fp32 rather than against the eager chain (no eager
// baseline exists at S = 100000).  q is scaled once by c = scale * log2(e)
// and rounded to T (q' = round(q c)); QK^T starts from the accumulator value
// -m, so that it yields acc = q' k - m directly in log2 units, with m the
// running row max of q' k.  Scores stay fp32 (no bf16 rounding): p =
// exp2(acc), rounded to T only as the MFMA operand of P V; o = round(sum p v /
// sum p).  The running max is re-based only when it grows past m + 8
// (p <= 2^8), so most tiles skip the rescale of o and l.
//
// At head_dim 64 a wave issues per 64-key tile 32 exponentials, 16
// conversions, 16 max3 and ~10 other vector ops beside 16 32x32x16 MFMAs and
// 4 16x16x32 MFMAs (the row sum).  Scores come from the key-permuted K
// operand, so P needs no lane exchange; the row sum runs on the matrix cores
// with a 0/1 selector operand instead of 32 vector adds; the max offset
// rides in the accumulator instead of 32 FMAs.  Together these took 7% off
// the kernel at S = 100000.  Measured slower and not used:
// issuing the next tile's QK^T among this tile's exponentials (a one-tile
// software pipeline, bit-identical: +10% with three or four ring stages; two
// score sets need 186 VGPRs, i.e. two waves per SIMD, and the loop-carried
// scores cost 32 moves per tile, or 34 accumulator moves when unrolled by
// two), the
// row sum as a full 32x32x16 MFMA with an all-ones operand (+8%), 128 VGPRs
// with a two-stage ring for four waves per SIMD (+2%), and raising the wave
// priority (s_setprio 1) around the QK^T MFMAs (-1%, within run-to-run
// spread) or around every MFMA group (+2%).
template <typename T, int HD, bool VNAT>
__global__ __launch_bounds__(AX_THREADS, 2) void attn_flash_kernel(AttnArgs a) {
  typedef typename Mfma<T>::vec vec;
  typedef AxK<T, HD> KL;
  typedef AxVTile<T, HD, VNAT> VL;
  constexpr int NST = (HD == 128) ? 2 : 3;
  constexpr int LPW = KL::LD + VL::LD;
  __shared__ __attribute__((aligned(16))) T kv_lds[NST][KL::ELEMS + VL::ELEMS];

  const int S = a.seq, H = a.heads;
  const int nq = (S + AX_BQ - 1) / AX_BQ;
  int bh, qb;
  ax_work_of(nq, a.causal, bh, qb);
  const int b = bh / H, h = bh - b * H;
  const int q0 = qb * AX_BQ;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int q0w = q0 + wave * 32, myq = q0w + (lane & 31);
  const float NEG_INF = -__builtin_inff();
  const float c = a.scale * 1.4426950408889634f;
  AxHead<T> hp;
  hp.init(a, b, h);

  KL kl;
  kl.init(hp.k, a.k_ss, S, wave, lane);
  VL vl;
  vl.init(hp, a, S, wave, lane);
  AxKOff<HD> ko;
  ko.init_perm(lane);
  vec qf[HD / 16];
  {
    const T* qrow = hp.q + (int64_t)min(myq, S - 1) * a.q_ss + 8 * half;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) qf[ks] = __builtin_bit_cast(vec, ld128(qrow + 16 * ks));
    // Scores in log2 units: q c, rounded to T once per row.
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) {
      const u32x4 w = __builtin_bit_cast(u32x4, qf[ks]);
      u32x4 sc;
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[j] = pack2<T>(unpack8<T>(w, 2 * j) * c, unpack8<T>(w, 2 * j + 1) * c);
      qf[ks] = __builtin_bit_cast(vec, sc);
    }
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) settle(qf[ks]);
  }
  const int n_tiles = ax_n_tiles(S, a.causal, q0);
  const uint8_t* kv = hp.kv;

  f32x16 o_acc[HD / 32];
#pragma unroll
  for (int t = 0; t < HD / 32; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[t][r] = 0.f;
  // m_run: running row max of q c k (log2 units); mc: the value the scores
  // are measured from (m_run, or 0 before the first admissible key), fed to
  // QK^T as the accumulator's initial value -mc so that p = exp2(acc).
  float m_run = NEG_INF, mc = 0.f;
  f32x16 negm;
#pragma unroll
  for (int r = 0; r < 16; ++r) negm[r] = 0.f;
  // Row sum on the matrix cores: D(16x16) += A(16x32) P^T(32x16) per 16-key
  // step, with P as the B operand (lane l: column l & 15, k-group l >> 4 =
  // query (l & 15) + 16 ((l >> 4) & 1), keys 8 (l >> 5) .. +7) and the 0/1
  // selector A[i][8 g + e] = ((g & 1) == ((i >> 2) & 1)).  Register e of lane
  // l holds D row 4 (l >> 4) + e, column l & 15: the sum over all 16 keys of
  // query (l & 15) + 16 ((l >> 4) & 1) = the lane's own query, in all four
  // registers.
  typedef typename Mfma16<T>::vec vec16;
  vec16 sel;
  {
    const uint32_t one2 = std::is_same<T, bf16>::value ? 0x3F803F80u : 0x3C003C00u;
    const uint32_t w = (((lane >> 4) & 1) == (((lane & 15) >> 2) & 1)) ? one2 : 0u;
    sel = __builtin_bit_cast(vec16, u32x4{w, w, w, w});
  }
  f32x4 lsum = {0.f, 0.f, 0.f, 0.f};

  auto issue = [&](int kt) {
    const int kk = min(kt, n_tiles - 1);
    T* base = kv_lds[kt % NST];
    kl.issue(kk, base);
    vl.issue(kk, base + KL::ELEMS);
  };
#pragma unroll
  for (int s = 0; s < NST - 1; ++s) issue(s);

  for (int kt = 0; kt < n_tiles; ++kt) {
    const int kt0 = kt * AX_BN;
    ring_barrier<LPW * (NST - 2)>();  // tile kt
    T* Vs = kv_lds[kt % NST] + KL::ELEMS;
    if (VL::ZERO_TAIL && kt0 + AX_BN > S) {
      // Keys >= S of the last tile: zero V (p is 0 there, and 0 * garbage
      // could be NaN), then make the zeros visible.
      for (int idx = tid; idx < HD * AX_BN; idx += AX_THREADS) {
        const int d = idx / AX_BN, key = idx % AX_BN;
        if (kt0 + key >= S) Vs[d * AX_BN + (((key >> 3) ^ ax_swz8(d)) << 3) + (key & 7)] = (T)0.f;
      }
      __syncthreads();
    }
    issue(kt + NST - 1);
    vl.begin(Vs);
    f32x16 sn[2];
    ax_scores<T, HD>(kv_lds[kt % NST], qf, ko, sn, &negm);
    // A use of -mc after both MFMAs: the second then also reads it in place
    // as its C operand instead of copying it into its accumulator first
    // (eight v_mov_b64 per tile).
    asm volatile("" ::"v"(negm));

    float x[2][16];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) x[t][r] = sn[t][r];
    // Without a key mask only the last tile can hold missing keys.
    const uint64_t kmask = (kv != nullptr || kt0 + AX_BN > S) ? ax_key_mask(kv, kt0, S, lane) : ~0ull;
    const bool need_mask = __builtin_amdgcn_readfirstlane(
        (int)((a.causal && (kt0 + AX_BN - 1 > q0w)) || (kmask != ~0ull))) != 0;
    if (need_mask) ax_mask<true>(x, kmask, a.causal, kt0, myq, lane);
    float mx = NEG_INF;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, x[t][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // Re-base when the row max grows past m_run + 8 (p <= 2^8 otherwise).
    if (__any(mx + mc > m_run + 8.f)) {
      const float m_new = fmaxf(m_run, mx + mc);
      const float corr = (m_run == NEG_INF) ? 0.f : exp2f(m_run - m_new);
#pragma unroll
      for (int j = 0; j < 4; ++j) lsum[j] *= corr;
#pragma unroll
      for (int t = 0; t < HD / 32; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o_acc[t][r] *= corr;
      m_run = m_new;
      const float mc_new = (m_run == NEG_INF) ? 0.f : m_run;
      const float sh = mc_new - mc;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) x[t][r] -= sh;
      mc = mc_new;
#pragma unroll
      for (int r = 0; r < 16; ++r) negm[r] = -mc;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = u >> 1, hh = u & 1;
      vl.load_step(u);  // natural V: this step's operand reads go out first
      float p8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // The hardware exp2: no subnormal handling; p < 2^-126 becomes 0,
        // against a row sum >= 1.
        p8[e] = __builtin_amdgcn_exp2f(x[t][8 * hh + e]);
      }
      // p comes straight out of the exponential: nothing to fuse with the
      // conversion, so no fp32 barrier (which would copy every p).  With the
      // key-permuted K operand the eight values are already the lane's eight
      // consecutive keys of this 16-key step.
      const u32x4 pk = u32x4{pack2_raw<T>(p8[0], p8[1]), pack2_raw<T>(p8[2], p8[3]),
                             pack2_raw<T>(p8[4], p8[5]), pack2_raw<T>(p8[6], p8[7])};
      const vec pf = __builtin_bit_cast(vec, pk);
      lsum = Mfma16<T>::mma(sel, __builtin_bit_cast(vec16, pk), lsum);
      vl.wait_step();
#pragma unroll
      for (int dt = 0; dt < HD / 32; ++dt) {
        const vec vf = vl.operand(Vs, u, dt);
        o_acc[dt] = Mfma<T>::mma32(vf, pf, o_acc[dt]);
      }
    }
  }
  const float l_tot = lsum[0];
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (myq < S) {
    T* orow = hp.o + (int64_t)myq * a.o_ss;
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt) {
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
  ring_drain();
}

// ------------------------------------------------------------------ launch
template <typename T, int HD, bool EXACT, bool VNAT>
static int launch_exact_hd(const AttnArgs& a, dim3 grid, hipStream_t st) {
  dim3 block(AX_THREADS);
  if (a.softmax_mode == TX_SOFTMAX_ONLINE) {
    attn_flash_kernel<T, HD, VNAT><<<grid, block, 0, st>>>(a);
  } else if (HD == 64 && a.seq <= AX_BN) {
    // One key tile: the PV kernel forms the row statistics itself.  At head
    // dim 128 that kernel needs more than 256 registers; those rows take the
    // two-kernel path below.
    if constexpr (HD == 64) {
      if constexpr (!VNAT) {
        // V^T layout: four waves per 32 queries (attn_tile4_kernel).
        const long total = (long)((a.seq + 31) / 32) * a.batch * a.heads;
        if (total > 0x7fffffffL) return TX_EUNSUPPORTED;
        attn_tile4_kernel<T, EXACT><<<dim3((unsigned)total), dim3(256), 0, st>>>(a);
      } else {
        attn_pv2_kernel<T, HD, EXACT, 0, true, VNAT><<<grid, block, 0, st>>>(a);
      }
    }
  } else if (a.seq <= 2048) {
    // Wave softmax.  Head dim 64, V^T layout, up to 1024 keys: the
    // row-resident kernel where it is faster
    // (measured, same bits): causal rows (runs of about half the tiles), and
    // shapes whose 128-query blocks would leave CUs idle (fewer than two
    // workgroups per CU; it launches four times as many).  Long full rows on
    // a full grid keep the two-kernel path: there the row-resident kernel's
    // four-tile runs (two waves per SIMD, waits at its hand-offs) measured
    // 13% slower (c3: 192 vs 169 us).  TX_ATTN_ROWRES=0 / =1 forces either
    // path (A/B timing only).
    static const int rowres_env = [] {
      const char* e = getenv("TX_ATTN_ROWRES");
      return e ? (e[0] == '0' ? 0 : 1) : -1;
    }();
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    const long blocks128 = (long)grid.x;
    const bool rowres = rowres_env >= 0 ? rowres_env == 1 : (a.causal || blocks128 < 2L * cus);
    if (HD == 64 && !VNAT && rowres && a.seq <= 1024) {
      const long total = (long)((a.seq + AXR_BQ - 1) / AXR_BQ) * a.batch * a.heads;
      if (total > 0x7fffffffL) return TX_EUNSUPPORTED;
      attn_rowres_kernel<T, EXACT><<<dim3((unsigned)total), block, 0, st>>>(a);
    } else {
      attn_stats2_kernel<T, HD, EXACT, 0><<<grid, block, 0, st>>>(a);
      attn_pv2_kernel<T, HD, EXACT, 0, false, VNAT><<<grid, block, 0, st>>>(a);
    }
  } else {
    attn_stats2_kernel<T, HD, EXACT, 1><<<grid, block, 0, st>>>(a);
    attn_pv2_kernel<T, HD, EXACT, 1, false, VNAT><<<grid, block, 0, st>>>(a);
  }
  return hipGetLastError() == hipSuccess ? TX_OK : TX_EHIP;
}

template <typename T, int HD, bool EXACT>
static int launch_layout(const AttnArgs& a, dim3 grid, hipStream_t st) {
  return a.vnat ? launch_exact_hd<T, HD, EXACT, true>(a, grid, st)
                : launch_exact_hd<T, HD, EXACT, false>(a, grid, st);
}

template <typename T>
static int launch_exact_typed(const AttnArgs& a0, hipStream_t st) {
  const AttnArgs& a = a0;
  // Eager softmax: only lengths whose ATen softmax order the kernels
  // reproduce (the rule and its reasons: eager_softmax_mirrorable).
  if (a.softmax_mode == TX_SOFTMAX_EAGER &&
      (!eager_softmax_mirrorable(a.seq, device_shared_mem_per_block()) ||
       (a.seq + AX_BN - 1) / AX_BN > AX_MAX_TILES))
    return TX_EUNSUPPORTED;
  const int nq = (a.seq + AX_BQ - 1) / AX_BQ;
  const long total = (long)nq * a.batch * a.heads;
  if (total > 0x7fffffffL) return TX_EUNSUPPORTED;
  dim3 grid((unsigned)total);
  // A power-of-two scale makes round(round(acc) * scale) = round(acc) *
  // scale exactly -- in bf16 always (fp32's exponent range), in fp16 only
  // while the product stays normal: below 2^-14 eager's fp16 multiply rounds
  // it to a subnormal and drops bits.  So only bf16 takes the fused form.
  int e2 = 0;
  const bool exact = std::is_same<T, bf16>::value && (frexpf(a.scale, &e2) == 0.5f);
  if (a.head_dim == 64)
    return exact ? launch_layout<T, 64, true>(a, grid, st) : launch_layout<T, 64, false>(a, grid, st);
  if (a.head_dim == 128)
    return exact ? launch_layout<T, 128, true>(a, grid, st) : launch_layout<T, 128, false>(a, grid, st);
  return TX_EUNSUPPORTED;
}

int launch_attention(const AttnArgs& a, int dt, hipStream_t st) {
  if (dt == TX_BF16) return launch_exact_typed<bf16>(a, st);
  if (dt == TX_F16) return launch_exact_typed<f16>(a, st);
  return TX_EUNSUPPORTED;
}

// ------------------------------------------------- fixed scratch (no-alloc)
// Row-statistics workspace of tx_flash_attn_fwd_noalloc: (max, sum) per
// query row, TX_NOALLOC_MAX_STAT_ROWS rows (8 MiB).  Each device holds its
// own copy from module load to process end.  Every call on a device shares
// it; the stats pass writes every row it covers before the PV pass of the
// same call reads it, so nothing needs clearing between calls, and calls that
// overlap on one device race.
static __device__ __align__(256) float scratch[2 * TX_NOALLOC_MAX_STAT_ROWS];

// Device address of this device's scratch, resolved once per device with
// that device current (the array's host-side name is not a device address).
float* scratch_device_ptr() {
  constexpr int MAX_DEV = 64;
  static float* ptr[MAX_DEV];
  static hipError_t err[MAX_DEV];
  static std::once_flag once[MAX_DEV];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) return nullptr;
  std::call_once(once[dev], [dev]() {
    void* p = nullptr;
    err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    ptr[dev] = (float*)p;
  });
  return err[dev] == hipSuccess ? ptr[dev] : nullptr;
}

}  // namespace tx
