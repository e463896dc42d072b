// Host-side predicates of the entry points' argument checks and of the GEMM
// kernel routing.  Plain C++ (no HIP): tests compile this header with the
// host compiler and check the rules at their boundaries.
#pragma once

#include <stdint.h>

namespace tx {

// gemm_hp_kernel forms each lane's DMA source offset within a 256-row tile
// as a 32-bit int: (row * ld + 8 * chunk) * element_size with row <= 255,
// chunk <= 7, and the k step offset k * element_size.  Shapes whose offsets
// could pass INT32_MAX take a kernel with 64-bit addressing instead.
inline bool hp_offsets_fit(int64_t lda, int64_t ldw, int64_t k, int64_t elem_size) {
  if (lda < 0 || ldw < 0 || k < 0 || elem_size <= 0) return false;
  const int64_t ld = lda > ldw ? lda : ldw;
  if (ld > (int64_t)1 << 40) return false;
  return (255 * ld + 8 * 7) * elem_size <= (int64_t)INT32_MAX && k * elem_size <= (int64_t)INT32_MAX;
}

// Largest element offset of a [batch, heads, seq, head_dim] view with element
// strides st[0..2] (st[3] = 1); -1 when it does not fit in 62 bits.
inline int64_t view_max_offset(const int64_t* st, int64_t batch, int64_t heads, int64_t seq,
                               int64_t head_dim) {
  const int64_t size[3] = {batch, heads, seq};
  __int128 off = head_dim - 1;
  for (int i = 0; i < 3; ++i) off += (__int128)(size[i] - 1) * st[i];
  if (off < 0 || off > ((__int128)1 << 62)) return -1;
  return (int64_t)off;
}

// True when no two (b, h, s) rows of the view share an element: with the
// dimensions of extent > 1 taken in ascending stride order, each stride
// reaches past everything the smaller ones cover (head_dim contiguous
// elements first).  Interleavings that this rule refuses are not used by
// any caller of the attention entry points.
inline bool view_is_nonoverlapping(const int64_t* st, int64_t batch, int64_t heads, int64_t seq,
                                   int64_t head_dim) {
  int64_t size[3] = {batch, heads, seq};
  int64_t stride[3] = {st[0], st[1], st[2]};
  int idx[3] = {0, 1, 2};
  for (int a = 0; a < 3; ++a)
    for (int b = a + 1; b < 3; ++b)
      if (stride[idx[b]] < stride[idx[a]]) {
        const int t = idx[a];
        idx[a] = idx[b];
        idx[b] = t;
      }
  __int128 reach = head_dim;  // elements [0, reach) covered so far
  for (int j = 0; j < 3; ++j) {
    const int i = idx[j];
    if (size[i] <= 1) continue;
    if (stride[i] < reach) return false;
    reach += (__int128)(size[i] - 1) * stride[i];
  }
  return true;
}

// Whether the byte ranges [a, a + a_len) and [b, b + b_len) intersect.
inline bool spans_overlap(uintptr_t a, int64_t a_len, uintptr_t b, int64_t b_len) {
  if (a_len <= 0 || b_len <= 0) return false;
  return a < b + (uintptr_t)b_len && b < a + (uintptr_t)a_len;
}

}  // namespace tx

namespace tx {

// Threads of ATen's block softmax (rows longer than 2048 fp32 values).
constexpr int ATEN_SOFTMAX_BLOCK_THREADS = 512;

// Rows whose eager softmax (the eager chain's torch.softmax(scores.float()),
// TTB:187) the kernels reproduce bit for bit.  Up to 2048 keys (2048 fp32
// values fill its 8 KB limit): ATen's warp softmax, one 64-lane wave per row,
// lane t summing the keys t + 64 i in order of i -- always.  Longer rows: its
// 512-thread block softmax, thread t summing the keys 4t + 2048 i + j (4-value
// vectors, j = 0..3, then i ascending).  That order holds when every row is
// read as whole vectors (S a multiple of 4) and either the row fits the
// block's shared-memory copy (S < (shared_mem_per_block - 32) / 4: the cached
// variant) or the uncached variant has no element-wise tail (S a multiple of
// 2048).  Other lengths start rows off 16-byte alignment or end them with a
// tail that ATen assigns to threads differently; they are refused.  The eager
// chain itself needs S^2 scores per head, so S is also capped at 65536.
inline bool eager_softmax_mirrorable(int64_t S, int64_t shared_mem_per_block) {
  if (S <= 0) return false;
  if (S <= 2048) return true;
  if (S > 65536 || S % 4 != 0) return false;
  const int64_t T = ATEN_SOFTMAX_BLOCK_THREADS;
  const int64_t cached_limit = (shared_mem_per_block - T / 64 * 4) / 4;
  return S < cached_limit || S % (4 * T) == 0;
}

}  // namespace tx
