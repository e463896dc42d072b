// Boundary checks of the host-side predicates in csrc/limits.hpp (the GEMM
// routing rule and the attention output-view rules).  Prints "ok" or the
// first failing check.
#include <stdio.h>

#include "limits.hpp"

static int fails = 0;
#define CHECK(c)                                   \
  do {                                             \
    if (!(c)) {                                    \
      printf("FAIL line %d: %s\n", __LINE__, #c); \
      ++fails;                                     \
    }                                              \
  } while (0)

int main() {
  using namespace tx;
  // (255 ld + 56) * 2 <= 2^31 - 1  <=>  ld <= 4210752 for 16-bit operands.
  CHECK(hp_offsets_fit(1024, 1024, 1024, 2));
  CHECK(hp_offsets_fit(4210752, 64, 64, 2));
  CHECK(!hp_offsets_fit(4210753, 64, 64, 2));
  CHECK(!hp_offsets_fit(64, 4210753, 64, 2));
  CHECK(!hp_offsets_fit(4210760, 64, 64, 2));  // the GPU routing test's stride
  CHECK(hp_offsets_fit(8192, 8192, (1 << 30) - 1, 2));
  CHECK(!hp_offsets_fit(8192, 8192, 1 << 30, 2));
  CHECK(hp_offsets_fit(2105375, 64, 64, 4));
  CHECK(!hp_offsets_fit(2105376, 64, 64, 4));  // 4-byte elements halve the limit
  CHECK(!hp_offsets_fit(-1, 64, 64, 2));

  const long B = 2, H = 16, S = 512, HD = 64, D = H * HD;
  const int64_t contiguous[4] = {H * S * HD, S * HD, HD, 1};   // [B, H, S, hd]
  const int64_t merged[4] = {S * D, HD, D, 1};                 // [B, S, H, hd] viewed as [B, H, S, hd]
  const int64_t col_slice[4] = {S * 3 * D, HD, 3 * D, 1};      // q of a packed [B, S, 3D]
  const int64_t head_zero[4] = {S * D, 0, D, 1};
  const int64_t rows_short[4] = {S * D, HD, HD / 2, 1};
  const int64_t batch_interleaved_bad[4] = {32, S * D, D, 1};
  const int64_t batch_interleaved_ok[4] = {64, 2 * S * D, 128 * 8, 1};
  CHECK(view_is_nonoverlapping(contiguous, B, H, S, HD));
  CHECK(view_is_nonoverlapping(merged, B, H, S, HD));
  CHECK(view_is_nonoverlapping(col_slice, B, H, S, HD));
  CHECK(!view_is_nonoverlapping(head_zero, B, H, S, HD));
  CHECK(view_is_nonoverlapping(head_zero, B, 1, S, HD));  // one head: its stride is unused
  CHECK(!view_is_nonoverlapping(rows_short, B, H, S, HD));
  CHECK(!view_is_nonoverlapping(batch_interleaved_bad, B, H, S, HD));
  CHECK(view_is_nonoverlapping(batch_interleaved_ok, B, H, S, HD));

  CHECK(view_max_offset(contiguous, B, H, S, HD) == B * H * S * HD - 1);
  CHECK(view_max_offset(col_slice, B, H, S, HD) == (B - 1) * S * 3 * D + (H - 1) * HD + (S - 1) * 3 * D + HD - 1);
  const int64_t huge[4] = {(int64_t)1 << 40, 0, 0, 1};
  CHECK(view_max_offset(huge, (int64_t)1 << 30, 1, 1, 64) == -1);

  CHECK(spans_overlap(1000, 100, 1099, 10));
  CHECK(!spans_overlap(1000, 100, 1100, 10));
  CHECK(!spans_overlap(1100, 10, 1000, 100));
  CHECK(spans_overlap(1000, 100, 900, 101));
  CHECK(!spans_overlap(1000, 0, 1000, 10));
  const int64_t K64 = 65536, K160 = 163840;
  CHECK(eager_softmax_mirrorable(1, K64));
  CHECK(eager_softmax_mirrorable(1023, K64));   // warp softmax: any length up to 2048
  CHECK(eager_softmax_mirrorable(1025, K64));
  CHECK(eager_softmax_mirrorable(2047, K64));
  CHECK(eager_softmax_mirrorable(2048, K64));
  CHECK(!eager_softmax_mirrorable(2049, K64));  // block softmax: whole 4-value vectors only
  CHECK(eager_softmax_mirrorable(2052, K64));
  CHECK(eager_softmax_mirrorable(8192, K64));
  CHECK(eager_softmax_mirrorable(16372, K64));   // (65536 - 32) / 4 = 16376
  CHECK(!eager_softmax_mirrorable(16376, K64));  // uncached, tail of 16376 % 2048
  CHECK(eager_softmax_mirrorable(18432, K64));   // uncached, 9 x 2048: no tail
  CHECK(eager_softmax_mirrorable(18432 + 4, K160));  // cached with 160 KiB
  CHECK(!eager_softmax_mirrorable(18432 + 4, K64));
  CHECK(eager_softmax_mirrorable(65536, K64));
  CHECK(!eager_softmax_mirrorable(65536 + 2048, K160));  // beyond the eager cap
  CHECK(!eager_softmax_mirrorable(0, K64));
  if (fails == 0) printf("ok\n");
  return fails ? 1 : 0;
}
