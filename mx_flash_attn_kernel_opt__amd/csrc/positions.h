// Token-position arithmetic of appends (paged_decode.hip, host and device).  Sequence lengths,
// positions and table widths are int32; these helpers never form a sum that could wrap.
#pragma once

#include <hip/hip_runtime.h>

#include <climits>

// Cache position of new token j (0 <= j) of a sequence that holds seq_len keys before the
// append: max(seq_len, 0) + j, or -1 when that is at or past table_tokens (the table row's
// max_pages * page_size slots, 0 <= table_tokens <= INT32_MAX).
__host__ __device__ inline int append_position(int seq_len, int j, int table_tokens) {
  const int at = seq_len > 0 ? seq_len : 0;
  return at >= table_tokens - j ? -1 : at + j;
}

// Keys of a sequence that held seq_len keys before `appended` (>= 0) new ones:
// max(seq_len, 0) + appended, saturated at INT32_MAX (which every capacity check then flags).
__host__ __device__ inline int keys_after_append(int seq_len, int appended) {
  const int at = seq_len > 0 ? seq_len : 0;
  return at > INT_MAX - appended ? INT_MAX : at + appended;
}
