"""TEST INFRASTRUCTURE ONLY: the CPU oracle (checker) of the paged GQA decode operator.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only to check or to time the CPU baseline.  The product path
(``mx_flash_attn_kernel_opt__amd``) never imports it and has no CPU fallback.

Pinning (what each function is checked against, in tests/test_oracle.py):
  paged_decode_reference  fp32 torch restatement of task.md:138-148.  Pinned by the fp64
                          brute force below, by torch's own scaled_dot_product_attention on
                          contiguous layouts (an independent library routine), by closed-form
                          known answers (L=1 -> the V row, constant V, q=0 -> mean of V,
                          identical K rows -> mean of V) and by invariants (page permutation,
                          poisoned padding, KV-head permutation).
  paged_decode_fp64       fp64 numpy brute force over tokens (small shapes only); pinned by the
                          same known answers.
  split_partials / combine_partials
                          the split-KV + log-sum-exp merge (optimized_c500_flash_attn.cu:537-551,
                          666-728); pinned by equality with the unsplit oracle for every split
                          size.
  paged_decode_partial_reference / lse_merge_reference
                          one shard's unmerged (o, lse) and the merge of gathered shards
                          (optimized_c500_flash_attn.cu:537-551, 666-728); lse pinned by
                          scipy.special.logsumexp and the closed form log(L) (zero keys), the
                          merge of any page sharding pinned by equality with the unsharded
                          decode (itself pinned by SDPA), including causal multi-token shards.
  paged_decode_append_reference
                          append then decode over the L + S keys (flash_attn_with_kvcache with
                          k / v); pinned by torch SDPA with an explicit end-aligned causal mask
                          over the independently concatenated keys.
  paged_kv_append_reference
                          the paged K/V append (flash_attn_with_kvcache's k / v); pinned by
                          the round trip through the decode oracle against plain attention
                          over the concatenated keys, computed by torch's SDPA.
  paged_decode_fp8_reference
                          the decode over a float8_e4m3fn cache with per-tensor scales
                          (beyond the reference, whose cache is bf16): the decode oracle on
                          caches dequantized by torch's e4m3fn conversion; pinned by known
                          e4m3fn codes (1, 448, the smallest subnormal, -0, NaN), by agreement
                          with the bf16 oracle on the same values and by scale linearity.
  fp8_quantize            what an append into an fp8 cache stores (x / scale saturated to
                          +-448, rounded to nearest even by torch's conversion); pinned by
                          closed-form codes (ties to even at normal and subnormal steps,
                          saturation, signed zero, NaN), by the round trip of all 256 codes
                          and by the half-step error bound.
No reference-held fixtures exist for this path (the reference checks live against the absent
third-party flash_attn_with_kvcache, verify_real.py:40-41), so parity with that library is
unpinned; the task.md:85-96 example is kept as a shape fixture under tests/golden/.
"""

from .paged_attention import (  # noqa: F401
    combine_partials,
    fp8_dequantize,
    fp8_quantize,
    kv_bytes,
    lse_merge_reference,
    paged_decode_append_reference,
    paged_decode_fp64,
    paged_decode_fp8_reference,
    paged_decode_partial_reference,
    paged_decode_reference,
    paged_kv_append_reference,
    split_partials,
)
