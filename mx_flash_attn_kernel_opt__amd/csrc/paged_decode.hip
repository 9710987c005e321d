// Paged GQA decode attention for MI355X (gfx950): split-KV main kernel, log-sum-exp combine
// kernel, split policy, argument validation and the C ABI declared in include/mx_paged_decode.h.
//
// Operator: reference task.md:138-148 (one query token per sequence, paged bf16 K/V cache,
// query head h reads KV head h / group).  The reference's kernel pair is
// submission_clean.cu:66-300 (main) and :307-360 (combine); its launcher is :432-504.  The
// softmax here is the running-max form of optimized_c500_flash_attn.cu:310-461 (page max,
// rescale) and its combine the LSE merge of optimized_c500_flash_attn.cu:666-728.
//
// Design (gfx950, wave64):
//  * One 64-lane wave per (KV head, split, sequence); grid (Hkv, splits, batch) so the Hkv
//    waves that stream the same physical pages are dispatched back to back.
//  * No LDS.  A 16-token chunk of K is loaded straight into the A operand of
//    v_mfma_f32_16x16x32_bf16 (lane = token r16, 8 consecutive dims per k-group g4) and the
//    product is S^T = K . Q^T with the query group as the N dimension.  The 16x16 fp32 result
//    leaves lane (head r16, g4) holding the scores of tokens 4*g4 .. 4*g4+3, which is exactly the
//    B-operand layout of v_mfma_f32_16x16x16_bf16 for O^T = V^T . P^T, so P never moves.
//  * V is loaded as whole 2*D-byte token rows (lane (r16, g4) reads rows 4*g4+r, dims
//    (D/16)*r16 ..) and v_perm_b32 regroups the bf16 halves into V^T operands; PV tile i holds
//    dims d = (D/16)*m + i, so lane (h, g4) ends with the contiguous dims [D/4*g4, D/4*(g4+1)).
//  * K/V chunks are double-buffered in registers; the loop body issues no conditional loads so
//    the compiler's vmcnt waits stay partial.
//  * Online softmax in fp32, log2 domain, with a lazy rescale: the running max only moves when
//    a chunk max exceeds it by more than 8, so p <= 2^8 and the O/l rescale is rare.  The final
//    normalisation uses the same max for numerator and denominator, so the result is exact.
//  * Sequences that fit one split write bf16 output directly; longer ones write normalised fp32
//    partials plus a log2-sum-exp per (head, split), merged by the combine kernel.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>
#include <vector>

#include "mx_paged_decode.h"

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

constexpr int kChunk = 16;             // tokens per PV k-step (one 16x16x16 MFMA)
constexpr float kRescaleSlack = 8.0f;  // log2 units the stale running max may lag behind
constexpr int kStatusBytes = 256;      // device status word region at the start of a workspace

// ------------------------------------------------------------------------------------------
// Device helpers
// ------------------------------------------------------------------------------------------

__device__ __forceinline__ float as_float(uint32_t x) { return __builtin_bit_cast(float, x); }
__device__ __forceinline__ uint32_t as_u32(float x) { return __builtin_bit_cast(uint32_t, x); }

// max over the four lanes {l, l^16, l^32, l^48}: the k-groups that share one head column.
__device__ __forceinline__ float group_max4(float x) {
  auto a = __builtin_amdgcn_permlane32_swap(as_u32(x), as_u32(x), false, false);
  x = fmaxf(as_float(a[0]), as_float(a[1]));
  auto b = __builtin_amdgcn_permlane16_swap(as_u32(x), as_u32(x), false, false);
  return fmaxf(as_float(b[0]), as_float(b[1]));
}

__device__ __forceinline__ float group_sum4(float x) {
  auto a = __builtin_amdgcn_permlane32_swap(as_u32(x), as_u32(x), false, false);
  x = as_float(a[0]) + as_float(a[1]);
  auto b = __builtin_amdgcn_permlane16_swap(as_u32(x), as_u32(x), false, false);
  return as_float(b[0]) + as_float(b[1]);
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

// Round-to-nearest-even pack of two floats into one dword of bf16 (lo in bits 0..15).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}


// Register image of one 16-token chunk of one KV head.
//   k[i]    : K[token r16][32*i + 8*g4 .. +7]            (A operand of QK MFMA i)
//   v[r][w] : V[token 4*g4 + r][(D/16)*r16 + 2w .. +1]   (D/32 dwords per row)
// Compile-time tuning knobs (defaults are the measured best on MI355X).
#ifndef MX_NBUF_D64
#define MX_NBUF_D64 2
#endif
#ifndef MX_NBUF_D128
#define MX_NBUF_D128 2
#endif
#ifndef MX_NBUF_D256
#define MX_NBUF_D256 2
#endif
#ifndef MX_KV_NONTEMPORAL
#define MX_KV_NONTEMPORAL 0
#endif

template <int D>
constexpr int ring_depth() {
  return D == 64 ? MX_NBUF_D64 : (D == 128 ? MX_NBUF_D128 : MX_NBUF_D256);
}

// K/V stream loads: wave-uniform base plus per-lane byte offset.
__device__ __forceinline__ u32x4 ld_kv16(const uint16_t* base, uint32_t byte_off) {
  const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + byte_off);
#if MX_KV_NONTEMPORAL
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}
__device__ __forceinline__ u32x2 ld_kv8(const uint16_t* base, uint32_t byte_off) {
  const u32x2* p = reinterpret_cast<const u32x2*>(reinterpret_cast<const char*>(base) + byte_off);
#if MX_KV_NONTEMPORAL
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}

// Register image of one 16-token chunk of one KV head.
//   k[i]    : K[token r16][32*i + 8*g4 .. +7]            (A operand of QK MFMA i)
//   v[r][w] : V[token 4*g4 + r][(D/16)*r16 + 2w .. +1]   (D/32 dwords per row)
template <int D>
struct Chunk {
  u32x4 k[D / 32];
  uint32_t v[4][D / 32];
};

template <int D>
__device__ __forceinline__ void load_v_row(uint32_t (&dst)[D / 32], const uint16_t* base,
                                           uint32_t byte_off) {
  if constexpr (D == 64) {
    const u32x2 x = ld_kv8(base, byte_off);
    dst[0] = x[0];
    dst[1] = x[1];
  } else {
#pragma unroll
    for (int w = 0; w < D / 32; w += 4) {
      const u32x4 x = ld_kv16(base, byte_off + 4 * w);
      dst[w + 0] = x[0];
      dst[w + 1] = x[1];
      dst[w + 2] = x[2];
      dst[w + 3] = x[3];
    }
  }
}

// Per-lane byte offsets of a chunk inside its page (constant for the whole wave).
struct LaneOffsets {
  uint32_t k;             // K[token r16][8*g4]
  uint32_t v;             // V[token 4*g4][(D/16)*r16]
  uint32_t token_bytes;   // bytes between consecutive tokens of a page
};

// Loads all 16 token rows of a chunk.  A chunk never crosses a page (page_size % 16 == 0),
// so rows past the sequence end in the last chunk are unused slots of an allocated page;
// they are discarded at process time by selects, never by arithmetic.
template <int D>
__device__ __forceinline__ void load_chunk(Chunk<D>& c, const uint16_t* kpage,
                                           const uint16_t* vpage, const LaneOffsets& lo) {
#pragma unroll
  for (int i = 0; i < D / 32; ++i) c.k[i] = ld_kv16(kpage, lo.k + 64 * i);
#pragma unroll
  for (int r = 0; r < 4; ++r) load_v_row<D>(c.v[r], vpage, lo.v + r * lo.token_bytes);
}

template <int D>
struct SoftmaxState {
  f32x4 o[D / 16];  // o[i][j] = O[head r16][(D/16)*(4*g4 + j) + i]
  float m;          // running max (log2 units), identical on the 4 lanes of a head
  float l;          // this lane's share of the running denominator
};

// One chunk of the online softmax.  kMasked: only the first `nvalid` tokens of the chunk are
// real; the scores of the others become -inf and their V rows are replaced by zeros (so NaN or
// Inf in unused page slots cannot reach the accumulators).
template <int D, bool kMasked>
__device__ __forceinline__ void process_chunk(SoftmaxState<D>& st, const Chunk<D>& c,
                                              const bf16x8 (&qop)[D / 32], float scale_log2,
                                              int g4, int nvalid) {
  // S^T[token][head] = K . Q^T  (16 tokens x 16 head slots, contraction over D)
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, c.k[i]), qop[i], s, 0,
                                                 0, 0);
  float x[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x[j] = s[j] * scale_log2;
    if constexpr (kMasked) {
      if (4 * g4 + j >= nvalid) x[j] = -INFINITY;
    }
  }
  float cm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
  cm = group_max4(cm);
  if (__builtin_amdgcn_ballot_w64(cm > st.m + kRescaleSlack)) {
    const float mn = fmaxf(st.m, cm);
    const float alpha = __builtin_amdgcn_exp2f(st.m - mn);
    st.m = mn;
    st.l *= alpha;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) st.o[i] *= alpha;
  }
  float p[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) p[j] = __builtin_amdgcn_exp2f(x[j] - st.m);
  st.l += (p[0] + p[1]) + (p[2] + p[3]);
  const u32x2 pw = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])};
  const s16x4 pop = __builtin_bit_cast(s16x4, pw);

  uint32_t v[4][D / 32];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const bool keep = !kMasked || (4 * g4 + r < nvalid);
#pragma unroll
    for (int w = 0; w < D / 32; ++w) v[r][w] = keep ? c.v[r][w] : 0u;
  }
  // O^T[d][head] += V^T . P^T  (tile i covers dims (D/16)*m + i, m = 0..15)
#pragma unroll
  for (int i = 0; i < D / 16; ++i) {
    const int w = i >> 1;
    const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
    const u32x2 vw = {__builtin_amdgcn_perm(v[1][w], v[0][w], sel),
                      __builtin_amdgcn_perm(v[3][w], v[2][w], sel)};
    st.o[i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, vw), pop,
                                                        st.o[i], 0, 0, 0);
  }
}

// ------------------------------------------------------------------------------------------
// Main split-KV kernel
// ------------------------------------------------------------------------------------------

struct MainShape {
  int64_t page_stride;   // elements between physical pages: page_size * Hkv * D
  int token_stride;      // elements between tokens of a page: Hkv * D
  int num_heads;
  int group;
  int max_pages;         // block_table row width
  int num_pages;         // pool size, 0 = unknown
  int chunk_shift;       // log2(page_size / 16)
  int num_splits;
  int tokens_per_split;  // multiple of page_size
  int cap_tokens;        // seq_lens above this are clamped and flagged
  float scale_log2;      // scale * log2(e)
};

// Grid (Hkv, batch, splits): consecutive workgroup ids, which the dispatcher deals round-robin
// to the 8 XCDs, walk the KV heads of one sequence first, then the sequences, then the splits.
// Every XCD therefore gets an even share of the first split of every sequence (where ragged
// batches keep most of their work), and the Hkv waves that read the same physical pages start
// together.
template <int D, int NBUF>
__global__ __launch_bounds__(64) void mx_paged_decode_splitkv(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, uint16_t* __restrict__ out,
    const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ block_table,
    float* __restrict__ part_o, float* __restrict__ part_lse, uint32_t* __restrict__ status,
    const MainShape sh) {
  constexpr int VW = D / 16;  // dims per lane per V row == number of PV tiles
  const int lane = threadIdx.x;
  const int r16 = lane & 15;
  const int g4 = lane >> 4;
  const int kv = blockIdx.x;
  const int b = blockIdx.y;
  const int split = blockIdx.z;
  const int h = r16;  // head slot inside the group (valid when h < group)
  const bool hvalid = h < sh.group;
  const int qhead = kv * sh.group + h;

  int seq = seq_lens[b];
  if (seq > sh.cap_tokens) {
    if (split == 0 && kv == 0 && lane == 0) atomicOr(status, (uint32_t)MX_DEVICE_SEQ_TOO_LONG);
    seq = sh.cap_tokens;
  }
  if (seq <= 0) {
    // Empty sequence: defined as a zero output.
    if (split == 0 && hvalid) {
      uint16_t* op = out + ((int64_t)b * sh.num_heads + qhead) * D + (D / 4) * g4;
#pragma unroll
      for (int w = 0; w < D / 4; w += 8) *reinterpret_cast<u32x4*>(op + w) = u32x4{0, 0, 0, 0};
    }
    return;
  }
  const int t0 = split * sh.tokens_per_split;
  if (t0 >= seq) return;
  const int t1 = min(t0 + sh.tokens_per_split, seq);
  const bool single = seq <= sh.tokens_per_split;

  // Query operand: lane (h, g4) holds Q[h][32*i + 8*g4 .. +7] for MFMA i.
  bf16x8 qop[D / 32];
  {
    const uint16_t* qp = q + ((int64_t)b * sh.num_heads + qhead) * D + 8 * g4;
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
      u32x4 x = {0, 0, 0, 0};
      if (hvalid) x = *reinterpret_cast<const u32x4*>(qp + 32 * i);
      qop[i] = __builtin_bit_cast(bf16x8, x);
    }
  }

  const int32_t* bt_row = block_table + (int64_t)b * sh.max_pages;
  const int chunk_mask = (1 << sh.chunk_shift) - 1;
  LaneOffsets lo;
  lo.token_bytes = 2u * (uint32_t)sh.token_stride;
  lo.k = 2u * (uint32_t)(r16 * sh.token_stride + kv * D + 8 * g4);
  lo.v = 2u * (uint32_t)(4 * g4 * sh.token_stride + kv * D + VW * r16);
  bool bad_page = false;

  // Element offset of chunk c (16 tokens) of this sequence inside the K/V pools.  Only table
  // entries below ceil(seq / page_size) are ever read.
  auto chunk_base = [&](int c) -> int64_t {
    int pid = bt_row[c >> sh.chunk_shift];
    if (pid < 0 || (sh.num_pages > 0 && pid >= sh.num_pages)) {
      bad_page = true;
      pid = 0;
    }
    return (int64_t)pid * sh.page_stride + (int64_t)((c & chunk_mask) * kChunk) * sh.token_stride;
  };

  SoftmaxState<D> st;
#pragma unroll
  for (int i = 0; i < VW; ++i) st.o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.l = 0.f;

  const int c0 = t0 / kChunk;
  const int c1 = (t1 + kChunk - 1) / kChunk;    // chunk range [c0, c1), last may be partial
  const int last_valid = t1 - (c1 - 1) * kChunk; // tokens of chunk c1-1 (1..16)
  const float sl2 = sh.scale_log2;
  auto nvalid_of = [&](int c) { return c == c1 - 1 ? last_valid : kChunk; };

  Chunk<D> buf[NBUF];
  auto load = [&](Chunk<D>& dst, int64_t base) { load_chunk<D>(dst, kc + base, vc + base, lo); };

  // Register ring of NBUF chunks.  The steady-state loop processes NBUF full chunks and
  // refills their buffers with the next NBUF, with no conditional loads (so the compiler's
  // vmcnt waits stay partial); the page lookups of the refills are issued before the math.
  const int n = c1 - c0;
  if (n >= NBUF) {
#pragma unroll
    for (int i = 0; i < NBUF; ++i) load(buf[i], chunk_base(c0 + i));
    int c = c0;
    while (c + 2 * NBUF <= c1) {
      int64_t nb[NBUF];
#pragma unroll
      for (int i = 0; i < NBUF; ++i) nb[i] = chunk_base(c + NBUF + i);
#pragma unroll
      for (int i = 0; i < NBUF; ++i) {
        process_chunk<D, false>(st, buf[i], qop, sl2, g4, kChunk);
        load(buf[i], nb[i]);
      }
      c += NBUF;
    }
    // c + NBUF <= c1 < c + 2*NBUF: buffers hold chunks c .. c+NBUF-1, `extra` more remain.
    const int extra = c1 - c - NBUF;
#pragma unroll
    for (int i = 0; i < NBUF; ++i) {
      if (i < extra) {
        const int64_t nbase = chunk_base(c + NBUF + i);
        process_chunk<D, true>(st, buf[i], qop, sl2, g4, nvalid_of(c + i));
        load(buf[i], nbase);
      } else {
        process_chunk<D, true>(st, buf[i], qop, sl2, g4, nvalid_of(c + i));
      }
    }
#pragma unroll
    for (int i = 0; i < NBUF; ++i)
      if (i < extra) process_chunk<D, true>(st, buf[i], qop, sl2, g4, nvalid_of(c + NBUF + i));
  } else {
#pragma unroll
    for (int i = 0; i < NBUF; ++i)
      if (i < n) load(buf[i], chunk_base(c0 + i));
#pragma unroll
    for (int i = 0; i < NBUF; ++i)
      if (i < n) process_chunk<D, true>(st, buf[i], qop, sl2, g4, nvalid_of(c0 + i));
  }

  if (bad_page && lane == 0) atomicOr(status, (uint32_t)MX_DEVICE_BAD_PAGE_ID);

  const float l_tot = group_sum4(st.l);
  const float inv = 1.0f / l_tot;
  if (!hvalid) return;
  const int64_t row = (int64_t)b * sh.num_heads + qhead;
  if (single) {
    // bf16 output: lane writes dims [D/4*g4, D/4*(g4+1)), element VW*j + i = o[i][j].
    uint16_t* op = out + row * D + (D / 4) * g4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (VW == 4) {
        const u32x2 w = {pack_bf16x2(st.o[0][j] * inv, st.o[1][j] * inv),
                         pack_bf16x2(st.o[2][j] * inv, st.o[3][j] * inv)};
        *reinterpret_cast<u32x2*>(op + VW * j) = w;
      } else {
#pragma unroll
        for (int i = 0; i < VW; i += 8) {
          u32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            w[e] = pack_bf16x2(st.o[i + 2 * e][j] * inv, st.o[i + 2 * e + 1][j] * inv);
          *reinterpret_cast<u32x4*>(op + VW * j + i) = w;
        }
      }
    }
  } else {
    float* pp = part_o + (row * sh.num_splits + split) * D + (D / 4) * g4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int i = 0; i < VW; i += 4) {
        const f32x4 w = {st.o[i][j] * inv, st.o[i + 1][j] * inv, st.o[i + 2][j] * inv,
                         st.o[i + 3][j] * inv};
        *reinterpret_cast<f32x4*>(pp + VW * j + i) = w;
      }
    }
    if (g4 == 0) part_lse[row * sh.num_splits + split] = st.m + log2f(l_tot);
  }
}

// ------------------------------------------------------------------------------------------
// Combine kernel: out[b, h] = sum_s 2^(lse_s - M) * O_s / sum_s 2^(lse_s - M), M = max_s lse_s
// over the splits that hold tokens of sequence b (optimized_c500_flash_attn.cu:666-728).
// ------------------------------------------------------------------------------------------

template <int D>
__global__ __launch_bounds__(64) void mx_paged_decode_combine(
    const float* __restrict__ part_o, const float* __restrict__ part_lse,
    const int32_t* __restrict__ seq_lens, uint16_t* __restrict__ out, int num_heads,
    int num_splits, int tokens_per_split, int cap_tokens) {
  constexpr int E = D / 64;  // output dims per lane
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x;
  int seq = min(seq_lens[b], cap_tokens);
  if (seq <= tokens_per_split) return;  // single split (or empty): main kernel wrote it
  const int nsv = (seq + tokens_per_split - 1) / tokens_per_split;
  const int64_t row = (int64_t)b * num_heads + h;
  const float* lse = part_lse + row * num_splits;
  const float* po = part_o + row * num_splits * D + E * lane;

  float mx = -INFINITY;
  for (int s = lane; s < nsv; s += 64) mx = fmaxf(mx, lse[s]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));

  float acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
  float wsum = 0.f;
#pragma unroll 4
  for (int s = 0; s < nsv; ++s) {
    const float w = __builtin_amdgcn_exp2f(lse[s] - mx);
    wsum += w;
    const float* src = po + (int64_t)s * D;
    if constexpr (E == 1) {
      acc[0] += w * src[0];
    } else if constexpr (E == 2) {
      const f32x2 x = *reinterpret_cast<const f32x2*>(src);
      acc[0] += w * x[0];
      acc[1] += w * x[1];
    } else {
      const f32x4 x = *reinterpret_cast<const f32x4*>(src);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += w * x[e];
    }
  }
  const float inv = 1.0f / wsum;
  uint16_t* op = out + row * D + E * lane;
  if constexpr (E == 1) {
    op[0] = __builtin_bit_cast(uint16_t, (__bf16)(acc[0] * inv));
  } else if constexpr (E == 2) {
    *reinterpret_cast<uint32_t*>(op) = pack_bf16x2(acc[0] * inv, acc[1] * inv);
  } else {
    const u32x2 w = {pack_bf16x2(acc[0] * inv, acc[1] * inv),
                     pack_bf16x2(acc[2] * inv, acc[3] * inv)};
    *reinterpret_cast<u32x2*>(op) = w;
  }
}

// ------------------------------------------------------------------------------------------
// Host side: errors, planning, workspace, launch
// ------------------------------------------------------------------------------------------

thread_local int g_last_status = MX_STATUS_OK;
thread_local std::string g_last_error;

int fail(int status, const std::string& msg) {
  g_last_status = status;
  g_last_error = msg;
  return status;
}

int ok() {
  g_last_status = MX_STATUS_OK;
  g_last_error.clear();
  return MX_STATUS_OK;
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
int64_t align_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// Split policy (replaces the 104-SM regime table of submission_clean.cu:375-430).  Measured
// on MI355X: the split-KV kernel reaches the device's streaming-read ceiling once about
// 8 MB of K/V loads are in flight, i.e. 2 single-wave workgroups per CU for D=128 (8 KB per
// 16-token chunk, 2 chunks in flight per wave) and 4 per CU for D=64 (4 KB chunks) and
// D=256 (one wave per SIMD, issue-bound).  Every extra split costs a wave prologue and a
// partial write, so the policy asks for just enough splits to reach that wave count.
constexpr int64_t kMinTokensPerSplit = 128;   // amortises Q load, pipeline fill and partials
constexpr int64_t kMaxTokensPerSplit = 4096;  // bounds one wave's share of a long sequence
constexpr int64_t kMaxGridDim = 65535;

int64_t target_waves_per_cu(int64_t head_dim) { return head_dim == 128 ? 2 : 4; }

struct Plan {
  int64_t splits = 1;
  int64_t tokens_per_split = 0;
  int64_t cap_tokens = 0;
  int64_t lse_offset = 0;
  int64_t o_offset = 0;
  int64_t workspace_bytes = kStatusBytes;
  int chunk_shift = 0;
};

int query_num_cus(int64_t* num_cus) {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MX_STATUS_HIP_ERROR, "hipGetDevice failed (no HIP device?)");
  }
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0) {
      (void)hipGetLastError();
      return fail(MX_STATUS_HIP_ERROR, "hipDeviceGetAttribute(MultiprocessorCount) failed");
    }
    cache[dev] = n;
  }
  *num_cus = cache[dev];
  return MX_STATUS_OK;
}

// Validates the shape and computes the split plan.  Performs no HIP call when num_cus > 0.
int make_plan(int64_t batch, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
              int64_t page_size, int64_t max_pages, int64_t max_seq_len, int64_t num_splits,
              int64_t num_cus, Plan* plan) {
  if (batch < 1 || num_heads < 1 || num_kv_heads < 1 || head_dim < 1 || page_size < 1 ||
      max_pages < 1)
    return fail(MX_STATUS_INVALID_SHAPE,
                "batch, num_heads, num_kv_heads, head_dim, page_size and max_pages_per_seq "
                "must all be >= 1");
  if (num_heads % num_kv_heads != 0)
    return fail(MX_STATUS_INVALID_SHAPE, "num_heads must be a multiple of num_kv_heads");
  if (num_heads / num_kv_heads > 16)
    return fail(MX_STATUS_UNSUPPORTED, "query group (num_heads / num_kv_heads) must be <= 16");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(MX_STATUS_UNSUPPORTED, "head_dim must be 64, 128 or 256");
  if (page_size != 16 && page_size != 32 && page_size != 64 && page_size != 128 &&
      page_size != 256)
    return fail(MX_STATUS_UNSUPPORTED, "page_size must be 16, 32, 64, 128 or 256");
  if (num_splits < 0) return fail(MX_STATUS_INVALID_SHAPE, "num_splits must be >= 0");
  if (batch > kMaxGridDim) return fail(MX_STATUS_UNSUPPORTED, "batch must be <= 65535");
  if (num_heads > kMaxGridDim) return fail(MX_STATUS_UNSUPPORTED, "num_heads must be <= 65535");
  if (max_pages > (int64_t)INT32_MAX / page_size)
    return fail(MX_STATUS_UNSUPPORTED, "max_pages_per_seq * page_size must fit in int32");
  if (num_kv_heads * head_dim * page_size > (int64_t)INT32_MAX / 4)
    return fail(MX_STATUS_UNSUPPORTED, "page too large for 32-bit in-page offsets");

  const int64_t table_tokens = max_pages * page_size;
  const int64_t cap = (max_seq_len > 0 && max_seq_len < table_tokens) ? max_seq_len : table_tokens;
  const int64_t cap_pages = ceil_div(cap, page_size);
  int64_t ns;
  if (num_splits > 0) {
    ns = num_splits;
  } else {
    if (num_cus <= 0) {
      const int st = query_num_cus(&num_cus);
      if (st != MX_STATUS_OK) return st;
    }
    const int64_t units = batch * num_kv_heads;
    ns = ceil_div(num_cus * target_waves_per_cu(head_dim), units);
    const int64_t max_by_len = ceil_div(cap, kMinTokensPerSplit);
    if (ns > max_by_len) ns = max_by_len;
    const int64_t min_by_len = ceil_div(cap, kMaxTokensPerSplit);
    if (ns < min_by_len) ns = min_by_len;
  }
  if (ns > cap_pages) ns = cap_pages;
  if (ns < 1) ns = 1;
  const int64_t pages_per_split = ceil_div(cap_pages, ns);
  ns = ceil_div(cap_pages, pages_per_split);  // page-aligned splits, none empty at capacity
  if (ns > kMaxGridDim) return fail(MX_STATUS_UNSUPPORTED, "split count exceeds 65535");

  plan->splits = ns;
  plan->tokens_per_split = pages_per_split * page_size;
  plan->cap_tokens = std::min<int64_t>(table_tokens, ns * plan->tokens_per_split);
  int shift = 0;
  while ((int64_t(kChunk) << shift) < page_size) ++shift;
  plan->chunk_shift = shift;
  if (ns > 1) {
    const int64_t rows = batch * num_heads * ns;
    plan->lse_offset = kStatusBytes;
    plan->o_offset = kStatusBytes + align_up(rows * 4, 256);
    plan->workspace_bytes = plan->o_offset + rows * head_dim * 4;
  } else {
    plan->lse_offset = plan->o_offset = 0;
    plan->workspace_bytes = kStatusBytes;
  }
  return MX_STATUS_OK;
}

// Library-owned workspace, one per device, grow-only (as submission_clean.cu:478-491).
struct DeviceWorkspace {
  void* ptr = nullptr;
  int64_t bytes = 0;
};
std::mutex g_ws_mu;
std::vector<DeviceWorkspace> g_ws;

int internal_workspace(int64_t need, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MX_STATUS_HIP_ERROR, "hipGetDevice failed");
  }
  std::lock_guard<std::mutex> lock(g_ws_mu);
  if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1);
  DeviceWorkspace& ws = g_ws[dev];
  if (ws.ptr == nullptr || ws.bytes < need) {
    const int64_t bytes = std::max<int64_t>(need, 1 << 20);
    if (ws.ptr != nullptr) {
      (void)hipDeviceSynchronize();
      (void)hipFree(ws.ptr);
      ws.ptr = nullptr;
      ws.bytes = 0;
    }
    void* p = nullptr;
    if (hipMalloc(&p, (size_t)bytes) != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      return fail(MX_STATUS_ALLOC_FAILED, "hipMalloc of the internal workspace failed");
    }
    if (hipMemset(p, 0, kStatusBytes) != hipSuccess) {
      (void)hipGetLastError();
      (void)hipFree(p);
      return fail(MX_STATUS_HIP_ERROR, "hipMemset of the internal workspace failed");
    }
    ws.ptr = p;
    ws.bytes = bytes;
  }
  *out = ws.ptr;
  return MX_STATUS_OK;
}

template <int D>
hipError_t launch(const Plan& plan, const void* q, const void* k, const void* v, void* out,
                  const int32_t* seq_lens, const int32_t* block_table, int64_t batch,
                  int64_t num_heads, int64_t num_kv_heads, int64_t page_size, int64_t num_pages,
                  int64_t max_pages, float scale, char* ws, int32_t phase, hipStream_t stream) {
  float* part_lse = plan.splits > 1 ? reinterpret_cast<float*>(ws + plan.lse_offset) : nullptr;
  float* part_o = plan.splits > 1 ? reinterpret_cast<float*>(ws + plan.o_offset) : nullptr;
  if (phase != MX_PHASE_COMBINE_ONLY) {
    MainShape sh;
    sh.page_stride = page_size * num_kv_heads * D;
    sh.token_stride = (int)(num_kv_heads * D);
    sh.num_heads = (int)num_heads;
    sh.group = (int)(num_heads / num_kv_heads);
    sh.max_pages = (int)max_pages;
    sh.num_pages = (num_pages > 0 && num_pages <= INT32_MAX) ? (int)num_pages : 0;
    sh.chunk_shift = plan.chunk_shift;
    sh.num_splits = (int)plan.splits;
    sh.tokens_per_split = (int)plan.tokens_per_split;
    sh.cap_tokens = (int)plan.cap_tokens;
    sh.scale_log2 = scale * 1.4426950408889634f;
    const dim3 grid((unsigned)num_kv_heads, (unsigned)batch, (unsigned)plan.splits);
    hipLaunchKernelGGL((mx_paged_decode_splitkv<D, ring_depth<D>()>), grid, dim3(64), 0, stream,
                       static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                       static_cast<const uint16_t*>(v), static_cast<uint16_t*>(out), seq_lens,
                       block_table, part_o, part_lse, reinterpret_cast<uint32_t*>(ws), sh);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (phase != MX_PHASE_MAIN_ONLY && plan.splits > 1) {
    const dim3 grid((unsigned)num_heads, (unsigned)batch);
    hipLaunchKernelGGL(mx_paged_decode_combine<D>, grid, dim3(64), 0, stream, part_o, part_lse,
                       seq_lens, static_cast<uint16_t*>(out), (int)num_heads, (int)plan.splits,
                       (int)plan.tokens_per_split, (int)plan.cap_tokens);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

// ------------------------------------------------------------------------------------------
// C ABI
// ------------------------------------------------------------------------------------------

extern "C" {

int mx_paged_gqa_decode_plan(int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                             int64_t head_dim, int64_t page_size, int64_t max_pages_per_seq,
                             int64_t max_seq_len, int64_t num_splits, int64_t num_cus,
                             int64_t* splits_out, int64_t* tokens_per_split_out,
                             int64_t* workspace_bytes_out) {
  Plan plan;
  const int st = make_plan(batch, num_heads, num_kv_heads, head_dim, page_size,
                           max_pages_per_seq, max_seq_len, num_splits, num_cus, &plan);
  if (st != MX_STATUS_OK) return st;
  if (splits_out) *splits_out = plan.splits;
  if (tokens_per_split_out) *tokens_per_split_out = plan.tokens_per_split;
  if (workspace_bytes_out) *workspace_bytes_out = plan.workspace_bytes;
  return ok();
}

int64_t mx_paged_gqa_decode_workspace_size(int64_t batch, int64_t num_heads,
                                           int64_t num_kv_heads, int64_t head_dim,
                                           int64_t page_size, int64_t max_pages_per_seq,
                                           int64_t max_seq_len, int64_t num_splits) {
  Plan plan;
  const int st = make_plan(batch, num_heads, num_kv_heads, head_dim, page_size,
                           max_pages_per_seq, max_seq_len, num_splits, 0, &plan);
  if (st != MX_STATUS_OK) return st;
  ok();
  return plan.workspace_bytes;
}

int mx_paged_gqa_decode(const void* q, const void* k_cache, const void* v_cache, void* out,
                        const int32_t* seq_lens, const int32_t* block_table, int64_t batch,
                        int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                        int64_t page_size, int64_t num_pages, int64_t max_pages_per_seq,
                        int64_t max_seq_len, float scale, int64_t num_splits, void* workspace,
                        int64_t workspace_bytes, int32_t phase, void* stream) {
  if (!q || !k_cache || !v_cache || !out || !seq_lens || !block_table)
    return fail(MX_STATUS_NULL_POINTER,
                "q, k_cache, v_cache, out, seq_lens and block_table must be non-NULL");
  if (phase != 0 && phase != MX_PHASE_MAIN_ONLY && phase != MX_PHASE_COMBINE_ONLY)
    return fail(MX_STATUS_INVALID_ARGUMENT, "phase must be 0, 1 or 2");
  if (!std::isfinite(scale)) return fail(MX_STATUS_INVALID_ARGUMENT, "scale must be finite");
  if (num_pages < 0) return fail(MX_STATUS_INVALID_SHAPE, "num_pages must be >= 0");
  Plan plan;
  int st = make_plan(batch, num_heads, num_kv_heads, head_dim, page_size, max_pages_per_seq,
                     max_seq_len, num_splits, 0, &plan);
  if (st != MX_STATUS_OK) return st;
  if (workspace != nullptr) {
    if (workspace_bytes < plan.workspace_bytes)
      return fail(MX_STATUS_WORKSPACE_TOO_SMALL,
                  "workspace_bytes " + std::to_string(workspace_bytes) + " < required " +
                      std::to_string(plan.workspace_bytes));
  } else {
    st = internal_workspace(plan.workspace_bytes, &workspace);
    if (st != MX_STATUS_OK) return st;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  hipError_t e;
  switch (head_dim) {
    case 64:
      e = launch<64>(plan, q, k_cache, v_cache, out, seq_lens, block_table, batch, num_heads,
                     num_kv_heads, page_size, num_pages, max_pages_per_seq, scale, ws, phase, s);
      break;
    case 128:
      e = launch<128>(plan, q, k_cache, v_cache, out, seq_lens, block_table, batch, num_heads,
                      num_kv_heads, page_size, num_pages, max_pages_per_seq, scale, ws, phase, s);
      break;
    default:
      e = launch<256>(plan, q, k_cache, v_cache, out, seq_lens, block_table, batch, num_heads,
                      num_kv_heads, page_size, num_pages, max_pages_per_seq, scale, ws, phase, s);
      break;
  }
  if (e != hipSuccess)
    return fail(MX_STATUS_HIP_ERROR, std::string("kernel launch failed: ") + hipGetErrorString(e));
  return ok();
}

void run_kernel(const void* q, const void* k_cache_paged, const void* v_cache_paged,
                void* output, const int32_t* cache_seqlens, const int32_t* block_table,
                int64_t batch_size, int64_t seqlen_k, int64_t seqlen_q, int64_t num_heads,
                int64_t num_heads_k, int64_t headdim, int64_t page_block_size,
                int64_t num_blocks, int64_t causal) {
  int st;
  if (seqlen_q != 1) {
    st = fail(MX_STATUS_UNSUPPORTED, "run_kernel: seqlen_q must be 1 (decode)");
  } else if (causal != 0) {
    st = fail(MX_STATUS_UNSUPPORTED, "run_kernel: causal must be 0");
  } else if (batch_size < 1 || num_blocks < batch_size || num_blocks % batch_size != 0) {
    st = fail(MX_STATUS_INVALID_SHAPE,
              "run_kernel: num_blocks must be a positive multiple of batch_size");
  } else if (seqlen_k < 1) {
    st = fail(MX_STATUS_INVALID_SHAPE, "run_kernel: seqlen_k must be >= 1");
  } else if (headdim < 1) {
    st = fail(MX_STATUS_INVALID_SHAPE, "run_kernel: headdim must be >= 1");
  } else {
    const float scale = 1.0f / sqrtf((float)headdim);
    // The legacy ABI carries no pool size (num_blocks is the table row width times batch),
    // so only negative page ids are flagged.
    st = mx_paged_gqa_decode(q, k_cache_paged, v_cache_paged, output, cache_seqlens,
                             block_table, batch_size, num_heads, num_heads_k, headdim,
                             page_block_size, 0, num_blocks / batch_size, seqlen_k, scale, 0,
                             nullptr, 0, 0, nullptr);
  }
  if (st != MX_STATUS_OK) fprintf(stderr, "run_kernel: %s\n", g_last_error.c_str());
}

int mx_read_device_status(void* workspace, int32_t reset, void* stream, int32_t* flags_out) {
  if (!flags_out) return fail(MX_STATUS_NULL_POINTER, "flags_out must be non-NULL");
  if (workspace == nullptr) {
    int st = internal_workspace(kStatusBytes, &workspace);
    if (st != MX_STATUS_OK) return st;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t word = 0;
  if (hipMemcpyAsync(&word, workspace, sizeof(word), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MX_STATUS_HIP_ERROR, "reading the device status word failed");
  }
  if (reset && word != 0) {
    if (hipMemsetAsync(workspace, 0, sizeof(word), s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
      (void)hipGetLastError();
      return fail(MX_STATUS_HIP_ERROR, "clearing the device status word failed");
    }
  }
  *flags_out = (int32_t)word;
  return ok();
}

int mx_last_status(void) { return g_last_status; }

const char* mx_last_error(void) { return g_last_error.c_str(); }

const char* mx_version(void) { return "mxattn 0.1.0 (gfx950 paged GQA decode)"; }

}  // extern "C"
