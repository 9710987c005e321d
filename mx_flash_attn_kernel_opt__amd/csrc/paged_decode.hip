// Paged GQA decode attention for MI355X (gfx950): split-KV and length-balanced main kernels,
// log-sum-exp combine kernel, schedule policy, argument validation and the C ABI declared in
// include/mx_paged_decode.h.
//
// Operator: reference task.md:138-148 (paged bf16 K/V cache, query head h reads KV head
// h / group), extended to seqlen_q query tokens per sequence with the optional end-aligned
// causal mask (task.md:47, 53).  The reference's kernel pair is submission_clean.cu:66-300
// (main) and :307-360 (combine); its launcher is :432-504.  The softmax is the running-max form
// of optimized_c500_flash_attn.cu:310-461 and the merge the LSE combine of :666-728.
//
// Design (gfx950, wave64):
//  * Query rows (token, head of the group) of one KV head are the N dimension of the MFMAs:
//    QK is S^T = K . Q^T with v_mfma_f32_16x16x32_bf16 (16 tokens x 16 rows), whose fp32 result
//    leaves lane (row r16, k-group g4) holding the scores of tokens 4*g4 .. 4*g4+3 -- exactly
//    the B operand of v_mfma_f32_16x16x16_bf16 for O^T = V^T . P^T, so P never moves.
//  * K and V are loaded as whole 2*D-byte token rows (nontemporal); K goes through a
//    wave-private XOR-swizzled LDS tile into the MFMA A layout, V is regrouped by v_perm_b32.
//  * Each wave streams 16-token chunks through a register ring with unconditional refills (so
//    vmcnt waits stay partial); NW waves of a workgroup interleave the chunks of one piece and
//    merge their (m, l, O) states through LDS.
//  * Online softmax in fp32, log2 domain, lazy rescale (the running max moves only when a
//    chunk max exceeds it by more than 8); the final O / l uses one max for both, so it is
//    exact.  Masked chunks (sequence tail, causal limits) use selects, never arithmetic on
//    unused page slots.
//  * Two schedules, both one launch: the split grid (Hkv * row groups, batch, splits), whose
//    splits merge their partials through an in-kernel tree of arrival counters (fan-in 8; a
//    combine kernel in a second launch only when the counters do not fit), and a
//    length-balanced launch that cuts the batch's chunk line into equal shares on the device
//    and merges cut units through a fan-in-8 tree of the same kind.
//  * Sharded decode: the same kernels can write each query row as fp32 output plus its
//    log-sum-exp (mx_paged_gqa_decode_partial) for a cross-device merge (mx_lse_merge).
//  * Paged K/V append (mx_paged_kv_append), and append-and-attend (mx_paged_gqa_decode_append):
//    for up to 16 new tokens the kernels' kAppend variants read the new keys from k_new / v_new
//    as one extra chunk per unit and write them to their cache slots in the same launch.
//  * fp8 (e4m3fn) caches with per-tensor scales (the _fp8kv entries; kFp8 variants): chunks of
//    one-byte K/V widened to bf16 on the way into the MFMA operands; head_dim-64 heads run in
//    adjacent pairs as heads of dim 128 (MainShape::pair_group); appends quantize on write.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "mx_paged_decode.h"
#include "positions.h"

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

constexpr int kChunk = 16;             // tokens per PV k-step (one 16x16x16 MFMA)
constexpr float kRescaleSlack = 8.0f;  // log2 units the stale running max may lag behind
// Workspace layout: [status word region][merge counters][partials].  The counter region has
// a fixed size and offset and holds the balanced kernel's merge-tree counters and the split
// grid's per-unit arrival counters; every kernel resets each counter it uses, so a zero-filled
// workspace keeps valid counters across calls of any shape, whatever the partials of earlier
// calls left behind.
constexpr int kStatusBytes = 256;
// XCD claim masks (xcd_slot): one 32-bit word per block of 8 workgroups, each in a 256-byte line
// of its own, so the claims of different blocks never contend for one line (packed into one
// line, 256 claims serialised and took config 2 from 156 to 165 us).
constexpr int kXcdMaskWords = 128;
constexpr int kXcdMaskStride = 64;  // words
constexpr int64_t kXcdMaskBytes = (int64_t)kXcdMaskWords * kXcdMaskStride * 4;
constexpr int kMaxSlots = 4096 + 8192;          // balanced: workgroups + batch * Hkv
constexpr int kBalancedBatch = 512;             // balanced: largest batch
constexpr int kCounterLevels = 4;               // fan-in-8 merge tree levels
constexpr int64_t kCounterBytes = (int64_t)kCounterLevels * kMaxSlots * 4;
constexpr int64_t kPartialBase = kStatusBytes + kXcdMaskBytes + kCounterBytes;

// ------------------------------------------------------------------------------------------
// Per-workgroup timeline (profiling builds only)
// ------------------------------------------------------------------------------------------

// Built with -DMX_WG_TIMELINE (a profiling build, never the shipped library), the main
// kernels record per workgroup (linear id below kTimelineSlots) the wall clock (100 MHz) at
// entry, at the start of its first streamed piece, at the end of its last one and at exit,
// plus the XCD it ran on and the number of pieces it streamed; mx_timeline_read copies the
// table out.  Thread 0 writes its workgroup's row with plain vector stores.  In the default
// build WgTimeline is an empty struct whose calls compile to nothing.
#ifdef MX_WG_TIMELINE
constexpr int kTimelineSlots = 16384;
constexpr int kTimelineFields = 6;  // entry, first stream begin, last stream end, exit, XCD, pieces
__device__ unsigned long long g_timeline[kTimelineSlots][kTimelineFields];
struct WgTimeline {
  int pieces = 0;
  __device__ static void put(int field, unsigned long long v) {
    const int slot = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    if (threadIdx.x == 0 && slot < kTimelineSlots) g_timeline[slot][field] = v;
  }
  __device__ WgTimeline() {
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    put(0, wall_clock64());
    put(4, xcc);
  }
  __device__ ~WgTimeline() {
    put(3, wall_clock64());
    put(5, (unsigned long long)pieces);
  }
  __device__ void stream_begin() {
    if (pieces++ == 0) put(1, wall_clock64());
  }
  __device__ void stream_end() { put(2, wall_clock64()); }
};
#else
struct WgTimeline {
  __device__ void stream_begin() {}
  __device__ void stream_end() {}
};
#endif

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

// floor(x / d) for 0 <= x < 2^31, given inv = 1.0 / d (d >= 1): (x + 1/2) / d lies at least
// 1/(2d) from every integer, while the double product's relative error is below 2^-51, i.e.
// (x + 1/2) / d * 2^-51 < 1/(2d) for every such x.
__device__ __forceinline__ int div_floor(int x, double inv) {
  return (int)(((double)x + 0.5) * inv);
}

// Inclusive prefix sum over the 64 lanes of a wave (row shifts, then the row broadcasts of
// lanes 15 and 31), without LDS.
__device__ __forceinline__ int wave_inclusive_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
  return x;
}

__device__ __forceinline__ float group_sum4(float x) {
  auto a = __builtin_amdgcn_permlane32_swap(as_u32(x), as_u32(x), false, false);
  x = as_float(a[0]) + as_float(a[1]);
  auto b = __builtin_amdgcn_permlane16_swap(as_u32(x), as_u32(x), false, false);
  return as_float(b[0]) + as_float(b[1]);
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

// XCD-stable workgroup order (thread 0 calls it; the caller hands the result to the workgroup).
// The dispatcher deals a launch's workgroups to the 8 XCDs in turn, starting at the XCD after
// the one its hardware queue dispatched to last, so the XCD of workgroup w varies between
// launches (eager calls back to back, graph replays, calls after other kernels).  A workgroup's
// streaming rate depends on its XCD and on the byte offsets of the rows it streams, so one
// mapping of shares to XCDs runs measurably faster than its rotations (config 2: 156 against
// 162-164 us).  xcd_slot fixes the mapping: workgroup w of the aligned block k = w / 8 takes
// logical index 8k + x, x its own XCC_ID, by claiming bit x of the block's mask word
// (atomicOr); when another workgroup of the block holds that bit (a block the dispatcher did
// not deal one to each XCD), it claims the first free bit.  The block's 8 workgroups claim 8
// distinct bits, so the mapping is a bijection whatever the dispatch; the claim that fills the
// mask clears it, when no other claim of the block is left, for the next launch.  Workgroups of
// a last, partial block keep their own index.  Relaxed agent-scope atomics: the mask only
// arbitrates indices, nothing is published through it.  The masks start at zero like the merge
// counters (a zero-filled workspace, each launch leaving them zero); were one not, a claim could
// find no free bit: xcd_slot then returns -1 and the kernel raises MX_DEVICE_WORKSPACE_STATE.
__device__ __forceinline__ int xcd_slot(int w, int n, uint32_t* masks) {
  const int k = w >> 3;
  if ((k + 1) * 8 > n) return w;
  unsigned xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  int slot = (int)(xcc & 7u);
  uint32_t bit = 1u << slot;
  uint32_t* m = masks + k * kXcdMaskStride;
  uint32_t old = __hip_atomic_fetch_or(m, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (old & bit) {
    // Taken: the first free bit (one exists: the block has 8 workgroups for 8 bits).
    for (slot = 0; slot < 8; ++slot) {
      bit = 1u << slot;
      if (old & bit) continue;
      old = __hip_atomic_fetch_or(m, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (!(old & bit)) break;
    }
    if (slot == 8) return -1;
  }
  if ((old | bit) == 0xffu) __hip_atomic_store(m, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return 8 * k + slot;
}

// Round-to-nearest-even pack of two floats into one dword of bf16 (lo in bits 0..15).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

// Shapes of the main kernels, each the best of interleaved A/B runs on MI355X:
//  * chunks in a wave's register ring (bf16 caches): 2 at head_dim 64 and 128, 1 at 256.  D=64
//    with 3 or 4 chunks ran 189-190 against 172 us, D=256 with 2 ran 178.5 against 174.9 us,
//    and D=128 with 3 or 4 (one wave per SIMD) stayed within 1 % everywhere;
//  * waves per workgroup: 2 at head_dim 64, 4 at 128 and 256.  D=64 with 4 waves ran 176.5
//    against 172 us, D=128 with 8 gained nothing, D=256 with 8 spilled to scratch (302 us);
//  * waves per SIMD the register allocation must leave room for: 2, or 1 at head_dim 256.
template <int D>
constexpr int ring_depth() {
  return D == 256 ? 1 : 2;
}

template <int D>
constexpr int waves_per_group() {
  return D == 64 ? 2 : 4;
}

template <int D, int KT>
constexpr int min_waves_per_simd() {
  return (KT == 2 || D == 256) ? 1 : 2;  // two row tiles hold two states: one wave per SIMD
}

// K/V stream loads: wave-uniform base plus per-lane byte offset, nontemporal (K/V are streamed
// once: the device's streaming-read rate rises from 6.1-6.4 to 7.15 TB/s with the hint).
__device__ __forceinline__ u32x4 ld_kv16(const uint16_t* base, uint32_t byte_off) {
  const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + byte_off);
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ u32x2 ld_kv8(const uint16_t* base, uint32_t byte_off) {
  const u32x2* p = reinterpret_cast<const u32x2*>(reinterpret_cast<const char*>(base) + byte_off);
  return __builtin_nontemporal_load(p);
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

// A load from a wave-uniform address of memory no kernel of the launch writes (the block table),
// made a scalar load: the address goes through SGPRs (readfirstlane) and is read through the
// constant address space, whatever registers the compiler gave its operands.  The page ids of
// the chunk stream must stay scalar loads: issued as vector loads behind the other ring slot's
// K/V loads and waited for before the refill, they serialise the ring (a register allocation
// that did that took config 2 from 156 to 164 us and head_dim 64 from 163 to 193 us).
typedef const int32_t __attribute__((address_space(4))) ConstInt32;
__device__ __forceinline__ int scalar_load(const int32_t* p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  // (readfirstlane returns an int: each half goes through uint32_t, so the low half is
  // zero-extended, never sign-extended into the high one.)
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return *reinterpret_cast<ConstInt32*>(((uint64_t)hi << 32) | (uint64_t)lo);
}

// Per-lane byte offsets of a chunk inside its page (constant for the whole wave).
struct LaneOffsets {
  uint32_t k;             // first K load of this lane
  uint32_t k_step;        // byte step between the lane's successive K loads
  uint32_t v;             // V[token 4*g4][(D/16)*r16]
  uint32_t token_bytes;   // bytes between consecutive tokens of a page
};

// K chunk staging through LDS: lane j loads row i*RPI + j/SPR, 16-byte segment j%SPR of the
// chunk (RPI = 512/D whole 2D-byte rows per instruction, the V access pattern), writes it to a
// wave-private 16 x 2D-byte LDS tile at an XOR-swizzled segment, and reads the MFMA A operand
// back with ds_read_b128; the swizzle keeps both the writes and the 16 rows of one read
// conflict-free.  (Loading the A operand directly, 16 rows x 64 B per instruction, streamed at
// 5.8 TB/s against 6.6 TB/s for whole nontemporal rows, and config 2 ran 177.6 us against 169.9.)
template <int D>
__device__ __forceinline__ int k_swizzle(int row) {
  return D == 64 ? ((row >> 1) & 7) : (row & 15);
}

template <int D>
__device__ __forceinline__ void k_lane_offsets(LaneOffsets& lo, int lane, int kv) {
  constexpr int SPR = D / 8;     // 16-byte segments per K row
  constexpr int RPI = 64 / SPR;  // rows per load instruction
  lo.k = (uint32_t)(lane / SPR) * lo.token_bytes + 2u * (uint32_t)(kv * D) + 16u * (lane % SPR);
  lo.k_step = RPI * lo.token_bytes;
}

// Loads all 16 token rows of a chunk.  A chunk never crosses a page (page_size % 16 == 0),
// so rows past the sequence end in the last chunk are unused slots of an allocated page;
// they are discarded at process time by selects, never by arithmetic.
template <int D>
__device__ __forceinline__ void load_chunk(Chunk<D>& c, const uint16_t* kpage,
                                           const uint16_t* vpage, const LaneOffsets& lo) {
#pragma unroll
  for (int i = 0; i < D / 32; ++i) c.k[i] = ld_kv16(kpage, lo.k + (uint32_t)i * lo.k_step);
#pragma unroll
  for (int r = 0; r < 4; ++r) load_v_row<D>(c.v[r], vpage, lo.v + r * lo.token_bytes);
}

// A operands of the QK MFMAs for one chunk (see k_lane_offsets for the two stagings).
template <int D>
__device__ __forceinline__ void k_operands(bf16x8 (&kop)[D / 32], const Chunk<D>& c,
                                           char* klds, int lane) {
  constexpr int SPR = D / 8;
  constexpr int RPI = 64 / SPR;
  const int wr = lane / SPR;
  const int ws = lane % SPR;
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    const int row = i * RPI + wr;
    *reinterpret_cast<u32x4*>(klds + row * 2 * D + 16 * (ws ^ k_swizzle<D>(row))) = c.k[i];
  }
  const int t = lane & 15;
  const int g4 = lane >> 4;
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
    kop[i] = __builtin_bit_cast(
        bf16x8, *reinterpret_cast<const u32x4*>(klds + t * 2 * D +
                                                16 * ((4 * i + g4) ^ k_swizzle<D>(t))));
}

// ------------------------------------------------------------------------------------------
// fp8 K/V cache (OCP e4m3fn, one byte per element, per-tensor scales)
// ------------------------------------------------------------------------------------------

// Register image of one 16-token chunk of one KV head of an fp8 cache (half the bytes of a
// bf16 chunk, loaded in the same row-major patterns):
//   k[i]    : 16 fp8 values, K[token i*(1024/D) + lane/(D/16)][16*(lane%(D/16)) .. +15]
//   v[r][w] : V[token 4*g4 + r][(D/16)*r16 + 4w .. +3]   (D/64 dwords per row)
template <int D>
struct Chunk8 {
  u32x4 k[D / 64];
  uint32_t v[4][D / 64];
};

// Two fp8 (e4m3fn) values of dword x (bytes 0-1, or 2-3 with kHi) as one dword of two bf16:
// exact, since every e4m3fn value is a bf16 value.  One gfx950 v_cvt_scalef32_pk_bf16_fp8 with
// scale 1, which reads the OCP e4m3fn format (checked against torch's float8_e4m3fn on all 256
// codes, NaN included).
template <bool kHi>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t x) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x, 1.0f, kHi));
}

// bf16 to fp8 (e4m3fn) for appends into an fp8 cache: four bf16 values (two dwords) as four
// bytes, each the e4m3fn value nearest to x / scale with the quotient saturated to [-448, 448]
// (NaN stays NaN).
__device__ __forceinline__ float fp8_saturate(float v) {
  return v > 448.f ? 448.f : (v < -448.f ? -448.f : v);  // comparisons pass NaN through
}

__device__ __forceinline__ uint32_t bf16x4_to_fp8x4(uint32_t lo, uint32_t hi, float scale) {
  // x / scale is the correctly rounded fp32 quotient (hipcc's default for fp32 division).
  const float a = fp8_saturate(__uint_as_float(lo << 16) / scale);
  const float b = fp8_saturate(__uint_as_float(lo & 0xffff0000u) / scale);
  const float c = fp8_saturate(__uint_as_float(hi << 16) / scale);
  const float d = fp8_saturate(__uint_as_float(hi & 0xffff0000u) / scale);
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);  // bytes 0, 1
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);       // bytes 2, 3
  return (uint32_t)w;
}

template <int D>
__device__ __forceinline__ void k_lane_offsets8(LaneOffsets& lo, int lane, int kv) {
  constexpr int SPR = D / 16;    // 16-byte segments per fp8 K row
  constexpr int RPI = 64 / SPR;  // rows per load instruction
  lo.k = (uint32_t)(lane / SPR) * lo.token_bytes + (uint32_t)(kv * D) + 16u * (lane % SPR);
  lo.k_step = RPI * lo.token_bytes;
}

template <int D>
__device__ __forceinline__ void load_chunk(Chunk8<D>& c, const uint8_t* kpage,
                                           const uint8_t* vpage, const LaneOffsets& lo) {
  const uint16_t* kp = reinterpret_cast<const uint16_t*>(kpage);
  const uint16_t* vp = reinterpret_cast<const uint16_t*>(vpage);
#pragma unroll
  for (int i = 0; i < D / 64; ++i) c.k[i] = ld_kv16(kp, lo.k + (uint32_t)i * lo.k_step);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t off = lo.v + r * lo.token_bytes;
    if constexpr (D == 64) {
      const uint32_t* p = reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(vp) + off);
      c.v[r][0] = __builtin_nontemporal_load(p);
    } else if constexpr (D == 128) {
      const u32x2 x = ld_kv8(vp, off);
      c.v[r][0] = x[0];
      c.v[r][1] = x[1];
    } else {
      const u32x4 x = ld_kv16(vp, off);
      c.v[r][0] = x[0];
      c.v[r][1] = x[1];
      c.v[r][2] = x[2];
      c.v[r][3] = x[3];
    }
  }
}

// K staging of an fp8 chunk: each lane widens its 16 values to bf16 and writes them as two
// 16-byte segments of the same swizzled LDS tile as a bf16 chunk, so the operand read back is
// unchanged.
template <int D>
__device__ __forceinline__ void k_operands(bf16x8 (&kop)[D / 32], const Chunk8<D>& c,
                                           char* klds, int lane) {
  constexpr int SPR = D / 16;
  constexpr int RPI = 64 / SPR;
  const int wr = lane / SPR;
  const int ws = lane % SPR;
#pragma unroll
  for (int i = 0; i < D / 64; ++i) {
    const int row = i * RPI + wr;
    const u32x4 x = c.k[i];
    const u32x4 lo = {fp8x2_to_bf16x2<false>(x[0]), fp8x2_to_bf16x2<true>(x[0]),
                      fp8x2_to_bf16x2<false>(x[1]), fp8x2_to_bf16x2<true>(x[1])};
    const u32x4 hi = {fp8x2_to_bf16x2<false>(x[2]), fp8x2_to_bf16x2<true>(x[2]),
                      fp8x2_to_bf16x2<false>(x[3]), fp8x2_to_bf16x2<true>(x[3])};
    char* base = klds + row * 2 * D;
    *reinterpret_cast<u32x4*>(base + 16 * ((2 * ws) ^ k_swizzle<D>(row))) = lo;
    *reinterpret_cast<u32x4*>(base + 16 * ((2 * ws + 1) ^ k_swizzle<D>(row))) = hi;
  }
  const int t = lane & 15;
  const int g4 = lane >> 4;
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
    kop[i] = __builtin_bit_cast(
        bf16x8, *reinterpret_cast<const u32x4*>(klds + t * 2 * D +
                                                16 * ((4 * i + g4) ^ k_swizzle<D>(t))));
}

// Dword w (elements 2w, 2w+1 of this lane's slice) of V row r of a chunk, as bf16.
template <int D>
__device__ __forceinline__ uint32_t v_word(const Chunk<D>& c, int r, int w) {
  return c.v[r][w];
}
template <int D>
__device__ __forceinline__ uint32_t v_word(const Chunk8<D>& c, int r, int w) {
  const uint32_t x = c.v[r][w >> 1];
  return (w & 1) ? fp8x2_to_bf16x2<true>(x) : fp8x2_to_bf16x2<false>(x);
}

// Initial running max: finite, so exp2(score - m) is 0 for a masked (-inf) score even before a
// row has seen any visible key; a row that never sees one keeps l == 0 and is written as zeros.
constexpr float kNoScore = -1.0e30f;

template <int D>
struct SoftmaxState {
  f32x4 o[D / 16];  // o[i][j] = O[row r16][(D/16)*(4*g4 + j) + i]
  float m;          // running max (log2 units), identical on the 4 lanes of a row
  float l;          // this lane's share of the running denominator
};

template <int D>
__device__ __forceinline__ void reset_state(SoftmaxState<D>& st) {
#pragma unroll
  for (int i = 0; i < D / 16; ++i) st.o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = kNoScore;
  st.l = 0.f;
}

// One chunk of the online softmax for KT tiles of 16 query rows (the K and V operands are
// shared by the tiles).  kMasked: only the first `nvalid` tokens of the chunk are real (their V
// rows are kept, the others are replaced by zeros, so NaN or Inf in unused page slots cannot
// reach the accumulators), and this lane's query row of tile t sees only the first
// row_valid[t] (<= nvalid) tokens: the causal limit of multi-token queries.  Scores of tokens
// a row does not see become -inf.
template <int D, bool kMasked, int KT, class ChunkT>
__device__ __forceinline__ void process_chunk(SoftmaxState<D> (&st)[KT], const ChunkT& c,
                                              const bf16x8 (&qop)[KT][D / 32], float scale_log2,
                                              int g4, int nvalid, const int (&row_valid)[KT],
                                              char* klds, int lane) {
  // S^T[token][row] = K . Q^T  (16 tokens x 16 rows per tile, contraction over D)
  bf16x8 kop[D / 32];
  k_operands<D>(kop, c, klds, lane);
  f32x4 s[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    s[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
      s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[i], qop[t][i], s[t], 0, 0, 0);
  }
  s16x4 pop[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    float x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[j] = s[t][j] * scale_log2;
      if constexpr (kMasked) {
        if (4 * g4 + j >= row_valid[t]) x[j] = -INFINITY;
      }
    }
    float cm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    cm = group_max4(cm);
    if (__builtin_amdgcn_ballot_w64(cm > st[t].m + kRescaleSlack)) {
      const float mn = fmaxf(st[t].m, cm);
      const float alpha = __builtin_amdgcn_exp2f(st[t].m - mn);
      st[t].m = mn;
      st[t].l *= alpha;
#pragma unroll
      for (int i = 0; i < D / 16; ++i) st[t].o[i] *= alpha;
    }
    float p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = __builtin_amdgcn_exp2f(x[j] - st[t].m);
    st[t].l += (p[0] + p[1]) + (p[2] + p[3]);
    const u32x2 pw = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])};
    pop[t] = __builtin_bit_cast(s16x4, pw);
  }

  uint32_t v[4][D / 32];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const bool keep = !kMasked || (4 * g4 + r < nvalid);
#pragma unroll
    for (int w = 0; w < D / 32; ++w) v[r][w] = keep ? v_word<D>(c, r, w) : 0u;
  }
  // O^T[d][row] += V^T . P^T  (tile i covers dims (D/16)*m + i, m = 0..15)
#pragma unroll
  for (int i = 0; i < D / 16; ++i) {
    const int w = i >> 1;
    const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
    const u32x2 vw = {__builtin_amdgcn_perm(v[1][w], v[0][w], sel),
                      __builtin_amdgcn_perm(v[3][w], v[2][w], sel)};
#pragma unroll
    for (int t = 0; t < KT; ++t)
      st[t].o[i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, vw),
                                                             pop[t], st[t].o[i], 0, 0, 0);
  }
}

// ------------------------------------------------------------------------------------------
// Shared pieces of the main kernels
// ------------------------------------------------------------------------------------------

// Query rows.  The seqlen_q query tokens of a sequence times the G query heads of one KV head
// form rows r = t * G + h (token t, head h); rows are processed in tiles of 16 (the N dimension
// of the QK MFMA), so a unit of work is one (sequence, KV head, row tile) and kvr = kv *
// row_tiles + tile indexes the second and third.
struct MainShape {
  int64_t page_stride;   // elements between physical pages: page_size * Hkv * D
  int token_stride;      // elements between tokens of a page: Hkv * D
  int num_heads;
  int num_kv_heads;
  int group;
  uint32_t group_magic;  // floor(2^32 / group) + 1 (0 when group == 1): r / group by mul-high
  // Paired heads (head_dim 128 kernels only): 0, or the query group of the stored heads when each
  // KV head of the kernel is two adjacent stored heads of dim 64.  A token's rows of the two are
  // contiguous, so K and V read as one head of dim 128.  Rows of the first stored head carry their
  // query in dims 0..63 of the operand and zeros above, rows of the second in dims 64..127, so
  // each row's scores use its own head's keys; of its PV output each row keeps its own half.
  int pair_group;
  // Mirrored pairs (MX_SCHEDULE_BALANCED_PAIRED on a bf16 cache of four KV heads, 1 KB token
  // rows): kernel head p is the stored heads p and 3 - p (byte offsets 0 and 768, or 256 and
  // 512, of the token row) instead of 2p and 2p + 1.  Its first G rows are head p's query rows,
  // the next G head 3 - p's (row_offset, stored_head).
  int pair_mirror;
  int seqlen_q;          // query tokens per sequence
  int causal;            // row t sees keys [0, L - seqlen_q + t + 1) (bottom-right aligned)
  int rows;              // seqlen_q * group
  int row_tiles;         // ceil(rows / 16)
  int tile_rows;         // min(rows, 16): rows per tile slot of the partial buffers
  int batch;
  int max_pages;         // block_table row width
  int num_pages;         // pool size, 0 = unknown
  int chunk_shift;       // log2(page_size / 16)
  int cap_tokens;        // seq_lens above this are clamped and flagged
  float scale_log2;      // scale * log2(e)
  // split grid
  int num_splits;
  int tokens_per_split;  // multiple of page_size
  int fused_combine;     // split grid: the splits of each unit merge their partials in-kernel
  int xcd_map;           // workgroups take XCD-stable indices (xcd_slot) instead of blockIdx
  int split_groups;      // split grid: ceil(num_splits / kMergeFanIn), merge counters per unit
  // balanced schedule
  int num_groups;        // workgroups of the launch
  int chunk_weight;      // balanced schedule: positions per chunk
  int unit_overhead;     // positions charged per (sequence, KV head) on top of its chunks
  int num_slots;         // partial slots: num_groups + batch * Hkv
  // Partial outputs (sharded decode): when o_out is set, each query row is written as its fp32
  // normalised output to o_out and its natural-log sum-exp to lse_out instead of bf16 to out.
  float* o_out;
  float* lse_out;
  // Append-and-attend: seq_lens are lengths before an append of this many tokens per sequence
  // (written by the append kernel just before), so sequence b has max(seq_lens[b], 0) + appended
  // keys.  0 = seq_lens are the key counts.
  int appended;
  // Append-and-attend in one launch (new_tokens = S in 1..16, else 0; the kAppend kernel
  // variants): the S new keys of each sequence are read from k_new / v_new [B, S, Hkv, D] as
  // one extra masked chunk by the split or piece holding the unit's last schedule chunk (see
  // NewTokens), and written to their cache slots at positions max(L, 0) + j through k_dst /
  // v_dst, the same memory as the kernels' K/V cache pointers.
  const uint16_t* k_new;
  const uint16_t* v_new;
  uint16_t* k_dst;
  uint16_t* v_dst;
  int new_tokens;
  // fp8 caches: V values are v_scale times the stored fp8 values (the K scale is folded into
  // scale_log2 on the host).  k_scale is kept for the fused append, which quantizes new keys.
  float v_scale;
  float k_scale;
};

// fp8 caches: a wave's output accumulators were built from unscaled V; O is linear in V, so
// scaling them once before the merge applies v_scale exactly as the per-element product would.
template <int D, int KT>
__device__ __forceinline__ void scale_o_by_v_scale(SoftmaxState<D> (&st)[KT],
                                                   const MainShape& sh) {
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int i = 0; i < D / 16; ++i) st[t].o[i] *= sh.v_scale;
}

// Keys of a sequence whose seq_lens entry is L, before clamping (see MainShape::appended).
__device__ __forceinline__ int key_count_of(int L, int appended) {
  return appended > 0 ? keys_after_append(L, appended) : L;
}
__device__ __forceinline__ int key_count(const int32_t* seq_lens, int b, int appended) {
  return key_count_of(seq_lens[b], appended);
}

// Sequence length as the kernels see it: clamped to the planned capacity (flagged).
__device__ __forceinline__ int clamped_len_of(int L, const MainShape& sh, uint32_t* status,
                                              bool report) {
  int seq = key_count_of(L, sh.appended);
  if (seq > sh.cap_tokens) {
    if (report) atomicOr(status, (uint32_t)MX_DEVICE_SEQ_TOO_LONG);
    seq = sh.cap_tokens;
  }
  return seq;
}

// Rows of q / out.  Row r = t*G + h of KV head kv of sequence b is q row
// (b*seqlen_q + t)*num_heads + kv*G + h = row_base(b, kv) + row_offset(kv, r): a wave-uniform
// base plus a per-lane offset that is r itself for a single query token.
__device__ __forceinline__ int64_t row_base(int b, int kv, const MainShape& sh) {
  return (int64_t)b * sh.seqlen_q * sh.num_heads + kv * sh.group;
}
// Query token of row r: r / group, exact for 0 <= r < 2^32 / group.
__device__ __forceinline__ int row_token(int r, const MainShape& sh) {
  return sh.group_magic ? (int)__umulhi((uint32_t)r, sh.group_magic) : r;
}
// Stored KV head of half s (rows s*G .. s*G + G - 1 of each token, waves 2s and 2s + 1) of the
// paired kernel head kv.
__device__ __forceinline__ int stored_head(int kv, int s, const MainShape& sh) {
  return sh.pair_mirror ? (s ? 3 - kv : kv) : 2 * kv + s;
}
__device__ __forceinline__ int row_offset(int kv, int r, const MainShape& sh) {
  const int t = row_token(r, sh);
  int off = r + t * (sh.num_heads - sh.group);
  if (sh.pair_mirror) {
    // Half s of kernel head kv is stored head h = stored_head(kv, s), whose query rows sit
    // (h - 2kv - s) heads' rows away from those of half s of an adjacent pair.
    const int g = sh.group >> 1;
    const int s = r - t * sh.group >= g;
    off += (stored_head(kv, s, sh) - 2 * kv - s) * g;
  }
  return off;
}

// Keys row r of a sequence of length seq sees: [0, limit).
__device__ __forceinline__ int row_key_limit(int r, int seq, const MainShape& sh) {
  if (!sh.causal) return seq;
  return seq - sh.seqlen_q + row_token(min(r, sh.rows - 1), sh) + 1;
}

// Query operand of row tile `tile` of (b, kv): lane (r16, g4) holds row tile*16 + r16,
// dims 32*i + 8*g4 .. +7, for MFMA i (zeros past the last row).
template <int D>
__device__ __forceinline__ void load_q(bf16x8 (&qop)[D / 32], const uint16_t* q, int b, int kv,
                                       int tile, const MainShape& sh, int lane) {
  const int g4 = lane >> 4;
  const int r = tile * 16 + (lane & 15);
  const bool live = r < sh.rows;
  if constexpr (D == 128) {
    if (sh.pair_group > 0) {  // q rows of 64 dims, placed in the row's half (MainShape)
      const int rr = live ? r : 0;
      const bool hi = rr - row_token(rr, sh) * sh.group >= sh.pair_group;
      const uint16_t* qp =
          q + (row_base(b, kv, sh) + row_offset(kv, rr, sh)) * (D / 2) + 8 * g4;
#pragma unroll
      for (int i = 0; i < D / 32; ++i) {
        u32x4 x = {0, 0, 0, 0};
        if (live && (i >= D / 64) == hi)
          x = *reinterpret_cast<const u32x4*>(qp + 32 * (i % (D / 64)));
        qop[i] = __builtin_bit_cast(bf16x8, x);
      }
      return;
    }
  }
  const uint16_t* qp = q + (row_base(b, kv, sh) + row_offset(kv, live ? r : 0, sh)) * D + 8 * g4;
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    u32x4 x = {0, 0, 0, 0};
    if (live) x = *reinterpret_cast<const u32x4*>(qp + 32 * i);
    qop[i] = __builtin_bit_cast(bf16x8, x);
  }
}

// A stream_chunks hook that does nothing (see NewTokens for the one that does).
struct NoExtraChunk {
  template <class ChunkT>
  __device__ __forceinline__ void load(ChunkT&) const {}
  template <int D, int KT, class ChunkT>
  __device__ __forceinline__ void process(SoftmaxState<D> (&)[KT], const ChunkT&,
                                          const bf16x8 (&)[KT][D / 32], const int (&)[KT],
                                          char*) const {}
  template <int D, int KT>
  __device__ __forceinline__ void finish(SoftmaxState<D> (&)[KT], const bf16x8 (&)[KT][D / 32],
                                         const int (&)[KT], char*) const {}
};

// K/V cache pointers: restrict-qualified, except where the same launch also writes the cache
// (the fused-append variants, through MainShape::k_dst / v_dst).
// Elements are uint16_t (bf16) or uint8_t (fp8).
template <bool kWrites, class Elem = uint16_t>
using CachePtr = std::conditional_t<kWrites, const Elem*, const Elem* __restrict__>;

// Cache element and chunk register image of a bf16 (kFp8 false) or fp8 cache.
template <bool kFp8>
using CacheElem = std::conditional_t<kFp8, uint8_t, uint16_t>;
template <int D, bool kFp8>
using ChunkOf = std::conditional_t<kFp8, Chunk8<D>, Chunk<D>>;

// Streams chunks c_lo + wv + k*NW (k >= 0, < c_hi) of one (sequence, KV head) through this
// wave's register ring, accumulating the KT row tiles into `st`.  The sequence holds `seq`
// tokens; chunks from c_mask on (at least the last one) are processed with masks: tokens past
// the sequence end, and with kCausal, for this lane's query row of tile t, the keys at or past
// row_lim[t].  Without kCausal c_mask is the last chunk and row_lim is ignored.  `hook` may add
// one more chunk from outside the cache (see NewTokens).
template <int D, int NBUF, int NW, bool kCausal, int KT, class Extra = NoExtraChunk,
          bool kFp8 = false>
__device__ __forceinline__ void stream_chunks(SoftmaxState<D> (&st)[KT],
                                              const bf16x8 (&qop)[KT][D / 32],
                                              CachePtr<!std::is_same_v<Extra, NoExtraChunk>,
                                                       CacheElem<kFp8>> kc,
                                              CachePtr<!std::is_same_v<Extra, NoExtraChunk>,
                                                       CacheElem<kFp8>> vc,
                                              const int32_t* __restrict__ bt_row, int kv,
                                              int c_lo, int c_hi, int seq, int c_mask,
                                              const int (&row_lim)[KT], int wv, char* klds,
                                              const MainShape& sh, bool& bad_page,
                                              const Extra& hook = Extra{}) {
  constexpr int VW = D / 16;
  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15;
  const int g4 = lane >> 4;
  constexpr uint32_t kElemBytes = sizeof(CacheElem<kFp8>);
  LaneOffsets lo;
  lo.token_bytes = kElemBytes * (uint32_t)sh.token_stride;
  if constexpr (kFp8) {
    k_lane_offsets8<D>(lo, lane, kv);
  } else {
    k_lane_offsets<D>(lo, lane, kv);
  }
  lo.v = kElemBytes * (uint32_t)(4 * g4 * sh.token_stride + kv * D + VW * r16);
  const int chunk_mask = (1 << sh.chunk_shift) - 1;
  const float sl2 = sh.scale_log2;

  // Element offset of chunk c (16 tokens) inside the K/V pools.  Only table entries below
  // ceil(seq / page_size) are ever read.
  // (c is below c_hi wherever a chunk is loaded; clamping the index to the stream's last chunk
  // keeps the load's address a valid table entry however the compiler schedules it.)
  const int c_top = max(c_hi - 1, 0);
  auto chunk_base = [&](int c) -> int64_t {
    int pid = scalar_load(bt_row + (min(c, c_top) >> sh.chunk_shift));
    if (pid < 0 || (sh.num_pages > 0 && pid >= sh.num_pages)) {
      bad_page = true;
      pid = 0;
    }
    return (int64_t)pid * sh.page_stride + (int64_t)((c & chunk_mask) * kChunk) * sh.token_stride;
  };
  const int n = (c_hi - c_lo > wv) ? (c_hi - c_lo - wv + NW - 1) / NW : 0;
  auto gc = [&](int k) { return c_lo + wv + k * NW; };
  // Masked processing of this wave's k-th chunk: tokens of the chunk inside the sequence, and
  // those this lane's row sees.
  using ChunkT = ChunkOf<D, kFp8>;
  auto masked = [&](ChunkT& cb, int k) {
    const int t0 = gc(k) * kChunk;
    const int nvalid = min(kChunk, seq - t0);
    int row_valid[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t) row_valid[t] = kCausal ? min(nvalid, row_lim[t] - t0) : nvalid;
    process_chunk<D, true, KT>(st, cb, qop, sl2, g4, nvalid, row_valid, klds, lane);
  };
  int all_valid[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) all_valid[t] = kChunk;

  ChunkT buf[NBUF];
  auto load = [&](ChunkT& dst, int64_t base) { load_chunk<D>(dst, kc + base, vc + base, lo); };
  // The hook's extra chunk is loaded before the ring's first chunks and processed once they
  // are in flight, so its memory latency overlaps theirs (or, where registers are short, all
  // of it runs in hook.finish after the ring).
  ChunkT xc;
  hook.load(xc);

  // Register ring of NBUF chunks.  The steady-state loops process NBUF chunks and refill their
  // buffers with the next NBUF, with no conditional loads (so the compiler's vmcnt waits stay
  // partial); the page lookups of the refills are issued before the math.  Chunks before
  // c_mask need no mask; the second loop only runs when masking starts early (causal queries
  // with many tokens).
  if (n >= NBUF) {
#pragma unroll
    for (int i = 0; i < NBUF; ++i) load(buf[i], chunk_base(gc(i)));
    hook.process(st, xc, qop, row_lim, klds);
    int k = 0;
    while (k + 2 * NBUF <= n && (!kCausal || gc(k + NBUF - 1) < c_mask)) {
      int64_t nb[NBUF];
#pragma unroll
      for (int i = 0; i < NBUF; ++i) nb[i] = chunk_base(gc(k + NBUF + i));
#pragma unroll
      for (int i = 0; i < NBUF; ++i) {
        process_chunk<D, false, KT>(st, buf[i], qop, sl2, g4, kChunk, all_valid, klds, lane);
        load(buf[i], nb[i]);
      }
      k += NBUF;
    }
    if constexpr (kCausal) {
      while (k + 2 * NBUF <= n) {
        int64_t nb[NBUF];
#pragma unroll
        for (int i = 0; i < NBUF; ++i) nb[i] = chunk_base(gc(k + NBUF + i));
#pragma unroll
        for (int i = 0; i < NBUF; ++i) {
          masked(buf[i], k + i);
          load(buf[i], nb[i]);
        }
        k += NBUF;
      }
    }
    // k + NBUF <= n < k + 2*NBUF: buffers hold chunks k .. k+NBUF-1, `extra` more remain.
    const int extra = n - k - NBUF;
#pragma unroll
    for (int i = 0; i < NBUF; ++i) {
      if (i < extra) {
        const int64_t nbase = chunk_base(gc(k + NBUF + i));
        masked(buf[i], k + i);
        load(buf[i], nbase);
      } else {
        masked(buf[i], k + i);
      }
    }
#pragma unroll
    for (int i = 0; i < NBUF; ++i)
      if (i < extra) masked(buf[i], k + NBUF + i);
  } else {
#pragma unroll
    for (int i = 0; i < NBUF; ++i)
      if (i < n) load(buf[i], chunk_base(gc(i)));
    hook.process(st, xc, qop, row_lim, klds);
#pragma unroll
    for (int i = 0; i < NBUF; ++i)
      if (i < n) masked(buf[i], i);
  }
  hook.finish(st, qop, row_lim, klds);
}

// Workgroup LDS: the per-wave K transpose tiles while streaming, then (after a barrier) the
// per-wave softmax states of the 16*KT rows for the merge.  Rows of s_o are padded by 4 floats
// so the 16 rows written by one store instruction fall in different banks.
template <int D, int NW, int KT>
struct GroupLds {
  static constexpr int kRows = 16 * KT;
  static constexpr int kRow = D + 4;
  static constexpr int kKTile = 16 * 2 * D;
  static constexpr int kMergeBytes = NW * kRows * kRow * 4 + 2 * NW * kRows * 4;
  static constexpr int kBytes = (NW * kKTile > kMergeBytes) ? NW * kKTile : kMergeBytes;
  __device__ __forceinline__ static char* ktile(char* base, int wv) { return base + wv * kKTile; }
  __device__ __forceinline__ static float* o(char* base) { return reinterpret_cast<float*>(base); }
  __device__ __forceinline__ static float* m(char* base) { return o(base) + NW * kRows * kRow; }
  __device__ __forceinline__ static float* l(char* base) { return m(base) + NW * kRows; }
};

// Writes every wave's state to LDS (after a barrier that ends the K-tile use of the same
// bytes) and synchronises, so merged_head() can combine them.
template <int D, int NW, int KT>
__device__ __forceinline__ void publish_wave_state(char* lds, const SoftmaxState<D> (&st)[KT],
                                                   int wv) {
  using L = GroupLds<D, NW, KT>;
  constexpr int VW = D / 16;
  const int lane = threadIdx.x & 63;
  const int h = lane & 15;
  const int g4 = lane >> 4;
  float l_w[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) l_w[t] = group_sum4(st[t].l);
  __syncthreads();
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    const int row = wv * L::kRows + t * 16 + h;
    float* dst = L::o(lds) + row * L::kRow + (D / 4) * g4;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < VW; i += 4)
        *reinterpret_cast<f32x4*>(dst + VW * j + i) =
            f32x4{st[t].o[i][j], st[t].o[i + 1][j], st[t].o[i + 2][j], st[t].o[i + 3][j]};
    if (g4 == 0) {
      L::m(lds)[row] = st[t].m;
      L::l(lds)[row] = l_w[t];
    }
  }
  __syncthreads();
}

// merged_head for a workgroup whose waves stream two stored KV heads (mx_paged_decode_splitkv
// with kPairW): row hh of the kernel head, whose rows of each query token are the stored first
// head's `g` rows then the second's, merges the states of the two waves that streamed its own
// head (waves 0-1 the first, 2-3 the second).
template <int D>
__device__ __forceinline__ f32x4 merged_head_pair(const char* lds, int hh, int d, float& lse,
                                                  const MainShape& sh) {
  using L = GroupLds<D, 4, 1>;
  const float* sm = L::m(const_cast<char*>(lds));
  const float* sl = L::l(const_cast<char*>(lds));
  const int w0 = hh - row_token(hh, sh) * sh.group >= sh.group / 2 ? 2 : 0;
  const int s0 = w0 * L::kRows + hh;
  const int s1 = s0 + L::kRows;
  const float mx = fmaxf(sm[s0], sm[s1]);
  const float a0 = __builtin_amdgcn_exp2f(sm[s0] - mx);
  const float a1 = __builtin_amdgcn_exp2f(sm[s1] - mx);
  const float lsum = a0 * sl[s0] + a1 * sl[s1];
  const float* so = L::o(const_cast<char*>(lds));
  const f32x4 acc = a0 * *reinterpret_cast<const f32x4*>(so + s0 * L::kRow + d) +
                    a1 * *reinterpret_cast<const f32x4*>(so + s1 * L::kRow + d);
  const bool seen = lsum > 0.f;
  lse = seen ? mx + log2f(lsum) : -INFINITY;
  return acc * (seen ? 1.0f / lsum : 0.f);
}

// Merged (normalised) dims d..d+3 of row slot hh (< 16*KT) and its log2-sum-exp; a row that
// saw no key (l == 0: causal rows before their first key) is zeros with log2-sum-exp -inf.
template <int D, int NW, int KT>
__device__ __forceinline__ f32x4 merged_head(const char* lds, int hh, int d, float& lse) {
  using L = GroupLds<D, NW, KT>;
  const float* sm = L::m(const_cast<char*>(lds));
  const float* sl = L::l(const_cast<char*>(lds));
  float mx = sm[hh];
#pragma unroll
  for (int w = 1; w < NW; ++w) mx = fmaxf(mx, sm[w * L::kRows + hh]);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float lsum = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float a = __builtin_amdgcn_exp2f(sm[w * L::kRows + hh] - mx);
    lsum += a * sl[w * L::kRows + hh];
    acc += a * *reinterpret_cast<const f32x4*>(L::o(const_cast<char*>(lds)) +
                                              (w * L::kRows + hh) * L::kRow + d);
  }
  const bool seen = lsum > 0.f;
  lse = seen ? mx + log2f(lsum) : -INFINITY;
  return acc * (seen ? 1.0f / lsum : 0.f);
}

__device__ __forceinline__ void store_bf16x4(uint16_t* p, f32x4 v) {
  const u32x2 w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  *reinterpret_cast<u32x2*>(p) = w;
}

constexpr float kLn2 = 0.69314718055994531f;
constexpr float kLog2e = 1.4426950408889634f;

// Final output of dims d..d+3 of query row `row` with log2-sum-exp lse2: bf16 into out, or, for
// partial outputs, fp32 into sh.o_out and (once per row) the natural-log sum-exp into sh.lse_out.
// With paired heads (MainShape::pair_group) rows are 64 dims and only the row's own half of
// the kernel's 128 is written.
template <int D>
__device__ __forceinline__ void store_row4(uint16_t* out, const MainShape& sh, int64_t row, int d,
                                           f32x4 o, float lse2) {
  int64_t at = row * D + d;
  bool first = d == 0;
  if constexpr (D == 128) {
    if (sh.pair_group > 0) {
      const int hi = ((uint32_t)row % (uint32_t)sh.num_heads / (uint32_t)sh.pair_group) & 1;
      if ((d >= D / 2) != (hi != 0)) return;
      at = row * (D / 2) + d - hi * (D / 2);
      first = d == hi * (D / 2);
    }
  }
  if (sh.o_out == nullptr) {
    store_bf16x4(out + at, o);
    return;
  }
  *reinterpret_cast<f32x4*>(sh.o_out + at) = o;
  if (first) sh.lse_out[row] = lse2 * kLn2;
}

// Row group g of a KV head: KT tiles of 16 rows, rows g*16*KT + t*16 + r16.  Loads the query
// operands, clears the states and computes each lane's causal key limit per tile.
template <int D, int KT>
__device__ __forceinline__ void setup_row_group(bf16x8 (&qop)[KT][D / 32],
                                                SoftmaxState<D> (&st)[KT], int (&row_lim)[KT],
                                                const uint16_t* q, int b, int kv, int g, int seq,
                                                const MainShape& sh, int lane) {
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    load_q<D>(qop[t], q, b, kv, g * KT + t, sh, lane);
    reset_state<D>(st[t]);
    row_lim[t] = row_key_limit((g * KT + t) * 16 + (lane & 15), seq, sh);
  }
}

// Extent of sequence b as the kernels see it.  keys: keys attended; cache: keys read from the
// paged cache; sched: tokens the schedules (splits, balanced positions) cover; at: cache position
// of the first new key (fused append only).  Without a fused append keys, cache and sched are
// the clamped key count.  With one (MainShape::new_tokens = S) the cache holds
// min(max(L, 0), cap) old keys and the S new ones come from k_new (L + S above the capacity is
// flagged); an empty cache still takes one schedule slot so the unit exists.
struct SeqExtent {
  int keys;
  int cache;
  int sched;
  int at;
};
template <bool kAppend>
__device__ __forceinline__ SeqExtent seq_extent_of(int L, const MainShape& sh, uint32_t* status,
                                                   bool report) {
  if constexpr (!kAppend) {
    const int s = clamped_len_of(L, sh, status, report);
    return SeqExtent{s, s, s, 0};
  }
  const int at = max(L, 0);
  if (at > sh.cap_tokens - sh.new_tokens && report)
    atomicOr(status, (uint32_t)MX_DEVICE_SEQ_TOO_LONG);
  const int c = min(at, sh.cap_tokens);
  return SeqExtent{c + sh.new_tokens, c, max(c, 1), at};
}
template <bool kAppend>
__device__ __forceinline__ SeqExtent seq_extent(const int32_t* seq_lens, int b,
                                                const MainShape& sh, uint32_t* status,
                                                bool report) {
  return seq_extent_of<kAppend>(seq_lens[b], sh, status, report);
}

// The fused append's extra chunk of unit (b, kv), a stream_chunks hook: in the wave that owns
// it (`active`), load() reads the S = sh.new_tokens new rows of KV head kv from k_new / v_new
// (rows past S re-read row S-1, so nothing past them is touched) and process() runs them as a
// masked chunk at attended positions `cache` + j: query row r of tile t sees new key j when
// cache + j < row_lim[t].  With `write` (one unit per KV head), process() first stores the
// rows to their cache slots at positions at + j, like the append kernel: positions past the
// table row and page ids outside the pool are skipped and flagged.  Those stores are issued at
// the start of the wave's streaming, so they complete long before its next barrier, and no
// slot written is read unmasked by the launch (cache chunks cover positions below `cache`).
// With head_dim 256 the chunk runs after the ring instead and the cache is written by
// copy_new_tokens at the end of the launch.
template <bool kFp8 = false>
struct NewTokens {
  const MainShape& sh;
  int b, kv, cache;
  bool active;                  // wave-uniform
  bool write;                   // wave-uniform
  int at;                       // cache position of new row 0: max(seq_lens[b], 0)
  const int32_t* bt_row;
  uint32_t* status;

  // With head_dim 256 the ring leaves no registers for a chunk in flight beside it, and an
  // fp8 ring's slots cannot hold bf16 rows: the new keys are then loaded and processed after
  // the ring (finish).
  template <int D>
  static constexpr bool kOverlap = D <= 128 && !kFp8;
  // bf16 caches at head_dim 256: the cache rows are written after the attention, by
  // copy_new_tokens.  (fp8 caches: finish writes the quantized rows.)
  template <int D>
  static constexpr bool kCopyAfter = D > 128 && !kFp8;

  template <int D>
  __device__ __forceinline__ void load(Chunk<D>& c) const {
    if constexpr (kOverlap<D>)
      if (active) load_rows(c);
  }
  template <int D>
  __device__ __forceinline__ void load(Chunk8<D>&) const {}
  template <int D, int KT>
  __device__ __forceinline__ void process(SoftmaxState<D> (&)[KT], const Chunk8<D>&,
                                          const bf16x8 (&)[KT][D / 32], const int (&)[KT],
                                          char*) const {}
  template <int D, int KT>
  __device__ __forceinline__ void process(SoftmaxState<D> (&st)[KT], const Chunk<D>& c,
                                          const bf16x8 (&qop)[KT][D / 32],
                                          const int (&row_lim)[KT], char* klds) const {
    if constexpr (kOverlap<D>) {
      if (active) {
        if (write) store_rows(c);
        run(st, c, qop, row_lim, klds);
      }
    }
  }
  template <int D, int KT>
  __device__ __forceinline__ void finish(SoftmaxState<D> (&st)[KT],
                                         const bf16x8 (&qop)[KT][D / 32],
                                         const int (&row_lim)[KT], char* klds) const {
    if constexpr (!kOverlap<D>) {
      if (active) {
        Chunk<D> c;
        load_rows(c);
        if constexpr (kFp8) quantize_and_store(c);
        run(st, c, qop, row_lim, klds);
      }
    }
  }

  // fp8 caches: every bf16 value x of the loaded rows becomes the e4m3fn value q nearest to
  // x / scale (saturated, as the append kernel stores it); q is written to the row's cache slot
  // (when this wave writes) and replaces x in the chunk, widened back to bf16, so the new keys
  // are attended as the cache will hold them (the scales multiply back in the softmax scale
  // and on the output).
  template <int D>
  __device__ __forceinline__ void quantize_and_store(Chunk<D>& c) const {
    constexpr int VW = D / 16;
    uint32_t k8[D / 32][2];
    uint32_t v8[4][VW / 4];
    const float ks = sh.k_scale, vs = sh.v_scale;
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
      u32x4& w = c.k[i];
      k8[i][0] = bf16x4_to_fp8x4(w[0], w[1], ks);
      k8[i][1] = bf16x4_to_fp8x4(w[2], w[3], ks);
      w = u32x4{fp8x2_to_bf16x2<false>(k8[i][0]), fp8x2_to_bf16x2<true>(k8[i][0]),
                fp8x2_to_bf16x2<false>(k8[i][1]), fp8x2_to_bf16x2<true>(k8[i][1])};
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int w = 0; w < VW / 4; ++w) {
        v8[r][w] = bf16x4_to_fp8x4(c.v[r][2 * w], c.v[r][2 * w + 1], vs);
        c.v[r][2 * w] = fp8x2_to_bf16x2<false>(v8[r][w]);
        c.v[r][2 * w + 1] = fp8x2_to_bf16x2<true>(v8[r][w]);
      }
    if (write) store_rows8<D>(k8, v8);
  }

  // store_rows for fp8 bytes: K segment i of a lane is 8 bytes at byte 8 * (lane % (D/8)) of
  // its row, V is VW bytes at byte VW * (lane & 15).
  template <int D>
  __device__ __forceinline__ void store_rows8(const uint32_t (&k8)[D / 32][2],
                                              const uint32_t (&v8)[4][D / 64]) const {
    int lane = threadIdx.x & 63;
    asm volatile("" : "+v"(lane));
    constexpr int SPR = D / 8;
    constexpr int RPI = 64 / SPR;
    constexpr int VW = D / 16;
    uint8_t* kd = reinterpret_cast<uint8_t*>(sh.k_dst);
    uint8_t* vd = reinterpret_cast<uint8_t*>(sh.v_dst);
    const RowSlots rs = row_slots<D>();
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
      const int64_t o = rs.slot(i * RPI + lane / SPR);
      if (o >= 0) *reinterpret_cast<u32x2*>(kd + o + 8 * (lane % SPR)) = u32x2{k8[i][0], k8[i][1]};
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t o = rs.slot(4 * (lane >> 4) + r);
      if (o >= 0) {
        uint8_t* dst = vd + o + VW * (lane & 15);
        if constexpr (D == 64) {
          *reinterpret_cast<uint32_t*>(dst) = v8[r][0];
        } else if constexpr (D == 128) {
          *reinterpret_cast<u32x2*>(dst) = u32x2{v8[r][0], v8[r][1]};
        } else {
          *reinterpret_cast<u32x4*>(dst) = u32x4{v8[r][0], v8[r][1], v8[r][2], v8[r][3]};
        }
      }
    }
  }

  template <int D>
  __device__ __forceinline__ void load_rows(Chunk<D>& c) const {
    // An opaque copy of the lane index: keeps the per-lane offsets of this rarely taken block
    // from being hoisted out of the callers' loops, where they would stay live (and spill)
    // across the streaming of every chunk.
    int lane = threadIdx.x & 63;
    asm volatile("" : "+v"(lane));
    constexpr int SPR = D / 8;     // 16-byte segments per K row
    constexpr int RPI = 64 / SPR;  // K rows per load instruction
    constexpr int VW = D / 16;     // V elements per lane and row
    const int S = sh.new_tokens;
    // Row 0 of stored head kv: k_new / v_new rows have the cache's token stride (the stored
    // heads', also where the kernel's heads are pairs of them).
    const int64_t head0 = (int64_t)b * S * sh.token_stride + (int64_t)kv * D;
    const uint16_t* kb = sh.k_new + head0;
    const uint16_t* vb = sh.v_new + head0;
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
      const int rr = min(i * RPI + lane / SPR, S - 1);
      c.k[i] = *reinterpret_cast<const u32x4*>(kb + (int64_t)rr * sh.token_stride +
                                               8 * (lane % SPR));
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int rr = min(4 * (lane >> 4) + r, S - 1);
      load_v_row<D>(c.v[r], vb + (int64_t)rr * sh.token_stride + VW * (lane & 15), 0u);
    }
  }

  // The loaded rows (K in the LDS-staged layout: lane j holds 16-byte segment j % (D/8) of row
  // i*(512/D) + j/(D/8); V: lane (r16, g4) holds elements (D/16)*r16 .. of row 4*g4 + r) go
  // to their page slots.  The S <= 16 <= page_size positions span at most two pages, whose ids
  // are two wave-uniform loads.
  // Cache slots of the new rows: the S <= 16 <= page_size positions span at most two pages.
  struct RowSlots {
    int n_ok, at, psize, page0, pid0, pid1, kvD;
    bool ok0, ok1;
    const MainShape* shp;
    // Element offset of new row j's KV head, or -1 when it is not written.
    __device__ __forceinline__ int64_t slot(int j) const {
      if (j >= n_ok) return -1;  // (at + j is formed only inside the table row)
      const int pos = at + j;
      const bool first = pos / psize == page0;
      if (!(first ? ok0 : ok1)) return -1;
      return (int64_t)(first ? pid0 : pid1) * shp->page_stride +
             (int64_t)(pos % psize) * shp->token_stride + kvD;
    }
  };
  // The two page ids (wave-uniform loads); flags rows past the table row or in pages outside
  // the pool.
  template <int D>
  __device__ __forceinline__ RowSlots row_slots() const {
    const int lane = threadIdx.x & 63;
    RowSlots rs;
    rs.shp = &sh;
    rs.at = at;
    rs.kvD = kv * D;
    rs.psize = kChunk << sh.chunk_shift;
    const int S = sh.new_tokens;
    const int table_tokens = sh.max_pages * rs.psize;
    rs.n_ok = max(0, min(S, table_tokens - at));  // rows whose position is in the row
    if (rs.n_ok < S && lane == 0) atomicOr(status, (uint32_t)MX_DEVICE_SEQ_TOO_LONG);
    rs.page0 = at / rs.psize;
    rs.pid0 = rs.n_ok > 0 ? bt_row[rs.page0] : -1;
    rs.pid1 = rs.n_ok > 0 ? bt_row[(at + rs.n_ok - 1) / rs.psize] : -1;
    auto valid = [&](int pid) { return pid >= 0 && (sh.num_pages <= 0 || pid < sh.num_pages); };
    rs.ok0 = valid(rs.pid0);
    rs.ok1 = valid(rs.pid1);
    if (rs.n_ok > 0 && !(rs.ok0 && rs.ok1) && lane == 0)
      atomicOr(status, (uint32_t)MX_DEVICE_BAD_PAGE_ID);
    return rs;
  }

  template <int D>
  __device__ __forceinline__ void store_rows(const Chunk<D>& c) const {
    int lane = threadIdx.x & 63;
    asm volatile("" : "+v"(lane));
    constexpr int SPR = D / 8;
    constexpr int RPI = 64 / SPR;
    constexpr int VW = D / 16;
    const RowSlots rs = row_slots<D>();
    if (rs.n_ok == 0) return;
    auto slot = [&](int j) -> int64_t { return rs.slot(j); };
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
      const int64_t o = slot(i * RPI + lane / SPR);
      if (o >= 0) *reinterpret_cast<u32x4*>(sh.k_dst + o + 8 * (lane % SPR)) = c.k[i];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t o = slot(4 * (lane >> 4) + r);
      if (o >= 0) {
        uint16_t* dst = sh.v_dst + o + VW * (lane & 15);
        if constexpr (D == 64) {
          *reinterpret_cast<u32x2*>(dst) = u32x2{c.v[r][0], c.v[r][1]};
        } else {
#pragma unroll
          for (int w = 0; w < D / 32; w += 4)
            *reinterpret_cast<u32x4*>(dst + 2 * w) =
                u32x4{c.v[r][w], c.v[r][w + 1], c.v[r][w + 2], c.v[r][w + 3]};
        }
      }
    }
  }

  template <int D, int KT>
  __device__ __forceinline__ void run(SoftmaxState<D> (&st)[KT], const Chunk<D>& c,
                                      const bf16x8 (&qop)[KT][D / 32], const int (&row_lim)[KT],
                                      char* klds) const {
    const int lane = threadIdx.x & 63;
    const int S = sh.new_tokens;
    int row_valid[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t) row_valid[t] = max(0, min(S, row_lim[t] - cache));
    process_chunk<D, true, KT>(st, c, qop, sh.scale_log2, lane >> 4, S, row_valid, klds, lane);
  }
};

// The fused append's cache write for KV head kv of sequence b: new row j of k_new / v_new goes
// to cache position max(seq_lens[b], 0) + j, like the append kernel (positions past the table
// row and page ids outside the pool are skipped and flagged).  One workgroup per (sequence, KV
// head) does it, as its last work: the stores' completion then delays no barrier or merge of
// the launch, and none of these slots is read unmasked by it (cache chunks cover positions
// below SeqExtent::cache only).
template <int D>
__device__ __forceinline__ void copy_new_tokens(const int32_t* __restrict__ seq_lens,
                                                const int32_t* __restrict__ block_table, int b,
                                                int kv, const MainShape& sh, uint32_t* status,
                                                int tid, int nthreads) {
  constexpr int SEG = D / 8;  // 16-byte segments per row of one KV head
  const int S = sh.new_tokens;
  const int at = max(seq_lens[b], 0);
  const int psize = kChunk << sh.chunk_shift;
  const int table_tokens = sh.max_pages * psize;
  const int32_t* bt_row = block_table + (int64_t)b * sh.max_pages;
  bool overflow = false, bad = false;
  for (int e = tid; e < 2 * S * SEG; e += nthreads) {
    const int is_v = e >= S * SEG;
    const int j = (e - is_v * S * SEG) / SEG;
    const int seg = e % SEG;
    const int pos = append_position(at, j, table_tokens);
    if (pos < 0) {  // past the table row
      overflow = true;
      continue;
    }
    const int pid = bt_row[pos / psize];
    if (pid < 0 || (sh.num_pages > 0 && pid >= sh.num_pages)) {
      bad = true;
      continue;
    }
    const int64_t src = ((int64_t)b * S + j) * sh.token_stride + (int64_t)kv * D + 8 * seg;
    const int64_t dst = (int64_t)pid * sh.page_stride + (int64_t)(pos % psize) * sh.token_stride +
                        kv * D + 8 * seg;
    const u32x4 x = *reinterpret_cast<const u32x4*>((is_v ? sh.v_new : sh.k_new) + src);
    *reinterpret_cast<u32x4*>((is_v ? sh.v_dst : sh.k_dst) + dst) = x;
  }
  if (__builtin_amdgcn_ballot_w64(overflow) != 0 && (tid & 63) == 0)
    atomicOr(status, (uint32_t)MX_DEVICE_SEQ_TOO_LONG);
  if (__builtin_amdgcn_ballot_w64(bad) != 0 && (tid & 63) == 0)
    atomicOr(status, (uint32_t)MX_DEVICE_BAD_PAGE_ID);
}

// Partials merged per step of a cross-workgroup merge tree (the balanced schedule's pieces, the
// split grid's splits); kCounterLevels levels cover 8^4 = 4096 items.  For the split grid 8
// matched the two-launch combine on long-context decode in interleaved A/B (B=1, 32K: 30.0
// against 30.0 us), where groups of 16 ran 30.7 and of 4 ran 31.3.
constexpr int kMergeFanIn = 8;
constexpr int kMaxMergeItems = 8 * 8 * 8 * 8;

// Cross-workgroup handoff of partials (the split grid's in-kernel merge and the balanced
// kernel's merge tree).  Partials are stored and loaded with agent-coherent accesses, which keep
// each location coherent across the device's XCDs with no L2 write-back: the sc1 cache policy
// that relaxed agent-scope atomic accesses carry on gfx950 (global_store / global_load ... sc1).
// The 16-byte row pieces go through buffer instructions with that policy (buffer_store_dwordx4
// / buffer_load_dwordx4 ... sc1) over a resource based at the partial region, whose byte
// offsets are 32-bit: the host keeps every region read this way below 2^31 bytes
// (kMaxHandoffBytes).  Two 8-byte atomic accesses per piece instead wrote each 64-byte line
// through twice (WRITE_SIZE twice the partial bytes); interleaved A/B against them, outputs
// bitwise equal: long B=1 128K 85.0 against 85.8 us, contest cases 10 and 14 (B=1, 64 splits)
// 11.35 against 11.75 and 27.0 against 27.6 us, the balanced shapes within +-0.3 us.  The
// order between the stores of the pieces and the loads of the workgroup that merges them comes
// from the arrival counter (arrive_last).  A plain-store variant with __threadfence() in every
// thread was measured first: it writes back the L2 per wave, and config 2 with 1 024 workgroups
// ran 505 us instead of 174.
// The merging workgroup's loads (rows and log-sum-exps) also carry the nontemporal hint: a
// partial is read once.  Interleaved A/B against sc1 loads without it, outputs bitwise equal:
// ragged 72.2 against 74.1 us (graph replays 72.4 against 74.4, seed 3 68.1 against 70.2),
// contest cases 11 and 8 42.5 against 43.1 and 19.3 against 19.6 us, long contexts 0.1-0.3 us
// faster.  The same hint on the partial stores was slower (long B=1 32K 28.6 against 27.4 us,
// ragged 75.0 against 74.3).
constexpr int kCachePolicySc1 = 16;  // buffer intrinsics' aux bit for sc1
constexpr int kCachePolicyNt = 2;    // buffer intrinsics' aux bit for nt
__device__ __forceinline__ __amdgpu_buffer_rsrc_t partial_rsrc(const float* base) {
  // Raw buffer over [base, base + 2^31 - 1): stride 0, dword 3 = 0x00020000 (32-bit data, no
  // swizzle), as for every gfx9 raw buffer.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, 0x7fffffff,
                                           0x00020000);
}
__device__ __forceinline__ void store_partial4(const float* base, float* p, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), partial_rsrc(base),
                                         (int)((const char*)p - (const char*)base), 0,
                                         kCachePolicySc1);
}
__device__ __forceinline__ void store_partial1(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x4 load_partial4(const float* base, const float* p) {
  return __builtin_bit_cast(
      f32x4, __builtin_amdgcn_raw_buffer_load_b128(partial_rsrc(base),
                                                   (int)((const char*)p - (const char*)base), 0,
                                                   kCachePolicySc1 | kCachePolicyNt));
}
// A log-sum-exp stored by store_partial1, read through a resource based at the log-sum-exp region
// (also below 2^31 bytes) with the same policy as load_partial4.
__device__ __forceinline__ float load_partial1(const float* base, const float* p) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_raw_buffer_load_b32(partial_rsrc(base),
                                                  (int)((const char*)p - (const char*)base), 0,
                                                  kCachePolicySc1 | kCachePolicyNt));
}

// Arrival of this workgroup at `counter`, which `expected` workgroups reach once each; returns,
// uniformly over the workgroup, whether it arrived last (and then resets the counter for the
// next call).  Called by every thread after its partial stores (store_partial4/1).  The steps:
//  1. each wave waits until its own stores have completed (s_waitcnt vmcnt(0)): with sc1 they
//     are then written through to the device-coherent level, past the XCD's own L2;
//  2. the barrier: every wave of the workgroup is past step 1 before thread 0 goes on, so all
//     of the workgroup's stores are complete before its increment is issued;
//  3. thread 0 increments with a relaxed agent-scope read-modify-write, performed at the
//     device-coherent level: the value returned counts the increments before it, each issued
//     after its workgroup's stores were complete;
//  4. the barrier hands thread 0's result to every thread, so the last arrival issues its
//     loads of the others' partials (load_partial4/1, sc1: served from the device-coherent
//     level) only after the read-modify-write has returned.
// The partials never sit in a non-coherent cache line (stores write through, loads do not hit
// stale lines), which is why no release or acquire fence is needed; an acq_rel increment adds
// an L2 write-back and invalidate per arrival and measured 98.6 against 86.2 us on ragged
// decode.
__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t expected, int* s_flag) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = prev == expected - 1;
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = last ? 1 : 0;
  }
  __syncthreads();
  return *s_flag != 0;
}

// One merge step of a cross-workgroup merge tree: the gsize (<= W) items of a group, at level-0
// slots gslot + t * stride, merged as
//   O = sum_t 2^(lse_t - M) O_t / sum_t 2^(lse_t - M),  lse = M + log2 sum_t 2^(lse_t - M),
// M = max_t lse_t (optimized_c500_flash_attn.cu:666-728, log2 domain).  A row no item saw a key
// for (every lse -inf: causal rows before their first key) stays zeros with lse -inf.  The
// merged rows go to the output (`final`) or to the group's first slot (lse to s_lse, which the
// caller stores after a barrier).
//
// The arithmetic of one element's merge over items t < gsize of W (items past gsize weigh 0):
// returns the merged dims and sets lse.
template <int W>
__device__ __forceinline__ f32x4 lse_merge(float (&ls)[W], const f32x4 (&vs)[W], int gsize,
                                           float& lse) {
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < W; ++t) {
    if (t >= gsize) ls[t] = -INFINITY;
    mx = fmaxf(mx, ls[t]);
  }
  const bool seen = mx > -INFINITY;
  const float mref = seen ? mx : 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float wsum = 0.f;
#pragma unroll
  for (int t = 0; t < W; ++t) {
    const float w = __builtin_amdgcn_exp2f(ls[t] - mref);  // 0 for t >= gsize
    wsum += w;
    acc += w * vs[t];
  }
  acc *= seen ? 1.0f / wsum : 0.f;
  lse = seen ? mx + log2f(wsum) : -INFINITY;
  return acc;
}

// merge_elems handles E four-dim elements e0, e0 + 64*NW, ... (< total) of the group's rows: it
// issues the loads of all items for all of them at once (unconditional: slots past the group
// re-read its first item and are masked by their lse, elements past the rows re-read e0's), so
// the step is one memory round trip.  A row's D/4 elements sit on D/4 consecutive lanes of one
// wave; when the group has at most that many items, lane j of the row loads item j's
// log-sum-exp and the row's lanes exchange them (ds_bpermute) instead of each loading all W:
// W loads per element fewer in flight, which keeps W = 32 items (64 loads per thread otherwise,
// past the 63 the memory counter tracks) to one round trip.
template <int D, int NW, int W, int E, class Tree>
__device__ __forceinline__ void merge_elems(const Tree& tree, int e0, int total, int gslot,
                                            int stride, int gsize, bool final, float* s_lse) {
  constexpr int kRowLanes = D / 4;
  constexpr bool kLaneLse = W <= kRowLanes;
  static_assert((64 * NW) % kRowLanes == 0 && kRowLanes <= 64, "a row's lanes in one wave");
  const int lane = e0 & 63;
  const int row_lane0 = lane & ~(kRowLanes - 1);  // first lane of this lane's row group
  float ls[E][W];
  float lsl[E];  // kLaneLse: item (lane - row_lane0)'s log-sum-exp of element q's row
  f32x4 vs[E][W];
  int hh[E], d[E];
  // Item t of the group sits t * stride slots after the first: the row's addresses are formed
  // once and stepped by a uniform stride (forming each item's address from its slot instead took
  // a dozen dependent integer instructions per load).
  const int lse_step = tree.lse_step() * stride;
  const int o_step = tree.o_step() * stride;
#pragma unroll
  for (int q = 0; q < E; ++q) {
    const int e = e0 + q * 64 * NW;
    const int ee = e < total ? e : e0;
    hh[q] = ee / (D / 4);
    d[q] = 4 * (ee - hh[q] * (D / 4));
    const float* lp = tree.lse(hh[q], gslot);
    const float* op = tree.o(hh[q], gslot) + d[q];
    if constexpr (kLaneLse) {
      const int j = lane - row_lane0;  // = d[q] / 4
      lsl[q] = load_partial1(tree.part_lse, lp + (j < gsize ? j : 0) * lse_step);
    }
#pragma unroll
    for (int t = 0; t < W; ++t) {
      const int tt = t < gsize ? t : 0;
      if constexpr (!kLaneLse) ls[q][t] = load_partial1(tree.part_lse, lp + tt * lse_step);
      vs[q][t] = load_partial4(tree.part_o, op + tt * o_step);
    }
  }
  if constexpr (kLaneLse) {
    // (Every lane of a row group runs this: total is a multiple of the row's lanes, and lanes
    // past it hold e0's row, the same for the whole group.)
#pragma unroll
    for (int q = 0; q < E; ++q)
#pragma unroll
      for (int t = 0; t < W; ++t) ls[q][t] = __shfl(lsl[q], row_lane0 + t);
  }
#pragma unroll
  for (int q = 0; q < E; ++q) {
    if (e0 + q * 64 * NW >= total) break;
    float lse;
    const f32x4 acc = lse_merge<W>(ls[q], vs[q], gsize, lse);
    if (final) {
      tree.store(hh[q], d[q], acc, lse);
    } else {
      store_partial4(tree.part_o, tree.o(hh[q], gslot) + d[q], acc);
      if (d[q] == 0) s_lse[hh[q]] = lse;
    }
  }
}

// The whole step: nrows * D/4 elements over the workgroup's 64*NW threads, two per thread and
// round when there are more elements than threads (16 rows at D=128 take one round instead of
// two; paired split grid at B=1, 32K tokens: 31.1 against 32.4 us per call with two rounds).
template <int D, int NW, int W, class Tree>
__device__ __forceinline__ void merge_group(const Tree& tree, int gslot, int stride, int gsize,
                                            int nrows, bool final, float* s_lse) {
  // An opaque copy of the thread index: keeps the per-thread addressing of this step from being
  // hoisted out of the callers' loops, where it would stay live across the chunk streaming.
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int total = nrows * (D / 4);
  if (total > 64 * NW && W <= 16) {
    for (int e0 = tid; e0 < total; e0 += 2 * 64 * NW)
      merge_elems<D, NW, W, 2>(tree, e0, total, gslot, stride, gsize, final, s_lse);
  } else {
    // (Groups of 32: one element per thread and round, so the loads in flight, 5 registers per
    // item, stay within a wave's registers.)
    for (int e0 = tid; e0 < total; e0 += 64 * NW)
      merge_elems<D, NW, W, 1>(tree, e0, total, gslot, stride, gsize, final, s_lse);
  }
}

// The merge tree of one cut unit: the balanced schedule's pieces, or the split grid's splits.
// Level-0 item i is the partial that workgroup has stored for it (normalised O / l per row and
// its log2-sum-exp); level-l item j covers level-0 items [j*F^l, (j+1)*F^l) and is stored in the
// slot of its first one.  The last arrival of each group of up to F items merges them
// (merge_group, with as many loads per thread as the group has items, rounded up to a power of
// two) into the group's slot, or into the output when it is the last level's only group.
// Returns when this workgroup is not the last arrival of its group, or after the output is
// written.
//
// `tree` provides o(hh, slot) / lse(hh, slot) (the fp32 partial row hh of a level-0 slot and its
// log2-sum-exp), o_step() / lse_step() (the floats between those of consecutive slots of a row),
// counter(level, slot) (the arrival counter of the level's group whose first item
// is at `slot`) and store(hh, d, o, lse) (the final store of dims d..d+3 of row hh).  s_lse holds
// nrows floats.
template <int D, int NW, int F, class Tree>
__device__ __forceinline__ void merge_tree(const Tree& tree, int item, int nitems, int nrows,
                                           float* s_lse, int* s_flag) {
  static_assert(F == 8 || F == 16 || F == 32, "fan-in of the merge trees");
  const int tid = threadIdx.x;
  int stride = 1;  // level-0 items per item of this level
  for (int level = 0;; ++level) {
    const int grp = item / F;
    const int gsize = min(F, nitems - grp * F);
    const int gslot = grp * F * stride;  // level-0 slot of the group's first item
    if (!arrive_last(tree.counter(level, gslot), (uint32_t)gsize, s_flag)) return;
    const int nnext = (nitems + F - 1) / F;
    const bool final = nnext == 1;
    if (gsize <= 2) {
      merge_group<D, NW, 2>(tree, gslot, stride, gsize, nrows, final, s_lse);
    } else if (gsize <= 4) {
      merge_group<D, NW, 4>(tree, gslot, stride, gsize, nrows, final, s_lse);
    } else if (F == 8 || gsize <= 8) {
      merge_group<D, NW, 8>(tree, gslot, stride, gsize, nrows, final, s_lse);
    } else if (F == 16 || gsize <= 16) {
      merge_group<D, NW, 16>(tree, gslot, stride, gsize, nrows, final, s_lse);
    } else {
      merge_group<D, NW, F>(tree, gslot, stride, gsize, nrows, final, s_lse);
    }
    if (final) return;
    // Every thread has read the group's log-sum-exps before the merged one overwrites the first.
    __syncthreads();
    if (tid < nrows) store_partial1(tree.lse(tid, gslot), s_lse[tid]);
    item = grp;
    nitems = nnext;
    stride *= F;
  }
}

// ------------------------------------------------------------------------------------------
// Split-grid kernel
// ------------------------------------------------------------------------------------------

// The split grid's merge tree over the splits of one unit (merge_tree).  Partials are row-major
// over the query rows with the splits innermost: part_o[(row * num_splits + split) * D + d],
// part_lse[row * num_splits + split] (the layout mx_paged_decode_combine reads).  Each level of
// the counter region holds split_groups = ceil(num_splits / kMergeFanIn) counters per unit.
template <int D>
struct SplitTree {
  const MainShape& sh;
  float* part_o;
  float* part_lse;
  uint32_t* counters;
  uint16_t* out;
  int64_t rbase;  // row_base of the unit
  int kv;         // kernel KV head of the unit
  int r0;         // first row of the unit's row group
  int unit;       // (sequence, KV head and row group) index
  __device__ __forceinline__ int64_t row(int hh) const {
    return rbase + row_offset(kv, r0 + hh, sh);
  }
  __device__ __forceinline__ float* o(int hh, int slot) const {
    return part_o + (row(hh) * sh.num_splits + slot) * D;
  }
  __device__ __forceinline__ float* lse(int hh, int slot) const {
    return part_lse + row(hh) * sh.num_splits + slot;
  }
  __device__ __forceinline__ uint32_t* counter(int level, int slot) const {
    return counters + (int64_t)level * kMaxSlots + (int64_t)unit * sh.split_groups +
           slot / kMergeFanIn;
  }
  // floats between the lse / o entries of consecutive slots of one row
  __device__ __forceinline__ int lse_step() const { return 1; }
  __device__ __forceinline__ int o_step() const { return D; }
  __device__ __forceinline__ void store(int hh, int d, f32x4 v, float l) const {
    store_row4<D>(out, sh, row(hh), d, v, l);
  }
};

// Grid (Hkv * row_tiles, batch, splits), NW waves per workgroup, row_tiles groups of KT 16-row
// tiles per KV head.  Consecutive workgroup ids, which the dispatcher deals round-robin to the
// 8 XCDs, walk the KV heads (and row groups) of one sequence first, then the sequences, then
// the splits.  Every XCD therefore gets an even share of the first split of every sequence
// (where ragged batches keep most of their work), and the workgroups that read the same
// physical pages start together.
//
// The NW waves of a workgroup share one (KV head, row group, sequence, split): wave wv streams
// chunks c0+wv, c0+wv+NW, ... through its own register ring (so NW times more K/V bytes are in
// flight per split, with no global partials), and the waves merge their (m, l, O) states
// through LDS.  KT = 2 holds two tiles' states per wave, so one wave per SIMD (512 registers).
//
// A sequence cut into several splits leaves one normalised partial (O/l, log2-sum-exp) per
// split and row.  With fused_combine the splits of each unit merge them through an in-kernel
// tree (merge_tree: groups of kMergeFanIn splits, the last arrival of a group merges it), so the
// whole call is one launch; otherwise mx_paged_decode_combine merges them in a second launch.
//
// kPairW (MX_SCHEDULE_SPLIT_GRID_PAIRED): kernel head p is the stored KV heads 2p and 2p+1, whose
// rows of one token are adjacent.  Waves 0-1 stream head 2p and waves 2-3 head 2p+1 over the same
// chunks of the split (wave wv takes chunks c0 + (wv & 1), c0 + (wv & 1) + 2, ...), each wave with
// the query rows of both heads, of which only its own head's rows are merged (merged_head_pair).
// The unit's rows are the two heads' rows; the strides in MainShape are the stored heads'.  A
// workgroup streaming one head's 256-byte rows reads more slowly the rows at some offsets in
// the 2 KB token row than at others when every head is streamed at once; two adjacent heads
// per workgroup even that out (the measurements are beside make_plan).
template <int D, int NBUF, int NW, bool kCausal, int KT, bool kAppend, bool kFp8,
          bool kPairW = false>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(min_waves_per_simd<D, KT>())))
void mx_paged_decode_splitkv(
    const uint16_t* __restrict__ q, CachePtr<kAppend, CacheElem<kFp8>> kc,
    CachePtr<kAppend, CacheElem<kFp8>> vc,
    uint16_t* __restrict__ out,
    const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ block_table,
    float* __restrict__ part_o, float* __restrict__ part_lse, uint32_t* __restrict__ counters,
    uint32_t* __restrict__ status, const MainShape sh) {
  using L = GroupLds<D, NW, KT>;
  __shared__ __attribute__((aligned(16))) char lds[L::kBytes];
  __shared__ int s_last;
  __shared__ float s_lse[16 * KT];
  WgTimeline timeline;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave index, made provably wave-uniform so the chunk indices derived from it stay in
  // SGPRs and the page lookups remain scalar loads (off the vector-memory counter).
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Grid position (unit of the sequence, sequence, split).  Paired launches take XCD-stable
  // positions (xcd_slot, as the paired balanced kernel): the claim's round trip overlaps the
  // length load, and its barrier comes before any other use of s_last.
  int bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
  if constexpr (kPairW) {
    if (sh.xcd_map) {
      const int X = gridDim.x, Y = gridDim.y;
      const int w0 = bx + X * (by + Y * bz);
      if (tid == 0) s_last = xcd_slot(w0, X * Y * (int)gridDim.z, status + kStatusBytes / 4);
      __syncthreads();
      int w = __builtin_amdgcn_readfirstlane(s_last);
      if (w < 0) {  // the claim masks were not zero (see xcd_slot)
        if (tid == 0) atomicOr(status, (uint32_t)MX_DEVICE_WORKSPACE_STATE);
        w = w0;
      }
      bx = w % X;
      by = (w / X) % Y;
      bz = w / (X * Y);
    }
  }
  const int kv = sh.row_tiles == 1 ? bx : bx / sh.row_tiles;
  const int grp = bx - kv * sh.row_tiles;  // row group: rows grp*16*KT ..
  const int r0 = grp * 16 * KT;
  const int b = by;
  const int split = bz;
  const int nrows = min(16 * KT, sh.rows - r0);  // query rows of this group

  const SeqExtent ext =
      seq_extent<kAppend>(seq_lens, b, sh, status, split == 0 && bx == 0 && tid == 0);
  const int seq = ext.sched;
  if (ext.keys <= 0) {
    // Empty sequence: defined as a zero output.
    if (split == 0)
      for (int e = tid; e < nrows * (D / 4); e += 64 * NW)
        store_row4<D>(out, sh, row_base(b, kv, sh) + row_offset(kv, r0 + e / (D / 4), sh),
                      4 * (e % (D / 4)), f32x4{0.f, 0.f, 0.f, 0.f}, -INFINITY);
    return;
  }
  const int t0 = split * sh.tokens_per_split;
  if (t0 >= seq) return;  // uniform over the workgroup: no barrier is skipped by part of it
  const int t1 = min(t0 + sh.tokens_per_split, seq);
  const bool single = seq <= sh.tokens_per_split;
  const int n_cache = (ext.cache + kChunk - 1) / kChunk;  // chunks read from the paged cache
  const int c_lo = t0 / kChunk;
  const int c_hi = (t1 + kChunk - 1) / kChunk;
  // First chunk any row of this group must mask (causal), else the last cache chunk.
  const int c_mask =
      kCausal ? min(n_cache - 1, max(0, row_key_limit(r0, ext.keys, sh)) / kChunk) : n_cache - 1;

  // Fused append with head_dim 256: the workgroup of split 0 and row group 0 writes the new
  // tokens of (b, kv) to the cache, after its share of the attention (and after its arrival at
  // the merge).
  auto copy_if_writer = [&]() {
    if constexpr (kAppend && NewTokens<kFp8>::template kCopyAfter<D>)
      if (split == 0 && grp == 0)
        copy_new_tokens<D>(seq_lens, block_table, b, kv, sh, status, tid, 64 * NW);
  };

  bf16x8 qop[KT][D / 32];
  SoftmaxState<D> st[KT];
  int row_lim[KT];
  setup_row_group<D, KT>(qop, st, row_lim, q, b, kv, grp, ext.keys, sh, lane);
  bool bad_page = false;
  const int32_t* bt_row = block_table + (int64_t)b * sh.max_pages;
  const int c_end = min(c_hi, n_cache);
  timeline.stream_begin();
  if constexpr (kAppend) {
    // Fused append: the split holding the last schedule chunk also takes the new keys, as one
    // more chunk after its cache chunks in the waves' round-robin order.
    // Paired waves: each head's two waves take the new keys of their own head.
    const bool last = c_hi * kChunk >= seq;
    const int hk = kPairW ? stored_head(kv, wv >> 1, sh) : kv;  // stored head of this wave
    const int wk = kPairW ? (wv & 1) : wv;  // its place among the head's waves
    constexpr int kHeadWaves = kPairW ? 2 : NW;
    const NewTokens<kFp8> nt{sh, b, hk, ext.cache, last && wk == (c_end - c_lo) % kHeadWaves,
                       grp == 0,    ext.at,     bt_row, status};
    stream_chunks<D, NBUF, kHeadWaves, kCausal, KT, NewTokens<kFp8>, kFp8>(
        st, qop, kc, vc, bt_row, hk, c_lo, c_end, ext.cache, c_mask, row_lim, wk,
        L::ktile(lds, wv), sh, bad_page, nt);
  } else if constexpr (kPairW) {
    static_assert(NW == 4 && KT == 1, "paired waves: four waves, one row tile");
    stream_chunks<D, NBUF, 2, kCausal, KT, NoExtraChunk, kFp8>(
        st, qop, kc, vc, bt_row, stored_head(kv, wv >> 1, sh), c_lo, c_end, ext.cache, c_mask,
        row_lim, wv & 1, L::ktile(lds, wv), sh, bad_page);
  } else {
    stream_chunks<D, NBUF, NW, kCausal, KT, NoExtraChunk, kFp8>(
        st, qop, kc, vc, bt_row, kv, c_lo, c_end, ext.cache, c_mask, row_lim, wv,
        L::ktile(lds, wv), sh, bad_page);
  }
  timeline.stream_end();
  if constexpr (kFp8) scale_o_by_v_scale<D, KT>(st, sh);
  if (bad_page && lane == 0) atomicOr(status, (uint32_t)MX_DEVICE_BAD_PAGE_ID);
  publish_wave_state<D, NW, KT>(lds, st, wv);
  for (int e = tid; e < nrows * (D / 4); e += 64 * NW) {
    const int hh = e / (D / 4);
    const int d = 4 * (e - hh * (D / 4));
    float lse;
    f32x4 o;
    if constexpr (kPairW)
      o = merged_head_pair<D>(lds, hh, d, lse, sh);
    else
      o = merged_head<D, NW, KT>(lds, hh, d, lse);
    const int64_t row = row_base(b, kv, sh) + row_offset(kv, r0 + hh, sh);
    if (single) {
      store_row4<D>(out, sh, row, d, o, lse);
    } else if (sh.fused_combine) {  // read back by another workgroup of this launch
      store_partial4(part_o, part_o + (row * sh.num_splits + split) * D + d, o);
      if (d == 0) store_partial1(part_lse + row * sh.num_splits + split, lse);
    } else {                        // read by the combine kernel of the next launch
      *reinterpret_cast<f32x4*>(part_o + (row * sh.num_splits + split) * D + d) = o;
      if (d == 0) part_lse[row * sh.num_splits + split] = lse;
    }
  }
  if (single || !sh.fused_combine) {
    copy_if_writer();
    return;
  }

  // This split's partial is level-0 item `split` of the unit's merge tree.
  const int nsv = (seq + sh.tokens_per_split - 1) / sh.tokens_per_split;  // splits with tokens
  const SplitTree<D> tree{sh,  part_o, part_lse, counters, out, row_base(b, kv, sh), kv, r0,
                          b * (int)gridDim.x + bx};
  // Up to 32 splits merge in one level: the last arrival loads every partial in one round trip
  // (long B=1 32K, 32 splits: 27.36-27.41 against 27.53-27.55 us; long B=4 32K, 16 paired
  // splits: 83.2 against 84.6 us), where fan-in 8 takes two levels of store, arrival and load.
  if (nsv > kMergeFanIn && nsv <= 32)
    merge_tree<D, NW, 32>(tree, split, nsv, nrows, s_lse, &s_last);
  else
    merge_tree<D, NW, kMergeFanIn>(tree, split, nsv, nrows, s_lse, &s_last);
  copy_if_writer();
}

// ------------------------------------------------------------------------------------------
// Length-balanced kernel
// ------------------------------------------------------------------------------------------

// The balanced schedule's merge tree over the pieces of one unit (merge_tree).  Piece k of a unit
// whose first piece is held by workgroup w0 has slot slot0 + k, slot0 = w0 + unit index: the
// slots of different units are disjoint, and so are the counters (kCounterLevels levels of 8,
// enough for 8^4 = 4096 pieces per unit), indexed like the slots.  A slot holds tile_rows rows.
template <int D>
struct BalancedTree {
  const MainShape& sh;
  float* part_o;
  float* part_lse;
  uint32_t* counters;
  uint16_t* out;
  int64_t rbase;  // row_base of the unit
  int kv;         // kernel KV head of the unit
  int r0;         // first row of the unit's row group
  int slot0;
  int tile_rows;
  __device__ __forceinline__ float* o(int hh, int slot) const {
    return part_o + ((int64_t)(slot0 + slot) * tile_rows + hh) * D;
  }
  __device__ __forceinline__ float* lse(int hh, int slot) const {
    return part_lse + (int64_t)(slot0 + slot) * tile_rows + hh;
  }
  __device__ __forceinline__ uint32_t* counter(int level, int slot) const {
    return counters + (int64_t)level * kMaxSlots + slot0 + slot;
  }
  // floats between the lse / o entries of consecutive slots of one row
  __device__ __forceinline__ int lse_step() const { return tile_rows; }
  __device__ __forceinline__ int o_step() const { return tile_rows * D; }
  __device__ __forceinline__ void store(int hh, int d, f32x4 v, float l) const {
    store_row4<D>(out, sh, rbase + row_offset(kv, r0 + hh, sh), d, v, l);
  }
};

// A unit cut into exactly two pieces, merged by the workgroup of its first piece without storing
// that piece: the first piece is the last of its workgroup's share (the unit starts inside the
// share and runs past its end) and the second the first of the next workgroup's, which has
// almost always stored its partial and arrived by then.  Thread 0 reads the unit's level-0
// counter (relaxed, agent scope, like the increments of arrive_last): when it reads 1, the
// second piece's stores were complete before its increment, so this workgroup resets the
// counter, loads that partial (sc1, after the barrier that hands the read to every thread) and
// writes the output with the same arithmetic as a merge step of two items (lse_merge).  Returns
// false, having changed nothing, when the second piece has not arrived: the caller then stores
// this piece and arrives as usual.  `own(hh, d, lse)` gives this piece's merged dims of row hh.
template <int D, int NW, int KT, class Own>
__device__ __forceinline__ bool merge_first_of_two(const BalancedTree<D>& tree, int nrows,
                                                   const Own& own, int* s_flag) {
  if (threadIdx.x == 0) {
    uint32_t* c = tree.counter(0, 0);
    const bool ready = __hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 1u;
    if (ready) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = ready ? 1 : 0;
  }
  __syncthreads();
  if (*s_flag == 0) return false;
  constexpr int kE = (16 * KT * (D / 4) + 64 * NW - 1) / (64 * NW);  // elements per thread
  const int total = nrows * (D / 4);
  const int tid = threadIdx.x;
  float ls[kE][2];
  f32x4 vs[kE][2];
#pragma unroll
  for (int q = 0; q < kE; ++q) {  // the second piece's loads first, all in one round
    const int e = min(tid + q * 64 * NW, total - 1);
    const int hh = e / (D / 4);
    const int d = 4 * (e - hh * (D / 4));
    ls[q][1] = load_partial1(tree.part_lse, tree.lse(hh, 1));
    vs[q][1] = load_partial4(tree.part_o, tree.o(hh, 1) + d);
  }
#pragma unroll
  for (int q = 0; q < kE; ++q) {
    const int e = tid + q * 64 * NW;
    if (e >= total) break;
    const int hh = e / (D / 4);
    const int d = 4 * (e - hh * (D / 4));
    vs[q][0] = own(hh, d, ls[q][0]);
    float lse;
    const f32x4 acc = lse_merge<2>(ls[q], vs[q], 2, lse);
    tree.store(hh, d, acc, lse);
  }
  return true;
}

// One launch of num_groups workgroups covers the whole batch whatever the length mix.  Every
// (sequence b, KV head and row group j) "unit" with n_b = ceil(L_b/16) > 0 chunks occupies n_b +
// unit_overhead consecutive positions of one global line (units in (b, j) order; the
// overhead charges the per-unit Q load and pipeline fill); workgroup w owns positions
// [w*q, (w+1)*q) with q = ceil(total / num_groups), found from seq_lens on the device, so a
// ragged batch is balanced without the host seeing its lengths.  A unit a workgroup covers
// entirely is written out as bf16; a unit cut into several pieces has each piece written as
// a normalised partial (O/l, log2-sum-exp) to its own slot, and the last piece to finish
// merges them through a fan-in-8 tree of per-unit counters, so the whole call is one launch.
//
// kPairW (MX_SCHEDULE_BALANCED_PAIRED): units are (sequence, pair of adjacent KV heads), streamed
// as in mx_paged_decode_splitkv with kPairW (waves 0-1 the first head, 2-3 the second), and a
// pair's chunk weighs twice a single head's on the line (MainShape::chunk_weight).
template <int D, int NBUF, int NW, bool kCausal, int KT, bool kAppend, bool kFp8,
          bool kPairW = false, bool kXcdMap = kPairW>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(min_waves_per_simd<D, KT>())))
void mx_paged_decode_balanced(
    const uint16_t* __restrict__ q, CachePtr<kAppend, CacheElem<kFp8>> kc,
    CachePtr<kAppend, CacheElem<kFp8>> vc,
    uint16_t* __restrict__ out,
    const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ block_table,
    float* __restrict__ part_o, float* __restrict__ part_lse, uint32_t* __restrict__ counters,
    uint32_t* __restrict__ status, const MainShape sh) {
  using L = GroupLds<D, NW, KT>;
  __shared__ __attribute__((aligned(16))) char lds[L::kBytes];
  __shared__ int s_int[NW + 4];
  __shared__ int s_mm[2 * NW];
  __shared__ float s_lse[16 * KT];
  __shared__ int s_len[kBalancedBatch];  // the batch's seq_lens entries
  WgTimeline timeline;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wg0 = blockIdx.x;                        // dispatch index (see wg below)
  const int TR = sh.tile_rows;                       // rows per partial slot
  const int UPS = sh.num_kv_heads * sh.row_tiles;    // units per sequence
  const int B = sh.batch;

  // Sequence weights (positions per sequence).  The batch is at most kBalancedBatch sequences:
  // thread tid reads the kScanPerThread consecutive entries from b = tid * kScanPerThread on
  // once and keeps their weights in registers for both the total and the scan that locates
  // this workgroup's first position.  The entries also go to LDS, where the empty-sequence
  // check and the unit walk read them.
  constexpr int kScanPerThread = (kBalancedBatch + 64 * NW - 1) / (64 * NW);
  int wts[kScanPerThread];  // chunks of the sequence, then its positions
  int nb_lo = INT_MAX, nb_hi = 0;
#pragma unroll
  for (int i = 0; i < kScanPerThread; ++i) {
    const int b = tid * kScanPerThread + i;
    const int len = b < B ? seq_lens[b] : 0;
    if (b < B) s_len[b] = len;
    const int seq = b < B ? seq_extent_of<kAppend>(len, sh, status, wg0 == 0).sched : 0;
    wts[i] = seq > 0 ? (seq + kChunk - 1) / kChunk : 0;
    if (b < B) {
      nb_lo = min(nb_lo, wts[i]);
      nb_hi = max(nb_hi, wts[i]);
    }
  }
  // Positions charged per unit on top of its chunks.  When every sequence has the same chunk
  // count and the workgroups divide into k equal pieces per unit, the overhead is instead the
  // smallest that makes k divide the unit's span: every workgroup then holds exactly one piece
  // of equal chunks (charging the full overhead to a unit's first piece would leave its other
  // pieces longer, and shares that straddle units would pay two pieces).
  int alpha = sh.unit_overhead;
  int wc = sh.chunk_weight;
  int equal_k = 0;  // k when every unit is cut into k equal pieces, one per share
  const int units = B * UPS;
  // (k = 1 needs no change: every workgroup then holds one whole unit whatever the charge.)
  if (sh.num_groups > units && sh.num_groups % units == 0) {  // the same in every thread
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      nb_lo = min(nb_lo, __shfl_xor(nb_lo, off));
      nb_hi = max(nb_hi, __shfl_xor(nb_hi, off));
    }
    if (lane == 0) {
      s_mm[wv] = nb_lo;
      s_mm[NW + wv] = nb_hi;
    }
    __syncthreads();
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) {
      nb_lo = min(nb_lo, s_mm[w2]);
      nb_hi = max(nb_hi, s_mm[NW + w2]);
    }
    // Values read back from LDS are uniform, which the compiler cannot see: without the
    // readfirstlane the unit walk below (and the page-id loads it feeds) would run per lane.
    nb_lo = __builtin_amdgcn_readfirstlane(nb_lo);
    nb_hi = __builtin_amdgcn_readfirstlane(nb_hi);
    if (nb_lo == nb_hi && nb_lo > 0) {
      const int k = sh.num_groups / units;
      wc = 1;
      alpha = (k - nb_lo % k) % k;
      equal_k = k;
    }
  }
  int mine = 0;
#pragma unroll
  for (int i = 0; i < kScanPerThread; ++i) {
    wts[i] = wts[i] > 0 ? UPS * (wts[i] * wc + alpha) : 0;
    mine += wts[i];
  }
  // This workgroup's index on the line: XCD-stable (xcd_slot) in the paired kernels, claimed
  // after the seq_lens loads so the claim's round trip overlaps the scan.  (Only there: the claim
  // code, even switched off, changed the other kernels' register allocation and cost them 1-2 %,
  // and only the paired units showed the placement effect in measurements.)
  if constexpr (kXcdMap) {
    if (tid == 0)
      s_int[NW + 3] = sh.xcd_map ? xcd_slot(wg0, sh.num_groups, status + kStatusBytes / 4) : wg0;
  }
  // One scan over the workgroup: positions before this thread's first sequence, and the total.
  const int incl = wave_inclusive_sum(mine);
  if (tid == 0) s_int[NW] = -1;
  if (lane == 63) s_int[wv] = incl;
  __syncthreads();
  int wg = wg0;
  if constexpr (kXcdMap) {
    wg = __builtin_amdgcn_readfirstlane(s_int[NW + 3]);
    if (wg < 0) {  // the claim masks were not zero (see xcd_slot)
      if (tid == 0) atomicOr(status, (uint32_t)MX_DEVICE_WORKSPACE_STATE);
      wg = wg0;
    }
  }
  // Equal pieces: consecutive workgroups take the same piece of consecutive units (as the split
  // grid's consecutive workgroups take consecutive KV heads), not the k pieces of one unit.
  // Uniform B=8-16, L=4096 batches: 1-3 % faster.
  if (equal_k > 0) wg = (wg % units) * equal_k + wg / units;
  // Empty sequences (L <= 0) are defined as zero output; sequence b's zeros (its seqlen_q *
  // num_heads consecutive rows) are written by workgroup b % num_groups.
  if constexpr (!kAppend) {
    for (int b = wg0; b < B; b += sh.num_groups) {
      if (key_count_of(s_len[b], sh.appended) <= 0) {
        const int64_t row0 = (int64_t)b * sh.seqlen_q * sh.num_heads;
        for (int e = tid; e < sh.seqlen_q * sh.num_heads * (D / 4); e += 64 * NW)
          store_row4<D>(out, sh, row0 + e / (D / 4), 4 * (e % (D / 4)),
                        f32x4{0.f, 0.f, 0.f, 0.f}, -INFINITY);
      }
    }
  }
  int total = 0, before = 0;
#pragma unroll
  for (int w2 = 0; w2 < NW; ++w2) {
    total += s_int[w2];
    before += w2 < wv ? s_int[w2] : 0;
  }
  if (total == 0) return;
  // (Shares of at least one chunk's weight: every workgroup a unit spans then holds a chunk.)
  const int qsz = max((total + sh.num_groups - 1) / sh.num_groups, wc);
  const int x_begin = wg * qsz;
  if (x_begin >= total) return;
  const int x_end = min(x_begin + qsz, total);
  // Positions are laid out sequence by sequence, so the sequence holding x_begin is found by
  // exactly one thread (the positions of non-empty sequences tile [0, total)).
  {
    int start = before + incl - mine;
#pragma unroll
    for (int i = 0; i < kScanPerThread; ++i) {
      if (wts[i] > 0 && start <= x_begin && x_begin < start + wts[i]) {
        s_int[NW] = tid * kScanPerThread + i;
        s_int[NW + 1] = start;
      }
      start += wts[i];
    }
    __syncthreads();
  }
  int b = __builtin_amdgcn_readfirstlane(s_int[NW]);
  int seq_start = __builtin_amdgcn_readfirstlane(s_int[NW + 1]);
  if (b < 0) return;  // unreachable: the positions of non-empty sequences tile [0, total)

  // (LDS values are uniform here; readfirstlane keeps the unit walk in scalar registers.)
  auto extent = [&](int bb) {
    return seq_extent_of<kAppend>(__builtin_amdgcn_readfirstlane(s_len[bb]), sh, status, false);
  };
  SeqExtent ext = extent(b);
  int n_b = (ext.sched + kChunk - 1) / kChunk;
  int span = n_b * wc + alpha;
  // The unit walk divides only through shifts (the chunk weight is a power of two) and
  // div_floor: with one wave per SIMD, every step of an integer division's ~35-instruction
  // sequence would wait out its full latency, on every piece.
  const int wshift = __builtin_ctz(wc);
  const double inv_qsz = 1.0 / qsz;
  int j = div_floor(x_begin - seq_start, 1.0 / span);  // (KV head, row group) of the unit
  int kv = sh.row_tiles == 1 ? j : j / sh.row_tiles;
  int grp = j - kv * sh.row_tiles;  // row group: rows grp*16*KT ..
  int u0 = seq_start + j * span;  // first position of unit (b, j)
  bool bad_page = false;

  for (;;) {
    // Unit (b, j): positions [u0, u0 + span), its chunk c at positions u0 + alpha + c * wc ..;
    // this workgroup takes the chunks that start in [x_begin, x_end).
    const int cpos = u0 + alpha;
    const int ca = min(n_b, (max(0, x_begin - cpos) + wc - 1) >> wshift);
    const int cb = min(n_b, (max(0, x_end - cpos) + wc - 1) >> wshift);
    if (ca < cb) {
      const int unit = b * UPS + j;
      const int r0 = grp * 16 * KT;
      const int nrows = min(16 * KT, sh.rows - r0);
      const int64_t rbase = row_base(b, kv, sh);
      // Workgroups holding the unit's first and last chunks: this one when that chunk starts
      // in [x_begin, x_end) (one does, as ca < cb).
      const int last = cpos + (n_b - 1) * wc;
      const int first_wg = cpos >= x_begin ? wg : div_floor(cpos, inv_qsz);
      const int npieces = (last < x_end ? wg : div_floor(last, inv_qsz)) - first_wg + 1;
      const int n_cache = (ext.cache + kChunk - 1) / kChunk;  // chunks read from the cache
      const int c_mask = kCausal ? min(n_cache - 1, max(0, row_key_limit(r0, ext.keys, sh)) / kChunk)
                                 : n_cache - 1;

      bf16x8 qop[KT][D / 32];
      SoftmaxState<D> st[KT];
      int row_lim[KT];
      setup_row_group<D, KT>(qop, st, row_lim, q, b, kv, grp, ext.keys, sh, lane);
      const int32_t* bt_row = block_table + (int64_t)b * sh.max_pages;
      const int c_end = min(cb, n_cache);
      timeline.stream_begin();
      if constexpr (kAppend) {
        // Fused append: the piece holding the unit's last schedule chunk also takes the new
        // keys, as one more chunk after its cache chunks in the waves' round-robin order.
        // Paired waves: each head's two waves take the new keys of their own head.
        const int hk = kPairW ? stored_head(kv, wv >> 1, sh) : kv;  // stored head of this wave
        const int wk = kPairW ? (wv & 1) : wv;  // its place among the head's waves
        constexpr int kHeadWaves = kPairW ? 2 : NW;
        const NewTokens<kFp8> nt{sh, b, hk, ext.cache, cb == n_b && wk == (c_end - ca) % kHeadWaves,
                           grp == 0, ext.at, bt_row, status};
        stream_chunks<D, NBUF, kHeadWaves, kCausal, KT, NewTokens<kFp8>, kFp8>(
            st, qop, kc, vc, bt_row, hk, ca, c_end, ext.cache, c_mask, row_lim, wk,
            L::ktile(lds, wv), sh, bad_page, nt);
      } else if constexpr (kPairW) {
        static_assert(NW == 4 && KT == 1, "paired waves: four waves, one row tile");
        stream_chunks<D, NBUF, 2, kCausal, KT, NoExtraChunk, kFp8>(
            st, qop, kc, vc, bt_row, stored_head(kv, wv >> 1, sh), ca, c_end, ext.cache, c_mask,
            row_lim, wv & 1, L::ktile(lds, wv), sh, bad_page);
      } else {
        stream_chunks<D, NBUF, NW, kCausal, KT, NoExtraChunk, kFp8>(
            st, qop, kc, vc, bt_row, kv, ca, c_end, ext.cache, c_mask, row_lim, wv,
            L::ktile(lds, wv), sh, bad_page);
      }
      timeline.stream_end();
      if constexpr (kFp8) scale_o_by_v_scale<D, KT>(st, sh);
      publish_wave_state<D, NW, KT>(lds, st, wv);

      if (npieces == 1) {
        for (int e = tid; e < nrows * (D / 4); e += 64 * NW) {
          const int hh = e / (D / 4);
          const int d = 4 * (e - hh * (D / 4));
          float lse;
          f32x4 o;
          if constexpr (kPairW)
            o = merged_head_pair<D>(lds, hh, d, lse, sh);
          else
            o = merged_head<D, NW, KT>(lds, hh, d, lse);
          store_row4<D>(out, sh, rbase + row_offset(kv, r0 + hh, sh), d, o, lse);
        }
      } else {
        // Piece k of the unit goes to slot slot0 + k and is level-0 item k of its merge tree.
        const int slot0 = first_wg + unit;
        const int item = wg - first_wg;
        const BalancedTree<D> tree{sh, part_o, part_lse, counters, out, rbase, kv, r0, slot0, TR};
        auto own = [&](int hh, int d, float& lse) -> f32x4 {
          if constexpr (kPairW)
            return merged_head_pair<D>(lds, hh, d, lse, sh);
          else
            return merged_head<D, NW, KT>(lds, hh, d, lse);
        };
        // (Not at head_dim 256: there its registers spilled in the causal kernel.)
        bool merged = false;
        if constexpr (D <= 128) {
          if (npieces == 2 && item == 0)
            merged = merge_first_of_two<D, NW, KT>(tree, nrows, own, &s_int[NW + 2]);
        }
        if (!merged) {
          float* po = part_o + (int64_t)(slot0 + item) * TR * D;
          float* pl = part_lse + (int64_t)(slot0 + item) * TR;
          for (int e = tid; e < nrows * (D / 4); e += 64 * NW) {
            const int hh = e / (D / 4);
            const int d = 4 * (e - hh * (D / 4));
            float lse;
            const f32x4 o = own(hh, d, lse);
            store_partial4(part_o, po + hh * D + d, o);
            if (d == 0) store_partial1(pl + hh, lse);
          }
          merge_tree<D, NW, kMergeFanIn>(tree, item, npieces, nrows, s_lse, &s_int[NW + 2]);
        }
      }
      // The merged states in LDS share bytes with the K tiles the next piece streams into:
      // no wave may start that piece until every wave has finished reading them.
      __syncthreads();
    }
    // Next unit.
    u0 += span;
    if (u0 >= x_end) break;
    if (++grp == sh.row_tiles) {
      grp = 0;
      ++kv;
    }
    if (++j == UPS) {
      j = 0;
      kv = 0;
      ext.sched = 0;
      while (ext.sched <= 0 && ++b < B) ext = extent(b);
      if (b >= B) break;  // unreachable: positions only exist for non-empty sequences
      n_b = (ext.sched + kChunk - 1) / kChunk;
      span = n_b * wc + alpha;
    }
  }
  if (bad_page && lane == 0) atomicOr(status, (uint32_t)MX_DEVICE_BAD_PAGE_ID);
  if constexpr (kAppend && NewTokens<kFp8>::template kCopyAfter<D>) {
    // Fused append with head_dim 256: the cache writes of the (sequence, KV head) pairs, spread
    // over the workgroups that hold positions, each doing its share after all its pieces.
    const int n_active = (total + qsz - 1) / qsz;
    for (int pr = wg; pr < B * sh.num_kv_heads; pr += n_active)
      copy_new_tokens<D>(seq_lens, block_table, pr / sh.num_kv_heads, pr % sh.num_kv_heads, sh,
                         status, tid, 64 * NW);
  }
}

// ------------------------------------------------------------------------------------------
// LSE merge of partials: out[row] = sum_s 2^(lse_s - M) * O_s / sum_s 2^(lse_s - M), M = max_s
// lse_s (optimized_c500_flash_attn.cu:666-728, log2 domain).  Partials with lse -inf (a causal
// row that saw no key in that part) weigh 0, and a row no part saw a key for is zeros.
// ------------------------------------------------------------------------------------------

// One wave merges the n partials of one row: lane holds dims E*lane .. E*lane+E-1.  Partial s
// sits at lse[s * lse_stride] (times lse_to_log2 in log2 units) and o[s * o_stride + E*lane ..].  One online pass, the loads of
// kBatch partials issued together per round (the pass is latency-bound).  Returns the merged
// log2-sum-exp (-inf when no part saw a key) and leaves the normalised dims in acc.
template <int D>
__device__ __forceinline__ float merge_row(float (&acc)[D / 64], const float* __restrict__ lse,
                                           int64_t lse_stride, float lse_to_log2,
                                           const float* __restrict__ o, int64_t o_stride, int n,
                                           int lane) {
  constexpr int E = D / 64;
  constexpr int kBatch = 16;
  const float* po = o + E * lane;
  float mx = -INFINITY;  // running max of the log2-sum-exps seen
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
  float wsum = 0.f;
  for (int s0 = 0; s0 < n; s0 += kBatch) {
    float ls[kBatch];
    float vs[kBatch][E];
    // Every slot loads (past the last part it re-reads the last one), so the loads are
    // unconditional and issue back to back; the extra slots are masked by their lse below.
#pragma unroll
    for (int t = 0; t < kBatch; ++t) {
      const int64_t sl = min(s0 + t, n - 1);
      ls[t] = lse[sl * lse_stride] * lse_to_log2;
      const float* src = po + sl * o_stride;
      if constexpr (E == 1) {
        vs[t][0] = src[0];
      } else if constexpr (E == 2) {
        const f32x2 x = *reinterpret_cast<const f32x2*>(src);
        vs[t][0] = x[0];
        vs[t][1] = x[1];
      } else {
        const f32x4 x = *reinterpret_cast<const f32x4*>(src);
#pragma unroll
        for (int e = 0; e < 4; ++e) vs[t][e] = x[e];
      }
    }
#pragma unroll
    for (int t = 0; t < kBatch; ++t)
      if (s0 + t >= n) ls[t] = -INFINITY;
    float bm = mx;
#pragma unroll
    for (int t = 0; t < kBatch; ++t) bm = fmaxf(bm, ls[t]);
    if (bm > -INFINITY) {  // else: no part so far saw a key for this row
      const float a = __builtin_amdgcn_exp2f(mx - bm);
      wsum *= a;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] *= a;
#pragma unroll
      for (int t = 0; t < kBatch; ++t) {
        const float w = __builtin_amdgcn_exp2f(ls[t] - bm);
        wsum += w;
#pragma unroll
        for (int e = 0; e < E; ++e) acc[e] += w * vs[t][e];
      }
      mx = bm;
    }
  }
  const bool seen = wsum > 0.f;
  const float inv = seen ? 1.0f / wsum : 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] *= inv;
  return seen ? mx + log2f(wsum) : -INFINITY;
}

// Writes a merged row (log2-sum-exp lse): bf16 to out, or (partial outputs) fp32 to o_out and
// the natural-log sum-exp to lse_out.  half >= 0 (paired heads, MainShape::pair_group): the
// row is 64 dims, taken from half `half` of the D merged ones.
template <int D>
__device__ __forceinline__ void store_merged_row(const float (&acc)[D / 64], float lse,
                                                 uint16_t* __restrict__ out,
                                                 float* __restrict__ o_out,
                                                 float* __restrict__ lse_out, int64_t row,
                                                 int lane, int half = -1) {
  constexpr int E = D / 64;
  int64_t at = row * D + E * lane;
  bool first = lane == 0;
  if constexpr (D == 128) {
    if (half >= 0) {
      if ((E * lane >= D / 2) != (half == 1)) return;
      at = row * (D / 2) + E * lane - half * (D / 2);
      first = E * lane == half * (D / 2);
    }
  }
  if (o_out != nullptr) {
#pragma unroll
    for (int e = 0; e < E; ++e) o_out[at + e] = acc[e];
    if (first) lse_out[row] = lse * kLn2;
    return;
  }
  uint16_t* op = out + at;
  if constexpr (E == 1) {
    op[0] = __builtin_bit_cast(uint16_t, (__bf16)acc[0]);
  } else if constexpr (E == 2) {
    *reinterpret_cast<uint32_t*>(op) = pack_bf16x2(acc[0], acc[1]);
  } else {
    const u32x2 w = {pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
    *reinterpret_cast<u32x2*>(op) = w;
  }
}

// Second launch of the split grid: one wave per (query head, sequence * query token) merges the
// splits that hold tokens of the row's sequence.
template <int D>
__global__ __launch_bounds__(64) void mx_paged_decode_combine(
    const float* __restrict__ part_o, const float* __restrict__ part_lse,
    const int32_t* __restrict__ seq_lens, uint16_t* __restrict__ out, float* __restrict__ o_out,
    float* __restrict__ lse_out, int num_heads, int seqlen_q, int num_splits,
    int tokens_per_split, int cap_tokens, int appended, int new_tokens, int pair_group) {
  const int h = blockIdx.x;
  const int bt = blockIdx.y;  // sequence * seqlen_q + query token
  const int b = bt / seqlen_q;
  const int lane = threadIdx.x;
  // Tokens the splits cover (SeqExtent::sched of the main kernel).
  const int seq = new_tokens > 0 ? max(min(max(seq_lens[b], 0), cap_tokens), 1)
                                 : min(key_count(seq_lens, b, appended), cap_tokens);
  if (seq <= tokens_per_split) return;  // single split (or empty): main kernel wrote it
  const int nsv = (seq + tokens_per_split - 1) / tokens_per_split;
  const int64_t row = (int64_t)bt * num_heads + h;
  float acc[D / 64];
  const float lse = merge_row<D>(acc, part_lse + row * num_splits, 1, 1.0f,
                                 part_o + row * num_splits * D, D, nsv, lane);
  store_merged_row<D>(acc, lse, out, o_out, lse_out, row, lane,
                      pair_group > 0 ? (h / pair_group) & 1 : -1);
}

// mx_lse_merge: rows merged over `parts` gathered partials, part-major ([parts, rows, D] and
// [parts, rows], natural-log sum-exps); one wave per row.
template <int D>
__global__ __launch_bounds__(64) void mx_lse_merge_kernel(const float* __restrict__ o_parts,
                                                          const float* __restrict__ lse_parts,
                                                          int64_t rows, int parts,
                                                          uint16_t* __restrict__ out) {
  const int64_t row = blockIdx.x;
  float acc[D / 64];
  const float lse = merge_row<D>(acc, lse_parts + row, rows, kLog2e, o_parts + row * D,
                                 rows * D, parts, threadIdx.x);
  store_merged_row<D>(acc, lse, out, nullptr, nullptr, row, threadIdx.x);
}

// ------------------------------------------------------------------------------------------
// Paged KV-cache append: the new tokens' K/V rows into their block-table slots
// ------------------------------------------------------------------------------------------

// One wave per (new token, K or V).  A token's Hkv * D values are contiguous both in the
// new-token tensor [batch, seqlen_new, Hkv, D] and in its page slot [page, offset, Hkv, D], so
// the copy is row_vec16 = Hkv * D / 8 16-byte vectors.  Token j of sequence b goes to position
// pos = max(seq_lens[b], 0) + j: page block_table[b, pos / page_size], offset
// pos % page_size.  A position past the table row or a page id outside [0, num_pages) is
// flagged and skipped, so nothing is ever written outside the pool.
__global__ __launch_bounds__(256) void mx_paged_kv_append_kernel(
    const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ block_table, int batch,
    int seqlen_new, int row_vec16, int page_size, int num_pages, int max_pages,
    uint32_t* __restrict__ status) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
  if (wave >= 2 * batch * seqlen_new) return;
  const int tok = wave >> 1;  // neighbouring waves copy the K and V rows of one token
  const bool is_v = (wave & 1) != 0;
  const int b = tok / seqlen_new;
  const int j = tok - b * seqlen_new;
  const int pos = append_position(seq_lens[b], j, max_pages * page_size);
  if (pos < 0) {
    if (lane == 0 && !is_v) atomicOr(status, (uint32_t)MX_DEVICE_SEQ_TOO_LONG);
    return;
  }
  const int pid = block_table[(int64_t)b * max_pages + pos / page_size];
  if (pid < 0 || pid >= num_pages) {
    if (lane == 0 && !is_v) atomicOr(status, (uint32_t)MX_DEVICE_BAD_PAGE_ID);
    return;
  }
  const u32x4* src = reinterpret_cast<const u32x4*>(is_v ? v_new : k_new) + (int64_t)tok * row_vec16;
  u32x4* dst = reinterpret_cast<u32x4*>(is_v ? v_cache : k_cache) +
               ((int64_t)pid * page_size + pos % page_size) * row_vec16;
  for (int i = lane; i < row_vec16; i += 64) dst[i] = src[i];
}

// The append into an fp8 (e4m3fn) cache: the same slots, each bf16 value x stored as the OCP
// e4m3fn value nearest to x / scale (ties to even), with x / scale clamped to [-448, 448]
// first (saturation; NaN stays NaN).  One wave per (new token, K or V); a lane converts 8
// values per step, one 16-byte load of bf16 into one 8-byte store of fp8.
__global__ __launch_bounds__(256) void mx_paged_kv_append_fp8_kernel(
    const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
    uint8_t* __restrict__ k_cache, uint8_t* __restrict__ v_cache,
    const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ block_table, int batch,
    int seqlen_new, int row_vec8, int page_size, int num_pages, int max_pages, float k_scale,
    float v_scale, uint32_t* __restrict__ status) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
  if (wave >= 2 * batch * seqlen_new) return;
  const int tok = wave >> 1;
  const bool is_v = (wave & 1) != 0;
  const int b = tok / seqlen_new;
  const int j = tok - b * seqlen_new;
  const int pos = append_position(seq_lens[b], j, max_pages * page_size);
  if (pos < 0) {
    if (lane == 0 && !is_v) atomicOr(status, (uint32_t)MX_DEVICE_SEQ_TOO_LONG);
    return;
  }
  const int pid = block_table[(int64_t)b * max_pages + pos / page_size];
  if (pid < 0 || pid >= num_pages) {
    if (lane == 0 && !is_v) atomicOr(status, (uint32_t)MX_DEVICE_BAD_PAGE_ID);
    return;
  }
  const u32x4* src = reinterpret_cast<const u32x4*>(is_v ? v_new : k_new) + (int64_t)tok * row_vec8;
  u32x2* dst = reinterpret_cast<u32x2*>(is_v ? v_cache : k_cache) +
               ((int64_t)pid * page_size + pos % page_size) * row_vec8;
  const float scale = is_v ? v_scale : k_scale;
  for (int i = lane; i < row_vec8; i += 64) {
    const u32x4 x = src[i];
    dst[i] = u32x2{bf16x4_to_fp8x4(x[0], x[1], scale), bf16x4_to_fp8x4(x[2], x[3], scale)};
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

// Schedule policy (replaces the 104-SM regime table of submission_clean.cu:375-430), from
// interleaved A/B sweeps on MI355X over the five north-star configurations:
//  * workgroups per CU: one cooperative 4-wave group for D=128 and D=256, two 2-wave groups
//    for D=64 -- more resident groups contend for HBM without adding bandwidth;
//  * batches with at least kBalancedMinUnits (sequence, KV head) units and a capacity of at
//    least kBalancedMinCap tokens (or half that with 512+ units) take the balanced single
//    launch (lengths balanced on the device, ~84% of 8 TB/s on Llama-3-8B decode);
//  * shorter capacities take the split grid: its one split per unit skips the length scan
//    and the merges, 15-50% faster below 1 024 tokens (e.g. B=64, Hkv=8, 64 tokens: 7.4 vs
//    14.9 us);
//  * fewer, long units (long-context decode) take the split grid, whose page-aligned splits
//    plus a separate combine beat the balanced merge tree by ~10% there;
//  * split counts: just enough splits for the workgroup target, each at least
//    kMinTokensPerSplit long and at most kMaxTokensPerSplit.
constexpr int64_t kMinTokensPerSplit = 128;   // amortises Q load, pipeline fill and partials
constexpr int64_t kMaxTokensPerSplit = 16384;  // bounds one workgroup's share of a sequence
constexpr int64_t kPairMinTokensPerSplit = 896;  // paired split grid: shortest paired split
constexpr int64_t kMaxGridDim = 65535;
// Query heads per KV head (MQA included).  Rows of one KV head are processed in 16- or 32-row
// groups whatever the group size, so the limit only bounds how often K/V is re-streamed.
constexpr int64_t kMaxGroup = 128;
constexpr int64_t kBalancedMinUnits = 64;
constexpr int64_t kBalancedMinCap = 2048;  // tokens of capacity (max_seq_len) for balanced
constexpr int64_t kMaxMergeRows = int64_t(1) << 25;  // mx_lse_merge: 64 * rows work-items < 2^31

int64_t groups_per_cu(int64_t head_dim) { return head_dim == 64 ? 2 : 1; }

// Whether the split grid's units merge their splits in-kernel (one launch): each level of the
// counter region must hold ceil(splits / kMergeFanIn) counters per unit, the tree's levels
// cover at most kMaxMergeItems splits, and the o partials (o_bytes) stay within the 32-bit
// offsets of the handoff's buffer accesses.  Otherwise the combine kernel merges in a second
// launch.
constexpr int64_t kMaxHandoffBytes = 0x7fffffff;
// The balanced kernel's partial slots always fit: slots <= kMaxSlots of at most 64 rows.
static_assert((int64_t)kMaxSlots * 64 * 256 * 4 <= kMaxHandoffBytes, "balanced partials");
bool split_tree_fits(int64_t units, int64_t splits, int64_t o_bytes) {
  return splits <= kMaxMergeItems && units * ceil_div(splits, kMergeFanIn) <= kMaxSlots &&
         o_bytes <= kMaxHandoffBytes;
}

// Balanced schedule: chunk positions charged per unit on top of its chunks, for its query load,
// pipeline fill and merge.  A per-workgroup timeline of ragged decode puts a piece at 0.26 us per
// chunk plus 2.3 us (1.5 us more when the unit is cut and merged): at 6 positions the units were
// undercharged, and the workgroups holding many one-chunk units ended last (84 us against a
// median of 68).  8 took ragged decode from 85.0 to 80.0 us (10 and 12: 81.1, 82.8), the other
// configurations unchanged.
constexpr int kChunkPositions = 8;
constexpr int kUnitOverhead = 8 * kChunkPositions;
// Mirrored pairs (MainShape::pair_mirror) are charged 80 positions per pair unit (the weight of
// 10 single-head chunks, 5 of their own).  Interleaved A/B on config 4: 64, 80, 96, 112 and 128
// positions 75.9-76.1, 74.7-74.8, 74.8-74.9, 74.9-75.0 and 75.1-75.2 us (single heads
// 75.6-75.9); config 4's lengths at page size 16: 80 positions 75.4, 96 75.9, 128 75.9 against
// 77.1 us single-head.
constexpr int kMirroredPairOverhead = 10 * kChunkPositions;
// fp8 caches: a chunk moves half a bf16 chunk's bytes in about half the time, while a unit's
// query load, pipeline fill and merge take as long, so a unit costs more chunk positions: 160
// (192 for the pairs of 512- and 768-byte token rows).  Interleaved A/B on ragged lengths
// (config 4's recipe, B=256, up to 8 192 tokens), charges 64 / 128 / 160 / 192 / 256 / 320:
// - 4 KV heads, fp8 pairs (config 4): 61.6 / 48.0 / 45.5 / 44.3 / 44.4 / 45.6 us;
// - 8 KV heads, pairs, page size 16: 103.1 / 78.6 / 78.5 / 79.5 / 81.1 / 82.9; page size 64:
//   101.7 / 77.8 / 77.9 / 79.0 / 79.8 / 82.4;
// - 2 KV heads, single heads: head_dim 128 35.7 / 27.9 / 27.0 / 27.5 / 28.4 / 29.7, head_dim
//   256 (B=128) 32.9 / 29.6 / 28.7 / 28.4 / 29.9 / 30.7.
constexpr int kFp8UnitOverhead = 20 * kChunkPositions;
constexpr int kFp8NarrowPairOverhead = 24 * kChunkPositions;
constexpr int kMaxUnitOverhead = kFp8NarrowPairOverhead;  // of every charge above
static_assert((kChunkPositions & (kChunkPositions - 1)) == 0,
              "the balanced kernels divide by the chunk weight with a shift");
// Balanced schedule limits: the largest batch whose seq_lens scan stays within two passes of
// one workgroup.
constexpr int64_t kBalancedMaxBatch = kBalancedBatch;
constexpr int64_t kBalancedMaxGroups = 4095;  // pieces per unit stay within the 8^4 merge tree
constexpr int64_t kBalancedMaxUnits = 8192;   // batch * Hkv * row tiles (counter region)
// The balanced kernels count a batch's chunks (plus per-unit overheads) in 32-bit integers.
constexpr int64_t kBalancedMaxLine = int64_t(1) << 30;

struct Plan {
  int schedule = MX_SCHEDULE_SPLIT_GRID;
  int64_t splits = 1;             // split grid: splits per sequence
  int64_t tokens_per_split = 0;   // split grid
  int64_t groups = 0;             // balanced: workgroups of the launch
  int64_t slots = 0;              // balanced: partial slots (groups + units)
  int64_t rows = 1;               // query rows per KV head: seqlen_q * group
  int64_t row_tiles = 1;          // row groups: ceil(rows / (16 * tiles_per_group))
  int tiles_per_group = 1;        // 16-row tiles one pass over K/V serves (1, or 2 above 16 rows)
  int64_t cap_tokens = 0;
  int64_t counter_offset = 0;
  int64_t lse_offset = 0;
  int64_t o_offset = 0;
  int64_t workspace_bytes = kStatusBytes;
  int chunk_shift = 0;
  bool pair_mirror = false;       // MX_SCHEDULE_BALANCED_PAIRED: mirrored pairs (MainShape)
};

// KV heads of the kernels' units: pairs of the (kernel) heads on the paired schedules.
int64_t plan_kv_heads(const Plan& plan, int64_t kv_heads) {
  return (plan.schedule == MX_SCHEDULE_SPLIT_GRID_PAIRED ||
          plan.schedule == MX_SCHEDULE_BALANCED_PAIRED)
             ? kv_heads / 2
             : kv_heads;
}

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
// Whether an automatic plan runs adjacent KV heads in pairs, two waves per head
// (MX_SCHEDULE_SPLIT_GRID_PAIRED, MX_SCHEDULE_BALANCED_PAIRED): calls that allow it (pair_ok:
// pair_ok_for), head_dim 128, at least 8 KV heads, an even count (token rows of at least 2 KB
// in bf16, 1 KB in fp8), and both heads' rows in one 16-row tile.
// pair_ok values (pair_ok_for): no pairs; bf16 rules; fp8 rules, where 4 KV heads (512-byte
// token rows) also pair on the balanced schedule when there are at least as many pair units as
// workgroups (a ragged batch: config 4's lengths on an fp8 cache, 63.7-63.9 against 67.5-68.5
// us; with fewer units, e.g. contest cases 8 and 11 on fp8, pairs lost 16 and 8 %).  bf16
// caches of 4 KV heads (1 KB token rows) pair on the balanced schedule as mirrored pairs
// (MainShape::pair_mirror) when there are more pair units than workgroups (mirrored_pairs).
constexpr int kPairNone = 0, kPairBf16 = 1, kPairFp8 = 2;
bool pair_heads(bool pair_ok, int64_t num_splits, int64_t head_dim, int64_t num_kv_heads,
                int64_t rows) {
  return pair_ok && num_splits == 0 && head_dim == 128 && num_kv_heads % 2 == 0 &&
         num_kv_heads * head_dim * 2 >= 2048 && 2 * rows <= 16;
}

// Mirrored pairs (MainShape::pair_mirror): balanced pairs of heads 0 and 3, 1 and 2 of a bf16
// cache with 4 KV heads at head_dim 128, when the batch has more pair units than workgroups.
// Interleaved A/B against single heads (B ragged or uniform lengths, Hq=28, page size 64 unless
// noted):
// - config 4 (B=256, lengths up to 8 192): 74.7-74.8 against 75.9-76.2 us, graph replays 74.9
//   against 76.6; the same lengths at page size 16: 75.4 against 77.1; ragged B=192: 55.7
//   against 57.2; ragged B=512 up to 4 096: 84.6 against 85.3;
// - uniform B=256 at 2 048 tokens: 163.3 against 163.3; B=192 at 4 096: 243.5 against 242.4.
// Adjacent pairs (0 and 1, 2 and 3) lost on config 4 (77.6-78.0 us), pairs 0 and 2, 1 and 3
// lost less (76.7-77.0), both at the 8 positions per unit of 2 KB pairs, where mirrored pairs
// took 75.6-75.7.  With as many pair units as workgroups (B=128) pairs lost: ragged 42.3
// against 41.9, uniform at 4 096 tokens 162.2 against 157.8 us.
bool mirrored_pairs(int pair_ok, int64_t num_splits, int64_t head_dim, int64_t num_kv_heads,
                    int64_t rows, int64_t units, int64_t groups) {
  return pair_ok == kPairBf16 && num_kv_heads == 4 &&
         pair_heads(true, num_splits, head_dim, 2 * num_kv_heads, rows) && units / 2 > groups;
}

// Automatic split count of the split grid: enough splits for `slots` resident workgroups over
// `units` units, each split holding at least kMinTokensPerSplit tokens at capacity `cap` (and
// splitting starts at four splits: the partial round trip and merge, ~3.5 us, are only repaid
// by cutting a unit's streaming time at least four ways; capacity 256: 1 split 7.8-8.1 us, 2
// splits 8.7-8.9 us; capacity 512 with 64 units: 4 splits 9.2 us, 1 split 10.2 us), and at most
// kMaxTokensPerSplit.
int64_t auto_splits(int64_t units, int64_t slots, int64_t cap) {
  int64_t ns = ceil_div(slots, units);
  int64_t max_by_len = cap / kMinTokensPerSplit;
  if (max_by_len < 4) max_by_len = 1;
  if (ns > max_by_len) ns = max_by_len;
  const int64_t min_by_len = ceil_div(cap, kMaxTokensPerSplit);
  if (ns < min_by_len) ns = min_by_len;
  return ns;
}

int make_plan(int64_t batch, int64_t seqlen_q, int64_t num_heads, int64_t num_kv_heads,
              int64_t head_dim, int64_t page_size, int64_t max_pages, int64_t max_seq_len,
              int64_t num_splits, int64_t num_cus, int pair_ok, Plan* plan) {
  if (batch < 1 || seqlen_q < 1 || num_heads < 1 || num_kv_heads < 1 || head_dim < 1 ||
      page_size < 1 || max_pages < 1)
    return fail(MX_STATUS_INVALID_SHAPE,
                "batch, seqlen_q, num_heads, num_kv_heads, head_dim, page_size and "
                "max_pages_per_seq must all be >= 1");
  if (num_heads % num_kv_heads != 0)
    return fail(MX_STATUS_INVALID_SHAPE, "num_heads must be a multiple of num_kv_heads");
  if (num_heads / num_kv_heads > kMaxGroup)
    return fail(MX_STATUS_UNSUPPORTED, "query group (num_heads / num_kv_heads) must be <= 128");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(MX_STATUS_UNSUPPORTED, "head_dim must be 64, 128 or 256");
  if (page_size != 16 && page_size != 32 && page_size != 64 && page_size != 128 &&
      page_size != 256)
    return fail(MX_STATUS_UNSUPPORTED, "page_size must be 16, 32, 64, 128 or 256");
  if (batch > kMaxGridDim) return fail(MX_STATUS_UNSUPPORTED, "batch must be <= 65535");
  if (batch * seqlen_q > kMaxGridDim)
    return fail(MX_STATUS_UNSUPPORTED, "batch * seqlen_q must be <= 65535");
  const int64_t group = num_heads / num_kv_heads;
  const int64_t rows = seqlen_q * group;
  // Above 16 rows, one pass over a head's K/V serves two 16-row tiles (32 rows); at
  // head_dim 256 two tiles' states do not fit the registers of a wave.
  const int tiles_per_group = (rows > 16 && head_dim <= 128) ? 2 : 1;
  const int64_t row_tiles = ceil_div(rows, 16 * tiles_per_group);
  const int64_t tile_rows = std::min<int64_t>(rows, 16 * tiles_per_group);
  if (num_kv_heads * row_tiles > kMaxGridDim)
    return fail(MX_STATUS_UNSUPPORTED, "num_kv_heads * ceil(seqlen_q * group / 16) must be <= 65535");
  plan->rows = rows;
  plan->row_tiles = row_tiles;
  plan->tiles_per_group = tiles_per_group;
  if (num_heads > kMaxGridDim) return fail(MX_STATUS_UNSUPPORTED, "num_heads must be <= 65535");
  // Token positions are int32, including a capacity plus the up to 16 keys a one-launch
  // append-and-attend adds.
  if (max_pages > ((int64_t)INT32_MAX - kChunk) / page_size)
    return fail(MX_STATUS_UNSUPPORTED, "max_pages_per_seq * page_size must be < 2^31 - 16");
  if (num_kv_heads * head_dim * page_size > (int64_t)INT32_MAX / 4)
    return fail(MX_STATUS_UNSUPPORTED, "page too large for 32-bit in-page offsets");

  const int64_t table_tokens = max_pages * page_size;
  const int64_t cap = (max_seq_len > 0 && max_seq_len < table_tokens) ? max_seq_len : table_tokens;
  const int64_t cap_pages = ceil_div(cap, page_size);
  int64_t ns;
  if (num_splits > 0) {
    ns = num_splits;
  } else if (num_splits < 0) {
    ns = 1;
  } else {
    if (num_cus <= 0) {
      const int st = query_num_cus(&num_cus);
      if (st != MX_STATUS_OK) return st;
    }
    ns = auto_splits(batch * num_kv_heads * row_tiles, num_cus * groups_per_cu(head_dim), cap);
  }
  if (ns > cap_pages) ns = cap_pages;
  if (ns < 1) ns = 1;
  int64_t pages_per_split = ceil_div(cap_pages, ns);
  ns = ceil_div(cap_pages, pages_per_split);  // page-aligned splits, none empty at capacity
  if (ns > kMaxGridDim) return fail(MX_STATUS_UNSUPPORTED, "split count exceeds 65535");

  plan->splits = ns;
  plan->tokens_per_split = pages_per_split * page_size;
  plan->cap_tokens = std::min<int64_t>(table_tokens, ns * plan->tokens_per_split);
  int shift = 0;
  while ((int64_t(kChunk) << shift) < page_size) ++shift;
  plan->chunk_shift = shift;
  const int64_t units = batch * num_kv_heads * row_tiles;
  const bool balanced_ok = batch <= kBalancedMaxBatch && units <= kBalancedMaxUnits &&
                           units * (ceil_div(cap, kChunk) * kChunkPositions + kMaxUnitOverhead) <
                               kBalancedMaxLine;
  // Short capacities favour one split per unit (no length scan, no merge): the balanced
  // schedule pays off from 2 048 tokens, or from 1 024 with at least 512 units.
  const bool long_enough = cap >= kBalancedMinCap || (cap >= kBalancedMinCap / 2 && units >= 512);
  const bool balanced_auto =
      num_splits == 0 && balanced_ok && units >= kBalancedMinUnits && long_enough;
  if ((num_splits < 0 && balanced_ok) || balanced_auto) {
    // Length-balanced single launch (automatic, or num_splits < 0 = that many workgroups).
    int64_t groups;
    if (num_splits < 0) {
      groups = -num_splits;
    } else {
      if (num_cus <= 0) {
        const int st = query_num_cus(&num_cus);
        if (st != MX_STATUS_OK) return st;
      }
      groups = num_cus * groups_per_cu(head_dim);
    }
    if (groups > kBalancedMaxGroups) groups = kBalancedMaxGroups;
    plan->schedule = MX_SCHEDULE_BALANCED;
    plan->splits = 0;
    plan->tokens_per_split = 0;
    plan->groups = groups;
    int64_t line_units = units;
    int64_t slot_rows = tile_rows;
    // Paired heads (MX_SCHEDULE_BALANCED_PAIRED): interleaved A/B against one head per unit,
    // sweep B=32 16K 331.9 against 344.9 us, B=128 16K 1294.5 against 1307.6, group 1 on config
    // 2's bytes 164.8 against 167.6, config 2 159.2/165.9 against 161.0/165.9 (two runs);
    // ragged lengths with 8 KV heads (B=256, G=4, P=64) 143.0 against 148.5.  With 4 KV heads
    // (1 KB token rows) pairing gained nothing (ragged P=16 82.2 against 81.9, uniform 165.4
    // against 165.9) or lost (config 4, P=64: 84.3 against 80.1), so it needs 2 KB token rows.
    const bool narrow_pairs =
        pair_ok == kPairFp8 && num_kv_heads >= 4 && num_kv_heads % 2 == 0 &&
        pair_heads(true, num_splits, head_dim, 2 * num_kv_heads, rows) && units / 2 >= groups;
    const bool mirrored =
        mirrored_pairs(pair_ok, num_splits, head_dim, num_kv_heads, rows, units, groups);
    if (pair_heads(pair_ok != kPairNone, num_splits, head_dim, num_kv_heads, rows) ||
        narrow_pairs || mirrored) {
      plan->schedule = MX_SCHEDULE_BALANCED_PAIRED;
      plan->pair_mirror = mirrored;
      plan->rows = 2 * rows;
      line_units = units / 2;
      slot_rows = 2 * rows;
    }
    plan->slots = groups + line_units;
    plan->cap_tokens = cap;
    plan->counter_offset = kStatusBytes + kXcdMaskBytes;
    plan->lse_offset = kPartialBase;
    plan->o_offset = plan->lse_offset + align_up(plan->slots * slot_rows * 4, 256);
    plan->workspace_bytes = plan->o_offset + plan->slots * slot_rows * head_dim * 4;
    return MX_STATUS_OK;
  }
  if (num_splits < 0)
    return fail(MX_STATUS_UNSUPPORTED,
                "the balanced schedule supports batch <= 512, batch * num_kv_heads * row "
                "groups <= 8192 and fewer than 2^30 chunks of capacity over all units");
  // Paired heads (MX_SCHEDULE_SPLIT_GRID_PAIRED, mx_paged_decode_splitkv with kPairW): units of
  // two adjacent KV heads, streamed two waves per head, when the split grid runs automatically
  // and each workgroup still streams >= kPairMinTokensPerSplit tokens.  A workgroup streaming one
  // 256-byte head row per token reads rows at some offsets of the 2 KB token row more slowly
  // than others while every head streams: on long B=4 at 128K the heads' workgroups ended
  // 267-332 us apart, paired 290-303 us.  Interleaved A/B against one head per workgroup: long
  // B=4 128K 329.7 against 349.1 us, B=1 128K 91.5 against 94.5, B=4 32K 90.5 against 92.5.
  // Shorter splits lose: B=1 at 32K (512 tokens per paired split) 31.1 against 30.0 us, where
  // the tree's partials of 16 rows lengthen the merge tail (with XCD-stable positions: 29.1
  // against 27.8 us); at 928 tokens (contest case 13, B=1, 58 976 tokens) pairs win, 43.2
  // against 44.3 us.
  if (pair_heads(pair_ok != kPairNone, num_splits, head_dim, num_kv_heads, rows)) {
    int64_t ns2 = auto_splits(batch * (num_kv_heads / 2), num_cus * groups_per_cu(head_dim), cap);
    if (ns2 > cap_pages) ns2 = cap_pages;
    if (ns2 < 1) ns2 = 1;
    const int64_t pages2 = ceil_div(cap_pages, ns2);
    ns2 = ceil_div(cap_pages, pages2);
    if (ns2 > 1 && pages2 * page_size >= kPairMinTokensPerSplit) {
      plan->schedule = MX_SCHEDULE_SPLIT_GRID_PAIRED;
      ns = ns2;
      pages_per_split = pages2;
      plan->splits = ns;
      plan->tokens_per_split = pages_per_split * page_size;
      plan->cap_tokens = std::min<int64_t>(table_tokens, ns * plan->tokens_per_split);
      plan->rows = 2 * rows;
    }
  }
  if (ns > kMaxGridDim) return fail(MX_STATUS_UNSUPPORTED, "split count exceeds 65535");
  if (ns > 1) {
    const int64_t prow = batch * seqlen_q * num_heads * ns;
    plan->lse_offset = kPartialBase;
    plan->o_offset = kPartialBase + align_up(prow * 4, 256);
    plan->workspace_bytes = plan->o_offset + prow * head_dim * 4;
  } else {
    plan->lse_offset = plan->o_offset = 0;
    plan->workspace_bytes = kStatusBytes;
  }
  return MX_STATUS_OK;
}

// Library-owned workspace, one per device, grow-only (as submission_clean.cu:478-491).  A grown
// workspace never frees its predecessors: kernels still in flight, and HIP graphs captured with
// the old address, keep valid memory until the process ends.  Growth doubles the size, so the
// retired allocations add up to less than the current one (up to 1 GiB; past it growth is to
// the size needed).  A call that grows it starts a fresh device status word.
struct DeviceWorkspace {
  void* ptr = nullptr;
  int64_t bytes = 0;
  std::vector<void*> retired;
};
std::mutex g_ws_mu;
std::vector<DeviceWorkspace> g_ws;

int internal_workspace(int64_t need, hipStream_t stream, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MX_STATUS_HIP_ERROR, "hipGetDevice failed");
  }
  std::lock_guard<std::mutex> lock(g_ws_mu);
  if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1);
  DeviceWorkspace& ws = g_ws[dev];
  if (ws.ptr == nullptr || ws.bytes < need) {
    // Allocating (and clearing) cannot be captured into a graph.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (stream != nullptr && hipStreamIsCapturing(stream, &capture) != hipSuccess) {
      (void)hipGetLastError();
      return fail(MX_STATUS_HIP_ERROR, "hipStreamIsCapturing failed");
    }
    if (capture != hipStreamCaptureStatusNone)
      return fail(MX_STATUS_INVALID_ARGUMENT,
                  "the library's workspace must grow, which cannot happen under stream capture: "
                  "pass a workspace, or make one call of this shape before capturing");
    // Doubling keeps the retired allocations below the current one; past 1 GiB it stops, and a
    // failed doubled allocation is retried at exactly `need`.
    const int64_t grown = ws.bytes < (int64_t(1) << 30) ? 2 * ws.bytes : ws.bytes;
    int64_t bytes = std::max<int64_t>({need, grown, int64_t(1) << 20});
    void* p = nullptr;
    if (hipMalloc(&p, (size_t)bytes) != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      p = nullptr;
      if (bytes > need && hipMalloc(&p, (size_t)need) == hipSuccess && p != nullptr) {
        bytes = need;
      } else {
        (void)hipGetLastError();
        return fail(MX_STATUS_ALLOC_FAILED, "hipMalloc of the internal workspace failed");
      }
    }
    // status word and merge counters must start at zero
    if (hipMemset(p, 0, (size_t)std::min<int64_t>(bytes, kPartialBase)) != hipSuccess) {
      (void)hipGetLastError();
      (void)hipFree(p);
      return fail(MX_STATUS_HIP_ERROR, "hipMemset of the internal workspace failed");
    }
    if (ws.ptr != nullptr) ws.retired.push_back(ws.ptr);
    ws.ptr = p;
    ws.bytes = bytes;
  }
  *out = ws.ptr;
  return MX_STATUS_OK;
}

// How a decode launch finds the newest keys of each sequence (see MainShape::appended and
// MainShape::new_tokens).
struct AppendArgs {
  int appended = 0;    // already appended to the cache: seq_lens exclude them
  int new_tokens = 0;  // fused append: read from k_new / v_new and written to the cache
  const void* k_new = nullptr;
  const void* v_new = nullptr;
};

// Format of the K/V cache: bf16, or fp8 (OCP e4m3fn) whose K and V values are k_scale and
// v_scale times the stored ones.
struct KvFormat {
  bool fp8 = false;
  float k_scale = 1.0f;
  float v_scale = 1.0f;
};

// KV heads as the kernels see them.  Stored heads of dim 64 run in adjacent pairs as kernel heads
// of dim 128 (MainShape::pair_group) when a head's query rows fit one 16-row tile, so that a
// pair is still one pass over its K/V.  For fp8 caches this is what makes the reads whole: an
// fp8 row of 64 dims is half a 128-byte line, which the workgroups of the two unpaired heads
// each fetch in full (FETCH_SIZE read 2.0x the cache bytes).  bf16 caches are not paired: a bf16
// row of 64 dims is a whole line already, and pairing measured 171.1 -> 168.8 us on B=128,
// Hkv=4, L=8192, within the spread of repeated runs.
struct KernelHeads {
  int64_t kv_heads;
  int64_t head_dim;
  int pair_group;  // 0: heads as stored; else the stored heads' query group
};

KernelHeads kernel_heads(int64_t seqlen_q, int64_t num_heads, int64_t num_kv_heads,
                         int64_t head_dim, bool fp8) {
  const bool pair = fp8 && head_dim == 64 && num_kv_heads >= 2 &&
                    num_kv_heads % 2 == 0 && num_heads % num_kv_heads == 0 && seqlen_q >= 1 &&
                    seqlen_q <= 16 && seqlen_q * (num_heads / num_kv_heads) <= 16;
  if (!pair) return {num_kv_heads, head_dim, 0};
  return {num_kv_heads / 2, 128, (int)(num_heads / num_kv_heads)};
}

// Whether a decode may run KV heads in pairs (pair_heads): bf16 caches, and fp8 caches whose
// kernel heads are the stored heads (not the head_dim-64 pairs of kernel_heads), with or
// without a fused append.  Paired fp8, interleaved A/B against single heads on cold pools:
// config 2's shape 89.5 and 94.7 against 94.0 and 96.8 us, the B=32 16K sweep 182.4 against
// 199.7 us, long B=1 128K 54.1 against 55.0, long B=4 32K 53.6 against 53.2.
int pair_ok_for(bool fp8, const KernelHeads& kh) {
  return !fp8 ? kPairBf16 : (kh.pair_group == 0 ? kPairFp8 : kPairNone);
}

// Register ring depth of the fp8 kernels (an fp8 chunk takes half the registers of a bf16 one).
// (A/B on 512 MB fp8 caches, chunks per ring 2/3/4/6: D=64 173.6/174.7/183.0/186.2 us, D=128
// config-2 shape 95.8/93.2/95.7/96.4 us, D=256 1/2/3/6 chunks 94.5/93.3-96.7/94.9/104.1 us.)
template <int D>
constexpr int ring_depth_fp8() {
  return D == 64 ? 2 : (D == 128 ? 3 : 1);
}

template <int D, bool kCausal, int KT>
hipError_t launch(const Plan& plan, const void* q, const void* k, const void* v, void* out,
                  const int32_t* seq_lens, const int32_t* block_table, int64_t batch,
                  int64_t seqlen_q, int64_t num_heads, int64_t num_kv_heads, int64_t page_size,
                  int64_t num_pages, int64_t max_pages, float scale, char* ws, int32_t phase,
                  float* o_out, float* lse_out, const AppendArgs& app, const KvFormat& kv,
                  int pair_group, hipStream_t stream) {
  constexpr int kNW = waves_per_group<D>();
  constexpr int kNBUF = ring_depth<D>();
  constexpr int kNBUF8 = ring_depth_fp8<D>();
  MainShape sh;
  // Strides are the stored heads'; the paired schedules' kernel heads are pairs of them.
  const bool paired = plan.schedule == MX_SCHEDULE_SPLIT_GRID_PAIRED ||
                      plan.schedule == MX_SCHEDULE_BALANCED_PAIRED;
  const int64_t kernel_kv = plan_kv_heads(plan, num_kv_heads);
  sh.page_stride = page_size * num_kv_heads * D;
  sh.token_stride = (int)(num_kv_heads * D);
  sh.num_heads = (int)num_heads;
  sh.num_kv_heads = (int)kernel_kv;
  sh.group = (int)(num_heads / kernel_kv);
  sh.group_magic = sh.group == 1 ? 0u : (uint32_t)((1ull << 32) / (uint64_t)sh.group + 1);
  if (pair_group > 0 && D != 128) return hipErrorInvalidValue;
  sh.pair_group = pair_group;
  sh.seqlen_q = (int)seqlen_q;
  sh.causal = kCausal ? 1 : 0;
  sh.rows = (int)plan.rows;
  sh.row_tiles = (int)plan.row_tiles;
  sh.tile_rows = (int)std::min<int64_t>(plan.rows, 16 * KT);
  sh.batch = (int)batch;
  sh.max_pages = (int)max_pages;
  sh.num_pages = (num_pages > 0 && num_pages <= INT32_MAX) ? (int)num_pages : 0;
  sh.chunk_shift = plan.chunk_shift;
  sh.cap_tokens = (int)plan.cap_tokens;
  sh.scale_log2 = scale * 1.4426950408889634f * (kv.fp8 ? kv.k_scale : 1.0f);
  sh.v_scale = kv.fp8 ? kv.v_scale : 1.0f;
  sh.k_scale = kv.fp8 ? kv.k_scale : 1.0f;
  sh.num_splits = (int)plan.splits;
  sh.fused_combine = 0;
  sh.split_groups = 1;
  // Paired launches (balanced and split grid) take XCD-stable shares or grid positions
  // (xcd_slot) when their blocks of 8 workgroups fit the claim masks.
  sh.xcd_map =
      (plan.schedule == MX_SCHEDULE_BALANCED_PAIRED && plan.groups <= 8 * kXcdMaskWords) ||
      (plan.schedule == MX_SCHEDULE_SPLIT_GRID_PAIRED &&
       batch * kernel_kv * plan.row_tiles * plan.splits <= 8 * kXcdMaskWords) ||
      (plan.schedule == MX_SCHEDULE_BALANCED && D == 128 && seqlen_q > 1 && !kv.fp8 &&
       app.new_tokens == 0 && plan.groups <= 8 * kXcdMaskWords);
  sh.tokens_per_split = (int)plan.tokens_per_split;
  sh.num_groups = (int)plan.groups;
  // A paired unit's chunk holds two heads' rows: twice a single head's weight on the line.
  sh.chunk_weight = paired ? 2 * kChunkPositions : kChunkPositions;
  sh.unit_overhead = !kv.fp8          ? (plan.pair_mirror ? kMirroredPairOverhead : kUnitOverhead)
                     : paired && num_kv_heads * D < 1024 ? kFp8NarrowPairOverhead
                                                         : kFp8UnitOverhead;
  sh.pair_mirror = plan.pair_mirror ? 1 : 0;
  sh.num_slots = (int)plan.slots;
  sh.o_out = o_out;
  sh.lse_out = lse_out;
  sh.appended = app.appended;
  sh.new_tokens = app.new_tokens;
  sh.k_new = static_cast<const uint16_t*>(app.k_new);
  sh.v_new = static_cast<const uint16_t*>(app.v_new);
  // The cache is written (fused append) only through the entry that takes it as mutable.
  sh.k_dst = app.new_tokens > 0 ? static_cast<uint16_t*>(const_cast<void*>(k)) : nullptr;
  sh.v_dst = app.new_tokens > 0 ? static_cast<uint16_t*>(const_cast<void*>(v)) : nullptr;
  uint32_t* status = reinterpret_cast<uint32_t*>(ws);
  const bool append = app.new_tokens > 0;
  const uint16_t* q16 = static_cast<const uint16_t*>(q);
  const uint16_t* k16 = static_cast<const uint16_t*>(k);
  const uint16_t* v16 = static_cast<const uint16_t*>(v);
  const uint8_t* k8 = static_cast<const uint8_t*>(k);
  const uint8_t* v8 = static_cast<const uint8_t*>(v);

  if (plan.schedule == MX_SCHEDULE_BALANCED || plan.schedule == MX_SCHEDULE_BALANCED_PAIRED) {
    // One launch does everything; MX_PHASE_COMBINE_ONLY has nothing left to do.
    if (phase == MX_PHASE_COMBINE_ONLY) return hipSuccess;
    auto go = [&](auto kernel, auto kc, auto vc) {
      hipLaunchKernelGGL(kernel, dim3((unsigned)plan.groups), dim3(64 * kNW), 0, stream, q16, kc,
                         vc, static_cast<uint16_t*>(out), seq_lens, block_table,
                         reinterpret_cast<float*>(ws + plan.o_offset),
                         reinterpret_cast<float*>(ws + plan.lse_offset),
                         reinterpret_cast<uint32_t*>(ws + plan.counter_offset), status, sh);
    };
    if (paired) {
      // make_plan pairs only head_dim 128 with one tile.
      if constexpr (D == 128 && KT == 1) {
        if (kv.fp8 && append)
          go(mx_paged_decode_balanced<D, kNBUF8, kNW, kCausal, KT, true, true, true>, k8, v8);
        else if (kv.fp8)
          go(mx_paged_decode_balanced<D, kNBUF8, kNW, kCausal, KT, false, true, true>, k8, v8);
        else if (append)
          go(mx_paged_decode_balanced<D, kNBUF, kNW, kCausal, KT, true, false, true>, k16, v16);
        else
          go(mx_paged_decode_balanced<D, kNBUF, kNW, kCausal, KT, false, false, true>, k16, v16);
      } else {
        return hipErrorInvalidValue;
      }
    } else if (kv.fp8 && append)
      go(mx_paged_decode_balanced<D, kNBUF8, kNW, kCausal, KT, true, true>, k8, v8);
    else if (kv.fp8)
      go(mx_paged_decode_balanced<D, kNBUF8, kNW, kCausal, KT, false, true>, k8, v8);
    else if (append)
      go(mx_paged_decode_balanced<D, kNBUF, kNW, kCausal, KT, true, false>, k16, v16);
    else if (sh.xcd_map) {
      if constexpr (D == 128)
        go(mx_paged_decode_balanced<D, kNBUF, kNW, kCausal, KT, false, false, false, true>, k16,
           v16);
      else
        return hipErrorInvalidValue;
    } else
      go(mx_paged_decode_balanced<D, kNBUF, kNW, kCausal, KT, false, false>, k16, v16);
    return hipGetLastError();
  }

  float* part_lse = plan.splits > 1 ? reinterpret_cast<float*>(ws + plan.lse_offset) : nullptr;
  float* part_o = plan.splits > 1 ? reinterpret_cast<float*>(ws + plan.o_offset) : nullptr;
  // One launch (the splits of each unit merge through an in-kernel tree) when the units' arrival
  // counters fit the counter region and the caller did not ask for the two phases separately.
  const bool fused = phase == 0 && plan.splits > 1 &&
                     split_tree_fits(batch * kernel_kv * plan.row_tiles, plan.splits,
                                     plan.workspace_bytes - plan.o_offset);
  sh.split_groups = (int)ceil_div(plan.splits, kMergeFanIn);
  sh.fused_combine = fused ? 1 : 0;
  if (phase != MX_PHASE_COMBINE_ONLY) {
    const dim3 grid((unsigned)(kernel_kv * plan.row_tiles), (unsigned)batch,
                    (unsigned)plan.splits);
    auto go = [&](auto kernel, auto kc, auto vc) {
      hipLaunchKernelGGL(kernel, grid, dim3(64 * kNW), 0, stream, q16, kc, vc,
                         static_cast<uint16_t*>(out), seq_lens, block_table, part_o, part_lse,
                         reinterpret_cast<uint32_t*>(ws + kStatusBytes + kXcdMaskBytes), status,
                         sh);
    };
    if (paired) {
      // make_plan pairs only head_dim 128 with one tile.
      if constexpr (D == 128 && KT == 1) {
        if (kv.fp8 && append)
          go(mx_paged_decode_splitkv<D, kNBUF8, kNW, kCausal, KT, true, true, true>, k8, v8);
        else if (kv.fp8)
          go(mx_paged_decode_splitkv<D, kNBUF8, kNW, kCausal, KT, false, true, true>, k8, v8);
        else if (append)
          go(mx_paged_decode_splitkv<D, kNBUF, kNW, kCausal, KT, true, false, true>, k16, v16);
        else
          go(mx_paged_decode_splitkv<D, kNBUF, kNW, kCausal, KT, false, false, true>, k16, v16);
      } else {
        return hipErrorInvalidValue;
      }
    } else if (kv.fp8 && append)
      go(mx_paged_decode_splitkv<D, kNBUF8, kNW, kCausal, KT, true, true>, k8, v8);
    else if (kv.fp8)
      go(mx_paged_decode_splitkv<D, kNBUF8, kNW, kCausal, KT, false, true>, k8, v8);
    else if (append)
      go(mx_paged_decode_splitkv<D, kNBUF, kNW, kCausal, KT, true, false>, k16, v16);
    else
      go(mx_paged_decode_splitkv<D, kNBUF, kNW, kCausal, KT, false, false>, k16, v16);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (phase != MX_PHASE_MAIN_ONLY && plan.splits > 1 && !fused) {
    const dim3 grid((unsigned)num_heads, (unsigned)(batch * seqlen_q));
    hipLaunchKernelGGL(mx_paged_decode_combine<D>, grid, dim3(64), 0, stream, part_o, part_lse,
                       seq_lens, static_cast<uint16_t*>(out), o_out, lse_out, (int)num_heads,
                       (int)seqlen_q, (int)plan.splits, (int)plan.tokens_per_split,
                       (int)plan.cap_tokens, app.appended, app.new_tokens, pair_group);
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

// The plan of a bf16 (fp8 = false) or fp8 cache call.
static int report_plan(bool fp8, int64_t batch, int64_t seqlen_q, int64_t num_heads,
                       int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                       int64_t max_pages_per_seq, int64_t max_seq_len, int64_t num_splits,
                       int64_t num_cus, int64_t* schedule_out, int64_t* splits_out,
                       int64_t* tokens_per_split_out, int64_t* workgroups_out,
                       int64_t* workspace_bytes_out) {
  Plan plan;
  const KernelHeads kh = kernel_heads(seqlen_q, num_heads, num_kv_heads, head_dim, fp8);
  const int st = make_plan(batch, seqlen_q, num_heads, kh.kv_heads, kh.head_dim, page_size,
                           max_pages_per_seq, max_seq_len, num_splits, num_cus,
                           pair_ok_for(fp8, kh), &plan);
  if (st != MX_STATUS_OK) return st;
  if (schedule_out) *schedule_out = plan.schedule;
  if (splits_out) *splits_out = plan.splits;
  if (tokens_per_split_out) *tokens_per_split_out = plan.tokens_per_split;
  if (workgroups_out)
    *workgroups_out = (plan.schedule == MX_SCHEDULE_BALANCED ||
                       plan.schedule == MX_SCHEDULE_BALANCED_PAIRED)
                          ? plan.groups
                          : batch * plan_kv_heads(plan, kh.kv_heads) * plan.row_tiles * plan.splits;
  if (workspace_bytes_out) *workspace_bytes_out = plan.workspace_bytes;
  return ok();
}

int mx_paged_gqa_decode_plan(int64_t batch, int64_t seqlen_q, int64_t num_heads,
                             int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                             int64_t max_pages_per_seq, int64_t max_seq_len, int64_t num_splits,
                             int64_t num_cus, int64_t* schedule_out, int64_t* splits_out,
                             int64_t* tokens_per_split_out, int64_t* workgroups_out,
                             int64_t* workspace_bytes_out) {
  return report_plan(false, batch, seqlen_q, num_heads, num_kv_heads, head_dim, page_size,
                     max_pages_per_seq, max_seq_len, num_splits, num_cus, schedule_out,
                     splits_out, tokens_per_split_out, workgroups_out, workspace_bytes_out);
}

int mx_paged_gqa_decode_plan_fp8kv(int64_t batch, int64_t seqlen_q, int64_t num_heads,
                                   int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                   int64_t max_pages_per_seq, int64_t max_seq_len,
                                   int64_t num_splits, int64_t num_cus, int64_t* schedule_out,
                                   int64_t* splits_out, int64_t* tokens_per_split_out,
                                   int64_t* workgroups_out, int64_t* workspace_bytes_out) {
  return report_plan(true, batch, seqlen_q, num_heads, num_kv_heads, head_dim, page_size,
                     max_pages_per_seq, max_seq_len, num_splits, num_cus, schedule_out,
                     splits_out, tokens_per_split_out, workgroups_out, workspace_bytes_out);
}

int64_t mx_paged_gqa_decode_workspace_size(int64_t batch, int64_t seqlen_q, int64_t num_heads,
                                           int64_t num_kv_heads, int64_t head_dim,
                                           int64_t page_size, int64_t max_pages_per_seq,
                                           int64_t max_seq_len, int64_t num_splits) {
  // The size covers the call on a bf16 and on an fp8 cache (whose kernel heads may differ).
  int64_t bytes = 0;
  for (const bool fp8 : {false, true}) {
    Plan plan;
    const KernelHeads kh = kernel_heads(seqlen_q, num_heads, num_kv_heads, head_dim, fp8);
    const int st = make_plan(batch, seqlen_q, num_heads, kh.kv_heads, kh.head_dim, page_size,
                             max_pages_per_seq, max_seq_len, num_splits, 0, pair_ok_for(fp8, kh),
                             &plan);
    if (st != MX_STATUS_OK) return st;
    bytes = std::max(bytes, plan.workspace_bytes);
  }
  ok();
  return bytes;
}

}  // extern "C"

namespace {

// Argument checks, plan and workspace of a decode call; launches nothing.
int prepare_decode(const void* q, const void* k_cache, const void* v_cache, const void* out,
                   int64_t batch, int64_t seqlen_q, int64_t num_heads, int64_t num_kv_heads,
                   int64_t head_dim, int64_t page_size, int64_t num_pages,
                   int64_t max_pages_per_seq, int64_t max_seq_len, int32_t causal, float scale,
                   int64_t num_splits, void** workspace, int64_t workspace_bytes,
                   int32_t phase, void* stream, int pair_ok, Plan* plan) {
  if (phase != 0 && phase != MX_PHASE_MAIN_ONLY && phase != MX_PHASE_COMBINE_ONLY)
    return fail(MX_STATUS_INVALID_ARGUMENT, "phase must be 0, 1 or 2");
  // The kernels read q, K and V rows as 16-byte vectors and write out in 8-byte pieces.
  for (const void* p : {q, k_cache, v_cache})
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return fail(MX_STATUS_INVALID_ARGUMENT, "q, k_cache and v_cache must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(out) % 8 != 0)
    return fail(MX_STATUS_INVALID_ARGUMENT, "out must be 8-byte aligned");
  if (causal != 0 && causal != 1) return fail(MX_STATUS_INVALID_ARGUMENT, "causal must be 0 or 1");
  if (!std::isfinite(scale)) return fail(MX_STATUS_INVALID_ARGUMENT, "scale must be finite");
  if (num_pages < 0) return fail(MX_STATUS_INVALID_SHAPE, "num_pages must be >= 0");
  int st = make_plan(batch, seqlen_q, num_heads, num_kv_heads, head_dim, page_size,
                     max_pages_per_seq, max_seq_len, num_splits, 0, pair_ok, plan);
  if (st != MX_STATUS_OK) return st;
  if (*workspace != nullptr) {
    if (workspace_bytes < plan->workspace_bytes)
      return fail(MX_STATUS_WORKSPACE_TOO_SMALL,
                  "workspace_bytes " + std::to_string(workspace_bytes) + " < required " +
                      std::to_string(plan->workspace_bytes));
    return MX_STATUS_OK;
  }
  return internal_workspace(plan->workspace_bytes, static_cast<hipStream_t>(stream), workspace);
}

// Launches a prepared decode: bf16 into out, or (partial outputs) fp32 rows into o_out and
// natural-log sum-exps into lse_out (out is then null).  `app`: see AppendArgs.
int run_decode(const Plan& plan, const void* q, const void* k_cache, const void* v_cache,
               void* out, float* o_out, float* lse_out, const int32_t* seq_lens,
               const int32_t* block_table, int64_t batch, int64_t seqlen_q, int64_t num_heads,
               int64_t num_kv_heads, int64_t head_dim, int64_t page_size, int64_t num_pages,
               int64_t max_pages_per_seq, int32_t causal, float scale, void* workspace,
               int32_t phase, const AppendArgs& app, void* stream,
               const KvFormat& kv = KvFormat{}, int pair_group = 0) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  hipError_t e;
  // A causal mask changes nothing for a single query token (it sees every key).
  const bool masked = causal != 0 && seqlen_q > 1;
#define MX_LAUNCH(DIM, CAUSAL, KT)                                                            \
  launch<DIM, CAUSAL, KT>(plan, q, k_cache, v_cache, out, seq_lens, block_table, batch, seqlen_q, \
                      num_heads, num_kv_heads, page_size, num_pages, max_pages_per_seq, scale, \
                      ws, phase, o_out, lse_out, app, kv, pair_group, s)
  const bool pair = plan.tiles_per_group == 2;
  switch (head_dim) {
    case 64:
      e = pair ? (masked ? MX_LAUNCH(64, true, 2) : MX_LAUNCH(64, false, 2))
               : (masked ? MX_LAUNCH(64, true, 1) : MX_LAUNCH(64, false, 1));
      break;
    case 128:
      e = pair ? (masked ? MX_LAUNCH(128, true, 2) : MX_LAUNCH(128, false, 2))
               : (masked ? MX_LAUNCH(128, true, 1) : MX_LAUNCH(128, false, 1));
      break;
    default:  // head_dim 256: single tiles only
      e = masked ? MX_LAUNCH(256, true, 1) : MX_LAUNCH(256, false, 1);
      break;
  }
#undef MX_LAUNCH
  if (e != hipSuccess)
    return fail(MX_STATUS_HIP_ERROR, std::string("kernel launch failed: ") + hipGetErrorString(e));
  return ok();
}

// Shared by mx_paged_gqa_decode (bf16 into out) and mx_paged_gqa_decode_partial (fp32 rows into
// o_out and natural-log sum-exps into lse_out; out is then null).
int decode_impl(const void* q, const void* k_cache, const void* v_cache, void* out, float* o_out,
                float* lse_out, const int32_t* seq_lens, const int32_t* block_table,
                int64_t batch, int64_t seqlen_q, int64_t num_heads, int64_t num_kv_heads,
                int64_t head_dim, int64_t page_size, int64_t num_pages, int64_t max_pages_per_seq,
                int64_t max_seq_len, int32_t causal, float scale, int64_t num_splits,
                void* workspace, int64_t workspace_bytes, int32_t phase, void* stream,
                const KvFormat& kv = KvFormat{}) {
  Plan plan;
  const KernelHeads kh = kernel_heads(seqlen_q, num_heads, num_kv_heads, head_dim, kv.fp8);
  const int st = prepare_decode(q, k_cache, v_cache, out, batch, seqlen_q, num_heads,
                                kh.kv_heads, kh.head_dim, page_size, num_pages, max_pages_per_seq,
                                max_seq_len, causal, scale, num_splits, &workspace,
                                workspace_bytes, phase, stream, pair_ok_for(kv.fp8, kh),
                                &plan);
  if (st != MX_STATUS_OK) return st;
  return run_decode(plan, q, k_cache, v_cache, out, o_out, lse_out, seq_lens, block_table, batch,
                    seqlen_q, num_heads, kh.kv_heads, kh.head_dim, page_size, num_pages,
                    max_pages_per_seq, causal, scale, workspace, phase, AppendArgs{}, stream, kv,
                    kh.pair_group);
}

// Argument checks of a paged K/V append (shared by mx_paged_kv_append and the fused
// append-and-attend entry); launches nothing.
int check_append(const void* k_new, const void* v_new, const void* k_cache, const void* v_cache,
                 const int32_t* seq_lens, const int32_t* block_table, int64_t batch,
                 int64_t seqlen_new, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                 int64_t num_pages, int64_t max_pages_per_seq) {
  // k_new / v_new may be NULL (an empty tensor) only when there is nothing to append.
  if ((seqlen_new > 0 && (!k_new || !v_new)) || !k_cache || !v_cache || !seq_lens ||
      !block_table)
    return fail(MX_STATUS_NULL_POINTER,
                "k_new, v_new, k_cache, v_cache, seq_lens and block_table must be non-NULL");
  for (const void* p : {k_new, v_new, k_cache, v_cache})
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return fail(MX_STATUS_INVALID_ARGUMENT, "K/V tensors must be 16-byte aligned");
  if (batch < 1 || seqlen_new < 0 || num_kv_heads < 1 || head_dim < 1 || page_size < 1 ||
      max_pages_per_seq < 1)
    return fail(MX_STATUS_INVALID_SHAPE,
                "batch, num_kv_heads, head_dim, page_size and max_pages_per_seq must be >= 1 "
                "and seqlen_new >= 0");
  if (num_pages < 1)
    return fail(MX_STATUS_INVALID_SHAPE,
                "num_pages (the pool size) must be >= 1: it bounds every write");
  if (head_dim % 8 != 0) return fail(MX_STATUS_UNSUPPORTED, "head_dim must be a multiple of 8");
  if (max_pages_per_seq > (int64_t)INT32_MAX / page_size || num_pages > INT32_MAX ||
      num_kv_heads * head_dim > INT32_MAX / 8 ||
      batch * seqlen_new > (int64_t)INT32_MAX / 2 - 4)
    return fail(MX_STATUS_UNSUPPORTED, "sizes must fit 32-bit indices");
  return MX_STATUS_OK;
}

int launch_append(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                  const int32_t* seq_lens, const int32_t* block_table, int64_t batch,
                  int64_t seqlen_new, int64_t num_kv_heads, int64_t head_dim,
                  int64_t page_size, int64_t num_pages, int64_t max_pages_per_seq,
                  void* workspace, void* stream, const KvFormat& kv = KvFormat{}) {
  const int64_t waves = 2 * batch * seqlen_new;
  if (kv.fp8)
    hipLaunchKernelGGL(mx_paged_kv_append_fp8_kernel, dim3((unsigned)ceil_div(waves, 4)),
                       dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(k_new), static_cast<const uint16_t*>(v_new),
                       static_cast<uint8_t*>(k_cache), static_cast<uint8_t*>(v_cache), seq_lens,
                       block_table, (int)batch, (int)seqlen_new,
                       (int)(num_kv_heads * head_dim / 8), (int)page_size, (int)num_pages,
                       (int)max_pages_per_seq, kv.k_scale, kv.v_scale,
                       static_cast<uint32_t*>(workspace));
  else
    hipLaunchKernelGGL(mx_paged_kv_append_kernel, dim3((unsigned)ceil_div(waves, 4)), dim3(256),
                       0, static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(k_new),
                       static_cast<const uint16_t*>(v_new), static_cast<uint16_t*>(k_cache),
                       static_cast<uint16_t*>(v_cache), seq_lens, block_table, (int)batch,
                       (int)seqlen_new, (int)(num_kv_heads * head_dim / 8), (int)page_size,
                       (int)num_pages, (int)max_pages_per_seq, static_cast<uint32_t*>(workspace));
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(MX_STATUS_HIP_ERROR, std::string("kernel launch failed: ") + hipGetErrorString(e));
  return ok();
}

// ------------------------------------------------------------------------------------------
// Workspace of the allocation-free entry point (mx_paged_gqa_decode_noalloc)
// ------------------------------------------------------------------------------------------

// Clears n words at p (a kernel rather than hipMemsetAsync, which a stream capture would record
// as a memset node).
__global__ __launch_bounds__(256) void mx_zero_words(uint32_t* __restrict__ p, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0u;
}

}  // namespace

// The workspace of every mx_paged_gqa_decode_noalloc call on a device: a file-scope device array
// that the HIP runtime places on each device when the library's code is loaded there, held until
// the process ends.  Host code never uses this name as an address (on the host it is only a
// stand-in): scratch_address() looks up each device's own copy.
static __device__ __align__(256) char scratch[MX_NOALLOC_SCRATCH_BYTES];

namespace {

struct ScratchState {
  void* ptr = nullptr;  // this device's copy of `scratch`
  bool cleared = false;  // status word and merge counters zeroed by a launch on some stream
};
std::mutex g_scratch_mu;
std::vector<ScratchState> g_scratch;

// This device's copy of `scratch`, found with hipGetSymbolAddress on the device's first call.
// The first call also launches a clear of the status word and the merge counters on `stream`,
// ahead of its decode (the kernels leave the counters at zero after every call).
int scratch_address(hipStream_t stream, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MX_STATUS_HIP_ERROR, "hipGetDevice failed");
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if ((int)g_scratch.size() <= dev) g_scratch.resize(dev + 1);
  ScratchState& sc = g_scratch[dev];
  if (sc.ptr == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      return fail(MX_STATUS_HIP_ERROR, "hipGetSymbolAddress of the no-alloc scratch failed");
    }
    sc.ptr = p;
  }
  if (!sc.cleared) {
    constexpr int kWords = (int)(kPartialBase / 4);
    hipLaunchKernelGGL(mx_zero_words, dim3((kWords + 255) / 256), dim3(256), 0, stream,
                       static_cast<uint32_t*>(sc.ptr), kWords);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      return fail(MX_STATUS_HIP_ERROR, std::string("clearing the no-alloc scratch failed: ") +
                                           hipGetErrorString(e));
    sc.cleared = true;
  }
  *out = sc.ptr;
  return MX_STATUS_OK;
}

}  // namespace

extern "C" {

int mx_paged_gqa_decode(const void* q, const void* k_cache, const void* v_cache, void* out,
                        const int32_t* seq_lens, const int32_t* block_table, int64_t batch,
                        int64_t seqlen_q, int64_t num_heads, int64_t num_kv_heads,
                        int64_t head_dim, int64_t page_size, int64_t num_pages,
                        int64_t max_pages_per_seq, int64_t max_seq_len, int32_t causal,
                        float scale, int64_t num_splits, void* workspace, int64_t workspace_bytes,
                        int32_t phase, void* stream) {
  if (!q || !k_cache || !v_cache || !out || !seq_lens || !block_table)
    return fail(MX_STATUS_NULL_POINTER,
                "q, k_cache, v_cache, out, seq_lens and block_table must be non-NULL");
  return decode_impl(q, k_cache, v_cache, out, nullptr, nullptr, seq_lens, block_table, batch,
                     seqlen_q, num_heads, num_kv_heads, head_dim, page_size, num_pages,
                     max_pages_per_seq, max_seq_len, causal, scale, num_splits, workspace,
                     workspace_bytes, phase, stream);
}

int mx_paged_gqa_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                void* out, const int32_t* seq_lens, const int32_t* block_table,
                                int64_t batch, int64_t seqlen_q, int64_t num_heads,
                                int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                int64_t num_pages, int64_t max_pages_per_seq,
                                int64_t max_seq_len, int32_t causal, float scale,
                                int64_t num_splits, void* stream) {
  if (!q || !k_cache || !v_cache || !out || !seq_lens || !block_table)
    return fail(MX_STATUS_NULL_POINTER,
                "q, k_cache, v_cache, out, seq_lens and block_table must be non-NULL");
  // The size check comes first, so a call that cannot run changes nothing on the device.  It
  // sizes the bf16 plan that decode_impl runs (not mx_paged_gqa_decode_workspace_size, which
  // also covers the fp8 plan's kernel heads and can be twice as large at head_dim 64).
  int64_t need = 0;
  const int pst = report_plan(false, batch, seqlen_q, num_heads, num_kv_heads, head_dim,
                              page_size, max_pages_per_seq, max_seq_len, num_splits, 0, nullptr,
                              nullptr, nullptr, nullptr, &need);
  if (pst != MX_STATUS_OK) return pst;
  if (need > MX_NOALLOC_SCRATCH_BYTES)
    return fail(MX_STATUS_UNSUPPORTED,
                "this call needs " + std::to_string(need) +
                    " bytes of workspace, more than the no-alloc scratch holds (" +
                    std::to_string((int64_t)MX_NOALLOC_SCRATCH_BYTES) +
                    "): call mx_paged_gqa_decode with a workspace instead");
  void* ws = nullptr;
  const int st = scratch_address(static_cast<hipStream_t>(stream), &ws);
  if (st != MX_STATUS_OK) return st;
  return decode_impl(q, k_cache, v_cache, out, nullptr, nullptr, seq_lens, block_table, batch,
                     seqlen_q, num_heads, num_kv_heads, head_dim, page_size, num_pages,
                     max_pages_per_seq, max_seq_len, causal, scale, num_splits, ws,
                     MX_NOALLOC_SCRATCH_BYTES, 0, stream);
}

int mx_paged_gqa_decode_fp8kv(const void* q, const void* k_cache, const void* v_cache,
                              void* out, const int32_t* seq_lens, const int32_t* block_table,
                              int64_t batch, int64_t seqlen_q, int64_t num_heads,
                              int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                              int64_t num_pages, int64_t max_pages_per_seq, int64_t max_seq_len,
                              int32_t causal, float scale, float k_scale, float v_scale,
                              int64_t num_splits, void* workspace, int64_t workspace_bytes,
                              int32_t phase, void* stream) {
  if (!q || !k_cache || !v_cache || !out || !seq_lens || !block_table)
    return fail(MX_STATUS_NULL_POINTER,
                "q, k_cache, v_cache, out, seq_lens and block_table must be non-NULL");
  if (!std::isfinite(k_scale) || !std::isfinite(v_scale))
    return fail(MX_STATUS_INVALID_ARGUMENT, "k_scale and v_scale must be finite");
  if (!std::isfinite(scale * k_scale))
    return fail(MX_STATUS_INVALID_ARGUMENT, "scale * k_scale must be finite");
  KvFormat kv;
  kv.fp8 = true;
  kv.k_scale = k_scale;
  kv.v_scale = v_scale;
  return decode_impl(q, k_cache, v_cache, out, nullptr, nullptr, seq_lens, block_table, batch,
                     seqlen_q, num_heads, num_kv_heads, head_dim, page_size, num_pages,
                     max_pages_per_seq, max_seq_len, causal, scale, num_splits, workspace,
                     workspace_bytes, phase, stream, kv);
}

int mx_paged_gqa_decode_partial(const void* q, const void* k_cache, const void* v_cache,
                                float* o_partial, float* lse_partial, const int32_t* seq_lens,
                                const int32_t* block_table, int64_t batch, int64_t seqlen_q,
                                int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                int64_t page_size, int64_t num_pages, int64_t max_pages_per_seq,
                                int64_t max_seq_len, int32_t causal, float scale,
                                int64_t num_splits, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  if (!q || !k_cache || !v_cache || !o_partial || !lse_partial || !seq_lens || !block_table)
    return fail(MX_STATUS_NULL_POINTER,
                "q, k_cache, v_cache, o_partial, lse_partial, seq_lens and block_table must be "
                "non-NULL");
  if (reinterpret_cast<uintptr_t>(o_partial) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(lse_partial) % 4 != 0)
    return fail(MX_STATUS_INVALID_ARGUMENT,
                "o_partial must be 16-byte aligned and lse_partial 4-byte aligned");
  return decode_impl(q, k_cache, v_cache, nullptr, o_partial, lse_partial, seq_lens,
                     block_table, batch, seqlen_q, num_heads, num_kv_heads, head_dim, page_size,
                     num_pages, max_pages_per_seq, max_seq_len, causal, scale, num_splits,
                     workspace, workspace_bytes, 0, stream);
}

int mx_lse_merge(const float* o_parts, const float* lse_parts, int64_t num_parts, int64_t rows,
                 int64_t head_dim, void* out, void* stream) {
  if (!o_parts || !lse_parts || !out)
    return fail(MX_STATUS_NULL_POINTER, "o_parts, lse_parts and out must be non-NULL");
  if (num_parts < 1 || rows < 0)
    return fail(MX_STATUS_INVALID_SHAPE, "num_parts must be >= 1 and rows >= 0");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(MX_STATUS_UNSUPPORTED, "head_dim must be 64, 128 or 256");
  if (reinterpret_cast<uintptr_t>(o_parts) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(lse_parts) % 4 != 0 ||
      reinterpret_cast<uintptr_t>(out) % 8 != 0)
    return fail(MX_STATUS_INVALID_ARGUMENT,
                "o_parts must be 16-byte, lse_parts 4-byte and out 8-byte aligned");
  if (rows > kMaxMergeRows || num_parts > INT32_MAX)
    return fail(MX_STATUS_UNSUPPORTED, "rows must be <= 2^25 and num_parts < 2^31");
  if (rows == 0) return ok();
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)rows);
  uint16_t* o = static_cast<uint16_t*>(out);
  switch (head_dim) {
    case 64:
      hipLaunchKernelGGL(mx_lse_merge_kernel<64>, grid, dim3(64), 0, s, o_parts, lse_parts, rows,
                         (int)num_parts, o);
      break;
    case 128:
      hipLaunchKernelGGL(mx_lse_merge_kernel<128>, grid, dim3(64), 0, s, o_parts, lse_parts,
                         rows, (int)num_parts, o);
      break;
    default:
      hipLaunchKernelGGL(mx_lse_merge_kernel<256>, grid, dim3(64), 0, s, o_parts, lse_parts,
                         rows, (int)num_parts, o);
      break;
  }
  const hipError_t e = hipGetLastError();
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
  if (seqlen_q < 1) {
    st = fail(MX_STATUS_INVALID_SHAPE, "run_kernel: seqlen_q must be >= 1");
  } else if (causal != 0 && causal != 1) {
    st = fail(MX_STATUS_INVALID_ARGUMENT, "run_kernel: causal must be 0 or 1");
  } else if (batch_size < 1 || num_blocks < batch_size || num_blocks % batch_size != 0) {
    st = fail(MX_STATUS_INVALID_SHAPE,
              "run_kernel: num_blocks must be a positive multiple of batch_size");
  } else if (seqlen_k < 1) {
    st = fail(MX_STATUS_INVALID_SHAPE, "run_kernel: seqlen_k must be >= 1");
  } else if (headdim < 1) {
    st = fail(MX_STATUS_INVALID_SHAPE, "run_kernel: headdim must be >= 1");
  } else {
    const float scale = 1.0f / sqrtf((float)headdim);
    // num_blocks is both the pool size (k_cache_paged holds num_blocks pages, task.md:57-58)
    // and the table's size (num_blocks / batch_size entries per row, task.md:61): page ids
    // outside [0, num_blocks) are flagged and read as page 0.
    st = mx_paged_gqa_decode(q, k_cache_paged, v_cache_paged, output, cache_seqlens,
                             block_table, batch_size, seqlen_q, num_heads, num_heads_k, headdim,
                             page_block_size, num_blocks, num_blocks / batch_size, seqlen_k,
                             (int32_t)causal, scale, 0, nullptr, 0, 0, nullptr);
  }
  if (st != MX_STATUS_OK) fprintf(stderr, "run_kernel: %s\n", g_last_error.c_str());
}

int mx_read_device_status(void* workspace, int32_t reset, void* stream, int32_t* flags_out) {
  if (!flags_out) return fail(MX_STATUS_NULL_POINTER, "flags_out must be non-NULL");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (workspace == MX_NOALLOC_WORKSPACE) {
    // The no-alloc array of this device (cleared on its first use, which may be this one).
    int st = scratch_address(s, &workspace);
    if (st != MX_STATUS_OK) return st;
  } else if (workspace == nullptr) {
    int st = internal_workspace(kStatusBytes, s, &workspace);
    if (st != MX_STATUS_OK) return st;
  }
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

// Shared by mx_paged_kv_append and mx_paged_kv_append_fp8kv.
static int kv_append_impl(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                          const int32_t* seq_lens, const int32_t* block_table, int64_t batch,
                          int64_t seqlen_new, int64_t num_kv_heads, int64_t head_dim,
                          int64_t page_size, int64_t num_pages, int64_t max_pages_per_seq,
                          void* workspace, void* stream, const KvFormat& kv) {
  int st = check_append(k_new, v_new, k_cache, v_cache, seq_lens, block_table, batch, seqlen_new,
                        num_kv_heads, head_dim, page_size, num_pages, max_pages_per_seq);
  if (st != MX_STATUS_OK) return st;
  if (seqlen_new == 0) return ok();
  if (workspace == nullptr) {
    st = internal_workspace(kStatusBytes, static_cast<hipStream_t>(stream), &workspace);
    if (st != MX_STATUS_OK) return st;
  }
  return launch_append(k_new, v_new, k_cache, v_cache, seq_lens, block_table, batch, seqlen_new,
                       num_kv_heads, head_dim, page_size, num_pages, max_pages_per_seq,
                       workspace, stream, kv);
}

// Shared by mx_paged_gqa_decode_append and mx_paged_gqa_decode_append_fp8kv.
static int decode_append_impl(const void* q, const void* k_new, const void* v_new,
                              void* k_cache, void* v_cache, void* out, const int32_t* seq_lens,
                              const int32_t* block_table, int64_t batch, int64_t seqlen_q,
                              int64_t seqlen_new, int64_t num_heads, int64_t num_kv_heads,
                              int64_t head_dim, int64_t page_size, int64_t num_pages,
                              int64_t max_pages_per_seq, int64_t max_seq_len, int32_t causal,
                              float scale, int64_t num_splits, void* workspace,
                              int64_t workspace_bytes, void* stream, const KvFormat& kv) {
  if (!q || !out)
    return fail(MX_STATUS_NULL_POINTER, "q and out must be non-NULL");
  int st = check_append(k_new, v_new, k_cache, v_cache, seq_lens, block_table, batch, seqlen_new,
                        num_kv_heads, head_dim, page_size, num_pages, max_pages_per_seq);
  if (st != MX_STATUS_OK) return st;
  if (seqlen_new > INT32_MAX / 2)
    return fail(MX_STATUS_UNSUPPORTED, "seqlen_new must be < 2^30");
  Plan plan;
  const KernelHeads kh = kernel_heads(seqlen_q, num_heads, num_kv_heads, head_dim, kv.fp8);
  st = prepare_decode(q, k_cache, v_cache, out, batch, seqlen_q, num_heads, kh.kv_heads,
                      kh.head_dim, page_size, num_pages, max_pages_per_seq, max_seq_len, causal,
                      scale, num_splits, &workspace, workspace_bytes, 0, stream,
                      pair_ok_for(kv.fp8, kh), &plan);
  if (st != MX_STATUS_OK) return st;
  AppendArgs app;
  if (seqlen_new >= 1 && seqlen_new <= kChunk) {
    // One launch: the new keys are one extra chunk of each unit, written to the cache by the
    // wave that loads them.
    app.new_tokens = (int)seqlen_new;
    app.k_new = k_new;
    app.v_new = v_new;
  } else if (seqlen_new > 0) {
    // Longer appends: the append kernel first, then the decode over seq_lens + seqlen_new.
    st = launch_append(k_new, v_new, k_cache, v_cache, seq_lens, block_table, batch, seqlen_new,
                       num_kv_heads, head_dim, page_size, num_pages, max_pages_per_seq,
                       workspace, stream, kv);
    if (st != MX_STATUS_OK) return st;
    app.appended = (int)seqlen_new;
  }
  return run_decode(plan, q, k_cache, v_cache, out, nullptr, nullptr, seq_lens, block_table,
                    batch, seqlen_q, num_heads, kh.kv_heads, kh.head_dim, page_size, num_pages,
                    max_pages_per_seq, causal, scale, workspace, 0, app, stream, kv,
                    kh.pair_group);
}

// Scales of an append into an fp8 cache: the stored values are x / scale.
static int check_fp8_append_scales(float k_scale, float v_scale) {
  if (!(std::isfinite(k_scale) && std::isfinite(v_scale) && k_scale > 0.f && v_scale > 0.f))
    return fail(MX_STATUS_INVALID_ARGUMENT, "k_scale and v_scale must be finite and > 0");
  return MX_STATUS_OK;
}

int mx_paged_kv_append(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                       const int32_t* seq_lens, const int32_t* block_table, int64_t batch,
                       int64_t seqlen_new, int64_t num_kv_heads, int64_t head_dim,
                       int64_t page_size, int64_t num_pages, int64_t max_pages_per_seq,
                       void* workspace, void* stream) {
  return kv_append_impl(k_new, v_new, k_cache, v_cache, seq_lens, block_table, batch, seqlen_new,
                        num_kv_heads, head_dim, page_size, num_pages, max_pages_per_seq,
                        workspace, stream, KvFormat{});
}

int mx_paged_kv_append_fp8kv(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                             const int32_t* seq_lens, const int32_t* block_table, int64_t batch,
                             int64_t seqlen_new, int64_t num_kv_heads, int64_t head_dim,
                             int64_t page_size, int64_t num_pages, int64_t max_pages_per_seq,
                             float k_scale, float v_scale, void* workspace, void* stream) {
  const int st = check_fp8_append_scales(k_scale, v_scale);
  if (st != MX_STATUS_OK) return st;
  KvFormat kv;
  kv.fp8 = true;
  kv.k_scale = k_scale;
  kv.v_scale = v_scale;
  return kv_append_impl(k_new, v_new, k_cache, v_cache, seq_lens, block_table, batch, seqlen_new,
                        num_kv_heads, head_dim, page_size, num_pages, max_pages_per_seq,
                        workspace, stream, kv);
}

int mx_paged_gqa_decode_append(const void* q, const void* k_new, const void* v_new,
                               void* k_cache, void* v_cache, void* out, const int32_t* seq_lens,
                               const int32_t* block_table, int64_t batch, int64_t seqlen_q,
                               int64_t seqlen_new, int64_t num_heads, int64_t num_kv_heads,
                               int64_t head_dim, int64_t page_size, int64_t num_pages,
                               int64_t max_pages_per_seq, int64_t max_seq_len, int32_t causal,
                               float scale, int64_t num_splits, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  return decode_append_impl(q, k_new, v_new, k_cache, v_cache, out, seq_lens, block_table,
                            batch, seqlen_q, seqlen_new, num_heads, num_kv_heads, head_dim,
                            page_size, num_pages, max_pages_per_seq, max_seq_len, causal, scale,
                            num_splits, workspace, workspace_bytes, stream, KvFormat{});
}

int mx_paged_gqa_decode_append_fp8kv(const void* q, const void* k_new, const void* v_new,
                                     void* k_cache, void* v_cache, void* out,
                                     const int32_t* seq_lens, const int32_t* block_table,
                                     int64_t batch, int64_t seqlen_q, int64_t seqlen_new,
                                     int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                     int64_t page_size, int64_t num_pages,
                                     int64_t max_pages_per_seq, int64_t max_seq_len,
                                     int32_t causal, float scale, float k_scale, float v_scale,
                                     int64_t num_splits, void* workspace, int64_t workspace_bytes,
                                     void* stream) {
  int st = check_fp8_append_scales(k_scale, v_scale);
  if (st != MX_STATUS_OK) return st;
  if (!std::isfinite(scale * k_scale))
    return fail(MX_STATUS_INVALID_ARGUMENT, "scale * k_scale must be finite");
  KvFormat kv;
  kv.fp8 = true;
  kv.k_scale = k_scale;
  kv.v_scale = v_scale;
  return decode_append_impl(q, k_new, v_new, k_cache, v_cache, out, seq_lens, block_table,
                            batch, seqlen_q, seqlen_new, num_heads, num_kv_heads, head_dim,
                            page_size, num_pages, max_pages_per_seq, max_seq_len, causal, scale,
                            num_splits, workspace, workspace_bytes, stream, kv);
}

int mx_last_status(void) { return g_last_status; }

const char* mx_last_error(void) { return g_last_error.c_str(); }

const char* mx_version(void) { return "mxattn 0.1.0 (gfx950 paged GQA decode)"; }

}  // extern "C"

#ifdef MX_WG_TIMELINE
// Timeline builds only: the per-workgroup stamp table of the current device, kTimelineSlots
// rows of kTimelineFields unsigned 64-bit values (see WgTimeline).  Synchronous.
extern "C" int64_t mx_timeline_bytes(void) { return (int64_t)sizeof(g_timeline); }

extern "C" int mx_timeline_clear(void) {
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_timeline)) != hipSuccess ||
      hipMemset(p, 0, sizeof(g_timeline)) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
    (void)hipGetLastError();
    return MX_STATUS_HIP_ERROR;
  }
  return MX_STATUS_OK;
}

extern "C" int mx_timeline_read(void* host, int64_t bytes) {
  if (host == nullptr || bytes < (int64_t)sizeof(g_timeline)) return MX_STATUS_INVALID_ARGUMENT;
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_timeline)) != hipSuccess ||
      hipMemcpy(host, p, sizeof(g_timeline), hipMemcpyDeviceToHost) != hipSuccess) {
    (void)hipGetLastError();
    return MX_STATUS_HIP_ERROR;
  }
  return MX_STATUS_OK;
}
#endif
