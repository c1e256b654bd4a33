// kvshift.hip -- gfx950 kernels and C ABI for the shift-connector KV reuse path.
//
// What is computed (reference semantics: src/marathon/shift_kernels.py:141-159 for the
// op order, :68-84 for the rotation tables, :89-132 for the fused scatter, and
// src/marathon/kvshift.py:44-61 for the RoPE identity):
//   for every span s, layer l, token i < n_s and KV head h
//     K' = rotate(K[src(s, i), h], delta_s)   fp32, separate mul/mul/add, RNE back
//     V' = V[src(s, i), h]                     raw bytes
//     write K', V' at dst(s, i), head h        paged: block = slot / bs, off = slot % bs
//
// Design (CDNA4, HBM-bound, no MFMA):
//   * The shift kernel is a one-shot grid over (token tiles) x (layers): a workgroup
//     moves tile_tokens tokens of one layer and exits.  Measured on MI355X, one-shot
//     workgroups stream ~25% faster than persistent grid-stride loops, where each
//     iteration's loads queue behind the previous iteration's stores (gfx9 counts
//     loads and stores on one vmcnt).
//   * A row is one (layer, token, head): K[D] then V[D].  Lane j of a row owns the
//     16-byte chunk j of K and the 16-byte chunk j of V, so each load/store
//     instruction moves whole, contiguous runs (full 128-byte lines).
//   * When heads is a multiple of the rows a wave covers, every row of a wave pass
//     belongs to one token: the token's metadata is read with scalar loads and the
//     lane address is (uniform base) + (per-lane 32-bit constant).  Otherwise (fewer
//     heads, e.g. one GPU's share under tensor parallelism) each lane reads its own
//     token's record, and the wave's shared base-address row comes through scalar
//     loads.
//   * rotate_half needs chunk j +- rotary/2: it comes from the partner lane through
//     ds_bpermute (no second global read of K).
//   * Batched shifts take one of three paths.  Two launches: a small plan kernel
//     resolves every token's source and destination row (slot arrays / block tables,
//     bounds-checked) into a record and evaluates each span's cos/sin once (double
//     precision, rounded to fp32), both in a caller-provided workspace; the shift kernel
//     then reads one record per token (optionally sorted by destination page first).
//     Direct (short shifts, caller-supplied prefix and tables): the shift kernel alone,
//     each workgroup resolving its token from the span table, whose entries the wave's
//     lanes hold in registers.  Small (a decode step): the spans and index windows
//     travel in the launch's arguments.  The library allocates nothing.
//   * Loads and stores are non-temporal: every byte is touched exactly once.  Where a
//     pass's destination row is wave-uniform, the stores also carry device scope
//     (sc1 nt, through a buffer resource), measured 2-3% faster for these write-once
//     rows.
//   * Workgroups move one token each (bf16: 128 threads = 8 rows of 512 B) and are
//     dealt so that each XCD walks one contiguous range of tokens, layer by layer:
//     measured against every other order tried (strided ranges, layers inner,
//     persistent walks), this is the fastest.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "fp8_e4m3.h"
#include "marathon_kvshift.h"
#include "rope_angle.h"

#pragma clang fp contract(off)

// Tuning knobs (compile-time): non-temporal loads / stores, wave passes per workgroup.
#ifndef MKV_NT_LOAD
#define MKV_NT_LOAD 1
#endif
#ifndef MKV_NT_STORE
#define MKV_NT_STORE 1
#endif
#ifndef MKV_PASSES_2B
#define MKV_PASSES_2B 1
#endif
#ifndef MKV_PASSES_4B
#define MKV_PASSES_4B 4
#endif
#ifndef MKV_PASSES_1B
#define MKV_PASSES_1B 2
#endif
// fp8's passes per wave in the per-lane form (heads not a multiple of a wave's rows).
#ifndef MKV_PASSES_1B_NU
#define MKV_PASSES_1B_NU MKV_PASSES_1B
#endif

// 1: store V before rotating K (frees its registers during the rotation).  Measured
// 11% slower for bf16: a row's K and V halves are adjacent, and writing them far apart
// in time costs write efficiency.  Off.
#ifndef MKV_V_FIRST
#define MKV_V_FIRST 0
#endif

#ifndef MKV_WG_THREADS
#define MKV_WG_THREADS 128
#endif
// Plan pass: the per-span cos/sin tables are made by workgroups of their own, which need
// no token prefix, instead of by the first record workgroups after their records' chain
// (0.5 us less per two-launch call on 2,048-token and one-head shifts; 0: off).
#ifndef MKV_PLAN_TABLE_GROUPS
#define MKV_PLAN_TABLE_GROUPS 1
#endif
// Record and direct paths with one token per wave pass: each wave stages its span's
// rotation table in LDS with one 16-byte load per lane, and every lane reads its chunk's
// cos/sin from there, instead of each lane loading its own 2 x C floats from the table
// in memory: one global load per lane where fp8's chunk of 16 elements took eight.
// Bit 1: fp8 (measured 1.4-3% faster on the fp8 Qwen3-14B shift); bit 2: 2-byte
// elements (four loads per lane before: one-span shifts 0.3-1.7% faster, the 8-span
// Qwen3-14B shift 0.2% slower, so off); bit 4: fp8 on the per-lane path, where a wave's
// rows span tokens (one-head to four-head shares 0.3-1.2% faster).
#ifndef MKV_TABLE_LDS
#define MKV_TABLE_LDS 5
#endif
#ifndef MKV_TABLE_WITH_DATA
#define MKV_TABLE_WITH_DATA 1
#endif
// The same for the record path's per-lane form (rows of several tokens in a wave): each
// lane's first rotation table is loaded beside the data rather than after it.  One
// GPU's share under tensor parallelism 4 / 8 (2 / 1 KV heads): bf16 2.0 / 2.7% faster,
// fp8 0.8 / 0.7%.
#ifndef MKV_TABLE_WITH_DATA_LANES
#define MKV_TABLE_WITH_DATA_LANES 1
#endif
// Cache policy of the shift kernel's stores where the destination row is wave-uniform
// (buffer stores): 18 = sc1 | nt (device-scope streaming).  -1: plain non-temporal
// global stores everywhere.
#ifndef MKV_STORE_CPOL
#define MKV_STORE_CPOL 18
#endif
// Cache policy of the data loads where the source row is wave-uniform: >= 0 loads
// through a buffer resource with these policy bits; -1 global loads (non-temporal
// with MKV_NT_LOAD).
#ifndef MKV_LOAD_CPOL
#define MKV_LOAD_CPOL -1
#endif
// Layers one workgroup moves (grid.y = ceil(layers / this)), each pass's token metadata
// resolved once for all of them.  The direct path moves MKV_DIRECT_WIDE_LAYERS layers per
// workgroup when a shift of 2-byte elements has more than MKV_DIRECT_WIDE_MIN_ROWS
// (token, layer) rows, and one layer otherwise; the record path MKV_LAYERS_RECORDS.
#ifndef MKV_DIRECT_WIDE_LAYERS
#define MKV_DIRECT_WIDE_LAYERS 4
#endif
#ifndef MKV_DIRECT_WIDE_MIN_ROWS
#define MKV_DIRECT_WIDE_MIN_ROWS 2560
#endif
#ifndef MKV_LAYERS_RECORDS
#define MKV_LAYERS_RECORDS 1
#endif
// The same for the record path's per-lane form (heads not a multiple of a wave's rows:
// one GPU's share of the KV heads under tensor parallelism), for 1-byte elements and
// for the others.  fp8 at 4 / 2 / 1 heads: two layers 3.0 / 3.0 / 1.7% faster than one
// (a token's record then serves twice the bytes); bf16 at 2 / 1 heads 1.6 / 2.4% slower.
#ifndef MKV_LAYERS_RECORDS_NU_1B
#define MKV_LAYERS_RECORDS_NU_1B 2
#endif
#ifndef MKV_LAYERS_RECORDS_NU
#define MKV_LAYERS_RECORDS_NU MKV_LAYERS_RECORDS
#endif
// 1: the batched kernels fetch group 0's base addresses for their layers before the
// token metadata (the usual single-session shift then needs no dependent fetch of
// them).  Direct path, record path.
#ifndef MKV_SPEC_BASE_DIRECT
#define MKV_SPEC_BASE_DIRECT 1
#endif
#ifndef MKV_SPEC_BASE_RECORDS
#define MKV_SPEC_BASE_RECORDS 0
#endif
// The record path's per-lane form: group 0's bases fetched ahead, used when every lane
// of the wave belongs to group 0 (its records' base rows then need no scalar fetch of
// their own).  fp8 shares at 4 / 2 / 1 KV heads 0.9 / 1.0 / 0.7% faster, bf16 neutral.
#ifndef MKV_SPEC_BASE_LANES
#define MKV_SPEC_BASE_LANES 1
#endif
// XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs; with
// the remap, XCD k walks the k-th contiguous eighth of the tiles (smaller per-XCD set
// of pages in flight).  1 = plain order everywhere.
#ifndef MKV_XCDS
#define MKV_XCDS 8
#endif
// Shifts whose token rows (K and V of every head of a token, one layer) span fewer
// bytes than this take the plain order: with the plan's tokens sorted by destination
// page, dealing consecutive tiles to all XCDs at once measured faster for them (fp8 at
// 8 heads, 2 KB a token: 3.8%; bf16 at 4 / 2 / 1 heads: 4.8 / 3.6 / 2.7%), while 4 KB
// tokens (bf16 at 8 heads, 64 KB paged blocks) keep the XCD-aware order (headline 0.6%,
// 32 sessions 3.4% faster with it).
#ifndef MKV_XCD_MIN_TOKEN_BYTES
#define MKV_XCD_MIN_TOKEN_BYTES 4096
#endif
static_assert(MKV_XCDS >= 1, "MKV_XCDS");
// Record-path shifts reading from at least MKV_LAYER_MAJOR_MIN_GROUPS source groups
// (sessions' stores) and moving at least MKV_LAYER_MAJOR_MIN_TOKENS tokens take a
// one-dimensional grid with the layer groups fastest: a tile's layers run back to back
// on one XCD, so the workgroups running together hold a few tokens' rows of every layer
// rather than many tokens of one layer, from few sessions' stores rather than from all
// of them.  Measured in one process against the two-dimensional grid (layers slowest):
// 32 sessions (250K tokens) 2.8-5.2% faster and 16 sessions (116K) 2.5-4.2% (the
// translation misses of the vector caches fall by 39% at 32 sessions); 1, 2, 4 or 8
// sessions, or 16 and 32 short ones, within +-1.5% or slower (up to 12% for the fp8
// single-session shift); the reverse, saves from one paged pool into 16 or 32 stores,
// 4.6% slower, so only source groups count.
#ifndef MKV_LAYER_MAJOR_MIN_GROUPS
#define MKV_LAYER_MAJOR_MIN_GROUPS 16
#endif
#ifndef MKV_LAYER_MAJOR_MIN_TOKENS
#define MKV_LAYER_MAJOR_MIN_TOKENS 100000
#endif
// Which rows a wave's passes take when it makes more than one (fp8, fp32): 0 = pass u of
// wave w takes the tile's row group w + waves * u (the waves interleave); 1 = w * passes + u
// (a wave's passes take adjacent row groups: for 8 heads, adjacent tokens).
#ifndef MKV_PASS_MAJOR
#define MKV_PASS_MAJOR 0
#endif

namespace {

constexpr int kThreads = MKV_WG_THREADS;  // shift kernel; a multiple of the 64-lane wave
constexpr int kWaves = kThreads / 64;

// layers per workgroup of the record path (the direct path picks its own per launch)
template <int DT, bool BATCHED, bool UNIFORM>
constexpr int layer_batch() {
  return !BATCHED   ? 1
         : UNIFORM ? MKV_LAYERS_RECORDS
                   : (DT == MKV_FP8_E4M3 ? MKV_LAYERS_RECORDS_NU_1B : MKV_LAYERS_RECORDS_NU);
}
constexpr int kPlanThreads = 256;  // plan kernel
// Buffer resources for the stores: raw (stride 0), the whole 32-bit range checked by
// the hardware (a lane's offset is below 2^31, checked on the host), and the gfx9
// default data-format word.
constexpr int kRsrcRange = -1;  // 0xFFFFFFFF bytes
constexpr int kRsrcWord3 = 0x00020000;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Global-address-space view: keeps the compiler on global_load/global_store rather
// than flat_* (whose counters would also wait on the LDS exchange).
typedef u32x4 __attribute__((address_space(1))) g_u32x4;

// ------------------------------------------------------------------ element traits

template <int DT>
struct Elem;
template <>
struct Elem<MKV_BF16> {
  static constexpr int kBytes = 2, kPerChunk = 8, kPasses = MKV_PASSES_2B;
};
template <>
struct Elem<MKV_F16> {
  static constexpr int kBytes = 2, kPerChunk = 8, kPasses = MKV_PASSES_2B;
};
template <>
struct Elem<MKV_F32> {
  static constexpr int kBytes = 4, kPerChunk = 4, kPasses = MKV_PASSES_4B;
};
template <>
struct Elem<MKV_FP8_E4M3> {
  static constexpr int kBytes = 1, kPerChunk = 16, kPasses = MKV_PASSES_1B;
};

// Wave passes per workgroup: the element type's, or fp8's per-lane count.
template <int DT, bool UNIFORM>
constexpr int passes() {
  return DT == MKV_FP8_E4M3 && !UNIFORM ? MKV_PASSES_1B_NU : Elem<DT>::kPasses;
}

int passes_of(int dt, bool uniform) {
  switch (dt) {
    case MKV_FP8_E4M3:
      return uniform ? MKV_PASSES_1B : MKV_PASSES_1B_NU;
    case MKV_F32:
      return MKV_PASSES_4B;
    default:
      return MKV_PASSES_2B;
  }
}

// ----------------------------------------------------------------- device structs

// How one side maps a token position to a byte offset inside its buffer.
struct DevSide {
  const void* index;
  const int64_t* group_slots;
  int64_t index_len;
  int64_t num_slots;
  int64_t bstride;  // BYTES
  int64_t ostride;  // BYTES
  int64_t block_size;
  int32_t bs_shift;  // log2(block_size), or -1 when block_size is not a power of two
  int32_t mode;
  int32_t groups;
  int32_t pad;
};

// One resolved token of a batched shift (32 bytes), written by plan_kernel.
struct TokRec {
  int64_t src_off;  // byte offset of the token's row (head 0, element 0) in its buffer
  int64_t dst_off;
  int32_t span;     // -1: nothing to do for this token
  int32_t delta;
  int32_t src_base;  // src_group * layers (row of the source base-address tables)
  int32_t dst_base;
};

struct PlanParams {
  const mkv_span_t* spans;
  const float* inv_freq;
  float* tables;  // [n_spans][2][rotary]: cos by element, then sgn by element
  TokRec* recs;   // [total_tokens]
  uint32_t* order_hist;  // ordered: [gridDim.x][kOrderBuckets] page counts per workgroup
  int64_t order_chunk;   // ordered: tokens per workgroup (contiguous)
  int32_t order_shift;   // ordered: destination offset >> this = bucket
  const int32_t* token_order;  // record i resolves token token_order[i] (NULL: token i)
  int32_t* err;
  int64_t total_tokens;
  int32_t n_spans;
  int32_t layers;
  int32_t rotary;
  int32_t rec_groups;  // workgroups 0 .. rec_groups - 1 resolve records; the rest, tables
  DevSide src;
  DevSide dst;
};

struct ShiftParams {
  // single span: bases, the source token stride, slots and the rotation tables
  const char* s_k;
  const char* s_v;
  char* d_k;
  char* d_v;
  const int64_t* slots;
  const float* cos;
  const float* sgn;
  int64_t src_tstride;  // BYTES
  DevSide dst;          // slot -> offset (single span)
  // batched: records (or, direct, the span table and its token prefix), per-span
  // tables, base-address tables
  const TokRec* recs;
  const mkv_span_t* spans;
  const int64_t* starts;  // direct: [n_spans + 1] exclusive prefix of n_tokens
  DevSide src;            // direct: source addressing (dst above is the destination's)
  const float* tables;
  const float* inv_freq;  // small: the tables are computed from it in the kernel
  const uint64_t* src_k_base;
  const uint64_t* src_v_base;
  const uint64_t* dst_k_base;
  const uint64_t* dst_v_base;
  // common
  const float* k_scale;
  int32_t* err;
  int64_t total_tokens;
  int64_t src_hstride;  // BYTES
  int64_t dst_hstride;  // BYTES
  int32_t layers;
  int32_t heads;
  int32_t rotary;
  int32_t tile_tokens;
  int32_t chunks_per_row;  // nK: 16-byte chunks in K (= lanes per row)
  int32_t rows_per_wave;
  uint32_t heads_magic;  // ceil(2^32 / heads): r / heads == umulhi(r, magic), r < 2^16
  int32_t rotate;        // single span: tables present
  int32_t n_spans;       // direct
  int32_t xcds;          // MKV_XCDS: XCD-aware tile order; 1: plain order
  int32_t xcd_per;       // set at launch: tiles per XCD with xcds > 1, else 0
  int32_t layer_groups;  // the layer-major grid: 1 = asked for (host), then the layer
                         // groups at launch; 0: two-dimensional
  int32_t pad3;
};

// A small shift's tables, carried in the launch's kernel arguments (no device copy):
// the span table, its token prefix and each side's index window (int64, block ids or
// slots).  ~1.5 KB of the 4 KB kernel-argument limit.
struct SmallPack {
  mkv_span_t spans[MKV_SMALL_MAX_SPANS];
  int64_t starts[MKV_SMALL_MAX_SPANS + 1];
  int64_t src_index[MKV_SMALL_MAX_INDEX];
  int64_t dst_index[MKV_SMALL_MAX_INDEX];
};

struct SmallParams {
  ShiftParams p;
  SmallPack q;
};

// ------------------------------------------------------------------ small helpers

// Read-only metadata through the constant address space: with a uniform address the
// compiler emits scalar loads (through the scalar cache; nothing is written there).
template <typename T>
__device__ __forceinline__ T ld_const(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

__device__ __forceinline__ u32x4 load16(const char* p) {
#if MKV_NT_LOAD
  return __builtin_nontemporal_load((const g_u32x4*)p);
#else
  return *(const g_u32x4*)p;
#endif
}
__device__ __forceinline__ void store16(char* p, u32x4 v) {
#if MKV_NT_STORE
  __builtin_nontemporal_store(v, (g_u32x4*)p);
#else
  *(g_u32x4*)p = v;
#endif
}

// Store through a buffer resource whose base is wave-uniform (`base`, a row of the
// destination) at a per-lane 32-bit offset, with the cache policy MKV_STORE_CPOL.  The
// default, device-scope streaming (sc1 nt), measured 2-3% faster than nt alone on gfx950
// for these write-once rows; the global-store builtins cannot set the scope bits.
// Policy bits: 1 sc0, 2 nt, 16 sc1.
__device__ __forceinline__ void store16_at(char* base, uint32_t lane_off, u32x4 v) {
#if MKV_STORE_CPOL >= 0
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(base, 0, kRsrcRange, kRsrcWord3);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, static_cast<int>(lane_off), 0, MKV_STORE_CPOL);
#else
  store16(base + lane_off, v);
#endif
}

// Load from a wave-uniform source row `base` at a per-lane 32-bit offset, with the
// cache policy MKV_LOAD_CPOL (same bits as the stores).
__device__ __forceinline__ u32x4 load16_at(const char* base, uint32_t lane_off) {
#if MKV_LOAD_CPOL >= 0
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(base), 0, kRsrcRange, kRsrcWord3);
  return __builtin_bit_cast(
      u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(lane_off), 0,
                                                   MKV_LOAD_CPOL));
#else
  return load16(base + lane_off);
#endif
}

__device__ __forceinline__ uint32_t bpermute(int lane_byte_addr, uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_ds_bpermute(lane_byte_addr, static_cast<int>(v)));
}

template <typename T>
__device__ __forceinline__ T uniform(T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "");
  if constexpr (sizeof(T) == 4) {
    return static_cast<T>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
  } else {
    const uint64_t u = static_cast<uint64_t>(v);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<int>(u & 0xFFFFFFFFu));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<int>(u >> 32));
    return static_cast<T>((static_cast<uint64_t>(hi) << 32) | lo);
  }
}

// The value lane `src` holds (src wave-uniform).
__device__ __forceinline__ int32_t lane_value(int32_t v, int src) {
  return __builtin_amdgcn_readlane(v, src);
}
__device__ __forceinline__ int64_t lane_value(int64_t v, int src) {
  const uint64_t u = static_cast<uint64_t>(v);
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(u & 0xFFFFFFFFu), src);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(u >> 32), src);
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// RN(RN(k*c) + RN(kp*s)): the torch path's separate fp32 multiply, multiply, add
// (shift_kernels.py:156).  `contract(off)` above keeps the compiler from fusing.
__device__ __forceinline__ float rot1(float k, float kp, float c, float s) {
  float a = k * c;
  float b = kp * s;
  return a + b;
}

// fp32 -> bf16, round to nearest even; NaN -> 0x7FC0 (torch's c10::BFloat16 rule).
__device__ __forceinline__ uint32_t bf16_rne(float y) {
  uint32_t u = __float_as_uint(y);
  uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  return (y != y) ? 0x7FC0u : r;
}

__device__ __forceinline__ uint32_t f16_rne(float y) {
  if (y != y) return 0x7E00u;
  return static_cast<uint32_t>(__half_as_ushort(__float2half_rn(y)));
}
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  return __half2float(__ushort_as_half(static_cast<unsigned short>(h & 0xFFFFu)));
}

// Rotate the C elements of one 16-byte chunk.  `mine` is this lane's K chunk,
// `part` the partner chunk (same element positions, other half of the rotation),
// c / s the cos and signed sin of those positions.
template <int DT>
struct Rotor;

template <>
struct Rotor<MKV_BF16> {
  static __device__ __forceinline__ u32x4 run(u32x4 mine, u32x4 part, const float* c,
                                              const float* s, const mkv_fp8::Divisor&) {
    u32x4 out;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float k0 = __uint_as_float(mine[w] << 16), k1 = __uint_as_float(mine[w] & 0xFFFF0000u);
      float p0 = __uint_as_float(part[w] << 16), p1 = __uint_as_float(part[w] & 0xFFFF0000u);
      uint32_t lo = bf16_rne(rot1(k0, p0, c[2 * w], s[2 * w]));
      uint32_t hi = bf16_rne(rot1(k1, p1, c[2 * w + 1], s[2 * w + 1]));
      out[w] = lo | (hi << 16);
    }
    return out;
  }
};

template <>
struct Rotor<MKV_F16> {
  static __device__ __forceinline__ u32x4 run(u32x4 mine, u32x4 part, const float* c,
                                              const float* s, const mkv_fp8::Divisor&) {
    u32x4 out;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float k0 = f16_to_f32(mine[w]), k1 = f16_to_f32(mine[w] >> 16);
      float p0 = f16_to_f32(part[w]), p1 = f16_to_f32(part[w] >> 16);
      uint32_t lo = f16_rne(rot1(k0, p0, c[2 * w], s[2 * w]));
      uint32_t hi = f16_rne(rot1(k1, p1, c[2 * w + 1], s[2 * w + 1]));
      out[w] = lo | (hi << 16);
    }
    return out;
  }
};

template <>
struct Rotor<MKV_F32> {
  static __device__ __forceinline__ u32x4 run(u32x4 mine, u32x4 part, const float* c,
                                              const float* s, const mkv_fp8::Divisor&) {
    u32x4 out;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float y = rot1(__uint_as_float(mine[w]), __uint_as_float(part[w]), c[w], s[w]);
      out[w] = (y != y) ? 0x7FC00000u : __float_as_uint(y);
    }
    return out;
  }
};

// fp8 e4m3fn: dequantise with the layer's K scale, rotate as above, requantise
// (codec in fp8_e4m3.h).  When any lane of the wave holds a NaN code, every lane
// recomputes which of its outputs are NaN and writes the canonical 0x7F there.  A lane's
// partner chunk is another active lane's own chunk (the partner sits in the same row,
// so it runs this code too), so one ballot over the lanes' own chunks covers both.
template <>
struct Rotor<MKV_FP8_E4M3> {
  static __device__ __forceinline__ u32x4 run(u32x4 mine, u32x4 part, const float* c,
                                              const float* s, const mkv_fp8::Divisor& dv) {
    using namespace mkv_fp8;
    u32x4 out;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float mk[4], pk[4], q[4];
      decode4(mine[w], mk);
      decode4(part[w], pk);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int e = 4 * w + b;
        q[b] = quant(rot1(mk[b] * dv.s, pk[b] * dv.s, c[e], s[e]), dv);
      }
      out[w] = encode4(q);
    }
    const bool own_nan = has_nan_code(mine[0]) || has_nan_code(mine[1]) ||
                         has_nan_code(mine[2]) || has_nan_code(mine[3]);
    if (__builtin_expect(__ballot(own_nan) != 0, 0)) {
      // y is NaN exactly when an input of its rotation is (every other input is finite)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        float mk[4], pk[4];
        decode4(mine[w], mk);
        decode4(part[w], pk);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int e = 4 * w + b;
          const float y = rot1(mk[b] * dv.s, pk[b] * dv.s, c[e], s[e]);
          if (y != y) out[w] = with_nan(out[w], b);
        }
      }
    }
    return out;
  }
};

// Byte offset of token position `pos0 + i` (index slot `index0 + i`) on one side; false
// when any index is out of range.  cap / cap_blocks: slots and blocks the buffer holds.
__device__ __forceinline__ bool resolve(const DevSide& sd, int64_t cap, int64_t cap_blocks,
                                        int64_t pos0, int64_t index0, int64_t i,
                                        int64_t& off_bytes) {
  int64_t blk, off;
  if (sd.mode == MKV_ADDR_TABLE) {
    const int64_t pos = pos0 + i;
    if (pos < 0) return false;
    const int64_t bi = sd.bs_shift >= 0 ? (pos >> sd.bs_shift) : (pos / sd.block_size);
    const int64_t ti = index0 + bi;
    if (ti < 0 || ti >= sd.index_len) return false;
    const int64_t b = static_cast<const int32_t*>(sd.index)[ti];
    if (b < 0 || b >= cap_blocks) return false;
    blk = b;
    off = pos - bi * sd.block_size;
  } else {
    int64_t slot;
    if (sd.mode == MKV_ADDR_SLOTS) {
      const int64_t ii = index0 + i;
      if (ii < 0 || ii >= sd.index_len) return false;
      slot = static_cast<const int64_t*>(sd.index)[ii];
    } else {
      slot = pos0 + i;
    }
    if (slot < 0 || slot >= cap) return false;
    if (sd.bs_shift >= 0) {
      blk = slot >> sd.bs_shift;
      off = slot & (sd.block_size - 1);
    } else {
      blk = slot / sd.block_size;
      off = slot - blk * sd.block_size;
    }
  }
  off_bytes = blk * sd.bstride + off * sd.ostride;
  return true;
}

// resolve() for the direct path: block sizes that are powers of two (shifts only, no
// 64-bit division) and wave-uniform indices (scalar loads).
// `small`: the index is the launch's own int64 window, not the side's device array.
__device__ __forceinline__ bool resolve_direct(const DevSide& sd, const int64_t* small,
                                               int64_t cap, int64_t pos0, int64_t index0,
                                               int64_t i, int64_t& off_bytes) {
  const int sh = sd.bs_shift;
  int64_t blk, off;
  if (sd.mode == MKV_ADDR_TABLE) {
    const int64_t pos = pos0 + i;
    if (pos < 0) return false;
    const int64_t ti = index0 + (pos >> sh);
    if (ti < 0 || ti >= sd.index_len) return false;
    blk = small != nullptr ? ld_const(small + ti)
                           : ld_const(static_cast<const int32_t*>(sd.index) + ti);
    if (blk < 0 || blk >= (cap >> sh)) return false;
    off = pos & ((int64_t{1} << sh) - 1);
  } else {
    int64_t slot = pos0 + i;
    if (sd.mode == MKV_ADDR_SLOTS) {
      const int64_t ii = index0 + i;
      if (ii < 0 || ii >= sd.index_len) return false;
      slot = ld_const((small != nullptr ? small : static_cast<const int64_t*>(sd.index)) + ii);
    }
    if (slot < 0 || slot >= cap) return false;
    blk = slot >> sh;
    off = slot & ((int64_t{1} << sh) - 1);
  }
  off_bytes = blk * sd.bstride + off * sd.ostride;
  return true;
}

// Destination-page order (MKV_ORDER_DST_PAGE): a record's bucket is its destination row's
// byte offset >> shift, where the host picks the smallest shift of at least 21 (2 MB
// translation pages) that maps the destination cache's extent into kOrderBuckets
// buckets; offsets past the last bucket share it.
constexpr int kOrderBuckets = 256;
constexpr int kOrderMaxGroups = 256;  // workgroups of an ordered plan pass (and scatter)

__device__ __forceinline__ uint32_t order_bucket(const TokRec& r, int shift) {
  if (r.span < 0) return 0;
  const uint64_t page = static_cast<uint64_t>(r.dst_off) >> shift;
  return page < kOrderBuckets ? static_cast<uint32_t>(page) : kOrderBuckets - 1;
}

// cos and sin of frequency f's angle for one delta: the fp32 angle fl32(delta * inv_freq[f])
// (shift_kernels.py:73), its sine and cosine evaluated in double precision and rounded
// once to fp32 (rope_angle.h).  Every table the device makes (the plan pass and the small
// path) and every table the host makes (mkv_rope_tables) comes from that one routine, so
// they hold the same bits.
__device__ __forceinline__ void angle_cos_sin(int delta, float inv_freq_f, float& c, float& s) {
  mkv_rope::angle_cos_sin(delta, inv_freq_f, c, s);
}

// A span's table in the layout every path reads: [2][rotary], the cos of each element's
// frequency, then its signed sine (-sin on the first half, +sin on the second).
__device__ __forceinline__ void put_table(float* t, int rotary, int f, float c, float s) {
  const int half = rotary / 2;
  t[f] = c;
  t[f + half] = c;
  t[rotary + f] = -s;
  t[rotary + f + half] = s;
}

// --------------------------------------------------------------------- plan kernel
//
// Every workgroup builds the token prefix over spans in LDS, then resolves a
// grid-stride share of the tokens into records and of (span, frequency) pairs into
// the cos/sin tables.

// cos / signed sin per span, element-indexed like the reference's tables: (span,
// frequency) pairs from `first` in steps of `stride`
__device__ __forceinline__ void plan_tables(const PlanParams& p, int64_t first, int64_t stride) {
  const int half = p.rotary / 2;
  const int64_t pairs = static_cast<int64_t>(p.n_spans) * half;
  for (int64_t idx = first; idx < pairs; idx += stride) {
    const int s = static_cast<int>(idx / half);
    const int f = static_cast<int>(idx - static_cast<int64_t>(s) * half);
    float c, sn;
    angle_cos_sin(p.spans[s].delta, p.inv_freq[f], c, sn);
    put_table(p.tables + static_cast<int64_t>(s) * 2 * p.rotary, p.rotary, f, c, sn);
  }
}

__global__ __launch_bounds__(kPlanThreads) void plan_kernel(PlanParams p) {
  extern __shared__ int64_t s_pre[];  // [n_spans + 1]: exclusive prefix of tokens
  __shared__ int64_t s_part[kPlanThreads];
  __shared__ int s_bad;
  const int tid = threadIdx.x;
  const int n = p.n_spans;
  const int rec_groups = p.rec_groups;
#if MKV_PLAN_TABLE_GROUPS
  if (static_cast<int>(blockIdx.x) >= rec_groups) {  // a table workgroup (uniform)
    plan_tables(p, static_cast<int64_t>(blockIdx.x - rec_groups) * kPlanThreads + tid,
                static_cast<int64_t>(gridDim.x - rec_groups) * kPlanThreads);
    return;
  }
#endif
  const bool checker = blockIdx.x == 0 && p.err != nullptr;  // workgroup 0 checks the spans
  if (tid == 0) s_bad = 0;

  // the spans' token counts into LDS: coalesced loads, 8 in flight per thread
  constexpr int kStage = 8;
  bool bad = false;
  for (int i0 = 0; i0 < n; i0 += kStage * kPlanThreads) {
    int32_t c[kStage];
#pragma unroll
    for (int k = 0; k < kStage; ++k) {
      const int i = i0 + k * kPlanThreads + tid;
      c[k] = i < n ? p.spans[i].n_tokens : 0;
    }
#pragma unroll
    for (int k = 0; k < kStage; ++k) {
      const int i = i0 + k * kPlanThreads + tid;
      if (i < n) {
        s_pre[i] = c[k] > 0 ? c[k] : 0;
        if (checker) {
          const mkv_span_t& sp = p.spans[i];
          bad |= c[k] < 0 || sp.src_group < 0 || sp.src_group >= p.src.groups ||
                 sp.dst_group < 0 || sp.dst_group >= p.dst.groups;
        }
      }
    }
  }
  __syncthreads();
  // exclusive prefix in place: per-thread contiguous chunks, then a scan of the chunks
  const int per = (n + kPlanThreads - 1) / kPlanThreads;
  const int b = tid * per;
  const int e = min(b + per, n);
  int64_t sum = 0;
  for (int i = b; i < e; ++i) sum += s_pre[i];
  s_part[tid] = sum;
  __syncthreads();
  for (int off = 1; off < kPlanThreads; off <<= 1) {
    const int64_t v = tid >= off ? s_part[tid - off] : 0;
    __syncthreads();
    s_part[tid] += v;
    __syncthreads();
  }
  int64_t run = s_part[tid] - sum;
  for (int i = b; i < e; ++i) {
    const int64_t c = s_pre[i];
    s_pre[i] = run;
    run += c;
  }
  if (tid == kPlanThreads - 1) s_pre[n] = s_part[kPlanThreads - 1];
  if (bad) s_bad = 1;
  __syncthreads();
  const int64_t actual = s_pre[n];
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * kPlanThreads + tid;
  const int64_t gstride = static_cast<int64_t>(rec_groups) * kPlanThreads;

  if (checker && tid == 0 && (s_bad != 0 || actual > p.total_tokens))
    atomicOr(p.err, MKV_FLAG_SPAN);

#if !MKV_PLAN_TABLE_GROUPS
  plan_tables(p, gtid, gstride);
#endif

  // token records: grid-stride, or (ordered) one contiguous chunk per workgroup with
  // its page histogram
  __shared__ uint32_t s_hist[kOrderBuckets];
  const bool ordered = p.order_hist != nullptr;
  int64_t g_lo = gtid, g_hi = p.total_tokens, g_step = gstride;
  if (ordered) {
    for (int b = tid; b < kOrderBuckets; b += kPlanThreads) s_hist[b] = 0;
    __syncthreads();
    g_lo = static_cast<int64_t>(blockIdx.x) * p.order_chunk;
    g_hi = min(g_lo + p.order_chunk, p.total_tokens);
    g_lo += tid;
    g_step = kPlanThreads;
  }
  for (int64_t g = g_lo; g < g_hi; g += g_step) {
    TokRec r;
    r.src_off = 0;
    r.dst_off = 0;
    r.span = -1;
    r.delta = 0;
    r.src_base = 0;
    r.dst_base = 0;
    // the token this record resolves: the caller's order, or span order
    int64_t tok = g;
    if (p.token_order != nullptr) {
      tok = p.token_order[g];
      if (tok < 0 || tok >= p.total_tokens) {
        if (p.err != nullptr) atomicOr(p.err, MKV_FLAG_SPAN);
        tok = actual;  // resolves nothing
      }
    }
    if (tok < actual) {
      int lo = 0, hi = n;  // largest s with s_pre[s] <= tok; then s_pre[s + 1] > tok
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (s_pre[mid] <= tok) lo = mid;
        else hi = mid;
      }
      const mkv_span_t sp = p.spans[lo];
      const bool groups_ok = sp.src_group >= 0 && sp.src_group < p.src.groups &&
                             sp.dst_group >= 0 && sp.dst_group < p.dst.groups;
      if (groups_ok) {
        const int64_t i = tok - s_pre[lo];
        int64_t s_cap = p.src.num_slots, d_cap = p.dst.num_slots;
        if (p.src.group_slots != nullptr) s_cap = p.src.group_slots[sp.src_group];
        if (p.dst.group_slots != nullptr) d_cap = p.dst.group_slots[sp.dst_group];
        int64_t so = 0, dof = 0;
        const bool s_ok =
            resolve(p.src, s_cap, s_cap / p.src.block_size, sp.src_pos, sp.src_index, i, so);
        const bool d_ok =
            resolve(p.dst, d_cap, d_cap / p.dst.block_size, sp.dst_pos, sp.dst_index, i, dof);
        if (s_ok && d_ok) {
          r.src_off = so;
          r.dst_off = dof;
          r.span = lo;
          r.delta = sp.delta;
          r.src_base = sp.src_group * p.layers;
          r.dst_base = sp.dst_group * p.layers;
        } else if (p.err != nullptr) {
          atomicOr(p.err, (s_ok ? 0 : MKV_FLAG_SRC_RANGE) | (d_ok ? 0 : MKV_FLAG_DST_RANGE));
        }
      }
    }
    p.recs[g] = r;
    if (ordered) atomicAdd(&s_hist[order_bucket(r, p.order_shift)], 1u);
  }
  if (ordered) {
    __syncthreads();
    for (int b = tid; b < kOrderBuckets; b += kPlanThreads)
      p.order_hist[static_cast<int64_t>(blockIdx.x) * kOrderBuckets + b] = s_hist[b];
  }
}

// -------------------------------------------------------------------- order kernels
//
// Optional (MKV_ORDER_DST_PAGE): the plan's records, sorted stably by the page of their
// destination row, so that the workgroups running together touch few destination pages
// while the tokens of one destination block stay together and in order (each record
// still carries its span, so the per-span tables are unchanged).  Two steps: the ordered
// plan pass resolves one contiguous chunk of tokens per workgroup and counts its pages
// ([groups][kOrderBuckets]); order_scatter_kernel, one workgroup per chunk, derives its
// chunk's first output position in every page from all the counts and writes the
// chunk's records there in token order (ranks within a wave from ballots, waves and
// batches in order).

constexpr int kScatterThreads = kOrderBuckets;  // thread b owns page bucket b

__global__ __launch_bounds__(kScatterThreads) void order_scatter_kernel(
    const TokRec* in, TokRec* out, const uint32_t* hist, int64_t total, int64_t chunk,
    int groups, int shift) {
  __shared__ uint32_t part[kOrderBuckets];     // records of each page, all chunks
  __shared__ uint32_t running[kOrderBuckets];  // next output position of each page
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // page tid: its records in every chunk, and in the chunks before this one (loads
  // coalesced across threads, 32 chunks in flight per round)
  constexpr int kRound = 32;
  uint32_t all = 0, before = 0;
  const int me = static_cast<int>(blockIdx.x);
  for (int w = 0; w < groups; w += kRound) {
    uint32_t c[kRound];
#pragma unroll
    for (int k = 0; k < kRound; ++k)
      c[k] = w + k < groups ? hist[static_cast<int64_t>(w + k) * kOrderBuckets + tid] : 0u;
#pragma unroll
    for (int k = 0; k < kRound; ++k) {
      all += c[k];
      before += w + k < me ? c[k] : 0u;
    }
  }
  part[tid] = all;
  __syncthreads();
  for (int off = 1; off < kOrderBuckets; off <<= 1) {  // inclusive scan over pages
    const uint32_t v = tid >= off ? part[tid - off] : 0u;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  running[tid] = part[tid] - all + before;
  const int64_t lo = static_cast<int64_t>(blockIdx.x) * chunk;
  const int64_t hi = min(lo + chunk, total);
  const uint64_t below = (uint64_t{1} << lane) - 1;
  for (int64_t b0 = lo; b0 < hi; b0 += kScatterThreads) {
    const int64_t g = b0 + tid;
    const bool valid = g < hi;
    TokRec r{};
    if (valid) r = in[g];
    const uint32_t key = valid ? order_bucket(r, shift) : 0u;
    uint32_t pos = 0;
    __syncthreads();  // `running` is set (first batch) or the previous batch is done
    for (int v = 0; v < kScatterThreads / 64; ++v) {
      if (wave == v) {
        // the distinct pages of this wave, one ballot each, in lane order
        uint64_t todo = __ballot(valid);
        while (todo != 0) {
          const int leader = __ffsll(static_cast<long long>(todo)) - 1;
          const uint32_t k = static_cast<uint32_t>(
              __builtin_amdgcn_readlane(static_cast<int>(key), leader));
          const uint64_t same = __ballot(valid && key == k);
          const uint32_t base = running[k];
          if (valid && key == k) pos = base + static_cast<uint32_t>(__popcll(same & below));
          if (lane == leader) running[k] = base + static_cast<uint32_t>(__popcll(same));
          todo &= ~same;
        }
      }
      __syncthreads();
    }
    if (valid) out[pos] = r;
  }
}

// -------------------------------------------------------------------- shift kernel
//
// Grid (token tiles, layer groups of LB layers).  Wave w of the workgroup runs passes
// q = w + kWaves * u (u < U); pass q covers rows [q * rpw, (q + 1) * rpw) of the tile's
// token-major (token, head) rows, in each of the workgroup's LB layers.  UNIFORM:
// heads % rpw == 0, so every row of a pass belongs to one token.  BATCHED: a span
// table (records from the plan pass, or DIRECT: resolved here); otherwise one span of
// one layer (mkv_scatter_shifted).  SMALL: the span table and index windows are the
// launch's arguments.

template <int DT, bool BATCHED, bool UNIFORM, bool DIRECT, bool SMALL, int LB>
__device__ __forceinline__ void shift_body(const ShiftParams& p, const SmallPack* q) {
  static_assert(!DIRECT || (BATCHED && UNIFORM), "direct shifts resolve one token per pass");
  static_assert(!SMALL || DIRECT, "small shifts take the direct path");
  using E = Elem<DT>;
  constexpr int C = E::kPerChunk;
  constexpr int U = passes<DT, UNIFORM>();
  static_assert(LB >= 1 && (BATCHED || LB == 1), "one layer per single-span launch");
  constexpr int N = U * LB;  // (pass, layer) units of one sweep: x = u * LB + lb

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int nK = p.chunks_per_row;
  const int rpw = p.rows_per_wave;
  const int row_in_wave = lane / nK;
  const int j = lane - row_in_wave * nK;  // chunk index inside K (and inside V)
  const bool lane_live = row_in_wave < rpw;
  const int P = p.rotary / (2 * C);  // rotate_half distance, in chunks
  const bool rot_lane = j < 2 * P;
  const int partner = j < P ? lane + P : (rot_lane ? lane - P : lane);
  const int partner_addr = (partner & 63) * 4;
  const uint32_t chunk_off = static_cast<uint32_t>(j) * 16u;
  const int H = p.heads;

  // The fields the first metadata and data fetches need are loaded in the kernel's first
  // batch of scalar loads, with those the tile decisions below read, rather than in a
  // second dependent batch behind the early exits (the compiler does not hoist loads
  // above them on its own): one kernel-argument round trip fewer ahead of the data.
  if constexpr (!BATCHED) {
    asm volatile("" ::"s"(p.s_k), "s"(p.s_v), "s"(p.d_k), "s"(p.d_v), "s"(p.src_tstride));
  } else if constexpr (!DIRECT) {
    asm volatile("" ::"s"(p.recs), "s"(p.src_k_base), "s"(p.src_v_base), "s"(p.dst_k_base),
                 "s"(p.dst_v_base), "s"(p.tables), "s"(p.k_scale), "s"(p.src_hstride),
                 "s"(p.dst_hstride));
  } else if constexpr (!SMALL) {
    asm volatile("" ::"s"(p.starts), "s"(p.spans), "s"(p.n_spans));
  }
  int64_t tile = blockIdx.x;
  int lgroup = blockIdx.y;
  if (BATCHED && !DIRECT && p.layer_groups > 0) {
    // gridDim.x == tiles * layer_groups: XCD k takes tiles [k * xcd_per, (k + 1) *
    // xcd_per), each tile's layer groups in turn; plain order: tile-major, layers fastest
    const int64_t b = blockIdx.x;
    const int LG = p.layer_groups;
    if (p.xcd_per > 0) {
      const int64_t local = b / MKV_XCDS;
      lgroup = static_cast<int>(local % LG);
      tile = (b % MKV_XCDS) * p.xcd_per + local / LG;
    } else {
      lgroup = static_cast<int>(b % LG);
      tile = b / LG;
    }
  } else if (p.xcd_per > 0) {
    // gridDim.x == MKV_XCDS * xcd_per (the launch pads the grid): a bijection on
    // [0, gridDim.x).  The launch passes xcd_per rather than the kernel reading
    // gridDim.x, whose hidden argument would be one more dependent scalar load ahead
    // of the first data load.
    tile = static_cast<int64_t>(blockIdx.x % MKV_XCDS) * p.xcd_per + blockIdx.x / MKV_XCDS;
  }
  const int layer0 = lgroup * LB;
  const int64_t g0 = tile * p.tile_tokens;
  if constexpr (DIRECT && !SMALL) {
    // one workgroup checks the caller's prefix against the span table: starts[0] == 0,
    // each step equals the span's token count, and the last is at most total_tokens
    if (blockIdx.x == 0 && blockIdx.y == 0 && wave == 0 && p.err != nullptr) {
      bool bad = false;
      if (lane < p.n_spans) {
        const int64_t lo = p.starts[lane], hi = p.starts[lane + 1];
        const int32_t n = p.spans[lane].n_tokens;
        bad = hi - lo != (n > 0 ? n : 0) || (lane == 0 && lo != 0) ||
              (lane == p.n_spans - 1 && hi > p.total_tokens) || n < 0;
      }
      if (__ballot(bad) != 0 && lane == 0) atomicOr(p.err, MKV_FLAG_SPAN);
    }
  }
  const int64_t left = p.total_tokens - g0;
  if (left <= 0) return;  // padding workgroups of the XCD-aware grid
  const int ntok = static_cast<int>(left < p.tile_tokens ? left : p.tile_tokens);
  const int nrows = ntok * H;
  // small: the spans of the workgroup's tokens [g0, g0 + ntok), whose rotation tables the
  // workgroup computes together into LDS ([span - small_lo][2][rotary])
  float* small_tab = nullptr;
  int small_lo = 0, small_hi = 0;
  if constexpr (SMALL) {
    extern __shared__ float small_lds[];
    small_tab = small_lds;
#pragma unroll
    for (int k = 0; k < MKV_SMALL_MAX_SPANS; ++k) {
      if (k < p.n_spans && q->starts[k] <= g0) small_lo = k;
      if (k < p.n_spans && q->starts[k] <= g0 + ntok - 1) small_hi = k;
    }
  }
  // per-lane constant part of the addresses (UNIFORM: lane head = pass head + row_in_wave)
  const uint32_t s_lane = UNIFORM ? static_cast<uint32_t>(row_in_wave) *
                                            static_cast<uint32_t>(p.src_hstride) + chunk_off
                                  : chunk_off;
  const uint32_t d_lane = UNIFORM ? static_cast<uint32_t>(row_in_wave) *
                                            static_cast<uint32_t>(p.dst_hstride) + chunk_off
                                  : chunk_off;
  // the workgroup's layers; the last batch of a layer count that LB does not divide
  // has layers past the end, which move nothing
  bool lay_ok[LB];
  int lay[LB];  // clamped: base-table and scale reads stay in range
#pragma unroll
  for (int lb = 0; lb < LB; ++lb) {
    lay_ok[lb] = layer0 + lb < p.layers;
    lay[lb] = lay_ok[lb] ? layer0 + lb : p.layers - 1;
  }

  mkv_fp8::Divisor dv[LB];  // fp8: the layers' K scales
  float cs[C], sg[C];
#pragma unroll
  for (int e = 0; e < C; ++e) cs[e] = 1.0f, sg[e] = 0.0f;
#pragma unroll
  for (int lb = 0; lb < LB; ++lb) dv[lb] = mkv_fp8::unit_divisor();
  int cur_span = -1;
  // MKV_TABLE_LDS: the wave's span table in LDS, staged by the whole wave
  constexpr bool kLdsTab =
      BATCHED && UNIFORM && !SMALL &&
      (((MKV_TABLE_LDS & 1) != 0 && DT == MKV_FP8_E4M3) || ((MKV_TABLE_LDS & 2) != 0 && E::kBytes == 2));
  constexpr bool kLdsTabLanes =
      BATCHED && !UNIFORM && !SMALL && (MKV_TABLE_LDS & 4) != 0 && DT == MKV_FP8_E4M3;
  float* wave_tab = nullptr;
  if constexpr (kLdsTab || kLdsTabLanes) {
    __shared__ __align__(16) float tab_lds[kWaves][2 * MKV_MAX_HEAD_SIZE];
    wave_tab = tab_lds[wave];
  }
  // stage span sp's [2][rotary] table (rotary / 2 chunks of 16 bytes) into the wave's LDS
  // copy, then give each rotating lane its chunk's values; wave-uniform calls only
  auto stage_table = [&](int sp) {
    const float* tb = p.tables + static_cast<int64_t>(sp) * 2 * p.rotary;
    for (int c = lane; c < p.rotary / 2; c += 64)
      *reinterpret_cast<u32x4*>(wave_tab + 4 * c) = *reinterpret_cast<const u32x4*>(tb + 4 * c);
    __builtin_amdgcn_wave_barrier();  // a wave's LDS accesses complete in order
    if (lane_live && rot_lane) {
#pragma unroll
      for (int e = 0; e < C; ++e) {
        cs[e] = wave_tab[j * C + e];
        sg[e] = wave_tab[p.rotary + j * C + e];
      }
    }
  };
  (void)stage_table;
  // the per-lane path's tables (kLdsTabLanes; the whole wave calls it): `need` lanes
  // rotate with span `sp` and lack its table.  The wave stages the span of the first such
  // lane in LDS and every lane needing that span reads it there, then the next span, until
  // none is left (a wave's rows rarely straddle two spans)
  auto lane_tables = [&](bool need, int sp) {
    for (uint64_t needs = __ballot(need); needs != 0; needs = __ballot(need)) {
      const int sp0 = __builtin_amdgcn_readlane(sp, __builtin_ctzll(needs));
      const float* tb = p.tables + static_cast<int64_t>(sp0) * 2 * p.rotary;
      for (int c = lane; c < p.rotary / 2; c += 64)
        *reinterpret_cast<u32x4*>(wave_tab + 4 * c) = *reinterpret_cast<const u32x4*>(tb + 4 * c);
      __builtin_amdgcn_wave_barrier();  // a wave's LDS accesses complete in order
      if (need && sp == sp0) {
#pragma unroll
        for (int e = 0; e < C; ++e) {
          cs[e] = wave_tab[j * C + e];
          sg[e] = wave_tab[p.rotary + j * C + e];
        }
        cur_span = sp;
        need = false;
      }
    }
  };
  (void)lane_tables;
  // a single span's cos/sin and fp8's K scales are loaded behind the first pass's data
  // (phase B), not here: they are needed only for the rotation, and a load in flight at
  // the pass loop's head would hold back the first data loads
  bool scale_ready = DT != MKV_FP8_E4M3;

  // direct (span table in memory): lane k holds span k's fields and prefix entry k,
  // loaded once; a pass finds its span with one ballot and reads the fields from that
  // lane, with no dependent load
  int64_t l_start = INT64_MAX, l_spos = 0, l_dpos = 0, l_sidx = 0, l_didx = 0;
  int32_t l_n = 0, l_delta = 0, l_sg = 0, l_dg = 0;
  if constexpr (DIRECT && !SMALL) {
    if (lane <= p.n_spans) l_start = p.starts[lane];
    if (lane < p.n_spans) {
      const mkv_span_t sp = p.spans[lane];
      l_spos = sp.src_pos;
      l_dpos = sp.dst_pos;
      l_sidx = sp.src_index;
      l_didx = sp.dst_index;
      l_n = sp.n_tokens;
      l_delta = sp.delta;
      l_sg = sp.src_group;
      l_dg = sp.dst_group;
    }
  }
  // group 0's base addresses for the workgroup's layers, fetched ahead (see
  // MKV_SPEC_BASE_*); a pass of another group fetches its own
  constexpr bool kSpec = BATCHED && (UNIFORM ? (DIRECT ? MKV_SPEC_BASE_DIRECT != 0
                                                       : MKV_SPEC_BASE_RECORDS != 0)
                                            : MKV_SPEC_BASE_LANES != 0);
  const char* g0_sk[LB];
  const char* g0_sv[LB];
  char* g0_dk[LB];
  char* g0_dv[LB];
  if constexpr (kSpec) {
#pragma unroll
    for (int lb = 0; lb < LB; ++lb) {
      g0_sk[lb] = reinterpret_cast<const char*>(ld_const(p.src_k_base + lay[lb]));
      g0_sv[lb] = reinterpret_cast<const char*>(ld_const(p.src_v_base + lay[lb]));
      g0_dk[lb] = reinterpret_cast<char*>(ld_const(p.dst_k_base + lay[lb]));
      g0_dv[lb] = reinterpret_cast<char*>(ld_const(p.dst_v_base + lay[lb]));
    }
  }

    if constexpr (SMALL) {
    // the workgroup computes the tables of its spans together (at most one cos/sin pair
    // per thread for a one-span step) into LDS, with the routine of the plan pass, so
    // every path holds the same table bits.  Done before the data loads: evaluated
    // beside them it kept the loads' registers live through the double-precision sine
    // and cosine (133 against 93 VGPRs for fp8).
    if (p.rotary > 0) {
      const int half = p.rotary / 2;
      const int pairs = (small_hi - small_lo + 1) * half;
      for (int idx = tid; idx < pairs; idx += kThreads) {
        const int k = idx / half;
        const int f = idx - k * half;
        const int dl = q->spans[small_lo + k].delta;
        if (dl != 0) {
          float c, sn;
          angle_cos_sin(dl, p.inv_freq[f], c, sn);
          put_table(small_tab + k * 2 * p.rotary, p.rotary, f, c, sn);
        }
      }
      __syncthreads();
    }
  }
  for (int r0 = 0; r0 < nrows; r0 += kWaves * U * rpw) {
    // ---- phase A: where each pass reads and writes (uniform when UNIFORM).  All token
    // metadata is fetched first, then all base addresses, so the workgroup pays two
    // metadata round trips in total rather than two per pass; a token's metadata serves
    // every layer of the workgroup.
    bool live[U];
    int span_u[U], delta_u[U], head_u[U];
    int64_t s_at[U], d_at[U];  // byte offsets of the pass's (first) row
    int64_t slot_u[U];         // single span: the pass's destination slot, resolved late
    // direct: the destination's inputs, resolved late (dchk: span and groups are valid)
    bool dchk_u[U];
    int64_t dpos_u[U], didx_u[U], di_u[U];
    int dg_u[U];
    int sb_u[U], db_u[U];      // the (group, layer 0) rows of the base tables
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row0 = r0 + (MKV_PASS_MAJOR ? wave * U + u : wave + kWaves * u) * rpw;
      const int r = UNIFORM ? row0 : row0 + row_in_wave;
      const int rr = r < nrows ? r : nrows - 1;  // clamp: metadata reads stay in range
      const int t = H == 1 ? rr
                           : static_cast<int>(__umulhi(static_cast<uint32_t>(rr), p.heads_magic));
      head_u[u] = rr - t * H;
      const int64_t g = g0 + t;
      live[u] = r < nrows;
      if constexpr (DIRECT) {
        // the token's span and rows, resolved here from the span table (no plan pass)
        int s;
        int64_t start, spos, dpos, sidx, didx;
        int32_t n_tok, delta, sg, dg;
        if constexpr (SMALL) {
          s = -1;  // the prefix is the launch's own: a uniform scan of at most 9 entries
#pragma unroll
          for (int k = 0; k <= MKV_SMALL_MAX_SPANS; ++k)
            if (k <= p.n_spans && q->starts[k] <= g) s = k;
          const int sc = s >= 0 && s < p.n_spans ? s : 0;  // clamped: reads stay in range
          const mkv_span_t* sp = q->spans + sc;
          start = ld_const(q->starts + sc);
          spos = ld_const(&sp->src_pos);
          dpos = ld_const(&sp->dst_pos);
          sidx = ld_const(&sp->src_index);
          didx = ld_const(&sp->dst_index);
          n_tok = ld_const(&sp->n_tokens);
          delta = ld_const(&sp->delta);
          sg = ld_const(&sp->src_group);
          dg = ld_const(&sp->dst_group);
        } else {
          s = static_cast<int>(__popcll(__ballot(l_start <= g))) - 1;
          const int sc = s >= 0 && s < p.n_spans ? s : 0;
          start = lane_value(l_start, sc);
          spos = lane_value(l_spos, sc);
          dpos = lane_value(l_dpos, sc);
          sidx = lane_value(l_sidx, sc);
          didx = lane_value(l_didx, sc);
          n_tok = lane_value(l_n, sc);
          delta = lane_value(l_delta, sc);
          sg = lane_value(l_sg, sc);
          dg = lane_value(l_dg, sc);
        }
        const int64_t i = g - start;
        const bool in_span = live[u] && s >= 0 && s < p.n_spans && i >= 0;
        bool ok = in_span && i < n_tok && sg >= 0 && sg < p.src.groups &&
                  dg >= 0 && dg < p.dst.groups;
        // the source row now; the destination row after the data loads have gone out
        // (they do not need it), with its inputs kept here
        dchk_u[u] = ok;
        dpos_u[u] = dpos;
        didx_u[u] = didx;
        di_u[u] = i;
        dg_u[u] = dg;
        int64_t so = 0;
        if (ok) {
          const int64_t s_cap = p.src.group_slots != nullptr ? ld_const(p.src.group_slots + sg)
                                                             : p.src.num_slots;
          if (!resolve_direct(p.src, SMALL ? q->src_index : nullptr, s_cap, spos, sidx, i, so)) {
            if (p.err != nullptr && lane == 0) atomicOr(p.err, MKV_FLAG_SRC_RANGE);
            ok = false;
          }
        } else if (in_span && p.err != nullptr && lane == 0) {
          atomicOr(p.err, MKV_FLAG_SPAN);  // a bad group, or a prefix the spans do not fill
        }
        span_u[u] = ok ? s : -1;
        delta_u[u] = delta;
        s_at[u] = so;
        d_at[u] = 0;
        sb_u[u] = (ok ? sg : 0) * p.layers;
        db_u[u] = (ok ? dg : 0) * p.layers;
      } else if constexpr (BATCHED) {
        const TokRec* rp = p.recs + g;
        span_u[u] = UNIFORM ? ld_const(&rp->span) : rp->span;
        delta_u[u] = UNIFORM ? ld_const(&rp->delta) : rp->delta;
        s_at[u] = UNIFORM ? ld_const(&rp->src_off) : rp->src_off;
        d_at[u] = UNIFORM ? ld_const(&rp->dst_off) : rp->dst_off;
        sb_u[u] = UNIFORM ? ld_const(&rp->src_base) : rp->src_base;
        db_u[u] = UNIFORM ? ld_const(&rp->dst_base) : rp->dst_base;
      } else {
        span_u[u] = 0;
        delta_u[u] = p.rotate;
        s_at[u] = g * p.src_tstride;
        sb_u[u] = db_u[u] = 0;
        // the destination slot is only read here; it is checked and turned into an
        // address after the data loads have gone out (the source row does not need it)
        slot_u[u] = UNIFORM ? ld_const(p.slots + g) : p.slots[g];
        d_at[u] = 0;
      }
      if constexpr (BATCHED) live[u] = live[u] && span_u[u] >= 0;
      s_at[u] += head_u[u] * p.src_hstride;
      d_at[u] += head_u[u] * p.dst_hstride;
    }

    // ---- the base address of every (pass, layer) unit
    bool xl[N];
    const char* sbk[N];
    const char* sbv[N];
    char* dbk[N];
    char* dbv[N];
#pragma unroll
    for (int x = 0; x < N; ++x) {
      const int u = x / LB, lb = x % LB;
      xl[x] = live[u] && lay_ok[lb];
      if constexpr (BATCHED) {
        const int sb = sb_u[u] + lay[lb], db = db_u[u] + lay[lb];
        if (UNIFORM && u > 0 && sb_u[u] == sb_u[0] && db_u[u] == db_u[0]) {
          // the usual case: every pass of the tile belongs to one group
          sbk[x] = sbk[lb];
          sbv[x] = sbv[lb];
          dbk[x] = dbk[lb];
          dbv[x] = dbv[lb];
        } else if (kSpec && (UNIFORM ? sb_u[u] == 0 && db_u[u] == 0
                                     : __all(sb_u[u] == 0 && db_u[u] == 0))) {
          sbk[x] = g0_sk[lb];
          sbv[x] = g0_sv[lb];
          dbk[x] = g0_dk[lb];
          dbv[x] = g0_dv[lb];
        } else if (UNIFORM) {
          sbk[x] = reinterpret_cast<const char*>(ld_const(p.src_k_base + sb));
          sbv[x] = reinterpret_cast<const char*>(ld_const(p.src_v_base + sb));
          dbk[x] = reinterpret_cast<char*>(ld_const(p.dst_k_base + db));
          dbv[x] = reinterpret_cast<char*>(ld_const(p.dst_v_base + db));
        } else {
          // rows of several tokens: they usually share one (group, layer) base row,
          // read with scalar loads (a per-lane gather measured 6-10% slower); the
          // gather runs only when the wave straddles groups
          const int sb0 = uniform(sb), db0 = uniform(db);
          sbk[x] = reinterpret_cast<const char*>(ld_const(p.src_k_base + sb0));
          sbv[x] = reinterpret_cast<const char*>(ld_const(p.src_v_base + sb0));
          dbk[x] = reinterpret_cast<char*>(ld_const(p.dst_k_base + db0));
          dbv[x] = reinterpret_cast<char*>(ld_const(p.dst_v_base + db0));
          if (!__all(sb == sb0 && db == db0)) {
            sbk[x] = reinterpret_cast<const char*>(p.src_k_base[sb]);
            sbv[x] = reinterpret_cast<const char*>(p.src_v_base[sb]);
            dbk[x] = reinterpret_cast<char*>(p.dst_k_base[db]);
            dbv[x] = reinterpret_cast<char*>(p.dst_v_base[db]);
          }
        }
        const bool aligned =
            ((reinterpret_cast<uint64_t>(sbk[x]) | reinterpret_cast<uint64_t>(sbv[x]) |
              reinterpret_cast<uint64_t>(dbk[x]) | reinterpret_cast<uint64_t>(dbv[x])) & 15u) == 0;
        if (xl[x] && !aligned) {
          if (p.err != nullptr && (!UNIFORM || lane == 0)) atomicOr(p.err, MKV_FLAG_ALIGN);
          xl[x] = false;
        }
      } else {
        sbk[x] = p.s_k;
        sbv[x] = p.s_v;
        dbk[x] = p.d_k;
        dbv[x] = p.d_v;
      }
    }

    // ---- phase B: every data load of the workgroup's passes in flight at once
    __builtin_amdgcn_sched_barrier(0);
    u32x4 kd[N], vd[N];
#pragma unroll
    for (int x = 0; x < N; ++x) {
      const int u = x / LB;
      kd[x] = u32x4{0, 0, 0, 0};
      vd[x] = u32x4{0, 0, 0, 0};
      if (xl[x] && lane_live) {
        if constexpr (UNIFORM) {
          kd[x] = load16_at(sbk[x] + s_at[u], s_lane);
          vd[x] = load16_at(sbv[x] + s_at[u], s_lane);
        } else {
          kd[x] = load16(sbk[x] + s_at[u] + s_lane);
          vd[x] = load16(sbv[x] + s_at[u] + s_lane);
        }
      }
    }
    if constexpr (DT == MKV_FP8_E4M3) {
      if (!scale_ready) {
        // the scale dequantises K for the rotation; with no rotation k_scale may be NULL
        if (BATCHED ? p.rotary > 0 : p.rotate != 0) {
#pragma unroll
          for (int lb = 0; lb < LB; ++lb)
            dv[lb] = mkv_fp8::divisor(ld_const(p.k_scale + (BATCHED ? lay[lb] : 0)));
        }
        scale_ready = true;
      }
    }
    if constexpr (!BATCHED) {
      // single span: the one rotation table, once per workgroup, behind the data
      if (cur_span < 0 && p.rotate && rot_lane) {
#pragma unroll
        for (int e = 0; e < C; ++e) {
          cs[e] = p.cos[j * C + e];
          sg[e] = p.sgn[j * C + e];
        }
      }
      cur_span = 0;
    }
#if MKV_TABLE_WITH_DATA
    if constexpr (BATCHED && UNIFORM && DT == MKV_FP8_E4M3) {
      // fp8 (5 waves per SIMD: too few to hide one more dependent round trip per
      // workgroup): the first pass's rotation table travels with the data, an L2 hit,
      // instead of being fetched after it.  A later pass of another span (rare) still
      // loads its own in phase C.  Measured +2-3% for fp8; for bf16, which runs at full
      // occupancy, 1-4% slower, so there the table follows the data.
      if constexpr (kLdsTab) {
        if (live[0] && delta_u[0] != 0 && span_u[0] != cur_span) {  // wave-uniform
          stage_table(span_u[0]);
          cur_span = span_u[0];
        }
      } else if (!SMALL && live[0] && lane_live && rot_lane && delta_u[0] != 0 &&
                 span_u[0] != cur_span) {
        const float* tb = p.tables + static_cast<int64_t>(span_u[0]) * 2 * p.rotary;
#pragma unroll
        for (int e = 0; e < C; ++e) {
          cs[e] = tb[j * C + e];
          sg[e] = tb[p.rotary + j * C + e];
        }
        cur_span = span_u[0];
      }
    }
#endif
#if MKV_TABLE_WITH_DATA_LANES
    if constexpr (kLdsTabLanes) {
      lane_tables(live[0] && lane_live && rot_lane && delta_u[0] != 0 && span_u[0] != cur_span,
                  span_u[0]);
    } else if constexpr (BATCHED && !UNIFORM) {
      if (live[0] && lane_live && rot_lane && delta_u[0] != 0 && span_u[0] != cur_span) {
        const float* tb = p.tables + static_cast<int64_t>(span_u[0]) * 2 * p.rotary;
#pragma unroll
        for (int e = 0; e < C; ++e) {
          cs[e] = tb[j * C + e];
          sg[e] = tb[p.rotary + j * C + e];
        }
        cur_span = span_u[0];
      }
    }
#endif
    __builtin_amdgcn_sched_barrier(0);

    // xs: the units that store.  A single span's destination slots, read in phase A,
    // are checked and turned into addresses only now, while the data loads are in
    // flight: an out-of-range slot raises its flag and its row is not stored.
    bool xs[N];
    if constexpr (!BATCHED) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t slot = slot_u[u];
        const bool ok = slot >= 0 && slot < p.dst.num_slots;
        if (live[u] && !ok && p.err != nullptr && (!UNIFORM || lane == 0))
          atomicOr(p.err, MKV_FLAG_DST_RANGE);
        int64_t blk, off;
        if (p.dst.bs_shift >= 0) {
          blk = slot >> p.dst.bs_shift;
          off = slot & (p.dst.block_size - 1);
        } else {
          blk = slot / p.dst.block_size;
          off = slot - blk * p.dst.block_size;
        }
        d_at[u] += blk * p.dst.bstride + off * p.dst.ostride;
#pragma unroll
        for (int lb = 0; lb < LB; ++lb) xs[u * LB + lb] = xl[u * LB + lb] && ok;
      }
    }
    if constexpr (DIRECT) {
      // the direct path's destination rows, likewise: a row whose source or destination
      // is out of range raises its flag and is not stored
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int64_t dof = 0;
        bool d_ok = false;
        if (dchk_u[u]) {
          const int64_t d_cap = p.dst.group_slots != nullptr
                                    ? ld_const(p.dst.group_slots + dg_u[u])
                                    : p.dst.num_slots;
          d_ok = resolve_direct(p.dst, SMALL ? q->dst_index : nullptr, d_cap, dpos_u[u],
                                didx_u[u], di_u[u], dof);
          if (!d_ok && p.err != nullptr && lane == 0) atomicOr(p.err, MKV_FLAG_DST_RANGE);
        }
        d_at[u] += dof;
#pragma unroll
        for (int lb = 0; lb < LB; ++lb) xs[u * LB + lb] = xl[u * LB + lb] && d_ok;
      }
    }
    // the record path resolved its rows in phase A: xl already says what stores
#define MKV_STORES(x) ((BATCHED && !DIRECT) ? xl[x] : xs[x])

    // ---- phase C: V goes out as it came in, then K is rotated (the whole wave joins
    // the partner exchange)
#if MKV_V_FIRST
#pragma unroll
    for (int x = 0; x < N; ++x) {
      if (MKV_STORES(x) && lane_live) store16(dbv[x] + d_at[x / LB] + d_lane, vd[x]);
    }
#endif
#pragma unroll
    for (int x = 0; x < N; ++x) {
      const int u = x / LB, lb = x % LB;
      const bool wave_rotates = UNIFORM ? (MKV_STORES(x) && delta_u[u] != 0 && p.rotary > 0)
                                        : (p.rotary > 0);
      if (!wave_rotates) continue;
      if constexpr (kLdsTab) {
        if (span_u[u] != cur_span) {  // wave-uniform
          stage_table(span_u[u]);
          cur_span = span_u[u];
        }
      }
      if constexpr (kLdsTabLanes)
        lane_tables(MKV_STORES(x) && lane_live && rot_lane && delta_u[u] != 0 &&
                        span_u[u] != cur_span,
                    span_u[u]);
      u32x4 pd;
      pd[0] = bpermute(partner_addr, kd[x][0]);
      pd[1] = bpermute(partner_addr, kd[x][1]);
      pd[2] = bpermute(partner_addr, kd[x][2]);
      pd[3] = bpermute(partner_addr, kd[x][3]);
      if (MKV_STORES(x) && lane_live && rot_lane && delta_u[u] != 0) {
        if constexpr (BATCHED && !kLdsTab && !kLdsTabLanes) {
          if (span_u[u] != cur_span) {
            if constexpr (SMALL) {
              // the workgroup's own table, computed into LDS in phase B
              const float* tb = small_tab + (span_u[u] - small_lo) * 2 * p.rotary;
#pragma unroll
              for (int e = 0; e < C; ++e) {
                cs[e] = tb[j * C + e];
                sg[e] = tb[p.rotary + j * C + e];
              }
            } else {
              const float* tb = p.tables + static_cast<int64_t>(span_u[u]) * 2 * p.rotary;
#pragma unroll
              for (int e = 0; e < C; ++e) {
                cs[e] = tb[j * C + e];
                sg[e] = tb[p.rotary + j * C + e];
              }
            }
            cur_span = span_u[u];
          }
        }
        kd[x] = Rotor<DT>::run(kd[x], pd, cs, sg, dv[lb]);
      }
    }

    // ---- phase D: stores (UNIFORM: the pass's destination row is wave-uniform, so the
    // stores go through buffer resources carrying the store cache policy)
#pragma unroll
    for (int x = 0; x < N; ++x) {
      const int u = x / LB;
      if (MKV_STORES(x) && lane_live) {
        if constexpr (UNIFORM) {
          store16_at(dbk[x] + d_at[u], d_lane, kd[x]);
#if !MKV_V_FIRST
          store16_at(dbv[x] + d_at[u], d_lane, vd[x]);
#endif
        } else {
          store16(dbk[x] + d_at[u] + d_lane, kd[x]);
#if !MKV_V_FIRST
          store16(dbv[x] + d_at[u] + d_lane, vd[x]);
#endif
        }
      }
    }
#undef MKV_STORES
  }
}

template <int DT, bool BATCHED, bool UNIFORM, bool DIRECT, int LB>
__global__ __launch_bounds__(kThreads) void shift_kernel(ShiftParams p) {
  shift_body<DT, BATCHED, UNIFORM, DIRECT, false, LB>(p, nullptr);
}

// A small shift: the span table, prefix and index windows arrive in the arguments.
template <int DT>
__global__ __launch_bounds__(kThreads) void shift_small_kernel(SmallParams a) {
  shift_body<DT, true, true, true, true, 1>(a.p, &a.q);
}

// --------------------------------------------------------------------- host side

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int elem_bytes(int dt) {
  switch (dt) {
    case MKV_BF16:
    case MKV_F16:
      return 2;
    case MKV_F32:
      return 4;
    case MKV_FP8_E4M3:
      return 1;
    default:
      return 0;
  }
}

int ilog2_exact(int64_t v) {
  if (v <= 0 || (v & (v - 1)) != 0) return -1;
  int s = 0;
  while ((int64_t{1} << s) < v) ++s;
  return s;
}

bool aligned16(uint64_t v) { return (v & 15u) == 0; }

int64_t align256(int64_t v) { return (v + 255) & ~int64_t{255}; }

// Validate one side's geometry and convert it to the device form.
int make_side(const mkv_side_t& in, int eb, DevSide& out, int64_t& hstride_b, const char* name) {
  memset(&out, 0, sizeof out);
  if (in.mode != MKV_ADDR_FLAT && in.mode != MKV_ADDR_SLOTS && in.mode != MKV_ADDR_TABLE)
    return fail(MKV_ERR_ARG, "%s: unknown addressing mode %d", name, in.mode);
  if (in.block_size <= 0) return fail(MKV_ERR_ARG, "%s: block_size %d", name, in.block_size);
  if (in.num_slots < 0) return fail(MKV_ERR_ARG, "%s: num_slots < 0", name);
  if (in.mode != MKV_ADDR_FLAT && in.index == nullptr && in.index_len > 0)
    return fail(MKV_ERR_ARG, "%s: index is NULL", name);
  if (in.groups <= 0) return fail(MKV_ERR_ARG, "%s: groups %d", name, in.groups);
  const int64_t bs = in.block_stride * eb;
  const int64_t hs = in.head_stride * eb;
  const int64_t os = in.offset_stride * eb;
  if (!aligned16(static_cast<uint64_t>(bs)) || !aligned16(static_cast<uint64_t>(hs)) ||
      !aligned16(static_cast<uint64_t>(os)))
    return fail(MKV_ERR_ALIGN, "%s: byte strides (%lld, %lld, %lld) not 16-byte aligned", name,
                (long long)bs, (long long)hs, (long long)os);
  out.index = in.index;
  out.group_slots = in.group_slots;
  out.index_len = in.index == nullptr ? 0 : in.index_len;
  out.num_slots = in.num_slots;
  out.bstride = bs;
  out.ostride = os;
  out.block_size = in.block_size;
  out.bs_shift = ilog2_exact(in.block_size);
  out.mode = in.mode;
  out.groups = in.groups;
  hstride_b = hs;
  return MKV_OK;
}

struct Geometry {
  int chunks_per_row;
  int rows_per_wave;
  int tile_tokens;
  bool uniform;
  uint32_t heads_magic;
  int xcds;  // the tile order (MKV_XCD_MIN_TOKEN_BYTES)
};

int check_geometry(int dtype, int heads, int head_size, int rotary, int64_t src_hs,
                   int64_t dst_hs, Geometry& g) {
  const int eb = elem_bytes(dtype);
  if (eb == 0) return fail(MKV_ERR_DTYPE, "unknown dtype %d", dtype);
  if (heads <= 0) return fail(MKV_ERR_ARG, "heads %d", heads);
  if (head_size <= 0 || head_size > MKV_MAX_HEAD_SIZE)
    return fail(MKV_ERR_UNSUPPORTED, "head_size %d outside (0, %d]", head_size,
                MKV_MAX_HEAD_SIZE);
  if ((head_size * eb) % 16 != 0)
    return fail(MKV_ERR_UNSUPPORTED, "head_size %d x %d bytes is not a multiple of 16 bytes",
                head_size, eb);
  if (rotary < 0 || rotary > head_size)
    return fail(MKV_ERR_ARG, "rotary %d > head_size %d", rotary, head_size);
  const int per_chunk = 16 / eb;
  if (rotary % (2 * per_chunk) != 0)
    return fail(MKV_ERR_UNSUPPORTED, "rotary %d is not a multiple of %d for this dtype", rotary,
                2 * per_chunk);
  g.chunks_per_row = head_size * eb / 16;
  if (g.chunks_per_row > 64)
    return fail(MKV_ERR_UNSUPPORTED, "row of %d chunks exceeds one wave", g.chunks_per_row);
  g.rows_per_wave = 64 / g.chunks_per_row;
  g.uniform = heads % g.rows_per_wave == 0;
  const int rows = g.rows_per_wave * kWaves * passes_of(dtype, g.uniform);
  g.tile_tokens = rows / heads > 0 ? rows / heads : 1;
  // row -> (token, head) uses a 32-bit reciprocal, exact while rows < 2^16
  if (static_cast<int64_t>(g.tile_tokens) * heads >= (1 << 16))
    return fail(MKV_ERR_UNSUPPORTED, "heads %d too large", heads);
  g.heads_magic =
      heads == 1 ? 0u : static_cast<uint32_t>(((uint64_t{1} << 32) + heads - 1) / heads);
  g.xcds = static_cast<int64_t>(heads) * 2 * head_size * eb >= MKV_XCD_MIN_TOKEN_BYTES ? MKV_XCDS
                                                                                       : 1;
  // per-lane address parts are 32-bit
  const int64_t hs_max = src_hs > dst_hs ? src_hs : dst_hs;
  const int64_t lane_max =
      (g.rows_per_wave - 1) * hs_max + static_cast<int64_t>(g.chunks_per_row) * 16;
  if (src_hs < 0 || dst_hs < 0 || lane_max >= (int64_t{1} << 31))
    return fail(MKV_ERR_UNSUPPORTED, "head strides out of range");
  return MKV_OK;
}

template <int DT, bool BATCHED, bool UNIFORM, bool DIRECT, int LB>
int launch_shift(const ShiftParams& sp, int64_t tiles, int layers, hipStream_t stream) {
  // tiles is rounded up to a multiple of MKV_XCDS below; extra workgroups exit at once
  if (tiles <= 0) return MKV_OK;
  tiles = (tiles + MKV_XCDS - 1) / MKV_XCDS * MKV_XCDS;
  const int layer_groups = (layers + LB - 1) / LB;
  if (tiles > 0x7FFFFFFF || layer_groups > 65535)
    return fail(MKV_ERR_UNSUPPORTED, "grid of %lld x %d tiles too large", (long long)tiles,
                layer_groups);
  ShiftParams q = sp;
  q.xcd_per = sp.xcds > 1 ? static_cast<int32_t>(tiles / MKV_XCDS) : 0;
  q.layer_groups = 0;
  dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(layer_groups));
  if (BATCHED && !DIRECT && sp.layer_groups != 0 && tiles * layer_groups <= 0x7FFFFFFF) {
    q.layer_groups = layer_groups;
    grid = dim3(static_cast<unsigned>(tiles * layer_groups), 1);
  }
  hipLaunchKernelGGL((shift_kernel<DT, BATCHED, UNIFORM, DIRECT, LB>), grid, dim3(kThreads), 0,
                     stream, q);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MKV_ERR_HIP, "launch failed: %s", hipGetErrorString(e));
  return MKV_OK;
}

// direct_layers: the direct path's layers per workgroup (1, or MKV_DIRECT_WIDE_LAYERS for
// a larger shift of 2-byte elements); 0 = the record path.
template <bool BATCHED>
int launch_any(int dtype, bool uniform, int direct_layers, const ShiftParams& sp,
               int64_t tiles, int layers, hipStream_t stream) {

#define MKV_CASE(DT)                                                                        \
  case DT:                                                                                  \
    if constexpr (BATCHED) {                                                                \
      if (uniform && direct_layers > 0) {                                                   \
        if constexpr (Elem<DT>::kBytes == 2 && MKV_DIRECT_WIDE_LAYERS > 1) {                \
          if (direct_layers > 1)                                                            \
            return launch_shift<DT, true, true, true, MKV_DIRECT_WIDE_LAYERS>(sp, tiles,    \
                                                                              layers, stream); \
        }                                                                                   \
        return launch_shift<DT, true, true, true, 1>(sp, tiles, layers, stream);            \
      }                                                                                     \
    }                                                                                       \
    return uniform                                                                          \
               ? launch_shift<DT, BATCHED, true, false, layer_batch<DT, BATCHED, true>()>(     \
                     sp, tiles, layers, stream)                                             \
               : launch_shift<DT, BATCHED, false, false, layer_batch<DT, BATCHED, false>()>(   \
                     sp, tiles, layers, stream);
  switch (dtype) {
    MKV_CASE(MKV_BF16)
    MKV_CASE(MKV_F16)
    MKV_CASE(MKV_F32)
    MKV_CASE(MKV_FP8_E4M3)
    default:
      return fail(MKV_ERR_DTYPE, "unknown dtype %d", dtype);
  }
#undef MKV_CASE
}

int64_t workspace_bytes(int64_t total_tokens, int32_t n_spans, int32_t rotary) {
  return align256(static_cast<int64_t>(n_spans) * 2 * rotary *
                  static_cast<int64_t>(sizeof(float))) +
         total_tokens * static_cast<int64_t>(sizeof(TokRec));
}

}  // namespace

// ------------------------------------------------------------ no-allocation scratch
//
// The workspace of mkv_shift_spans_noalloc: one array per GPU, in the code object's
// device memory, held from the library's first use on that GPU until the process ends.
// Host code never passes `scratch` itself to a kernel (on the host its name is only a
// handle): each device's address comes from hipGetSymbolAddress, resolved once per
// device with that device current, and that address is what the kernels receive.
// Nothing in it needs clearing: the plan kernel writes every record and table entry the
// shift kernel of the same call reads.

__device__ __align__(256) unsigned char scratch[MKV_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 256;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, once resolved

// This call's scratch address: the current device's copy, which must also be the
// device of `st` (a NULL stream is the current device's).
int scratch_of(hipStream_t st, void** out) {
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return fail(MKV_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (st != nullptr) {
    hipDevice_t sd = -1;
    e = hipStreamGetDevice(st, &sd);
    if (e != hipSuccess)
      return fail(MKV_ERR_HIP, "hipStreamGetDevice: %s", hipGetErrorString(e));
    if (sd != cur)
      return fail(MKV_ERR_ARG, "stream is on device %d but device %d is current; make the "
                  "stream's device current", static_cast<int>(sd), cur);
  }
  if (cur < 0 || cur >= kMaxDevices) return fail(MKV_ERR_UNSUPPORTED, "device %d", cur);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[cur] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(MKV_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", cur,
                  hipGetErrorString(e));
    g_scratch_ptr[cur] = p;
  }
  *out = g_scratch_ptr[cur];
  return MKV_OK;
}

}  // namespace

// ------------------------------------------------------------------------ C ABI

extern "C" const char* mkv_last_error(void) { return g_err; }

extern "C" int32_t mkv_abi_version(void) { return MKV_ABI_VERSION; }

extern "C" int mkv_rope_tables(const int32_t* deltas, int32_t n_spans, const float* inv_freq,
                               int32_t rotary, float* tables) {
  if (n_spans < 0 || rotary < 0 || rotary % 2 != 0)
    return fail(MKV_ERR_ARG, "n_spans %d, rotary %d", n_spans, rotary);
  if (n_spans == 0 || rotary == 0) return MKV_OK;
  if (deltas == nullptr || inv_freq == nullptr || tables == nullptr)
    return fail(MKV_ERR_ARG, "null pointer");
  const int half = rotary / 2;
  for (int32_t sp = 0; sp < n_spans; ++sp) {
    float* t = tables + static_cast<int64_t>(sp) * 2 * rotary;
    for (int f = 0; f < half; ++f) {
      float c, sn;
      mkv_rope::angle_cos_sin(deltas[sp], inv_freq[f], c, sn);
      t[f] = c;
      t[f + half] = c;
      t[rotary + f] = -sn;
      t[rotary + f + half] = sn;
    }
  }
  return MKV_OK;
}

extern "C" int64_t mkv_shift_workspace_size(int64_t total_tokens, int32_t n_spans,
                                            int32_t rotary) {
  if (total_tokens < 0 || n_spans < 0 || rotary < 0) return -1;
  return workspace_bytes(total_tokens, n_spans, rotary);
}

extern "C" int mkv_scatter_shifted(const void* src, int64_t src_token_stride,
                                   int64_t src_head_stride, void* kv, int64_t kv_block_stride,
                                   int64_t kv_head_stride, int64_t kv_offset_stride,
                                   int64_t kv_num_blocks, const int64_t* slots,
                                   int64_t n_tokens, int32_t heads, int32_t head_size,
                                   int32_t block_size, int32_t dtype, const float* cos,
                                   const float* sgn, int32_t rotary, const float* k_scale,
                                   int32_t* error_flags, void* stream) {
  g_err[0] = '\0';
  const int eb = elem_bytes(dtype);
  if (eb == 0) return fail(MKV_ERR_DTYPE, "unknown dtype %d", dtype);
  Geometry g;
  int rc = check_geometry(dtype, heads, head_size, rotary, src_head_stride * eb,
                          kv_head_stride * eb, g);
  if (rc != MKV_OK) return rc;
  if (n_tokens < 0) return fail(MKV_ERR_ARG, "n_tokens %lld < 0", (long long)n_tokens);
  if (n_tokens == 0) return MKV_OK;  // the reference returns early (shift_kernels.py:185)
  if (src == nullptr || kv == nullptr || slots == nullptr)
    return fail(MKV_ERR_ARG, "NULL src, kv or slots");
  if (block_size <= 0) return fail(MKV_ERR_ARG, "block_size %d", block_size);
  if (kv_num_blocks < 0) return fail(MKV_ERR_ARG, "kv_num_blocks < 0");
  const bool rot = cos != nullptr && rotary > 0;
  if (cos != nullptr && sgn == nullptr) return fail(MKV_ERR_ARG, "cos without sgn");
  if (dtype == MKV_FP8_E4M3 && rot && k_scale == nullptr)
    return fail(MKV_ERR_ARG, "fp8 needs k_scale");
  const uint64_t s0 = reinterpret_cast<uint64_t>(src);
  const uint64_t d0 = reinterpret_cast<uint64_t>(kv);
  const uint64_t vofs = static_cast<uint64_t>(head_size) * eb;
  if (!aligned16(s0) || !aligned16(d0))
    return fail(MKV_ERR_ALIGN, "src or kv base address not 16-byte aligned");
  if (!aligned16(static_cast<uint64_t>(src_token_stride * eb)))
    return fail(MKV_ERR_ALIGN, "src token stride not 16-byte aligned");
  if (!aligned16(static_cast<uint64_t>(src_head_stride * eb)))
    return fail(MKV_ERR_ALIGN, "src head stride not 16-byte aligned");

  mkv_side_t d_in{};
  d_in.index = slots;
  d_in.index_len = n_tokens;
  d_in.num_slots = kv_num_blocks * static_cast<int64_t>(block_size);
  d_in.block_stride = kv_block_stride;
  d_in.head_stride = kv_head_stride;
  d_in.offset_stride = kv_offset_stride;
  d_in.block_size = block_size;
  d_in.mode = MKV_ADDR_SLOTS;
  d_in.groups = 1;

  ShiftParams sp;
  memset(&sp, 0, sizeof sp);
  int64_t dst_hs = 0;
  rc = make_side(d_in, eb, sp.dst, dst_hs, "dst");
  if (rc != MKV_OK) return rc;
  sp.s_k = reinterpret_cast<const char*>(s0);
  sp.s_v = reinterpret_cast<const char*>(s0 + vofs);
  sp.d_k = reinterpret_cast<char*>(d0);
  sp.d_v = reinterpret_cast<char*>(d0 + vofs);
  sp.slots = slots;
  sp.cos = cos;
  sp.sgn = sgn;
  sp.src_tstride = src_token_stride * eb;
  sp.k_scale = k_scale;
  sp.err = error_flags;
  sp.total_tokens = n_tokens;
  sp.src_hstride = src_head_stride * eb;
  sp.dst_hstride = dst_hs;
  sp.layers = 1;
  sp.heads = heads;
  sp.rotary = rot ? rotary : 0;
  sp.tile_tokens = g.tile_tokens;
  sp.xcds = g.xcds;
  sp.chunks_per_row = g.chunks_per_row;
  sp.rows_per_wave = g.rows_per_wave;
  sp.heads_magic = g.heads_magic;
  sp.rotate = rot ? 1 : 0;
  const int64_t tiles = (n_tokens + g.tile_tokens - 1) / g.tile_tokens;
  return launch_any<false>(dtype, g.uniform, 0, sp, tiles, 1,
                           static_cast<hipStream_t>(stream));
}

namespace {

// The batched shift.  noalloc: the workspace is this device's `scratch` array and the
// descriptor's workspace fields are ignored.
int shift_spans(const mkv_shift_desc_t* d, void* stream, bool noalloc) {
  g_err[0] = '\0';
  if (d == nullptr) return fail(MKV_ERR_ARG, "NULL descriptor");
  const int eb = elem_bytes(d->dtype);
  if (eb == 0) return fail(MKV_ERR_DTYPE, "unknown dtype %d", d->dtype);
  Geometry g;
  int rc = check_geometry(d->dtype, d->heads, d->head_size, d->rotary,
                          d->src.head_stride * eb, d->dst.head_stride * eb, g);
  if (rc != MKV_OK) return rc;
  if (d->n_spans < 0 || d->n_spans > MKV_MAX_SPANS)
    return fail(MKV_ERR_UNSUPPORTED, "n_spans %d outside [0, %d]", d->n_spans, MKV_MAX_SPANS);
  if (d->total_tokens < 0) return fail(MKV_ERR_ARG, "total_tokens < 0");
  if (d->n_spans == 0 || d->total_tokens == 0) return MKV_OK;
  if (d->spans == nullptr) return fail(MKV_ERR_ARG, "NULL span table");
  if (d->layers <= 0) return fail(MKV_ERR_ARG, "layers %d", d->layers);
  if (d->rotary > 0 && d->inv_freq == nullptr) return fail(MKV_ERR_ARG, "inv_freq is NULL");
  if (d->dtype == MKV_FP8_E4M3 && d->rotary > 0 && d->k_scale == nullptr)
    return fail(MKV_ERR_ARG, "fp8 needs k_scale");
  if (d->src.k_base == nullptr || d->src.v_base == nullptr || d->dst.k_base == nullptr ||
      d->dst.v_base == nullptr)
    return fail(MKV_ERR_ARG, "NULL base-address table");
  if (d->token_order != nullptr && d->order != MKV_ORDER_NONE)
    return fail(MKV_ERR_ARG, "token_order and order %d together: one order or the other",
                d->order);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t tiles = (d->total_tokens + g.tile_tokens - 1) / g.tile_tokens;
  if (tiles > 0x7FFFFFFF) return fail(MKV_ERR_UNSUPPORTED, "total_tokens too large");

  ShiftParams sp;
  memset(&sp, 0, sizeof sp);
  sp.src_k_base = d->src.k_base;
  sp.src_v_base = d->src.v_base;
  sp.dst_k_base = d->dst.k_base;
  sp.dst_v_base = d->dst.v_base;
  sp.k_scale = d->k_scale;
  sp.err = d->error_flags;
  sp.total_tokens = d->total_tokens;
  sp.layers = d->layers;
  sp.heads = d->heads;
  sp.rotary = d->rotary;
  sp.tile_tokens = g.tile_tokens;
  sp.xcds = g.xcds;
  sp.chunks_per_row = g.chunks_per_row;
  sp.rows_per_wave = g.rows_per_wave;
  sp.heads_magic = g.heads_magic;

  // one launch and no workspace: the shift kernel resolves every token from the span
  // table, the caller's token prefix and the caller's per-span tables
  if (d->span_starts != nullptr && d->span_tables != nullptr && g.uniform &&
      d->n_spans <= MKV_DIRECT_MAX_SPANS && ilog2_exact(d->src.block_size) >= 0 &&
      ilog2_exact(d->dst.block_size) >= 0) {
    if (!aligned16(reinterpret_cast<uint64_t>(d->span_tables)))
      return fail(MKV_ERR_ALIGN, "span_tables not 16-byte aligned");
    rc = make_side(d->src, eb, sp.src, sp.src_hstride, "src");
    if (rc != MKV_OK) return rc;
    rc = make_side(d->dst, eb, sp.dst, sp.dst_hstride, "dst");
    if (rc != MKV_OK) return rc;
    sp.spans = d->spans;
    sp.starts = d->span_starts;
    sp.n_spans = d->n_spans;
    sp.tables = d->span_tables;
    // several layers per workgroup only for 2-byte elements: fp8 would hold 16 rows' data
    // across its two passes per wave, fp32 its four passes' (255 VGPRs, 2 waves per SIMD)
    const int direct_layers =
        eb == 2 && d->total_tokens * d->layers > MKV_DIRECT_WIDE_MIN_ROWS
            ? MKV_DIRECT_WIDE_LAYERS
            : 1;
    return launch_any<true>(d->dtype, true, direct_layers, sp, tiles, d->layers, st);
  }

  if (d->order != MKV_ORDER_NONE && d->order != MKV_ORDER_DST_PAGE)
    return fail(MKV_ERR_ARG, "unknown order %d", d->order);
  const bool ordered = d->order == MKV_ORDER_DST_PAGE;
  const int64_t need = workspace_bytes(d->total_tokens, d->n_spans, d->rotary) +
                       (ordered ? MKV_ORDER_EXTRA_BYTES(d->total_tokens) : 0);
  void* ws_ptr = d->workspace;
  int64_t ws_bytes = d->workspace_bytes;
  if (noalloc) {
    if (need > MKV_NOALLOC_SCRATCH_BYTES)
      return fail(MKV_ERR_UNSUPPORTED,
                  "this shift needs %lld bytes of workspace, more than the %lld bytes of "
                  "the no-allocation scratch buffer (use mkv_shift_spans with a workspace)",
                  (long long)need, (long long)MKV_NOALLOC_SCRATCH_BYTES);
    rc = scratch_of(st, &ws_ptr);
    if (rc != MKV_OK) return rc;
    ws_bytes = MKV_NOALLOC_SCRATCH_BYTES;
  }
  if (ws_ptr == nullptr || ws_bytes < need)
    return fail(MKV_ERR_ARG, "workspace of %lld bytes needed (mkv_shift_workspace_size)",
                (long long)need);
  if (!aligned16(reinterpret_cast<uint64_t>(ws_ptr)))
    return fail(MKV_ERR_ALIGN, "workspace not 16-byte aligned");

  PlanParams pp;
  memset(&pp, 0, sizeof pp);
  int64_t src_hs = 0, dst_hs = 0;
  rc = make_side(d->src, eb, pp.src, src_hs, "src");
  if (rc != MKV_OK) return rc;
  rc = make_side(d->dst, eb, pp.dst, dst_hs, "dst");
  if (rc != MKV_OK) return rc;
  char* ws = static_cast<char*>(ws_ptr);
  float* tables = reinterpret_cast<float*>(ws);
  TokRec* recs = reinterpret_cast<TokRec*>(
      ws + align256(static_cast<int64_t>(d->n_spans) * 2 * d->rotary *
                    static_cast<int64_t>(sizeof(float))));
  pp.spans = d->spans;
  pp.inv_freq = d->inv_freq;
  pp.tables = tables;
  pp.recs = recs;
  pp.token_order = d->token_order;
  pp.err = d->error_flags;
  pp.total_tokens = d->total_tokens;
  pp.n_spans = d->n_spans;
  pp.layers = d->layers;
  pp.rotary = d->rotary;

  const int64_t pairs = static_cast<int64_t>(d->n_spans) * (d->rotary / 2);
#if MKV_PLAN_TABLE_GROUPS
  // record workgroups for the tokens, then table workgroups for the (span, frequency) pairs
  const int64_t work = d->total_tokens;
  int64_t tab_grid = (pairs + kPlanThreads - 1) / kPlanThreads;
  if (tab_grid > 256) tab_grid = 256;
#else
  // every workgroup resolves records, then makes tables
  const int64_t work = d->total_tokens > pairs ? d->total_tokens : pairs;
  const int64_t tab_grid = 0;
#endif
  int64_t plan_grid = (work + kPlanThreads - 1) / kPlanThreads;
  if (plan_grid > 4096) plan_grid = 4096;
  if (plan_grid < 1) plan_grid = 1;
  TokRec* sorted = nullptr;
  if (ordered) {  // sorted records, then the page counts, after the plan's records
    int64_t groups = (d->total_tokens + kPlanThreads - 1) / kPlanThreads;
    if (groups > kOrderMaxGroups) groups = kOrderMaxGroups;
    if (groups < 1) groups = 1;
    plan_grid = groups;
    pp.order_chunk = (d->total_tokens + groups - 1) / groups;
    sorted = recs + d->total_tokens;
    pp.order_hist = reinterpret_cast<uint32_t*>(sorted + d->total_tokens);
    // the destination's extent per (group, layer), in bytes, sets the bucket width
    const int64_t cap = pp.dst.num_slots > 0 ? pp.dst.num_slots : 0;
    const int64_t extent = (cap / pp.dst.block_size + 1) * pp.dst.bstride;
    int shift = 21;
    while (shift < 62 && (extent >> shift) >= kOrderBuckets) ++shift;
    pp.order_shift = shift;
  }
  const size_t lds = sizeof(int64_t) * (static_cast<size_t>(d->n_spans) + 1);
  pp.rec_groups = static_cast<int32_t>(plan_grid);  // the order kernel's groups too
  hipLaunchKernelGGL(plan_kernel, dim3(static_cast<unsigned>(plan_grid + tab_grid)),
                     dim3(kPlanThreads), lds, st, pp);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MKV_ERR_HIP, "plan launch failed: %s", hipGetErrorString(e));
  if (ordered) {
    hipLaunchKernelGGL(order_scatter_kernel, dim3(static_cast<unsigned>(plan_grid)),
                       dim3(kScatterThreads), 0, st, recs, sorted, pp.order_hist,
                       d->total_tokens, pp.order_chunk, static_cast<int>(plan_grid),
                       pp.order_shift);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(MKV_ERR_HIP, "order launch failed: %s", hipGetErrorString(e));
    recs = sorted;
  }

  sp.recs = recs;
  sp.tables = tables;
  sp.src_hstride = src_hs;
  sp.dst_hstride = dst_hs;
  sp.layer_groups = d->src.groups >= MKV_LAYER_MAJOR_MIN_GROUPS &&
                    d->total_tokens >= MKV_LAYER_MAJOR_MIN_TOKENS;
  return launch_any<true>(d->dtype, g.uniform, 0, sp, tiles, d->layers, st);
}

template <int DT>
int launch_small(SmallParams& a, int64_t tiles, int layers, hipStream_t stream) {
  tiles = (tiles + MKV_XCDS - 1) / MKV_XCDS * MKV_XCDS;
  if (tiles > 0x7FFFFFFF) return fail(MKV_ERR_UNSUPPORTED, "grid of %lld tiles too large", (long long)tiles);
  a.p.xcd_per = a.p.xcds > 1 ? static_cast<int32_t>(tiles / MKV_XCDS) : 0;
  // LDS for the rotation tables of the spans one workgroup may touch
  const size_t lds = static_cast<size_t>(a.p.n_spans) * 2 * a.p.rotary * sizeof(float);
  hipLaunchKernelGGL(shift_small_kernel<DT>,
                     dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(layers)),
                     dim3(kThreads), lds, stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MKV_ERR_HIP, "launch failed: %s", hipGetErrorString(e));
  return MKV_OK;
}

// One side's index window, from the caller's host array into the launch's int64 window.
int pack_index(const mkv_side_t& in, int64_t* out, const char* name) {
  if (in.mode == MKV_ADDR_FLAT) return MKV_OK;
  if (in.index_len < 0 || in.index_len > MKV_SMALL_MAX_INDEX)
    return fail(MKV_ERR_UNSUPPORTED, "%s: index of %lld entries, more than %d for a small shift",
                name, (long long)in.index_len, MKV_SMALL_MAX_INDEX);
  if (in.index_len > 0 && in.index == nullptr) return fail(MKV_ERR_ARG, "%s: index is NULL", name);
  for (int64_t k = 0; k < in.index_len; ++k)
    out[k] = in.mode == MKV_ADDR_TABLE ? static_cast<const int32_t*>(in.index)[k]
                                       : static_cast<const int64_t*>(in.index)[k];
  return MKV_OK;
}

}  // namespace

extern "C" int mkv_shift_spans(const mkv_shift_desc_t* d, void* stream) {
  return shift_spans(d, stream, false);
}

extern "C" int mkv_shift_spans_small(const mkv_shift_desc_t* d, void* stream) {
  g_err[0] = '\0';
  if (d == nullptr) return fail(MKV_ERR_ARG, "NULL descriptor");
  const int eb = elem_bytes(d->dtype);
  if (eb == 0) return fail(MKV_ERR_DTYPE, "unknown dtype %d", d->dtype);
  Geometry g;
  int rc = check_geometry(d->dtype, d->heads, d->head_size, d->rotary,
                          d->src.head_stride * eb, d->dst.head_stride * eb, g);
  if (rc != MKV_OK) return rc;
  if (d->n_spans < 0 || d->n_spans > MKV_SMALL_MAX_SPANS)
    return fail(MKV_ERR_UNSUPPORTED, "n_spans %d outside [0, %d] for a small shift", d->n_spans,
                MKV_SMALL_MAX_SPANS);
  if (d->total_tokens < 0) return fail(MKV_ERR_ARG, "total_tokens < 0");
  if (d->n_spans == 0 || d->total_tokens == 0) return MKV_OK;
  if (d->spans == nullptr) return fail(MKV_ERR_ARG, "NULL span table");
  if (d->layers <= 0) return fail(MKV_ERR_ARG, "layers %d", d->layers);
  if (d->rotary > 0 && d->inv_freq == nullptr) return fail(MKV_ERR_ARG, "inv_freq is NULL");
  if (d->dtype == MKV_FP8_E4M3 && d->rotary > 0 && d->k_scale == nullptr)
    return fail(MKV_ERR_ARG, "fp8 needs k_scale");
  if (d->src.k_base == nullptr || d->src.v_base == nullptr || d->dst.k_base == nullptr ||
      d->dst.v_base == nullptr)
    return fail(MKV_ERR_ARG, "NULL base-address table");
  if (!g.uniform || ilog2_exact(d->src.block_size) < 0 || ilog2_exact(d->dst.block_size) < 0)
    return fail(MKV_ERR_UNSUPPORTED,
                "a small shift needs power-of-two block sizes and heads a multiple of %d",
                g.rows_per_wave);
  const int64_t tiles = (d->total_tokens + g.tile_tokens - 1) / g.tile_tokens;
  if (tiles > 0x7FFFFFFF) return fail(MKV_ERR_UNSUPPORTED, "total_tokens too large");

  static thread_local SmallParams a;  // ~2 KB: kept off the stack, rewritten every call
  memset(&a, 0, sizeof a);
  int64_t acc = 0;
  for (int k = 0; k < d->n_spans; ++k) {
    a.q.spans[k] = d->spans[k];
    if (d->spans[k].n_tokens < 0)
      return fail(MKV_ERR_ARG, "span %d has n_tokens %d", k, d->spans[k].n_tokens);
    a.q.starts[k] = acc;
    acc += d->spans[k].n_tokens;
  }
  for (int k = d->n_spans; k <= MKV_SMALL_MAX_SPANS; ++k) a.q.starts[k] = acc;
  // the prefix is computed here, so a total that disagrees with it is the caller's error
  // (fewer would leave tokens unmoved, more would launch workgroups with no span)
  if (acc != d->total_tokens)
    return fail(MKV_ERR_ARG, "the spans hold %lld tokens, total_tokens is %lld", (long long)acc,
                (long long)d->total_tokens);
  rc = pack_index(d->src, a.q.src_index, "src");
  if (rc != MKV_OK) return rc;
  rc = pack_index(d->dst, a.q.dst_index, "dst");
  if (rc != MKV_OK) return rc;

  ShiftParams& sp = a.p;
  rc = make_side(d->src, eb, sp.src, sp.src_hstride, "src");
  if (rc != MKV_OK) return rc;
  rc = make_side(d->dst, eb, sp.dst, sp.dst_hstride, "dst");
  if (rc != MKV_OK) return rc;
  sp.src.index = nullptr;  // host arrays: the kernel reads the launch's own windows
  sp.dst.index = nullptr;
  sp.src_k_base = d->src.k_base;
  sp.src_v_base = d->src.v_base;
  sp.dst_k_base = d->dst.k_base;
  sp.dst_v_base = d->dst.v_base;
  sp.k_scale = d->k_scale;
  sp.inv_freq = d->inv_freq;
  sp.err = d->error_flags;
  sp.total_tokens = d->total_tokens;
  sp.layers = d->layers;
  sp.heads = d->heads;
  sp.rotary = d->rotary;
  sp.tile_tokens = g.tile_tokens;
  sp.xcds = g.xcds;
  sp.chunks_per_row = g.chunks_per_row;
  sp.rows_per_wave = g.rows_per_wave;
  sp.heads_magic = g.heads_magic;
  sp.n_spans = d->n_spans;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (d->dtype) {
    case MKV_BF16:
      return launch_small<MKV_BF16>(a, tiles, d->layers, st);
    case MKV_F16:
      return launch_small<MKV_F16>(a, tiles, d->layers, st);
    case MKV_F32:
      return launch_small<MKV_F32>(a, tiles, d->layers, st);
    default:
      return launch_small<MKV_FP8_E4M3>(a, tiles, d->layers, st);
  }
}

extern "C" int mkv_shift_spans_noalloc(const mkv_shift_desc_t* d, void* stream) {
  return shift_spans(d, stream, true);
}
