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
//   * One persistent launch covers every span x every layer.  Work is cut into tiles
//     of (span, layer, run of tile_tokens tokens); a workgroup walks tiles with a
//     grid stride.  The per-span tile prefix lives in LDS (built once per workgroup).
//   * A row is one (layer, token, head): K[D] then V[D].  Lane j of a row owns the
//     16-byte chunk j of K and the 16-byte chunk j of V, so each load/store
//     instruction moves whole, contiguous 16*nK-byte runs (full 128-byte lines).
//   * rotate_half needs chunk j +- rotary/2: it comes from the partner lane through
//     ds_bpermute (no second global read of K).
//   * cos/sin of fl32(delta * inv_freq[f]) are evaluated once per span per workgroup
//     in double precision, rounded to fp32 and kept in LDS; each lane then holds the
//     values of its own chunk in registers.
//   * Loads and stores are non-temporal: every byte is touched exactly once.
//   * Every slot, block id and table index is checked against the capacities given
//     by the caller; a row that fails is skipped and flagged, never accessed.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "marathon_kvshift.h"

#pragma clang fp contract(off)

namespace {

constexpr int kThreads = 256;            // 4 waves of 64
constexpr int kWaves = kThreads / 64;
constexpr int kMaxHalf = MKV_MAX_HEAD_SIZE / 2;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Global-address-space view: keeps the compiler on global_load/global_store rather
// than flat_* (whose counters would also wait on the LDS exchange).
typedef u32x4 __attribute__((address_space(1))) g_u32x4;

// ------------------------------------------------------------------ element traits

template <int DT>
struct Elem;
template <>
struct Elem<MKV_BF16> {
  static constexpr int kBytes = 2, kPerChunk = 8, kUnroll = 4;
};
template <>
struct Elem<MKV_F16> {
  static constexpr int kBytes = 2, kPerChunk = 8, kUnroll = 4;
};
template <>
struct Elem<MKV_F32> {
  static constexpr int kBytes = 4, kPerChunk = 4, kUnroll = 4;
};
template <>
struct Elem<MKV_FP8_E4M3> {
  static constexpr int kBytes = 1, kPerChunk = 16, kUnroll = 2;
};

// -------------------------------------------------------------------- kernel params

struct DevSide {
  const uint64_t* k_base;  // [groups * layers] (batched) or nullptr (single span)
  const uint64_t* v_base;
  uint64_t k_inline;       // single span: K / V base address of the one (group, layer)
  uint64_t v_inline;
  const void* index;
  const int64_t* group_slots;  // per-group num_slots, or nullptr
  int64_t index_len;
  int64_t num_slots;
  int64_t bstride;  // BYTES
  int64_t hstride;  // BYTES
  int64_t ostride;  // BYTES
  int64_t block_size;
  int32_t bs_shift;  // log2(block_size), or -1 when block_size is not a power of two
  int32_t mode;
  int32_t groups;
  int32_t pad;
};

struct KParams {
  const mkv_span_t* spans;  // batched: device table; single span: nullptr
  mkv_span_t one;           // single span, passed by value
  const float* inv_freq;
  const float* k_scale;
  int32_t* err;
  int32_t n_spans;
  int32_t layers;
  int32_t heads;
  int32_t head_size;
  int32_t rotary;
  int32_t tile_tokens;
  int32_t chunks_per_row;  // nK: 16-byte chunks in K (= lanes per row)
  int32_t rows_per_wave;
  uint32_t heads_magic;    // ceil(2^32 / heads): r / heads == umulhi(r, magic) for r < 2^16
  int32_t pad;
  DevSide src;
  DevSide dst;
};

// ------------------------------------------------------------------ small helpers

__device__ __forceinline__ u32x4 load16(const char* p) {
  return __builtin_nontemporal_load((const g_u32x4*)p);
}
__device__ __forceinline__ void store16(char* p, u32x4 v) {
  __builtin_nontemporal_store(v, (g_u32x4*)p);
}

__device__ __forceinline__ uint32_t bpermute(int lane_byte_addr, uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_ds_bpermute(lane_byte_addr, static_cast<int>(v)));
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

// e4m3fn (OCP) decode, exact: sign | 4-bit exponent (bias 7) | 3-bit mantissa;
// exponent 0 is subnormal (m * 2^-9); S.1111.111 is NaN; there is no infinity.
__device__ __forceinline__ float e4m3_decode(uint32_t b) {
  uint32_t s = (b & 0x80u) << 24;
  uint32_t e = (b >> 3) & 0xFu;
  uint32_t m = b & 7u;
  float mag;
  if (e == 0) {
    mag = static_cast<float>(m) * 0x1p-9f;
  } else if (e == 15 && m == 7) {
    return __uint_as_float(0x7FC00000u);
  } else {
    mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
  }
  return __uint_as_float(__float_as_uint(mag) | s);
}

// e4m3fn encode of a value already clamped to [-448, 448] (or NaN), round to nearest
// even.  NaN -> 0x7F.  Subnormals: |x| < 2^-6 encodes rint(|x| * 2^9) (exact scaling,
// so one rounding); the carry into code 8 is the smallest normal, as it should be.
__device__ __forceinline__ uint32_t e4m3_encode(float x) {
  if (x != x) return 0x7Fu;
  uint32_t u = __float_as_uint(x);
  uint32_t sign = (u >> 24) & 0x80u;
  float a = __uint_as_float(u & 0x7FFFFFFFu);
  uint32_t code;
  if (a < 0x1p-6f) {
    code = static_cast<uint32_t>(__builtin_rintf(a * 512.0f));
  } else {
    uint32_t v = __float_as_uint(a);
    v = v + 0x7FFFFu + ((v >> 20) & 1u);  // RNE at mantissa bit 20
    uint32_t e = (v >> 23) - 120u;        // rebias 127 -> 7
    code = (e << 3) | ((v >> 20) & 7u);
  }
  return code | sign;
}

__device__ __forceinline__ float clamp448(float q) {
  return q > 448.0f ? 448.0f : (q < -448.0f ? -448.0f : q);
}

// Rotate the C elements of one 16-byte chunk.  `mine` is this lane's K chunk,
// `part` the partner chunk (same element positions, other half of the rotation).
template <int DT>
struct Rotor;

template <>
struct Rotor<MKV_BF16> {
  static __device__ __forceinline__ u32x4 run(u32x4 mine, u32x4 part, const float* c,
                                              const float* s, float, float) {
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
                                              const float* s, float, float) {
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
                                              const float* s, float, float) {
    u32x4 out;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float y = rot1(__uint_as_float(mine[w]), __uint_as_float(part[w]), c[w], s[w]);
      out[w] = (y != y) ? 0x7FC00000u : __float_as_uint(y);
    }
    return out;
  }
};

template <>
struct Rotor<MKV_FP8_E4M3> {
  static __device__ __forceinline__ u32x4 run(u32x4 mine, u32x4 part, const float* c,
                                              const float* s, float scale, float) {
    u32x4 out;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t word = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int e = 4 * w + b;
        float x = e4m3_decode((mine[w] >> (8 * b)) & 0xFFu) * scale;
        float xp = e4m3_decode((part[w] >> (8 * b)) & 0xFFu) * scale;
        float y = rot1(x, xp, c[e], s[e]);
        word |= e4m3_encode(clamp448(y / scale)) << (8 * b);
      }
      out[w] = word;
    }
    return out;
  }
};

// Slot of token i of a span on one side; false when any index is out of range.
__device__ __forceinline__ bool resolve(const DevSide& sd, int64_t cap, int64_t cap_blocks,
                                        int64_t pos0, int64_t index0, int64_t i, int64_t& blk,
                                        int64_t& off) {
  int64_t slot;
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
    return true;
  }
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
  return true;
}

__device__ __forceinline__ int64_t span_tiles(const mkv_span_t& sp, const KParams& p) {
  if (sp.n_tokens <= 0) return 0;
  if (sp.src_group < 0 || sp.src_group >= p.src.groups) return 0;
  if (sp.dst_group < 0 || sp.dst_group >= p.dst.groups) return 0;
  return static_cast<int64_t>(p.layers) *
         ((static_cast<int64_t>(sp.n_tokens) + p.tile_tokens - 1) / p.tile_tokens);
}

__device__ __forceinline__ bool span_bad(const mkv_span_t& sp, const KParams& p) {
  return sp.n_tokens < 0 || sp.src_group < 0 || sp.src_group >= p.src.groups ||
         sp.dst_group < 0 || sp.dst_group >= p.dst.groups;
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

// ------------------------------------------------------------------------- kernel

template <int DT, bool SINGLE>
__global__ __launch_bounds__(kThreads) void shift_kernel(KParams p) {
  using E = Elem<DT>;
  constexpr int C = E::kPerChunk;
  constexpr int U = E::kUnroll;

  extern __shared__ int64_t s_prefix[];  // batched: tile prefix [n_spans + 1]
  __shared__ float s_cos[kMaxHalf];
  __shared__ float s_sin[kMaxHalf];
  __shared__ int64_t s_part[kThreads];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nK = p.chunks_per_row;
  const int rpw = p.rows_per_wave;
  const int row_in_wave = lane / nK;
  const int j = lane - row_in_wave * nK;  // chunk index inside K (and inside V)
  const bool lane_live = row_in_wave < rpw;
  const int wg_rows = rpw * kWaves;
  const int wg_row = wave * rpw + row_in_wave;
  const int P = p.rotary / (2 * C);  // rotate_half distance, in chunks
  const bool rot_lane = j < 2 * P;
  const int partner = j < P ? lane + P : (rot_lane ? lane - P : lane);
  const int partner_addr = partner * 4;
  const int64_t chunk_off = static_cast<int64_t>(j) * 16;
  const int H = p.heads;
  const int half = p.rotary / 2;

  // ---- tile prefix over spans
  int64_t total;
  if constexpr (SINGLE) {
    total = span_tiles(p.one, p);
  } else {
    const int n = p.n_spans;
    const int per = (n + kThreads - 1) / kThreads;
    const int b = tid * per;
    const int e = min(b + per, n);
    int64_t sum = 0;
    bool bad = false;
    for (int i = b; i < e; ++i) {
      const mkv_span_t sp = p.spans[i];
      sum += span_tiles(sp, p);
      bad |= span_bad(sp, p);
    }
    if (bad && p.err != nullptr && blockIdx.x == 0) atomicOr(p.err, MKV_FLAG_SPAN);
    s_part[tid] = sum;
    __syncthreads();
    for (int off = 1; off < kThreads; off <<= 1) {
      const int64_t v = tid >= off ? s_part[tid - off] : 0;
      __syncthreads();
      s_part[tid] += v;
      __syncthreads();
    }
    int64_t run = s_part[tid] - sum;
    for (int i = b; i < e; ++i) {
      s_prefix[i] = run;
      run += span_tiles(p.spans[i], p);
    }
    if (tid == kThreads - 1) s_prefix[n] = s_part[kThreads - 1];
    __syncthreads();
    total = s_prefix[n];
  }

  int cur = -1;
  mkv_span_t sp = p.one;
  int64_t sp_t0 = 0, sp_t1 = 0, chunks = 1;
  bool rotate = false;
  float cs[C], sg[C];
#pragma unroll
  for (int e = 0; e < C; ++e) cs[e] = 1.0f, sg[e] = 0.0f;

  for (int64_t tile = blockIdx.x; tile < total; tile += gridDim.x) {
    if (tile >= sp_t1) {
      // advance to the span holding this tile (tiles only move forward)
      int s;
      if constexpr (SINGLE) {
        s = 0;
        sp_t0 = 0;
        sp_t1 = total;
      } else {
        s = cur + 1;
        while (s_prefix[s + 1] <= tile) ++s;
        s = uniform(s);
        sp = p.spans[s];
        sp_t0 = s_prefix[s];
        sp_t1 = s_prefix[s + 1];
      }
      cur = s;
      chunks = (static_cast<int64_t>(sp.n_tokens) + p.tile_tokens - 1) / p.tile_tokens;
      rotate = sp.delta != 0 && p.rotary > 0;
      if (rotate) {
        __syncthreads();  // nobody still reads the previous span's table
        for (int f = tid; f < half; f += kThreads) {
          const float ang = static_cast<float>(sp.delta) * p.inv_freq[f];
          double sd, cd;
          sincos(static_cast<double>(ang), &sd, &cd);
          s_cos[f] = static_cast<float>(cd);
          s_sin[f] = static_cast<float>(sd);
        }
        __syncthreads();
        if (rot_lane) {
          const bool first = j < P;
#pragma unroll
          for (int e = 0; e < C; ++e) {
            int f = j * C + e;
            if (f >= half) f -= half;
            cs[e] = s_cos[f];
            sg[e] = first ? -s_sin[f] : s_sin[f];
          }
        }
      }
    }

    // tile counts stay far below 2^31 (a span holds < 2^31 tokens), so 32-bit math
    const uint32_t local = static_cast<uint32_t>(tile - sp_t0);
    const uint32_t layer = local / static_cast<uint32_t>(chunks);
    const int64_t tok0 =
        static_cast<int64_t>(local - layer * static_cast<uint32_t>(chunks)) * p.tile_tokens;
    const int ntok = static_cast<int>(min(static_cast<int64_t>(p.tile_tokens),
                                          static_cast<int64_t>(sp.n_tokens) - tok0));
    const int nrows = ntok * H;

    const char* sk;
    const char* sv;
    char* dk;
    char* dv;
    if constexpr (SINGLE) {
      sk = reinterpret_cast<const char*>(p.src.k_inline);
      sv = reinterpret_cast<const char*>(p.src.v_inline);
      dk = reinterpret_cast<char*>(p.dst.k_inline);
      dv = reinterpret_cast<char*>(p.dst.v_inline);
    } else {
      const int64_t si = static_cast<int64_t>(sp.src_group) * p.layers + layer;
      const int64_t di = static_cast<int64_t>(sp.dst_group) * p.layers + layer;
      sk = reinterpret_cast<const char*>(p.src.k_base[si]);
      sv = reinterpret_cast<const char*>(p.src.v_base[si]);
      dk = reinterpret_cast<char*>(p.dst.k_base[di]);
      dv = reinterpret_cast<char*>(p.dst.v_base[di]);
    }
    if (((reinterpret_cast<uint64_t>(sk) | reinterpret_cast<uint64_t>(sv) |
          reinterpret_cast<uint64_t>(dk) | reinterpret_cast<uint64_t>(dv)) & 15u) != 0) {
      if (p.err != nullptr && tid == 0) atomicOr(p.err, MKV_FLAG_ALIGN);
      continue;  // uniform: the whole workgroup skips this tile
    }
    int64_t s_cap = p.src.num_slots, d_cap = p.dst.num_slots;
    if constexpr (!SINGLE) {
      if (p.src.group_slots != nullptr) s_cap = p.src.group_slots[sp.src_group];
      if (p.dst.group_slots != nullptr) d_cap = p.dst.group_slots[sp.dst_group];
    }
    // block capacity of a TABLE side, once per tile (block ids are checked against it)
    const int64_t s_cap_blocks = s_cap / p.src.block_size;
    const int64_t d_cap_blocks = d_cap / p.dst.block_size;
    float scale = 1.0f;
    if constexpr (DT == MKV_FP8_E4M3) {
      if (rotate) scale = p.k_scale[layer];  // k_scale may be NULL when nothing rotates
    }

    for (int r0 = 0; r0 < nrows; r0 += wg_rows * U) {
      u32x4 kd[U], vd[U];
      int64_t doff[U];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = r0 + u * wg_rows + wg_row;
        ok[u] = lane_live && r < nrows;
        kd[u] = u32x4{0, 0, 0, 0};
        vd[u] = u32x4{0, 0, 0, 0};
        doff[u] = 0;
        if (ok[u]) {
          const int t = H == 1 ? r
                               : static_cast<int>(__umulhi(static_cast<uint32_t>(r), p.heads_magic));
          const int h = r - t * H;
          const int64_t ti = tok0 + t;
          int64_t sb, so, db, dof;
          const bool s_ok =
              resolve(p.src, s_cap, s_cap_blocks, sp.src_pos, sp.src_index, ti, sb, so);
          const bool d_ok =
              resolve(p.dst, d_cap, d_cap_blocks, sp.dst_pos, sp.dst_index, ti, db, dof);
          if (!(s_ok && d_ok)) {
            if (p.err != nullptr)
              atomicOr(p.err, (s_ok ? 0 : MKV_FLAG_SRC_RANGE) | (d_ok ? 0 : MKV_FLAG_DST_RANGE));
            ok[u] = false;
          } else {
            const int64_t soff = sb * p.src.bstride + so * p.src.ostride + h * p.src.hstride + chunk_off;
            doff[u] = db * p.dst.bstride + dof * p.dst.ostride + h * p.dst.hstride + chunk_off;
            kd[u] = load16(sk + soff);
            vd[u] = load16(sv + soff);
          }
        }
      }
      if (rotate) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          u32x4 pd;
          pd[0] = bpermute(partner_addr, kd[u][0]);
          pd[1] = bpermute(partner_addr, kd[u][1]);
          pd[2] = bpermute(partner_addr, kd[u][2]);
          pd[3] = bpermute(partner_addr, kd[u][3]);
          if (rot_lane) kd[u] = Rotor<DT>::run(kd[u], pd, cs, sg, scale, 0.0f);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (ok[u]) {
          store16(dk + doff[u], kd[u]);
          store16(dv + doff[u], vd[u]);
        }
      }
    }
  }
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

struct DevInfo {
  int cus = 0;
};

std::mutex g_mu;
DevInfo g_dev[64];

int device_cus(int dev) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (dev < 0 || dev >= 64) return 0;
  if (g_dev[dev].cus == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    g_dev[dev].cus = cus;
  }
  return g_dev[dev].cus;
}

bool aligned16(uint64_t v) { return (v & 15u) == 0; }

// Validate one side's geometry and convert it to the device form.
int make_side(const mkv_side_t& in, int eb, bool single, DevSide& out, const char* name) {
  memset(&out, 0, sizeof out);
  if (in.mode != MKV_ADDR_FLAT && in.mode != MKV_ADDR_SLOTS && in.mode != MKV_ADDR_TABLE)
    return fail(MKV_ERR_ARG, "%s: unknown addressing mode %d", name, in.mode);
  if (in.block_size <= 0) return fail(MKV_ERR_ARG, "%s: block_size %d", name, in.block_size);
  if (in.num_slots < 0) return fail(MKV_ERR_ARG, "%s: num_slots < 0", name);
  if (in.mode != MKV_ADDR_FLAT && in.index == nullptr && in.index_len > 0)
    return fail(MKV_ERR_ARG, "%s: index is NULL", name);
  if (!single && (in.k_base == nullptr || in.v_base == nullptr))
    return fail(MKV_ERR_ARG, "%s: base-address table is NULL", name);
  if (!single && in.groups <= 0) return fail(MKV_ERR_ARG, "%s: groups %d", name, in.groups);
  const int64_t bs = static_cast<int64_t>(in.block_stride) * eb;
  const int64_t hs = static_cast<int64_t>(in.head_stride) * eb;
  const int64_t os = static_cast<int64_t>(in.offset_stride) * eb;
  if (!aligned16(static_cast<uint64_t>(bs)) || !aligned16(static_cast<uint64_t>(hs)) ||
      !aligned16(static_cast<uint64_t>(os)))
    return fail(MKV_ERR_ALIGN, "%s: byte strides (%lld, %lld, %lld) not 16-byte aligned", name,
                (long long)bs, (long long)hs, (long long)os);
  out.k_base = in.k_base;
  out.v_base = in.v_base;
  out.index = in.index;
  out.group_slots = single ? nullptr : in.group_slots;
  out.index_len = in.index == nullptr ? 0 : in.index_len;
  out.num_slots = in.num_slots;
  out.bstride = bs;
  out.hstride = hs;
  out.ostride = os;
  out.block_size = in.block_size;
  out.bs_shift = ilog2_exact(in.block_size);
  out.mode = in.mode;
  out.groups = single ? 1 : in.groups;
  return MKV_OK;
}

struct Geometry {
  int chunks_per_row;
  int rows_per_wave;
  int tile_tokens;
  uint32_t heads_magic;
};

int check_geometry(int dtype, int heads, int head_size, int rotary, Geometry& g) {
  const int eb = elem_bytes(dtype);
  if (eb == 0) return fail(MKV_ERR_DTYPE, "unknown dtype %d", dtype);
  if (heads <= 0) return fail(MKV_ERR_ARG, "heads %d", heads);
  if (head_size <= 0 || head_size > MKV_MAX_HEAD_SIZE)
    return fail(MKV_ERR_UNSUPPORTED, "head_size %d outside (0, %d]", head_size, MKV_MAX_HEAD_SIZE);
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
  int unroll = dtype == MKV_FP8_E4M3 ? Elem<MKV_FP8_E4M3>::kUnroll : 4;
  const int rows = g.rows_per_wave * kWaves * unroll;
  g.tile_tokens = rows / heads > 0 ? rows / heads : 1;
  // the row -> (token, head) split uses a 32-bit reciprocal, exact while
  // tile_tokens * heads < 2^16 and heads < 2^16
  if (static_cast<int64_t>(g.tile_tokens) * heads >= (1 << 16))
    return fail(MKV_ERR_UNSUPPORTED, "heads %d too large", heads);
  g.heads_magic =
      heads == 1 ? 0u : static_cast<uint32_t>(((uint64_t{1} << 32) + heads - 1) / heads);
  return MKV_OK;
}

template <int DT, bool SINGLE>
int launch_typed(const KParams& kp, int64_t single_tiles, size_t lds, hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(MKV_ERR_HIP, "hipGetDevice failed");
  const int cus = device_cus(dev);
  if (cus <= 0) return fail(MKV_ERR_HIP, "could not query the CU count of device %d", dev);
  int per_cu = 0;
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
      &per_cu, reinterpret_cast<const void*>(&shift_kernel<DT, SINGLE>), kThreads, lds);
  if (e != hipSuccess || per_cu <= 0) per_cu = 1;
  int64_t grid = static_cast<int64_t>(cus) * per_cu;
  if (SINGLE && single_tiles < grid) grid = single_tiles;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL((shift_kernel<DT, SINGLE>), dim3(static_cast<unsigned>(grid)),
                     dim3(kThreads), lds, stream, kp);
  e = hipGetLastError();
  if (e != hipSuccess) return fail(MKV_ERR_HIP, "launch failed: %s", hipGetErrorString(e));
  return MKV_OK;
}

template <bool SINGLE>
int launch(int dtype, const KParams& kp, int64_t single_tiles, size_t lds, hipStream_t stream) {
  switch (dtype) {
    case MKV_BF16:
      return launch_typed<MKV_BF16, SINGLE>(kp, single_tiles, lds, stream);
    case MKV_F16:
      return launch_typed<MKV_F16, SINGLE>(kp, single_tiles, lds, stream);
    case MKV_F32:
      return launch_typed<MKV_F32, SINGLE>(kp, single_tiles, lds, stream);
    case MKV_FP8_E4M3:
      return launch_typed<MKV_FP8_E4M3, SINGLE>(kp, single_tiles, lds, stream);
    default:
      return fail(MKV_ERR_DTYPE, "unknown dtype %d", dtype);
  }
}

}  // namespace

// ------------------------------------------------------------------------ C ABI

extern "C" const char* mkv_last_error(void) { return g_err; }

extern "C" int32_t mkv_abi_version(void) { return MKV_ABI_VERSION; }

extern "C" int mkv_scatter_shifted(const void* src, int64_t src_token_stride,
                                   int64_t src_head_stride, void* kv, int64_t kv_block_stride,
                                   int64_t kv_head_stride, int64_t kv_offset_stride,
                                   int64_t kv_num_blocks, const int64_t* slots,
                                   int64_t n_tokens, int32_t heads, int32_t head_size,
                                   int32_t block_size, int32_t dtype, const float* inv_freq,
                                   int32_t rotary, int32_t delta, const float* k_scale,
                                   int32_t* error_flags, void* stream) {
  g_err[0] = '\0';
  Geometry g;
  int rc = check_geometry(dtype, heads, head_size, rotary, g);
  if (rc != MKV_OK) return rc;
  if (n_tokens < 0) return fail(MKV_ERR_ARG, "n_tokens %lld < 0", (long long)n_tokens);
  if (n_tokens > INT32_MAX) return fail(MKV_ERR_UNSUPPORTED, "n_tokens exceeds 2^31-1");
  if (n_tokens == 0) return MKV_OK;  // the reference returns early (shift_kernels.py:185)
  if (src == nullptr || kv == nullptr || slots == nullptr)
    return fail(MKV_ERR_ARG, "NULL src, kv or slots");
  if (block_size <= 0) return fail(MKV_ERR_ARG, "block_size %d", block_size);
  if (kv_num_blocks < 0) return fail(MKV_ERR_ARG, "kv_num_blocks < 0");
  const bool rot = delta != 0 && rotary > 0;
  if (rot && inv_freq == nullptr) return fail(MKV_ERR_ARG, "inv_freq is NULL");
  if (dtype == MKV_FP8_E4M3 && rot && k_scale == nullptr)
    return fail(MKV_ERR_ARG, "fp8 needs k_scale");
  const int eb = elem_bytes(dtype);
  const uint64_t s0 = reinterpret_cast<uint64_t>(src);
  const uint64_t d0 = reinterpret_cast<uint64_t>(kv);
  const uint64_t vofs = static_cast<uint64_t>(head_size) * eb;
  if (!aligned16(s0) || !aligned16(d0))
    return fail(MKV_ERR_ALIGN, "src or kv base address not 16-byte aligned");

  mkv_side_t s_in{};
  s_in.index = nullptr;
  s_in.num_slots = n_tokens;
  s_in.block_stride = src_token_stride;
  s_in.head_stride = src_head_stride;
  s_in.offset_stride = 0;
  s_in.block_size = 1;
  s_in.mode = MKV_ADDR_FLAT;
  mkv_side_t d_in{};
  d_in.index = slots;
  d_in.index_len = n_tokens;
  d_in.num_slots = kv_num_blocks * static_cast<int64_t>(block_size);
  d_in.block_stride = kv_block_stride;
  d_in.head_stride = kv_head_stride;
  d_in.offset_stride = kv_offset_stride;
  d_in.block_size = block_size;
  d_in.mode = MKV_ADDR_SLOTS;

  KParams kp;
  memset(&kp, 0, sizeof kp);
  rc = make_side(s_in, eb, true, kp.src, "src");
  if (rc != MKV_OK) return rc;
  rc = make_side(d_in, eb, true, kp.dst, "dst");
  if (rc != MKV_OK) return rc;
  kp.src.k_inline = s0;
  kp.src.v_inline = s0 + vofs;
  kp.dst.k_inline = d0;
  kp.dst.v_inline = d0 + vofs;
  kp.spans = nullptr;
  kp.one.src_pos = 0;
  kp.one.dst_pos = 0;
  kp.one.src_index = 0;
  kp.one.dst_index = 0;
  kp.one.n_tokens = static_cast<int32_t>(n_tokens);
  kp.one.delta = rot ? delta : 0;
  kp.one.src_group = 0;
  kp.one.dst_group = 0;
  kp.inv_freq = inv_freq;
  kp.k_scale = k_scale;
  kp.err = error_flags;
  kp.n_spans = 1;
  kp.layers = 1;
  kp.heads = heads;
  kp.head_size = head_size;
  kp.rotary = rot ? rotary : 0;
  kp.tile_tokens = g.tile_tokens;
  kp.chunks_per_row = g.chunks_per_row;
  kp.rows_per_wave = g.rows_per_wave;
  kp.heads_magic = g.heads_magic;
  const int64_t tiles = (n_tokens + g.tile_tokens - 1) / g.tile_tokens;
  return launch<true>(dtype, kp, tiles, 0, static_cast<hipStream_t>(stream));
}

extern "C" int mkv_shift_spans(const mkv_shift_desc_t* d, void* stream) {
  g_err[0] = '\0';
  if (d == nullptr) return fail(MKV_ERR_ARG, "NULL descriptor");
  Geometry g;
  int rc = check_geometry(d->dtype, d->heads, d->head_size, d->rotary, g);
  if (rc != MKV_OK) return rc;
  if (d->n_spans < 0 || d->n_spans > MKV_MAX_SPANS)
    return fail(MKV_ERR_UNSUPPORTED, "n_spans %d outside [0, %d]", d->n_spans, MKV_MAX_SPANS);
  if (d->n_spans == 0) return MKV_OK;
  if (d->spans == nullptr) return fail(MKV_ERR_ARG, "NULL span table");
  if (d->layers <= 0) return fail(MKV_ERR_ARG, "layers %d", d->layers);
  if (d->rotary > 0 && d->inv_freq == nullptr) return fail(MKV_ERR_ARG, "inv_freq is NULL");
  if (d->dtype == MKV_FP8_E4M3 && d->rotary > 0 && d->k_scale == nullptr)
    return fail(MKV_ERR_ARG, "fp8 needs k_scale");
  const int eb = elem_bytes(d->dtype);
  KParams kp;
  memset(&kp, 0, sizeof kp);
  rc = make_side(d->src, eb, false, kp.src, "src");
  if (rc != MKV_OK) return rc;
  rc = make_side(d->dst, eb, false, kp.dst, "dst");
  if (rc != MKV_OK) return rc;
  kp.spans = d->spans;
  kp.inv_freq = d->inv_freq;
  kp.k_scale = d->k_scale;
  kp.err = d->error_flags;
  kp.n_spans = d->n_spans;
  kp.layers = d->layers;
  kp.heads = d->heads;
  kp.head_size = d->head_size;
  kp.rotary = d->rotary;
  kp.tile_tokens = g.tile_tokens;
  kp.chunks_per_row = g.chunks_per_row;
  kp.rows_per_wave = g.rows_per_wave;
  kp.heads_magic = g.heads_magic;
  const size_t lds = sizeof(int64_t) * (static_cast<size_t>(d->n_spans) + 1);
  return launch<false>(d->dtype, kp, 0, lds, static_cast<hipStream_t>(stream));
}
