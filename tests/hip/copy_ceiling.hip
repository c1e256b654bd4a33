// Benchmark and test library (not product code): two copy kernels that set the practical
// ceiling the shift kernel is measured against, with no rotation and as little metadata
// as a copy of each pattern can have.
//
//  * ceil_stream_copy: one contiguous buffer into another, one 16-byte vector per
//    thread, 256-thread workgroups of a one-shot grid dealt so that each XCD walks one
//    contiguous range, non-temporal loads, and stores either non-temporal (global) or
//    device-scope streaming (sc1 nt, through a buffer resource whose base is the
//    workgroup's first byte).
//  * ceil_stream_copy_persistent: the same copy with a fixed grid whose workgroups walk
//    the buffer in grid-sized strides (a persistent kernel), for comparison with the
//    one-shot grid.
//  * ceil_paged_copy: token positions [0, n) of a paged source into positions [0, n) of
//    a paged destination, both through 16-token block tables, every layer: the shift's
//    access pattern (a token's K and V rows of every head, 16 bytes per lane, lane j of a
//    row owning chunk j of K and chunk j of V) with nothing resolved but the two block
//    ids, and no arithmetic on the data.
//  * ceil_paged_copy_ex: ceil_paged_copy with K and V optionally moved by separate waves
//    (a wave pair per row group) and K's store optionally held behind one dependent read
//    of a small table, as the shift's rotation holds it behind its cos/sin table.
//  * ceil_paged_copy_lanes: the same copy with each lane finding its own (token, head)
//    row, so a wave's rows may span tokens (one GPU's 1, 2 or 4 KV heads under tensor
//    parallelism); block ids are per-lane loads and the stores go through the layer's
//    buffer resource (sc1 nt) or plain non-temporal global stores.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef u32x4 __attribute__((address_space(1))) g_u32x4;

constexpr int kXcds = 8;
constexpr int kRsrcRange = -1;
constexpr int kRsrcWord3 = 0x00020000;

// Read-only metadata through the constant address space: a wave-uniform address becomes
// a scalar load, so the buffer stores' bases stay scalar (no waterfall loop).
template <typename T>
__device__ __forceinline__ T ld_const(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

__device__ __forceinline__ u32x4 load_nt(const char* p) {
  return __builtin_nontemporal_load((const g_u32x4*)p);
}

template <int CPOL>
__device__ __forceinline__ void store_at(char* base, uint32_t off, u32x4 v) {
  if constexpr (CPOL < 0) {
    __builtin_nontemporal_store(v, (g_u32x4*)(base + off));
  } else {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, kRsrcRange, kRsrcWord3);
    __builtin_amdgcn_raw_buffer_store_b128(v, r, static_cast<int>(off), 0, CPOL);
  }
}

// blockIdx.x -> tile, each XCD taking one contiguous eighth (gridDim.x is a multiple of 8)
__device__ __forceinline__ int64_t xcd_tile() {
  const int64_t per = gridDim.x / kXcds;
  return (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
}

template <int CPOL>
__global__ __launch_bounds__(256) void stream_copy_kernel(const char* src, char* dst, int64_t n16) {
  const int64_t tile = xcd_tile();
  const int64_t i = tile * 256 + threadIdx.x;
  if (i >= n16) return;
  const u32x4 v = load_nt(src + i * 16);
  store_at<CPOL>(dst + tile * 4096, threadIdx.x * 16u, v);
}

// Persistent: workgroup b copies 4 KB tiles b, b + gridDim.x, ... (256 threads, one
// 16-byte vector each per tile).
template <int CPOL>
__global__ __launch_bounds__(256) void stream_copy_persistent_kernel(const char* src, char* dst,
                                                                      int64_t n16, int64_t tiles) {
  for (int64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const int64_t i = tile * 256 + threadIdx.x;
    if (i < n16) store_at<CPOL>(dst + tile * 4096, threadIdx.x * 16u, load_nt(src + i * 16));
  }
}

struct PagedCopy {
  const uint64_t* src_k;  // [layers] byte addresses
  const uint64_t* src_v;
  const uint64_t* dst_k;
  const uint64_t* dst_v;
  const int32_t* src_table;  // block ids of positions [16 b, 16 b + 16)
  const int32_t* dst_table;
  int64_t src_blocks, dst_blocks;  // blocks each layer's buffer holds
  int64_t n_tokens;
  int64_t s_block, s_head, s_off;  // byte strides
  int64_t d_block, d_head, d_off;
  int32_t heads, chunks, rows_per_wave, tile_tokens;
};

// 128 threads: two waves of rows_per_wave (token, head) rows each; heads is a multiple of
// rows_per_wave, so every wave's rows belong to one token.
__global__ __launch_bounds__(128) void paged_copy_kernel(PagedCopy p) {
  const int64_t tile = xcd_tile();
  const int layer = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row_in_wave = lane / p.chunks;
  const int j = lane - row_in_wave * p.chunks;
  const int row0 = wave * p.rows_per_wave;  // first row of the wave, in the tile
  const int t = row0 / p.heads;
  const int h0 = row0 - t * p.heads;
  const int64_t pos = tile * p.tile_tokens + t;
  if (pos >= p.n_tokens || row_in_wave >= p.rows_per_wave) return;
  const int64_t sb = ld_const(p.src_table + (pos >> 4));
  const int64_t db = ld_const(p.dst_table + (pos >> 4));
  if (sb < 0 || sb >= p.src_blocks || db < 0 || db >= p.dst_blocks) return;
  const int64_t off = pos & 15;
  const int64_t s_row = sb * p.s_block + off * p.s_off + h0 * p.s_head;
  const int64_t d_row = db * p.d_block + off * p.d_off + h0 * p.d_head;
  const uint32_t s_lane = static_cast<uint32_t>(row_in_wave * p.s_head) + j * 16u;
  const uint32_t d_lane = static_cast<uint32_t>(row_in_wave * p.d_head) + j * 16u;
  const char* sk = reinterpret_cast<const char*>(ld_const(p.src_k + layer)) + s_row;
  const char* sv = reinterpret_cast<const char*>(ld_const(p.src_v + layer)) + s_row;
  char* dk = reinterpret_cast<char*>(ld_const(p.dst_k + layer)) + d_row;
  char* dv = reinterpret_cast<char*>(ld_const(p.dst_v + layer)) + d_row;
  const u32x4 k = load_nt(sk + s_lane);
  const u32x4 v = load_nt(sv + s_lane);
  store_at<18>(dk, d_lane, k);
  store_at<18>(dv, d_lane, v);
}

// ceil_paged_copy's rows, two row groups of rows_per_wave rows per workgroup.  SPLIT: 256
// threads, wave w moving only K (w even) or only V (w odd) of row group w / 2; else 128
// threads, each wave moving K and V of its group.  KREAD: K's chunk is stored only after
// a read of k_read[its first word & 15] (zeros, so the copy stays exact) has returned.
template <bool SPLIT, bool KREAD>
__global__ __launch_bounds__(256) void paged_copy_ex_kernel(PagedCopy p, const uint32_t* k_read) {
  const int64_t tile = xcd_tile();
  const int layer = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int group = SPLIT ? wave >> 1 : wave;
  const bool v_only = SPLIT && (wave & 1) != 0;
  const bool k_only = SPLIT && !v_only;
  const int row_in_wave = lane / p.chunks;
  const int j = lane - row_in_wave * p.chunks;
  const int row0 = group * p.rows_per_wave;
  const int t = row0 / p.heads;
  const int h0 = row0 - t * p.heads;
  const int64_t pos = tile * p.tile_tokens + t;
  if (pos >= p.n_tokens || row_in_wave >= p.rows_per_wave) return;
  const int64_t sb = ld_const(p.src_table + (pos >> 4));
  const int64_t db = ld_const(p.dst_table + (pos >> 4));
  if (sb < 0 || sb >= p.src_blocks || db < 0 || db >= p.dst_blocks) return;
  const int64_t off = pos & 15;
  const int64_t s_row = sb * p.s_block + off * p.s_off + h0 * p.s_head;
  const int64_t d_row = db * p.d_block + off * p.d_off + h0 * p.d_head;
  const uint32_t s_lane = static_cast<uint32_t>(row_in_wave * p.s_head) + j * 16u;
  const uint32_t d_lane = static_cast<uint32_t>(row_in_wave * p.d_head) + j * 16u;
  u32x4 k{0, 0, 0, 0}, v{0, 0, 0, 0};
  if (!v_only) k = load_nt(reinterpret_cast<const char*>(ld_const(p.src_k + layer)) + s_row + s_lane);
  if (!k_only) v = load_nt(reinterpret_cast<const char*>(ld_const(p.src_v + layer)) + s_row + s_lane);
  if (KREAD && !v_only) k[0] ^= k_read[k[0] & 15u];
  if (!v_only) store_at<18>(reinterpret_cast<char*>(ld_const(p.dst_k + layer)) + d_row, d_lane, k);
  if (!k_only) store_at<18>(reinterpret_cast<char*>(ld_const(p.dst_v + layer)) + d_row, d_lane, v);
}

// 128 threads: two waves of rows_per_wave rows each, rows (token, head) in token order;
// a lane's token and head come from its own row number.  Destination byte offsets within
// a layer stay below 2^31 (checked on the host), so a layer's base is the store's
// wave-uniform resource and the lane's offset its 32-bit voffset.
template <int CPOL>
__global__ __launch_bounds__(128) void paged_copy_lane_kernel(PagedCopy p) {
  const int64_t tile = xcd_tile();
  const int layer = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row_in_wave = lane / p.chunks;
  const int j = lane - row_in_wave * p.chunks;
  if (row_in_wave >= p.rows_per_wave) return;
  // rows (n_tokens * heads, padded to whole tiles) stay below 2^31: 32-bit division
  const uint32_t row = static_cast<uint32_t>((tile * 2 + wave) * p.rows_per_wave + row_in_wave);
  const uint32_t pos = row / static_cast<uint32_t>(p.heads);
  const int64_t h = row - pos * static_cast<uint32_t>(p.heads);
  if (pos >= p.n_tokens) return;
  const int64_t sb = p.src_table[pos >> 4];
  const int64_t db = p.dst_table[pos >> 4];
  if (sb < 0 || sb >= p.src_blocks || db < 0 || db >= p.dst_blocks) return;
  const int64_t off = pos & 15;
  const int64_t s_at = sb * p.s_block + off * p.s_off + h * p.s_head + j * 16;
  const uint32_t d_at = static_cast<uint32_t>(db * p.d_block + off * p.d_off + h * p.d_head + j * 16);
  const char* sk = reinterpret_cast<const char*>(ld_const(p.src_k + layer));
  const char* sv = reinterpret_cast<const char*>(ld_const(p.src_v + layer));
  char* dk = reinterpret_cast<char*>(ld_const(p.dst_k + layer));
  char* dv = reinterpret_cast<char*>(ld_const(p.dst_v + layer));
  const u32x4 k = load_nt(sk + s_at);
  const u32x4 v = load_nt(sv + s_at);
  store_at<CPOL>(dk, d_at, k);
  store_at<CPOL>(dv, d_at, v);
}

int grid_x(int64_t tiles, unsigned* out) {
  tiles = (tiles + kXcds - 1) / kXcds * kXcds;
  if (tiles <= 0 || tiles > 0x7FFFFFFF) return 1;
  *out = static_cast<unsigned>(tiles);
  return 0;
}

}  // namespace

// bytes: a multiple of 16; both buffers 16-byte aligned.  device_scope: 1 = sc1 nt
// buffer stores, 0 = non-temporal global stores.  Returns 0, or 1 on a bad argument,
// 2 when the launch failed.
extern "C" int ceil_stream_copy(const void* src, void* dst, int64_t bytes, int32_t device_scope,
                                void* stream) {
  if (src == nullptr || dst == nullptr || bytes <= 0 || bytes % 16 != 0 ||
      (reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 != 0)
    return 1;
  const int64_t n16 = bytes / 16;
  unsigned gx = 0;
  if (grid_x((n16 + 255) / 256, &gx) != 0) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (device_scope)
    hipLaunchKernelGGL(stream_copy_kernel<18>, dim3(gx), dim3(256), 0, st,
                       static_cast<const char*>(src), static_cast<char*>(dst), n16);
  else
    hipLaunchKernelGGL(stream_copy_kernel<-1>, dim3(gx), dim3(256), 0, st,
                       static_cast<const char*>(src), static_cast<char*>(dst), n16);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

namespace {

// The two paged copies' shared argument checks; fills p (tile_tokens unset).
int paged_args(PagedCopy& p, const uint64_t* src_k, const uint64_t* src_v, const uint64_t* dst_k,
               const uint64_t* dst_v, int32_t layers, const int32_t* src_table,
               int64_t src_table_len, int64_t src_blocks, const int32_t* dst_table,
               int64_t dst_table_len, int64_t dst_blocks, int64_t n_tokens, int32_t heads,
               int32_t row_bytes, int64_t s_block, int64_t s_head, int64_t s_off, int64_t d_block,
               int64_t d_head, int64_t d_off) {
  if (!src_k || !src_v || !dst_k || !dst_v || !src_table || !dst_table) return 1;
  if (layers <= 0 || layers > 65535 || n_tokens <= 0 || heads <= 0) return 1;
  if (src_blocks <= 0 || dst_blocks <= 0) return 1;
  if (row_bytes <= 0 || row_bytes % 16 != 0 || row_bytes > 1024) return 1;
  const int64_t need = (n_tokens + 15) / 16;
  if (src_table_len < need || dst_table_len < need) return 1;
  const int64_t strides[6] = {s_block, s_head, s_off, d_block, d_head, d_off};
  for (int64_t s : strides)
    if (s < 0 || s % 16 != 0) return 1;
  p.src_k = src_k;
  p.src_v = src_v;
  p.dst_k = dst_k;
  p.dst_v = dst_v;
  p.src_table = src_table;
  p.dst_table = dst_table;
  p.src_blocks = src_blocks;
  p.dst_blocks = dst_blocks;
  p.n_tokens = n_tokens;
  p.s_block = s_block;
  p.s_head = s_head;
  p.s_off = s_off;
  p.d_block = d_block;
  p.d_head = d_head;
  p.d_off = d_off;
  p.heads = heads;
  p.chunks = row_bytes / 16;
  p.rows_per_wave = 64 / p.chunks;
  return 0;
}

}  // namespace

// As ceil_stream_copy (sc1 nt stores) with a fixed grid of `workgroups` workgroups
// (1..65535) walking the buffer.  Returns 0, 1 on a bad argument, 2 on a failed launch.
extern "C" int ceil_stream_copy_persistent(const void* src, void* dst, int64_t bytes,
                                           int32_t workgroups, void* stream) {
  if (src == nullptr || dst == nullptr || bytes <= 0 || bytes % 16 != 0 || workgroups <= 0 ||
      workgroups > 65535 ||
      (reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 != 0)
    return 1;
  const int64_t n16 = bytes / 16;
  const int64_t tiles = (n16 + 255) / 256;
  hipLaunchKernelGGL(stream_copy_persistent_kernel<18>, dim3(static_cast<unsigned>(workgroups)),
                     dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const char*>(src), static_cast<char*>(dst), n16, tiles);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Positions [0, n_tokens) of every layer, block size 16.  Tables hold at least
// ceil(n_tokens / 16) entries (src_table_len, dst_table_len); block ids outside
// [0, *_blocks) skip their rows.  row_bytes: bytes of K (and of V) per (token, head),
// a multiple of 16 of at most 1 KB; heads a multiple of 64 / (row_bytes / 16).  Strides
// in bytes, multiples of 16, lane offsets within 2^31.
extern "C" int ceil_paged_copy(const uint64_t* src_k, const uint64_t* src_v, const uint64_t* dst_k,
                               const uint64_t* dst_v, int32_t layers, const int32_t* src_table,
                               int64_t src_table_len, int64_t src_blocks,
                               const int32_t* dst_table, int64_t dst_table_len,
                               int64_t dst_blocks, int64_t n_tokens, int32_t heads,
                               int32_t row_bytes, int64_t s_block, int64_t s_head, int64_t s_off,
                               int64_t d_block, int64_t d_head, int64_t d_off, void* stream) {
  PagedCopy p;
  if (paged_args(p, src_k, src_v, dst_k, dst_v, layers, src_table, src_table_len, src_blocks,
                 dst_table, dst_table_len, dst_blocks, n_tokens, heads, row_bytes, s_block, s_head,
                 s_off, d_block, d_head, d_off) != 0)
    return 1;
  const int rpw = p.rows_per_wave;
  if (heads % rpw != 0) return 1;
  if ((rpw - 1) * (s_head > d_head ? s_head : d_head) + row_bytes >= (int64_t{1} << 31)) return 1;
  const int rows = 2 * rpw;  // two waves
  p.tile_tokens = rows / heads > 0 ? rows / heads : 1;
  if (p.tile_tokens * heads != rows) return 1;  // a tile is whole tokens
  unsigned gx = 0;
  if (grid_x((n_tokens + p.tile_tokens - 1) / p.tile_tokens, &gx) != 0) return 1;
  hipLaunchKernelGGL(paged_copy_kernel, dim3(gx, static_cast<unsigned>(layers)), dim3(128), 0,
                     static_cast<hipStream_t>(stream), p);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// As ceil_paged_copy; kv_split 1 moves K and V by separate waves, and a non-NULL k_read
// (device, 16 zero words) holds each K store behind one dependent read of it.
extern "C" int ceil_paged_copy_ex(const uint64_t* src_k, const uint64_t* src_v,
                                  const uint64_t* dst_k, const uint64_t* dst_v, int32_t layers,
                                  const int32_t* src_table, int64_t src_table_len,
                                  int64_t src_blocks, const int32_t* dst_table,
                                  int64_t dst_table_len, int64_t dst_blocks, int64_t n_tokens,
                                  int32_t heads, int32_t row_bytes, int64_t s_block,
                                  int64_t s_head, int64_t s_off, int64_t d_block, int64_t d_head,
                                  int64_t d_off, int32_t kv_split, const uint32_t* k_read,
                                  void* stream) {
  PagedCopy p;
  if (paged_args(p, src_k, src_v, dst_k, dst_v, layers, src_table, src_table_len, src_blocks,
                 dst_table, dst_table_len, dst_blocks, n_tokens, heads, row_bytes, s_block, s_head,
                 s_off, d_block, d_head, d_off) != 0)
    return 1;
  const int rpw = p.rows_per_wave;
  if (heads % rpw != 0) return 1;
  if ((rpw - 1) * (s_head > d_head ? s_head : d_head) + row_bytes >= (int64_t{1} << 31)) return 1;
  const int rows = 2 * rpw;  // two row groups
  p.tile_tokens = rows / heads > 0 ? rows / heads : 1;
  if (p.tile_tokens * heads != rows) return 1;  // a tile is whole tokens
  unsigned gx = 0;
  if (grid_x((n_tokens + p.tile_tokens - 1) / p.tile_tokens, &gx) != 0) return 1;
  const dim3 grid(gx, static_cast<unsigned>(layers));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (kv_split && k_read)
    hipLaunchKernelGGL((paged_copy_ex_kernel<true, true>), grid, dim3(256), 0, st, p, k_read);
  else if (kv_split)
    hipLaunchKernelGGL((paged_copy_ex_kernel<true, false>), grid, dim3(256), 0, st, p, k_read);
  else if (k_read)
    hipLaunchKernelGGL((paged_copy_ex_kernel<false, true>), grid, dim3(128), 0, st, p, k_read);
  else
    hipLaunchKernelGGL((paged_copy_ex_kernel<false, false>), grid, dim3(128), 0, st, p, k_read);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// As ceil_paged_copy for any number of heads, each lane resolving its own row.  The
// destination's last byte of a layer ((dst_blocks - 1) * d_block + 15 * d_off +
// (heads - 1) * d_head + row_bytes) must stay below 2^31.  device_scope: 1 = sc1 nt
// buffer stores, 0 = non-temporal global stores.
extern "C" int ceil_paged_copy_lanes(const uint64_t* src_k, const uint64_t* src_v,
                                     const uint64_t* dst_k, const uint64_t* dst_v, int32_t layers,
                                     const int32_t* src_table, int64_t src_table_len,
                                     int64_t src_blocks, const int32_t* dst_table,
                                     int64_t dst_table_len, int64_t dst_blocks, int64_t n_tokens,
                                     int32_t heads, int32_t row_bytes, int64_t s_block,
                                     int64_t s_head, int64_t s_off, int64_t d_block, int64_t d_head,
                                     int64_t d_off, int32_t device_scope, void* stream) {
  PagedCopy p;
  if (paged_args(p, src_k, src_v, dst_k, dst_v, layers, src_table, src_table_len, src_blocks,
                 dst_table, dst_table_len, dst_blocks, n_tokens, heads, row_bytes, s_block, s_head,
                 s_off, d_block, d_head, d_off) != 0)
    return 1;
  const int64_t limit = int64_t{1} << 31;
  if (dst_blocks > limit || d_block > limit || d_off > limit || d_head > limit) return 1;
  const int64_t last = (dst_blocks - 1) * d_block + 15 * d_off + (heads - 1) * d_head + row_bytes;
  if (last >= limit) return 1;
  const int64_t rows = n_tokens * heads;
  const int64_t per_tile = 2 * p.rows_per_wave;
  if (rows > limit - per_tile * kXcds) return 1;
  p.tile_tokens = 0;  // unused: rows, not tokens, make the tiles
  unsigned gx = 0;
  if (grid_x((rows + per_tile - 1) / per_tile, &gx) != 0) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (device_scope)
    hipLaunchKernelGGL(paged_copy_lane_kernel<18>, dim3(gx, static_cast<unsigned>(layers)),
                       dim3(128), 0, st, p);
  else
    hipLaunchKernelGGL(paged_copy_lane_kernel<-1>, dim3(gx, static_cast<unsigned>(layers)),
                       dim3(128), 0, st, p);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
