/*
 * marathon_kvshift.h -- C ABI of the MI355X (gfx950) KV-shift library.
 *
 * The library moves reused spans of cached K/V into a paged KV cache.  For every
 * (layer, token, KV head) row it reads K[head_size] and V[head_size] from the source,
 * re-rotates K by the span's token offset delta with NeoX rotate-half RoPE
 *
 *     out[i] = RN(RN(k[i] * cos[i]) + RN(k[partner(i)] * sgn[i]))       (fp32, no FMA)
 *     partner(i) = i + rotary/2 (i < rotary/2),  i - rotary/2 (rotary/2 <= i < rotary)
 *     sgn[i]     = -sin(a[i mod rotary/2]) (i < rotary/2),  +sin(...) (otherwise)
 *     a[f]       = fl32((float)delta * inv_freq[f])
 *
 * rounds K back to the cache element type (RNE), copies V bit for bit, and writes the
 * row at its destination slot (block = slot / block_size, offset = slot % block_size).
 * Dimensions at or above `rotary`, and every element of a delta == 0 span, are copied
 * bit for bit.  cos/sin are the cosine and sine of the fp32 angle evaluated in double
 * precision and rounded to fp32, by one routine for the device and the host
 * (marathon_amd/csrc/rope_angle.h; mkv_rope_tables below), so every path's tables hold
 * the same bits.
 *
 * Conventions shared by every entry point:
 *   - All pointers named "device" are HIP device addresses; nothing is allocated and
 *     nothing is synchronised (the batched entry point works in a caller-provided
 *     device workspace).  Work is enqueued on `stream` (a hipStream_t; NULL is
 *     the legacy default stream) and the call returns as soon as it is enqueued.
 *   - Strides are in ELEMENTS of the cache element type.  16-byte alignment of every
 *     base address and of every stride in bytes is required (MKV_ERR_ALIGN otherwise).
 *   - Every slot, block id and block-table index is bounds-checked on the device
 *     against the capacities given here; a row that fails is not read or written and,
 *     when `error_flags` is non-NULL, sets MKV_FLAG_* bits there (atomic OR).
 *   - Return value: MKV_OK or one of the MKV_ERR_* codes below; on error nothing was
 *     enqueued.  mkv_last_error() returns a human-readable reason for the last error
 *     raised on the calling thread.
 *
 * Element types (`dtype`): bf16, fp16 and fp32 rotate in fp32 and round to nearest
 * even (NaN -> canonical quiet NaN); fp8 e4m3fn (OCP, max 448) dequantises K with the
 * per-layer scale, rotates in fp32 and requantises:
 *     x = fl32(decode(code) * k_scale[layer]);   y = rotation of x as above;
 *     q = e4m3fn_RNE(clamp(fl32(y / k_scale[layer]), -448, 448))   (NaN -> 0x7F)
 * The quotient is evaluated without a division per element (marathon_amd/csrc/fp8_e4m3.h:
 * the reciprocal split in two, then one Markstein correction); it equals the correctly
 * rounded fl32(y / k_scale) for every finite y at every k_scale in [2^-90, 2^100], the
 * range a K scale must lie in.
 * V bytes are copied raw for every element type.
 */
#ifndef MARATHON_KVSHIFT_H
#define MARATHON_KVSHIFT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------------- */
#define MKV_OK 0
#define MKV_ERR_ARG 1         /* geometry or argument rejected (row size, rotary, NULL) */
#define MKV_ERR_DTYPE 2       /* unknown element type */
#define MKV_ERR_ALIGN 3       /* a base address or byte stride is not 16-byte aligned */
#define MKV_ERR_UNSUPPORTED 4 /* geometry outside what the kernels handle */
#define MKV_ERR_HIP 5         /* the HIP runtime refused the launch */

/* ---- device error flags (bits OR-ed into *error_flags) ---------------------------- */
#define MKV_FLAG_SRC_RANGE 1  /* a source slot / block id / table index out of range */
#define MKV_FLAG_DST_RANGE 2  /* a destination slot / block id / table index out of range */
#define MKV_FLAG_SPAN 4       /* a span with n_tokens < 0 or a group id out of range */
#define MKV_FLAG_ALIGN 8      /* a base address from a k_base/v_base table not 16-byte aligned */

/* ---- element types ---------------------------------------------------------------- */
#define MKV_BF16 0
#define MKV_F16 1
#define MKV_F32 2
#define MKV_FP8_E4M3 3

/* ---- how one side maps a token position to a slot -------------------------------- */
#define MKV_ADDR_FLAT 0  /* slot = position (a position-indexed store, block_size 1) */
#define MKV_ADDR_SLOTS 1 /* slot = ((const int64_t*)index)[span.*_index + i] */
#define MKV_ADDR_TABLE 2 /* slot = tbl[span.*_index + pos / bs] * bs + pos % bs,
                            tbl = (const int32_t*)index, pos = span.*_pos + i */

/* Token orders of the batched entry point (mkv_shift_desc_t.order). */
#define MKV_ORDER_NONE 0
#define MKV_ORDER_DST_PAGE 1
#define MKV_ORDER_EXTRA_BYTES(total_tokens) ((int64_t)(total_tokens) * 32 + (1 << 20))

/* Limits of the batched entry point. */
#define MKV_MAX_SPANS 4096
#define MKV_MAX_HEAD_SIZE 512
#define MKV_DIRECT_MAX_SPANS 63 /* spans of a direct (single-launch) shift */
#define MKV_SMALL_MAX_SPANS 8   /* spans of a small shift (mkv_shift_spans_small) */
#define MKV_SMALL_MAX_INDEX 64  /* index entries per side of a small shift */

/*
 * One reused span: n_tokens consecutive tokens whose K moves by `delta` positions.
 * Token i of the span is read at source position src_pos + i and written at
 * destination position dst_pos + i (FLAT/TABLE), or through the slot arrays at
 * src_index + i / dst_index + i (SLOTS).  src_group / dst_group select the row of the
 * side's base-address tables (for example the session whose store holds the span).
 * 48 bytes, naturally aligned; arrays of it are read by the device.
 */
typedef struct mkv_span {
  int64_t src_pos;
  int64_t dst_pos;
  int64_t src_index;
  int64_t dst_index;
  int32_t n_tokens;
  int32_t delta;
  int32_t src_group;
  int32_t dst_group;
} mkv_span_t;

/*
 * One side (source or destination) of a batched shift.
 *   k_base, v_base : device arrays [groups * layers] of byte addresses of element 0 of
 *                    K and V for (group, layer), row-major in group.  For the fused
 *                    [..., 2 * head_size] layout v_base = k_base + head_size elements.
 *   index          : device int64 slots (SLOTS) or int32 block ids (TABLE); NULL (FLAT).
 *   index_len      : number of entries in `index`.
 *   num_slots      : slots one (group, layer) buffer holds: blocks * block_size, or
 *                    rows for FLAT.
 *   group_slots    : optional device int64 [groups]: per-group num_slots (groups whose
 *                    buffers differ in size, e.g. sessions' stores); NULL = num_slots.
 *   block_stride, head_stride, offset_stride : element strides of (block, head,
 *                    in-block offset).  FLAT uses block_size 1 and block_stride = the
 *                    token stride.
 */
typedef struct mkv_side {
  const uint64_t* k_base;
  const uint64_t* v_base;
  const void* index;
  const int64_t* group_slots;
  int64_t index_len;
  int64_t num_slots;
  int64_t block_stride;
  int64_t head_stride;
  int64_t offset_stride;
  int32_t block_size;
  int32_t mode;
  int32_t groups;
  int32_t reserved;
} mkv_side_t;

/*
 * A batched shift: every span x every layer, enqueued as two launches (a small plan
 * kernel that resolves every token's source and destination row and each span's
 * cos/sin into the workspace, then the shift itself).
 *   spans        : device [n_spans], 0 <= n_spans <= MKV_MAX_SPANS.
 *   total_tokens : sum of the spans' n_tokens, known to the caller (it sizes the
 *                  launch and the workspace); tokens beyond it are not moved and raise
 *                  MKV_FLAG_SPAN.
 *   inv_freq     : device fp32 [rotary / 2]; may be NULL when rotary == 0.
 *   k_scale      : device fp32 [layers] for MKV_FP8_E4M3 when rotary > 0, each in
 *                  [2^-90, 2^100]; otherwise ignored and may be NULL (with rotary 0 every
 *                  K byte is copied).
 *   error_flags  : device int32 [1] or NULL.
 *   workspace    : device, >= mkv_shift_workspace_size(total_tokens, n_spans, rotary)
 *                  bytes, 16-byte aligned; overwritten by every call, so calls that
 *                  overlap on one workspace race.  Not needed on the direct path.
 *   span_starts, span_tables : optional, together: the direct path, one launch and no
 *                  workspace.  span_starts is device int64 [n_spans + 1], the exclusive
 *                  prefix sum of the spans' max(n_tokens, 0) (span_starts[0] == 0,
 *                  span_starts[n_spans] <= total_tokens); span_tables is device fp32
 *                  [n_spans][2][rotary], 16-byte aligned: for span s, the rotary cos
 *                  values by element, then the rotary signed sines by element, in the
 *                  header's notation cos(a[i mod rotary/2]) and sgn[i], each rounded to
 *                  fp32 (the values the plan pass would compute).  Taken when
 *                  n_spans <= MKV_DIRECT_MAX_SPANS, both sides' block sizes are powers
 *                  of two, and heads is a multiple of the rows one wave covers
 *                  (64 / (head_size * element bytes / 16)); otherwise
 *                  ignored, and the two-launch path with its workspace runs.  A prefix
 *                  that disagrees with the spans raises MKV_FLAG_SPAN; its tokens are
 *                  bounds-checked like any other.
 *   order        : MKV_ORDER_NONE, or MKV_ORDER_DST_PAGE: on the two-launch path, the
 *                  resolved tokens are sorted by the page of their destination row (2 MB,
 *                  or wider where the destination spans more than 256 such pages)
 *                  before the shift (a stable sort: the tokens of one page keep their
 *                  order; one more small launch), so that the workgroups running
 *                  together touch few destination pages.  The workspace then needs
 *                  MKV_ORDER_EXTRA_BYTES(total_tokens) more bytes.  Results are the same
 *                  bytes either way.  Ignored on the direct path.
 *   token_order  : optional device int32 [total_tokens], the same kind of order chosen
 *                  by the caller, with no extra launch: on the two-launch path the plan
 *                  pass resolves record i from token token_order[i] (tokens numbered in
 *                  span order, 0 <= token_order[i] < total_tokens), and the shift moves
 *                  the records in that order.  A permutation moves every token once and
 *                  writes the same bytes as span order; an entry out of range raises
 *                  MKV_FLAG_SPAN and moves nothing.  NULL = span order.  Not together
 *                  with MKV_ORDER_DST_PAGE (MKV_ERR_ARG).  Ignored on the direct path.
 */
typedef struct mkv_shift_desc {
  const mkv_span_t* spans;
  const float* inv_freq;
  const float* k_scale;
  int32_t* error_flags;
  void* workspace;
  int64_t workspace_bytes;
  int64_t total_tokens;
  int32_t n_spans;
  int32_t layers;
  int32_t heads;
  int32_t head_size;
  int32_t rotary;
  int32_t dtype;
  mkv_side_t src;
  mkv_side_t dst;
  const int64_t* span_starts;
  const float* span_tables;
  int32_t order;
  int32_t reserved;
  const int32_t* token_order;
} mkv_shift_desc_t;

/*
 * Single span, single layer: the drop-in for
 *   scatter_shifted(src, kv, slots, block_size, hnd, shift)
 *   (src/marathon/shift_kernels.py:166-210; its Triton kernel :89-132 and its torch
 *   path :141-159).
 * src       : device [n_tokens, heads, 2 * head_size] rows with the given token/head
 *             strides (K in [..., :head_size], V in [..., head_size:]).
 * kv        : device fused paged cache; (block, head, offset) strides select HND
 *             [blocks, heads, bs, 2D] or NHD [blocks, bs, heads, 2D]
 *             (shift_kernels.py:135-138).  kv_num_blocks bounds the slots.
 * slots     : device int64 [n_tokens] flat destination slots (shift_store.py:56-60).
 * cos, sgn  : device fp32 [head_size]: the RopeShift tables of one delta
 *             (shift_kernels.py:50-84: cos[i], and -sin for i < rotary/2, +sin for
 *             rotary/2 <= i < rotary); cos == NULL is a plain scatter (delta 0).
 * rotary    : rotated dimensions (2 * len(inv_freq)); dims >= rotary are copied.
 *             n_tokens == 0 is a no-op.
 * k_scale   : device fp32 [1], in [2^-90, 2^100], for MKV_FP8_E4M3 when rotating, else NULL.
 * Tokens move concurrently, as in the Triton kernel: a slot repeated in `slots` gets
 * one of its tokens, which one is unspecified; `src` must not alias `kv`.
 */
int mkv_scatter_shifted(const void* src, int64_t src_token_stride, int64_t src_head_stride,
                        void* kv, int64_t kv_block_stride, int64_t kv_head_stride,
                        int64_t kv_offset_stride, int64_t kv_num_blocks,
                        const int64_t* slots, int64_t n_tokens, int32_t heads,
                        int32_t head_size, int32_t block_size, int32_t dtype,
                        const float* cos, const float* sgn, int32_t rotary,
                        const float* k_scale, int32_t* error_flags, void* stream);

/*
 * Batched multi-span, multi-layer, multi-session shift in one launch: replaces the
 * connector's per-load, per-layer loop of store.read + scatter_shifted
 * (src/marathon/vllm_shift_connector.py:481-534, loop at :505-518) and the HF
 * prototype's per-segment stitch (src/marathon/kvshift.py:242-268, :265-266).
 * Every row of every span and layer moves concurrently: destination rows must be
 * distinct, and no destination row may also be read as a source row by the same call.
 * If two rows share a destination, which one lands is unspecified.  The reference's
 * sequential loop lets the later load win, but its loads cover disjoint destination
 * ranges.
 */
int mkv_shift_spans(const mkv_shift_desc_t* desc, void* stream);

/*
 * A small batched shift -- a decode step's saves, a short load -- as one launch that
 * carries its span table, token prefix and index windows in the launch's own kernel
 * arguments: nothing is copied to the device first and no workspace is used.  Same
 * semantics, checks and results as mkv_shift_spans, with these differences:
 *   - desc->spans and desc->src.index / desc->dst.index are HOST pointers, read during
 *     the call (the caller may reuse them as soon as it returns);
 *   - n_spans <= MKV_SMALL_MAX_SPANS and each side's index_len <= MKV_SMALL_MAX_INDEX;
 *     both sides' block sizes powers of two; heads a multiple of the rows one wave covers
 *     (64 / (head_size * element bytes / 16)); otherwise MKV_ERR_UNSUPPORTED;
 *   - the token prefix is computed here: a span with n_tokens < 0, or spans whose
 *     n_tokens do not sum to total_tokens, are MKV_ERR_ARG;
 *   - the rotation tables are computed in the kernel from inv_freq as the plan pass
 *     computes them; desc->workspace, span_starts and span_tables are ignored.
 * Replaces the reference connector's per-layer, per-save launches for a decode step
 * (src/marathon/vllm_shift_connector.py:539-553) and short loads (:505-518).
 */
int mkv_shift_spans_small(const mkv_shift_desc_t* desc, void* stream);

/*
 * mkv_shift_spans without a workspace argument: the same shift, the same checks and the
 * same results, with its workspace in a library-owned device buffer of
 * MKV_NOALLOC_SCRATCH_BYTES on each GPU (held from the library's first use on that GPU
 * until the process ends).  desc->workspace and desc->workspace_bytes are ignored.
 * No counterpart in the reference: this entry point is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc); it allocates nothing and calls no allocating routine.
 *   - A shift whose mkv_shift_workspace_size() exceeds MKV_NOALLOC_SCRATCH_BYTES is
 *     refused with MKV_ERR_UNSUPPORTED before anything is enqueued.
 *   - `stream` must belong to the current device (MKV_ERR_ARG otherwise).
 *   - Every call on one GPU shares that GPU's buffer, which keeps the last call's
 *     contents: calls that overlap on one GPU (on different streams, or from different
 *     threads without ordering) race.  Calls ordered on one stream do not.
 *   - The first call on a GPU resolves that GPU's buffer address (hipGetSymbolAddress);
 *     make that call eagerly, before capturing calls into a HIP graph.  A captured call
 *     records its kernels only (no memset or copy nodes), and each replay reuses the
 *     buffer: graphs of this entry point must not replay concurrently on one GPU.
 */
int mkv_shift_spans_noalloc(const mkv_shift_desc_t* desc, void* stream);
#define MKV_NOALLOC_SCRATCH_BYTES (16LL << 20)

/* Workspace bytes mkv_shift_spans needs for these sizes (-1 on negative input). */
int64_t mkv_shift_workspace_size(int64_t total_tokens, int32_t n_spans, int32_t rotary);

/*
 * Host function (no GPU call): the rotation tables of n_spans deltas, [n_spans][2][rotary]
 * fp32 in the span_tables layout (the cos of each element's angle, then its signed sine),
 * evaluated by the very routine the plan pass and the small path run on the device
 * (double-precision reduction and series in IEEE operations, marathon_amd/csrc/
 * rope_angle.h), so the direct path's tables and the device's are the same bits by
 * construction.  Replaces the reference's torch cos/sin table build
 * (shift_kernels.py:73-84) for callers that want this library's tables on the host.
 * inv_freq: host fp32 [rotary / 2]; deltas: host int32 [n_spans].
 */
int mkv_rope_tables(const int32_t* deltas, int32_t n_spans, const float* inv_freq,
                    int32_t rotary, float* tables);

/* Human-readable reason for the last non-MKV_OK return on this thread ("" if none). */
const char* mkv_last_error(void);

/* ABI version of this header: (major << 16) | minor. */
int32_t mkv_abi_version(void);
#define MKV_ABI_VERSION ((3 << 16) | 4)

#ifdef __cplusplus
}
#endif

#endif /* MARATHON_KVSHIFT_H */
