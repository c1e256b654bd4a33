/* A C host program that drives the library through its C ABI alone: no Python, no
 * torch.  It builds a small batched shift (two layers, one session's flat store ->
 * an HND paged cache through a slot array, two spans with different deltas), runs
 * it with mkv_shift_spans, checks the ABI's error path, and writes every input and
 * output to a file that a GPU test compares with the oracle.
 *
 *   usage: shift_spans_example OUT_FILE
 *
 * OUT_FILE layout (little endian): int32 header[12] = {LAYERS, HEADS, HEAD_SIZE,
 * BLOCK_SIZE, HISTORY, BLOCKS, N_SPANS, N_SLOTS, rc, flags, abi_version, error_path_ok},
 * then fp32 inv_freq[HEAD_SIZE / 2], mkv_span_t spans[N_SPANS], int64 slots[N_SLOTS],
 * bf16 src[LAYERS][HISTORY][HEADS][2 * HEAD_SIZE],
 * bf16 dst_before[LAYERS][BLOCKS][HEADS][BLOCK_SIZE][2 * HEAD_SIZE], bf16 dst_after[...].
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "marathon_kvshift.h"

enum { LAYERS = 2, HEADS = 8, HEAD_SIZE = 128, BLOCK_SIZE = 16, HISTORY = 300, BLOCKS = 32 };
enum { ROW = 2 * HEAD_SIZE, N_SPANS = 2 };

#define HIP_OK(call)                                                             \
  do {                                                                           \
    hipError_t e_ = (call);                                                      \
    if (e_ != hipSuccess) {                                                      \
      fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));          \
      return 2;                                                                  \
    }                                                                            \
  } while (0)

static uint32_t next_random(uint64_t* state) {
  *state = *state * 6364136223846793005ull + 1442695040888963407ull;
  return (uint32_t)(*state >> 33);
}

/* fp32 -> bf16 bits, round to nearest even (inputs are finite) */
static uint16_t to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

static void fill(uint16_t* p, size_t n, uint64_t* state) {
  for (size_t i = 0; i < n; ++i)
    p[i] = to_bf16(((float)(next_random(state) % 20001u) - 10000.0f) / 2500.0f);
}

int main(int argc, char** argv) {
  if (argc != 2) {
    fprintf(stderr, "usage: %s OUT_FILE\n", argv[0]);
    return 1;
  }
  const size_t src_layer = (size_t)HISTORY * HEADS * ROW;             /* elements */
  const size_t dst_layer = (size_t)BLOCKS * HEADS * BLOCK_SIZE * ROW; /* elements */
  uint16_t* src = malloc(LAYERS * src_layer * 2);
  uint16_t* dst_before = malloc(LAYERS * dst_layer * 2);
  uint16_t* dst_after = malloc(LAYERS * dst_layer * 2);
  if (!src || !dst_before || !dst_after) return 1;
  uint64_t state = 2024;
  fill(src, LAYERS * src_layer, &state);
  fill(dst_before, LAYERS * dst_layer, &state);

  float inv_freq[HEAD_SIZE / 2];
  for (int f = 0; f < HEAD_SIZE / 2; ++f)
    inv_freq[f] = 1.0f / powf(1.0e6f, (float)(2 * f) / (float)HEAD_SIZE);

  /* the request's block table: a shuffled pool of BLOCKS blocks */
  int table[BLOCKS];
  for (int b = 0; b < BLOCKS; ++b) table[b] = b;
  for (int b = BLOCKS - 1; b > 0; --b) {
    const int k = (int)(next_random(&state) % (uint32_t)(b + 1));
    const int t = table[b];
    table[b] = table[k];
    table[k] = t;
  }
  /* span 0: store rows 5..125 -> positions 3..123, delta -41;
     span 1: store rows 150..250 -> positions 200..300, delta 777 */
  const mkv_span_t spans[N_SPANS] = {{5, 0, 0, 0, 120, -41, 0, 0},
                                     {150, 0, 0, 120, 100, 777, 0, 0}};
  enum { N_SLOTS = 220 };
  int64_t slots[N_SLOTS];
  for (int i = 0; i < 120; ++i) slots[i] = (int64_t)table[(3 + i) / BLOCK_SIZE] * BLOCK_SIZE + (3 + i) % BLOCK_SIZE;
  for (int i = 0; i < 100; ++i)
    slots[120 + i] = (int64_t)table[(200 + i) / BLOCK_SIZE] * BLOCK_SIZE + (200 + i) % BLOCK_SIZE;

  /* device copies */
  void *src_d, *dst_d, *inv_d, *spans_d, *slots_d, *tables_d, *flags_d, *ws_d;
  HIP_OK(hipMalloc(&src_d, LAYERS * src_layer * 2));
  HIP_OK(hipMalloc(&dst_d, LAYERS * dst_layer * 2));
  HIP_OK(hipMalloc(&inv_d, sizeof inv_freq));
  HIP_OK(hipMalloc(&spans_d, sizeof spans));
  HIP_OK(hipMalloc(&slots_d, sizeof slots));
  HIP_OK(hipMalloc(&tables_d, 4 * LAYERS * sizeof(uint64_t)));
  HIP_OK(hipMalloc(&flags_d, sizeof(int32_t)));
  HIP_OK(hipMemcpy(src_d, src, LAYERS * src_layer * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dst_d, dst_before, LAYERS * dst_layer * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(inv_d, inv_freq, sizeof inv_freq, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(spans_d, spans, sizeof spans, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(slots_d, slots, sizeof slots, hipMemcpyHostToDevice));
  HIP_OK(hipMemset(flags_d, 0, sizeof(int32_t)));

  /* per-layer base addresses: src K, src V, dst K, dst V (V = K + HEAD_SIZE elements) */
  uint64_t bases[4 * LAYERS];
  for (int l = 0; l < LAYERS; ++l) {
    bases[0 * LAYERS + l] = (uint64_t)(uintptr_t)src_d + (uint64_t)l * src_layer * 2;
    bases[1 * LAYERS + l] = bases[0 * LAYERS + l] + HEAD_SIZE * 2;
    bases[2 * LAYERS + l] = (uint64_t)(uintptr_t)dst_d + (uint64_t)l * dst_layer * 2;
    bases[3 * LAYERS + l] = bases[2 * LAYERS + l] + HEAD_SIZE * 2;
  }
  HIP_OK(hipMemcpy(tables_d, bases, sizeof bases, hipMemcpyHostToDevice));
  const uint64_t* tab = (const uint64_t*)tables_d;

  mkv_shift_desc_t d;
  memset(&d, 0, sizeof d);
  d.spans = (const mkv_span_t*)spans_d;
  d.n_spans = N_SPANS;
  d.total_tokens = N_SLOTS;
  d.layers = LAYERS;
  d.heads = HEADS;
  d.head_size = HEAD_SIZE;
  d.rotary = HEAD_SIZE;
  d.dtype = MKV_BF16;
  d.inv_freq = (const float*)inv_d;
  d.error_flags = (int32_t*)flags_d;
  d.src.k_base = tab + 0 * LAYERS;
  d.src.v_base = tab + 1 * LAYERS;
  d.src.num_slots = HISTORY;
  d.src.block_stride = HEADS * ROW; /* FLAT: the token stride */
  d.src.head_stride = ROW;
  d.src.block_size = 1;
  d.src.mode = MKV_ADDR_FLAT;
  d.src.groups = 1;
  d.dst.k_base = tab + 2 * LAYERS;
  d.dst.v_base = tab + 3 * LAYERS;
  d.dst.index = slots_d;
  d.dst.index_len = N_SLOTS;
  d.dst.num_slots = BLOCKS * BLOCK_SIZE;
  d.dst.block_stride = HEADS * BLOCK_SIZE * ROW; /* HND [blocks, heads, bs, 2D] */
  d.dst.head_stride = BLOCK_SIZE * ROW;
  d.dst.offset_stride = ROW;
  d.dst.block_size = BLOCK_SIZE;
  d.dst.mode = MKV_ADDR_SLOTS;
  d.dst.groups = 1;
  d.workspace_bytes = mkv_shift_workspace_size(d.total_tokens, d.n_spans, d.rotary);
  HIP_OK(hipMalloc(&ws_d, (size_t)d.workspace_bytes));
  d.workspace = ws_d;

  const int rc = mkv_shift_spans(&d, NULL);
  if (rc != MKV_OK) fprintf(stderr, "mkv_shift_spans: %d (%s)\n", rc, mkv_last_error());
  HIP_OK(hipDeviceSynchronize());
  int32_t flags = -1;
  HIP_OK(hipMemcpy(dst_after, dst_d, LAYERS * dst_layer * 2, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(&flags, flags_d, sizeof flags, hipMemcpyDeviceToHost));

  /* the error path: a NULL descriptor is refused with a reason, nothing enqueued */
  const int error_path_ok = mkv_shift_spans(NULL, NULL) == MKV_ERR_ARG && mkv_last_error()[0] != 0;

  FILE* out = fopen(argv[1], "wb");
  if (!out) return 1;
  const int32_t header[12] = {LAYERS, HEADS, HEAD_SIZE, BLOCK_SIZE, HISTORY, BLOCKS, N_SPANS,
                              N_SLOTS, rc, flags, mkv_abi_version(), error_path_ok};
  fwrite(header, sizeof header, 1, out);
  fwrite(inv_freq, sizeof inv_freq, 1, out);
  fwrite(spans, sizeof spans, 1, out);
  fwrite(slots, sizeof slots, 1, out);
  fwrite(src, LAYERS * src_layer * 2, 1, out);
  fwrite(dst_before, LAYERS * dst_layer * 2, 1, out);
  fwrite(dst_after, LAYERS * dst_layer * 2, 1, out);
  fclose(out);
  hipFree(src_d);
  hipFree(dst_d);
  hipFree(inv_d);
  hipFree(spans_d);
  hipFree(slots_d);
  hipFree(tables_d);
  hipFree(flags_d);
  hipFree(ws_d);
  free(src);
  free(dst_before);
  free(dst_after);
  printf("shift_spans_example: rc=%d flags=%d\n", rc, flags);
  return rc == MKV_OK && flags == 0 && error_path_ok ? 0 : 3;
}
