/*
 * hexkv.h -- C ABI of the MI355X (gfx950) KV-cache data path of HexGen-2's
 * disaggregated prefill/decode pilot.
 *
 * The steps, each a hand-written HIP kernel:
 *   pack    gather the live positions of every layer's prefill cache into one
 *           contiguous handoff buffer (ragged, prefix-sum offsets, no padding);
 *   unpack  scatter that buffer into the decode phase's preallocated cache;
 *   append  write the new token's K/V at each sequence's current length;
 *   attend  single-query (GQA) attention over the cache, optionally with the
 *           append fused in;
 * plus the legacy KV formats (flat packet, zero-padded batch, tensor-parallel
 * head concatenation) and the same-GPU cross-process handoff (IPC).
 *
 * Conventions (all entry points):
 *   - Every pointer named *_dev or documented "device" is device memory on
 *     the current HIP device; everything else is host memory read during the
 *     call only.  The library never allocates device memory: callers own
 *     every buffer, including the attention workspace.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream)
 *     and the call returns without synchronising.
 *   - Return value: HEXKV_OK (0) or a negative hexkv_status.  A failed call
 *     launches nothing; hexkv_last_error() then returns a message for the
 *     calling thread.
 *   - Cache layout (one layer): [batch][capacity][2][kv_heads][head_dim], the
 *     layout hexgen_core allocates (hexgen/hexgen_core/modules/mha.py:260-265);
 *     one "row" = one position's K and V for all KV heads = 2*Hkv*D*elem bytes.
 *   - Packed (handoff) layout (one layer): [sum(lens)][row], sequences in batch
 *     order, i.e. the per-sequence live slices of hexgen2/model.py:81 laid end
 *     to end in send order (hexgen2/transport.py:56-59).
 */
#ifndef HEXKV_H_
#define HEXKV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *hexkv_stream_t; /* hipStream_t */

enum hexkv_dtype {
  HEXKV_F16 = 0,  /* torch.float16  */
  HEXKV_BF16 = 1, /* torch.bfloat16 */
  HEXKV_F32 = 2   /* torch.float32  */
};

/* Attention kernels.  AUTO picks MFMA for 16-bit data with head_dim 64 or
 * 128 and 8+ query heads per KV head, VALU otherwise; a work list is planned
 * and launched with hexkv_attend_plan_kernel's choice, which is ROWS for
 * AUTO on large calls. */
enum hexkv_kernel {
  HEXKV_KERNEL_AUTO = 0,
  HEXKV_KERNEL_VALU = 1, /* packed dot products on the vector ALUs     */
  HEXKV_KERNEL_MFMA = 2, /* scores and P.V on the matrix cores           */
  HEXKV_KERNEL_ROWS = 3  /* work lists planned for the XCDs only: each item
                            covers a block of adjacent KV heads (contiguous
                            bytes of every cache row); 16-bit, head_dim 128,
                            1, 2 or 4 query heads per KV head; see
                            hexkv_attend_plan_kernel */
};

enum hexkv_status {
  HEXKV_OK = 0,
  HEXKV_EINVAL = -1,       /* bad argument: shape, length, alignment, null */
  HEXKV_ERANGE = -2,       /* a length or position exceeds the capacity    */
  HEXKV_EHIP = -3,         /* the HIP runtime reported an error            */
  HEXKV_EUNSUPPORTED = -4, /* valid request outside the compiled variants  */
  HEXKV_EWORKSPACE = -5    /* workspace missing or too small               */
};

/* Largest layer count / batch one pack or unpack launch carries in its kernel
 * arguments; larger requests are split into several launches by the library. */
#define HEXKV_MAX_LAYERS_PER_LAUNCH 96
#define HEXKV_MAX_SEQS_PER_LAUNCH 256

/* Library version, major*10000 + minor*100 + patch. */
int hexkv_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char *hexkv_last_error(void);

/*
 * Device status flags: conditions a kernel met in values it read from device
 * memory (which the host could not check before the launch), handled
 * without a fault and recorded in one status word per GPU.
 */
#define HEXKV_STATUS_APPEND_SKIPPED 1u /* hexkv_append: a position outside [0, capacity); that row was not written */
#define HEXKV_STATUS_LENGTH_CLAMPED 2u /* hexkv_attend / hexkv_ft_attend: a row length above max_seqlen, cut to it
                                          (with kv_new, a new row past that bound was neither written nor attended) */
#define HEXKV_STATUS_PLACEMENT 4u      /* hexkv_attend: the items of a split segment ran on more than one XCD
                                          (work_xcds > 0), so its in-kernel merge may have read stale partials */
#define HEXKV_STATUS_DISPATCH 8u       /* hexkv_attend, information only: workgroup 0 of a list merged in the
                                          kernel started on an XCD other than 0 modulo work_xcds (the queue's
                                          dispatch starts elsewhere; the items still run on the XCDs they were
                                          planned for) */
#define HEXKV_STATUS_LIST 16u          /* hexkv_attend: a work item planned for another head-group size (another
                                          kernel) was skipped, so its outputs were not written */

/*
 * Waits for `stream`, then reads the status word of the stream's device into
 * *flags (HEXKV_STATUS_* bits) and, when `clear` is nonzero, resets it.  Not
 * for use under graph capture (it synchronises).
 *
 * The reference checks the append position on the host before every write
 * (assert sequence_end <= kv_cache.shape[1], hexgen/hexgen_core/modules/
 * mha.py:281-282) because its offset is a host integer; with per-sequence
 * positions in device memory the check happens in the kernels, and this
 * call reports it at the caller's next synchronisation point.
 */
int hexkv_device_status(uint32_t *flags, int clear, hexkv_stream_t stream);

/* Number of XCDs (dies with their own L2) of the current HIP device, for
 * hexkv_attend_params.work_xcds.  No counterpart in the reference. */
int hexkv_device_xcds(int32_t *xcds);

/*
 * Pack: for every layer l < n_layers and sequence b < batch, copy rows
 * [0, lens[b]) of sequence b of cache_layers[l] to packed_layers[l] at row
 * offset lens[0] + ... + lens[b-1].
 *
 * Replaces the per-layer live-slice gather of Engine.prefill,
 *   cache = {i: t[:, :len(input_ids)].contiguous() ...}  (hexgen2/model.py:81)
 * generalised from batch 1 to a ragged batch, all layers in one launch.
 *
 *   cache_layers   host array [n_layers] of device pointers, each the base of
 *                  one layer's cache [batch..][capacity][row]
 *   packed_layers  host array [n_layers] of device pointers, each the base of
 *                  that layer's packed region [sum(lens)][row]
 *   seq_stride_rows  rows between consecutive sequences in the cache
 *                  (= capacity for a [B][capacity][row] cache)
 *   capacity       rows of one sequence in the cache; lens[b] <= capacity
 *   row_bytes      bytes of one row; a multiple of 4
 *   lens           host array [batch] of live lengths (0 allowed)
 * Returns HEXKV_ERANGE if some lens[b] is negative or exceeds capacity.
 */
int hexkv_pack(const void *const *cache_layers, void *const *packed_layers,
               int n_layers, int batch, int64_t seq_stride_rows,
               int64_t capacity, int64_t row_bytes, const int64_t *lens,
               hexkv_stream_t stream);

/*
 * Unpack: the mirror of hexkv_pack.  Rows [0, lens[b]) of every sequence of
 * cache_layers[l] are overwritten from packed_layers[l]; every other cache row
 * is left untouched.
 *
 * Replaces the per-layer cache rebuild of Engine.decode,
 *   full = torch.empty((1, max_sequence_len, ...)); full[:, :L].copy_(live)
 *   (hexgen2/model.py:104-108), writing into a cache the caller preallocated.
 */
int hexkv_unpack(const void *const *packed_layers, void *const *cache_layers,
                 int n_layers, int batch, int64_t seq_stride_rows,
                 int64_t capacity, int64_t row_bytes, const int64_t *lens,
                 hexkv_stream_t stream);

/*
 * Append: for every sequence b < batch, copy row b of kv_new ([batch][row],
 * contiguous) into the cache at position
 *   pos_b = (positions_dev ? positions_dev[b] : 0) + position_bias.
 * Rows with pos_b outside [0, capacity) are skipped on the device and raise
 * HEXKV_STATUS_APPEND_SKIPPED (the host wrapper rejects them first whenever
 * positions are known on the host).
 *
 * Replaces the slice assignment of _update_kv_cache,
 *   kv_cache[batch_start:batch_end, sequence_start:sequence_end, ...] = kv
 *   (hexgen/hexgen_core/modules/mha.py:286), with per-sequence positions in
 *   place of the single sequence_len_offset (mha.py:276-279).
 *
 *   cache             device base of [batch..][capacity][row] (the caller
 *                     adds batch_size_offset * seq_stride_rows * row_bytes)
 *   positions_dev     device int32 [batch] or NULL
 */
int hexkv_append(const void *kv_new, void *cache, int batch,
                 int64_t seq_stride_rows, int64_t capacity, int64_t row_bytes,
                 const int32_t *positions_dev, int32_t position_bias,
                 hexkv_stream_t stream);

/*
 * One workgroup's share of decode attention in a work list (32 bytes): the
 * `count` positions from `first` of query row `row` for the query heads of
 * head group `head_group` (head groups of `heads` query heads, the size
 * hexkv_attend_plan planned for), which is partition `part` of the `parts`
 * partitions that row and head group is cut into.  `len` is the row's
 * attended length (with kv_new, the new row is position len - 1).  A launch
 * whose head groups have another size skips the item and raises
 * HEXKV_STATUS_LIST (`heads` 0: the launch's own size is assumed).
 */
typedef struct hexkv_work_item {
  int32_t row, head_group, part, parts;
  int32_t first, count, len, heads;
} hexkv_work_item;

/*
 * Geometry and inputs of one attention call.  Strides are in elements.
 * Query row r = (b, t), b < batch, t < q_len; q and out are
 * [batch][q_len][q_heads][head_dim] with the two innermost dims contiguous.
 * The cache is one layer: K of position s, head h at
 *   cache + b*cache_batch_stride + s*cache_pos_stride + h*head_dim
 * and V at that address + cache_kv_stride.
 */
typedef struct hexkv_attend_params {
  int dtype;      /* enum hexkv_dtype, shared by q, cache, kv_new, out    */
  int batch;      /* B                                                    */
  int q_len;      /* queries per sequence (1 for decode)                  */
  int q_heads;    /* Hq                                                   */
  int kv_heads;   /* Hkv, divides Hq                                      */
  int head_dim;   /* D: 16, 32, 64, 128 or 256                            */
  int causal;     /* q_len > 1 only: query t sees keys < len - q_len + t + 1 */
  float softmax_scale;
  const void *q;
  int64_t q_batch_stride, q_row_stride;
  const void *cache;
  int64_t cache_batch_stride, cache_pos_stride, cache_kv_stride;
  int64_t capacity; /* positions per sequence in the cache */
  void *out;
  int64_t out_batch_stride, out_row_stride;
  /* Keys attended by sequence b: len_b = (seqlens_dev ? seqlens_dev[b] : 0)
   * + seqlen_bias, plus one when kv_new is set.  max_seqlen bounds every
   * len_b (including that +1) and sizes the grid. */
  const int32_t *seqlens_dev;
  int32_t seqlen_bias;
  int32_t max_seqlen;
  /* Optional fused append (q_len == 1 only): kv_new is [batch][2][kv_heads]
   * [head_dim] contiguous; its row is written to cache position len_b - 1 and
   * attended from registers. */
  const void *kv_new;
  /* Split-K partition size in positions; 0 = chosen by the library. */
  int partition;
  /* enum hexkv_kernel: which kernel computes the scores. */
  int kernel;
  /* Optional work list (device memory, from hexkv_attend_plan), decode rows
   * only (q_len 1, not causal): one workgroup per item, in list order.  The
   * items carry the row lengths, so seqlens_dev and seqlen_bias are not
   * read.  work_parts_dev[row * head_groups + head group] is the partition
   * count of that (row, head group) for the split merge; work_max_parts
   * bounds every count and sizes the workspace.  NULL: the library's
   * uniform partitions over the lengths in seqlens_dev. */
  const hexkv_work_item *work_items_dev;
  const int32_t *work_parts_dev;
  int32_t n_work_items;
  int32_t work_max_parts;
  /* XCDs the work list is planned for (hexkv_attend_plan reads it too).
   * 0: the partials of a split (row, head group) are merged by a second
   * kernel on the same stream.  N > 0 (the device's XCD count,
   * hexkv_device_xcds): every item of a split segment sits at one index
   * modulo N, so its items share one XCD's L2, and the segment's last item
   * to finish merges the partials inside the attention kernel: one launch
   * per call.  Workgroups reach the XCDs round-robin by index from a start
   * XCD that depends on the hardware queue; when N divides the device's XCD
   * count and the list length is a multiple of N (as planned), each
   * workgroup runs the item of its own XCD within its group of N, so index
   * j * N + x always runs on XCD x.  Each workgroup checks its XCD and raises
   * HEXKV_STATUS_PLACEMENT if a segment's items still met on two.  A list
   * whose split segments would merge in the attention kernel and whose N is
   * not the device's XCD count is refused (HEXKV_EINVAL): its segments
   * would straddle XCDs. */
  int32_t work_xcds;
  /* Work-list calls with kv_new only, else NULL: row b's new cached length
   * (its attended keys, the appended row included) is stored to
   * lengths_out_dev[b], so a captured decode step advances the caller's
   * lengths in the same launch. */
  int32_t *lengths_out_dev;
} hexkv_attend_params;

/* Workspace bytes hexkv_attend needs for these parameters (0 when one
 * partition covers every sequence).  The workspace is scratch (partial
 * outputs of the split-K merge) behind HEXKV_ATTEND_COUNTER_BYTES of
 * arrival counters, which single-launch merges (work_xcds > 0) use and
 * leave zero: zero the workspace once after allocating it.  Calls sharing
 * one workspace must not overlap. */
#define HEXKV_ATTEND_COUNTER_BYTES (256u << 10)
size_t hexkv_attend_workspace_bytes(const hexkv_attend_params *p);

/* The kernel hexkv_attend runs for these parameters, HEXKV_KERNEL_VALU or
 * HEXKV_KERNEL_MFMA (HEXKV_KERNEL_AUTO resolved by head group, head_dim and
 * dtype), or a negative error code.  No counterpart in the reference: it
 * lets profiling and benchmarks name the kernel they measure. */
int hexkv_attend_kernel(const hexkv_attend_params *p);

/*
 * Single-query GQA attention over the cache, optionally appending first:
 *   out[b,t,h] = sum_s softmax_s(q[b,t,h] . K[b,s,h/g] * scale) V[b,s,h/g]
 * over s < len(b,t), g = q_heads / kv_heads, fp32 accumulation.
 *
 * Replaces the decode-time attention of MHA.forward,
 *   context = self.inner_cross_attn(q, kv, causal=False)
 *   (hexgen/hexgen_core/modules/mha.py:568-569) -> FlashCrossAttention.forward
 *   (mha.py:105-142), whose CPU semantics are CrossAttention.forward
 *   (mha.py:209-244, GQA head repeat mha.py:223-224).  With kv_new set it also
 *   replaces the preceding _update_kv_cache call (mha.py:565, 286).
 */
int hexkv_attend(const hexkv_attend_params *p, void *workspace,
                 size_t workspace_bytes, hexkv_stream_t stream);

/*
 * Work list for hexkv_attend over decode rows whose lengths the host knows:
 * row b attends len_b = lens[b] + p->seqlen_bias (+1 with kv_new) keys,
 * each within [0, p->max_seqlen].  Every (row, head group) segment is cut
 * into chunks of p->partition positions (0: the library's choice by the
 * bytes the call reads, see hexkv_attend_plan_chunk; else a multiple of 64,
 * of 16 for HEXKV_KERNEL_ROWS, whose segments are blocks of KV heads),
 * and the items are ordered for the launch: empty
 * rows, then the full chunks across all segments, then each segment's last,
 * shorter chunk from the longest down.  With p->work_xcds = N > 0 the
 * segments are first dealt to the N XCDs (longest first, each to the XCD with
 * the fewest positions so far), that order is kept within each XCD's items,
 * and XCD x's j-th item goes to index j * N + x; shorter XCD lists are padded
 * with items the kernels skip (row = batch), so n_items is a multiple of N.
 * Host memory only; the caller copies `items` and `parts` to the device and
 * passes them in hexkv_attend_params.work_*.
 *
 *   lens            host int32 [batch]
 *   items, parts    host outputs: up to items_capacity items and
 *                   parts_capacity (>= batch * head groups; batch * q_heads
 *                   always suffices) partition counts; the device copy of
 *                   `parts` must hold all batch * head groups of them, the
 *                   merge reads them by (row, head group); items == NULL
 *                   only sizes the plan
 *   n_items, max_parts   outputs: the item count and the largest partition
 *                   count (work_max_parts)
 *
 * The reference has no planning step: this replaces nothing in it.  It is
 * how the call of mha.py:568-569 (FlashCrossAttention over the cache) is
 * cut into workgroups when the lengths are known on the host.
 */
int hexkv_attend_plan(const hexkv_attend_params *p, const int32_t *lens, hexkv_work_item *items,
                      int32_t items_capacity, int32_t *parts, int32_t parts_capacity,
                      int32_t *n_items, int32_t *max_parts);

/*
 * The chunk (positions per work item) hexkv_attend_plan uses for these
 * lengths: p->partition when set, else the library's choice -- below 4 MB
 * read one chunk per segment (or, with work_xcds > 0, about a twelfth of the
 * longest row, 64 positions at least), about 240 items below 64 MB, 896
 * positions above (1280 from 2^20 positions up).  A caller that replays one
 * captured launch over several steps can plan every step with the chunk of
 * its last (longest) step, passed as p->partition, so the item and
 * partition counts only grow and the last step's sizes bound every step
 * (without work_xcds; planned for the XCDs, a list's length is the longest
 * XCD share times the XCD count, which need not grow).  Returns HEXKV_OK
 * with *chunk set, or an error as hexkv_attend_plan.  No counterpart in the
 * reference (it has no planning step).
 */
int hexkv_attend_plan_chunk(const hexkv_attend_params *p, const int32_t *lens, int32_t *chunk);

/*
 * The kernel value to plan and launch these lengths with: p->kernel when it
 * is not HEXKV_KERNEL_AUTO; for AUTO, HEXKV_KERNEL_ROWS when the call reads
 * at least 64 MB, fits the row-block kernel and is planned for the XCDs
 * (p->work_xcds 1-8), else AUTO's own choice (HEXKV_KERNEL_VALU or _MFMA).
 * The row-block kernel streams 2 adjacent KV heads per item for grouped
 * queries, 8 for one query head per KV head, and reads those heads' bytes of
 * every cache row contiguously; at Llama-3-8B's and Llama-2-7B's shapes it
 * measured 7-8% and ~4% faster per call than one head per item.  A caller
 * sets the returned value in p->kernel for hexkv_attend_plan and for the
 * launches of that list.  Returns HEXKV_OK with *kernel set, or an error as
 * hexkv_attend_plan.  No counterpart in the reference (it has no planning
 * step).
 */
int hexkv_attend_plan_kernel(const hexkv_attend_params *p, const int32_t *lens, int32_t *kernel);

/* Size of the static scratch array behind hexkv_attend_noalloc (per GPU). */
#define HEXKV_NOALLOC_SCRATCH_BYTES (32u << 20)

/*
 * hexkv_attend without a workspace argument: the same kernels and results,
 * with the split-K partials in a static device array of
 * HEXKV_NOALLOC_SCRATCH_BYTES (32 MiB) that the library holds on each GPU it
 * runs on until the process ends.  The call allocates nothing (no hipMalloc,
 * no library allocation); the caller still passes q, the cache and out.
 * Returns HEXKV_EWORKSPACE when hexkv_attend_workspace_bytes(p) exceeds the
 * array.  The array's address on a device is looked up on that device's
 * first call (the stream's device; the current device for the null stream).
 * Calls on one GPU share its array, which keeps the last call's contents:
 * calls that overlap on one GPU (different streams, no ordering) race.
 *
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory -- code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.
 */
int hexkv_attend_noalloc(const hexkv_attend_params *p, hexkv_stream_t stream);

/*
 * The FasterTransformer ("FT") cache layout of hexgen_core's fused decode
 * path (fused_ft_kernel=True; the layout the reference's CUDA-graph decode
 * uses): per layer
 *   K  [batch][kv_heads][head_dim / pack][capacity][pack]
 *   V  [batch][kv_heads][capacity][head_dim]
 * with pack = 8 for 16-bit data and 4 for float32, so one K position of one
 * head is head_dim / pack chunks of 16 bytes, capacity * 16 bytes apart.
 */

/*
 * Writes positions [0, seq_len) of kv ([batch][.. seq_len ..][2][kv_heads]
 * [head_dim], heads and head_dim contiguous; strides in elements, kv_stride
 * from K to V) into the FT caches, positions [0, seq_len) of each sequence.
 * A bit copy.
 *
 * Replaces the FT branch of _update_kv_cache
 * (hexgen/hexgen_core/modules/mha.py:289-305): the conversion of a filled
 * [B, S, 2, H, D] cache into the FT pair (rearranges at mha.py:296-298) and
 * the direct prefill write into FT caches (mha.py:301-305).
 */
int hexkv_ft_store(const void *kv, int64_t kv_batch_stride, int64_t kv_pos_stride, int64_t kv_stride,
                   void *k_cache, void *v_cache, int batch, int seq_len, int64_t capacity,
                   int kv_heads, int head_dim, int dtype, hexkv_stream_t stream);

/* One decode step over FT caches: rotary on q and on the new K, append of
 * the new K/V at each sequence's position, single-query GQA attention over
 * positions [0, position]. */
typedef struct hexkv_ft_attend_params {
  int dtype;       /* enum hexkv_dtype, shared by every tensor            */
  int batch;
  int q_heads;
  int kv_heads;    /* divides q_heads                                      */
  int head_dim;    /* 16, 32, 64, 128 or 256                               */
  float softmax_scale;
  const void *q;   /* [batch][q_heads][head_dim], heads contiguous         */
  int64_t q_batch_stride;
  const void *k_new, *v_new; /* [batch][kv_heads][head_dim] each          */
  int64_t new_batch_stride;
  void *k_cache, *v_cache;   /* FT layouts above                           */
  int64_t capacity;
  void *out;       /* [batch][q_heads][head_dim]                           */
  int64_t out_batch_stride;
  /* Position of sequence b's new token: pos_b = (positions_dev ?
   * positions_dev[b] : 0) + position_bias; max_position bounds every pos_b
   * and must be below capacity. */
  const int32_t *positions_dev;
  int32_t position_bias;
  int32_t max_position;
  /* Rotary embedding of q and the new K at pos_b: the first rotary_dim
   * dimensions of each head turn in pairs, pair j by pos_b *
   * rotary_base^(-2j / rotary_dim) radians; pairs (j, j + rotary_dim/2) when
   * rotary_neox, else (2j, 2j + 1).  rotary_dim 0: no rotation. */
  int rotary_dim;
  float rotary_base;
  int rotary_neox;
  int partition;   /* as in hexkv_attend_params */
} hexkv_ft_attend_params;

/* Workspace bytes hexkv_ft_attend needs (same role as for hexkv_attend). */
size_t hexkv_ft_attend_workspace_bytes(const hexkv_ft_attend_params *p);

/*
 * Replaces the fused decode attention of the FT path,
 *   _apply_rotary_single_query_attention
 *   (hexgen/hexgen_core/modules/mha.py:310-337), which calls
 *   ft_attention.single_query_attention (FasterTransformer's masked
 *   multi-head attention, an extension the reference does not vendor) with
 *   lengths_per_sample or sequence_len_offset as the position
 *   (mha.py:325-335).  q and the new K are rotated and rounded to the data
 *   type, the new K/V are written at pos_b, and
 *   out[b,h] = sum_{s <= pos_b} softmax_s(q.K[b,s,h/g] * scale) V[b,s,h/g].
 */
int hexkv_ft_attend(const hexkv_ft_attend_params *p, void *workspace, size_t workspace_bytes,
                    hexkv_stream_t stream);

/*
 * Legacy KV formats of HexGen's earlier disaggregation scripts
 * (hexgen/llama/): the flat-concatenated packet, zero-padded request
 * batching and the tensor-parallel head concatenation.  Each is a strided
 * gather of byte rows, described by blocks.
 *
 * A block is depth x height rows of `width` contiguous bytes at
 *   data + k * slice_pitch + r * row_pitch      (k < depth, r < height),
 * e.g. a cache view [B, L, 2, Hkv, D] of one layer is depth = B sequences,
 * height = L positions, width = one row (2*Hkv*D*elem), row_pitch and
 * slice_pitch its position and batch strides in bytes.  A block's "compact"
 * order is slice by slice, row by row.  Sources may alias each other; a
 * destination must not overlap any source.
 */
typedef struct hexkv_block {
  const void *data;    /* device address of byte 0 of row 0 of slice 0 */
  int64_t width;       /* contiguous bytes per row                      */
  int64_t height;      /* rows per slice                                */
  int64_t depth;       /* slices                                        */
  int64_t row_pitch;   /* bytes from one row to the next                */
  int64_t slice_pitch; /* bytes from one slice to the next              */
} hexkv_block;

/*
 * Flat concatenation: the bytes of src[0], src[1], ... src[n-1], each in
 * compact order, laid end to end at dst.
 *
 * Replaces the payload build of send_key_value_memory_dict,
 *   torch.cat([t.flatten() for t in key_value_memory_dict.values()])
 *   (hexgen/llama/kv_cache_communication.py:21-26); the receiver's per-layer
 *   tensors are views of the flat buffer (:50-57).
 */
int hexkv_flat_concat(const hexkv_block *src, int n, void *dst, hexkv_stream_t stream);

/*
 * Zero-padded batching: for every layer l < n_layers the requests' caches
 * src[l * n_req + i] (depth b_i sequences x height len_i positions x width
 * row bytes) are stacked into dst_layers[l], a contiguous
 * [sum_i b_i][max_rows][row] buffer, request i's sequences after those of
 * requests < i; rows [len_i, max_rows) of each of its sequences are zero.
 * b_i and len_i of request i must agree over layers, the width over all
 * blocks, and len_i <= max_rows.
 *
 * Replaces the per-layer F.pad + torch.cat of
 * batch_logits_and_key_value_memory_dict (hexgen/llama/kv_cache_batch.py:
 * 4-28) with max_rows = max_i len_i.
 */
int hexkv_batch_pad(const hexkv_block *src, int n_layers, int n_req, void *const *dst_layers,
                    int64_t max_rows, hexkv_stream_t stream);

/*
 * Head concatenation of tensor-parallel shards: for every layer l the
 * shards src[l * n_shards + j] (depth x height rows of w_j bytes, one row =
 * one (sequence, position, K|V) slice of shard j's heads, rows numbered
 * slice by slice) are joined row by row into dst_layers[l], a contiguous
 * [rows][sum_j w_j] buffer, shard j at byte column w_0 + ... + w_{j-1}.  The
 * row count depth x height must agree over a layer's shards, w_j over
 * layers.
 *
 * Replaces concat_dicts(list_of_dicts, dim=3), torch.cat over the KV-head
 * dimension of [B, S, 2, H_j, D] (hexgen/llama/tensor_parallel_dim_concat.py:
 * 9-19): depth = B, height = 2 S, w_j = H_j * D * elem.
 */
int hexkv_head_concat(const hexkv_block *src, int n_layers, int n_shards, void *const *dst_layers,
                      hexkv_stream_t stream);

/*
 * Cross-process handoff on one GPU.  Two processes sharing the GPU (the
 * prefill and decode ranks of the pilot, hexgen2/run.py:141-198) hand the
 * packed KV buffer over in device memory: the sender exports an IPC handle of
 * the allocation holding each tensor, the handle and offset travel in the
 * packet header's host message, and the receiver maps the allocation and
 * reads the bytes where they lie.  These calls replace the payload leg of
 * send_packet/recv_packet (hexgen2/transport.py:56-59, 75-78); the header
 * leg is unchanged.
 *
 * The mapped allocation must stay alive in the sender until the receiver has
 * closed every mapping of it.  On this platform an exported allocation must
 * be smaller than 2 GiB.
 */
typedef struct hexkv_ipc_handle {
  unsigned char bytes[64];
} hexkv_ipc_handle;

/* Handle of the device allocation containing `ptr`, the byte offset of `ptr`
 * in it, and the allocation's size.  HEXKV_ERANGE (no handle) when the
 * allocation is 2 GiB or larger. */
int hexkv_ipc_export(const void *ptr, hexkv_ipc_handle *handle, uint64_t *offset,
                     uint64_t *alloc_bytes);

/* Maps an exported allocation into this process (or takes one more reference
 * to an existing mapping of the same handle); *base is its first byte. */
int hexkv_ipc_open(const hexkv_ipc_handle *handle, void **base);

/* Drops one reference to a mapping; the last one synchronises the device (no
 * enqueued work may still read it) and unmaps it. */
int hexkv_ipc_close(void *base);

/* A DLPack (v0.8 `DLManagedTensor`, device kDLROCM) view of `ndim`-dimensional
 * compact row-major data at base + offset, for a framework's from_dlpack.  It
 * takes over one reference of the mapping from hexkv_ipc_open: the view's
 * deleter closes it.  dtype_code/bits follow DLPack (kDLInt 0, kDLUInt 1,
 * kDLFloat 2, kDLBfloat 4, kDLBool 6).  Returns NULL on bad arguments. */
void *hexkv_ipc_dlpack(void *base, uint64_t offset, int ndim, const int64_t *shape,
                       int dtype_code, int dtype_bits, int device_id);

#ifdef __cplusplus
}
#endif

#endif /* HEXKV_H_ */
