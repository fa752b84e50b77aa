// Ragged live-position copies of the KV-cache handoff: pack (cache -> packed
// handoff buffer), unpack (packed -> decode cache) and per-step append.
//
// All three are pure byte movement, bound by HBM bandwidth.  Design for gfx950:
//  * one launch covers every layer of a request (grid.y = layer) and every
//    sequence of the batch; the per-sequence row offsets (prefix sums of the
//    live lengths) and the per-layer base pointers travel in the kernel
//    arguments, so no metadata is read from HBM and no padded row is moved;
//  * grid.x tiles each layer's packed region into fixed-size byte chunks, so
//    work per workgroup is uniform however ragged the lengths are; a chunk
//    crosses at most a few sequence boundaries, found by one scalar binary
//    search per workgroup;
//  * each lane moves 16-byte vectors with nontemporal (streaming) loads and
//    stores, eight in flight per lane (four in the 256-thread workgroups of
//    copies below 128 MB), so the 256 MB MALL is not polluted by data that
//    is touched exactly once.
#include "hexkv_common.h"

#include <algorithm>

namespace hexkv {

// 1024 threads x 8 vectors of 16 bytes in flight per workgroup: a whole
// 128 KB chunk is loaded before any of it is stored.  Measured on MI355X
// with the Llama-3-8B handoff (pack + unpack of 2 x 63.9 GB), every variant
// on the same buffers in one process (medians of 4-5 interleaved rounds):
// 1024 x 8 21.15 ms; 512 x 8 22.2; 512 x 16 22.5; 1024 x 8 with 256 KB
// chunks 21.4, with 64 KB 22.4; 1024 x 4 21.9; 1024 x 16 with 256 KB 21.9;
// 512 x 4 (the earlier choice) 23.3; 256 x 8 23.6.  Nontemporal loads and
// stores both matter: 1024 x 8 with ordinary stores 23.3 ms, with ordinary
// loads 21.7, against 21.1 with neither.  For reference a plain
// chunked copy of 512 x 4 reached 5.55-5.76 TB/s (read + write), a
// device-to-device hipMemcpy 4.90, a write-only stream 6.2-6.4 and a
// read-only stream 7.1.
constexpr int kCopyThreads = 1024;
constexpr int kCopyUnroll = 8;
// Copies below 128 MB (16 KB chunks, the smallest; TinyLlama's 22-layer
// handoff moves 11.5 MB each way) run 256 threads x 4 vectors: the same 16 KB
// per workgroup, all of it loaded before any store, and a quarter of the
// threads, so the grid is resident at once instead of in two rounds of
// 1024-thread workgroups.
constexpr int kSmallCopyThreads = 256;
constexpr int kSmallCopyUnroll = 4;
constexpr int64_t kSmallCopyChunk = INT64_C(16384);
// The per-step append moves one row per sequence: 512 threads, one vector each.
constexpr int kAppendThreads = 512;

// Kernel arguments of one launch over L layers and S sequences at most.  The
// block is copied into the kernel-argument segment on every launch, and its
// size shows in the host's cost per call: a hexkv_pack call of TinyLlama's
// 22-layer handoff took 5.9 us with the 2.6 KB block of 96 layers x 256
// sequences and 3.4-3.9 us with a 0.46 KB one (MI355X host, back-to-back
// calls; the kernel itself takes 6.8 us, so the host set the rate of
// isolated calls).  Launches of up to 32 layers and 16 sequences use the
// 0.6 KB block.
template <int L, int S>
struct RaggedCopyArgs {
  const char *src[L];
  char *dst[L];
  int64_t row_bytes;
  int64_t seq_stride_bytes;  // padded (cache) side: bytes between sequences
  int64_t chunk_bytes;       // packed bytes per workgroup
  int64_t layer_bytes;       // packed bytes per layer in this launch
  int32_t batch;
  int32_t cu[S + 1];  // packed row offset of each sequence
};
using WideCopyArgs = RaggedCopyArgs<HEXKV_MAX_LAYERS_PER_LAUNCH, HEXKV_MAX_SEQS_PER_LAUNCH>;
using SmallCopyArgs = RaggedCopyArgs<32, 16>;
static_assert(sizeof(WideCopyArgs) <= 4096, "kernel arguments above 4 KiB");

// Every pass issues UN loads per lane (NT lanes) before its stores; the last,
// partial pass masks lanes instead of falling back to one vector at a time.
template <typename V, int NT, int UN>
__device__ __forceinline__ void copy_span(const char *__restrict__ s, char *__restrict__ d,
                                          int64_t n) {
  const V *sv = reinterpret_cast<const V *>(s);
  V *dv = reinterpret_cast<V *>(d);
  const int64_t nv = n / static_cast<int64_t>(sizeof(V));
  int64_t i = threadIdx.x;
  for (; i + (UN - 1) * NT < nv; i += UN * NT) {
    V r[UN];
#pragma unroll
    for (int u = 0; u < UN; ++u) r[u] = __builtin_nontemporal_load(sv + i + u * NT);
#pragma unroll
    for (int u = 0; u < UN; ++u) __builtin_nontemporal_store(r[u], dv + i + u * NT);
  }
  if (i < nv) {
    V r[UN];
#pragma unroll
    for (int u = 0; u < UN; ++u)
      if (i + u * NT < nv) r[u] = __builtin_nontemporal_load(sv + i + u * NT);
#pragma unroll
    for (int u = 0; u < UN; ++u)
      if (i + u * NT < nv) __builtin_nontemporal_store(r[u], dv + i + u * NT);
  }
}

// PACK: src = padded cache, dst = packed buffer.  UNPACK: the reverse.
template <typename V, bool PACK, typename A, int NT, int UN>
__global__ __launch_bounds__(NT) void ragged_copy_kernel(const A a) {
  const int64_t start = static_cast<int64_t>(blockIdx.x) * a.chunk_bytes;
  if (start >= a.layer_bytes) return;
  const int64_t end = min(start + a.chunk_bytes, a.layer_bytes);
  const char *src = a.src[blockIdx.y];
  char *dst = a.dst[blockIdx.y];
  const int64_t row = a.row_bytes;
  // Last sequence whose packed range starts at or before `start`.
  int lo = 0, hi = a.batch;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (static_cast<int64_t>(a.cu[mid]) * row <= start) lo = mid; else hi = mid;
  }
  for (int b = lo; b < a.batch; ++b) {
    const int64_t seg0 = static_cast<int64_t>(a.cu[b]) * row;
    if (seg0 >= end) break;
    const int64_t seg1 = static_cast<int64_t>(a.cu[b + 1]) * row;
    const int64_t p0 = max(start, seg0), p1 = min(end, seg1);
    if (p0 >= p1) continue;
    const int64_t padded = static_cast<int64_t>(b) * a.seq_stride_bytes + (p0 - seg0);
    if constexpr (PACK) copy_span<V, NT, UN>(src + padded, dst + p0, p1 - p0);
    else copy_span<V, NT, UN>(src + p0, dst + padded, p1 - p0);
  }
}

template <typename V>
__global__ __launch_bounds__(kAppendThreads) void append_kernel(
    const char *__restrict__ kv_new, char *__restrict__ cache, int64_t seq_stride_bytes,
    int64_t capacity, int64_t row_bytes, const int32_t *__restrict__ positions, int32_t bias,
    unsigned int *status) {
  const int b = blockIdx.y;
  const int64_t pos = (positions ? static_cast<int64_t>(positions[b]) : 0) + bias;
  if (pos < 0 || pos >= capacity) {
    if (blockIdx.x == 0 && threadIdx.x == 0) raise_status(status, HEXKV_STATUS_APPEND_SKIPPED);
    return;
  }
  const int64_t nv = row_bytes / static_cast<int64_t>(sizeof(V));
  const V *s = reinterpret_cast<const V *>(kv_new + b * row_bytes);
  V *d = reinterpret_cast<V *>(cache + b * seq_stride_bytes + pos * row_bytes);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kAppendThreads + threadIdx.x; i < nv;
       i += static_cast<int64_t>(gridDim.x) * kAppendThreads)
    d[i] = s[i];
}

// ------------------------------------------------------------------ host ---

// The status word of each GPU (HEXKV_STATUS_* bits, raised by kernels with
// atomicOr), defined beside kernels so that its code object is one the
// runtime loads with them.  Host code passes kernels the per-device address
// that hipGetSymbolAddress returns, never the name itself.
static __device__ unsigned int device_status;
static std::atomic<void *> g_status_addr[kMaxDevices];

int status_word(hexkv_stream_t stream, unsigned int **word, const char *what) {
  void *ptr = nullptr;
  const int rc = symbol_address(reinterpret_cast<const void *>(&HIP_SYMBOL(device_status)), g_status_addr, stream,
                                &ptr, what);
  *word = static_cast<unsigned int *>(ptr);
  return rc;
}


// Packed bytes per workgroup: large enough to amortise the per-workgroup
// sequence search, small enough to give every CU many workgroups.
static int64_t choose_chunk(int64_t total_bytes) {
  const int64_t target_wgs = 8192;
  int64_t chunk = (total_bytes / target_wgs + 4095) / 4096 * 4096;
  return std::min<int64_t>(std::max<int64_t>(chunk, kSmallCopyChunk), 131072);
}

// One launch: layers [l0, l0 + nl) of sequences [b0, b0 + nb), whose packed
// row offsets are cu[0..nb]; A is the argument block it fits.
template <typename A>
static int launch_copy(bool pack, bool vec16, const void *const *src_layers, void *const *dst_layers, int l0,
                       int nl, int nb, const int32_t *cu, int64_t row_bytes, int64_t seq_stride_bytes,
                       int64_t chunk, int64_t padded_off, int64_t packed_off, hipStream_t stream,
                       const char *what) {
  A a;
  a.row_bytes = row_bytes;
  a.seq_stride_bytes = seq_stride_bytes;
  a.chunk_bytes = chunk;
  a.batch = nb;
  for (int b = 0; b <= nb; ++b) a.cu[b] = cu[b];
  a.layer_bytes = static_cast<int64_t>(cu[nb]) * row_bytes;
  for (int l = 0; l < nl; ++l) {
    const char *s = static_cast<const char *>(src_layers[l0 + l]);
    char *d = static_cast<char *>(dst_layers[l0 + l]);
    a.src[l] = s + (pack ? padded_off : packed_off);
    a.dst[l] = d + (pack ? packed_off : padded_off);
  }
  const int64_t gx = (a.layer_bytes + chunk - 1) / chunk;
  if (gx > INT32_MAX) return fail(HEXKV_ERANGE, "%s: grid too large", what);
  dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(nl));
  if (vec16 && chunk == kSmallCopyChunk) {
    constexpr int NT = kSmallCopyThreads, UN = kSmallCopyUnroll;
    if (pack) ragged_copy_kernel<u32x4, true, A, NT, UN><<<grid, NT, 0, stream>>>(a);
    else ragged_copy_kernel<u32x4, false, A, NT, UN><<<grid, NT, 0, stream>>>(a);
  } else if (vec16) {
    constexpr int NT = kCopyThreads, UN = kCopyUnroll;
    if (pack) ragged_copy_kernel<u32x4, true, A, NT, UN><<<grid, NT, 0, stream>>>(a);
    else ragged_copy_kernel<u32x4, false, A, NT, UN><<<grid, NT, 0, stream>>>(a);
  } else {
    constexpr int NT = kCopyThreads, UN = kCopyUnroll;
    if (pack) ragged_copy_kernel<unsigned int, true, A, NT, UN><<<grid, NT, 0, stream>>>(a);
    else ragged_copy_kernel<unsigned int, false, A, NT, UN><<<grid, NT, 0, stream>>>(a);
  }
  return check_launch(what);
}

static int ragged_copy(bool pack, const void *const *src_layers, void *const *dst_layers,
                       int n_layers, int batch, int64_t seq_stride_rows, int64_t capacity,
                       int64_t row_bytes, const int64_t *lens, hipStream_t stream) {
  clear_error();
  const char *what = pack ? "hexkv_pack" : "hexkv_unpack";
  if (n_layers < 0 || batch < 0) return fail(HEXKV_EINVAL, "%s: negative layer count or batch", what);
  if (n_layers == 0 || batch == 0) return HEXKV_OK;
  if (!src_layers || !dst_layers || !lens) return fail(HEXKV_EINVAL, "%s: null argument", what);
  if (row_bytes <= 0 || row_bytes % 4 != 0)
    return fail(HEXKV_EINVAL, "%s: row_bytes %lld is not a positive multiple of 4", what,
                static_cast<long long>(row_bytes));
  if (capacity < 0 || (batch > 1 && seq_stride_rows < capacity) || seq_stride_rows < 0)
    return fail(HEXKV_EINVAL, "%s: sequence stride %lld rows is below capacity %lld", what,
                static_cast<long long>(seq_stride_rows), static_cast<long long>(capacity));
  int64_t total_rows = 0;
  for (int b = 0; b < batch; ++b) {
    if (lens[b] < 0 || lens[b] > capacity)
      return fail(HEXKV_ERANGE, "%s: length %lld of sequence %d outside [0, %lld]", what,
                  static_cast<long long>(lens[b]), b, static_cast<long long>(capacity));
    total_rows += lens[b];
  }
  if (total_rows > INT32_MAX) return fail(HEXKV_ERANGE, "%s: more than 2^31-1 live rows", what);
  if (total_rows == 0) return HEXKV_OK;
  bool vec16 = row_bytes % 16 == 0;
  for (int l = 0; l < n_layers; ++l) {
    if (!src_layers[l] || !dst_layers[l]) return fail(HEXKV_EINVAL, "%s: null layer pointer %d", what, l);
    if ((reinterpret_cast<uintptr_t>(src_layers[l]) | reinterpret_cast<uintptr_t>(dst_layers[l])) & 3)
      return fail(HEXKV_EINVAL, "%s: layer %d pointer not 4-byte aligned", what, l);
    vec16 = vec16 && aligned16(src_layers[l]) && aligned16(dst_layers[l]);
  }
  const int64_t chunk = choose_chunk(total_rows * row_bytes * n_layers);

  // Sequences in groups of HEXKV_MAX_SEQS_PER_LAUNCH, layers in groups of
  // HEXKV_MAX_LAYERS_PER_LAUNCH; one launch per (group, group) pair.
  int64_t row_base = 0;
  int32_t cu[HEXKV_MAX_SEQS_PER_LAUNCH + 1];
  const int64_t seq_stride_bytes = seq_stride_rows * row_bytes;
  for (int b0 = 0; b0 < batch; b0 += HEXKV_MAX_SEQS_PER_LAUNCH) {
    const int nb = std::min(batch - b0, HEXKV_MAX_SEQS_PER_LAUNCH);
    cu[0] = 0;
    for (int b = 0; b < nb; ++b) cu[b + 1] = cu[b] + static_cast<int32_t>(lens[b0 + b]);
    const int64_t padded_off = static_cast<int64_t>(b0) * seq_stride_bytes;
    const int64_t packed_off = row_base * row_bytes;
    row_base += cu[nb];
    if (cu[nb] == 0) continue;
    for (int l0 = 0; l0 < n_layers; l0 += HEXKV_MAX_LAYERS_PER_LAUNCH) {
      const int nl = std::min(n_layers - l0, HEXKV_MAX_LAYERS_PER_LAUNCH);
      const int rc = nl <= 32 && nb <= 16
          ? launch_copy<SmallCopyArgs>(pack, vec16, src_layers, dst_layers, l0, nl, nb, cu, row_bytes,
                                       seq_stride_bytes, chunk, padded_off, packed_off, stream, what)
          : launch_copy<WideCopyArgs>(pack, vec16, src_layers, dst_layers, l0, nl, nb, cu, row_bytes,
                                      seq_stride_bytes, chunk, padded_off, packed_off, stream, what);
      if (rc != HEXKV_OK) return rc;
    }
  }
  return HEXKV_OK;
}

}  // namespace hexkv

extern "C" int hexkv_pack(const void *const *cache_layers, void *const *packed_layers, int n_layers,
                          int batch, int64_t seq_stride_rows, int64_t capacity, int64_t row_bytes,
                          const int64_t *lens, hexkv_stream_t stream) {
  return hexkv::ragged_copy(true, cache_layers, packed_layers, n_layers, batch, seq_stride_rows,
                            capacity, row_bytes, lens, static_cast<hipStream_t>(stream));
}

extern "C" int hexkv_unpack(const void *const *packed_layers, void *const *cache_layers,
                            int n_layers, int batch, int64_t seq_stride_rows, int64_t capacity,
                            int64_t row_bytes, const int64_t *lens, hexkv_stream_t stream) {
  return hexkv::ragged_copy(false, packed_layers, cache_layers, n_layers, batch, seq_stride_rows,
                            capacity, row_bytes, lens, static_cast<hipStream_t>(stream));
}

extern "C" int hexkv_append(const void *kv_new, void *cache, int batch, int64_t seq_stride_rows,
                            int64_t capacity, int64_t row_bytes, const int32_t *positions_dev,
                            int32_t position_bias, hexkv_stream_t stream) {
  using namespace hexkv;
  clear_error();
  if (batch < 0) return fail(HEXKV_EINVAL, "hexkv_append: negative batch");
  if (batch == 0) return HEXKV_OK;
  if (!kv_new || !cache) return fail(HEXKV_EINVAL, "hexkv_append: null argument");
  if (row_bytes <= 0 || row_bytes % 4 != 0)
    return fail(HEXKV_EINVAL, "hexkv_append: row_bytes %lld is not a positive multiple of 4",
                static_cast<long long>(row_bytes));
  if (capacity <= 0 || (batch > 1 && seq_stride_rows < capacity))
    return fail(HEXKV_EINVAL, "hexkv_append: bad capacity/stride");
  if (batch > 65535) return fail(HEXKV_EINVAL, "hexkv_append: batch above 65535");
  if (!positions_dev && (position_bias < 0 || position_bias >= capacity))
    return fail(HEXKV_ERANGE, "hexkv_append: position %d outside [0, %lld)", position_bias,
                static_cast<long long>(capacity));
  if ((reinterpret_cast<uintptr_t>(kv_new) | reinterpret_cast<uintptr_t>(cache)) & 3)
    return fail(HEXKV_EINVAL, "hexkv_append: pointers not 4-byte aligned");
  const bool vec16 = row_bytes % 16 == 0 && aligned16(kv_new) && aligned16(cache);
  const int64_t nv = row_bytes / (vec16 ? 16 : 4);
  const unsigned gx = static_cast<unsigned>(std::min<int64_t>((nv + kAppendThreads - 1) / kAppendThreads, 64));
  dim3 grid(gx, static_cast<unsigned>(batch));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t stride = seq_stride_rows * row_bytes;
  // Positions read on the device can fall outside the cache: such rows are
  // skipped and reported through the status word.
  unsigned int *status = nullptr;
  if (positions_dev) {
    const int rc = status_word(stream, &status, "hexkv_append");
    if (rc != HEXKV_OK) return rc;
  }
  if (vec16)
    append_kernel<u32x4><<<grid, kAppendThreads, 0, s>>>(static_cast<const char *>(kv_new),
        static_cast<char *>(cache), stride, capacity, row_bytes, positions_dev, position_bias, status);
  else
    append_kernel<unsigned int><<<grid, kAppendThreads, 0, s>>>(static_cast<const char *>(kv_new),
        static_cast<char *>(cache), stride, capacity, row_bytes, positions_dev, position_bias, status);
  return check_launch("hexkv_append");
}

extern "C" int hexkv_device_status(uint32_t *flags, int clear, hexkv_stream_t stream) {
  using namespace hexkv;
  clear_error();
  const char *what = "hexkv_device_status";
  if (!flags) return fail(HEXKV_EINVAL, "%s: null argument", what);
  unsigned int *word = nullptr;
  int rc = status_word(stream, &word, what);
  if (rc != HEXKV_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = hipStreamSynchronize(s);
  if (e == hipSuccess) e = hipMemcpyAsync(flags, word, sizeof(*flags), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess && clear) e = hipMemsetAsync(word, 0, sizeof(*word), s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return fail(HEXKV_EHIP, "%s: %s", what, hipGetErrorString(e));
  return HEXKV_OK;
}
