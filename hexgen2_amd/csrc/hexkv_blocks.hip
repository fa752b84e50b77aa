// Strided byte-row gathers of the legacy KV formats: hexkv_flat_concat,
// hexkv_batch_pad and hexkv_head_concat (hexkv.h).
//
// All three reduce to one engine.  A launch carries up to kMaxSpans spans in
// its kernel arguments; a span is depth x height rows of `width` bytes to
// move from a source block (or to zero-fill) to a destination with pitches
// of its own.  The host normalises each span (rows contiguous on both sides
// merge into one long row; slices that follow each other become rows) and
// cuts it into tiles of about one chunk of bytes: whole rows when rows are
// short, row pieces when they are long.  When every layer's spans have one
// shape and advance by fixed strides from layer to layer (layers that are
// views of one stacked allocation), the layers fold into a fourth dimension
// of each span and one launch moves them all.  One workgroup moves one tile with
// nontemporal 16-byte loads and stores (narrower vectors only when an
// address, pitch or width is not a multiple of 16): eight in flight per lane
// when every tile of the launch is a wide row, four otherwise, where short
// rows are spread over the workgroup several per pass, so a 256-byte head
// slice keeps every lane busy.  The tile -> span lookup is one scalar
// binary search over the prefix sums of tile counts.
#include "hexkv_common.h"

#include <algorithm>
#include <vector>

namespace hexkv {

// Tiles of at most 128 KB.  A launch whose tiles are all wide rows (at least
// kWideThreads vectors) runs kWideThreads threads with kWideUnroll vectors in
// flight per lane, a whole tile loaded before it is stored, as the ragged
// copy does; any other launch runs kSpanThreads x kSpanUnroll, which spreads
// short rows over the workgroup.  On MI355X (all variants on the same
// buffers in one process): flat packet 6.02 TB/s with 1024 x 8 against 5.72
// with 512 x 4, zero-pad batching 5.47 against 5.11, but TP head
// concatenation (256-byte rows) 4.87 against 5.17.  The FT store has its own
// thread count and tile shape.
constexpr int kSpanThreads = 512;
constexpr int kSpanUnroll = 4;
constexpr int kWideThreads = 1024;
constexpr int kWideUnroll = 8;
constexpr int kFtThreads = 1024;
constexpr int kMaxSpans = 32;

struct Span {
  const char *src;  // nullptr: zero-fill the destination rows
  char *dst;
  int64_t width;                                   // bytes per row
  int64_t src_row, src_slice, dst_row, dst_slice;  // pitches, bytes
  int64_t src_layer, dst_layer;                    // pitches between layers, bytes
  int64_t tile_cols;                               // bytes of one row per tile
  int32_t height;                                  // rows per slice
  int32_t depth;                                   // slices per layer
  int32_t tile_rows;                               // rows per tile
  int32_t row_tiles;                               // tiles down one slice
  int32_t col_tiles;                               // tiles along one row
};

struct SpanArgs {
  Span span[kMaxSpans];
  int32_t first_tile[kMaxSpans + 1];  // prefix sums of tiles per span
  int32_t n;
};
static_assert(sizeof(SpanArgs) <= 4096, "kernel arguments above 4 KiB");

// The work of one span_copy_kernel workgroup (`tile`): rows [r0, r1) of
// one slice of one layer of one span, `bytes` of each row from column c0.
// Host and device share this decode (the CPU emulation of the kernel calls
// it), so the arithmetic that is bounds-checked is the one that runs.
struct SpanTile {
  const char *src;  // the tile's first byte in row 0 (nullptr: zero fill)
  char *dst;
  int64_t src_row, dst_row;  // row pitches, bytes
  int64_t bytes;             // bytes of each row this tile moves
  int r0, r1;
};

__host__ __device__ inline int span_of_tile(const SpanArgs &a, int tile) {
  int lo = 0, hi = a.n;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (a.first_tile[mid] <= tile) lo = mid; else hi = mid;
  }
  return lo;
}

__host__ __device__ inline SpanTile span_tile(const SpanArgs &a, int tile) {
  const int i = span_of_tile(a, tile);
  const Span &s = a.span[i];
  int t = tile - a.first_tile[i];
  const int ct = t % s.col_tiles;
  t /= s.col_tiles;
  const int rt = t % s.row_tiles;
  t /= s.row_tiles;
  const int64_t k = t % s.depth;  // slice
  const int64_t m = t / s.depth;  // layer
  const int64_t c0 = static_cast<int64_t>(ct) * s.tile_cols;
  const int64_t c1 = s.width < c0 + s.tile_cols ? s.width : c0 + s.tile_cols;
  SpanTile w;
  w.src = s.src ? s.src + m * s.src_layer + k * s.src_slice + c0 : nullptr;
  w.dst = s.dst + m * s.dst_layer + k * s.dst_slice + c0;
  w.src_row = s.src_row;
  w.dst_row = s.dst_row;
  w.bytes = c1 - c0;
  w.r0 = rt * s.tile_rows;
  w.r1 = s.height < w.r0 + s.tile_rows ? s.height : w.r0 + s.tile_rows;
  return w;
}

// Short rows (fewer vectors than threads): `per` rows per pass, lane `tid`
// at (row in pass tr, vector tc); lanes with tr >= per idle.
struct RowLane {
  int per, tr, tc;
};

__host__ __device__ inline RowLane row_lane(int threads, int vectors, int tid) {
  RowLane l;
  l.per = threads / vectors;
  l.tr = tid / vectors;
  l.tc = tid - l.tr * vectors;
  return l;
}

// A wide row piece: the workgroup strides along it.  A zero fill (no
// source) has its own loop with eight stores in flight per lane: on MI355X
// zero-pad batching moved 5.12 TB/s with it against 5.05 with the copy loop
// storing zeros, and the copy loop without the per-element source test moved
// the flat packet at 5.72 against 5.63.
template <typename V, int T, int UR>
__device__ __forceinline__ void move_row(const char *__restrict__ s, char *__restrict__ d, int64_t nv) {
  const V *sv = reinterpret_cast<const V *>(s);
  V *dv = reinterpret_cast<V *>(d);
  int64_t i = threadIdx.x;
  if (!sv) {
    constexpr int kZeroUnroll = 8;
    for (; i + (kZeroUnroll - 1) * T < nv; i += kZeroUnroll * T) {
#pragma unroll
      for (int u = 0; u < kZeroUnroll; ++u) __builtin_nontemporal_store(V{}, dv + i + u * T);
    }
    for (; i < nv; i += T) __builtin_nontemporal_store(V{}, dv + i);
    return;
  }
  for (; i + (UR - 1) * T < nv; i += UR * T) {
    V r[UR];
#pragma unroll
    for (int u = 0; u < UR; ++u) r[u] = __builtin_nontemporal_load(sv + i + u * T);
#pragma unroll
    for (int u = 0; u < UR; ++u) __builtin_nontemporal_store(r[u], dv + i + u * T);
  }
  for (; i < nv; i += T) __builtin_nontemporal_store(__builtin_nontemporal_load(sv + i), dv + i);
}

template <typename V, int T, int UR>
__global__ __launch_bounds__(T) void span_copy_kernel(const SpanArgs a) {
  const SpanTile w = span_tile(a, blockIdx.x);
  const int64_t nv = w.bytes / static_cast<int64_t>(sizeof(V));
  if (nv >= T) {
    for (int r = w.r0; r < w.r1; ++r)
      move_row<V, T, UR>(w.src ? w.src + r * w.src_row : nullptr, w.dst + r * w.dst_row, nv);
    return;
  }
  const RowLane l = row_lane(T, static_cast<int>(nv), threadIdx.x);
  if (l.tr >= l.per) return;
  const int64_t col = static_cast<int64_t>(l.tc) * static_cast<int64_t>(sizeof(V));
  for (int r = w.r0 + l.tr; r < w.r1; r += l.per * UR) {
    V v[UR];
#pragma unroll
    for (int u = 0; u < UR; ++u) {
      const int rr = r + u * l.per;
      v[u] = V{};
      if (w.src && rr < w.r1) v[u] = __builtin_nontemporal_load(reinterpret_cast<const V *>(w.src + rr * w.src_row + col));
    }
#pragma unroll
    for (int u = 0; u < UR; ++u) {
      const int rr = r + u * l.per;
      if (rr < w.r1) __builtin_nontemporal_store(v[u], reinterpret_cast<V *>(w.dst + rr * w.dst_row + col));
    }
  }
}

// Head concatenation as a gather (hexkv_head_concat's fast path): a
// workgroup takes a tile of destination rows and its lanes lie across one
// destination row, each lane in the shard its column falls in; every pass
// loads kWideUnroll rows per lane from the shards' own rows, then stores the
// whole destination rows.  Reads stay contiguous per shard, writes become
// whole-row runs instead of one shard's slice per row (the span engine
// writes 256-byte pieces 2 KB apart for eight one-head shards).
constexpr int kGatherShards = 16;

struct GatherArgs {
  const char *src[kGatherShards];
  int64_t src_pitch[kGatherShards];   // bytes between a shard's rows
  int64_t src_layer[kGatherShards];   // bytes between a shard's layers
  int32_t vec_start[kGatherShards + 1];  // first 16-byte column of each shard
  char *dst;
  int64_t dst_layer;
  int64_t rows;           // rows per layer
  int32_t wvec;           // 16-byte vectors per destination row (<= kWideThreads)
  int32_t n;              // shards
  int32_t rows_per_tile;
};

// What lane `tid` of head_gather_kernel's workgroup (tile, layer) moves:
// destination rows r0 + tr, r0 + tr + per, ... below r1, 16 bytes at column
// vector tc, read from shard `shard`.  Shared with the CPU emulation.
struct GatherLane {
  const char *src;  // the lane's 16 bytes in source row 0
  char *dst;        // the lane's 16 bytes in destination row 0
  int64_t src_pitch, dst_pitch, r0, r1;
  int per, tr, tc, shard;
};

__host__ __device__ inline GatherLane gather_lane(const GatherArgs &a, int64_t tile, int64_t layer, int tid) {
  GatherLane g;
  const RowLane rl = row_lane(kWideThreads, a.wvec, tid);
  g.per = rl.per;
  g.tr = rl.tr;
  g.tc = rl.tc;
  g.r0 = tile * a.rows_per_tile;
  g.r1 = a.rows < g.r0 + a.rows_per_tile ? a.rows : g.r0 + a.rows_per_tile;
  int j = 0;
  while (j + 1 < a.n && a.vec_start[j + 1] <= g.tc) ++j;
  g.shard = j;
  g.src = a.src[j] + layer * a.src_layer[j] + static_cast<int64_t>(g.tc - a.vec_start[j]) * 16;
  g.src_pitch = a.src_pitch[j];
  g.dst = a.dst + layer * a.dst_layer + static_cast<int64_t>(g.tc) * 16;
  g.dst_pitch = static_cast<int64_t>(a.wvec) * 16;
  return g;
}

// The row lane u of a pass starting at row r loads: past the tile's last
// row it reloads that row (a clamped, in-bounds load whose value is not
// stored), so every lane issues kWideUnroll loads before any store.
__host__ __device__ inline int64_t gather_load_row(const GatherLane &g, int64_t r, int u) {
  const int64_t rr = r + static_cast<int64_t>(u) * g.per;
  return rr < g.r1 - 1 ? rr : g.r1 - 1;
}

__global__ __launch_bounds__(kWideThreads) void head_gather_kernel(const GatherArgs a) {
  const GatherLane g = gather_lane(a, blockIdx.x, blockIdx.y, threadIdx.x);
  if (g.tr >= g.per) return;
  for (int64_t r = g.r0 + g.tr; r < g.r1; r += static_cast<int64_t>(g.per) * kWideUnroll) {
    u32x4 v[kWideUnroll];
#pragma unroll
    for (int u = 0; u < kWideUnroll; ++u)
      v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(g.src + gather_load_row(g, r, u) * g.src_pitch));
#pragma unroll
    for (int u = 0; u < kWideUnroll; ++u) {
      const int64_t rr = r + u * g.per;
      if (rr < g.r1) __builtin_nontemporal_store(v[u], reinterpret_cast<u32x4 *>(g.dst + rr * g.dst_pitch));
    }
  }
}

// FT store (hexkv_ft_store): kv rows [2][H][D] -> K chunk planes and
// head-major V.  A workgroup takes up to kFtRows positions x kFtCols 16-byte
// chunks of one sequence: it reads the K chunks row by row (kFtCols x 16-byte
// pieces) into LDS and writes them out plane by plane (kFtRows x 16-byte
// runs); the V chunks go straight from the rows to their head rows.  Long
// plane runs matter more than long row reads: on MI355X with a 64 x 4096
// position Llama-3-8B prefill and 256 threads, 16 x 128 tiles moved 4.0
// TB/s, 64 x 32 5.1, 128 x 16 5.4 and 256 x 8 5.6; 1024 threads on 512 x 8
// tiles take 0.374 ms against 0.384 for 256 on 256 x 8 (5.74 TB/s; 512
// threads on 256 x 8 0.398, on 512 x 8 0.376; 1024 on 1024 x 8 0.410, and
// on whole-head 256 x 16 or 512 x 16 tiles, which write V in one run per
// head, 0.403-0.406).
constexpr int kFtRows = 512, kFtCols = 8;

struct FtStoreArgs {
  const char *src;  // K of sequence 0, position 0
  int64_t src_batch, src_pos, src_kv;
  char *k, *v;
  int64_t k_batch, v_batch, k_plane, v_head;  // bytes
  int32_t head_chunks;                        // 16-byte chunks per head row
  int32_t chunks;                             // 16-byte chunks of a row's K (= of its V)
  int32_t seq_len;
};

__global__ __launch_bounds__(kFtThreads) void ft_store_kernel(const FtStoreArgs a) {
  __shared__ u32x4 s_tile[kFtRows][kFtCols + 1];  // padded: plane-wise reads spread over the banks
  const int tid = threadIdx.x;
  const int p0 = blockIdx.x * kFtRows, c0 = blockIdx.y * kFtCols;
  const int64_t b = blockIdx.z;
  const int np = min(kFtRows, a.seq_len - p0), nc = min(kFtCols, a.chunks - c0);
  const char *rows = a.src + b * a.src_batch + static_cast<int64_t>(p0) * a.src_pos;
  // Every load of the tile is issued before the first store: a store may
  // alias the source as far as the compiler knows, so loads interleaved with
  // stores would wait for each other and leave one load in flight per lane.
  // A thread keeps one chunk column and steps down kPass rows at a time; the
  // loads of rows and columns past the tile's edge are clamped to its last
  // row and column (in bounds, never stored), so no load is conditional.
  constexpr int kPass = kFtThreads / kFtCols, kPer = kFtRows / kPass;
  static_assert(kFtThreads % kFtCols == 0 && kFtRows % kPass == 0, "FT tile does not split over the workgroup");
  const int c = tid % kFtCols, pb = tid / kFtCols;
  const bool col = c < nc;
  const int g = c0 + min(c, nc - 1), h = g / a.head_chunks, cc = g - h * a.head_chunks;
  const char *src = rows + static_cast<int64_t>(g) * 16;
  char *vdst = a.v + b * a.v_batch + h * a.v_head + (static_cast<int64_t>(p0) * a.head_chunks + cc) * 16;
  u32x4 kr[kPer], vr[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int p = min(pb + i * kPass, np - 1);
    kr[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src + p * a.src_pos));
    vr[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src + p * a.src_pos + a.src_kv));
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int p = pb + i * kPass;
    if (col && p < np) {
      s_tile[p][c] = kr[i];
      __builtin_nontemporal_store(vr[i], reinterpret_cast<u32x4 *>(vdst + static_cast<int64_t>(p) * a.head_chunks * 16));
    }
  }
  __syncthreads();
  for (int q = tid; q < kFtRows * kFtCols; q += kFtThreads) {
    const int c = q / kFtRows, p = q % kFtRows;
    if (p < np && c < nc) {
      char *dst = a.k + b * a.k_batch + (c0 + c) * a.k_plane + static_cast<int64_t>(p0 + p) * 16;
      __builtin_nontemporal_store(s_tile[p][c], reinterpret_cast<u32x4 *>(dst));
    }
  }
}

// ------------------------------------------------------------------ host ---

// One span before tiling (all sizes in bytes): `layers` copies of a
// depth x height x width block, layer pitches apart.
struct Move {
  const char *src;  // nullptr: zero fill
  char *dst;
  int64_t width, height, depth;
  int64_t src_row, src_slice, dst_row, dst_slice;
  int64_t layers = 1, src_layer = 0, dst_layer = 0;
};

static int64_t move_bytes(const Move &m) { return m.width * m.height * m.depth * m.layers; }

static bool same_shape(const Move &a, const Move &b) {
  return a.width == b.width && a.height == b.height && a.depth == b.depth && a.src_row == b.src_row &&
         a.src_slice == b.src_slice && a.dst_row == b.dst_row && a.dst_slice == b.dst_slice &&
         (a.src == nullptr) == (b.src == nullptr) && a.layers == 1 && b.layers == 1;
}

// `moves` holds n_layers groups of equally many moves, layer by layer.  When
// move j of every layer has one shape and its source and destination advance
// by fixed strides from layer to layer (the layers are views of one stacked
// allocation), the n_layers copies become one move with a layer dimension:
// one launch carries every layer.  Otherwise `moves` is left as it is.
static void merge_layers(std::vector<Move> &moves, int n_layers) {
  if (n_layers < 2 || moves.empty() || moves.size() % n_layers) return;
  const size_t per = moves.size() / n_layers;
  std::vector<Move> merged(moves.begin(), moves.begin() + per);
  for (size_t j = 0; j < per; ++j) {
    const Move &m0 = moves[j], &m1 = moves[per + j];
    if (!same_shape(m0, m1)) return;
    const int64_t ds = m0.src ? m1.src - m0.src : 0, dd = m1.dst - m0.dst;
    for (int l = 2; l < n_layers; ++l) {
      const Move &ml = moves[l * per + j];
      if (!same_shape(m0, ml) || (m0.src && ml.src - m0.src != ds * l) || ml.dst - m0.dst != dd * l) return;
    }
    merged[j].layers = n_layers;
    merged[j].src_layer = ds;
    merged[j].dst_layer = dd;
  }
  moves.swap(merged);
}

// Merges dimensions that are contiguous on both sides, so the engine moves
// the longest possible rows and tiles several short rows together.
static void normalise(Move &m) {
  auto merge_rows = [&m] {  // rows follow each other on both sides: one row
    if (m.height > 1 && m.dst_row == m.width && (!m.src || m.src_row == m.width)) {
      m.width *= m.height;
      m.height = 1;
      m.src_row = m.dst_row = m.width;
    }
  };
  merge_rows();
  if (m.depth > 1 && m.dst_slice == m.height * m.dst_row && (!m.src || m.src_slice == m.height * m.src_row)) {
    m.height *= m.depth;  // slices follow each other: one slice
    m.depth = 1;
  } else if (m.height == 1 && m.depth > 1) {
    m.height = m.depth;  // single-row slices become rows, so short ones share a tile
    m.src_row = m.src_slice;
    m.dst_row = m.dst_slice;
    m.depth = 1;
  }
  merge_rows();
}

// Bytes per tile: about total / 8192 workgroups, 16 KB to 128 KB.
static int64_t tile_bytes(int64_t total) {
  const int64_t chunk = (total / 8192 + 4095) / 4096 * 4096;
  return std::min<int64_t>(std::max<int64_t>(chunk, 16384), 131072);
}

template <typename V>
static void launch_spans(const SpanArgs &a, int tiles, bool wide, hipStream_t s) {
  if (wide) span_copy_kernel<V, kWideThreads, kWideUnroll><<<dim3(static_cast<unsigned>(tiles)), kWideThreads, 0, s>>>(a);
  else span_copy_kernel<V, kSpanThreads, kSpanUnroll><<<dim3(static_cast<unsigned>(tiles)), kSpanThreads, 0, s>>>(a);
}

// Moves every span, kMaxSpans per launch, in order on `stream`.
static int run_moves(std::vector<Move> &moves, hipStream_t stream, const char *what) {
  int64_t total = 0;
  uint64_t align = 0;  // OR of every address, pitch and width in use
  std::vector<Move> live;
  live.reserve(moves.size());
  for (Move &m : moves) {
    if (move_bytes(m) == 0) continue;
    normalise(m);
    if (m.height > INT32_MAX) return fail(HEXKV_ERANGE, "%s: more than 2^31-1 rows in one block", what);
    total += move_bytes(m);
    align |= reinterpret_cast<uintptr_t>(m.dst) | static_cast<uint64_t>(m.width);
    if (m.src) align |= reinterpret_cast<uintptr_t>(m.src);
    if (m.height > 1) align |= static_cast<uint64_t>(m.dst_row) | static_cast<uint64_t>(m.src ? m.src_row : 0);
    if (m.depth > 1)
      align |= static_cast<uint64_t>(m.dst_slice) | static_cast<uint64_t>(m.src ? m.src_slice : 0);
    if (m.layers > 1)
      align |= static_cast<uint64_t>(m.dst_layer) | static_cast<uint64_t>(m.src ? m.src_layer : 0);
    if (m.depth > INT32_MAX || m.layers * m.depth > INT32_MAX)
      return fail(HEXKV_ERANGE, "%s: more than 2^31-1 slices in one block set", what);
    live.push_back(m);
  }
  if (live.empty()) return HEXKV_OK;
  const int vec = (align & 15) == 0 ? 16 : (align & 3) == 0 ? 4 : (align & 1) == 0 ? 2 : 1;
  const int64_t chunk = tile_bytes(total);

  size_t i = 0;
  while (i < live.size()) {
    SpanArgs a;
    int64_t tiles = 0;
    int n = 0;
    for (; i < live.size() && n < kMaxSpans; ++i, ++n) {
      const Move &m = live[i];
      Span &s = a.span[n];
      s.src = m.src;
      s.dst = m.dst;
      s.width = m.width;
      s.src_row = m.src_row;
      s.src_slice = m.src_slice;
      s.dst_row = m.dst_row;
      s.dst_slice = m.dst_slice;
      s.src_layer = m.src_layer;
      s.dst_layer = m.dst_layer;
      s.height = static_cast<int32_t>(m.height);
      s.depth = static_cast<int32_t>(m.depth);
      int64_t col_tiles, row_tiles, tile_rows;
      if (m.width >= chunk) {
        s.tile_cols = chunk;
        col_tiles = (m.width + chunk - 1) / chunk;
        tile_rows = 1;
        row_tiles = m.height;
      } else {
        s.tile_cols = m.width;
        col_tiles = 1;
        tile_rows = std::max<int64_t>(1, chunk / m.width);
        row_tiles = (m.height + tile_rows - 1) / tile_rows;
      }
      const int64_t span_tiles = m.layers * m.depth * row_tiles * col_tiles;
      if (span_tiles > INT32_MAX || tiles + span_tiles > INT32_MAX) {
        if (n == 0) return fail(HEXKV_ERANGE, "%s: block too large for one launch", what);
        break;  // next launch
      }
      s.tile_rows = static_cast<int32_t>(std::min<int64_t>(tile_rows, m.height));
      s.row_tiles = static_cast<int32_t>(row_tiles);
      s.col_tiles = static_cast<int32_t>(col_tiles);
      a.first_tile[n] = static_cast<int32_t>(tiles);
      tiles += span_tiles;
    }
    a.first_tile[n] = static_cast<int32_t>(tiles);
    a.n = n;
    // Wide launch: every span's tiles are rows of at least kWideThreads vectors.
    bool wide = true;
    for (int q = 0; q < n; ++q) wide = wide && a.span[q].tile_cols >= static_cast<int64_t>(kWideThreads) * vec;
    switch (vec) {
      case 16: launch_spans<u32x4>(a, static_cast<int>(tiles), wide, stream); break;
      case 4: launch_spans<unsigned int>(a, static_cast<int>(tiles), wide, stream); break;
      case 2: launch_spans<unsigned short>(a, static_cast<int>(tiles), wide, stream); break;
      default: launch_spans<unsigned char>(a, static_cast<int>(tiles), wide, stream); break;
    }
    const int rc = check_launch(what);
    if (rc != HEXKV_OK) return rc;
  }
  return HEXKV_OK;
}

// hexkv_head_concat through head_gather_kernel when the shapes allow it
// (validated blocks): at most kGatherShards shards, destination rows of at
// most kWideThreads 16-byte vectors, every shard's rows one level (depth 1,
// or slices that follow each other) with 16-byte aligned data and pitch,
// every layer holding rows.  Layers whose pointers advance by fixed strides
// share one launch; otherwise one launch per layer.  Returns false (nothing
// launched) when the shapes do not qualify.
static bool head_gather(const hexkv_block *src, int n_layers, int n_shards, void *const *dst_layers, int64_t row,
                        hipStream_t stream) {
  if (n_shards > kGatherShards || row <= 0 || row % 16 || row / 16 > kWideThreads) return false;
  const int64_t rows = src[0].depth * src[0].height;
  if (rows <= 0 || rows > INT64_C(1) << 40) return false;
  // Bytes between consecutive rows of a one-level block.
  const auto pitch = [](const hexkv_block &b) { return b.height > 1 || b.depth == 1 ? b.row_pitch : b.slice_pitch; };
  for (int l = 0; l < n_layers; ++l) {
    if (!dst_layers[l] || !aligned16(dst_layers[l])) return false;
    for (int j = 0; j < n_shards; ++j) {
      const hexkv_block &b = src[static_cast<int64_t>(l) * n_shards + j];
      if (b.depth * b.height != rows || b.width % 16) return false;
      if (b.width == 0) continue;
      if (!aligned16(b.data) || b.row_pitch % 16) return false;
      if (b.depth > 1 && b.slice_pitch != b.height * b.row_pitch) return false;
      if (pitch(b) != pitch(src[j])) return false;  // one pitch per shard over every layer
    }
  }
  GatherArgs a{};
  a.n = n_shards;
  a.wvec = static_cast<int32_t>(row / 16);
  a.rows = rows;
  a.rows_per_tile = static_cast<int32_t>(std::max<int64_t>(1, 131072 / row));
  a.vec_start[0] = 0;
  for (int j = 0; j < n_shards; ++j) {
    a.vec_start[j + 1] = a.vec_start[j] + static_cast<int32_t>(src[j].width / 16);
    a.src_pitch[j] = pitch(src[j]);
  }
  // One launch for every layer when the layers advance by fixed strides.
  bool fold = n_layers > 1 && n_layers <= 65535;
  const auto at = [&](int l, int j) { return static_cast<const char *>(src[static_cast<int64_t>(l) * n_shards + j].data); };
  for (int l = 2; fold && l < n_layers; ++l) {
    fold = static_cast<char *>(dst_layers[l]) - static_cast<char *>(dst_layers[0]) ==
           (static_cast<char *>(dst_layers[1]) - static_cast<char *>(dst_layers[0])) * l;
    for (int j = 0; fold && j < n_shards; ++j)
      fold = src[j].width == 0 || at(l, j) - at(0, j) == (at(1, j) - at(0, j)) * l;
  }
  const int64_t tiles = (rows + a.rows_per_tile - 1) / a.rows_per_tile;
  if (tiles > INT32_MAX) return false;
  for (int l0 = 0; l0 < n_layers; l0 += fold ? n_layers : 1) {
    const int nl = fold ? n_layers : 1;
    for (int j = 0; j < n_shards; ++j) {
      a.src[j] = at(l0, j);
      a.src_layer[j] = fold && src[j].width ? at(1, j) - at(0, j) : 0;
    }
    a.dst = static_cast<char *>(dst_layers[l0]);
    a.dst_layer = fold ? static_cast<char *>(dst_layers[1]) - static_cast<char *>(dst_layers[0]) : 0;
    head_gather_kernel<<<dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(nl)), kWideThreads, 0, stream>>>(a);
  }
  return true;
}

// Shape checks shared by the entry points: non-negative sizes, bytes that
// fit int64, a device address whenever the block holds bytes.
constexpr int64_t kMaxBytes = INT64_C(1) << 46;  // 64 TiB: no product below overflows

static int check_block(const hexkv_block &b, const char *what, int index) {
  if (b.width < 0 || b.height < 0 || b.depth < 0)
    return fail(HEXKV_EINVAL, "%s: block %d has a negative size", what, index);
  if (b.width == 0 || b.height == 0 || b.depth == 0) return HEXKV_OK;
  if (b.row_pitch < 0 || b.slice_pitch < 0)
    return fail(HEXKV_EINVAL, "%s: block %d has a negative pitch", what, index);
  if (b.width > kMaxBytes || b.height > kMaxBytes || b.depth > kMaxBytes ||
      b.width * b.height > kMaxBytes || b.width * b.height * b.depth > kMaxBytes)
    return fail(HEXKV_ERANGE, "%s: block %d is larger than 64 TiB", what, index);
  if (!b.data) return fail(HEXKV_EINVAL, "%s: block %d has no data pointer", what, index);
  return HEXKV_OK;
}

}  // namespace hexkv

extern "C" int hexkv_flat_concat(const hexkv_block *src, int n, void *dst, hexkv_stream_t stream) {
  using namespace hexkv;
  clear_error();
  const char *what = "hexkv_flat_concat";
  if (n < 0) return fail(HEXKV_EINVAL, "%s: negative block count", what);
  if (n > 0 && !src) return fail(HEXKV_EINVAL, "%s: null block array", what);
  std::vector<Move> moves;
  int64_t off = 0;
  for (int i = 0; i < n; ++i) {
    int rc = check_block(src[i], what, i);
    if (rc != HEXKV_OK) return rc;
    const hexkv_block &b = src[i];
    const int64_t bytes = b.width * b.height * b.depth;
    if (bytes == 0) continue;
    if (!dst) return fail(HEXKV_EINVAL, "%s: null destination", what);
    if (off > kMaxBytes) return fail(HEXKV_ERANGE, "%s: concatenation larger than 64 TiB", what);
    moves.push_back(Move{static_cast<const char *>(b.data), static_cast<char *>(dst) + off, b.width,
                         b.height, b.depth, b.row_pitch, b.slice_pitch, b.width, b.width * b.height});
    off += bytes;
  }
  merge_layers(moves, static_cast<int>(moves.size()));
  return run_moves(moves, static_cast<hipStream_t>(stream), what);
}

extern "C" int hexkv_batch_pad(const hexkv_block *src, int n_layers, int n_req, void *const *dst_layers,
                               int64_t max_rows, hexkv_stream_t stream) {
  using namespace hexkv;
  clear_error();
  const char *what = "hexkv_batch_pad";
  if (n_layers < 0 || n_req < 0 || max_rows < 0) return fail(HEXKV_EINVAL, "%s: negative count", what);
  if (n_layers == 0 || n_req == 0) return HEXKV_OK;
  if (!src || !dst_layers) return fail(HEXKV_EINVAL, "%s: null argument", what);
  const int64_t width = src[0].width;
  int64_t seqs = 0;
  for (int l = 0; l < n_layers; ++l) {
    for (int i = 0; i < n_req; ++i) {
      const hexkv_block &b = src[static_cast<int64_t>(l) * n_req + i];
      int rc = check_block(b, what, l * n_req + i);
      if (rc != HEXKV_OK) return rc;
      const hexkv_block &first = src[i];
      if (b.width != width)
        return fail(HEXKV_EINVAL, "%s: request %d of layer %d has rows of %lld bytes, not %lld", what, i, l,
                    static_cast<long long>(b.width), static_cast<long long>(width));
      if (b.depth != first.depth || b.height != first.height)
        return fail(HEXKV_EINVAL, "%s: request %d has other sizes in layer %d than in layer 0", what, i, l);
      if (b.height > max_rows)
        return fail(HEXKV_ERANGE, "%s: request %d holds %lld rows, above max_rows %lld", what, i,
                    static_cast<long long>(b.height), static_cast<long long>(max_rows));
    }
  }
  for (int i = 0; i < n_req && seqs <= kMaxBytes; ++i) seqs += src[i].depth;
  if (width > 0 && max_rows > kMaxBytes / width)
    return fail(HEXKV_ERANGE, "%s: padded sequence larger than 64 TiB", what);
  const int64_t seq_bytes = max_rows * width;
  if (seqs > kMaxBytes || (seq_bytes > 0 && seqs > kMaxBytes / seq_bytes))
    return fail(HEXKV_ERANGE, "%s: batched layer larger than 64 TiB", what);
  std::vector<Move> moves;
  for (int l = 0; l < n_layers; ++l) {
    if (seqs * seq_bytes == 0) break;
    if (!dst_layers[l]) return fail(HEXKV_EINVAL, "%s: null destination of layer %d", what, l);
    char *base = static_cast<char *>(dst_layers[l]);
    for (int i = 0; i < n_req; ++i) {
      const hexkv_block &b = src[static_cast<int64_t>(l) * n_req + i];
      moves.push_back(Move{static_cast<const char *>(b.data), base, width, b.height, b.depth, b.row_pitch,
                           b.slice_pitch, width, seq_bytes});
      moves.push_back(Move{nullptr, base + b.height * width, width, max_rows - b.height, b.depth, 0, 0,
                           width, seq_bytes});
      base += b.depth * seq_bytes;
    }
  }
  merge_layers(moves, n_layers);
  // Every copy before any zero fill (the destinations are disjoint): on
  // MI355X 5.59 TB/s against 5.47 with each request's fill after its copy.
  std::stable_partition(moves.begin(), moves.end(), [](const Move &m) { return m.src != nullptr; });
  return run_moves(moves, static_cast<hipStream_t>(stream), what);
}

extern "C" int hexkv_head_concat(const hexkv_block *src, int n_layers, int n_shards, void *const *dst_layers,
                                 hexkv_stream_t stream) {
  using namespace hexkv;
  clear_error();
  const char *what = "hexkv_head_concat";
  if (n_layers < 0 || n_shards < 0) return fail(HEXKV_EINVAL, "%s: negative count", what);
  if (n_layers == 0 || n_shards == 0) return HEXKV_OK;
  if (!src || !dst_layers) return fail(HEXKV_EINVAL, "%s: null argument", what);
  int64_t row = 0;  // destination row bytes
  for (int j = 0; j < n_shards; ++j) {
    if (src[j].width < 0 || src[j].width > kMaxBytes || row > kMaxBytes)
      return fail(HEXKV_ERANGE, "%s: shard %d row width out of range", what, j);
    row += src[j].width;
  }
  std::vector<Move> moves;
  for (int l = 0; l < n_layers; ++l) {
    const hexkv_block *shards = src + static_cast<int64_t>(l) * n_shards;
    for (int j = 0; j < n_shards; ++j) {
      int rc = check_block(shards[j], what, l * n_shards + j);
      if (rc != HEXKV_OK) return rc;
      if (shards[j].width != src[j].width)
        return fail(HEXKV_EINVAL, "%s: shard %d of layer %d has rows of %lld bytes, %lld in layer 0", what, j,
                    l, static_cast<long long>(shards[j].width), static_cast<long long>(src[j].width));
      if (shards[j].depth * shards[j].height != shards[0].depth * shards[0].height)
        return fail(HEXKV_EINVAL, "%s: the shards of layer %d hold different numbers of rows", what, l);
    }
    const int64_t rows = shards[0].depth * shards[0].height;
    if (row == 0 || rows == 0) continue;
    if (row > kMaxBytes / rows) return fail(HEXKV_ERANGE, "%s: concatenated layer larger than 64 TiB", what);
    if (!dst_layers[l]) return fail(HEXKV_EINVAL, "%s: null destination of layer %d", what, l);
    int64_t col = 0;
    for (int j = 0; j < n_shards; ++j) {
      // Destination row k * height_j + r of shard j's (slice k, row r).
      const hexkv_block &b = shards[j];
      moves.push_back(Move{static_cast<const char *>(b.data), static_cast<char *>(dst_layers[l]) + col, b.width,
                           b.height, b.depth, b.row_pitch, b.slice_pitch, row, row * b.height});
      col += b.width;
    }
  }
  if (head_gather(src, n_layers, n_shards, dst_layers, row, static_cast<hipStream_t>(stream)))
    return check_launch(what);
  merge_layers(moves, n_layers);
  return run_moves(moves, static_cast<hipStream_t>(stream), what);
}

extern "C" int hexkv_ft_store(const void *kv, int64_t kv_batch_stride, int64_t kv_pos_stride, int64_t kv_stride,
                              void *k_cache, void *v_cache, int batch, int seq_len, int64_t capacity,
                              int kv_heads, int head_dim, int dtype, hexkv_stream_t stream) {
  using namespace hexkv;
  clear_error();
  const char *what = "hexkv_ft_store";
  if (dtype != HEXKV_F16 && dtype != HEXKV_BF16 && dtype != HEXKV_F32)
    return fail(HEXKV_EINVAL, "%s: unknown dtype %d", what, dtype);
  const int64_t es = dtype == HEXKV_F32 ? 4 : 2, pack = 16 / es;
  if (batch < 0 || seq_len < 0 || kv_heads < 1 || head_dim < 1 || capacity < 0)
    return fail(HEXKV_EINVAL, "%s: negative or empty size", what);
  if (head_dim % pack) return fail(HEXKV_EINVAL, "%s: head_dim %d not a multiple of %lld", what, head_dim,
                                   static_cast<long long>(pack));
  if (seq_len > capacity)
    return fail(HEXKV_ERANGE, "%s: seq_len %d above capacity %lld", what, seq_len, static_cast<long long>(capacity));
  if (kv_batch_stride < 0 || kv_pos_stride < 0 || kv_stride < 0)
    return fail(HEXKV_EINVAL, "%s: negative stride", what);
  if (batch == 0 || seq_len == 0) return HEXKV_OK;
  if (!kv || !k_cache || !v_cache) return fail(HEXKV_EINVAL, "%s: null tensor", what);
  const int64_t head = static_cast<int64_t>(head_dim) * es;  // bytes of one head row
  const int64_t heads = static_cast<int64_t>(kv_heads) * head;
  if (capacity > kMaxBytes / heads || batch > kMaxBytes / (capacity * heads))
    return fail(HEXKV_ERANGE, "%s: caches larger than 64 TiB", what);
  const char *src = static_cast<const char *>(kv);
  if (aligned16(kv) && aligned16(k_cache) && aligned16(v_cache) && (kv_batch_stride * es) % 16 == 0 &&
      (kv_pos_stride * es) % 16 == 0 && (kv_stride * es) % 16 == 0 && head % 16 == 0 && heads / 16 <= INT32_MAX &&
      batch <= 65535) {
    FtStoreArgs a;
    a.src = src;
    a.src_batch = kv_batch_stride * es;
    a.src_pos = kv_pos_stride * es;
    a.src_kv = kv_stride * es;
    a.k = static_cast<char *>(k_cache);
    a.v = static_cast<char *>(v_cache);
    a.k_batch = a.v_batch = capacity * heads;
    a.k_plane = capacity * 16;
    a.v_head = capacity * head;
    a.head_chunks = static_cast<int32_t>(head / 16);
    a.chunks = static_cast<int32_t>(heads / 16);
    a.seq_len = seq_len;
    const dim3 grid((seq_len + kFtRows - 1) / kFtRows, (a.chunks + kFtCols - 1) / kFtCols, batch);
    if (grid.y > 65535) return fail(HEXKV_ERANGE, "%s: rows of more than %d chunks", what, 65535 * kFtCols);
    ft_store_kernel<<<grid, kFtThreads, 0, static_cast<hipStream_t>(stream)>>>(a);
    return check_launch(what);
  }
  // Unaligned views: the span engine.
  // K: for every (head, 16-byte chunk) slice, seq_len positions of 16 bytes,
  // from rows kv_pos_stride apart into chunk rows packed back to back.
  Move k{src, static_cast<char *>(k_cache), 16, seq_len, heads / 16, kv_pos_stride * es, 16, 16, capacity * 16};
  k.layers = batch;
  k.src_layer = kv_batch_stride * es;
  k.dst_layer = capacity * heads;
  // V: per head, seq_len head rows into rows head bytes apart.
  Move v{src + kv_stride * es, static_cast<char *>(v_cache), head, seq_len, kv_heads, kv_pos_stride * es, head,
         head, capacity * head};
  v.layers = batch;
  v.src_layer = kv_batch_stride * es;
  v.dst_layer = capacity * heads;
  std::vector<Move> moves{k, v};
  return run_moves(moves, static_cast<hipStream_t>(stream), what);
}
