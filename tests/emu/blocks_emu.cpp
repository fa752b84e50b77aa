// CPU emulation of the legacy-format kernels (span_copy_kernel in both launch
// shapes, head_gather_kernel) for bounds and correctness checks without a
// GPU.  The real host code of hexkv_blocks.hip is compiled in; its kernel
// launches are intercepted (hipLaunchKernel and the call-configuration hooks
// are defined here) and each workgroup and lane is replayed on the CPU
// through the kernels' own __host__ __device__ index functions (span_tile,
// row_lane, gather_lane, gather_load_row).  Every source and destination access
// must fall inside a registered buffer and be aligned to its vector width;
// the bytes are moved, so the caller can compare the result with the
// oracle.  Used by tests/test_blocks_emulated.py.
#include "hexkv_blocks.hip"
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <vector>

struct Buf { uintptr_t lo, hi; bool dst; };
static std::vector<Buf> g_bufs;
static long g_violations = 0, g_launches = 0, g_tiles = 0;

extern "C" void emu_register(uintptr_t p, uint64_t n, int is_dst) { g_bufs.push_back({p, p + n, is_dst != 0}); }
extern "C" void emu_clear() { g_bufs.clear(); }
extern "C" long emu_violations() { return g_violations; }
extern "C" long emu_launches() { return g_launches; }
extern "C" long emu_tiles() { return g_tiles; }

static bool inside(uintptr_t p, size_t n, bool dst) {
  for (auto &b : g_bufs) if (b.dst == dst && p >= b.lo && p + n <= b.hi) return true;
  return false;
}

static void move(const char *s, char *d, size_t vs) {
  if (s && !inside((uintptr_t)s, vs, false)) { if (g_violations++ < 10) fprintf(stderr, "src OOB %p\n", s); return; }
  if (!inside((uintptr_t)d, vs, true)) { if (g_violations++ < 10) fprintf(stderr, "dst OOB %p\n", d); return; }
  if ((uintptr_t)d % vs || (s && (uintptr_t)s % vs)) { if (g_violations++ < 10) fprintf(stderr, "misaligned\n"); return; }
  if (s) memcpy(d, s, vs); else memset(d, 0, vs);
}

// span_copy_kernel, workgroup by workgroup and lane by lane: the tile decode
// (span_tile) and the short-row lane mapping (row_lane) are the kernel's
// own functions; the loops visit the rows and vectors the kernel's loops do.
static void emulate(const hexkv::SpanArgs &a, unsigned grid, size_t vs, int T) {
  using namespace hexkv;
  for (unsigned tile = 0; tile < grid; ++tile) {
    const int i = span_of_tile(a, (int)tile);
    const int t = (int)tile - a.first_tile[i];
    if (i < 0 || i >= a.n || t < 0 || t >= a.first_tile[i + 1] - a.first_tile[i]) {
      g_violations++;
      fprintf(stderr, "tile map\n");
      continue;
    }
    const SpanTile w = span_tile(a, (int)tile);
    const int64_t nv = w.bytes / (int64_t)vs;
    if (w.bytes % (int64_t)vs || nv < 1) { g_violations++; fprintf(stderr, "tile width %lld\n", (long long)w.bytes); }
    g_tiles++;
    for (int tid = 0; tid < T; ++tid) {
      if (nv >= T) {
        for (int r = w.r0; r < w.r1; ++r)
          for (int64_t v = tid; v < nv; v += T)
            move(w.src ? w.src + r * w.src_row + v * vs : nullptr, w.dst + r * w.dst_row + v * vs, vs);
      } else {
        const RowLane l = row_lane(T, (int)nv, tid);
        if (l.tr >= l.per) continue;
        for (int r = w.r0 + l.tr; r < w.r1; r += l.per)
          move(w.src ? w.src + r * w.src_row + l.tc * vs : nullptr, w.dst + r * w.dst_row + l.tc * vs, vs);
      }
    }
  }
}

// head_gather_kernel, lane by lane, through the kernel's own gather_lane and
// gather_load_row (clamped loads included: every load address is checked).
static void emulate_gather(const hexkv::GatherArgs &a, dim3 grid) {
  using namespace hexkv;
  if (a.wvec < 1 || a.wvec > kWideThreads || a.n < 1 || a.n > kGatherShards) { g_violations++; fprintf(stderr, "gather args\n"); return; }
  for (unsigned ly = 0; ly < grid.y; ++ly)
    for (unsigned bx = 0; bx < grid.x; ++bx) {
      g_tiles++;
      for (int tid = 0; tid < kWideThreads; ++tid) {
        const GatherLane g = gather_lane(a, bx, ly, tid);
        if (g.tr >= g.per) continue;
        if (g.tc < a.vec_start[g.shard] || g.tc >= a.vec_start[g.shard + 1]) { g_violations++; fprintf(stderr, "shard map\n"); continue; }
        for (int64_t r = g.r0 + g.tr; r < g.r1; r += (int64_t)g.per * kWideUnroll)
          for (int u = 0; u < kWideUnroll; ++u) {
            const int64_t lr = gather_load_row(g, r, u);
            if (!inside((uintptr_t)(g.src + lr * g.src_pitch), 16, false)) { if (g_violations++ < 10) fprintf(stderr, "gather load OOB\n"); }
            const int64_t rr = r + (int64_t)u * g.per;
            if (rr < g.r1) move(g.src + rr * g.src_pitch, g.dst + rr * g.dst_pitch, 16);
          }
      }
    }
}

extern "C" hipError_t hipLaunchKernel(const void *f, dim3 grid, dim3 block, void **args, size_t, hipStream_t) {
  using namespace hexkv;
  g_launches++;
  if (f == reinterpret_cast<const void *>(&head_gather_kernel)) {
    if (block.x != kWideThreads || grid.z != 1) { g_violations++; fprintf(stderr, "gather launch shape\n"); }
    emulate_gather(*static_cast<const GatherArgs *>(args[0]), grid);
    return hipSuccess;
  }
  if (grid.y != 1 || grid.z != 1) { g_violations++; fprintf(stderr, "launch shape\n"); }
  const SpanArgs &a = *static_cast<const SpanArgs *>(args[0]);
  size_t vs = 0;
  int T = 0;
#define K(VT, BYTES) \
  if (f == reinterpret_cast<const void *>(&span_copy_kernel<VT, kSpanThreads, kSpanUnroll>)) { vs = BYTES; T = kSpanThreads; } \
  else if (f == reinterpret_cast<const void *>(&span_copy_kernel<VT, kWideThreads, kWideUnroll>)) { vs = BYTES; T = kWideThreads; }
  K(u32x4, 16) else K(unsigned int, 4) else K(unsigned short, 2) else K(unsigned char, 1)
  else { g_violations++; fprintf(stderr, "unknown kernel\n"); return hipSuccess; }
#undef K
  if ((int)block.x != T) { g_violations++; fprintf(stderr, "block size\n"); }
  emulate(a, grid.x, vs, T);
  return hipSuccess;
}
extern "C" hipError_t hipGetLastError(void) { return hipSuccess; }
static thread_local dim3 t_grid, t_block;
static thread_local size_t t_shm;
static thread_local hipStream_t t_stream;
extern "C" hipError_t __hipPushCallConfiguration(dim3 g, dim3 b, size_t shm, hipStream_t s) {
  t_grid = g; t_block = b; t_shm = shm; t_stream = s; return hipSuccess;
}
extern "C" hipError_t __hipPopCallConfiguration(dim3 *g, dim3 *b, size_t *shm, hipStream_t *s) {
  *g = t_grid; *b = t_block; *shm = t_shm; *s = t_stream; return hipSuccess;
}
