// CPU emulation of the legacy-format kernels (span_copy_kernel in both launch
// shapes, head_gather_kernel) for bounds and correctness checks without a
// GPU.  The real host code of hexkv_blocks.hip is compiled in; its kernel
// launches are intercepted (hipLaunchKernel and the call-configuration hooks
// are defined here) and each workgroup and lane is replayed on the CPU with
// the kernel's own index arithmetic.  Every source and destination access
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

static void emulate(const hexkv::SpanArgs &a, unsigned grid, size_t vs, int T) {
  using namespace hexkv;
  for (unsigned tile = 0; tile < grid; ++tile) {
    int lo = 0, hi = a.n;
    while (hi - lo > 1) { int mid = (lo + hi) >> 1; if (a.first_tile[mid] <= (int)tile) lo = mid; else hi = mid; }
    const Span &s = a.span[lo];
    int t = tile - a.first_tile[lo];
    if (t < 0 || t >= a.first_tile[lo + 1] - a.first_tile[lo]) { g_violations++; fprintf(stderr, "tile map\n"); }
    const int ct = t % s.col_tiles; t /= s.col_tiles;
    const int rt = t % s.row_tiles; t /= s.row_tiles;
    const int64_t k = t % s.depth, m = t / s.depth;
    const int r0 = rt * s.tile_rows, r1 = std::min(s.height, r0 + s.tile_rows);
    const int64_t c0 = (int64_t)ct * s.tile_cols;
    const int64_t nv = (std::min(s.width, c0 + s.tile_cols) - c0) / (int64_t)vs;
    const char *src = s.src ? s.src + m * s.src_layer + k * s.src_slice + c0 : nullptr;
    char *dst = s.dst + m * s.dst_layer + k * s.dst_slice + c0;
    g_tiles++;
    for (int tid = 0; tid < T; ++tid) {
      if (nv >= T) {
        for (int r = r0; r < r1; ++r)
          for (int64_t i = tid; i < nv; i += T)
            move(src ? src + r * s.src_row + i * vs : nullptr, dst + r * s.dst_row + i * vs, vs);
      } else {
        const int per = T / (int)nv, tr = tid / (int)nv, tc = tid - tr * (int)nv;
        if (tr >= per) continue;
        for (int r = r0 + tr; r < r1; r += per)
          move(src ? src + r * s.src_row + tc * vs : nullptr, dst + r * s.dst_row + tc * vs, vs);
      }
    }
  }
}

// head_gather_kernel, lane by lane, with the kernel's own index arithmetic
// (clamped loads included: every load address is checked).
static void emulate_gather(const hexkv::GatherArgs &a, dim3 grid) {
  using namespace hexkv;
  if (a.wvec < 1 || a.wvec > kWideThreads || a.n < 1 || a.n > kGatherShards) { g_violations++; fprintf(stderr, "gather args\n"); return; }
  for (unsigned ly = 0; ly < grid.y; ++ly)
    for (unsigned bx = 0; bx < grid.x; ++bx) {
      g_tiles++;
      const int64_t l = ly, r0 = (int64_t)bx * a.rows_per_tile, r1 = std::min(a.rows, r0 + a.rows_per_tile);
      const int per = kWideThreads / a.wvec;
      for (int tid = 0; tid < kWideThreads; ++tid) {
        const int tr = tid / a.wvec, tc = tid - tr * a.wvec;
        if (tr >= per) continue;
        int j = 0;
        while (j + 1 < a.n && a.vec_start[j + 1] <= tc) ++j;
        if (tc < a.vec_start[j] || tc >= a.vec_start[j + 1]) { g_violations++; fprintf(stderr, "shard map\n"); continue; }
        const char *src = a.src[j] + l * a.src_layer[j] + (int64_t)(tc - a.vec_start[j]) * 16;
        const int64_t sp = a.src_pitch[j], dp = (int64_t)a.wvec * 16;
        char *dst = a.dst + l * a.dst_layer + (int64_t)tc * 16;
        for (int64_t r = r0 + tr; r < r1; r += (int64_t)per * kWideUnroll)
          for (int u = 0; u < kWideUnroll; ++u) {
            const int64_t rr = std::min(r + u * per, r1 - 1);
            if (!inside((uintptr_t)(src + rr * sp), 16, false)) { if (g_violations++ < 10) fprintf(stderr, "gather load OOB\n"); }
            if (r + u * per < r1) move(src + (r + u * per) * sp, dst + (r + u * per) * dp, 16);
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
