// Single-query GQA decode attention over the KV cache, with optional fused
// append of the new token's K/V (hexkv_attend in hexkv.h), and the same over
// the FasterTransformer cache layouts with rotary embedding (hexkv_ft_attend:
// the VALU kernel with a rotary prologue, K tiles staged through LDS to turn
// the FT chunk planes back into position-major rows, V read directly).
//
// Work decomposition (split-K, "flash-decoding"): a workgroup (4 waves) owns
// consecutive cache positions of one sequence for the G query heads that
// share one KV head, so every K/V byte is read by exactly one workgroup.  Two
// ways to hand out those pieces:
//   * grid = (partition, q-head group, query row), partitions of `part`
//     positions, row lengths read from seqlens on the device; ragged lengths
//     only change how many partitions a row has.
//   * a work list (decode rows, lengths known on the host): workgroup i runs
//     item i, planned by hexkv_attend_plan -- full chunks first, chunk index
//     by chunk index across every (row, head group) segment, then each
//     segment's shorter last chunk from the longest down -- so the grid has
//     no empty partitions and the launch ends on its smallest items.
//
// Two kernels stream a partition; both keep every load in flight without a
// barrier, address K/V as a uniform (SGPR) base plus a 32-bit lane offset,
// run an online softmax in the log2 domain whose running maximum moves
// lazily (only when a score exceeds it by more than kRescaleSlack, so the
// accumulator rescale is a rare wave-uniform branch), and accumulate
// o += p * V in fp32 registers:
//
// attend_valu_kernel (any dtype, any group): positions are dealt to "lane
//   groups" of LPP lanes; a lane group reads one position's K and V head
//   slice (LPP x 16 bytes each) per load slot, U slots per iteration.  Scores
//   are v_dot2_f32_{bf16,f16} (fp32: fma) of the lane's K slice with its
//   slice of the G query vectors, summed over the LPP lanes by DPP moves.
//
// attend_mfma_kernel (16-bit, head_dim >= 64): both products on the matrix
//   cores.  A wave takes tiles of 16 positions; S = K Q^T is
//   v_mfma_f32_16x16x32 with K in the A-operand layout (lane = position,
//   16-byte head slices) and the G query heads as the B operand, and the
//   resulting score layout is directly the A operand of O += P V
//   (v_mfma_f32_16x16x16, probabilities as hi + lo 16-bit pairs).  V passes
//   through a per-wave LDS tile and comes back transposed
//   (ds_read_b64_tr_b16) as the B operand.  The VALU only runs the softmax.
//
// With kv_new (fused append) the new row is the last position of the row: it
// is never read from the cache; one wave attends it from kv_new after the
// streaming loop, and the workgroup owning it writes it to the cache.
//
// A row with one partition writes its normalised output directly.  With
// several, each partition stores (unnormalised o, max, sum) to the workspace,
// and the partials are merged in one of two ways:
//   * XCD-local, in the attention kernel (work lists planned for the device's
//     XCDs, work_xcds > 0): every item of a split segment sits at one index
//     modulo the XCD count, and workgroups reach the XCDs round-robin by
//     index, so all of them run on one XCD and share its L2.  Each stores its
//     partial, waits for the stores (s_waitcnt vmcnt(0): they are in that
//     L2), and counts its arrival with an L2 atomic; the last one drops its
//     L1 lines (buffer_inv sc0), reads the partials from the L2, writes the
//     output and resets the counter.  No L2 writeback is needed.  (The
//     device-wide form -- an agent-scope release per workgroup, which writes
//     back the XCD's whole L2 -- measured 17x slower than the XCD-local one
//     in an in-bounds probe, and with partials spread over XCDs the plain
//     form reads stale data: the XCDs' L2s are not coherent.)
//   * otherwise `combine_kernel`, launched next on the same stream.
#include "hexkv_common.h"

#include <algorithm>
#include <atomic>
#include <mutex>
#include <utility>
#include <vector>

namespace hexkv {

constexpr int kAttThreads = 256;
constexpr int kAttWaves = kAttThreads / 64;
constexpr float kRescaleSlack = 8.f;  // log2 units
constexpr float kNoScore = -1e30f;    // finite "minus infinity" of the running max

struct AttendArgs {
  const void *q;
  int64_t q_bs, q_rs;
  const void *cache;
  int64_t c_bs, c_ps, c_kv;
  void *out;
  int64_t o_bs, o_rs;
  const void *kv_new;
  const int32_t *seqlens;
  int32_t bias;
  int32_t q_len;
  int32_t causal;
  int32_t q_heads;
  int32_t kv_heads;
  int32_t group;  // q heads per KV head
  int32_t part;   // positions per partition
  int32_t max_parts;
  int32_t max_seqlen;  // host bound; every row length is clamped to it
  int64_t capacity;
  float scale_log2;    // softmax_scale * log2(e), > 0
  float *ws_o;         // [rows][q_heads][max_parts][D]
  float *ws_ml;        // [rows][q_heads][max_parts][2]
  // Work-list mode (items != nullptr, decode rows only): workgroup i runs
  // items[i], which carries its row's length, so the kernel reads no
  // seqlens; seg_parts[row * n_groups + head group] is that segment's
  // partition count for the merge (partitions of one segment may differ in
  // size).  Grid mode otherwise: grid (partition, head group, row),
  // partitions of `part` positions, lengths from seqlens.
  const hexkv_work_item *items;
  const int32_t *seg_parts;
  int32_t n_groups;
  int32_t rows;  // query rows (batch * q_len)
  // XCD-local merge (work lists planned for n_xcd XCDs): arrival counters
  // [rows * n_groups], zero between calls; nullptr: combine_kernel merges.
  uint64_t *seg_count;
  int32_t n_xcd;
  // 1: the list holds XCD x's share at indices j * n_xcd + x and n_xcd
  // divides the device's XCD count; each workgroup then runs the item of its
  // own XCD within its group of n_xcd (see begin_work).
  int32_t xcd_remap;
  int32_t *lengths_out;  // work lists with kv_new: row b's new length, or nullptr
  unsigned int *status;  // HEXKV_STATUS_* word of this device, or nullptr
  // FasterTransformer cache layouts (hexkv_ft_attend only): K is
  // [batch][kv_heads][D / pack][capacity][pack] (one 16-byte chunk of D per
  // position), V is [batch][kv_heads][capacity][D]; strides in bytes.  The
  // new row's K comes from kv_new, its V from v_new, both [batch][kv_heads][D]
  // rows new_bs elements apart, and q and k are rotated first when rot_dim > 0.
  const void *k_ft, *v_ft;
  int64_t k_ft_batch, k_ft_head, k_ft_chunk;
  int64_t v_ft_batch, v_ft_head;
  const void *v_new;
  int64_t new_bs;
  int32_t rot_dim;      // leading dims of each head that rotate (0: none)
  int32_t rot_neox;     // 1: pairs (i, i + rot_dim / 2); 0: pairs (2i, 2i + 1)
  double rot_log2_base;  // log2 of the rotary base
};

// Number of keys query row (b, t) attends to; *pos_new = cache position of the
// fused-append row (or -1).
__device__ __forceinline__ int row_length(const AttendArgs &a, int b, int t, int *pos_new, bool *clamped) {
  int len = (a.seqlens ? a.seqlens[b] : 0) + a.bias;
  *pos_new = -1;
  if (a.kv_new) {
    *pos_new = len;
    len += 1;
  }
  if (a.causal) len = len - a.q_len + t + 1;
  // Lengths come from device memory: clamp to the host bound that sized the
  // grid and the workspace (max_seqlen <= capacity is checked on the host),
  // so no row can reach past either, and report it.
  *clamped = len > a.max_seqlen;
  if (len > a.max_seqlen) len = a.max_seqlen;
  return len;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// What one workgroup does: query row (b, t), head group qh0.., KV head hk,
// positions [p0, p0 + n) of which the first n_cache come from the cache and,
// when has_new, the last one (pos_new) from kv_new.
struct Work {
  int row, b, t, len, part, p0, n, n_cache, nparts, qh0, hk, pos_new;
  bool has_new, writer, clamped;
};

// Fills `w`; returns false when the workgroup has nothing to do (after
// writing the defined zero output of an empty row).
template <typename T, int D, int G>
__device__ __forceinline__ bool begin_work(const AttendArgs &a, Work &w) {
  int hg;
  w.clamped = false;
  if (a.items) {
    // The dispatcher hands workgroup b to XCD (b + r) mod 8, with a rotation
    // r that depends on the hardware queue.  Run XCD x's share on XCD x
    // whatever r is: the workgroup takes the item of its own XCD within its
    // group of n_xcd consecutive workgroups (round-robin dispatch gives the
    // n_xcd of a group distinct XCDs, so each item runs once), the same items
    // in the same order per XCD.  Measured on MI355X at Llama-3-8B: a share's
    // reads concentrate on a few KV heads of every cache row, and with r = 7
    // the call took 159 us against 150-152 at r = 0 and r = 6.
    unsigned idx = blockIdx.x;
    if (a.xcd_remap) idx = idx - idx % a.n_xcd + static_cast<unsigned>(xcd_id()) % a.n_xcd;
    // The rotation is shared by the whole launch, so workgroup 0 alone
    // reports it.  (One device-scope atomic per workgroup, as every split
    // item once did at its merge, cost ~1 us per call at the Llama-2-70B
    // TP-8 share whenever the rotation was not 0.)
    if (a.seg_count && a.n_xcd > 0 && blockIdx.x == 0 && threadIdx.x == 0 &&
        static_cast<unsigned>(xcd_id()) % a.n_xcd != 0)
      raise_status(a.status, HEXKV_STATUS_DISPATCH);
    const hexkv_work_item it = a.items[idx];
    // Items come from device memory: one naming a row, head group, partition
    // or positions outside this call's geometry does nothing; one planned
    // for head groups of another size (another kernel) does nothing either,
    // and says so.
    if (!work_item_fits(it, a.rows, a.n_groups, a.max_parts, a.max_seqlen)) return false;
    if (it.heads != 0 && it.heads != G) {
      if (threadIdx.x == 0) raise_status(a.status, HEXKV_STATUS_LIST);
      return false;
    }
    // The item holding a row's last position of head group 0 records the
    // row's new length (work lists read no seqlens, so this may alias them).
    if (a.lengths_out && threadIdx.x == 0 && it.head_group == 0 && it.len > 0 && it.count == it.len - it.first)
      a.lengths_out[it.row] = it.len;
    w.row = w.b = it.row;
    w.t = 0;
    hg = it.head_group;
    w.part = it.part;
    w.nparts = it.parts;
    w.p0 = it.first;
    w.n = it.count;
    w.len = it.len;
    w.pos_new = a.kv_new ? w.len - 1 : -1;
  } else {
    w.row = blockIdx.z;
    w.b = w.row / a.q_len;
    w.t = w.row - w.b * a.q_len;
    w.len = row_length(a, w.b, w.t, &w.pos_new, &w.clamped);
    hg = blockIdx.y;
    w.part = blockIdx.x;
    w.p0 = w.part * a.part;
  }
  w.qh0 = hg * G;
  if (w.len <= 0) {
    if (w.part == 0) {
      T *out_row = static_cast<T *>(a.out) + w.b * a.o_bs + w.t * a.o_rs + w.qh0 * D;
      for (int i = threadIdx.x; i < G * D; i += kAttThreads) out_row[i] = Elem<T>::from_float(0.f);
    }
    return false;
  }
  if (!a.items) {
    if (w.p0 >= w.len) return false;
    w.n = min(a.part, w.len - w.p0);
    w.nparts = (w.len + a.part - 1) / a.part;
  } else if (w.n <= 0) {
    return false;
  }
  w.hk = w.qh0 / a.group;
  // The new row, when attended at all, is the row's last position.
  w.has_new = a.kv_new != nullptr && w.pos_new == w.p0 + w.n - 1;
  w.n_cache = w.n - (w.has_new ? 1 : 0);
  // Head groups sharing a KV head (G < group) hold the same new row; only
  // the first writes it.
  w.writer = w.has_new && (w.qh0 % a.group) == 0;
  return true;
}

// Largest partition count a single-launch merge takes (the host sends calls
// with more to combine_kernel): one wave holds a head's (max, sum) pairs.
constexpr int kMergeMaxParts = 64;  // also keeps each XCD's 8-bit arrival count from overflowing

// Four consecutive outputs at p, one vector store when p is aligned for it
// (output rows may have any element stride).
template <typename T>
__device__ __forceinline__ void store4(T *p, f32x4 v) {
  if ((reinterpret_cast<uintptr_t>(p) & (4 * sizeof(T) - 1)) == 0) {
    typedef T t4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<t4 *>(p) = t4{Elem<T>::from_float(v[0]), Elem<T>::from_float(v[1]),
                                    Elem<T>::from_float(v[2]), Elem<T>::from_float(v[3])};
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) p[k] = Elem<T>::from_float(v[k]);
  }
}

// The XCD-local merge of a split segment (row, head group qh0 / G), after
// this workgroup stored its partial: count the arrival; the last of the
// segment's w.nparts items reads every partial from the XCD's L2 and writes
// the normalised output, parts in index order (the result does not depend
// on which item arrives last).
//
// Each thread owns 4 consecutive outputs of the G x D block per pass (1024
// outputs a pass), so the D / 4 lanes of a head sit in one wave.  Every lane
// loads its 4 outputs of each part (one 16-byte load per part, parts past
// w.nparts not issued) and lane k of a head the (max, sum) pairs of parts k,
// k + D / 4, ...; the head's lanes then reduce the pairs into the part
// weights w_p = 2^(m_p - max m) / sum_q 2^(m_q - max m) l_q, exchange them
// through LDS (s_w, G x kMergeMaxParts floats) within the wave, and
// accumulate.  One L2 round trip per pass, no barrier after the arrival,
// and one load instruction per wave and part.
template <typename T, int D, int G>
__device__ __forceinline__ void merge_split(const AttendArgs &a, const Work &w, float (*s_w)[kMergeMaxParts]) {
  constexpr int OUT = G * D;
  constexpr int LPH = D / 4;  // lanes per head
  constexpr int R = (kMergeMaxParts + LPH - 1) / LPH;  // (max, sum) pairs per lane
  constexpr int kDepth = 16;
  static_assert(D % 16 == 0 && LPH <= 64, "a head's outputs lie in one wave");
  static_assert(kMergeMaxParts % kDepth == 0, "weight blocks stay inside s_w");
  __shared__ int s_last;
  // Every wave's partial stores have reached the L2 before the arrival counts.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  // One 64-bit counter per segment, an 8-bit arrival count per XCD: the last
  // arrival sees whether every part ran on its own XCD (the L2 it reads).
  uint64_t *count = a.seg_count + static_cast<int64_t>(w.row) * a.n_groups + w.qh0 / G;
  if (threadIdx.x == 0) {
    const int x = xcd_id() & 7;
    const uint64_t mine = UINT64_C(1) << (8 * x);
    const uint64_t old = __hip_atomic_fetch_add(count, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int arrived = static_cast<int>((old * UINT64_C(0x0101010101010101)) >> 56);  // byte sum (< 256)
    s_last = arrived == w.nparts - 1;
    if (s_last && old + mine != static_cast<uint64_t>(w.nparts) << (8 * x))
      raise_status(a.status, HEXKV_STATUS_PLACEMENT);
    if (s_last) __hip_atomic_store(count, static_cast<uint64_t>(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  // Drop this CU's L1 lines so the partials come from the L2.
  asm volatile("buffer_inv sc0" ::: "memory");
  const int n = w.nparts;
  for (int i0 = 4 * static_cast<int>(threadIdx.x); i0 < OUT; i0 += 4 * kAttThreads) {
    const int g = i0 / D, d = i0 - g * D, k = d / 4;
    const int64_t slot = (static_cast<int64_t>(w.row) * a.q_heads + w.qh0 + g) * a.max_parts;
    const float *o = a.ws_o + slot * D + d;
    const float2 *ml = reinterpret_cast<const float2 *>(a.ws_ml + slot * 2);
    // The partials first: the pairs' loads then wait for nothing else.
    f32x4 ov[kDepth];
#pragma unroll
    for (int u = 0; u < kDepth; ++u)
      if (u < n) ov[u] = *reinterpret_cast<const f32x4 *>(o + static_cast<int64_t>(u) * D);
    float2 mlv[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int p = k + j * LPH;
      mlv[j] = p < n ? ml[p] : float2{kNoScore, 0.f};
    }
    float mx = kNoScore;
#pragma unroll
    for (int j = 0; j < R; ++j) mx = fmaxf(mx, mlv[j].x);
    mx = group_max<LPH>(mx);
    float e[R], den = 0.f;
#pragma unroll
    for (int j = 0; j < R; ++j) {
      e[j] = fast_exp2(mlv[j].x - mx);
      den = fmaf(e[j], mlv[j].y, den);
    }
    const float inv = 1.f / group_sum<LPH>(den);
#pragma unroll
    for (int j = 0; j < R; ++j)
      if (k + j * LPH < n) s_w[g][k + j * LPH] = e[j] * inv;
    __builtin_amdgcn_wave_barrier();  // the weights come from lanes of this wave
    f32x4 acc{};
    for (int p0 = 0; p0 < n; p0 += kDepth) {
      if (p0 > 0) {
#pragma unroll
        for (int u = 0; u < kDepth; ++u)
          if (p0 + u < n) ov[u] = *reinterpret_cast<const f32x4 *>(o + static_cast<int64_t>(p0 + u) * D);
      }
      f32x4 wq[kDepth / 4];  // weights of parts p0.. (p0 + kDepth <= kMergeMaxParts)
#pragma unroll
      for (int q = 0; q < kDepth / 4; ++q) wq[q] = *reinterpret_cast<const f32x4 *>(&s_w[g][p0 + 4 * q]);
#pragma unroll
      for (int u = 0; u < kDepth; ++u)
        if (p0 + u < n) acc += wq[u / 4][u % 4] * ov[u];
    }
    store4(static_cast<T *>(a.out) + w.b * a.o_bs + w.t * a.o_rs + w.qh0 * D + i0, acc);
  }
}

// Merges the NS slots' (max, sum, o) held in LDS (the 4 waves' of the
// attention kernels, the position slots' of the row-block kernel) into this
// partition's result: the normalised output for a single-partition row,
// else a workspace partial (merged here, XCD-locally, when the call has
// arrival counters).  Each thread takes 4 consecutive outputs of a head per
// pass (D is a multiple of 16): one 16-byte LDS read per slot and one set of
// slot weights per pass.  With W_IN_ACC the merge's weights reuse s_acc
// (read completely before the merge's first barrier).
template <typename T, int D, int G, int NS = kAttWaves, bool W_IN_ACC = false>
__device__ __forceinline__ void finish_work(const AttendArgs &a, const Work &w,
                                            const float (*s_acc)[G][D], const float (*s_m)[G],
                                            const float (*s_l)[G]) {
  T *out_row = static_cast<T *>(a.out) + w.b * a.o_bs + w.t * a.o_rs + w.qh0 * D;
  const int64_t slot0 = (static_cast<int64_t>(w.row) * a.q_heads + w.qh0) * a.max_parts;
  for (int i = 4 * threadIdx.x; i < G * D; i += 4 * kAttThreads) {
    const int g = i / D, d = i - g * D;
    float mx = s_m[0][g];
#pragma unroll
    for (int ww = 1; ww < NS; ++ww) mx = fmaxf(mx, s_m[ww][g]);
    f32x4 o{};
    float sum = 0.f;
#pragma unroll
    for (int ww = 0; ww < NS; ++ww) {
      const float c = fast_exp2(s_m[ww][g] - mx);
      o += c * *reinterpret_cast<const f32x4 *>(&s_acc[ww][g][d]);
      sum = fmaf(c, s_l[ww][g], sum);
    }
    if (w.nparts == 1) {
      store4(out_row + i, o * (1.f / sum));
    } else {
      const int64_t slot = slot0 + static_cast<int64_t>(g) * a.max_parts + w.part;
      *reinterpret_cast<f32x4 *>(a.ws_o + slot * D + d) = o;
      if (d == 0) *reinterpret_cast<float2 *>(a.ws_ml + slot * 2) = float2{mx, sum};
    }
  }
  if (w.clamped && threadIdx.x == 0) raise_status(a.status, HEXKV_STATUS_LENGTH_CLAMPED);
  if (w.nparts > 1 && a.seg_count) {
    if constexpr (W_IN_ACC) {
      static_assert(NS * D >= kMergeMaxParts, "the merge's weights fit in s_acc");
      merge_split<T, D, G>(a, w, reinterpret_cast<float (*)[kMergeMaxParts]>(const_cast<float *>(&s_acc[0][0][0])));
    } else if constexpr (G * D <= 4 * kAttThreads) {  // the host merges larger blocks with combine_kernel
      __shared__ __attribute__((aligned(16))) float s_w[G][kMergeMaxParts];
      merge_split<T, D, G>(a, w, s_w);
    }
  }
}

__device__ __forceinline__ u32x4 load16(const char *base, uint32_t off) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base + off));
}

// Lane geometry of one (dtype, head_dim) for reading a head row: each lane
// owns EPL consecutive elements (NV 16-byte vectors), LPP lanes cover it.
template <typename T, int D>
struct Lanes {
  static constexpr int VEC = 16 / static_cast<int>(sizeof(T));
  static constexpr int NV = D / VEC > 16 ? D / (VEC * 16) : 1;
  static constexpr int EPL = VEC * NV;
  static constexpr int LPP = D / EPL;
  static constexpr int GPW = 64 / LPP;
  static constexpr int NG = GPW * kAttWaves;
  static_assert(LPP >= 1 && LPP <= 16 && EPL * LPP == D, "head_dim does not map onto a wave");
};

// Running-softmax state update for one tile of scores: moves the running
// maximum of head g to the tile maximum `mt[g]` (scaled) when it exceeds the
// old one by more than kRescaleSlack, rescaling l and the accumulators.
template <int G, int EPL>
__device__ __forceinline__ void lazy_rescale(const float (&mt)[G], float (&m)[G], float (&l)[G],
                                             float (&acc)[G][EPL]) {
  bool grow = false;
  float mnew[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const bool up = mt[g] > m[g] + kRescaleSlack;
    mnew[g] = up ? mt[g] : m[g];
    grow |= up;
  }
  if (__any(grow)) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float c = fast_exp2(m[g] - mnew[g]);
      m[g] = mnew[g];
      l[g] *= c;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[g][e] *= c;
    }
  }
}

// 16 bytes of T rounded from VEC floats.
template <typename T>
__device__ __forceinline__ u32x4 pack16(const float *f) {
  constexpr int VEC = 16 / static_cast<int>(sizeof(T));
  T t[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) t[i] = Elem<T>::from_float(f[i]);
  u32x4 r;
  __builtin_memcpy(&r, t, 16);
  return r;
}

// FT layout prologue: the workgroup's G query heads (sq, G x D) and, for the
// workgroup that attends the new row, its K (skn, D) as fp32 in LDS, rotated
// in place at the new row's position when rot_dim > 0: pair (x0, x1) of
// dimension pair j turns by pos * base^(-2j / rot_dim) radians.  The angle
// and its sine and cosine are evaluated in fp64 (an fp32 angle is off by
// ~pos * 2^-24 radians, 6e-5 at position 1000); the turn itself is fp32.
// The caller rounds both back to T when it packs them, as the reference
// kernel does.
template <typename T, int D, int G>
__device__ __forceinline__ void ft_prologue(const AttendArgs &a, const Work &w, float *sq, float *skn) {
  const T *q = static_cast<const T *>(a.q) + w.b * a.q_bs + w.qh0 * D;
  for (int i = threadIdx.x; i < G * D; i += kAttThreads) sq[i] = static_cast<float>(q[i]);
  if (w.has_new) {
    const T *k = static_cast<const T *>(a.kv_new) + w.b * a.new_bs + static_cast<int64_t>(w.hk) * D;
    for (int i = threadIdx.x; i < D; i += kAttThreads) skn[i] = static_cast<float>(k[i]);
  }
  __syncthreads();
  const int half = a.rot_dim / 2;
  if (half > 0) {
    const int pos = w.pos_new;
    const int vecs = w.has_new ? G + 1 : G;
    for (int i = threadIdx.x; i < vecs * half; i += kAttThreads) {
      const int g = i / half, j = i - g * half;
      float *x = g < G ? sq + g * D : skn;
      const int i0 = a.rot_neox ? j : 2 * j, i1 = a.rot_neox ? j + half : 2 * j + 1;
      const double theta = static_cast<double>(pos) * exp2(-static_cast<double>(2 * j) / a.rot_dim * a.rot_log2_base);
      double sd, cd;
      sincos(theta, &sd, &cd);
      const float sn = static_cast<float>(sd), cs = static_cast<float>(cd);
      const float x0 = x[i0], x1 = x[i1];
      x[i0] = x0 * cs - x1 * sn;
      x[i1] = x0 * sn + x1 * cs;
    }
  }
  __syncthreads();
}

// ------------------------------------------------------------- VALU path ---

template <typename T, int D, int G, int U, bool PF = true, bool FT = false>
__global__ __launch_bounds__(kAttThreads) void attend_valu_kernel(const AttendArgs a) {
  using E = Elem<T>;
  using L = Lanes<T, D>;
  constexpr int VEC = L::VEC, NV = L::NV, EPL = L::EPL, LPP = L::LPP, GPW = L::GPW, NG = L::NG;
  constexpr int STEP = NG * U;  // positions per workgroup iteration
  __shared__ __attribute__((aligned(16))) float s_acc[kAttWaves][G][D];
  __shared__ float s_m[kAttWaves][G], s_l[kAttWaves][G];
  __shared__ float s_kn[FT ? D : 1];
  // FT: two staged K tiles, STEP positions of D / VEC 16-byte chunks each,
  // one padded row per position.
  constexpr int KT_PITCH = D / VEC * 16 + 16;
  __shared__ __attribute__((aligned(16))) char s_kt[FT ? 2 * STEP * KT_PITCH : 16];
  Work w;
  if (!begin_work<T, D, G>(a, w)) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane % LPP, gid = wave * GPW + lane / LPP;
  const float scale = a.scale_log2;

  u32x4 qv[G][NV];
  if constexpr (FT) {
    ft_prologue<T, D, G>(a, w, &s_acc[0][0][0], s_kn);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int v = 0; v < NV; ++v) qv[g][v] = pack16<T>(&s_acc[0][g][sub * EPL + v * VEC]);
    __syncthreads();  // every wave holds its query before s_acc is written again
  } else {
    const T *qrow = static_cast<const T *>(a.q) + w.b * a.q_bs + w.t * a.q_rs + w.qh0 * D + sub * EPL;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int v = 0; v < NV; ++v) qv[g][v] = *reinterpret_cast<const u32x4 *>(qrow + g * D + v * VEC);
  }

  // Uniform bases of this sequence's K and V head slices; lane offsets are
  // 32-bit (the host checks capacity * position stride fits).  In the
  // standard layout K and V of a position share one offset; in the FT layout
  // a K position is one 16-byte chunk (the lane's chunks kchunk apart) and a
  // V position one head row.
  const char *kseq, *vseq;
  uint32_t row_bytes, vrow_bytes, kchunk, klane;
  const uint32_t lane_off = static_cast<uint32_t>(sub * EPL * sizeof(T));
  if constexpr (FT) {
    kseq = static_cast<const char *>(a.k_ft) + w.b * a.k_ft_batch + w.hk * a.k_ft_head;
    vseq = static_cast<const char *>(a.v_ft) + w.b * a.v_ft_batch + w.hk * a.v_ft_head;
    row_bytes = 16;
    vrow_bytes = static_cast<uint32_t>(D * sizeof(T));
    kchunk = static_cast<uint32_t>(a.k_ft_chunk);
    klane = static_cast<uint32_t>(sub * NV) * kchunk;
  } else {
    kseq = static_cast<const char *>(a.cache) +
           (w.b * a.c_bs + static_cast<int64_t>(w.hk) * D) * static_cast<int64_t>(sizeof(T));
    vseq = kseq + a.c_kv * static_cast<int64_t>(sizeof(T));
    row_bytes = vrow_bytes = static_cast<uint32_t>(a.c_ps * sizeof(T));
    kchunk = 16;
    klane = lane_off;
  }
  const uint32_t lane_base = static_cast<uint32_t>(w.p0 + gid) * row_bytes + klane;
  const uint32_t vlane_base = static_cast<uint32_t>(w.p0 + gid) * vrow_bytes + lane_off;

  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNoScore;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
  }

  // One iteration covers U slots of one position per lane group.  `fetch`
  // issues its loads; TAIL clamps the positions past n_cache to the last
  // cached one (finite data) and `consume` masks their scores.
  using Slots = u32x4[U][NV];
  auto fetch = [&](int i0, Slots &kr, Slots &vr, auto tail) {
    constexpr bool TAIL = decltype(tail)::value;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      uint32_t off, voff;
      if constexpr (TAIL) {
        const int p = min(i0 + u * NG + gid, w.n_cache - 1);
        off = static_cast<uint32_t>(w.p0 + p) * row_bytes + klane;
        if constexpr (FT) voff = static_cast<uint32_t>(w.p0 + p) * vrow_bytes + lane_off;
      } else {
        off = lane_base + static_cast<uint32_t>(i0 + u * NG) * row_bytes;
        if constexpr (FT) voff = vlane_base + static_cast<uint32_t>(i0 + u * NG) * vrow_bytes;
      }
      if constexpr (!FT) voff = off;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        kr[u][v] = load16(kseq, off + v * kchunk);
        vr[u][v] = load16(vseq, voff + v * 16);
      }
    }
  };
  auto consume = [&](int i0, const Slots &kr, const Slots &vr, auto tail) {
    constexpr bool TAIL = decltype(tail)::value;
    float sc[U][G];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = E::dot(qv[g][0], kr[u][0], 0.f);
#pragma unroll
        for (int v = 1; v < NV; ++v) d = E::dot(qv[g][v], kr[u][v], d);
        sc[u][g] = group_sum<LPP>(d);
      }
    if constexpr (TAIL) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool valid = i0 + u * NG + gid < w.n_cache;
#pragma unroll
        for (int g = 0; g < G; ++g) sc[u][g] = valid ? sc[u][g] : -INFINITY;
      }
    }
    float mt[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float x = sc[0][g];
#pragma unroll
      for (int u = 1; u < U; ++u) x = fmaxf(x, sc[u][g]);
      mt[g] = x * scale;
    }
    lazy_rescale<G, EPL>(mt, m, l, acc);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float vf[EPL];
#pragma unroll
      for (int v = 0; v < NV; ++v) E::to_float(vr[u][v], vf + v * VEC);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pr = fast_exp2(fmaf(sc[u][g], scale, -m[g]));
        l[g] += pr;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(pr, vf[e], acc[g][e]);
      }
    }
  };

  // Full iterations, software-pipelined PF deep: the loads of iteration
  // i + 1 are in flight while iteration i computes.  Then the tail.
  const int n_full = w.n_cache / STEP * STEP;
  int i0 = 0;
  if constexpr (FT) {
    // K of the FT layout is staged through LDS: the workgroup loads a tile of
    // STEP positions plane by plane (consecutive threads, consecutive
    // positions: STEP x 16-byte runs), stores it position-major, and every
    // lane group then reads its position's chunks as in the standard layout.
    // Double-buffered: tile t + 1's loads are in flight while tile t
    // computes, one barrier per tile.  V is read directly, as before.
    constexpr int CH = D / VEC, CPT = STEP * CH / kAttThreads;
    static_assert(STEP * CH % kAttThreads == 0, "K tile does not split over the workgroup");
    auto kt_fetch = [&](int t0, u32x4 (&kt)[CPT]) {
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const int q = tid + c * kAttThreads, r = q % STEP, j = q / STEP;
        const int p = min(t0 + r, w.n_cache - 1);
        kt[c] = load16(kseq, static_cast<uint32_t>(w.p0 + p) * 16u + static_cast<uint32_t>(j) * kchunk);
      }
    };
    auto kt_store = [&](int buf, const u32x4 (&kt)[CPT]) {
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const int q = tid + c * kAttThreads, r = q % STEP, j = q / STEP;
        *reinterpret_cast<u32x4 *>(s_kt + (buf * STEP + r) * KT_PITCH + j * 16) = kt[c];
      }
    };
    auto v_fetch = [&](int t0, Slots &vr) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int p = min(t0 + u * NG + gid, w.n_cache - 1);
        const uint32_t voff = static_cast<uint32_t>(w.p0 + p) * vrow_bytes + lane_off;
#pragma unroll
        for (int v = 0; v < NV; ++v) vr[u][v] = load16(vseq, voff + v * 16);
      }
    };
    auto k_read = [&](int buf, Slots &kr) {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int v = 0; v < NV; ++v)
          kr[u][v] = *reinterpret_cast<const u32x4 *>(s_kt + (buf * STEP + u * NG + gid) * KT_PITCH +
                                                      (sub * NV + v) * 16);
    };
    const int nfull = w.n_cache / STEP, ntiles = (w.n_cache + STEP - 1) / STEP;
    if (ntiles > 0) {
      u32x4 kt[CPT];
      Slots vr;
      kt_fetch(0, kt);
      v_fetch(0, vr);
      kt_store(0, kt);
      __syncthreads();
      for (int t = 0; t < nfull; ++t) {
        const int t0 = t * STEP;
        const bool more = t + 1 < ntiles;
        Slots vnext;
        if (more) {
          kt_fetch(t0 + STEP, kt);
          v_fetch(t0 + STEP, vnext);
        }
        Slots kr;
        k_read(t & 1, kr);
        consume(t0, kr, vr, std::false_type{});
        if (more) {
          kt_store((t + 1) & 1, kt);
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int v = 0; v < NV; ++v) vr[u][v] = vnext[u][v];
        }
        __syncthreads();
      }
      if (nfull < ntiles) {  // the partial last tile, loaded and staged above
        Slots kr;
        k_read(nfull & 1, kr);
        consume(nfull * STEP, kr, vr, std::true_type{});
      }
    }
    i0 = w.n_cache;
  } else if constexpr (PF) {
    if (n_full > 0) {
      Slots ka, va;
      fetch(0, ka, va, std::false_type{});
      for (; i0 + STEP < n_full; i0 += STEP) {
        Slots kb, vb;
        fetch(i0 + STEP, kb, vb, std::false_type{});
        consume(i0, ka, va, std::false_type{});
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int v = 0; v < NV; ++v) {
            ka[u][v] = kb[u][v];
            va[u][v] = vb[u][v];
          }
      }
      consume(i0, ka, va, std::false_type{});
      i0 += STEP;
    }
  } else {
    for (; i0 < n_full; i0 += STEP) {
      Slots kr, vr;
      fetch(i0, kr, vr, std::false_type{});
      consume(i0, kr, vr, std::false_type{});
    }
  }
  if (i0 < w.n_cache) {
    Slots kr, vr;
    fetch(i0, kr, vr, std::true_type{});
    consume(i0, kr, vr, std::true_type{});
  }

  if (w.has_new) {
    // The new row: attended by lane group 0 from kv_new, written to the cache
    // by that lane group of the writer workgroup.
    u32x4 kn[NV], vn[NV];
    if constexpr (FT) {
      const char *vnew = static_cast<const char *>(a.v_new) +
                         (w.b * a.new_bs + static_cast<int64_t>(w.hk) * D) * static_cast<int64_t>(sizeof(T));
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        kn[v] = pack16<T>(s_kn + sub * EPL + v * VEC);
        vn[v] = *reinterpret_cast<const u32x4 *>(vnew + lane_off + v * 16);
      }
    } else {
      const char *knew = static_cast<const char *>(a.kv_new) +
                         ((static_cast<int64_t>(w.b) * 2 * a.kv_heads + w.hk) * D) * static_cast<int64_t>(sizeof(T));
      const char *vnew = knew + static_cast<int64_t>(a.kv_heads) * D * sizeof(T);
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        kn[v] = *reinterpret_cast<const u32x4 *>(knew + lane_off + v * 16);
        vn[v] = *reinterpret_cast<const u32x4 *>(vnew + lane_off + v * 16);
      }
    }
    float sc[G], mt[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float d = E::dot(qv[g][0], kn[0], 0.f);
#pragma unroll
      for (int v = 1; v < NV; ++v) d = E::dot(qv[g][v], kn[v], d);
      sc[g] = gid == 0 ? group_sum<LPP>(d) : -INFINITY;
      mt[g] = sc[g] * scale;
    }
    lazy_rescale<G, EPL>(mt, m, l, acc);
    float vf[EPL];
#pragma unroll
    for (int v = 0; v < NV; ++v) E::to_float(vn[v], vf + v * VEC);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float pr = fast_exp2(fmaf(sc[g], scale, -m[g]));
      l[g] += pr;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(pr, vf[e], acc[g][e]);
    }
    if (w.writer && gid == 0) {
      const uint32_t off = static_cast<uint32_t>(w.pos_new) * row_bytes + klane;
      const uint32_t voff = static_cast<uint32_t>(w.pos_new) * vrow_bytes + lane_off;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        *reinterpret_cast<u32x4 *>(const_cast<char *>(kseq) + off + v * kchunk) = kn[v];
        *reinterpret_cast<u32x4 *>(const_cast<char *>(vseq) + voff + v * 16) = vn[v];
      }
    }
  }

  // Merge the GPW lane groups of this wave (lanes with equal `sub`).
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float mw = max_from<LPP>(m[g]);
    const float c = fast_exp2(m[g] - mw);
    m[g] = mw;
    l[g] = sum_from<LPP>(l[g] * c);
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = sum_from<LPP>(acc[g][e] * c);
  }
  if (lane < LPP) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < EPL; ++e) s_acc[wave][g][sub * EPL + e] = acc[g][e];
    if (lane == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();
  finish_work<T, D, G>(a, w, s_acc, s_m, s_l);
}

// ------------------------------------------------------ row-block path ---
//
// attend_rows_kernel: a work item covers HB consecutive KV heads of one
// row's positions [p0, p0 + n), with the GQ query heads of each, so the
// workgroup reads whole cache rows (HB = the row's KV head count) instead of
// one head's 2 D-element slices out of every row.  Measured on MI355X in a
// read-only probe over 4 KB rows of 8 heads: one head per workgroup and XCD
// 6.6-6.7 TB/s with the odd heads' slices served last (the XCDs reading
// them finished ~55 us after the others in a ~320 us stream; each head
// alone streams at the same rate as any other), whole rows per workgroup
// 7.1 TB/s with the XCDs finishing within ~18 us.
//
// Lane group gid (LPP lanes, one D-element head slice) takes KV head
// hh = gid % HB at position slot ps = gid / HB: NG / HB positions per load
// slot, U slots per iteration.  Each lane keeps the running-softmax state of
// its head's GQ query heads; the slots of a head are merged through LDS at
// the end (finish_work over NG / HB slots), and a split segment
// (row, head block) merges XCD-locally like the other kernels'.
template <typename T, int D, int GQ, int HB, int U>
__global__ __launch_bounds__(kAttThreads) void attend_rows_kernel(const AttendArgs a) {
  using E = Elem<T>;
  using L = Lanes<T, D>;
  constexpr int VEC = L::VEC, NV = L::NV, EPL = L::EPL, LPP = L::LPP, GPW = L::GPW, NG = L::NG;
  constexpr int PS = NG / HB, QH = HB * GQ, STEP = PS * U;
  static_assert(NG % HB == 0, "the head block divides the lane groups");
  __shared__ __attribute__((aligned(16))) float s_acc[PS][QH][D];
  __shared__ float s_m[PS][QH], s_l[PS][QH];
  Work w;
  if (!begin_work<T, D, QH>(a, w)) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane % LPP, gid = wave * GPW + lane / LPP;
  const int hh = gid % HB, ps = gid / HB;
  const float scale = a.scale_log2;

  u32x4 qv[GQ][NV];
  {
    const T *qrow = static_cast<const T *>(a.q) + w.b * a.q_bs + w.t * a.q_rs + (w.qh0 + hh * GQ) * D + sub * EPL;
#pragma unroll
    for (int g = 0; g < GQ; ++g)
#pragma unroll
      for (int v = 0; v < NV; ++v) qv[g][v] = *reinterpret_cast<const u32x4 *>(qrow + g * D + v * VEC);
  }

  // Uniform bases at the block's first KV head; each lane's 32-bit offset
  // adds its head's slice within the row.
  const char *kseq = static_cast<const char *>(a.cache) +
                     (w.b * a.c_bs + static_cast<int64_t>(w.hk) * D) * static_cast<int64_t>(sizeof(T));
  const char *vseq = kseq + a.c_kv * static_cast<int64_t>(sizeof(T));
  const uint32_t row_bytes = static_cast<uint32_t>(a.c_ps * sizeof(T));
  const uint32_t lane_off = static_cast<uint32_t>((hh * D + sub * EPL) * sizeof(T));
  const uint32_t lane_base = static_cast<uint32_t>(w.p0 + ps) * row_bytes + lane_off;

  float m[GQ], l[GQ], acc[GQ][EPL];
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
    m[g] = kNoScore;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
  }

  // Slot u of the iteration at i0 holds position i0 + u * PS + ps; TAIL
  // clamps positions past n_cache to the last cached one (finite data) and
  // `consume` masks their scores.
  using Slots = u32x4[U][NV];
  auto fetch = [&](int i0, Slots &kr, Slots &vr, auto tail) {
    constexpr bool TAIL = decltype(tail)::value;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      uint32_t off;
      if constexpr (TAIL) {
        const int pp = min(i0 + u * PS + ps, w.n_cache - 1);
        off = static_cast<uint32_t>(w.p0 + pp) * row_bytes + lane_off;
      } else {
        off = lane_base + static_cast<uint32_t>(i0 + u * PS) * row_bytes;
      }
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        kr[u][v] = load16(kseq, off + v * 16);
        vr[u][v] = load16(vseq, off + v * 16);
      }
    }
  };
  auto consume = [&](int i0, const Slots &kr, const Slots &vr, auto tail) {
    constexpr bool TAIL = decltype(tail)::value;
    float sc[U][GQ];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int g = 0; g < GQ; ++g) {
        float d = E::dot(qv[g][0], kr[u][0], 0.f);
#pragma unroll
        for (int v = 1; v < NV; ++v) d = E::dot(qv[g][v], kr[u][v], d);
        sc[u][g] = group_sum<LPP>(d);
      }
    if constexpr (TAIL) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool valid = i0 + u * PS + ps < w.n_cache;
#pragma unroll
        for (int g = 0; g < GQ; ++g) sc[u][g] = valid ? sc[u][g] : -INFINITY;
      }
    }
    float mt[GQ];
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
      float x = sc[0][g];
#pragma unroll
      for (int u = 1; u < U; ++u) x = fmaxf(x, sc[u][g]);
      mt[g] = x * scale;
    }
    lazy_rescale<GQ, EPL>(mt, m, l, acc);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float vf[EPL];
#pragma unroll
      for (int v = 0; v < NV; ++v) E::to_float(vr[u][v], vf + v * VEC);
#pragma unroll
      for (int g = 0; g < GQ; ++g) {
        const float pr = fast_exp2(fmaf(sc[u][g], scale, -m[g]));
        l[g] += pr;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(pr, vf[e], acc[g][e]);
      }
    }
  };

  // Full iterations with the next one's loads in flight, then the tail.
  const int n_full = w.n_cache / STEP * STEP;
  int i0 = 0;
  if (n_full > 0) {
    Slots ka, va;
    fetch(0, ka, va, std::false_type{});
    for (; i0 + STEP < n_full; i0 += STEP) {
      Slots kb, vb;
      fetch(i0 + STEP, kb, vb, std::false_type{});
      consume(i0, ka, va, std::false_type{});
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          ka[u][v] = kb[u][v];
          va[u][v] = vb[u][v];
        }
    }
    consume(i0, ka, va, std::false_type{});
    i0 += STEP;
  }
  if (i0 < w.n_cache) {
    Slots kr, vr;
    fetch(i0, kr, vr, std::true_type{});
    consume(i0, kr, vr, std::true_type{});
  }

  if (w.has_new) {
    // The new row of every head of the block: attended by the lane groups of
    // slot 0 from kv_new, written to the cache by them (one head each).
    const char *knew = static_cast<const char *>(a.kv_new) +
                       ((static_cast<int64_t>(w.b) * 2 * a.kv_heads + w.hk + hh) * D + sub * EPL) *
                           static_cast<int64_t>(sizeof(T));
    const char *vnew = knew + static_cast<int64_t>(a.kv_heads) * D * sizeof(T);
    u32x4 kn[NV], vn[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      kn[v] = *reinterpret_cast<const u32x4 *>(knew + v * 16);
      vn[v] = *reinterpret_cast<const u32x4 *>(vnew + v * 16);
    }
    float sc[GQ], mt[GQ];
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
      float d = E::dot(qv[g][0], kn[0], 0.f);
#pragma unroll
      for (int v = 1; v < NV; ++v) d = E::dot(qv[g][v], kn[v], d);
      sc[g] = ps == 0 ? group_sum<LPP>(d) : -INFINITY;
      mt[g] = sc[g] * scale;
    }
    lazy_rescale<GQ, EPL>(mt, m, l, acc);
    float vf[EPL];
#pragma unroll
    for (int v = 0; v < NV; ++v) E::to_float(vn[v], vf + v * VEC);
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
      const float pr = fast_exp2(fmaf(sc[g], scale, -m[g]));
      l[g] += pr;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(pr, vf[e], acc[g][e]);
    }
    if (w.writer && ps == 0) {
      const uint32_t off = static_cast<uint32_t>(w.pos_new) * row_bytes + lane_off;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        *reinterpret_cast<u32x4 *>(const_cast<char *>(kseq) + off + v * 16) = kn[v];
        *reinterpret_cast<u32x4 *>(const_cast<char *>(vseq) + off + v * 16) = vn[v];
      }
    }
  }

#pragma unroll
  for (int g = 0; g < GQ; ++g) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) s_acc[ps][hh * GQ + g][sub * EPL + e] = acc[g][e];
    if (sub == 0) {
      s_m[ps][hh * GQ + g] = m[g];
      s_l[ps][hh * GQ + g] = l[g];
    }
  }
  __syncthreads();
  finish_work<T, D, QH, PS, true>(a, w, s_acc, s_m, s_l);
}

// ------------------------------------------------------------- MFMA path ---

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// LDS view of a byte offset into a __shared__ array.
__device__ __forceinline__ lds_s16x4 *lds_at(char *shared, uint32_t off) {
  return (lds_s16x4 *)((__attribute__((address_space(3))) char *)shared + off);
}

template <typename T>
struct Mfma;

template <>
struct Mfma<__bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  // 16x16x32: scores, K slices (A) against the group's query heads (B)
  __device__ __forceinline__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
  // 16x16x16: probabilities (A) against transposed V (B)
  __device__ __forceinline__ static f32x4 mma16(s16x4 a, s16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  // f rounded to bf16: (bits, value as float)
  __device__ __forceinline__ static short round(float f, float *r) {
    const short b = __builtin_bit_cast(short, static_cast<__bf16>(f));
    *r = __uint_as_float(static_cast<unsigned int>(static_cast<unsigned short>(b)) << 16);
    return b;
  }
};

template <>
struct Mfma<_Float16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 v4 __attribute__((ext_vector_type(4)));
  __device__ __forceinline__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static f32x4 mma16(s16x4 a, s16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4, a), __builtin_bit_cast(v4, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static short round(float f, float *r) {
    const _Float16 h = static_cast<_Float16>(f);
    *r = static_cast<float>(h);
    return __builtin_bit_cast(short, h);
  }
};

// Both products of a 16-position tile on the matrix cores.
//
//   scores  S = K Q^T with v_mfma_f32_16x16x32: lane l = (kg = l / 16,
//           r = l % 16) holds, as the A operand, position r's 16-byte K
//           slices 4j + kg (j < D/32) and, as the B operand, the same slices
//           of query head r (zero for r >= G).  The result gives lane l the
//           scores of positions 4 kg + e (e < 4) for head r.
//   values  O += P V with v_mfma_f32_16x16x16 per 16 columns of V: that
//           score layout is already the A operand (lane (kg, r): head r,
//           positions 4 kg + e), so the probabilities stay in registers.  V
//           is staged row-major in a per-wave LDS tile and read back
//           transposed by ds_read_b64_tr_b16, which hands lane 4c + d of each
//           16-lane group element d of the 8 bytes addressed by lanes c,
//           c + 4, c + 8, c + 12: with lane s of group kg addressing V row
//           4 kg + s / 4, columns n0 + 4 (s % 4).., lane (kg, n) receives
//           V[4 kg + e][n0 + n], e < 4 -- the B operand.  The accumulator lane
//           (kg, n) holds O[head 4 kg + e][n0 + n].
//
// The probabilities enter the product as hi + lo pairs of the input type, so
// the products carry about 17 bits of each probability; scores, sums and O
// stay in fp32.
//
// Three waves per SIMD (at most 168 registers per lane): measured faster than
// two (more registers, accumulators in AGPRs) and than four on the
// Llama-2-70B TP-8 share (16.8 vs 19.7 and 18.4 us per layer).
template <typename T, int D, int G>
__global__ __launch_bounds__(kAttThreads, 3) void attend_mfma_kernel(const AttendArgs a) {
  static_assert(sizeof(T) == 2 && G <= 16, "MFMA path: 16-bit types, up to 16 heads per group");
  using M = Mfma<T>;
  constexpr int NJ = D / 32;         // score k-steps of 32 elements
  constexpr int NC = D / 16;         // value column chunks of 16
  constexpr int VLPP = D / 8;        // lanes per V row (16 bytes each)
  constexpr int VPPI = 64 / VLPP;    // V rows per load
  constexpr int UV = 16 / VPPI;      // V loads per tile
  constexpr int PITCH = 2 * D + 32;  // LDS bytes per staged V row (padded: transposed reads spread over banks)
  static_assert(NJ >= 1 && VLPP <= 64 && UV >= 1 && UV * VPPI == 16, "head_dim");
  __shared__ __attribute__((aligned(16))) char s_v[kAttWaves][16 * PITCH];
  __shared__ __attribute__((aligned(16))) float s_acc[kAttWaves][G][D];
  __shared__ float s_m[kAttWaves][G], s_l[kAttWaves][G];
  Work w;
  if (!begin_work<T, D, G>(a, w)) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kg = lane >> 4, r = lane & 15;
  const int vg = lane / VLPP, vs = lane % VLPP;
  const float scale = a.scale_log2;
  const bool head_lane = r < G;

  const T *qrow = static_cast<const T *>(a.q) + w.b * a.q_bs + w.t * a.q_rs + w.qh0 * D;
  u32x4 qb[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    qb[j] = head_lane ? *reinterpret_cast<const u32x4 *>(qrow + r * D + (4 * j + kg) * 8) : u32x4{0u, 0u, 0u, 0u};

  const char *kseq = static_cast<const char *>(a.cache) +
                     (w.b * a.c_bs + static_cast<int64_t>(w.hk) * D) * static_cast<int64_t>(sizeof(T));
  const char *vseq = kseq + a.c_kv * static_cast<int64_t>(sizeof(T));
  const uint32_t row_bytes = static_cast<uint32_t>(a.c_ps * sizeof(T));
  const uint32_t k_lane = static_cast<uint32_t>(w.p0 + r) * row_bytes + kg * 16;
  const uint32_t v_lane = static_cast<uint32_t>(w.p0 + vg) * row_bytes + vs * 16;

  // This wave's V tile: row-major stores, transposed reads.
  char *vtile = s_v[wave];
  const uint32_t v_store = vg * PITCH + vs * 16;
  const uint32_t v_read = (4 * kg + r / 4) * PITCH + (r % 4) * 8;

  float m = kNoScore, lp = 0.f;  // head r's running max and this lane's share of its sum
  f32x4 acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One tile of 16 positions starting at p0 + i0: `fetch` issues its loads
  // (MODE 0 full, 1 tail: positions past n_cache clamped to the last cached
  // one, 2: the new row from kv_new in every slot, written to the cache by
  // the writer); `consume` computes it (masking what MODE 1 and 2 do not
  // attend).  Every staged V row holds finite data, so masked (zero)
  // probabilities contribute exact zeros.
  auto fetch = [&](int i0, u32x4 (&kr)[NJ], u32x4 (&vr)[UV], auto mode) {
    constexpr int MODE = decltype(mode)::value;
    if constexpr (MODE == 2) {
      const char *knew = static_cast<const char *>(a.kv_new) +
                         ((static_cast<int64_t>(w.b) * 2 * a.kv_heads + w.hk) * D) * static_cast<int64_t>(sizeof(T));
      const char *vnew = knew + static_cast<int64_t>(a.kv_heads) * D * sizeof(T);
#pragma unroll
      for (int j = 0; j < NJ; ++j) kr[j] = *reinterpret_cast<const u32x4 *>(knew + (4 * j + kg) * 16);
#pragma unroll
      for (int u = 0; u < UV; ++u) vr[u] = *reinterpret_cast<const u32x4 *>(vnew + vs * 16);
      if (w.writer && lane < VLPP) {
        const uint32_t off = static_cast<uint32_t>(w.pos_new) * row_bytes + vs * 16;
        *reinterpret_cast<u32x4 *>(const_cast<char *>(kseq) + off) = *reinterpret_cast<const u32x4 *>(knew + vs * 16);
        *reinterpret_cast<u32x4 *>(const_cast<char *>(vseq) + off) = vr[0];
      }
    } else {
      uint32_t koff, voff[UV];
      if constexpr (MODE == 1) {
        const int last = w.n_cache - 1;
        koff = static_cast<uint32_t>(w.p0 + min(i0 + r, last)) * row_bytes + kg * 16;
#pragma unroll
        for (int u = 0; u < UV; ++u)
          voff[u] = static_cast<uint32_t>(w.p0 + min(i0 + u * VPPI + vg, last)) * row_bytes + vs * 16;
      } else {
        koff = k_lane + static_cast<uint32_t>(i0) * row_bytes;
#pragma unroll
        for (int u = 0; u < UV; ++u) voff[u] = v_lane + static_cast<uint32_t>(i0 + u * VPPI) * row_bytes;
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j) kr[j] = load16(kseq, koff + j * 64);
#pragma unroll
      for (int u = 0; u < UV; ++u) vr[u] = load16(vseq, voff[u]);
    }
  };
  auto consume = [&](int i0, const u32x4 (&kr)[NJ], const u32x4 (&vr)[UV], auto mode) {
    constexpr int MODE = decltype(mode)::value;
    // Stage V while the scores are computed.
#pragma unroll
    for (int u = 0; u < UV; ++u) *reinterpret_cast<u32x4 *>(vtile + v_store + u * VPPI * PITCH) = vr[u];
    f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NJ; ++j) c = M::mma(kr[j], qb[j], c);
    float s[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s[e] = c[e];
      if constexpr (MODE == 1) s[e] = i0 + 4 * kg + e < w.n_cache ? s[e] : -INFINITY;
      if constexpr (MODE == 2) s[e] = (kg == 0 && e == 0) ? s[e] : -INFINITY;
    }
    const float mt = max_from<16>(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]))) * scale;
    const bool up = head_lane && mt > m + kRescaleSlack;
    if (__any(up)) {
      const float mnew = up ? mt : m;
      const float cf = fast_exp2(m - mnew);
      m = mnew;
      lp *= cf;
      // accumulator rows are heads 4 kg + e; lane h (< 16) holds head h's factor
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float ce = __shfl(cf, 4 * kg + e);
#pragma unroll
        for (int ch = 0; ch < NC; ++ch) acc[ch][e] *= ce;
      }
    }
    // Each probability enters the product as the sum of two 16-bit values
    // (p = hi + lo to about 2^-17 relative); both products with the 16-bit V
    // are exact in the fp32 accumulator, and the sum takes hi + lo too.
    s16x4 pa_hi, pa_lo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p = head_lane ? fast_exp2(fmaf(s[e], scale, -m)) : 0.f;
      float hi, lo;
      pa_hi[e] = M::round(p, &hi);
      pa_lo[e] = M::round(p - hi, &lo);
      lp += hi + lo;
    }
    __builtin_amdgcn_wave_barrier();
    // (V is read twice from LDS rather than held: fewer registers.)
#pragma unroll
    for (int ch = 0; ch < NC; ++ch)
      acc[ch] = M::mma16(pa_hi, __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_at(vtile, v_read + ch * 32)), acc[ch]);
#pragma unroll
    for (int ch = 0; ch < NC; ++ch)
      acc[ch] = M::mma16(pa_lo, __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_at(vtile, v_read + ch * 32)), acc[ch]);
    __builtin_amdgcn_wave_barrier();
  };

  // Tiles of 16 positions, dealt round-robin to the waves; the next full
  // tile's loads are in flight while the current one computes.
  using Full = std::integral_constant<int, 0>;
  const int full_tiles = w.n_cache / 16;
  int ti = wave;
  if (ti < full_tiles) {
    u32x4 ka[NJ], va[UV];
    fetch(ti * 16, ka, va, Full{});
    for (; ti + kAttWaves < full_tiles; ti += kAttWaves) {
      u32x4 kb[NJ], vb[UV];
      fetch((ti + kAttWaves) * 16, kb, vb, Full{});
      consume(ti * 16, ka, va, Full{});
#pragma unroll
      for (int j = 0; j < NJ; ++j) ka[j] = kb[j];
#pragma unroll
      for (int u = 0; u < UV; ++u) va[u] = vb[u];
    }
    consume(ti * 16, ka, va, Full{});
    ti += kAttWaves;
  }
  if (ti * 16 < w.n_cache) {
    u32x4 kr[NJ], vr[UV];
    fetch(ti * 16, kr, vr, std::integral_constant<int, 1>{});
    consume(ti * 16, kr, vr, std::integral_constant<int, 1>{});
  }
  if (w.has_new && wave == 0) {
    u32x4 kr[NJ], vr[UV];
    fetch(0, kr, vr, std::integral_constant<int, 2>{});
    consume(0, kr, vr, std::integral_constant<int, 2>{});
  }

  // Wave totals: l over the 4 kg lanes of each head; O rows from the
  // accumulator layout.
  lp = sum_from<16>(lp);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int h = 4 * kg + e;
    if (h < G) {
#pragma unroll
      for (int ch = 0; ch < NC; ++ch) s_acc[wave][h][ch * 16 + r] = acc[ch][e];
    }
  }
  if (lane < G) {
    s_m[wave][lane] = m;
    s_l[wave][lane] = lp;
  }
  __syncthreads();
  finish_work<T, D, G>(a, w, s_acc, s_m, s_l);
}

// Merges the partitions of one (query row, query head) of a split row:
// o = sum_p w_p o_p with w_p = 2^(m_p - max m) / sum_p 2^(m_p - max m) l_p.
// One workgroup per (head, row) keeps the per-workgroup chain short when a
// few long rows carry many partitions.  The 256 threads split the partitions
// into 256 / D slices of D outputs each and add the slices through LDS.
//
// Fast path (up to kCombineDepth partitions per slice, the decode shapes):
// once the row length is in, every partition's (max, sum) and this thread's
// partial outputs are loaded at once, so the workgroup waits for two rounds
// of memory latency instead of three (length, then (max, sum), then the
// outputs behind a barrier) and reads only the row's own partitions.
// Otherwise the weights are staged in LDS kCombineChunk partitions at a time.
constexpr int kCombineChunk = 256;  // partitions whose weights sit in LDS at once

// kCombineDepth: partial outputs per thread held in registers, 8 or 32,
// chosen by the host from max_parts (the smaller instance keeps every
// workgroup of a large decode batch resident at once).
template <typename T, int D, int G, int kCombineDepth>
__global__ __launch_bounds__(kAttThreads) void combine_kernel(const AttendArgs a) {
  using E = Elem<T>;
  constexpr int SL = kAttThreads / D >= 1 ? kAttThreads / D : 1;  // partition slices
  constexpr int PER = (D + kAttThreads - 1) / kAttThreads;        // outputs per thread (D > 256)
  __shared__ float s_w[kCombineChunk];
  __shared__ float s_red[SL][D];
  __shared__ float s_wmax[kAttWaves], s_wsum[kAttWaves];
  __shared__ float s_mx, s_inv;
  const int h = blockIdx.x, row = blockIdx.y;
  const int b = row / a.q_len, t = row - b * a.q_len;
  const int tid = threadIdx.x, wave = tid >> 6;
  const int64_t base = (static_cast<int64_t>(row) * a.q_heads + h) * a.max_parts;
  const float *ml = a.ws_ml + base * 2;
  const int d0 = tid % D, sl = tid / D;
  T *out = static_cast<T *>(a.out) + b * a.o_bs + t * a.o_rs + static_cast<int64_t>(h) * D;

  if constexpr (PER == 1) {
    if (a.max_parts <= kCombineChunk && a.max_parts <= SL * kCombineDepth) {
      int nparts;
      if (a.items) {
        nparts = min(a.seg_parts[row * a.n_groups + h / G], a.max_parts);
      } else {
        int pos_new;
        bool clamped;
        const int len = row_length(a, b, t, &pos_new, &clamped);
        nparts = len > 0 ? (len + a.part - 1) / a.part : 0;
      }
      if (nparts <= 1) return;  // written by the attention kernel
      const bool valid = tid < nparts;
      float2 mlv = {-INFINITY, 0.f};
      if (valid) mlv = *reinterpret_cast<const float2 *>(ml + 2 * tid);
      float ov[kCombineDepth];
      const float *o = a.ws_o + base * D + d0;
#pragma unroll
      for (int k = 0; k < kCombineDepth; ++k) {
        const int p = sl + k * SL;
        ov[k] = 0.f;
        if (sl < SL && p < nparts) ov[k] = o[static_cast<int64_t>(p) * D];
      }
      const float mp = valid ? mlv.x : -INFINITY;
      float mx = wave_max(mp);
      if ((tid & 63) == 0) s_wmax[wave] = mx;
      __syncthreads();
      mx = s_wmax[0];
#pragma unroll
      for (int w = 1; w < kAttWaves; ++w) mx = fmaxf(mx, s_wmax[w]);
      const float c = valid ? fast_exp2(mp - mx) : 0.f;
      s_w[tid] = c;
      const float sum = sum_from<1>(valid ? c * mlv.y : 0.f);
      if ((tid & 63) == 0) s_wsum[wave] = sum;
      __syncthreads();
      float total = 0.f;
#pragma unroll
      for (int w = 0; w < kAttWaves; ++w) total += s_wsum[w];
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < kCombineDepth; ++k) {
        const int p = sl + k * SL;
        if (sl < SL && p < nparts) acc = fmaf(s_w[p], ov[k], acc);
      }
      if constexpr (SL > 1) {
        if (sl < SL) s_red[sl][d0] = acc;
        __syncthreads();
        if (tid < D) {
          float r = 0.f;
#pragma unroll
          for (int k = 0; k < SL; ++k) r += s_red[k][tid];
          out[tid] = E::from_float(r / total);
        }
      } else {
        if (sl == 0) out[d0] = E::from_float(acc / total);
      }
      return;
    }
  }

  int nparts;
  if (a.items) {
    nparts = min(a.seg_parts[row * a.n_groups + h / G], a.max_parts);
  } else {
    int pos_new;
    bool clamped;
    const int len = row_length(a, b, t, &pos_new, &clamped);
    nparts = len > 0 ? (len + a.part - 1) / a.part : 0;
  }
  if (nparts <= 1) return;
  if (tid < 64) {
    float mx = kNoScore;
    for (int p = tid; p < nparts; p += 64) mx = fmaxf(mx, ml[2 * p]);
    mx = max_from<1>(mx);
    float sum = 0.f;
    for (int p = tid; p < nparts; p += 64) sum = fmaf(fast_exp2(ml[2 * p] - mx), ml[2 * p + 1], sum);
    sum = sum_from<1>(sum);
    if (tid == 0) {
      s_mx = mx;
      s_inv = 1.f / sum;
    }
  }
  float acc[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) acc[k] = 0.f;
  for (int c0 = 0; c0 < nparts; c0 += kCombineChunk) {
    const int nc = min(kCombineChunk, nparts - c0);
    __syncthreads();  // s_mx/s_inv ready; the previous chunk's weights consumed
    for (int p = tid; p < nc; p += kAttThreads) s_w[p] = fast_exp2(ml[2 * (c0 + p)] - s_mx) * s_inv;
    __syncthreads();
    if (sl < SL) {
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const float *o = a.ws_o + (base + c0) * D + d0 + k * kAttThreads;
        int p = sl;
        for (; p + 7 * SL < nc; p += 8 * SL) {
          float v[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) v[u] = o[static_cast<int64_t>(p + u * SL) * D];
#pragma unroll
          for (int u = 0; u < 8; ++u) acc[k] = fmaf(s_w[p + u * SL], v[u], acc[k]);
        }
        for (; p < nc; p += SL) acc[k] = fmaf(s_w[p], o[static_cast<int64_t>(p) * D], acc[k]);
      }
    }
  }
  if constexpr (SL > 1) {
    if (sl < SL) s_red[sl][d0] = acc[0];
    __syncthreads();
    if (tid < D) {
      float o = 0.f;
#pragma unroll
      for (int k = 0; k < SL; ++k) o += s_red[k][tid];
      out[tid] = E::from_float(o);
    }
  } else {
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int d = d0 + k * kAttThreads;
      if (sl == 0 && d < D) out[d] = E::from_float(acc[k]);
    }
  }
}

// ------------------------------------------------------------------ host ---

static int elem_size(int dtype) { return dtype == HEXKV_F32 ? 4 : 2; }

// Largest group size the kernels are compiled for that divides q/kv heads.
static int kernel_group(int group) {
  for (int g : {8, 4, 2, 1})
    if (group % g == 0) return g;
  return 1;
}

// KV heads per work item of the row-block kernel (HEXKV_KERNEL_ROWS), or 0
// when these parameters do not fit it (16-bit data, head_dim 128, 2+ KV
// heads, 1, 2 or 4 query heads per KV head).  2 for grouped queries, 8 (else
// the largest of 4, 2 dividing the KV heads) for one query head per KV head:
// measured per call at Llama-3-8B's shape (bf16, 8 KV heads, group 4;
// decode steps 0 / 128 / 255, ~400 items) 152.3 / 158.9 / 163.2 us with 2
// heads per item, 157.3 / 160.8 / 164.6 with 4 and 155.7 / 161.6 / 166.8
// with 8, against 166.2 / 170.3 / 175.7 with one head per item; at
// Llama-2-7B's (fp16, 32 KV heads, group 1; steps 0 / 32 / 63) 29.9 / 30.6 /
// 31.3 with 8, 31.3 / 31.8 / 32.5 with 2 and 31.4 / 32.7 / 33.4 with 4,
// against 31.2 / 32.1 / 32.5.
static int rows_block(const hexkv_attend_params *p) {
  if (p->dtype == HEXKV_F32 || p->head_dim != 128 || p->kv_heads < 2) return 0;
  const int group = p->q_heads / p->kv_heads;
  if (group != 1 && group != 2 && group != 4) return 0;
  if (group > 1) return p->kv_heads % 2 == 0 ? 2 : 0;
  for (int hb : {8, 4, 2})
    if (p->kv_heads % hb == 0) return hb;
  return 0;
}

// Query heads per (row, head group) segment: a head block's for the
// row-block kernel, a kernel group's otherwise.
static int segment_heads(const hexkv_attend_params *p) {
  const int group = p->q_heads / p->kv_heads;
  if (p->kernel == HEXKV_KERNEL_ROWS) return rows_block(p) * group;
  return kernel_group(group);
}

// Partition size: about (rows x head groups x positions) / 2048 positions,
// as a power of two in [128, 512], counting half of max_seqlen per row
// (ragged batches average about that).  Measured on MI355X (attention +
// combine per layer, interleaved A/B in one process): Llama-3-8B's shape
// (64 rows x 8 groups, lengths to 8K) 165.3 us at 512, 166.5 at 768, 169.3 at
// 1024, 168.1 at 384; the Llama-2-70B TP-8 share (32 x 1, to 4K) is fastest
// at 128-256, TinyLlama (1 x 4, 512) at 64-256; Llama-2-7B (8 x 32, to 2K)
// gets 256 (33.5 us; 1024 measured 32.4, 512 35.5 -- not monotonic, left
// alone).  An evenly split persistent schedule (one wave of workgroups, each
// an equal share of all positions, pieces merged after) was built and
// measured slower on every one of these shapes (Llama-3-8B 172.5 vs 171.1 us,
// the 70B TP-8 share 26.3 vs 15.9): at 512 positions the partitions already
// balance the launch, and finer pieces only add partials to merge.
static int choose_partition(const hexkv_attend_params *p) {
  if (p->partition > 0) return p->partition;
  const int64_t rows = static_cast<int64_t>(p->batch) * p->q_len;
  const int64_t groups = p->q_heads / kernel_group(p->q_heads / p->kv_heads);
  const int64_t half = std::max<int64_t>(1, (p->max_seqlen + 1) / 2);
  const int64_t want = rows * groups * half / 2048;
  int part = 128;
  while (part < 512 && part < want) part <<= 1;
  return part;
}

// Partitions per (row, head group) the workspace holds: from the work list
// when there is one, else from the partition size and max_seqlen.
static int64_t max_parts_of(const hexkv_attend_params *p, int part) {
  if (p->work_items_dev) return std::max<int64_t>(1, p->work_max_parts);
  return std::max<int64_t>(1, (p->max_seqlen + part - 1) / part);
}

// Arrival counters of the XCD-local merge at the front of every workspace
// (one 64-bit word per (row, head group) segment), whatever the call's mode,
// so that one workspace serves calls of either mode.
constexpr int64_t kCounterWords = HEXKV_ATTEND_COUNTER_BYTES / sizeof(uint64_t);

// Workspace: the arrival counters, then the partial outputs
// [rows][q_heads][max_parts][D], then their (max, sum) pairs
// [rows][q_heads][max_parts][2], all fp32.
static size_t workspace_bytes(const hexkv_attend_params *p, int part) {
  const int64_t max_parts = max_parts_of(p, part);
  if (max_parts <= 1) return 0;
  const int64_t rows = static_cast<int64_t>(p->batch) * p->q_len;
  return HEXKV_ATTEND_COUNTER_BYTES +
         static_cast<size_t>(rows * p->q_heads * max_parts * (p->head_dim + 2)) * sizeof(float);
}

static int validate(const hexkv_attend_params *p) {
  if (!p) return fail(HEXKV_EINVAL, "hexkv_attend: null params");
  if (p->dtype != HEXKV_F16 && p->dtype != HEXKV_BF16 && p->dtype != HEXKV_F32)
    return fail(HEXKV_EINVAL, "hexkv_attend: unknown dtype %d", p->dtype);
  if (p->batch < 0 || p->q_len < 1 || p->q_heads < 1 || p->kv_heads < 1)
    return fail(HEXKV_EINVAL, "hexkv_attend: bad batch/q_len/heads");
  if (p->q_heads % p->kv_heads != 0)
    return fail(HEXKV_EINVAL, "hexkv_attend: q_heads %d not a multiple of kv_heads %d", p->q_heads,
                p->kv_heads);
  const int d = p->head_dim;
  if (d != 16 && d != 32 && d != 64 && d != 128 && d != 256)
    return fail(HEXKV_EUNSUPPORTED, "hexkv_attend: head_dim %d (compiled: 16, 32, 64, 128, 256)", d);
  if (static_cast<int64_t>(p->batch) * p->q_len > 65535)
    return fail(HEXKV_EINVAL, "hexkv_attend: batch*q_len above 65535");
  if (p->kv_new && p->q_len != 1) return fail(HEXKV_EINVAL, "hexkv_attend: fused append needs q_len 1");
  if (p->max_seqlen < 0 || p->max_seqlen > p->capacity)
    return fail(HEXKV_ERANGE, "hexkv_attend: max_seqlen %d outside [0, capacity %lld]",
                p->max_seqlen, static_cast<long long>(p->capacity));
  // With a work list the items carry the positions and the partition is not
  // read; it may then hold the list's chunk, which can exceed 4096.
  // (Row-block lists are cut in multiples of 16 positions.)
  const int grain = p->kernel == HEXKV_KERNEL_ROWS ? 16 : 64;
  if (p->partition < 0 || (p->partition > 0 && p->partition % grain != 0) ||
      (!p->work_items_dev && p->partition > 4096))
    return fail(HEXKV_EINVAL, "hexkv_attend: partition must be 0 or a multiple of %d (up to 4096 without a work list)",
                grain);
  if (!(p->softmax_scale > 0.f) || p->softmax_scale > 3.0e38f)
    return fail(HEXKV_EINVAL, "hexkv_attend: softmax_scale must be positive and finite");
  if (p->kernel < HEXKV_KERNEL_AUTO || p->kernel > HEXKV_KERNEL_ROWS)
    return fail(HEXKV_EINVAL, "hexkv_attend: unknown kernel %d", p->kernel);
  if (p->kernel == HEXKV_KERNEL_MFMA && (p->dtype == HEXKV_F32 || p->head_dim < 64))
    return fail(HEXKV_EUNSUPPORTED, "hexkv_attend: the MFMA kernel takes float16/bfloat16 with head_dim >= 64");
  if (p->kernel == HEXKV_KERNEL_ROWS && !rows_block(p))
    return fail(HEXKV_EUNSUPPORTED, "hexkv_attend: the row-block kernel takes float16/bfloat16, head_dim 128, "
                                    "2+ KV heads and 1, 2 or 4 query heads per KV head");
  if (p->work_xcds < 0 || p->work_xcds > 64) return fail(HEXKV_EINVAL, "hexkv_attend: work_xcds outside [0, 64]");
  if (p->lengths_out_dev && (!p->work_items_dev || !p->kv_new))
    return fail(HEXKV_EINVAL, "hexkv_attend: lengths_out_dev needs a work list and kv_new");
  if (p->batch == 0) return HEXKV_OK;  // nothing to launch, with or without a work list
  if (p->work_items_dev) {
    if (p->n_work_items < 1 || !p->work_parts_dev || p->work_max_parts < 1 || p->work_max_parts > 65535)
      return fail(HEXKV_EINVAL, "hexkv_attend: a work list needs n_work_items >= 1, work_parts_dev and "
                                "1 <= work_max_parts <= 65535");
    if (!aligned16(p->work_items_dev) || (reinterpret_cast<uintptr_t>(p->work_parts_dev) & 3u))
      return fail(HEXKV_EINVAL, "hexkv_attend: work_items_dev must be 16-byte aligned, work_parts_dev 4-byte");
    if (p->q_len != 1 || p->causal)
      return fail(HEXKV_EINVAL, "hexkv_attend: a work list is for decode rows (q_len 1, not causal)");
    if (p->work_xcds > 0 && static_cast<int64_t>(p->batch) * (p->q_heads / segment_heads(p)) > kCounterWords)
      return fail(HEXKV_EINVAL, "hexkv_attend: the single-launch merge counts at most %lld (row, head group) "
                                "segments; use work_xcds 0", static_cast<long long>(kCounterWords));
    if (p->kernel == HEXKV_KERNEL_ROWS &&
        (p->work_xcds < 1 || p->work_xcds > 8 || p->work_max_parts > kMergeMaxParts))
      return fail(HEXKV_EUNSUPPORTED, "hexkv_attend: the row-block kernel merges in the kernel: a list planned "
                                      "for 1-8 XCDs with at most %d partitions per segment", kMergeMaxParts);
  } else if (p->work_xcds > 0) {
    return fail(HEXKV_EINVAL, "hexkv_attend: work_xcds is for work lists");
  } else if (p->kernel == HEXKV_KERNEL_ROWS) {
    return fail(HEXKV_EUNSUPPORTED, "hexkv_attend: the row-block kernel runs work lists only");
  }
  if (p->lengths_out_dev && (reinterpret_cast<uintptr_t>(p->lengths_out_dev) & 3u))
    return fail(HEXKV_EINVAL, "hexkv_attend: lengths_out_dev must be 4-byte aligned");
  if (!p->q || !p->cache || !p->out) return fail(HEXKV_EINVAL, "hexkv_attend: null tensor");
  const int vec = 16 / elem_size(p->dtype);
  if (!aligned16(p->q) || !aligned16(p->cache) || (p->kv_new && !aligned16(p->kv_new)))
    return fail(HEXKV_EINVAL, "hexkv_attend: q/cache/kv_new must be 16-byte aligned");
  if (p->q_batch_stride % vec || p->q_row_stride % vec || p->cache_batch_stride % vec ||
      p->cache_pos_stride % vec || p->cache_kv_stride % vec)
    return fail(HEXKV_EINVAL, "hexkv_attend: strides must be multiples of 16 bytes");
  if ((reinterpret_cast<uintptr_t>(p->out) & (elem_size(p->dtype) - 1)) != 0)
    return fail(HEXKV_EINVAL, "hexkv_attend: out misaligned");
  // K/V are addressed as a per-sequence base plus a 32-bit byte offset.
  if (p->cache_pos_stride <= 0 || p->cache_kv_stride < 0 ||
      (static_cast<int64_t>(p->max_seqlen) * p->cache_pos_stride + p->cache_kv_stride +
       static_cast<int64_t>(p->kv_heads) * d) * elem_size(p->dtype) > INT64_C(0xffffffff))
    return fail(HEXKV_EUNSUPPORTED, "hexkv_attend: one sequence of the cache spans more than 4 GiB");
  return HEXKV_OK;
}

// Load slots per lane group and iteration of the VALU kernel (with the next
// iteration's loads in flight): 2 for one 16-byte vector per lane, 1 for two
// or more.  Measured at Llama-3-8B, 1024-position partitions: 2 slots +
// prefetch 171.4 us, 4 slots + prefetch 172.7, 2 slots without 178.3,
// 1 slot without 187.8.
template <typename T, int D, int G>
constexpr int slots() {
  return Lanes<T, D>::NV >= 2 ? 1 : 2;
}

// Kernel choice: the MFMA kernel for 16-bit data with head_dim >= 64 and 8+
// query heads per KV head, where it beats the VALU kernel (Llama-2-70B TP-8
// share: 16.0 vs 23.8 us per layer at the best partition of each; TinyLlama:
// 10.6 vs 11.9); the VALU kernel otherwise (Llama-3-8B, group 4: 176.4 vs
// 180.6; Llama-2-7B, group 1: 34.8 vs 38.1).
// head_dim 256 stays on the VALU kernel: the MFMA kernel's accumulators spill
// to scratch there.
static bool use_mfma(const hexkv_attend_params *p, int G) {
  if (p->kernel == HEXKV_KERNEL_MFMA) return true;
  if (p->kernel == HEXKV_KERNEL_VALU) return false;
  return p->dtype != HEXKV_F32 && p->head_dim >= 64 && p->head_dim <= 128 && G >= 8;
}

// Which attention kernel a launch runs.
enum LaunchKind { kLaunchValu = 0, kLaunchMfma = 1, kLaunchFt = 2 };

template <typename T, int D, int G>
static void launch(const AttendArgs &a, dim3 grid, int kind, hipStream_t s) {
  if (kind == kLaunchFt) {
    attend_valu_kernel<T, D, G, slots<T, D, G>(), true, true><<<grid, kAttThreads, 0, s>>>(a);
  } else if constexpr (sizeof(T) == 2 && D >= 64) {
    if (kind == kLaunchMfma) attend_mfma_kernel<T, D, G><<<grid, kAttThreads, 0, s>>>(a);
    else attend_valu_kernel<T, D, G, slots<T, D, G>()><<<grid, kAttThreads, 0, s>>>(a);
  } else {
    attend_valu_kernel<T, D, G, slots<T, D, G>()><<<grid, kAttThreads, 0, s>>>(a);
  }
  if (a.max_parts > 1 && !a.seg_count) {
    const dim3 cgrid(a.q_heads, a.rows);
    constexpr int SL = kAttThreads / D >= 1 ? kAttThreads / D : 1;
    if (a.max_parts <= 8 * SL) combine_kernel<T, D, G, 8><<<cgrid, kAttThreads, 0, s>>>(a);
    else combine_kernel<T, D, G, 32><<<cgrid, kAttThreads, 0, s>>>(a);
  }
}

// The row-block kernel (head_dim 128, 16-bit): GQ query heads per KV head,
// HB KV heads per item.
template <typename T, int GQ>
static int dispatch_rows_hb(int HB, const AttendArgs &a, dim3 grid, hipStream_t s) {
  // The head blocks rows_block picks: 2 KV heads for grouped queries; 8, 4
  // or 2 for one query head per KV head.
  constexpr int U = slots<T, 128, GQ>();
  if (HB == 2) {
    attend_rows_kernel<T, 128, GQ, 2, U><<<grid, kAttThreads, 0, s>>>(a);
    return HEXKV_OK;
  }
  if constexpr (GQ == 1) {
    if (HB == 4) {
      attend_rows_kernel<T, 128, GQ, 4, U><<<grid, kAttThreads, 0, s>>>(a);
      return HEXKV_OK;
    }
    if (HB == 8) {
      attend_rows_kernel<T, 128, GQ, 8, U><<<grid, kAttThreads, 0, s>>>(a);
      return HEXKV_OK;
    }
  }
  return fail(HEXKV_EUNSUPPORTED, "hexkv_attend: head block %d with %d query heads per KV head", HB, GQ);
}

template <typename T>
static int dispatch_rows(int GQ, int HB, const AttendArgs &a, dim3 grid, hipStream_t s) {
  switch (GQ) {
    case 1: return dispatch_rows_hb<T, 1>(HB, a, grid, s);
    case 2: return dispatch_rows_hb<T, 2>(HB, a, grid, s);
    case 4: return dispatch_rows_hb<T, 4>(HB, a, grid, s);
    default: return fail(HEXKV_EUNSUPPORTED, "hexkv_attend: group %d", GQ);
  }
}

template <typename T, int D>
static int dispatch_g(int G, const AttendArgs &a, dim3 grid, int kind, hipStream_t s) {
  switch (G) {
    case 1: launch<T, D, 1>(a, grid, kind, s); break;
    case 2: launch<T, D, 2>(a, grid, kind, s); break;
    case 4: launch<T, D, 4>(a, grid, kind, s); break;
    case 8: launch<T, D, 8>(a, grid, kind, s); break;
    default: return fail(HEXKV_EUNSUPPORTED, "hexkv_attend: group %d", G);
  }
  return HEXKV_OK;
}

template <typename T>
static int dispatch_d(int D, int G, const AttendArgs &a, dim3 grid, int kind, hipStream_t s) {
  switch (D) {
    case 16: return dispatch_g<T, 16>(G, a, grid, kind, s);
    case 32: return dispatch_g<T, 32>(G, a, grid, kind, s);
    case 64: return dispatch_g<T, 64>(G, a, grid, kind, s);
    case 128: return dispatch_g<T, 128>(G, a, grid, kind, s);
    case 256: return dispatch_g<T, 256>(G, a, grid, kind, s);
    default: return fail(HEXKV_EUNSUPPORTED, "hexkv_attend: head_dim %d", D);
  }
}

}  // namespace hexkv

namespace hexkv {

// Home XCD of each (row, head group) segment of a list planned for X XCDs
// (segment s = row * groups + group, len[row] positions): longest first,
// each to the XCD with the fewest positions so far.  All 0 for X = 1.
static std::vector<int> segment_homes(const std::vector<int64_t> &len, int groups, int X) {
  const int64_t segs = static_cast<int64_t>(len.size()) * groups;
  std::vector<int> home(static_cast<size_t>(segs), 0);
  if (X <= 1) return home;
  std::vector<int64_t> order(static_cast<size_t>(segs));
  for (int64_t i = 0; i < segs; ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(),
                   [&](int64_t x, int64_t y) { return len[x / groups] > len[y / groups]; });
  std::vector<int64_t> load(X, 0);
  for (const int64_t sg : order) {
    const int x = static_cast<int>(std::min_element(load.begin(), load.end()) - load.begin());
    home[sg] = x;
    load[x] += std::max<int64_t>(len[sg / groups], 1);
  }
  return home;
}

// Chunk size (positions) of a work list when the caller leaves the choice to
// the library, by the bytes one call reads (W positions over all (row, head
// group) segments, row_bytes per position of one KV head).  Measured on
// MI355X against the uniform grid and against each other (attention +
// merge per layer, interleaved A/B in one process): below 4 MB the call is
// launch-bound and no split at all is fastest (TinyLlama: 6.5 vs 8.1 us --
// no merge launch).  Up to 64 MB a workgroup's stream, not HBM, is the
// limit (about 22 GB/s per workgroup, one per CU, 4 or 8 waves alike), so
// about 240 items, close to one per CU, are fastest: the Llama-2-70B TP-8
// share (36 MB, read from HBM: twenty caches per measurement, more than the
// 256 MB MALL) 13.4-13.7 us at 320 positions against 14.1 at 384, 14.2 at
// 352, 14.8 at 448, 15.5 at 512 and 16.1 at 256.  Above 64 MB,
// 896-position chunks, or 1280 from a million positions up (Llama-2-7B,
// 0.34 M positions, single-launch merge, HBM-resident, first and last
// decode step: 30.2-31.7 us at 832-896 against 30.9-32.0 at 1024, 30.9-32.6
// at 768, 32.6-33.4 at 1152, 32.0-34.0 at 640; with the second-launch merge
// 896 had also led by 1-2%; Llama-3-8B, 2.0 M: 170.3-170.9 us at 1280
// against 173.0-173.2 at 1024, 179 for the grid and 179.6 at 512, over
// three boxes).
//
// Planned for the XCDs (split segments merged in the attention kernel, no
// second launch), calls below 4 MB are split too, in pieces of about a
// twelfth of the longest row (64 positions at least): TinyLlama's 577-640
// positions as 10 items of 64 per segment, 6.7 us per call against 9.1 for
// one item per segment (7.2 at 128 positions, 7.7 at 192, 8.3 at 256;
// HBM-resident A/B in one process).
static int plan_chunk(int64_t positions, int64_t row_bytes, int64_t longest, bool xcd_merge) {
  const int64_t bytes = positions * row_bytes;
  if (bytes < (INT64_C(4) << 20) && xcd_merge)
    return static_cast<int>(std::max<int64_t>(64, (longest / 12 + 63) / 64 * 64));
  if (bytes < (INT64_C(4) << 20)) return static_cast<int>(std::max<int64_t>(64, (longest + 63) / 64 * 64));
  if (bytes < (INT64_C(64) << 20)) return static_cast<int>(std::min<int64_t>(1024, std::max<int64_t>(64, (positions / 240 + 63) / 64 * 64)));
  return positions >= (INT64_C(1) << 20) ? 1280 : 896;
}

// Chunk of a row-block list (positions, a multiple of 16).  Each XCD runs
// its share of the list in order on its 32 CUs, as many workgroups per CU
// at once as registers and LDS allow (4 for 4 query heads per KV head: 103
// VGPRs and 33 KB of LDS; 5 otherwise: 84 VGPRs; the build records the
// compiler's figures and tests/test_kernel_resources.py holds them to
// these counts), so the first 32 x (workgroups per CU) items of a share
// start together and each later one starts when a slot frees.  A share is its segments' full chunks (all the same
// size), then their shorter last pieces from the longest down.  The chunk
// is the smallest one at which no share holds more than 27/32 of its slots
// in full chunks: the full chunks all start at once, and the slots left
// over hold the longest last pieces, which finish early and hand their
// slots to the short ones still waiting.  Measured on MI355X at Llama-3-8B
// (one layer, decode steps 0-255, HBM-resident, interleaved A/B in one
// process): 107-109 full chunks in a share of 128 slots 149.8-159.8 us per
// call (0.83 of 8 TB/s), 109-111 153.3-164.3, 113 or more 166.6-178.1 (the
// last pieces then wait for the full chunks: a second round), 95-102
// 157.8-168.1 (fewer, longer full chunks per CU); the earlier target of
// ~400 items (528 with the last pieces) 154.9-162.5; this rule 152.4-160.6.
// A model of the dispatch (each share in order onto 128 slots, each CU's
// bandwidth shared by its items) puts the best chunk at the same place and
// the cliff on its finer side, hence the margin.  Small calls are bound by
// each item's fixed latency instead: no item under kRowsItemBytes
// (Llama-2-7B, 8-head items of 4 KB per position: 112 positions, ~400
// items, 29.7-31.3 us per call over decode steps 0-63, against 33.2-35.2 at
// 80-96 and 34.8-37.2 at 64).  At most kMergeMaxParts pieces per row.
constexpr int kCusPerXcd = 32;
constexpr int64_t kRowsItemBytes = INT64_C(448) << 10;

static int rows_chunk(const hexkv_attend_params *p, const int32_t *lens, int hb, int64_t longest) {
  const int groups = p->kv_heads / hb;
  const int X = std::max(1, p->work_xcds);
  const int extra = p->kv_new ? 1 : 0;
  std::vector<int64_t> len(p->batch);
  for (int b = 0; b < p->batch; ++b) len[b] = static_cast<int64_t>(lens[b]) + p->seqlen_bias + extra;
  const std::vector<int> home = segment_homes(len, groups, X);
  const int64_t per_cu = p->q_heads / p->kv_heads == 4 ? 4 : 5;
  const int64_t full_limit = kCusPerXcd * per_cu * 27 / 32;
  const int64_t block_bytes = 2 * static_cast<int64_t>(hb) * p->head_dim * elem_size(p->dtype);
  const int64_t fewest = (longest + kMergeMaxParts - 1) / kMergeMaxParts;  // positions per piece
  auto up16 = [](int64_t v) { return (v + 15) / 16 * 16; };
  const int64_t lo = std::max<int64_t>({16, up16((kRowsItemBytes + block_bytes - 1) / block_bytes), up16(fewest)});
  auto fits = [&](int64_t c) {
    std::vector<int64_t> full(X, 0);
    for (size_t sg = 0; sg < home.size(); ++sg) full[home[sg]] += len[sg / groups] / c;
    return *std::max_element(full.begin(), full.end()) <= full_limit;
  };
  // full chunks per share only fall as the chunk grows: binary search over
  // multiples of 16 in [lo, hi], hi past the longest row (no full chunk)
  int64_t a = lo / 16, z = std::max(lo, up16(longest + 1)) / 16;
  if (fits(a * 16)) return static_cast<int>(a * 16);
  while (z - a > 1) {
    const int64_t m = (a + z) / 2;
    (fits(m * 16) ? z : a) = m;
  }
  return static_cast<int>(z * 16);
}

// Checks a planning request and returns the chunk hexkv_attend_plan cuts
// segments into (> 0), or a negative error code.
static int plan_request(const hexkv_attend_params *p, const int32_t *lens, const char *what) {
  if (!p || !lens) return fail(HEXKV_EINVAL, "%s: null argument", what);
  if (p->q_heads < 1 || p->kv_heads < 1 || p->q_heads % p->kv_heads || p->batch < 0 || p->batch > 65535)
    return fail(HEXKV_EINVAL, "%s: bad batch or head counts", what);
  if (p->q_len != 1 || p->causal) return fail(HEXKV_EINVAL, "%s: work lists are for decode rows (q_len 1, not causal)", what);
  if (p->kernel < HEXKV_KERNEL_AUTO || p->kernel > HEXKV_KERNEL_ROWS)
    return fail(HEXKV_EINVAL, "%s: unknown kernel %d", what, p->kernel);
  // Row-block items hold several heads per position: finer chunks.
  const int grain = p->kernel == HEXKV_KERNEL_ROWS ? 16 : 64;
  if (p->partition < 0 || (p->partition > 0 && (p->partition % grain != 0 || p->partition > (1 << 30))))
    return fail(HEXKV_EINVAL, "%s: partition must be 0 or a positive multiple of %d", what, grain);
  const int hb = p->kernel == HEXKV_KERNEL_ROWS ? rows_block(p) : 1;
  if (!hb || (p->kernel == HEXKV_KERNEL_ROWS && p->work_xcds < 1))
    return fail(HEXKV_EUNSUPPORTED, "%s: the row-block kernel takes float16/bfloat16, head_dim 128, 2+ KV heads, "
                                    "1, 2 or 4 query heads per KV head, and a list planned for the XCDs", what);
  // Segment positions as the per-KV-head kernels count them (the chunk rule
  // below is measured in those); a row-block item holds hb of them per
  // position.
  const int groups = p->q_heads / kernel_group(p->q_heads / p->kv_heads);
  const int extra = p->kv_new ? 1 : 0;
  int64_t positions = 0, longest = 0;
  for (int b = 0; b < p->batch; ++b) {
    const int64_t len = static_cast<int64_t>(lens[b]) + p->seqlen_bias + extra;
    if (len < 0 || len > p->max_seqlen)
      return fail(HEXKV_ERANGE, "%s: row %d attends %lld keys, outside [0, max_seqlen %d]", what, b,
                  static_cast<long long>(len), p->max_seqlen);
    positions += len * groups;
    longest = std::max(longest, len);
  }
  if (p->partition > 0) {
    if (hb > 1 && (longest + p->partition - 1) / p->partition > kMergeMaxParts)
      return fail(HEXKV_EUNSUPPORTED, "%s: partition %d cuts a %lld-key row into more than %d pieces, which the "
                                      "row-block kernel cannot merge", what, p->partition,
                  static_cast<long long>(longest), kMergeMaxParts);
    return p->partition;
  }
  const int64_t row_bytes = 2 * static_cast<int64_t>(p->head_dim) * elem_size(p->dtype);
  if (hb == 1) return plan_chunk(positions, row_bytes, longest, p->work_xcds > 0);
  return rows_chunk(p, lens, hb, longest);
}

}  // namespace hexkv

extern "C" int hexkv_attend_plan_chunk(const hexkv_attend_params *p, const int32_t *lens, int32_t *chunk) {
  using namespace hexkv;
  clear_error();
  if (!chunk) return fail(HEXKV_EINVAL, "hexkv_attend_plan_chunk: null argument");
  const int c = plan_request(p, lens, "hexkv_attend_plan_chunk");
  if (c < 0) return c;
  *chunk = c;
  return HEXKV_OK;
}

extern "C" int hexkv_attend_plan_kernel(const hexkv_attend_params *p, const int32_t *lens, int32_t *kernel) {
  using namespace hexkv;
  clear_error();
  if (!kernel) return fail(HEXKV_EINVAL, "hexkv_attend_plan_kernel: null argument");
  const int c = plan_request(p, lens, "hexkv_attend_plan_kernel");
  if (c < 0) return c;
  if (p->kernel != HEXKV_KERNEL_AUTO) {
    *kernel = p->kernel;
    return HEXKV_OK;
  }
  *kernel = use_mfma(p, kernel_group(p->q_heads / p->kv_heads)) ? HEXKV_KERNEL_MFMA : HEXKV_KERNEL_VALU;
  if (rows_block(p) && p->work_xcds >= 1 && p->work_xcds <= 8) {
    // Bytes the call reads: every attended position of every KV head.
    int64_t positions = 0;
    const int extra = p->kv_new ? 1 : 0;
    for (int b = 0; b < p->batch; ++b) positions += static_cast<int64_t>(lens[b]) + p->seqlen_bias + extra;
    const int64_t bytes = positions * p->kv_heads * 2 * p->head_dim * elem_size(p->dtype);
    if (bytes >= (INT64_C(64) << 20)) *kernel = HEXKV_KERNEL_ROWS;
  }
  return HEXKV_OK;
}

namespace hexkv {

// The work list of a planning request, in launch order (see hexkv_attend_plan),
// and each (row, head group) segment's partition count.
static int build_plan(const hexkv_attend_params *p, const int32_t *lens, int64_t chunk,
                      std::vector<hexkv_work_item> &out, std::vector<int32_t> &seg_parts, int32_t *max_parts,
                      const char *what) {
  const int G = segment_heads(p);
  const int groups = p->q_heads / G;
  const int64_t segs = static_cast<int64_t>(p->batch) * groups;
  const int extra = p->kv_new ? 1 : 0;
  const int X = std::max(1, p->work_xcds);
  if (p->work_xcds < 0 || p->work_xcds > 64) return fail(HEXKV_EINVAL, "%s: work_xcds outside [0, 64]", what);
  if (p->work_xcds > 0 && segs > kCounterWords)
    return fail(HEXKV_EINVAL, "%s: the single-launch merge counts at most %lld segments", what,
                static_cast<long long>(kCounterWords));
  std::vector<int64_t> len(p->batch);
  int64_t count = 0, most = 1, full_rounds = 0;
  for (int b = 0; b < p->batch; ++b) {
    len[b] = static_cast<int64_t>(lens[b]) + p->seqlen_bias + extra;
    const int64_t k = len[b] == 0 ? 1 : (len[b] + chunk - 1) / chunk;
    count += k * groups;
    most = std::max(most, k);
    full_rounds = std::max(full_rounds, len[b] / chunk);
  }
  if (most > 65535 || count > INT32_MAX / 2) return fail(HEXKV_EUNSUPPORTED, "%s: more than 65535 partitions per row", what);
  *max_parts = static_cast<int32_t>(most);
  seg_parts.assign(static_cast<size_t>(segs), 0);
  for (int b = 0; b < p->batch; ++b)
    for (int hg = 0; hg < groups; ++hg)
      seg_parts[static_cast<size_t>(b) * groups + hg] = static_cast<int32_t>(len[b] == 0 ? 1 : (len[b] + chunk - 1) / chunk);

  const std::vector<int> home = segment_homes(len, groups, X);
  // Each XCD's items: empty rows (a zero output each), then the full chunks,
  // chunk index by chunk index across its segments, then every segment's
  // last, shorter chunk from the longest down, so its share ends on its
  // smallest items.
  std::vector<std::vector<hexkv_work_item>> lists(X);
  auto make = [&](int b, int hg, int64_t part, int64_t first, int64_t cnt) {
    hexkv_work_item it;
    it.row = b;
    it.head_group = hg;
    it.part = static_cast<int32_t>(part);
    it.parts = seg_parts[static_cast<size_t>(b) * groups + hg];
    it.first = static_cast<int32_t>(first);
    it.count = static_cast<int32_t>(cnt);
    it.len = static_cast<int32_t>(len[b]);
    it.heads = G;
    lists[home[static_cast<size_t>(b) * groups + hg]].push_back(it);
  };
  std::vector<std::pair<int64_t, int64_t>> tails;  // (positions, b * groups + hg)
  for (int b = 0; b < p->batch; ++b)
    for (int hg = 0; hg < groups; ++hg) {
      if (len[b] == 0) make(b, hg, 0, 0, 0);
      else if (len[b] % chunk) tails.emplace_back(len[b] % chunk, static_cast<int64_t>(b) * groups + hg);
    }
  for (int64_t c = 0; c < full_rounds; ++c)
    for (int b = 0; b < p->batch; ++b) {
      if ((c + 1) * chunk > len[b]) continue;
      for (int hg = 0; hg < groups; ++hg) make(b, hg, c, c * chunk, chunk);
    }
  std::stable_sort(tails.begin(), tails.end(),
                   [](const std::pair<int64_t, int64_t> &x, const std::pair<int64_t, int64_t> &y) { return x.first > y.first; });
  for (const auto &t : tails) {
    const int b = static_cast<int>(t.second / groups), hg = static_cast<int>(t.second % groups);
    const int64_t k = (len[b] + chunk - 1) / chunk;
    make(b, hg, k - 1, (k - 1) * chunk, t.first);
  }
  // XCD x's j-th item at index j * X + x; shorter lists padded with items
  // outside the call's geometry (row = batch), which the kernels skip.
  size_t longest = 0;
  for (const auto &l : lists) longest = std::max(longest, l.size());
  hexkv_work_item pad{};
  pad.row = p->batch;
  out.assign(longest * X, pad);
  for (int x = 0; x < X; ++x)
    for (size_t j = 0; j < lists[x].size(); ++j) out[j * X + x] = lists[x][j];
  if (X == 1 && static_cast<int64_t>(out.size()) != count)
    return fail(HEXKV_EINVAL, "%s: internal count mismatch %zu vs %lld", what, out.size(), static_cast<long long>(count));
  if (out.size() > static_cast<size_t>(INT32_MAX)) return fail(HEXKV_EUNSUPPORTED, "%s: work list too long", what);
  return HEXKV_OK;
}

}  // namespace hexkv

extern "C" int hexkv_attend_plan(const hexkv_attend_params *p, const int32_t *lens, hexkv_work_item *items,
                                 int32_t items_capacity, int32_t *parts, int32_t parts_capacity,
                                 int32_t *n_items, int32_t *max_parts) {
  using namespace hexkv;
  clear_error();
  const char *what = "hexkv_attend_plan";
  if (!n_items || !max_parts) return fail(HEXKV_EINVAL, "%s: null argument", what);
  const int chunk_or_error = plan_request(p, lens, what);
  if (chunk_or_error < 0) return chunk_or_error;
  std::vector<hexkv_work_item> list;
  std::vector<int32_t> seg_parts;
  int32_t most = 1;
  const int rc = build_plan(p, lens, chunk_or_error, list, seg_parts, &most, what);
  if (rc != HEXKV_OK) return rc;
  *n_items = static_cast<int32_t>(list.size());
  *max_parts = most;
  if (!items) return HEXKV_OK;  // a size query
  if (items_capacity < static_cast<int64_t>(list.size()) || !parts || parts_capacity < static_cast<int64_t>(seg_parts.size()))
    return fail(HEXKV_EINVAL, "%s: room for %d items and %d segment counts given, %zu and %zu needed", what,
                items_capacity, parts_capacity, list.size(), seg_parts.size());
  std::copy(list.begin(), list.end(), items);
  std::copy(seg_parts.begin(), seg_parts.end(), parts);
  return HEXKV_OK;
}

extern "C" size_t hexkv_attend_workspace_bytes(const hexkv_attend_params *p) {
  using namespace hexkv;
  if (!p || p->q_heads < 1 || p->kv_heads < 1 || p->q_heads % p->kv_heads || p->q_len < 1 ||
      p->batch < 0 || p->max_seqlen < 0)
    return 0;
  return workspace_bytes(p, choose_partition(p));
}

extern "C" int hexkv_attend_kernel(const hexkv_attend_params *p) {
  using namespace hexkv;
  clear_error();
  if (!p || p->q_heads < 1 || p->kv_heads < 1 || p->q_heads % p->kv_heads != 0)
    return fail(HEXKV_EINVAL, "hexkv_attend_kernel: bad q_heads/kv_heads");
  if (p->kernel < HEXKV_KERNEL_AUTO || p->kernel > HEXKV_KERNEL_ROWS)
    return fail(HEXKV_EINVAL, "hexkv_attend_kernel: unknown kernel %d", p->kernel);
  if (p->kernel == HEXKV_KERNEL_ROWS) return HEXKV_KERNEL_ROWS;
  return use_mfma(p, kernel_group(p->q_heads / p->kv_heads)) ? HEXKV_KERNEL_MFMA : HEXKV_KERNEL_VALU;
}

namespace hexkv {

// The launch behind hexkv_attend and hexkv_attend_noalloc: validated
// parameters, a workspace of ws_bytes bytes (device memory), one stream.
static int attend_launch(const hexkv_attend_params *p, void *workspace, size_t ws_bytes,
                         hexkv_stream_t stream, const char *what) {
  int rc = validate(p);
  if (rc != HEXKV_OK || p->batch == 0) return rc;
  const int part = choose_partition(p);
  const int G = kernel_group(p->q_heads / p->kv_heads);
  const int64_t max_parts = max_parts_of(p, part);
  const size_t need = workspace_bytes(p, part);
  if (need > 0 && (!workspace || ws_bytes < need))
    return fail(HEXKV_EWORKSPACE, "%s: workspace of %zu bytes needed, %zu given", what, need, ws_bytes);
  if (need > 0 && !aligned16(workspace))
    return fail(HEXKV_EINVAL, "%s: workspace must be 16-byte aligned", what);
  const int64_t rows = static_cast<int64_t>(p->batch) * p->q_len;

  AttendArgs a{};
  a.q = p->q;
  a.q_bs = p->q_batch_stride;
  a.q_rs = p->q_row_stride;
  a.cache = p->cache;
  a.c_bs = p->cache_batch_stride;
  a.c_ps = p->cache_pos_stride;
  a.c_kv = p->cache_kv_stride;
  a.out = p->out;
  a.o_bs = p->out_batch_stride;
  a.o_rs = p->out_row_stride;
  a.kv_new = p->kv_new;
  a.seqlens = p->seqlens_dev;
  a.bias = p->seqlen_bias;
  a.q_len = p->q_len;
  a.causal = p->causal ? 1 : 0;
  a.q_heads = p->q_heads;
  a.kv_heads = p->kv_heads;
  a.group = p->q_heads / p->kv_heads;
  a.part = part;
  a.max_parts = static_cast<int32_t>(max_parts);
  a.max_seqlen = p->max_seqlen;
  a.capacity = p->capacity;
  a.scale_log2 = p->softmax_scale * 1.4426950408889634f;
  a.ws_o = nullptr;
  a.ws_ml = nullptr;
  if (need > 0) {
    a.ws_o = reinterpret_cast<float *>(static_cast<char *>(workspace) + HEXKV_ATTEND_COUNTER_BYTES);
    a.ws_ml = a.ws_o + rows * p->q_heads * max_parts * p->head_dim;
  }
  const bool rows_kernel = p->kernel == HEXKV_KERNEL_ROWS;
  a.n_groups = p->q_heads / segment_heads(p);
  a.rows = static_cast<int32_t>(rows);
  a.items = p->work_items_dev;
  a.seg_parts = p->work_parts_dev;
  // Split segments of a list planned for the XCDs merge in the attention
  // kernel, counting arrivals in the workspace's counter words (the
  // row-block kernel's always: validate() holds it to such lists).
  a.seg_count = (a.items && p->work_xcds > 0 && p->work_xcds <= 8 && need > 0 && max_parts <= kMergeMaxParts &&
                 (rows_kernel || G * p->head_dim <= 4 * kAttThreads))
                    ? static_cast<uint64_t *>(workspace) : nullptr;
  a.n_xcd = p->work_xcds;
  a.xcd_remap = 0;
  if (a.items && p->work_xcds > 0) {
    int device_xcds = 1;
    if ((rc = stream_xcds(stream, &device_xcds, what)) != HEXKV_OK) return rc;
    // The in-kernel merge needs every item of a split segment on one XCD:
    // only a list dealt over this device's XCDs puts them there.
    if (a.seg_count && device_xcds != p->work_xcds)
      return fail(HEXKV_EINVAL, "%s: a work list planned for %d XCDs merges split rows on one XCD, and this "
                                "device has %d (hexkv_device_xcds)", what, p->work_xcds, device_xcds);
    a.xcd_remap = p->work_xcds > 1 && device_xcds % p->work_xcds == 0 && p->n_work_items % p->work_xcds == 0;
  }
  a.lengths_out = p->lengths_out_dev;
  // The status word, where a kernel may raise a flag: lengths read from
  // seqlens (clamped), XCD placement of a single-launch merge, work items
  // planned for another kernel.
  if ((a.seqlens || a.items) && (rc = status_word(stream, &a.status, what)) != HEXKV_OK)
    return rc;

  dim3 grid;
  if (a.items) {
    grid = dim3(static_cast<unsigned>(p->n_work_items));  // one workgroup per item, in list order
  } else {
    // Workgroups reach the 8 XCDs round-robin by linear index, and the later
    // partitions exist only in long rows.  With an even partition count the
    // same partition indices would always land on the same XCDs (measured
    // 1.6x slower at 32 than at 31); an odd count rotates them across the
    // XCDs from one (head group, row) to the next.  The extra column is empty.
    const unsigned grid_x = static_cast<unsigned>(max_parts | 1);
    grid = dim3(grid_x, static_cast<unsigned>(p->q_heads / G), static_cast<unsigned>(rows));
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (rows_kernel) {
    const int GQ = p->q_heads / p->kv_heads, HB = rows_block(p);
    rc = p->dtype == HEXKV_BF16 ? dispatch_rows<__bf16>(GQ, HB, a, grid, s) : dispatch_rows<_Float16>(GQ, HB, a, grid, s);
    if (rc != HEXKV_OK) return rc;
    return check_launch(what);
  }
  const int kind = use_mfma(p, G) ? kLaunchMfma : kLaunchValu;
  switch (p->dtype) {
    case HEXKV_BF16: rc = dispatch_d<__bf16>(p->head_dim, G, a, grid, kind, s); break;
    case HEXKV_F16: rc = dispatch_d<_Float16>(p->head_dim, G, a, grid, kind, s); break;
    default: rc = dispatch_d<float>(p->head_dim, G, a, grid, kind, s); break;
  }
  if (rc != HEXKV_OK) return rc;
  return check_launch(what);
}

// hexkv_attend_noalloc's workspace: one array per GPU the library runs on,
// held until the process ends.  Host code never passes `scratch` itself to a
// kernel (in host code the name is a stand-in, not a device address); it
// uses the per-device address hipGetSymbolAddress returns.  Like every
// file-scope variable it starts zero, so its arrival counters (the first
// HEXKV_ATTEND_COUNTER_BYTES, which every call leaves zero) need no clearing.
static __device__ __align__(256) unsigned char scratch[HEXKV_NOALLOC_SCRATCH_BYTES];
static std::atomic<void *> g_scratch_addr[kMaxDevices];

// Device address of `scratch` on the device that runs `stream` (the current
// device for the null stream), looked up once per device with that device
// current.
static int scratch_address(hexkv_stream_t stream, void **addr, const char *what) {
  return symbol_address(reinterpret_cast<const void *>(&HIP_SYMBOL(scratch)), g_scratch_addr, stream, addr, what);
}

}  // namespace hexkv

extern "C" int hexkv_attend(const hexkv_attend_params *p, void *workspace, size_t ws_bytes,
                            hexkv_stream_t stream) {
  hexkv::clear_error();
  return hexkv::attend_launch(p, workspace, ws_bytes, stream, "hexkv_attend");
}

extern "C" int hexkv_attend_noalloc(const hexkv_attend_params *p, hexkv_stream_t stream) {
  using namespace hexkv;
  clear_error();
  const char *what = "hexkv_attend_noalloc";
  int rc = validate(p);
  if (rc != HEXKV_OK || p->batch == 0) return rc;
  const size_t need = workspace_bytes(p, choose_partition(p));
  if (need > HEXKV_NOALLOC_SCRATCH_BYTES)
    return fail(HEXKV_EWORKSPACE,
                "%s: this call needs %zu bytes of split-K workspace, above the %u-byte static scratch "
                "(use hexkv_attend with a workspace, or fewer rows / a shorter max_seqlen)",
                what, need, static_cast<unsigned>(HEXKV_NOALLOC_SCRATCH_BYTES));
  void *ws = nullptr;
  if (need > 0 && (rc = scratch_address(stream, &ws, what)) != HEXKV_OK) return rc;
  return attend_launch(p, ws, need, stream, what);
}

// ------------------------------------------------------------ FT layout ---

namespace hexkv {

// The geometry of an FT call as hexkv_attend parameters (q_len 1, the VALU
// kernel, keys up to max_position + 1): partition, workspace and grid follow
// the same rules.
static hexkv_attend_params ft_geometry(const hexkv_ft_attend_params *p) {
  hexkv_attend_params g{};
  g.dtype = p->dtype;
  g.batch = p->batch;
  g.q_len = 1;
  g.q_heads = p->q_heads;
  g.kv_heads = p->kv_heads;
  g.head_dim = p->head_dim;
  g.softmax_scale = p->softmax_scale;
  g.capacity = p->capacity;
  g.max_seqlen = p->max_position + 1;
  g.partition = p->partition;
  g.kernel = HEXKV_KERNEL_VALU;
  return g;
}

static int validate_ft(const hexkv_ft_attend_params *p) {
  const char *what = "hexkv_ft_attend";
  if (!p) return fail(HEXKV_EINVAL, "%s: null params", what);
  if (p->dtype != HEXKV_F16 && p->dtype != HEXKV_BF16 && p->dtype != HEXKV_F32)
    return fail(HEXKV_EINVAL, "%s: unknown dtype %d", what, p->dtype);
  if (p->batch < 0 || p->q_heads < 1 || p->kv_heads < 1 || p->q_heads % p->kv_heads != 0)
    return fail(HEXKV_EINVAL, "%s: bad batch or head counts", what);
  const int d = p->head_dim;
  if (d != 16 && d != 32 && d != 64 && d != 128 && d != 256)
    return fail(HEXKV_EUNSUPPORTED, "%s: head_dim %d (compiled: 16, 32, 64, 128, 256)", what, d);
  if (p->batch > 65535) return fail(HEXKV_EINVAL, "%s: batch above 65535", what);
  if (p->capacity < 1 || p->max_position < 0 || p->max_position >= p->capacity)
    return fail(HEXKV_ERANGE, "%s: max_position %d outside [0, capacity %lld)", what, p->max_position,
                static_cast<long long>(p->capacity));
  if (p->rotary_dim < 0 || p->rotary_dim > d || p->rotary_dim % 2 != 0)
    return fail(HEXKV_EINVAL, "%s: rotary_dim %d must be even and at most head_dim", what, p->rotary_dim);
  if (p->rotary_dim > 0 && !(p->rotary_base > 0.f && p->rotary_base < 3.0e38f))
    return fail(HEXKV_EINVAL, "%s: rotary_base must be positive and finite", what);
  if (!(p->softmax_scale > 0.f) || p->softmax_scale > 3.0e38f)
    return fail(HEXKV_EINVAL, "%s: softmax_scale must be positive and finite", what);
  if (p->partition < 0 || (p->partition > 0 && (p->partition % 64 != 0 || p->partition > 4096)))
    return fail(HEXKV_EINVAL, "%s: partition must be 0 or a multiple of 64 up to 4096", what);
  if (p->batch == 0) return HEXKV_OK;
  if (!p->q || !p->k_new || !p->v_new || !p->k_cache || !p->v_cache || !p->out)
    return fail(HEXKV_EINVAL, "%s: null tensor", what);
  const int es = elem_size(p->dtype), vec = 16 / es;
  if (!aligned16(p->q) || !aligned16(p->k_new) || !aligned16(p->v_new) || !aligned16(p->k_cache) ||
      !aligned16(p->v_cache))
    return fail(HEXKV_EINVAL, "%s: q, k_new, v_new and the caches must be 16-byte aligned", what);
  if (p->q_batch_stride % vec || p->new_batch_stride % vec)
    return fail(HEXKV_EINVAL, "%s: strides must be multiples of 16 bytes", what);
  if ((reinterpret_cast<uintptr_t>(p->out) & (es - 1)) != 0) return fail(HEXKV_EINVAL, "%s: out misaligned", what);
  // K chunks and V rows of one (sequence, head) are addressed by 32-bit offsets.
  if (p->capacity > (INT64_C(1) << 31) / (static_cast<int64_t>(d) * es))
    return fail(HEXKV_EUNSUPPORTED, "%s: capacity * head_dim * element above 2 GiB", what);
  return HEXKV_OK;
}

}  // namespace hexkv

extern "C" size_t hexkv_ft_attend_workspace_bytes(const hexkv_ft_attend_params *p) {
  using namespace hexkv;
  if (!p || p->q_heads < 1 || p->kv_heads < 1 || p->q_heads % p->kv_heads || p->batch < 0 ||
      p->max_position < 0)
    return 0;
  const hexkv_attend_params g = ft_geometry(p);
  return workspace_bytes(&g, choose_partition(&g));
}

extern "C" int hexkv_ft_attend(const hexkv_ft_attend_params *p, void *workspace, size_t ws_bytes,
                               hexkv_stream_t stream) {
  using namespace hexkv;
  clear_error();
  int rc = validate_ft(p);
  if (rc != HEXKV_OK || p->batch == 0) return rc;
  const hexkv_attend_params g = ft_geometry(p);
  const int part = choose_partition(&g);
  const int G = kernel_group(p->q_heads / p->kv_heads);
  const int64_t max_parts = max_parts_of(&g, part);
  const size_t need = workspace_bytes(&g, part);
  if (need > 0 && (!workspace || ws_bytes < need))
    return fail(HEXKV_EWORKSPACE, "hexkv_ft_attend: workspace of %zu bytes needed, %zu given", need, ws_bytes);
  if (need > 0 && !aligned16(workspace))
    return fail(HEXKV_EINVAL, "hexkv_ft_attend: workspace must be 16-byte aligned");
  const int64_t rows = p->batch;
  const int64_t es = elem_size(p->dtype), d = p->head_dim, cap = p->capacity;

  AttendArgs a{};
  a.q = p->q;
  a.q_bs = p->q_batch_stride;
  a.out = p->out;
  a.o_bs = p->out_batch_stride;
  a.kv_new = p->k_new;
  a.v_new = p->v_new;
  a.new_bs = p->new_batch_stride;
  a.seqlens = p->positions_dev;
  a.bias = p->position_bias;
  a.q_len = 1;
  a.q_heads = p->q_heads;
  a.kv_heads = p->kv_heads;
  a.group = p->q_heads / p->kv_heads;
  a.part = part;
  a.max_parts = static_cast<int32_t>(max_parts);
  a.max_seqlen = p->max_position + 1;
  a.capacity = cap;
  a.scale_log2 = p->softmax_scale * 1.4426950408889634f;
  if (need > 0) {
    a.ws_o = reinterpret_cast<float *>(static_cast<char *>(workspace) + HEXKV_ATTEND_COUNTER_BYTES);
    a.ws_ml = a.ws_o + rows * p->q_heads * max_parts * p->head_dim;
  }
  a.rows = static_cast<int32_t>(rows);
  a.n_groups = p->q_heads / G;
  a.k_ft = p->k_cache;
  a.v_ft = p->v_cache;
  a.k_ft_head = d * cap * es;  // D / pack chunks of capacity x 16 bytes
  a.k_ft_batch = p->kv_heads * a.k_ft_head;
  a.k_ft_chunk = cap * 16;
  a.v_ft_head = cap * d * es;
  a.v_ft_batch = p->kv_heads * a.v_ft_head;
  a.rot_dim = p->rotary_dim;
  a.rot_neox = p->rotary_neox ? 1 : 0;
  a.rot_log2_base = p->rotary_dim > 0 ? log2(static_cast<double>(p->rotary_base)) : 0.0;
  if (p->positions_dev && (rc = status_word(stream, &a.status, "hexkv_ft_attend")) != HEXKV_OK) return rc;

  const unsigned grid_x = static_cast<unsigned>(max_parts | 1);  // odd: see hexkv_attend
  dim3 grid(grid_x, static_cast<unsigned>(p->q_heads / G), static_cast<unsigned>(rows));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (p->dtype) {
    case HEXKV_BF16: rc = dispatch_d<__bf16>(p->head_dim, G, a, grid, kLaunchFt, s); break;
    case HEXKV_F16: rc = dispatch_d<_Float16>(p->head_dim, G, a, grid, kLaunchFt, s); break;
    default: rc = dispatch_d<float>(p->head_dim, G, a, grid, kLaunchFt, s); break;
  }
  if (rc != HEXKV_OK) return rc;
  return check_launch("hexkv_ft_attend");
}
