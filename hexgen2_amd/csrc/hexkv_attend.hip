// Single-query GQA decode attention over the KV cache, with optional fused
// append of the new token's K/V (hexkv_attend in hexkv.h).
//
// Work decomposition (split-K, "flash-decoding"):
//   grid = (partition, q-head group, query row).  A workgroup (4 waves) owns
//   `part` consecutive cache positions of one sequence for G query heads that
//   share one KV head, so every K/V byte is read by exactly one workgroup.
//   Ragged lengths only change how many partitions a row has; every
//   partition but the last is full, so work per workgroup is uniform.
//
// Inside a workgroup, per partition:
//   1. scores: lanes are grouped LPP = D*elem/16 per position; each lane
//      loads one 16-byte slice of a K row (coalesced: a group reads the whole
//      D-wide row) and dots it with its slice of the G query vectors held in
//      registers (v_dot2_f32_{bf16,f16} for 16-bit types).  The LPP partial
//      sums are combined with DPP lane moves and the scaled score (log2
//      domain) goes to LDS as scores[p][G];
//   2. softmax: workgroup max per head, exp2 in place in LDS, sum per head;
//   3. values: the same lane mapping loads V slices and accumulates
//      p * V in fp32 registers (G x 8 accumulators per lane); lane groups and
//      waves are then reduced through LDS.
//   K/V go straight from HBM to VGPRs with nontemporal loads: each byte is
//   consumed by exactly one lane, so staging them in LDS would add LDS traffic
//   without any reuse.  LDS holds what is shared: the score tile.
// A row with one partition writes its normalised output directly; otherwise
// each partition writes (unnormalised o, max, sum) to the workspace and
// `combine_kernel` merges them.
#include "hexkv_common.h"

#include <algorithm>

namespace hexkv {

constexpr int kAttThreads = 256;
constexpr int kAttWaves = kAttThreads / 64;

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
  float scale_log2;  // softmax_scale * log2(e)
  float *ws_o;       // [rows][q_heads][max_parts][D]
  float *ws_ml;      // [rows][q_heads][max_parts][2]
};

// Number of keys query row (b, t) attends to; *pos_new = cache position of the
// fused-append row (or -1).
__device__ __forceinline__ int row_length(const AttendArgs &a, int b, int t, int *pos_new) {
  int len = (a.seqlens ? a.seqlens[b] : 0) + a.bias;
  *pos_new = -1;
  if (a.kv_new) {
    *pos_new = len;
    len += 1;
  }
  if (a.causal) len = len - a.q_len + t + 1;
  // Lengths come from device memory: clamp to the host bound that sized the
  // grid and the workspace (max_seqlen <= capacity is checked on the host),
  // so no row can reach past either.
  if (len > a.max_seqlen) len = a.max_seqlen;
  return len;
}

template <typename T, int D, int G>
__global__ __launch_bounds__(kAttThreads) void attend_kernel(const AttendArgs a) {
  using E = Elem<T>;
  constexpr int VEC = 16 / static_cast<int>(sizeof(T));  // elements per 16-byte slice
  constexpr int LPP = D / VEC;                           // lanes per position
  static_assert(LPP >= 1 && LPP <= 64, "head_dim does not map onto a wave");
  constexpr int PPW = 64 / LPP;          // positions per wave per load
  constexpr int PPI = PPW * kAttWaves;   // positions per workgroup per load
  constexpr int U = 4;                   // loads in flight per lane
  extern __shared__ float smem[];        // scores [part][G]; later [waves][G][D]
  __shared__ float s_red[kAttWaves][G];
  __shared__ float s_m[G], s_l[G];

  const int row = blockIdx.z;
  const int b = row / a.q_len, t = row - b * a.q_len;
  int pos_new;
  const int len = row_length(a, b, t, &pos_new);
  const int part = blockIdx.x;
  const int p0 = part * a.part;
  const int qh0 = blockIdx.y * G;
  T *out_row = static_cast<T *>(a.out) + b * a.o_bs + t * a.o_rs + qh0 * D;
  if (len <= 0) {  // nothing to attend to: defined zero output
    if (part == 0)
      for (int i = threadIdx.x; i < G * D; i += kAttThreads) out_row[i] = E::from_float(0.f);
    return;
  }
  if (p0 >= len) return;
  const int n = min(a.part, len - p0);
  const int nparts = (len + a.part - 1) / a.part;
  const int hk = qh0 / a.group;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int sub = lane % LPP, grp = lane / LPP;
  const int slot = w * PPW + grp;  // position of this lane within a PPI tile

  const T *qrow = static_cast<const T *>(a.q) + b * a.q_bs + t * a.q_rs + qh0 * D + sub * VEC;
  u32x4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qv[g] = *reinterpret_cast<const u32x4 *>(qrow + g * D);

  T *kbase = const_cast<T *>(static_cast<const T *>(a.cache)) + b * a.c_bs + hk * D + sub * VEC;
  T *vbase = kbase + a.c_kv;
  const T *knew = a.kv_new
      ? static_cast<const T *>(a.kv_new) + (static_cast<int64_t>(b) * 2 * a.kv_heads + hk) * D + sub * VEC
      : nullptr;
  const T *vnew = knew ? knew + a.kv_heads * D : nullptr;
  // The fused-append row is read from kv_new (never from the cache) and
  // written to the cache by the lanes that load it; K by phase 1, V by
  // phase 3, of the one workgroup per (row, head group) owning position
  // pos_new.  Head groups sharing a KV head (G < group) all hold the same
  // bytes; only the first writes.
  const bool writer = (qh0 % a.group) == 0;

  // ---- phase 1: scores -----------------------------------------------------
  float mx[G];
#pragma unroll
  for (int g = 0; g < G; ++g) mx[g] = -INFINITY;
  for (int i0 = 0; i0 < n; i0 += PPI * U) {
    u32x4 kr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = i0 + u * PPI + slot;
      const int s = p0 + p;
      kr[u] = u32x4{0u, 0u, 0u, 0u};
      if (p < n) {
        if (s == pos_new) kr[u] = *reinterpret_cast<const u32x4 *>(knew);
        else kr[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(kbase + s * a.c_ps));
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = i0 + u * PPI + slot;
      float sc[G];
#pragma unroll
      for (int g = 0; g < G; ++g) sc[g] = group_sum<LPP>(E::dot(qv[g], kr[u], 0.f)) * a.scale_log2;
      if (p < n) {
#pragma unroll
        for (int g = 0; g < G; ++g) mx[g] = fmaxf(mx[g], sc[g]);
        if (sub == 0) {
#pragma unroll
          for (int g = 0; g < G; ++g) smem[p * G + g] = sc[g];
        }
        if (p0 + p == pos_new && writer)
          *reinterpret_cast<u32x4 *>(kbase + static_cast<int64_t>(pos_new) * a.c_ps) = kr[u];
      }
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float m = wave_max(mx[g]);
    if (lane == 0) s_red[w][g] = m;
  }
  __syncthreads();
  if (tid < G) {
    float m = s_red[0][tid];
#pragma unroll
    for (int i = 1; i < kAttWaves; ++i) m = fmaxf(m, s_red[i][tid]);
    s_m[tid] = m;
  }
  __syncthreads();

  // ---- phase 2: exponentiate in place, sum per head -----------------------
  {
    const int g = tid % G;  // G divides 256: a thread always sees one head
    const float m = s_m[g];
    float l = 0.f;
    for (int i = tid; i < n * G; i += kAttThreads) {
      const float e = exp2f(smem[i] - m);
      smem[i] = e;
      l += e;
    }
#pragma unroll
    for (int off = 32; off >= G; off >>= 1) l += __shfl_xor(l, off);
    if (lane < G) s_red[w][lane] = l;
  }
  __syncthreads();
  if (tid < G) {
    float l = 0.f;
#pragma unroll
    for (int i = 0; i < kAttWaves; ++i) l += s_red[i][tid];
    s_l[tid] = l;
  }
  // (s_l is read only after the barrier that follows phase 3.)

  // ---- phase 3: o = sum_p e_p * V_p ---------------------------------------
  float acc[G][VEC];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[g][e] = 0.f;
  for (int i0 = 0; i0 < n; i0 += PPI * U) {
    u32x4 vr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = i0 + u * PPI + slot;
      const int s = p0 + p;
      vr[u] = u32x4{0u, 0u, 0u, 0u};
      if (p < n) {
        if (s == pos_new) vr[u] = *reinterpret_cast<const u32x4 *>(vnew);
        else vr[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(vbase + s * a.c_ps));
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = i0 + u * PPI + slot;
      if (p < n) {
        float pr[G];
#pragma unroll
        for (int g = 0; g < G; ++g) pr[g] = smem[p * G + g];
        float vf[VEC];
        E::to_float(vr[u], vf);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[g][e] = fmaf(pr[g], vf[e], acc[g][e]);
        if (p0 + p == pos_new && writer)
          *reinterpret_cast<u32x4 *>(vbase + static_cast<int64_t>(pos_new) * a.c_ps) = vr[u];
      }
    }
  }
  // Reduce over the PPW lane groups of each wave (lanes with equal `sub`).
#pragma unroll
  for (int off = LPP; off < 64; off <<= 1)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[g][e] += __shfl_xor(acc[g][e], off);
  __syncthreads();  // all score reads done: smem becomes [waves][G][D]
  if (grp == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < VEC; ++e) smem[(w * G + g) * D + sub * VEC + e] = acc[g][e];
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += kAttThreads) {
    float o = 0.f;
#pragma unroll
    for (int ww = 0; ww < kAttWaves; ++ww) o += smem[ww * G * D + i];
    const int g = i / D, d = i - g * D;
    if (nparts == 1) {
      out_row[i] = E::from_float(o / s_l[g]);
    } else {
      const int64_t slot_idx = (static_cast<int64_t>(row) * a.q_heads + qh0 + g) * a.max_parts + part;
      a.ws_o[slot_idx * D + d] = o;
      if (d == 0) {
        a.ws_ml[slot_idx * 2] = s_m[g];
        a.ws_ml[slot_idx * 2 + 1] = s_l[g];
      }
    }
  }
}

// Merges the partitions of one (query row, q head): o = sum_p w_p o_p / sum_p
// w_p l_p with w_p = 2^(m_p - max m).
template <typename T>
__global__ __launch_bounds__(64) void combine_kernel(const AttendArgs a, int D) {
  using E = Elem<T>;
  const int h = blockIdx.x, row = blockIdx.y;
  const int b = row / a.q_len, t = row - b * a.q_len;
  int pos_new;
  const int len = row_length(a, b, t, &pos_new);
  if (len <= 0) return;
  const int nparts = (len + a.part - 1) / a.part;
  if (nparts <= 1) return;
  const int64_t base = (static_cast<int64_t>(row) * a.q_heads + h) * a.max_parts;
  const float *ml = a.ws_ml + base * 2;
  float m = -INFINITY;
  for (int p = 0; p < nparts; ++p) m = fmaxf(m, ml[2 * p]);
  float l = 0.f;
  for (int p = 0; p < nparts; ++p) l += exp2f(ml[2 * p] - m) * ml[2 * p + 1];
  const float inv = 1.f / l;
  T *out = static_cast<T *>(a.out) + b * a.o_bs + t * a.o_rs + static_cast<int64_t>(h) * D;
  const float *o = a.ws_o + base * D;
  for (int d = threadIdx.x; d < D; d += 64) {
    float acc = 0.f;
    for (int p = 0; p < nparts; ++p) acc += exp2f(ml[2 * p] - m) * o[p * D + d];
    out[d] = E::from_float(acc * inv);
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

static int choose_partition(const hexkv_attend_params *p) {
  if (p->partition > 0) return p->partition;
  const int64_t rows = static_cast<int64_t>(p->batch) * p->q_len;
  const int64_t groups = p->q_heads / kernel_group(p->q_heads / p->kv_heads);
  const int64_t target = 1024;  // >= 4 workgroups per CU on a 256-CU part
  for (int part = 1024; part >= 64; part >>= 1) {
    const int64_t parts = (p->max_seqlen + part - 1) / part;
    if (rows * groups * parts >= target) return part;
  }
  return 64;
}

static size_t workspace_bytes(const hexkv_attend_params *p, int part) {
  const int64_t max_parts = (p->max_seqlen + part - 1) / part;
  if (max_parts <= 1) return 0;
  const int64_t rows = static_cast<int64_t>(p->batch) * p->q_len;
  return static_cast<size_t>(rows * p->q_heads * max_parts * (p->head_dim + 2)) * sizeof(float);
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
  if (p->partition < 0 || (p->partition > 0 && (p->partition % 64 != 0 || p->partition > 4096)))
    return fail(HEXKV_EINVAL, "hexkv_attend: partition must be 0 or a multiple of 64 up to 4096");
  if (p->batch == 0) return HEXKV_OK;
  if (!p->q || !p->cache || !p->out) return fail(HEXKV_EINVAL, "hexkv_attend: null tensor");
  const int vec = 16 / elem_size(p->dtype);
  if (!aligned16(p->q) || !aligned16(p->cache) || (p->kv_new && !aligned16(p->kv_new)))
    return fail(HEXKV_EINVAL, "hexkv_attend: q/cache/kv_new must be 16-byte aligned");
  if (p->q_batch_stride % vec || p->q_row_stride % vec || p->cache_batch_stride % vec ||
      p->cache_pos_stride % vec || p->cache_kv_stride % vec)
    return fail(HEXKV_EINVAL, "hexkv_attend: strides must be multiples of 16 bytes");
  if ((reinterpret_cast<uintptr_t>(p->out) & (elem_size(p->dtype) - 1)) != 0)
    return fail(HEXKV_EINVAL, "hexkv_attend: out misaligned");
  return HEXKV_OK;
}

template <typename T, int D, int G>
static void launch(const AttendArgs &a, dim3 grid, size_t smem, hipStream_t s) {
  attend_kernel<T, D, G><<<grid, kAttThreads, smem, s>>>(a);
}

template <typename T, int D>
static int dispatch_g(int G, const AttendArgs &a, dim3 grid, size_t smem, hipStream_t s) {
  switch (G) {
    case 1: launch<T, D, 1>(a, grid, smem, s); break;
    case 2: launch<T, D, 2>(a, grid, smem, s); break;
    case 4: launch<T, D, 4>(a, grid, smem, s); break;
    case 8: launch<T, D, 8>(a, grid, smem, s); break;
    default: return fail(HEXKV_EUNSUPPORTED, "hexkv_attend: group %d", G);
  }
  return HEXKV_OK;
}

template <typename T>
static int dispatch_d(int D, int G, const AttendArgs &a, dim3 grid, size_t smem, hipStream_t s) {
  switch (D) {
    case 16: return dispatch_g<T, 16>(G, a, grid, smem, s);
    case 32: return dispatch_g<T, 32>(G, a, grid, smem, s);
    case 64: return dispatch_g<T, 64>(G, a, grid, smem, s);
    case 128: return dispatch_g<T, 128>(G, a, grid, smem, s);
    case 256: return dispatch_g<T, 256>(G, a, grid, smem, s);
    default: return fail(HEXKV_EUNSUPPORTED, "hexkv_attend: head_dim %d", D);
  }
}

}  // namespace hexkv

extern "C" size_t hexkv_attend_workspace_bytes(const hexkv_attend_params *p) {
  using namespace hexkv;
  if (!p || p->q_heads < 1 || p->kv_heads < 1 || p->q_heads % p->kv_heads) return 0;
  return workspace_bytes(p, choose_partition(p));
}

extern "C" int hexkv_attend(const hexkv_attend_params *p, void *workspace, size_t ws_bytes,
                            hexkv_stream_t stream) {
  using namespace hexkv;
  clear_error();
  int rc = validate(p);
  if (rc != HEXKV_OK || p->batch == 0) return rc;
  const int part = choose_partition(p);
  const int G = kernel_group(p->q_heads / p->kv_heads);
  const int max_parts = std::max(1, (p->max_seqlen + part - 1) / part);
  const size_t need = workspace_bytes(p, part);
  if (need > 0 && (!workspace || ws_bytes < need))
    return fail(HEXKV_EWORKSPACE, "hexkv_attend: workspace of %zu bytes needed, %zu given", need,
                ws_bytes);
  if (need > 0 && !aligned16(workspace))
    return fail(HEXKV_EINVAL, "hexkv_attend: workspace must be 16-byte aligned");
  const int64_t rows = static_cast<int64_t>(p->batch) * p->q_len;

  AttendArgs a;
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
  a.max_parts = max_parts;
  a.max_seqlen = p->max_seqlen;
  a.capacity = p->capacity;
  a.scale_log2 = p->softmax_scale * 1.4426950408889634f;
  a.ws_o = static_cast<float *>(workspace);
  const int64_t slots = rows * p->q_heads * max_parts;
  a.ws_ml = need > 0 ? a.ws_o + slots * p->head_dim : nullptr;

  dim3 grid(static_cast<unsigned>(max_parts), static_cast<unsigned>(p->q_heads / G),
            static_cast<unsigned>(rows));
  const size_t smem = sizeof(float) * std::max<size_t>(static_cast<size_t>(part) * G,
                                                       static_cast<size_t>(kAttWaves) * G * p->head_dim);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (p->dtype) {
    case HEXKV_BF16: rc = dispatch_d<__bf16>(p->head_dim, G, a, grid, smem, s); break;
    case HEXKV_F16: rc = dispatch_d<_Float16>(p->head_dim, G, a, grid, smem, s); break;
    default: rc = dispatch_d<float>(p->head_dim, G, a, grid, smem, s); break;
  }
  if (rc != HEXKV_OK) return rc;
  rc = check_launch("hexkv_attend");
  if (rc != HEXKV_OK || max_parts <= 1) return rc;
  dim3 cgrid(static_cast<unsigned>(p->q_heads), static_cast<unsigned>(rows));
  switch (p->dtype) {
    case HEXKV_BF16: combine_kernel<__bf16><<<cgrid, 64, 0, s>>>(a, p->head_dim); break;
    case HEXKV_F16: combine_kernel<_Float16><<<cgrid, 64, 0, s>>>(a, p->head_dim); break;
    default: combine_kernel<float><<<cgrid, 64, 0, s>>>(a, p->head_dim); break;
  }
  return check_launch("hexkv_attend(combine)");
}
