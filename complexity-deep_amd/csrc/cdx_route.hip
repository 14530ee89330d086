// Routing plan for the token-routed MoE on gfx950 (piece 1a of the hot path).
//
// Reference behaviour: core/token_routed_mlp.py:149-150 (expert = map[clamp(id)]),
// :166-170 (mask dispatch, i.e. a stable partition by expert id) and the operator
// API cuda/triton_token_routed.py:37-61 (counts = bincount, offsets = [0, cumsum]).
//
// Design: a stable counting sort in two launches, bit-exact and deterministic.
// Tokens are split into at most kMaxBlocks blocks of tpb consecutive tokens (tpb a
// multiple of 1024, the smallest that keeps the block count within kMaxBlocks); a
// block walks its tokens in rounds of 1024 = 16 chunks of 64, one chunk per wave.
//   1. count:   each block looks up the expert of its tokens (written to expert_id)
//               and, per chunk and expert, takes a 64-bit ballot; the popcounts summed
//               in LDS (integer adds: order-free) are the block's per-expert totals,
//               written to row [block][E] of a small count table.
//   2. scatter: every block reads the whole count table (at most kMaxBlocks x E ints)
//               and derives, per expert, the total (hence counts and offsets; block 0
//               writes them) and the tokens of earlier blocks (its base).  It then
//               recomputes its ballots round by round: a token's sorted position is
//               base[e] + (tokens of e in earlier chunks) + popcount(ballot & lanes
//               below).  Token order inside an expert is the original index order,
//               which is exactly argsort(expert, stable=True).
// The count table is the only scratch: caller workspace (cdx_route_plan) or a
// library-owned device array (cdx_route_plan_noalloc).  Nothing needs zeroing: the
// count launch writes every entry the scatter launch reads.
// cdx_route_plans runs L plans over the same ids, one per expert map (a model's
// layers each route through their own map), in the same two launches: the plan
// index is blockIdx.y, and every output and the count table gain a leading [L] axis.
#include <mutex>

#include "cdx_common.h"

namespace cdx {
namespace {

constexpr int kRound = 1024;                 // tokens per round of a block
constexpr int kChunks = kRound / kWave;      // 16 chunks of 64
constexpr int kMaxE = 64;
constexpr int kMaxBlocks = 256;
constexpr int kScratchInts = kMaxBlocks * kMaxE;  // 64 KB: the largest count table
// Plans per launch of cdx_route_plans (blockIdx.y); the maps travel in the kernel
// arguments (1 KB), so that the host never copies a pointer table to the device.
constexpr int kMaxMaps = 128;
struct MapSet {
  const int64_t* m[kMaxMaps];
};

// Tokens per block: a multiple of kRound such that the block count is <= kMaxBlocks.
inline int64_t tokens_per_block(int64_t T) {
  const int64_t rounds = (T + (int64_t)kRound * kMaxBlocks - 1) / ((int64_t)kRound * kMaxBlocks);
  return kRound * (rounds < 1 ? 1 : rounds);
}

__device__ __forceinline__ int lookup_expert(const int64_t* ids, const int64_t* map, int64_t V,
                                             int E, int64_t t) {
  int64_t id = ids[t];
  int64_t e;
  if (map != nullptr) {
    id = id < 0 ? 0 : (id > V - 1 ? V - 1 : id);
    e = map[id];
  } else {
    e = id;
  }
  // Out-of-range expert ids only arise from a corrupt map; clamp to stay in bounds.
  e = e < 0 ? 0 : (e > E - 1 ? E - 1 : e);
  return (int)e;
}

// Plan y = blockIdx.y routes through maps.m[y] and writes expert_id[y T ..] and its
// count table rows [y nblk ..].
__global__ __launch_bounds__(256) void route_count_kernel(const int64_t* __restrict__ ids, const MapSet maps,
                                                          int64_t V, int E, int64_t T, int64_t tpb,
                                                          int32_t* __restrict__ expert_id,
                                                          int32_t* __restrict__ blk_counts) {
  __shared__ int cnt[kMaxE];
  const int64_t* map = maps.m[blockIdx.y];
  expert_id += (int64_t)blockIdx.y * T;
  blk_counts += (int64_t)blockIdx.y * gridDim.x * E;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (threadIdx.x < E) cnt[threadIdx.x] = 0;
  __syncthreads();
  const int64_t b0 = (int64_t)blockIdx.x * tpb;
  const int64_t b1 = min(T, b0 + tpb);
  for (int64_t r0 = b0; r0 < b1; r0 += kRound) {
    // The four chunks of a wave: lookups first (independent loads in flight), then
    // the ballots.
    int ev[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t t = r0 + (wave * 4 + j) * kWave + lane;
      ev[j] = t < b1 ? lookup_expert(ids, map, V, E, t) : -1;
      if (t < b1) expert_id[t] = ev[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      for (int x = 0; x < E; ++x) {
        const uint64_t m = __ballot(ev[j] == x);
        if (lane == 0 && m) atomicAdd(&cnt[x], __popcll(m));
      }
  }
  __syncthreads();
  if (threadIdx.x < E) blk_counts[(int64_t)blockIdx.x * E + threadIdx.x] = cnt[threadIdx.x];
}

__global__ __launch_bounds__(256) void route_scatter_kernel(const int32_t* __restrict__ expert_id, int E,
                                                            int64_t T, int64_t tpb, int nblk,
                                                            const int32_t* __restrict__ blk_counts,
                                                            int32_t* __restrict__ perm, int32_t* __restrict__ inv_perm,
                                                            int32_t* __restrict__ counts,
                                                            int32_t* __restrict__ offsets) {
  __shared__ int cnt[kChunks][kMaxE];
  __shared__ int pre[kChunks][kMaxE];
  __shared__ int total[kMaxE];
  __shared__ int base[kMaxE];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int blk = blockIdx.x;
  // Plan blockIdx.y: its rows of every output and of the count table.
  const int64_t y = blockIdx.y;
  expert_id += y * T;
  perm += y * T;
  inv_perm += y * T;
  counts += y * E;
  offsets += y * (E + 1);
  blk_counts += y * nblk * E;

  // Per expert: all blocks' tokens (total) and those of blocks before this one.
  for (int x = wave; x < E; x += 4) {
    int tot = 0, before = 0;
    for (int b = lane; b < nblk; b += kWave) {
      const int v = blk_counts[(int64_t)b * E + x];
      tot += v;
      before += b < blk ? v : 0;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      tot += __shfl_xor(tot, off, 64);
      before += __shfl_xor(before, off, 64);
    }
    if (lane == 0) {
      total[x] = tot;
      base[x] = before;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int x = 0; x < E; ++x) {
      if (blk == 0) {
        counts[x] = total[x];
        offsets[x] = run;
      }
      base[x] += run;
      run += total[x];
    }
    if (blk == 0) offsets[E] = run;
  }
  __syncthreads();

  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t b0 = (int64_t)blk * tpb;
  const int64_t b1 = min(T, b0 + tpb);
  for (int64_t r0 = b0; r0 < b1; r0 += kRound) {
    int my_e[4], my_rank[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t t = r0 + (wave * 4 + j) * kWave + lane;
      my_e[j] = t < b1 ? expert_id[t] : -1;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = wave * 4 + j;
      int rank = 0;
      for (int x = 0; x < E; ++x) {
        const uint64_t m = __ballot(my_e[j] == x);
        if (my_e[j] == x) rank = __popcll(m & below);
        if (lane == 0) cnt[c][x] = __popcll(m);
      }
      my_rank[j] = rank;
    }
    __syncthreads();
    for (int x = threadIdx.x; x < E; x += blockDim.x) {
      int s = base[x];
#pragma unroll
      for (int c = 0; c < kChunks; ++c) {
        pre[c][x] = s;
        s += cnt[c][x];
      }
      base[x] = s;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t t = r0 + (wave * 4 + j) * kWave + lane;
      if (t < b1) {
        const int pos = pre[wave * 4 + j][my_e[j]] + my_rank[j];
        perm[pos] = (int32_t)t;
        inv_perm[t] = pos;
      }
    }
    __syncthreads();  // cnt / pre are rewritten by the next round
  }
}

// Both launches of L <= kMaxMaps plans over the same ids (plan y through maps[y],
// outputs at row y of each [L, ...] array); blk_counts holds L * nblk * E ints.
int route_plan_launch(const int64_t* ids, int64_t T, const int64_t* const* maps, int32_t L, int64_t V, int32_t E,
                      int32_t* expert_id, int32_t* perm, int32_t* inv_perm, int32_t* counts, int32_t* offsets,
                      int32_t* blk_counts, hipStream_t s, const char* name) {
  const int64_t tpb = tokens_per_block(T);
  const int nblk = (int)((T + tpb - 1) / tpb);
  MapSet ms{};
  for (int y = 0; y < L; ++y) ms.m[y] = maps[y];
  if (nblk > 0) {
    route_count_kernel<<<dim3((unsigned)nblk, (unsigned)L), dim3(256), 0, s>>>(ids, ms, V, E, T, tpb, expert_id,
                                                                                blk_counts);
    if (int rc = check_launch(name)) return rc;
  }
  // At least one block per plan: with T == 0 it writes the zero counts and offsets.
  route_scatter_kernel<<<dim3((unsigned)(nblk > 0 ? nblk : 1), (unsigned)L), dim3(256), 0, s>>>(
      expert_id, E, T, tpb, nblk, blk_counts, perm, inv_perm, counts, offsets);
  return check_launch(name);
}

int route_plan_check(const int64_t* ids, int64_t T, const int64_t* map, int64_t V, int32_t E, int32_t* expert_id,
                     int32_t* perm, int32_t* inv_perm, int32_t* counts, int32_t* offsets, const char* name) {
  if (T < 0 || T > INT32_MAX) return fail(CDX_EINVAL, "%s: T=%lld out of range", name, (long long)T);
  if (E <= 0 || E > kMaxE) return fail(CDX_EUNSUPPORTED, "%s: E=%d must be in [1, %d]", name, E, kMaxE);
  if (map != nullptr && V <= 0) return fail(CDX_EINVAL, "%s: V=%lld must be > 0", name, (long long)V);
  if (!counts || !offsets) return fail(CDX_EINVAL, "%s: null counts/offsets", name);
  if (T > 0 && (!ids || !expert_id || !perm || !inv_perm))
    return fail(CDX_EINVAL, "%s: null ids/expert_id/perm/inv_perm", name);
  return CDX_OK;
}

// out[i] = in[perm[i]] (gather) or out[perm[i]] = in[i] (scatter).  HBM-bound: one
// wave per row, each lane moving up to kPermVec 16-byte vectors of it with all its
// loads issued before its stores; both sides are streamed (non-temporal), as no row
// is read twice.  A permutation entry outside [0, T) copies nothing.
constexpr int kPermVec = 4;

template <bool GATHER>
__global__ __launch_bounds__(256) void permute_rows_kernel(const uint4* __restrict__ in,
                                                           const int32_t* __restrict__ perm,
                                                           int64_t T, int64_t vec_per_row,
                                                           uint4* __restrict__ out) {
  typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= T) return;
  const int64_t p = perm[i];
  if (p < 0 || p >= T) return;
  const u32x4_t* src = reinterpret_cast<const u32x4_t*>(in + (GATHER ? p : i) * vec_per_row);
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(out + (GATHER ? i : p) * vec_per_row);
  for (int64_t v0 = 0; v0 < vec_per_row; v0 += kPermVec * kWave) {
    u32x4_t r[kPermVec];
#pragma unroll
    for (int u = 0; u < kPermVec; ++u) {
      const int64_t v = v0 + u * kWave + lane;
      if (v < vec_per_row) r[u] = __builtin_nontemporal_load(src + v);
    }
#pragma unroll
    for (int u = 0; u < kPermVec; ++u) {
      const int64_t v = v0 + u * kWave + lane;
      if (v < vec_per_row) __builtin_nontemporal_store(r[u], dst + v);
    }
  }
}

// Rows whose length or base is not a multiple of 16 bytes (a token matrix of any
// width, as tokens[sorted_indices] takes): one wave per row moving W-byte words, W the
// widest power of two below 16 that divides the row length and both bases.
template <bool GATHER, typename W>
__global__ __launch_bounds__(256) void permute_rows_narrow_kernel(const W* __restrict__ in,
                                                                  const int32_t* __restrict__ perm, int64_t T,
                                                                  int64_t words, W* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= T) return;
  const int64_t p = perm[i];
  if (p < 0 || p >= T) return;
  const W* src = in + (GATHER ? p : i) * words;
  W* dst = out + (GATHER ? i : p) * words;
  for (int64_t v = lane; v < words; v += kWave) dst[v] = src[v];
}

template <bool GATHER>
int permute_narrow_launch(const void* in, const int32_t* perm, int64_t T, int64_t row_bytes, void* out,
                          hipStream_t s) {
  const uintptr_t a = (uintptr_t)in | (uintptr_t)out | (uintptr_t)row_bytes;
  const dim3 grid((unsigned)((T + 3) / 4)), block(256);
  if (a % 8 == 0)
    permute_rows_narrow_kernel<GATHER, uint64_t><<<grid, block, 0, s>>>(
        static_cast<const uint64_t*>(in), perm, T, row_bytes / 8, static_cast<uint64_t*>(out));
  else if (a % 4 == 0)
    permute_rows_narrow_kernel<GATHER, uint32_t><<<grid, block, 0, s>>>(
        static_cast<const uint32_t*>(in), perm, T, row_bytes / 4, static_cast<uint32_t*>(out));
  else if (a % 2 == 0)
    permute_rows_narrow_kernel<GATHER, uint16_t><<<grid, block, 0, s>>>(
        static_cast<const uint16_t*>(in), perm, T, row_bytes / 2, static_cast<uint16_t*>(out));
  else
    permute_rows_narrow_kernel<GATHER, uint8_t><<<grid, block, 0, s>>>(
        static_cast<const uint8_t*>(in), perm, T, row_bytes, static_cast<uint8_t*>(out));
  return CDX_OK;
}

}  // namespace
}  // namespace cdx

extern "C" size_t cdx_route_workspace_bytes(int64_t T, int32_t E) {
  if (T <= 0 || E <= 0) return 0;
  const int64_t tpb = cdx::tokens_per_block(T);
  return (size_t)(((T + tpb - 1) / tpb) * E) * sizeof(int32_t);
}

extern "C" int cdx_route_plan(const int64_t* ids, int64_t T, const int64_t* map, int64_t V,
                              int32_t E, int32_t* expert_id, int32_t* perm, int32_t* inv_perm,
                              int32_t* counts, int32_t* offsets, void* workspace,
                              size_t workspace_bytes, void* stream) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_route_plan";
  if (int rc = route_plan_check(ids, T, map, V, E, expert_id, perm, inv_perm, counts, offsets, name)) return rc;
  const size_t need = cdx_route_workspace_bytes(T, E);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(CDX_EWORKSPACE, "%s: workspace needs %zu bytes, got %zu", name, need, workspace_bytes);
  return route_plan_launch(ids, T, &map, 1, V, E, expert_id, perm, inv_perm, counts, offsets,
                           static_cast<int32_t*>(workspace), reinterpret_cast<hipStream_t>(stream), name);
}

extern "C" size_t cdx_route_plans_workspace_bytes(int64_t T, int32_t E, int32_t L) {
  if (L <= 0) return 0;
  return cdx_route_workspace_bytes(T, E) * (size_t)L;
}

extern "C" int cdx_route_plans(const int64_t* ids, int64_t T, const int64_t* const* maps, int32_t L, int64_t V,
                               int32_t E, int32_t* expert_id, int32_t* perm, int32_t* inv_perm, int32_t* counts,
                               int32_t* offsets, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_route_plans";
  if (L < 0) return fail(CDX_EINVAL, "%s: L=%d must be >= 0", name, L);
  if (L == 0) return CDX_OK;
  if (!maps) return fail(CDX_EINVAL, "%s: null map table", name);
  for (int32_t y = 0; y < L; ++y)
    if (!maps[y]) return fail(CDX_EINVAL, "%s: map %d is NULL", name, y);
  if (int rc = route_plan_check(ids, T, maps[0], V, E, expert_id, perm, inv_perm, counts, offsets, name)) return rc;
  if ((int64_t)L * T > INT32_MAX)
    return fail(CDX_EUNSUPPORTED, "%s: L * T = %lld exceeds 2^31 - 1", name, (long long)L * T);
  const size_t need = cdx_route_plans_workspace_bytes(T, E, L);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(CDX_EWORKSPACE, "%s: workspace needs %zu bytes, got %zu", name, need, workspace_bytes);
  const size_t per = cdx_route_workspace_bytes(T, E) / sizeof(int32_t);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // Launches of at most kMaxMaps plans each (the map table travels in the arguments).
  for (int32_t y0 = 0; y0 < L; y0 += kMaxMaps) {
    const int32_t n = L - y0 < kMaxMaps ? L - y0 : kMaxMaps;
    const int64_t r = (int64_t)y0;
    if (int rc = route_plan_launch(ids, T, maps + y0, n, V, E, expert_id + r * T, perm + r * T, inv_perm + r * T,
                                   counts + r * E, offsets + r * (E + 1),
                                   static_cast<int32_t*>(workspace) + r * per, s, name))
      return rc;
  }
  return CDX_OK;
}

// ---- allocation-free variant --------------------------------------------------
// The count table of cdx_route_plan_noalloc lives in this file-scope device array,
// one copy per GPU, held until the process ends.  In host code the name `scratch`
// denotes a host-side shadow, not device memory: the device address is looked up
// once per device (hipGetSymbolAddress with that device current) and only that
// address is ever handed to a kernel.  Calls on one GPU share the array, so calls
// that overlap in time on one GPU (different streams, or host threads) race; calls
// ordered on one stream do not.  Nothing in it needs clearing between calls: the
// count launch writes every entry the scatter launch then reads.
static __device__ __align__(256) int32_t scratch[cdx::kScratchInts];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
int32_t* g_scratch_dev[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on first use).
int scratch_on_current_device(int32_t** out, const char* name) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0)
    return cdx::fail(CDX_ELAUNCH, "%s: hipGetDevice failed", name);
  if (dev >= kMaxDevices) return cdx::fail(CDX_EUNSUPPORTED, "%s: device %d >= %d", name, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return cdx::fail(CDX_ELAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", name, dev,
                       hipGetErrorString(e));
    g_scratch_dev[dev] = static_cast<int32_t*>(p);
  }
  *out = g_scratch_dev[dev];
  return CDX_OK;
}
}  // namespace

extern "C" size_t cdx_route_noalloc_scratch_bytes(void) { return sizeof(scratch); }

extern "C" int cdx_route_plan_noalloc(const int64_t* ids, int64_t T, const int64_t* map, int64_t V, int32_t E,
                                      int32_t* expert_id, int32_t* perm, int32_t* inv_perm, int32_t* counts,
                                      int32_t* offsets, void* stream) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_route_plan_noalloc";
  if (int rc = route_plan_check(ids, T, map, V, E, expert_id, perm, inv_perm, counts, offsets, name)) return rc;
  const size_t need = cdx_route_workspace_bytes(T, E);
  if (need > sizeof(scratch))
    return fail(CDX_EWORKSPACE, "%s: the count table needs %zu bytes, the library scratch holds %zu", name, need,
                sizeof(scratch));
  int32_t* table = nullptr;
  if (int rc = scratch_on_current_device(&table, name)) return rc;
  return route_plan_launch(ids, T, &map, 1, V, E, expert_id, perm, inv_perm, counts, offsets, table,
                           reinterpret_cast<hipStream_t>(stream), name);
}

static int permute_common(const void* in, const int32_t* perm, int64_t T, int64_t row_bytes,
                          void* out, void* stream, bool gather, const char* name) {
  using namespace cdx;
  clear_error();
  if (T < 0 || row_bytes <= 0) return fail(CDX_EINVAL, "%s: bad shape", name);
  if (T > INT32_MAX) return fail(CDX_EUNSUPPORTED, "%s: T=%lld exceeds 2^31 - 1", name, (long long)T);
  if (T == 0) return CDX_OK;
  if (!in || !perm || !out) return fail(CDX_EINVAL, "%s: null pointer", name);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (row_bytes % 16 != 0 || !aligned16(in) || !aligned16(out)) {
    const int rc = gather ? permute_narrow_launch<true>(in, perm, T, row_bytes, out, s)
                          : permute_narrow_launch<false>(in, perm, T, row_bytes, out, s);
    return rc ? rc : check_launch(name);
  }
  const dim3 grid((unsigned)((T + 3) / 4));
  if (gather)
    permute_rows_kernel<true><<<grid, dim3(256), 0, s>>>(static_cast<const uint4*>(in), perm, T, row_bytes / 16, static_cast<uint4*>(out));
  else
    permute_rows_kernel<false><<<grid, dim3(256), 0, s>>>(static_cast<const uint4*>(in), perm, T, row_bytes / 16, static_cast<uint4*>(out));
  return check_launch(name);
}

extern "C" int cdx_permute_rows(const void* in, const int32_t* perm, int64_t T, int64_t row_bytes,
                                void* out, void* stream) {
  return permute_common(in, perm, T, row_bytes, out, stream, true, "cdx_permute_rows");
}

extern "C" int cdx_unpermute_rows(const void* in, const int32_t* perm, int64_t T, int64_t row_bytes,
                                  void* out, void* stream) {
  return permute_common(in, perm, T, row_bytes, out, stream, false, "cdx_unpermute_rows");
}
