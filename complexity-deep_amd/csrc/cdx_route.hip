// Routing plan for the token-routed MoE on gfx950 (piece 1a of the hot path).
//
// Reference behaviour: core/token_routed_mlp.py:149-150 (expert = map[clamp(id)]),
// :166-170 (mask dispatch, i.e. a stable partition by expert id) and the operator
// API cuda/triton_token_routed.py:37-61 (counts = bincount, offsets = [0, cumsum]).
//
// Design: a stable counting sort in three launches, bit-exact and free of atomics.
//   1. count:   each 256-thread block owns 1024 consecutive tokens, split into 16
//               chunks of 64 (one chunk per wave per step).  A wave looks up the
//               expert of its 64 tokens and, per expert, takes a 64-bit ballot; the
//               popcount is the chunk's count.  The block writes its per-expert
//               totals to workspace row [block][E].
//   2. scan:    one block turns the [nblk][E] counts into counts/offsets and into the
//               first sorted position of every (block, expert) pair, scanning in
//               expert-major, block-minor order.
//   3. scatter: each block recomputes its ballots; a token's sorted position is
//               base[block][e] + (tokens of e in earlier chunks of the block) +
//               popcount(ballot & lanes-below).  Token order inside an expert is the
//               original index order, which is exactly argsort(expert, stable=True).
#include "cdx_common.h"

namespace cdx {
namespace {

constexpr int kTokPerBlock = 1024;
constexpr int kChunks = kTokPerBlock / kWave;  // 16
constexpr int kMaxE = 64;

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

__global__ __launch_bounds__(256) void route_count_kernel(const int64_t* __restrict__ ids,
                                                          const int64_t* __restrict__ map,
                                                          int64_t V, int E, int64_t T,
                                                          int32_t* __restrict__ expert_id,
                                                          int32_t* __restrict__ blk_counts) {
  __shared__ int cnt[kChunks][kMaxE];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t base = (int64_t)blockIdx.x * kTokPerBlock;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = wave * 4 + j;
    const int64_t t = base + c * kWave + lane;
    int e = -1;
    if (t < T) {
      e = lookup_expert(ids, map, V, E, t);
      expert_id[t] = e;
    }
    for (int x = 0; x < E; ++x) {
      const uint64_t m = __ballot(e == x);
      if (lane == 0) cnt[c][x] = __popcll(m);
    }
  }
  __syncthreads();
  for (int x = threadIdx.x; x < E; x += blockDim.x) {
    int s = 0;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) s += cnt[c][x];
    blk_counts[(int64_t)blockIdx.x * E + x] = s;
  }
}

// Inclusive scan of one int per thread over a 1024-thread block.
__device__ __forceinline__ int block_inclusive_scan(int v, int* lds_wave_tot, int& block_total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(v, off, 64);
    if (lane >= off) v += y;
  }
  if (lane == 63) lds_wave_tot[wave] = v;
  __syncthreads();
  int prefix = 0, total = 0;
  const int nw = blockDim.x >> 6;
  for (int w = 0; w < nw; ++w) {
    const int tw = lds_wave_tot[w];
    if (w < wave) prefix += tw;
    total += tw;
  }
  __syncthreads();
  block_total = total;
  return v + prefix;
}

__global__ __launch_bounds__(1024) void route_scan_kernel(int64_t nblk, int E,
                                                          const int32_t* __restrict__ blk_counts,
                                                          int32_t* __restrict__ blk_base,
                                                          int32_t* __restrict__ counts,
                                                          int32_t* __restrict__ offsets) {
  __shared__ int wave_tot[16];
  __shared__ int totals[kMaxE];
  __shared__ int offs[kMaxE + 1];
  for (int x = 0; x < E; ++x) {
    int carry = 0;
    for (int64_t b0 = 0; b0 < nblk; b0 += blockDim.x) {
      const int64_t b = b0 + threadIdx.x;
      const int v = b < nblk ? blk_counts[b * E + x] : 0;
      int tot;
      const int incl = block_inclusive_scan(v, wave_tot, tot);
      if (b < nblk) blk_base[b * E + x] = carry + incl - v;  // exclusive, within expert x
      carry += tot;
    }
    if (threadIdx.x == 0) totals[x] = carry;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    offs[0] = 0;
    for (int x = 0; x < E; ++x) {
      run += totals[x];
      offs[x + 1] = run;
    }
  }
  __syncthreads();
  for (int x = threadIdx.x; x < E; x += blockDim.x) counts[x] = totals[x];
  for (int x = threadIdx.x; x <= E; x += blockDim.x) offsets[x] = offs[x];
  for (int64_t i = threadIdx.x; i < nblk * E; i += blockDim.x) blk_base[i] += offs[i % E];
}

__global__ __launch_bounds__(256) void route_scatter_kernel(const int32_t* __restrict__ expert_id,
                                                            int E, int64_t T,
                                                            const int32_t* __restrict__ blk_base,
                                                            int32_t* __restrict__ perm,
                                                            int32_t* __restrict__ inv_perm) {
  __shared__ int cnt[kChunks][kMaxE];
  __shared__ int pre[kChunks][kMaxE];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t base = (int64_t)blockIdx.x * kTokPerBlock;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int my_e[4], my_rank[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = wave * 4 + j;
    const int64_t t = base + c * kWave + lane;
    const int e = (t < T) ? expert_id[t] : -1;
    int rank = 0;
    for (int x = 0; x < E; ++x) {
      const uint64_t m = __ballot(e == x);
      if (e == x) rank = __popcll(m & below);
      if (lane == 0) cnt[c][x] = __popcll(m);
    }
    my_e[j] = e;
    my_rank[j] = rank;
  }
  __syncthreads();
  for (int x = threadIdx.x; x < E; x += blockDim.x) {
    int s = blk_base[(int64_t)blockIdx.x * E + x];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      pre[c][x] = s;
      s += cnt[c][x];
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = wave * 4 + j;
    const int64_t t = base + c * kWave + lane;
    if (t < T) {
      const int pos = pre[c][my_e[j]] + my_rank[j];
      perm[pos] = (int32_t)t;
      inv_perm[t] = pos;
    }
  }
}

// out[i] = in[perm[i]] (gather) or out[perm[i]] = in[i] (scatter); one wave per row.
template <bool GATHER>
__global__ __launch_bounds__(256) void permute_rows_kernel(const uint4* __restrict__ in,
                                                           const int32_t* __restrict__ perm,
                                                           int64_t T, int64_t vec_per_row,
                                                           uint4* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= T) return;
  const int64_t p = perm[i];
  const uint4* src = in + (GATHER ? p : i) * vec_per_row;
  uint4* dst = out + (GATHER ? i : p) * vec_per_row;
  for (int64_t v = lane; v < vec_per_row; v += kWave) dst[v] = src[v];
}

}  // namespace
}  // namespace cdx

extern "C" size_t cdx_route_workspace_bytes(int64_t T, int32_t E) {
  if (T < 0 || E <= 0) return 0;
  const int64_t nblk = (T + cdx::kTokPerBlock - 1) / cdx::kTokPerBlock;
  return (size_t)(2 * nblk * E) * sizeof(int32_t);
}

extern "C" int cdx_route_plan(const int64_t* ids, int64_t T, const int64_t* map, int64_t V,
                              int32_t E, int32_t* expert_id, int32_t* perm, int32_t* inv_perm,
                              int32_t* counts, int32_t* offsets, void* workspace,
                              size_t workspace_bytes, void* stream) {
  using namespace cdx;
  clear_error();
  if (T < 0 || T > INT32_MAX) return fail(CDX_EINVAL, "cdx_route_plan: T=%lld out of range", (long long)T);
  if (E <= 0 || E > kMaxE) return fail(CDX_EUNSUPPORTED, "cdx_route_plan: E=%d must be in [1, %d]", E, kMaxE);
  if (map != nullptr && V <= 0) return fail(CDX_EINVAL, "cdx_route_plan: V=%lld must be > 0", (long long)V);
  if (!counts || !offsets) return fail(CDX_EINVAL, "cdx_route_plan: null counts/offsets");
  if (T > 0 && (!ids || !expert_id || !perm || !inv_perm))
    return fail(CDX_EINVAL, "cdx_route_plan: null ids/expert_id/perm/inv_perm");
  const size_t need = cdx_route_workspace_bytes(T, E);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(CDX_EWORKSPACE, "cdx_route_plan: workspace needs %zu bytes, got %zu", need, workspace_bytes);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t nblk = (T + kTokPerBlock - 1) / kTokPerBlock;
  int32_t* blk_counts = static_cast<int32_t*>(workspace);
  int32_t* blk_base = blk_counts + nblk * E;
  if (nblk > 0) {
    route_count_kernel<<<dim3((unsigned)nblk), dim3(256), 0, s>>>(ids, map, V, E, T, expert_id, blk_counts);
    if (int rc = check_launch("cdx_route_plan/count")) return rc;
  }
  route_scan_kernel<<<dim3(1), dim3(1024), 0, s>>>(nblk, E, blk_counts, blk_base, counts, offsets);
  if (int rc = check_launch("cdx_route_plan/scan")) return rc;
  if (nblk > 0) {
    route_scatter_kernel<<<dim3((unsigned)nblk), dim3(256), 0, s>>>(expert_id, E, T, blk_base, perm, inv_perm);
    if (int rc = check_launch("cdx_route_plan/scatter")) return rc;
  }
  return CDX_OK;
}

static int permute_common(const void* in, const int32_t* perm, int64_t T, int64_t row_bytes,
                          void* out, void* stream, bool gather, const char* name) {
  using namespace cdx;
  clear_error();
  if (T < 0 || row_bytes <= 0) return fail(CDX_EINVAL, "%s: bad shape", name);
  if (row_bytes % 16 != 0) return fail(CDX_EUNSUPPORTED, "%s: row_bytes=%lld must be a multiple of 16", name, (long long)row_bytes);
  if (T == 0) return CDX_OK;
  if (!in || !perm || !out) return fail(CDX_EINVAL, "%s: null pointer", name);
  if (!aligned16(in) || !aligned16(out)) return fail(CDX_EUNSUPPORTED, "%s: pointers must be 16-byte aligned", name);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
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
