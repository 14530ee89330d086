/*
 * CPU oracle for the integer part of the hot path — TEST INFRASTRUCTURE ONLY.
 *
 * Nothing in the product links this file; only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load liboracle.so, as the checker.
 *
 * Restates, in plain C:
 *   oracle_binpack_map  core/token_routed_mlp.py:105-116 (greedy Zipf bin-packing)
 *   oracle_modulo_map   core/token_routed_mlp.py:118-119 (token_id % E fallback)
 *   oracle_route_plan   core/token_routed_mlp.py:149-150,166-170 and
 *                       cuda/triton_token_routed.py:37-61 (lookup, bincount,
 *                       offsets, stable order by expert)
 */
#include <stdint.h>
#include <stdlib.h>

/* Order tokens by descending frequency; equal frequencies keep ascending token id
 * (the Zipf pmf used by the benchmarks has no ties, so this choice is never hit). */
static const float* g_freq;
static int cmp_desc(const void* a, const void* b) {
  const int64_t i = *(const int64_t*)a, j = *(const int64_t*)b;
  const float fi = g_freq[i], fj = g_freq[j];
  if (fi > fj) return -1;
  if (fi < fj) return 1;
  return (i > j) - (i < j);
}

/*
 * Greedy bin-packing: walk tokens by descending frequency and give each to the expert
 * with the smallest accumulated load (first such expert on ties); loads accumulate in
 * double precision, adding the float32 frequency exactly as Python's float does.
 * Returns 0, or -1 on bad arguments / allocation failure.
 */
int oracle_binpack_map(const float* freq, int64_t V, int32_t E, int64_t* map) {
  if (!freq || !map || V <= 0 || E <= 0) return -1;
  int64_t* order = (int64_t*)malloc(sizeof(int64_t) * (size_t)V);
  double* load = (double*)calloc((size_t)E, sizeof(double));
  if (!order || !load) {
    free(order);
    free(load);
    return -1;
  }
  for (int64_t i = 0; i < V; ++i) order[i] = i;
  g_freq = freq;
  qsort(order, (size_t)V, sizeof(int64_t), cmp_desc);
  for (int64_t r = 0; r < V; ++r) {
    const int64_t tid = order[r];
    int32_t best = 0;
    for (int32_t e = 1; e < E; ++e)
      if (load[e] < load[best]) best = e;
    map[tid] = best;
    load[best] += (double)freq[tid];
  }
  free(order);
  free(load);
  return 0;
}

void oracle_modulo_map(int64_t V, int32_t E, int64_t* map) {
  for (int64_t i = 0; i < V; ++i) map[i] = i % E;
}

/*
 * Routing plan.  expert_id[t] = map[clamp(ids[t], 0, V-1)] (map == NULL: ids are the
 * expert ids).  counts = bincount, offsets = [0, cumsum(counts)], perm = stable
 * argsort of expert_id, inv_perm = perm^-1.  Expert ids are clamped into [0, E).
 * Two passes over the tokens (count, then place): a textbook stable counting sort.
 */
int oracle_route_plan(const int64_t* ids, int64_t T, const int64_t* map, int64_t V, int32_t E,
                      int32_t* expert_id, int32_t* perm, int32_t* inv_perm, int64_t* counts,
                      int64_t* offsets) {
  if (T < 0 || E <= 0 || !counts || !offsets) return -1;
  for (int32_t e = 0; e < E; ++e) counts[e] = 0;
  for (int64_t t = 0; t < T; ++t) {
    int64_t e;
    if (map) {
      int64_t id = ids[t];
      if (id < 0) id = 0;
      if (id > V - 1) id = V - 1;
      e = map[id];
    } else {
      e = ids[t];
    }
    if (e < 0) e = 0;
    if (e > E - 1) e = E - 1;
    expert_id[t] = (int32_t)e;
    counts[e] += 1;
  }
  offsets[0] = 0;
  for (int32_t e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
  int64_t* next = (int64_t*)malloc(sizeof(int64_t) * (size_t)E);
  if (!next) return -1;
  for (int32_t e = 0; e < E; ++e) next[e] = offsets[e];
  for (int64_t t = 0; t < T; ++t) {
    const int64_t pos = next[expert_id[t]]++;
    perm[pos] = (int32_t)t;
    inv_perm[t] = (int32_t)pos;
  }
  free(next);
  return 0;
}
