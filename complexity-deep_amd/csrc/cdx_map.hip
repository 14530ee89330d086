// Greedy bin-packing of a vocabulary onto experts (host code, no kernels): the
// token -> expert map the routing plan looks up.
//
// Reference behaviour: core/token_routed_mlp.py:87-119 (_build_token_mapping with
// token_frequencies): tokens in descending frequency, each assigned to the expert with
// the lowest accumulated load (the first such expert on ties, as min(range(E),
// key=loads) picks), loads accumulated in double from the float32 frequencies.
//
// Here: one stable sort of the token ids by descending frequency (ties keep the
// lower id first) and a binary min-heap of (load, expert) pairs, so each assignment
// costs O(log E) instead of the reference's O(E) scan; the heap order (load, then
// expert index) selects exactly the first least-loaded expert.
#include <algorithm>
#include <cmath>
#include <numeric>
#include <queue>
#include <vector>

#include "cdx_common.h"

extern "C" int cdx_binpack_map(const float* freq, int64_t V, int32_t E, int64_t* map) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_binpack_map";
  if (V <= 0 || E <= 0 || E > 65536) return fail(CDX_EINVAL, "%s: bad shape V=%lld E=%d", name, (long long)V, E);
  if (!freq || !map) return fail(CDX_EINVAL, "%s: null pointer", name);
  for (int64_t i = 0; i < V; ++i)
    if (std::isnan(freq[i])) return fail(CDX_EINVAL, "%s: frequency of token %lld is NaN", name, (long long)i);
  std::vector<int64_t> order((size_t)V);
  std::iota(order.begin(), order.end(), int64_t(0));
  std::stable_sort(order.begin(), order.end(), [freq](int64_t a, int64_t b) { return freq[a] > freq[b]; });
  struct Bin {
    double load;
    int32_t expert;
  };
  auto later = [](const Bin& a, const Bin& b) {  // heap top = least load, then lowest expert
    return a.load > b.load || (a.load == b.load && a.expert > b.expert);
  };
  std::priority_queue<Bin, std::vector<Bin>, decltype(later)> heap(later);
  for (int32_t e = 0; e < E; ++e) heap.push({0.0, e});
  for (const int64_t tid : order) {
    Bin b = heap.top();
    heap.pop();
    map[tid] = b.expert;
    b.load += (double)freq[tid];
    heap.push(b);
  }
  return CDX_OK;
}
