// Token embedding gather for gfx950 (the input side of the tied LM head).
//
// Reference behaviour: models/modeling.py:74,177 — nn.Embedding(vocab, hidden) looked
// up with the token ids: out[t, :] = table[ids[t], :], an exact copy of bf16 rows.
//
// Design: one wave64 per token row.  The id is read once per wave (wave-uniform, so
// the row base is scalar), then every lane copies 16-byte chunks of the row: all
// loads of a lane first, then all stores, so a wave keeps the whole row in flight.
// An id outside [0, vocab) yields a row of bf16 quiet NaNs.  nn.Embedding raises
// there, which a kernel cannot do without a host round trip; a NaN row reads nothing
// out of bounds and cannot pass for a result: every logit that depends on the token
// (its own row, and through attention every later position of its sequence) is NaN.
#include "cdx_common.h"

namespace cdx {
namespace {

constexpr int kEmbedRowsPerBlock = 4;  // 4 waves of 64 lanes, one row each

template <int VPL>
__global__ __launch_bounds__(256) void embedding_kernel(const int64_t* __restrict__ ids, int64_t T,
                                                        const uint16_t* __restrict__ table, int64_t V, int H,
                                                        uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kEmbedRowsPerBlock + (threadIdx.x >> 6);
  if (row >= T) return;
  const int64_t id = ids[row];
  const bool valid = id >= 0 && id < V;
  const int nvec = H >> 3;
  const uint4* src = reinterpret_cast<const uint4*>(table + (valid ? id : 0) * (int64_t)H);
  uint4* dst = reinterpret_cast<uint4*>(out + row * (int64_t)H);
  constexpr uint32_t kNaN2 = 0x7FC07FC0u;  // two bf16 quiet NaNs
  uint4 v[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int idx = i * kWave + lane;
    v[i] = make_uint4(kNaN2, kNaN2, kNaN2, kNaN2);
    if (valid && idx < nvec) v[i] = src[idx];
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int idx = i * kWave + lane;
    if (idx < nvec) dst[idx] = v[i];
  }
}

template <int VPL>
int launch_embed(const int64_t* ids, int64_t T, const uint16_t* table, int64_t V, int H, uint16_t* out,
                 hipStream_t s) {
  const dim3 grid((unsigned)((T + kEmbedRowsPerBlock - 1) / kEmbedRowsPerBlock));
  embedding_kernel<VPL><<<grid, dim3(256), 0, s>>>(ids, T, table, V, H, out);
  return check_launch("cdx_embedding_fwd");
}

}  // namespace
}  // namespace cdx

extern "C" int cdx_embedding_fwd(const int64_t* ids, int64_t T, const uint16_t* table, int64_t V, int32_t H,
                                 uint16_t* out, void* stream) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_embedding_fwd";
  if (T < 0 || V <= 0 || H <= 0)
    return fail(CDX_EINVAL, "%s: bad shape T=%lld V=%lld H=%d", name, (long long)T, (long long)V, H);
  if (H % 8 != 0 || H > 16384)
    return fail(CDX_EUNSUPPORTED, "%s: H=%d must be a multiple of 8 and <= 16384", name, H);
  if (T == 0) return CDX_OK;
  if ((T + kEmbedRowsPerBlock - 1) / kEmbedRowsPerBlock > INT32_MAX)
    return fail(CDX_EUNSUPPORTED, "%s: too many tokens", name);
  if (!ids || !table || !out) return fail(CDX_EINVAL, "%s: null pointer", name);
  if (!aligned16(table) || !aligned16(out))
    return fail(CDX_EUNSUPPORTED, "%s: table and out must be 16-byte aligned", name);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int nvec = H / 8;
  if (nvec <= 64) return launch_embed<1>(ids, T, table, V, H, out, s);
  if (nvec <= 128) return launch_embed<2>(ids, T, table, V, H, out, s);
  if (nvec <= 256) return launch_embed<4>(ids, T, table, V, H, out, s);
  if (nvec <= 512) return launch_embed<8>(ids, T, table, V, H, out, s);
  if (nvec <= 1024) return launch_embed<16>(ids, T, table, V, H, out, s);
  return launch_embed<32>(ids, T, table, V, H, out, s);
}
