// Residual add + RMSNorm for gfx950 (piece 3 of the hot path).
//
// Reference behaviour: core/normalization.py:29-32 (RMSNorm in the input dtype) and
// core/layer.py:174,183 (bf16 residual adds); operator API of
// cuda/fused_residual.py:333-399.
//
// Design: one wave64 normalises one row at a time and walks rows with a stride of the
// grid's wave count, prefetching its next row (x and residual, 128-bit loads, VPL
// vectors of 8 bf16 per lane) before it works on the current one, so a CU keeps
// many KB in flight and the kernel runs at HBM speed.  The weight row is loaded once
// per wave.  The row's sum of squares is reduced with DPP adds inside each 16-lane
// row and four readlanes (no LDS round trips).  h = bf16(x + residual) is rounded
// exactly like the reference's bf16 add, the sum of squares is accumulated in fp32
// over the rounded h, and the normalised output is rounded to bf16 once.  Traffic
// per row is the algorithmic minimum: read x, residual (2H bytes each), write h and
// out.  The output rows may sit at a stride wider than H (cdx_rmsnorm_ld_fwd): the
// model writes the next layer's normalised x beside its mu in one [T, 2H] buffer.
#include <algorithm>

#include "cdx_common.h"

namespace cdx {
namespace {

constexpr int kWavesPerBlock = 4;

// Sum over the wave, returned to every lane: DPP butterflies within each 16-lane
// row (xor 1, xor 2, half-row mirror, row mirror), then the four row sums.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (a + b) + (c + d);
}

// FULL: H == 512 VPL (every lane owns VPL whole vectors, no guards).  Otherwise lanes
// past the row's end load a clamped vector (never used) so the loads stay unguarded.
template <int VPL, bool FULL, bool HAS_RES, bool STORE_RES>
__global__ __launch_bounds__(64 * kWavesPerBlock) void add_rmsnorm_kernel(
    const uint16_t* x, const uint16_t* res, const uint16_t* __restrict__ w, float eps,
    int64_t T, int H, uint16_t* out, int64_t ldo, uint16_t* res_out) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
  int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= T) return;
  const int nvec = H >> 3;
  int vi[VPL];  // vector index of each of the lane's vectors, clamped in range
  bool ok[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int idx = v * kWave + lane;
    ok[v] = FULL || idx < nvec;
    vi[v] = FULL ? idx : min(idx, nvec - 1);
  }
  float wf[VPL][8];
  {
    const uint4* wr = reinterpret_cast<const uint4*>(w);
#pragma unroll
    for (int v = 0; v < VPL; ++v) unpack8(wr[vi[v]], wf[v]);
  }
  auto load_row = [&](int64_t r, uint4* xv, uint4* rv) __attribute__((always_inline)) {
    const uint4* xr = reinterpret_cast<const uint4*>(x + r * H);
    const uint4* rr = reinterpret_cast<const uint4*>((HAS_RES ? res : x) + r * H);
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      xv[v] = xr[vi[v]];
      if (HAS_RES) rv[v] = rr[vi[v]];
    }
  };
  uint4 xv[VPL], rv[VPL];
  load_row(row, xv, rv);
  for (; row < T; row += nwaves) {
    // Next row in flight while this one is reduced and written.
    uint4 xn[VPL], rn[VPL];
    const int64_t next = row + nwaves;
    if (next < T) load_row(next, xn, rn);

    float h[VPL][8];
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      unpack8(xv[v], h[v]);
      if (HAS_RES) {
        float r[8];
        unpack8(rv[v], r);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          // bf16 + bf16 rounded to bf16, as torch does for a bf16 add.
          h[v][i] = bf16_bits_to_f32(f32_to_bf16_bits(h[v][i] + r[i]));
        }
      }
      if (!ok[v]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) h[v][i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += h[v][i] * h[v][i];
    }
    const float inv = rsqrtf(wave_sum_dpp(ss) / (float)H + eps);

    uint4* orow = reinterpret_cast<uint4*>(out + row * ldo);
    uint4* hrow = STORE_RES ? reinterpret_cast<uint4*>(res_out + row * H) : nullptr;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      if (!ok[v]) continue;
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = wf[v][i] * (h[v][i] * inv);
      if (STORE_RES) hrow[vi[v]] = pack8(h[v]);
      orow[vi[v]] = pack8(y);
    }
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      xv[v] = xn[v];
      if (HAS_RES) rv[v] = rn[v];
    }
  }
}

template <int VPL, bool FULL>
int launch_vpl(const uint16_t* x, const uint16_t* res, const uint16_t* w, float eps, int64_t T,
               int H, uint16_t* out, int64_t ldo, uint16_t* res_out, hipStream_t s) {
  // Four blocks (16 waves) per CU; each wave walks about T / waves rows, so that its
  // prefetch of the next row has work to hide behind.
  const int64_t max_blocks = (int64_t)device_cu_count() * 4;
  const int64_t blocks = std::min<int64_t>((T + kWavesPerBlock - 1) / kWavesPerBlock, max_blocks);
  const dim3 grid((unsigned)blocks);
  const dim3 block(64 * kWavesPerBlock);
  if (res == nullptr) {
    add_rmsnorm_kernel<VPL, FULL, false, false><<<grid, block, 0, s>>>(x, res, w, eps, T, H, out, ldo, res_out);
  } else if (res_out == nullptr) {
    add_rmsnorm_kernel<VPL, FULL, true, false><<<grid, block, 0, s>>>(x, res, w, eps, T, H, out, ldo, res_out);
  } else {
    add_rmsnorm_kernel<VPL, FULL, true, true><<<grid, block, 0, s>>>(x, res, w, eps, T, H, out, ldo, res_out);
  }
  return check_launch("cdx_add_rmsnorm_fwd");
}

template <int VPL>
int launch_h(const uint16_t* x, const uint16_t* res, const uint16_t* w, float eps, int64_t T, int H,
             uint16_t* out, int64_t ldo, uint16_t* res_out, hipStream_t s) {
  if (H == 512 * VPL) return launch_vpl<VPL, true>(x, res, w, eps, T, H, out, ldo, res_out, s);
  return launch_vpl<VPL, false>(x, res, w, eps, T, H, out, ldo, res_out, s);
}

int launch(const uint16_t* x, const uint16_t* res, const uint16_t* w, float eps, int64_t T, int H,
           uint16_t* out, int64_t ldo, uint16_t* res_out, hipStream_t s) {
  const int nvec = H / 8;
  if (nvec <= 64) return launch_h<1>(x, res, w, eps, T, H, out, ldo, res_out, s);
  if (nvec <= 128) return launch_h<2>(x, res, w, eps, T, H, out, ldo, res_out, s);
  if (nvec <= 256) return launch_h<4>(x, res, w, eps, T, H, out, ldo, res_out, s);
  if (nvec <= 512) return launch_h<8>(x, res, w, eps, T, H, out, ldo, res_out, s);
  return launch_h<16>(x, res, w, eps, T, H, out, ldo, res_out, s);
}

}  // namespace
}  // namespace cdx

extern "C" int cdx_add_rmsnorm_fwd(const uint16_t* x, const uint16_t* residual,
                                   const uint16_t* weight, float eps, int64_t T, int32_t H,
                                   uint16_t* out, uint16_t* residual_out, void* stream) {
  using namespace cdx;
  clear_error();
  if (T < 0 || H <= 0) return fail(CDX_EINVAL, "cdx_add_rmsnorm_fwd: bad shape T=%lld H=%d", (long long)T, H);
  if (H % 8 != 0 || H > 8192)
    return fail(CDX_EUNSUPPORTED, "cdx_add_rmsnorm_fwd: H=%d must be a multiple of 8 and <= 8192", H);
  if (!(eps >= 0.f)) return fail(CDX_EINVAL, "cdx_add_rmsnorm_fwd: eps must be >= 0");
  if (T == 0) return CDX_OK;
  if (!x || !weight || !out) return fail(CDX_EINVAL, "cdx_add_rmsnorm_fwd: null x/weight/out");
  if (!residual && residual_out)
    return fail(CDX_EINVAL, "cdx_add_rmsnorm_fwd: residual_out given without residual");
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out) || (residual && !aligned16(residual)) ||
      (residual_out && !aligned16(residual_out)))
    return fail(CDX_EUNSUPPORTED, "cdx_add_rmsnorm_fwd: pointers must be 16-byte aligned");
  return launch(x, residual, weight, eps, T, H, out, H, residual_out, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int cdx_rmsnorm_ld_fwd(const uint16_t* x, const uint16_t* weight, float eps, int64_t T, int32_t H,
                                  uint16_t* out, int64_t ldo, void* stream) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_rmsnorm_ld_fwd";
  if (T < 0 || H <= 0) return fail(CDX_EINVAL, "%s: bad shape T=%lld H=%d", name, (long long)T, H);
  if (H % 8 != 0 || H > 8192) return fail(CDX_EUNSUPPORTED, "%s: H=%d must be a multiple of 8 and <= 8192", name, H);
  if (!(eps >= 0.f)) return fail(CDX_EINVAL, "%s: eps must be >= 0", name);
  if (ldo < H) return fail(CDX_EINVAL, "%s: ldo=%lld is smaller than H=%d", name, (long long)ldo, H);
  if (ldo % 8 != 0) return fail(CDX_EUNSUPPORTED, "%s: ldo=%lld must be a multiple of 8", name, (long long)ldo);
  if (T == 0) return CDX_OK;
  if (!x || !weight || !out) return fail(CDX_EINVAL, "%s: null x/weight/out", name);
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out))
    return fail(CDX_EUNSUPPORTED, "%s: pointers must be 16-byte aligned", name);
  return launch(x, nullptr, weight, eps, T, H, out, ldo, nullptr, reinterpret_cast<hipStream_t>(stream));
}
