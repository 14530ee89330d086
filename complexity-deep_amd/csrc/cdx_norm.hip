// Residual add + RMSNorm for gfx950 (piece 3 of the hot path).
//
// Reference behaviour: core/normalization.py:29-32 (RMSNorm in the input dtype) and
// core/layer.py:174,183 (bf16 residual adds); operator API of
// cuda/fused_residual.py:333-399.
//
// Design: one wave64 owns one row.  Every lane issues all of its 128-bit loads for x
// and residual up front (VPL vectors of 8 bf16 each), so a CU keeps many KB in flight
// and the kernel runs at HBM speed.  h = bf16(x + residual) is rounded exactly like
// the reference's bf16 add, the sum of squares is accumulated in fp32 over the
// rounded h, and the normalised output is rounded to bf16 once.  Traffic per row is
// the algorithmic minimum: read x, residual (2H bytes each), write h and out.
#include "cdx_common.h"

namespace cdx {
namespace {

constexpr int kRowsPerBlock = 4;  // 4 waves of 64 lanes, one row each

template <int VPL, bool HAS_RES, bool STORE_RES>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(
    const uint16_t* x, const uint16_t* res, const uint16_t* __restrict__ w, float eps,
    int64_t T, int H, uint16_t* out, uint16_t* res_out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= T) return;
  const int nvec = H >> 3;
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * H);
  const uint4* rr = HAS_RES ? reinterpret_cast<const uint4*>(res + row * H) : nullptr;

  uint4 xv[VPL], rv[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int idx = v * kWave + lane;
    if (idx < nvec) {
      xv[v] = xr[idx];
      if (HAS_RES) rv[v] = rr[idx];
    }
  }

  float h[VPL][8];
  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int idx = v * kWave + lane;
    if (idx < nvec) {
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
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += h[v][i] * h[v][i];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) h[v][i] = 0.f;
    }
  }
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / (float)H + eps);

  const uint4* wr = reinterpret_cast<const uint4*>(w);
  uint4* orow = reinterpret_cast<uint4*>(out + row * H);
  uint4* hrow = STORE_RES ? reinterpret_cast<uint4*>(res_out + row * H) : nullptr;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int idx = v * kWave + lane;
    if (idx < nvec) {
      float wf[8], y[8];
      unpack8(wr[idx], wf);
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = wf[i] * (h[v][i] * inv);
      if (STORE_RES) hrow[idx] = pack8(h[v]);
      orow[idx] = pack8(y);
    }
  }
}

template <int VPL>
int launch_vpl(const uint16_t* x, const uint16_t* res, const uint16_t* w, float eps, int64_t T,
               int H, uint16_t* out, uint16_t* res_out, hipStream_t s) {
  const dim3 grid((unsigned)((T + kRowsPerBlock - 1) / kRowsPerBlock));
  const dim3 block(256);
  if (res == nullptr) {
    add_rmsnorm_kernel<VPL, false, false><<<grid, block, 0, s>>>(x, res, w, eps, T, H, out, res_out);
  } else if (res_out == nullptr) {
    add_rmsnorm_kernel<VPL, true, false><<<grid, block, 0, s>>>(x, res, w, eps, T, H, out, res_out);
  } else {
    add_rmsnorm_kernel<VPL, true, true><<<grid, block, 0, s>>>(x, res, w, eps, T, H, out, res_out);
  }
  return check_launch("cdx_add_rmsnorm_fwd");
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
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int nvec = H / 8;
  if (nvec <= 64) return launch_vpl<1>(x, residual, weight, eps, T, H, out, residual_out, s);
  if (nvec <= 128) return launch_vpl<2>(x, residual, weight, eps, T, H, out, residual_out, s);
  if (nvec <= 256) return launch_vpl<4>(x, residual, weight, eps, T, H, out, residual_out, s);
  if (nvec <= 512) return launch_vpl<8>(x, residual, weight, eps, T, H, out, residual_out, s);
  return launch_vpl<16>(x, residual, weight, eps, T, H, out, residual_out, s);
}
