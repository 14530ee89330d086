// Elementwise SwiGLU, out = silu(gate) * up, for the reference's operator API around
// the grouped GEMMs (gfx950).
//
// Reference behaviour:
//   cuda/triton_token_routed.py:163-188,234-257 (fused_swiglu_triton): silu in fp32,
//     rounded to the input dtype, then multiplied by up in that dtype
//     (round_silu = 1: two roundings, as F.silu(gate) * up does in bf16);
//   cuda/persistent_cggr.py:411-478 (fused_swiglu_simple): gate and up widened to fp32,
//     silu(gate) * up in fp32, one rounding (round_silu = 0).
// silu(g) = g / (1 + exp(-g)), evaluated in fp32.
//
// HBM-bound (reads 2n elements, writes n): each lane moves 16-byte vectors, a block of
// 256 lanes covers 4 KB of each operand per step and the grid strides over the rest;
// the ragged tail (n not a multiple of the vector) is done elementwise by block 0.
#include "cdx_common.h"

namespace cdx {
namespace {

enum : int { kBF16 = 0, kF16 = 1, kF32 = 2 };

template <int DT>
struct Elt;
template <>
struct Elt<kBF16> {
  typedef uint16_t T;
  static constexpr int kVec = 8;
  __device__ static float load(T v) { return bf16_bits_to_f32(v); }
  __device__ static T store(float f) { return f32_to_bf16_bits(f); }
};
template <>
struct Elt<kF16> {
  typedef uint16_t T;
  static constexpr int kVec = 8;
  __device__ static float load(T v) { return (float)__builtin_bit_cast(_Float16, v); }
  __device__ static T store(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
};
template <>
struct Elt<kF32> {
  typedef float T;
  static constexpr int kVec = 4;
  __device__ static float load(T v) { return v; }
  __device__ static T store(float f) { return f; }
};

template <int DT, bool ROUND>
__device__ __forceinline__ typename Elt<DT>::T swiglu1(typename Elt<DT>::T g, typename Elt<DT>::T u) {
  using E = Elt<DT>;
  const float gf = E::load(g);
  // The accurate expf (the kernel is bandwidth-bound): the fast form's relative error
  // grows with |g| and reaches several fp32 ulps of silu at |g| ~ 15.
  float s = gf / (1.0f + expf(-gf));
  if (ROUND) s = E::load(E::store(s));
  return E::store(s * E::load(u));
}

template <int DT, bool ROUND>
__global__ __launch_bounds__(256) void swiglu_kernel(const typename Elt<DT>::T* __restrict__ gate,
                                                     const typename Elt<DT>::T* __restrict__ up, int64_t n,
                                                     typename Elt<DT>::T* __restrict__ out) {
  using E = Elt<DT>;
  using T = typename E::T;
  constexpr int V = E::kVec;
  const int64_t nvec = n / V;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nvec; i += stride) {
    const uint4 g4 = reinterpret_cast<const uint4*>(gate)[i];
    const uint4 u4 = reinterpret_cast<const uint4*>(up)[i];
    const T* g = reinterpret_cast<const T*>(&g4);
    const T* u = reinterpret_cast<const T*>(&u4);
    uint4 o4;
    T* o = reinterpret_cast<T*>(&o4);
#pragma unroll
    for (int j = 0; j < V; ++j) o[j] = swiglu1<DT, ROUND>(g[j], u[j]);
    reinterpret_cast<uint4*>(out)[i] = o4;
  }
  if (blockIdx.x == 0) {
    for (int64_t i = nvec * V + threadIdx.x; i < n; i += blockDim.x) out[i] = swiglu1<DT, ROUND>(gate[i], up[i]);
  }
}

template <int DT>
int launch_swiglu(const void* gate, const void* up, int64_t n, bool round_silu, void* out, hipStream_t s) {
  using T = typename Elt<DT>::T;
  const int64_t nvec = n / Elt<DT>::kVec;
  // Enough blocks to keep every CU streaming (8 blocks of 256 lanes per CU), no more.
  const int64_t want = (nvec + 255) / 256;
  const unsigned blocks = (unsigned)(want < 1 ? 1 : (want > 2048 ? 2048 : want));
  if (round_silu)
    swiglu_kernel<DT, true><<<dim3(blocks), dim3(256), 0, s>>>(static_cast<const T*>(gate),
                                                                static_cast<const T*>(up), n, static_cast<T*>(out));
  else
    swiglu_kernel<DT, false><<<dim3(blocks), dim3(256), 0, s>>>(static_cast<const T*>(gate),
                                                                 static_cast<const T*>(up), n, static_cast<T*>(out));
  return check_launch("cdx_swiglu_fwd");
}

}  // namespace
}  // namespace cdx

extern "C" int cdx_swiglu_fwd(const void* gate, const void* up, int64_t n, int32_t dtype, int32_t round_silu,
                              void* out, void* stream) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_swiglu_fwd";
  if (n < 0) return fail(CDX_EINVAL, "%s: n=%lld must be >= 0", name, (long long)n);
  if (dtype != kBF16 && dtype != kF16 && dtype != kF32)
    return fail(CDX_EUNSUPPORTED, "%s: dtype code %d (0 bf16, 1 fp16, 2 fp32)", name, dtype);
  if (n == 0) return CDX_OK;
  if (!gate || !up || !out) return fail(CDX_EINVAL, "%s: null pointer", name);
  if (!aligned16(gate) || !aligned16(up) || !aligned16(out))
    return fail(CDX_EUNSUPPORTED, "%s: pointers must be 16-byte aligned", name);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case kBF16: return launch_swiglu<kBF16>(gate, up, n, round_silu != 0, out, s);
    case kF16: return launch_swiglu<kF16>(gate, up, n, round_silu != 0, out, s);
    default: return launch_swiglu<kF32>(gate, up, n, round_silu != 0, out, s);
  }
}
