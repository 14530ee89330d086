// Internal helpers shared by the gfx950 kernels of libcdx.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/cdx.h"

namespace cdx {

// ---- error reporting -------------------------------------------------------
// Sets the thread-local message returned by cdx_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// Checks hipGetLastError() after a launch; returns CDX_OK or CDX_ELAUNCH.
int check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Compute units of the current device (256 on MI355X, the fallback if the query fails),
// looked up once per device: launch paths call this several times per GEMM, and a
// small forward is paced by its host-side launch cost.
inline int device_cu_count() {
  constexpr int kMaxDev = 64;
  static int cached[kMaxDev] = {};  // 0 = not looked up yet (benign race: same value)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < kMaxDev) {
    const int c = __atomic_load_n(&cached[dev], __ATOMIC_RELAXED);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (dev >= 0 && dev < kMaxDev) __atomic_store_n(&cached[dev], cus, __ATOMIC_RELAXED);
  return cus;
}

// ---- bf16 <-> f32 ----------------------------------------------------------
typedef __bf16 bf16_t;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
// Round-to-nearest-even f32 -> bf16 bits (gfx950 lowers this to v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  bf16_t b = static_cast<bf16_t>(f);
  return __builtin_bit_cast(uint16_t, b);
}
// Two values in one v_cvt_pk_bf16_f32 (the same rounding as f32_to_bf16_bits).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) float f32x2_t;
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Eight bf16 sums a + b, each added in fp32 and rounded once (a bf16 tensor add).
__device__ __forceinline__ uint4 add_bf16x8(const uint4& a, const uint4& b) {
  const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
  uint32_t r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = __uint_as_float(aw[i] << 16) + __uint_as_float(bw[i] << 16);
    const float hi = __uint_as_float(aw[i] & 0xFFFF0000u) + __uint_as_float(bw[i] & 0xFFFF0000u);
    r[i] = pack_bf16x2(lo, hi);
  }
  return make_uint4(r[0], r[1], r[2], r[3]);
}
// 16-byte store with the non-temporal hint (streamed output that the kernel does
// not read back).
__device__ __forceinline__ void store_nt16(void* p, const uint4& v) {
  typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;
  const u32x4_t w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(p));
}

// Unpack the 8 bf16 values held in a 16-byte vector into floats.
__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ uint4 pack8(const float* f) {
  uint4 v;
  v.x = pack_bf16x2(f[0], f[1]);
  v.y = pack_bf16x2(f[2], f[3]);
  v.z = pack_bf16x2(f[4], f[5]);
  v.w = pack_bf16x2(f[6], f[7]);
  return v;
}

// ---- wavefront size --------------------------------------------------------
constexpr int kWave = 64;

}  // namespace cdx
