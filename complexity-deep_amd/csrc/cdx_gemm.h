// MFMA tile engine shared by the mu-QKV projection and the MoE grouped GEMMs (gfx950).
//
// C[m, n] = sum_k A[m, k] * B[n, k]: both operands K-contiguous ("NT"), which is the
// natural layout of nn.Linear weights ([out, in]) and of packed expert weights.
//
// Block tile BM x BN x 64, 256 threads = 2 x 2 waves, each wave owning a
// (BM/2) x (BN/2) sub-tile made of 32x32 blocks computed with
// v_mfma_f32_32x32x16_bf16 (fp32 accumulators).
//
// Data movement per K-step of 64:
//   global -> registers: every thread loads 16-byte chunks (8 bf16 along K); eight
//     consecutive threads cover one 128-byte row segment, so a wave reads eight full
//     rows per instruction.
//   registers -> LDS: rows of 128 bytes, 16-byte chunk c of row r stored at chunk
//     c ^ (r & 7).  The MFMA fragment reads (32 rows x one chunk per half-wave) then
//     touch eight different chunk positions per eight lanes: no bank conflicts.
//   LDS is double buffered; the global loads of step k+1 are in flight while the
//   MFMAs of step k run, and one barrier per step separates the phases.
//
// Operand order: the MFMA is issued as mfma(B_frag, A_frag), producing D = C^T for
// the 32x32 block.  In the gfx950 32x32 output layout lane l holds column l%32 and
// rows 8*(v/4) + 4*(l/32) + v%4 of D, i.e. one row m of C and four consecutive
// columns n per group of four accumulators, so the epilogue stores 8 contiguous bytes.
//
// Grid: one block per (M tile, N tile).  Block ids are first remapped so that the
// blocks the hardware sends to one XCD (round robin over 8 XCDs) form one contiguous
// range of logical tiles, then ordered in groups of kGroupM M-tiles so that the
// blocks resident on an XCD at the same time share A rows and B rows in its L2.
#pragma once

#include "cdx_common.h"

namespace cdx {

enum class ALoad { kDense, kConcat, kGather };
enum class Epi { kStore, kSwiGLU, kScatter };

struct GemmParams {
  // A operand
  const uint16_t* a;   // dense rows / x for concat / gather source
  int64_t lda;
  const uint16_t* a2;  // mu (concat); row stride lda2, 0 = broadcast one row
  int64_t lda2;
  int32_t k_split;     // first K index served by a2 (concat); == K when a2 unused
  const int32_t* perm; // sorted position -> token (gather rows / scatter rows)
  // segments (grouped GEMM); offsets == nullptr means one segment [0, M)
  const int32_t* offsets;
  int32_t E;
  int64_t M;
  // B operand: expert e uses b + e * b_estride, rows n with stride ldb
  const uint16_t* b;
  int64_t ldb;
  int64_t b_estride;
  int32_t N;
  int32_t K;
  // C
  uint16_t* c;
  int64_t ldc;
  // grid decomposition
  int32_t mt_count;  // number of M tiles (upper bound for grouped GEMMs)
  int32_t nt_count;
};

constexpr int kGroupM = 4;
constexpr int kNumXcd = 8;

__device__ __forceinline__ int xcd_remap(int b, int nb) {
  const int q = nb / kNumXcd, r = nb % kNumXcd;
  const int xcd = b % kNumXcd, k = b / kNumXcd;
  return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + k;
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + __expf(-g)); }

template <int BM, int BN, ALoad AL, Epi EP>
__global__ __launch_bounds__(256, 1) void gemm_nt_kernel(const GemmParams p) {
  constexpr int BK = 64;
  constexpr int ROW_BYTES = BK * 2;       // 128 bytes per tile row
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int MI = WM / 32, NI = WN / 32;
  constexpr int A_LD = BM * BK / 8 / 256;  // 16-byte chunks per thread per step
  constexpr int B_LD = BN * BK / 8 / 256;
  constexpr int A_BYTES = BM * ROW_BYTES, B_BYTES = BN * ROW_BYTES;
  static_assert(MI >= 1 && NI >= 1 && A_LD >= 1 && B_LD >= 1, "tile too small");
  static_assert(EP != Epi::kSwiGLU || (WN % 64) == 0, "SwiGLU needs gate/up pairs per wave");

  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * (A_BYTES + B_BYTES)];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // ---- tile decode -------------------------------------------------------
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int per_group = kGroupM * p.nt_count;
  const int group = L / per_group;
  const int first_m = group * kGroupM;
  const int gsz = min(p.mt_count - first_m, kGroupM);
  const int in_group = L - group * per_group;
  const int mt = first_m + in_group % gsz;
  const int nt = in_group / gsz;

  int64_t m0, m_end;
  int e = 0;
  if (p.offsets != nullptr) {
    int before = 0;
    e = -1;
    for (int x = 0; x < p.E; ++x) {
      const int s0 = p.offsets[x], s1 = p.offsets[x + 1];
      const int ntile = (s1 - s0 + BM - 1) / BM;
      if (mt < before + ntile) {
        e = x;
        m0 = s0 + (int64_t)(mt - before) * BM;
        m_end = s1;
        break;
      }
      before += ntile;
    }
    if (e < 0) return;
  } else {
    m0 = (int64_t)mt * BM;
    m_end = p.M;
    if (m0 >= m_end) return;
  }
  const int n0 = nt * BN;

  // ---- per-thread global source rows ----------------------------------------
  const int ld_row = tid >> 3;  // 0..31
  const int ld_chunk = tid & 7;
  const uint16_t* a_src[A_LD];
  const uint16_t* a2_src[A_LD];
#pragma unroll
  for (int i = 0; i < A_LD; ++i) {
    int64_t gm = m0 + ld_row + i * 32;
    gm = gm < m_end ? gm : m_end - 1;  // rows past the segment are loaded but never stored
    const int64_t row = (AL == ALoad::kGather) ? (int64_t)p.perm[gm] : gm;
    a_src[i] = p.a + row * p.lda + ld_chunk * 8;
    if (AL == ALoad::kConcat) a2_src[i] = p.a2 + row * p.lda2 + ld_chunk * 8;
  }
  const uint16_t* bexp = p.b + (int64_t)e * p.b_estride;
  const uint16_t* b_src[B_LD];
#pragma unroll
  for (int i = 0; i < B_LD; ++i) {
    int n = n0 + ld_row + i * 32;
    n = n < p.N ? n : p.N - 1;
    b_src[i] = bexp + (int64_t)n * p.ldb + ld_chunk * 8;
  }
  // LDS destination of this thread's chunks: row ld_row + 32 i, swizzled chunk.
  const int st_off = ld_row * ROW_BYTES + ((ld_chunk ^ (ld_row & 7)) << 4);

  uint4 ra[A_LD], rb[B_LD];
  auto gload = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const uint16_t* src;
      if (AL == ALoad::kConcat) {
        src = (k0 < p.k_split) ? a_src[i] + k0 : a2_src[i] + (k0 - p.k_split);
      } else {
        src = a_src[i] + k0;
      }
      ra[i] = *reinterpret_cast<const uint4*>(src);
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) rb[i] = *reinterpret_cast<const uint4*>(b_src[i] + k0);
  };
  auto sstore = [&](int buf) {
    uint8_t* As = lds + buf * (A_BYTES + B_BYTES);
    uint8_t* Bs = As + A_BYTES;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) *reinterpret_cast<uint4*>(As + st_off + i * 32 * ROW_BYTES) = ra[i];
#pragma unroll
    for (int i = 0; i < B_LD; ++i) *reinterpret_cast<uint4*>(Bs + st_off + i * 32 * ROW_BYTES) = rb[i];
  };

  f32x16 acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][ni][v] = 0.f;

  // Fragment read offsets: row (lane & 31) of a 32-row block, chunk 2 s + (lane >> 5).
  const int fr_row = lane & 31;
  int fr_off[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) fr_off[s] = fr_row * ROW_BYTES + (((2 * s + (lane >> 5)) ^ (fr_row & 7)) << 4);

  const int KT = p.K / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
    const uint8_t* As = lds + cur * (A_BYTES + B_BYTES) + wm * WM * ROW_BYTES;
    const uint8_t* Bs = lds + cur * (A_BYTES + B_BYTES) + A_BYTES + wn * WN * ROW_BYTES;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x8 af[MI], bfg[NI];
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
        af[mi] = *reinterpret_cast<const bf16x8*>(As + mi * 32 * ROW_BYTES + fr_off[s]);
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        bfg[ni] = *reinterpret_cast<const bf16x8*>(Bs + ni * 32 * ROW_BYTES + fr_off[s]);
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfg[ni], af[mi], acc[mi][ni], 0, 0, 0);
    }
    if (kt + 1 < KT) sstore(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue --------------------------------------------------------------
  const int hi = lane >> 5;
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
    const int64_t gm = m0 + wm * WM + mi * 32 + (lane & 31);
    if (gm >= m_end) continue;
    if constexpr (EP == Epi::kSwiGLU) {
      // Packed B rows come in groups of 64: 32 gate rows then the matching 32 up rows.
      uint16_t* crow = p.c + gm * p.ldc;
#pragma unroll
      for (int ni = 0; ni < NI; ni += 2) {
        const int nb = n0 + wn * WN + ni * 32;  // multiple of 64
        if (nb >= p.N) continue;
        const int colb = (nb >> 6) * 32;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float a4[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float gate = acc[mi][ni][4 * g + j];
            const float up = acc[mi][ni + 1][4 * g + j];
            a4[j] = silu_f32(gate) * up;
          }
          uint2 v;
          v.x = pack_bf16x2(a4[0], a4[1]);
          v.y = pack_bf16x2(a4[2], a4[3]);
          *reinterpret_cast<uint2*>(crow + colb + 8 * g + 4 * hi) = v;
        }
      }
    } else {
      const int64_t orow = (EP == Epi::kScatter) ? (int64_t)p.perm[gm] : gm;
      uint16_t* crow = p.c + orow * p.ldc;
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + wn * WN + ni * 32 + 8 * g + 4 * hi;
          if (n < p.N) {
            uint2 v;
            v.x = pack_bf16x2(acc[mi][ni][4 * g + 0], acc[mi][ni][4 * g + 1]);
            v.y = pack_bf16x2(acc[mi][ni][4 * g + 2], acc[mi][ni][4 * g + 3]);
            *reinterpret_cast<uint2*>(crow + n) = v;
          }
        }
      }
    }
  }
}

}  // namespace cdx
