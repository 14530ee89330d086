// MFMA tile engine shared by the mu-QKV projection and the MoE grouped GEMMs (gfx950).
//
// C[m, n] = sum_k A[m, k] * B[n, k]: both operands K-contiguous ("NT"), which is the
// natural layout of nn.Linear weights ([out, in]) and of packed expert weights.
//
// Block tile 256 x 256 x 64, 256 threads = 2 x 2 waves (one wave per SIMD), each wave
// owning a 128 x 128 sub-tile made of 4 x 4 blocks of 32 x 32 computed with
// v_mfma_f32_32x32x16_bf16 (256 fp32 accumulators per lane, held in AGPRs).
//
// Global -> LDS: direct-to-LDS loads (global_load_lds_dwordx4).  One wave instruction
// writes 64 x 16 bytes = 1 KB of LDS contiguously (lane i at base + 16 i), i.e. eight
// 128-byte tile rows.  The LDS tile is row-major, 128 bytes per row (64 bf16 of K),
// with 16-byte chunk c of row r stored at chunk position c ^ (r & 7); the swizzle is
// applied on the load side: lane i of a block fetches global chunk (i & 7) ^ (i >> 3)
// of row (i >> 3).  Fragment reads (32 rows x one chunk per half wave) then touch
// eight distinct chunk positions per eight lanes: no LDS bank conflicts.
//
// Pipeline (two LDS stages of 64 KB each; four K16 sub-steps per 64-wide K step):
//   sub-steps 0..2:  read the fragments of sub-step s+1 into the spare register set,
//                    then issue the 16 MFMAs of sub-step s.
//   sub-step 3:      wait for this wave's DMA of step k+1 (vmcnt(0)), barrier (now
//                    every wave's DMA landed and every wave finished reading stage
//                    k), issue the DMA of step k+2 into stage k, read sub-step 0 of
//                    step k+1, then issue the MFMAs of sub-step 3.
// One barrier per K step; its latency is covered by the MFMAs of sub-step 3, whose
// operands are already in registers.  The DMA of a step has a whole K step to land.
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

constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kBK = 64;
constexpr int kGemmThreads = 256;
constexpr int kGroupM = 4;
constexpr int kNumXcd = 8;

__device__ __forceinline__ int xcd_remap(int b, int nb) {
  const int q = nb / kNumXcd, r = nb % kNumXcd;
  const int xcd = b % kNumXcd, k = b / kNumXcd;
  return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + k;
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + __expf(-g)); }

// s_waitcnt immediate (gfx9 layout: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | ((lgkm & 15) << 8);
}

// 16 bytes from global memory straight into LDS at lds_block + 16 * lane.
__device__ __forceinline__ void dma16(const uint16_t* g, uint8_t* lds_block) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                   (__attribute__((address_space(3))) void*)lds_block, 16, 0, 0);
}

template <ALoad AL, Epi EP>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_nt_kernel(const GemmParams p) {
  constexpr int ROW_BYTES = kBK * 2;                // 128 bytes per tile row
  constexpr int TILE_BYTES = kBM * ROW_BYTES;       // 32 KB per operand and stage
  constexpr int STAGE_BYTES = 2 * TILE_BYTES;
  constexpr int WM = kBM / 2, WN = kBN / 2;
  constexpr int MI = WM / 32, NI = WN / 32;         // 4 x 4 blocks of 32 x 32
  constexpr int LD_PER_WAVE = kBM / 8 / 4;          // 1 KB DMA blocks per wave and operand: 8
  static_assert(kBM == kBN, "A and B tiles share the DMA layout");
  static_assert(EP != Epi::kSwiGLU || (WN % 64) == 0, "SwiGLU needs gate/up pairs per wave");

  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * STAGE_BYTES];

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
      const int ntile = (s1 - s0 + kBM - 1) / kBM;
      if (mt < before + ntile) {
        e = x;
        m0 = s0 + (int64_t)(mt - before) * kBM;
        m_end = s1;
        break;
      }
      before += ntile;
    }
    if (e < 0) return;
  } else {
    m0 = (int64_t)mt * kBM;
    m_end = p.M;
    if (m0 >= m_end) return;
  }
  const int n0 = nt * kBN;

  // ---- per-lane DMA sources ------------------------------------------------
  // Wave w fills tile rows [64 w, 64 w + 64) of both operands, eight rows per
  // instruction; lane i of instruction j covers row 64 w + 8 j + (i >> 3) and
  // fetches its swizzled chunk.
  const int dr = lane >> 3;
  const int dchunk = (lane & 7) ^ dr;
  const uint16_t* a_src[LD_PER_WAVE];
  const uint16_t* a2_src[LD_PER_WAVE];
  const uint16_t* b_src[LD_PER_WAVE];
  const uint16_t* bexp = p.b + (int64_t)e * p.b_estride;
#pragma unroll
  for (int j = 0; j < LD_PER_WAVE; ++j) {
    const int r = wave * 64 + j * 8 + dr;
    int64_t gm = m0 + r;
    gm = gm < m_end ? gm : m_end - 1;  // rows past the segment are loaded but never stored
    const int64_t row = (AL == ALoad::kGather) ? (int64_t)p.perm[gm] : gm;
    a_src[j] = p.a + row * p.lda + dchunk * 8;
    if (AL == ALoad::kConcat) a2_src[j] = p.a2 + row * p.lda2 + dchunk * 8;
    int n = n0 + r;
    n = n < p.N ? n : p.N - 1;
    b_src[j] = bexp + (int64_t)n * p.ldb + dchunk * 8;
  }
  const int dma_off = wave * 64 * ROW_BYTES;  // this wave's first 1 KB block in a tile

  auto issue = [&](int kt, int stage) __attribute__((always_inline)) {
    const int k0 = kt * kBK;
    uint8_t* As = lds + stage * STAGE_BYTES + dma_off;
    uint8_t* Bs = As + TILE_BYTES;
#pragma unroll
    for (int j = 0; j < LD_PER_WAVE; ++j) {
      const uint16_t* src;
      if (AL == ALoad::kConcat) {
        src = (k0 < p.k_split) ? a_src[j] + k0 : a2_src[j] + (k0 - p.k_split);
      } else {
        src = a_src[j] + k0;
      }
      dma16(src, As + j * 1024);
      dma16(b_src[j] + k0, Bs + j * 1024);
    }
  };

  // ---- fragments -------------------------------------------------------------
  // Row (lane & 31) of a 32-row block, chunk 2 s + (lane >> 5) for sub-step s.
  const int fr_row = lane & 31;
  int fr_off[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) fr_off[s] = fr_row * ROW_BYTES + (((2 * s + (lane >> 5)) ^ (fr_row & 7)) << 4);
  const int a_frag_base = wm * WM * ROW_BYTES;
  const int b_frag_base = TILE_BYTES + wn * WN * ROW_BYTES;

  bf16x8 fa[2][MI], fb[2][NI];
  auto read_frags = [&](int stage, int s, int set) __attribute__((always_inline)) {
    const uint8_t* base = lds + stage * STAGE_BYTES;
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
      fa[set][mi] = *reinterpret_cast<const bf16x8*>(base + a_frag_base + mi * 32 * ROW_BYTES + fr_off[s]);
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
      fb[set][ni] = *reinterpret_cast<const bf16x8*>(base + b_frag_base + ni * 32 * ROW_BYTES + fr_off[s]);
  };

  f32x16 acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][ni][v] = 0.f;

  auto mfmas = [&](int set) __attribute__((always_inline)) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[set][ni], fa[set][mi], acc[mi][ni], 0, 0, 0);
  };

  // ---- main loop --------------------------------------------------------------
  // Scheduling masks of __builtin_amdgcn_sched_group_barrier.
  constexpr int kSchedMfma = 0x008, kSchedVmem = 0x010, kSchedDsRead = 0x100;

  // Sub-steps 0..2 of a K step: MFMAs of sub-step s from register set s & 1, with
  // the eight fragment reads of sub-step s+1 slotted behind the first eight MFMAs,
  // so they have landed long before the next sub-step needs them.
  auto substep = [&](int stage, int s) __attribute__((always_inline)) {
    read_frags(stage, s + 1, (s + 1) & 1);
    mfmas(s & 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 8, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  // Sub-step 3: barrier, then its MFMAs (set 1) interleaved with the DMA of step
  // kt+2 into this stage and the reads of sub-step 0 of step kt+1 from the other.
  auto last_substep = [&](int kt, int stage, bool dma, bool next) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));  // own DMA of kt+1 landed, own reads done
    __syncthreads();
    if (dma) issue(kt + 2, stage);
    if (next) read_frags(stage ^ 1, 0, 0);
    mfmas(1);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedVmem, 1, 0);
      if (i < 8) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto kstep = [&](int kt, bool dma, bool next) __attribute__((always_inline)) {
    const int stage = kt & 1;
    substep(stage, 0);
    substep(stage, 1);
    substep(stage, 2);
    last_substep(kt, stage, dma, next);
  };

  const int KT = p.K / kBK;
  issue(0, 0);
  if (KT > 1) {
    issue(1, 1);
    // step 0's 2 * LD_PER_WAVE loads of this wave landed (step 1's may be in flight)
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(2 * LD_PER_WAVE, 15));
  } else {
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
  }
  __syncthreads();
  read_frags(0, 0, 0);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
  __builtin_amdgcn_sched_barrier(0);

  int kt = 0;
  for (; kt + 2 < KT; ++kt) kstep(kt, true, true);
  if (kt + 1 < KT) kstep(kt++, false, true);
  kstep(kt, false, false);

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
