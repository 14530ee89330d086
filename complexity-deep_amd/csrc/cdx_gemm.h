// MFMA tile engine shared by the mu-QKV projection and the MoE grouped GEMMs (gfx950).
//
// C[m, n] = sum_k A[m, k] * B[n, k]: both operands K-contiguous ("NT"), which is the
// natural layout of nn.Linear weights ([out, in]) and of packed expert weights.
//
// Block tile 256 x 256 (x BK = 64 per LDS stage), 256 threads = 2 x 2 waves (one wave
// per SIMD), each wave owning a 128 x 128 sub-tile made of 8 x 8 blocks of 16 x 16
// computed with v_mfma_f32_16x16x32_bf16 (256 fp32 accumulators per lane, in AGPRs).
// On random bf16 data this instruction sustains about 15% more throughput than the
// 32x32x16 form at the chip's power limit, for the same LDS traffic per flop.
//
// Global -> LDS: direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds).  One wave
// instruction writes 64 x 16 bytes = 1 KB of LDS contiguously (lane i at base + 16 i),
// i.e. eight 128-byte tile rows.  The LDS tile is row-major, 128 bytes per row (64
// bf16 of K), with 16-byte chunk c of row r stored at chunk position c ^ ((r / 2) % 8):
// the 16 rows that one 16-lane phase of a fragment read touches then cover all 64
// banks once.  The swizzle is applied on the load side (each lane fetches the global
// chunk that belongs at its LDS position).
//
// Pipeline (two LDS stages of 64 KB each; two K32 sub-steps per 64-wide K step):
//   sub-step 0:  the 64 MFMAs of sub-step 0, the 16 fragment reads of sub-step 1
//                slotted behind the first of them;
//   sub-step 1:  wait for this wave's DMA of step k+1 (vmcnt), barrier (now every
//                wave's DMA landed and every wave finished reading stage k), then the
//                MFMAs of sub-step 1 with the DMA of step k+2 into stage k and the
//                fragment reads of step k+1's sub-step 0 slotted behind them.
// One barrier per K step; its latency is covered by MFMAs whose operands are already
// in registers.  The DMA of a step has a whole K step to land.
//
// Operand order: the MFMA is issued as mfma(B_frag, A_frag), producing D = C^T for
// the 16x16 block.  In the 16x16 output layout lane l holds column l%16 and rows
// 4*(l/16) .. 4*(l/16)+3 of D, i.e. one row m of C and four consecutive columns n.
// The epilogue stages the bf16 results through LDS and stores whole row segments,
// 16 bytes per lane.
//
// Grid: one block per (M tile, N tile).  Block ids are first remapped so that the
// blocks the hardware sends to one XCD (round robin over 8 XCDs) form one contiguous
// range of logical tiles, then ordered in groups of kGroupM M-tiles so that the
// blocks resident on an XCD at the same time share A rows and B rows in its L2.
#pragma once

#include "cdx_common.h"

namespace cdx {

// kSegmented (the MoE down pass): M tiles of kBM consecutive sorted rows regardless of
// the expert segments (offsets); a tile runs the shared K columns [0, k_split) once
// for all its rows, then the expert columns [k_split, K) once per expert it touches,
// with that expert's B and the other experts' A rows read as zeros.  No tile is
// padded to an expert boundary, so the grid holds ceil(M / kBM) M tiles.
enum class ALoad { kDense, kConcat, kGather, kSegmented };
// kScatterAdd: like kScatter, but the scattered rows are added to what C holds (the
// caller's residual stream, updated in place) with one bf16 rounding of the sum.
enum class Epi { kStore, kSwiGLU, kScatter, kQKRope, kBiasClamp, kScatterAdd };

// Parameters of the kQKRope epilogue (mu-QKV with QK RMSNorm and RoPE fused): the
// packed [M, (nq + 2 nkv) * HD] projection is never stored; q, k and v go straight
// to head-major [B, heads, S, HD] buffers, q and k normalised and rotated.
struct QKRopeParams {
  int64_t S;                 // tokens per sequence; row m is token (m / S, m % S)
  int32_t nq, nkv;           // query and key/value heads
  const uint16_t* q_norm_w;  // [HD] bf16, nullptr = no QK RMSNorm
  const uint16_t* k_norm_w;  // [HD] bf16
  float eps;
  const float* cos_sin;      // [pos][HD/2] (cos, sin) pairs, fp32
  int64_t pos0;              // position of token s = 0 (KV-cache length)
  uint16_t* q_out;           // [B, nq, S, HD]
  uint16_t* k_out;           // [B, nkv, S, HD]
  uint16_t* v_out;           // [B, nkv, S, HD], or transposed (vt_ld > 0)
  // vt_ld > 0: v_out is V transposed for the attention kernel, [B, nkv, HD, vt_ld]
  // (vt_ld >= S, a multiple of 64), with token s stored at column vt_col(s).
  int64_t vt_ld;
};

// Column of token s in the transposed V layout: inside every group of 16 tokens the
// middle two quads swap places (s = 16 u + 4 q + j -> 16 u + 4 sigma(q) + j, sigma =
// (0 2 1 3)).  The attention kernel's P fragments hold, per lane half, keys
// {16 u + 4 h + j, 16 u + 8 + 4 h + j}; this order makes those eight keys one
// contiguous 16-byte run of a V^T row.
__host__ __device__ __forceinline__ int64_t vt_col(int64_t s) {
  const int64_t q = (s >> 2) & 3;
  const int64_t qs = q == 1 ? 2 : (q == 2 ? 1 : q);
  return (s & ~int64_t(15)) + 4 * qs + (s & 3);
}

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
  // concat: B columns [k_split, K) come from b2 (rows n, stride ldb).
  // Scatter epilogues (the MoE down pass): b2 is the shared expert's [N][ldb] block,
  // which serves K columns [0, k_split); expert e serves [k_split, K) from its own
  // block b + e * b_estride, whose column 0 is K column k_split.
  const uint16_t* b2;
  int64_t ldb;
  int64_t b_estride;
  // kSwiGLU (the MoE gate/up pass): b is the [blocks][2][gu_P][ldb] weights, gate rows
  // then up rows of each block; block 0 is the shared expert when gu_shared, then one
  // block per routed expert (gu_tile maps a tile's logical rows onto them).
  int32_t gu_P;
  int32_t gu_shared;
  int32_t N;
  int32_t K;
  // C
  uint16_t* c;
  int64_t ldc;
  // grid decomposition
  int32_t mt_count;  // number of M tiles (upper bound for grouped GEMMs)
  int32_t nt_count;
  QKRopeParams qk;  // kQKRope epilogue only
  // kBiasClamp epilogue: c = clamp(acc + clamp(bias[n], bias_lo, bias_hi), lo, hi)
  const uint16_t* bias;  // [N] bf16
  float bias_lo, bias_hi;
  float lo, hi;
};

constexpr int kBM = 256;
constexpr int kGemmThreads = 256;
#ifndef CDX_GROUP_M
#define CDX_GROUP_M 4
#endif
constexpr int kGroupM = CDX_GROUP_M;  // M tiles per group in the tile order
constexpr int kNumXcd = 8;

// Tile configuration: BN output columns per block, BK-deep LDS stages, STAGES of
// them in flight, compiled for MINB blocks per CU (the launch bound, which sets the
// register budget; RESIDENT blocks fit the LDS at once).  Stage s holds the A (256 x BK) and B
// (BN x BK) tiles of one K step; the DMA of step k + STAGES is issued as soon as
// stage k is consumed, so a load has STAGES - 1 K steps to land.
// DMA_EVERY / DMA_OFF place the refill DMA instructions of a K step behind MFMAs
// DMA_OFF, DMA_OFF + DMA_EVERY, ... of its last sub-step (1, 0 = a burst behind the
// first ones); READ_EVERY likewise spaces the fragment reads.
// BM rows per tile: 256 (waves of 128 rows), or 128 (waves of 64 rows) for products
// whose 256-row tiles leave most CUs idle.  The tile shape does not change any output
// element's accumulation (the same MFMAs over the same K order), so every shape gives
// the same bits.
template <int BN_, int BK_, int STAGES_, int MINB_, int DMA_EVERY_ = 1, int DMA_OFF_ = 0, int READ_EVERY_ = 1,
          int BM_ = kBM>
struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, STAGES = STAGES_, MINB = MINB_;
  static constexpr int DMA_EVERY = DMA_EVERY_, DMA_OFF = DMA_OFF_, READ_EVERY = READ_EVERY_;
  static_assert(DMA_OFF < DMA_EVERY, "DMA slot offset must be below its spacing");
  static_assert(BM == 256 || BM == 128, "BM must be 128 or 256");
  static_assert(BN == 256 || BN == 128 || BN == 64, "BN must be 64, 128 or 256");
  static_assert(BK == 64, "BK must be 64 (two K32 sub-steps per stage)");
  static constexpr int STAGE_BYTES = (BM + BN) * BK * 2;
  static_assert(STAGES >= 2 && STAGES * STAGE_BYTES <= 160 * 1024, "stages must fit 160 KB of LDS");
  static constexpr int RESIDENT = (160 * 1024) / (STAGES * STAGE_BYTES) < MINB ? (160 * 1024) / (STAGES * STAGE_BYTES)
                                                                                : MINB;
};
#ifndef CDX_GEMM_CFG
#define CDX_GEMM_CFG 256, 64, 2, 1, 4, 1, 1
#endif
using DefaultCfg = GemmCfg<CDX_GEMM_CFG>;

// Logical tile of block b when `tiles` real tiles run on a grid of at least that many
// blocks: the hardware deals blocks to the XCDs round robin (XCD b % 8), so XCD x
// gets an equal share of the real tiles as one contiguous logical range (its L2 then
// serves neighbouring tiles).  Blocks beyond their XCD's share get -1.
__device__ __forceinline__ int xcd_remap(int b, int tiles) {
  const int q = tiles / kNumXcd, r = tiles % kNumXcd;
  const int xcd = b % kNumXcd, k = b / kNumXcd;
  if (k >= q + (xcd < r ? 1 : 0)) return -1;
  return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + k;
}

// g * sigmoid(g) with the hardware reciprocal (1 ulp) in place of an IEEE division,
// which costs about ten vector instructions per element; the result is rounded to
// bf16 afterwards.  exp(-g) overflowing to +inf gives rcp = 0 and silu = -0.
__device__ __forceinline__ float silu_f32(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// Four bf16 bias values (8 bytes) as fp32, each clamped to [lo, hi] (the clamp on the
// mu parameter, core/layer.py:60, applied where the epilogue reads it).
__device__ __forceinline__ float4 load_bias4(const uint16_t* src, float lo, float hi) {
  const uint2 w = *reinterpret_cast<const uint2*>(src);
  auto cl = [&](float v) __attribute__((always_inline)) { return fminf(fmaxf(v, lo), hi); };
  return make_float4(cl(__uint_as_float(w.x << 16)), cl(__uint_as_float(w.x & 0xffff0000u)),
                     cl(__uint_as_float(w.y << 16)), cl(__uint_as_float(w.y & 0xffff0000u)));
}

// s_waitcnt immediate (gfx9 layout: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | ((lgkm & 15) << 8);
}

// Raw buffer descriptor over [base, base + records): stride 0, 32-bit data format
// (descriptor word 3 = 0x00020000, the gfx9 layout).  The default range passes every
// 32-bit offset; records = 0 makes every access out of range, so a load through it
// fetches nothing and returns zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t records = 0xFFFFFFFFu) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)records, 0x00020000);
}

// 16 bytes per lane from buffer offset voff + soff straight into LDS at
// lds_block + 16 * lane (buffer_load_dwordx4 ... lds).
__device__ __forceinline__ void buf_dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                          uint8_t* lds_block) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_block, 16, voff, soff,
                                           0, 0);
}

// kSwiGLU B tiles.  Logical row n of expert e's gate/up operand (n < S * 2P, S = 2
// with the shared expert, else 1) is in block n / (2P) of the expert's sequence
// (shared block, then its own); inside it, w = n % (2P) is the gate (w / 32 even) or
// up row of unit (w / 64) * 32 + w % 32, so that a tile's rows interleave 32 gate rows
// with the 32 up rows of the same units.  Storage keeps gate and up rows in unit
// order ([blocks][2][P][H]), which is what makes the module's weight Parameters views
// of the operand.  For a tile starting at logical row n0 (a multiple of 128; P is a
// multiple of 64), row r < BN sits at
//     lo + gu_row(r) * ldb            for r <  split
//     hi + gu_row(r) * ldb            for r >= split
// with gu_row(r) = ((r / 32) % 2) * P + (r / 64) * 32 + r % 32 and split, a multiple of
// 128, where the tile crosses into the next block (tiles past the last block read
// rows of that block again: computed, never stored).  A DMA instruction's eight rows
// never straddle split, so the choice of base is one scalar select per instruction.
struct GuTile {
  uintptr_t lo, hi;
  int split;
};
__device__ __forceinline__ int gu_row(int r, int P) { return ((r >> 5) & 1) * P + (r >> 6) * 32 + (r & 31); }
__device__ __forceinline__ GuTile gu_tile(const uint16_t* b, int64_t ldb, int P, bool shared, int e, int n0) {
  const int twoP = 2 * P;
  const int bl = n0 / twoP;
  const int w0 = n0 - bl * twoP;
  const int last = shared ? 1 : 0;
  const int64_t blk_lo = shared && bl == 0 ? 0 : last + e;
  const int64_t blk_hi = last + e;  // the next block, when bl == 0 and there is one
  GuTile t;
  t.split = twoP - w0;
  t.lo = (uintptr_t)(b + (blk_lo * twoP + w0 / 2) * ldb);
  t.hi = bl < last ? (uintptr_t)(b + (blk_hi * twoP - t.split / 2) * ldb)
                   : (uintptr_t)(b + (blk_lo * twoP + w0 / 2 - t.split / 2) * ldb);
  return t;
}

// ---- QK-norm + RoPE epilogue pieces (shared by the engine's two kernel forms) ----
// For one 16-row block of one head: lane l holds row l & 15 and, in x[nb][0..3], the
// head's columns 16 nb + 4 (l >> 4) + (0..3) (lanes l, l ^ 16, l ^ 32, l ^ 48 together
// hold the row's HD = 16 BPH values).  In place: RMSNorm over the head (weights wf,
// all ones and a unit scale without QK norm), then RoPE on each pair (c, c + HD/2),
// whose elements sit in blocks nb and nb + BPH/2 of the same lane:
//   y[c] = x[c] cos - x[c + HD/2] sin,  y[c + HD/2] = x[c + HD/2] cos + x[c] sin,
// with cs[nb] the (cos, sin) pairs of this lane's first-half columns for its row.
template <int BPH>
__device__ __forceinline__ void qk_norm_rope(float (&x)[BPH][4], const float (&wf)[BPH][4],
                                             const float4 (&cs)[BPH / 2][2], bool norm, float eps) {
  // Four independent partial sums keep the chain short; the partners' sums come in
  // through a swizzle (l ^ 16) and v_permlane32_swap (l ^ 32), neither touching LDS.
  float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int nb = 0; nb < BPH; ++nb)
#pragma unroll
    for (int v = 0; v < 4; ++v) s4[v] = __builtin_fmaf(x[nb][v], x[nb][v], s4[v]);
  float ss = (s4[0] + s4[1]) + (s4[2] + s4[3]);
  // ds_swizzle bit mode, and-mask 0x1f, xor-mask 0x10: lane l reads lane l ^ 16.
  ss += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(ss), 0x401F));
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
  ss = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  // ss / HD + eps >= eps > 0 is a normal number: the plain hardware reciprocal square
  // root needs no denormal scaling.  Without QK norm the weights are 1 and the scale
  // is 1: both products are then exact, and there is no branch between the norm and
  // the rotation (a branch there made the compiler pass the values through AGPRs).
  const float rs = norm ? __builtin_amdgcn_rsqf(ss / (float)(16 * BPH) + eps) : 1.f;
#pragma unroll
  for (int nb = 0; nb < BPH; ++nb)
#pragma unroll
    for (int j = 0; j < 4; ++j) x[nb][j] = wf[nb][j] * (x[nb][j] * rs);
#pragma unroll
  for (int nb = 0; nb < BPH / 2; ++nb) {
    const float4 t01 = cs[nb][0], t23 = cs[nb][1];
    const float cv[4] = {t01.x, t01.z, t23.x, t23.z};
    const float sv[4] = {t01.y, t01.w, t23.y, t23.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // Explicit FMAs: the contraction is then the same wherever this is inlined.
      const float a = x[nb][j], bq = x[nb + BPH / 2][j];
      x[nb][j] = __builtin_fmaf(a, cv[j], -(bq * sv[j]));
      x[nb + BPH / 2][j] = __builtin_fmaf(bq, cv[j], a * sv[j]);
    }
  }
}

// V^T quad transpose: lanes 4j + t (same l >> 4) hold tokens 4j + t of dims
// 4 (l >> 4) + (0..3) in x0..x3; afterwards lane 4j + t holds dim 4 (l >> 4) + t of
// tokens 4j + (0..3), as two packed bf16 pairs, after two exchanges (lane t ^ 1, then
// t ^ 2) over the quad.
__device__ __forceinline__ uint2 vt_quad_transpose(float x0, float x1, float x2, float x3, int lane) {
  const int t = lane & 3;
  const bool odd = t & 1, upper = t & 2;
  const uint32_t p0 = pack_bf16x2(x0, x1), p1 = pack_bf16x2(x2, x3);
  // first exchange: even lanes give dims 1, 3 and keep 0, 2; odd lanes the reverse.
  const uint32_t give = __builtin_amdgcn_perm(p1, p0, odd ? 0x05040100u : 0x07060302u);
  const uint32_t got = (uint32_t)__builtin_amdgcn_mov_dpp((int)give, 0xB1, 0xF, 0xF, true);
  const uint32_t a0 = __builtin_amdgcn_perm(got, p0, odd ? 0x03020504u : 0x05040100u);
  const uint32_t a1 = __builtin_amdgcn_perm(got, p1, odd ? 0x03020706u : 0x07060100u);
  // second exchange: lanes t < 2 give their second pair, t >= 2 their first.
  const uint32_t give2 = upper ? a0 : a1;
  const uint32_t got2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)give2, 0x4E, 0xF, 0xF, true);
  uint2 w;
  w.x = upper ? got2 : a0;  // tokens 4j, 4j + 1
  w.y = upper ? a1 : got2;  // tokens 4j + 2, 4j + 3
  return w;
}

template <class Cfg, ALoad AL, Epi EP, int HD = 0>
__global__ __launch_bounds__(kGemmThreads, Cfg::MINB) void gemm_nt_kernel(const GemmParams p) {
  constexpr int kBN = Cfg::BN, kBK = Cfg::BK, kStages = Cfg::STAGES;
  constexpr int kTM = Cfg::BM;                      // rows per tile
  constexpr int ROW_BYTES = kBK * 2;                // bytes per tile row in LDS
  constexpr int CPR = kBK / 8;                      // 16-byte chunks per row
  constexpr int RPL = 256 / ROW_BYTES;              // rows per 256-byte bank line (64 banks)
  constexpr int A_TILE_BYTES = kTM * ROW_BYTES;     // one stage of A
  constexpr int STAGE_BYTES = Cfg::STAGE_BYTES;     // A then B
  constexpr int WM = kTM / 2, WN = kBN / 2;
  constexpr int MI = WM / 16, NI = WN / 16;         // blocks of 16 x 16 per wave
  constexpr int ROWS_PER_DMA = 1024 / ROW_BYTES;    // rows one wave instruction fills
  constexpr int LD_A = kTM / ROWS_PER_DMA / 4;      // DMA instructions per wave and K step, A
  constexpr int LD_B = kBN / ROWS_PER_DMA / 4;      // and B
  constexpr int LD_PER_STEP = LD_A + LD_B;
  constexpr int NSUB = kBK / 32;                    // K32 sub-steps per K step
  constexpr int NFRAG = MI + NI;                    // fragment reads per sub-step
  constexpr int DMA_EVERY = Cfg::DMA_EVERY, DMA_OFF = Cfg::DMA_OFF, RD_EVERY = Cfg::READ_EVERY;
  static_assert(LD_B >= 1, "B tile too small for the DMA layout");
  static_assert(NSUB % 2 == 0, "fragment register sets alternate per sub-step: K step must hold an even count");
  static_assert(EP != Epi::kSwiGLU || (WN % 64) == 0, "SwiGLU needs gate/up pairs per wave");
  static_assert(LD_PER_STEP * (kStages - 1) <= 63, "vmcnt range");

  // Scatter epilogues: after the stages, the output row (permutation entry) of each of
  // the tile's kTM rows, loaded in the prologue.
  constexpr bool kScatterRows = EP == Epi::kScatter || EP == Epi::kScatterAdd;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * STAGE_BYTES + (kScatterRows ? kTM * 4 : 0)];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave-uniform, so LDS addresses (the DMA's M0 in particular) stay scalar.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // ---- tile decode -------------------------------------------------------
  // Segment offsets are read clamped to [0, M] and a segment that ends before it
  // starts is empty, so that offsets that are not a valid plan (the C-ABI cannot check
  // device data) give wrong rows but no access outside the operands.
  auto seg_off = [&](int x) __attribute__((always_inline)) {
    const int v = p.offsets[x];
    return v < 0 ? 0 : (v > (int)p.M ? (int)p.M : v);
  };
  // Grouped GEMMs launch an upper bound of M tiles; the real count follows from the
  // segment offsets, so that the surplus blocks neither take an XCD's share nor sit
  // in the middle of the logical order.
  int mt_real = p.mt_count;
  if (AL != ALoad::kSegmented && p.offsets != nullptr) {
    mt_real = 0;
    for (int x = 0; x < p.E; ++x) mt_real += max(0, (seg_off(x + 1) - seg_off(x) + kTM - 1) / kTM);
    mt_real = min(mt_real, p.mt_count);
  }
  const int L = xcd_remap(blockIdx.x, mt_real * p.nt_count);
  if (L < 0) return;
  const int per_group = kGroupM * p.nt_count;
  const int group = L / per_group;
  const int first_m = group * kGroupM;
  const int gsz = min(mt_real - first_m, kGroupM);
  const int in_group = L - group * per_group;
  // The divisions above run on the vector unit; pinning the tile indices to scalar
  // registers keeps every descriptor built from them scalar (a descriptor operand in
  // vector registers turns each DMA into a loop over lanes).
  const int mt = __builtin_amdgcn_readfirstlane(first_m + in_group % gsz);
  const int nt = __builtin_amdgcn_readfirstlane(in_group / gsz);

  // The tile computes rows [m0, m0 + kTM) and stores rows [m_lo, m_end).
  int64_t m0, m_end, m_lo;
  int e = 0;
  int e_lo = 0, n_exp = 1;  // kSegmented: first expert of the tile, experts it touches
  // kSegmented: lane x holds segment start offsets[x] for x < E (E <= 64), read in one
  // vector load instead of a chain of scalar ones; the tile's experts follow by ballots.
  int seg_lane = 0;
  if constexpr (AL == ALoad::kSegmented) {
    // Rows outside [offsets[0], offsets[E]) belong to no expert and are not stored.
    m0 = (int64_t)mt * kTM;
    seg_lane = lane < p.E ? seg_off(lane) : (int)p.M;
    m_lo = max(m0, (int64_t)__builtin_amdgcn_readfirstlane(seg_lane));
    m_end = min(min(p.M, m0 + kTM), (int64_t)__builtin_amdgcn_readfirstlane(seg_off(p.E)));
    if (m_lo >= m_end) return;
    // Experts holding rows m_lo and m_end - 1: for consecutive sorted segments, the
    // number of segments after the first that start at or before the row (a segment
    // that is empty or out of order gives wrong rows, never an expert outside [0, E)).
    // (Pinned to scalar registers: the B descriptor is built from e_lo.)
    const bool mid = lane >= 1 && lane < p.E;
    e_lo = __builtin_amdgcn_readfirstlane(__builtin_popcountll(__builtin_amdgcn_ballot_w64(mid && seg_lane <= m_lo)));
    const int e_hi =
        __builtin_amdgcn_readfirstlane(__builtin_popcountll(__builtin_amdgcn_ballot_w64(mid && seg_lane <= m_end - 1)));
    n_exp = max(1, e_hi - e_lo + 1);
  } else if (p.offsets != nullptr) {
    int before = 0;
    e = -1;
    for (int x = 0; x < p.E; ++x) {
      const int s0 = seg_off(x), s1 = seg_off(x + 1);
      const int ntile = max(0, (s1 - s0 + kTM - 1) / kTM);
      if (mt < before + ntile) {
        e = x;
        m0 = s0 + (int64_t)(mt - before) * kTM;
        m_end = s1;
        break;
      }
      before += ntile;
    }
    if (e < 0) return;
    m_lo = m0;
  } else {
    m0 = (int64_t)mt * kTM;
    m_end = p.M;
    m_lo = m0;
    if (m0 >= m_end) return;
  }
  const int n0 = nt * kBN;

  // ---- per-lane DMA sources ------------------------------------------------
  // LDS rows are ROW_BYTES long; 16-byte chunk c of tile row r sits at chunk
  // position c ^ ((r / RPL) % CPR).  The LDS serves a 128-bit read 16 lanes at a
  // time from 64 banks (256 bytes); the 16 rows one fragment read touches per 16
  // lanes then cover every bank exactly once.  The swizzle is applied on the load
  // side: lane i of a DMA instruction fills position i % CPR of row i / CPR of its
  // 1 KB block and therefore fetches global chunk (i % CPR) ^ ((row / RPL) % CPR).
  // Wave w fills rows [64 w, 64 w + 64) of both operands.
  // The DMA goes through buffer descriptors: each lane's byte offset inside its
  // operand is fixed for the whole K loop and the K position travels in the
  // instruction's scalar offset, so a DMA costs no vector instruction.  Dense and
  // concat A and B offsets are relative to the tile's first row (< 4 GB for any
  // practical leading dimension); gathered A offsets are relative to the matrix,
  // which the host bounds to 4 GB.  The concat descriptors' bases (mu for A, the mu
  // weights for B) sit k_split columns before their first column, so that both halves
  // of K take the same scalar offset (2 k0) and the choice between the two sources is
  // a select, not a branch.
  const int dr = lane / CPR;
  constexpr bool kGuTiles = EP == Epi::kSwiGLU;
  // Scatter epilogues on per-expert tiles (the down pass, kDense): K columns below
  // k_split come from the shared block b2.
  constexpr bool kSharedB = kScatterRows && AL == ALoad::kDense;
  const uint16_t* bexp = p.b + (int64_t)e * p.b_estride;
  const uintptr_t a_base = (uintptr_t)(AL == ALoad::kGather ? p.a : p.a + m0 * p.lda);
  const uintptr_t a2_base =
      AL == ALoad::kConcat ? (uintptr_t)(p.a2 + m0 * p.lda2) - (uintptr_t)p.k_split * 2 : a_base;
  // kSegmented: the A descriptor covers the tile's rows only, so that a masked row's
  // offset (kMaskedOff) reads zeros; each row remembers its expert (-1 past m_end).
  const __amdgpu_buffer_rsrc_t rs_a =
      AL == ALoad::kSegmented ? make_rsrc((const void*)a_base, (uint32_t)((m_end - m0) * p.lda * 2))
                              : make_rsrc((const void*)a_base);
  // SwiGLU tiles: this wave's B rows come from before or after the tile's block switch
  // (gu_tile).  The switch row is a multiple of 128 and a wave's B rows one aligned run
  // of BN / 4 (64, 32 or 16) rows, so they all lie on one side of it: one descriptor
  // for the whole K loop.
  const __amdgpu_buffer_rsrc_t rs_b = [&]() __attribute__((always_inline)) {
    if constexpr (kGuTiles) {
      const GuTile gu = gu_tile(p.b, p.ldb, p.gu_P, p.gu_shared != 0, e, n0);
      return make_rsrc((const void*)(wave * (kBN / 4) >= gu.split ? gu.hi : gu.lo));
    } else {
      return make_rsrc(bexp + (int64_t)n0 * p.ldb);
    }
  }();
  // kSharedB: b_base serves the expert columns (column 0 = K column k_split), b2_base
  // the shared ones.
  const uintptr_t b_base =
      (uintptr_t)(bexp + (int64_t)n0 * p.ldb) - (kSharedB ? (uintptr_t)p.k_split * 2 : (uintptr_t)0);
  const uintptr_t b2_base =
      AL == ALoad::kConcat ? (uintptr_t)(p.b2 + (int64_t)n0 * p.ldb) - (uintptr_t)p.k_split * 2
                           : (kSharedB && p.b2 != nullptr ? (uintptr_t)(p.b2 + (int64_t)n0 * p.ldb) : b_base);
  constexpr uint32_t kMaskedOff = 0x80000000u;
  uint32_t a_off[LD_A], a2_off[LD_A], b_off[LD_B];
  int a_exp[AL == ALoad::kSegmented ? LD_A : 1];
#pragma unroll
  for (int j = 0; j < LD_A; ++j) {
    const int r = wave * (kTM / 4) + j * ROWS_PER_DMA + dr;
    const int dchunk = (lane % CPR) ^ ((r / RPL) % CPR);
    int64_t gm = m0 + r;
    if constexpr (AL == ALoad::kSegmented) {
      int ex = -1;
      if (gm >= m_lo && gm < m_end) {
        ex = e_lo;
        for (int x = e_lo + 1; x < e_lo + n_exp; ++x) ex += __builtin_amdgcn_readlane(seg_lane, x) <= gm ? 1 : 0;
      }
      a_exp[j] = ex;
    }
    gm = gm < m_end ? gm : m_end - 1;  // rows past the segment are loaded but never stored
    if (AL == ALoad::kGather) {
      // A permutation entry outside [0, M) is clamped into it (negative entries wrap
      // to large unsigned values first): a corrupt permutation reads wrong rows but
      // stays inside the operand.  The host bounds M * lda * 2 to 4 GB.  (This kernel
      // runs at the register limit: a select here pushed the compiler into moving
      // values through AGPRs inside the K loop.)
      const uint32_t src = min((uint32_t)p.perm[gm], (uint32_t)(p.M - 1));
      a_off[j] = (src * (uint32_t)p.lda + (uint32_t)dchunk * 8u) * 2u;
    } else {
      a_off[j] = (uint32_t)(((gm - m0) * p.lda + dchunk * 8) * 2);
    }
    a2_off[j] = AL == ALoad::kConcat ? (uint32_t)(((gm - m0) * p.lda2 + dchunk * 8) * 2) : 0u;
  }
#pragma unroll
  for (int j = 0; j < LD_B; ++j) {
    const int r = wave * (kBN / 4) + j * ROWS_PER_DMA + dr;
    const int dchunk = (lane % CPR) ^ ((r / RPL) % CPR);
    if constexpr (kGuTiles) {
      b_off[j] = (uint32_t)(((int64_t)gu_row(r, p.gu_P) * p.ldb + dchunk * 8) * 2);
    } else {
      int n = n0 + r;
      n = n < p.N ? n : p.N - 1;
      b_off[j] = (uint32_t)(((int64_t)(n - n0) * p.ldb + dchunk * 8) * 2);
    }
  }
  const int a_dma_off = wave * (kTM / 4) * ROW_BYTES;  // this wave's first DMA block in A
  const int b_dma_off = A_TILE_BYTES + wave * (kBN / 4) * ROW_BYTES;

  // Where K step kt reads: k0 = its first K column (the same for A and B), and for
  // kSegmented the expert whose columns and B it is (-1: the shared columns).
  // Steps past the end (kt >= KT) go through the empty descriptor: the pipeline
  // issues the same instructions every step, and those fetch nothing.
  const int ks0 = AL == ALoad::kSegmented ? p.k_split / kBK : 0;          // shared K steps
  const int ks1 = AL == ALoad::kSegmented ? (p.K - p.k_split) / kBK : 1;  // K steps per expert
  const int KT = AL == ALoad::kSegmented ? ks0 + n_exp * ks1 : p.K / kBK;
  const __amdgpu_buffer_rsrc_t rs_none = make_rsrc(p.b, 0u);
  struct StepSrc {
    int k0;
    int e;
    bool live;
  };
  auto step_src = [&](int kt) __attribute__((always_inline)) { return StepSrc{kt * kBK, -1, kt < KT}; };
  // kSegmented: the DMA steps are issued in order, so their sources advance by scalar
  // selects instead of a division per step: the shared columns, then each expert's.
  StepSrc seg_next{ks0 > 0 ? 0 : p.k_split, ks0 > 0 ? -1 : e_lo, true};
  int seg_step = 0;
  // B of the step: the shared block b2 for the shared columns, else the step's expert
  // block (addressed so that K column k_split is its column 0), or the empty
  // descriptor past the end.  Kept as addresses, not as descriptors: a loop-carried
  // descriptor is not kept in scalar registers.
  const uintptr_t b_estep = (uintptr_t)p.b_estride * 2;
  const uintptr_t seg_sptr = AL == ALoad::kSegmented && p.b2 != nullptr ? (uintptr_t)(p.b2 + (int64_t)n0 * p.ldb) : 0;
  uintptr_t seg_bptr = (uintptr_t)(p.b + (int64_t)n0 * p.ldb + (int64_t)e_lo * p.b_estride) - (uintptr_t)p.k_split * 2;
  auto seg_advance = [&]() __attribute__((always_inline)) {
    const int k1 = seg_next.k0 + kBK;
    const bool shared = seg_next.e < 0;
    const bool wrap = shared ? k1 >= p.k_split : k1 >= p.K;
    const bool next_e = wrap && !shared;
    seg_next.e = wrap ? (shared ? e_lo : seg_next.e + 1) : seg_next.e;
    seg_next.k0 = wrap ? p.k_split : k1;
    seg_bptr += next_e ? b_estep : 0;
    ++seg_step;
    seg_next.live = seg_step < KT;
  };
  // One DMA instruction of step st into `stage`: d < LD_A covers A rows, then B.
  auto dma1 = [&](const StepSrc& st, int stage, int d) __attribute__((always_inline)) {
    const int k0 = st.k0;
    const bool live = st.live;
    uint8_t* dst = lds + stage * STAGE_BYTES;
    if (d < LD_A) {
      if constexpr (AL == ALoad::kConcat) {
        const bool second = k0 >= p.k_split;
        const __amdgpu_buffer_rsrc_t r = make_rsrc((const void*)(second ? a2_base : a_base));
        buf_dma16(live ? r : rs_none, second ? a2_off[d] : a_off[d], (uint32_t)k0 * 2, dst + a_dma_off + d * 1024);
      } else if constexpr (AL == ALoad::kSegmented) {
        const bool mine = st.e < 0 || a_exp[d] == st.e;
        buf_dma16(live ? rs_a : rs_none, mine ? a_off[d] : kMaskedOff, (uint32_t)k0 * 2, dst + a_dma_off + d * 1024);
      } else {
        buf_dma16(live ? rs_a : rs_none, a_off[d], (uint32_t)k0 * 2, dst + a_dma_off + d * 1024);
      }
    } else {
      if constexpr (AL == ALoad::kSegmented) {
        const __amdgpu_buffer_rsrc_t r = make_rsrc((const void*)(st.e < 0 ? seg_sptr : seg_bptr));
        buf_dma16(live ? r : rs_none, b_off[d - LD_A], (uint32_t)k0 * 2, dst + b_dma_off + (d - LD_A) * 1024);
      } else if constexpr (AL == ALoad::kConcat) {
        const __amdgpu_buffer_rsrc_t r = make_rsrc((const void*)(k0 >= p.k_split ? b2_base : b_base));
        buf_dma16(live ? r : rs_none, b_off[d - LD_A], (uint32_t)k0 * 2, dst + b_dma_off + (d - LD_A) * 1024);
      } else if constexpr (kSharedB) {
        const __amdgpu_buffer_rsrc_t r = make_rsrc((const void*)(k0 < p.k_split ? b2_base : b_base));
        buf_dma16(live ? r : rs_none, b_off[d - LD_A], (uint32_t)k0 * 2, dst + b_dma_off + (d - LD_A) * 1024);
      } else {
        buf_dma16(live ? rs_b : rs_none, b_off[d - LD_A], (uint32_t)k0 * 2, dst + b_dma_off + (d - LD_A) * 1024);
      }
    }
  };
  auto issue = [&](int kt, int stage) __attribute__((always_inline)) {
    const StepSrc st = AL == ALoad::kSegmented ? seg_next : step_src(kt);
#pragma unroll
    for (int d = 0; d < LD_PER_STEP; ++d) dma1(st, stage, d);
    if constexpr (AL == ALoad::kSegmented) seg_advance();
  };

  // ---- fragments -------------------------------------------------------------
  // Row (lane & 15) of a 16-row block, chunk 4 s + (lane >> 4) for sub-step s.  A
  // 16-row block spans a whole swizzle period (16 rows for 128- and 64-byte rows),
  // so the same offsets serve every block.
  const int fr_row = lane & 15;
  int fr_off[NSUB];
#pragma unroll
  for (int s = 0; s < NSUB; ++s)
    fr_off[s] = fr_row * ROW_BYTES + (((4 * s + (lane >> 4)) ^ ((fr_row / RPL) % CPR)) << 4);
  const int a_frag_base = wm * WM * ROW_BYTES;
  const int b_frag_base = A_TILE_BYTES + wn * WN * ROW_BYTES;

  bf16x8 fa[2][MI], fb[2][NI];
  // Fragment f of sub-step s into register set `set`: f < MI is A block f, then B.
  auto read1 = [&](int stage, int s, int set, int f) __attribute__((always_inline)) {
    const uint8_t* base = lds + stage * STAGE_BYTES;
    if (f < MI) {
      fa[set][f] = *reinterpret_cast<const bf16x8*>(base + a_frag_base + f * 16 * ROW_BYTES + fr_off[s]);
    } else {
      fb[set][f - MI] = *reinterpret_cast<const bf16x8*>(base + b_frag_base + (f - MI) * 16 * ROW_BYTES + fr_off[s]);
    }
  };
  auto read_frags = [&](int stage, int s, int set) __attribute__((always_inline)) {
#pragma unroll
    for (int f = 0; f < NFRAG; ++f) read1(stage, s, set, f);
  };

  f32x4 acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[mi][ni][v] = 0.f;

  auto mfma1 = [&](int set, int i) __attribute__((always_inline)) {
    const int mi = i / NI, ni = i % NI;
    acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[set][ni], fa[set][mi], acc[mi][ni], 0, 0, 0);
  };

  // ---- main loop --------------------------------------------------------------
  // The order of MFMAs, fragment reads and DMA instructions inside a sub-step is
  // fixed by hand: each MFMA is followed by at most one read and one DMA, and a
  // scheduling fence closes the group, so the memory instructions issue in the
  // shadow of the MFMAs instead of in bursts.
  //
  // Sub-steps 0..NSUB-2 of a K step: MFMAs of sub-step s from register set s & 1,
  // the NFRAG fragment reads of sub-step s+1 slotted behind the first MFMAs.
  auto substep = [&](int stage, int s) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < MI * NI; ++i) {
      mfma1(s & 1, i);
      if (i % RD_EVERY == 0 && i / RD_EVERY < NFRAG) read1(stage, s + 1, (s + 1) & 1, i / RD_EVERY);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Last sub-step: wait until step kt+1 has landed (the DMA of later steps may stay
  // in flight) and every wave is done with `stage`; then its MFMAs, each followed by
  // one DMA instruction of step kt + kStages into the freed stage and one fragment
  // read of sub-step 0 of step kt+1.  Every step issues the same count of DMA
  // instructions (past the end they fetch nothing), so one vmcnt threshold serves
  // all steps.  The final step (last = true) only computes.
  auto last_substep = [&](int kt, int stage, int next_stage, bool last) __attribute__((always_inline)) {
    const StepSrc st = AL == ALoad::kSegmented ? seg_next : step_src(kt + kStages);
    if (!last) {
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(LD_PER_STEP * (kStages - 2), 0));
      __syncthreads();
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < MI * NI; ++i) {
      mfma1((NSUB - 1) & 1, i);
      if (!last && i % DMA_EVERY == DMA_OFF && i / DMA_EVERY < LD_PER_STEP) dma1(st, stage, i / DMA_EVERY);
      if (!last && i % RD_EVERY == 0 && i / RD_EVERY < NFRAG) read1(next_stage, 0, 0, i / RD_EVERY);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!last) {
#pragma unroll
      for (int d = (MI * NI - DMA_OFF + DMA_EVERY - 1) / DMA_EVERY; d < LD_PER_STEP; ++d) dma1(st, stage, d);
      if constexpr (AL == ALoad::kSegmented) seg_advance();
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto kstep = [&](int kt, int stage, int next_stage, bool last) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s + 1 < NSUB; ++s) substep(stage, s);
    last_substep(kt, stage, next_stage, last);
  };

  // Prologue: steps 0 .. kStages-1 in flight, step 0 landed.  Scatter epilogues: thread
  // r < kTM first loads row r's permutation entry, which lands with step 0 and goes to
  // LDS, so that the epilogue's residual loads need no dependent global load.
  // Entries are clamped into [0, M) (a corrupt permutation scrambles rows but stays in
  // C); rows past the segment repeat its last row's (read, never stored).
  int32_t* perm_lds = reinterpret_cast<int32_t*>(lds + kStages * STAGE_BYTES);
  int32_t perm_pre = 0;
  if constexpr (kScatterRows) {
    // (No permutation: identity rows, the residual add of a plain product.)
    if (tid < kTM) {
      const int64_t r = m0 + tid < m_end ? m0 + tid : m_end - 1;
      perm_pre = p.perm != nullptr ? p.perm[r] : (int32_t)r;
    }
  }
  for (int i = 0; i < kStages; ++i) issue(i, i);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(LD_PER_STEP * (kStages - 1), 15));
  if constexpr (kScatterRows) {
    if (tid < kTM) perm_lds[tid] = perm_pre < 0 ? 0 : (perm_pre >= (int32_t)p.M ? (int32_t)p.M - 1 : perm_pre);
  }
  __syncthreads();
  read_frags(0, 0, 0);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
  __builtin_amdgcn_sched_barrier(0);

  // Steps 0 .. KT-2, then the final step peeled (its MFMAs then sit in the block of
  // the epilogue that reads their results).
  int stage = 0, kt = 0;
  for (; kt + 1 < KT; ++kt) {
    const int nxt = stage + 1 == kStages ? 0 : stage + 1;
    kstep(kt, stage, nxt, false);
    stage = nxt;
  }
  kstep(kt, stage, 0, true);
  // The refills issued by the last steps write (zeros) into the LDS the epilogue uses.
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));

  // ---- epilogue --------------------------------------------------------------
  // Results are staged through LDS: each wave writes its WM rows in the MFMA output
  // layout (8 bytes per lane and 4-column group) into its own region, rows of
  // OUT_ROWB bytes with 16-byte chunk c of row r at position c ^ (r % OUT_CH), then
  // reads them back 16 bytes per lane along the rows and stores whole row segments.
  // A store instruction then covers a few contiguous row pieces (1 KB in total)
  // instead of 8 bytes in each of 32 rows, which costs the L1 and L2 four times
  // fewer accesses.  Transposed V (kQKRope with vt_ld > 0) is stored directly.
  // In the 16 x 16 output layout lane l holds row l & 15 of a block and its four
  // consecutive columns 4 (l >> 4) .. 4 (l >> 4) + 3.
  const int q4 = lane >> 4;
  const int rl = lane & 15;
  constexpr int OUT_COLS = EP == Epi::kSwiGLU ? WN / 2 : WN;  // output columns per wave
  constexpr int OUT_ROWB = OUT_COLS * 2;
  constexpr int OUT_CH = OUT_ROWB / 16;
  constexpr int RPI = 64 / OUT_CH;  // rows per store instruction
  static_assert(4 * WM * OUT_ROWB <= kStages * STAGE_BYTES, "epilogue staging must fit the LDS");
  __syncthreads();  // every wave is done with the pipeline's LDS stages
  uint8_t* ep = lds + wave * (WM * OUT_ROWB);
  // Scatter epilogues: the output row of every store-loop iteration (from the LDS copy
  // of the permutation) and, for kScatterAdd, every residual piece this lane adds to
  // are loaded up front, before the accumulators are staged, so that the residual
  // loads' latency runs under the staging instead of after it (loads interleaved with
  // the stores below would wait one by one: a store may alias a later row's load).
  // Rows past the segment and columns past N read a clamped, valid piece (never
  // stored): guarded loads would become branches, each waiting for its load.
  constexpr int NIT = WM / RPI;  // store-loop iterations per lane
  int32_t prow[kScatterRows ? NIT : 1];
  uint4 resid[EP == Epi::kScatterAdd ? NIT : 1];
  if constexpr (kScatterRows) {
#pragma unroll
    for (int i = 0; i < NIT; ++i) prow[i] = perm_lds[wm * WM + i * RPI + lane / OUT_CH];
  }
  if constexpr (EP == Epi::kScatterAdd) {
    const int n = min(n0 + wn * WN + (lane % OUT_CH) * 8, p.N - 8);
#pragma unroll
    for (int i = 0; i < NIT; ++i) resid[i] = *reinterpret_cast<const uint4*>(p.c + (int64_t)prow[i] * p.ldc + n);
  }
  auto stage4 = [&](int r, int col, float y0, float y1, float y2, float y3) __attribute__((always_inline)) {
    uint2 o;
    o.x = pack_bf16x2(y0, y1);
    o.y = pack_bf16x2(y2, y3);
    const int ch = (col >> 3) ^ (r % OUT_CH);
    *reinterpret_cast<uint2*>(ep + r * OUT_ROWB + ch * 16 + ((col >> 2) & 1) * 8) = o;
  };

  // kQKRope: token (b, s) of wave row r, from one division per wave for its first
  // row (the host bounds S below 2^31 - 256, so s0 + r fits 32 bits).
  int64_t tok_b0 = 0;
  uint32_t tok_s0 = 0;
  if constexpr (EP == Epi::kQKRope) {
    const int64_t row_base = m0 + wm * WM;
    tok_b0 = row_base / p.qk.S;
    tok_s0 = (uint32_t)(row_base - tok_b0 * p.qk.S);
  }
  // kQKRope, V^T output: a wave whose columns are all V heads and whose WM rows are
  // one run of tokens of one sequence starting at a multiple of 16 stages V^T through
  // LDS (rows d of 2 WM bytes = its WM tokens in vt_col order) and stores whole row
  // segments; other waves store V^T element by element.
  constexpr int VT_ROWB = WM * 2, VT_CH = VT_ROWB / 16;  // staged V^T row: bytes, 16-byte chunks
  static_assert(EP != Epi::kQKRope || WN * VT_ROWB <= WM * OUT_ROWB,
                "staged V^T rows must fit the wave's staging region");
  bool vt_fast = false;
  if constexpr (EP == Epi::kQKRope) {
    vt_fast = p.qk.vt_ld > 0 && n0 + wn * WN >= (p.qk.nq + p.qk.nkv) * HD && (tok_s0 & 15) == 0 &&
              (int64_t)tok_s0 + WM <= p.qk.S && m0 + wm * WM + WM <= m_end;
  }
  // A wave whose WM rows lie in one sequence (every wave when S % WM == 0) needs no
  // division per row.
  bool one_seq = false;
  if constexpr (EP == Epi::kQKRope) one_seq = (int64_t)tok_s0 + WM <= p.qk.S;
  auto tok = [&](int r, int64_t& b, uint32_t& s) __attribute__((always_inline)) {
    const uint32_t t = tok_s0 + (uint32_t)r, S32 = (uint32_t)p.qk.S;
    if (one_seq) {
      s = t;
      b = tok_b0;
      return;
    }
    const uint32_t w = t / S32;
    s = t - w * S32;
    b = tok_b0 + w;
  };

  if constexpr (EP == Epi::kQKRope) {
    // Head-wise epilogue.  A wave's WN columns hold WN / HD whole heads of BPH
    // 16-column blocks; for row m a lane holds a quarter of the head's HD values
    // (lanes l, l ^ 16, l ^ 32, l ^ 48 together hold all of it) and both elements of
    // every RoPE pair (c, c + HD/2): blocks nb and nb + BPH/2, same slot.
    static_assert(HD == 32 || HD == 64 || HD == 128, "head dim must be 32, 64 or 128");
    constexpr int BPH = HD / 16, HPW = WN / HD, HALF = HD / 2;
    const QKRopeParams& q = p.qk;
    const int qd = q.nq * HD, kvd = q.nkv * HD;
#pragma unroll
    for (int hb = 0; hb < HPW; ++hb) {
      const int c0 = n0 + wn * WN + hb * HD;  // first global column of this head
      if (c0 >= p.N) continue;
      const int kind = c0 < qd ? 0 : (c0 < qd + kvd ? 1 : 2);  // q, k, v
      const int head = kind == 0 ? c0 / HD : (kind == 1 ? (c0 - qd) / HD : (c0 - qd - kvd) / HD);
      const uint16_t* nw = kind == 0 ? q.q_norm_w : (kind == 1 ? q.k_norm_w : nullptr);
      const bool norm = kind != 2 && nw != nullptr;
      // Norm weights of this lane's columns (the same for every row).
      // Without QK norm the weights are 1 and the scale below is 1: both products are
      // then exact, and the code has no branch between the norm and the rotation (a
      // branch there made the compiler pass the values through AGPRs).
      uint2 wpk[BPH];  // 4 bf16 each; one uniform branch around all the loads
#pragma unroll
      for (int nb = 0; nb < BPH; ++nb) wpk[nb] = make_uint2(0x3F803F80u, 0x3F803F80u);
      if (norm) {
#pragma unroll
        for (int nb = 0; nb < BPH; ++nb) wpk[nb] = *reinterpret_cast<const uint2*>(nw + nb * 16 + 4 * q4);
      }
      float wf[BPH][4];  // the same weights in fp32, unpacked once for all rows
#pragma unroll
      for (int nb = 0; nb < BPH; ++nb) {
        wf[nb][0] = __uint_as_float(wpk[nb].x << 16);
        wf[nb][1] = __uint_as_float(wpk[nb].x & 0xffff0000u);
        wf[nb][2] = __uint_as_float(wpk[nb].y << 16);
        wf[nb][3] = __uint_as_float(wpk[nb].y & 0xffff0000u);
      }
      // cos / sin of this lane's first-half columns for the rows of block mi, read at
      // the top of the block so that the latency hides behind the norm arithmetic.
      // Every row's s lies in [0, S), so the reads stay inside the table even past
      // m_end.
      // Narrow tiles (the small products, whose blocks have no neighbours on their CU
      // to hide a wait) read block mi + 1's pairs while block mi is computed; the wide
      // tile has no registers to spare for them.
      constexpr bool kCsAhead = kBN == 128;
      float4 cs_cur[BPH / 2][2], cs_nxt[BPH / 2][2];
      auto fetch_cs = [&](int mi, float4 (&dst)[BPH / 2][2]) __attribute__((always_inline)) {
        int64_t b;
        uint32_t s;
        tok(mi * 16 + rl, b, s);
        const float2* cs = reinterpret_cast<const float2*>(q.cos_sin) + (q.pos0 + s) * HALF;
#pragma unroll
        for (int nb = 0; nb < BPH / 2; ++nb) {
          const int c = nb * 16 + 4 * q4;
          dst[nb][0] = *reinterpret_cast<const float4*>(cs + c);
          dst[nb][1] = *reinterpret_cast<const float4*>(cs + c + 2);
        }
      };
      if (kCsAhead && kind != 2) fetch_cs(0, cs_nxt);
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
        __builtin_amdgcn_sched_barrier(0);  // one block of accumulators live at a time
        const int r = mi * 16 + rl;
        const int64_t gm = m0 + wm * WM + r;
        float x[BPH][4];
#pragma unroll
        for (int nb = 0; nb < BPH; ++nb)
#pragma unroll
          for (int v = 0; v < 4; ++v) x[nb][v] = acc[mi][hb * BPH + nb][v];
        if (kind == 2) {
          if (vt_fast) {
            // Quad transpose: lanes 4j + t (same q4) hold tokens 4j + t of dims
            // 4 q4 + (0..3); afterwards lane 4j + t holds dim 4 q4 + t of tokens
            // 4j + (0..3), as two packed bf16 pairs, in two exchanges (lane t ^ 1,
            // then t ^ 2) over the quad.
            const int t = lane & 3, j = (lane >> 2) & 3;
#pragma unroll
            for (int nb = 0; nb < BPH; ++nb) {
              const uint2 w = vt_quad_transpose(x[nb][0], x[nb][1], x[nb][2], x[nb][3], lane);
              // Tokens r .. r + 3 (r = 16 mi + 4 j) sit at V^T positions
              // 16 mi + 4 sigma(j) .. + 3; rows are VT_ROWB bytes with 16-byte chunk
              // k at position k ^ (row % VT_CH).
              const int row = hb * HD + nb * 16 + 4 * q4 + t;
              const int sj = j == 1 ? 2 : (j == 2 ? 1 : j);
              const int chunk = 2 * mi + (sj >> 1);
              *reinterpret_cast<uint2*>(ep + row * VT_ROWB + ((chunk ^ (row & (VT_CH - 1))) << 4) + (sj & 1) * 8) = w;
            }
            continue;
          }
          if (gm >= m_end) continue;
          if (q.vt_ld > 0) {
            // V^T: column vt_col(s) of rows d; 16 consecutive tokens per quarter wave.
            int64_t b;
            uint32_t s;
            tok(r, b, s);
            uint16_t* vt = q.v_out + ((b * q.nkv + head) * HD) * q.vt_ld + vt_col(s);
#pragma unroll
            for (int nb = 0; nb < BPH; ++nb)
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                const int d = nb * 16 + 4 * q4 + v;
                vt[(int64_t)d * q.vt_ld] = f32_to_bf16_bits(x[nb][v]);
              }
            continue;
          }
#pragma unroll
          for (int nb = 0; nb < BPH; ++nb)
            stage4(r, hb * HD + nb * 16 + 4 * q4, x[nb][0], x[nb][1], x[nb][2], x[nb][3]);
          continue;
        }
        if constexpr (kCsAhead) {
#pragma unroll
          for (int nb = 0; nb < BPH / 2; ++nb) {
            cs_cur[nb][0] = cs_nxt[nb][0];
            cs_cur[nb][1] = cs_nxt[nb][1];
          }
          if (mi + 1 < MI) fetch_cs(mi + 1, cs_nxt);
        } else {
          fetch_cs(mi, cs_cur);
        }
        qk_norm_rope<BPH>(x, wf, cs_cur, norm, q.eps);
        if (gm >= m_end) continue;
#pragma unroll
        for (int nb = 0; nb < BPH; ++nb)
          stage4(r, hb * HD + nb * 16 + 4 * q4, x[nb][0], x[nb][1], x[nb][2], x[nb][3]);
      }
    }
  } else if constexpr (EP == Epi::kSwiGLU) {
    // Packed B rows come in groups of 64: 32 gate rows then the matching 32 up rows,
    // i.e. blocks 4 g, 4 g + 1 (gate) and 4 g + 2, 4 g + 3 (up); the wave's output
    // columns are 32 g + 16 (ni % 4) + 4 q4.
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      const int r = mi * 16 + rl;
#pragma unroll
      for (int ni = 0; ni < NI; ni += 4)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float a4[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) a4[j] = silu_f32(acc[mi][ni + h][j]) * acc[mi][ni + h + 2][j];
          stage4(r, (ni >> 2) * 32 + 16 * h + 4 * q4, a4[0], a4[1], a4[2], a4[3]);
        }
    }
  } else {
    // kBiasClamp: the lane's NI groups of 4 bias values, loaded once for every row.
    float4 bias4[EP == Epi::kBiasClamp ? NI : 1];
    if constexpr (EP == Epi::kBiasClamp) {
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        const int n = n0 + wn * WN + ni * 16 + 4 * q4;
        bias4[ni] = n < p.N ? load_bias4(p.bias + n, p.bias_lo, p.bias_hi) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      const int r = mi * 16 + rl;
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        const int col = ni * 16 + 4 * q4;
        float y[4] = {acc[mi][ni][0], acc[mi][ni][1], acc[mi][ni][2], acc[mi][ni][3]};
        if constexpr (EP == Epi::kBiasClamp) {
          const float bb[4] = {bias4[ni].x, bias4[ni].y, bias4[ni].z, bias4[ni].w};
#pragma unroll
          for (int j = 0; j < 4; ++j) y[j] = fminf(fmaxf(y[j] + bb[j], p.lo), p.hi);
        }
        stage4(r, col, y[0], y[1], y[2], y[3]);
      }
    }
  }

  // Own LDS writes are complete before the reads (LDS operations of a wave execute
  // in order; the wait also keeps the compiler from reordering them).  The outputs
  // are streamed (non-temporal stores), which keeps the operands' panels in L2.
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
  if constexpr (EP == Epi::kQKRope) {
    if (vt_fast) {
      // V^T rows: VT_CH lanes per row, 64 / VT_CH rows per instruction.
      const QKRopeParams& q = p.qk;
      constexpr int VT_RPI = 64 / VT_CH;
      const int k = lane % VT_CH;
#pragma unroll 4
      for (int i = 0; i < WN / VT_RPI; ++i) {
        const int row = i * VT_RPI + lane / VT_CH;
        const int c0 = n0 + wn * WN + (row / HD) * HD;
        if (c0 >= p.N) continue;
        const int head = (c0 - (q.nq + q.nkv) * HD) / HD, d = row % HD;
        const uint4 v = *reinterpret_cast<const uint4*>(ep + row * VT_ROWB + ((k ^ (row & (VT_CH - 1))) << 4));
        uint16_t* dst = q.v_out + ((tok_b0 * q.nkv + head) * HD + d) * q.vt_ld + tok_s0 + k * 8;
        store_nt16(dst, v);
      }
      return;
    }
  }
  const int jc = lane % OUT_CH;  // this lane's chunk of a row
  auto store_row = [&](int i) __attribute__((always_inline)) {
    const int r = i * RPI + lane / OUT_CH;
    const int64_t gm = m0 + wm * WM + r;
    if (gm < m_lo || gm >= m_end) return;
    const uint4 v = *reinterpret_cast<const uint4*>(ep + r * OUT_ROWB + ((jc ^ (r % OUT_CH)) << 4));
    const int col = jc * 8;  // first output column of the chunk within the wave
    uint16_t* dst;
    if constexpr (EP == Epi::kQKRope) {
      const QKRopeParams& q = p.qk;
      const int qd = q.nq * HD, kvd = q.nkv * HD;
      const int c0 = n0 + wn * WN + (col / HD) * HD;
      if (c0 >= p.N) return;
      const int kind = c0 < qd ? 0 : (c0 < qd + kvd ? 1 : 2);
      if (kind == 2 && q.vt_ld > 0) return;  // stored directly above
      const int head = kind == 0 ? c0 / HD : (kind == 1 ? (c0 - qd) / HD : (c0 - qd - kvd) / HD);
      const int nheads = kind == 0 ? q.nq : q.nkv;
      uint16_t* obase = kind == 0 ? q.q_out : (kind == 1 ? q.k_out : q.v_out);
      int64_t b;
      uint32_t s;
      tok(r, b, s);
      dst = obase + ((b * nheads + head) * q.S + s) * HD + (col % HD);
    } else if constexpr (EP == Epi::kSwiGLU) {
      const int n = (n0 + wn * WN) / 2 + col;
      if (2 * n >= p.N) return;
      dst = p.c + gm * p.ldc + n;
    } else {
      const int n = n0 + wn * WN + col;
      if (n >= p.N) return;
      int64_t orow = gm;
      if constexpr (kScatterRows) orow = prow[i];
      dst = p.c + orow * p.ldc + n;
    }
    if constexpr (EP == Epi::kScatterAdd) {
      // Each output row belongs to one tile and each 16-byte piece to one lane, so the
      // read-add-write has no other writer.
      store_nt16(dst, add_bf16x8(v, resid[i]));
    } else {
      store_nt16(dst, v);
    }
  };
  if constexpr (kScatterRows) {
#pragma unroll
    for (int i = 0; i < NIT; ++i) store_row(i);  // prow[] and resid[] are indexed by constants only
  } else {
#pragma unroll 4
    for (int i = 0; i < NIT; ++i) store_row(i);
  }
}

}  // namespace cdx
