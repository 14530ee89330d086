// Persistent form of the MFMA tile engine (cdx_gemm.h): whole tiles of a dense or
// concat A operand (M and N multiples of the tile) with the store or bias-clamp
// epilogue, mu-QKV with the QK-norm + RoPE epilogue (head dim 128, V transposed), and
// the MoE gate/up pass (rows gathered through the routing permutation, per-expert M
// tiles, SwiGLU epilogue).
//
// gemm_nt_kernel runs one tile per block, so every tile pays a block launch, its setup
// and a prologue that waits for its first K step to arrive from L2 or HBM.  Here a grid
// of one block per CU walks the tiles of its XCD's range (the same logical order as
// gemm_nt_kernel: contiguous per XCD, groups of kGroupM M tiles; with the QK-norm + RoPE
// epilogue, odd groups take their N tiles in reverse).  The refill issued by
// a tile's second-to-last K step is the next tile's first step, so that step lands
// while the tile finishes and writes its results.  The epilogue stages the results
// through the other LDS stage in two halves of 64 rows per wave (16 KB per wave, one
// stage in all; the SwiGLU output, half as wide, fits at once); the next tile's second
// step is issued when it is done.  For gathered rows the next tile's per-lane source
// offsets are computed from the permutation when the current tile starts.  The
// accumulators are cleared between tiles.
//
// K loop, fragment reads, LDS layout, DMA placement and the staged-store layout are
// those of gemm_nt_kernel.
#pragma once

#include "cdx_gemm.h"

namespace cdx {

template <class Cfg, ALoad AL, Epi EP, int HD = 0>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_persist_kernel(const GemmParams p) {
  constexpr bool kGathered = AL == ALoad::kGather;
  // kScatterAdd here has identity rows (no permutation): c += the tile, the residual
  // add fused into a plain product.
  static_assert(((AL == ALoad::kDense || AL == ALoad::kConcat) && (EP == Epi::kStore || EP == Epi::kBiasClamp)) ||
                    (AL == ALoad::kDense && EP == Epi::kScatterAdd) || (kGathered && EP == Epi::kSwiGLU) ||
                    ((AL == ALoad::kConcat || AL == ALoad::kDense) && EP == Epi::kQKRope && HD == 128),
                "persistent tiles: dense/concat A with store or bias-clamp, dense A with the residual add, "
                "gathered A with SwiGLU, or mu-QKV (dense or concat A) with the QK-norm + RoPE epilogue at "
                "head dim 128");
  static_assert(Cfg::STAGES == 2 && Cfg::MINB == 1 && Cfg::BN == 256 && Cfg::BM == kBM,
                "persistent tiles: 256 x 256, two stages");
  constexpr int kBN = Cfg::BN, kBK = Cfg::BK, kStages = 2;
  constexpr int ROW_BYTES = kBK * 2;
  constexpr int CPR = kBK / 8;
  constexpr int RPL = 256 / ROW_BYTES;
  constexpr int A_TILE_BYTES = kBM * ROW_BYTES;
  constexpr int STAGE_BYTES = Cfg::STAGE_BYTES;
  constexpr int WM = kBM / 2, WN = kBN / 2;
  constexpr int MI = WM / 16, NI = WN / 16;
  constexpr int ROWS_PER_DMA = 1024 / ROW_BYTES;
  constexpr int LD_A = kBM / ROWS_PER_DMA / 4;
  constexpr int LD_B = kBN / ROWS_PER_DMA / 4;
  constexpr int LD_PER_STEP = LD_A + LD_B;
  constexpr int NSUB = kBK / 32;
  constexpr int NFRAG = MI + NI;
  constexpr int DMA_EVERY = Cfg::DMA_EVERY, DMA_OFF = Cfg::DMA_OFF, RD_EVERY = Cfg::READ_EVERY;
  // Epilogue staging: per wave and half, 64 rows of WN bf16 (256 bytes); SwiGLU: all
  // WM rows of WN / 2 columns (128 bytes).  16-byte chunk c of row r sits at position
  // c ^ (r % OUT_CH).
  constexpr int OUT_ROWB = (EP == Epi::kSwiGLU ? WN / 2 : WN) * 2, OUT_CH = OUT_ROWB / 16;
  constexpr int HALF_ROWS = WM / 2, RPI = 64 / OUT_CH;
  static_assert(NSUB == 2, "one K step is two K32 sub-steps");
  static_assert(4 * HALF_ROWS * OUT_ROWB <= STAGE_BYTES, "a staged half must fit one stage");
  static_assert(EP != Epi::kSwiGLU || 4 * WM * OUT_ROWB <= STAGE_BYTES, "the SwiGLU tile must fit one stage");

  // Gathered tiles: after the stages, a table of 3 x 64 ints (segment starts, ends and
  // the running count of M tiles, one entry per expert).
  constexpr int SEG_TAB_BYTES = kGathered ? 3 * 64 * 4 : 0;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * STAGE_BYTES + SEG_TAB_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // ---- this block's tiles ------------------------------------------------------
  // Segment offsets are read clamped to [0, M], and a segment that ends before it
  // starts is empty (as in gemm_nt_kernel): offsets that are not a valid plan give
  // wrong rows but no access outside the operands.  Grouped tiles: each M tile lies in
  // one expert's segment; the launch bound p.mt_count caps the real count.
  auto seg_off = [&](int x) __attribute__((always_inline)) {
    const int v = p.offsets[x];
    return v < 0 ? 0 : (v > (int)p.M ? (int)p.M : v);
  };
  // Gathered: lane x < E holds segment x's start and end and the number of M tiles of
  // segments 0..x (an inclusive scan over the lanes), from two vector loads per block;
  // tile decodes then take ballots and lane reads instead of a loop of dependent loads
  // (a load in that loop waited for every outstanding memory operation, the previous
  // tile's stores included).  Wave 0 keeps a copy in LDS for the decodes at tile
  // switches, so that the values are not held in registers through the K loop.
  int mt_real = p.mt_count;
  int g_s0 = 0, g_s1 = 0, g_ci = 0;
  int* seg_tab = reinterpret_cast<int*>(lds + kStages * STAGE_BYTES);
  if constexpr (kGathered) {
    g_s0 = lane < p.E ? seg_off(lane) : (int)p.M;
    g_s1 = lane < p.E ? seg_off(lane + 1) : (int)p.M;
    g_ci = lane < p.E ? max(0, (g_s1 - g_s0 + kBM - 1) / kBM) : 0;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int up = __shfl_up(g_ci, d);
      g_ci += lane >= d ? up : 0;
    }
    mt_real = min(__builtin_amdgcn_readlane(g_ci, 63), p.mt_count);
    if (wave == 0) {
      seg_tab[lane] = g_s0;
      seg_tab[64 + lane] = g_s1;
      seg_tab[128 + lane] = g_ci;
    }
  }
  // XCD x (blocks b with b % 8 == x) owns logical tiles [x_first, x_first + x_count);
  // its k-th block takes tiles x_first + k, x_first + k + x_blocks, ...
  const int tiles = mt_real * p.nt_count;
  const int xcd = blockIdx.x % kNumXcd, kx = blockIdx.x / kNumXcd;
  const int tq = tiles / kNumXcd, tr = tiles % kNumXcd;
  const int x_first = xcd < tr ? xcd * (tq + 1) : tr * (tq + 1) + (xcd - tr) * tq;
  const int x_count = tq + (xcd < tr ? 1 : 0);
  const int x_blocks = (int)(gridDim.x / kNumXcd) + (xcd < (int)(gridDim.x % kNumXcd) ? 1 : 0);
  if (kx >= x_count) return;

  // Tile i of the XCD's range: first row and column and the DMA bases (A rows and B
  // rows of the tile; concat: also the mu and mu-weight sources, k_split columns before
  // their first column, so that both K halves take the scalar offset 2 k0).  Separate
  // scalars: a struct selected through a reference ends up in scratch memory.
  // Grouped: m0 / m_end are the tile's rows in the sorted order, its expert's B rows
  // start at b + e * b_estride, and A is the whole gather source.
  // Gathered (SwiGLU) tiles: b is the base of this wave's B rows, taken before or
  // after the tile's block switch (gu_tile).  The switch row is a multiple of 128 and a
  // wave's rows are one 64-aligned run of 64, so they all lie on one side of it: the
  // choice is made once per tile, not for every DMA.
  auto tile_at = [&](int i, int64_t& m0, int64_t& m_end, int& n0, uintptr_t& a, uintptr_t& a2, uintptr_t& b,
                     uintptr_t& b2, int s0v, int s1v, int civ) __attribute__((always_inline)) {
    const int L = x_first + i;
    const int per_group = kGroupM * p.nt_count;
    const int group = L / per_group;
    const int first_m = group * kGroupM;
    const int gsz = min(mt_real - first_m, kGroupM);
    const int in_group = L - group * per_group;
    const int mt = __builtin_amdgcn_readfirstlane(first_m + in_group % gsz);
    // QK-norm + RoPE: odd groups walk the N tiles backwards (a serpentine), so that a
    // block's tiles i and i + 2 x_blocks sit at mirrored columns and every block gets
    // a mix of q, k and v heads, whose epilogues differ in cost (at the 1B shape half
    // the blocks otherwise ran two q and two k tiles).  Measured slower for the MoE
    // gate/up pass, so the other epilogues keep the plain order.
    const int nt = in_group / gsz;
    const bool rev = EP == Epi::kQKRope && (group & 1);
    n0 = __builtin_amdgcn_readfirstlane(rev ? p.nt_count - 1 - nt : nt) * kBN;
    int e = 0;
    if constexpr (kGathered) {
      // The segment holding M tile mt: the first whose running tile count exceeds mt
      // (mt < mt_real keeps it below E).
      e = min((int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < p.E && civ <= mt)), p.E - 1);
      e = __builtin_amdgcn_readfirstlane(e);
      const int before = e > 0 ? __builtin_amdgcn_readlane(civ, e - 1) : 0;
      m0 = __builtin_amdgcn_readlane(s0v, e) + (int64_t)(mt - before) * kBM;
      m_end = __builtin_amdgcn_readlane(s1v, e);
      a = (uintptr_t)p.a;
    } else {
      m0 = (int64_t)mt * kBM;
      m_end = m0 + kBM;
      a = (uintptr_t)(p.a + m0 * p.lda);
    }
    b = (uintptr_t)(p.b + (int64_t)e * p.b_estride + (int64_t)n0 * p.ldb);
    if constexpr (kGathered) {
      const GuTile g = gu_tile(p.b, p.ldb, p.gu_P, p.gu_shared != 0, e, n0);
      b = wave * (kBN / 4) >= g.split ? g.hi : g.lo;
      b2 = b;
    } else if constexpr (AL == ALoad::kConcat) {
      a2 = (uintptr_t)(p.a2 + m0 * p.lda2) - (uintptr_t)p.k_split * 2;
      b2 = (uintptr_t)(p.b2 + (int64_t)n0 * p.ldb) - (uintptr_t)p.k_split * 2;
    } else {
      b2 = b;
    }
    if constexpr (AL != ALoad::kConcat) a2 = a;
  };

  // ---- per-lane DMA offsets (the same for every whole tile) ----------------------
  // Gathered rows: per tile, from the permutation (see gather_offsets below).
  const int dr = lane / CPR;
  uint32_t a_off[LD_A], a2_off[LD_A], b_off[LD_B];
#pragma unroll
  for (int j = 0; j < LD_A; ++j) {
    const int r = wave * (kBM / 4) + j * ROWS_PER_DMA + dr;
    const int dchunk = (lane % CPR) ^ ((r / RPL) % CPR);
    a_off[j] = (uint32_t)(((int64_t)r * p.lda + dchunk * 8) * 2);
    a2_off[j] = AL == ALoad::kConcat ? (uint32_t)(((int64_t)r * p.lda2 + dchunk * 8) * 2) : 0u;
  }
#pragma unroll
  for (int j = 0; j < LD_B; ++j) {
    const int r = wave * (kBN / 4) + j * ROWS_PER_DMA + dr;
    const int dchunk = (lane % CPR) ^ ((r / RPL) % CPR);
    const int64_t row = kGathered ? (int64_t)gu_row(r, p.gu_P) : (int64_t)r;
    b_off[j] = (uint32_t)((row * p.ldb + dchunk * 8) * 2);
  }
  const int a_dma_off = wave * (kBM / 4) * ROW_BYTES;
  const int b_dma_off = A_TILE_BYTES + wave * (kBN / 4) * ROW_BYTES;

  const int KT = p.K / kBK;  // the host guarantees KT >= 2
  const __amdgpu_buffer_rsrc_t rs_none = make_rsrc(p.b, 0u);
  int ti = kx;  // index of the current tile in the XCD's range
  int64_t cur_m0, nxt_m0, cur_m_end, nxt_m_end;
  int cur_n0, nxt_n0;
  uintptr_t cur_a, cur_a2, cur_b, cur_b2, nxt_a, nxt_a2, nxt_b, nxt_b2;
  tile_at(ti, cur_m0, cur_m_end, cur_n0, cur_a, cur_a2, cur_b, cur_b2, g_s0, g_s1, g_ci);
  bool has_next = ti + x_blocks < x_count;
  tile_at(has_next ? ti + x_blocks : ti, nxt_m0, nxt_m_end, nxt_n0, nxt_a, nxt_a2, nxt_b, nxt_b2, g_s0,
          g_s1, g_ci);
  // Gathered rows: the source row of each lane's DMA rows, through the permutation;
  // rows past the segment repeat its last row (loaded, never stored), and an entry
  // outside [0, M) is clamped into it (a corrupt permutation reads wrong rows but stays
  // inside the operand; the host bounds M * lda * 2 to 4 GB).
  uint32_t cur_goff[kGathered ? LD_A : 1], nxt_goff[kGathered ? LD_A : 1];
  auto gather_offsets = [&](int64_t m0, int64_t m_end, uint32_t (&off)[kGathered ? LD_A : 1])
                            __attribute__((always_inline)) {
    if constexpr (kGathered) {
#pragma unroll
      for (int j = 0; j < LD_A; ++j) {
        const int r = wave * (kBM / 4) + j * ROWS_PER_DMA + dr;
        const int dchunk = (lane % CPR) ^ ((r / RPL) % CPR);
        const int64_t gm = max(min(m0 + r, m_end - 1), (int64_t)0);
        const uint32_t src = min((uint32_t)p.perm[gm], (uint32_t)(p.M - 1));
        off[j] = (src * (uint32_t)p.lda + (uint32_t)dchunk * 8u) * 2u;
      }
    }
  };
  gather_offsets(cur_m0, cur_m_end, cur_goff);
  // Without a next tile the "next" tile is the current one again (its offsets are set
  // but never read from: the DMA that would fetch it takes the empty descriptor).
  gather_offsets(nxt_m0, nxt_m_end, nxt_goff);

  // Where a DMA reads: k0, the current or the next tile, and whether there is one.
  struct StepSrc {
    int k0;
    bool next;
    bool live;
  };
  auto dma1 = [&](const StepSrc st, int stage, int d) __attribute__((always_inline)) {
    const int k0 = st.k0;
    const bool second = AL == ALoad::kConcat && k0 >= p.k_split;
    uint8_t* dst = lds + stage * STAGE_BYTES;
    if (d < LD_A) {
      const uintptr_t first_src = st.next ? nxt_a : cur_a, second_src = st.next ? nxt_a2 : cur_a2;
      const __amdgpu_buffer_rsrc_t r = make_rsrc((const void*)(second ? second_src : first_src));
      uint32_t off = second ? a2_off[d] : a_off[d];
      if constexpr (kGathered) off = st.next ? nxt_goff[d] : cur_goff[d];
      buf_dma16(st.live ? r : rs_none, off, (uint32_t)k0 * 2, dst + a_dma_off + d * 1024);
    } else {
      const uintptr_t first_src = st.next ? nxt_b : cur_b, second_src = st.next ? nxt_b2 : cur_b2;
      const __amdgpu_buffer_rsrc_t r = make_rsrc((const void*)(second ? second_src : first_src));
      buf_dma16(st.live ? r : rs_none, b_off[d - LD_A], (uint32_t)k0 * 2, dst + b_dma_off + (d - LD_A) * 1024);
    }
  };

  // ---- fragments ---------------------------------------------------------------
  const int fr_row = lane & 15;
  int fr_off[NSUB];
#pragma unroll
  for (int s = 0; s < NSUB; ++s)
    fr_off[s] = fr_row * ROW_BYTES + (((4 * s + (lane >> 4)) ^ ((fr_row / RPL) % CPR)) << 4);
  const int a_frag_base = wm * WM * ROW_BYTES;
  const int b_frag_base = A_TILE_BYTES + wn * WN * ROW_BYTES;
  bf16x8 fa[2][MI], fb[2][NI];
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
  // Cleared between tiles.  The empty asm makes the zeros opaque: with them known,
  // the compiler feeds the first MFMAs a constant C operand and then moves their
  // results between AGPRs and VGPRs to reach the K loop's registers.
  auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};
        asm volatile("" : "+a"(acc[mi][ni]));
      }
  };
  auto mfma1 = [&](int set, int i) __attribute__((always_inline)) {
    const int mi = i / NI, ni = i % NI;
    acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[set][ni], fa[set][mi], acc[mi][ni], 0, 0, 0);
  };

  // ---- K step --------------------------------------------------------------------
  // Sub-step 0: its MFMAs with the fragment reads of sub-step 1 behind them.
  // Sub-step 1: wait for the next step's DMA and the barrier, then its MFMAs with the
  // refill of the freed stage and the fragment reads of step kt + 1.
  // The refill is step kt + 2 of the tile, or the next tile's first step (none after
  // the block's last tile); the tile's last step neither refills nor reads the next
  // step's fragments (its stage then stages the results).
  auto kstep = [&](int kt, int stage, int next_stage, bool last) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < MI * NI; ++i) {
      mfma1(0, i);
      if (i % RD_EVERY == 0 && i / RD_EVERY < NFRAG) read1(stage, 1, 1, i / RD_EVERY);
      __builtin_amdgcn_sched_barrier(0);
    }
    const int g = kt + kStages;
    const StepSrc st = g < KT ? StepSrc{g * kBK, false, true} : StepSrc{0, true, has_next};
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < MI * NI; ++i) {
      mfma1(1, i);
      if (!last && i % DMA_EVERY == DMA_OFF && i / DMA_EVERY < LD_PER_STEP) dma1(st, stage, i / DMA_EVERY);
      if (!last && i % RD_EVERY == 0 && i / RD_EVERY < NFRAG) read1(next_stage, 0, 0, i / RD_EVERY);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!last) {
#pragma unroll
      for (int d = (MI * NI - DMA_OFF + DMA_EVERY - 1) / DMA_EVERY; d < LD_PER_STEP; ++d) dma1(st, stage, d);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // ---- epilogue --------------------------------------------------------------------
  // Lane l holds row l & 15 of each 16 x 16 block and its columns 4 (l >> 4) .. + 3.
  const int q4 = lane >> 4;
  const int rl = lane & 15;
  float4 bias4[EP == Epi::kBiasClamp ? NI : 1];
  auto load_bias = [&](int n0) __attribute__((always_inline)) {
    if constexpr (EP == Epi::kBiasClamp) {
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        bias4[ni] = load_bias4(p.bias + n0 + wn * WN + ni * 16 + 4 * q4, p.bias_lo, p.bias_hi);
    }
  };
  // Staged through `stage`: each wave's region holds 64 rows; the wave writes the
  // results of four 16-row blocks, reads them back 16 bytes per lane along the rows
  // and stores whole row segments, then does the same for the other four blocks.
  // Only the wave's own region is touched between the two barriers around the
  // epilogue, so the halves need no barrier of their own.
  // QK-norm + RoPE (head dim 128, V transposed, S a multiple of WM): the wave's
  // WN = HD columns are one head and its WM rows one run of tokens of one sequence.
  // q and k heads are normalised and rotated block by block from the accumulators
  // (qk_norm_rope) and staged like the plain store; a V head is staged transposed,
  // per half as HD rows d of its 64 tokens (128 bytes, 16-byte chunk k of row d at
  // position k ^ (d % 8)) in vt_col order, and stored as V^T row segments.  The lane
  // index is passed through an empty asm first, so that nothing derived from it here
  // is computed once and held through the K loop.
  auto epilogue_rope = [&](int stage, int64_t m0, int n0) __attribute__((always_inline)) {
    // (The lambda exists in every instance of the kernel; kHD keeps it well formed.)
    constexpr int kHD = EP == Epi::kQKRope ? HD : 32, BPH = kHD / 16;
    const QKRopeParams& q = p.qk;
    int lo = lane;
    asm volatile("" : "+v"(lo));
    const int eq4 = lo >> 4, erl = lo & 15;
    const int c0 = n0 + wn * WN;
    const int qd = q.nq * kHD, kvd = q.nkv * kHD;
    const int kind = c0 < qd ? 0 : (c0 < qd + kvd ? 1 : 2);  // q, k, v
    const int head = kind == 0 ? c0 / kHD : (kind == 1 ? (c0 - qd) / kHD : (c0 - qd - kvd) / kHD);
    const int64_t row0 = m0 + wm * WM;
    const int64_t tb = row0 / q.S;
    const int64_t ts0 = row0 - tb * q.S;
    uint8_t* ep = lds + stage * STAGE_BYTES + wave * (HALF_ROWS * OUT_ROWB);
    if (kind == 2) {
      const int t = lo & 3, j = (lo >> 2) & 3;
      const int sj = j == 1 ? 2 : (j == 2 ? 1 : j);
      const int k = lo & 7;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int mh = 0; mh < MI / 2; ++mh) {
          const int mi = h * (MI / 2) + mh;
#pragma unroll
          for (int nb = 0; nb < BPH; ++nb) {
            const uint2 w = vt_quad_transpose(acc[mi][nb][0], acc[mi][nb][1], acc[mi][nb][2], acc[mi][nb][3], lo);
            const int row = nb * 16 + 4 * eq4 + t;
            const int chunk = 2 * mh + (sj >> 1);
            *reinterpret_cast<uint2*>(ep + row * 128 + ((chunk ^ (row & 7)) << 4) + (sj & 1) * 8) = w;
          }
        }
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
        uint16_t* vrow = q.v_out + ((tb * q.nkv + head) * kHD + (lo >> 3)) * q.vt_ld + ts0 + h * HALF_ROWS + k * 8;
#pragma unroll 4
        for (int i = 0; i < kHD / 8; ++i) {
          const int row = i * 8 + (lo >> 3);
          const uint4 v = *reinterpret_cast<const uint4*>(ep + row * 128 + ((k ^ (row & 7)) << 4));
          store_nt16(vrow + (int64_t)i * 8 * q.vt_ld, v);
        }
      }
      return;
    }
    // Norm weights of this lane's columns, fp32; all ones without QK norm (no branch
    // between the norm and the rotation).
    const uint16_t* nw = kind == 0 ? q.q_norm_w : q.k_norm_w;
    const bool norm = nw != nullptr;
    // Two bf16 ones, made opaque here: as a known constant the pair was set up once
    // before the tile loop and spilled.
    uint32_t one2 = 0x3F803F80u;
    asm volatile("" : "+v"(one2));
    uint2 wpk[BPH];
#pragma unroll
    for (int nb = 0; nb < BPH; ++nb) wpk[nb] = make_uint2(one2, one2);
    if (norm) {
#pragma unroll
      for (int nb = 0; nb < BPH; ++nb) wpk[nb] = *reinterpret_cast<const uint2*>(nw + nb * 16 + 4 * eq4);
    }
    float wf[BPH][4];
#pragma unroll
    for (int nb = 0; nb < BPH; ++nb) {
      wf[nb][0] = __uint_as_float(wpk[nb].x << 16);
      wf[nb][1] = __uint_as_float(wpk[nb].x & 0xffff0000u);
      wf[nb][2] = __uint_as_float(wpk[nb].y << 16);
      wf[nb][3] = __uint_as_float(wpk[nb].y & 0xffff0000u);
    }
    const int jc = lo % OUT_CH;
    uint16_t* obase = kind == 0 ? q.q_out : q.k_out;
    const int nheads = kind == 0 ? q.nq : q.nkv;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int mh = 0; mh < MI / 2; ++mh) {
        __builtin_amdgcn_sched_barrier(0);  // one block of accumulators live at a time
        const int mi = h * (MI / 2) + mh;
        const int r = mh * 16 + erl;
        float x[BPH][4];
#pragma unroll
        for (int nb = 0; nb < BPH; ++nb)
#pragma unroll
          for (int v = 0; v < 4; ++v) x[nb][v] = acc[mi][nb][v];
        // (cos, sin) of this lane's first-half columns at the row's position.
        const float2* csp = reinterpret_cast<const float2*>(q.cos_sin) + (q.pos0 + ts0 + mi * 16 + erl) * (kHD / 2);
        float4 cs[BPH / 2][2];
#pragma unroll
        for (int nb = 0; nb < BPH / 2; ++nb) {
          const int c = nb * 16 + 4 * eq4;
          cs[nb][0] = *reinterpret_cast<const float4*>(csp + c);
          cs[nb][1] = *reinterpret_cast<const float4*>(csp + c + 2);
        }
        qk_norm_rope<BPH>(x, wf, cs, norm, q.eps);
#pragma unroll
        for (int nb = 0; nb < BPH; ++nb) {
          const int col = nb * 16 + 4 * eq4;
          uint2 o;
          o.x = pack_bf16x2(x[nb][0], x[nb][1]);
          o.y = pack_bf16x2(x[nb][2], x[nb][3]);
          const int ch = (col >> 3) ^ (r % OUT_CH);
          *reinterpret_cast<uint2*>(ep + r * OUT_ROWB + ch * 16 + ((col >> 2) & 1) * 8) = o;
        }
      }
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
      uint16_t* orow = obase + ((tb * nheads + head) * q.S + ts0 + h * HALF_ROWS + lo / OUT_CH) * kHD + jc * 8;
#pragma unroll 4
      for (int i = 0; i < HALF_ROWS / RPI; ++i) {
        const int r = i * RPI + lo / OUT_CH;
        const uint4 v = *reinterpret_cast<const uint4*>(ep + r * OUT_ROWB + ((jc ^ (r % OUT_CH)) << 4));
        store_nt16(orow + (int64_t)i * RPI * kHD, v);
      }
    }
  };
  // SwiGLU: packed B rows come in groups of 64, 32 gate rows then the matching 32 up
  // rows (blocks 4 g, 4 g + 1 gate, 4 g + 2, 4 g + 3 up); the wave's output columns
  // are 32 g + 16 (ni % 4) + 4 q4, all WM rows staged at once; rows at or past the
  // segment's end are not stored.
  auto epilogue = [&](int stage, int64_t m0, int64_t m_end, int n0) __attribute__((always_inline)) {
    const int jc = lane % OUT_CH;
    if constexpr (EP == Epi::kQKRope) {
      epilogue_rope(stage, m0, n0);
      return;
    }
    if constexpr (EP == Epi::kSwiGLU) {
      uint8_t* ep = lds + stage * STAGE_BYTES + wave * (WM * OUT_ROWB);
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
            const int col = (ni >> 2) * 32 + 16 * h + 4 * q4;
            uint2 o;
            o.x = pack_bf16x2(a4[0], a4[1]);
            o.y = pack_bf16x2(a4[2], a4[3]);
            const int ch = (col >> 3) ^ (r % OUT_CH);
            *reinterpret_cast<uint2*>(ep + r * OUT_ROWB + ch * 16 + ((col >> 2) & 1) * 8) = o;
          }
      }
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
      const int n = (n0 + wn * WN) / 2 + jc * 8;
#pragma unroll 4
      for (int i = 0; i < WM / RPI; ++i) {
        const int r = i * RPI + lane / OUT_CH;
        const int64_t gm = m0 + wm * WM + r;
        const uint4 v = *reinterpret_cast<const uint4*>(ep + r * OUT_ROWB + ((jc ^ (r % OUT_CH)) << 4));
        if (gm < m_end && 2 * n < p.N) store_nt16(p.c + gm * p.ldc + n, v);
      }
      return;
    }
    uint8_t* ep = lds + stage * STAGE_BYTES + wave * (HALF_ROWS * OUT_ROWB);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint16_t* crow = p.c + (m0 + wm * WM + h * HALF_ROWS + lane / OUT_CH) * p.ldc + n0 + wn * WN + jc * 8;
      // Residual add: the half's pieces of c are loaded before the staging, so that
      // their latency runs under it; each piece belongs to this lane alone.
      uint4 resid[EP == Epi::kScatterAdd ? HALF_ROWS / RPI : 1];
      if constexpr (EP == Epi::kScatterAdd) {
#pragma unroll
        for (int i = 0; i < HALF_ROWS / RPI; ++i)
          resid[i] = *reinterpret_cast<const uint4*>(crow + (int64_t)i * RPI * p.ldc);
      }
#pragma unroll
      for (int mh = 0; mh < MI / 2; ++mh) {
        const int mi = h * (MI / 2) + mh;
        const int r = mh * 16 + rl;
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
          float y[4] = {acc[mi][ni][0], acc[mi][ni][1], acc[mi][ni][2], acc[mi][ni][3]};
          if constexpr (EP == Epi::kBiasClamp) {
            const float bb[4] = {bias4[ni].x, bias4[ni].y, bias4[ni].z, bias4[ni].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) y[j] = fminf(fmaxf(y[j] + bb[j], p.lo), p.hi);
          }
          const int col = ni * 16 + 4 * q4;
          uint2 o;
          o.x = pack_bf16x2(y[0], y[1]);
          o.y = pack_bf16x2(y[2], y[3]);
          const int ch = (col >> 3) ^ (r % OUT_CH);
          *reinterpret_cast<uint2*>(ep + r * OUT_ROWB + ch * 16 + ((col >> 2) & 1) * 8) = o;
        }
      }
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
      // Each store takes its data from a read of the region, so the region is read
      // in full before the next half overwrites it.
      if constexpr (EP == Epi::kScatterAdd) {
#pragma unroll
        for (int i = 0; i < HALF_ROWS / RPI; ++i) {  // resid[] is indexed by constants only
          const int r = i * RPI + lane / OUT_CH;
          const uint4 v = *reinterpret_cast<const uint4*>(ep + r * OUT_ROWB + ((jc ^ (r % OUT_CH)) << 4));
          store_nt16(crow + (int64_t)i * RPI * p.ldc, add_bf16x8(v, resid[i]));
        }
      } else {
#pragma unroll 4
        for (int i = 0; i < HALF_ROWS / RPI; ++i) {
          const int r = i * RPI + lane / OUT_CH;
          const uint4 v = *reinterpret_cast<const uint4*>(ep + r * OUT_ROWB + ((jc ^ (r % OUT_CH)) << 4));
          store_nt16(crow + (int64_t)i * RPI * p.ldc, v);
        }
      }
    }
  };

  // ---- prologue: the first tile's steps 0 and 1 in flight, step 0 landed ---------
#pragma unroll
  for (int s = 0; s < kStages; ++s) {
#pragma unroll
    for (int d = 0; d < LD_PER_STEP; ++d) dma1(StepSrc{s * kBK, false, true}, s, d);
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(LD_PER_STEP, 15));
  __syncthreads();
  read_frags(0, 0, 0);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
  __builtin_amdgcn_sched_barrier(0);

  int stage = 0;
  zero_acc();
  while (true) {
    for (int kt = 0; kt + 1 < KT; ++kt) {
      kstep(kt, stage, stage ^ 1, false);
      stage ^= 1;
    }
    load_bias(cur_n0);
    // The tile's last step: its wait and barrier also cover the next tile's step 0;
    // afterwards nobody reads `stage`.
    kstep(KT - 1, stage, stage ^ 1, true);
    epilogue(stage, cur_m0, cur_m_end, cur_n0);
    if (!has_next) break;
    // Every wave is done with the staging region (its reads were waited for above):
    // the next tile's step 1 goes there.  A plain barrier: the stores just issued
    // need not be complete.
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    ti += x_blocks;
    cur_m0 = nxt_m0;
    cur_m_end = nxt_m_end;
    cur_n0 = nxt_n0;
    cur_a = nxt_a;
    cur_a2 = nxt_a2;
    cur_b = nxt_b;
    cur_b2 = nxt_b2;
    has_next = ti + x_blocks < x_count;
    int t_s0 = 0, t_s1 = 0, t_ci = 0;
    if constexpr (kGathered) {
      t_s0 = seg_tab[lane];
      t_s1 = seg_tab[64 + lane];
      t_ci = seg_tab[128 + lane];
    }
    tile_at(has_next ? ti + x_blocks : ti, nxt_m0, nxt_m_end, nxt_n0, nxt_a, nxt_a2, nxt_b, nxt_b2, t_s0,
            t_s1, t_ci);
    if constexpr (kGathered) {
#pragma unroll
      for (int j = 0; j < LD_A; ++j) cur_goff[j] = nxt_goff[j];
      if (has_next) gather_offsets(nxt_m0, nxt_m_end, nxt_goff);
    }
    // An opaque K position: with kBK known, the compiler reused the prologue's A-offset
    // selects for these DMAs and kept them (spilled) through the whole tile loop.
    int k1 = kBK;
    asm volatile("" : "+s"(k1));
#pragma unroll
    for (int d = 0; d < LD_PER_STEP; ++d) dma1(StepSrc{k1, false, true}, stage, d);
    stage ^= 1;  // the next tile's step 0
    read_frags(stage, 0, 0);
    zero_acc();
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
    __builtin_amdgcn_sched_barrier(0);
  }
}

}  // namespace cdx
