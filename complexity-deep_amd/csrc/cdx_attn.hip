// Causal GQA attention forward for gfx950: the attention core that follows the fused
// mu-QKV + QK-norm + RoPE projection.
//
// Reference behaviour: core/attention.py:162-181 — K and V repeated over query-head
// groups (repeat_interleave), F.scaled_dot_product_attention(q, k, v, is_causal=True)
// (top-left causal mask, scale 1/sqrt(head_dim)), then the [B, S, heads * D] merge
// fed to o_proj.  Here query head h reads key/value head h / (nq / nkv) directly and
// the output is written in the merged [B, S, nq * D] layout.
//
// Design (one block = 128 queries of one (batch, head); 4 waves x 32 query rows):
//   * S^T = K Q^T per 64-key tile with v_mfma_f32_32x32x16_bf16 issued as
//     mfma(K_frag, Q_frag): each lane then holds one query row m = lane % 32 and 32
//     of the tile's 64 scores (its partner lane l ^ 32 the other 32), so the online
//     softmax statistics are per-lane scalars plus one cross-half exchange.
//   * O^T += V^T P as mfma(V^T_frag, P_frag): P never leaves registers; the score
//     layout is exactly the B-operand layout once the key order inside each 16-key
//     group matches.  V therefore arrives transposed, [B, nkv, D, vt_ld], with that key
//     order (vt_col in cdx_gemm.h), written so by the projection's epilogue.
//   * K and V^T tiles are DMA'd (buffer_load_dwordx4 ... lds, one buffer descriptor
//     per (batch, kv head) slice) into two K and two V^T LDS buffers with the same
//     256-byte-line chunk swizzle as the GEMM engine; one barrier per tile.
//   * Software pipeline inside each wave: while the softmax of tile t runs on the
//     vector ALU, the QK MFMAs of tile t + 1 and the PV MFMAs of tile t are issued
//     between its pieces, so the matrix pipe is fed during the softmax.  The loop is
//     unrolled by buffer parity (offsets are instruction immediates) and split so
//     that every loop body is straight-line code: only a wave's last tile is masked.
//   * Causal work: the block visits key tiles up to its last query; a wave skips the
//     MFMAs of tiles entirely above its rows; the last query tiles, which do the most
//     work, are launched first.
//   * Softmax in the log2 domain: t = s * log2(e) / sqrt(D) folded into one FMA
//     before exp2; running max m and sum l, with the rescale of O and l by
//     exp2(m_old - m_new) done only when a row's max passes m by more than kLazy;
//     l sums the bf16-rounded P that the PV product uses (v_dot2 with ones); the
//     lane-half exchanges use v_permlane32_swap; one division by l at the end; one
//     bf16 rounding of O.
#include <type_traits>

#include "cdx_gemm.h"

namespace cdx {
namespace {

struct AttnParams {
  const uint16_t* q;   // [B, nq, S, HD]
  const uint16_t* k;   // [B, nkv, S, HD]
  const uint16_t* vt;  // [B, nkv, HD, vt_ld], keys in vt_col order
  uint16_t* out;       // [B, S, nq * HD]
  int64_t S;
  int64_t vt_ld;
  int32_t B, nq, nkv;
  int32_t q_tiles;
  float scale_log2;    // log2(e) * scale
};

constexpr int kAttnBM = 128;  // queries per block, 32 per wave
constexpr int kAttnBN = 64;   // keys per tile
constexpr float kLazy = 8.f;  // log2-domain headroom before the running max is moved

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

// Both values of x held by lanes l and l ^ 32 (v_permlane32_swap: no LDS round trip).
__device__ __forceinline__ void halves(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

template <int HD>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(const AttnParams p) {
  constexpr int KROW = HD * 2;              // bytes per K row
  constexpr int K_CPR = HD / 8;             // 16-byte chunks per K row
  constexpr int K_RPL = 256 / KROW;         // K rows per 256-byte bank line
  constexpr int K_BYTES = kAttnBN * KROW;   // one K tile
  constexpr int V_ROWB = kAttnBN * 2;       // 128 bytes per V^T row (64 keys)
  constexpr int V_BYTES = HD * V_ROWB;      // one V^T tile
  constexpr int V_BASE = 2 * K_BYTES;       // two K buffers, then two V^T buffers
  constexpr int NKD = HD / 16;              // K16 steps over the head dim
  constexpr int NDB = HD / 32;              // 32-row blocks of O^T
  constexpr int KPW = K_BYTES / 1024 / 4;   // K DMA instructions per wave and tile
  constexpr int VPW = V_BYTES / 1024 / 4;   // V^T DMA instructions per wave and tile
  constexpr int K_ROWS_DMA = 1024 / KROW;   // K rows one DMA instruction fills
  static_assert(HD == 32 || HD == 64 || HD == 128, "head dim must be 32, 64 or 128");
  static_assert(KPW >= 1 && VPW >= 1, "tile too small for the DMA layout");

  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * K_BYTES + 2 * V_BYTES];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hi = lane >> 5;
  const int r32 = lane & 31;

  // ---- block -> (query tile, batch, head), heaviest query tiles first ----------
  const int bh_count = p.B * p.nq;
  const int qt = p.q_tiles - 1 - (int)(blockIdx.x / bh_count);
  const int bh = blockIdx.x % bh_count;
  const int b = bh / p.nq, h = bh % p.nq;
  const int kvh = h / (p.nq / p.nkv);
  const int64_t S = p.S;
  const int64_t q0 = (int64_t)qt * kAttnBM;
  const int64_t mw = q0 + wave * 32;  // first query row of this wave
  const int64_t m = mw + r32;         // this lane's query row
  // Key n is visible to query m iff n <= m (top-left causal) and n < S.
  const int64_t kv_end = min(S, q0 + kAttnBM);
  const int nt = (int)((kv_end + kAttnBN - 1) / kAttnBN);  // tiles of the block
  // Tiles of this wave (0 when all its rows are past the end).
  const int ntw = mw < S ? (int)((min(S, mw + 32) + kAttnBN - 1) / kAttnBN) : 0;

  // ---- Q fragments: B operand, row m, head dims 16 k + 8 hi .. + 8 ---------------
  bf16x8 qf[NKD];
  {
    const int64_t mr = m < S ? m : S - 1;
    const uint16_t* qrow = p.q + (((int64_t)b * p.nq + h) * S + mr) * HD + 8 * hi;
#pragma unroll
    for (int k = 0; k < NKD; ++k) qf[k] = *reinterpret_cast<const bf16x8*>(qrow + 16 * k);
  }

  // ---- DMA sources ---------------------------------------------------------------
  // K tile row r (key n0 + r): chunk c at position c ^ ((r / K_RPL) % K_CPR).
  // V^T tile row d (keys n0 .. n0 + 63, 128 bytes): chunk c at position c ^ ((d / 2) % 8).
  // Buffer loads straight to LDS, one descriptor per (batch, kv head) slice.  The K
  // descriptor covers exactly S rows and the tile's row offset is added to each lane's
  // vector offset, which the buffer range check always covers, so rows past the end
  // read as zeros (and are masked) without leaving the K allocation; whether the
  // check also covers the instruction's scalar offset is not relied on.  V^T tiles
  // move along a row by their key position (scalar offset): columns up to vt_ld are
  // inside the slice and finite by contract.
  const __amdgpu_buffer_rsrc_t rs_k =
      make_rsrc(p.k + ((int64_t)b * p.nkv + kvh) * S * HD, (uint32_t)(S * HD * 2));
  const __amdgpu_buffer_rsrc_t rs_v = make_rsrc(p.vt + ((int64_t)b * p.nkv + kvh) * HD * p.vt_ld);
  uint32_t k_off[KPW], v_off[VPW];
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    const int r = (wave * KPW + j) * K_ROWS_DMA + lane / K_CPR;
    k_off[j] = (uint32_t)(r * HD + ((lane % K_CPR) ^ ((r / K_RPL) % K_CPR)) * 8) * 2;
  }
#pragma unroll
  for (int j = 0; j < VPW; ++j) {
    const int d = (wave * VPW + j) * 8 + lane / 8;
    v_off[j] = (uint32_t)((int64_t)d * p.vt_ld + ((lane % 8) ^ ((d / 2) % 8)) * 8) * 2;
  }
  auto issue_k = [&](int t, int buf) __attribute__((always_inline)) {
    const uint32_t tile_off = (uint32_t)t * (kAttnBN * HD * 2);
#pragma unroll
    for (int j = 0; j < KPW; ++j)
      buf_dma16(rs_k, k_off[j] + tile_off, 0u, lds + buf * K_BYTES + (wave * KPW + j) * 1024);
  };
  auto issue_v = [&](int t, int buf) __attribute__((always_inline)) {
    const uint32_t n0 = (uint32_t)t * kAttnBN;
#pragma unroll
    for (int j = 0; j < VPW; ++j)
      buf_dma16(rs_v, v_off[j], n0 * 2, lds + V_BASE + buf * V_BYTES + (wave * VPW + j) * 1024);
  };

  // ---- fragment offsets ----------------------------------------------------------
  // Key block kb (rows 32 kb + r32) and head-dim block db (rows 32 db + r32) see the
  // same swizzle as block 0, so one offset per K16 step / key slab serves all blocks.
  int kf_off[NKD];
#pragma unroll
  for (int k = 0; k < NKD; ++k) kf_off[k] = r32 * KROW + (((2 * k + hi) ^ ((r32 / K_RPL) % K_CPR)) << 4);
  int vf_off[4];
#pragma unroll
  for (int sl = 0; sl < 4; ++sl) vf_off[sl] = r32 * V_ROWB + (((2 * sl + hi) ^ ((r32 / 2) % 8)) << 4);

  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[db][v] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  // Scores S^T of two tiles (the one in softmax and the next one): [set][key block].
  f32x16 sacc[2][2];

  // QK MFMA j of a tile (j < 2 NKD, key-block major: kb = j / NKD, K16 step
  // k = j % NKD) reads K fragment j; fragments are read two MFMAs ahead.
  constexpr int NQK = 2 * NKD;
  bf16x8 kfr[3];
  auto k_read = [&](int kbuf, int j) __attribute__((always_inline)) {
    kfr[j % 3] = *reinterpret_cast<const bf16x8*>(lds + kbuf * K_BYTES + kf_off[j % NKD] + (j / NKD) * 32 * KROW);
  };
  auto qk_mfma = [&](int set, int j) __attribute__((always_inline)) {
    const int kb = j / NKD, k = j % NKD;
    sacc[set][kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfr[j % 3], qf[k], k == 0 ? f32x16{} : sacc[set][kb], 0, 0, 0);
  };

  // Softmax of tile t (scores in set `set`), in pieces: piece 0 masks (the wave's last
  // tile only) and takes the row max (and moves the running max when needed), pieces
  // 1..4 turn one 16-key slab into bf16 P and its row sum, piece 5 folds the lane
  // halves of the row sum.
  bf16x8 pf[4];  // [16-key slab], the B operand of O^T += V^T P
  float rsum[4];
  auto softmax_piece = [&](int set, int t, int piece, auto msk) __attribute__((always_inline)) {
    if (piece == 0) {
      if constexpr (decltype(msk)::value) {
        // Causal / length mask of the wave's last tile, the only one that reaches its
        // rows (its 32 rows lie inside one 64-key tile) or the end of the sequence:
        // key n0 + idx is visible iff idx <= lim; idx = c + 4 hi with c a per-score
        // constant, so comparing c against lim - 4 hi keeps the constants immediates.
        const int64_t n0 = (int64_t)t * kAttnBN;
        const int64_t last = (m < S ? m : S - 1) - n0;
        const int lim = (int)(last < kAttnBN ? last : kAttnBN) - 4 * hi;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int c = kb * 32 + 8 * (v >> 2) + (v & 3);
            sacc[set][kb][v] = c > lim ? -INFINITY : sacc[set][kb][v];
          }
      }
      // Row max in log2 units: two independent three-input max chains over the
      // lane's 32 scores, then the partner lane's half.
      float x[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        x[kb] = fmaxf(sacc[set][kb][0], sacc[set][kb][1]);
#pragma unroll
        for (int v = 2; v < 16; v += 2) x[kb] = fmaxf(fmaxf(x[kb], sacc[set][kb][v]), sacc[set][kb][v + 1]);
      }
      float a, c;
      halves(fmaxf(x[0], x[1]), a, c);
      const float mx = fmaxf(a, c) * p.scale_log2;
      // Lazy rescale: the reference max m_run (log2 units) moves only when a row's
      // max passes it by more than kLazy; until then P = 2^(t - m_run) <= 2^kLazy,
      // which bf16 and fp32 hold, and the final division by l cancels the reference.
      // Tile 0 holds key 0, visible to every row, so m_run is finite from then on.
      if (__builtin_amdgcn_ballot_w64(mx > m_run + kLazy) != 0) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
        m_run = m_new;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int v = 0; v < 16; ++v) o[db][v] *= alpha;
      }
    } else if (piece <= 4) {
      // P of one 16-key slab and its row sum (of the rounded P, the weights the PV
      // product uses; two per instruction).
      const int sl = piece - 1, kb = sl >> 1, g = sl & 1;
      const bf16x2_t ones = __builtin_bit_cast(bf16x2_t, 0x3F803F80u);
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[set][kb][8 * g + 2 * j], p.scale_log2, -m_run));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[set][kb][8 * g + 2 * j + 1], p.scale_log2, -m_run));
        w[j] = pack_bf16x2(p0, p1);
      }
      const float r01 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[0]), ones, 0.f, false);
      const float r23 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[2]), ones, 0.f, false);
      rsum[sl] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[1]), ones, r01, false) +
                 __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[3]), ones, r23, false);
      pf[sl] = __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
    } else {
      float a, c;
      halves((rsum[0] + rsum[1]) + (rsum[2] + rsum[3]), a, c);
      l_run += a + c;
    }
  };

  // O^T += V^T P: V^T fragments of one 16-key slab (double-buffered by slab parity),
  // and the slab's NDB MFMAs.
  bf16x8 vfr[2][NDB];
  auto v_read = [&](int vbuf, int sl) __attribute__((always_inline)) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      vfr[sl & 1][db] =
          *reinterpret_cast<const bf16x8*>(lds + V_BASE + vbuf * V_BYTES + vf_off[sl] + db * 32 * V_ROWB);
  };
  auto pv_slab = [&](int sl) __attribute__((always_inline)) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfr[sl & 1][db], pf[sl], o[db], 0, 0, 0);
  };

  // ---- pipeline ------------------------------------------------------------------
  // LDS holds two K buffers and two V^T buffers.  Iteration t runs the softmax of
  // tile t (scores already in registers) and O += V(t)^T P(t) (V buffer t % 2)
  // interleaved with the QK MFMAs of tile t + 1 (K buffer (t + 1) % 2), so that the
  // matrix pipe and the vector ALU of one wave work side by side.  The iteration's
  // DMAs, issued after its barrier, fetch K(t + 2) into the K buffer tile t used and
  // V(t + 1) into the V buffer tile t - 1 used; both land before the next barrier.
  //
  // Event order of an iteration, each behind the QK MFMA of its slot (positions are
  // for 16 QK MFMAs and scale with the head dim):
  //   softmax piece 0 @0, piece 1 @2, V slab 0 @3, piece 2 @4, PV slab 0 @5,
  //   V slab 1 @5, piece 3 @6, PV slab 1 @7, V slab 2 @7, piece 4 @8, PV slab 2 @9,
  //   V slab 3 @9, piece 5 @10, PV slab 3 @11.
  constexpr int kEvents = 14;
  constexpr int kEvPos[kEvents] = {0, 2, 3, 4, 5, 5, 6, 7, 7, 8, 9, 9, 10, 11};
  // event kind: 0..5 softmax piece, 10 + s V read of slab s, 20 + s PV slab s
  constexpr int kEvKind[kEvents] = {0, 1, 10, 2, 20, 11, 3, 21, 12, 4, 22, 13, 5, 23};
  auto event = [&](int t, int cur, int e, auto msk) __attribute__((always_inline)) {
    const int kind = kEvKind[e];
    if (kind < 10) softmax_piece(cur, t, kind, msk);
    else if (kind < 20) v_read(cur, kind - 10);
    else pv_slab(kind - 20);
  };

  // Block-uniform part of iteration t: wait until K(t + 1) and V(t) have landed and
  // every wave is done with K(t) and V(t - 1), then refill those buffers.
  auto sync = [&](int t, int cur) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
    __syncthreads();
    if (t + 2 < nt) issue_k(t + 2, cur);
    if (t + 1 < nt) issue_v(t + 1, cur ^ 1);
  };
  // Tile t of parity `par` with the next tile's QK MFMAs interleaved; never masked.
  auto body = [&](int t, auto par) __attribute__((always_inline)) {
    constexpr int cur = decltype(par)::value;
    constexpr int nxt = cur ^ 1;
    sync(t, cur);
    k_read(nxt, 0);
    k_read(nxt, 1);
#pragma unroll
    for (int j = 0; j < NQK; ++j) {
      if (j + 2 < NQK) k_read(nxt, j + 2);
      qk_mfma(nxt, j);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int e = 0; e < kEvents; ++e)
        if (kEvPos[e] * NQK / 16 == j) event(t, cur, e, std::false_type{});
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // The wave's last tile: masked, nothing to overlap.
  auto last = [&](int t, auto par) __attribute__((always_inline)) {
    constexpr int cur = decltype(par)::value;
    sync(t, cur);
#pragma unroll
    for (int e = 0; e < kEvents; ++e) event(t, cur, e, std::true_type{});
  };

  issue_k(0, 0);
  if (nt > 1) issue_k(1, 1);
  issue_v(0, 0);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
  __syncthreads();
  if (ntw > 0) {
    k_read(0, 0);
    k_read(0, 1);
#pragma unroll
    for (int j = 0; j < NQK; ++j) {
      if (j + 2 < NQK) k_read(0, j + 2);
      qk_mfma(0, j);
    }
  }

  // Every wave passes sync(t) once for each t < nt, in order, so the barriers pair up.
  int t = 0;
  for (; t + 2 < ntw; t += 2) {
    body(t, std::integral_constant<int, 0>{});
    body(t + 1, std::integral_constant<int, 1>{});
  }
  if (t + 1 < ntw) {
    body(t, std::integral_constant<int, 0>{});
    ++t;
  }
  if (t < ntw) {
    if (t & 1) last(t, std::integral_constant<int, 1>{});
    else last(t, std::integral_constant<int, 0>{});
    ++t;
  }
  for (; t < nt; ++t) sync(t, t & 1);

  // ---- O = O^T / l -> out[b, m, h * HD + d] ----------------------------------------
  // A lane holds 8-byte pieces of one query row, so direct stores would write 16-byte
  // runs of 32 rows per instruction.  The rows are staged through the K buffers
  // instead (free once every wave is past its last tile; 32 rows of HD values per
  // wave fill them exactly), 16-byte chunk c of row r at position c ^ (r % OCH), and
  // go out as whole HD * 2-byte rows.
  constexpr int OROWB = HD * 2, OCH = OROWB / 16, ORPI = 64 / OCH;
  static_assert(4 * 32 * OROWB <= 2 * K_BYTES, "output staging must fit the K buffers");
  __syncthreads();
  uint8_t* ost = lds + wave * 32 * OROWB;
  const float inv_l = 1.f / l_run;  // rows past S (l = 0) are staged but never stored
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint2 w;
      w.x = pack_bf16x2(o[db][4 * g + 0] * inv_l, o[db][4 * g + 1] * inv_l);
      w.y = pack_bf16x2(o[db][4 * g + 2] * inv_l, o[db][4 * g + 3] * inv_l);
      const int ch = (db * 4 + g) ^ (r32 % OCH);
      *reinterpret_cast<uint2*>(ost + r32 * OROWB + ch * 16 + hi * 8) = w;
    }
  // The wave's own LDS writes complete before its reads (and stay ahead of them).
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
  const int jc = lane % OCH;
  uint16_t* obase = p.out + (int64_t)h * HD + jc * 8;
#pragma unroll
  for (int i = 0; i < 32 / ORPI; ++i) {
    const int r = i * ORPI + lane / OCH;
    const uint4 v = *reinterpret_cast<const uint4*>(ost + r * OROWB + ((jc ^ (r % OCH)) << 4));
    const int64_t mr = mw + r;
    if (mr < S) *reinterpret_cast<uint4*>(obase + ((int64_t)b * S + mr) * ((int64_t)p.nq * HD)) = v;
  }
}

template <int HD>
int launch_attn(const AttnParams& p, hipStream_t s) {
  const int64_t blocks = (int64_t)p.q_tiles * p.B * p.nq;
  if (blocks > INT32_MAX) return fail(CDX_EUNSUPPORTED, "cdx_attention_fwd: problem too large");
  attn_fwd_kernel<HD><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(p);
  return check_launch("cdx_attention_fwd");
}

}  // namespace
}  // namespace cdx

extern "C" int cdx_attention_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* vt, int64_t B,
                                 int64_t S, int32_t nq, int32_t nkv, int32_t hd, int64_t vt_ld, float scale,
                                 uint16_t* out, void* stream) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_attention_fwd";
  if (B < 0 || S < 0 || nq <= 0 || nkv <= 0 || nq % nkv != 0)
    return fail(CDX_EINVAL, "%s: bad shape B=%lld S=%lld nq=%d nkv=%d", name, (long long)B, (long long)S, nq, nkv);
  if (hd != 32 && hd != 64 && hd != 128)
    return fail(CDX_EUNSUPPORTED, "%s: head dim %d must be 32, 64 or 128", name, hd);
  if (vt_ld < S || vt_ld % 64 != 0)
    return fail(CDX_EINVAL, "%s: vt_ld=%lld must be a multiple of 64 that is >= S", name, (long long)vt_ld);
  if (!(scale > 0.f)) return fail(CDX_EINVAL, "%s: scale must be > 0", name);
  if (B == 0 || S == 0) return CDX_OK;
  if ((S + kAttnBM - 1) / kAttnBM > INT32_MAX || B * nq > INT32_MAX)
    return fail(CDX_EUNSUPPORTED, "%s: problem too large", name);
  // The kernel addresses one (batch, kv head) slice of K and of V^T with 32-bit offsets;
  // a K tile's offsets reach up to 64 rows past the slice (those rows read as zeros).
  if ((S + 64) * hd * 2 > (int64_t)UINT32_MAX || vt_ld * hd * 2 > (int64_t)UINT32_MAX)
    return fail(CDX_EUNSUPPORTED, "%s: a K or V^T head slice must fit 4 GB (S=%lld)", name, (long long)S);
  if (!q || !k || !vt || !out) return fail(CDX_EINVAL, "%s: null pointer", name);
  if (!aligned16(q) || !aligned16(k) || !aligned16(vt) || !aligned16(out))
    return fail(CDX_EUNSUPPORTED, "%s: pointers must be 16-byte aligned", name);
  AttnParams p{};
  p.q = q;
  p.k = k;
  p.vt = vt;
  p.out = out;
  p.S = S;
  p.vt_ld = vt_ld;
  p.B = (int32_t)B;
  p.nq = nq;
  p.nkv = nkv;
  p.q_tiles = (int32_t)((S + kAttnBM - 1) / kAttnBM);
  p.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (hd) {
    case 32: return launch_attn<32>(p, s);
    case 64: return launch_attn<64>(p, s);
    default: return launch_attn<128>(p, s);
  }
}
