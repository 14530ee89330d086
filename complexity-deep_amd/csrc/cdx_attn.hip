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
//     per (batch, kv head) slice) into two LDS stages with the same 256-byte-line
//     chunk swizzle as the GEMM engine; the next tile's DMA is in flight while the
//     current one is consumed; one barrier per tile.  The tile loop is unrolled by
//     the two stages so that stage offsets are instruction immediates, and K
//     fragments are read through a rolling window ahead of their MFMAs.
//   * Causal work: the block visits key tiles up to its last query; a wave skips the
//     MFMAs of tiles entirely above its rows; the last query tiles, which do the most
//     work, are launched first.
//   * Softmax in the log2 domain: t = s * log2(e) / sqrt(D) folded into one FMA
//     before exp2; running max m and sum l, with the rescale of O and l by
//     exp2(m_old - m_new) done only when a row's max passes m by more than kLazy;
//     one division by l at the end; one bf16 rounding of O.
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

template <int HD>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(const AttnParams p) {
  constexpr int KROW = HD * 2;              // bytes per K row
  constexpr int K_CPR = HD / 8;             // 16-byte chunks per K row
  constexpr int K_RPL = 256 / KROW;         // K rows per 256-byte bank line
  constexpr int K_BYTES = kAttnBN * KROW;   // one K tile
  constexpr int V_ROWB = kAttnBN * 2;       // 128 bytes per V^T row (64 keys)
  constexpr int V_BYTES = HD * V_ROWB;      // one V^T tile
  constexpr int STAGE = K_BYTES + V_BYTES;
  constexpr int NKD = HD / 16;              // K16 steps over the head dim
  constexpr int NDB = HD / 32;              // 32-row blocks of O^T
  constexpr int KPW = K_BYTES / 1024 / 4;   // K DMA instructions per wave and tile
  constexpr int VPW = V_BYTES / 1024 / 4;   // V^T DMA instructions per wave and tile
  constexpr int K_ROWS_DMA = 1024 / KROW;   // K rows one DMA instruction fills
  static_assert(HD == 32 || HD == 64 || HD == 128, "head dim must be 32, 64 or 128");
  static_assert(KPW >= 1 && VPW >= 1, "tile too small for the DMA layout");

  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * STAGE];

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
  const int64_t mw = q0 + wave * 32;   // first query row of this wave
  const int64_t m = mw + r32;          // this lane's query row
  // Key n is visible to query m iff n <= m (top-left causal) and n < S.
  const int64_t kv_end = min(S, q0 + kAttnBM);
  const int nt = (int)((kv_end + kAttnBN - 1) / kAttnBN);
  const int nt_wave = (int)((min(S, mw + 32) + kAttnBN - 1) / kAttnBN);

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
  // Buffer loads straight to LDS: each lane's byte offset inside the (batch, kv head)
  // slice is fixed and the tile's key position travels in the scalar offset.  The K
  // descriptor covers exactly S rows, so rows past the end read as zeros (and are
  // masked); V^T columns up to vt_ld are in range and finite by contract.
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
  auto issue = [&](int t, int stage) __attribute__((always_inline)) {
    const uint32_t n0 = (uint32_t)t * kAttnBN;
    uint8_t* ks = lds + stage * STAGE;
    uint8_t* vs = ks + K_BYTES;
#pragma unroll
    for (int j = 0; j < KPW; ++j) buf_dma16(rs_k, k_off[j], n0 * HD * 2, ks + (wave * KPW + j) * 1024);
#pragma unroll
    for (int j = 0; j < VPW; ++j) buf_dma16(rs_v, v_off[j], n0 * 2, vs + (wave * VPW + j) * 1024);
  };

  // ---- fragment offsets in a stage -------------------------------------------------
  int kf_off[2][NKD];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int k = 0; k < NKD; ++k) {
      const int r = nb * 32 + r32;
      kf_off[nb][k] = r * KROW + (((2 * k + hi) ^ ((r / K_RPL) % K_CPR)) << 4);
    }
  int vf_off[NDB][4];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) {
      const int d = db * 32 + r32;
      vf_off[db][sl] = K_BYTES + d * V_ROWB + (((2 * sl + hi) ^ ((d / 2) % 8)) << 4);
    }

  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[db][v] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  issue(0, 0);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
  __syncthreads();

  // One key tile; STG is the tile's LDS stage as a compile-time constant, so the
  // stage offset folds into the LDS instructions' immediate offsets.
  auto tile = [&](int t, auto stg) __attribute__((always_inline)) {
    constexpr int stage = decltype(stg)::value;
    if (t + 1 < nt) issue(t + 1, stage ^ 1);
    if (t < nt_wave) {
      const uint8_t* st = lds + stage * STAGE;
      // S^T = K Q^T for the tile's two 32-key blocks.  The 2 NKD K fragments are read
      // through a rolling window: fragment i + KWIN is read behind the MFMA of
      // fragment i, so KWIN reads are in flight while the MFMAs run (the full set
      // does not fit next to O, the Q fragments and the V^T fragments).
      constexpr int NKF = 2 * NKD, KWIN = NKF < 6 ? NKF : 6;
      auto kfrag = [&](int i) __attribute__((always_inline)) {
        return *reinterpret_cast<const bf16x8*>(st + kf_off[i & 1][i >> 1]);
      };
      bf16x8 kfr[NKF];
#pragma unroll
      for (int i = 0; i < KWIN; ++i) kfr[i] = kfrag(i);
      f32x16 sacc[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int v = 0; v < 16; ++v) sacc[nb][v] = 0.f;
#pragma unroll
      for (int i = 0; i < NKF; ++i) {
        sacc[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfr[i], qf[i >> 1], sacc[i & 1], 0, 0, 0);
        if (i + KWIN < NKF) kfr[i + KWIN] = kfrag(i + KWIN);
        __builtin_amdgcn_sched_barrier(0);
      }
      // V^T fragments of the tile, in flight during the softmax.
      bf16x8 vfr[4 * NDB];
#pragma unroll
      for (int sl = 0; sl < 4; ++sl)
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          vfr[sl * NDB + db] = *reinterpret_cast<const bf16x8*>(st + vf_off[db][sl]);
      // Causal / length mask on the tiles that reach this wave's rows: key
      // n0 + idx is visible iff idx <= lim (one compare per score, no branches).
      const int64_t n0 = (int64_t)t * kAttnBN;
      if (n0 + kAttnBN - 1 > mw) {
        const int64_t last = (m < S ? m : S - 1) - n0;
        const int lim = (int)(last < kAttnBN ? last : kAttnBN);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int idx = nb * 32 + 8 * (v >> 2) + 4 * hi + (v & 3);
            sacc[nb][v] = idx > lim ? -INFINITY : sacc[nb][v];
          }
      }
      // Row max of the tile's raw scores.
      float mx = -INFINITY;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sacc[nb][v]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * p.scale_log2;
      // Lazy rescale: the reference max m_run (log2 units) moves only when a row's max
      // passes it by more than kLazy; until then P = 2^(t - m_run) <= 2^kLazy, which
      // bf16 and fp32 hold, and the final division by l cancels the reference.  Tile 0
      // holds key 0, visible to every row, so m_run is finite from then on.
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
      float rs = 0.f;
      bf16x8 pf[4];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          uint32_t w[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[nb][8 * g + 2 * j], p.scale_log2, -m_run));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[nb][8 * g + 2 * j + 1], p.scale_log2, -m_run));
            rs += p0 + p1;
            w[j] = pack_bf16x2(p0, p1);
          }
          pf[nb * 2 + g] = __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
        }
      rs += __shfl_xor(rs, 32, 64);
      l_run += rs;
      // O^T += V^T P over the tile's four 16-key slabs
#pragma unroll
      for (int sl = 0; sl < 4; ++sl)
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfr[sl * NDB + db], pf[sl], o[db], 0, 0, 0);
    }
    // next tile landed (own DMA) and this wave is done with `stage`
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
    __syncthreads();
  };
  for (int t = 0; t < nt; t += 2) {
    tile(t, std::integral_constant<int, 0>{});
    if (t + 1 < nt) tile(t + 1, std::integral_constant<int, 1>{});
  }

  // ---- O = O^T / l -> out[b, m, h * HD + d] ----------------------------------------
  if (m >= S) return;
  const float inv_l = 1.f / l_run;
  uint16_t* orow = p.out + ((int64_t)b * S + m) * ((int64_t)p.nq * HD) + (int64_t)h * HD;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint2 w;
      w.x = pack_bf16x2(o[db][4 * g + 0] * inv_l, o[db][4 * g + 1] * inv_l);
      w.y = pack_bf16x2(o[db][4 * g + 2] * inv_l, o[db][4 * g + 3] * inv_l);
      *reinterpret_cast<uint2*>(orow + db * 32 + 8 * g + 4 * hi) = w;
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
  // The kernel addresses one (batch, kv head) slice of K and of V^T with 32-bit offsets.
  if (S * hd * 2 > (int64_t)UINT32_MAX || vt_ld * hd * 2 > (int64_t)UINT32_MAX)
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
