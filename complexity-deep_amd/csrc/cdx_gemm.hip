// C-ABI entry points built on the MFMA tile engine (cdx_gemm.h):
//   cdx_mu_qkv_fwd       piece 2: one K = 2H contraction over [x | mu_prev] against
//                        [W_x | W_mu] (two weight sources, selected by the K half)
//   cdx_mu_qkv_rope_fwd  the same contraction with QK RMSNorm + RoPE fused into the
//                        epilogue, writing head-major q, k, v
//   cdx_mu_qkv_rope_bcast_fwd  the same for one broadcast mu row, its product with
//                        W_mu folded into a single 64-column K block
//   cdx_moe_swiglu_fwd   piece 1b: gather + gate/up + SwiGLU, then down + scatter,
//                        with the shared expert folded into both passes
//   cdx_moe_swiglu_residual_fwd  the same, the scattered rows added to the residual
//                        stream in place (the block's h = h + mlp(x))
//   cdx_grouped_gemm_fwd plain grouped GEMM over expert segments
//   cdx_mu_guidance_fwd  mu = clamp(h @ W_mu^T + clamp(mu_param), lo, hi), the
//                        producer of the next layer's mu operand (the parameter is
//                        read and clamped in the epilogue)
//   cdx_linear_fwd       y = x @ W^T (the tied LM head)
#include <type_traits>

#include "cdx_gemm_persist.h"

namespace cdx {
namespace {

// Tiles of 256 x 128 for products too small to fill the chip with 256 x 256 tiles.
// Their K steps are half as long, so three stages (144 KB) give each load two steps
// to land; refills ride behind every fourth MFMA of the step.
using NarrowCfg = GemmCfg<128, 64, 3, 1, 4, 1, 1>;
// Tiles of 256 x 64 for the plain epilogues (store, bias-clamp, scatter) of products
// that leave most CUs idle even with 256 x 128 tiles; the SwiGLU and QK-norm epilogues
// need a wave's 64 or more columns together.  Their ten refills per step ride behind
// every second MFMA.
using XNarrowCfg = GemmCfg<64, 64, 3, 1, 2, 1, 1>;
// Tiles of 128 rows (waves of 64 x 64 or 64 x 32) for products whose 256-row tiles
// leave many CUs idle (the small model's QKV, mu and MLP products): up to twice the
// blocks, each with half the MFMA work per K step.  128 x 128: three stages (96 KB,
// one block per CU), so that a load has two short K steps to land; in a forward,
// where each layer's weights come from HBM, that beat two stages by 4% although the
// register allocator then copies some accumulators between AGPRs on every K step
// (store, SwiGLU and QK-norm epilogues).  128 x 64: three stages of 24 KB, compiled
// for two blocks per CU (with that register budget its K loops keep the
// accumulators in place).
using SmallCfg = GemmCfg<128, 64, 3, 1, 2, 1, 1, 128>;
using XSmallCfg = GemmCfg<64, 64, 3, 2, 1, 0, 1, 128>;

template <ALoad AL, Epi EP, class Cfg = DefaultCfg, int HD = 0>
int launch(GemmParams p, hipStream_t s, const char* name) {
  p.nt_count = (p.N + Cfg::BN - 1) / Cfg::BN;
  const int64_t nb = (int64_t)p.mt_count * p.nt_count;
  if (nb == 0) return CDX_OK;
  // At most half as many 256 x 256 tiles as CUs (launch bound): half-width tiles give
  // twice the blocks, each with half the MFMA work per K step, still in one round.
  // (A head of 128 columns does not fit a narrow tile's 64-column waves.)
  if constexpr (Cfg::BN == 256 && (EP != Epi::kQKRope || HD <= 64)) {
    if (2 * nb <= device_cu_count()) return launch<AL, EP, NarrowCfg, HD>(p, s, name);
  }
  if constexpr (Cfg::BN == 128 && Cfg::BM == kBM && EP != Epi::kQKRope && EP != Epi::kSwiGLU) {
    if (2 * nb <= device_cu_count()) return launch<AL, EP, XNarrowCfg, HD>(p, s, name);
  }
  // 128-row tiles when they are all resident at once (RESIDENT blocks per CU).  The M
  // tile count is recounted for them (for the grouped passes, again an upper bound
  // with one partial tile per expert).
  if constexpr (Cfg::BM == kBM && Cfg::BN <= 128) {
    using Small = std::conditional_t<Cfg::BN == 128, SmallCfg, XSmallCfg>;
    const bool grouped = p.offsets != nullptr && AL != ALoad::kSegmented;
    const int64_t mt_small = (p.M + Small::BM - 1) / Small::BM + (grouped ? p.E : 0);
    if (mt_small * p.nt_count <= (int64_t)Small::RESIDENT * device_cu_count()) {
      p.mt_count = (int32_t)mt_small;
      return launch<AL, EP, Small, HD>(p, s, name);
    }
  }
  if (nb > INT32_MAX) return fail(CDX_EUNSUPPORTED, "%s: problem too large (%lld tiles)", name, (long long)nb);
  // The kernel's K loop runs at least once and whole steps only.
  if (p.K < Cfg::BK || p.K % Cfg::BK != 0)
    return fail(CDX_EUNSUPPORTED, "%s: K=%d must be a positive multiple of %d", name, p.K, Cfg::BK);
  // Whole tiles of a plain (unsegmented) product, the gathered SwiGLU pass with whole
  // N tiles, and mu-QKV with the QK-norm + RoPE epilogue (head dim 128, V transposed,
  // A from two sources switching at K = H, or from one: x alone, or x and mu side by
  // side in one [T, 2H] buffer;
  // whole M tiles, sequences a multiple of 128 tokens) run on the persistent form when
  // they have more tiles than CUs: one block per CU (a multiple of 8, so that every
  // XCD's share of the tiles has blocks) walking its XCD's tiles.  (For the gathered
  // pass nb is the launch bound on the per-expert tiles; the kernel counts the real
  // ones.)
  constexpr bool kDenseTiles =
      ((AL == ALoad::kDense || AL == ALoad::kConcat) && (EP == Epi::kStore || EP == Epi::kBiasClamp)) ||
      (AL == ALoad::kDense && EP == Epi::kScatterAdd);
  constexpr bool kGatherTiles = AL == ALoad::kGather && EP == Epi::kSwiGLU;
  constexpr bool kRopeTiles = (AL == ALoad::kConcat || AL == ALoad::kDense) && EP == Epi::kQKRope && HD == 128;
  if constexpr ((kDenseTiles || kGatherTiles || kRopeTiles) && Cfg::BN == 256) {
    const int64_t grid = (device_cu_count() + kNumXcd - 1) / kNumXcd * kNumXcd;
    bool whole = kGatherTiles ? p.offsets != nullptr : (p.offsets == nullptr && p.M % kBM == 0);
    if (EP == Epi::kScatterAdd) whole = whole && p.perm == nullptr;  // identity rows only
    if (kRopeTiles) whole = whole && p.qk.vt_ld > 0 && p.qk.S % (kBM / 2) == 0;
    if (whole && p.N % Cfg::BN == 0 && p.K >= 2 * Cfg::BK && nb > grid) {
      gemm_persist_kernel<Cfg, AL, EP, HD><<<dim3((unsigned)grid), dim3(kGemmThreads), 0, s>>>(p);
      return check_launch(name);
    }
  }
  gemm_nt_kernel<Cfg, AL, EP, HD><<<dim3((unsigned)nb), dim3(kGemmThreads), 0, s>>>(p);
  return check_launch(name);
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace
}  // namespace cdx

using cdx::ALoad;
using cdx::Epi;
using cdx::GemmParams;

extern "C" int cdx_mu_qkv_fwd(const uint16_t* x, int64_t ldx, const uint16_t* mu, int64_t ldmu,
                              const uint16_t* w, const uint16_t* w_mu, int64_t ldw, int64_t M, int32_t H,
                              int32_t N, uint16_t* out, int64_t ldo, void* stream) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_mu_qkv_fwd";
  if (M < 0 || H <= 0 || N <= 0) return fail(CDX_EINVAL, "%s: bad shape M=%lld H=%d N=%d", name, (long long)M, H, N);
  if (H % 64 != 0) return fail(CDX_EUNSUPPORTED, "%s: H=%d must be a multiple of 64", name, H);
  if (N % 8 != 0) return fail(CDX_EUNSUPPORTED, "%s: N=%d must be a multiple of 8", name, N);
  const int64_t K = mu ? 2 * (int64_t)H : (int64_t)H;
  if (ldx < H || ldo < N || ldw < H || (mu && ldmu != 0 && ldmu < H))
    return fail(CDX_EINVAL, "%s: leading dimension too small", name);
  if (ldx % 8 || ldo % 8 || ldw % 8 || (mu && ldmu % 8))
    return fail(CDX_EUNSUPPORTED, "%s: leading dimensions must be multiples of 8", name);
  if (M == 0) return CDX_OK;
  if (!x || !w || !out || (mu && !w_mu)) return fail(CDX_EINVAL, "%s: null pointer", name);
  if (!aligned16(x) || !aligned16(w) || !aligned16(out) || (mu && (!aligned16(mu) || !aligned16(w_mu))))
    return fail(CDX_EUNSUPPORTED, "%s: pointers must be 16-byte aligned", name);
  GemmParams p{};
  p.a = x;
  p.lda = ldx;
  p.a2 = mu;
  p.lda2 = ldmu;
  p.k_split = H;
  p.perm = nullptr;
  p.offsets = nullptr;
  p.E = 1;
  p.M = M;
  p.b = w;
  p.b2 = w_mu;
  p.ldb = ldw;
  p.b_estride = 0;
  p.N = N;
  p.K = (int32_t)K;
  p.c = out;
  p.ldc = ldo;
  if (cdiv(M, kBM) > INT32_MAX) return fail(CDX_EUNSUPPORTED, "%s: M too large", name);
  p.mt_count = (int32_t)cdiv(M, kBM);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (mu) return launch<ALoad::kConcat, Epi::kStore>(p, s, name);
  return launch<ALoad::kDense, Epi::kStore>(p, s, name);
}

namespace cdx {
namespace {

// Both MoE passes; with `residual`, the down pass adds its rows to `out` in place.
int moe_swiglu(const uint16_t* x, int64_t T, int32_t H, int32_t Ie, int32_t E, int32_t has_shared,
               const int32_t* perm, const int32_t* offsets, const uint16_t* w_gu, const uint16_t* w_down,
               uint16_t* inter, uint16_t* out, void* stream, bool residual, const char* name) {
  clear_error();
  if (T < 0 || T > INT32_MAX || H <= 0 || Ie <= 0 || E <= 0 || E > 64)
    return fail(CDX_EINVAL, "%s: bad shape T=%lld H=%d Ie=%d E=%d", name, (long long)T, H, Ie, E);
  if (H % 64 != 0) return fail(CDX_EUNSUPPORTED, "%s: H=%d must be a multiple of 64", name, H);
  if (T * (int64_t)H * 2 > (int64_t)UINT32_MAX)
    return fail(CDX_EUNSUPPORTED, "%s: x must fit 4 GB (T=%lld, H=%d)", name, (long long)T, H);
  if (T == 0) return CDX_OK;
  if (!x || !perm || !offsets || !w_gu || !w_down || !inter || !out)
    return fail(CDX_EINVAL, "%s: null pointer", name);
  if (!aligned16(x) || !aligned16(w_gu) || !aligned16(w_down) || !aligned16(inter) || !aligned16(out))
    return fail(CDX_EUNSUPPORTED, "%s: pointers must be 16-byte aligned", name);
  const int32_t P = (Ie + 63) / 64 * 64;
  const int32_t S = has_shared ? 2 : 1;
  const int32_t n_gu = 2 * S * P;
  const int32_t k_down = S * P;
  const int64_t blocks = (int64_t)E + (has_shared ? 1 : 0);
  // The kernels address each weight operand with 32-bit offsets from a tile base.
  if (blocks * 2 * P * (int64_t)H * 2 > (int64_t)UINT32_MAX)
    return fail(CDX_EUNSUPPORTED, "%s: the gate/up weights must fit 4 GB (E=%d, P=%d, H=%d)", name, E, P, H);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int32_t mt = (int32_t)(cdiv(T, kBM) + E);

  // Pass 1: gathered rows x[perm] times the gate/up rows of the shared block and the
  // token's expert block (w_gu [blocks][2][P][H]), SwiGLU epilogue; logical N rows
  // [0, S 2P) per expert (gu_tile).
  GemmParams p1{};
  p1.a = x;
  p1.lda = H;
  p1.k_split = H;
  p1.perm = perm;
  p1.offsets = offsets;
  p1.E = E;
  p1.M = T;
  p1.b = w_gu;
  p1.ldb = H;
  p1.b_estride = 0;
  p1.gu_P = P;
  p1.gu_shared = has_shared ? 1 : 0;
  p1.N = n_gu;
  p1.K = H;
  p1.c = inter;
  p1.ldc = k_down;
  p1.mt_count = mt;
  if (int rc = launch<ALoad::kGather, Epi::kSwiGLU>(p1, s, name)) return rc;

  // Pass 2: activations (sorted order) times [shared_down | down[e]], rows scattered back.
  // Two tile layouts.  Per-expert tiles (as in pass 1) leave up to one partial tile per
  // expert; tiles that ignore the expert boundaries (kSegmented) leave none, but a tile
  // that spans experts runs the expert columns once per expert.  The kernel holds one
  // block per CU, so price each in K steps per CU: whole rounds of tiles, plus one
  // spanning tile's extra expert columns for kSegmented.  At the 1B shape (8 experts,
  // 2048 columns) per-expert tiles take 2.2 rounds, i.e. 3 x 22 steps, the segmented
  // ones 2 x 22 + 11.
  const int64_t ks_shared = has_shared ? P / DefaultCfg::BK : 0, ks_expert = P / DefaultCfg::BK;
  const int64_t nt2 = cdiv(H, DefaultCfg::BN), cus = device_cu_count();
  const int64_t cost_expert = cdiv((cdiv(T, kBM) + E - 1) * nt2, cus) * (ks_shared + ks_expert);
  const int64_t cost_segmented = cdiv(cdiv(T, kBM) * nt2, cus) * (ks_shared + ks_expert) + ks_expert;
  const bool segmented = cost_segmented < cost_expert;
  // B: w_down [blocks][H][P]; the shared block (if any) serves K columns [0, P), the
  // token's expert block K columns [k_split, K).
  GemmParams p2{};
  p2.a = inter;
  p2.lda = k_down;
  p2.k_split = has_shared ? P : 0;
  p2.perm = perm;
  p2.offsets = offsets;
  p2.E = E;
  p2.M = T;
  p2.b = w_down + (has_shared ? (int64_t)H * P : 0);
  p2.b2 = has_shared ? w_down : nullptr;
  p2.ldb = P;
  p2.b_estride = (int64_t)H * P;
  p2.N = H;
  p2.K = k_down;
  p2.c = out;
  p2.ldc = H;
  if (segmented) {
    p2.mt_count = (int32_t)cdiv(T, kBM);
    if (residual) return launch<ALoad::kSegmented, Epi::kScatterAdd>(p2, s, name);
    return launch<ALoad::kSegmented, Epi::kScatter>(p2, s, name);
  }
  p2.mt_count = mt;
  if (residual) return launch<ALoad::kDense, Epi::kScatterAdd>(p2, s, name);
  return launch<ALoad::kDense, Epi::kScatter>(p2, s, name);
}

}  // namespace
}  // namespace cdx

extern "C" int cdx_moe_swiglu_fwd(const uint16_t* x, int64_t T, int32_t H, int32_t Ie, int32_t E,
                                  int32_t has_shared, const int32_t* perm, const int32_t* offsets,
                                  const uint16_t* w_gu, const uint16_t* w_down, uint16_t* inter,
                                  uint16_t* out, void* stream) {
  return cdx::moe_swiglu(x, T, H, Ie, E, has_shared, perm, offsets, w_gu, w_down, inter, out, stream, false,
                         "cdx_moe_swiglu_fwd");
}

extern "C" int cdx_moe_swiglu_residual_fwd(const uint16_t* x, int64_t T, int32_t H, int32_t Ie, int32_t E,
                                           int32_t has_shared, const int32_t* perm, const int32_t* offsets,
                                           const uint16_t* w_gu, const uint16_t* w_down, uint16_t* inter,
                                           uint16_t* residual, void* stream) {
  return cdx::moe_swiglu(x, T, H, Ie, E, has_shared, perm, offsets, w_gu, w_down, inter, residual, stream, true,
                         "cdx_moe_swiglu_residual_fwd");
}

extern "C" int cdx_grouped_gemm_fwd(const uint16_t* a, int64_t T, int32_t K, int32_t N, int32_t E,
                                    const int32_t* offsets, const uint16_t* w, uint16_t* out,
                                    void* stream) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_grouped_gemm_fwd";
  if (T < 0 || T > INT32_MAX || K <= 0 || N <= 0 || E <= 0 || E > 64)
    return fail(CDX_EINVAL, "%s: bad shape T=%lld K=%d N=%d E=%d", name, (long long)T, K, N, E);
  if (K % 64 != 0) return fail(CDX_EUNSUPPORTED, "%s: K=%d must be a multiple of 64", name, K);
  if (N % 8 != 0) return fail(CDX_EUNSUPPORTED, "%s: N=%d must be a multiple of 8", name, N);
  if (T == 0) return CDX_OK;
  if (!a || !offsets || !w || !out) return fail(CDX_EINVAL, "%s: null pointer", name);
  if (!aligned16(a) || !aligned16(w) || !aligned16(out))
    return fail(CDX_EUNSUPPORTED, "%s: pointers must be 16-byte aligned", name);
  GemmParams p{};
  p.a = a;
  p.lda = K;
  p.k_split = K;
  p.offsets = offsets;
  p.E = E;
  p.M = T;
  p.b = w;
  p.ldb = K;
  p.b_estride = (int64_t)N * K;
  p.N = N;
  p.K = K;
  p.c = out;
  p.ldc = N;
  p.mt_count = (int32_t)(cdiv(T, kBM) + E);
  return launch<ALoad::kDense, Epi::kStore>(p, reinterpret_cast<hipStream_t>(stream), name);
}

namespace cdx {
namespace {

// The mu-QKV + QK-norm + RoPE launch shared by both entry points.  A = [x | a2] and
// B = [w | b2] switch source at K column H; K_total columns in all (2H for a per-token
// mu, H + 64 for the folded broadcast row, H without a mu term: a2 == NULL).
int mu_qkv_rope(const char* name, const uint16_t* x, int64_t ldx, const uint16_t* a2, int64_t lda2,
                const uint16_t* w, const uint16_t* b2, int64_t ldw, int64_t B, int64_t S, int32_t H, int64_t K,
                int32_t nq, int32_t nkv, int32_t hd, const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                float eps, const float* cos_sin, int64_t n_pos, int64_t pos0, uint16_t* q_out,
                uint16_t* k_out, uint16_t* v_out, int64_t vt_ld, void* stream) {
  const int64_t M = B * S;
  const int64_t N = (int64_t)(nq + 2 * nkv) * hd;
  GemmParams p{};
  p.a = x;
  p.lda = ldx;
  p.a2 = a2;
  p.lda2 = lda2;
  p.k_split = H;
  p.E = 1;
  p.M = M;
  p.b = w;
  p.b2 = b2;
  p.ldb = ldw;
  p.N = (int32_t)N;
  p.K = (int32_t)K;
  p.qk.S = S;
  p.qk.nq = nq;
  p.qk.nkv = nkv;
  p.qk.q_norm_w = q_norm_w;
  p.qk.k_norm_w = k_norm_w;
  p.qk.eps = eps;
  p.qk.cos_sin = cos_sin;
  p.qk.pos0 = pos0;
  p.qk.q_out = q_out;
  p.qk.k_out = k_out;
  p.qk.v_out = v_out;
  p.qk.vt_ld = vt_ld;
  if (cdiv(M, kBM) > INT32_MAX) return fail(CDX_EUNSUPPORTED, "%s: M too large", name);
  p.mt_count = (int32_t)cdiv(M, kBM);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool concat = a2 != nullptr;
  switch (hd) {
    case 32:
      return concat ? launch<ALoad::kConcat, Epi::kQKRope, DefaultCfg, 32>(p, st, name)
                    : launch<ALoad::kDense, Epi::kQKRope, DefaultCfg, 32>(p, st, name);
    case 64:
      return concat ? launch<ALoad::kConcat, Epi::kQKRope, DefaultCfg, 64>(p, st, name)
                    : launch<ALoad::kDense, Epi::kQKRope, DefaultCfg, 64>(p, st, name);
    default:
      return concat ? launch<ALoad::kConcat, Epi::kQKRope, DefaultCfg, 128>(p, st, name)
                    : launch<ALoad::kDense, Epi::kQKRope, DefaultCfg, 128>(p, st, name);
  }
}

// Checks shared by both entry points (mu NULL: no mu term; ldmu 0: one broadcast row).
int check_rope_args(const char* name, const uint16_t* x, int64_t ldx, const uint16_t* mu, int64_t ldmu,
                    const uint16_t* w, const uint16_t* w_mu, int64_t ldw,
                    int64_t B, int64_t S, int32_t H, int32_t nq, int32_t nkv, int32_t hd,
                    const uint16_t* q_norm_w, const uint16_t* k_norm_w, float eps, const float* cos_sin,
                    int64_t n_pos, int64_t pos0, uint16_t* q_out, uint16_t* k_out, uint16_t* v_out,
                    int64_t vt_ld) {
  if (B < 0 || S < 0 || H <= 0 || nq <= 0 || nkv <= 0 || pos0 < 0 || n_pos < 0)
    return fail(CDX_EINVAL, "%s: bad shape B=%lld S=%lld H=%d nq=%d nkv=%d", name, (long long)B, (long long)S,
                H, nq, nkv);
  if (hd != 32 && hd != 64 && hd != 128)
    return fail(CDX_EUNSUPPORTED, "%s: head dim %d must be 32, 64 or 128", name, hd);
  if (H % 64 != 0) return fail(CDX_EUNSUPPORTED, "%s: H=%d must be a multiple of 64", name, H);
  if ((q_norm_w == nullptr) != (k_norm_w == nullptr))
    return fail(CDX_EINVAL, "%s: q and k norm weights must both be given or both be NULL", name);
  if (!(eps >= 0.f)) return fail(CDX_EINVAL, "%s: eps must be >= 0", name);
  if ((int64_t)(nq + 2 * nkv) * hd > INT32_MAX) return fail(CDX_EUNSUPPORTED, "%s: too many heads", name);
  if (S > INT32_MAX - 256) return fail(CDX_EUNSUPPORTED, "%s: S=%lld too long", name, (long long)S);
  if (ldx < H || ldw < H || (mu && ldmu != 0 && ldmu < H))
    return fail(CDX_EINVAL, "%s: leading dimension too small", name);
  if (ldx % 8 || ldw % 8 || (mu && ldmu % 8))
    return fail(CDX_EUNSUPPORTED, "%s: leading dimensions must be multiples of 8", name);
  if (vt_ld < 0 || (vt_ld > 0 && (vt_ld < S || vt_ld % 64 != 0)))
    return fail(CDX_EINVAL, "%s: vt_ld=%lld must be 0 or a multiple of 64 that is >= S", name, (long long)vt_ld);
  if (B * S == 0) return CDX_OK;
  if (pos0 + S > n_pos)
    return fail(CDX_EINVAL, "%s: cos/sin table has %lld positions, needs %lld", name, (long long)n_pos,
                (long long)(pos0 + S));
  if (!x || !w || !cos_sin || !q_out || !k_out || !v_out || (mu && !w_mu))
    return fail(CDX_EINVAL, "%s: null pointer", name);
  if (!aligned16(x) || !aligned16(w) || !aligned16(cos_sin) || !aligned16(q_out) || !aligned16(k_out) ||
      !aligned16(v_out) || (mu && (!aligned16(mu) || !aligned16(w_mu))) ||
      (q_norm_w && (!aligned16(q_norm_w) || !aligned16(k_norm_w))))
    return fail(CDX_EUNSUPPORTED, "%s: pointers must be 16-byte aligned", name);
  return CDX_OK;
}

// A broadcast mu row (layer 0's mu_init.expand) has one product with W_mu for every
// token: bias[n] = sum_k mu[k] W_mu[n, k].  This kernel computes it in fp32 (one wave
// per row n) and writes it as a 64-column K block for the projection: row n of `fold`
// (row stride ldw, the projection's B stride) gets (hi, lo, 0, ..., 0) with
// hi = bf16(bias[n]) and lo = bf16(bias[n] - hi), and `unit` (the A row, broadcast)
// gets (1, 1, 0, ..., 0).  The MFMA adds hi + lo exactly in fp32, which carries the
// bias to about 2^-17 of its size, so the projection needs one K step for the mu
// term instead of H / 64.  (A bias that is not finite keeps lo = 0, so that
// hi + lo is the bias itself.)
__global__ __launch_bounds__(256) void mu_fold_kernel(const uint16_t* __restrict__ mu,
                                                      const uint16_t* __restrict__ w, int64_t ldw, int32_t H,
                                                      int32_t N, uint16_t* __restrict__ fold,
                                                      uint16_t* __restrict__ unit) {
  const int lane = threadIdx.x & 63;
  if (blockIdx.x == 0 && threadIdx.x < 8)
    *reinterpret_cast<uint4*>(unit + threadIdx.x * 8) =
        threadIdx.x == 0 ? make_uint4(0x3F803F80u, 0u, 0u, 0u) : make_uint4(0u, 0u, 0u, 0u);
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const uint16_t* row = w + (int64_t)n * ldw;
  float acc = 0.f;
  for (int k = lane * 8; k < H; k += 64 * 8) {
    float a[8], b[8];
    unpack8(*reinterpret_cast<const uint4*>(row + k), a);
    unpack8(*reinterpret_cast<const uint4*>(mu + k), b);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = __builtin_fmaf(a[i], b[i], acc);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane < 8) {
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (lane == 0) {
      const uint16_t hi = f32_to_bf16_bits(acc);
      const float rest = acc - bf16_bits_to_f32(hi);
      const uint16_t lo = __builtin_isfinite(rest) ? f32_to_bf16_bits(rest) : (uint16_t)0;
      v.x = (uint32_t)hi | ((uint32_t)lo << 16);
    }
    *reinterpret_cast<uint4*>(fold + (int64_t)n * ldw + lane * 8) = v;
  }
}

}  // namespace
}  // namespace cdx

extern "C" int cdx_mu_qkv_rope_fwd(const uint16_t* x, int64_t ldx, const uint16_t* mu, int64_t ldmu,
                                   const uint16_t* w, const uint16_t* w_mu, int64_t ldw, int64_t B, int64_t S,
                                   int32_t H,
                                   int32_t nq, int32_t nkv, int32_t hd, const uint16_t* q_norm_w,
                                   const uint16_t* k_norm_w, float eps, const float* cos_sin,
                                   int64_t n_pos, int64_t pos0, uint16_t* q_out, uint16_t* k_out,
                                   uint16_t* v_out, int64_t vt_ld, void* stream) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_mu_qkv_rope_fwd";
  const int rc = check_rope_args(name, x, ldx, mu, ldmu, w, w_mu, ldw, B, S, H, nq, nkv, hd, q_norm_w, k_norm_w,
                                 eps, cos_sin, n_pos, pos0, q_out, k_out, v_out, vt_ld);
  if (rc != CDX_OK || B * S == 0) return rc;
  const int64_t K = mu ? 2 * (int64_t)H : (int64_t)H;
  return mu_qkv_rope(name, x, ldx, mu, ldmu, w, mu ? w_mu : nullptr, ldw, B, S, H, K, nq, nkv, hd, q_norm_w,
                     k_norm_w, eps, cos_sin, n_pos, pos0, q_out, k_out, v_out, vt_ld, stream);
}

extern "C" int cdx_mu_qkv_rope_bcast_fwd(const uint16_t* x, int64_t ldx, const uint16_t* mu_row,
                                         const uint16_t* w, const uint16_t* w_mu, int64_t ldw, int64_t B,
                                         int64_t S, int32_t H, int32_t nq, int32_t nkv, int32_t hd,
                                         const uint16_t* q_norm_w, const uint16_t* k_norm_w, float eps,
                                         const float* cos_sin, int64_t n_pos, int64_t pos0, uint16_t* q_out,
                                         uint16_t* k_out, uint16_t* v_out, int64_t vt_ld, uint16_t* work,
                                         void* stream) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_mu_qkv_rope_bcast_fwd";
  if (!mu_row) return fail(CDX_EINVAL, "%s: null pointer", name);
  int rc = check_rope_args(name, x, ldx, mu_row, 0, w, w_mu, ldw, B, S, H, nq, nkv, hd, q_norm_w, k_norm_w, eps,
                           cos_sin, n_pos, pos0, q_out, k_out, v_out, vt_ld);
  if (rc != CDX_OK || B * S == 0) return rc;
  if (!work) return fail(CDX_EINVAL, "%s: null pointer", name);
  if (!aligned16(work)) return fail(CDX_EUNSUPPORTED, "%s: pointers must be 16-byte aligned", name);
  const int32_t N = (nq + 2 * nkv) * hd;
  // work: the fold block, N rows of stride ldw (64 columns of each written), then the
  // 64-value unit row.
  uint16_t* fold = work;
  uint16_t* unit = work + (int64_t)N * ldw;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  mu_fold_kernel<<<dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st>>>(mu_row, w_mu, ldw, H, N, fold, unit);
  rc = check_launch(name);
  if (rc != CDX_OK) return rc;
  return mu_qkv_rope(name, x, ldx, unit, 0, w, fold, ldw, B, S, H, (int64_t)H + 64, nq, nkv, hd, q_norm_w,
                     k_norm_w, eps, cos_sin, n_pos, pos0, q_out, k_out, v_out, vt_ld, stream);
}

extern "C" int cdx_mu_guidance_fwd(const uint16_t* h, int64_t T, int32_t H, const uint16_t* w,
                                   const uint16_t* mu, float mu_lo, float mu_hi, float lo, float hi, uint16_t* out,
                                   int64_t ldo, void* stream) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_mu_guidance_fwd";
  if (T < 0 || H <= 0) return fail(CDX_EINVAL, "%s: bad shape T=%lld H=%d", name, (long long)T, H);
  if (H % 64 != 0) return fail(CDX_EUNSUPPORTED, "%s: H=%d must be a multiple of 64", name, H);
  if (!(lo <= hi) || !(mu_lo <= mu_hi)) return fail(CDX_EINVAL, "%s: clamp ranges must satisfy lo <= hi", name);
  if (ldo < H) return fail(CDX_EINVAL, "%s: ldo=%lld is smaller than H=%d", name, (long long)ldo, H);
  if (ldo % 8 != 0) return fail(CDX_EUNSUPPORTED, "%s: ldo=%lld must be a multiple of 8", name, (long long)ldo);
  if (T == 0) return CDX_OK;
  if (!h || !w || !mu || !out) return fail(CDX_EINVAL, "%s: null pointer", name);
  if (!aligned16(h) || !aligned16(w) || !aligned16(mu) || !aligned16(out))
    return fail(CDX_EUNSUPPORTED, "%s: pointers must be 16-byte aligned", name);
  GemmParams p{};
  p.a = h;
  p.lda = H;
  p.k_split = H;
  p.E = 1;
  p.M = T;
  p.b = w;
  p.ldb = H;
  p.N = H;
  p.K = H;
  p.c = out;
  p.ldc = ldo;
  p.bias = mu;
  p.bias_lo = mu_lo;
  p.bias_hi = mu_hi;
  p.lo = lo;
  p.hi = hi;
  if (cdiv(T, kBM) > INT32_MAX) return fail(CDX_EUNSUPPORTED, "%s: T too large", name);
  p.mt_count = (int32_t)cdiv(T, kBM);
  return launch<ALoad::kDense, Epi::kBiasClamp>(p, reinterpret_cast<hipStream_t>(stream), name);
}

extern "C" int cdx_linear_fwd(const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t ldw, int64_t M, int32_t K,
                              int32_t N, uint16_t* out, int64_t ldo, void* stream) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_linear_fwd";
  if (M < 0 || K <= 0 || N <= 0) return fail(CDX_EINVAL, "%s: bad shape M=%lld K=%d N=%d", name, (long long)M, K, N);
  if (K % 64 != 0) return fail(CDX_EUNSUPPORTED, "%s: K=%d must be a multiple of 64", name, K);
  // Results are stored in 16-byte pieces: columns [N, round_up(N, 8)) of each output
  // row receive values of no meaning, so ldo must leave room for them.
  const int64_t n8 = ((int64_t)N + 7) / 8 * 8;
  if (ldx < K || ldw < K || ldo < n8)
    return fail(CDX_EINVAL, "%s: leading dimension too small (ldo must be >= round_up(N, 8) = %lld)", name,
                (long long)n8);
  if (ldx % 8 || ldw % 8 || ldo % 8)
    return fail(CDX_EUNSUPPORTED, "%s: leading dimensions must be multiples of 8", name);
  if (M == 0) return CDX_OK;
  if (!x || !w || !out) return fail(CDX_EINVAL, "%s: null pointer", name);
  if (!aligned16(x) || !aligned16(w) || !aligned16(out))
    return fail(CDX_EUNSUPPORTED, "%s: pointers must be 16-byte aligned", name);
  GemmParams p{};
  p.a = x;
  p.lda = ldx;
  p.k_split = K;
  p.E = 1;
  p.M = M;
  p.b = w;
  p.ldb = ldw;
  p.N = N;
  p.K = K;
  p.c = out;
  p.ldc = ldo;
  if (cdiv(M, kBM) > INT32_MAX) return fail(CDX_EUNSUPPORTED, "%s: M too large", name);
  p.mt_count = (int32_t)cdiv(M, kBM);
  return launch<ALoad::kDense, Epi::kStore>(p, reinterpret_cast<hipStream_t>(stream), name);
}

extern "C" int cdx_linear_residual_fwd(const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t ldw, int64_t M,
                                       int32_t K, int32_t N, uint16_t* residual, int64_t ldr, void* stream) {
  using namespace cdx;
  clear_error();
  const char* name = "cdx_linear_residual_fwd";
  if (M < 0 || K <= 0 || N <= 0) return fail(CDX_EINVAL, "%s: bad shape M=%lld K=%d N=%d", name, (long long)M, K, N);
  if (K % 64 != 0) return fail(CDX_EUNSUPPORTED, "%s: K=%d must be a multiple of 64", name, K);
  // The residual is read and written in whole 16-byte pieces.
  if (N % 8 != 0) return fail(CDX_EUNSUPPORTED, "%s: N=%d must be a multiple of 8", name, N);
  if (M > INT32_MAX) return fail(CDX_EUNSUPPORTED, "%s: M=%lld too large", name, (long long)M);
  if (ldx < K || ldw < K || ldr < N) return fail(CDX_EINVAL, "%s: leading dimension too small", name);
  if (ldx % 8 || ldw % 8 || ldr % 8)
    return fail(CDX_EUNSUPPORTED, "%s: leading dimensions must be multiples of 8", name);
  if (M == 0) return CDX_OK;
  if (!x || !w || !residual) return fail(CDX_EINVAL, "%s: null pointer", name);
  if (!aligned16(x) || !aligned16(w) || !aligned16(residual))
    return fail(CDX_EUNSUPPORTED, "%s: pointers must be 16-byte aligned", name);
  GemmParams p{};
  p.a = x;
  p.lda = ldx;
  p.k_split = 0;     // every K column from b (the residual-add kernels' B has no shared block)
  p.perm = nullptr;  // identity rows
  p.E = 1;
  p.M = M;
  p.b = w;
  p.ldb = ldw;
  p.N = N;
  p.K = K;
  p.c = residual;
  p.ldc = ldr;
  p.mt_count = (int32_t)cdiv(M, kBM);
  return launch<ALoad::kDense, Epi::kScatterAdd>(p, reinterpret_cast<hipStream_t>(stream), name);
}
