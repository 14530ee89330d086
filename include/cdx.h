/*
 * cdx.h — C-ABI of the MI355X (gfx950) kernel library for the complexity-deep hot path.
 *
 * The library (libcdx.so) holds hand-written HIP kernels for three pieces of the
 * reference's forward pass:
 *   1. token-ID-routed MoE: routing plan (lookup, histogram, scan, stable permute)
 *      and the grouped SwiGLU GEMM with the shared lexical expert folded in;
 *   2. the mu-guided QKV projection as one contraction over [x | mu_prev];
 *   3. residual add + RMSNorm.
 *
 * Conventions (all entry points):
 *   - Every pointer argument named *_dev is device memory owned by the caller.
 *     The library never allocates or frees device memory.
 *   - `stream` is a hipStream_t passed as void*; all work is enqueued on it and
 *     nothing synchronises the host.  NULL means the default stream.
 *   - bf16 tensors are passed as uint16_t* (raw IEEE bfloat16 bits).
 *   - Return value: 0 on success, a negative CDX_E* code otherwise.  The message
 *     for the last failure on the calling thread is returned by cdx_last_error().
 *     Arguments are validated on the host before any launch; an invalid call
 *     enqueues nothing.
 *   - Row-major, unit stride in the last dimension; leading dimensions (ld*) are
 *     in elements.  16-byte alignment is required for every bf16 base pointer and
 *     leading dimensions must be multiples of 8 elements.
 *
 * No entry point has a counterpart in the reference as native code: the reference
 * hot path is PyTorch/ATen (and unwired Triton).  Each declaration cites the Python
 * function whose behaviour it replaces.
 */
#ifndef CDX_H_
#define CDX_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------------- */
#define CDX_OK 0
#define CDX_EINVAL (-1)      /* bad argument: null pointer, negative size, ... */
#define CDX_EUNSUPPORTED (-2) /* shape or alignment outside what the kernels handle */
#define CDX_ELAUNCH (-3)     /* the HIP runtime rejected a launch */
#define CDX_EWORKSPACE (-4)  /* workspace too small */

/* Library version (major*10000 + minor*100 + patch). */
int cdx_version(void);

/* Message for the last failing call on this host thread ("" if none). */
const char* cdx_last_error(void);

/* ---- piece 3: residual add + RMSNorm ------------------------------------- */

/*
 * h   = x + residual                      (rounded to bf16, written to residual_out)
 * out = weight * h * rsqrt(mean(h^2) + eps)   (fp32 math, rounded once to bf16)
 *
 * residual == NULL  -> plain RMSNorm of x (residual_out must then be NULL).
 * residual_out may alias residual (in-place update) or x.
 * Shapes: x, residual, out, residual_out [T, H] contiguous; weight [H].
 * H must be a multiple of 8 and at most 8192.
 *
 * Replaces: core/normalization.py:29-32 (RMSNorm.forward), core/layer.py:174,183
 * (residual adds), cuda/fused_residual.py:333-399 (fused_residual_rmsnorm) and
 * cuda/fused_residual.py:478-533 (fused_add_rmsnorm_inplace).
 */
int cdx_add_rmsnorm_fwd(const uint16_t* x_dev, const uint16_t* residual_dev,
                        const uint16_t* weight_dev, float eps, int64_t T, int32_t H,
                        uint16_t* out_dev, uint16_t* residual_out_dev, void* stream);

/*
 * Plain RMSNorm (cdx_add_rmsnorm_fwd with residual == NULL) whose output rows sit at
 * a stride ldo >= H (a multiple of 8): out[t * ldo + c] for c < H; the columns past
 * H are not touched.  x [T, H] contiguous.  The model writes the next layer's
 * normalised x into the left half of a [T, 2H] buffer whose right half
 * cdx_mu_guidance_fwd fills with mu, so that the projection reads [x | mu] as one
 * operand.
 *
 * Replaces: core/normalization.py:29-32 (the block's input_layernorm, core/layer.py:166).
 */
int cdx_rmsnorm_ld_fwd(const uint16_t* x_dev, const uint16_t* weight_dev, float eps, int64_t T, int32_t H,
                       uint16_t* out_dev, int64_t ldo, void* stream);

/* ---- piece 1a: routing plan ------------------------------------------------ */

/* Bytes of workspace cdx_route_plan needs for T tokens and E experts: one int32 per
 * (token block, expert), with at most 256 blocks, so never more than 64 KB. */
size_t cdx_route_workspace_bytes(int64_t T, int32_t E);

/*
 * expert_id[t] = map[clamp(ids[t], 0, V-1)]        (map == NULL: expert_id[t] = ids[t])
 * counts[e]    = #{t : expert_id[t] == e}
 * offsets      = [0, counts[0], counts[0]+counts[1], ...]   (E+1 entries)
 * perm         = stable argsort of expert_id (sorted position -> token index)
 * inv_perm     = inverse of perm                  (token index -> sorted position)
 *
 * All outputs are int32 and bit-exact against a stable counting sort.  E <= 64.
 * Expert ids outside [0, E) (possible only through a corrupt map or map == NULL)
 * are clamped into range so that no access leaves its buffer.
 * T == 0 is valid (counts and offsets are zeroed).
 *
 * Replaces: core/token_routed_mlp.py:149-150 (lookup), :166-170 (mask dispatch),
 * cuda/triton_token_routed.py:37-61 (sort_tokens_by_expert: sort, bincount, cumsum).
 */
int cdx_route_plan(const int64_t* ids_dev, int64_t T, const int64_t* map_dev, int64_t V,
                   int32_t E, int32_t* expert_id_dev, int32_t* perm_dev,
                   int32_t* inv_perm_dev, int32_t* counts_dev, int32_t* offsets_dev,
                   void* workspace_dev, size_t workspace_bytes, void* stream);

/*
 * L routing plans over the same ids, plan y through its own map maps[y] (`maps` is a host array
 * of L device pointers, none NULL, all of V entries), in two launches for all of them.
 * Outputs gain a leading [L] axis: expert_id / perm / inv_perm [L][T], counts [L][E],
 * offsets [L][E+1]; row y is exactly cdx_route_plan(ids, T, maps[y], ...).  The
 * workspace holds one count table per plan (cdx_route_plans_workspace_bytes).
 * L * T must stay below 2^31.  L == 0 does nothing.
 *
 * Replaces: core/token_routed_mlp.py:149-150 called from each layer's MLP
 * (core/layer.py:180): every layer looks its tokens up in its own token_to_expert.
 */
size_t cdx_route_plans_workspace_bytes(int64_t T, int32_t E, int32_t L);
int cdx_route_plans(const int64_t* ids_dev, int64_t T, const int64_t* const* maps, int32_t L,
                    int64_t V, int32_t E, int32_t* expert_id_dev, int32_t* perm_dev,
                    int32_t* inv_perm_dev, int32_t* counts_dev, int32_t* offsets_dev,
                    void* workspace_dev, size_t workspace_bytes, void* stream);

/*
 * cdx_route_plan without a workspace argument and without any allocation: the
 * per-block count table lives in a library-owned device array of
 * cdx_route_noalloc_scratch_bytes() bytes (64 KB: 256 blocks x 64 experts of int32),
 * one per GPU, held until the process ends.  Outputs and limits as cdx_route_plan
 * (E <= 64, T <= 2^31 - 1); a plan whose table would not fit is rejected with
 * CDX_EWORKSPACE.  The array's device address is looked up on the first call on each
 * device, which must then be the current device.  All calls on one GPU share the
 * array: calls that overlap in time on one GPU (two streams, two host threads) race
 * and must be ordered by the caller; calls on one stream are ordered already.
 *
 * No counterpart in the reference: this entry point exists for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).
 */
size_t cdx_route_noalloc_scratch_bytes(void);
int cdx_route_plan_noalloc(const int64_t* ids_dev, int64_t T, const int64_t* map_dev, int64_t V,
                           int32_t E, int32_t* expert_id_dev, int32_t* perm_dev,
                           int32_t* inv_perm_dev, int32_t* counts_dev, int32_t* offsets_dev,
                           void* stream);

/*
 * Row gather / scatter by a permutation (rows of `row_bytes` bytes, any length and
 * alignment; rows that are 16-byte multiples at 16-byte aligned bases take the wide path):
 *   permute:    out[i]       = in[perm[i]]
 *   unpermute:  out[perm[i]] = in[i]
 * An entry of perm outside [0, T) moves nothing.  T <= 2^31 - 1.
 * Replaces: cuda/triton_token_routed.py:55 (tokens[sorted_indices]) and
 * :385-386 (output[sorted_indices] = sorted_output); core/token_routed_mlp.py:170,174.
 */
int cdx_permute_rows(const void* in_dev, const int32_t* perm_dev, int64_t T,
                     int64_t row_bytes, void* out_dev, void* stream);
int cdx_unpermute_rows(const void* in_dev, const int32_t* perm_dev, int64_t T,
                       int64_t row_bytes, void* out_dev, void* stream);

/* ---- piece 1b: token-routed SwiGLU MoE ------------------------------------ */

/*
 * Weight operands (bf16, K-contiguous), laid out so that the module's Parameters can
 * be views of them (strided slices, no copy):
 *   P   = round_up(Ie, 64)                  padded expert width
 *   S   = has_shared ? 2 : 1                number of SwiGLU blocks per token
 *   NB  = E + (has_shared ? 1 : 0)          weight blocks: the shared expert (if any)
 *                                           is block 0, routed expert e block NB-E+e
 *   w_gu   [NB][2][P][H]   w_gu[b][0][i] = gate weights of unit i (row i of the
 *                          nn.Linear weight, column i of gate_proj_w[e]),
 *                          w_gu[b][1][i] = the up weights of unit i.
 *   w_down [NB][H][P]      w_down[b][n][i] = weight from unit i to output feature n
 *                          (down_proj_w[e][i][n], the shared nn.Linear's [n][i]).
 *   Units i in [Ie, P) are padding and must be zero.  Each block is stored once.
 *   ((E + 1) * 2 * P * H * 2 bytes must stay below 4 GB.)
 *
 * Computes, for every token t with e = expert_id[t]:
 *   a_s = silu(x_t Wsg^T) * (x_t Wsu^T)          (if has_shared)
 *   a_r = silu(x_t Wg[e]) * (x_t Wu[e])
 *   out_t = a_s Wsd^T + a_r Wd[e]                 (one fp32 accumulation, one rounding)
 * `inter_dev` is a caller workspace of [T, S*P] bf16 holding the activations in
 * sorted (perm) order.  x and out are [T, H] in original token order.
 * perm/offsets come from cdx_route_plan (offsets is [E+1] int32 on the device).
 * H must be a multiple of 64.
 *
 * Replaces: core/token_routed_mlp.py:157-178 (shared expert, per-expert loop,
 * combine), cuda/triton_token_routed.py:339-388 (_cggr_forward),
 * cuda/persistent_cggr.py:479-530 (persistent_swiglu_cggr).
 */
int cdx_moe_swiglu_fwd(const uint16_t* x_dev, int64_t T, int32_t H, int32_t Ie, int32_t E,
                       int32_t has_shared, const int32_t* perm_dev,
                       const int32_t* offsets_dev, const uint16_t* w_gu_dev,
                       const uint16_t* w_down_dev, uint16_t* inter_dev, uint16_t* out_dev,
                       void* stream);

/*
 * cdx_moe_swiglu_fwd with the block's residual add fused into the down pass:
 *   residual[t, :] = residual[t, :] + (shared(x) + expert_{e(t)}(x))[t, :]
 * in place, the MLP rows rounded to bf16 and then added with one more bf16 rounding
 * (the same two roundings as the reference's bf16 `residual + hidden_states`).
 * Arguments as cdx_moe_swiglu_fwd, with residual_dev [T, H] in place of out_dev.
 * Replaces: core/layer.py:176-183 (residual = h; h = mlp(norm(h)); h = residual + h),
 * the MLP half of the block.
 */
int cdx_moe_swiglu_residual_fwd(const uint16_t* x_dev, int64_t T, int32_t H, int32_t Ie, int32_t E,
                                int32_t has_shared, const int32_t* perm_dev,
                                const int32_t* offsets_dev, const uint16_t* w_gu_dev,
                                const uint16_t* w_down_dev, uint16_t* inter_dev,
                                uint16_t* residual_dev, void* stream);

/*
 * Grouped GEMM over expert segments of an already sorted token matrix:
 *   out[offsets[e]:offsets[e+1], :] = a[offsets[e]:offsets[e+1], :] @ W[e]
 * with W given K-contiguous: w_dev is [E][N][K] (W[e] transposed).  K % 64 == 0.
 * Replaces: cuda/triton_token_routed.py:197-231 (cggr_grouped_gemm_triton) and
 * :64-86 (grouped_gemm_pytorch).
 */
int cdx_grouped_gemm_fwd(const uint16_t* a_dev, int64_t T, int32_t K, int32_t N, int32_t E,
                         const int32_t* offsets_dev, const uint16_t* w_dev,
                         uint16_t* out_dev, void* stream);

/*
 * Elementwise SwiGLU, out[i] = silu(gate[i]) * up[i], silu(g) = g / (1 + exp(-g)) in
 * fp32.  dtype: 0 bf16, 1 fp16, 2 fp32 (gate, up and out all of it).
 *   round_silu = 1: silu(gate) rounded to dtype, then multiplied by up and rounded
 *                   (the reference's fused_swiglu_triton, and F.silu(g) * u);
 *   round_silu = 0: silu(gate) * up in fp32, rounded once (fused_swiglu_simple).
 * Pointers 16-byte aligned; any n >= 0.
 *
 * Replaces: cuda/triton_token_routed.py:234-257 (fused_swiglu_triton) and
 * cuda/persistent_cggr.py:450-476 (fused_swiglu_simple).
 */
int cdx_swiglu_fwd(const void* gate_dev, const void* up_dev, int64_t n, int32_t dtype, int32_t round_silu,
                   void* out_dev, void* stream);

/* ---- piece 2: mu-guided QKV projection ------------------------------------- */

/*
 * out[M, N] = [x | mu] @ [w_x | w_mu]^T, one K = 2H contraction, fp32 accumulate.
 *   x      [M, H]  leading dim ldx
 *   mu     [M, H]  leading dim ldmu; ldmu == 0 broadcasts one row (layer 0's
 *                  mu_init.expand); mu == NULL means no mu term (K = H)
 *   w_x    [N, H]  rows = output features: the q_proj, k_proj, v_proj weights
 *                  stacked ([out, in], as nn.Linear stores them), leading dim ldw
 *   w_mu   [N, H]  the mu_to_q, mu_to_k, mu_to_v weights stacked, leading dim ldw;
 *                  ignored when mu == NULL.  The two may be separate buffers or the
 *                  two halves of one [N, 2H] pack (w_mu = w_x + H, ldw = 2H).
 *   out    [M, N]  leading dim ldo; q = cols [0, Nq*D), k, v follow.
 * H % 64 == 0.
 * When x and mu are the two halves of one [M, 2H] buffer and w_x and w_mu the two
 * halves of one [N, 2H] buffer, the same product is the call with mu == NULL, x = that
 * buffer (ldx = 2H), w_x = the weight buffer (ldw = 2H) and 2H in place of H: one
 * operand on each side, the same sums in the same order (bit-identical), and no
 * choice between two sources on every load (this holds for cdx_mu_qkv_rope_fwd too).
 *
 * Replaces: core/attention.py:120-131 (cat + three F.linear),
 * cuda/triton_mu_qkv.py:195-283 (fused_mu_qkv_projection).
 */
int cdx_mu_qkv_fwd(const uint16_t* x_dev, int64_t ldx, const uint16_t* mu_dev, int64_t ldmu,
                   const uint16_t* w_x_dev, const uint16_t* w_mu_dev, int64_t ldw, int64_t M, int32_t H,
                   int32_t N, uint16_t* out_dev, int64_t ldo, void* stream);

/*
 * mu-QKV projection with the attention prologue fused into its epilogue:
 *   [q | k | v] = [x | mu] @ w_pack^T              (as cdx_mu_qkv_fwd; N = (nq + 2 nkv) hd)
 *   q_h = RoPE(q_norm_w * q_h / rms(q_h))          per head, per token; likewise k
 *   v_h = v_h
 * and writes q, k, v head-major: q_out [B, nq, S, hd], k_out / v_out [B, nkv, S, hd]
 * (row m = b * S + s of x is token s of sequence b).  The packed projection never
 * reaches memory; the norm and rotation run in fp32 on the accumulators and each
 * output is rounded to bf16 once.
 *   rms(z)   = sqrt(mean(z^2) + eps) over the hd values of the head.
 *   RoPE     y[c] = z[c] cos(t_c) - z[c + hd/2] sin(t_c)   for c <  hd/2
 *            y[c] = z[c] cos(t_c) + z[c - hd/2] sin(t_c)   for c >= hd/2
 *            with (cos, sin)(t_c) = cos_sin[pos0 + s][c mod hd/2], fp32 pairs, a table of
 *            n_pos >= pos0 + S positions (pos0 = tokens already in the KV cache).
 * q_norm_w / k_norm_w ([hd] bf16) both NULL: no QK norm.  hd must be 32, 64 or 128
 * and H a multiple of 64.  mu / ldmu / w_x / w_mu / ldw as in cdx_mu_qkv_fwd.
 * vt_ld == 0: v_out is [B, nkv, S, hd].  vt_ld > 0 (a multiple of 64, >= S): v_out is
 * V transposed for cdx_attention_fwd, [B, nkv, hd, vt_ld], token s of a sequence at
 * column 16*(s/16) + 4*sigma((s/4)%4) + s%4 with sigma = (0 2 1 3); the columns of
 * positions >= S are not written (cdx_attention_fwd needs them finite: clear them).
 *
 * Replaces: core/attention.py:120-155 (cat + three F.linear, head split, q_norm /
 * k_norm, rotary tables and apply_rotary_pos_emb), core/rotary.py:57-86.
 */
int cdx_mu_qkv_rope_fwd(const uint16_t* x_dev, int64_t ldx, const uint16_t* mu_dev, int64_t ldmu,
                        const uint16_t* w_x_dev, const uint16_t* w_mu_dev, int64_t ldw, int64_t B, int64_t S,
                        int32_t H,
                        int32_t nq, int32_t nkv, int32_t hd, const uint16_t* q_norm_w_dev,
                        const uint16_t* k_norm_w_dev, float eps, const float* cos_sin_dev,
                        int64_t n_pos, int64_t pos0, uint16_t* q_out_dev, uint16_t* k_out_dev,
                        uint16_t* v_out_dev, int64_t vt_ld, void* stream);

/*
 * cdx_mu_qkv_rope_fwd for a mu operand that is one row broadcast to every token
 * (layer 0's mu_init.expand, i.e. ldmu == 0), with the mu term folded:
 *   bias[n] = sum_k mu_row[k] w_mu[n, k]      (fp32, once per call)
 *   [q | k | v] = x @ w_x^T + bias            (then QK-norm + RoPE as cdx_mu_qkv_rope_fwd)
 * The bias enters the contraction as one 64-column K block whose row n holds
 * (bf16(bias[n]), bf16(bias[n] - bf16(bias[n])), 0, ...), so the product runs
 * K = H + 64 instead of 2H; hi + lo carries the fp32 bias to about 2^-17 of its
 * size and everything else is rounded as in cdx_mu_qkv_rope_fwd.
 *   mu_row  [H] bf16;  w_x / w_mu / ldw and the other arguments as cdx_mu_qkv_rope_fwd.
 *   work    device scratch of N * ldw + 64 bf16 (N = (nq + 2 nkv) hd), 16-byte
 *           aligned: the fold block (64 columns of each row written) and its unit A
 *           row.  Written on every call; calls that share it on one stream are ordered.
 *
 * Replaces: core/attention.py:120-155 for layer 0, whose mu_prev is
 * models/modeling.py:182 (mu_init.expand(B, S, -1)).
 */
int cdx_mu_qkv_rope_bcast_fwd(const uint16_t* x_dev, int64_t ldx, const uint16_t* mu_row_dev,
                              const uint16_t* w_x_dev, const uint16_t* w_mu_dev, int64_t ldw, int64_t B,
                              int64_t S, int32_t H, int32_t nq, int32_t nkv, int32_t hd,
                              const uint16_t* q_norm_w_dev, const uint16_t* k_norm_w_dev, float eps,
                              const float* cos_sin_dev, int64_t n_pos, int64_t pos0, uint16_t* q_out_dev,
                              uint16_t* k_out_dev, uint16_t* v_out_dev, int64_t vt_ld, uint16_t* work_dev,
                              void* stream);

/*
 * mu guidance, the producer of the next layer's mu operand:
 *   out[t, n] = clamp(sum_k h[t, k] w[n, k] + clamp(mu[n], mu_lo, mu_hi), lo, hi)
 * h [T, H] bf16, w [H, H] bf16 (nn.Linear layout, [out, in]), mu [H] bf16 (the
 * MuGuidance parameter, read on every call), out [T, H] bf16 with rows at stride
 * ldo >= H (a multiple of 8; H for a contiguous output); fp32 accumulation, one
 * rounding.  (mu_lo, mu_hi) are the module's (mu_min, mu_max); the model passes
 * (lo, hi) = (-2, 2), its clamp of mu between layers, the module API (-inf, +inf).
 * H must be a multiple of 64.
 *
 * Replaces: core/layer.py:54-61 (MuGuidance.forward: clamp(mu) + mu_proj(h)) and
 * models/modeling.py:199-200 (mu_prev = clamp(mu, -2, 2)).
 */
int cdx_mu_guidance_fwd(const uint16_t* h_dev, int64_t T, int32_t H, const uint16_t* w_dev,
                        const uint16_t* mu_dev, float mu_lo, float mu_hi, float lo, float hi,
                        uint16_t* out_dev, int64_t ldo, void* stream);

/*
 * Causal GQA attention over the fused projection's outputs:
 *   out[b, s, h*hd : (h+1)*hd] = sum_{n <= s} softmax_n(scale * q[b,h,s] . k[b,g,n]) v[b,g,n]
 * with g = h / (nq / nkv) (query heads share key/value heads in groups), the causal
 * mask top-left aligned (key n visible to query s iff n <= s) and fp32 softmax.
 *   q   [B, nq, S, hd] bf16;  k [B, nkv, S, hd] bf16
 *   vt  V transposed, [B, nkv, hd, vt_ld] bf16, token n at column
 *       16*(n/16) + 4*sigma((n/4)%4) + n%4, sigma = (0 2 1 3); vt_ld a multiple of 64
 *       >= S; the columns of positions n >= S (masked keys) must hold finite values
 *   out [B, S, nq * hd] bf16 (heads merged, the layout o_proj consumes)
 * hd must be 32, 64 or 128 and nkv must divide nq.
 *
 * Replaces: core/attention.py:163-181 (repeat_interleave of K and V, SDPA with
 * is_causal=True, transpose + merge of the heads).
 */
int cdx_attention_fwd(const uint16_t* q_dev, const uint16_t* k_dev, const uint16_t* vt_dev, int64_t B,
                      int64_t S, int32_t nq, int32_t nkv, int32_t hd, int64_t vt_ld, float scale,
                      uint16_t* out_dev, void* stream);

/* ---- expert map (host) ---------------------------------------------------- */

/*
 * Host function (no device work): the token -> expert map of greedy bin-packing.
 * freq [V] float32 and map [V] int64 are host arrays.  Tokens are taken in
 * descending frequency (ties: lower token id first) and each is assigned to the
 * expert with the least accumulated load (ties: lowest expert index); loads are
 * accumulated in double.  NaN frequencies are rejected.  1 <= E <= 65536.
 *
 * Replaces: core/token_routed_mlp.py:87-116 (_build_token_mapping with
 * token_frequencies).
 */
int cdx_binpack_map(const float* freq, int64_t V, int32_t E, int64_t* map);

/* ---- the model's ends: embedding gather and the tied LM head --------------- */

/*
 * out[t, :] = table[ids[t], :] for t < T; table [V, H] bf16 (the embedding weight),
 * ids int64 on the device, out [T, H] bf16.  An id outside [0, V) yields a row of
 * bf16 quiet NaNs (0x7FC0), so that every output depending on it is NaN: nn.Embedding
 * raises there, which needs a host round trip.  H must be a multiple of 8 and <= 16384.
 *
 * Replaces: models/modeling.py:74,177 (nn.Embedding and its lookup).
 */
int cdx_embedding_fwd(const int64_t* ids_dev, int64_t T, const uint16_t* table_dev, int64_t V, int32_t H,
                      uint16_t* out_dev, void* stream);

/*
 * out[M, N] = x[M, K] @ w[N, K]^T, bf16 in and out, fp32 accumulation, one rounding:
 * nn.Linear without bias with its weight as stored ([out, in]).  The model calls it
 * for the tied LM head, w = the embedding table.  K % 64 == 0; any N >= 1, with
 * ldo >= round_up(N, 8): the columns [N, round_up(N, 8)) of every output row are
 * written with values of no meaning.  Leading dimensions multiples of 8, pointers
 * 16-byte aligned.
 *
 * Replaces: models/modeling.py:101-103,206 (lm_head, weight tied to embed_tokens).
 */
int cdx_linear_fwd(const uint16_t* x_dev, int64_t ldx, const uint16_t* w_dev, int64_t ldw, int64_t M, int32_t K,
                   int32_t N, uint16_t* out_dev, int64_t ldo, void* stream);

/*
 * residual[M, N] = bf16(residual + bf16(x[M, K] @ w[N, K]^T)), in place: a bias-free
 * nn.Linear whose bf16 output is added to the residual stream with the rounding of a
 * separate bf16 add: o_proj and the block's first residual add.  (ComplexityModel
 * keeps hipBLASLt's GEMM with beta = 1 there, which ran the 1B forward 0.8% faster.)
 * K % 64 == 0, N % 8 == 0, M <= INT32_MAX, leading dimensions multiples of 8,
 * pointers 16-byte aligned.
 *
 * Replaces: core/attention.py:71,181 (o_proj) with core/layer.py:174
 * (hidden_states = residual + hidden_states).
 */
int cdx_linear_residual_fwd(const uint16_t* x_dev, int64_t ldx, const uint16_t* w_dev, int64_t ldw, int64_t M,
                            int32_t K, int32_t N, uint16_t* residual_dev, int64_t ldr, void* stream);

/* ---- measurement ---------------------------------------------------------- */

/*
 * Streaming probe of the HBM ceilings the bandwidth-bound kernels are compared with:
 *   mode 0  read `bytes` of in_dev (out_dev: a 4-byte sink, almost never written)
 *   mode 1  write `bytes` to out_dev (in_dev ignored)
 *   mode 2  copy `bytes` from in_dev to out_dev
 * 16-byte non-temporal accesses; bytes a multiple of 16, pointers 16-byte aligned.
 *
 * No counterpart in the reference: it measures the hardware, for the benchmark.
 */
int cdx_hbm_probe(int32_t mode, const void* in_dev, void* out_dev, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CDX_H_ */
