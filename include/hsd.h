/* libhsd -- the MI355X (gfx950) hot path of hsd as a C ABI.
 *
 * Every entry point takes raw device pointers, int64 sizes and a HIP stream passed as
 * `void*` (a hipStream_t; NULL = the default stream). The library never allocates and
 * never synchronises: every buffer, workspace included, is owned by the caller, and
 * launches are queued on the given stream. Return value: HSD_OK (0) or a negative
 * HSD_ERR_* code with a message in hsd_last_error() (per host thread).
 *
 * bf16 / f16 tensors are passed as uint16_t bit patterns. Layout names follow the
 * reference: the STOCK down projection is w [.., D, F/8] uint32 (8 nibbles of one
 * output row per word, low nibble first) with scales/biases [.., D, F/64] bf16; the
 * NEURON-MAJOR layout is pw [.., F, D/8] uint32 (row i = neuron i, word w packs
 * W[8w..8w+7, i]) with ps/pb [.., F/64, D] bf16.
 */
#ifndef HSD_H_
#define HSD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  HSD_OK = 0,
  HSD_ERR_ARG = -1,        /* null pointer or invalid argument */
  HSD_ERR_SHAPE = -2,      /* a size the kernels do not support */
  HSD_ERR_DTYPE = -3,      /* unsupported dtype tag */
  HSD_ERR_ALIGN = -4,      /* a pointer is not aligned as required */
  HSD_ERR_WORKSPACE = -5,  /* workspace missing or too small */
  HSD_ERR_LAUNCH = -6      /* the HIP runtime refused a launch */
};

enum { HSD_DT_BF16 = 0, HSD_DT_F16 = 1, HSD_DT_F32 = 2 };

/* hsd_linear: what x holds, the weight format, and what is written. */
enum { HSD_X_BF16 = 0, HSD_X_RMS = 1, HSD_X_GATED = 2, HSD_X_GATED_Z = 3 };
enum { HSD_W_Q4 = 0, HSD_W_BF16 = 1 };
enum { HSD_Y_BF16 = 0, HSD_Y_F32 = 1, HSD_Y_RESID = 2, HSD_Y_ARGMAX = 3 };

/* Bits of the device status word some kernels OR into (`dev_status`, nullable). */
enum { HSD_STATUS_BAD_EXPERT = 1, HSD_STATUS_BAD_STATE = 2, HSD_STATUS_BAD_TOKEN = 4 };

/* The sequence state of a generation (a device int32 array of HSD_SEQ_LEN entries), read
 * and advanced by the step kernels so that a decode or verify step replays as one graph:
 *   POS      tokens in the target's attention caches (the position of the next row)
 *   CUR      the Mamba ring index shared by every Mamba layer
 *   N        tokens emitted so far; TOK the last one (the next step's input)
 *   HEAD_POS rows in the MTP head's attention cache; HEAD_POS2 the chained call's row
 *   R        rows the head has not seen yet (the last verify's accepted count + 1)
 *   ACCEPT   the last verify's accepted drafts; ACC_SUM their sum; STEPS steps taken */
enum {
  HSD_SEQ_POS = 0, HSD_SEQ_CUR = 1, HSD_SEQ_N = 2, HSD_SEQ_TOK = 3, HSD_SEQ_HEAD_POS = 4,
  HSD_SEQ_R = 5, HSD_SEQ_HEAD_POS2 = 6, HSD_SEQ_ACCEPT = 7, HSD_SEQ_STEPS = 8, HSD_SEQ_ACC_SUM = 9,
  HSD_SEQ_LEN = 16
};

const char* hsd_last_error(void);
int hsd_abi_version(void);

/* ------------------------------------------------------------------ layout
 * Replaces hsd/layout.py:34-50 `nibble_transpose(w)`:
 * w [batch, rows, words] uint32 -> out [batch, 8*words, rows/8] uint32 with
 * out[b, c, wo] packing W[8*wo + n, c] at nibble n. Exact and self-inverse.
 * rows % 8 == 0. 16-byte aligned pointers are not required. */
int hsd_permute_nibbles(const uint32_t* w, uint32_t* out, int64_t batch, int64_t rows,
                        int64_t words, void* stream);

/* Replaces the scale/bias half of hsd/layout.py:72-73 (`mx.swapaxes(s, -1, -2)`):
 * in [batch, rows, cols] 16-bit -> out [batch, cols, rows], bit for bit. */
int hsd_transpose_u16(const uint16_t* in, uint16_t* out, int64_t batch, int64_t rows,
                      int64_t cols, void* stream);

/* ------------------------------------------------------------------ decode
 * Replaces hsd/decode.py:164-186 `sparse_down(h, sel, gains, pw, ps, pb, spw, sps,
 * spb, *, F, FS, D, topk, ...)` (kernels decode.py:37-144).
 *   h      [B, topk*F + FS] (h_dtype: bf16, f16 or f32), routed slots then the shared
 *          expert's FS neurons (model.py:123-129)
 *   sel    [B, topk] int32 routed expert ids; gains [B, topk+1] f32 (scores, then the
 *          shared expert's gain)
 *   pw [E, F, D/8] u32, ps/pb [E, F/64, D] bf16; spw [FS, D/8], sps/spb [FS/64, D]
 *   y      [B, D] (y_dtype)
 * Only rows whose activation is nonzero (+0/-0 dead, NaN live) and only 64-groups with
 * a live row are read. dense=1 reads every row (the dense-h control: bit-identical
 * result to dense=0 for finite data, every byte touched). live_masks (nullable,
 * [B, topk*F/64 + FS/64] uint64): bit j of entry g is the liveness of neuron 64g+j of
 * the slot (the canonical compaction). dev_status (nullable int32): ORed with
 * HSD_STATUS_BAD_EXPERT when an id is outside [0, E); such a slot contributes 0.
 * Requirements: D % 128 == 0, F % 64 == 0, FS % 64 == 0, 16-byte aligned ps/pb/sps/spb.
 * Per row of the batch the arithmetic does not depend on B (verify rows == single rows).
 * workspace: hsd_sparse_down_workspace_bytes() bytes, 256-byte aligned. */
size_t hsd_sparse_down_workspace_bytes(int64_t B, int64_t D, int64_t F, int64_t FS,
                                       int64_t topk);
int hsd_sparse_down_decode(const void* h, int h_dtype, const int32_t* sel, const float* gains,
                           const uint32_t* pw, const uint16_t* ps, const uint16_t* pb,
                           const uint32_t* spw, const uint16_t* sps, const uint16_t* spb,
                           void* y, int y_dtype, int64_t B, int64_t D, int64_t F, int64_t FS,
                           int64_t topk, int64_t E, int dense, uint64_t* live_masks,
                           int32_t* dev_status, void* workspace, size_t workspace_bytes,
                           void* stream);

/* Replaces hsd/model.py:136-139 after the front end: y = bf16(x + bf16(sparse_down(...)))
 * -- the MoE block's residual add fused into the partial sum. x, y [B, D] bf16 (y may be
 * x). Other arguments and requirements as hsd_sparse_down_decode. */
int hsd_sparse_down_residual(const void* h, int h_dtype, const int32_t* sel, const float* gains,
                             const uint32_t* pw, const uint16_t* ps, const uint16_t* pb,
                             const uint32_t* spw, const uint16_t* sps, const uint16_t* spb,
                             const uint16_t* x, uint16_t* y, int64_t B, int64_t D, int64_t F,
                             int64_t FS, int64_t topk, int64_t E, int dense, uint64_t* live_masks,
                             int32_t* dev_status, void* workspace, size_t workspace_bytes,
                             void* stream);

/* No counterpart in the reference. For callers that cannot allocate device memory (code
 * under HIP graph capture that must not call hipMalloc, tight serving loops, harnesses
 * that forbid allocation): hsd_sparse_down_decode without the workspace argument. The
 * partial sums live in a static 4 MiB device array inside libhsd (one per GPU, held
 * until the process ends; looked up with hipGetSymbolAddress on the first call on a
 * device, with that device current -- `stream` must belong to the current device).
 * Sizes whose partial sums exceed 4 MiB (hsd_sparse_down_workspace_bytes) are rejected
 * with HSD_ERR_SHAPE: B <= 12 rows at the Nemotron-3.5 MoE shape. Every element of the
 * array is written before it is read, so nothing is cleared between calls. Calls that
 * overlap on one GPU (distinct streams, or concurrent host threads) share the array and
 * race: serialise them. Same arguments, results and bit-for-bit output as
 * hsd_sparse_down_decode. */
int hsd_sparse_down_decode_noalloc(const void* h, int h_dtype, const int32_t* sel,
                                   const float* gains, const uint32_t* pw, const uint16_t* ps,
                                   const uint16_t* pb, const uint32_t* spw, const uint16_t* sps,
                                   const uint16_t* spb, void* y, int y_dtype, int64_t B, int64_t D,
                                   int64_t F, int64_t FS, int64_t topk, int64_t E, int dense,
                                   uint64_t* live_masks, int32_t* dev_status, void* stream);

/* ------------------------------------------------------------------ MoE front end
 * Replaces the MoE block's front end after the router, hsd/model.py:110-121: the routed
 * experts' up projection `gather_qmm(xn, fc1.weight, fc1.scales, fc1.biases,
 * rhs_indices=inds, transpose=True)`, the shared expert's `up_proj(xn)` and `relu2` =
 * square(relu(.)) (model.py:49-50), written in pack's hcat layout (model.py:123-129). The
 * router (`mix.gate`) is not part of it.
 *   x    [B, D] bf16 (the normed token), sel [B, topk] int32 expert ids
 *   w1 [E, F, D/8] u32, s1/b1 [E, F, D/64] bf16 (stock layout, rows = outputs);
 *   sw1 [FS, D/8], ss1/sb1 [FS, D/64] (the shared expert)
 *   hcat [B, topk*F + FS] bf16: square(relu(bf16(x W^T))) rounded to bf16, W = s q + b
 *   live_masks (nullable, [B, (topk*F + FS)/64] uint64): the canonical live masks of hcat
 *   (bit j of entry g: element 64g + j is nonzero; NaN live)
 *   dev_status (nullable int32): ORed with HSD_STATUS_BAD_EXPERT for an id outside
 *   [0, E); that slot's h is 0.
 * Requirements: D % 64 == 0, D <= 4096, F % 64 == 0, FS % 64 == 0, 16-byte aligned x, w1,
 * sw1 and the four scale/bias arrays. No workspace. */
int hsd_moe_up_relu2(const void* x, int x_dtype, const int32_t* sel, const uint32_t* w1,
                     const uint16_t* s1, const uint16_t* b1, const uint32_t* sw1,
                     const uint16_t* ss1, const uint16_t* sb1, void* hcat, int64_t B, int64_t D,
                     int64_t F, int64_t FS, int64_t topk, int64_t E, uint64_t* live_masks,
                     int32_t* dev_status, void* stream);

/* Replaces the MoE block's front end WITH the router, hsd/model.py:110-121 from `mix.gate`
 * on (the gate of mlx-lm's NemotronH MoE, restated from the model family's published
 * gate): from the gate's logits [B, E] bf16 (hsd_linear of the normed token with the bf16
 * gate weight), score = sigmoid(logit) (fp32), choice = score + e_bias (nullable, [E] f32);
 * sel[b] = the topk largest choices, descending (equal choices: the smaller expert id);
 * gains[b] = score_k / (sum of the selected scores + 1e-20) * routed_scale (norm_topk),
 * else score_k * routed_scale, then 1.0 for the shared expert; then hcat as
 * hsd_moe_up_relu2. E <= 256, topk <= 8. sel [B, topk] int32 and gains [B, topk+1] f32 are
 * written for the down projection. */
int hsd_moe_route_up_relu2(const void* x, int x_dtype, const uint16_t* logits, const float* e_bias,
                           float routed_scale, int norm_topk, int32_t* sel, float* gains,
                           const uint32_t* w1, const uint16_t* s1, const uint16_t* b1,
                           const uint32_t* sw1, const uint16_t* ss1, const uint16_t* sb1, void* hcat,
                           int64_t B, int64_t D, int64_t F, int64_t FS, int64_t topk, int64_t E,
                           uint64_t* live_masks, void* stream);

/* The router half of hsd_moe_route_up_relu2 on its own: sel [B, topk] and gains
 * [B, topk+1] from the gate's logits, by the same rule (one workgroup per token row). */
int hsd_router_topk(const uint16_t* logits, const float* e_bias, float routed_scale, int norm_topk,
                    int32_t* sel, float* gains, int64_t B, int64_t E, int64_t topk, void* stream);

/* The dense 4-bit down projection on the STOCK layout -- the comparator that
 * mlx-lm's gather_qmm + quantized_matmul compute in dense mode (model.py:132-133;
 * test_layout_decode.py:145-151). w [E, D, F/8], s/b [E, D, F/64]; sw [D, FS/8],
 * ss/sb [D, FS/64]. Same h/sel/gains/y conventions as hsd_sparse_down_decode.
 * Requirements: F % 64 == 0, FS % 64 == 0, D % 4 == 0. No workspace. */
int hsd_dense_down_decode(const void* h, int h_dtype, const int32_t* sel, const float* gains,
                          const uint32_t* w, const uint16_t* s, const uint16_t* b,
                          const uint32_t* sw, const uint16_t* ss, const uint16_t* sb,
                          void* y, int y_dtype, int64_t B, int64_t D, int64_t F, int64_t FS,
                          int64_t topk, int64_t E, int32_t* dev_status, void* stream);

/* ------------------------------------------------------------------ dense projections
 * Replaces mlx `quantized_matmul(x, w, scales, biases, transpose=True, group_size=64,
 * bits=4)` -- the QuantizedLinear layers of the model (Mamba in_proj/out_proj at
 * hsd/mamba.py:26,44; the attention q/k/v/o projections and lm_head, model.py:226-230,
 * 287, 343) -- and the bf16 `x @ W.T` of the router gate (model.py:115) and of the MTP
 * head's eh_proj (mtp.py:83), for B <= 4 token rows: y[b, o] = sum_i xn[b, i] W[o, i].
 *   w_kind HSD_W_Q4: w [O, I/8] u32 (8 nibbles per word, low first), scales/biases
 *     [O, I/64] bf16, W = s q + b; HSD_W_BF16: w [O, I] bf16 (scales/biases unused).
 *   x_kind HSD_X_BF16: xn = x [B, I] bf16 (row stride x_ld);
 *          HSD_X_RMS:  xn = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * norm_w)
 *                      (mx.fast.rms_norm, the block pre-norm, model.py:114, mamba.py:25);
 *          HSD_X_GATED: x = y [B, I] f32, z = x * silu(gate) (gate bf16, stride gate_ld),
 *                      per group of 512: xn = bf16(bf16(z * rsqrt(mean(z^2) + eps)) * norm_w)
 *                      (the Mamba-2 gated RMSNorm, mamba.py:43);
 *          HSD_X_GATED_Z: the same norm from hsd_mamba_ssm_gated's rows: x [B, I + I/16] f32
 *                      holds z, then the sums of z^2 over every 16 channels (x_ld >= I + I/16);
 *                      a group's sum is its 32 partials added in order (gate unused).
 *   y_kind HSD_Y_BF16 / HSD_Y_F32: y [B, O] (stride y_ld);
 *          HSD_Y_RESID: y = bf16(res + bf16(x W^T)) (res bf16, stride res_ld; y may be res:
 *                      the residual add `x + mixer(x)` of every block);
 *          HSD_Y_ARGMAX: the per-workgroup best (value, index) of the bf16-rounded outputs
 *                      into argmax_keys [B, key_ld] (key_ld >= hsd_linear_argmax_slots),
 *                      for hsd_argmax_keys; y, when non-null, receives the bf16 outputs.
 *   xn_out (nullable): receives xn (bf16 [B, I], stride xn_ld).
 * Instantiated pairs (x_kind, y_kind): 4-bit -- (RMS, BF16), (RMS, F32), (RMS, ARGMAX),
 * (GATED, RESID), (GATED_Z, RESID), (BF16, RESID), (BF16, BF16); bf16 weights -- (RMS,
 * BF16), (BF16, BF16).
 * Requirements: O a multiple of 8 (4-bit) or 4 (bf16); I a multiple of 64 and at most 4096
 * (4-bit) or a multiple of 8 and at most 6144 (bf16), of 512 for the gated norm; x, gate, norm_w, w, xn_out 16-byte aligned with
 * row strides of whole 16-byte pieces. A token row's arithmetic does not depend on B. */
int64_t hsd_linear_argmax_slots(int64_t O, int w_kind);
int hsd_linear(const void* x, int64_t x_ld, int x_kind, const uint16_t* gate, int64_t gate_ld,
               const uint16_t* norm_w, float eps, const void* w, const uint16_t* scales,
               const uint16_t* biases, int w_kind, void* y, int64_t y_ld, int y_kind,
               const uint16_t* res, int64_t res_ld, uint16_t* xn_out, int64_t xn_ld,
               uint64_t* argmax_keys, int64_t key_ld, int64_t B, int64_t O, int64_t I,
               void* stream);

/* Replaces `mx.argmax(logits, axis=-1)` after lm_head (model.py:302, 419): tok[b] = the
 * index of the largest key of argmax_keys[b, :slots] written by hsd_linear's HSD_Y_ARGMAX
 * (the first index among equal bf16 values; NaN beats numbers). */
int hsd_argmax_keys(const uint64_t* argmax_keys, int64_t key_ld, int64_t slots, int64_t B,
                    int32_t* tok, void* stream);

/* ------------------------------------------------------------------ attention
 * Replaces the attention block's scaled_dot_product_attention over mlx-lm's KVCache for
 * decode (model.py:287) and verify steps (model.py:343, causal mask): B <= 4 rows at
 * positions P .. P+B-1, P = *pos (device; the cache length before the call).
 *   qkv [B, (HQ + 2 HKV) * HD] bf16 (row stride qkv_ld): q heads, then k, then v
 *   k_cache, v_cache [HKV, smax, HD] bf16: rows P .. P+B-1 are written from qkv; rows
 *   below P are read. A rollback is a smaller *pos (KVCache.trim, model.py:355).
 *   out [B, HQ * HD] bf16: softmax(scale q k^T over keys 0 .. P+r) v per query head;
 *   query head h reads kv head h / (HQ / HKV).
 * P + B > smax: the call writes zeros and sets HSD_STATUS_BAD_STATE. Requirements:
 * HD == 128, (HQ / HKV) % 4 == 0, smax % 32 == 0, smax <= 16384. A row's arithmetic does not depend on
 * B. workspace: hsd_attn_workspace_bytes(B, HQ, smax). */
size_t hsd_attn_workspace_bytes(int64_t B, int64_t HQ, int64_t smax);
int hsd_attn_decode(const uint16_t* qkv, int64_t qkv_ld, int64_t B, uint16_t* k_cache,
                    uint16_t* v_cache, int64_t smax, const int32_t* pos, uint16_t* out,
                    int64_t out_ld, int64_t HQ, int64_t HKV, int64_t HD, float scale,
                    int32_t* dev_status, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ step glue
 * Replaces the quantised embedding lookup (model.py:223-224, mlx QuantizedEmbedding):
 * out[b] = bf16(s q + b) of row tok[b] of w [V, D/8] u32, s/b [V, D/64] bf16. A token
 * outside [0, V) gives zeros and HSD_STATUS_BAD_TOKEN. */
int hsd_embed_q4(const int32_t* tok, int64_t B, const uint32_t* w, const uint16_t* scales,
                 const uint16_t* biases, int64_t V, int64_t D, uint16_t* out, int64_t out_ld,
                 int32_t* dev_status, void* stream);

/* Replaces the MTP head's input, hsd/mtp.py:81-83: out[b] = concat(rms_norm(e[b], we),
 * rms_norm(h[b], wh)) in bf16, [B, 2D]. */
int hsd_pair_norm(const uint16_t* e, int64_t e_ld, const uint16_t* h, int64_t h_ld,
                  const uint16_t* we, const uint16_t* wh, float eps, int64_t B, int64_t D,
                  uint16_t* out, int64_t out_ld, void* stream);

/* Replaces the loop body of hsd/model.py:314-321 after the step: the greedy token (the
 * argmax of hsd_linear's keys for the last row), out_tokens[N] = it (N < cap), and the
 * sequence state after one row: N, POS += 1, CUR = (CUR + 1) % nslab, TOK = the token. */
int hsd_decode_advance(const uint64_t* argmax_keys, int64_t slots, int32_t* seq, int32_t* out_tokens,
                       int64_t cap, int64_t nslab, void* stream);

/* Replaces hsd/model.py:419-427 on the device: tgt[r] = argmax of verify row r (keys
 * [k+1, key_ld]); a = first i < k with ids[1+i] != tgt[i], else k; the emitted tokens
 * ids[1:1+a] + [tgt[a]] go to out_tokens at N (up to cap) and to pend (nullable, the MTP
 * head's next token rows); then the rollback: POS and N += a+1, CUR = (CUR + a + 1) %
 * nslab (model.py:348-356 with the Mamba checkpoint ring), HEAD_POS += R, R = a+1
 * (mtp.trim, model.py:427), TOK = tgt[a]. tgt (nullable) receives the k+1 targets. */
int hsd_spec_accept(const uint64_t* argmax_keys, int64_t key_ld, int64_t slots, int64_t k,
                    const int32_t* ids, int32_t* seq, int32_t* out_tokens, int64_t cap, int64_t nslab,
                    int32_t* pend, int32_t* tgt, void* stream);

/* Replaces the chaining of hsd/model.py:408-414: from the MTP head's first call over 3
 * pending rows (R = seq[HSD_SEQ_R] valid), d1[0] = the argmax of row R-1, h2 = its normed
 * hidden row hn[R-1] (D bf16), and seq[HSD_SEQ_HEAD_POS2] = HEAD_POS + R (the cache row of
 * the chained call). key_ld = 0 and hn_ld = 0: the keys and hn hold that one row already
 * (hsd_seq_select_row before lm_head). */
int hsd_mtp_chain(const uint64_t* argmax_keys, int64_t key_ld, int64_t slots, const uint16_t* hn,
                  int64_t hn_ld, int64_t D, int32_t* seq, int32_t* d1, uint16_t* h2, void* stream);

/* The row of the MTP head's first call whose prediction is the first draft (model.py:408-411:
 * only the last confirmed row's argmax is used): dst [D] = src[R-1] (bf16, row stride src_ld;
 * R = seq[HSD_SEQ_R] clamped to [1, 3]), so that lm_head runs on one row. */
int hsd_seq_select_row(const uint16_t* src, int64_t src_ld, const int32_t* seq, uint16_t* dst, int64_t D,
                       void* stream);

/* The verify ids of hsd/model.py:416: ids = [TOK, d1[0], argmax(keys2)] for k = 2 drafts.
 * With `script` (the true continuation, indexed by N) and `accepts` (an accepted count
 * per step, indexed by STEPS), the drafts are forced: the true token for i < a_t and a
 * wrong one at i = a_t (scripted acceptance; the head's own drafts are not used). */
int hsd_draft_ids(const int32_t* d1, const uint64_t* argmax_keys2, int64_t slots, int64_t k,
                  int32_t* seq, const int32_t* script, int64_t script_len, const int32_t* accepts,
                  int64_t n_accepts, int64_t V, int32_t* ids, void* stream);

/* The MTP head's input in one launch (hsd_embed_q4 then hsd_pair_norm, the same bits):
 * out[b] = concat(rms_norm(embed(t_b), we), rms_norm(h[b], wh)), [B, 2D] bf16, t_b = tok[b]
 * (mtp.py:81-83 with the head's token embedding, model.py:223-224). With tok NULL (the
 * chained call of hsd/model.py:408-414, B = 1): t = the argmax of argmax_keys (slots keys,
 * hsd_linear's HSD_Y_ARGMAX for the selected row), d1[0] = t and seq[HSD_SEQ_HEAD_POS2] =
 * HEAD_POS + R as hsd_mtp_chain does, h being that row's normed hidden row. A token outside
 * [0, V) embeds as zeros and sets HSD_STATUS_BAD_TOKEN. D % 64 == 0. */
int hsd_head_input(const int32_t* tok, const uint64_t* argmax_keys, int64_t slots, const uint32_t* w,
                   const uint16_t* scales, const uint16_t* biases, int64_t V, const uint16_t* h,
                   int64_t h_ld, const uint16_t* we, const uint16_t* wh, float eps, int64_t B, int64_t D,
                   int32_t* seq, int32_t* d1, uint16_t* out, int64_t out_ld, int32_t* dev_status,
                   void* stream);

/* hsd_draft_ids and the embedding of the k + 1 verify rows in one launch (model.py:416 and
 * 223-224): ids as hsd_draft_ids, out[r] = hsd_embed_q4 of ids[r] (out 16-byte aligned,
 * out_ld % 8 == 0, D % 64 == 0). */
int hsd_verify_input(const int32_t* d1, const uint64_t* argmax_keys2, int64_t slots, int64_t k,
                     int32_t* seq, const int32_t* script, int64_t script_len, const int32_t* accepts,
                     int64_t n_accepts, int64_t V, const uint32_t* w, const uint16_t* scales,
                     const uint16_t* biases, int64_t D, int32_t* ids, uint16_t* out, int64_t out_ld,
                     int32_t* dev_status, void* stream);

/* dst[i] = src[clamp(POS + offset + i, 0, n-1)] for i < count: the next rows of a prompt
 * held on the device, so a prefill step (model.py:259-279, here in steps of a few rows)
 * replays as one graph. */
int hsd_gather_tokens(const int32_t* src, int64_t n, const int32_t* seq, int64_t offset, int64_t count,
                      int32_t* dst, void* stream);

/* The sequence state after a prefill step of B rows of a T-token prompt at POS (the
 * chunk loop of model.py:265-279 and the MTP head's prefill hook, model.py:385-391):
 * POS and CUR advance by min(B, T - POS); HEAD_POS by min(B, T - 1 - POS) (>= 0). */
int hsd_prefill_advance(int32_t* seq, int64_t T, int64_t B, int64_t nslab, void* stream);

/* Replaces NemotronModel.rollback (model.py:348-356) after a verify that advanced the
 * state by B rows: POS -= n_drop (KVCache.trim) and CUR -= n_drop mod nslab (the
 * checkpoint ring still holds the kept rows' state). n_drop = B - n_keep < nslab. */
int hsd_seq_rollback(int32_t* seq, int64_t n_drop, int64_t nslab, void* stream);

/* seq[idx] += delta on the stream (host-known adjustments, e.g. the head's prefill rows). */
int hsd_seq_add(int32_t* seq, int64_t idx, int64_t delta, void* stream);

/* ------------------------------------------------------------------ prefill
 * Replaces hsd/prefill.py:247-278 `build_tiles(sel, E, tt)`: slots t*topk+k stably
 * sorted by expert (ties by slot id), ceil(count/tt) tiles per expert, then
 * ceil(T/tt) shared tiles (expert E); fixed NT = T*topk/tt + E + ceil(T/tt), -1 pads.
 * tile_e [NT] int32, tile_slot [NT*tt] int32. workspace: hsd_prefill_tiles_workspace_bytes. */
int64_t hsd_prefill_num_tiles(int64_t T, int64_t topk, int64_t E, int64_t tt);
size_t hsd_prefill_tiles_workspace_bytes(int64_t T, int64_t topk, int64_t E);
int hsd_prefill_tiles(const int32_t* sel, int64_t T, int64_t topk, int64_t E, int64_t tt,
                      int32_t* tile_e, int32_t* tile_slot, int32_t* dev_status,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Replaces hsd/prefill.py:281-291 `build_union` (kernel prefill.py:48-93): per tile the
 * ascending columns live in any of its valid slots, -1 padded to umax; ucount = size.
 * h [T, topk*F + FS] (h_dtype, 16-byte aligned); ulist [NT, umax] int32;
 * ucount [NT] int32. umax >= FS; F, FS multiples of 8. */
int hsd_prefill_union(const void* h, int h_dtype, const int32_t* tile_e,
                      const int32_t* tile_slot, int32_t* ulist, int32_t* ucount, int64_t T,
                      int64_t F, int64_t FS, int64_t topk, int64_t E, int64_t tt, int64_t NT,
                      int64_t umax, void* stream);

/* Replaces hsd/prefill.py:294-321 `sparse_down_prefill` (gather kernel prefill.py:95-117,
 * GEMM kernel prefill.py:119-222, partial sum prefill.py:320): per tile a bf16 MFMA GEMM
 * over the tile's union rows (the union list given here decides which rows are read),
 * the affine dequantisation factored per 64-row group (exact bf16 128+q operands, fp32
 * accumulation, per-group scale and bias applied in fp32), the gain epilogue, then
 * y[t] = sum over the topk+1 partials in slot order. Routed slots whose sel entry is out
 * of range contribute nothing (their tiles never held them).
 * h [T, topk*F+FS] bf16 (16-byte aligned); sel [T, topk] int32; gains [T, topk+1] f32;
 * y [T, D] (y_dtype). Requirements: tt in {32, 64}, D % 128 == 0, F and FS multiples of
 * 64 and at most 4032. workspace: hsd_prefill_gemm_workspace_bytes() bytes. */
size_t hsd_prefill_gemm_workspace_bytes(int64_t T, int64_t D, int64_t F, int64_t FS,
                                        int64_t topk, int64_t E, int64_t tt);
int hsd_prefill_gemm(const uint16_t* h, const int32_t* sel, const float* gains,
                     const int32_t* tile_e, const int32_t* tile_slot, const int32_t* ulist,
                     const int32_t* ucount, const uint32_t* pw, const uint16_t* ps,
                     const uint16_t* pb, const uint32_t* spw, const uint16_t* sps,
                     const uint16_t* spb, void* y, int y_dtype, int64_t T, int64_t D, int64_t F,
                     int64_t FS, int64_t topk, int64_t E, int64_t tt, int64_t NT, int64_t umax,
                     void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ Mamba-2
 * Replaces the state update of hsd/mamba.py:19-44 `mamba_verify` (depthwise conv,
 * silu, mlx-lm `ssm_update` over L rows, gated RMSNorm) for L in 1..nslab-1 rows.
 * State lives in a ring of nslab slabs: ssm_slabs [nslab, H, P, N] f32 (16-byte aligned),
 * conv_slabs [nslab, K-1, CD] bf16 (K = 4); *cur (device int32) names the current slab.
 * Row r (0-based) reads the state after row r-1 and writes the state after row r to
 * slab (cur+1+r) % nslab -- the per-row checkpoints. *cur is not changed here.
 *   conv_in [L, CD] bf16 (row stride conv_in_ld), dt_raw [L, H] bf16 (stride dt_ld),
 *   gate [L, H*P] bf16 (stride gate_ld); conv_w [CD, K] bf16, conv_b [CD] bf16;
 *   A_log, dt_bias, Dp [H] f32; norm_w [H*P] bf16;
 *   y [L, H*P] (y_dtype): rmsnorm over groups of norm_group of y_ssm*silu(gate), times
 *   norm_w. CD = H*P + 2*G*N. Requirements: N == 128, P % 16 == 0, H % G == 0,
 *   (H*P) % norm_group == 0, norm_group % 256 == 0.
 * D is used rounded to bf16 (the reference passes m.D.astype(x.dtype), mamba.py:38).
 * A ring index outside [0, nslab) reads and writes no state, makes y NaN and sets
 * HSD_STATUS_BAD_STATE in dev_status (nullable).
 * A row's arithmetic does not depend on L: a verify of L rows is bit-identical to L
 * single-row calls. workspace: hsd_mamba_workspace_bytes(). */
size_t hsd_mamba_workspace_bytes(int64_t L, int64_t H, int64_t P);
int hsd_mamba_verify(const uint16_t* conv_in, int64_t conv_in_ld, const uint16_t* dt_raw,
                     int64_t dt_ld, const uint16_t* gate, int64_t gate_ld,
                     const uint16_t* conv_w, const uint16_t* conv_b, const float* A_log,
                     const float* dt_bias, const float* Dp, const uint16_t* norm_w,
                     float* ssm_slabs, uint16_t* conv_slabs, const int32_t* cur, int64_t nslab,
                     void* y, int y_dtype, int64_t L, int64_t H, int64_t P, int64_t N,
                     int64_t G, int64_t norm_group, float eps, float dt_lo, float dt_hi,
                     int32_t* dev_status, void* workspace, size_t workspace_bytes, void* stream);

/* The conv + SSM half of hsd_mamba_verify without the gated norm: y [L, H*P] f32 =
 * sum_n S C + D x per row, the per-row checkpoints written to the ring as above, for
 * hsd_linear's HSD_X_GATED prologue. (The model's Mamba block takes hsd_mamba_ssm_gated
 * and HSD_X_GATED_Z.) */
int hsd_mamba_ssm(const uint16_t* conv_in, int64_t conv_in_ld, const uint16_t* dt_raw, int64_t dt_ld,
                  const uint16_t* conv_w, const uint16_t* conv_b, const float* A_log,
                  const float* dt_bias, const float* Dp, float* ssm_slabs, uint16_t* conv_slabs,
                  const int32_t* cur, int64_t nslab, float* y, int64_t L, int64_t H, int64_t P,
                  int64_t N, int64_t G, float dt_lo, float dt_hi, int32_t* dev_status, void* stream);

/* hsd_mamba_ssm with the gate of the gated norm applied (the first half of mamba.py:43):
 * z [L, z_ld] f32 with z_ld >= H*P + H*P/16: columns 0 .. H*P-1 hold z = y * silu(gate)
 * (gate [L, H*P] bf16, stride gate_ld), column H*P + k the sum of z^2 over channels
 * 16k .. 16k+15 (in channel order), for hsd_linear's HSD_X_GATED_Z prologue (the model's
 * out_proj then does no silu and loads no gate). A ring index outside [0, nslab) makes
 * both NaN and sets HSD_STATUS_BAD_STATE. */
int hsd_mamba_ssm_gated(const uint16_t* conv_in, int64_t conv_in_ld, const uint16_t* dt_raw, int64_t dt_ld,
                        const uint16_t* gate, int64_t gate_ld, const uint16_t* conv_w, const uint16_t* conv_b,
                        const float* A_log, const float* dt_bias, const float* Dp, float* ssm_slabs,
                        uint16_t* conv_slabs, const int32_t* cur, int64_t nslab, float* z, int64_t z_ld,
                        int64_t L, int64_t H, int64_t P, int64_t N, int64_t G, float dt_lo, float dt_hi,
                        int32_t* dev_status, void* stream);

/* Replaces hsd/mamba.py:47-56 `mamba_rollback(records, n_keep)` and the cache half of
 * model.py:348-356: the state after the first n_keep rows of the last verify is its
 * checkpoint slab, so the rollback is *cur = (*cur + n_keep) % nslab, on the device.
 * n_keep comes from *n_keep_dev when non-null (e.g. written by hsd_greedy_accept),
 * else from n_keep_host. n_keep == 0 keeps the state from before the verify; n_keep
 * outside [0, L] (L = the rows of that verify) leaves cur unchanged and sets
 * HSD_STATUS_BAD_STATE in dev_status (nullable). */
int hsd_mamba_select_row(int32_t* cur, const int32_t* n_keep_dev, int64_t n_keep_host,
                         int64_t L, int64_t nslab, int32_t* dev_status, void* stream);

/* ------------------------------------------------------------------ acceptance
 * Replaces the greedy acceptance of hsd/model.py:419-427 on the device (no host
 * round trip): tgt[r] = first argmax of logits[r, :V] for r < k+1; a = the first i < k
 * with draft[i] != tgt[i], else k; tokens[:a+1] = draft[:a] + [tgt[a]], -1 after;
 * *n_accept = a; *n_keep = a + 1. When cur is non-null also applies the rollback:
 * *cur = (*cur + a + 1) % nslab. logits [k+1, V] (dtype), draft [k] int32. */
int hsd_greedy_accept(const void* logits, int dtype, int64_t k, int64_t V,
                      const int32_t* draft, int32_t* tgt, int32_t* tokens, int32_t* n_accept,
                      int32_t* n_keep, int32_t* cur, int64_t nslab, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HSD_H_ */
