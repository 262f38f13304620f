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

/* Bits of the device status word some kernels OR into (`dev_status`, nullable). */
enum { HSD_STATUS_BAD_EXPERT = 1 };

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
                     void* workspace, size_t workspace_bytes, void* stream);

/* Replaces hsd/mamba.py:47-56 `mamba_rollback(records, n_keep)` and the cache half of
 * model.py:348-356: the state after the first n_keep rows of the last verify is its
 * checkpoint slab, so the rollback is *cur = (*cur + n_keep) % nslab, on the device.
 * n_keep comes from *n_keep_dev when non-null (e.g. written by hsd_greedy_accept),
 * else from n_keep_host. n_keep == 0 keeps the state from before the verify. */
int hsd_mamba_select_row(int32_t* cur, const int32_t* n_keep_dev, int64_t n_keep_host,
                         int64_t nslab, void* stream);

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
