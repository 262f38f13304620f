// The MoE front end after the router (hsd/model.py:110-121) in pack's layout
// (model.py:123-129): for token b the 4-bit up projection of each selected expert and of
// the shared expert, ReLU^2, written to hcat [B, topk*F + FS] (bf16), plus the canonical
// live mask of every 64-row group (the decode kernels' compaction input).
//
// k_moe_up (instanced for D <= 3072 and D <= 4096, see UpShape): one workgroup per (token,
// 16-row block of hcat): 4 wavefronts x 4 rows, so a
// 64-row mask group takes four workgroups (each writes its 16 bits of the group's mask).
//   1. one round trip: the token's x, the block's expert id (a scalar load), the 16 rows'
//      scales and biases (contiguous: 4 of each per thread, to LDS as the affine step's
//      factors (16 s, b - 16 s) per row and group), and the wave's
//      4 rows' 16-byte pieces (16 lanes per row, D/32 pieces per row dealt over them);
//   2. x goes to LDS as bf16 pairs (x[i], x[i+4]) in the order of a word's nibble pairs,
//      and the sum of x over every 32-input piece;
//   3. per piece: a shift, a mask and an OR with bf16 1.0 put each nibble in the top four
//      mantissa bits of a bf16, so a word becomes four bf16 pairs (1 + q_n/16,
//      1 + q_{n+4}/16) (exact); v_dot2_f32_bf16 accumulates x (1 + q/16) in fp32, and
//      u += 16 s * acc + (b - 16 s) * sum(x): the affine dequantisation W = s q + b folded
//      per piece. (An offset of 1 against q/16 <= 15/16 keeps the cancellation in
//      acc - sum(x) small: 128 + q, exact as well, lost about four more bits.)
//   4. the 16 lanes' partials of each row: a DPP sum inside the 16-lane row (a lane's
//      row never changes, so it keeps one partial and the x words it reads are those of
//      the other three rows' lanes); h = square(relu(bf16(u))) rounded to bf16.
// Bytes per token: every row of the 7 selected matrices (D/2 + 4 D/64 bytes per row),
// 22.45 MB at the reference shape: an HBM-bound batched GEMV.
#include "hsd_common.h"

namespace hsd {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kUpWaves = 4;
constexpr int kUpThreads = 64 * kUpWaves;
constexpr int kUpRows = 4;                      // rows per wavefront
constexpr int kUpBlk = kUpRows * kUpWaves;      // rows per workgroup (an eighth of a mask group)
constexpr int kUpMaxD = 4096;                   // inputs per token held in LDS (the larger instance)
constexpr int kUpSmallD = 3072;                 // the smaller instance (the reference shape's 2688)
static_assert((kUpBlk == 16 || kUpBlk == 8) && kUpBlk * (kUpMaxD / 64) / 4 <= kUpThreads,
              "a block is a quarter or an eighth of a mask group; 4 scales and biases per thread");
// Two instances by the largest D: the register arrays (x words, the lane's weight pieces)
// are sized for it, so D <= 3072 runs 8 wavefronts per SIMD (64 VGPRs) and the 4096
// instance 6. A single instance for D <= 4096 (96 VGPRs, 5 per SIMD) had made the
// MTP-2 step 2.221 against 2.196 ms for 72 VGPRs and 7 per SIMD; the x rows in LDS sit at
// a compile-time pitch (no per-piece address registers).
template <int MAXD> struct UpShape {
  static constexpr int kMaxP = MAXD / 32;
  static constexpr int kXIt = (MAXD / 8 + kUpThreads - 1) / kUpThreads;  // x words per thread
  // per SIMD: 8 for D <= 3072 (64 VGPRs, 2048 resident workgroups: 1.36 rounds at three
  // token rows), once the wavefront index and the routed expert id are scalars; with the
  // nibble mask in a register the routed instance had needed 65-68 VGPRs before that (7
  // wavefronts: MTP-2 step 1.854 / 1.846 against 1.860 / 1.863 ms for 8 with the
  // two-instruction decode).
  static constexpr int kWaves = MAXD <= kUpSmallD ? 8 : 6;
};
// 16-row workgroups (4 rows per wavefront): at three token rows 19.0 against 19.8 us per
// call for 8-row ones (fewer rounds of workgroups), at one row the same. Small workgroups
// measured faster than 64-row ones (1024 threads; 9.0 us per call with 8
// rows, 9.1 with 16, 10.1 with 64): a workgroup starts its arithmetic as soon as its own
// loads are in, and 1856 workgroups fill all CUs at the reference shape where 232 left 24
// idle.
constexpr uint32_t kBfOne2 = 0x3F803F80u;   // bf16 1.0 in both halves
constexpr uint32_t kNibHi = 0x00780078u;    // mantissa bits 3..6 of both halves

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                         false);
}

// The router's top-k (the gate of mlx-lm's NemotronH MoE, model.py:115; restated from the
// model family's published gate): score = sigmoid(logit) in fp32, choice = score + bias
// (a NaN choice ranks below every number); the topk largest choices in descending order
// (equal choices: the smaller expert id); gain_k = score_k / (sum of the selected scores +
// 1e-20) * scale (norm_topk), else score_k * scale. E <= 256.
// One wavefront ranks the experts: lane l holds experts l, l + 64, l + 128, l + 192 as keys
// (the choice's order-preserving bits << 32 | ~id, so a larger key is a larger choice, then
// a smaller id); topk rounds of a 64-lane maximum pick them in order. No LDS and no
// barrier, so a workgroup of the up projection can afford it in front of its weight loads.
struct Router {
  const uint16_t* logits;   // [B, E] bf16
  const float* bias;        // [E] f32 (nullable)
  int32_t* sel_out;         // [B, topk]
  float* gains_out;         // [B, topk + 1]
  float scale;
  int norm_topk;
};
constexpr int kMaxTopk = 8;
constexpr int kMaxE = 256;

__device__ __forceinline__ uint32_t ordered_bits(float c) {
  const uint32_t u = __float_as_uint(c);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Token row b's experts e[0..rounds) in rank order, and with rounds == topk the gains
// g[0..topk) (every lane gets them); every lane of one wavefront calls it. rounds < topk
// stops after the first rounds experts (the gains are then not the selection's).
__device__ __forceinline__ void route_topk_wave(const Router& rt, int b, int E, int topk, int rounds, int lane,
                                                int (&e_out)[kMaxTopk], float (&g_out)[kMaxTopk]) {
  uint64_t key[4];
  float sg[4];
  // every logit and bias load first, in one round trip: none under a branch (without a
  // bias the loads read the 4-byte word holding the logits' first element, and the value
  // is dropped), and the values pinned to registers after the last load is issued, so the
  // compiler cannot sink a load into the branch that uses it (a load under a branch ends
  // in a wait for every load where the paths merge: one round trip per key)
  uint32_t lg[4], bv[4];
  const bool has_bias = rt.bias != nullptr;
  const float* bp = has_bias ? rt.bias
                             : reinterpret_cast<const float*>(reinterpret_cast<uintptr_t>(rt.logits) & ~uintptr_t(3));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ec = min(lane + 64 * i, E - 1);
    lg[i] = rt.logits[(size_t)b * E + ec];
    bv[i] = __float_as_uint(bp[has_bias ? ec : 0]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lg[i] = opaque_vgpr(lg[i]);
    bv[i] = opaque_vgpr(bv[i]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    const float x = bf16_bits_to_f32(lg[i]);
    const float s = 1.0f / (1.0f + expf(-x));
    float c = s + (has_bias ? __uint_as_float(bv[i]) : 0.0f);
    c = c != c ? -INFINITY : c;
    key[i] = e < E ? ((uint64_t)ordered_bits(c) << 32) | (uint32_t)~(uint32_t)e : 0;
    sg[i] = s;
  }
  float ssum = 0.0f;
  float sc[kMaxTopk];
#pragma unroll
  for (int r = 0; r < kMaxTopk; ++r) {
    e_out[r] = 0;
    sc[r] = 0.0f;
    if (r < rounds) {                                  // uniform
      uint64_t m = key[0];
#pragma unroll
      for (int i = 1; i < 4; ++i) m = key[i] > m ? key[i] : m;
      m = wave_max_u64(m);
      const int e = __builtin_amdgcn_readfirstlane((int)~(uint32_t)m);  // the same in every lane
#pragma unroll
      for (int i = 0; i < 4; ++i) key[i] = key[i] == m ? 0 : key[i];
      const int ii = e >> 6;
      const float own = ii == 0 ? sg[0] : ii == 1 ? sg[1] : ii == 2 ? sg[2] : sg[3];
      const float s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(own), e & 63));
      e_out[r] = e;
      sc[r] = s;
      ssum += s;
    }
  }
#pragma unroll
  for (int r = 0; r < kMaxTopk; ++r)
    g_out[r] = rt.norm_topk ? sc[r] / (ssum + 1e-20f) * rt.scale : sc[r] * rt.scale;
}

template <bool ROUTE, int MAXD>
__global__ __launch_bounds__(kUpThreads)
__attribute__((amdgpu_waves_per_eu(UpShape<MAXD>::kWaves, UpShape<MAXD>::kWaves))) void k_moe_up(
    int D, int F, int FS, int topk, int E, const uint16_t* __restrict__ x, const int32_t* __restrict__ sel,
    const uint16_t* __restrict__ logits, const float* __restrict__ e_bias, const uint32_t* __restrict__ w1,
    const uint16_t* __restrict__ s1, const uint16_t* __restrict__ b1, const uint32_t* __restrict__ sw1,
    const uint16_t* __restrict__ ss1, const uint16_t* __restrict__ sb1, uint16_t* __restrict__ hcat,
    uint64_t* __restrict__ live_out, int32_t* __restrict__ status, Router rt_) {
  // the shape and the first round trip's pointers (x, the selection or the gate's logits
  // and bias) are the leading scalar arguments, which the dispatch preloads into SGPRs
  Router rt = rt_;
  rt.logits = logits;
  rt.bias = e_bias;
  // x pairs: piece j, word m, pair n at xp[4 (m kUpMaxP + j) + n] = (x[32 j + 8 m + n], x[.. + 4])
  // (a row of kUpMaxP pieces: the readers' addresses are a lane base plus constant offsets)
  constexpr int kUpMaxP = UpShape<MAXD>::kMaxP, kUpXIt = UpShape<MAXD>::kXIt;
  __shared__ __attribute__((aligned(16))) uint32_t xp[MAXD / 2];
  __shared__ float xh[kUpMaxP];  // sum of x over each 32-input piece
  __shared__ int nib[kUpWaves];
  // per (row, group) of the block: (16 s, b - 16 s), the factors of the affine step
  __shared__ __attribute__((aligned(16))) float2 sbt[kUpBlk * (MAXD / 64)];  // [row][group]
  const int b = blockIdx.y, blk = blockIdx.x;
  // the wavefront index as a scalar: the rows' addresses are then a scalar base plus the
  // lane's offset (8 wavefronts per SIMD fit 64 VGPRs only so)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int NR = topk * F + FS, NP = D / 32, NW = D / 8, NGD = D / 64;
  const int r0 = kUpBlk * blk;
  const bool routed = r0 < topk * F;
  const int k = routed ? r0 / F : topk;
  const int f0 = routed ? r0 - k * F : r0 - topk * F;

  // ---- round trip: x, the expert id, the rows' pieces and their scales (no load under a
  // branch: indices past the end are clamped and the values dropped); with the router,
  // the expert id is the top-k of the gate's logits, computed by every wavefront while x
  // is in flight
  uint4 xv[kUpXIt];
#pragma unroll
  for (int i = 0; i < kUpXIt; ++i)
    xv[i] = reinterpret_cast<const uint4*>(x + (size_t)b * D)[min(tid + kUpThreads * i, NW - 1)];
  int e;
  if constexpr (ROUTE) {
    // wavefront 0 ranks the experts (a routed block needs its id; block 0 writes the row's
    // selection and gains); the shared expert's blocks skip it
    __shared__ int tsel[kMaxTopk];
    if (routed) {
      if (wave == 0) {
        int es[kMaxTopk];
        float gs[kMaxTopk];
        // the block's own slot needs the first k + 1 experts; block 0 writes the whole
        // selection and the gains
        route_topk_wave(rt, b, E, topk, blk == 0 ? topk : k + 1, lane, es, gs);
        int ek = es[0];
        float gk = gs[0];
#pragma unroll
        for (int r = 1; r < kMaxTopk; ++r) {
          ek = lane == r ? es[r] : ek;
          gk = lane == r ? gs[r] : gk;
        }
        if (lane < topk) tsel[lane] = ek;
        if (blk == 0 && lane <= topk) {               // one writer per token row
          if (lane < topk) rt.sel_out[b * topk + lane] = ek;
          rt.gains_out[b * (topk + 1) + lane] = lane < topk ? gk : 1.0f;
        }
      }
      lds_barrier();
      e = __builtin_amdgcn_readfirstlane(tsel[k]);
    } else {
      e = 0;
    }
  } else {
    e = routed ? sel[b * topk + k] : 0;
  }
  const bool ok = !routed || (unsigned)e < (unsigned)E;
  const size_t row0 = routed ? (size_t)(ok ? e : 0) * F + f0 : (size_t)f0;
  const uint32_t* wb = routed ? w1 : sw1;
  const uint16_t* sb = routed ? s1 : ss1;
  const uint16_t* bb = routed ? b1 : sb1;
  // the block's scales and biases: kUpBlk NGD bf16 each, contiguous; thread t < nsc loads
  // entries 4t .. 4t+3 of both
  const int nsc = kUpBlk * NGD / 4;
  const int sc_i = min(tid, nsc - 1);
  const uint2 sv2 = reinterpret_cast<const uint2*>(sb + row0 * NGD)[sc_i];
  const uint2 bv2 = reinterpret_cast<const uint2*>(bb + row0 * NGD)[sc_i];
  // pieces: lanes 16 i .. 16 i + 15 take row i of the wave's 4, lane l its pieces
  // j = l % 16 + 16 it (it < NP / 16 rounded up)
  constexpr int kIt = (kUpMaxP + 15) / 16;
  const int rw = lane >> 4, jl = lane & 15, nit = (NP + 15) / 16;
  uint4 q[kIt];
  {
    const uint4* wr = reinterpret_cast<const uint4*>(wb + (row0 + kUpRows * wave + rw) * NW);
#pragma unroll
    for (int it = 0; it < kIt; ++it) q[it] = wr[min(jl + 16 * it, NP - 1)];  // past NP: re-read, unused
  }

  // ---- x pairs and piece sums into LDS: word t = tid + 256 i holds inputs 8t .. 8t+7
#pragma unroll
  for (int i = 0; i < kUpXIt; ++i) {
    const int t = tid + kUpThreads * i;
    const uint32_t w[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};  // bf16 pairs (x[8t+2c], x[8t+2c+1])
    if (t < NW) {
      // pairs (x[8t+n], x[8t+n+4]): the low or high halves of words n/2 and n/2 + 2, one
      // v_perm_b32 each
      uint4 pr;
      pr.x = __builtin_amdgcn_perm(w[2], w[0], 0x05040100u);
      pr.y = __builtin_amdgcn_perm(w[2], w[0], 0x07060302u);
      pr.z = __builtin_amdgcn_perm(w[3], w[1], 0x05040100u);
      pr.w = __builtin_amdgcn_perm(w[3], w[1], 0x07060302u);
      // word m of piece j at [m][j]: lanes holding consecutive pieces read consecutive
      // 16-byte words (no LDS bank conflicts)
      *reinterpret_cast<uint4*>(&xp[4 * ((t & 3) * kUpMaxP + (t >> 2))]) = pr;
    }
    // the word's 8 inputs summed by v_dot2_f32_bf16 against (1.0, 1.0)
    float s8 = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) s8 = dot2_bf16(w[c], kBfOne2, s8);
    s8 += dpp_f32<0xB1>(s8);  // the 4 words of a piece: quad_perm xor 1, xor 2
    s8 += dpp_f32<0x4E>(s8);
    if (t < NW && (t & 3) == 0) xh[t >> 2] = s8;
  }
  if (tid < nsc) {
    const uint32_t sw[2] = {sv2.x, sv2.y}, bw[2] = {bv2.x, bv2.y};
    float f[8];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float sc = bf16_bits_to_f32((c & 1) ? sw[c >> 1] >> 16 : sw[c >> 1] & 0xFFFFu);
      const float bi = bf16_bits_to_f32((c & 1) ? bw[c >> 1] >> 16 : bw[c >> 1] & 0xFFFFu);
      f[2 * c] = 16.0f * sc;
      f[2 * c + 1] = fmaf(-16.0f, sc, bi);
    }
    float4* dst = reinterpret_cast<float4*>(&sbt[4 * sc_i]);
    dst[0] = make_float4(f[0], f[1], f[2], f[3]);
    dst[1] = make_float4(f[4], f[5], f[6], f[7]);
  }
  lds_barrier();

  // ---- the lane's pieces into its row partial, then the row's 16-lane sum
  const uint32_t nibm = opaque_vgpr(kNibHi);         // (w & nibm) | one: one v_and_or_b32
  float pr = 0.0f;
  const int rl = kUpRows * wave + rw;                 // row within the block
#pragma unroll
  for (int it = 0; it < kIt; ++it) {
    if (it < nit) {  // uniform
      const int j = jl + 16 * it;                      // < kUpMaxP: inside the LDS pitch
      const bool use = j < NP;                         // past NP: read, then dropped
      const uint32_t qw[4] = {q[it].x, q[it].y, q[it].z, q[it].w};
      float acc = 0.0f;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        // the four rows' lanes read the same words (one LDS access serves all four)
        const uint4 xq = *reinterpret_cast<const uint4*>(&xp[4 * (m * kUpMaxP + j)]);
        const uint32_t xw[4] = {xq.x, xq.y, xq.z, xq.w};
        // nibble n (bits 4n..4n+3 of each half) to bits 3..6: a left shift by 3 for n = 0,
        // right shifts by 1, 5, 9 for the others
        const uint32_t w0 = qw[m] << 3, w1 = qw[m] >> 1, w2 = qw[m] >> 5, w3 = qw[m] >> 9;
        acc = dot2_bf16(xw[0], (w0 & nibm) | kBfOne2, acc);
        acc = dot2_bf16(xw[1], (w1 & nibm) | kBfOne2, acc);
        acc = dot2_bf16(xw[2], (w2 & nibm) | kBfOne2, acc);
        acc = dot2_bf16(xw[3], (w3 & nibm) | kBfOne2, acc);
      }
      const float2 f = sbt[rl * NGD + min(j, NP - 1) / 2];
      pr += use ? fmaf(f.x, acc, f.y * xh[j]) : 0.0f;
    }
  }
  // 16-lane sum (quad_perm xor 1, xor 2, row_half_mirror, row_mirror): every lane of a row
  // ends with the row's total
  pr += dpp_f32<0xB1>(pr);
  pr += dpp_f32<0x4E>(pr);
  pr += dpp_f32<0x141>(pr);
  pr += dpp_f32<0x140>(pr);
  const float ui = ok ? pr : 0.0f;

  // ---- h = square(relu(bf16(u))) in bf16; lane 16 i writes row i of the wave
  const float ub = bf16_bits_to_f32(f32_to_bf16_bits(ui));
  const float r = ub != ub ? ub : fmaxf(ub, 0.0f);
  const uint16_t hb = f32_to_bf16_bits(r * r);
  if (jl == 0) hcat[(size_t)b * NR + r0 + kUpRows * wave + rw] = hb;
  const uint64_t lv = __ballot(jl == 0 && (hb & 0x7FFFu) != 0);  // bits 0, 16, 32, 48
  const uint32_t lb = (uint32_t)((lv & 1u) | ((lv >> 15) & 2u) | ((lv >> 30) & 4u) | ((lv >> 45) & 8u));
  if (lane == 0) nib[wave] = (int)lb;
  if (live_out) {
    lds_barrier();
    if (tid == 0) {
      // this block's 16 bits of the group's 64-bit mask (little-endian: quarter q of
      // group g is 16-bit word 4 g + q)
      uint32_t m = 0;
#pragma unroll
      for (int w = 0; w < kUpWaves; ++w) m |= (uint32_t)nib[w] << (kUpRows * w);
      const size_t piece = ((size_t)b * (NR / 64) + r0 / 64) * (64 / kUpBlk) + (r0 % 64) / kUpBlk;
      if constexpr (kUpBlk == 16)
        reinterpret_cast<uint16_t*>(live_out)[piece] = (uint16_t)m;
      else
        reinterpret_cast<uint8_t*>(live_out)[piece] = (uint8_t)m;
    }
  }
  if (!ok && tid == 0 && f0 == 0 && status) atomicOr(status, (int32_t)HSD_STATUS_BAD_EXPERT);
}

// The router's top-k alone: one wavefront per token row writes sel and gains (the shared
// expert's gain 1.0 last).
__global__ __launch_bounds__(64) void k_router_topk(Router rt, int E, int topk) {
  const int b = blockIdx.x, lane = threadIdx.x;
  int es[kMaxTopk];
  float gs[kMaxTopk];
  route_topk_wave(rt, b, E, topk, topk, lane, es, gs);
  int ek = es[0];
  float gk = gs[0];
#pragma unroll
  for (int r = 1; r < kMaxTopk; ++r) {
    ek = lane == r ? es[r] : ek;
    gk = lane == r ? gs[r] : gk;
  }
  if (lane <= topk) {
    if (lane < topk) rt.sel_out[b * topk + lane] = ek;
    rt.gains_out[b * (topk + 1) + lane] = lane < topk ? gk : 1.0f;
  }
}

}  // namespace
}  // namespace hsd

using namespace hsd;

extern "C" int hsd_moe_up_relu2(const void* x, int x_dtype, const int32_t* sel, const uint32_t* w1,
                                const uint16_t* s1, const uint16_t* b1, const uint32_t* sw1,
                                const uint16_t* ss1, const uint16_t* sb1, void* hcat, int64_t B,
                                int64_t D, int64_t F, int64_t FS, int64_t topk, int64_t E,
                                uint64_t* live_masks, int32_t* dev_status, void* stream) {
  const char* fn = "hsd_moe_up_relu2";
  if (!x || !sel || !w1 || !s1 || !b1 || !sw1 || !ss1 || !sb1 || !hcat)
    return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (x_dtype != HSD_DT_BF16) return set_error(HSD_ERR_DTYPE, "%s: x must be bf16", fn);
  if (B < 0 || topk <= 0 || E <= 0 || D <= 0 || D % 64 || D > kUpMaxD || F <= 0 || F % 64 || FS <= 0 ||
      FS % 64)
    return set_error(HSD_ERR_SHAPE, "%s: need D %% 64 == 0 and D <= %d, F %% 64 == 0, FS %% 64 == 0", fn,
                     kUpMaxD);
  if (B > 65535 || (topk * F + FS) / 64 > 0x7FFFFFFF || E * F * (D / 8) >= ((int64_t)1 << 40))
    return set_error(HSD_ERR_SHAPE, "%s: sizes too large", fn);
  const uintptr_t al = (uintptr_t)x | (uintptr_t)w1 | (uintptr_t)sw1 | (uintptr_t)s1 | (uintptr_t)b1 |
                       (uintptr_t)ss1 | (uintptr_t)sb1;
  if (al & 15u)
    return set_error(HSD_ERR_ALIGN, "%s: x, the weights, scales and biases must be 16-byte aligned", fn);
  if (B == 0) return HSD_OK;
  const dim3 grid((unsigned)((topk * F + FS) / kUpBlk), (unsigned)B);
#define HSD_UP(MD)                                                                              \
  hipLaunchKernelGGL((k_moe_up<false, MD>), grid, dim3(kUpThreads), 0, as_stream(stream),      \
                     (int)D, (int)F, (int)FS, (int)topk, (int)E, reinterpret_cast<const uint16_t*>(x), \
                     sel, nullptr, nullptr, w1, s1, b1, sw1, ss1, sb1,                          \
                     reinterpret_cast<uint16_t*>(hcat), live_masks, dev_status, Router{})
  if (D <= kUpSmallD)
    HSD_UP(kUpSmallD);
  else
    HSD_UP(kUpMaxD);
#undef HSD_UP
  return check_launch(fn);
}

extern "C" int hsd_moe_route_up_relu2(const void* x, int x_dtype, const uint16_t* logits, const float* e_bias,
                                      float routed_scale, int norm_topk, int32_t* sel, float* gains,
                                      const uint32_t* w1, const uint16_t* s1, const uint16_t* b1,
                                      const uint32_t* sw1, const uint16_t* ss1, const uint16_t* sb1, void* hcat,
                                      int64_t B, int64_t D, int64_t F, int64_t FS, int64_t topk, int64_t E,
                                      uint64_t* live_masks, void* stream) {
  const char* fn = "hsd_moe_route_up_relu2";
  if (!x || !logits || !sel || !gains || !w1 || !s1 || !b1 || !sw1 || !ss1 || !sb1 || !hcat)
    return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (x_dtype != HSD_DT_BF16) return set_error(HSD_ERR_DTYPE, "%s: x must be bf16", fn);
  if (B < 0 || topk <= 0 || topk > kMaxTopk || E < topk || E > kMaxE || E % 4 || D <= 0 || D % 64 || D > kUpMaxD ||
      F <= 0 || F % 64 || FS <= 0 || FS % 64)
    return set_error(HSD_ERR_SHAPE,
                     "%s: need topk <= %d, topk <= E <= %d, E %% 4 == 0, D %% 64 == 0, D <= %d, F and FS %% 64 == 0", fn,
                     kMaxTopk, kMaxE, kUpMaxD);
  if (B > 65535 || E * F * (D / 8) >= ((int64_t)1 << 40)) return set_error(HSD_ERR_SHAPE, "%s: sizes too large", fn);
  const uintptr_t al = (uintptr_t)x | (uintptr_t)w1 | (uintptr_t)sw1 | (uintptr_t)s1 | (uintptr_t)b1 |
                       (uintptr_t)ss1 | (uintptr_t)sb1;
  if (al & 15u)
    return set_error(HSD_ERR_ALIGN, "%s: x, the weights, scales and biases must be 16-byte aligned", fn);
  if (B == 0) return HSD_OK;
  const dim3 grid((unsigned)((topk * F + FS) / kUpBlk), (unsigned)B);
  Router rt{logits, e_bias, sel, gains, routed_scale, norm_topk};
#define HSD_UP(MD)                                                                                   \
  hipLaunchKernelGGL((k_moe_up<true, MD>), grid, dim3(kUpThreads), 0, as_stream(stream),            \
                     (int)D, (int)F, (int)FS, (int)topk, (int)E, reinterpret_cast<const uint16_t*>(x), \
                     nullptr, rt.logits, rt.bias, w1, s1, b1, sw1, ss1, sb1,                         \
                     reinterpret_cast<uint16_t*>(hcat), live_masks, nullptr, rt)
  if (D <= kUpSmallD)
    HSD_UP(kUpSmallD);
  else
    HSD_UP(kUpMaxD);
#undef HSD_UP
  return check_launch(fn);
}

extern "C" int hsd_router_topk(const uint16_t* logits, const float* e_bias, float routed_scale, int norm_topk,
                               int32_t* sel, float* gains, int64_t B, int64_t E, int64_t topk, void* stream) {
  const char* fn = "hsd_router_topk";
  if (!logits || !sel || !gains) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (B < 0 || B > 65535 || topk <= 0 || topk > kMaxTopk || E < topk || E > kMaxE || E % 4)
    return set_error(HSD_ERR_SHAPE, "%s: need topk <= %d, topk <= E <= %d, E %% 4 == 0", fn, kMaxTopk, kMaxE);
  if (B == 0) return HSD_OK;
  Router rt{logits, e_bias, sel, gains, routed_scale, norm_topk};
  hipLaunchKernelGGL(k_router_topk, dim3((unsigned)B), dim3(64), 0, as_stream(stream), rt, (int)E, (int)topk);
  return check_launch(fn);
}
