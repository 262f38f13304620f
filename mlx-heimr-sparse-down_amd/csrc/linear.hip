// The dense projections of a decode step: y = x W^T for B <= 4 token rows, with W in
// the checkpoint's affine 4-bit group-64 layout (mlx `quantized_matmul(x, w, scales,
// biases, transpose=True)`, the QuantizedLinear of every Mamba in/out projection,
// attention projection and lm_head) or in bf16 (the router gate, the MTP head's eh_proj).
//
// Optional fused prologues on x (each workgroup recomputes them for its rows, so no
// separate normalisation launch):
//   HSD_X_RMS    xn = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)    (mx.fast.rms_norm)
//   HSD_X_GATED  z = y * silu(gate); per group of 512: xn = bf16(bf16(z * rsqrt(mean(z^2)
//                + eps)) * w)     (the Mamba-2 gated RMSNorm in front of out_proj)
// and epilogues: bf16 or f32 output, a residual add y = bf16(res + bf16(x W^T)), or the
// greedy argmax of the bf16-rounded outputs (per-workgroup best keys, reduced by
// hsd_argmax_keys; lm_head + argmax without writing the logits).
//
// Work split: a workgroup (4 wavefronts) owns 16 consecutive output rows (4-bit: 4 per
// wavefront) or 4 (bf16: 1 per wavefront) and loops over row blocks strided by the grid
// (as many workgroups as are resident at once, so the prologue is paid once per
// workgroup; every 4-bit projection of the model is one block per workgroup).
// 4-bit: the lanes of half-wavefront h own rows 2h and 2h + 1, lane l the 16-byte pieces
// l % 32, l % 32 + 32, ... of both: an x piece read from LDS serves two rows, and a lane
// adds into one partial per (row, token row) with no selects (VALU-bound at three token
// rows: 253 -> 150 VGPRs and 3 workgroups per CU for in_proj). The pieces become bf16 pairs
// (1 + q/16) with a shift, a mask and an OR, and v_dot2_f32_bf16 accumulates x (1 + q/16);
// per 32-input piece u += 16 s acc + (b - 16 s) sum(x) (the affine dequantisation folded per
// piece). A row's 32 lane partials are summed with DPP and v_permlane16_swap in a fixed
// order. bf16: lane l owns the pieces l, l + 64, ... of the wavefront's row; the next
// block's pieces are loaded while the current one is computed.
// 4-bit projections of more 16-row blocks than one grid (lm_head) run on the matrix cores
// instead (k_linear_q4 below): at several token rows the per-row dot products above bound
// them.
//
// Every token row is computed by the same instruction sequence whatever B is: a row of a
// B-row call is bit-identical to the same row alone (verify rows == decode rows).
#include "hsd_common.h"

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>

namespace hsd {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kLT = 256;                 // threads per workgroup
constexpr int kLMaxB = 4;                // token rows per launch
constexpr int kLMaxI = 6144;             // inputs per row
constexpr int kLSmallQ4 = 4096;          // 4-bit rows up to this length: 2 pieces per lane
constexpr int kLMaxGrid = 2048;
constexpr int kRowsMaxO = 512;           // bf16 rows with the RMS prologue up to this: k_linear_rows
constexpr uint32_t kBfOne2 = 0x3F803F80u;
constexpr uint32_t kNibHi = 0x00780078u;

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                         false);
}

__device__ __forceinline__ float rne_bf16(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

// Order key of a bf16 value for a max: larger values give larger keys; NaN (the
// canonical positive 0x7FC0) beats every number. Low 32 bits: ~index, so equal values
// prefer the smaller index.
__device__ __forceinline__ uint64_t argmax_key(uint16_t bits, int idx) {
  const uint32_t ord = (bits & 0x8000u) ? (uint32_t)(~bits & 0xFFFFu) : (uint32_t)(bits | 0x8000u);
  const uint32_t o2 = ((bits & 0x7FFFu) > 0x7F80u) ? 0x1FFFFu : ord;  // NaN above +inf
  return ((uint64_t)o2 << 32) | (uint32_t)~(uint32_t)idx;
}

template <int WF> struct WTraits;
template <> struct WTraits<HSD_W_Q4> {
  static constexpr int kIn = 32;                        // inputs per 16-byte piece
};
template <> struct WTraits<HSD_W_BF16> {
  static constexpr int kIn = 8;
};

struct LinArgs {
  const void* x;
  int64_t x_ld;
  const uint16_t* gate;
  int64_t gate_ld;
  const uint16_t* nw;
  float eps;
  const void* w;
  const uint16_t* s;
  const uint16_t* bq;
  void* y;
  int64_t y_ld;
  const uint16_t* res;
  int64_t res_ld;
  uint16_t* xn_out;
  int64_t xn_ld;
  uint64_t* keys;
  int64_t key_ld;
  int key_slots;
  int O, I;
};

// The fields a workgroup's first loads need (x, the weights, scales and biases, the norm
// weight, the shape, the grid) go ahead of the struct as scalar arguments: the dispatch
// preloads a kernel's leading scalar arguments into SGPRs (56 bytes here), while a struct
// argument (or gridDim, a hidden argument) is read from the argument segment by scalar
// loads, which the first global loads would wait for. The kernels rebuild the whole struct
// from both; grid_ is the launch's workgroup count.
#define HSD_LIN_PARAMS                                                                                  \
  const void *x_, const void *w_, const uint16_t *s_, const uint16_t *bq_, const uint16_t *nw_,          \
      int x_ld_, int grid_, int O_, int I_, LinArgs a_
#define HSD_LIN_UNPACK                                                                                  \
  LinArgs a = a_;                                                                                       \
  a.x = x_;                                                                                             \
  a.w = w_;                                                                                             \
  a.s = s_;                                                                                             \
  a.bq = bq_;                                                                                           \
  a.nw = nw_;                                                                                           \
  a.x_ld = x_ld_;                                                                                       \
  a.O = O_;                                                                                             \
  a.I = I_
#define HSD_LIN_ARGS(a, g) a.x, a.w, a.s, a.bq, a.nw, (int)a.x_ld, (int)(g), a.O, a.I, a

// Two floats to packed bf16 (round to nearest even; v_cvt_pk_bf16_f32 on gfx950). Used for
// the normalised activations, which are finite.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const __bf16 a = (__bf16)lo, b = (__bf16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}
__device__ __forceinline__ float lo_f(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float hi_f(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

// The prologue on x, shared by the kernels: this workgroup's copy of the NB input rows,
// normalised if asked, into LDS as bf16 pairs (4-bit weights: pairs (x[i], x[i+4]) in the
// order of a word's nibble pairs, word m of 32-input piece j at [m][j]; bf16: natural
// pairs), and for 4-bit weights the input sums of every PS inputs (32: a piece, 64: a
// group). load() issues the loads; the caller issues its first weight loads next, so
// finish() waits for x only (loads complete in issue order) while the weights are still
// on their way. Words t = tid + 256 i hold inputs 8t .. 8t+7.
// PX (4-bit weights): the LDS pitch of a token row in 32-input pieces (the instance's
// largest row), so that the readers' addresses are a lane base plus compile-time offsets.
template <int WF, int NB, int XK, int XIT, int PX>
struct XIn {
  static constexpr bool kF32 = XK == HSD_X_GATED || XK == HSD_X_GATED_Z;  // x is f32
  uint4 xv[XK == HSD_X_GATED_Z ? 1 : NB][XIT];
  float4 yv0[kF32 ? NB : 1][XIT], yv1[kF32 ? NB : 1][XIT];
  float zp[XK == HSD_X_GATED_Z ? NB : 1][XIT];   // HSD_X_GATED_Z: a partial of the group's sum
  uint4 nwv[XIT];

  __device__ __forceinline__ void load(const LinArgs& a, int tid) {
    const int NW = a.I / 8;
#pragma unroll
    for (int i = 0; i < XIT; ++i) {
      const int tc = min(tid + kLT * i, NW - 1);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if constexpr (kF32) {
          const float* xr = reinterpret_cast<const float*>(a.x) + b * a.x_ld;
          const float4* yr = reinterpret_cast<const float4*>(xr);
          yv0[b][i] = yr[2 * tc];
          yv1[b][i] = yr[2 * tc + 1];
          if constexpr (XK == HSD_X_GATED)
            xv[b][i] = reinterpret_cast<const uint4*>(a.gate + b * a.gate_ld)[tc];
          else  // the group of word tc (64 words) has partials 32 (tc / 64) .. + 31
            zp[b][i] = xr[a.I + 32 * (tc >> 6) + (tid & 31)];
        } else {
          xv[b][i] = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.x) + b * a.x_ld)[tc];
        }
      }
      if constexpr (XK != HSD_X_BF16) nwv[i] = reinterpret_cast<const uint4*>(a.nw)[tc];
    }
  }

  template <int PS>
  __device__ __forceinline__ void finish(const LinArgs& a, uint32_t* xp, float* xs, float (*wsum)[4], int tid,
                                         int lane, int wave) {
    const int I = a.I, NW = I / 8;
    // xo[b][i][c]: the prologue's output elements 8t + 2c, 8t + 2c + 1 as a bf16 pair
    uint32_t xo[NB][XIT][4];
    if constexpr (XK == HSD_X_BF16) {
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < XIT; ++i) {
          xo[b][i][0] = xv[b][i].x; xo[b][i][1] = xv[b][i].y; xo[b][i][2] = xv[b][i].z; xo[b][i][3] = xv[b][i].w;
        }
    } else if constexpr (XK == HSD_X_RMS) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < XIT; ++i) {
          const bool tv = tid + kLT * i < NW;
          const uint32_t xw[4] = {xv[b][i].x, xv[b][i].y, xv[b][i].z, xv[b][i].w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const uint32_t v = tv ? xw[c] : 0u;
            ss = dot2_bf16(v, v, ss);
          }
        }
        ss = wave_sum_dpp(ss);
        if (lane == 0) wsum[b][wave] = ss;
      }
      lds_barrier();
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float tot = ((wsum[b][0] + wsum[b][1]) + wsum[b][2]) + wsum[b][3];
        const float inv = __builtin_amdgcn_rsqf(tot / (float)I + a.eps);
#pragma unroll
        for (int i = 0; i < XIT; ++i) {
          const uint32_t xw[4] = {xv[b][i].x, xv[b][i].y, xv[b][i].z, xv[b][i].w};
          const uint32_t nw4[4] = {nwv[i].x, nwv[i].y, nwv[i].z, nwv[i].w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const uint32_t t = pack_bf16x2(lo_f(xw[c]) * inv, hi_f(xw[c]) * inv);
            xo[b][i][c] = pack_bf16x2(lo_f(t) * lo_f(nw4[c]), hi_f(t) * hi_f(nw4[c]));
          }
        }
      }
    } else if constexpr (XK == HSD_X_GATED_Z) {
      // a wavefront's 64 words of iteration i are one 512-element group; its 32 partials
      // (in lanes 0-31, repeated in 32-63) summed with DPP inside 16-lane rows, then the
      // lower row's total plus the upper's (v_permlane16_swap)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int i = 0; i < XIT; ++i) {
          float g = zp[b][i];
          g += dpp_f32<0xB1>(g);
          g += dpp_f32<0x4E>(g);
          g += dpp_f32<0x141>(g);
          g += dpp_f32<0x140>(g);
          const uint32_t gb = __float_as_uint(g);
          const auto pg = __builtin_amdgcn_permlane16_swap(gb, gb, false, false);
          g = __uint_as_float(pg[0]) + __uint_as_float(pg[1]);
          const float inv = __builtin_amdgcn_rsqf(g / 512.0f + a.eps);
          const float z[8] = {yv0[b][i].x, yv0[b][i].y, yv0[b][i].z, yv0[b][i].w,
                              yv1[b][i].x, yv1[b][i].y, yv1[b][i].z, yv1[b][i].w};
          const uint32_t nw4[4] = {nwv[i].x, nwv[i].y, nwv[i].z, nwv[i].w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const uint32_t t = pack_bf16x2(z[2 * c] * inv, z[2 * c + 1] * inv);
            xo[b][i][c] = pack_bf16x2(lo_f(t) * lo_f(nw4[c]), hi_f(t) * hi_f(nw4[c]));
          }
        }
      }
    } else {  // HSD_X_GATED: a wavefront's 64 words of iteration i are one 512-element group
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int i = 0; i < XIT; ++i) {
          const bool tv = tid + kLT * i < NW;
          const uint32_t gw[4] = {xv[b][i].x, xv[b][i].y, xv[b][i].z, xv[b][i].w};
          const float yy[8] = {yv0[b][i].x, yv0[b][i].y, yv0[b][i].z, yv0[b][i].w,
                               yv1[b][i].x, yv1[b][i].y, yv1[b][i].z, yv1[b][i].w};
          float z[8];
          float g = 0.0f;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            z[2 * c] = tv ? yy[2 * c] * silu_f32(lo_f(gw[c])) : 0.0f;
            z[2 * c + 1] = tv ? yy[2 * c + 1] * silu_f32(hi_f(gw[c])) : 0.0f;
            g = fmaf(z[2 * c], z[2 * c], g);
            g = fmaf(z[2 * c + 1], z[2 * c + 1], g);
          }
          g = wave_sum_dpp(g);
          const float inv = __builtin_amdgcn_rsqf(g / 512.0f + a.eps);
          const uint32_t nw4[4] = {nwv[i].x, nwv[i].y, nwv[i].z, nwv[i].w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const uint32_t t = pack_bf16x2(z[2 * c] * inv, z[2 * c + 1] * inv);
            xo[b][i][c] = pack_bf16x2(lo_f(t) * lo_f(nw4[c]), hi_f(t) * hi_f(nw4[c]));
          }
        }
      }
    }
    // ---- into LDS (and the side output)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int i = 0; i < XIT; ++i) {
        const int t = tid + kLT * i;
        const uint32_t* w = xo[b][i];
        if (t < NW) {
          uint4 pr;
          if constexpr (WF == HSD_W_Q4) {
            // pairs (x[8t + n], x[8t + n + 4]): element n of the word is half (n & 1) of w[n / 2]
            pr.x = (w[0] & 0xFFFFu) | (w[2] << 16);
            pr.y = (w[0] >> 16) | (w[2] & 0xFFFF0000u);
            pr.z = (w[1] & 0xFFFFu) | (w[3] << 16);
            pr.w = (w[1] >> 16) | (w[3] & 0xFFFF0000u);
          } else {
            pr.x = w[0]; pr.y = w[1]; pr.z = w[2]; pr.w = w[3];
          }
          // 4-bit: word m of piece j at [m][j] with a row of PX pieces (lanes holding
          // consecutive pieces then read consecutive 16-byte words, free of bank
          // conflicts); bf16: word t at t
          const int slot = WF == HSD_W_Q4 ? (t & 3) * PX + (t >> 2) : t;
          *reinterpret_cast<uint4*>(&xp[b * (WF == HSD_W_Q4 ? 16 * PX : I / 2) + 4 * slot]) = pr;
          if (a.xn_out && blockIdx.x == 0)
            reinterpret_cast<uint4*>(a.xn_out + b * a.xn_ld)[t] = make_uint4(w[0], w[1], w[2], w[3]);
        }
        if constexpr (WF == HSD_W_Q4) {
          float s8 = 0.0f;
#pragma unroll
          for (int c = 0; c < 4; ++c) s8 = dot2_bf16(w[c], kBfOne2, s8);
          s8 += dpp_f32<0xB1>(s8);  // the 4 words of a piece: quad_perm xor 1, xor 2
          s8 += dpp_f32<0x4E>(s8);
          if constexpr (PS == 64) s8 += dpp_f32<0x141>(s8);  // the other piece: row_half_mirror
          constexpr int kWS = PS / 8;                        // words per sum
          if (t < NW && (t & (kWS - 1)) == 0) xs[b * (PX * 32 / PS) + t / kWS] = s8;
        }
      }
    }
  }
};

// IMAX: the largest row length the instance serves (kFull full passes of 64 pieces, XIT x
// words of 8 inputs per thread in the prologue).
// RW: output rows per wavefront (a block = 4 RW rows). Lane l owns pieces l, l + 64, ... of
// each of its wavefront's RW rows, so an x piece read from LDS serves RW rows.
// At one token row the projections with a single block per workgroup (in_proj: 644
// blocks) want three workgroups per CU (8.5 against 9.1 us); the argmax instances (many
// blocks per workgroup, the next block in flight: lm_head took 49 against 59 us here before
// it moved to the matrix cores) are faster with the registers of two.
// ROWSY: a one-row residual instance launched over (blocks, token rows), blockIdx.y the
// token row (its own instance, so the one-row launches keep their code).
template <int WF, int NB, int XK, int YK, int IMAX, int RW, bool REM, bool ROWSY = false>
__global__ __launch_bounds__(kLT, WF == HSD_W_Q4 ? (IMAX == 3072 && NB < 4 ? 3 : 2) : (NB == 1 && YK != HSD_Y_ARGMAX) ? 3 : 2)
void k_linear(HSD_LIN_PARAMS) {
  HSD_LIN_UNPACK;
  using T = WTraits<WF>;
  constexpr bool Q4 = WF == HSD_W_Q4;
  static_assert(!Q4 || RW == 4 || RW == 2, "4-bit weights: 4 or 2 rows per wavefront, 2 or 1 per half-wavefront");
  constexpr int kRW = RW;
  constexpr int kRH = Q4 ? RW / 2 : 1;                 // 4-bit: rows per half-wavefront (each lane's)
  constexpr int kIt32 = (IMAX / 32 + 31) / 32;          // 4-bit: pieces per lane and row (max)
  constexpr int kFull = (IMAX / T::kIn) / 64 > 0 ? (IMAX / T::kIn) / 64 : 1;  // full passes (max)
  constexpr int kRP = REM ? (kRW * 63 + 63) / 64 : 1;  // remainder passes (max; none without REM)
  constexpr int XIT = (IMAX / 8 + kLT - 1) / kLT;
  constexpr int kRows = 4 * kRW;                       // rows per block
  extern __shared__ __attribute__((aligned(16))) uint32_t lsm[];
  // LDS: x as bf16 pairs [NB][I/2] (4-bit: pairs (x[i], x[i+4]) in a word's nibble
  // order, word m of 32-input piece j at [m][j]; bf16: natural pairs), then the 32-input
  // piece sums [NB][I/32] (4-bit only)
  __shared__ float wsum[NB][4];
  __shared__ uint64_t kbest[4][NB];
  const int I = a.I, O = a.O, NW = I / 8;
  uint32_t* xp = lsm;
  constexpr int PX = IMAX / 32;                        // 4-bit: LDS pitch of a token row in pieces
  float* xh = reinterpret_cast<float*>(lsm + NB * (Q4 ? 16 * PX : I / 2));
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t nibm = opaque_vgpr(kNibHi);         // (w & nibm) | one: one v_and_or_b32
  const int nblk = (O + kRows - 1) / kRows;            // the last block may be partial
  const int NPr = I / T::kIn;                          // pieces per row
  // 4-bit: lanes 32 h .. 32 h + 31 take rows 2 h and 2 h + 1 of the wavefront's 4, lane l
  // pieces l % 32 + 32 it of both (84 pieces a row at I = 2688: 3 each, the last taken by
  // 20 lanes of a half): an x piece read from LDS serves two rows, and a lane's rows never
  // change, so it keeps one partial per (row, token row).
  const int hw = lane >> 5, jl = lane & 31, nit32 = (NPr + 31) / 32;
  // bf16: pieces 0 .. 64 nfull - 1 of every row: lane l owns pieces l + 64 it of each of the
  // wavefront's kRW rows; the nrem pieces left of each row are dealt as (row, piece) pairs
  // over the lanes, so no pass runs with most lanes idle
  const int nfull = NPr / 64, nrem = REM ? NPr - 64 * nfull : 0;
  const int npair = kRW * nrem, npass = (npair + 63) / 64;
  int prr[kRP], prj[kRP];                              // a pair's row and piece
#pragma unroll
  for (int ps = 0; ps < kRP; ++ps) {
    const int p = min(lane + 64 * ps, max(npair - 1, 0));
    prr[ps] = nrem > 0 ? p / nrem : 0;
    prj[ps] = min(64 * nfull + (p - prr[ps] * max(nrem, 1)), NPr - 1);
  }

  // ---- weight pieces of a block (rows past O re-read row O-1, pieces past the row re-read
  // its last piece; unused)
  struct BlkQ4 {
    uint4 q[kIt32][kRH];
    uint32_t s[kIt32][kRH];
  };
  struct BlkBf {
    uint4 q[kRW][kFull];
    uint32_t s[kRW][kFull];
    uint4 qr[kRP];
    uint32_t sr[kRP];
  };
  using Blk = typename std::conditional<Q4, BlkQ4, BlkBf>::type;
  auto load_piece = [&](int row, int j, uint4& qq, uint32_t& sq) {
    if constexpr (WF == HSD_W_Q4) {
      const uint32_t* wr = reinterpret_cast<const uint32_t*>(a.w) + (size_t)row * NW;
      qq = reinterpret_cast<const uint4*>(wr)[j];
      const size_t gi = (size_t)row * (I / 64) + (j >> 1);
      sq = (uint32_t)a.s[gi] | ((uint32_t)a.bq[gi] << 16);
    } else {
      const uint16_t* wr = reinterpret_cast<const uint16_t*>(a.w) + (size_t)row * I;
      qq = reinterpret_cast<const uint4*>(wr)[j];
      sq = 0;
    }
  };
  auto load_block = [&](int blk, Blk& bk) {
    const int r0 = blk * kRows + kRW * wave;
    if constexpr (Q4) {
#pragma unroll
      for (int it = 0; it < kIt32; ++it)
#pragma unroll
        for (int i = 0; i < kRH; ++i)
          load_piece(min(r0 + kRH * hw + i, O - 1), min(jl + 32 * it, NPr - 1), bk.q[it][i], bk.s[it][i]);
    } else {
#pragma unroll
      for (int r = 0; r < kRW; ++r) {
        const int row = min(r0 + r, O - 1);
#pragma unroll
        for (int it = 0; it < kFull; ++it) load_piece(row, min(lane + 64 * it, NPr - 1), bk.q[r][it], bk.s[r][it]);
      }
      if constexpr (REM) {
#pragma unroll
        for (int ps = 0; ps < kRP; ++ps) load_piece(min(r0 + prr[ps], O - 1), prj[ps], bk.qr[ps], bk.sr[ps]);
      }
    }
  };

  // a one-row residual instance launched over several token rows (blockIdx.y = the token
  // row: a three-row call of a projection with few blocks, whose x needs no gate and writes
  // no normed copy): each y-slice is that row's one-row call, so the row's bits are those
  // of the one-row and the three-row kernels. x moves here (its stride is a preloaded
  // argument); the residual and the output take the row where they are used, so no wait for
  // the other arguments moves ahead of the first loads
  constexpr bool kRowsY = ROWSY;
  static_assert(!ROWSY || (NB == 1 && YK == HSD_Y_RESID), "token rows over blockIdx.y: one-row residual instances");
  const size_t yrow = kRowsY ? (size_t)blockIdx.y : 0;
  if constexpr (kRowsY) {
    constexpr size_t kXE = XIn<WF, NB, XK, XIT, PX>::kF32 ? 4 : 2;
    a.x = reinterpret_cast<const char*>(a.x) + yrow * (size_t)x_ld_ * kXE;
  }

  // ---- the output slot of this lane in a block's epilogue: token row ob, row orr of the
  // wavefront's rows (lane_out: the lane writes one)
  auto out_slot = [&](int& ob, int& orr, bool& lane_out) {
    if constexpr (Q4) {
      ob = jl / kRH;
      orr = kRH * hw + jl % kRH;
      lane_out = jl < kRH * NB;
    } else {
      ob = lane / kRW;
      orr = lane - ob * kRW;
      lane_out = lane < NB * kRW;
    }
  };
  // the residual of the lane's output in block blk_ (HSD_Y_RESID), loaded ahead of the
  // block's weights rather than in the epilogue, where it was one more round trip at the
  // end of every block (slots the lane does not write re-read a valid element)
  auto load_res = [&](int blk_) -> uint32_t {
    if constexpr (YK == HSD_Y_RESID) {
      int ob, orr;
      bool lane_out;
      out_slot(ob, orr, lane_out);
      const int o = min(blk_ * kRows + kRW * wave + orr, O - 1);
      return a.res[(yrow + min(ob, NB - 1)) * a.res_ld + o];
    } else {
      return 0u;
    }
  };

  // ---- prologue: this workgroup's copy of the NB input rows, normalised if asked
  XIn<WF, NB, XK, XIT, PX> xin;
  xin.load(a, tid);
  // the residual and the first block's weight pieces, issued after x: the prologue waits
  // for x only (loads complete in issue order), while the weights are still on their way
  Blk cur;
  int blk = blockIdx.x;
  uint32_t resv = load_res(blk);
  load_block(blk, cur);
  // every load above is issued before the prologue's arithmetic: the scheduler had moved
  // the gated norm's partial sums (which wait for their loads) ahead of the weight loads
  __builtin_amdgcn_sched_barrier(0);
  xin.template finish<32>(a, xp, xh, wsum, tid, lane, wave);
  lds_barrier();                                       // x in LDS; the weights may still be in flight
  // the residual in a register here (its load was issued before the weights', so this
  // waits for it alone): the compiler cannot move the load into the epilogue's branch
  if constexpr (YK == HSD_Y_RESID) resv = opaque_vgpr(resv);

  // bf16: one 16-byte piece j of a row against the token rows: the partial of each token row
  auto piece_terms = [&](int j, const uint4& qv, float (&t)[NB]) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const uint4 xq = *reinterpret_cast<const uint4*>(&xp[b * (I / 2) + 4 * j]);
      float acc = 0.0f;
      acc = dot2_bf16(xq.x, qv.x, acc);
      acc = dot2_bf16(xq.y, qv.y, acc);
      acc = dot2_bf16(xq.z, qv.z, acc);
      acc = dot2_bf16(xq.w, qv.w, acc);
      t[b] = acc;
    }
  };

  // ---- one block: the lane's pieces into per-row partials, the 64-lane sums, the epilogue
  uint64_t best[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) best[b] = 0;
  auto do_block = [&](int blk_, const Blk& bk, uint32_t resv_) {
    float outv = 0.0f;
    int ob, orr;
    bool lane_out;
    if constexpr (Q4) {
      // the lane's pieces of its kRH rows against every token row, then the 32-lane sums
      float pq[NB][kRH];
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < kRH; ++i) pq[b][i] = 0.0f;
#pragma unroll
      for (int it = 0; it < kIt32; ++it) {
        if (it < nit32) {                                // uniform
          const int j = jl + 32 * it;                    // < PX: inside the row's LDS pitch
          const bool use = j < NPr;                      // past NPr: read, then dropped
          // the token rows' x words of piece j (the two half-wavefronts read the same)
          uint4 xq[NB][4];
          float xs[NB];
#pragma unroll
          for (int b = 0; b < NB; ++b) {
#pragma unroll
            for (int m = 0; m < 4; ++m) xq[b][m] = *reinterpret_cast<const uint4*>(&xp[b * 16 * PX + (m * PX + j) * 4]);
            xs[b] = xh[b * PX + j];
          }
#pragma unroll
          for (int i = 0; i < kRH; ++i) {
            const uint32_t qw[4] = {bk.q[it][i].x, bk.q[it][i].y, bk.q[it][i].z, bk.q[it][i].w};
            uint32_t wc[4][4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
              wc[m][0] = ((qw[m] << 3) & nibm) | kBfOne2;
              wc[m][1] = ((qw[m] >> 1) & nibm) | kBfOne2;
              wc[m][2] = ((qw[m] >> 5) & nibm) | kBfOne2;
              wc[m][3] = ((qw[m] >> 9) & nibm) | kBfOne2;
            }
            const float sv = lo_f(bk.s[it][i]), bv = hi_f(bk.s[it][i]);
            const float s16 = 16.0f * sv, bo = fmaf(-16.0f, sv, bv);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
              float acc = 0.0f;
#pragma unroll
              for (int m = 0; m < 4; ++m) {
                acc = dot2_bf16(xq[b][m].x, wc[m][0], acc);
                acc = dot2_bf16(xq[b][m].y, wc[m][1], acc);
                acc = dot2_bf16(xq[b][m].z, wc[m][2], acc);
                acc = dot2_bf16(xq[b][m].w, wc[m][3], acc);
              }
              pq[b][i] += use ? fmaf(s16, acc, bo * xs[b]) : 0.0f;
            }
          }
        }
      }
      // 32-lane sums: DPP inside each 16-lane row (quad_perm xor 1, xor 2, row_half_mirror,
      // row_mirror), then v_permlane16_swap puts the even and the odd row's totals side by
      // side and they are added in that order; lane 32 h + 2 b + i keeps (token row b, row
      // 2 h + i)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int i = 0; i < kRH; ++i) {
          float v = pq[b][i];
          v += dpp_f32<0xB1>(v);
          v += dpp_f32<0x4E>(v);
          v += dpp_f32<0x141>(v);
          v += dpp_f32<0x140>(v);
          const uint32_t vb = __float_as_uint(v);
          const auto pv = __builtin_amdgcn_permlane16_swap(vb, vb, false, false);
          const float u = __uint_as_float(pv[0]) + __uint_as_float(pv[1]);
          outv = jl == kRH * b + i ? u : outv;
        }
      }
    } else {
      float pr[NB][kRW];
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < kRW; ++r) pr[b][r] = 0.0f;
#pragma unroll
      for (int it = 0; it < kFull; ++it) {
        if (it < nfull) {                                // uniform
          const int j = lane + 64 * it;
          uint4 xq[NB];
#pragma unroll
          for (int b = 0; b < NB; ++b) xq[b] = *reinterpret_cast<const uint4*>(&xp[b * (I / 2) + 4 * j]);
#pragma unroll
          for (int r = 0; r < kRW; ++r) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
              float acc = 0.0f;
              acc = dot2_bf16(xq[b].x, bk.q[r][it].x, acc);
              acc = dot2_bf16(xq[b].y, bk.q[r][it].y, acc);
              acc = dot2_bf16(xq[b].z, bk.q[r][it].z, acc);
              acc = dot2_bf16(xq[b].w, bk.q[r][it].w, acc);
              pr[b][r] += acc;
            }
          }
        }
      }
      // pair passes: lane l's pair p = l + 64 ps is piece prj of row prr of the wavefront
#pragma unroll
      for (int ps = 0; ps < kRP; ++ps) {
        if (REM && ps < npass) {                         // uniform
          const bool use = lane + 64 * ps < npair;
          float t[NB];
          piece_terms(prj[ps], bk.qr[ps], t);
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int r = 0; r < kRW; ++r) pr[b][r] += (use && prr[ps] == r) ? t[b] : 0.0f;
        }
      }
      // row sums: lane b*kRW + r ends with row r of token row b
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int r = 0; r < kRW; ++r) {
          float v = pr[b][r];
          v += dpp_f32<0xB1>(v);
          v += dpp_f32<0x4E>(v);
          v += dpp_f32<0x141>(v);
          v += dpp_f32<0x140>(v);
          const float t0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
          const float t1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
          const float t2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
          const float t3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
          const float u = ((t0 + t1) + t2) + t3;
          outv = lane == b * kRW + r ? u : outv;
        }
      }
    }
    out_slot(ob, orr, lane_out);
    const int o = blk_ * kRows + kRW * wave + orr;
    const bool live = lane_out && o < O;
    if constexpr (YK == HSD_Y_ARGMAX) {
      const uint16_t lb = f32_to_bf16_bits(outv);
      const uint64_t key = live ? argmax_key(lb, o) : 0;
      if (a.y && live) reinterpret_cast<uint16_t*>(a.y)[ob * a.y_ld + o] = lb;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        uint64_t kb = 0;
#pragma unroll
        for (int r = 0; r < kRW; ++r) {
          const int ln = Q4 ? 32 * (r / kRH) + kRH * b + r % kRH : b * kRW + r;  // (token row b, row r)
          const uint64_t kr = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(key >> 32), ln) << 32) |
                              (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key, ln);
          kb = kr > kb ? kr : kb;
        }
        best[b] = kb > best[b] ? kb : best[b];
      }
    } else if (live) {
      const int64_t yi = ((int64_t)yrow + ob) * a.y_ld + o;
      if constexpr (YK == HSD_Y_F32) {
        reinterpret_cast<float*>(a.y)[yi] = outv;
      } else if constexpr (YK == HSD_Y_RESID) {
        const float rv = bf16_bits_to_f32(resv_);
        reinterpret_cast<uint16_t*>(a.y)[yi] = f32_to_bf16_bits(rv + rne_bf16(outv));
      } else {
        reinterpret_cast<uint16_t*>(a.y)[yi] = f32_to_bf16_bits(outv);
      }
    }
  };

  if ((int)gridDim.x >= nblk) {
    do_block(blk, cur, resv);                          // one block per workgroup
  } else if constexpr (Q4) {
    // several blocks, one after the other: a second block's registers in flight would
    // cost the occupancy that makes every projection of the model one block per workgroup
    // (in_proj: 644 blocks, 768 resident workgroups)
    for (;;) {
      do_block(blk, cur, resv);
      blk += (int)gridDim.x;
      if (blk >= nblk) break;
      __builtin_amdgcn_sched_barrier(0);
      resv = load_res(blk);
      load_block(blk, cur);
      if constexpr (YK == HSD_Y_RESID) resv = opaque_vgpr(resv);
    }
  } else {
    // several blocks: the next block's pieces are in flight while one is computed; the
    // load is unconditional (the last block re-reads its own lines), so the compiler's
    // wait before the arithmetic counts only the current block's loads
    for (;;) {
      const int nxt = blk + (int)gridDim.x;
      Blk nx;
      uint32_t resn = load_res(nxt < nblk ? nxt : blk);
      load_block(nxt < nblk ? nxt : blk, nx);
      if constexpr (YK == HSD_Y_RESID) resn = opaque_vgpr(resn);
      do_block(blk, cur, resv);
      if (nxt >= nblk) break;
      blk = nxt;
      cur = nx;
      resv = resn;
    }
  }
  if constexpr (YK == HSD_Y_ARGMAX) {
    if (lane == 0)
#pragma unroll
      for (int b = 0; b < NB; ++b) kbest[wave][b] = best[b];
    __syncthreads();
    if (tid < NB) {
      uint64_t k = kbest[0][tid];
#pragma unroll
      for (int w = 1; w < 4; ++w) k = kbest[w][tid] > k ? kbest[w][tid] : k;
      a.keys[tid * a.key_ld + blockIdx.x] = k;
      // slots past the grid (the grid follows the occupancy) read as the smallest key
      for (int sl = blockIdx.x + gridDim.x; sl < a.key_slots; sl += gridDim.x) a.keys[tid * a.key_ld + sl] = 0;
    }
  }
}

// bf16 weights with few output rows (the MoE router gate: 128 rows of 2688 inputs) and the
// RMS prologue: one workgroup per output row, the row's 16-byte pieces split over the four
// wavefronts (wavefront w takes the w-th quarter, lane l its pieces l and l + 64), each
// wavefront's 64-lane sum per token row to LDS, the four added in wavefront order. The
// workgroup-per-four-rows form of k_linear left most CUs idle (32 workgroups) with a whole
// row per wavefront; here the prologue is the same and the dot products a quarter as long.
template <int NB, int IMAX>
__global__ __launch_bounds__(kLT) void k_linear_rows(HSD_LIN_PARAMS) {
  HSD_LIN_UNPACK;
  constexpr int XIT = (IMAX / 8 + kLT - 1) / kLT;
  constexpr int kP = (IMAX / 8 / 4 + 63) / 64;         // passes per wavefront (max)
  extern __shared__ __attribute__((aligned(16))) uint32_t lsm[];  // x as bf16 pairs [NB][I/2]
  __shared__ float wsum[NB][4];
  __shared__ float red[4][NB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int I = a.I, NPr = I / 8;                      // 16-byte pieces per row
  const int o = blockIdx.x;                            // the grid is the row count
  XIn<HSD_W_BF16, NB, HSD_X_RMS, XIT, 1> xin;
  xin.load(a, tid);
  // the wavefront's quarter of the row: pieces q0 .. q1 - 1 (past q1: re-read, unused)
  const int per = (NPr + 3) / 4, q0 = wave * per, q1 = min(q0 + per, NPr);
  const uint4* wr = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.w) + (size_t)o * I);
  uint4 qv[kP];
#pragma unroll
  for (int p = 0; p < kP; ++p) qv[p] = wr[min(q0 + lane + 64 * p, NPr - 1)];
  __builtin_amdgcn_sched_barrier(0);
  xin.template finish<32>(a, lsm, nullptr, wsum, tid, lane, wave);
  lds_barrier();
  float pr[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) pr[b] = 0.0f;
  const int npass = (per + 63) / 64;
#pragma unroll
  for (int p = 0; p < kP; ++p) {
    if (p < npass) {                                   // uniform
      const int j = q0 + lane + 64 * p;
      const bool use = j < q1;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const uint4 xq = *reinterpret_cast<const uint4*>(&lsm[b * (I / 2) + 4 * min(j, NPr - 1)]);
        float acc = 0.0f;
        acc = dot2_bf16(xq.x, qv[p].x, acc);
        acc = dot2_bf16(xq.y, qv[p].y, acc);
        acc = dot2_bf16(xq.z, qv[p].z, acc);
        acc = dot2_bf16(xq.w, qv[p].w, acc);
        pr[b] += use ? acc : 0.0f;
      }
    }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const float v = wave_sum_dpp(pr[b]);
    if (lane == 0) red[wave][b] = v;
  }
  lds_barrier();
  if (tid < NB) {
    const float v = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
    reinterpret_cast<uint16_t*>(a.y)[tid * a.y_ld + o] = f32_to_bf16_bits(v);
  }
}

// 4-bit weights on the matrix cores, for projections with more 16-row blocks than
// resident workgroups (lm_head: 8192), where the per-token-row dot products of the kernel
// above bound the time at several token rows. A workgroup (4 wavefronts) loops over blocks
// of 16 consecutive output rows strided by the grid, the next block's weights and scales in
// flight while one is computed; wavefront w takes the 64-input groups g = w, w + 4, ... of
// the block's rows, and the four partial sums meet in LDS, added in wavefront order.
// Per group, lane l (n = l % 16, q = l / 16) holds 8 bytes of row n: words 2 (q % 2) and
// 2 (q % 2) + 1 of the group's piece q / 2. A word's 8 nibbles become the lane's B operand
// of one v_mfma_f32_16x16x32_bf16 as four bf16 pairs (1 + q_j/16, 1 + q_{j+4}/16) (a shift,
// a mask and an OR each, exact); the A operand is the same 8 inputs of token row l % 16
// from LDS (rows from B on repeat row B-1; their outputs are not used). Two MFMAs give
// acc[m][n] = sum over the group of x (1 + q/16) in fp32; then lane n adds
// 16 s acc + (b - 16 s) sum_g(x) (W = s q + b folded per group) for the group's scale and
// bias of row n, staged in LDS per block ([group][row]: the 16 lanes read 16 banks). The
// vector-ALU work is the unpacking and the scale step, the same for any number of token
// rows; a token row's result depends on its own row of A only, so it is the same bits
// whatever B is. At one token row the kernel above is as fast (lm_head 49.7 against 51.8
// us); at three, 51.0 against 84.0 us.
// For projections of one round of blocks it was slower at one token row: in_proj 9.5
// against 8.5 us, out_proj 8.3 against 5.9 (the MFMA chains of a wavefront's groups and the
// cross-wavefront sum are on the critical path of a single block), and loading a 16-byte
// piece per lane (two groups per load, the other group's lanes multiplying a zero A operand:
// four MFMAs per group) slower still (in_proj 9.9, lm_head 57.0 us).
constexpr int kQR = 16;                  // output rows per block (the MFMA's N)

template <int NB, int XK, int YK, int IMAX>
__global__ __launch_bounds__(kLT, 2) void k_linear_q4(HSD_LIN_PARAMS) {
  HSD_LIN_UNPACK;
  constexpr int kGW = (IMAX / 64 + 3) / 4;             // groups per wavefront (max)
  constexpr int XIT = (IMAX / 8 + kLT - 1) / kLT;
  extern __shared__ __attribute__((aligned(16))) uint32_t lsm[];
  __shared__ float wsum[NB][4];
  __shared__ float red[2][8][NB][kQR];                 // [block parity][chain][token row][row]
  const int I = a.I, O = a.O, G = I / 64;
  // LDS: x pairs [NB][I/2] words, the group sums [NB][G], then per block parity the
  // (scale | bias << 16) words of the block's rows [2][G][16]
  uint32_t* xp = lsm;
  constexpr int PX = IMAX / 32;                        // LDS pitch of a token row in pieces
  float* xg = reinterpret_cast<float*>(lsm + NB * 16 * PX);
  uint32_t* sbl = lsm + NB * 16 * PX + NB * (PX / 2);
  // the wavefront index as a scalar: the group loops below branch on it uniformly (a
  // vector index made each group an exec-masked branch, serialising the groups)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t nibm = opaque_vgpr(kNibHi);         // (w & nibm) | one: one v_and_or_b32
  const int n = lane & 15, q = lane >> 4;
  const int nblk = (O + kQR - 1) / kQR;

  // a block's scales and biases: thread t < 16 G / 8 loads 8 consecutive (row, group)
  // entries of each (the rows of a block are contiguous in [O][G])
  auto load_sc = [&](int blk_, uint4& sv, uint4& bv) {
    const int lim = min(kQR, O - blk_ * kQR) * G / 8;
    const int t = min(tid, lim - 1);
    sv = reinterpret_cast<const uint4*>(a.s + (size_t)blk_ * kQR * G)[t];
    bv = reinterpret_cast<const uint4*>(a.bq + (size_t)blk_ * kQR * G)[t];
  };
  auto store_sc = [&](int par, int blk_, const uint4& sv, const uint4& bv) {
    const int lim = min(kQR, O - blk_ * kQR) * G / 8;
    if (tid < lim) {
      const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w}, bw[4] = {bv.x, bv.y, bv.z, bv.w};
      uint32_t* dst = sbl + par * kQR * G;
      int r = (8 * tid) / G, g = 8 * tid - r * G;      // entry 8 tid + c: row r, group g
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t sh = (c & 1) ? 16 : 0;
        dst[g * kQR + r] = ((sw[c >> 1] >> sh) & 0xFFFFu) | (((bw[c >> 1] >> sh) & 0xFFFFu) << 16);
        if (++g == G) { g = 0; ++r; }
      }
    }
  };
  // a block's weight words for this lane (groups past the row re-read the last group)
  struct Wq {
    uint2 w[kGW];
  };
  auto load_w = [&](int blk_, Wq& wb) {
    const int row = min(blk_ * kQR + n, O - 1);
    const uint32_t* wr = reinterpret_cast<const uint32_t*>(a.w) + (size_t)row * (I / 8) + 4 * (q >> 1) + 2 * (q & 1);
#pragma unroll
    for (int it = 0; it < kGW; ++it) wb.w[it] = *reinterpret_cast<const uint2*>(wr + 8 * min(wave + 4 * it, G - 1));
  };

  // ---- prologue: scales of the first block, x, the first block's weights
  int blk = blockIdx.x;
  uint4 sv, bv;
  load_sc(blk, sv, bv);
  XIn<HSD_W_Q4, NB, XK, XIT, PX> xin;
  xin.load(a, tid);
  Wq cur;
  load_w(blk, cur);
  store_sc(0, blk, sv, bv);
  xin.template finish<64>(a, xp, xg, wsum, tid, lane, wave);
  lds_barrier();                                       // x and scales in LDS; weights may be in flight

  uint64_t best = 0;                                   // wavefront 0, lanes of token row l / 16
  const int arow = min(n, NB - 1);                     // the token row of this lane's A operand
  // one block: the wavefront's groups (two chains), their partial sums to LDS, then
  // wavefront 0 adds the eight partials and runs the epilogue. With next_sc, the next
  // block's scales go to the other LDS parity before the barrier (their last readers were
  // the previous block's).
  auto do_block = [&](int blk_, const Wq& wb, int par, bool next_sc, int nblk_, const uint4& nsv,
                      const uint4& nbv) {
    // two chains per wavefront: the even group slots (groups wave + 8 k) and the odd ones
    // (wave + 4 + 8 k), so that the 8 partials and their order are those of the 8-wavefront
    // LDS ring below (one chain per wavefront there)
    float y[2][NB];
#pragma unroll
    for (int r = 0; r < NB; ++r) y[0][r] = y[1][r] = 0.0f;
    const uint32_t* sb = sbl + par * kQR * G;
    // a group slot's x words (the lane's token row, 2 x 16 bytes), read for the next slot
    // before the current slot's arithmetic so the LDS latency is off the chain of groups
    auto ldx = [&](int it, uint4& xa0, uint4& xa1) {
      const int p = 2 * min(wave + 4 * it, G - 1) + (q >> 1);
      xa0 = *reinterpret_cast<const uint4*>(&xp[arow * 16 * PX + 4 * ((2 * (q & 1) + 0) * PX + p)]);
      xa1 = *reinterpret_cast<const uint4*>(&xp[arow * 16 * PX + 4 * ((2 * (q & 1) + 1) * PX + p)]);
    };
    uint4 xa0n, xa1n;
    ldx(0, xa0n, xa1n);
    // the first 8 group slots unconditionally (a group past G re-reads group G - 1 and adds
    // nothing: a select, not a branch), so their LDS reads, unpacking and MFMAs interleave;
    // the slots after them stop at the row's last group (a uniform branch)
#pragma unroll
    for (int it = 0; it < kGW; ++it) {
      if (it >= 8 && wave + 4 * it >= G) break;
      const int g0 = wave + 4 * it, g = min(g0, G - 1);
      const uint4 xa0 = xa0n, xa1 = xa1n;
      if (it + 1 < kGW) ldx(it + 1, xa0n, xa1n);
      floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t qw = i ? wb.w[it].y : wb.w[it].x;
        const uint4 wq = make_uint4(((qw << 3) & nibm) | kBfOne2, ((qw >> 1) & nibm) | kBfOne2,
                                    ((qw >> 5) & nibm) | kBfOne2, ((qw >> 9) & nibm) | kBfOne2);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, i ? xa1 : xa0),
                                                      __builtin_bit_cast(bf16x8, wq), acc, 0, 0, 0);
      }
      const uint32_t sq = sb[g * kQR + n];
      const float sv_ = lo_f(sq), bv_ = hi_f(sq);
      const float s16 = 16.0f * sv_, bo = fmaf(-16.0f, sv_, bv_);
#pragma unroll
      for (int r = 0; r < NB; ++r) {
        const float yn = y[it & 1][r] + fmaf(s16, acc[r], bo * xg[r * (PX / 2) + g]);
        y[it & 1][r] = g0 < G ? yn : y[it & 1][r];
      }
    }
    // lanes 0..15 hold token rows 0..3 of output row n (acc[r]: token row 4 (l / 16) + r)
    if (q == 0) {
#pragma unroll
      for (int r = 0; r < NB; ++r) {
        red[par][wave][r][n] = y[0][r];
        red[par][wave + 4][r][n] = y[1][r];
      }
    }
    if (next_sc) store_sc(par ^ 1, nblk_, nsv, nbv);
    // LDS only: the next block's weights stay in flight across the barrier (53.9 against
    // 54.1 us at three token rows with __syncthreads, which waits for them)
    lds_barrier();
    if (wave == 0) {
      const int m = q;                                 // token row of this lane
      const int o = blk_ * kQR + n;
      const bool live = m < NB && o < O;
      const int mm = min(m, NB - 1);
      float v = red[par][0][mm][n];
#pragma unroll
      for (int c = 1; c < 8; ++c) v += red[par][c][mm][n];
      if constexpr (YK == HSD_Y_ARGMAX) {
        const uint16_t lb = f32_to_bf16_bits(v);
        uint64_t key = live ? argmax_key(lb, o) : 0;
        if (a.y && live) reinterpret_cast<uint16_t*>(a.y)[m * a.y_ld + o] = lb;
        key = row16_max_u64(key);                      // the best of the 16 lanes of token row m
        best = key > best ? key : best;
      } else if (live) {
        const int64_t yi = m * a.y_ld + o;
        if constexpr (YK == HSD_Y_F32) {
          reinterpret_cast<float*>(a.y)[yi] = v;
        } else if constexpr (YK == HSD_Y_RESID) {
          const float rv = bf16_bits_to_f32(a.res[m * a.res_ld + o]);
          reinterpret_cast<uint16_t*>(a.y)[yi] = f32_to_bf16_bits(rv + rne_bf16(v));
        } else {
          reinterpret_cast<uint16_t*>(a.y)[yi] = f32_to_bf16_bits(v);
        }
      }
    }
  };

  if ((int)gridDim.x >= nblk) {
    do_block(blk, cur, 0, false, blk, sv, bv);         // one block per workgroup
  } else {
    // several blocks: the next block's scales and weights are in flight while one is
    // computed (issued unconditionally: the last block re-reads its own lines)
    int par = 0;
    for (;;) {
      const int nxt = blk + (int)gridDim.x;
      const int nb = nxt < nblk ? nxt : blk;
      uint4 nsv, nbv;
      load_sc(nb, nsv, nbv);
      Wq nx;
      load_w(nb, nx);
      do_block(blk, cur, par, nxt < nblk, nb, nsv, nbv);
      if (nxt >= nblk) break;
      blk = nxt;
      cur = nx;
      par ^= 1;
    }
  }
  if constexpr (YK == HSD_Y_ARGMAX) {
    if (wave == 0 && n == 0 && q < NB) {
      a.keys[q * a.key_ld + blockIdx.x] = best;
      // slots past the grid (the grid follows the occupancy) read as the smallest key
      for (int sl = blockIdx.x + gridDim.x; sl < a.key_slots; sl += gridDim.x) a.keys[q * a.key_ld + sl] = 0;
    }
  }
}

// lm_head at NB = 1 or 3 token rows (argmax keys, no logits written): k_linear_q4's
// arithmetic with the weights streamed into LDS instead of registers. A workgroup of 8
// wavefronts keeps a ring of 2 blocks in flight (direct global-to-LDS loads, no registers
// held), where the register form holds one: 2 workgroups per CU (LDS: 2 x 24 KB + x), so 4
// wavefronts per SIMD hide the latency of the group arithmetic (4 wavefronts and 3 slots
// took 41.5 against 40.2 us per call at one row; 8 wavefronts and 3 slots 41.2). Each ring
// slot holds a block's 16 weight rows (a 16-byte pad after each, so the 16 rows of a read
// fall in different banks), then its scales and biases, 24 loads of 1 KB (3 per wavefront:
// every wavefront waits on the same counts). Wavefront w adds the groups w, w + 8, ... of a
// block; the 8 partials are summed in wavefront order. k_linear_q4 keeps the same 8 chains
// (two per wavefront), so a row's bf16 logits (and argmax) are bit-identical to that
// kernel's for any number of token rows.
constexpr int kRingI = 2688;             // inputs per row the ring is sized for (the hidden size)
constexpr int kRingW = 8;                // wavefronts per ring workgroup
constexpr int kRingSlots1 = 2;           // ring slots at one token row (three at three rows do not fit)
constexpr int kRingChunks = 1536;        // 16-byte chunks per slot: 16 (I/32 + 1) + 2 I/32 <= 1536
static_assert(16 * (kRingI / 32 + 1) + 2 * (kRingI / 32) <= kRingChunks && kRingChunks % 256 == 0, "ring slot");
typedef __attribute__((address_space(3))) void lds_void_t;

template <int XK, int NB, int kRW>
__global__ __launch_bounds__(64 * kRW, 2) void k_lm_ring(HSD_LIN_PARAMS) {
  HSD_LIN_UNPACK;
  constexpr int IMAX = kRingI, PX = IMAX / 32;
  constexpr int kGW = (IMAX / 64 + kRW - 1) / kRW;     // groups per wavefront (max)
  constexpr int XIT = (IMAX / 8 + kLT - 1) / kLT;
  constexpr int kSlots = NB == 1 ? kRingSlots1 : 2;  // ring slots
  constexpr int kPW = kRingChunks / 64 / kRW;          // 1-KB loads per wavefront and block
  static_assert(NB == 1 || NB == 3, "ring instances: one row (decode) and three (verify)");
  // wavefronts 4-7 meet the x prologue's one barrier with a barrier of their own: the RMS
  // prologue has exactly one (the other prologues have none or more)
  static_assert(XK == HSD_X_RMS && (kRW == 4 || kRW == 8), "ring instances: the RMS prologue, 4 or 8 wavefronts");
  __shared__ __attribute__((aligned(16))) uint4 ring[kSlots][kRingChunks];
  __shared__ __attribute__((aligned(16))) uint32_t xp[NB * 16 * PX];
  __shared__ float xg[NB * (PX / 2)];
  __shared__ float wsum[NB][4];
  __shared__ float red[2][kRW][NB][kQR];               // [block parity][wavefront][token row][row]
  const int I = a.I, O = a.O, G = I / 64, NPr = I / 32, rowc = NPr + 1;
  // the wavefront index as a scalar: the group loops below branch on it uniformly (a
  // vector index made each group an exec-masked branch, serialising the groups)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t nibm = opaque_vgpr(kNibHi);         // (w & nibm) | one: one v_and_or_b32
  const int n = lane & 15, q = lane >> 4;
  const int nblk = (O + kQR - 1) / kQR;
  const int nmine = nblk > (int)blockIdx.x ? (nblk - 1 - (int)blockIdx.x) / grid_ + 1 : 0;
  // this lane's source of each of its ring loads for block k = 0, and the step to block
  // k + 1: chunk c = 64 i + lane of a slot takes weight row c / rowc, chunk c % rowc (the pad
  // chunk re-reads the row's last), then the block's scales, then its biases; chunks past
  // those re-read the last bias chunk (O % 16 == 0: no row past O)
  const char* src[kPW];
  uint32_t step[kPW];
#pragma unroll
  for (int j = 0; j < kPW; ++j) {
    const int c = 64 * (wave + kRW * j) + lane;
    if (c < 16 * rowc) {
      const int r = c / rowc, ch = min(c - r * rowc, NPr - 1);
      src[j] = reinterpret_cast<const char*>(a.w) + (size_t)((int)blockIdx.x * kQR + r) * (I / 2) + 16 * ch;
      step[j] = (uint32_t)grid_ * 8u * (uint32_t)I;
    } else {
      const int k2 = c - 16 * rowc;
      const bool isb = k2 >= NPr;
      src[j] = reinterpret_cast<const char*>(isb ? a.bq : a.s) + (size_t)blockIdx.x * kQR * G * 2 +
               16 * min(isb ? k2 - NPr : k2, NPr - 1);
      step[j] = (uint32_t)grid_ * 32u * (uint32_t)G;
    }
  }
  const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
  // the next block of this workgroup into a slot: 1-KB direct loads (M0 = the LDS address of
  // the wavefront's 1 KB, one wait state before the load uses it); a block past the last
  // re-reads the last. The loads are issued by inline assembly so that the ring's reads wait
  // only on the explicit counts below (the compiler's own count would wait for every load in
  // flight before any LDS read). M0 is listed as clobbered; it is a reserved register, which
  // the compiler only sets right before its own M0 users, and this kernel's generated code
  // has none besides these loads (checked in its gfx950 assembly).
  auto issue = [&](int k, uint4* slot) {
    const uint32_t base = (uint32_t)(uintptr_t)(lds_void_t*)slot;
#pragma unroll
    for (int j = 0; j < kPW; ++j) {
      const uint32_t m0 = base + 1024u * (wv + (uint32_t)kRW * j);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(src[j])
                   : "memory", "m0");
#pragma clang diagnostic pop
      if (k + 1 < nmine) src[j] += step[j];
    }
  };

  // ---- prologue: x, the first blocks (one per slot), x into LDS
  // (the x prologue is written for 256 threads: with 8 wavefronts, wavefronts 4-7 only
  // meet its barrier)
  XIn<HSD_W_Q4, NB, XK, XIT, PX> xin;
  if (kRW == 4 || wave < 4) xin.load(a, tid);
#pragma unroll
  for (int k = 0; k < kSlots; ++k) issue(k, ring[k]);
  if (kRW == 4 || wave < 4)
    xin.template finish<64>(a, xp, xg, wsum, tid, lane, wave);
  else
    lds_barrier();

  uint64_t best = 0;                                   // lanes of token row l / 16
  const int arow = min(n, NB - 1);                     // the token row of this lane's A operand
  // block k from a slot: the wavefront's groups, its partial sums into red[k & 1]
  auto compute = [&](int k, const uint4* slot) {
    const char* sl = reinterpret_cast<const char*>(slot);
    const uint16_t* ss = reinterpret_cast<const uint16_t*>(sl + 16 * 16 * rowc);
    const uint16_t* sbb = ss + 8 * NPr;
    float y[NB];
#pragma unroll
    for (int r = 0; r < NB; ++r) y[r] = 0.0f;
    // a group slot's LDS words (its 8 weight bytes and the 2 x 16 bytes of x they meet); the
    // next slot's are read before the current slot's arithmetic, so the LDS latency is not
    // on the chain of one group after another
    auto ld = [&](int it, uint2& w2, uint4& xa0, uint4& xa1) {
      const int g = min(wave + kRW * it, G - 1);
      const int p = 2 * g + (q >> 1);
      w2 = *reinterpret_cast<const uint2*>(sl + 16 * (n * rowc + p) + 8 * (q & 1));
      xa0 = *reinterpret_cast<const uint4*>(&xp[arow * 16 * PX + 4 * ((2 * (q & 1) + 0) * PX + p)]);
      xa1 = *reinterpret_cast<const uint4*>(&xp[arow * 16 * PX + 4 * ((2 * (q & 1) + 1) * PX + p)]);
    };
    uint2 w2n;
    uint4 xa0n, xa1n;
    ld(0, w2n, xa0n, xa1n);
    // every group slot (a slot past G re-reads group G - 1 and adds nothing: a select, not a
    // branch); the sum over the wavefront's groups keeps its order
#pragma unroll
    for (int it = 0; it < kGW; ++it) {
      const int g0 = wave + kRW * it, g = min(g0, G - 1);
      const uint2 w2 = w2n;
      const uint4 xa0 = xa0n, xa1 = xa1n;
      if (it + 1 < kGW) ld(it + 1, w2n, xa0n, xa1n);
      floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t qw = i ? w2.y : w2.x;
        const uint4 wq = make_uint4(((qw << 3) & nibm) | kBfOne2, ((qw >> 1) & nibm) | kBfOne2,
                                    ((qw >> 5) & nibm) | kBfOne2, ((qw >> 9) & nibm) | kBfOne2);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, i ? xa1 : xa0),
                                                      __builtin_bit_cast(bf16x8, wq), acc, 0, 0, 0);
      }
      const float sv_ = bf16_bits_to_f32(ss[n * G + g]), bv_ = bf16_bits_to_f32(sbb[n * G + g]);
      const float s16 = 16.0f * sv_, bo = fmaf(-16.0f, sv_, bv_);
#pragma unroll
      for (int r = 0; r < NB; ++r) {
        const float yn = y[r] + fmaf(s16, acc[r], bo * xg[r * (PX / 2) + g]);
        y[r] = g0 < G ? yn : y[r];
      }
    }
    // lanes 0..15 hold token rows 0..3 of output row n (acc[r]: token row 4 (l / 16) + r)
    if (q == 0) {
#pragma unroll
      for (int r = 0; r < NB; ++r) red[k & 1][wave][r][n] = y[r];
    }
  };
  // after block k's barrier: wavefront k % 8 adds the 8 partials of each row and keeps the
  // best key, while the others go on to block k + 1 (which writes red[(k + 1) & 1]); taking
  // turns keeps one wavefront from running behind the others at every block's barrier
  auto epilogue = [&](int k) {
    if (wave == k % kRW) {                              // the wavefronts take turns
      const int o = ((int)blockIdx.x + k * grid_) * kQR + n;
      const int m = min(q, NB - 1);                      // token row of this lane
      const bool live = q < NB && o < O;
      float v = red[k & 1][0][m][n];
#pragma unroll
      for (int w = 1; w < kRW; ++w) v += red[k & 1][w][m][n];
      uint64_t key = live ? argmax_key(f32_to_bf16_bits(v), o) : 0;
      key = row16_max_u64(key);
      best = key > best ? key : best;
    }
  };
  // the end of block k: this wavefront's loads of block k + 1 in (a wavefront's ring loads
  // complete in issue order, 6 per block; with three slots block k + 2's may be outstanding,
  // when it was issued), then one barrier: every wavefront's part of block k + 1 is in, the
  // slot of block k is free and red[k & 1] complete
  auto end_block = [&](int k) {
    if (kSlots == 3 && (k + 2 <= 2 || k + 2 < nmine)) __builtin_amdgcn_s_waitcnt(0x0F70 | kPW);  // vmcnt(kPW)
    else __builtin_amdgcn_s_waitcnt(0x0F70);                                             // vmcnt(0)
    lds_barrier();
  };
  static_assert(2 * kPW < 16, "vmcnt immediates below");
  if constexpr (kSlots == 3)
    __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * kPW));    // vmcnt(2 kPW): block 0 in
  else
    __builtin_amdgcn_s_waitcnt(0x0F70 | kPW);          // vmcnt(kPW): block 0 in
  lds_barrier();                                       // x and block 0 in LDS
  for (int k = 0; k < nmine; k += kSlots) {
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      if (i > 0 && k + i >= nmine) break;
      compute(k + i, ring[i]);
      end_block(k + i);
      if (k + i + kSlots < nmine) issue(k + i + kSlots, ring[i]);
      epilogue(k + i);
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);                  // no ring load outlives the workgroup
  // each wavefront's best key per token row (lane 16 m holds row m's), then their maximum
  __shared__ uint64_t wbest[kRW][NB];
  if (n == 0 && q < NB) wbest[wave][q] = best;
  lds_barrier();
  if (wave == 0 && lane < NB) {
    uint64_t m = wbest[0][lane];
#pragma unroll
    for (int w = 1; w < kRW; ++w) m = wbest[w][lane] > m ? wbest[w][lane] : m;
    a.keys[lane * a.key_ld + blockIdx.x] = m;
    for (int sl2 = (int)blockIdx.x + grid_; sl2 < a.key_slots; sl2 += grid_) a.keys[lane * a.key_ld + sl2] = 0;
  }
}

// tok[b] = the index of the best key of row b (argmax with NaN first, then the larger
// value, then the smaller index). One workgroup per row.
__global__ __launch_bounds__(1024) void k_argmax_keys(const uint64_t* __restrict__ keys, int64_t key_ld,
                                                      int slots, int32_t* __restrict__ tok) {
  __shared__ uint64_t wbest[16];
  const int b = blockIdx.x;
  uint64_t k = 0;
  for (int i = threadIdx.x; i < slots; i += 1024) {
    const uint64_t v = keys[b * key_ld + i];
    k = v > k ? v : k;
  }
  k = wave_max_u64(k);
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = k;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t m = wbest[0];
    for (int w = 1; w < 16; ++w) m = wbest[w] > m ? wbest[w] : m;
    tok[b] = (int32_t)~(uint32_t)m;
  }
}

// Output rows per wavefront: 4 for 4-bit weights (an x piece read from LDS serves 4 rows),
// 1 for bf16. Two rows per wavefront for the shorter projections (more workgroups: 336
// rather than 168 for out_proj) measured slower for out_proj (6.3 against 5.9 us at one
// token row, 10.6 against 9.8 at three) and the decode step as a whole.
int rows_per_wave(int O, int w_kind) { (void)O; return w_kind == HSD_W_Q4 ? 4 : 1; }

int linear_grid(int O, int w_kind) {
  const int rows = 4 * rows_per_wave(O, w_kind);
  return std::min((O + rows - 1) / rows, kLMaxGrid);
}


// The checks and the launch of hsd_linear.
int launch_linear(const char* fn, const void* x, int64_t x_ld, int x_kind, const uint16_t* gate, int64_t gate_ld,
                  const uint16_t* norm_w, float eps, const void* w, const uint16_t* scales, const uint16_t* biases,
                  int w_kind, void* y, int64_t y_ld, int y_kind, const uint16_t* res, int64_t res_ld,
                  uint16_t* xn_out, int64_t xn_ld, uint64_t* argmax_keys, int64_t key_ld, int64_t B, int64_t O,
                  int64_t I, void* stream) {
  if (!x || !w || (y_kind != HSD_Y_ARGMAX && !y)) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (w_kind == HSD_W_Q4 && (!scales || !biases)) return set_error(HSD_ERR_ARG, "%s: 4-bit weights need scales and biases", fn);
  if (w_kind != HSD_W_Q4 && w_kind != HSD_W_BF16) return set_error(HSD_ERR_DTYPE, "%s: w_kind %d", fn, w_kind);
  if (x_kind != HSD_X_BF16 && x_kind != HSD_X_RMS && x_kind != HSD_X_GATED && x_kind != HSD_X_GATED_Z)
    return set_error(HSD_ERR_DTYPE, "%s: x_kind %d", fn, x_kind);
  if (y_kind < HSD_Y_BF16 || y_kind > HSD_Y_ARGMAX) return set_error(HSD_ERR_DTYPE, "%s: y_kind %d", fn, y_kind);
  if (x_kind != HSD_X_BF16 && !norm_w) return set_error(HSD_ERR_ARG, "%s: the normalisation needs norm_w", fn);
  if (x_kind == HSD_X_GATED && !gate) return set_error(HSD_ERR_ARG, "%s: the gated norm needs the gate", fn);
  if (y_kind == HSD_Y_RESID && !res) return set_error(HSD_ERR_ARG, "%s: the residual epilogue needs res", fn);
  if (y_kind == HSD_Y_ARGMAX && !argmax_keys) return set_error(HSD_ERR_ARG, "%s: argmax needs the key buffer", fn);
  const int rows = w_kind == HSD_W_Q4 ? 8 : 4;
  if (B < 0 || B > kLMaxB) return set_error(HSD_ERR_SHAPE, "%s: B must be in [0, %d]", fn, kLMaxB);
  if (O <= 0 || O % rows || O > (1 << 28))
    return set_error(HSD_ERR_SHAPE, "%s: O must be a positive multiple of %d", fn, rows);
  // 4-bit rows up to 4096 inputs (every 4-bit projection of the model; the register arrays
  // of longer rows spill), bf16 rows up to 6144 (the MTP head's eh_proj: 5376)
  const int imax = w_kind == HSD_W_Q4 ? kLSmallQ4 : kLMaxI;
  if (I <= 0 || I > imax || I % (w_kind == HSD_W_Q4 ? 64 : 8))
    return set_error(HSD_ERR_SHAPE, "%s: I must be a multiple of %d and at most %d", fn,
                     w_kind == HSD_W_Q4 ? 64 : 8, imax);
  const bool gated = x_kind == HSD_X_GATED || x_kind == HSD_X_GATED_Z;
  if (gated && I % 512) return set_error(HSD_ERR_SHAPE, "%s: the gated norm needs I %% 512 == 0", fn);
  if (x_kind == HSD_X_GATED_Z && x_ld < I + I / 16)
    return set_error(HSD_ERR_SHAPE, "%s: HSD_X_GATED_Z rows hold I + I/16 values (x_ld >= %lld)", fn,
                     (long long)(I + I / 16));
  const int64_t xe = gated ? 4 : 2;                   // x element bytes
  if (x_ld > 0x7FFFFFFF) return set_error(HSD_ERR_SHAPE, "%s: x_ld must be below 2^31", fn);
  if (x_ld < I || (x_ld * xe) % 16 || ((uintptr_t)x & 15u) || (norm_w && ((uintptr_t)norm_w & 15u)) ||
      ((uintptr_t)w & 15u) || (gate && (((uintptr_t)gate & 15u) || gate_ld % 8 || gate_ld < I)) ||
      (xn_out && (((uintptr_t)xn_out & 15u) || xn_ld % 8 || xn_ld < I)))
    return set_error(HSD_ERR_ALIGN, "%s: x, gate, norm_w, w and xn_out must be 16-byte aligned with row "
                     "strides of whole 16-byte pieces", fn);
  if (y_kind != HSD_Y_ARGMAX && y_ld < O) return set_error(HSD_ERR_SHAPE, "%s: y_ld < O", fn);
  if (y_kind == HSD_Y_RESID && res_ld < O) return set_error(HSD_ERR_SHAPE, "%s: res_ld < O", fn);
  const int slots = linear_grid((int)O, w_kind);     // argmax key slots (an upper bound of the grid)
  if (y_kind == HSD_Y_ARGMAX && key_ld < slots)
    return set_error(HSD_ERR_SHAPE, "%s: key_ld must be >= hsd_linear_argmax_slots() = %d", fn, slots);
  if (B == 0) return HSD_OK;
  LinArgs a{x, x_ld, gate, gate_ld, norm_w, eps, w, scales, biases, y, y_ld, res, res_ld, xn_out, xn_ld,
            argmax_keys, key_ld, slots, (int)O, (int)I};
  const size_t lds = (size_t)B * (I / 2) * 4;          // bf16 weights (4-bit: per instance below)
  // 4-bit projections of more 16-row blocks than one grid (lm_head) take the MFMA kernel;
  // the choice depends on O only, so a token row is computed the same way at any B
  const bool mfma = w_kind == HSD_W_Q4 && (O + kQR - 1) / kQR > kLMaxGrid;
  if (mfma && (((uintptr_t)scales & 15u) || ((uintptr_t)biases & 15u)))
    return set_error(HSD_ERR_ALIGN, "%s: scales and biases must be 16-byte aligned", fn);
  hipStream_t st = as_stream(stream);
  // IMAX 3072, then 4096 for 4-bit rows and 6144 for bf16 rows (bf16: pieces left over
  // after full passes dealt as pairs). A 4-bit row's pieces, their order and its sums do not
  // depend on IMAX.
  const int isz = I <= 3072 ? 0 : 1;
  const int grid = slots;
  // the (x_kind, y_kind) pairs this library instantiates
  const int pair = x_kind * 8 + y_kind;
  constexpr int kRB = HSD_X_RMS * 8 + HSD_Y_BF16, kRA = HSD_X_RMS * 8 + HSD_Y_ARGMAX,
                kRF = HSD_X_RMS * 8 + HSD_Y_F32, kGR = HSD_X_GATED * 8 + HSD_Y_RESID,
                kZR = HSD_X_GATED_Z * 8 + HSD_Y_RESID,
                kBR = HSD_X_BF16 * 8 + HSD_Y_RESID, kBB = HSD_X_BF16 * 8 + HSD_Y_BF16;
  // one token row of a 4-bit projection with a bf16 or residual output and fewer than 512
  // 16-row blocks (out_proj, o_proj, q|k|v; not in_proj's 644): 2 rows per wavefront (one
  // per half-wavefront), twice the workgroups. A row's pieces, their order and its 32-lane
  // sum are those of 4 rows per wavefront, so its bits do not depend on the choice
  // (out_proj and o_proj: the decode step 1.054 -> 1.050 ms; q|k|v too: the MTP-2 step
  // 1.894 -> 1.889 ms; in_proj too: the decode step slower, 1.062 against 1.058 ms; at
  // three token rows the MTP-2 step was slower, 1.905 against 1.899 ms)
  const bool rw2 = w_kind == HSD_W_Q4 && !mfma && B == 1 && (y_kind == HSD_Y_RESID || y_kind == HSD_Y_BF16) &&
                   (O + 15) / 16 < 512;
  const bool ok = w_kind == HSD_W_Q4 ? (pair == kRB || pair == kRA || pair == kRF || pair == kGR ||
                                        pair == kZR || pair == kBR || pair == kBB)
                                     : (pair == kRB || pair == kBB);
  if (!ok)
    return set_error(HSD_ERR_SHAPE, "%s: unsupported combination x_kind %d, y_kind %d, w_kind %d", fn, x_kind,
                     y_kind, w_kind);
#define HSD_LIN_R(WF, NB, XK, YK, IM, RW)                                                             \
  {                                                                                                   \
    constexpr bool REM = !(WF == HSD_W_Q4 && IM == kLSmallQ4);                                        \
    const void* kf = reinterpret_cast<const void*>(&k_linear<WF, NB, XK, YK, IM, RW, REM>);          \
    const size_t ldsx = WF == HSD_W_Q4 ? (size_t)B * 17 * (IM / 32) * 4 : lds;                        \
    const int gr = RW == 2 ? std::min((int)((O + 7) / 8), kLMaxGrid) : grid;                          \
    const int g = std::max(1, std::min(gr, resident_workgroups(kf, kLT, ldsx, kLMaxGrid)));           \
    hipLaunchKernelGGL((k_linear<WF, NB, XK, YK, IM, RW, REM>), dim3(g), dim3(kLT), ldsx, st,        \
                       HSD_LIN_ARGS(a, g));                                                       \
  }
#define HSD_LIN(WF, NB, XK, YK, IM)                                   \
  {                                                                   \
    if constexpr (WF == HSD_W_Q4 && NB == 1 && (YK == HSD_Y_RESID || YK == HSD_Y_BF16)) { \
      if (rw2) HSD_LIN_R(WF, NB, XK, YK, IM, 2)                       \
      else HSD_LIN_R(WF, NB, XK, YK, IM, 4)                           \
    } else if constexpr (WF == HSD_W_Q4) {                            \
      HSD_LIN_R(WF, NB, XK, YK, IM, 4)                                \
    } else {                                                          \
      HSD_LIN_R(WF, NB, XK, YK, IM, 1)                                \
    }                                                                 \
  }
  // several token rows of a residual projection with few blocks (out_proj, o_proj: 168
  // 16-row blocks): the one-row instance over (2-row wavefront blocks, token rows), three
  // times the workgroups of the three-row instance, each doing a third of the arithmetic
  const bool rows1 = w_kind == HSD_W_Q4 && !mfma && B > 1 && y_kind == HSD_Y_RESID && (O + 15) / 16 < 256 &&
                     !xn_out;
#define HSD_LIN_Y(XK, IM)                                                                             \
  {                                                                                                   \
    constexpr bool REM = IM != kLSmallQ4;                                                            \
    const void* kf = reinterpret_cast<const void*>(&k_linear<HSD_W_Q4, 1, XK, HSD_Y_RESID, IM, 2, REM, true>); \
    const size_t ldsx = (size_t)17 * (IM / 32) * 4;                                                   \
    const int gr = std::min((int)((O + 7) / 8), kLMaxGrid);                                           \
    const int g = std::max(1, std::min(gr, resident_workgroups(kf, kLT, ldsx, kLMaxGrid)));          \
    hipLaunchKernelGGL((k_linear<HSD_W_Q4, 1, XK, HSD_Y_RESID, IM, 2, REM, true>), dim3(g, (unsigned)B), \
                       dim3(kLT), ldsx, st, HSD_LIN_ARGS(a, g));                                      \
  }
#define HSD_LIN_I(WF, NB, XK, YK)                                       \
  if (isz == 0) HSD_LIN(WF, NB, XK, YK, 3072)                           \
  else if constexpr (WF == HSD_W_Q4) HSD_LIN(WF, NB, XK, YK, kLSmallQ4) \
  else HSD_LIN(WF, NB, XK, YK, kLMaxI)
#define HSD_LIN_P(WF, NB)                                                  \
  switch (pair) {                                                          \
    case kRB: HSD_LIN_I(WF, NB, HSD_X_RMS, HSD_Y_BF16); break;             \
    case kBB: HSD_LIN_I(WF, NB, HSD_X_BF16, HSD_Y_BF16); break;            \
    default:                                                               \
      if constexpr (WF == HSD_W_Q4) {                                      \
        switch (pair) {                                                    \
          case kRA: HSD_LIN_I(WF, NB, HSD_X_RMS, HSD_Y_ARGMAX); break;      \
          case kRF: HSD_LIN_I(WF, NB, HSD_X_RMS, HSD_Y_F32); break;         \
          case kGR: HSD_LIN_I(WF, NB, HSD_X_GATED, HSD_Y_RESID); break;     \
          case kZR: HSD_LIN_I(WF, NB, HSD_X_GATED_Z, HSD_Y_RESID); break;   \
          default: HSD_LIN_I(WF, NB, HSD_X_BF16, HSD_Y_RESID); break;      \
        }                                                                  \
      }                                                                    \
  }
#define HSD_LIN_B(WF)                        \
  switch (B) {                               \
    case 1: HSD_LIN_P(WF, 1); break;         \
    case 2: HSD_LIN_P(WF, 2); break;         \
    case 3: HSD_LIN_P(WF, 3); break;         \
    default: HSD_LIN_P(WF, 4); break;        \
  }
#define HSD_Q4_R(NB, XK, YK, IM)                                                                  \
  {                                                                                               \
    const void* kf = reinterpret_cast<const void*>(&k_linear_q4<NB, XK, YK, IM>);                 \
    const size_t ldsq = (size_t)NB * (16 * (IM / 32) + IM / 64) * 4 + (size_t)2 * kQR * (I / 64) * 4; \
    const int g = std::max(1, std::min(grid, resident_workgroups(kf, kLT, ldsq, kLMaxGrid)));     \
    hipLaunchKernelGGL((k_linear_q4<NB, XK, YK, IM>), dim3(g), dim3(kLT), ldsq, st, HSD_LIN_ARGS(a, g)); \
  }
#define HSD_Q4_I(NB, XK, YK)                                    \
  if (I <= 3072) HSD_Q4_R(NB, XK, YK, 3072)                     \
  else HSD_Q4_R(NB, XK, YK, kLSmallQ4)
#define HSD_Q4_P(NB)                                                   \
  switch (pair) {                                                      \
    case kRB: HSD_Q4_I(NB, HSD_X_RMS, HSD_Y_BF16); break;              \
    case kBB: HSD_Q4_I(NB, HSD_X_BF16, HSD_Y_BF16); break;             \
    case kRA: HSD_Q4_I(NB, HSD_X_RMS, HSD_Y_ARGMAX); break;            \
    case kRF: HSD_Q4_I(NB, HSD_X_RMS, HSD_Y_F32); break;               \
    case kGR: HSD_Q4_I(NB, HSD_X_GATED, HSD_Y_RESID); break;           \
    case kZR: HSD_Q4_I(NB, HSD_X_GATED_Z, HSD_Y_RESID); break;         \
    default: HSD_Q4_I(NB, HSD_X_BF16, HSD_Y_RESID); break;             \
  }
  // one or three token rows of argmax keys with no logits (the decode and verify steps'
  // lm_head): the LDS ring
  const bool ring = mfma && (B == 1 || B == 3) && pair == kRA && !y && I <= kRingI && O % kQR == 0;
  if (ring) {
#define HSD_RING(NB)                                                                          \
  {                                                                                           \
    const void* kf = reinterpret_cast<const void*>(&k_lm_ring<HSD_X_RMS, NB, kRingW>);        \
    const int g = std::max(1, std::min(grid, resident_workgroups(kf, 64 * kRingW, 0, kLMaxGrid))); \
    hipLaunchKernelGGL((k_lm_ring<HSD_X_RMS, NB, kRingW>), dim3(g), dim3(64 * kRingW), 0, st,  \
                       HSD_LIN_ARGS(a, g));                                                   \
  }
    if (B == 1)
      HSD_RING(1)
    else
      HSD_RING(3)
#undef HSD_RING
  } else if (mfma) {
    switch (B) {
      case 1: HSD_Q4_P(1); break;
      case 2: HSD_Q4_P(2); break;
      case 3: HSD_Q4_P(3); break;
      default: HSD_Q4_P(4); break;
    }
  } else if (rows1 && (pair == kZR || pair == kBR)) {
    if (pair == kZR) {
      if (isz == 0) HSD_LIN_Y(HSD_X_GATED_Z, 3072) else HSD_LIN_Y(HSD_X_GATED_Z, kLSmallQ4)
    } else {
      if (isz == 0) HSD_LIN_Y(HSD_X_BF16, 3072) else HSD_LIN_Y(HSD_X_BF16, kLSmallQ4)
    }
  } else if (w_kind == HSD_W_Q4) {
    HSD_LIN_B(HSD_W_Q4);
  } else if (pair == kRB && O <= kRowsMaxO && I <= 3072) {
    // few bf16 rows with the RMS prologue (the router gate): a workgroup per row
#define HSD_ROWS(NB)                                                                              \
  hipLaunchKernelGGL((k_linear_rows<NB, 3072>), dim3((unsigned)O), dim3(kLT), lds, st, HSD_LIN_ARGS(a, O));
    switch (B) {
      case 1: HSD_ROWS(1); break;
      case 2: HSD_ROWS(2); break;
      case 3: HSD_ROWS(3); break;
      default: HSD_ROWS(4); break;
    }
#undef HSD_ROWS
  } else {
    HSD_LIN_B(HSD_W_BF16);
  }
#undef HSD_Q4_P
#undef HSD_Q4_I
#undef HSD_Q4_R
#undef HSD_LIN_B
#undef HSD_LIN_P
#undef HSD_LIN_I
#undef HSD_LIN
#undef HSD_LIN_R
#undef HSD_LIN_Y
  return check_launch(fn);
}

}  // namespace
}  // namespace hsd

using namespace hsd;

extern "C" int64_t hsd_linear_argmax_slots(int64_t O, int w_kind) {
  if (O <= 0 || (w_kind != HSD_W_Q4 && w_kind != HSD_W_BF16)) return 0;
  return linear_grid((int)std::min<int64_t>(O, 1 << 30), w_kind);
}

extern "C" int hsd_linear(const void* x, int64_t x_ld, int x_kind, const uint16_t* gate, int64_t gate_ld,
                          const uint16_t* norm_w, float eps, const void* w, const uint16_t* scales,
                          const uint16_t* biases, int w_kind, void* y, int64_t y_ld, int y_kind,
                          const uint16_t* res, int64_t res_ld, uint16_t* xn_out, int64_t xn_ld,
                          uint64_t* argmax_keys, int64_t key_ld, int64_t B, int64_t O, int64_t I,
                          void* stream) {
  return launch_linear("hsd_linear", x, x_ld, x_kind, gate, gate_ld, norm_w, eps, w, scales, biases, w_kind, y,
                       y_ld, y_kind, res, res_ld, xn_out, xn_ld, argmax_keys, key_ld, B, O, I, stream);
}

extern "C" int hsd_argmax_keys(const uint64_t* keys, int64_t key_ld, int64_t slots, int64_t B, int32_t* tok,
                               void* stream) {
  if (!keys || !tok) return set_error(HSD_ERR_ARG, "hsd_argmax_keys: null pointer");
  if (B < 0 || B > 65535 || slots <= 0 || slots > key_ld || slots > (1 << 30))
    return set_error(HSD_ERR_SHAPE, "hsd_argmax_keys: bad B/slots");
  if (B == 0) return HSD_OK;
  hipLaunchKernelGGL(k_argmax_keys, dim3((unsigned)B), dim3(1024), 0, as_stream(stream), keys, key_ld, (int)slots,
                     tok);
  return check_launch("hsd_argmax_keys");
}
