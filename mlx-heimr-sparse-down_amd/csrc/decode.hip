// The MoE down projection at decode: sparse over the live ReLU^2 neurons on the
// neuron-major layout (hsd/decode.py), plus the dense 4-bit comparator on the stock
// layout.
//
// Split over (D chunk x groups) so that every CU gets an even share of the bytes and of
// the arithmetic, then a fixed-order sum (the reference's partial + reduce structure,
// decode.py:37-144). At the Nemotron-3.5 MoE shape (D=2688, F=1856, FS=3712, top-6 of 128 +
// shared) a token row has 232 64-neuron groups:
//   * k_sparse_down_part: one workgroup = (128-output chunk c, part p of <=8 groups of
//     one slot): 21 x 32 = 672 workgroups per row. 256 threads = 16 teams of 16 lanes;
//     team (j, phase) owns the live rows n of group g0+j with n % 2 == phase; lane l owns
//     weight word 16c+l (8 outputs, a 64-byte piece of every row per team).
//       1. one round trip: the slot's expert id and gain, and the group's 64 activations
//          (4 per lane); the group's 16-byte scale and bias vectors follow as soon as the
//          id is in, overlapping the activations' latency; 4 wave ballots give the live
//          mask and an ascending live-row list in LDS (+-0 dead, NaN live), each entry of
//          a 16-bit activation carrying its bits beside the row index (64 VGPRs, 8
//          wavefronts per SIMD: at three token rows the 2016 workgroups are one round);
//       2. one round trip: the live rows' words (4 B per lane), up to 16 rows per team;
//       3. acc[t] = sum h_i q_{i,t}, hsum = sum h_i (fp32); term = s*acc + b*hsum (the
//          group factorisation of decode.py:125-128);
//       4. terms summed in (group, phase) order, times the slot's gain -> part[b, p, chunk].
//   * k_sum_parts: y[b, o] = sum over the 32 parts in part order.
// Eight groups per workgroup measured fastest: 16 (512 threads) and 32 (1024) were 4 % and
// 6 % slower per call, 4 (128 threads, 63 parts) 6 % slower.
// k_sum_parts runs one wavefront per workgroup (42 per token row at D = 2688): 2.5 %
// faster per call than 256-thread workgroups (11).
// Two row phases per group: one phase (128-thread workgroups) was 0.9 % faster at 90 % zeros
// but needs a second batch of row loads once a group has more than 16 live rows (denser
// activations, the dense-h control); four phases were 17 % slower.
// No atomics, no inter-workgroup signalling: results are bit-reproducible, and a row
// of a B-row call is computed exactly as that row alone.
#include "hsd_common.h"

#include <mutex>

namespace hsd {
namespace {

constexpr int kRS = 2;                   // row phases per group
constexpr int kGPW = 8;                  // groups per workgroup
constexpr int kWPC = 16;                 // weight words per D chunk (one lane each)
constexpr int kThreads = kGPW * kWPC * kRS;
constexpr int kDC = kWPC * 8;            // outputs per D chunk
constexpr int kL1 = kThreads / kDC;      // first-level sub-sums per output
constexpr int kRB = 16;                  // rows per team per batch (a phase has 32 rows)

struct Geom {
  int D, F, FS, topk, E, NR, NW;
  int nchunk;  // D / 128
  int gpr;     // groups per routed expert (F/64)
  int gsh;     // groups of the shared expert (FS/64)
  int ppr;     // parts per routed slot
  int nparts;  // parts per token row
  int nwg;     // workgroups per token row
  int ngt;     // groups per token row (live mask entries)
};

Geom make_geom(int64_t D, int64_t F, int64_t FS, int64_t topk, int64_t E) {
  Geom g;
  g.D = (int)D; g.F = (int)F; g.FS = (int)FS; g.topk = (int)topk; g.E = (int)E;
  g.NR = (int)(topk * F + FS);
  g.NW = (int)(D / 8);
  g.nchunk = (int)(D / kDC);
  g.gpr = (int)(F / 64);
  g.gsh = (int)(FS / 64);
  g.ppr = (g.gpr + kGPW - 1) / kGPW;
  g.nparts = g.topk * g.ppr + (g.gsh + kGPW - 1) / kGPW;
  g.nwg = g.nparts * g.nchunk;
  g.ngt = g.topk * g.gpr + g.gsh;
  return g;
}

__device__ __forceinline__ float lo_bf16(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

// nonzero test on the element's bits: +-0 dead, NaN live
template <int HDT> __device__ __forceinline__ bool live_bits(typename Elem<HDT>::T v);
template <> __device__ __forceinline__ bool live_bits<HSD_DT_BF16>(uint16_t v) { return (v & 0x7FFFu) != 0; }
template <> __device__ __forceinline__ bool live_bits<HSD_DT_F16>(uint16_t v) { return (v & 0x7FFFu) != 0; }
template <> __device__ __forceinline__ bool live_bits<HSD_DT_F32>(float v) { return !(v == 0.0f); }

template <int HDT>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(HDT == HSD_DT_F32 ? 7 : 8, HDT == HSD_DT_F32 ? 7 : 8))) void k_sparse_down_part(
    const typename Elem<HDT>::T* __restrict__ h, const int32_t* __restrict__ sel,
    const float* __restrict__ gains, int nwg_, int nchunk_, int topk_, int ppr_, int gpr_, int gsh_, int nblk_,
    int F_, const uint32_t* __restrict__ pw, const uint16_t* __restrict__ ps, const uint16_t* __restrict__ pb,
    const uint32_t* __restrict__ spw, const uint16_t* __restrict__ sps,
    const uint16_t* __restrict__ spb, float* __restrict__ part, uint64_t* __restrict__ live_out,
    int32_t* __restrict__ status, Geom g_, int dense) {
  // the first round trip's pointers and geometry come as the leading scalar arguments,
  // which the dispatch preloads into SGPRs (the struct is read by scalar loads, which the
  // first loads would wait for). nwg_, nchunk_ and nblk_ are not needed by the (chunk,
  // part, token row) grid; this layout measured 0.07 us per call faster than one that
  // preloads D, E and the part count in their place.
  Geom g = g_;
  g.nwg = nwg_;
  g.nchunk = nchunk_;
  g.topk = topk_;
  g.ppr = ppr_;
  g.gpr = gpr_;
  g.gsh = gsh_;
  g.NR = topk_ * F_ + 64 * gsh_;
  g.F = F_;
  using HT = typename Elem<HDT>::T;
  // Per-team rows padded by 64 bytes, so that the team strides are 16 banks mod 32 and
  // the four teams of a wavefront (16 lanes each) write different LDS banks.
  constexpr int kHP = 64 + 64 / (int)sizeof(HT);
  constexpr int kRedP = 8 * kWPC + 16;
  // 16-bit activations: each list entry carries the row's activation bits beside its index
  // ((bits << 16) | row), so one LDS read per row gives both and a lane holds one register
  // per row instead of two (64 VGPRs: 8 wavefronts per SIMD); fp32: index list + table
  constexpr bool kPack = sizeof(HT) == 2;
  __shared__ HT hs[kPack ? 1 : kGPW * kRS][kHP];    // per team: the group's activations
  __shared__ uint8_t lst[kPack ? 1 : kGPW * kRS][64];  // per team: the group's live rows, ascending
  __shared__ uint32_t lsp[kPack ? kGPW * kRS : 1][64];  // the same with the activation bits
  __shared__ float red[kGPW * kRS][kRedP];          // per team: group terms [t][word]
  __shared__ float sum2[kDC][kL1 + 1];

  // grid (chunk, part, token row): the coordinates need no division (a one-dimensional
  // grid placed on the XCDs by part took 3 divisions ahead of the first loads: one call
  // 7.60 against 7.32 us, three rows 11.06 against 10.39)
  const int c = blockIdx.x, p = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, team = tid >> 4, l = tid & 15;
  const int j = team % kGPW, phase = team / kGPW;   // group slot, row phase
  const bool routed = p < g.topk * g.ppr;
  const int k = routed ? (int)((unsigned)p / (unsigned)g.ppr) : g.topk;
  const int g0 = (routed ? p - k * g.ppr : p - g.topk * g.ppr) * kGPW;
  const int ng = min(kGPW, (routed ? g.gpr : g.gsh) - g0);
  const int grp = g0 + j;
  const bool jv = j < ng;

  // ---- round trip 1: expert id, gain and activations, issued together and never under a
  // branch (a load inside a branch makes the compiler wait for all earlier loads where the
  // paths merge). The id/gain are vector loads (an opaque zero lane offset) so that the
  // activation loads do not wait on them through the scalar-load counter.
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  const int eraw = sel[b * g.topk + (routed ? k : g.topk - 1) + z];  // shared: unused
  const float gain = gains[b * (g.topk + 1) + k + z];
  const int grc = jv ? grp : g0;                     // groups past the end re-read g0, unused
  const uint32_t hoff = (uint32_t)b * (uint32_t)g.NR + (uint32_t)(routed ? k * g.F : g.topk * g.F) +
                        (uint32_t)grc * 64u;
  HT hr4[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) hr4[v] = h[hoff + 16 * v + l];
  __builtin_amdgcn_sched_barrier(0);
  const int e = routed ? eraw : 0;
  const bool ok = !routed || (unsigned)e < (unsigned)g.E;
  // the group's scale and bias vectors depend on the expert id alone: issued as soon as
  // the id is in, while the activations are still on their way
  const int w = c * kWPC + l;
  const size_t es = ok ? (size_t)e : 0;
  const uint16_t* sb = routed ? ps + es * (size_t)g.gpr * g.D : sps;
  const uint16_t* bb = routed ? pb + es * (size_t)g.gpr * g.D : spb;
  const size_t soff = ((size_t)grc * g.D + 8u * (uint32_t)w) * 2u;
  const uint4 sv = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(sb) + soff);
  const uint4 bv = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(bb) + soff);
  __builtin_amdgcn_sched_barrier(0);
  HT hv[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) hv[v] = jv ? hr4[v] : (HT)0;

  // ---- live mask (4 ballots over the wave's 4 teams) and the compacted row list
  const int sh = 16 * (team & 3);
  int cnt = 0;
  uint64_t live = 0;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const bool nz = ok && jv && live_bits<HDT>(hv[v]);
    // a team walks the rows n = 16v + l with n % kRS == phase: the phase of a row depends
    // on the row alone, so the dense control sums in the same grouping and order
    const bool use = jv && (dense ? ok : nz) && (l % kRS) == phase;
    const uint32_t mnz = (uint32_t)(__ballot(nz) >> sh) & 0xFFFFu;
    const uint32_t muse = (uint32_t)(__ballot(use) >> sh) & 0xFFFFu;
    live |= (uint64_t)mnz << (16 * v);
    const int pos = cnt + __popc(muse & ((1u << l) - 1u));
    if constexpr (kPack) {
      if (use) lsp[team][pos] = ((uint32_t)hv[v] << 16) | (uint32_t)(16 * v + l);
    } else {
      if (use) lst[team][pos] = (uint8_t)(16 * v + l);
      hs[team][16 * v + l] = hv[v];
    }
    cnt += __popc(muse);
  }
  if (live_out && c == 0 && phase == 0 && l == 0 && jv)
    live_out[(size_t)b * g.ngt + (routed ? k * g.gpr : g.topk * g.gpr) + grp] = live;
  // the team's LDS rows were written by lanes of this wave: a wave-level hand-off
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- round trip 2: live rows of this phase
  const uint32_t* wb = routed ? pw + es * (size_t)g.F * g.NW : spw;
  const uint32_t row0 = (uint32_t)grp * 64u * (uint32_t)g.NW + (uint32_t)w;
  float acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = 0.0f;
  float hsum = 0.0f;
  const int nmine = cnt;                              // this team's rows
  // most rows of any team of the wave: a team is one 16-lane row, so lanes 0, 16, 32
  // and 48 hold the four counts (scalar reads, no LDS permute in front of the row loads)
  const int nmax = max(max(__builtin_amdgcn_readlane(nmine, 0), __builtin_amdgcn_readlane(nmine, 16)),
                       max(__builtin_amdgcn_readlane(nmine, 32), __builtin_amdgcn_readlane(nmine, 48)));
  for (int r0 = 0; r0 < nmax; r0 += kRB) {            // one batch unless > 16 live rows
    // ent[r]: the row index in the low bits (16-bit activations: the activation bits above)
    uint32_t ent[kRB];
#pragma unroll
    for (int r = 0; r < kRB; ++r) {
      if constexpr (kPack)
        ent[r] = r0 + r < nmine ? lsp[team][r0 + r] : 0u;
      else
        ent[r] = r0 + r < nmine ? (uint32_t)lst[team][r0 + r] : 0u;
    }
    uint32_t q[kRB];
#pragma unroll
    for (int r = 0; r < kRB; ++r) {
      q[r] = 0u;
      if (r0 + r < nmine)
        q[r] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(wb) +
                                                  (size_t)(row0 + (ent[r] & 63u) * (uint32_t)g.NW) * 4u);
    }
    float hx[kPack ? 1 : kRB];
    if constexpr (!kPack) {
#pragma unroll
      for (int r = 0; r < kRB; ++r) hx[r] = Elem<HDT>::load(&hs[team][ent[r] & 63u], 0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < kRB; ++r) {
      if (r0 + r < nmax) {                            // wave-uniform bound
        float x;
        if constexpr (kPack) {
          const HT hb = (HT)(ent[r] >> 16);
          x = Elem<HDT>::load(&hb, 0);
        } else {
          x = hx[r];
        }
        x = r0 + r < nmine ? x : 0.0f;
        hsum += x;
        const uint32_t lo = q[r] & 0x0F0F0F0Fu, hi = (q[r] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[2 * i] = fmaf(x, (float)((lo >> (8 * i)) & 0xFFu), acc[2 * i]);
          acc[2 * i + 1] = fmaf(x, (float)((hi >> (8 * i)) & 0xFFu), acc[2 * i + 1]);
        }
      }
    }
  }

  // ---- group terms, then the ordered sum over (group, phase), two levels
  const uint32_t s32[4] = {sv.x, sv.y, sv.z, sv.w};
  const uint32_t b32[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    red[team][(2 * i) * kWPC + l] = fmaf(lo_bf16(s32[i]), acc[2 * i], lo_bf16(b32[i]) * hsum);
    red[team][(2 * i + 1) * kWPC + l] = fmaf(hi_bf16(s32[i]), acc[2 * i + 1], hi_bf16(b32[i]) * hsum);
  }
  __syncthreads();
  // level 1: kThreads/kDC threads per output, each over a contiguous run of groups. A
  // thread takes word lw = o % 16 and nibble t = o / 16 (output 8 lw + t), so the lanes of
  // a wavefront read consecutive words of red.
  constexpr int kGPS = kGPW / kL1;                    // groups per sub-sum
  {
    const int o = tid % kDC, s = tid / kDC;
    const int lw = o % kWPC, t = o / kWPC, col = 8 * lw + t;
    float acc2 = 0.0f;
    bool first = true;
#pragma unroll
    for (int i = 0; i < kGPS; ++i) {
      const int jj = s * kGPS + i;
      if (jj < ng) {
#pragma unroll
        for (int ph = 0; ph < kRS; ++ph) {
          const float v = red[ph * kGPW + jj][t * kWPC + lw];
          acc2 = first ? v : acc2 + v;
          first = false;
        }
      }
    }
    sum2[col][s] = acc2;
  }
  __syncthreads();
  if (tid < kDC) {
    float v = sum2[tid][0];
#pragma unroll
    for (int s = 1; s < kL1; ++s) v += sum2[tid][s];
    part[((size_t)b * g.nparts + p) * g.D + (size_t)c * kDC + tid] = gain * v;
  }
  if (!ok && tid == 0 && c == 0 && status) atomicOr(status, (int32_t)HSD_STATUS_BAD_EXPERT);
}

constexpr int kSumThreads = 64;          // one wavefront per workgroup: 42 per token row at D = 2688

// y = the parts summed in part order; with res (bf16 y only): y = bf16(res + bf16(sum)),
// the MoE block's residual add (model.py:139).
template <int YDT, int NP>
__global__ __launch_bounds__(kSumThreads) void k_sum_parts(const float* __restrict__ part,
                                                   typename Elem<YDT>::T* __restrict__ y, int D,
                                                   int nparts, const uint16_t* __restrict__ res) {
  // grid (output columns / 64, token rows): no division for the coordinates
  const int b = blockIdx.y, o = blockIdx.x * kSumThreads + threadIdx.x;
  if (o >= D) return;
  const int idx = b * D + o;
  const float* pp = part + (size_t)b * nparts * D + o;
  // the residual (bf16 output) is loaded with the parts, not after their sum (a load used
  // only under a branch is issued there, one more round trip): without a residual the load
  // reads the parts' first word and the value is dropped
  constexpr bool kRes = YDT == HSD_DT_BF16;
  const bool has_res = kRes && res != nullptr;
  const uint16_t* rp = has_res ? res : reinterpret_cast<const uint16_t*>(part);
  uint32_t rv = kRes ? rp[has_res ? idx : 0] : 0u;
  float s;
  if (NP > 0) {
    float v[NP > 0 ? NP : 1];
#pragma unroll
    for (int q = 0; q < NP; ++q) v[q] = pp[(size_t)q * D];
    if constexpr (kRes) rv = opaque_vgpr(rv);
    s = v[0];
#pragma unroll
    for (int q = 1; q < NP; ++q) s += v[q];
  } else {
    s = pp[0];
    if constexpr (kRes) rv = opaque_vgpr(rv);
    for (int q = 1; q < nparts; ++q) s += pp[(size_t)q * D];
  }
  if (has_res) s = bf16_bits_to_f32(rv) + bf16_bits_to_f32(f32_to_bf16_bits(s));
  Elem<YDT>::store(y, idx, s);
}

// ----------------------------------------------------------------- dense comparator
// The stock layout w [E, D, F/8]: output row o of a slot is F/8 contiguous words. One
// wavefront computes kOPW outputs over all topk+1 slots: the slots' rows, seen as one
// run of 16-byte pieces (32 neurons each; piece u covers h[32u .. 32u+31] because the
// slots are contiguous in h), are split over the 64 lanes (piece u -> lane u % 64). Every
// lane issues all its weight/scale/bias loads for the kOPW outputs before using any;
// h comes from LDS. Per piece: gain * (s*acc + b*hsum); a butterfly sum gives y.
constexpr int kOPW = 2;
constexpr int kDenseWaves = 4;
constexpr int kMaxPieces = 8;            // pieces per lane: (topk*F + FS)/32 <= 512

template <int HDT, int YDT>
__global__ __launch_bounds__(64 * kDenseWaves) void k_dense_down(
    const typename Elem<HDT>::T* __restrict__ h, const int32_t* __restrict__ sel,
    const float* __restrict__ gains, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ s, const uint16_t* __restrict__ bias,
    const uint32_t* __restrict__ sw, const uint16_t* __restrict__ ss,
    const uint16_t* __restrict__ sbias, typename Elem<YDT>::T* __restrict__ y,
    int32_t* __restrict__ status, int D, int F, int FS, int topk, int E) {
  using HT = typename Elem<HDT>::T;
  extern __shared__ __attribute__((aligned(16))) unsigned char dsm[];
  HT* hsh = reinterpret_cast<HT*>(dsm);
  const int NR = topk * F + FS;
  const int b = blockIdx.y;
  for (int i = threadIdx.x; i < NR; i += blockDim.x) hsh[i] = h[(size_t)b * NR + i];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int o0 = (blockIdx.x * kDenseWaves + wave) * kOPW;
  const int ur = F / 32, nu = NR / 32;
  // this lane's pieces: slot, piece within the slot's row, gain, row base
  const uint32_t* rowp[kMaxPieces];
  const uint16_t* scp[kMaxPieces];
  const uint16_t* bip[kMaxPieces];
  int rowstride[kMaxPieces], gstride[kMaxPieces];
  float gn[kMaxPieces];
  bool pv[kMaxPieces];
#pragma unroll
  for (int i = 0; i < kMaxPieces; ++i) {
    const int u = lane + 64 * i;
    pv[i] = u < nu;
    rowp[i] = sw; scp[i] = ss; bip[i] = sbias; rowstride[i] = 0; gstride[i] = 0; gn[i] = 0.0f;
    if (!pv[i]) continue;
    int k, uu;
    if (u < topk * ur) { k = u / ur; uu = u - k * ur; } else { k = topk; uu = u - topk * ur; }
    gn[i] = gains[b * (topk + 1) + k];
    if (k < topk) {
      const int e = sel[b * topk + k];
      if ((unsigned)e >= (unsigned)E) {
        if (status && uu == 0) atomicOr(status, (int32_t)HSD_STATUS_BAD_EXPERT);
        pv[i] = false;
        continue;
      }
      rowstride[i] = F / 8; gstride[i] = F / 64;
      rowp[i] = w + (size_t)e * D * (F / 8) + 4 * uu;
      scp[i] = s + (size_t)e * D * (F / 64) + uu / 2;
      bip[i] = bias + (size_t)e * D * (F / 64) + uu / 2;
    } else {
      rowstride[i] = FS / 8; gstride[i] = FS / 64;
      rowp[i] = sw + 4 * uu;
      scp[i] = ss + uu / 2;
      bip[i] = sbias + uu / 2;
    }
  }
  uint4 q[kOPW][kMaxPieces];
  float sc[kOPW][kMaxPieces], bi[kOPW][kMaxPieces];
#pragma unroll
  for (int oi = 0; oi < kOPW; ++oi) {
    const int o = min(o0 + oi, D - 1);
#pragma unroll
    for (int i = 0; i < kMaxPieces; ++i) {
      q[oi][i] = make_uint4(0, 0, 0, 0);
      sc[oi][i] = 0.0f;
      bi[oi][i] = 0.0f;
      if (pv[i]) {
        q[oi][i] = *reinterpret_cast<const uint4*>(rowp[i] + (size_t)o * rowstride[i]);
        sc[oi][i] = bf16_bits_to_f32(scp[i][(size_t)o * gstride[i]]);
        bi[oi][i] = bf16_bits_to_f32(bip[i][(size_t)o * gstride[i]]);
      }
    }
  }
  __syncthreads();
  float tot[kOPW];
#pragma unroll
  for (int oi = 0; oi < kOPW; ++oi) tot[oi] = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxPieces; ++i) {
    if (!pv[i]) continue;
    const int u = lane + 64 * i;
    float hv[32];
    float hs = 0.0f;
#pragma unroll
    for (int n = 0; n < 32; ++n) {
      hv[n] = Elem<HDT>::load(hsh, 32 * u + n);
      hs += hv[n];
    }
#pragma unroll
    for (int oi = 0; oi < kOPW; ++oi) {
      const uint32_t qw[4] = {q[oi][i].x, q[oi][i].y, q[oi][i].z, q[oi][i].w};
      float acc = 0.0f;
#pragma unroll
      for (int wi = 0; wi < 4; ++wi)
#pragma unroll
        for (int n = 0; n < 8; ++n) acc = fmaf(hv[8 * wi + n], (float)((qw[wi] >> (4 * n)) & 0xFu), acc);
      tot[oi] = fmaf(gn[i], fmaf(sc[oi][i], acc, bi[oi][i] * hs), tot[oi]);
    }
  }
#pragma unroll
  for (int oi = 0; oi < kOPW; ++oi) {
    const float v = wave_sum(tot[oi]);
    const int o = o0 + oi;
    if (lane == 0 && o < D) Elem<YDT>::store(y, (size_t)b * D + o, v);
  }
}

// The comparator for bf16 h, organised like the projections' GEMV: a workgroup (4
// wavefronts) owns kDQRows consecutive outputs of one token row, kDQRW per wavefront.
// Lane l owns pieces l, l + 64, ... (16 bytes, 32 neurons) of the slots' concatenated rows
// (topk F + FS neurons: 464 pieces at the reference shape) for its wavefront's outputs.
// The slot ids and h are loaded first, then every weight, scale and bias load is issued
// before the lane waits for h. h goes to LDS once per
// workgroup as bf16 pairs in a word's nibble order, with the sum of every piece. Per
// piece: a shift, a mask and an OR turn each nibble into a bf16 (1 + q/16) pair,
// v_dot2_f32_bf16 accumulates h (1 + q/16) in fp32, and the lane adds
// gain * (16 s acc + (b - 16 s) hsum) (W = s q + b folded per piece); a DPP sum gives y.
// Loads are never under a branch: a piece past the row or of a bad slot reads a valid
// address and is dropped by a select.
// Measured per call at the reference shape: 11.7 us with one output per wavefront, 13.1
// with two. With the weights issued before h (the wait for h then waited for every
// weight): 14.7 us with one output per wavefront, 15.7 with two, 17.3 with four, 16.1 with
// 8-wavefront workgroups, 18.3 with 2-wavefront ones.
constexpr int kDQRW = 1;                 // outputs per wavefront
constexpr int kDQWaves = 4;
constexpr int kDQRows = kDQRW * kDQWaves;
constexpr int kDQPass = 8;               // pieces per lane: (topk F + FS) / 32 <= 512
constexpr int kDQXIt = kDQPass * 64 * 4 / (64 * kDQWaves);  // h words (8 values) per thread
constexpr uint32_t kBfOne2 = 0x3F803F80u;
constexpr uint32_t kNibHi = 0x00780078u;

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                         false);
}

template <int YDT>
__global__ __launch_bounds__(64 * kDQWaves) void k_dense_down_q(
    const uint16_t* __restrict__ h, const int32_t* __restrict__ sel, const float* __restrict__ gains,
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ s, const uint16_t* __restrict__ bias,
    const uint32_t* __restrict__ sw, const uint16_t* __restrict__ ss, const uint16_t* __restrict__ sbias,
    typename Elem<YDT>::T* __restrict__ y, int32_t* __restrict__ status, int D, int F, int FS, int topk,
    int E) {
  extern __shared__ __attribute__((aligned(16))) uint32_t qsm[];
  const int NR = topk * F + FS, NP = NR / 32, NW = NR / 8;
  uint32_t* xp = qsm;                                    // word m of piece j at 4 (m NP + j)
  float* xh = reinterpret_cast<float*>(qsm + NR / 2);    // piece sums
  const int b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int o0 = blockIdx.x * kDQRows + wave * kDQRW;
  const int ur = F / 32;
  // ---- loads in the order they are waited for: the slots' ids and gains, h (neither
  // depends on the other), then the weights, whose addresses need the ids
  int ek[kDQPass];
  float gn[kDQPass];
#pragma unroll
  for (int it = 0; it < kDQPass; ++it) {
    const int u = min(lane + 64 * it, NP - 1);
    const int k = u < topk * ur ? u / ur : topk;
    gn[it] = gains[b * (topk + 1) + k];
    ek[it] = sel[b * topk + min(k, topk - 1)];
  }
  // words t = tid + 64 kDQWaves i hold neurons 8t .. 8t+7
  uint4 hv[kDQXIt];
#pragma unroll
  for (int i = 0; i < kDQXIt; ++i)
    hv[i] = reinterpret_cast<const uint4*>(h + (size_t)b * NR)[min(tid + 64 * kDQWaves * i, NW - 1)];
  // this lane's pieces: where row o of the piece's matrix starts
  const uint32_t* rowp[kDQPass];
  const uint16_t* scp[kDQPass];
  const uint16_t* bip[kDQPass];
  int rstride[kDQPass], gstride[kDQPass];
  bool pv[kDQPass];
#pragma unroll
  for (int it = 0; it < kDQPass; ++it) {
    const int u = min(lane + 64 * it, NP - 1);
    const bool routed = u < topk * ur;
    const int k = routed ? u / ur : topk;
    const int uu = routed ? u - k * ur : u - topk * ur;
    const int e = routed ? ek[it] : 0;
    const bool ok = (unsigned)e < (unsigned)E;
    pv[it] = lane + 64 * it < NP && ok;
    if (routed && !ok && uu == 0 && lane + 64 * it < NP && status) atomicOr(status, (int32_t)HSD_STATUS_BAD_EXPERT);
    const size_t eo = ok ? (size_t)e : 0;
    rstride[it] = routed ? F / 8 : FS / 8;
    gstride[it] = routed ? F / 64 : FS / 64;
    rowp[it] = routed ? w + eo * D * (F / 8) + 4 * uu : sw + 4 * uu;
    scp[it] = routed ? s + eo * D * (F / 64) + uu / 2 : ss + uu / 2;
    bip[it] = routed ? bias + eo * D * (F / 64) + uu / 2 : sbias + uu / 2;
  }
  uint4 q[kDQRW][kDQPass];
  uint32_t sb[kDQRW][kDQPass];
#pragma unroll
  for (int it = 0; it < kDQPass; ++it) {
#pragma unroll
    for (int r = 0; r < kDQRW; ++r) {
      const size_t o = (size_t)min(o0 + r, D - 1);
      q[r][it] = *reinterpret_cast<const uint4*>(rowp[it] + o * rstride[it]);
      sb[r][it] = (uint32_t)scp[it][o * gstride[it]] | ((uint32_t)bip[it][o * gstride[it]] << 16);
    }
  }
  // ---- h into LDS as bf16 pairs (h[8t + n], h[8t + n + 4]) in the order of a word's
  // nibble pairs, and the piece sums
#pragma unroll
  for (int i = 0; i < kDQXIt; ++i) {
    const int t = tid + 64 * kDQWaves * i;
    const uint32_t hw[4] = {hv[i].x, hv[i].y, hv[i].z, hv[i].w};
    if (t < NW) {
      uint4 pr;
      pr.x = (hw[0] & 0xFFFFu) | (hw[2] << 16);
      pr.y = (hw[0] >> 16) | (hw[2] & 0xFFFF0000u);
      pr.z = (hw[1] & 0xFFFFu) | (hw[3] << 16);
      pr.w = (hw[1] >> 16) | (hw[3] & 0xFFFF0000u);
      *reinterpret_cast<uint4*>(&xp[4 * ((t & 3) * NP + (t >> 2))]) = pr;
    }
    float s8 = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) s8 = dot2_bf16(hw[c], kBfOne2, s8);
    s8 += dpp_f32<0xB1>(s8);  // the 4 words of a piece: quad_perm xor 1, xor 2
    s8 += dpp_f32<0x4E>(s8);
    if (t < NW && (t & 3) == 0) xh[t >> 2] = s8;
  }
  lds_barrier();
  // ---- the lane's pieces against its wavefront's outputs
  const uint32_t nibm = opaque_vgpr(kNibHi);          // (w & nibm) | one: one v_and_or_b32
  float tot[kDQRW];
#pragma unroll
  for (int r = 0; r < kDQRW; ++r) tot[r] = 0.0f;
#pragma unroll
  for (int it = 0; it < kDQPass; ++it) {
    const int j = min(lane + 64 * it, NP - 1);
    uint4 xq[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) xq[m] = *reinterpret_cast<const uint4*>(&xp[4 * (m * NP + j)]);
    const float xs = xh[j];
#pragma unroll
    for (int r = 0; r < kDQRW; ++r) {
      const uint32_t qw[4] = {q[r][it].x, q[r][it].y, q[r][it].z, q[r][it].w};
      float acc = 0.0f;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        acc = dot2_bf16(xq[m].x, ((qw[m] << 3) & nibm) | kBfOne2, acc);
        acc = dot2_bf16(xq[m].y, ((qw[m] >> 1) & nibm) | kBfOne2, acc);
        acc = dot2_bf16(xq[m].z, ((qw[m] >> 5) & nibm) | kBfOne2, acc);
        acc = dot2_bf16(xq[m].w, ((qw[m] >> 9) & nibm) | kBfOne2, acc);
      }
      const float sv = lo_bf16(sb[r][it]), bv = hi_bf16(sb[r][it]);
      const float u = fmaf(16.0f * sv, acc, fmaf(-16.0f, sv, bv) * xs);
      tot[r] = pv[it] ? fmaf(gn[it], u, tot[r]) : tot[r];
    }
  }
#pragma unroll
  for (int r = 0; r < kDQRW; ++r) {
    const float v = wave_sum_dpp(tot[r]);
    const int o = o0 + r;
    if (lane == 0 && o < D) Elem<YDT>::store(y, (size_t)b * D + o, v);
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace hsd

using namespace hsd;

extern "C" size_t hsd_sparse_down_workspace_bytes(int64_t B, int64_t D, int64_t F, int64_t FS,
                                                  int64_t topk) {
  if (B <= 0 || D <= 0 || F <= 0 || FS <= 0 || topk <= 0) return 0;
  const Geom g = make_geom(D, F, FS, topk, 1);
  const size_t bytes = (size_t)B * g.nparts * (size_t)D * sizeof(float);
  return (bytes + 255) & ~(size_t)255;
}

namespace hsd {
namespace {

// The checks and the two launches of a sparse decode call, with the partial sums in
// `part` (B * nparts * D floats; every element is written before it is read).
int launch_sparse_down(const char* fn, const void* h, int h_dtype, const int32_t* sel,
                       const float* gains, const uint32_t* pw, const uint16_t* ps,
                       const uint16_t* pb, const uint32_t* spw, const uint16_t* sps,
                       const uint16_t* spb, void* y, int y_dtype, int64_t B, int64_t D,
                       int64_t F, int64_t FS, int64_t topk, int64_t E, int dense,
                       uint64_t* live_masks, int32_t* dev_status, float* part, hipStream_t st,
                       const uint16_t* res = nullptr) {
  const Geom g = make_geom(D, F, FS, topk, E);
  // the grid is (chunks, parts, token rows): at most 65535 token rows per call
  if (B > 65535 || g.nparts > 65535) return set_error(HSD_ERR_SHAPE, "%s: too many token rows or parts", fn);
  const int64_t nblk = B * (int64_t)g.nwg;
#define HSD_PART(DT)                                                                          \
  hipLaunchKernelGGL(k_sparse_down_part<DT>, dim3((unsigned)g.nchunk, (unsigned)g.nparts, (unsigned)B),      \
                     dim3(kThreads), 0, st,                                                               \
                     reinterpret_cast<const typename Elem<DT>::T*>(h), sel, gains, g.nwg, g.nchunk,   \
                     g.topk, g.ppr, g.gpr, g.gsh, (int)nblk, g.F, pw, ps, pb, spw, sps, spb, part,    \
                     live_masks, dev_status, g, dense)
  switch (h_dtype) {
    case HSD_DT_BF16: HSD_PART(HSD_DT_BF16); break;
    case HSD_DT_F16: HSD_PART(HSD_DT_F16); break;
    case HSD_DT_F32: HSD_PART(HSD_DT_F32); break;
    default: return set_error(HSD_ERR_DTYPE, "%s: h_dtype %d", fn, h_dtype);
  }
#undef HSD_PART
  int rc = check_launch(fn);
  if (rc) return rc;
  const dim3 rgrid((unsigned)((D + kSumThreads - 1) / kSumThreads), (unsigned)B);
#define HSD_SUM(DT)                                                                                  \
  if (g.nparts == 32)                                                                                \
    hipLaunchKernelGGL((k_sum_parts<DT, 32>), rgrid, dim3(kSumThreads), 0, st, part,                         \
                       reinterpret_cast<typename Elem<DT>::T*>(y), (int)D, g.nparts, res);          \
  else                                                                                               \
    hipLaunchKernelGGL((k_sum_parts<DT, 0>), rgrid, dim3(kSumThreads), 0, st, part,                          \
                       reinterpret_cast<typename Elem<DT>::T*>(y), (int)D, g.nparts, res);
  switch (y_dtype) {
    case HSD_DT_BF16: HSD_SUM(HSD_DT_BF16); break;
    case HSD_DT_F16: HSD_SUM(HSD_DT_F16); break;
    case HSD_DT_F32: HSD_SUM(HSD_DT_F32); break;
    default: return set_error(HSD_ERR_DTYPE, "%s: y_dtype %d", fn, y_dtype);
  }
#undef HSD_SUM
  return check_launch(fn);
}

// Argument checks shared by both sparse decode entry points.
int check_sparse_down_args(const char* fn, const void* h, const int32_t* sel, const float* gains,
                           const uint32_t* pw, const uint16_t* ps, const uint16_t* pb,
                           const uint32_t* spw, const uint16_t* sps, const uint16_t* spb,
                           const void* y, int64_t B, int64_t D, int64_t F, int64_t FS,
                           int64_t topk, int64_t E) {
  if (!h || !sel || !gains || !pw || !ps || !pb || !spw || !sps || !spb || !y)
    return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (B < 0 || topk <= 0 || E <= 0) return set_error(HSD_ERR_SHAPE, "%s: bad B/topk/E", fn);
  if (D <= 0 || D % kDC || F <= 0 || F % 64 || FS <= 0 || FS % 64)
    return set_error(HSD_ERR_SHAPE, "%s: need D %% %d == 0, F %% 64 == 0, FS %% 64 == 0 (D=%lld F=%lld FS=%lld)",
                     fn, kDC, (long long)D, (long long)F, (long long)FS);
  if (topk * F + FS > (int64_t)1 << 30 || D > 65536 || B > 65535 ||
      B * (topk * F + FS) >= ((int64_t)1 << 32) || F * (D / 8) >= ((int64_t)1 << 32) ||
      FS * (D / 8) >= ((int64_t)1 << 32))
    return set_error(HSD_ERR_SHAPE, "%s: sizes too large", fn);
  if (!aligned16(ps) || !aligned16(pb) || !aligned16(sps) || !aligned16(spb))
    return set_error(HSD_ERR_ALIGN, "%s: scales/biases must be 16-byte aligned", fn);
  return HSD_OK;
}

// ---------------------------------------------------------------- no-allocation variant
// The partial sums of hsd_sparse_down_decode_noalloc live in this file-scope device array
// (one copy per GPU, held until the process ends). Host code never passes the array's
// name to a kernel: on the host it is only a stand-in for the symbol. Its device address
// is looked up once per device with hipGetSymbolAddress and kept in g_scratch_dev.
constexpr size_t kNoAllocScratchBytes = (size_t)4 << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_dev[kMaxDevices] = {};

// The current device's copy of `scratch` (looked up on the first call on that device,
// with that device current). nullptr with the error set on failure.
float* scratch_for_current_device(const char* fn) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error(HSD_ERR_LAUNCH, "%s: hipGetDevice failed (%s)", fn, hipGetErrorString(e));
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error(HSD_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d (%s)", fn, dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_dev[dev] = reinterpret_cast<float*>(p);
  }
  return g_scratch_dev[dev];
}

}  // namespace
}  // namespace hsd

extern "C" int hsd_sparse_down_decode(const void* h, int h_dtype, const int32_t* sel,
                                      const float* gains, const uint32_t* pw, const uint16_t* ps,
                                      const uint16_t* pb, const uint32_t* spw, const uint16_t* sps,
                                      const uint16_t* spb, void* y, int y_dtype, int64_t B,
                                      int64_t D, int64_t F, int64_t FS, int64_t topk, int64_t E,
                                      int dense, uint64_t* live_masks, int32_t* dev_status,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "hsd_sparse_down_decode";
  int rc = check_sparse_down_args(fn, h, sel, gains, pw, ps, pb, spw, sps, spb, y, B, D, F, FS, topk, E);
  if (rc) return rc;
  if (B == 0) return HSD_OK;
  const size_t need = hsd_sparse_down_workspace_bytes(B, D, F, FS, topk);
  if (!workspace || workspace_bytes < need)
    return set_error(HSD_ERR_WORKSPACE, "%s: workspace needs %zu bytes", fn, need);
  return launch_sparse_down(fn, h, h_dtype, sel, gains, pw, ps, pb, spw, sps, spb, y, y_dtype, B, D, F, FS,
                            topk, E, dense, live_masks, dev_status, reinterpret_cast<float*>(workspace),
                            as_stream(stream));
}

extern "C" int hsd_sparse_down_residual(const void* h, int h_dtype, const int32_t* sel, const float* gains,
                                        const uint32_t* pw, const uint16_t* ps, const uint16_t* pb,
                                        const uint32_t* spw, const uint16_t* sps, const uint16_t* spb,
                                        const uint16_t* x, uint16_t* y, int64_t B, int64_t D, int64_t F,
                                        int64_t FS, int64_t topk, int64_t E, int dense, uint64_t* live_masks,
                                        int32_t* dev_status, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  const char* fn = "hsd_sparse_down_residual";
  if (!x) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  int rc = check_sparse_down_args(fn, h, sel, gains, pw, ps, pb, spw, sps, spb, y, B, D, F, FS, topk, E);
  if (rc) return rc;
  if (B == 0) return HSD_OK;
  const size_t need = hsd_sparse_down_workspace_bytes(B, D, F, FS, topk);
  if (!workspace || workspace_bytes < need)
    return set_error(HSD_ERR_WORKSPACE, "%s: workspace needs %zu bytes", fn, need);
  return launch_sparse_down(fn, h, h_dtype, sel, gains, pw, ps, pb, spw, sps, spb, y, HSD_DT_BF16, B, D, F, FS,
                            topk, E, dense, live_masks, dev_status, reinterpret_cast<float*>(workspace),
                            as_stream(stream), x);
}

extern "C" int hsd_sparse_down_decode_noalloc(const void* h, int h_dtype, const int32_t* sel,
                                              const float* gains, const uint32_t* pw,
                                              const uint16_t* ps, const uint16_t* pb,
                                              const uint32_t* spw, const uint16_t* sps,
                                              const uint16_t* spb, void* y, int y_dtype, int64_t B,
                                              int64_t D, int64_t F, int64_t FS, int64_t topk,
                                              int64_t E, int dense, uint64_t* live_masks,
                                              int32_t* dev_status, void* stream) {
  const char* fn = "hsd_sparse_down_decode_noalloc";
  int rc = check_sparse_down_args(fn, h, sel, gains, pw, ps, pb, spw, sps, spb, y, B, D, F, FS, topk, E);
  if (rc) return rc;
  if (B == 0) return HSD_OK;
  const size_t need = hsd_sparse_down_workspace_bytes(B, D, F, FS, topk);
  if (need > kNoAllocScratchBytes)
    return set_error(HSD_ERR_SHAPE,
                     "%s: the partial sums need %zu bytes, more than the %zu-byte static scratch "
                     "(at most B = %zu rows at this shape)",
                     fn, need, kNoAllocScratchBytes, kNoAllocScratchBytes / (need / (size_t)B));
  float* part = scratch_for_current_device(fn);
  if (!part) return HSD_ERR_LAUNCH;
  return launch_sparse_down(fn, h, h_dtype, sel, gains, pw, ps, pb, spw, sps, spb, y, y_dtype, B, D, F, FS,
                            topk, E, dense, live_masks, dev_status, part, as_stream(stream));
}

extern "C" int hsd_dense_down_decode(const void* h, int h_dtype, const int32_t* sel,
                                     const float* gains, const uint32_t* w, const uint16_t* s,
                                     const uint16_t* b, const uint32_t* sw, const uint16_t* ss,
                                     const uint16_t* sb, void* y, int y_dtype, int64_t B,
                                     int64_t D, int64_t F, int64_t FS, int64_t topk, int64_t E,
                                     int32_t* dev_status, void* stream) {
  const char* fn = "hsd_dense_down_decode";
  if (!h || !sel || !gains || !w || !s || !b || !sw || !ss || !sb || !y)
    return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (B < 0 || topk <= 0 || E <= 0 || D <= 0 || F <= 0 || FS <= 0 || F % 64 || FS % 64)
    return set_error(HSD_ERR_SHAPE, "%s: need F %% 64 == 0 and FS %% 64 == 0", fn);
  if (!aligned16(w) || !aligned16(sw)) return set_error(HSD_ERR_ALIGN, "%s: weights must be 16-byte aligned", fn);
  const int64_t NR = topk * F + FS;
  if (NR > 64 * 32 * kMaxPieces || (h_dtype == HSD_DT_F32 && NR * 4 > 65536))
    return set_error(HSD_ERR_SHAPE, "%s: h row of %lld elements too long", fn, (long long)NR);
  if (B == 0) return HSD_OK;
  if (B > 65535 || D > (1 << 24)) return set_error(HSD_ERR_SHAPE, "%s: sizes too large", fn);
  const int per_wg = kOPW * kDenseWaves;
  dim3 grid((unsigned)((D + per_wg - 1) / per_wg), (unsigned)B);
  hipStream_t st = as_stream(stream);
  const size_t lds = (size_t)NR * (h_dtype == HSD_DT_F32 ? 4 : 2);
#define HSD_DENSE(HD, YD)                                                                        \
  hipLaunchKernelGGL((k_dense_down<HD, YD>), grid, dim3(64 * kDenseWaves), lds, st,              \
                     reinterpret_cast<const typename Elem<HD>::T*>(h), sel, gains, w, s, b, sw, ss, \
                     sb, reinterpret_cast<typename Elem<YD>::T*>(y), dev_status, (int)D, (int)F,   \
                     (int)FS, (int)topk, (int)E)
#define HSD_DENSE_Y(HD)                                          \
  switch (y_dtype) {                                             \
    case HSD_DT_BF16: HSD_DENSE(HD, HSD_DT_BF16); break;         \
    case HSD_DT_F16: HSD_DENSE(HD, HSD_DT_F16); break;           \
    case HSD_DT_F32: HSD_DENSE(HD, HSD_DT_F32); break;           \
    default: return set_error(HSD_ERR_DTYPE, "%s: y_dtype %d", fn, y_dtype); \
  }
  if (h_dtype == HSD_DT_BF16 && aligned16(h)) {  // bf16 h: the GEMV-shaped kernel
    if (NR > 64 * 32 * kDQPass) return set_error(HSD_ERR_SHAPE, "%s: h row of %lld elements too long", fn, (long long)NR);
    dim3 gq((unsigned)((D + kDQRows - 1) / kDQRows), (unsigned)B);
    const size_t lq = (size_t)NR * 2 + (size_t)(NR / 32) * 4;
#define HSD_DENSE_Q(YD)                                                                           \
  hipLaunchKernelGGL((k_dense_down_q<YD>), gq, dim3(64 * kDQWaves), lq, st,                       \
                     reinterpret_cast<const uint16_t*>(h), sel, gains, w, s, b, sw, ss, sb,        \
                     reinterpret_cast<typename Elem<YD>::T*>(y), dev_status, (int)D, (int)F, (int)FS, \
                     (int)topk, (int)E)
    switch (y_dtype) {
      case HSD_DT_BF16: HSD_DENSE_Q(HSD_DT_BF16); break;
      case HSD_DT_F16: HSD_DENSE_Q(HSD_DT_F16); break;
      case HSD_DT_F32: HSD_DENSE_Q(HSD_DT_F32); break;
      default: return set_error(HSD_ERR_DTYPE, "%s: y_dtype %d", fn, y_dtype);
    }
#undef HSD_DENSE_Q
    return check_launch(fn);
  }
  switch (h_dtype) {
    case HSD_DT_BF16: HSD_DENSE_Y(HSD_DT_BF16); break;
    case HSD_DT_F16: HSD_DENSE_Y(HSD_DT_F16); break;
    case HSD_DT_F32: HSD_DENSE_Y(HSD_DT_F32); break;
    default: return set_error(HSD_ERR_DTYPE, "%s: h_dtype %d", fn, h_dtype);
  }
#undef HSD_DENSE_Y
#undef HSD_DENSE
  return check_launch(fn);
}
