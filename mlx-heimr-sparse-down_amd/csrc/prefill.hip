// The MoE down projection over a prompt chunk: tile order, per-tile union of live
// neurons, and a bf16 MFMA grouped GEMM on the neuron-major layout (hsd/prefill.py).
//
//   k_tiles      one workgroup: stable expert sort of the T*topk slots (wave ballots
//                give each slot its rank among equal experts), tile bases by a scan,
//                fixed NT = T*topk/tt + E + ceil(T/tt) with -1 padding, no host readback.
//   k_union      one workgroup per tile, 8 columns per thread: OR over the tile's slots
//                of h != 0 (16-byte loads), prefix compaction into the ascending union
//                list (ulist, ucount).
//   k_stage, k_gemm, k_sum_slots: the grouped GEMM, described above k_stage.
#include "hsd_common.h"

namespace hsd {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------------ tiles
constexpr int kTT = 1024;  // threads of the tile-order kernel

__global__ __launch_bounds__(kTT) void k_tiles(const int32_t* __restrict__ sel, int T, int topk,
                                               int E, int tt, int P,
                                               int32_t* __restrict__ tile_e,
                                               int32_t* __restrict__ tile_slot,
                                               int32_t* __restrict__ status,
                                               int32_t* __restrict__ rank_ws) {
  extern __shared__ int sh[];
  int* cnt = sh;                    // [E] running count per expert, then counts
  int* tbase = sh + E;              // [E + 1] tile base per expert (exclusive scan)
  int* wcnt = sh + 2 * E + 1;       // [P][16][E] per-(chunk, wave) counts of a pass
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = T * topk;
  const int nbits = 32 - __builtin_clz((unsigned)max(E - 1, 1));  // bits of an expert id
  for (int e = tid; e < E; e += kTT) cnt[e] = 0;
  // The slots are ranked kTT at a time (chunk k: slots k kTT + tid), P chunks per pass
  // (P = kTR when the pass's counts fit in LDS, else 1) with one set of barriers per pass.
  // With P = kTR the first pass's ids are loaded up front and its ranks stay in
  // registers; the other ranks go through rank_ws. Loads are never under a branch: ids
  // past n re-read slot n - 1.
  constexpr int kTR = 4;
  const int nch = (n + kTT - 1) / kTT;
  int e_r[kTR], rank_r[kTR];
#pragma unroll
  for (int k = 0; k < kTR; ++k) e_r[k] = sel[min(k * kTT + tid, n - 1)];
  // ranks of chunks k0 .. k0 + np - 1 (np <= P), ids in ev; ranks (stable among the slots
  // of an expert, or -1) into rk
  auto pass = [&](int k0, int np, int (&ev)[kTR], int (&rk)[kTR]) {
    for (int i = tid; i < np * 16 * E; i += kTT) wcnt[i] = 0;
    __syncthreads();
    int rw[kTR];
#pragma unroll
    for (int k = 0; k < kTR; ++k) {
      rw[k] = 0;
      if (k >= np) continue;  // uniform
      const int s = (k0 + k) * kTT + tid;
      int e = ev[k];
      if (s >= n) e = -1;
      if (s < n && (unsigned)e >= (unsigned)E) {
        if (status) atomicOr(status, (int32_t)HSD_STATUS_BAD_EXPERT);
        e = -1;
      }
      ev[k] = e;
      // rank among the lanes of this wave with the same expert, lowest lane first: the
      // lanes whose id equals this lane's are the AND over the id's bits of that bit's
      // ballot or its complement (one ballot per bit, no loop over distinct experts);
      // the lowest such lane writes the wave's count
      uint64_t eq = __ballot(e >= 0);
      for (int b = 0; b < nbits; ++b) {  // uniform
        const bool bit = (e >> b) & 1;
        const uint64_t m = __ballot(bit);
        eq &= bit ? m : ~m;
      }
      const uint64_t below = eq & ((1ull << lane) - 1ull);
      rw[k] = __popcll(below);
      if (e >= 0 && below == 0ull) wcnt[(k * 16 + wave) * E + e] = __popcll(eq);
    }
    __syncthreads();
    // exclusive scan over (chunk, wave) in slot order, per expert: 16 lanes per expert
    // (one DPP row, lane w = wave w), four experts per wave and round
    for (int e0 = wave * 4; e0 < E; e0 += 64) {
      const int ee = e0 + (lane >> 4), w = lane & 15;
      int run = ee < E ? cnt[ee] : 0;  // read by all 16 lanes before lane 15 updates it
#pragma unroll
      for (int k = 0; k < kTR; ++k) {
        if (k >= np) continue;  // uniform
        const int c = ee < E ? wcnt[(k * 16 + w) * E + ee] : 0;
        // inclusive scan over the 16 lanes of a DPP row: row_shr:1,2,4,8 (lanes shifted
        // in from outside the row read 0)
        int incl = c;
        incl += __builtin_amdgcn_update_dpp(0, incl, 0x111, 0xF, 0xF, true);
        incl += __builtin_amdgcn_update_dpp(0, incl, 0x112, 0xF, 0xF, true);
        incl += __builtin_amdgcn_update_dpp(0, incl, 0x114, 0xF, 0xF, true);
        incl += __builtin_amdgcn_update_dpp(0, incl, 0x118, 0xF, 0xF, true);
        const int tot = __shfl(incl, lane | 15, 64);
        if (ee < E) wcnt[(k * 16 + w) * E + ee] = run + incl - c;
        run += tot;
      }
      if (ee < E && w == 15) cnt[ee] = run;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kTR; ++k)
      if (k < np) rk[k] = ev[k] >= 0 ? wcnt[(k * 16 + wave) * E + ev[k]] + rw[k] : -1;
    __syncthreads();  // the counts are read before the next pass clears them
  };
  int k0 = 0;
  if (P == kTR) {
    pass(0, min(kTR, nch), e_r, rank_r);
    k0 = kTR;
  }
  for (; k0 < nch; k0 += P) {
    const int np = min(P, nch - k0);
    int ev[kTR], rk[kTR];
#pragma unroll
    for (int k = 0; k < kTR; ++k) ev[k] = sel[min((k0 + min(k, np - 1)) * kTT + tid, n - 1)];
    pass(k0, np, ev, rk);
#pragma unroll
    for (int k = 0; k < kTR; ++k) {
      const int s = (k0 + k) * kTT + tid;
      if (k < np && s < n) rank_ws[s] = rk[k];
    }
  }
  {  // tile base per expert: exclusive scan of the tile counts over the workgroup
    int* wtot = wcnt;  // 16 wave totals (the per-wave counts are no longer needed)
    const int nt = tid < E ? (cnt[tid] + tt - 1) / tt : 0;
    const int incl = wave_incl_scan(nt, lane);
    if (lane == 63) wtot[wave] = incl;
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; ++w) before += wtot[w];
    if (tid < E) tbase[tid] = before + incl - nt;
    if (tid == kTT - 1) tbase[E] = before + incl;
  }
  __syncthreads();
  const int nt_routed = n / tt + E;
  const int total = tbase[E];
  for (int t = tid; t < nt_routed; t += kTT) {
    int ee = -1;
    if (t < total) {  // the last expert whose base is <= t (experts with tiles are unique)
      int lo = 0, hi = E - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tbase[mid] <= t) lo = mid; else hi = mid - 1;
      }
      ee = lo;
    }
    tile_e[t] = ee;
  }
  for (int i = tid; i < nt_routed * tt; i += kTT) tile_slot[i] = -1;
  __syncthreads();  // the -1 fill is ordered before the scatter below (same workgroup)
  const int nreg = P == kTR ? min(kTR, nch) : 0;  // chunks whose ranks stayed in registers
#pragma unroll
  for (int k = 0; k < kTR; ++k) {
    const int s = k * kTT + tid;
    if (k < nreg && s < n && rank_r[k] >= 0)
      tile_slot[(tbase[e_r[k]] + rank_r[k] / tt) * tt + rank_r[k] % tt] = s;
  }
  for (int s = nreg * kTT + tid; s < n; s += kTT) {
    const int r = rank_ws[s];
    if (r < 0) continue;
    const int ee = sel[s];
    tile_slot[(tbase[ee] + r / tt) * tt + r % tt] = s;
  }
  const int nt_shared = (T + tt - 1) / tt;
  for (int t = tid; t < nt_shared; t += kTT) tile_e[nt_routed + t] = E;
  for (int i = tid; i < nt_shared * tt; i += kTT)
    tile_slot[(size_t)nt_routed * tt + i] = i < T ? i : -1;
}

// ------------------------------------------------------------------ union
constexpr int kUT = 512;  // threads of the union kernel; each owns 8 consecutive columns

// Bit j set when element j of the 8 activations in v is nonzero (+-0 are dead, NaN is live).
template <int HDT> struct Live8;
template <> struct Live8<HSD_DT_BF16> {
  __device__ __forceinline__ static uint32_t get(const void* p) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      m |= (((w[i] & 0x7FFFu) != 0u) ? 1u : 0u) << (2 * i) |
           (((w[i] & 0x7FFF0000u) != 0u) ? 1u : 0u) << (2 * i + 1);
    return m;
  }
};
template <> struct Live8<HSD_DT_F16> : Live8<HSD_DT_BF16> {};
template <> struct Live8<HSD_DT_F32> {
  __device__ __forceinline__ static uint32_t get(const void* p) {
    const uint4 a = reinterpret_cast<const uint4*>(p)[0], b = reinterpret_cast<const uint4*>(p)[1];
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) m |= (((w[i] & 0x7FFFFFFFu) != 0u) ? 1u : 0u) << i;
    return m;
  }
};

template <int HDT>
__global__ __launch_bounds__(kUT) void k_union(const typename Elem<HDT>::T* __restrict__ h,
                                               const int32_t* __restrict__ tile_e,
                                               const int32_t* __restrict__ tile_slot,
                                               int32_t* __restrict__ ulist,
                                               int32_t* __restrict__ ucount, int F, int FS,
                                               int topk, int E, int tt, int umax) {
  __shared__ int hoff[64];
  __shared__ int wsum[kUT / 64];
  const int tile = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int NR = topk * F + FS;
  int32_t* out = ulist + (size_t)tile * umax;
  // the tile's expert and slot together (one round trip; loads never under a branch)
  const int e = tile_e[tile];
  const int s = tile_slot[tile * tt + min(tid, tt - 1)];
  if (e < 0) {
    for (int i = tid; i < umax; i += kUT) out[i] = -1;
    if (tid == 0) ucount[tile] = 0;
    return;
  }
  const bool shared = e >= E;
  const int FF = shared ? FS : F;
  if (tid < tt)
    hoff[tid] = s < 0 ? -1 : (shared ? s * NR + topk * F : (s / topk) * NR + (s % topk) * F);
  __syncthreads();
  int base = 0;
  for (int c0 = 0; c0 < FF; c0 += 8 * kUT) {
    const int c = c0 + 8 * tid;
    uint32_t live = 0;  // bit j: column c + j is live in some slot of the tile
    // kUB slots' loads in flight at a time (a whole 32-slot tile for 16-bit h), then
    // their OR; dead slots and columns past the row read h[0..7] and are dropped after
    // the load (no load under a branch)
    constexpr int kUB = sizeof(typename Elem<HDT>::T) == 2 ? 32 : 16;
    for (int m0 = 0; m0 < tt; m0 += kUB) {
      uint32_t lm[kUB];
#pragma unroll
      for (int i = 0; i < kUB; ++i) {
        const int o = m0 + i < tt ? hoff[m0 + i] : -1;
        const bool ok = o >= 0 && c < FF;
        lm[i] = Live8<HDT>::get(h + (ok ? (size_t)o + c : 0));
        lm[i] = ok ? lm[i] : 0u;
      }
#pragma unroll
      for (int i = 0; i < kUB; ++i) live |= lm[i];
    }
    // exclusive prefix of the live counts over the workgroup, in column order
    const int n = __popc(live);
    const int incl = wave_incl_scan(n, lane);
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int before = base, tot = 0;
#pragma unroll
    for (int w = 0; w < kUT / 64; ++w) {
      before += w < wave ? wsum[w] : 0;
      tot += wsum[w];
    }
    int pos = before + incl - n;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if ((live >> j) & 1u) out[pos++] = c + j;
    base += tot;
    __syncthreads();
  }
  for (int i = base + tid; i < umax; i += kUT) out[i] = -1;
  if (tid == 0) ucount[tile] = base;
}

// ------------------------------------------------------------------ GEMM
// The grouped GEMM factors the affine dequantisation by 64-row group g:
//   y[m, n] = sum_g s[g, n] * sum_{k in g} h[m, k] * q[k, n]  +  sum_g hs[m, g] * b[g, n],
//   hs[m, g] = sum_{k in g} h[m, k].
// The MFMA B operand is the exact bf16 value 128 + q, made from a packed nibble word by
// a mask and an OR with 0x4300 (bf16 128.0); the extra 128 * hs[m, g] per group is
// removed in the correction term below. The K dimension is the tile's union rows, laid
// out group by group, each group padded to whole 16-row k-blocks, so one k-block never
// mixes two groups' scales.
//
//   k_stage   4 MS workgroups per tile, each for every (4 MS)-th slot: the union list
//             copied to LDS, group starts in it, the padded row
//             list (row byte offsets, kPadRow for padding), the A fragments of every
//             k-block in MFMA lane order (h at the padded rows, bf16), hs[m, g] summed
//             over each group's fragments in a fixed order, and the correction A
//             fragments.
//   k_sched   one workgroup: the GEMM's block schedule, column stripes of each expert
//             dealt over the XCDs, longest tiles first (see the kernel).
//   k_gemm    one wavefront per (tile, column block): 128 columns for 32-slot tiles, 64
//             for 64-slot tiles. Per k-block each lane loads 16 bytes of one row's
//             segment with a buffer load, kPD k-blocks ahead of their use; the words
//             pass through a double-buffered LDS transpose to the lanes that hold their
//             word column, which turn them into bf16 B fragments with v_perm_b32 +
//             shift/and_or, and run
//             v_mfma_f32_32x32x16_bf16. acc accumulates over all groups; at the end of
//             group g, y += (s_g - s_next) * acc, which sums to sum_g s_g * acc_g (Abel
//             summation, so acc is never cleared). Before the loop, y starts as the
//             correction sum_g [hs_hi, hs_lo, -128 hs_hi, -128 hs_lo] x [b, b, s, s]:
//             4 MFMA k-blocks per 16 groups, their B side staged in an LDS ring.
//             Epilogue: gain * y into part[token*(topk+1) + k], float4 per lane.
//   k_sum_slots  y[t] = sum over the topk+1 partials in slot order; routed slots whose
//             expert id is out of range contribute nothing.
constexpr int kGMax = 63;          // groups per expert (F/64, FS/64), one per lane
constexpr int kST = 256;           // threads of the staging kernel
// staging workgroups per tile (slot m goes to workgroup m % stage_split(MS)): 8 slots each
__host__ __device__ constexpr int stage_split(int ms) { return 4 * ms; }
constexpr int kPadRow = 0x7FFF0000;  // padding row offset: past every expert's weights
constexpr int kPD = 8;             // k-blocks in flight per wavefront (32-slot tiles); tiles pad to it
constexpr uint32_t kMagic = 0x43004300u;  // bf16 128.0 in both halves

// k-blocks per tile: at most 4 per group, plus the padding to a multiple of kPD
__host__ __device__ constexpr int kb_max(int gmx) { return 4 * gmx + kPD; }
__host__ __device__ constexpr int nch_max(int gmx) { return (gmx + 15) / 16; }

// The GEMM's block schedule. GEMM workgroup b runs on XCD b % 8 (the hardware deals
// workgroups to the XCDs in turn) and takes entry xcd_remap(b, n) of blk, so XCD x owns
// the contiguous range [start_x, start_x + q_x) of blk, q_x = n / 8 or n / 8 + 1. An
// entry is a block (tile * nblk + nb for column block nb of the tile, and the tile's
// expert), or (-1, -1): no work.
// Work is dealt by column stripe: span consecutive column blocks of one expert, 128
// bytes of each weight row (whole cache lines). The tiles of an expert read the same
// weight bytes in a stripe, so a stripe stays on one XCD with its tiles side by side in
// the dispatch order, where they share those bytes in the XCD's L2. An expert deals its
// stripes to the XCDs in turn, starting as many XCDs further on than the expert before
// it as it has stripes (so the remainders rotate), which gives every XCD nearly the same
// share of every expert. Within an XCD the experts come in descending order of their
// largest tile and then by id: the longest blocks start first and the launch ends on
// short ones. When the blocks do not fit the XCD ranges (too few empty tiles to spare),
// blk is the identity. Only the schedule depends on blk; every block writes its own
// outputs.
constexpr int kOT = 1024;
constexpr int kOrderMaxE = kOT - 1;  // experts the schedule supports (E + 1 runs <= kOT)

// LDS ints the schedule uses with NTH threads (NTH >= E + 1)
__host__ __device__ constexpr int sched_lds_ints(int nth) {
  return 14 * nth + 2 * (nth / 64) * kXcds + 2 * kXcds + 1;
}

// The schedule, computed by one workgroup of NTH threads (thread r handles run r: expert
// r, or the shared expert for r = E). The order key of an expert is its largest union
// (ucount), which k_stage turns into the tile's k-block count, group padding aside.
template <int NTH>
__device__ __forceinline__ void sched_body(int tid, int* __restrict__ lds,
                                           const int32_t* __restrict__ tile_e,
                                           const int32_t* __restrict__ ucount,
                                           int2* __restrict__ blk, int NT, int nblk, int span,
                                           int E) {
  int* rkey = lds;                    // 16-byte aligned: read as int4
  int* rlen = rkey + NTH;
  int* rmax = rlen + NTH;
  int* rrank = rmax + NTH;
  int* byrank = rrank + NTH;
  int* rcnt = byrank + NTH;
  int* base = rcnt + NTH;             // [kXcds][NTH]: blocks of the higher-ranked experts
  int* wsum = base + kXcds * NTH;     // [NTH / 64][kXcds]
  int* wbase = wsum + (NTH / 64) * kXcds;
  int* tot = wbase + (NTH / 64) * kXcds;
  int* st = tot + kXcds;              // [kXcds + 1]
  const int R = E + 1, n = NT * nblk;
  const int q = n / kXcds, rr = n % kXcds;
  rlen[tid] = 0;
  rmax[tid] = 0;
  rcnt[tid] = 0;
  byrank[tid] = -1;
  if (tid <= kXcds) st[tid] = tid < rr ? tid * (q + 1) : rr * (q + 1) + (tid - rr) * q;
  __syncthreads();
  for (int t = tid; t < NT; t += NTH) {
    const int e = tile_e[t], u = ucount[t];
    if (e < 0 || e > E) continue;
    atomicAdd(&rlen[e], 1);
    atomicMax(&rmax[e], min(max(u, 0), 0xFFFF));
  }
  __syncthreads();
  // unique keys, larger first: the largest union, then the lower id; -1 for no tiles
  rkey[tid] = tid < R && rlen[tid] > 0 ? (rmax[tid] << 10 | (NTH - 1 - tid)) : -1;
  __syncthreads();
  if (rkey[tid] >= 0) {
    const int k = rkey[tid];
    const int4* k4 = reinterpret_cast<const int4*>(rkey);
    int rk = 0;
#pragma unroll 4
    for (int r = 0; r < (R + 3) / 4; ++r) {
      const int4 u = k4[r];
      rk += (u.x > k) + (u.y > k) + (u.z > k) + (u.w > k);
    }
    rrank[tid] = rk;
    byrank[rk] = tid;
  }
  __syncthreads();
  // blocks the expert of rank tid puts on each XCD, and their exclusive prefix over ranks.
  // Stripe u (column blocks u*span ..) goes to XCD (u + off) % 8; the last may be short.
  const int U = (nblk + span - 1) / span, last = nblk - (U - 1) * span;
  int v[kXcds], inc[kXcds];
  const int off = (tid * U) & (kXcds - 1), me = byrank[tid];
#pragma unroll
  for (int x = 0; x < kXcds; ++x) {
    const int x0 = (x - off) & (kXcds - 1);
    const int nu = x0 < U ? (U - 1 - x0) / kXcds + 1 : 0;
    const int nbx = nu * span - ((U - 1) % kXcds == x0 ? span - last : 0);
    v[x] = me >= 0 ? rlen[me] * nbx : 0;
    inc[x] = v[x];
  }
  const int lane = tid & 63, wv = tid >> 6;
#pragma unroll
  for (int x = 0; x < kXcds; ++x) inc[x] = wave_incl_scan(inc[x], lane);
  if (lane == 63) {
#pragma unroll
    for (int x = 0; x < kXcds; ++x) wsum[wv * kXcds + x] = inc[x];
  }
  __syncthreads();
  if (tid < kXcds) {
    int sm = 0;
    for (int w = 0; w < NTH / 64; ++w) {
      wbase[w * kXcds + tid] = sm;
      sm += wsum[w * kXcds + tid];
    }
    tot[tid] = sm;
  }
  __syncthreads();
  bool fits = true;
#pragma unroll
  for (int x = 0; x < kXcds; ++x) {
    base[x * NTH + tid] = wbase[wv * kXcds + x] + inc[x] - v[x];
    fits = fits && tot[x] <= st[x + 1] - st[x];
  }
  __syncthreads();
  if (!fits) {  // identity: entry l is block l where its tile has an expert
    for (int l = tid; l < n; l += NTH) {
      const int e = tile_e[l / nblk];
      blk[l] = e >= 0 && e <= E ? make_int2(l, e) : make_int2(-1, -1);
    }
    return;
  }
  for (int l = tid; l < n; l += NTH) {  // the unused tail of each XCD's range
    int x = 0;
#pragma unroll
    for (int y = 1; y < kXcds; ++y) x += l >= st[y];
    if (l - st[x] >= tot[x]) blk[l] = make_int2(-1, -1);
  }
  for (int t = tid; t < NT; t += NTH) {
    const int e = tile_e[t];
    if (e < 0 || e > E) continue;
    const int k = atomicAdd(&rcnt[e], 1), i = rrank[e], L = rlen[e];
    const int o = (i * U) & (kXcds - 1);
    for (int nb = 0; nb < nblk; ++nb) {
      const int u = nb / span, j = nb - u * span, x = (u + o) & (kXcds - 1);
      blk[st[x] + base[x * NTH + i] + ((u / kXcds) * span + j) * L + k] = make_int2(t * nblk + nb, e);
    }
  }
}

// The schedule as a kernel of its own, for more experts than a staging workgroup has
// threads.
__global__ __launch_bounds__(kOT) void k_sched(const int32_t* __restrict__ tile_e,
                                               const int32_t* __restrict__ ucount,
                                               int2* __restrict__ blk, int NT, int nblk,
                                               int span, int E) {
  __shared__ __attribute__((aligned(16))) int lds[sched_lds_ints(kOT)];
  sched_body<kOT>((int)threadIdx.x, lds, tile_e, ucount, blk, NT, nblk, span, E);
}

template <int MS>
__global__ __launch_bounds__(kST) void k_stage(
    const uint16_t* __restrict__ h, const int32_t* __restrict__ tile_e,
    const int32_t* __restrict__ tile_slot, const int32_t* __restrict__ ulist,
    const int32_t* __restrict__ ucount, int32_t* __restrict__ kbg, int32_t* __restrict__ krow,
    uint4* __restrict__ hc, uint4* __restrict__ hcor, uint4* __restrict__ dump, int D, int F,
    int FS, int topk, int E, int umax, int GMX, int2* __restrict__ blk, int NT, int nblk,
    int span, int fuse, int sh0) {
  constexpr int TT = 32 * MS, kSplit = stage_split(MS), SPM = TT / kSplit;  // slots staged here
  constexpr int NUL = (kGMax * 64 + kST - 1) / kST;  // union list entries per thread
  // h rows of a gather batch, per slot GB groups x 64 values plus 8 of padding, so that
  // the slots' rows start in different LDS banks: they share the union list's space
  constexpr int GB = 16, HP = GB * 64 + 8;
  constexpr int ULS = NUL * kST > SPM * HP / 2 ? NUL * kST : SPM * HP / 2;
  __shared__ __attribute__((aligned(16))) int uls[ULS];  // the tile's union list (entries past
                                                         // its end unused)
  __shared__ int gs[kGMax + 1];    // first union position of each group
  __shared__ int kbs[kGMax + 1];   // first k-block of each group
  __shared__ __attribute__((aligned(16))) int prow[16 * kb_max(kGMax)];
  __shared__ float hsl[SPM][kGMax];
  __shared__ int kreal;            // k-blocks before the padding to a multiple of kPD
  static_assert(ULS >= sched_lds_ints(kST), "the schedule reuses the union list's LDS");
  // fuse: workgroup 0 computes the GEMM's block schedule (dispatched first, it runs
  // beside the staging workgroups), the others stage tiles
  if (fuse && blockIdx.x == 0) {
    sched_body<kST>((int)threadIdx.x, uls, tile_e, ucount, blk, NT, nblk, span, E);
    return;
  }
  // Workgroups past NT kSplit take the second half of a shared-expert tile (tiles sh0..):
  // a shared tile has twice the groups of a routed one, so its batches of GB groups (and
  // their correction chunks) alternate between two workgroups per slot set.
  const int bid = (int)blockIdx.x - fuse;
  const bool second = bid >= NT * kSplit;
  const int bb = second ? bid - NT * kSplit : bid;
  const int tile = second ? sh0 + bb / kSplit : bb / kSplit, sp = bb % kSplit, tid = threadIdx.x;
  const int nhalf = tile >= sh0 ? 2 : 1, half = second ? 1 : 0;
  const int KMX = 16 * kb_max(GMX), KBMX = kb_max(GMX), NCHMX = nch_max(GMX);
  int32_t* kbgT = kbg + (size_t)tile * (GMX + 1);
  // h is gathered in batches of GB groups: a batch is every 16-byte piece (8 per group,
  // the group's 64 values) of each of the SPM slots' rows, NLI pieces per thread.
  constexpr int NBT = (kGMax + GB - 1) / GB;
  constexpr int NLI = SPM * GB * 8 / kST;
  // Two memory round trips: the tile's expert, union size and the slots of this thread's
  // pieces; then the whole union list and every batch's pieces. Loads are never under a
  // branch (a load inside a branch makes the compiler wait for every earlier load where
  // the paths merge), and only LDS barriers follow them, so they stay in flight through
  // the list work below. A dead piece (slot not in the tile, group past the expert's end)
  // reads h[0..7]: its values reach only rows that are never written out or read.
  const int e = tile_e[tile];
  const int ucnt = ucount[tile];
  int slot[NLI];
#pragma unroll
  for (int i = 0; i < NLI; ++i) slot[i] = tile_slot[tile * TT + sp + kSplit * ((tid + kST * i) / (GB * 8))];
  if (e < 0) {
    if (sp == 0 && half == 0)
      for (int g = tid; g <= GMX; g += kST) kbgT[g] = 0;
    return;
  }
  const bool shared = e >= E;
  const int FF = shared ? FS : F, G = FF / 64;
  const int NR = topk * F + FS;
  const int U = min(max(ucnt, 0), min(umax, FF));
  const int32_t* ul = ulist + (size_t)tile * umax;
  int uv[NUL];  // entries past the list's end re-read its last slot and are unused
#pragma unroll
  for (int i = 0; i < NUL; ++i) uv[i] = ul[min(tid + kST * i, umax - 1)];
  uint4 pv[NBT][NLI];
#pragma unroll
  for (int i = 0; i < NLI; ++i) {
    const int s = slot[i];
    const int o = s < 0 ? -1 : (shared ? s * NR + topk * F : (s / topk) * NR + (s % topk) * F);
    const int item = tid + kST * i, pc = item % 8;
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) {
      const int g = GB * bt + (item / 8) % GB;
      const bool ok = o >= 0 && g < G && bt % nhalf == half;
      pv[bt][i] = *reinterpret_cast<const uint4*>(h + (ok ? (size_t)o + 64 * g + 8 * pc : 0));
    }
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < NUL; ++i) uls[tid + kST * i] = uv[i];
  lds_barrier();
  for (int g = tid; g <= G; g += kST) {  // lower bound of 64 g in the ascending list
    int lo = 0, hi = U;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (uls[mid] < 64 * g) lo = mid + 1; else hi = mid;
    }
    gs[g] = lo;
  }
  lds_barrier();
  if (tid < 64) {  // k-blocks per group, exclusive scan over the groups (one wavefront)
    const int n = tid < G ? (min(max(gs[tid + 1] - gs[tid], 0), 64) + 15) >> 4 : 0;  // <= 4
    const int incl = wave_incl_scan(n, tid);
    const int run = __builtin_amdgcn_readlane(incl, 63);
    // zero k-blocks (pad rows, A = 0) extend the last group to a multiple of kPD, so the
    // GEMM loop runs whole rounds of its prefetch ring
    const int padded = (run + kPD - 1) / kPD * kPD;
    if (tid <= G) kbs[tid] = incl - n == run ? padded : incl - n;
    if (tid == 0) kreal = run;
  }
  lds_barrier();
  const int nkb = kbs[G], nreal = kreal;
  if (sp == 0 && half == 0)
    for (int g = tid; g <= GMX; g += kST) kbgT[g] = kbs[g < G ? g : G];
  // padded row list: position 16 kbs[g] + j holds union row gs[g] + j of group g; the
  // rest of the group's k-blocks and the trailing zero k-blocks are padding
#pragma unroll 4
  for (int it = tid; it < 64 * G; it += kST) {
    const int g = it >> 6, j = it & 63;
    const int nb_g = min(kbs[g + 1], nreal) - kbs[g];  // real k-blocks of group g
    if (j >= 16 * nb_g) continue;
    const int p = 16 * kbs[g] + j;
    int r = -1;
    if (j < min(max(gs[g + 1] - gs[g], 0), 64)) {
      r = uls[gs[g] + j];
      if ((unsigned)r >= (unsigned)FF) r = -1;
    }
    prow[p] = r;
    if (sp == 0 && half == 0) krow[(size_t)tile * KMX + p] = r >= 0 ? r * (D / 2) : kPadRow;
  }
  for (int p = 16 * nreal + tid; p < 16 * nkb; p += kST) {
    prow[p] = -1;
    if (sp == 0 && half == 0) krow[(size_t)tile * KMX + p] = kPadRow;
  }
  lds_barrier();
  // A fragments, a batch of GB groups at a time: its pieces (loaded above) go to LDS over
  // the union list, no longer needed, and the 8 lanes of a (slot, group) sum hs[m, g] in a
  // fixed butterfly order (a column outside the union is zero in every slot of the tile,
  // so the sum over the row is the sum over the union); then each fragment (slot,
  // k-block, half) picks its 8 padded rows from LDS.
  uint16_t* hbuf = reinterpret_cast<uint16_t*>(uls);  // [SPM][HP]: group gl at gl * 64
#pragma unroll
  for (int bt = 0; bt < NBT; ++bt) {
    const int g0 = GB * bt;
    if (g0 >= G) break;
    if (bt % nhalf != half) continue;  // the other workgroup's batch (uniform)
    lds_barrier();  // the previous batch is assembled (the union list read)
#pragma unroll
    for (int i = 0; i < NLI; ++i) {
      const int item = tid + kST * i, jj = item / (GB * 8), gl = (item / 8) % GB, pc = item % 8;
      *reinterpret_cast<uint4*>(&hbuf[jj * HP + gl * 64 + 8 * pc]) = pv[bt][i];
      const uint32_t w[4] = {pv[bt][i].x, pv[bt][i].y, pv[bt][i].z, pv[bt][i].w};
      float s8 = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) s8 += bf16_bits_to_f32((j & 1) ? w[j >> 1] >> 16 : w[j >> 1] & 0xFFFFu);
      // the 8-lane sum with DPP (quad_perm xor 1, xor 2, then the other quad of the 8 by
      // row_half_mirror), no LDS permute
      s8 += dpp_f32<0xB1>(s8);
      s8 += dpp_f32<0x4E>(s8);
      s8 += dpp_f32<0x141>(s8);
      if (pc == 0 && g0 + gl < G) hsl[jj][g0 + gl] = s8;
    }
    lds_barrier();
    // A batch has at most 4 k-blocks per group, so NFR fragments per thread. All are made,
    // then all are stored, fragments past the batch's end to a dump row: the number of
    // stores is fixed, so the waits for later batches' pieces never wait for these stores
    // (the hardware counts loads and stores together, in issue order).
    const int kb0 = kbs[g0], nfr = (min(kbs[min(g0 + GB, G)], nreal) - kb0) * SPM * 2;
    constexpr int NFR = 4 * GB * SPM * 2 / kST;
    uint4 fr[NFR];
    uint4* dst[NFR];
#pragma unroll
    for (int f = 0; f < NFR; ++f) {
      const int it = tid + kST * f;
      const bool live = it < nfr;
      const int kb = kb0 + (live ? it / (2 * SPM) : 0), jj = (it >> 1) % SPM, half = it & 1;
      const int4 r0 = *reinterpret_cast<const int4*>(&prow[16 * kb + 8 * half]);
      const int4 r1 = *reinterpret_cast<const int4*>(&prow[16 * kb + 8 * half + 4]);
      const int r[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
      uint32_t v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)  // a union row r of this batch: group r / 64, column r % 64
        v[i] = live && r[i] >= 0 ? hbuf[jj * HP + r[i] - 64 * g0] : 0u;
      const int m = sp + kSplit * jj;
      fr[f] = make_uint4(v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16),
                         v[6] | (v[7] << 16));
      dst[f] = live ? hc + (((size_t)tile * KBMX + kb) * MS + (m >> 5)) * 64 + (m & 31) + 32 * half
                    : dump + tid;
    }
#pragma unroll
    for (int f = 0; f < NFR; ++f) *dst[f] = fr[f];
  }
  // the padding k-blocks (at most kPD - 1) hold zero fragments
  for (int it = tid; it < (half == 0 ? nkb - nreal : 0) * SPM * 2; it += kST) {
    const int kb = nreal + it / (2 * SPM), jj = (it >> 1) % SPM, half = it & 1;
    const int m = sp + kSplit * jj;
    hc[(((size_t)tile * KBMX + kb) * MS + (m >> 5)) * 64 + (m & 31) + 32 * half] = make_uint4(0, 0, 0, 0);
  }
  lds_barrier();
  // correction A fragments of this workgroup's slots, 16 groups per chunk: sections
  // [hs_hi, hs_lo, -128 hs_hi, -128 hs_lo]; hs = hs_hi + hs_lo to about 16 bits, -128 x
  // is exact in bf16
  static_assert(GB == 16, "a correction chunk (16 groups) is one gather batch");
  const int NCH = (G + 15) >> 4;
  for (int it = tid; it < NCH * 4 * SPM * 2; it += kST) {
    const int khalf = it & 1, jj = (it >> 1) % SPM, sec = (it / (2 * SPM)) & 3,
              ch = it / (8 * SPM);
    if (ch % nhalf != half) continue;  // the other workgroup's chunk: its groups' hs
    const int m = sp + kSplit * jj;
    uint32_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int g = 16 * ch + 8 * khalf + i;
      const float s = g < G ? hsl[jj][g] : 0.0f;
      const uint16_t hi = f32_to_bf16_bits(s);
      uint16_t b = (sec & 1) ? f32_to_bf16_bits(s - bf16_bits_to_f32(hi)) : hi;
      if (sec >= 2) b = f32_to_bf16_bits(-128.0f * bf16_bits_to_f32(b));
      v[i] = b;
    }
    hcor[((((size_t)tile * NCHMX + ch) * 4 + sec) * MS + (m >> 5)) * 64 + (m & 31) + 32 * khalf] =
        make_uint4(v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16),
                   v[6] | (v[7] << 16));
  }
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return __builtin_bit_cast(bf16x8, make_uint4(a, b, c, d));
}
__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

template <int MS>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm(
    const int32_t* __restrict__ tile_slot, const float* __restrict__ gains,
    const int32_t* __restrict__ kbg,
    const int32_t* __restrict__ krow, const uint4* __restrict__ hc,
    const uint4* __restrict__ hcor, const uint32_t* __restrict__ pw,
    const uint16_t* __restrict__ ps, const uint16_t* __restrict__ pb,
    const uint32_t* __restrict__ spw, const uint16_t* __restrict__ sps,
    const uint16_t* __restrict__ spb, float* __restrict__ part, const int2* __restrict__ blk,
    int D, int F, int FS, int topk, int E, int NT, int GMX) {
  constexpr int TT = 32 * MS, NWC = 16 / MS, NMF = 4 / MS, NCOL = 8 * NWC;
  // The correction ring: per column 8 blocks of 8 bf16 (RP = 64), of which 4 are used (b of
  // groups 0-7, 8-15, s of groups 0-7, 8-15); block beta of column col sits at block
  // beta ^ (col / 8 % 8), so the 16 columns that one write instruction covers (8 apart)
  // fall in different LDS banks.
  constexpr int RP = 64;
  // LDS: first the correction ring [NCOL][RP], then the scale table [G][NCOL] of this block
  constexpr int kLds = NCOL * RP > kGMax * NCOL ? NCOL * RP : kGMax * NCOL;
  __shared__ __attribute__((aligned(16))) uint16_t ring[kLds];
  // k-block words in transit: [word column][row], pitch 20 (with the row swizzle of put
  // and get, their 4-byte writes and 16-byte reads are free of bank conflicts)
  constexpr int TP = 20;
  __shared__ __attribute__((aligned(16))) uint32_t tbuf[2][NWC * TP];  // double buffered
  constexpr int PD = MS == 1 ? kPD : kPD / 2;  // register ring depth (a divisor of kPD)
  constexpr int LPR = NWC / 4;                 // lanes loading one row segment, 16 B each
  const int nblk = D / NCOL;
  const int2 bv = blk[xcd_remap((int)blockIdx.x, NT * nblk)];  // (tile * nblk + nb, expert)
  if (bv.x < 0 || bv.y < 0) return;
  const int tile = bv.x / nblk, nb = bv.x - (bv.x / nblk) * nblk;
  const int e = bv.y;
  const bool shared = e >= E;
  const int FF = shared ? FS : F, G = FF / 64;
  const int l = threadIdx.x, khalf = l >> 5, c = (l & 31) % NWC, jq = (l & 31) / NWC;
  const int KMX = 16 * kb_max(GMX), KBMX = kb_max(GMX), NCHMX = nch_max(GMX);
  const int n0 = nb * NCOL;
  const int lcol = 8 * c + NMF * jq;  // first of this lane's NMF columns within the block
  // the partial row and gain of slot l of the tile (lanes past TT repeat a slot), loaded
  // here and passed to the epilogue through LDS
  __shared__ int2 sinfo[TT];
  const int sl = tile_slot[(size_t)tile * TT + (l & (TT - 1))];
  const int gi = sl < 0 ? -1 : shared ? sl * (topk + 1) + topk : (sl / topk) * (topk + 1) + (sl % topk);
  const float gn = gains[max(gi, 0)];
  // The correction's first chunk (below) depends on the tile and expert only: its loads
  // go out now, with the tile's group starts and slots.
  const uint16_t* sb = (shared ? sps : ps + (size_t)e * (F / 64) * D) + n0 + lcol;
  const uint16_t* bb = (shared ? spb : pb + (size_t)e * (F / 64) * D) + n0 + lcol;
  const uint4* hq = hcor + (size_t)tile * NCHMX * 4 * MS * 64 + l;
  const int NCH = (G + 15) >> 4;
  constexpr int V8 = NCOL / 8;       // uint4 pieces per row segment
  constexpr int NIT = 32 * V8 / 64;  // 32 row segments (b, s of 16 groups)
  auto load_chunk = [&](int ch, uint4 (&a)[4][MS], uint4 (&v)[NIT]) {
#pragma unroll
    for (int sec = 0; sec < 4; ++sec)
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) a[sec][ms] = hq[(((size_t)ch * 4 + sec) * MS + ms) * 64];
#pragma unroll
    for (int t = 0; t < NIT; ++t) {
      const int item = l + 64 * t, r = item / V8, c8 = item % V8;
      const int gg = min(16 * ch + (r & 15), G - 1);
      v[t] = *reinterpret_cast<const uint4*>((r < 16 ? bb : sb) - lcol + (size_t)gg * D + 8 * c8);
    }
  };
  uint4 a0[4][MS], v0[NIT], a1[4][MS], v1[NIT];
  load_chunk(0, a0, v0);
  // the tile's k-block group starts: with the first round trip too (unconditional loads)
  const int32_t* kbgT = kbg + (size_t)tile * (GMX + 1);
  const int kv0 = kbgT[min(l, G)], kn0 = kbgT[min(l + 1, G)];
  f32x16 y[MS][NMF];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int i = 0; i < NMF; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) y[ms][i][v] = 0.0f;

  // The correction sum_g [hs_hi, hs_lo, -128 hs_hi, -128 hs_lo] x [b, b, s, s], 16 groups
  // at a time: the groups' b and s rows of this column block go through the LDS ring
  // [column][b of 16 groups | s of 16 groups | pad], then 4 MFMA k-blocks start y. The
  // next chunk's loads are in flight while a chunk is processed. Loads are never
  // conditional (a branch around a load makes the compiler wait for every load at the
  // merge): rows past G re-read row G - 1 and are zeroed, chunks past the last re-read it.
  auto process = [&](int ch, const uint4 (&a)[4][MS], const uint4 (&v)[NIT]) {
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NIT; ++t) {
      const int item = l + 64 * t, r = item / V8, c8 = item % V8;
      const bool live = 16 * ch + (r & 15) < G;
      const uint32_t w[4] = {live ? v[t].x : 0u, live ? v[t].y : 0u, live ? v[t].z : 0u,
                             live ? v[t].w : 0u};
#pragma unroll
      for (int j = 0; j < 8; ++j)
        ring[(8 * c8 + j) * RP + 8 * (((r >> 3) & 3) ^ (c8 & 7)) + (r & 7)] =
            (uint16_t)((j & 1) ? w[j >> 1] >> 16 : w[j >> 1]);
    }
    __syncthreads();
#pragma unroll
    for (int sec = 0; sec < 4; ++sec)
#pragma unroll
      for (int i = 0; i < NMF; ++i) {
        const int col = lcol + i, beta = 2 * (sec >> 1) + khalf;
        const uint4 bv = *reinterpret_cast<const uint4*>(&ring[col * RP + 8 * (beta ^ ((col >> 3) & 7))]);
#pragma unroll
        for (int ms = 0; ms < MS; ++ms)
          y[ms][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a[sec][ms]), as_bf16x8(bv), y[ms][i], 0, 0, 0);
      }
  };
  // Chunks go in pairs; a chunk past the last one (odd NCH) has all rows zeroed and adds
  // exact zeros. Nothing is conditional, so no load sinks into a branch, and the
  // scheduling barriers keep each chunk's loads ahead of the work before them. The
  // correction runs for every tile: with no k-block, hs and so y are zero.
  {
    for (int ch = 0; ch < NCH; ch += 2) {
      load_chunk(min(ch + 1, NCH - 1), a1, v1);
      __builtin_amdgcn_sched_barrier(0);
      process(ch, a0, v0);
      load_chunk(min(ch + 2, NCH - 1), a0, v0);
      __builtin_amdgcn_sched_barrier(0);
      process(ch + 1, a1, v1);
    }
  }

  const int kv = l <= G ? kv0 : 0;
  const int kn = l < G ? kn0 : 0;
  const uint64_t nonempty = __ballot(l < G && kn > kv);
  // k-blocks of this tile: a multiple of kPD and at most kb_max(G) by construction; the
  // clamp keeps a corrupted workspace from driving the loop out of its buffers
  const int nkb = min(max(__builtin_amdgcn_readlane(kv, G), 0), kb_max(G)) / kPD * kPD;

  if (nkb > 0) {
    f32x16 acc[MS][NMF];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int i = 0; i < NMF; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[ms][i][v] = 0.0f;
    const uint32_t* wb = shared ? spw : pw + (size_t)e * F * (D / 8);
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc((void*)wb, (short)0, FF * (D / 2), 0x00020000);
    const int lr = (l / LPR) & 15, la = l % LPR;     // this lane's row and 16-byte piece
    const uint32_t colbyte = (uint32_t)(n0 / 8) * 4u + 16u * (uint32_t)la;
    // the nibble mask as an opaque register, so (x & mask) | magic is one v_and_or_b32
    // (two literal operands would not fit the instruction)
    uint32_t nmask;
    asm volatile("v_mov_b32 %0, 0xf000f" : "=v"(nmask));
    const uint32_t bsel = MS == 1 ? 2u * jq : (uint32_t)jq;
    const uint32_t psel = MS == 1 ? (bsel | (bsel + 1) << 8 | (bsel + 4) << 16 | (bsel + 5) << 24)
                                  : (bsel | 0x0C00u | (bsel + 4) << 16 | 0x0C000000u);
    const int32_t* kr = krow + (size_t)tile * KMX + lr;
    const uint4* ha = hc + (size_t)tile * KBMX * MS * 64 + l;

    // the scale table s[g][n0 .. n0 + NCOL) of all groups, so that the k-block loop issues
    // no global load inside its group-end branch: every load first, then the stores.
    // Pieces past the table repeat its last piece (same source, same place).
    {
      constexpr int NST = (kGMax * V8 + 63) / 64;
      uint32_t sv[NST][4];
      __syncthreads();
#pragma unroll
      for (int t = 0; t < NST; ++t) {
        const int idx = min(l + 64 * t, G * V8 - 1), gg = idx / V8, c8 = idx % V8;
        const uint4 u = *reinterpret_cast<const uint4*>(sb - lcol + (size_t)gg * D + 8 * c8);
        sv[t][0] = u.x; sv[t][1] = u.y; sv[t][2] = u.z; sv[t][3] = u.w;
      }
#pragma unroll
      for (int t = 0; t < NST; ++t)  // piece idx = (g, c8) goes to ring[g * NCOL + 8 * c8]
        *reinterpret_cast<uint4*>(&ring[8 * min(l + 64 * t, G * V8 - 1)]) =
            make_uint4(sv[t][0], sv[t][1], sv[t][2], sv[t][3]);
    }
    __syncthreads();
    auto scales = [&](int g, float (&s)[NMF]) {  // this lane's NMF scales of group g
      uint32_t w[NMF / 2];
      if constexpr (NMF == 4) {
        const uint2 v = *reinterpret_cast<const uint2*>(&ring[g * NCOL + lcol]);
        w[0] = v.x; w[1] = v.y;
      } else {
        w[0] = *reinterpret_cast<const uint32_t*>(&ring[g * NCOL + lcol]);
      }
#pragma unroll
      for (int i = 0; i < NMF; ++i) s[i] = bf16_bits_to_f32((i & 1) ? w[i >> 1] >> 16 : w[i >> 1] & 0xFFFFu);
    };
    // group state: current group g, its end k-block, its scales
    int g = __builtin_ctzll(nonempty);
    int gend = __builtin_amdgcn_readlane(kn, g);
    float scur[NMF];
    scales(g, scur);

    // Register ring of PD k-blocks: per lane one row offset, one 16-byte piece of a row
    // segment (4 lanes per 64-byte segment) and the A fragment(s). A k-block's words
    // reach their lanes through tbuf one step before use.
    int rq[PD];
    uint4 wq[PD];
    uint4 aq[PD][MS];
    // A k-block's words reach their lanes through tbuf: k-block kb is written to
    // tbuf[kb & 1] LA + 1 steps before its use and read back LA steps before it, into
    // w8[kb % LA], so the LDS round trip hides behind LA steps of work. One wavefront per
    // workgroup executes its LDS operations in order.
    constexpr int LA = PD >= 8 ? 2 : 1;
    uint32_t w8[LA][8];  // this lane's 8 words (rows 8 khalf + 0..7, word column c)
    auto load_row = [&](int kb, int& r) { r = kr[16 * kb]; };
    auto load_kb = [&](int kb, int r, uint4& w, uint4 (&a)[MS]) {
      // 16-byte aligned: row offsets are multiples of D/2 = 16 * D/32, colbyte of 16
      w = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, (uint32_t)r + colbyte, 0, 0));
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) a[ms] = ha[((size_t)kb * MS + ms) * 64];
    };
    // word column w keeps its rows at [w][row ^ 8 (w / 8 % 2)]: the 8-row halves of
    // columns 8-15 are swapped, so that the four 16-byte pieces of a row (words 4 la ..)
    // that one write instruction covers fall in different LDS banks
    auto put = [&](int buf, const uint4& w) {  // row lr, words 4 la .. 4 la + 3
      const int pr = lr ^ (8 * ((la >> 1) & 1));
      tbuf[buf][(4 * la + 0) * TP + pr] = w.x;
      tbuf[buf][(4 * la + 1) * TP + pr] = w.y;
      tbuf[buf][(4 * la + 2) * TP + pr] = w.z;
      tbuf[buf][(4 * la + 3) * TP + pr] = w.w;
    };
    auto get = [&](int buf, uint32_t (&w)[8]) {  // this lane's rows 8 khalf + 0..7 of column c
      const int ph = 8 * (khalf ^ ((c >> 3) & 1));
      const uint4 u0 = *reinterpret_cast<const uint4*>(&tbuf[buf][c * TP + ph]);
      const uint4 u1 = *reinterpret_cast<const uint4*>(&tbuf[buf][c * TP + ph + 4]);
      w[0] = u0.x; w[1] = u0.y; w[2] = u0.z; w[3] = u0.w;
      w[4] = u1.x; w[5] = u1.y; w[6] = u1.z; w[7] = u1.w;
    };
    // Prefetches past the last k-block re-read the last one (in bounds, never used), so
    // every path issues the same loads and the waits stay partial.
    const int klast = nkb - 1;
#pragma unroll
    for (int d = 0; d < PD; ++d) load_row(min(d, klast), rq[d]);
    // issue order = consumption order (slot 0 first), so the loop's waits stay partial
#pragma unroll
    for (int d = 0; d < PD; ++d) {
      __builtin_amdgcn_sched_barrier(0);
      load_kb(min(d, klast), rq[d], wq[d], aq[d]);
      load_row(min(d + PD, klast), rq[d]);
    }
    __builtin_amdgcn_sched_barrier(0);
    put(0, wq[0]);
    put(1, wq[1]);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < LA; ++j) get(j, w8[j]);
    __builtin_amdgcn_wave_barrier();
    if constexpr (LA == 2) put(0, wq[2]);

    for (int kb0 = 0; kb0 < nkb; kb0 += PD) {
#pragma unroll
      for (int d = 0; d < PD; ++d) {  // nkb is a multiple of PD
        const int kb = kb0 + d;
        // B fragments: P_i holds column lcol + i of rows (2p, 2p+1) as bf16 128 + q
        uint32_t bf[NMF][4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint32_t x = __builtin_amdgcn_perm(w8[d % LA][2 * p + 1], w8[d % LA][2 * p], psel);
#pragma unroll
          for (int i = 0; i < NMF; ++i) bf[i][p] = ((x >> (4 * i)) & nmask) | kMagic;
        }
#pragma unroll
        for (int i = 0; i < NMF; ++i) {
          const bf16x8 bv = as_bf16x8(bf[i][0], bf[i][1], bf[i][2], bf[i][3]);
#pragma unroll
          for (int ms = 0; ms < MS; ++ms)
            acc[ms][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(aq[d][ms]), bv, acc[ms][i], 0, 0, 0);
        }
        load_kb(min(kb + PD, klast), rq[d], wq[d], aq[d]);
        load_row(min(kb + 2 * PD, klast), rq[d]);
        // The wave barriers order the lanes' LDS accesses for the compiler and document
        // the wavefront-synchronous exchange (no instruction is emitted).
        put((d + 1 + LA) & 1, wq[(d + 1 + LA) % PD]);  // k-block kb + LA + 1
        __builtin_amdgcn_wave_barrier();
        get((d + LA) & 1, w8[d % LA]);                 // k-block kb + LA (written a step ago)
        __builtin_amdgcn_wave_barrier();
        if (kb + 1 == gend) {  // end of group g: y += (s_g - s_next) * acc
          const uint64_t rest = nonempty & ~((2ull << g) - 1ull);
          const int gp = rest ? __builtin_ctzll(rest) : -1;
          float sn[NMF], ds[NMF];
          scales(gp >= 0 ? gp : g, sn);
#pragma unroll
          for (int i = 0; i < NMF; ++i) {
            if (gp < 0) sn[i] = 0.0f;
            ds[i] = scur[i] - sn[i];
            scur[i] = sn[i];
          }
#pragma unroll
          for (int ms = 0; ms < MS; ++ms)
#pragma unroll
            for (int i = 0; i < NMF; ++i)
#pragma unroll
              for (int v = 0; v < 16; ++v) y[ms][i][v] = fmaf(ds[i], acc[ms][i][v], y[ms][i][v]);
          if (gp >= 0) {
            g = gp;
            gend = __builtin_amdgcn_readlane(kn, g);
          }
        }
      }
    }
  }

  // epilogue: C[i][j], j = lane%32 -> column lcol + i, row 32 ms + 8 (v/4) + 4 (lane/32) + v%4
  if (l < TT) sinfo[l] = make_int2(gi, __float_as_int(gn));
  __syncthreads();
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int2 si = sinfo[32 * ms + 8 * (v >> 2) + 4 * khalf + (v & 3)];
      if (si.x < 0) continue;
      const float gn = __int_as_float(si.y);
      float* dst = part + (size_t)si.x * D + n0 + lcol;
      if constexpr (NMF == 4)
        *reinterpret_cast<float4*>(dst) =
            make_float4(gn * y[ms][0][v], gn * y[ms][1][v], gn * y[ms][2][v], gn * y[ms][3][v]);
      else
        *reinterpret_cast<float2*>(dst) = make_float2(gn * y[ms][0][v], gn * y[ms][1][v]);
    }
}

// One thread per 4 consecutive outputs of a token. K > 0: topk known at compile time, all
// ids and partials are loaded before any is used (out-of-range slots are dropped by a
// select, not a branch around a load); K == 0: any topk.
template <int YDT, int K>
__global__ __launch_bounds__(256) void k_sum_slots(const float* __restrict__ part,
                                                   const int32_t* __restrict__ sel,
                                                   typename Elem<YDT>::T* __restrict__ y, int T,
                                                   int D, int topk, int E) {
  const int D4 = D / 4;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)T * D4) return;
  const size_t t = idx / D4, o = (idx - t * D4) * 4;
  const float4* p = reinterpret_cast<const float4*>(part + t * (topk + 1) * D + o);
  const int32_t* st = sel + t * topk;
  auto add = [](float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); };
  float4 s;
  if constexpr (K > 0) {
    int e[K];
    float4 v[K + 1];
#pragma unroll
    for (int k = 0; k < K; ++k) e[k] = st[k];
#pragma unroll
    for (int k = 0; k <= K; ++k) v[k] = p[(size_t)k * D4];
    s = (unsigned)e[0] < (unsigned)E ? v[0] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int k = 1; k < K; ++k) s = (unsigned)e[k] < (unsigned)E ? add(s, v[k]) : s;
    s = add(s, v[K]);
  } else {
    s = (unsigned)st[0] < (unsigned)E ? p[0] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int k = 1; k < topk; ++k)
      if ((unsigned)st[k] < (unsigned)E) s = add(s, p[(size_t)k * D4]);
    s = add(s, p[(size_t)topk * D4]);
  }
  const size_t yo = t * D + o;
  Elem<YDT>::store(y, yo, s.x);
  Elem<YDT>::store(y, yo + 1, s.y);
  Elem<YDT>::store(y, yo + 2, s.z);
  Elem<YDT>::store(y, yo + 3, s.w);
}

}  // namespace
}  // namespace hsd

using namespace hsd;

extern "C" int64_t hsd_prefill_num_tiles(int64_t T, int64_t topk, int64_t E, int64_t tt) {
  if (T <= 0 || topk <= 0 || E <= 0 || tt <= 0) return 0;
  return T * topk / tt + E + (T + tt - 1) / tt;
}

extern "C" size_t hsd_prefill_tiles_workspace_bytes(int64_t T, int64_t topk, int64_t E) {
  (void)E;
  if (T <= 0 || topk <= 0) return 0;
  return ((size_t)T * topk * sizeof(int32_t) + 255) & ~(size_t)255;
}

extern "C" int hsd_prefill_tiles(const int32_t* sel, int64_t T, int64_t topk, int64_t E,
                                 int64_t tt, int32_t* tile_e, int32_t* tile_slot,
                                 int32_t* dev_status, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  const char* fn = "hsd_prefill_tiles";
  if (!sel || !tile_e || !tile_slot) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (T <= 0 || topk <= 0 || E <= 0 || tt <= 0 || tt > 64)
    return set_error(HSD_ERR_SHAPE, "%s: need T, topk, E > 0 and 0 < tt <= 64", fn);
  if (T * topk > (1 << 24) || E > 4096) return set_error(HSD_ERR_SHAPE, "%s: sizes too large", fn);
  const size_t need = hsd_prefill_tiles_workspace_bytes(T, topk, E);
  if (!workspace || workspace_bytes < need)
    return set_error(HSD_ERR_WORKSPACE, "%s: workspace needs %zu bytes", fn, need);
  // four chunks of 1024 slots per pass when their per-wave counts fit in 64 KB of LDS
  const int P = (2 * E + 1 + 4 * 16 * E) * sizeof(int) <= 65536 ? 4 : 1;
  const size_t lds = (size_t)(2 * E + 1 + P * 16 * E) * sizeof(int);
  if (lds > 65536) return set_error(HSD_ERR_SHAPE, "%s: E too large for LDS", fn);
  hipLaunchKernelGGL(k_tiles, dim3(1), dim3(kTT), lds, as_stream(stream), sel, (int)T, (int)topk,
                     (int)E, (int)tt, P, tile_e, tile_slot, dev_status,
                     reinterpret_cast<int32_t*>(workspace));
  return check_launch(fn);
}

extern "C" int hsd_prefill_union(const void* h, int h_dtype, const int32_t* tile_e,
                                 const int32_t* tile_slot, int32_t* ulist, int32_t* ucount,
                                 int64_t T, int64_t F, int64_t FS, int64_t topk, int64_t E,
                                 int64_t tt, int64_t NT, int64_t umax, void* stream) {
  const char* fn = "hsd_prefill_union";
  if (!h || !tile_e || !tile_slot || !ulist || !ucount) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (T <= 0 || F <= 0 || FS <= 0 || topk <= 0 || E <= 0 || tt <= 0 || tt > 64 || NT <= 0)
    return set_error(HSD_ERR_SHAPE, "%s: bad sizes", fn);
  if (F % 8 || FS % 8) return set_error(HSD_ERR_SHAPE, "%s: F and FS must be multiples of 8", fn);
  if (umax < FS || umax < F) return set_error(HSD_ERR_SHAPE, "%s: umax must be >= FS and F", fn);
  if (NT != hsd_prefill_num_tiles(T, topk, E, tt)) return set_error(HSD_ERR_SHAPE, "%s: NT mismatch", fn);
  if ((topk * F + FS) * T > ((int64_t)1 << 31)) return set_error(HSD_ERR_SHAPE, "%s: sizes too large", fn);
  if ((uintptr_t)h & 15u) return set_error(HSD_ERR_ALIGN, "%s: h must be 16-byte aligned", fn);
  hipStream_t st = as_stream(stream);
  switch (h_dtype) {
#define HSD_UNION(DT)                                                                             \
  case DT:                                                                                        \
    hipLaunchKernelGGL(k_union<DT>, dim3((unsigned)NT), dim3(kUT), 0, st,                        \
                       reinterpret_cast<const typename Elem<DT>::T*>(h), tile_e, tile_slot, ulist, \
                       ucount, (int)F, (int)FS, (int)topk, (int)E, (int)tt, (int)umax);           \
    break;
    HSD_UNION(HSD_DT_BF16)
    HSD_UNION(HSD_DT_F16)
    HSD_UNION(HSD_DT_F32)
#undef HSD_UNION
    default: return set_error(HSD_ERR_DTYPE, "%s: h_dtype %d", fn, h_dtype);
  }
  return check_launch(fn);
}

namespace {
// Workspace of hsd_prefill_gemm, in this order, each piece 256-byte aligned:
//   part [T*(topk+1), D] f32 | kbg [NT, GMX+1] i32 | krow [NT, 16 KB] i32 |
//   hc [NT, KB, MS, 64] uint4 | hcor [NT, ceil(GMX/16), 4, MS, 64] uint4 |
//   blk [NT * D * MS / 128] int2 (the GEMM's block schedule) | dump [256] uint4 (staging
//   stores of unused fragments), KB = kb_max(GMX)
struct GemmWs {
  size_t part, kbg, krow, hc, hcor, blk, dump, total;
};
inline size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }
GemmWs gemm_ws(int64_t T, int64_t D, int64_t F, int64_t FS, int64_t topk, int64_t E, int64_t tt) {
  GemmWs w{};
  const int64_t NT = hsd_prefill_num_tiles(T, topk, E, tt);
  const int64_t GMX = (F > FS ? F : FS) / 64, MS = tt / 32;
  w.part = 0;
  w.kbg = al256((size_t)T * (topk + 1) * D * sizeof(float));
  w.krow = w.kbg + al256((size_t)NT * (GMX + 1) * sizeof(int32_t));
  w.hc = w.krow + al256((size_t)NT * 16 * kb_max((int)GMX) * sizeof(int32_t));
  w.hcor = w.hc + al256((size_t)NT * kb_max((int)GMX) * MS * 64 * sizeof(uint4));
  w.blk = w.hcor + al256((size_t)NT * nch_max((int)GMX) * 4 * MS * 64 * sizeof(uint4));
  w.dump = w.blk + al256((size_t)NT * (D * MS / 128) * sizeof(int2));
  w.total = w.dump + al256((size_t)kST * sizeof(uint4));
  return w;
}
}  // namespace

extern "C" size_t hsd_prefill_gemm_workspace_bytes(int64_t T, int64_t D, int64_t F, int64_t FS,
                                                   int64_t topk, int64_t E, int64_t tt) {
  if (T <= 0 || D <= 0 || F <= 0 || FS <= 0 || topk <= 0 || E <= 0 || (tt != 32 && tt != 64))
    return 0;
  return gemm_ws(T, D, F, FS, topk, E, tt).total;
}

extern "C" int hsd_prefill_gemm(const uint16_t* h, const int32_t* sel, const float* gains,
                                const int32_t* tile_e, const int32_t* tile_slot,
                                const int32_t* ulist, const int32_t* ucount, const uint32_t* pw,
                                const uint16_t* ps, const uint16_t* pb, const uint32_t* spw,
                                const uint16_t* sps, const uint16_t* spb, void* y, int y_dtype,
                                int64_t T, int64_t D, int64_t F, int64_t FS, int64_t topk,
                                int64_t E, int64_t tt, int64_t NT, int64_t umax, void* workspace,
                                size_t workspace_bytes, void* stream) {
  const char* fn = "hsd_prefill_gemm";
  if (!h || !sel || !gains || !tile_e || !tile_slot || !ulist || !ucount || !pw || !ps || !pb ||
      !spw || !sps || !spb || !y)
    return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (tt != 32 && tt != 64) return set_error(HSD_ERR_SHAPE, "%s: tt must be 32 or 64", fn);
  if (T <= 0 || D <= 0 || D % 128 || F <= 0 || F % 64 || FS <= 0 || FS % 64 || topk <= 0 || E <= 0)
    return set_error(HSD_ERR_SHAPE, "%s: need D %% 128 == 0, F %% 64 == 0, FS %% 64 == 0", fn);
  if (F / 64 > kGMax || FS / 64 > kGMax)
    return set_error(HSD_ERR_SHAPE, "%s: F and FS must be <= %d", fn, 64 * kGMax);
  if (NT != hsd_prefill_num_tiles(T, topk, E, tt)) return set_error(HSD_ERR_SHAPE, "%s: NT mismatch", fn);
  if (umax < FS || umax < F) return set_error(HSD_ERR_SHAPE, "%s: umax must be >= FS", fn);
  if (E > kOrderMaxE) return set_error(HSD_ERR_SHAPE, "%s: at most %d experts", fn, kOrderMaxE);
  if (NT * (D / 64) > 0x7FFFFFFF || (topk * F + FS) * T > ((int64_t)1 << 31) ||
      (int64_t)(F > FS ? F : FS) * (D / 2) >= (int64_t)kPadRow)
    return set_error(HSD_ERR_SHAPE, "%s: sizes too large", fn);
  const uintptr_t al = (uintptr_t)ps | (uintptr_t)pb | (uintptr_t)sps | (uintptr_t)spb;
  if (al & 15u) return set_error(HSD_ERR_ALIGN, "%s: scales/biases must be 16-byte aligned", fn);
  if ((uintptr_t)h & 15u) return set_error(HSD_ERR_ALIGN, "%s: h must be 16-byte aligned", fn);
  const GemmWs w = gemm_ws(T, D, F, FS, topk, E, tt);
  if (!workspace || workspace_bytes < w.total)
    return set_error(HSD_ERR_WORKSPACE, "%s: workspace needs %zu bytes", fn, w.total);
  hipStream_t st = as_stream(stream);
  char* ws = reinterpret_cast<char*>(workspace);
  float* part = reinterpret_cast<float*>(ws + w.part);
  int32_t* kbg = reinterpret_cast<int32_t*>(ws + w.kbg);
  int32_t* krow = reinterpret_cast<int32_t*>(ws + w.krow);
  uint4* hc = reinterpret_cast<uint4*>(ws + w.hc);
  uint4* hcor = reinterpret_cast<uint4*>(ws + w.hcor);
  int2* blk = reinterpret_cast<int2*>(ws + w.blk);
  uint4* dump = reinterpret_cast<uint4*>(ws + w.dump);
  const int GMX = (int)((F > FS ? F : FS) / 64);
  // The schedule runs inside the staging launch (its workgroup 0) when a staging
  // workgroup has a thread per expert; otherwise as a kernel of its own.
  const int fuse = E + 1 <= kST ? 1 : 0;
  const int MS = tt == 32 ? 1 : 2;
  const int nblk = (int)(D / (128 / MS)), span = 2 * MS;
  if (!fuse) {
    hipLaunchKernelGGL(k_sched, dim3(1), dim3(kOT), 0, st, tile_e, ucount, blk, (int)NT, nblk,
                       span, (int)E);
    const int rc = check_launch(fn);
    if (rc) return rc;
  }
  const int64_t nt_shared = (T + tt - 1) / tt, sh0 = NT - nt_shared;
  const dim3 sgrid((unsigned)((NT + nt_shared) * stage_split(MS) + fuse));
  if (MS == 1)
    hipLaunchKernelGGL(k_stage<1>, sgrid, dim3(kST), 0, st, h, tile_e, tile_slot, ulist, ucount, kbg,
                       krow, hc, hcor, dump, (int)D, (int)F, (int)FS, (int)topk, (int)E, (int)umax,
                       GMX, blk, (int)NT, nblk, span, fuse, (int)sh0);
  else
    hipLaunchKernelGGL(k_stage<2>, sgrid, dim3(kST), 0, st, h, tile_e, tile_slot, ulist, ucount, kbg,
                       krow, hc, hcor, dump, (int)D, (int)F, (int)FS, (int)topk, (int)E, (int)umax,
                       GMX, blk, (int)NT, nblk, span, fuse, (int)sh0);
  {
    const int rc = check_launch(fn);
    if (rc) return rc;
  }
  if (MS == 1)
    hipLaunchKernelGGL(k_gemm<1>, dim3((unsigned)(NT * nblk)), dim3(64), 0, st, tile_slot, gains,
                       kbg, krow, hc, hcor, pw, ps, pb, spw, sps, spb, part, blk, (int)D, (int)F,
                       (int)FS, (int)topk, (int)E, (int)NT, GMX);
  else
    hipLaunchKernelGGL(k_gemm<2>, dim3((unsigned)(NT * nblk)), dim3(64), 0, st, tile_slot, gains,
                       kbg, krow, hc, hcor, pw, ps, pb, spw, sps, spb, part, blk, (int)D, (int)F,
                       (int)FS, (int)topk, (int)E, (int)NT, GMX);
  int rc = check_launch(fn);
  if (rc) return rc;
  const unsigned sg = (unsigned)((T * (D / 4) + 255) / 256);
  switch (y_dtype) {
#define HSD_SUMS(DT)                                                                          \
  case DT:                                                                                    \
    if (topk == 6)                                                                            \
      hipLaunchKernelGGL((k_sum_slots<DT, 6>), dim3(sg), dim3(256), 0, st, part, sel,        \
                         reinterpret_cast<typename Elem<DT>::T*>(y), (int)T, (int)D,         \
                         (int)topk, (int)E);                                                  \
    else                                                                                      \
      hipLaunchKernelGGL((k_sum_slots<DT, 0>), dim3(sg), dim3(256), 0, st, part, sel,        \
                         reinterpret_cast<typename Elem<DT>::T*>(y), (int)T, (int)D,         \
                         (int)topk, (int)E);                                                  \
    break;
    HSD_SUMS(HSD_DT_BF16)
    HSD_SUMS(HSD_DT_F16)
    HSD_SUMS(HSD_DT_F32)
#undef HSD_SUMS
    default: return set_error(HSD_ERR_DTYPE, "%s: y_dtype %d", fn, y_dtype);
  }
  return check_launch(fn);
}
