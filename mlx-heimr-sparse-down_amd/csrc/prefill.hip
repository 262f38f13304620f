// The MoE down projection over a prompt chunk: tile order, per-tile union of live
// neurons, and a bf16 MFMA grouped GEMM on the neuron-major layout (hsd/prefill.py).
//
//   k_tiles      one workgroup: stable expert sort of the T*topk slots (wave ballots
//                give each slot its rank among equal experts), tile bases by a scan,
//                fixed NT = T*topk/tt + E + ceil(T/tt) with -1 padding, no host readback.
//   k_union      one workgroup per tile: OR of h != 0 over the tile's slots, ballot +
//                prefix compaction into an ascending union list (ulist, ucount).
//   k_gemm       one workgroup per (tile, 128-column block of D): K = the tile's union
//                rows in chunks of 64. Per chunk the B tile (64 rows x 128 columns) is
//                dequantised from the 4-bit rows and their groups' bf16 scale/bias as
//                bf16(s*q + b) into LDS (n-major), the A tile (tt slots x 64 union
//                columns of h, bf16) is gathered into LDS, and 4 waves run
//                v_mfma_f32_32x32x16_bf16 with fp32 accumulators (wave w: columns
//                32w..32w+31, all tt rows). Epilogue: gain * acc into part[token*(topk+1)+k].
//   k_sum_slots  y[t] = sum over the topk+1 partials in slot order.
#include "hsd_common.h"

namespace hsd {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------------ tiles
constexpr int kTT = 1024;  // threads of the tile-order kernel

__global__ __launch_bounds__(kTT) void k_tiles(const int32_t* __restrict__ sel, int T, int topk,
                                               int E, int tt, int32_t* __restrict__ tile_e,
                                               int32_t* __restrict__ tile_slot,
                                               int32_t* __restrict__ status,
                                               int32_t* __restrict__ rank_ws) {
  extern __shared__ int sh[];
  int* cnt = sh;                    // [E] running count per expert, then counts
  int* tbase = sh + E;              // [E + 1] tile base per expert (exclusive scan)
  int* wcnt = sh + 2 * E + 1;       // [16][E] per-wave counts of the current chunk
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = T * topk;
  for (int e = tid; e < E; e += kTT) cnt[e] = 0;
  __syncthreads();
  for (int base = 0; base < n; base += kTT) {
    for (int i = tid; i < 16 * E; i += kTT) wcnt[i] = 0;
    __syncthreads();
    const int s = base + tid;
    int e = s < n ? sel[s] : -1;
    if (s < n && (unsigned)e >= (unsigned)E) {
      if (status) atomicOr(status, (int32_t)HSD_STATUS_BAD_EXPERT);
      e = -1;
    }
    // rank among the lanes of this wave with the same expert, lowest lane first
    uint64_t todo = __ballot(e >= 0);
    int rank_w = 0;
    while (todo) {
      const int leader = __builtin_ctzll(todo);
      const int le = __shfl(e, leader, 64);
      const uint64_t mk = __ballot(e == le);
      if (e == le) rank_w = __popcll(mk & ((1ull << lane) - 1ull));
      if (lane == leader) wcnt[wave * E + le] = __popcll(mk);
      todo &= ~mk;
    }
    __syncthreads();
    for (int ee = tid; ee < E; ee += kTT) {  // exclusive scan over the waves, per expert
      int run = cnt[ee];
      for (int w = 0; w < 16; ++w) {
        const int c = wcnt[w * E + ee];
        wcnt[w * E + ee] = run;
        run += c;
      }
      cnt[ee] = run;
    }
    __syncthreads();
    if (s < n) rank_ws[s] = e >= 0 ? wcnt[wave * E + e] + rank_w : -1;
    __syncthreads();
  }
  if (tid == 0) {
    int run = 0;
    for (int ee = 0; ee < E; ++ee) {
      tbase[ee] = run;
      run += (cnt[ee] + tt - 1) / tt;
    }
    tbase[E] = run;
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
  for (int s = tid; s < n; s += kTT) {
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
constexpr int kUT = 256;

template <int HDT>
__global__ __launch_bounds__(kUT) void k_union(const typename Elem<HDT>::T* __restrict__ h,
                                               const int32_t* __restrict__ tile_e,
                                               const int32_t* __restrict__ tile_slot,
                                               int32_t* __restrict__ ulist,
                                               int32_t* __restrict__ ucount, int F, int FS,
                                               int topk, int E, int tt, int umax) {
  __shared__ int hoff[64];
  __shared__ int wtot[kUT / 64];
  const int tile = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int NR = topk * F + FS;
  int32_t* out = ulist + (size_t)tile * umax;
  const int e = tile_e[tile];
  if (e < 0) {
    for (int i = tid; i < umax; i += kUT) out[i] = -1;
    if (tid == 0) ucount[tile] = 0;
    return;
  }
  const bool shared = e >= E;
  const int FF = shared ? FS : F;
  if (tid < tt) {
    const int s = tile_slot[tile * tt + tid];
    hoff[tid] = s < 0 ? -1 : (shared ? s * NR + topk * F : (s / topk) * NR + (s % topk) * F);
  }
  __syncthreads();
  int base = 0;
  for (int c0 = 0; c0 < FF; c0 += kUT) {
    const int c = c0 + tid;
    bool live = false;
    if (c < FF)
      for (int m = 0; m < tt; ++m) {
        const int o = hoff[m];
        if (o >= 0) {
          const float v = Elem<HDT>::load(h, (size_t)o + c);
          live = live || !(v == 0.0f);
        }
      }
    const uint64_t bal = __ballot(live);
    if (lane == 0) wtot[wave] = __popcll(bal);
    __syncthreads();
    int before = base;
    for (int w = 0; w < wave; ++w) before += wtot[w];
    if (live) out[before + __popcll(bal & ((1ull << lane) - 1ull))] = c;
    for (int w = 0; w < kUT / 64; ++w) base += wtot[w];
    __syncthreads();
  }
  for (int i = base + tid; i < umax; i += kUT) out[i] = -1;
  if (tid == 0) ucount[tile] = base;
}

// ------------------------------------------------------------------ GEMM
constexpr int kGT = 256;  // 4 waves
constexpr int kNB = 128;  // output columns per workgroup
constexpr int kKC = 64;   // union rows per chunk
constexpr int kKP = kKC + 8;  // LDS row pitch (bf16) of the A and B tiles

template <int MS>  // MS = tt / 32 row blocks
__global__ __launch_bounds__(kGT) void k_gemm(
    const uint16_t* __restrict__ h, const float* __restrict__ gains,
    const int32_t* __restrict__ tile_e, const int32_t* __restrict__ tile_slot,
    const int32_t* __restrict__ ulist, const int32_t* __restrict__ ucount,
    const uint32_t* __restrict__ pw, const uint16_t* __restrict__ ps,
    const uint16_t* __restrict__ pb, const uint32_t* __restrict__ spw,
    const uint16_t* __restrict__ sps, const uint16_t* __restrict__ spb, float* __restrict__ part,
    int D, int F, int FS, int topk, int E, int NT, int umax) {
  constexpr int TT = 32 * MS;
  __shared__ __attribute__((aligned(16))) uint16_t As[TT * kKP];    // [m][k]
  __shared__ __attribute__((aligned(16))) uint16_t Bs[kNB * kKP];   // [n][k]
  __shared__ int hoff[TT];
  __shared__ int rows[kKC];
  const int nblk = D / kNB;
  const int logical = xcd_remap((int)blockIdx.x, NT * nblk);
  const int tile = logical / nblk, nb = logical - (logical / nblk) * nblk;
  const int e = tile_e[tile];
  if (e < 0) return;
  const int U = ucount[tile];
  if (U == 0) return;  // all-dead tile: its slots' partials were zeroed by the caller
  const bool shared = e >= E;
  const int NR = topk * F + FS;
  const int NW = D / 8;
  const int n0 = nb * kNB;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t* wb = shared ? spw : pw + (size_t)e * F * NW;
  const uint16_t* sb = shared ? sps : ps + (size_t)e * (F / 64) * D;
  const uint16_t* bb = shared ? spb : pb + (size_t)e * (F / 64) * D;
  const int32_t* ul = ulist + (size_t)tile * umax;
  if (tid < TT) {
    const int s = tile_slot[tile * TT + tid];
    hoff[tid] = s < 0 ? -1 : (shared ? s * NR + topk * F : (s / topk) * NR + (s % topk) * F);
  }
  f32x16 acc[MS];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[ms][v] = 0.0f;

  // B staging task of this thread: rows 4*kq .. 4*kq+3 of the chunk, columns 8*wv .. +7
  const int kq = tid >> 4, wv = tid & 15;
  for (int u0 = 0; u0 < U; u0 += kKC) {
    if (tid < kKC) rows[tid] = (u0 + tid < U) ? ul[u0 + tid] : -1;
    __syncthreads();
    // ---- B: dequantise 4 rows x 8 columns -> Bs[n][k]
    {
      uint32_t q[4];
      uint4 s4[4], b4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = rows[4 * kq + i];
        q[i] = 0u;
        s4[i] = make_uint4(0, 0, 0, 0);
        b4[i] = make_uint4(0, 0, 0, 0);
        if (r >= 0) {
          q[i] = wb[(size_t)r * NW + (n0 >> 3) + wv];
          s4[i] = *reinterpret_cast<const uint4*>(sb + (size_t)(r >> 6) * D + n0 + 8 * wv);
          b4[i] = *reinterpret_cast<const uint4*>(bb + (size_t)(r >> 6) * D + n0 + 8 * wv);
        }
      }
#pragma unroll
      for (int c = 0; c < 8; ++c) {  // column n0 + 8*wv + c
        uint16_t v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t sw = (&s4[i].x)[c >> 1], bw = (&b4[i].x)[c >> 1];
          const float sc = (c & 1) ? __uint_as_float(sw & 0xFFFF0000u) : __uint_as_float(sw << 16);
          const float bi = (c & 1) ? __uint_as_float(bw & 0xFFFF0000u) : __uint_as_float(bw << 16);
          const float qv = (float)((q[i] >> (4 * c)) & 0xFu);
          v[i] = f32_to_bf16_bits(fmaf(sc, qv, bi));
        }
        uint2 pk;
        pk.x = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
        pk.y = (uint32_t)v[2] | ((uint32_t)v[3] << 16);
        *reinterpret_cast<uint2*>(&Bs[(8 * wv + c) * kKP + 4 * kq]) = pk;
      }
    }
    // ---- A: gather h[slot m, rows k] -> As[m][k]
#pragma unroll
    for (int it = 0; it < (TT * kKC / 8) / kGT; ++it) {
      const int task = tid + it * kGT;
      const int m = task >> 3, ko = (task & 7) * 8;
      const int o = hoff[m];
      uint32_t pk[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r0 = rows[ko + 2 * i], r1 = rows[ko + 2 * i + 1];
        const uint32_t v0 = (o >= 0 && r0 >= 0) ? h[(size_t)o + r0] : 0u;
        const uint32_t v1 = (o >= 0 && r1 >= 0) ? h[(size_t)o + r1] : 0u;
        pk[i] = v0 | (v1 << 16);
      }
      *reinterpret_cast<uint4*>(&As[m * kKP + ko]) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
    __syncthreads();
    // ---- MFMA: wave owns columns 32*wave .. +31
#pragma unroll
    for (int ks = 0; ks < kKC / 16; ++ks) {
      const int kk = ks * 16 + 8 * (lane >> 5);
      const bf16x8 bfrag =
          *reinterpret_cast<const bf16x8*>(&Bs[(32 * wave + (lane & 31)) * kKP + kk]);
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
        const bf16x8 afrag = *reinterpret_cast<const bf16x8*>(&As[(32 * ms + (lane & 31)) * kKP + kk]);
        acc[ms] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afrag, bfrag, acc[ms], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  // ---- epilogue: C[i][j], j = lane%32, i = 8*(v/4) + 4*(lane/32) + v%4
  const int j = n0 + 32 * wave + (lane & 31);
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int i = 32 * ms + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
      const int s = tile_slot[tile * TT + i];
      if (s >= 0) {
        const int gi = shared ? s * (topk + 1) + topk : (s / topk) * (topk + 1) + (s % topk);
        part[(size_t)gi * D + j] = gains[gi] * acc[ms][v];
      }
    }
}

// Partials of slots that no GEMM workgroup writes (an empty union, a bad expert id)
// must read as 0: cleared by a fill kernel (graph-capture safe, no memset node).
__global__ void k_zero_f32(float* __restrict__ p, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = 0.0f;
}

template <int YDT>
__global__ __launch_bounds__(256) void k_sum_slots(const float* __restrict__ part,
                                                   typename Elem<YDT>::T* __restrict__ y, int T,
                                                   int D, int nk) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)T * D) return;
  const size_t t = idx / D, o = idx - t * D;
  const float* p = part + t * nk * D + o;
  float s = p[0];
  for (int k = 1; k < nk; ++k) s += p[(size_t)k * D];
  Elem<YDT>::store(y, idx, s);
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
  const size_t lds = (size_t)(2 * E + 1 + 16 * E) * sizeof(int);
  if (lds > 65536) return set_error(HSD_ERR_SHAPE, "%s: E too large for LDS", fn);
  hipLaunchKernelGGL(k_tiles, dim3(1), dim3(kTT), lds, as_stream(stream), sel, (int)T, (int)topk,
                     (int)E, (int)tt, tile_e, tile_slot, dev_status,
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
  if (umax < FS || umax < F) return set_error(HSD_ERR_SHAPE, "%s: umax must be >= FS and F", fn);
  if (NT != hsd_prefill_num_tiles(T, topk, E, tt)) return set_error(HSD_ERR_SHAPE, "%s: NT mismatch", fn);
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

extern "C" size_t hsd_prefill_gemm_workspace_bytes(int64_t T, int64_t D, int64_t topk) {
  if (T <= 0 || D <= 0 || topk <= 0) return 0;
  return ((size_t)T * (topk + 1) * D * sizeof(float) + 255) & ~(size_t)255;
}

extern "C" int hsd_prefill_gemm(const uint16_t* h, const float* gains, const int32_t* tile_e,
                                const int32_t* tile_slot, const int32_t* ulist,
                                const int32_t* ucount, const uint32_t* pw, const uint16_t* ps,
                                const uint16_t* pb, const uint32_t* spw, const uint16_t* sps,
                                const uint16_t* spb, void* y, int y_dtype, int64_t T, int64_t D,
                                int64_t F, int64_t FS, int64_t topk, int64_t E, int64_t tt,
                                int64_t NT, int64_t umax, void* workspace,
                                size_t workspace_bytes, void* stream) {
  const char* fn = "hsd_prefill_gemm";
  if (!h || !gains || !tile_e || !tile_slot || !ulist || !ucount || !pw || !ps || !pb || !spw ||
      !sps || !spb || !y)
    return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (tt != 32 && tt != 64) return set_error(HSD_ERR_SHAPE, "%s: tt must be 32 or 64", fn);
  if (T <= 0 || D <= 0 || D % kNB || F <= 0 || F % 64 || FS <= 0 || FS % 64 || topk <= 0 || E <= 0)
    return set_error(HSD_ERR_SHAPE, "%s: need D %% 128 == 0, F %% 64 == 0, FS %% 64 == 0", fn);
  if (NT != hsd_prefill_num_tiles(T, topk, E, tt)) return set_error(HSD_ERR_SHAPE, "%s: NT mismatch", fn);
  if (umax < FS || umax < F) return set_error(HSD_ERR_SHAPE, "%s: umax must be >= FS", fn);
  if (NT * (D / kNB) > 0x7FFFFFFF || (topk * F + FS) * T > ((int64_t)1 << 31))
    return set_error(HSD_ERR_SHAPE, "%s: sizes too large", fn);
  const uintptr_t al = (uintptr_t)ps | (uintptr_t)pb | (uintptr_t)sps | (uintptr_t)spb;
  if (al & 15u) return set_error(HSD_ERR_ALIGN, "%s: scales/biases must be 16-byte aligned", fn);
  const size_t need = hsd_prefill_gemm_workspace_bytes(T, D, topk);
  if (!workspace || workspace_bytes < need)
    return set_error(HSD_ERR_WORKSPACE, "%s: workspace needs %zu bytes", fn, need);
  hipStream_t st = as_stream(stream);
  float* part = reinterpret_cast<float*>(workspace);
  const size_t npart = (size_t)T * (topk + 1) * D;
  hipLaunchKernelGGL(k_zero_f32, dim3(1024), dim3(256), 0, st, part, npart);
  int rc = check_launch(fn);
  if (rc) return rc;
  const unsigned grid = (unsigned)(NT * (D / kNB));
  if (tt == 32)
    hipLaunchKernelGGL(k_gemm<1>, dim3(grid), dim3(kGT), 0, st, h, gains, tile_e, tile_slot,
                       ulist, ucount, pw, ps, pb, spw, sps, spb, part, (int)D, (int)F, (int)FS,
                       (int)topk, (int)E, (int)NT, (int)umax);
  else
    hipLaunchKernelGGL(k_gemm<2>, dim3(grid), dim3(kGT), 0, st, h, gains, tile_e, tile_slot,
                       ulist, ucount, pw, ps, pb, spw, sps, spb, part, (int)D, (int)F, (int)FS,
                       (int)topk, (int)E, (int)NT, (int)umax);
  rc = check_launch(fn);
  if (rc) return rc;
  const unsigned sg = (unsigned)((T * D + 255) / 256);
  switch (y_dtype) {
#define HSD_SUMS(DT)                                                                        \
  case DT:                                                                                  \
    hipLaunchKernelGGL(k_sum_slots<DT>, dim3(sg), dim3(256), 0, st, part,                  \
                       reinterpret_cast<typename Elem<DT>::T*>(y), (int)T, (int)D, (int)(topk + 1)); \
    break;
    HSD_SUMS(HSD_DT_BF16)
    HSD_SUMS(HSD_DT_F16)
    HSD_SUMS(HSD_DT_F32)
#undef HSD_SUMS
    default: return set_error(HSD_ERR_DTYPE, "%s: y_dtype %d", fn, y_dtype);
  }
  return check_launch(fn);
}
