// The MoE down projection at decode: sparse over the live ReLU^2 neurons on the
// neuron-major layout (hsd/decode.py), plus the dense 4-bit comparator on the stock
// layout.
//
// Work split of the sparse kernel (one token row b, BASELINE shape D=2688, F=1856,
// FS=3712, top-6 + shared):
//   * D is cut into chunks of 128 outputs = 16 weight words = 64 bytes of every row.
//   * A slot's 64-neuron groups are cut into "parts" of up to 16 groups (routed: 16+13,
//     shared: 16+16+16+10), 16 parts per token.
//   * One workgroup = (part, D chunk): 256 threads = 16 lane-groups of 16 lanes; lane-
//     group j owns group g0+j, lane l owns weight word 16c+l (8 outputs). 336
//     workgroups per token row.
// Compaction: each lane loads 4 of its group's 64 activations; 4 wave ballots give every
// lane-group the 64-bit live mask of its group (bit n = neuron 64g+n live). A lane then
// walks the set bits in ascending order, 8 rows in flight, loading only the live rows'
// 4-byte words and, if the group has a live row, the group's 16-byte scale and bias
// vectors. Per group: acc[t] = sum h_i q_{i,t}, hsum = sum h_i (fp32), and
// term = s*acc + b*hsum (the factorisation of decode.py:125-128). The 16 group terms
// are summed in ascending group order through LDS, times the slot's gain, into one fp32
// partial per (part, chunk); a second kernel sums the 16 parts in part order.
// Every row of a batch is computed by the same code independently of B.
#include "hsd_common.h"

namespace hsd {
namespace {

constexpr int kThreads = 256;
constexpr int kDC = 128;                 // outputs per D chunk
constexpr int kWPC = kDC / 8;            // weight words per chunk (one lane each)
constexpr int kGPW = kThreads / kWPC;    // groups per workgroup (one per lane-group)
constexpr int kRB = 8;                   // live rows in flight per lane

struct Geom {
  int D, F, FS, topk, E, NR, NW;
  int nchunk;  // D / 128
  int gpr;     // groups per routed expert (F/64)
  int gsh;     // groups of the shared expert (FS/64)
  int ppr;     // parts per routed slot
  int psh;     // parts of the shared slot
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
  g.psh = (g.gsh + kGPW - 1) / kGPW;
  g.nparts = g.topk * g.ppr + g.psh;
  g.nwg = g.nparts * g.nchunk;
  g.ngt = g.topk * g.gpr + g.gsh;
  return g;
}

__device__ __forceinline__ float lo_bf16(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

template <int HDT>
__global__ __launch_bounds__(kThreads) void k_sparse_down_part(
    const typename Elem<HDT>::T* __restrict__ h, const int32_t* __restrict__ sel,
    const float* __restrict__ gains, const uint32_t* __restrict__ pw,
    const uint16_t* __restrict__ ps, const uint16_t* __restrict__ pb,
    const uint32_t* __restrict__ spw, const uint16_t* __restrict__ sps,
    const uint16_t* __restrict__ spb, float* __restrict__ part, uint64_t* __restrict__ live_out,
    int32_t* __restrict__ status, Geom g, int B, int dense) {
  __shared__ float hsh[kGPW][64];
  __shared__ float red[kGPW * 8 * kWPC];  // [j][t][l]

  const int logical = xcd_remap((int)blockIdx.x, B * g.nwg);
  const int b = logical / g.nwg;
  const int rem = logical - b * g.nwg;
  const int p = rem / g.nchunk, c = rem - p * g.nchunk;
  const int tid = threadIdx.x, j = tid >> 4, l = tid & 15;

  int k, g0, ng, gbase;
  if (p < g.topk * g.ppr) {
    k = p / g.ppr;
    g0 = (p - k * g.ppr) * kGPW;
    ng = min(kGPW, g.gpr - g0);
    gbase = k * g.gpr;
  } else {
    k = g.topk;
    g0 = (p - g.topk * g.ppr) * kGPW;
    ng = min(kGPW, g.gsh - g0);
    gbase = g.topk * g.gpr;
  }

  const uint32_t* wb;
  const uint16_t* sb;
  const uint16_t* bb;
  int hoff;
  bool ok = true;
  if (k < g.topk) {
    const int e = sel[b * g.topk + k];
    ok = (unsigned)e < (unsigned)g.E;
    const size_t es = ok ? (size_t)e : 0;
    wb = pw + es * (size_t)g.F * g.NW;
    sb = ps + es * (size_t)g.gpr * g.D;
    bb = pb + es * (size_t)g.gpr * g.D;
    hoff = k * g.F;
  } else {
    wb = spw;
    sb = sps;
    bb = spb;
    hoff = g.topk * g.F;
  }
  if (!ok && tid == 0 && status) atomicOr(status, (int32_t)HSD_STATUS_BAD_EXPERT);
  const float gain = gains[b * (g.topk + 1) + k];

  // ---- compaction: the group's 64-bit live mask from four wave ballots
  const int grp = g0 + j;
  const bool gvalid = ok && j < ng;
  const typename Elem<HDT>::T* hrow = h + (size_t)b * g.NR + hoff + (size_t)grp * 64;
  uint64_t live = 0;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float x = gvalid ? Elem<HDT>::load(hrow, 16 * v + l) : 0.0f;
    const uint64_t bal = __ballot(gvalid && !(x == 0.0f));  // +-0 dead, NaN live
    live |= ((bal >> (16 * (j & 3))) & 0xFFFFull) << (16 * v);
    hsh[j][16 * v + l] = x;
  }
  const uint64_t rows = dense ? (gvalid ? ~0ull : 0ull) : live;
  if (live_out && c == 0 && l == 0 && j < ng) live_out[(size_t)b * g.ngt + gbase + grp] = live;

  // ---- the group's scales and biases, only if it has a row to read
  const int w = c * kWPC + l;
  uint4 sv = make_uint4(0, 0, 0, 0), bv = make_uint4(0, 0, 0, 0);
  if (rows) {
    sv = *reinterpret_cast<const uint4*>(sb + (size_t)grp * g.D + 8 * w);
    bv = *reinterpret_cast<const uint4*>(bb + (size_t)grp * g.D + 8 * w);
  }
  __syncthreads();

  // ---- live rows, ascending, kRB in flight
  const uint32_t* wrow = wb + (size_t)grp * 64 * g.NW + w;
  float acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = 0.0f;
  float hsum = 0.0f;
  uint64_t m = rows;
  while (m) {
    uint32_t q[kRB];
    float hv[kRB];
#pragma unroll
    for (int r = 0; r < kRB; ++r) {
      if (m) {
        const int n = __builtin_ctzll(m);
        m &= m - 1;
        q[r] = wrow[(size_t)n * g.NW];
        hv[r] = hsh[j][n];
      } else {
        q[r] = 0u;
        hv[r] = 0.0f;
      }
    }
#pragma unroll
    for (int r = 0; r < kRB; ++r) {
      hsum += hv[r];
      const uint32_t lo = q[r] & 0x0F0F0F0Fu, hi = (q[r] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = fmaf(hv[r], (float)((lo >> (8 * i)) & 0xFFu), acc[2 * i]);
        acc[2 * i + 1] = fmaf(hv[r], (float)((hi >> (8 * i)) & 0xFFu), acc[2 * i + 1]);
      }
    }
  }

  // ---- group term s*acc + b*hsum, then the ordered sum over the workgroup's groups
  const uint32_t s32[4] = {sv.x, sv.y, sv.z, sv.w};
  const uint32_t b32[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    red[(j * 8 + 2 * i) * kWPC + l] = fmaf(lo_bf16(s32[i]), acc[2 * i], lo_bf16(b32[i]) * hsum);
    red[(j * 8 + 2 * i + 1) * kWPC + l] =
        fmaf(hi_bf16(s32[i]), acc[2 * i + 1], hi_bf16(b32[i]) * hsum);
  }
  __syncthreads();
  if (tid < kDC) {
    const int lw = tid >> 3, t = tid & 7;  // output 8*lw + t of the chunk
    float s = red[t * kWPC + lw];
    for (int jj = 1; jj < ng; ++jj) s += red[(jj * 8 + t) * kWPC + lw];
    part[((size_t)b * g.nparts + p) * g.D + (size_t)c * kDC + tid] = gain * s;
  }
}

template <int YDT>
__global__ __launch_bounds__(256) void k_sum_parts(const float* __restrict__ part,
                                                   typename Elem<YDT>::T* __restrict__ y, int D,
                                                   int nparts) {
  const int o = blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (o >= D) return;
  const float* pp = part + (size_t)b * nparts * D + o;
  float s = pp[0];
  for (int q = 1; q < nparts; ++q) s += pp[(size_t)q * D];
  Elem<YDT>::store(y, (size_t)b * D + o, s);
}

// ----------------------------------------------------------------- dense comparator
// One wavefront per kOPW outputs, all topk+1 slots: lane u reads the 16-byte word
// group (32 neurons) u of each output row, with that half-group's scale and bias; the
// token's h is staged once per workgroup in LDS (fp32). Per lane and slot:
// gain * (s*acc + b*hsum) over its 32 neurons; a butterfly sum over the wave gives y.
constexpr int kOPW = 2;
constexpr int kDenseWaves = 4;

template <int HDT, int YDT>
__global__ __launch_bounds__(64 * kDenseWaves) void k_dense_down(
    const typename Elem<HDT>::T* __restrict__ h, const int32_t* __restrict__ sel,
    const float* __restrict__ gains, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ s, const uint16_t* __restrict__ bias,
    const uint32_t* __restrict__ sw, const uint16_t* __restrict__ ss,
    const uint16_t* __restrict__ sbias, typename Elem<YDT>::T* __restrict__ y,
    int32_t* __restrict__ status, int D, int F, int FS, int topk, int E) {
  extern __shared__ float hsh[];
  const int NR = topk * F + FS;
  const int b = blockIdx.y;
  for (int i = threadIdx.x; i < NR; i += blockDim.x) hsh[i] = Elem<HDT>::load(h, (size_t)b * NR + i);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int o0 = (blockIdx.x * kDenseWaves + wave) * kOPW;
  float tot[kOPW];
#pragma unroll
  for (int i = 0; i < kOPW; ++i) tot[i] = 0.0f;
  for (int k = 0; k <= topk; ++k) {
    const uint32_t* wk;
    const uint16_t *sk, *bk;
    int width, hoff;
    if (k < topk) {
      int e = sel[b * topk + k];
      if ((unsigned)e >= (unsigned)E) {
        if (lane == 0 && status) atomicOr(status, (int32_t)HSD_STATUS_BAD_EXPERT);
        continue;
      }
      width = F;
      hoff = k * F;
      wk = w + (size_t)e * D * (F / 8);
      sk = s + (size_t)e * D * (F / 64);
      bk = bias + (size_t)e * D * (F / 64);
    } else {
      width = FS;
      hoff = topk * F;
      wk = sw;
      sk = ss;
      bk = sbias;
    }
    const float gain = gains[b * (topk + 1) + k];
    const int nu = width / 32, ngr = width / 64, nwd = width / 8;
    for (int u = lane; u < nu; u += 64) {
      const float* hv = hsh + hoff + 32 * u;
      float hs = 0.0f;
#pragma unroll
      for (int i = 0; i < 32; ++i) hs += hv[i];
#pragma unroll
      for (int oi = 0; oi < kOPW; ++oi) {
        const int o = o0 + oi;
        if (o >= D) break;
        const uint4 q4 = *reinterpret_cast<const uint4*>(wk + (size_t)o * nwd + 4 * u);
        const float sc = bf16_bits_to_f32(sk[(size_t)o * ngr + u / 2]);
        const float bi = bf16_bits_to_f32(bk[(size_t)o * ngr + u / 2]);
        const uint32_t qw[4] = {q4.x, q4.y, q4.z, q4.w};
        float acc = 0.0f;
#pragma unroll
        for (int wi = 0; wi < 4; ++wi)
#pragma unroll
          for (int n = 0; n < 8; ++n)
            acc = fmaf(hv[8 * wi + n], (float)((qw[wi] >> (4 * n)) & 0xFu), acc);
        tot[oi] = fmaf(gain, fmaf(sc, acc, bi * hs), tot[oi]);
      }
    }
  }
#pragma unroll
  for (int oi = 0; oi < kOPW; ++oi) {
    const float v = wave_sum(tot[oi]);
    const int o = o0 + oi;
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

extern "C" int hsd_sparse_down_decode(const void* h, int h_dtype, const int32_t* sel,
                                      const float* gains, const uint32_t* pw, const uint16_t* ps,
                                      const uint16_t* pb, const uint32_t* spw, const uint16_t* sps,
                                      const uint16_t* spb, void* y, int y_dtype, int64_t B,
                                      int64_t D, int64_t F, int64_t FS, int64_t topk, int64_t E,
                                      int dense, uint64_t* live_masks, int32_t* dev_status,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "hsd_sparse_down_decode";
  if (!h || !sel || !gains || !pw || !ps || !pb || !spw || !sps || !spb || !y)
    return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (B < 0 || topk <= 0 || E <= 0) return set_error(HSD_ERR_SHAPE, "%s: bad B/topk/E", fn);
  if (D <= 0 || D % kDC || F <= 0 || F % 64 || FS <= 0 || FS % 64)
    return set_error(HSD_ERR_SHAPE, "%s: need D %% 128 == 0, F %% 64 == 0, FS %% 64 == 0 (D=%lld F=%lld FS=%lld)",
                     fn, (long long)D, (long long)F, (long long)FS);
  if (topk * F + FS > (int64_t)1 << 30 || D > 65536 || B > 65535)
    return set_error(HSD_ERR_SHAPE, "%s: sizes too large", fn);
  if (!aligned16(ps) || !aligned16(pb) || !aligned16(sps) || !aligned16(spb))
    return set_error(HSD_ERR_ALIGN, "%s: scales/biases must be 16-byte aligned", fn);
  if (B == 0) return HSD_OK;
  const Geom g = make_geom(D, F, FS, topk, E);
  const size_t need = hsd_sparse_down_workspace_bytes(B, D, F, FS, topk);
  if (!workspace || workspace_bytes < need)
    return set_error(HSD_ERR_WORKSPACE, "%s: workspace needs %zu bytes", fn, need);
  float* part = reinterpret_cast<float*>(workspace);
  hipStream_t st = as_stream(stream);
  const int64_t nblk = B * (int64_t)g.nwg;
  if (nblk > 0x7FFFFFFF) return set_error(HSD_ERR_SHAPE, "%s: too many workgroups", fn);
#define HSD_PART(DT)                                                                        \
  hipLaunchKernelGGL(k_sparse_down_part<DT>, dim3((unsigned)nblk), dim3(kThreads), 0, st,  \
                     reinterpret_cast<const typename Elem<DT>::T*>(h), sel, gains, pw, ps, pb, \
                     spw, sps, spb, part, live_masks, dev_status, g, (int)B, dense)
  switch (h_dtype) {
    case HSD_DT_BF16: HSD_PART(HSD_DT_BF16); break;
    case HSD_DT_F16: HSD_PART(HSD_DT_F16); break;
    case HSD_DT_F32: HSD_PART(HSD_DT_F32); break;
    default: return set_error(HSD_ERR_DTYPE, "%s: h_dtype %d", fn, h_dtype);
  }
#undef HSD_PART
  int rc = check_launch(fn);
  if (rc) return rc;
  dim3 rgrid((unsigned)((D + 255) / 256), (unsigned)B);
#define HSD_SUM(DT)                                                                   \
  hipLaunchKernelGGL(k_sum_parts<DT>, rgrid, dim3(256), 0, st, part,                 \
                     reinterpret_cast<typename Elem<DT>::T*>(y), (int)D, g.nparts)
  switch (y_dtype) {
    case HSD_DT_BF16: HSD_SUM(HSD_DT_BF16); break;
    case HSD_DT_F16: HSD_SUM(HSD_DT_F16); break;
    case HSD_DT_F32: HSD_SUM(HSD_DT_F32); break;
    default: return set_error(HSD_ERR_DTYPE, "%s: y_dtype %d", fn, y_dtype);
  }
#undef HSD_SUM
  return check_launch(fn);
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
  if (NR * 4 > 65536) return set_error(HSD_ERR_SHAPE, "%s: h row of %lld floats exceeds LDS", fn, (long long)NR);
  if (B == 0) return HSD_OK;
  if (B > 65535 || D > (1 << 24)) return set_error(HSD_ERR_SHAPE, "%s: sizes too large", fn);
  const int per_wg = kOPW * kDenseWaves;
  dim3 grid((unsigned)((D + per_wg - 1) / per_wg), (unsigned)B);
  hipStream_t st = as_stream(stream);
  const size_t lds = (size_t)NR * sizeof(float);
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
