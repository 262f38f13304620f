// Mamba-2 multi-row verify with per-row state checkpoints, the rollback by slab
// selection, and greedy acceptance -- all on the device.
//
// hsd/mamba.py keeps the verify's inputs and RECOMPUTES the SSM over the accepted
// prefix on rollback (and mlx-lm's L>1 path is not bit-identical to single steps).
// Here the state lives in a ring of slabs; row r of a verify writes the (ssm, conv)
// state after row r into slab (cur+1+r) % nslab, so a rollback to n_keep rows is
// cur += n_keep -- no recompute, no copy, no host round trip. A row is computed by the
// same instruction sequence whatever L is, so L rows equal L single-row calls bit for
// bit.
//
// Work split of the state update (BASELINE: H=64 heads x P=64 head_dim x N=128 state,
// G=8 groups, conv K=4, CD = 4096 + 2*8*128 = 6144 channels):
//   one workgroup = (head h, block of 16 head_dim rows p): 256 WGs. It computes the conv
//   + silu of its 16 x channels and of its group's 128 B and 128 C channels for all L
//   rows (LDS), then each wave streams 4 state rows S[h, p, :] (128 fp32 = 2 per lane)
//   through the L rows: S = dA*S + (x*dt)*B, y = sum_n S*C + D*x (butterfly sum), and
//   writes each row's S to its checkpoint slab. HBM: read S once, write L checkpoints.
// The gated RMSNorm (groups of 512 = 8 heads) runs as a second small kernel.
#include "hsd_common.h"

namespace hsd {
namespace {

constexpr int kMT = 256;
constexpr int kPB = 16;      // head_dim rows per workgroup
constexpr int kN = 128;      // state size (2 per lane)
constexpr int kK = 4;        // conv kernel
constexpr int kLMax = 7;     // rows per verify (nslab <= 8)

__global__ __launch_bounds__(kMT) void k_mamba_ssm(
    const uint16_t* __restrict__ conv_in, int64_t cin_ld, const uint16_t* __restrict__ dt_raw,
    int64_t dt_ld, const uint16_t* __restrict__ conv_w, const uint16_t* __restrict__ conv_b,
    const float* __restrict__ A_log, const float* __restrict__ dt_bias,
    const float* __restrict__ Dp, float* __restrict__ ssm, uint16_t* __restrict__ convs,
    const int32_t* __restrict__ cur_ptr, int nslab, float* __restrict__ y_pre, int L, int H,
    int P, int G, float dt_lo, float dt_hi) {
  __shared__ float xs[kLMax][kPB];
  __shared__ float Bs[kLMax][kN];
  __shared__ float Cs[kLMax][kN];
  __shared__ float dtv[kLMax], dA[kLMax];
  const int npb = P / kPB;
  const int hh = blockIdx.x / npb, pblk = blockIdx.x - (blockIdx.x / npb) * npb;
  const int tid = threadIdx.x;
  const int cur = *cur_ptr;
  if ((unsigned)cur >= (unsigned)nslab) return;  // a corrupt ring index: touch nothing
  const int DI = H * P, GN = G * kN, CD = DI + 2 * GN;
  const int hpg = H / G;
  const int g = hh / hpg;
  const bool owner_bc = (hh % hpg == 0) && pblk == 0;  // writes the B/C conv checkpoints

  // ---- the state rows this workgroup streams: issued first, they do not depend on the
  // conv, so their latency overlaps it
  const int lane = tid & 63, wave = tid >> 6;
  constexpr int kRPW = kPB / (kMT / 64);
  float2 S[kRPW];
  const size_t slab_sz = (size_t)H * P * kN;
#pragma unroll
  for (int i = 0; i < kRPW; ++i) {
    const int p = pblk * kPB + wave * kRPW + i;
    S[i] = *reinterpret_cast<const float2*>(ssm + (size_t)cur * slab_sz +
                                            ((size_t)hh * P + p) * kN + 2 * lane);
  }

  // ---- depthwise causal conv + silu of the channels this workgroup needs
  const uint16_t* cs0 = convs + (size_t)cur * (kK - 1) * CD;
  for (int t = tid; t < kPB + 2 * kN; t += kMT) {
    int ch;
    if (t < kPB) ch = hh * P + pblk * kPB + t;
    else if (t < kPB + kN) ch = DI + g * kN + (t - kPB);
    else ch = DI + GN + g * kN + (t - kPB - kN);
    uint16_t win[kK - 1 + kLMax];
#pragma unroll
    for (int i = 0; i < kK - 1; ++i) win[i] = cs0[(size_t)i * CD + ch];
#pragma unroll
    for (int r = 0; r < kLMax; ++r)
      win[kK - 1 + r] = r < L ? conv_in[(size_t)r * cin_ld + ch] : (uint16_t)0;
    float wj[kK];
#pragma unroll
    for (int j = 0; j < kK; ++j) wj[j] = bf16_bits_to_f32(conv_w[(size_t)ch * kK + j]);
    const float bias = bf16_bits_to_f32(conv_b[ch]);
#pragma unroll
    for (int r = 0; r < kLMax; ++r) {
      if (r < L) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < kK; ++j) acc = fmaf(wj[j], bf16_bits_to_f32(win[r + j]), acc);
        const float co = silu_f32(acc + bias);
        if (t < kPB) xs[r][t] = co;
        else if (t < kPB + kN) Bs[r][t - kPB] = co;
        else Cs[r][t - kPB - kN] = co;
      }
    }
    if (t < kPB || owner_bc) {  // conv checkpoint after row r: window rows r+1 .. r+3
#pragma unroll
      for (int r = 0; r < kLMax; ++r) {
        if (r < L) {
          uint16_t* dst = convs + (size_t)((cur + 1 + r) % nslab) * (kK - 1) * CD + ch;
#pragma unroll
          for (int i = 0; i < kK - 1; ++i) dst[(size_t)i * CD] = win[r + 1 + i];
        }
      }
    }
  }
  if (tid < L) {
    const float A = -expf(A_log[hh]);
    const float v = softplus_f32(bf16_bits_to_f32(dt_raw[(size_t)tid * dt_ld + hh]) + dt_bias[hh]);
    const float d = fminf(fmaxf(v, dt_lo), dt_hi);
    dtv[tid] = d;
    dA[tid] = expf(A * d);
  }
  const float Dh = Dp[hh];
  __syncthreads();

  // ---- the state rows: 4 per wave, 2 state elements per lane
  for (int r = 0; r < L; ++r) {
    const float B0 = Bs[r][2 * lane], B1 = Bs[r][2 * lane + 1];
    const float C0 = Cs[r][2 * lane], C1 = Cs[r][2 * lane + 1];
    float* dst = ssm + (size_t)((cur + 1 + r) % nslab) * slab_sz;
#pragma unroll
    for (int i = 0; i < kRPW; ++i) {
      const int pl = wave * kRPW + i, p = pblk * kPB + pl;
      const float x = xs[r][pl];
      const float xdt = x * dtv[r];
      S[i].x = fmaf(dA[r], S[i].x, xdt * B0);
      S[i].y = fmaf(dA[r], S[i].y, xdt * B1);
      *reinterpret_cast<float2*>(dst + ((size_t)hh * P + p) * kN + 2 * lane) = S[i];
      const float y = wave_sum(fmaf(S[i].y, C1, S[i].x * C0));
      if (lane == 0) y_pre[(size_t)r * DI + (size_t)hh * P + p] = y + x * Dh;
    }
  }
}

// out[r, i] = norm_w[i] * z_i / sqrt(mean_group(z^2) + eps), z = y_pre * silu(gate);
// one workgroup per (row, norm group).
template <int YDT>
__global__ __launch_bounds__(kMT) void k_gated_norm(const float* __restrict__ y_pre,
                                                    const uint16_t* __restrict__ gate,
                                                    int64_t gate_ld,
                                                    const uint16_t* __restrict__ norm_w,
                                                    typename Elem<YDT>::T* __restrict__ y, int DI,
                                                    int NG, float eps) {
  __shared__ float wsum[kMT / 64];
  const int ngrp = DI / NG;
  const int r = blockIdx.x / ngrp, gi = blockIdx.x - (blockIdx.x / ngrp) * ngrp;
  const int per = NG / kMT;
  float z[8], nw[8];
  float ss = 0.0f;
  for (int i = 0; i < per; ++i) {  // every load (activations, gate, weight) before the reduction
    const int c = gi * NG + i * kMT + threadIdx.x;
    nw[i] = bf16_bits_to_f32(norm_w[c]);
    z[i] = y_pre[(size_t)r * DI + c] * silu_f32(bf16_bits_to_f32(gate[(size_t)r * gate_ld + c]));
    ss = fmaf(z[i], z[i], ss);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = wsum[0];
  for (int w = 1; w < kMT / 64; ++w) tot += wsum[w];
  const float inv = 1.0f / sqrtf(tot / (float)NG + eps);
  for (int i = 0; i < per; ++i) {
    const int c = gi * NG + i * kMT + threadIdx.x;
    Elem<YDT>::store(y, (size_t)r * DI + c, (z[i] * inv) * nw[i]);
  }
}

__global__ void k_select_row(int32_t* cur, const int32_t* n_keep_dev, int n_keep_host,
                             int nslab) {
  if (threadIdx.x == 0) {
    const int nk = n_keep_dev ? *n_keep_dev : n_keep_host;
    const int c = *cur;
    if (nk >= 0 && nk < nslab && c >= 0 && c < nslab) *cur = (c + nk) % nslab;
  }
}

// ---------------------------------------------------------------- acceptance
// a "better" b for argmax: NaN beats numbers (numpy/MLX return the first NaN), then
// the larger value, then the smaller index.
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  const bool na = va != va, nb = vb != vb;
  if (na != nb) return na;
  if (!na && va != vb) return va > vb;
  return ia < ib;
}

constexpr int kAT = 1024;
template <int DT>
__global__ __launch_bounds__(kAT) void k_argmax_rows(const typename Elem<DT>::T* __restrict__ x,
                                                     int64_t V, int32_t* __restrict__ out) {
  __shared__ float sv[kAT / 64];
  __shared__ int si[kAT / 64];
  const int r = blockIdx.x;
  float bv = 0.0f;
  int bi = 0x7FFFFFFF;
  for (int64_t i = threadIdx.x; i < V; i += kAT) {
    const float v = Elem<DT>::load(x, (size_t)r * V + i);
    if (bi == 0x7FFFFFFF || better(v, (int)i, bv, bi)) { bv = v; bi = (int)i; }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (oi != 0x7FFFFFFF && (bi == 0x7FFFFFFF || better(ov, oi, bv, bi))) { bv = ov; bi = oi; }
  }
  if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = sv[0];
    int i = si[0];
    for (int w = 1; w < kAT / 64; ++w)
      if (si[w] != 0x7FFFFFFF && (i == 0x7FFFFFFF || better(sv[w], si[w], v, i))) { v = sv[w]; i = si[w]; }
    out[r] = i;
  }
}

__global__ void k_accept(const int32_t* __restrict__ draft, const int32_t* __restrict__ tgt,
                         int k, int32_t* __restrict__ tokens, int32_t* __restrict__ n_accept,
                         int32_t* __restrict__ n_keep, int32_t* __restrict__ cur, int nslab) {
  if (threadIdx.x != 0) return;
  int a = k;
  for (int i = 0; i < k; ++i)
    if (draft[i] != tgt[i]) { a = i; break; }
  for (int i = 0; i <= k; ++i) tokens[i] = i < a ? draft[i] : (i == a ? tgt[a] : -1);
  if (n_accept) *n_accept = a;
  if (n_keep) *n_keep = a + 1;
  if (cur && *cur >= 0 && *cur < nslab) *cur = (*cur + a + 1) % nslab;
}

}  // namespace
}  // namespace hsd

using namespace hsd;

extern "C" size_t hsd_mamba_workspace_bytes(int64_t L, int64_t H, int64_t P) {
  if (L <= 0 || H <= 0 || P <= 0) return 0;
  return ((size_t)L * H * P * sizeof(float) + 255) & ~(size_t)255;
}

extern "C" int hsd_mamba_verify(const uint16_t* conv_in, int64_t conv_in_ld,
                                const uint16_t* dt_raw, int64_t dt_ld, const uint16_t* gate,
                                int64_t gate_ld, const uint16_t* conv_w, const uint16_t* conv_b,
                                const float* A_log, const float* dt_bias, const float* Dp,
                                const uint16_t* norm_w, float* ssm_slabs, uint16_t* conv_slabs,
                                const int32_t* cur, int64_t nslab, void* y, int y_dtype,
                                int64_t L, int64_t H, int64_t P, int64_t N, int64_t G,
                                int64_t norm_group, float eps, float dt_lo, float dt_hi,
                                void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "hsd_mamba_verify";
  if (!conv_in || !dt_raw || !gate || !conv_w || !conv_b || !A_log || !dt_bias || !Dp ||
      !norm_w || !ssm_slabs || !conv_slabs || !cur || !y)
    return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (N != kN) return set_error(HSD_ERR_SHAPE, "%s: state size N must be %d (got %lld)", fn, kN, (long long)N);
  if (L < 1 || L > kLMax || nslab < L + 1 || nslab > kLMax + 1)
    return set_error(HSD_ERR_SHAPE, "%s: need 1 <= L <= nslab-1 <= %d (L=%lld nslab=%lld)", fn, kLMax,
                     (long long)L, (long long)nslab);
  if (H <= 0 || P <= 0 || P % kPB || G <= 0 || H % G)
    return set_error(HSD_ERR_SHAPE, "%s: need P %% %d == 0 and H %% G == 0", fn, kPB);
  const int64_t DI = H * P, CD = DI + 2 * G * N;
  if (norm_group <= 0 || norm_group % kMT || DI % norm_group || norm_group / kMT > 8)
    return set_error(HSD_ERR_SHAPE, "%s: norm_group must be a multiple of 256, <= 2048, dividing H*P", fn);
  if (conv_in_ld < CD || dt_ld < H || gate_ld < DI)
    return set_error(HSD_ERR_SHAPE, "%s: row strides smaller than the rows", fn);
  if ((uintptr_t)ssm_slabs & 7u) return set_error(HSD_ERR_ALIGN, "%s: ssm_slabs must be 8-byte aligned", fn);
  if (H * (P / kPB) > 0x7FFFFFFF) return set_error(HSD_ERR_SHAPE, "%s: too large", fn);
  const size_t need = hsd_mamba_workspace_bytes(L, H, P);
  if (!workspace || workspace_bytes < need)
    return set_error(HSD_ERR_WORKSPACE, "%s: workspace needs %zu bytes", fn, need);
  hipStream_t st = as_stream(stream);
  float* y_pre = reinterpret_cast<float*>(workspace);
  hipLaunchKernelGGL(k_mamba_ssm, dim3((unsigned)(H * (P / kPB))), dim3(kMT), 0, st, conv_in,
                     conv_in_ld, dt_raw, dt_ld, conv_w, conv_b, A_log, dt_bias, Dp, ssm_slabs,
                     conv_slabs, cur, (int)nslab, y_pre, (int)L, (int)H, (int)P, (int)G, dt_lo,
                     dt_hi);
  int rc = check_launch(fn);
  if (rc) return rc;
  const unsigned ngrid = (unsigned)(L * (DI / norm_group));
#define HSD_NORM(DT)                                                                        \
  hipLaunchKernelGGL(k_gated_norm<DT>, dim3(ngrid), dim3(kMT), 0, st, y_pre, gate, gate_ld, \
                     norm_w, reinterpret_cast<typename Elem<DT>::T*>(y), (int)DI,           \
                     (int)norm_group, eps)
  switch (y_dtype) {
    case HSD_DT_BF16: HSD_NORM(HSD_DT_BF16); break;
    case HSD_DT_F16: HSD_NORM(HSD_DT_F16); break;
    case HSD_DT_F32: HSD_NORM(HSD_DT_F32); break;
    default: return set_error(HSD_ERR_DTYPE, "%s: y_dtype %d", fn, y_dtype);
  }
#undef HSD_NORM
  return check_launch(fn);
}

extern "C" int hsd_mamba_select_row(int32_t* cur, const int32_t* n_keep_dev, int64_t n_keep_host,
                                    int64_t nslab, void* stream) {
  if (!cur) return set_error(HSD_ERR_ARG, "hsd_mamba_select_row: null cur");
  if (nslab < 2 || nslab > kLMax + 1) return set_error(HSD_ERR_SHAPE, "hsd_mamba_select_row: bad nslab");
  if (!n_keep_dev && (n_keep_host < 0 || n_keep_host >= nslab))
    return set_error(HSD_ERR_ARG, "hsd_mamba_select_row: n_keep %lld outside [0, nslab)", (long long)n_keep_host);
  hipLaunchKernelGGL(k_select_row, dim3(1), dim3(64), 0, as_stream(stream), cur, n_keep_dev,
                     (int)n_keep_host, (int)nslab);
  return check_launch("hsd_mamba_select_row");
}

extern "C" int hsd_greedy_accept(const void* logits, int dtype, int64_t k, int64_t V,
                                 const int32_t* draft, int32_t* tgt, int32_t* tokens,
                                 int32_t* n_accept, int32_t* n_keep, int32_t* cur, int64_t nslab,
                                 void* stream) {
  const char* fn = "hsd_greedy_accept";
  if (!logits || !tgt || !tokens || (k > 0 && !draft)) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (k < 0 || k > 64 || V <= 0 || V > 0x7FFFFFFE) return set_error(HSD_ERR_SHAPE, "%s: bad k/V", fn);
  if (cur && (nslab < k + 2 || nslab > kLMax + 1))
    return set_error(HSD_ERR_SHAPE, "%s: nslab must be in [k+2, %d]", fn, kLMax + 1);
  hipStream_t st = as_stream(stream);
  switch (dtype) {
    case HSD_DT_BF16:
      hipLaunchKernelGGL(k_argmax_rows<HSD_DT_BF16>, dim3((unsigned)(k + 1)), dim3(kAT), 0, st,
                         reinterpret_cast<const uint16_t*>(logits), V, tgt);
      break;
    case HSD_DT_F16:
      hipLaunchKernelGGL(k_argmax_rows<HSD_DT_F16>, dim3((unsigned)(k + 1)), dim3(kAT), 0, st,
                         reinterpret_cast<const uint16_t*>(logits), V, tgt);
      break;
    case HSD_DT_F32:
      hipLaunchKernelGGL(k_argmax_rows<HSD_DT_F32>, dim3((unsigned)(k + 1)), dim3(kAT), 0, st,
                         reinterpret_cast<const float*>(logits), V, tgt);
      break;
    default: return set_error(HSD_ERR_DTYPE, "%s: dtype %d", fn, dtype);
  }
  int rc = check_launch(fn);
  if (rc) return rc;
  hipLaunchKernelGGL(k_accept, dim3(1), dim3(64), 0, st, draft, tgt, (int)k, tokens, n_accept,
                     n_keep, cur, (int)nslab);
  return check_launch(fn);
}
