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
// Work split of the state update (Nemotron-3.5 Mamba-2 layer: H=64 heads x P=64 head_dim x N=128 state,
// G=8 groups, conv K=4, CD = 4096 + 2*8*128 = 6144 channels):
//   one workgroup = (head h, block of 16 head_dim rows p): 256 WGs. It computes the conv
//   + silu of its 16 x channels and of its group's 128 B and 128 C channels for all L
//   rows (LDS), then each wave streams 4 state rows S[h, p, :] (128 fp32: 16 lanes per
//   row, 8 elements each) through the L rows: S = dA*S + (x*dt)*B, y = sum_n S*C + D*x
//   (a lane's 8 products, then a butterfly over the row's 16 lanes), and writes each
//   row's S to its checkpoint slab. HBM: read S once, write L checkpoints; all loads in
//   two round trips (the ring index, then what depends on it).
// The gated RMSNorm (groups of 512 = 8 heads) runs as a second small kernel
// (hsd_mamba_verify), or in out_proj's prologue: hsd_mamba_ssm_gated has this kernel apply
// the gate (z = y silu(gate)) and write, after each row's z, every 16-channel block's sum
// of z^2, so the prologue only adds 32 partials per group (no silu, no gate loads).
#include "hsd_common.h"

namespace hsd {
namespace {

constexpr int kMT = 256;
constexpr int kPB = 16;      // head_dim rows per workgroup
constexpr int kN = 128;      // state size (16 lanes per state row, 8 elements each)
constexpr int kK = 4;        // conv kernel
constexpr int kLMax = 7;     // rows per verify (nslab <= 8)

// The shape (L | G << 16, H | P << 16), the ring index, the conv inputs and weights and dt
// lead the arguments: the dispatch preloads leading scalar arguments into SGPRs, so the
// first round trip's loads need no scalar load of the argument segment before they issue.
__global__ __launch_bounds__(kMT) void k_mamba_ssm(
    int LG, int HP, int cin_ld, const int32_t* __restrict__ cur_ptr, const uint16_t* __restrict__ conv_in,
    const uint16_t* __restrict__ conv_w, const uint16_t* __restrict__ conv_b, const uint16_t* __restrict__ dt_raw,
    int64_t dt_ld, const float* __restrict__ A_log, const float* __restrict__ dt_bias, const float* __restrict__ Dp,
    float* __restrict__ ssm, uint16_t* __restrict__ convs, int nslab, float* __restrict__ y_pre, int64_t y_ld,
    const uint16_t* __restrict__ gate, int64_t gate_ld, float dt_lo, float dt_hi, int32_t* __restrict__ status) {
  const int L = LG & 0xFFFF, G = LG >> 16, H = HP & 0xFFFF, P = HP >> 16;
  __shared__ float xs[kLMax][kPB];
  __shared__ float zsq[kLMax][kPB];
  __shared__ __attribute__((aligned(16))) float Bs[kLMax][kN];
  __shared__ __attribute__((aligned(16))) float Cs[kLMax][kN];
  __shared__ float dtv[kLMax], dA[kLMax];
  const int npb = P / kPB;
  // xcd_remap: consecutive heads (a B/C group's, and a norm group's) run on one XCD, so
  // their shared B/C conv inputs and their y rows stay in that XCD's L2; k_gated_norm's
  // workgroup for norm group g runs on XCD g % 8 as well
  // (the grid is H x P / kPB workgroups, from preloaded arguments: gridDim would be a
  // scalar load of the dispatch's hidden arguments ahead of every load)
  const int lb = xcd_remap((int)blockIdx.x, H * (P / kPB));
  const int hh = lb / npb, pblk = lb - (lb / npb) * npb;
  const int tid = threadIdx.x;
  const int DI = H * P, GN = G * kN, CD = DI + 2 * GN;
  const int hpg = H / G;
  const int g = hh / hpg;
  const bool owner_bc = (hh % hpg == 0) && pblk == 0;  // writes the B/C conv checkpoints
  // Loads in two round trips, never under a branch (a load inside a branch makes the
  // compiler wait for every earlier load where the paths merge): first the ring index
  // with every input that does not depend on it, then the state rows and conv windows.
  // Rows past L re-read row L - 1 and are unused.
  const int cur = *cur_ptr;
  // conv channels: thread t owns channel t of [16 x | 128 B | 128 C]; the last NCH - kMT
  // threads (wave 3) also own channels kMT .. NCH - 1, and wave 1 computes dt and dA, so
  // no wave carries both extras; the others repeat channel t for the second and drop it
  constexpr int NCH = kPB + 2 * kN;
  auto chan = [&](int t) {
    return t < kPB ? hh * P + pblk * kPB + t
                   : (t < kPB + kN ? DI + g * kN + (t - kPB) : DI + GN + g * kN + (t - kPB - kN));
  };
  constexpr int kExtra = NCH - kMT;  // channels past one per thread
  static_assert(kExtra > 0 && kExtra <= 64 && kMT >= 128, "the extra channels fit the last wave");
  const int t1 = tid, t2 = tid >= kMT - kExtra ? tid + kExtra : tid;
  const int ch1 = chan(t1), ch2 = chan(t2);
  uint16_t in1[kLMax], in2[kLMax];
#pragma unroll
  for (int r = 0; r < kLMax; ++r) {
    in1[r] = conv_in[(size_t)min(r, L - 1) * cin_ld + ch1];
    in2[r] = conv_in[(size_t)min(r, L - 1) * cin_ld + ch2];
  }
  uint16_t w1[kK], w2[kK];
#pragma unroll
  for (int j = 0; j < kK; ++j) {
    w1[j] = conv_w[(size_t)ch1 * kK + j];
    w2[j] = conv_w[(size_t)ch2 * kK + j];
  }
  const uint16_t b1 = conv_b[ch1], b2 = conv_b[ch2];
  const int rd = min(max(tid - 64, 0), L - 1);  // wave 1's first L lanes: dt and dA
  const uint16_t dtr = dt_raw[(size_t)rd * dt_ld + hh];
  // the gate of this thread's output channel (state row p below) for every row: read from
  // conv_in (in bounds, unused) when there is no gate, so the load is unconditional
  const uint16_t* gsrc = gate ? gate : conv_in;
  const int64_t gld = gate ? gate_ld : cin_ld;
  const int pg = pblk * kPB + (tid >> 6) * (kPB / (kMT / 64)) + ((tid & 63) >> 4);
  uint16_t gv[kLMax];
#pragma unroll
  for (int r = 0; r < kLMax; ++r) gv[r] = gsrc[(size_t)min(r, L - 1) * gld + (size_t)hh * P + pg];
  // D enters the recurrence rounded to bf16, as the reference passes m.D.astype(x.dtype)
  // to ssm_update (mamba.py:38)
  const float Alog = A_log[hh], dtb = dt_bias[hh], Dh = bf16_bits_to_f32(f32_to_bf16_bits(Dp[hh]));
  if ((unsigned)cur >= (unsigned)nslab) {
    // a corrupt ring index: no state is read or written; the rows' outputs become NaN and
    // the status word says why
    if (tid < kPB * L) y_pre[(size_t)(tid / kPB) * y_ld + (size_t)hh * P + pblk * kPB + tid % kPB] = __int_as_float(0x7FC00000);
    if (gate && tid < L) y_pre[(size_t)tid * y_ld + DI + (size_t)hh * npb + pblk] = __int_as_float(0x7FC00000);
    if (tid == 0 && status) atomicOr(status, (int32_t)HSD_STATUS_BAD_STATE);
    return;
  }

  // the state rows: wave w owns rows 4w .. 4w+3 of the block, lane = 16 i + c holds
  // elements 8c .. 8c+7 of row 4w + i
  const int lane = tid & 63, wave = tid >> 6, ri = lane >> 4, c8 = lane & 15;
  const int pl = wave * (kPB / (kMT / 64)) + ri, p = pblk * kPB + pl;
  const size_t slab_sz = (size_t)H * P * kN;
  const size_t soff = ((size_t)hh * P + p) * kN + 8 * c8;
  float4 S0 = *reinterpret_cast<const float4*>(ssm + (size_t)cur * slab_sz + soff);
  float4 S1 = *reinterpret_cast<const float4*>(ssm + (size_t)cur * slab_sz + soff + 4);
  const uint16_t* cs0 = convs + (size_t)cur * (kK - 1) * CD;
  uint16_t s1[kK - 1], s2[kK - 1];
#pragma unroll
  for (int i = 0; i < kK - 1; ++i) {
    s1[i] = cs0[(size_t)i * CD + ch1];
    s2[i] = cs0[(size_t)i * CD + ch2];
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- depthwise causal conv + silu of the channels this workgroup needs, and the conv
  // checkpoint after row r (window rows r+1 .. r+3)
  auto conv = [&](int t, int ch, const uint16_t (&st)[kK - 1], const uint16_t (&in)[kLMax],
                  const uint16_t (&wr)[kK], uint16_t bb) {
    uint16_t win[kK - 1 + kLMax];
#pragma unroll
    for (int i = 0; i < kK - 1; ++i) win[i] = st[i];
#pragma unroll
    for (int r = 0; r < kLMax; ++r) win[kK - 1 + r] = in[r];
    float wj[kK];
#pragma unroll
    for (int j = 0; j < kK; ++j) wj[j] = bf16_bits_to_f32(wr[j]);
    const float bias = bf16_bits_to_f32(bb);
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
    if (t < kPB || owner_bc) {
#pragma unroll
      for (int r = 0; r < kLMax; ++r) {
        if (r < L) {
          uint16_t* dst = convs + (size_t)((cur + 1 + r) % nslab) * (kK - 1) * CD + ch;
#pragma unroll
          for (int i = 0; i < kK - 1; ++i) dst[(size_t)i * CD] = win[r + 1 + i];
        }
      }
    }
  };
  conv(t1, ch1, s1, in1, w1, b1);
  if (t2 != t1) conv(t2, ch2, s2, in2, w2, b2);
  if (tid >= 64 && tid < 64 + L) {
    const float A = -expf(Alog);
    const float v = softplus_f32(bf16_bits_to_f32(dtr) + dtb);
    const float d = fminf(fmaxf(v, dt_lo), dt_hi);
    dtv[tid - 64] = d;
    dA[tid - 64] = expf(A * d);
  }
  lds_barrier();

  // ---- the state rows through the L rows: S = dA*S + (x*dt)*B, written to the row's
  // checkpoint slab; y = sum_n S*C (8 elements per lane, then 16 lanes) + D*x
  for (int r = 0; r < L; ++r) {
    const float4 B0 = *reinterpret_cast<const float4*>(&Bs[r][8 * c8]);
    const float4 B1 = *reinterpret_cast<const float4*>(&Bs[r][8 * c8 + 4]);
    const float4 C0 = *reinterpret_cast<const float4*>(&Cs[r][8 * c8]);
    const float4 C1 = *reinterpret_cast<const float4*>(&Cs[r][8 * c8 + 4]);
    const float x = xs[r][pl];
    const float xdt = x * dtv[r], a = dA[r];
    S0.x = fmaf(a, S0.x, xdt * B0.x);
    S0.y = fmaf(a, S0.y, xdt * B0.y);
    S0.z = fmaf(a, S0.z, xdt * B0.z);
    S0.w = fmaf(a, S0.w, xdt * B0.w);
    S1.x = fmaf(a, S1.x, xdt * B1.x);
    S1.y = fmaf(a, S1.y, xdt * B1.y);
    S1.z = fmaf(a, S1.z, xdt * B1.z);
    S1.w = fmaf(a, S1.w, xdt * B1.w);
    float* dst = ssm + (size_t)((cur + 1 + r) % nslab) * slab_sz + soff;
    *reinterpret_cast<float4*>(dst) = S0;
    *reinterpret_cast<float4*>(dst + 4) = S1;
    float y = S0.x * C0.x;
    y = fmaf(S0.y, C0.y, y);
    y = fmaf(S0.z, C0.z, y);
    y = fmaf(S0.w, C0.w, y);
    y = fmaf(S1.x, C1.x, y);
    y = fmaf(S1.y, C1.y, y);
    y = fmaf(S1.z, C1.z, y);
    y = fmaf(S1.w, C1.w, y);
    // the 16-lane sum with DPP, no LDS permute: xor 1 and xor 2 inside each quad
    // (quad_perm), then the other quad of each 8 (row_half_mirror) and the other 8 of the
    // row (row_mirror); after the first two steps a quad holds one value, so the mirrors
    // add the same partial sums as xor 4 and xor 8
    y += dpp_f32<0xB1>(y);   // quad_perm [1, 0, 3, 2]
    y += dpp_f32<0x4E>(y);   // quad_perm [2, 3, 0, 1]
    y += dpp_f32<0x141>(y);  // row_half_mirror
    y += dpp_f32<0x140>(y);  // row_mirror
    if (c8 == 0) {
      float yo = y + x * Dh;
      if (gate) {                                      // uniform
        yo *= silu_f32(bf16_bits_to_f32(gv[r]));
        zsq[r][pl] = yo * yo;
      }
      y_pre[(size_t)r * y_ld + (size_t)hh * P + p] = yo;
    }
  }
  if (gate) {
    // this block's sum of z^2 over its 16 channels (in channel order) per row, after the
    // row's z values: the gated norm's group sums start from these partials
    lds_barrier();
    if (tid < L) {
      float s = zsq[tid][0];
#pragma unroll
      for (int i = 1; i < kPB; ++i) s += zsq[tid][i];
      y_pre[(size_t)tid * y_ld + DI + (size_t)hh * npb + pblk] = s;
    }
  }
}

// out[r, i] = norm_w[i] * z_i / sqrt(mean_group(z^2) + eps), z = y_pre * silu(gate);
// one workgroup per (row, norm group).
// PER > 0: NG = PER kMT at compile time (no slice past the group is loaded); PER == 0:
// any NG <= 8 kMT.
template <int YDT, int PER>
__global__ __launch_bounds__(kMT) void k_gated_norm(const float* __restrict__ y_pre,
                                                    const uint16_t* __restrict__ gate,
                                                    int64_t gate_ld,
                                                    const uint16_t* __restrict__ norm_w,
                                                    typename Elem<YDT>::T* __restrict__ y, int DI,
                                                    int NG, float eps) {
  __shared__ float wsum[kMT / 64];
  const int ngrp = DI / NG;
  const int r = blockIdx.x / ngrp, gi = blockIdx.x - (blockIdx.x / ngrp) * ngrp;
  const int per = PER > 0 ? PER : NG / kMT;
  constexpr int kPerMax = PER > 0 ? PER : 8;  // NG <= 8 kMT (checked by the host)
  // every load (activations, gate, weight) in one round trip: slices past per re-read
  // the last one and are dropped (no load under a branch)
  float yv[kPerMax], gv[kPerMax], nw[kPerMax];
#pragma unroll
  for (int i = 0; i < kPerMax; ++i) {
    const int c = gi * NG + min(i, per - 1) * kMT + threadIdx.x;
    nw[i] = bf16_bits_to_f32(norm_w[c]);
    yv[i] = y_pre[(size_t)r * DI + c];
    gv[i] = bf16_bits_to_f32(gate[(size_t)r * gate_ld + c]);
  }
  float z[kPerMax];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kPerMax; ++i) {
    z[i] = i < per ? yv[i] * silu_f32(gv[i]) : 0.0f;
    ss = fmaf(z[i], z[i], ss);
  }
  ss = wave_sum_dpp(ss);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = ss;
  lds_barrier();
  float tot = wsum[0];
#pragma unroll
  for (int w = 1; w < kMT / 64; ++w) tot += wsum[w];
  const float inv = __builtin_amdgcn_rsqf(tot / (float)NG + eps);
#pragma unroll
  for (int i = 0; i < kPerMax; ++i) {
    if (i >= per) break;
    const int c = gi * NG + i * kMT + threadIdx.x;
    Elem<YDT>::store(y, (size_t)r * DI + c, (z[i] * inv) * nw[i]);
  }
}

// cur += n_keep (mod nslab) for 0 <= n_keep <= L (the rows of the last verify); anything
// else leaves cur unchanged and sets HSD_STATUS_BAD_STATE.
__global__ void k_select_row(int32_t* cur, const int32_t* n_keep_dev, int n_keep_host,
                             int nslab, int L, int32_t* status) {
  if (threadIdx.x == 0) {
    const int nk = n_keep_dev ? *n_keep_dev : n_keep_host;
    const int c = *cur;
    if (nk >= 0 && nk <= L && nk < nslab && c >= 0 && c < nslab)
      *cur = (c + nk) % nslab;
    else if (status)
      atomicOr(status, (int32_t)HSD_STATUS_BAD_STATE);
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
                                int32_t* dev_status, void* workspace, size_t workspace_bytes,
                                void* stream) {
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
  if ((uintptr_t)ssm_slabs & 15u) return set_error(HSD_ERR_ALIGN, "%s: ssm_slabs must be 16-byte aligned", fn);
  if (H * (P / kPB) > 0x7FFFFFFF) return set_error(HSD_ERR_SHAPE, "%s: too large", fn);
  const size_t need = hsd_mamba_workspace_bytes(L, H, P);
  if (!workspace || workspace_bytes < need)
    return set_error(HSD_ERR_WORKSPACE, "%s: workspace needs %zu bytes", fn, need);
  hipStream_t st = as_stream(stream);
  float* y_pre = reinterpret_cast<float*>(workspace);
  if (conv_in_ld > 0x7FFFFFFF || H > 0xFFFF || P > 0xFFFF || G > 0xFFFF)
    return set_error(HSD_ERR_SHAPE, "%s: sizes too large", fn);
  hipLaunchKernelGGL(k_mamba_ssm, dim3((unsigned)(H * (P / kPB))), dim3(kMT), 0, st, (int)(L | (G << 16)),
                     (int)(H | (P << 16)), (int)conv_in_ld, cur, conv_in, conv_w, conv_b, dt_raw, dt_ld, A_log,
                     dt_bias, Dp, ssm_slabs, conv_slabs, (int)nslab, y_pre, (int64_t)DI, nullptr, (int64_t)0, dt_lo,
                     dt_hi, dev_status);
  int rc = check_launch(fn);
  if (rc) return rc;
  const unsigned ngrid = (unsigned)(L * (DI / norm_group));
#define HSD_NORM_P(DT, PER)                                                                   \
  hipLaunchKernelGGL((k_gated_norm<DT, PER>), dim3(ngrid), dim3(kMT), 0, st, y_pre, gate, gate_ld, \
                     norm_w, reinterpret_cast<typename Elem<DT>::T*>(y), (int)DI,               \
                     (int)norm_group, eps)
#define HSD_NORM(DT)                                          \
  switch (norm_group / kMT) {                                 \
    case 1: HSD_NORM_P(DT, 1); break;                         \
    case 2: HSD_NORM_P(DT, 2); break;                         \
    case 4: HSD_NORM_P(DT, 4); break;                         \
    default: HSD_NORM_P(DT, 0); break;                        \
  }
  switch (y_dtype) {
    case HSD_DT_BF16: HSD_NORM(HSD_DT_BF16); break;
    case HSD_DT_F16: HSD_NORM(HSD_DT_F16); break;
    case HSD_DT_F32: HSD_NORM(HSD_DT_F32); break;
    default: return set_error(HSD_ERR_DTYPE, "%s: y_dtype %d", fn, y_dtype);
  }
#undef HSD_NORM
#undef HSD_NORM_P
  return check_launch(fn);
}

extern "C" int hsd_mamba_select_row(int32_t* cur, const int32_t* n_keep_dev, int64_t n_keep_host,
                                    int64_t L, int64_t nslab, int32_t* dev_status, void* stream) {
  if (!cur) return set_error(HSD_ERR_ARG, "hsd_mamba_select_row: null cur");
  if (nslab < 2 || nslab > kLMax + 1) return set_error(HSD_ERR_SHAPE, "hsd_mamba_select_row: bad nslab");
  if (L < 0 || L >= nslab) return set_error(HSD_ERR_SHAPE, "hsd_mamba_select_row: L must be in [0, nslab)");
  if (!n_keep_dev && (n_keep_host < 0 || n_keep_host > L))
    return set_error(HSD_ERR_ARG, "hsd_mamba_select_row: n_keep %lld outside [0, L = %lld]", (long long)n_keep_host,
                     (long long)L);
  hipLaunchKernelGGL(k_select_row, dim3(1), dim3(64), 0, as_stream(stream), cur, n_keep_dev,
                     (int)n_keep_host, (int)nslab, (int)L, dev_status);
  return check_launch("hsd_mamba_select_row");
}

namespace {
int launch_ssm(const char* fn, const uint16_t* conv_in, int64_t conv_in_ld, const uint16_t* dt_raw, int64_t dt_ld,
               const uint16_t* conv_w, const uint16_t* conv_b, const float* A_log, const float* dt_bias,
               const float* Dp, float* ssm_slabs, uint16_t* conv_slabs, const int32_t* cur, int64_t nslab, float* y,
               int64_t y_ld, const uint16_t* gate, int64_t gate_ld, int64_t L, int64_t H, int64_t P, int64_t N,
               int64_t G, float dt_lo, float dt_hi, int32_t* dev_status, void* stream) {
  if (!conv_in || !dt_raw || !conv_w || !conv_b || !A_log || !dt_bias || !Dp || !ssm_slabs || !conv_slabs ||
      !cur || !y)
    return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (N != kN) return set_error(HSD_ERR_SHAPE, "%s: state size N must be %d (got %lld)", fn, kN, (long long)N);
  if (L < 1 || L > kLMax || nslab < L + 1 || nslab > kLMax + 1)
    return set_error(HSD_ERR_SHAPE, "%s: need 1 <= L <= nslab-1 <= %d (L=%lld nslab=%lld)", fn, kLMax,
                     (long long)L, (long long)nslab);
  if (H <= 0 || P <= 0 || P % kPB || G <= 0 || H % G)
    return set_error(HSD_ERR_SHAPE, "%s: need P %% %d == 0 and H %% G == 0", fn, kPB);
  const int64_t DI = H * P, CD = DI + 2 * G * N;
  if (conv_in_ld < CD || dt_ld < H) return set_error(HSD_ERR_SHAPE, "%s: row strides smaller than the rows", fn);
  if (y_ld < (gate ? DI + DI / kPB : DI) || (gate && gate_ld < DI))
    return set_error(HSD_ERR_SHAPE, "%s: row strides smaller than the rows", fn);
  if ((uintptr_t)ssm_slabs & 15u) return set_error(HSD_ERR_ALIGN, "%s: ssm_slabs must be 16-byte aligned", fn);
  if (conv_in_ld > 0x7FFFFFFF || H > 0xFFFF || P > 0xFFFF || G > 0xFFFF)
    return set_error(HSD_ERR_SHAPE, "%s: sizes too large", fn);
  hipLaunchKernelGGL(k_mamba_ssm, dim3((unsigned)(H * (P / kPB))), dim3(kMT), 0, as_stream(stream),
                     (int)(L | (G << 16)), (int)(H | (P << 16)), (int)conv_in_ld, cur, conv_in, conv_w, conv_b,
                     dt_raw, dt_ld, A_log, dt_bias, Dp, ssm_slabs, conv_slabs, (int)nslab, y, y_ld, gate, gate_ld,
                     dt_lo, dt_hi, dev_status);
  return check_launch(fn);
}
}  // namespace

extern "C" int hsd_mamba_ssm(const uint16_t* conv_in, int64_t conv_in_ld, const uint16_t* dt_raw, int64_t dt_ld,
                             const uint16_t* conv_w, const uint16_t* conv_b, const float* A_log,
                             const float* dt_bias, const float* Dp, float* ssm_slabs, uint16_t* conv_slabs,
                             const int32_t* cur, int64_t nslab, float* y, int64_t L, int64_t H, int64_t P,
                             int64_t N, int64_t G, float dt_lo, float dt_hi, int32_t* dev_status, void* stream) {
  return launch_ssm("hsd_mamba_ssm", conv_in, conv_in_ld, dt_raw, dt_ld, conv_w, conv_b, A_log, dt_bias, Dp,
                    ssm_slabs, conv_slabs, cur, nslab, y, H * P, nullptr, 0, L, H, P, N, G, dt_lo, dt_hi,
                    dev_status, stream);
}

extern "C" int hsd_mamba_ssm_gated(const uint16_t* conv_in, int64_t conv_in_ld, const uint16_t* dt_raw,
                                   int64_t dt_ld, const uint16_t* gate, int64_t gate_ld, const uint16_t* conv_w,
                                   const uint16_t* conv_b, const float* A_log, const float* dt_bias,
                                   const float* Dp, float* ssm_slabs, uint16_t* conv_slabs, const int32_t* cur,
                                   int64_t nslab, float* z, int64_t z_ld, int64_t L, int64_t H, int64_t P,
                                   int64_t N, int64_t G, float dt_lo, float dt_hi, int32_t* dev_status,
                                   void* stream) {
  if (!gate) return set_error(HSD_ERR_ARG, "hsd_mamba_ssm_gated: null gate");
  return launch_ssm("hsd_mamba_ssm_gated", conv_in, conv_in_ld, dt_raw, dt_ld, conv_w, conv_b, A_log, dt_bias,
                    Dp, ssm_slabs, conv_slabs, cur, nslab, z, z_ld, gate, gate_ld, L, H, P, N, G, dt_lo, dt_hi,
                    dev_status, stream);
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
