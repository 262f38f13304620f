// GQA attention for decode and verify steps over a KV cache that rollback trims by
// moving its length: mlx-lm's NemotronH attention block as hsd runs it (model.py:287 for
// a decode step, model.py:343 with a causal mask for a verify step; no positional
// encoding in this model family), after the q/k/v projections.
//
// B <= 4 consecutive positions P .. P+B-1 (P = the cache length before the call, a
// device int, so a captured graph replays at any length). Row r attends to keys
// 0 .. P+r. The new keys and values come from the projection output itself and are also
// written into the cache at P .. P+B-1; the cache is read only below P, so no kernel reads
// what this launch writes.
//
//   k_attn_part: one workgroup per (kv head, 32-key chunk, 16 of the kv head's query
//     heads: all of them in this model; 8 or 4 for other ratios), a wavefront per query head, so a chunk's keys and
//     values are loaded once (4 heads per 256-thread workgroup: the MTP-2 step 1.922
//     against 1.915 ms, the decode step 1.075 against 1.064). 32-key chunks halve each
//     thread's value sum for twice the workgroups and partials (against 64-key ones:
//     1.907 against 1.915 ms, 1.061 against 1.067; 16-key ones: 1.997 and 1.085, the
//     combine then past its up-front loads). The chunk's keys go to LDS
//     (rows padded by 16 bytes against bank conflicts); lane 32 u + j of wave w scores
//     key j against query head w + u HPW/2 (a q.k dot in fp32 with v_dot2_f32_bf16 in four
//     partial sums, times the scale), so half the wavefronts score (one head per
//     wavefront with lanes 32-63 idle had taken 1.913 against 1.901 ms); a
//     half-wavefront's max and sum over the chunk's keys (DPP); then
//     p = exp(s - m) times V (LDS) into acc[128] (even and odd keys in separate sums).
//     Writes the chunk's (m, l, acc) per row and head.
//   k_attn_combine: one workgroup per (row, query head): the chunks of keys 0 .. P+r in
//     chunk order: M = max m, L = sum l e^(m-M), o = sum acc e^(m-M) / L, rounded to bf16.
// The chunk boundaries are absolute positions and each row's chunks are combined in the
// same order whatever B is, so a row of a B-row verify is bit-identical to that row
// computed by a single-row decode step.
#include "hsd_common.h"

namespace hsd {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kHD = 128;        // head dim
constexpr int kCH = 32;         // keys per chunk (lanes kCH .. 63 of the scores idle)
constexpr int kAMaxB = 4;
constexpr int kKP = kHD / 2 + 4;  // padded K row in u32 (272 bytes)
constexpr int kMaxHPW = 16;      // query heads per workgroup: 16, or 8 or 4 for other GQA ratios
constexpr int kRec = kHD + 4;     // partial record: m, l, 2 unused, acc[128] (16-byte aligned)

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

struct AttnArgs {
  const uint16_t* qkv;
  int64_t qkv_ld;
  uint16_t* kc;
  uint16_t* vc;
  int64_t smax;
  const int32_t* pos;
  float* part;            // [B][HQ][nch][kRec]
  uint16_t* out;
  int64_t out_ld;
  int32_t* status;
  int B, HQ, HKV, nch;
  float scale;
};

// The fields each kernel's first loads need go ahead of the struct as scalar arguments,
// which the dispatch preloads into SGPRs (a struct argument is read by scalar loads from
// the argument segment, which the first global loads would wait for); the kernels rebuild
// the whole struct from both.
#define HSD_ATTN_PART_PARAMS                                                                    \
  const int32_t *pos_, const uint16_t *qkv_, uint16_t *kc_, uint16_t *vc_, int64_t qkv_ld_,      \
      int64_t smax_, int HQ_, int nch_, AttnArgs a_
#define HSD_ATTN_PART_ARGS(a) a.pos, a.qkv, a.kc, a.vc, a.qkv_ld, a.smax, a.HQ, a.nch, a
#define HSD_ATTN_COMB_PARAMS                                                                    \
  const int32_t *pos_, float *part_, uint16_t *out_, int64_t out_ld_, int64_t smax_,       \
      int HQ_, int nch_, int B_, AttnArgs a_
#define HSD_ATTN_COMB_ARGS(a) a.pos, a.part, a.out, a.out_ld, a.smax, a.HQ, a.nch, a.B, a

template <int kHPW>  // query heads per workgroup, one wavefront each
__global__ __launch_bounds__(64 * kHPW) void k_attn_part(HSD_ATTN_PART_PARAMS) {
  AttnArgs a = a_;
  a.pos = pos_;
  a.qkv = qkv_;
  a.kc = kc_;
  a.vc = vc_;
  a.qkv_ld = qkv_ld_;
  a.smax = smax_;
  a.HQ = HQ_;
  a.nch = nch_;
  constexpr int kAT = 64 * kHPW;
  constexpr int kAW = kAT / 64;     // wavefronts per workgroup
  constexpr int kTPH = kAT / kHPW;  // threads per head in the value sum
  constexpr int kDPT = 128 / kTPH;  // head dims per thread there
  constexpr int kLT = kCH * 16 < kAT ? kCH * 16 : kAT;  // threads loading K and V (16 bytes each)
  constexpr int kLI = kCH * 16 / kLT;  // 16-byte K (and V) pieces per loading thread
  static_assert(kHPW == kAW && kHPW % 2 == 0 && kCH <= 64 && kCH * 16 % kLT == 0 && kLT % 64 == 0 && kHPW <= kMaxHPW,
                "attention workgroup shape");
  __shared__ __attribute__((aligned(16))) uint32_t ks[kCH][kKP];
  __shared__ __attribute__((aligned(16))) float vs[kCH][kHD];     // V in fp32 (converted once)
  __shared__ __attribute__((aligned(16))) uint32_t qs[kAMaxB][kHPW][kHD / 2];
  __shared__ float ps[kAMaxB][kHPW][kCH];
  // the device length first: its load (preloaded pointer) leaves before the workgroup's
  // coordinates, which wait for the rest of the arguments
  const int P = *a.pos;
  __builtin_amdgcn_sched_barrier(0);
  const int nhalf = a.HQ / a.HKV / kHPW;       // workgroups per (kv head, chunk)
  const int g = blockIdx.x / (a.nch * nhalf);
  const int rem = blockIdx.x - g * a.nch * nhalf;
  const int c = rem / nhalf, hh = rem - c * nhalf;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int B = a.B;
  if (P < 0 || P + B > a.smax) {
    if (blockIdx.x == 0 && tid == 0 && a.status) atomicOr(a.status, (int32_t)HSD_STATUS_BAD_STATE);
    return;
  }
  const int j0 = c * kCH;
  if (j0 > P + B - 1) return;                  // no key of this chunk is visible to any row
  const int HQ = a.HQ, QD = HQ * kHD, KD = a.HKV * kHD;
  const int hq0 = g * (HQ / a.HKV) + hh * kHPW;  // first query head of this workgroup

  // ---- loads: the chunk's K and V rows (256 bytes each: 16 lanes x 16 bytes), from the
  // cache below P and from the projection rows at P .. P+B-1; this workgroup's query
  // heads for every row (8 heads x 256 bytes per row)
  {
    const int piece = tid & 15;
#pragma unroll
    for (int i = 0; i < kLI; ++i) {
      if (tid >= kLT) break;                     // whole wavefronts
      const int jl = (tid >> 4) + (kLT / 16) * i, j = j0 + jl;
      const bool cached = j < P;
      const int r = min(max(j - P, 0), B - 1);
      const uint16_t* ksrc = cached ? a.kc + ((size_t)g * a.smax + j) * kHD
                                    : a.qkv + (size_t)r * a.qkv_ld + QD + g * kHD;
      const uint16_t* vsrc = cached ? a.vc + ((size_t)g * a.smax + j) * kHD
                                    : a.qkv + (size_t)r * a.qkv_ld + QD + KD + g * kHD;
      const uint4 kv = reinterpret_cast<const uint4*>(ksrc)[piece];
      const uint4 vv = reinterpret_cast<const uint4*>(vsrc)[piece];
      *reinterpret_cast<uint4*>(&ks[jl][4 * piece]) = kv;
      {
        const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
        float vf[8];
#pragma unroll
        for (int c2 = 0; c2 < 4; ++c2) {
          vf[2 * c2] = bf16_bits_to_f32(vw[c2] & 0xFFFFu);
          vf[2 * c2 + 1] = bf16_bits_to_f32(vw[c2] >> 16);
        }
        *reinterpret_cast<float4*>(&vs[jl][8 * piece]) = make_float4(vf[0], vf[1], vf[2], vf[3]);
        *reinterpret_cast<float4*>(&vs[jl][8 * piece + 4]) = make_float4(vf[4], vf[5], vf[6], vf[7]);
      }
      // the new rows also go to the cache (hh == 0: one writer per position)
      if (!cached && j < P + B && hh == 0) {
        reinterpret_cast<uint4*>(a.kc + ((size_t)g * a.smax + j) * kHD)[piece] = kv;
        reinterpret_cast<uint4*>(a.vc + ((size_t)g * a.smax + j) * kHD)[piece] = vv;
      }
    }
    // queries: B rows x kHPW heads x 16 pieces
    for (int i = tid; i < B * kHPW * 16; i += kAT) {
      const int r = i / (kHPW * 16), rem2 = i - r * kHPW * 16, h = rem2 >> 4, pc = rem2 & 15;
      const uint4 qv = reinterpret_cast<const uint4*>(a.qkv + (size_t)r * a.qkv_ld + (hq0 + h) * kHD)[pc];
      *reinterpret_cast<uint4*>(&qs[r][h][4 * pc]) = qv;
    }
  }
  __syncthreads();

  // ---- scores: a half-wavefront per query head, lane 32 u + j on key j; wavefront w <
  // kSW takes heads w and w + kSW (the other wavefronts wait at the barrier)
  constexpr int kSW = kHPW / 2;                        // wavefronts that score
  static_assert(kCH == 32, "a half-wavefront's 32 lanes are the chunk's keys");
  const int half = lane >> 5, jk = lane & 31;
  const int hs = wave + kSW * half;                    // this lane's query head
  const int j = j0 + jk;
  float m[kAMaxB], l[kAMaxB];
  if (wave < kSW) {                                    // uniform
    uint32_t kr[kHD / 2];
#pragma unroll
    for (int i = 0; i < kHD / 8; ++i) {
      const uint4 v = *reinterpret_cast<const uint4*>(&ks[jk][4 * i]);
      kr[4 * i] = v.x; kr[4 * i + 1] = v.y; kr[4 * i + 2] = v.z; kr[4 * i + 3] = v.w;
    }
#pragma unroll
    for (int r = 0; r < kAMaxB; ++r) {
      if (r < B) {                                     // uniform
        const bool vis = j <= P + r;
        // four partial dot products (16-byte pieces i % 4), so that four dependency chains
        // of 16 interleave instead of one of 64
        float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < kHD / 8; ++i) {
          const uint4 qv = *reinterpret_cast<const uint4*>(&qs[r][hs][4 * i]);
          float t = s4[i & 3];
          t = dot2(qv.x, kr[4 * i], t);
          t = dot2(qv.y, kr[4 * i + 1], t);
          t = dot2(qv.z, kr[4 * i + 2], t);
          t = dot2(qv.w, kr[4 * i + 3], t);
          s4[i & 3] = t;
        }
        float s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
        s = vis ? s * a.scale : -INFINITY;
        // the half-wavefront's max: DPP inside rows of 16, then its two row maxima
        float mx = s;
        mx = fmaxf(mx, dpp_f32<0xB1>(mx));
        mx = fmaxf(mx, dpp_f32<0x4E>(mx));
        mx = fmaxf(mx, dpp_f32<0x141>(mx));
        mx = fmaxf(mx, dpp_f32<0x140>(mx));
        const float m0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 0));
        const float m1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 16));
        const float m2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 32));
        const float m3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 48));
        const float M = half ? fmaxf(m2, m3) : fmaxf(m0, m1);  // finite: key j0 is visible
        const float p = vis ? __expf(s - M) : 0.0f;
        ps[r][hs][jk] = p;
        m[r] = M;
        // the half-wavefront's sum of p: DPP inside rows, then its two row sums
        float v = p;
        v += dpp_f32<0xB1>(v);
        v += dpp_f32<0x4E>(v);
        v += dpp_f32<0x141>(v);
        v += dpp_f32<0x140>(v);
        const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
        const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
        const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
        const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
        l[r] = half ? r2 + r3 : r0 + r1;
      }
    }
  }
  __syncthreads();

  // ---- acc = sum_j p_j v_j: thread = (head h = tid / kTPH, dims kDPT (tid % kTPH) ..)
  {
    const int h = tid / kTPH, d0 = kDPT * (tid % kTPH);
    // two accumulator sets (even and odd keys), added at the end: twice the independent
    // chains for the latency of the fma and LDS reads
    float acc[kAMaxB][kDPT], acc2[kAMaxB][kDPT];
#pragma unroll
    for (int r = 0; r < kAMaxB; ++r)
#pragma unroll
      for (int e = 0; e < kDPT; ++e) acc[r][e] = acc2[r][e] = 0.0f;
#pragma unroll 4
    for (int jl = 0; jl < kCH; jl += 2) {
      float va[kDPT], vb[kDPT];
#pragma unroll
      for (int e = 0; e < kDPT; e += 2) {
        const float2 fa = *reinterpret_cast<const float2*>(&vs[jl][d0 + e]);
        const float2 fb = *reinterpret_cast<const float2*>(&vs[jl + 1][d0 + e]);
        va[e] = fa.x;
        va[e + 1] = fa.y;
        vb[e] = fb.x;
        vb[e + 1] = fb.y;
      }
#pragma unroll
      for (int r = 0; r < kAMaxB; ++r) {
        if (r < B) {
          const float2 p = *reinterpret_cast<const float2*>(&ps[r][h][jl]);
#pragma unroll
          for (int e = 0; e < kDPT; ++e) {
            acc[r][e] = fmaf(p.x, va[e], acc[r][e]);
            acc2[r][e] = fmaf(p.y, vb[e], acc2[r][e]);
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kAMaxB; ++r)
#pragma unroll
      for (int e = 0; e < kDPT; ++e) acc[r][e] += acc2[r][e];
#pragma unroll
    for (int r = 0; r < kAMaxB; ++r) {
      if (r < B && j0 <= P + r) {
        float* dst = a.part + (((size_t)r * HQ + hq0 + h) * a.nch + c) * kRec + 4 + d0;
#pragma unroll
        for (int e = 0; e < kDPT; e += 2) *reinterpret_cast<float2*>(dst + e) = make_float2(acc[r][e], acc[r][e + 1]);
      }
    }
  }
  // m and l of each (row, head): the first lane of the half-wavefront that computed them
  if (wave < kSW && jk == 0) {
#pragma unroll
    for (int r = 0; r < kAMaxB; ++r) {
      if (r < B && j0 <= P + r) {
        float* dst = a.part + (((size_t)r * HQ + hq0 + hs) * a.nch + c) * kRec;
        dst[0] = m[r];
        dst[1] = l[r];
      }
    }
  }
}

constexpr int kMaxCh = 512;      // chunks per row the combine stages in LDS (smax <= 16384)
constexpr int kPre = 64;         // chunks whose values the combine loads up front (2048 keys;
                                 // 128 measured no faster, 158 VGPRs)

__global__ __launch_bounds__(kHD) void k_attn_combine(HSD_ATTN_COMB_PARAMS) {
  AttnArgs a = a_;
  a.pos = pos_;
  a.part = part_;
  a.out = out_;
  a.out_ld = out_ld_;
  a.smax = smax_;
  a.HQ = HQ_;
  a.nch = nch_;
  a.B = B_;
  __shared__ float mw[kMaxCh];    // the chunks' maxima, then their weights e^(m - M)
  __shared__ float lw[kMaxCh];
  __shared__ float red[2];
  const int r = blockIdx.x / a.HQ, h = blockIdx.x - r * a.HQ;
  const int d = threadIdx.x;
  const int P = *a.pos;
  uint16_t* o = a.out + (size_t)r * a.out_ld + (size_t)h * kHD;
  if (P < 0 || P + a.B > a.smax) {
    o[d] = 0;
    return;
  }
  const int nc = (P + r) / kCH + 1;
  const float* src = a.part + ((size_t)r * a.HQ + h) * a.nch * kRec;
  // this dimension's values of the first kPre chunks, all issued with the (m, l) loads
  // (they do not depend on the maximum), in blocks of 8 so that a short row issues few
  float v0[kPre];
#pragma unroll
  for (int b = 0; b < kPre; b += 8) {
    if (b < nc) {
#pragma unroll
      for (int u = b; u < b + 8; ++u) v0[u] = src[(size_t)min(u, nc - 1) * kRec + 4 + d];
    }
  }
  // (m, l) of every chunk in one round trip, into LDS
  for (int c = d; c < nc; c += kHD) {
    mw[c] = src[(size_t)c * kRec];
    lw[c] = src[(size_t)c * kRec + 1];
  }
  __syncthreads();
  if (d < 64) {
    float M = -INFINITY;
    for (int c = d; c < nc; c += 64) M = fmaxf(M, mw[c]);
    M = wave_max_f32(M);
    if (d == 0) red[0] = M;
  }
  __syncthreads();
  const float M = red[0];
  for (int c = d; c < nc; c += kHD) mw[c] = __expf(mw[c] - M);
  __syncthreads();
  // L and this dimension's sum over the chunks in chunk order; chunks past kPre (contexts
  // above kPre * kCH keys) load in passes of 16 whose loads are all issued before the sums
  float L = 0.0f, acc = 0.0f;
#pragma unroll
  for (int u = 0; u < kPre; ++u) {
    if (u < nc) {
      L = fmaf(lw[u], mw[u], L);
      acc = fmaf(v0[u], mw[u], acc);
    }
  }
  for (int c = kPre; c < nc; c += 16) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = src[(size_t)min(c + u, nc - 1) * kRec + 4 + d];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      if (c + u < nc) {
        L = fmaf(lw[c + u], mw[c + u], L);
        acc = fmaf(v[u], mw[c + u], acc);
      }
    }
  }
  o[d] = f32_to_bf16_bits(acc / L);
}

}  // namespace
}  // namespace hsd

using namespace hsd;

extern "C" size_t hsd_attn_workspace_bytes(int64_t B, int64_t HQ, int64_t smax) {
  if (B <= 0 || HQ <= 0 || smax <= 0) return 0;
  const int64_t nch = (smax + kCH - 1) / kCH;
  return ((size_t)B * HQ * nch * kRec * sizeof(float) + 255) & ~(size_t)255;
}

extern "C" int hsd_attn_decode(const uint16_t* qkv, int64_t qkv_ld, int64_t B, uint16_t* k_cache,
                               uint16_t* v_cache, int64_t smax, const int32_t* pos, uint16_t* out,
                               int64_t out_ld, int64_t HQ, int64_t HKV, int64_t HD, float scale,
                               int32_t* dev_status, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "hsd_attn_decode";
  if (!qkv || !k_cache || !v_cache || !pos || !out) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (HD != kHD) return set_error(HSD_ERR_SHAPE, "%s: head_dim must be %d", fn, kHD);
  if (B < 1 || B > kAMaxB) return set_error(HSD_ERR_SHAPE, "%s: B must be in [1, %d]", fn, kAMaxB);
  if (HKV <= 0 || HQ <= 0 || HQ % HKV || (HQ / HKV) % 4)
    return set_error(HSD_ERR_SHAPE, "%s: query heads per kv head must be a multiple of 4", fn);
  // heads per workgroup: all 16 of a kv head where the ratio allows (each chunk's keys and
  // values loaded once), else 8 or 4
  const int ratio = (int)(HQ / HKV);
  const int hpw = ratio % 16 == 0 ? 16 : ratio % 8 == 0 ? 8 : 4;
  if (smax <= 0 || smax % kCH || smax > kCH * kMaxCh)
    return set_error(HSD_ERR_SHAPE, "%s: the cache length must be a multiple of %d and at most %d", fn, kCH,
                     kCH * kMaxCh);
  if (qkv_ld < (HQ + 2 * HKV) * kHD || qkv_ld % 8 || out_ld < HQ * kHD)
    return set_error(HSD_ERR_SHAPE, "%s: row strides", fn);
  if (((uintptr_t)qkv | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15u)
    return set_error(HSD_ERR_ALIGN, "%s: qkv and the caches must be 16-byte aligned", fn);
  const size_t need = hsd_attn_workspace_bytes(B, HQ, smax);
  if (!workspace || workspace_bytes < need) return set_error(HSD_ERR_WORKSPACE, "%s: workspace needs %zu bytes", fn, need);
  const int nch = (int)(smax / kCH);
  AttnArgs a{qkv, qkv_ld, k_cache, v_cache, smax, pos, reinterpret_cast<float*>(workspace), out, out_ld,
             dev_status, (int)B, (int)HQ, (int)HKV, nch, scale};
  hipStream_t st = as_stream(stream);
  const int64_t nwg = HKV * nch * (ratio / hpw);
  if (nwg > 0x7FFFFFFF) return set_error(HSD_ERR_SHAPE, "%s: too large", fn);
  if (hpw == 16)
    hipLaunchKernelGGL(k_attn_part<16>, dim3((unsigned)nwg), dim3(64 * 16), 0, st, HSD_ATTN_PART_ARGS(a));
  else if (hpw == 8)
    hipLaunchKernelGGL(k_attn_part<8>, dim3((unsigned)nwg), dim3(64 * 8), 0, st, HSD_ATTN_PART_ARGS(a));
  else
    hipLaunchKernelGGL(k_attn_part<4>, dim3((unsigned)nwg), dim3(64 * 4), 0, st, HSD_ATTN_PART_ARGS(a));
  int rc = check_launch(fn);
  if (rc) return rc;
  hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)(B * HQ)), dim3(kHD), 0, st, HSD_ATTN_COMB_ARGS(a));
  return check_launch(fn);
}
