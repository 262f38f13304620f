// The small kernels that tie a decode / verify step together on the device, so a whole
// step is one captured graph with no host round trip (hsd/model.py:281-323 `step` /
// `generate`, 333-356 `verify_step` / `rollback`, 366-443 `generate_mtp`):
//   k_embed_q4       the quantised token embedding (mlx QuantizedEmbedding, model.py:223)
//   k_pair_norm      concat(rms_norm(e, enorm), rms_norm(h, hnorm)): the MTP head's input
//                    (mtp.py:81-83)
//   k_head_in        the two above in one launch (the head's token rows embedded and
//                    normed in place), or for the head's chained call with the chaining
//                    of k_mtp_chain in front
//   k_verify_in      k_draft and the verify rows' embedding in one launch
//   k_decode_advance argmax of the last row + the sequence state after a plain step
//   k_spec_accept    greedy acceptance of a verify step + the rollback of every cache
//   k_mtp_chain      the inputs of the MTP head's chained call (mtp.py, model.py:408-414)
//   k_draft          the verify ids [tok, drafts], optionally with scripted acceptance
//
// The sequence state is a device int32 array (HSD_SEQ_* indices in hsd.h): the attention
// caches' length, the Mamba ring index, the count of emitted tokens, the last token, the
// MTP head's cache length and pending-row count, ...
#include "hsd_common.h"

namespace hsd {
namespace {

// ---------------------------------------------------------------- embedding
// out[b, i] = bf16(s[t, i/64] * q[t, i] + b[t, i/64]), t = tok[b] (one workgroup per row;
// thread = 8 outputs = one word). A token outside [0, V) gives a zero row and the status
// bit HSD_STATUS_BAD_TOKEN.
__device__ __forceinline__ void embed_row(int t, const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
                                          const uint16_t* __restrict__ bq, int V, int D, uint16_t* __restrict__ orow,
                                          int32_t* __restrict__ status) {
  const bool ok = (unsigned)t < (unsigned)V;
  const size_t row = ok ? (size_t)t : 0;
  // passes of 4 words per thread, each pass's loads issued before they are used
  constexpr int kIt = 4;
  const int NW = D / 8;
  for (int p0 = 0; p0 < NW; p0 += 256 * kIt) {
    uint32_t qv[kIt];
    uint16_t sv[kIt], bv[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int wi = min(p0 + (int)threadIdx.x + 256 * it, NW - 1);
      qv[it] = w[row * (D / 8) + wi];
      sv[it] = s[row * (D / 64) + wi / 8];
      bv[it] = bq[row * (D / 64) + wi / 8];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int wi = p0 + (int)threadIdx.x + 256 * it;
      const uint32_t q = qv[it];
      const float sc = bf16_bits_to_f32(sv[it]), bi = bf16_bits_to_f32(bv[it]);
      uint32_t o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t lo = ok ? f32_to_bf16_bits(fmaf(sc, (float)((q >> (8 * c)) & 0xFu), bi)) : 0u;
        const uint32_t hi = ok ? f32_to_bf16_bits(fmaf(sc, (float)((q >> (8 * c + 4)) & 0xFu), bi)) : 0u;
        o[c] = lo | (hi << 16);
      }
      if (wi < NW) reinterpret_cast<uint4*>(orow)[wi] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  if (!ok && threadIdx.x == 0 && status) atomicOr(status, (int32_t)HSD_STATUS_BAD_TOKEN);
}

__global__ __launch_bounds__(256) void k_embed_q4(const int32_t* __restrict__ tok, const uint32_t* __restrict__ w,
                                                  const uint16_t* __restrict__ s, const uint16_t* __restrict__ bq,
                                                  int V, int D, uint16_t* __restrict__ out, int64_t out_ld,
                                                  int32_t* __restrict__ status) {
  const int b = blockIdx.x;
  embed_row(tok[b], w, s, bq, V, D, out + (size_t)b * out_ld, status);
}

// ---------------------------------------------------------------- pair norm
// One row's rms_norm by one 256-thread workgroup: o[i] = bf16(bf16(x_i * rsqrt(mean(x^2) +
// eps)) * w_i), x_i the bf16 value src gives for element i. A pass of 16 elements per
// thread: every load issued before the first is used (a loop with one load per step waits
// for each in turn); the sum keeps the element order.
struct RowBf16 {                                       // a bf16 row in memory
  const uint16_t* p;
  struct Raw {
    uint16_t v;
  };
  __device__ __forceinline__ Raw load(int i) const { return {p[i]}; }
  __device__ __forceinline__ uint16_t bits(const Raw& r, int) const { return r.v; }
};
struct RowEmbed {                                      // row `row` of the 4-bit embedding, as k_embed_q4 writes it
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  size_t row;
  int D;
  bool ok;
  struct Raw {
    uint32_t q;
    uint16_t s, b;
  };
  __device__ __forceinline__ Raw load(int i) const {
    return {w[row * (D / 8) + i / 8], s[row * (D / 64) + i / 64], b[row * (D / 64) + i / 64]};
  }
  __device__ __forceinline__ uint16_t bits(const Raw& r, int i) const {
    // element i is nibble i % 8 of word i / 8 (k_embed_q4: bits 8c and 8c + 4 of a word
    // are elements 2c and 2c + 1)
    return ok ? f32_to_bf16_bits(fmaf(bf16_bits_to_f32(r.s), (float)((r.q >> (4 * (i & 7))) & 0xFu),
                                      bf16_bits_to_f32(r.b)))
              : (uint16_t)0;
  }
};
template <class Src>
__device__ __forceinline__ void rms_norm_row(const Src& x, const uint16_t* __restrict__ w, float eps, int D,
                                             uint16_t* __restrict__ o, float* wsum) {
  constexpr int kIt = 16;
  float ss = 0.0f;
  for (int p0 = 0; p0 < D; p0 += 256 * kIt) {
    typename Src::Raw v[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) v[it] = x.load(min(p0 + (int)threadIdx.x + 256 * it, D - 1));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int i = p0 + (int)threadIdx.x + 256 * it;
      const float f = i < D ? bf16_bits_to_f32(x.bits(v[it], i)) : 0.0f;
      ss = i < D ? fmaf(f, f, ss) : ss;
    }
  }
  ss = wave_sum_dpp(ss);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
  const float inv = __builtin_amdgcn_rsqf(tot / (float)D + eps);
  for (int p0 = 0; p0 < D; p0 += 256 * kIt) {
    typename Src::Raw xv[kIt];
    uint16_t wv[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int i = min(p0 + (int)threadIdx.x + 256 * it, D - 1);
      xv[it] = x.load(i);
      wv[it] = w[i];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int i = p0 + (int)threadIdx.x + 256 * it;
      const float t = bf16_bits_to_f32(f32_to_bf16_bits(bf16_bits_to_f32(x.bits(xv[it], min(i, D - 1))) * inv));
      if (i < D) o[i] = f32_to_bf16_bits(t * bf16_bits_to_f32(wv[it]));
    }
  }
}

// out[b, :D] = rms_norm(e[b], w_e), out[b, D:] = rms_norm(h[b], w_h). One workgroup
// (256 threads) per row and half.
__global__ __launch_bounds__(256) void k_pair_norm(const uint16_t* __restrict__ e, int64_t e_ld,
                                                   const uint16_t* __restrict__ h, int64_t h_ld,
                                                   const uint16_t* __restrict__ we, const uint16_t* __restrict__ wh,
                                                   float eps, int D, uint16_t* __restrict__ out, int64_t out_ld) {
  __shared__ float wsum[4];
  const int b = blockIdx.x >> 1, half = blockIdx.x & 1;
  const uint16_t* x = half ? h + (size_t)b * h_ld : e + (size_t)b * e_ld;
  rms_norm_row(RowBf16{x}, half ? wh : we, eps, D, out + (size_t)b * out_ld + half * D, wsum);
}

// dst[i] = src[i] for i < n by one 256-thread workgroup, each pass's loads issued before
// its stores
__device__ __forceinline__ void copy_row_u16(uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, int n) {
  constexpr int kIt = 16;
  for (int p0 = 0; p0 < n; p0 += 256 * kIt) {
    uint16_t v[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) v[it] = src[min(p0 + (int)threadIdx.x + 256 * it, n - 1)];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int it = 0; it < kIt; ++it)
      if (p0 + (int)threadIdx.x + 256 * it < n) dst[p0 + threadIdx.x + 256 * it] = v[it];
  }
}

// ---------------------------------------------------------------- argmax of keys
// The best key of row b over `slots` per-workgroup keys (hsd_linear's HSD_Y_ARGMAX), by
// one wavefront: the index (low 32 bits inverted) of the largest key.
// Up to 2048 keys (hsd_linear's most) are loaded in one pass, every load issued before the
// first is used: a loop with one load per step waited for each in turn (32 dependent round
// trips at 2048 slots). Indices past `slots` re-read the last key, which leaves the maximum
// unchanged.
__device__ int wave_argmax_keys(const uint64_t* keys, int slots, int lane) {
  constexpr int kPer = 32;
  uint64_t k = 0;
  for (int base = 0; base < slots; base += 64 * kPer) {
    uint64_t v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) v[i] = keys[min(base + lane + 64 * i, slots - 1)];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kPer; ++i) k = v[i] > k ? v[i] : k;
  }
  return (int)~(uint32_t)wave_max_u64(k);
}

// A plain decode step's end: tok = argmax; out_tokens[n] = tok (if n < cap); n += 1;
// pos += 1; cur = (cur + 1) % nslab. One wavefront.
__global__ __launch_bounds__(64) void k_decode_advance(const uint64_t* __restrict__ keys, int slots,
                                                       int32_t* __restrict__ seq, int32_t* __restrict__ out_tokens,
                                                       int cap, int nslab) {
  const int tok = wave_argmax_keys(keys, slots, threadIdx.x);
  if (threadIdx.x == 0) {
    const int n = seq[HSD_SEQ_N];
    if (n < cap) out_tokens[n] = tok;
    seq[HSD_SEQ_N] = n + 1;
    seq[HSD_SEQ_TOK] = tok;
    seq[HSD_SEQ_POS] += 1;
    if (nslab > 0) seq[HSD_SEQ_CUR] = (seq[HSD_SEQ_CUR] + 1) % nslab;
    seq[HSD_SEQ_STEPS] += 1;
  }
}

// A verify step's end: tgt[r] = argmax of row r (r <= k); a = first i < k with
// draft[i] != tgt[i], else k; the emitted tokens draft[:a] + [tgt[a]] go to out_tokens
// at n (up to cap) and to pend[0..a] (the MTP head's next rows); n, pos and cur advance
// by a + 1 (the rollback of the attention caches and of the Mamba rings); the head's
// cache keeps the rows of its last first call (head_pos += R) and R = a + 1.
// One workgroup of (k+1) wavefronts.
__global__ __launch_bounds__(256) void k_spec_accept(const uint64_t* __restrict__ keys, int64_t key_ld, int slots,
                                                     int k, const int32_t* __restrict__ ids,
                                                     int32_t* __restrict__ seq, int32_t* __restrict__ out_tokens,
                                                     int cap, int nslab, int32_t* __restrict__ pend,
                                                     int32_t* __restrict__ tgt_out) {
  __shared__ int tgt[8];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (w <= k) {
    const int t = wave_argmax_keys(keys + (size_t)w * key_ld, slots, lane);
    if (lane == 0) tgt[w] = t;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int a = k;
    for (int i = 0; i < k; ++i)
      if (ids[1 + i] != tgt[i]) { a = i; break; }
    const int n = seq[HSD_SEQ_N];
    for (int i = 0; i <= a; ++i) {
      const int tk = i < a ? ids[1 + i] : tgt[a];
      if (n + i < cap) out_tokens[n + i] = tk;
      if (pend) pend[i] = tk;
    }
    if (tgt_out)
      for (int i = 0; i <= k; ++i) tgt_out[i] = tgt[i];
    seq[HSD_SEQ_N] = n + a + 1;
    seq[HSD_SEQ_TOK] = tgt[a];
    seq[HSD_SEQ_POS] += a + 1;
    if (nslab > 0) seq[HSD_SEQ_CUR] = (seq[HSD_SEQ_CUR] + a + 1) % nslab;
    seq[HSD_SEQ_HEAD_POS] += seq[HSD_SEQ_R];
    seq[HSD_SEQ_R] = a + 1;
    seq[HSD_SEQ_ACCEPT] = a;
    seq[HSD_SEQ_STEPS] += 1;
    seq[HSD_SEQ_ACC_SUM] += a;
  }
}

// The chained call's inputs: row R-1 of the first call (its prediction and its normed
// hidden state), and that row's cache position head_pos + R.
__global__ __launch_bounds__(256) void k_mtp_chain(const uint64_t* __restrict__ keys, int64_t key_ld, int slots,
                                                   const uint16_t* __restrict__ hn, int64_t hn_ld, int D,
                                                   int32_t* __restrict__ seq, int32_t* __restrict__ d1,
                                                   uint16_t* __restrict__ h2) {
  const int R = seq[HSD_SEQ_R];
  const int r = min(max(R, 1), 3) - 1;
  if (threadIdx.x < 64) {
    const int t = wave_argmax_keys(keys + (size_t)r * key_ld, slots, threadIdx.x);
    if (threadIdx.x == 0) {
      d1[0] = t;
      seq[HSD_SEQ_HEAD_POS2] = seq[HSD_SEQ_HEAD_POS] + r + 1;
    }
  }
  copy_row_u16(h2, hn + (size_t)r * hn_ld, D);
}

// dst = src row R-1 (R = the pending-row count, clamped to [1, 3]).
__global__ __launch_bounds__(256) void k_select_row(const uint16_t* __restrict__ src, int64_t src_ld,
                                                    const int32_t* __restrict__ seq, uint16_t* __restrict__ dst,
                                                    int D) {
  const int r = min(max(seq[HSD_SEQ_R], 1), 3) - 1;
  copy_row_u16(dst, src + (size_t)r * src_ld, D);
}

// The verify ids [tok, d_0 .. d_{k-1}]: d_0 = the chained call's input prediction, d_1
// = the chained call's argmax (k = 2). With `script` (true tokens, indexed by the count
// of emitted tokens) and `accepts` (one accepted-draft count per step), the drafts are
// forced: d_i = true[n + i] for i < a_t, a guaranteed-wrong token at i = a_t.
__global__ __launch_bounds__(64) void k_draft(const int32_t* __restrict__ d1, const uint64_t* __restrict__ keys2,
                                              int slots, int k, int32_t* __restrict__ seq,
                                              const int32_t* __restrict__ script, int script_len,
                                              const int32_t* __restrict__ accepts, int n_accepts, int V,
                                              int32_t* __restrict__ ids) {
  int d2 = 0;
  if (k >= 2 && keys2) d2 = wave_argmax_keys(keys2, slots, threadIdx.x);
  if (threadIdx.x == 0) {
    ids[0] = seq[HSD_SEQ_TOK];
    int d[8];
    d[0] = d1 ? d1[0] : 0;
    if (k >= 2) d[1] = d2;
    for (int i = 2; i < k; ++i) d[i] = 0;
    if (script) {
      const int n = seq[HSD_SEQ_N];
      const int st = seq[HSD_SEQ_STEPS];
      const int at = accepts ? accepts[min(st, n_accepts - 1)] : k;
      for (int i = 0; i < k; ++i) {
        const int tt = script[min(n + i, script_len - 1)];
        d[i] = i < at ? tt : (i == at ? (tt + 1) % V : tt);
      }
    }
    for (int i = 0; i < k; ++i) ids[1 + i] = d[i];
  }
}

// The MTP head's input rows in one launch: out[b, :D] = rms_norm(embed(t_b), w_e),
// out[b, D:] = rms_norm(h[b], w_h) (k_embed_q4 then k_pair_norm, the same arithmetic; one
// workgroup per row and half). t_b = tok[b]; without tok (the chained call, B = 1) t is the
// argmax of `keys` and the chaining of k_mtp_chain happens here: d1[0] = t and HEAD_POS2 =
// HEAD_POS + R (R = seq[HSD_SEQ_R] clamped to [1, 3]); h is then the normed hidden row.
__global__ __launch_bounds__(256) void k_head_in(const int32_t* __restrict__ tok, const uint64_t* __restrict__ keys,
                                                 int slots, const uint32_t* __restrict__ ew,
                                                 const uint16_t* __restrict__ es, const uint16_t* __restrict__ eb,
                                                 int V, const uint16_t* __restrict__ h, int64_t h_ld,
                                                 const uint16_t* __restrict__ we, const uint16_t* __restrict__ wh,
                                                 float eps, int D, int32_t* __restrict__ seq, int32_t* __restrict__ d1,
                                                 uint16_t* __restrict__ out, int64_t out_ld,
                                                 int32_t* __restrict__ status) {
  __shared__ float wsum[4];
  __shared__ int tsh;
  const int b = blockIdx.x >> 1, half = blockIdx.x & 1;
  uint16_t* o = out + (size_t)b * out_ld + half * D;
  if (half) {
    rms_norm_row(RowBf16{h + (size_t)b * h_ld}, wh, eps, D, o, wsum);
    return;
  }
  int t;
  if (tok) {
    t = tok[b];
  } else {
    if (threadIdx.x < 64) {
      const int a = wave_argmax_keys(keys, slots, threadIdx.x);
      if (threadIdx.x == 0) {
        tsh = a;
        d1[0] = a;
        const int r = min(max(seq[HSD_SEQ_R], 1), 3) - 1;
        seq[HSD_SEQ_HEAD_POS2] = seq[HSD_SEQ_HEAD_POS] + r + 1;
      }
    }
    __syncthreads();
    t = tsh;
  }
  const bool ok = (unsigned)t < (unsigned)V;
  rms_norm_row(RowEmbed{ew, es, eb, ok ? (size_t)t : 0, D, ok}, we, eps, D, o, wsum);
  if (!ok && threadIdx.x == 0 && status) atomicOr(status, (int32_t)HSD_STATUS_BAD_TOKEN);
}

// k_draft and the embedding of the verify rows in one launch: workgroup r takes row r of
// [tok, d_0 .. d_{k-1}] (k_draft's rule, each workgroup for its own row: only the row of
// the chained call's draft ranks keys2), writes ids[r] and embeds it (k_embed_q4's rows).
__global__ __launch_bounds__(256) void k_verify_in(const int32_t* __restrict__ d1, const uint64_t* __restrict__ keys2,
                                                   int slots, int k, int32_t* __restrict__ seq,
                                                   const int32_t* __restrict__ script, int script_len,
                                                   const int32_t* __restrict__ accepts, int n_accepts, int V,
                                                   const uint32_t* __restrict__ ew, const uint16_t* __restrict__ es,
                                                   const uint16_t* __restrict__ eb, int D, int32_t* __restrict__ ids,
                                                   uint16_t* __restrict__ out, int64_t out_ld,
                                                   int32_t* __restrict__ status) {
  __shared__ int tsh;
  const int r = blockIdx.x;                            // 0: TOK, i = r - 1 >= 0: draft i
  if (threadIdx.x < 64) {
    int t;
    if (r == 0) {
      t = seq[HSD_SEQ_TOK];
    } else {
      const int i = r - 1;
      if (script) {
        const int n = seq[HSD_SEQ_N];
        const int st = seq[HSD_SEQ_STEPS];
        const int at = accepts ? accepts[min(st, n_accepts - 1)] : k;
        const int tt = script[min(n + i, script_len - 1)];
        t = i < at ? tt : (i == at ? (tt + 1) % V : tt);
      } else if (i == 0) {
        t = d1 ? d1[0] : 0;
      } else if (i == 1) {
        t = wave_argmax_keys(keys2, slots, threadIdx.x);
      } else {
        t = 0;
      }
    }
    if (threadIdx.x == 0) {
      tsh = t;
      ids[r] = t;
    }
  }
  __syncthreads();
  embed_row(tsh, ew, es, eb, V, D, out + (size_t)r * out_ld, status);
}

// dst[i] = src[clamp(POS + offset + i, 0, n - 1)]: the next rows' tokens of a prompt held
// on the device (a prefill step replays as one graph).
__global__ void k_gather_tokens(const int32_t* __restrict__ src, int n, const int32_t* __restrict__ seq,
                                int offset, int count, int32_t* __restrict__ dst) {
  const int i = threadIdx.x;
  if (i < count) dst[i] = src[min(max(seq[HSD_SEQ_POS] + offset + i, 0), n - 1)];
}

// The state after a prefill step of B rows at POS of a T-token prompt: the rows up to the
// prompt's end are kept (POS and CUR advance by min(B, T - POS)); the MTP head keeps the
// rows whose next token is a prompt token (HEAD_POS += min(B, T - 1 - POS), >= 0).
__global__ void k_prefill_advance(int32_t* seq, int T, int B, int nslab) {
  if (threadIdx.x == 0) {
    const int p = seq[HSD_SEQ_POS];
    const int valid = min(max(T - p, 0), B);
    const int head = min(max(T - 1 - p, 0), B);
    seq[HSD_SEQ_POS] = p + valid;
    if (nslab > 0) seq[HSD_SEQ_CUR] = (seq[HSD_SEQ_CUR] + valid) % nslab;
    seq[HSD_SEQ_HEAD_POS] += head;
  }
}

// POS -= n_drop and CUR -= n_drop (mod nslab): the rollback of a verify step's last
// n_drop rows (KVCache.trim, model.py:355; the checkpoint ring still holds the state).
__global__ void k_seq_rollback(int32_t* seq, int n_drop, int nslab) {
  if (threadIdx.x == 0) {
    seq[HSD_SEQ_POS] -= n_drop;
    if (nslab > 0) seq[HSD_SEQ_CUR] = ((seq[HSD_SEQ_CUR] - n_drop) % nslab + nslab) % nslab;
  }
}

// seq[idx] += delta (host-known adjustments outside a graph, e.g. the head's prefill rows)
__global__ void k_seq_add(int32_t* seq, int idx, int delta) {
  if (threadIdx.x == 0) seq[idx] += delta;
}

}  // namespace
}  // namespace hsd

using namespace hsd;

extern "C" int hsd_embed_q4(const int32_t* tok, int64_t B, const uint32_t* w, const uint16_t* scales,
                            const uint16_t* biases, int64_t V, int64_t D, uint16_t* out, int64_t out_ld,
                            int32_t* dev_status, void* stream) {
  const char* fn = "hsd_embed_q4";
  if (!tok || !w || !scales || !biases || !out) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (B < 0 || B > 65535 || V <= 0 || V > 0x7FFFFFFF || D <= 0 || D % 64 || out_ld < D || out_ld % 8)
    return set_error(HSD_ERR_SHAPE, "%s: need D %% 64 == 0 and out_ld >= D, a multiple of 8", fn);
  if ((uintptr_t)out & 15u) return set_error(HSD_ERR_ALIGN, "%s: out must be 16-byte aligned", fn);
  if (B == 0) return HSD_OK;
  hipLaunchKernelGGL(k_embed_q4, dim3((unsigned)B), dim3(256), 0, as_stream(stream), tok, w, scales, biases, (int)V,
                     (int)D, out, out_ld, dev_status);
  return check_launch(fn);
}

extern "C" int hsd_pair_norm(const uint16_t* e, int64_t e_ld, const uint16_t* h, int64_t h_ld, const uint16_t* we,
                             const uint16_t* wh, float eps, int64_t B, int64_t D, uint16_t* out, int64_t out_ld,
                             void* stream) {
  const char* fn = "hsd_pair_norm";
  if (!e || !h || !we || !wh || !out) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (B < 0 || B > 65535 || D <= 0 || e_ld < D || h_ld < D || out_ld < 2 * D)
    return set_error(HSD_ERR_SHAPE, "%s: row strides", fn);
  if (B == 0) return HSD_OK;
  hipLaunchKernelGGL(k_pair_norm, dim3((unsigned)(2 * B)), dim3(256), 0, as_stream(stream), e, e_ld, h, h_ld, we, wh,
                     eps, (int)D, out, out_ld);
  return check_launch(fn);
}

extern "C" int hsd_decode_advance(const uint64_t* argmax_keys, int64_t slots, int32_t* seq, int32_t* out_tokens,
                                  int64_t cap, int64_t nslab, void* stream) {
  const char* fn = "hsd_decode_advance";
  if (!argmax_keys || !seq || (cap > 0 && !out_tokens)) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (slots <= 0 || slots > (1 << 30) || cap < 0 || cap > 0x7FFFFFFF || nslab < 0 || nslab > 64)
    return set_error(HSD_ERR_SHAPE, "%s: bad sizes", fn);
  hipLaunchKernelGGL(k_decode_advance, dim3(1), dim3(64), 0, as_stream(stream), argmax_keys, (int)slots, seq,
                     out_tokens, (int)cap, (int)nslab);
  return check_launch(fn);
}

extern "C" int hsd_spec_accept(const uint64_t* argmax_keys, int64_t key_ld, int64_t slots, int64_t k,
                               const int32_t* ids, int32_t* seq, int32_t* out_tokens, int64_t cap, int64_t nslab,
                               int32_t* pend, int32_t* tgt, void* stream) {
  const char* fn = "hsd_spec_accept";
  if (!argmax_keys || !ids || !seq || (cap > 0 && !out_tokens)) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (k < 1 || k > 3 || slots <= 0 || slots > key_ld || cap < 0 || cap > 0x7FFFFFFF || nslab < 0 || nslab > 64 ||
      (nslab > 0 && nslab < k + 2))
    return set_error(HSD_ERR_SHAPE, "%s: need 1 <= k <= 3, slots <= key_ld, nslab 0 or >= k + 2", fn);
  hipLaunchKernelGGL(k_spec_accept, dim3(1), dim3(256), 0, as_stream(stream), argmax_keys, key_ld, (int)slots, (int)k,
                     ids, seq, out_tokens, (int)cap, (int)nslab, pend, tgt);
  return check_launch(fn);
}

extern "C" int hsd_mtp_chain(const uint64_t* argmax_keys, int64_t key_ld, int64_t slots, const uint16_t* hn,
                             int64_t hn_ld, int64_t D, int32_t* seq, int32_t* d1, uint16_t* h2, void* stream) {
  const char* fn = "hsd_mtp_chain";
  if (!argmax_keys || !hn || !seq || !d1 || !h2) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (slots <= 0 || (key_ld != 0 && slots > key_ld) || D <= 0 || (hn_ld != 0 && hn_ld < D) || key_ld < 0 || hn_ld < 0)
    return set_error(HSD_ERR_SHAPE, "%s: bad sizes", fn);
  hipLaunchKernelGGL(k_mtp_chain, dim3(1), dim3(256), 0, as_stream(stream), argmax_keys, key_ld, (int)slots, hn,
                     hn_ld, (int)D, seq, d1, h2);
  return check_launch(fn);
}

extern "C" int hsd_seq_select_row(const uint16_t* src, int64_t src_ld, const int32_t* seq, uint16_t* dst, int64_t D,
                                  void* stream) {
  const char* fn = "hsd_seq_select_row";
  if (!src || !seq || !dst) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (D <= 0 || D > (1 << 24) || src_ld < D) return set_error(HSD_ERR_SHAPE, "%s: bad sizes", fn);
  hipLaunchKernelGGL(k_select_row, dim3(1), dim3(256), 0, as_stream(stream), src, src_ld, seq, dst, (int)D);
  return check_launch(fn);
}

extern "C" int hsd_draft_ids(const int32_t* d1, const uint64_t* argmax_keys2, int64_t slots, int64_t k, int32_t* seq,
                             const int32_t* script, int64_t script_len, const int32_t* accepts, int64_t n_accepts,
                             int64_t V, int32_t* ids, void* stream) {
  const char* fn = "hsd_draft_ids";
  if (!seq || !ids || (k >= 2 && !script && !argmax_keys2)) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (k < 1 || k > 7 || V <= 0 || (script && script_len <= 0) || (accepts && n_accepts <= 0) ||
      (argmax_keys2 && slots <= 0))
    return set_error(HSD_ERR_SHAPE, "%s: bad sizes", fn);
  hipLaunchKernelGGL(k_draft, dim3(1), dim3(64), 0, as_stream(stream), d1, argmax_keys2, (int)slots, (int)k, seq,
                     script, (int)script_len, accepts, (int)n_accepts, (int)V, ids);
  return check_launch(fn);
}

extern "C" int hsd_head_input(const int32_t* tok, const uint64_t* argmax_keys, int64_t slots, const uint32_t* w,
                              const uint16_t* scales, const uint16_t* biases, int64_t V, const uint16_t* h,
                              int64_t h_ld, const uint16_t* we, const uint16_t* wh, float eps, int64_t B, int64_t D,
                              int32_t* seq, int32_t* d1, uint16_t* out, int64_t out_ld, int32_t* dev_status,
                              void* stream) {
  const char* fn = "hsd_head_input";
  if (!w || !scales || !biases || !h || !we || !wh || !out) return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (!tok && (!argmax_keys || !seq || !d1))
    return set_error(HSD_ERR_ARG, "%s: without tok, argmax_keys, seq and d1 are needed", fn);
  if (B < 0 || B > 65535 || (!tok && B != 1) || V <= 0 || V > 0x7FFFFFFF || D <= 0 || D % 64 || h_ld < D ||
      out_ld < 2 * D || (!tok && (slots <= 0 || slots > (1 << 30))))
    return set_error(HSD_ERR_SHAPE, "%s: need D %% 64 == 0, row strides h_ld >= D and out_ld >= 2 D, B == 1 without tok",
                     fn);
  if (B == 0) return HSD_OK;
  hipLaunchKernelGGL(k_head_in, dim3((unsigned)(2 * B)), dim3(256), 0, as_stream(stream), tok, argmax_keys, (int)slots,
                     w, scales, biases, (int)V, h, h_ld, we, wh, eps, (int)D, seq, d1, out, out_ld, dev_status);
  return check_launch(fn);
}

extern "C" int hsd_verify_input(const int32_t* d1, const uint64_t* argmax_keys2, int64_t slots, int64_t k, int32_t* seq,
                                const int32_t* script, int64_t script_len, const int32_t* accepts, int64_t n_accepts,
                                int64_t V, const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int64_t D,
                                int32_t* ids, uint16_t* out, int64_t out_ld, int32_t* dev_status, void* stream) {
  const char* fn = "hsd_verify_input";
  if (!seq || !ids || !w || !scales || !biases || !out || (k >= 2 && !script && !argmax_keys2))
    return set_error(HSD_ERR_ARG, "%s: null pointer", fn);
  if (k < 1 || k > 7 || V <= 0 || V > 0x7FFFFFFF || (script && script_len <= 0) || (accepts && n_accepts <= 0) ||
      (argmax_keys2 && slots <= 0) || D <= 0 || D % 64 || out_ld < D || out_ld % 8)
    return set_error(HSD_ERR_SHAPE, "%s: bad sizes", fn);
  if ((uintptr_t)out & 15u) return set_error(HSD_ERR_ALIGN, "%s: out must be 16-byte aligned", fn);
  hipLaunchKernelGGL(k_verify_in, dim3((unsigned)(k + 1)), dim3(256), 0, as_stream(stream), d1, argmax_keys2,
                     (int)slots, (int)k, seq, script, (int)script_len, accepts, (int)n_accepts, (int)V, w, scales,
                     biases, (int)D, ids, out, out_ld, dev_status);
  return check_launch(fn);
}

extern "C" int hsd_seq_add(int32_t* seq, int64_t idx, int64_t delta, void* stream) {
  if (!seq) return set_error(HSD_ERR_ARG, "hsd_seq_add: null pointer");
  if (idx < 0 || idx >= HSD_SEQ_LEN) return set_error(HSD_ERR_SHAPE, "hsd_seq_add: bad index");
  hipLaunchKernelGGL(k_seq_add, dim3(1), dim3(64), 0, as_stream(stream), seq, (int)idx, (int)delta);
  return check_launch("hsd_seq_add");
}

extern "C" int hsd_gather_tokens(const int32_t* src, int64_t n, const int32_t* seq, int64_t offset, int64_t count,
                                 int32_t* dst, void* stream) {
  if (!src || !seq || !dst) return set_error(HSD_ERR_ARG, "hsd_gather_tokens: null pointer");
  if (n <= 0 || n > 0x7FFFFFFF || count < 0 || count > 64 || offset < -65536 || offset > 65536)
    return set_error(HSD_ERR_SHAPE, "hsd_gather_tokens: bad sizes");
  if (count == 0) return HSD_OK;
  hipLaunchKernelGGL(k_gather_tokens, dim3(1), dim3(64), 0, as_stream(stream), src, (int)n, seq, (int)offset,
                     (int)count, dst);
  return check_launch("hsd_gather_tokens");
}

extern "C" int hsd_prefill_advance(int32_t* seq, int64_t T, int64_t B, int64_t nslab, void* stream) {
  if (!seq) return set_error(HSD_ERR_ARG, "hsd_prefill_advance: null pointer");
  if (T < 0 || T > 0x7FFFFFFF || B < 1 || B > 64 || nslab < 0 || nslab > 64)
    return set_error(HSD_ERR_SHAPE, "hsd_prefill_advance: bad sizes");
  hipLaunchKernelGGL(k_prefill_advance, dim3(1), dim3(64), 0, as_stream(stream), seq, (int)T, (int)B, (int)nslab);
  return check_launch("hsd_prefill_advance");
}

extern "C" int hsd_seq_rollback(int32_t* seq, int64_t n_drop, int64_t nslab, void* stream) {
  if (!seq) return set_error(HSD_ERR_ARG, "hsd_seq_rollback: null pointer");
  if (n_drop < 0 || n_drop > 64 || nslab < 0 || nslab > 64 || (nslab > 0 && n_drop >= nslab))
    return set_error(HSD_ERR_SHAPE, "hsd_seq_rollback: need 0 <= n_drop < nslab");
  hipLaunchKernelGGL(k_seq_rollback, dim3(1), dim3(64), 0, as_stream(stream), seq, (int)n_drop, (int)nslab);
  return check_launch("hsd_seq_rollback");
}
