// Shared helpers of libhsd: error state, launch checks, bf16/f16 conversion, the
// XCD-aware workgroup remap. gfx950 (MI355X) only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/hsd.h"

namespace hsd {

// ---------------------------------------------------------------- error state
// One message per host thread; entry points return a negative code and leave the
// message here (hsd_last_error).
int set_error(int code, const char* fmt, ...);

// Checks the launch that was just issued on this thread.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Workgroups of `kernel` (`threads` each, `lds` bytes of dynamic LDS) resident at once on
// the current device (occupancy x CUs), looked up once per kernel, size and device;
// `fallback` when the runtime cannot say. A grid no larger than this has no workgroup
// waiting for another to finish.
int resident_workgroups(const void* kernel, int threads, size_t lds, int fallback);

// ---------------------------------------------------------------- bf16 / f16
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits) {
  return __uint_as_float(bits << 16);
}

// Round to nearest even; every NaN becomes the canonical quiet NaN 0x7FC0.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t bits) {
  return (float)__builtin_bit_cast(_Float16, bits);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Element loads/stores by dtype tag (HSD_DT_*).
template <int DT> struct Elem;
template <> struct Elem<HSD_DT_BF16> {
  using T = uint16_t;
  __device__ __forceinline__ static float load(const T* p, size_t i) { return bf16_bits_to_f32(p[i]); }
  __device__ __forceinline__ static void store(T* p, size_t i, float v) { p[i] = f32_to_bf16_bits(v); }
};
template <> struct Elem<HSD_DT_F16> {
  using T = uint16_t;
  __device__ __forceinline__ static float load(const T* p, size_t i) { return f16_bits_to_f32(p[i]); }
  __device__ __forceinline__ static void store(T* p, size_t i, float v) { p[i] = f32_to_f16_bits(v); }
};
template <> struct Elem<HSD_DT_F32> {
  using T = float;
  __device__ __forceinline__ static float load(const T* p, size_t i) { return p[i]; }
  __device__ __forceinline__ static void store(T* p, size_t i, float v) { p[i] = v; }
};

// ---------------------------------------------------------------- XCD remap
// MI355X dispatches workgroup i of a launch to XCD i % 8 (round robin). This maps a
// hardware workgroup id to a logical one so that logically consecutive workgroups run
// on the same XCD and share its L2 (neighbouring 64-byte pieces of one weight row,
// one tile's column blocks). Bijective for any n.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  const int q = n / kXcds, r = n % kXcds;
  const int x = bid % kXcds, i = bid / kXcds;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + i;
}

// Workgroup barrier that orders LDS accesses only. __syncthreads() also waits for every
// outstanding global access of the wave (the hardware counts loads and stores together),
// which would end the flight of loads issued ahead of the barrier for later use.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// v in a vector register the compiler cannot see through. The 4-bit decodes build a bf16
// pair as ((w >> k) & mask) | one: with both constants as literals that compiles to a
// v_and_b32 and a v_or_b32 (the three-operand v_and_or_b32 takes no literal on this
// target); with the mask in a register and the other constant in a scalar register it is one
// v_and_or_b32. Call once per kernel, outside the loops.
__device__ __forceinline__ uint32_t opaque_vgpr(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// v read from another lane of the same 16-lane row by a DPP control (quad_perm, row
// mirrors: every source lane is inside the row)
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, false);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// The maximum of a 64-bit key over each 16-lane row, in every lane of the row: DPP
// quad_perm xor 1, xor 2, row_half_mirror, row_mirror (no LDS). Needs the row's lanes
// active.
__device__ __forceinline__ uint64_t row16_max_u64(uint64_t k) {
  k = max_u64(k, dpp_u64<0xB1>(k));
  k = max_u64(k, dpp_u64<0x4E>(k));
  k = max_u64(k, dpp_u64<0x141>(k));
  k = max_u64(k, dpp_u64<0x140>(k));
  return k;
}

// The maximum of a 64-bit key over the 64 lanes, in every lane: the row maxima, then
// v_permlane16_swap and v_permlane32_swap (each lane then holds its value and that of lane
// l ^ 16, then l ^ 32, in some order). No LDS; needs every lane active.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
  k = row16_max_u64(k);
  {
    const uint32_t hi = (uint32_t)(k >> 32), lo = (uint32_t)k;
    const auto h = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    const auto l = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    k = max_u64(((uint64_t)h[0] << 32) | l[0], ((uint64_t)h[1] << 32) | l[1]);
  }
  {
    const uint32_t hi = (uint32_t)(k >> 32), lo = (uint32_t)k;
    const auto h = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    const auto l = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    k = max_u64(((uint64_t)h[0] << 32) | l[0], ((uint64_t)h[1] << 32) | l[1]);
  }
  return k;
}

// The maximum of a float over the 64 lanes, in every lane (fmaxf: a NaN loses to a
// number), by the same moves as wave_max_u64. Needs every lane active.
__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  const uint32_t b = __float_as_uint(v);
  const auto p16 = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  v = fmaxf(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
  const uint32_t c = __float_as_uint(v);
  const auto p32 = __builtin_amdgcn_permlane32_swap(c, c, false, false);
  return fmaxf(__uint_as_float(p32[0]), __uint_as_float(p32[1]));
}

// silu(x) = x / (1 + e^-x), with the hardware exponential and reciprocal (a few ulp;
// the IEEE division and the libm exponential are long dependent sequences).
__device__ __forceinline__ float silu_f32(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// softplus(x) = log(1 + e^x); above 20 it equals x in fp32.
__device__ __forceinline__ float softplus_f32(float x) {
  return x > 20.0f ? x : log1pf(expf(x));
}

// Inclusive prefix sum over the 64 lanes of a wavefront without LDS: a DPP scan inside
// each 16-lane row (row_shr 1, 2, 4, 8; lanes shifted in from outside the row read 0),
// then the totals of the lower rows (v_readlane of lanes 15, 31, 47) added per row.
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);
  const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31),
            r2 = __builtin_amdgcn_readlane(v, 47);
  const int row = lane >> 4;
  return v + (row > 0 ? r0 : 0) + (row > 1 ? r1 : 0) + (row > 2 ? r2 : 0);
}

// Sum over the 64 lanes of a wavefront without LDS, the same in every lane: DPP sums
// inside each 16-lane row (quad_perm xor 1, xor 2, row_half_mirror, row_mirror), then the
// four row sums in a fixed order. Needs every lane active.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x141>(v);
  v += dpp_f32<0x140>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return ((r0 + r1) + r2) + r3;
}

// Deterministic butterfly sum over the 64 lanes of a wavefront (same tree on every
// call, so equal inputs give equal bits).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace hsd
