// Shared device helpers for the gfx950 attention kernels: element types, 16-byte vector
// access, wave64 cross-lane reductions and the thread-local error channel of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/miattn.h"

namespace miattn {

// ------------------------------------------------------------------ error channel
// Set by every failing entry point; mi_last_error() returns it. Thread-local so two host
// threads driving different streams never read each other's message.
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int launch_status(const char* what);

// ------------------------------------------------------------------ element types
// bf16 and fp16 travel as raw 16-bit patterns; arithmetic is always fp32.
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float(uint32_t(x.bits) << 16); }
__device__ __forceinline__ float to_f32(f16_t x) {
  return __half2float(__ushort_as_half(x.bits));
}

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
// Round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950), NaN kept quiet: the same rounding
// torch uses for .to(bfloat16).
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) {
  return bf16_t{__builtin_bit_cast(uint16_t, (__bf16)x)};
}
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float x) {
  return f16_t{__half_as_ushort(__float2half_rn(x))};
}

// Unpack the i-th element of a 16-byte vector holding 16/sizeof(T) elements.
template <typename T> struct Vec16;
template <> struct Vec16<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static float get(const uint4& v, int i) {
    const uint32_t w = i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
    return __uint_as_float(w);
  }
};
template <> struct Vec16<bf16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static float get(const uint4& v, int i) {
    const uint32_t w = (i >> 1) == 0 ? v.x : (i >> 1) == 1 ? v.y : (i >> 1) == 2 ? v.z : v.w;
    return (i & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
  }
};
template <> struct Vec16<f16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static float get(const uint4& v, int i) {
    const uint32_t w = (i >> 1) == 0 ? v.x : (i >> 1) == 1 ? v.y : (i >> 1) == 2 ? v.z : v.w;
    const uint16_t h = (i & 1) ? uint16_t(w >> 16) : uint16_t(w & 0xffffu);
    return __half2float(__ushort_as_half(h));
  }
};

__device__ __forceinline__ uint4 load16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}
__device__ __forceinline__ void store16(void* p, const uint4& v) {
  *reinterpret_cast<uint4*>(p) = v;
}

// Sum over s = 0 .. parts-1 (parts >= 1) of f[s * plane], added in that order in fp32 (the
// split-K partial sums of one output element), split into a load and a sum step so a kernel
// can issue the loads of all its elements before any arithmetic (an empty asm in a rounding
// helper is a scheduling barrier the loads would otherwise not cross). kU > 0 needs
// parts <= kU: kU loads with the index clamped to the last partial (always in bounds) and a
// straight-line sum. kU = 0: a plain loop for any count, summed at load time.
template <int kU>
struct PartSum {
  static constexpr int N = kU > 0 ? kU : 1;
  float v[N];
  __device__ __forceinline__ void load(const float* f, int parts, int64_t plane) {
    if constexpr (kU == 0) {
      float acc = f[0];
      for (int s = 1; s < parts; ++s) acc += f[s * plane];
      v[0] = acc;
    } else {
#pragma unroll
      for (int s = 0; s < kU; ++s) v[s] = f[int64_t(s < parts ? s : parts - 1) * plane];
    }
  }
  __device__ __forceinline__ float sum(int parts) const {
    float acc = v[0];
#pragma unroll
    for (int s = 1; s < N; ++s) acc = s < parts ? acc + v[s] : acc;
    return acc;
  }
};

// Unroll class of PartSum for a partial count; -1: no partials (the input holds T values).
constexpr int parts_unroll(int parts) { return parts == 0 ? -1 : (parts <= 2 ? 2 : (parts <= 8 ? 8 : 0)); }

// 16-byte global load and store with the nontemporal (streaming) hint, for data that one
// kernel touches once.
typedef unsigned u32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load16_nt(const void* p) {
  const u32x4_nt w = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
  return make_uint4(w.x, w.y, w.z, w.w);
}
__device__ __forceinline__ void store16_nt(void* p, const uint4& v) {
  const u32x4_nt w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4_nt*>(p));
}

// ------------------------------------------------------------------ cross-lane reductions
// DPP butterflies inside one 16-lane DPP row. quad_perm [1,0,3,2] and [2,3,0,1] exchange
// lanes xor 1 and xor 2; once every quad holds one value, row_half_mirror (lane i <- 7-i)
// pairs the two quads of a half-row, and once every half-row is uniform, row_mirror
// (lane i <- 15-i) pairs the two halves. Each step is a single DPP-modified VALU op.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
constexpr int kDppQuadXor1 = 0xB1;
constexpr int kDppQuadXor2 = 0x4E;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
// row_ror:8: lane i of each 16-lane row reads lane (i + 8) mod 16 (the other half-row).
constexpr int kDppRowRor8 = 0x128;

// Exchange with lane ^ 16 (inside each 32-lane half) via ds_swizzle bitmask mode.
__device__ __forceinline__ float swap16(float x) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401F));
}
// Exchange with lane ^ 32: gfx950 v_permlane32_swap.
__device__ __forceinline__ float swap32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(__lane_id() < 32 ? r[1] : r[0]);
}

// max / sum of x over lanes i and i ^ 32: swapped with a copy of itself, the two results
// of v_permlane32_swap hold x's low and high half in every lane, so one op combines them
// (no lane select after the swap)
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

struct SumOp {
  __device__ __forceinline__ static float op(float a, float b) { return a + b; }
};
struct MaxOp {
  __device__ __forceinline__ static float op(float a, float b) { return fmaxf(a, b); }
};

// All-reduce over aligned groups of W consecutive lanes (W in 1..64, power of two).
template <int W, typename Op>
__device__ __forceinline__ float group_allreduce(float x) {
  if constexpr (W >= 2) x = Op::op(x, dpp<kDppQuadXor1>(x));
  if constexpr (W >= 4) x = Op::op(x, dpp<kDppQuadXor2>(x));
  if constexpr (W >= 8) x = Op::op(x, dpp<kDppRowHalfMirror>(x));
  if constexpr (W >= 16) x = Op::op(x, dpp<kDppRowMirror>(x));
  if constexpr (W >= 32) x = Op::op(x, swap16(x));
  if constexpr (W >= 64) x = Op::op(x, swap32(x));
  return x;
}

// Round an fp32 result to T (the rounding a tensor op of dtype T applies to its result).
// The value goes through an empty asm first: without it the compiler may fold
// round_T(op_f32(a, b)) into the native fp16 op (division, square root), whose rounding
// differs from the fp32 op rounded once (measured: 21% of fp16 outputs one ulp off the
// tensor ops).
template <typename T>
__device__ __forceinline__ float rt(float x) {
  asm volatile("" : "+v"(x));
  return to_f32(from_f32<T>(x));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace miattn
