// Decode-step attention epilogue of one layer, fused: per-head RMSNorm of q and k, NeoX
// RoPE at each row's position, q out contiguous for the paged decode, k and v scattered into
// the paged pool at each row's write slot.
//
// The reference runs these as separate tensor ops between the projections and the paged
// decode: q_norm / k_norm (RMSNorm, reference model/layers.py:342-350, applied at :193-194),
// apply_rotary_emb (:59-89, applied at :210-211), then PagedKV.write, whose slot scatter is
// mi_kv_slot_write (model/paged.py:503-520). At the decode shape (B = 32 rows, 16 + 8 + 8
// heads of 128) every one of those ops is a few microseconds of launch for kilobytes of
// data; here the whole epilogue is one launch.
//
// Arithmetic follows the reference's tensor ops step by step in the activation dtype: each
// elementwise result is rounded to the dtype as the op it restates would store it (x^2, the
// mean, mean + eps, its square root, x / rms, (x / rms) * w, and each product and sum of the
// rotation), with the mean's sum accumulated in fp32 as the reduction kernel does. The
// result equals the tensor-op chain's except where the fp32 sum's order moves a rounding
// boundary.
//
// With k_out / v_out the roped k and the v of each row are also written packed, (B, H_kv, D)
// contiguous, for a packed prefill's attention (the decode reads them from the pool).
//
// Layout: one wave per (row, head) over q, k and v heads of a packed projection row
// [q (H x D) | k (H_kv x D) | v (H_kv x D)]; lane l holds the rotation pairs (p, p + D/2)
// for p = l, l + 64, ... < D/2, so the pair partner is in the same lane. The projection
// rows are T, or fp32 split-K partial sums [parts][B][row_stride] of mi_rows_gemm, summed
// in split order and rounded once to T (the value the projection's own output would hold).
#include <type_traits>

#include "common.h"

namespace miattn {
namespace {

// Round an fp32 result to T. The value goes through an empty asm first: without it the
// compiler may fold round_T(op_f32(a, b)) into the native fp16 op (division, square root),
// whose rounding differs from the fp32 op rounded once (measured: 21% of fp16 outputs one
// ulp off the tensor ops).
template <typename T>
__device__ __forceinline__ float rt(float x) {
  asm volatile("" : "+v"(x));
  return to_f32(from_f32<T>(x));
}

template <typename T, int D, typename IdxT, int kU>
__global__ __launch_bounds__(256) void qk_norm_rope_write_kernel(
    const void* __restrict__ qkv, int64_t row_stride, int parts, int64_t plane, const T* __restrict__ q_w,
    const T* __restrict__ k_w,
    const T* __restrict__ cos_tab, const T* __restrict__ sin_tab, int64_t n_pos,
    const int64_t* __restrict__ pos, const IdxT* __restrict__ slots, T* __restrict__ q_out,
    T* __restrict__ k_pool, T* __restrict__ v_pool, T* __restrict__ k_out, T* __restrict__ v_out, int B, int H,
    int H_kv, int64_t n_slots, float eps, int32_t* __restrict__ err) {
  constexpr int HALF = D / 2;
  constexpr int PPL = (HALF + 63) / 64;  // rotation pairs per lane
  const int lane = threadIdx.x & 63;
  const int head = blockIdx.y * (blockDim.x / 64) + (threadIdx.x >> 6);  // over q, k, v heads
  const int b = blockIdx.x;
  const int n_heads = H + 2 * H_kv;
  if (head >= n_heads || b >= B) return;  // wave-uniform
  // a row whose position is outside the RoPE table or whose slot is outside the pool is
  // not written at all and is reported (row + 1) through the error word
  const int64_t pb = pos[b];
  const IdxT slot = slots[b];
  if (pb < 0 || pb >= n_pos || !(slot >= 0 && int64_t(slot) < n_slots)) {
    if (lane == 0 && head == 0 && err != nullptr) atomicCAS(err, 0, b + 1);
    return;
  }
  const int64_t src = int64_t(b) * row_stride + int64_t(head) * D;
  // every load of this wave's inputs first, then the arithmetic (the rounding helper's empty
  // asm is a scheduling barrier)
  constexpr int kP = kU < 0 ? 1 : kU;
  PartSum<kP> r1[PPL], r2[PPL];
#pragma unroll
  for (int j = 0; j < PPL; ++j) {
    const int p = min(lane + 64 * j, HALF - 1);
    if constexpr (kU < 0) {
      r1[j].v[0] = to_f32(static_cast<const T*>(qkv)[src + p]);
      r2[j].v[0] = to_f32(static_cast<const T*>(qkv)[src + p + HALF]);
    } else {
      r1[j].load(static_cast<const float*>(qkv) + src + p, parts, plane);
      r2[j].load(static_cast<const float*>(qkv) + src + p + HALF, parts, plane);
    }
  }
  // norm weights and this row's RoPE table entries (read here, used after the reduction)
  const bool is_q = head < H;
  const T* w = is_q ? q_w : k_w;
  const T* cr = cos_tab + pb * HALF;
  const T* sr = sin_tab + pb * HALF;
  float w1[PPL], w2[PPL], cs[PPL], sn[PPL];
#pragma unroll
  for (int j = 0; j < PPL; ++j) {
    const int p = min(lane + 64 * j, HALF - 1);
    w1[j] = to_f32(w[p]);
    w2[j] = to_f32(w[p + HALF]);
    cs[j] = to_f32(cr[p]);
    sn[j] = to_f32(sr[p]);
  }
  float x1[PPL], x2[PPL];
#pragma unroll
  for (int j = 0; j < PPL; ++j) {
    const bool live = lane + 64 * j < HALF;
    if constexpr (kU < 0) {
      x1[j] = live ? r1[j].v[0] : 0.0f;
      x2[j] = live ? r2[j].v[0] : 0.0f;
    } else {
      x1[j] = live ? rt<T>(r1[j].sum(parts)) : 0.0f;
      x2[j] = live ? rt<T>(r2[j].sum(parts)) : 0.0f;
    }
  }

  if (head >= H + H_kv) {  // v head: copied as is (exact: x1/x2 hold T values)
    const int vh = head - H - H_kv;
    T* dst = v_pool + (int64_t(slot) * H_kv + vh) * D;
    T* dst2 = v_out != nullptr ? v_out + (int64_t(b) * H_kv + vh) * D : nullptr;
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
      const int p = lane + 64 * j;
      if (p < HALF) {
        dst[p] = from_f32<T>(x1[j]);
        dst[p + HALF] = from_f32<T>(x2[j]);
        if (dst2 != nullptr) {
          dst2[p] = from_f32<T>(x1[j]);
          dst2[p + HALF] = from_f32<T>(x2[j]);
        }
      }
    }
    return;
  }

  // RMSNorm: mean of the rounded squares (fp32 sum), then the reference's rounding steps
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < PPL; ++j) ss += rt<T>(x1[j] * x1[j]) + rt<T>(x2[j] * x2[j]);
  ss = group_allreduce<64, SumOp>(ss);
  const float ms = rt<T>(ss * (1.0f / D));
  const float rms = rt<T>(sqrtf(rt<T>(ms + eps)));
  // RoPE at this row's position (table rows of D/2)
  float o1[PPL], o2[PPL];
#pragma unroll
  for (int j = 0; j < PPL; ++j) {
    const int p = lane + 64 * j;
    if (p < HALF) {
      const float a = rt<T>(rt<T>(x1[j] / rms) * w1[j]);
      const float c = rt<T>(rt<T>(x2[j] / rms) * w2[j]);
      o1[j] = rt<T>(rt<T>(a * cs[j]) - rt<T>(c * sn[j]));
      o2[j] = rt<T>(rt<T>(a * sn[j]) + rt<T>(c * cs[j]));
    }
  }

  T* dst;
  T* dst2 = nullptr;  // the packed k copy, when asked for
  if (is_q) {
    dst = q_out + (int64_t(b) * H + head) * D;
  } else {
    dst = k_pool + (int64_t(slot) * H_kv + (head - H)) * D;
    if (k_out != nullptr) dst2 = k_out + (int64_t(b) * H_kv + (head - H)) * D;
  }
#pragma unroll
  for (int j = 0; j < PPL; ++j) {
    const int p = lane + 64 * j;
    if (p < HALF) {
      dst[p] = from_f32<T>(o1[j]);
      dst[p + HALF] = from_f32<T>(o2[j]);
      if (dst2 != nullptr) {
        dst2[p] = from_f32<T>(o1[j]);
        dst2[p + HALF] = from_f32<T>(o2[j]);
      }
    }
  }
}

template <typename T, int D>
int launch_d(const void* qkv, int64_t row_stride, int parts, const void* q_w, const void* k_w, const void* cos_tab,
             const void* sin_tab, int64_t n_pos, const int64_t* pos, const void* slots, int slot_bits,
             void* q_out, void* k_pool, void* v_pool, void* k_out, void* v_out, int B, int H, int H_kv,
             int64_t n_slots, float eps, int32_t* err, hipStream_t s) {
  constexpr int kWaves = 4;
  const dim3 grid(B, (H + 2 * H_kv + kWaves - 1) / kWaves);
  const int64_t plane = int64_t(B) * row_stride;
  auto go = [&](auto idx_tag, auto unroll) {
    using IdxT = decltype(idx_tag);
    hipLaunchKernelGGL((qk_norm_rope_write_kernel<T, D, IdxT, decltype(unroll)::value>), grid, dim3(64 * kWaves), 0, s, qkv,
                       row_stride, parts, plane, static_cast<const T*>(q_w), static_cast<const T*>(k_w),
                       static_cast<const T*>(cos_tab), static_cast<const T*>(sin_tab), n_pos, pos,
                       static_cast<const IdxT*>(slots), static_cast<T*>(q_out), static_cast<T*>(k_pool),
                       static_cast<T*>(v_pool), static_cast<T*>(k_out), static_cast<T*>(v_out), B, H, H_kv,
                       n_slots, eps, err);
  };
  auto by_slots = [&](auto unroll) {
    if (slot_bits == 32) go(int32_t{}, unroll); else go(int64_t{}, unroll);
  };
  switch (parts_unroll(parts)) {
    case -1: by_slots(std::integral_constant<int, -1>{}); break;
    case 2: by_slots(std::integral_constant<int, 2>{}); break;
    case 8: by_slots(std::integral_constant<int, 8>{}); break;
    default: by_slots(std::integral_constant<int, 0>{}); break;
  }
  return launch_status("mi_qk_norm_rope_write");
}

template <typename T>
int launch_t(int D, const void* qkv, int64_t row_stride, int parts, const void* q_w, const void* k_w, const void* cos_tab,
             const void* sin_tab, int64_t n_pos, const int64_t* pos, const void* slots, int slot_bits,
             void* q_out, void* k_pool, void* v_pool, void* k_out, void* v_out, int B, int H, int H_kv,
             int64_t n_slots, float eps, int32_t* err, hipStream_t s) {
  switch (D) {
    case 64: return launch_d<T, 64>(qkv, row_stride, parts, q_w, k_w, cos_tab, sin_tab, n_pos, pos, slots, slot_bits,
                                    q_out, k_pool, v_pool, k_out, v_out, B, H, H_kv, n_slots, eps, err, s);
    case 128: return launch_d<T, 128>(qkv, row_stride, parts, q_w, k_w, cos_tab, sin_tab, n_pos, pos, slots, slot_bits,
                                      q_out, k_pool, v_pool, k_out, v_out, B, H, H_kv, n_slots, eps, err, s);
    case 256: return launch_d<T, 256>(qkv, row_stride, parts, q_w, k_w, cos_tab, sin_tab, n_pos, pos, slots, slot_bits,
                                      q_out, k_pool, v_pool, k_out, v_out, B, H, H_kv, n_slots, eps, err, s);
    default:
      return fail(MI_ERR_UNSUPPORTED, "mi_qk_norm_rope_write: head_dim %d is not supported (64, 128, 256)", D);
  }
}

}  // namespace
}  // namespace miattn

extern "C" int mi_qk_norm_rope_write(const void* qkv, int64_t row_stride, int qkv_parts, const void* q_norm_w,
                                     const void* k_norm_w, const void* cos_tab, const void* sin_tab,
                                     int64_t n_pos, const int64_t* pos, const void* slot_ids, int slot_bits,
                                     void* q_out, void* k_pool, void* v_pool, void* k_out, void* v_out, int B,
                                     int H, int H_kv, int D, int64_t n_slots, float eps, int dtype,
                                     int32_t* error_word, void* stream) {
  using namespace miattn;
  if (B < 0 || H < 1 || H_kv < 1 || H % H_kv != 0) {
    return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: n_head (%d) must be a multiple of n_kv_head (%d)", H, H_kv);
  }
  if (slot_bits != 32 && slot_bits != 64) {
    return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: slot_bits must be 32 or 64, got %d", slot_bits);
  }
  if (n_pos < 1) return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: the RoPE table is empty");
  if (qkv_parts < 0) return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: qkv_parts %d < 0", qkv_parts);
  if (row_stride < int64_t(H + 2 * H_kv) * D) {
    return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: row stride %lld < %d packed q/k/v elements",
                (long long)row_stride, (H + 2 * H_kv) * D);
  }
  if (qkv == nullptr || q_norm_w == nullptr || k_norm_w == nullptr || cos_tab == nullptr || sin_tab == nullptr ||
      pos == nullptr || slot_ids == nullptr || q_out == nullptr || k_pool == nullptr || v_pool == nullptr) {
    return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: NULL pointer argument");
  }
  if (B == 0) return MI_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MI_BF16: return launch_t<bf16_t>(D, qkv, row_stride, qkv_parts, q_norm_w, k_norm_w, cos_tab, sin_tab, n_pos, pos,
                                          slot_ids, slot_bits, q_out, k_pool, v_pool, k_out, v_out, B, H, H_kv, n_slots, eps,
                                          error_word, s);
    case MI_F16: return launch_t<f16_t>(D, qkv, row_stride, qkv_parts, q_norm_w, k_norm_w, cos_tab, sin_tab, n_pos, pos,
                                        slot_ids, slot_bits, q_out, k_pool, v_pool, k_out, v_out, B, H, H_kv, n_slots, eps,
                                        error_word, s);
    case MI_F32: return launch_t<float>(D, qkv, row_stride, qkv_parts, q_norm_w, k_norm_w, cos_tab, sin_tab, n_pos, pos,
                                        slot_ids, slot_bits, q_out, k_pool, v_pool, k_out, v_out, B, H, H_kv, n_slots, eps,
                                        error_word, s);
    default:
      return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: unknown dtype %d", dtype);
  }
}
